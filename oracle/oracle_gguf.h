/* Oracle GGUF structures (internal).  TEST INFRASTRUCTURE ONLY. */
#ifndef QWEN_ORACLE_GGUF_H
#define QWEN_ORACLE_GGUF_H
#include <stddef.h>
#include <stdint.h>

enum { M_UINT = 1, M_INT, M_FLOAT, M_BOOL, M_STR, M_ARRAY };

typedef struct {
    int tag;
    uint64_t u;
    int64_t i;
    double f;
    char *s;
} or_meta;

typedef struct {
    char *name;
    uint32_t rank;
    uint64_t dims[3];
    uint32_t kind;
    size_t offset, len;
} or_tensor;

struct or_gguf {
    const uint8_t *data;
    size_t len;
    char **keys;
    or_meta *vals;
    size_t nmeta;
    or_tensor *t;
    size_t nt;
};

const or_tensor *or_gguf_find(const or_gguf *g, const char *name);
const char *or_gguf_str(const or_gguf *g, const char *key);

#endif
