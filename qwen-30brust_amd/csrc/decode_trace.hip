// Phase-trace build of the persistent token step: the same kernel with
// QH_MARK(k, p) recording the wall clock (s_memrealtime, 100 MHz) of each
// workgroup at mark p of part k (the last layer of a launch overwrites the
// earlier ones).  Linked into libqwen_hip_trace.so in place of decode.o; read
// with qh_dtrace_dump after a step.  Not part of the product library.
#define QH_PHASE_TRACE 1
#include "decode.hip"

namespace qh {
__device__ unsigned long long g_dtrace[8][512][8];
__device__ void qh_phase_mark(int k, int p) {
    if (threadIdx.x == 0) g_dtrace[k][blockIdx.x][p] = wall_clock64();
}
__device__ void qh_phase_mark_last(int k, int p) {
    if ((threadIdx.x & 63) == 0) atomicMax(&g_dtrace[k][blockIdx.x][p], (unsigned long long)wall_clock64());
}
}  // namespace qh

// Copies the [8][512][8] mark table to host memory.
extern "C" int qh_dtrace_dump(void* host) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(qh::g_dtrace), sizeof(qh::g_dtrace));
}
// Clears the mark table.
extern "C" int qh_dtrace_clear() {
    static unsigned long long zero[8][512][8];
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(qh::g_dtrace), zero, sizeof(zero));
}
