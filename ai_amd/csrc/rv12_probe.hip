// Measurement probe (not part of the C ABI of librv12): the pure weight
// stream of the vector linear, for the ceiling a launch of that shape can
// reach.  Same grid, waves, step order, buffer loads and prefetch depth as
// k_gemv at one token, with the decode, the activations, the FMAs and the
// exceptions left out: each lane folds its 12-byte groups with xor and
// writes one word, so no load is dead.  Built into librv12probe.so for
// bench.py only.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rv12_device.h"

namespace rv12 {

template <int RB, int D>
__global__ __launch_bounds__(1024) void k_stream(const uint32_t* __restrict__ tiles, int N, int K,
                                                 uint32_t* __restrict__ out) {
    const int W = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wu = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nsteps = K >> 5;
    const int64_t nblk = (N + 15) / 16;
    const int64_t blk0 = (int64_t)blockIdx.x * RB;
    const int nvalid = (int)min((int64_t)RB, nblk - blk0);
    const uint32_t blk_bytes = (uint32_t)nsteps * kStepBytes;
    const char* wbase = reinterpret_cast<const char*>(tiles) + blk0 * (int64_t)blk_bytes;
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(wbase, (uint32_t)nvalid * blk_bytes);
    const __amdgpu_buffer_rsrc_t rnull = make_rsrc(wbase, 0u);
    int voff[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) voff[b] = (int)(b * blk_bytes) + lane * 12;
    u32x3 buf[D][RB];
    const int s0 = wu;
#pragma unroll
    for (int u = 0; u < D; ++u) {
        const int s = s0 + u * W;
        const __amdgpu_buffer_rsrc_t r = s < nsteps ? rv : rnull;
#pragma unroll
        for (int b = 0; b < RB; ++b) buf[u][b] = load_group(r, voff[b], (s < nsteps ? s : 0) * kStepBytes);
    }
    uint32_t acc = 0;
    const int rounds = ((nsteps - s0 + W - 1) / W + D - 1) / D;
    for (int rr = 0; rr < rounds; ++rr) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
#pragma unroll
            for (int b = 0; b < RB; ++b) acc ^= buf[u][b].x ^ buf[u][b].y ^ buf[u][b].z;
            const int s = s0 + (rr * D + u + D) * W;
            const __amdgpu_buffer_rsrc_t r = s < nsteps ? rv : rnull;
#pragma unroll
            for (int b = 0; b < RB; ++b) buf[u][b] = load_group(r, voff[b], (s < nsteps ? s : 0) * kStepBytes);
        }
    }
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

}  // namespace rv12

extern "C" int rv12_probe_stream(const void* tiles, int n, int k, int rb, int waves, int depth, void* out,
                                 void* stream) {
    using namespace rv12;
    if (!tiles || !out || n < 1 || k < 32 || k % 32 || waves < 1 || waves > 16) return -1;
    const int64_t nblk = ((int64_t)n + 15) / 16;
    const dim3 grid((unsigned)((nblk + rb - 1) / rb)), block((unsigned)(waves * 64));
    hipStream_t st = (hipStream_t)stream;
#define RV12_PROBE(R, DD) hipLaunchKernelGGL((k_stream<R, DD>), grid, block, 0, st, (const uint32_t*)tiles, n, k, (uint32_t*)out)
    if (rb == 1 && depth == 4) RV12_PROBE(1, 4);
    else if (rb == 1 && depth == 6) RV12_PROBE(1, 6);
    else if (rb == 1 && depth == 8) RV12_PROBE(1, 8);
    else if (rb == 2 && depth == 4) RV12_PROBE(2, 4);
    else if (rb == 2 && depth == 6) RV12_PROBE(2, 6);
    else if (rb == 2 && depth == 8) RV12_PROBE(2, 8);
    else return -1;
#undef RV12_PROBE
    return hipGetLastError() == hipSuccess ? 0 : -20;
}
