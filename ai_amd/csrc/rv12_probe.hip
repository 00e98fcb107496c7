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
    int voff[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) voff[b] = (int)(b * blk_bytes) + lane * 12;
    // the linear's addressing: the step's offset in the vector offset, a step
    // past the end at 2^31 + the row-block offset (past the descriptor: zeros,
    // no memory access)
    auto issue = [&](u32x3 (&dst)[RB], int s) {
        const uint32_t off = s < nsteps ? (uint32_t)s * kStepBytes : 0x80000000u;
#pragma unroll
        for (int b = 0; b < RB; ++b) dst[b] = load_group(rv, (int)((uint32_t)voff[b] + off), 0);
    };
    u32x3 buf[D][RB];
    const int s0 = wu;
#pragma unroll
    for (int u = 0; u < D; ++u) {
        issue(buf[u], s0 + u * W);
        asm volatile("" ::: "memory");  // issued in step order, as the linear's
    }
    uint32_t acc = 0;
    // the linear's loop: a step's words are used before the load D steps
    // ahead reuses their registers (the fence keeps the compiler's scheduler
    // from hoisting the load), so D loads stay in flight across the rounds
    for (int sr = s0; sr < nsteps; sr += D * W) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
#pragma unroll
            for (int b = 0; b < RB; ++b) acc ^= buf[u][b].x ^ buf[u][b].y ^ buf[u][b].z;
            asm volatile("" : "+v"(acc)::"memory");
            issue(buf[u], sr + (u + D) * W);
        }
    }
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

// The same stream with 16-byte loads: the row block's bytes in 3 KB chunks
// (four steps of 768 bytes), chunk c read by wave c % W as three 1 KB loads
// (lane l the 16 bytes at 16 l of each), D chunks in flight per wave (D = 2
// holds the bytes of 8 steps).  Host condition: K % 128 == 0.
template <int D>
__global__ __launch_bounds__(1024) void k_stream16(const uint32_t* __restrict__ tiles, int N, int K,
                                                   uint32_t* __restrict__ out) {
    const int W = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wu = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nchunk = K >> 7;
    const int64_t nblk = (N + 15) / 16;
    const int64_t blk0 = blockIdx.x;
    const uint32_t blk_bytes = (uint32_t)(K >> 5) * kStepBytes;
    const char* wbase = reinterpret_cast<const char*>(tiles) + blk0 * (int64_t)blk_bytes;
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(wbase, blk0 < nblk ? blk_bytes : 0u);
    const __amdgpu_buffer_rsrc_t rnull = make_rsrc(wbase, 0u);
    u32x4 buf[D][3];
    auto issue = [&](u32x4 (&b)[3], int c) {
        const __amdgpu_buffer_rsrc_t r = c < nchunk ? rv : rnull;
        const int soff = (c < nchunk ? c : 0) * 3072;
#pragma unroll
        for (int i = 0; i < 3; ++i)
            b[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, i * 1024 + lane * 16, soff,
                                                                                   kNonTemporal));
    };
#pragma unroll
    for (int u = 0; u < D; ++u) issue(buf[u], wu + u * W);
    uint32_t acc = 0;
    const int rounds = ((nchunk - wu + W - 1) / W + D - 1) / D;
    for (int rr = 0; rr < rounds; ++rr) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
#pragma unroll
            for (int i = 0; i < 3; ++i) acc ^= buf[u][i].x ^ buf[u][i].y ^ buf[u][i].z ^ buf[u][i].w;
            issue(buf[u], wu + (rr * D + u + D) * W);
        }
    }
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

// The first `depth` weight steps of every wave of the vector linear's
// one-row-block launch (the bytes its prefetch asks for first), read with
// ordinary (temporal) loads, so that a launch right after it finds them in
// the caches if the caches keep them across the kernel boundary.
__global__ __launch_bounds__(1024) void k_warm(const uint32_t* __restrict__ tiles, int N, int K, int depth,
                                               uint32_t* __restrict__ out) {
    const int W = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wu = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nsteps = K >> 5;
    const int64_t nblk = (N + 15) / 16;
    const int64_t blk0 = blockIdx.x;
    const uint32_t blk_bytes = (uint32_t)nsteps * kStepBytes;
    const char* wbase = reinterpret_cast<const char*>(tiles) + blk0 * (int64_t)blk_bytes;
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(wbase, blk0 < nblk ? blk_bytes : 0u);
    uint32_t acc = 0;
    for (int u = 0; u < depth; ++u) {
        const int s = wu + u * W;
        const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(rv, lane * 12, (s < nsteps ? s : 0) * kStepBytes, 0);
        acc ^= v.x ^ v.y ^ v.z;
    }
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

}  // namespace rv12

extern "C" int rv12_probe_warm(const void* tiles, int n, int k, int waves, int depth, void* out, void* stream) {
    using namespace rv12;
    if (!tiles || !out || n < 1 || k < 32 || k % 32 || waves < 1 || waves > 16 || depth < 1 || depth > 64) return -1;
    const dim3 grid((unsigned)(((int64_t)n + 15) / 16)), block((unsigned)(waves * 64));
    hipLaunchKernelGGL(k_warm, grid, block, 0, (hipStream_t)stream, (const uint32_t*)tiles, n, k, depth, (uint32_t*)out);
    return hipGetLastError() == hipSuccess ? 0 : -20;
}

extern "C" int rv12_probe_stream16(const void* tiles, int n, int k, int waves, int depth, void* out, void* stream) {
    using namespace rv12;
    if (!tiles || !out || n < 1 || k < 128 || k % 128 || waves < 1 || waves > 16) return -1;
    const dim3 grid((unsigned)(((int64_t)n + 15) / 16)), block((unsigned)(waves * 64));
    hipStream_t st = (hipStream_t)stream;
    if (depth == 1) hipLaunchKernelGGL((k_stream16<1>), grid, block, 0, st, (const uint32_t*)tiles, n, k, (uint32_t*)out);
    else if (depth == 2) hipLaunchKernelGGL((k_stream16<2>), grid, block, 0, st, (const uint32_t*)tiles, n, k, (uint32_t*)out);
    else if (depth == 3) hipLaunchKernelGGL((k_stream16<3>), grid, block, 0, st, (const uint32_t*)tiles, n, k, (uint32_t*)out);
    else return -1;
    return hipGetLastError() == hipSuccess ? 0 : -20;
}

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

namespace rv12 {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef const __attribute__((address_space(4))) f32x16 cf32x16;

// Arrival of the activations inside one launch of the vector linear's shape
// at one token (one row block per workgroup, D = 6 weight steps in flight
// per wave).  Every workgroup stages the K activations into LDS, then
// streams its weights (WS) and folds them with the staged values; lane 0 of
// each wave records the 100 MHz real-time counter at entry, after the
// workgroup barrier that ends the staging, and at the end.
// SC = false: vector loads, NX float4 chunks per thread issued before the
//   weight prefetch and written to LDS after it (the linear's order);
// SC = true: scalar loads (a uniform address in the constant address space),
//   each wave 32-float pieces of its K / W slice, two pieces in flight (scalar
//   loads return out of order, so the wave waits for both), each
//   piece moved to VGPRs of lane 0 (v_mov from the SGPRs) and written with
//   eight 16-byte LDS stores; the weight prefetch is issued after the first
//   two pieces.
// Host conditions: K == 4 * NX * 64 * W, K <= 16384 (LDS of K floats).
template <bool SC, bool WS, int NX>
__global__ __launch_bounds__(1024) void k_arrival(const uint32_t* __restrict__ tiles, int N, int K,
                                                  const float* __restrict__ x, uint32_t* __restrict__ out,
                                                  uint64_t* __restrict__ ts) {
    constexpr int D = 6;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    extern __shared__ float xl[];
    const int W = blockDim.x >> 6;
    const int nthr = blockDim.x;
    const int lane = threadIdx.x & 63;
    const int wu = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nsteps = K >> 5;
    const int64_t nblk = (N + 15) / 16;
    const int64_t blk0 = blockIdx.x;
    const uint32_t blk_bytes = (uint32_t)nsteps * kStepBytes;
    const char* wbase = reinterpret_cast<const char*>(tiles) + blk0 * (int64_t)blk_bytes;
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(wbase, blk0 < nblk ? blk_bytes : 0u);
    const __amdgpu_buffer_rsrc_t rnull = make_rsrc(wbase, 0u);
    const int voff = lane * 12;
    const int s0 = wu;
    u32x3 buf[D];
    auto prefetch = [&]() {
        if constexpr (WS) {
#pragma unroll
            for (int u = 0; u < D; ++u) {
                const int s = s0 + u * W;
                buf[u] = load_group(s < nsteps ? rv : rnull, voff, (s < nsteps ? s : 0) * kStepBytes);
            }
        }
    };
    if constexpr (!SC) {
        f32x4 xr[NX];
#pragma unroll
        for (int j = 0; j < NX; ++j) xr[j] = *reinterpret_cast<const f32x4*>(x + (threadIdx.x + j * nthr) * 4);
        __builtin_amdgcn_s_barrier();
        prefetch();
#pragma unroll
        for (int j = 0; j < NX; ++j) *reinterpret_cast<f32x4*>(xl + (threadIdx.x + j * nthr) * 4) = xr[j] * kXScale;
    } else {
        const int sl = K / W;  // floats of this wave's slice, a multiple of 64
        const cf32x16* cx = (const cf32x16*)(x + (int64_t)wu * sl);
        float* xw = xl + wu * sl;
        auto put = [&](f32x16 a, f32x16 b, int c) {
            if (lane == 0) {
                f32x4* dst = reinterpret_cast<f32x4*>(xw + c * 32);
#pragma unroll
                for (int g = 0; g < 4; ++g) dst[g] = f32x4{a[4 * g], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]} * kXScale;
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    dst[4 + g] = f32x4{b[4 * g], b[4 * g + 1], b[4 * g + 2], b[4 * g + 3]} * kXScale;
            }
        };
        const int np = sl / 32;  // even
        // the loads are written as asm so that the compiler issues them here,
        // before the barrier and the weight prefetch (it would sink loads of
        // the constant address space past both); the asm wait below ties the
        // four values, so no use of them is scheduled before it
        f32x16 a0, b0, a1, b1;
        auto load4 = [&](const cf32x16* src) {
            asm volatile("s_load_dwordx16 %0, %4, 0x0\n\t"
                         "s_load_dwordx16 %1, %4, 0x40\n\t"
                         "s_load_dwordx16 %2, %4, 0x80\n\t"
                         "s_load_dwordx16 %3, %4, 0xc0"
                         : "=s"(a0), "=s"(b0), "=s"(a1), "=s"(b1)
                         : "s"(src)
                         : "memory");
        };
        load4(cx);
        asm volatile("s_barrier" ::: "memory");
        prefetch();
        for (int c = 0; c < np; c += 2) {
            asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(a0), "+s"(b0), "+s"(a1), "+s"(b1)::"memory");
            put(a0, b0, c);
            put(a1, b1, c + 1);
            if (c + 2 < np) load4(cx + 2 * c + 4);
        }
    }
    __syncthreads();
    const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
    uint32_t acc = 0;
    if constexpr (WS) {
        const int rounds = ((nsteps - s0 + W - 1) / W + D - 1) / D;
        for (int rr = 0; rr < rounds; ++rr) {
#pragma unroll
            for (int u = 0; u < D; ++u) {
                const int s = s0 + (rr * D + u) * W;
                acc ^= buf[u].x ^ buf[u].y ^ buf[u].z ^ __float_as_uint(xl[(s < nsteps ? s : 0) * 32 + (lane & 31)]);
                const int sn = s + D * W;
                buf[u] = load_group(sn < nsteps ? rv : rnull, voff, (sn < nsteps ? sn : 0) * kStepBytes);
            }
        }
    } else {
        acc = __float_as_uint(xl[threadIdx.x % K]);
    }
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
    const uint64_t t2 = __builtin_amdgcn_s_memrealtime();
    if (lane == 0) {
        uint64_t* tw = ts + ((int64_t)blockIdx.x * W + wu) * 3;
        tw[0] = t0;
        tw[1] = t1;
        tw[2] = t2;
    }
}

}  // namespace rv12

// mode bit 0: scalar staging; bit 1: with the weight stream.  ts receives
// three 100 MHz counter values per wave: [workgroup][wave][entry, staged, end]
extern "C" int rv12_probe_arrival(const void* tiles, int n, int k, int waves, int mode, const void* x, void* out,
                                  void* ts, void* stream) {
    using namespace rv12;
    if (!tiles || !x || !out || !ts || n < 1 || k < 32 || k > 16384 || waves < 1 || waves > 16 ||
        k % (64 * waves) || mode < 0 || mode > 3)
        return -1;
    const int nx = k / (256 * waves);  // float4 chunks per thread
    if (nx < 1 || nx > 4 || nx * 256 * waves != k) return -1;
    const dim3 grid((unsigned)(((int64_t)n + 15) / 16)), block((unsigned)(waves * 64));
    const size_t lds = (size_t)k * 4;
    hipStream_t st = (hipStream_t)stream;
#define RV12_ARR(S, WW, X) hipLaunchKernelGGL((k_arrival<S, WW, X>), grid, block, lds, st, (const uint32_t*)tiles, n, \
                                              k, (const float*)x, (uint32_t*)out, (uint64_t*)ts)
#define RV12_ARR_X(S, WW)                 \
    if (nx == 1) RV12_ARR(S, WW, 1);      \
    else if (nx == 2) RV12_ARR(S, WW, 2); \
    else if (nx == 3) RV12_ARR(S, WW, 3); \
    else RV12_ARR(S, WW, 4);
    if (mode == 0) { RV12_ARR_X(false, false) }
    else if (mode == 1) { RV12_ARR_X(true, false) }
    else if (mode == 2) { RV12_ARR_X(false, true) }
    else { RV12_ARR_X(true, true) }
#undef RV12_ARR_X
#undef RV12_ARR
    return hipGetLastError() == hipSuccess ? 0 : -20;
}
