// rv12 prefill linear: the 12-bit decode fused into a bf16x3 MFMA GEMM over
// all the prompt's tokens at once (gfx950).  Replaces the blocked prefill's
// decode_rows + fp32 GEMM (ramvi/engine/ramvi_engine/kernels/prefill.py:66-78,
// prefill_kernels.py:8-26 and 58-110): every weight is read once per prompt
// in its 12-bit form, never written back in a wider format.
//
// y[t] (=|+=) W_dec . x'[t], t < T, with the MODE prologue (2: x' =
// silu(x[0:K]) * x[K:2K]) or the RMSNorm prologue of mode 0 (x' = lnw x,
// the token's rs = 1 / sqrt(mean x^2 + eps) applied to its outputs, as the
// decode kernels apply it).  Two passes:
//   1. k_prefill_x: one workgroup per 16 tokens: each token's exponent scale
//      P_t (64 when its largest |x'| lies in [2^-40, 2^63), else 100 minus
//      the exponent of the largest) and, with RMS, its rs (sum of squares of
//      x 2^-32), then x' 2^P_t split into bf16 parts
//      hi + mid + lo (24 significand bits, as the reference's _x3 split,
//      wcomp.py:130-140) in B-operand lane order: for token block tb, step
//      s (32 columns) and part, 64 lanes x 8 bf16 (lane l: token l%16,
//      k = 8(l/16) + 0..7).  Token rows past T are zeros.
//   2. k_prefill_mm: workgroup = 256 rows x 128 tokens, 8 waves of 64 rows x
//      64 tokens.  Per 32-column step each wave reads its 4 row blocks' Q16
//      tiles straight from memory, three steps ahead (they are the A operand
//      of v_mfma_f32_16x16x32_bf16, the h values w 2^-sc); the step's B parts
//      of the workgroup's 8 token blocks are loaded three steps ahead into
//      registers and pass through LDS (double-buffered, one barrier per
//      step); 4 x 4 tiles x 3 parts = 48 MFMAs accumulate in 16 independent
//      fp32 accumulators.  Epilogue: v = acc 2^(sc_row - P_t) (exact); the
//      packed form's exception entries of the wave's rows (weights outside a
//      row's window, zeros in the tiles) add ev * x'[t][col] in list order,
//      x' gathered from x in fp32; with RMS v is scaled by rs_t; then y is
//      stored or added; rows past N and tokens past T are skipped.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rv12_device.h"
#include "rv12_internal.h"

namespace rv12 {

constexpr int kPfRowBlocks = 16;  // row blocks (of 16 rows) per workgroup
constexpr int kPfTokBlocks = 8;   // token blocks (of 16 tokens) per workgroup
constexpr int kPfThreads = 512;
constexpr int kPfDepth = 2;       // weight steps in flight per wave beyond the current one
static_assert((kPfDepth + 1) % 3 == 0, "the B register ring (3 sets) is indexed by the unrolled step");

// x' of token row xr at columns k..k+7 (MODE 2: silu(g) * u; lnw: the RMS
// weight times x)
__device__ __forceinline__ void prefill_xprime(const float* xr, int K, int k, bool m2, const uint16_t* lnw,
                                               float (&v)[8]) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(xr + k);
    const f32x4 b = *reinterpret_cast<const f32x4*>(xr + k + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    if (lnw) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(lnw + k);
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] *= __uint_as_float(ww[i] << 16);
            v[2 * i + 1] *= __uint_as_float(ww[i] & 0xFFFF0000u);
        }
    }
    if (m2) {
        const f32x4 c = *reinterpret_cast<const f32x4*>(xr + K + k);
        const f32x4 d = *reinterpret_cast<const f32x4*>(xr + K + k + 4);
        const float u[8] = {c.x, c.y, c.z, c.w, d.x, d.y, d.z, d.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = silu_mul(v[e], u[e]);
    }
}

// 1. grid (token blocks of the padded T), kPxThreads threads: 16 waves per
// 16 tokens, so the few workgroups of a prompt keep enough loads in flight
constexpr int kPxThreads = 1024;
constexpr int kPxWaves = kPxThreads / 64;
__global__ __launch_bounds__(kPxThreads) void k_prefill_x(const float* __restrict__ x, int T, int K, int xs, int m2,
                                                   const uint16_t* __restrict__ lnw, float eps,
                                                   u32x4* __restrict__ xb, int* __restrict__ P,
                                                   float* __restrict__ R) {
    __shared__ int emax[kPxWaves][16];
    __shared__ float ssq[kPxWaves][16];
    __shared__ int ps[16];
    const int tb = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nsteps = K >> 5;
    // (a) the largest exponent of |x'| per token and, with RMS, the sum of
    // squares of x 2^-32: thread (tok, sub) over columns 8 sub + 8 kPxThreads / 16 i
    {
        const int tok = tid & 15, sub = tid >> 4;
        const int t = tb * 16 + tok;
        int e = -1000;
        float sq = 0.0f;
        if (t < T) {
            const float* xr = x + (int64_t)t * xs;
            for (int k = sub * 8; k < K; k += kPxThreads / 2) {
                float v[8];
                prefill_xprime(xr, K, k, m2 != 0, nullptr, v);
                if (lnw) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) sq += (v[i] * kSsqScale) * (v[i] * kSsqScale);
                    const u32x4 w = *reinterpret_cast<const u32x4*>(lnw + k);
                    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        v[2 * i] *= __uint_as_float(ww[i] << 16);
                        v[2 * i + 1] *= __uint_as_float(ww[i] & 0xFFFF0000u);
                    }
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) e = max(e, exp_or_min(v[i]));
            }
        }
        e = max(e, __shfl_xor(e, 16));
        e = max(e, __shfl_xor(e, 32));
        sq += __shfl_xor(sq, 16);
        sq += __shfl_xor(sq, 32);
        if (lane < 16) {
            emax[wave][lane] = e;
            ssq[wave][lane] = sq;
        }
    }
    __syncthreads();
    if (tid < 16) {
        int e = emax[0][tid];
        float q = ssq[0][tid];
        for (int w = 1; w < kPxWaves; ++w) {  // a fixed order
            e = max(e, emax[w][tid]);
            q += ssq[w][tid];
        }
        const int p = (e >= -39 && e <= kXRangeHi) ? kXScaleExp : slow_scale_exp(e);
        ps[tid] = p;
        P[tb * 16 + tid] = p;
        if (lnw) R[tb * 16 + tid] = rms_scale(q, K, eps);
    }
    __syncthreads();
    // (b) the parts: thread (tok, k8, ss) writes steps ss + kPxWaves i, lane 16 k8 + tok
    const int tok = tid & 15, k8 = (tid >> 4) & 3, ss = tid >> 6;
    const int t = tb * 16 + tok;
    const int p = ps[tok];
    const float* xr = x + (int64_t)min(t, T - 1) * xs;
    for (int s = ss; s < nsteps; s += kPxWaves) {
        u32x4 hi = {0, 0, 0, 0}, mid = {0, 0, 0, 0}, lo = {0, 0, 0, 0};
        if (t < T) {
            float v[8];
            prefill_xprime(xr, K, s * 32 + k8 * 8, m2 != 0, lnw, v);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = ldexpf(v[i], p);
            split3(v, hi, mid, lo);
        }
        u32x4* d = xb + ((int64_t)tb * nsteps + s) * 192 + k8 * 16 + tok;
        d[0] = hi;
        d[64] = mid;
        d[128] = lo;
    }
}

// 2. grid (row tiles of 256 rows, token tiles of 128), 512 threads.  M2 / LN
// (the silu(g) * u and RMS prologues) are template arguments, so that the
// exception gathers of the epilogue are straight-line loads per variant.
template <bool M2, bool LN>
__global__ __launch_bounds__(kPfThreads) void k_prefill_mm(const uint32_t* __restrict__ tiles,
                                                           const int32_t* __restrict__ rbase,
                                                           const u32x4* __restrict__ xb, const int* __restrict__ P,
                                                           const int32_t* __restrict__ rp,
                                                           const int32_t* __restrict__ er,
                                                           const int32_t* __restrict__ ec,
                                                           const float* __restrict__ ev, const float* __restrict__ x,
                                                           const uint16_t* __restrict__ lnw,
                                                           const float* __restrict__ R, float* __restrict__ y, int N,
                                                           int K, int T, int xs, int m2, int add) {
    __shared__ u32x4 bs[2][kPfTokBlocks * 3 * 64];  // 2 x 24 KB
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave & 3, wc = wave >> 2;
    const int nsteps = K >> 5;
    const int64_t nblk = (N + 15) / 16;
    const int64_t blk0 = (int64_t)blockIdx.x * kPfRowBlocks + wr * 4;  // this wave's first row block
    const int tb0 = blockIdx.y * kPfTokBlocks;                            // the workgroup's first token block
    const int nvalid = (int)max((int64_t)0, min((int64_t)4, nblk - blk0));
    const uint32_t blk_bytes = (uint32_t)nsteps * kStepBytes;
    const char* wbase = reinterpret_cast<const char*>(tiles) + blk0 * (int64_t)blk_bytes;
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(wbase, (uint32_t)nvalid * blk_bytes);
    const __amdgpu_buffer_rsrc_t rnull = make_rsrc(wbase, 0u);
    int voff[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) voff[b] = (int)(b * blk_bytes) + lane * 12;
    auto issue_a = [&](u32x3 (&dst)[4], int s) {
        const __amdgpu_buffer_rsrc_t r = s < nsteps ? rv : rnull;
        const int soff = (s < nsteps ? s : 0) * kStepBytes;
#pragma unroll
        for (int b = 0; b < 4; ++b) dst[b] = load_group(r, voff[b], soff);
    };
    // the B parts of step s for the workgroup's token blocks: 3 groups per
    // thread, through a descriptor over the workgroup's parts (a step past the
    // end reads zeros through a 0-byte one), so no load sits behind a branch
    // and every wait counts only the loads it needs
    const u32x4* xbw = xb + (int64_t)tb0 * nsteps * 192;
    const __amdgpu_buffer_rsrc_t rbx = make_rsrc(xbw, (uint32_t)kPfTokBlocks * nsteps * 192 * 16);
    const __amdgpu_buffer_rsrc_t rbnull = make_rsrc(xbw, 0u);
    int boff[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int idx = tid + j * kPfThreads;  // (token block, part, lane) of the step
        boff[j] = ((idx / 192) * nsteps * 192 + idx % 192) * 16;
    }
    auto load_b = [&](u32x4 (&dst)[3], int s) {
        const __amdgpu_buffer_rsrc_t r = s < nsteps ? rbx : rbnull;
        const int soff = (s < nsteps ? s : 0) * 192 * 16;
#pragma unroll
        for (int j = 0; j < 3; ++j)
            dst[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, boff[j], soff, 0));
    };
    auto store_b = [&](const u32x4 (&src)[3], int buf) {
#pragma unroll
        for (int j = 0; j < 3; ++j) bs[buf][tid + j * kPfThreads] = src[j];
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[b][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    u32x3 ring[kPfDepth + 1][4];
#pragma unroll
    for (int u = 0; u <= kPfDepth; ++u) issue_a(ring[u], u);
    // B parts: loaded three steps ahead into a ring of three register sets
    // (the set of step s + 3 is the one step s's parts left, stored to LDS at
    // the end of step s - 1), stored to LDS one step ahead (double buffer), so
    // a store waits for a load issued two steps earlier while the later loads
    // stay in flight
    // The loop runs the steps in whole rounds of the unroll: steps past
    // nsteps read zeros (A and B), add nothing, and keep the loop body free of
    // branches around loads.
    u32x4 breg[3][3];
    load_b(breg[0], 0);
    load_b(breg[1], 1);
    load_b(breg[2], 2);
    store_b(breg[0], 0);
    __syncthreads();

    const int nround = (nsteps + kPfDepth) / (kPfDepth + 1) * (kPfDepth + 1);
    for (int s0 = 0; s0 < nround; s0 += kPfDepth + 1) {
#pragma unroll
        for (int u = 0; u <= kPfDepth; ++u) {
            const int s = s0 + u;
            {
                load_b(breg[u % 3], s + 3);  // u % 3 == s % 3: step s's set, already in LDS
                // this wave's B fragments: 4 token blocks x 3 parts
                u32x4 bf[4][3];
                const u32x4* src = bs[s & 1] + (wc * 4) * 192 + lane;
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int q = 0; q < 3; ++q) bf[c][q] = src[c * 192 + q * 64];
                u32x4 a[4];
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    uint32_t pr[4];
                    unpack_pairs(ring[u][b].x, ring[u][b].y, ring[u][b].z, pr);
                    a[b] = u32x4{pr[0], pr[1], pr[2], pr[3]};
                }
                issue_a(ring[u], s + kPfDepth + 1);
                // every fragment read is issued before the first MFMA, so the
                // LDS latency is paid once per step, not between MFMAs
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < 3; ++q)
#pragma unroll
                    for (int b = 0; b < 4; ++b)
#pragma unroll
                        for (int c = 0; c < 4; ++c) acc[b][c] = mfma(a[b], bf[c][q], acc[b][c]);
                store_b(breg[(u + 1) % 3], (s + 1) & 1);  // past the end: zeros nobody reads
                __syncthreads();
            }
        }
    }

    // epilogue: lane l holds token 16 c + l%16 and rows 4(l/16) + 0..3 of each tile
    const int q = lane >> 4, jj = lane & 15;
    // (a) rescale: v = acc 2^(sc_row - P_t), exact
    float v[4][4][4];
    int tok[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        tok[c] = (tb0 + wc * 4 + c) * 16 + jj;
        const int pt = tok[c] < T ? P[tok[c]] : 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int64_t n = (blk0 + b) * 16 + q * 4;
            const float av[4] = {acc[b][c].x, acc[b][c].y, acc[b][c].z, acc[b][c].w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                v[b][c][i] = ldexpf(av[i], scale_exp(rbase[min(n + i, (int64_t)N - 1)]) - pt);
        }
    }
    // (b) the exceptions of the wave's 64 rows (the tiles hold zeros there), in
    // list order, 8 entries at a time: x' of the lane's 4 tokens at each
    // entry's column gathered from x (fp32), the product added to the output
    // that holds the entry's row
    const int64_t rlo = blk0 * 16;
    if (rlo < N) {
        const int32_t e_lo = rp[rlo], e_hi = rp[min(rlo + 64, (int64_t)N)];
        for (int32_t e0 = e_lo; e0 < e_hi; e0 += 8) {
            int rr[8];
            float evv[8], xv[8][4];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int32_t e = min(e0 + j, e_hi - 1);
                rr[j] = (int)(er[e] - rlo);
                evv[j] = e0 + j < e_hi ? ev[e] : 0.0f;
                const int col = ec[e];
                float wl = 1.0f;
                if constexpr (LN) wl = __uint_as_float((uint32_t)lnw[col] << 16);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float* xr = x + (int64_t)min(tok[c], T - 1) * xs;
                    const float g = xr[col];
                    if constexpr (M2) xv[j][c] = silu_mul(g, xr[K + col]);
                    else xv[j][c] = LN ? g * wl : g;
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int eb = rr[j] >> 4, eq = (rr[j] & 15) >> 2, ei = rr[j] & 3;
#pragma unroll
                for (int b = 0; b < 4; ++b)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const bool hit = b == eb && i == ei && q == eq;
#pragma unroll
                        for (int c = 0; c < 4; ++c) v[b][c][i] += hit ? evv[j] * xv[j][c] : 0.0f;
                    }
            }
        }
    }
    // (c) with RMS the token's rs; store or add; rows past N and tokens past
    // T are skipped
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        if (tok[c] >= T) continue;
        if constexpr (LN) {
            const float rs = R[tok[c]];
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i) v[b][c][i] *= rs;
        }
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int64_t n = (blk0 + b) * 16 + q * 4;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (n + i >= N) continue;
                float* yp = y + (int64_t)tok[c] * N + n + i;
                *yp = add ? *yp + v[b][c][i] : v[b][c][i];
            }
        }
    }
}

int prefill_tokens_padded(int T) { return (T + kPfTokBlocks * 16 - 1) / (kPfTokBlocks * 16) * (kPfTokBlocks * 16); }

size_t prefill_ws_bytes(int K, int T) {
    const size_t tp = (size_t)prefill_tokens_padded(T);
    return tp * (size_t)K * 6 + tp * 8;
}

void launch_prefill(const rv12_matrix& w, const float* x, float* y, int T, int mode, const uint16_t* lnw, float eps,
                    void* ws, hipStream_t st) {
    const int K = w.k, N = w.n;
    const int tp = prefill_tokens_padded(T);
    u32x4* xb = reinterpret_cast<u32x4*>(ws);
    int* P = reinterpret_cast<int*>(reinterpret_cast<char*>(ws) + (size_t)tp * K * 6);
    float* R = reinterpret_cast<float*>(P + tp);
    const int xs = mode == 2 ? 2 * K : K;
    hipLaunchKernelGGL(k_prefill_x, dim3(tp / 16), dim3(kPxThreads), 0, st, x, T, K, xs, mode == 2 ? 1 : 0, lnw, eps, xb, P,
                       R);
    const int64_t nblk = ((int64_t)N + 15) / 16;
    const dim3 grid((unsigned)((nblk + kPfRowBlocks - 1) / kPfRowBlocks), (unsigned)(tp / (kPfTokBlocks * 16)));
    const auto kern = mode == 2 ? k_prefill_mm<true, false> : (lnw ? k_prefill_mm<false, true> : k_prefill_mm<false, false>);
    hipLaunchKernelGGL(kern, grid, dim3(kPfThreads), 0, st, reinterpret_cast<const uint32_t*>(w.tiles), w.rbase, xb,
                       P, w.rp, w.er, w.ec, w.ev, x, lnw, R, y, N, K, T, xs, mode == 2 ? 1 : 0, mode != 0 ? 1 : 0);
}

}  // namespace rv12
