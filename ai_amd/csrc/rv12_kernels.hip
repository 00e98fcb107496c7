// rv12 HIP kernels for gfx950: 12-bit codec encode, Q16 re-tile, bit-exact
// row decode, and the fused decode + split-K linear for 1..16 tokens.
//
// Q16 layout (written by k_retile, read by every other kernel)
// -------------------------------------------------------------
// Rows are grouped in blocks of 16, K in steps of 32.  For row block b, step s
// and lane l (0..63) one 12-byte group holds the 8 weights of row 16b + l%16 at
// k = 32s + 8(l/16) + 0..7.  The groups of one (b, s) are contiguous
// (64 x 12 = 768 bytes, one coalesced global_load_dwordx3 per wave), and the
// lane -> (row, k) map is the A-operand map of v_mfma_f32_16x16x32_bf16.
//
// Each weight is kept as a 16-bit "h" = sign << 15 | c << 7 | mantissa7 with a
// 4-bit exponent code c in bits 7..10:
//   c = code + 1       weight in the window, exponent e = code + base
//   c = 0, s, m kept   exponent 0 inside the window (zero or subnormal)
//   c = 0, s = m = 0   exception (its value is in the codec's ev list)
// As a float32, h << 16 is the weight times 2^(1 - base) for every in-window
// weight with e > 0, and exactly +0 for an exception, so a dot product can use
// the raw h values and rescale the sum once by 2^(base - 1).
// Weights 0..7 pair up as P0 = h0 | h1 << 16 ... P3 = h6 | h7 << 16.  The
// pairs never use bits 11..14 and 27..30, so three dwords carry four pairs:
//   D0 = P0 | (P3 & 0x000F000F) << 11
//   D1 = P1 | (P3 & 0x00F000F0) << 7
//   D2 = P2 | (P3 & 0x07000700) << 3 | (P3 & 0x80008000) >> 1
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rv12_internal.h"

namespace rv12 {

// ---------------------------------------------------------------- helpers
__device__ __forceinline__ void unpack_pairs(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t p[4]) {
    p[0] = d0 & 0x87FF87FFu;
    p[1] = d1 & 0x87FF87FFu;
    p[2] = d2 & 0x87FF87FFu;
    p[3] = ((d0 >> 11) & 0x000F000Fu) | ((d1 >> 7) & 0x00F000F0u) | ((d2 >> 3) & 0x07000700u) |
           ((d2 << 1) & 0x80008000u);
}

__device__ __forceinline__ float lo_f(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float hi_f(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }

// h -> original bf16 bits
__device__ __forceinline__ uint32_t h_to_bf16(uint32_t h, int base) {
    uint32_t c = (h >> 7) & 15u;
    return c ? ((h + ((uint32_t)(base - 1) << 7)) & 0xFFFFu) : h;
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// ------------------------------------------------------------------ encode
__global__ void k_zero_i32(int32_t* p, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

// exponent histogram of all N*K weights (atomic integer counts: exact)
__global__ __launch_bounds__(256) void k_hist(const uint16_t* __restrict__ w, int64_t count,
                                              int32_t* __restrict__ hist) {
    __shared__ int32_t h[256];
    h[threadIdx.x] = 0;
    __syncthreads();
    int64_t stride = (int64_t)gridDim.x * blockDim.x * 8;
    for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8; i < count; i += stride) {
        if (i + 8 <= count) {
            uint4 v = *reinterpret_cast<const uint4*>(w + i);
            uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                atomicAdd(&h[(d[j] >> 7) & 0xFF], 1);
                atomicAdd(&h[(d[j] >> 23) & 0xFF], 1);
            }
        } else {
            for (int64_t j = i; j < count; ++j) atomicAdd(&h[(w[j] >> 7) & 0xFF], 1);
        }
    }
    __syncthreads();
    if (h[threadIdx.x]) atomicAdd(&hist[threadIdx.x], h[threadIdx.x]);
}

// one workgroup per row: m8, e4 and the row's exception count
__global__ __launch_bounds__(256) void k_encode_rows(const uint16_t* __restrict__ w, int K, int CH, int base,
                                                     uint8_t* __restrict__ m8, uint8_t* __restrict__ e4,
                                                     int32_t* __restrict__ row_exc) {
    const int n = blockIdx.x;
    const uint16_t* row = w + (int64_t)n * K;
    const int half = CH / 2;
    int cnt = 0;
    for (int jb = threadIdx.x; jb < K / 2; jb += blockDim.x) {
        int c = jb / half, i = jb % half;
        int k0 = c * CH + i, k1 = k0 + half;
        uint32_t b0 = row[k0], b1 = row[k1];
        int c0 = (int)((b0 >> 7) & 0xFF) - base, c1 = (int)((b1 >> 7) & 0xFF) - base;
        if (c0 < 0 || c0 > 14) { c0 = 15; ++cnt; }
        if (c1 < 0 || c1 > 14) { c1 = 15; ++cnt; }
        m8[(int64_t)n * K + k0] = (uint8_t)(((b0 >> 15) << 7) | (b0 & 0x7F));
        m8[(int64_t)n * K + k1] = (uint8_t)(((b1 >> 15) << 7) | (b1 & 0x7F));
        e4[(int64_t)n * (K / 2) + jb] = (uint8_t)(c0 | (c1 << 4));
    }
    __shared__ int red[4];
    for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = cnt;
    __syncthreads();
    if (threadIdx.x == 0) {
        int s = 0;
        for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s += red[i];
        row_exc[n] = s;
    }
}

// one workgroup per row: exceptions in column order at rp[n]
__global__ __launch_bounds__(256) void k_encode_exc(const uint16_t* __restrict__ w, int K, int base,
                                                    const int32_t* __restrict__ rp, int32_t* __restrict__ er,
                                                    int32_t* __restrict__ ec, float* __restrict__ ev) {
    const int n = blockIdx.x;
    const int32_t start = rp[n];
    if (rp[n + 1] == start) return;  // uniform across the workgroup
    const uint16_t* row = w + (int64_t)n * K;
    const int per = (K + blockDim.x - 1) / blockDim.x;
    const int k0 = threadIdx.x * per, k1 = min(K, k0 + per);
    int cnt = 0;
    for (int k = k0; k < k1; ++k) {
        int c = (int)((row[k] >> 7) & 0xFF) - base;
        cnt += (c < 0 || c > 14);
    }
    // exclusive scan of cnt over the workgroup
    __shared__ int wsum[4];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int inc = cnt;
    for (int d = 1; d < 64; d <<= 1) {
        int v = __shfl_up(inc, d);
        if (lane >= d) inc += v;
    }
    if (lane == 63) wsum[wv] = inc;
    __syncthreads();
    int off = inc - cnt;
    for (int i = 0; i < wv; ++i) off += wsum[i];
    int pos = start + off;
    for (int k = k0; k < k1; ++k) {
        uint32_t b = row[k];
        int c = (int)((b >> 7) & 0xFF) - base;
        if (c < 0 || c > 14) {
            er[pos] = n;
            ec[pos] = k;
            ev[pos] = __uint_as_float(b << 16);
            ++pos;
        }
    }
}

// ------------------------------------------------------------------ retile
// one thread per 12-byte group (row block b, step s, lane l)
__global__ __launch_bounds__(256) void k_retile(const uint8_t* __restrict__ m8, const uint8_t* __restrict__ e4,
                                                int N, int K, int CH, int base, uint32_t* __restrict__ tiles,
                                                int64_t groups) {
    int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= groups) return;
    const int nsteps = K / 32;
    const int l = (int)(gid & 63);
    const int64_t bs = gid >> 6;
    const int s = (int)(bs % nsteps);
    const int64_t b = bs / nsteps;
    const int64_t n = b * 16 + (l & 15);
    const int k0 = s * 32 + (l >> 4) * 8;
    uint32_t h[8];
    if (n < N) {
        const int half = CH / 2;
        const int c = k0 / CH, i = k0 % CH;
        const uint8_t* mrow = m8 + n * K + k0;
        const uint8_t* erow = e4 + n * (K / 2) + (int64_t)c * half + (i % half);
        const int shift = i < half ? 0 : 4;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t m = mrow[j];
            uint32_t code = (erow[j] >> shift) & 15u;
            uint32_t sm = ((m >> 7) << 15) | (m & 0x7Fu);
            if (code == 15u) h[j] = 0u;
            else if (code + (uint32_t)base == 0u) h[j] = sm;
            else h[j] = sm | ((code + 1u) << 7);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = 0u;
    }
    uint32_t p0 = h[0] | (h[1] << 16), p1 = h[2] | (h[3] << 16), p2 = h[4] | (h[5] << 16), p3 = h[6] | (h[7] << 16);
    uint32_t* o = tiles + gid * 3;
    o[0] = p0 | ((p3 & 0x000F000Fu) << 11);
    o[1] = p1 | ((p3 & 0x00F000F0u) << 7);
    o[2] = p2 | ((p3 & 0x07000700u) << 3) | ((p3 & 0x80008000u) >> 1);
}

// ------------------------------------------------------------------ decode
// one thread per 12-byte group of the row blocks covering [first, last)
__global__ __launch_bounds__(256) void k_decode(const uint32_t* __restrict__ tiles, int K, int base, int first,
                                                int last, int64_t b0, int64_t groups, void* __restrict__ out,
                                                int out_f32) {
    int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= groups) return;
    const int nsteps = K / 32;
    const int l = (int)(gid & 63);
    const int64_t bs = gid >> 6;
    const int s = (int)(bs % nsteps);
    const int64_t b = b0 + bs / nsteps;
    const int64_t n = b * 16 + (l & 15);
    if (n < first || n >= last) return;
    const int k0 = s * 32 + (l >> 4) * 8;
    const uint32_t* t = tiles + ((b * nsteps + s) * 64 + l) * 3;
    uint32_t p[4];
    unpack_pairs(t[0], t[1], t[2], p);
    uint32_t v[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[2 * j] = h_to_bf16(p[j] & 0xFFFFu, base);
        v[2 * j + 1] = h_to_bf16(p[j] >> 16, base);
    }
    const int64_t o = (n - first) * (int64_t)K + k0;
    if (out_f32) {
        uint4* d = reinterpret_cast<uint4*>(reinterpret_cast<uint32_t*>(out) + o);
        d[0] = make_uint4(v[0] << 16, v[1] << 16, v[2] << 16, v[3] << 16);
        d[1] = make_uint4(v[4] << 16, v[5] << 16, v[6] << 16, v[7] << 16);
    } else {
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(out) + o) =
            make_uint4(v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16), v[6] | (v[7] << 16));
    }
}

// scatter the exceptions with index in [e0, e1) whose row is in [first, last)
__global__ __launch_bounds__(256) void k_decode_exc(const int32_t* __restrict__ er, const int32_t* __restrict__ ec,
                                                    const float* __restrict__ ev, int64_t e0, int64_t e1, int K,
                                                    int first, int last, void* __restrict__ out, int out_f32) {
    int64_t j = e0 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= e1) return;
    const int r = er[j];
    if (r < first || r >= last) return;
    const int64_t o = (int64_t)(r - first) * K + ec[j];
    const uint32_t bits = __float_as_uint(ev[j]);
    if (out_f32) reinterpret_cast<uint32_t*>(out)[o] = bits;
    else reinterpret_cast<uint16_t*>(out)[o] = (uint16_t)(bits >> 16);
}

// ------------------------------------------------------------------ linear
// Workgroup = `waves` waves (1..16) over 16*RB rows and the K steps
// [s_lo, s_hi) of split blockIdx.y.  Order of work, chosen so that every
// long-latency load is in flight before anything waits on it:
//   1. each wave issues the loads of its first kDepth steps of weights;
//   2. every wave fetches its 64-entry slice of the first round of the
//      workgroup's exceptions (row, column, value; a round is waves * 64
//      entries of the row-major exception list);
//   3. all threads stage x'[t][k] for the split's K range in LDS (MODE / RMS
//      transform, sum of squares for RMS), then one barrier;
//   4. main loop: wave w takes steps s_lo + w, s_lo + w + waves, ...; per step
//      it decodes 8 weights per row block and does 8 FMAs per token into fp32
//      accumulators while the load kDepth steps ahead is in flight;
//   5. epilogue: lane quarters and waves are summed in a fixed order (no
//      atomics), rescaled by 2^(base-1); the exceptions whose column lies in
//      the split are added (per wave a segmented scan over its slice, per-wave
//      LDS sums added in wave order); the result is stored (one split) or
//      written as a partial for k_splitk_reduce.
constexpr int kDepth = 8;
constexpr int kMaxThreads = 1024;

template <int RB>
__device__ __forceinline__ void load_step(uint32_t (&dst)[RB][3], const uint32_t* tb, const int64_t (&bofs)[RB],
                                          int s, int lo3) {
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        const uint32_t* g = tb + bofs[b] + (int64_t)s * 192 + lo3;
        dst[b][0] = __builtin_nontemporal_load(g);
        dst[b][1] = __builtin_nontemporal_load(g + 1);
        dst[b][2] = __builtin_nontemporal_load(g + 2);
    }
}

template <int T, int RB>
__global__ __launch_bounds__(kMaxThreads) void k_linear(LinearParams p) {
    extern __shared__ float smem[];
    const int W = blockDim.x >> 6;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, q = lane >> 4;
    const int wu = __builtin_amdgcn_readfirstlane(wave);
    const int S = gridDim.y, sp = blockIdx.y;
    const int nsteps = p.K >> 5;
    const int s_lo = (int)((int64_t)sp * nsteps / S), s_hi = (int)((int64_t)(sp + 1) * nsteps / S);
    const int k_lo = s_lo * 32, krange = (s_hi - s_lo) * 32;
    const int64_t blk0 = (int64_t)blockIdx.x * RB;
    const int n0 = (int)(blk0 * 16);

    float* xl = smem;                        // [T][krange]
    float* red = xl + T * krange;            // [W][RB][T][16]
    float* exc = red + W * RB * T * 16;      // [W][RB*16][T] per-wave exception sums
    float* ssq = exc + W * RB * 16 * T;      // [W][T]

    // ---- 1. first kDepth steps of weights
    // wave-uniform step indices (scalar branches); loads are issued
    // unconditionally at a clamped step so no load sits under a branch.
    // Row blocks past the last one (grid rounded up to RB) re-read the last
    // block; their rows are >= N and are never stored.
    const uint32_t* tb = p.tiles + (blk0 * nsteps) * 192;
    const int64_t nblk = (p.N + 15) / 16;
    int64_t bofs[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) bofs[b] = (min(blk0 + b, nblk - 1) - blk0) * (int64_t)nsteps * 192;
    const int lo3 = lane * 3;
    const int s0 = s_lo + wu;
    const int slast = s_hi - 1;
    uint32_t buf[kDepth][RB][3];
#pragma unroll
    for (int u = 0; u < kDepth; ++u) load_step<RB>(buf[u], tb, bofs, min(s0 + u * W, slast), lo3);

    // ---- 2. exception range and this wave's slice of the first round
    int32_t e_lo = 0, e_hi = 0;
    int er0 = 0x7FFFFFFF, ec0 = 0;
    float ev0 = 0.0f;
    if (p.n_exc > 0) {
        e_lo = p.rp[n0];
        e_hi = p.rp[min(n0 + RB * 16, p.N)];
        const int32_t j = e_lo + wu * 64 + lane;
        if (j < e_hi) {
            er0 = p.er[j] - n0;
            ec0 = p.ec[j];
            ev0 = p.ev[j];
        }
    }

    // ---- 3. x' into LDS
    float sq[T];
#pragma unroll
    for (int t = 0; t < T; ++t) sq[t] = 0.0f;
    for (int i = threadIdx.x * 4; i < krange; i += blockDim.x * 4) {
        const int k = k_lo + i;
        float4 lw = make_float4(1.f, 1.f, 1.f, 1.f);
        if (p.lnw) {
            uint2 b = *reinterpret_cast<const uint2*>(p.lnw + k);
            lw = make_float4(__uint_as_float(b.x << 16), __uint_as_float(b.x & 0xFFFF0000u),
                             __uint_as_float(b.y << 16), __uint_as_float(b.y & 0xFFFF0000u));
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float* xr = p.x + (int64_t)t * p.xs;
            float4 v = *reinterpret_cast<const float4*>(xr + k);
            if (p.lnw) sq[t] += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            if (p.mode == 2) {
                float4 u = *reinterpret_cast<const float4*>(xr + p.K + k);
                v = make_float4(silu_mul(v.x, u.x), silu_mul(v.y, u.y), silu_mul(v.z, u.z), silu_mul(v.w, u.w));
            }
            if (p.lnw) v = make_float4(lw.x * v.x, lw.y * v.y, lw.z * v.z, lw.w * v.w);
            *reinterpret_cast<float4*>(xl + t * krange + i) = v;
        }
    }
    for (int i = threadIdx.x; i < W * RB * 16 * T; i += blockDim.x) exc[i] = 0.0f;
    if (p.lnw) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
            float v = sq[t];
            for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
            if (lane == 0) ssq[wave * T + t] = v;
        }
    }
    __syncthreads();

    // ---- 4. main loop
    float acc[RB][T];
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[b][t] = 0.0f;

    for (int sb = s0; sb < s_hi; sb += kDepth * W) {
#pragma unroll
        for (int u = 0; u < kDepth; ++u) {
            const int s = sb + u * W;
            uint32_t cur[RB][3];
#pragma unroll
            for (int b = 0; b < RB; ++b) {
                cur[b][0] = buf[u][b][0];
                cur[b][1] = buf[u][b][1];
                cur[b][2] = buf[u][b][2];
            }
            load_step<RB>(buf[u], tb, bofs, min(s + kDepth * W, slast), lo3);
            if (s < s_hi) {
                uint32_t pr[RB][4];
#pragma unroll
                for (int b = 0; b < RB; ++b) unpack_pairs(cur[b][0], cur[b][1], cur[b][2], pr[b]);
                const float* xs = xl + (s - s_lo) * 32 + q * 8;
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    const float4 xa = *reinterpret_cast<const float4*>(xs + t * krange);
                    const float4 xb = *reinterpret_cast<const float4*>(xs + t * krange + 4);
#pragma unroll
                    for (int b = 0; b < RB; ++b) {
                        float a = acc[b][t];
                        a = fmaf(lo_f(pr[b][0]), xa.x, a);
                        a = fmaf(hi_f(pr[b][0]), xa.y, a);
                        a = fmaf(lo_f(pr[b][1]), xa.z, a);
                        a = fmaf(hi_f(pr[b][1]), xa.w, a);
                        a = fmaf(lo_f(pr[b][2]), xb.x, a);
                        a = fmaf(hi_f(pr[b][2]), xb.y, a);
                        a = fmaf(lo_f(pr[b][3]), xb.z, a);
                        a = fmaf(hi_f(pr[b][3]), xb.w, a);
                        acc[b][t] = a;
                    }
                }
            }
        }
    }

    // ---- 5. epilogue: lane quarters, then waves
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int t = 0; t < T; ++t) {
            float v = acc[b][t];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            if (lane < 16) red[((wave * RB + b) * T + t) * 16 + lane] = v;
        }

    // exceptions of this workgroup's rows with a column inside the split:
    // rounds of waves*64 entries, wave w takes entries [w*64, w*64+64) of each
    float* excw = exc + wave * RB * 16 * T;
    for (int32_t j0 = e_lo; j0 < e_hi; j0 += W * 64) {
        const int32_t j = j0 + wu * 64 + lane;
        const bool valid = j < e_hi;
        int r = 0x7FFFFFFF, c = 0;
        float v = 0.0f;
        if (j0 == e_lo) {
            r = er0;
            c = ec0;
            v = ev0;
        } else if (valid) {
            r = p.er[j] - n0;
            c = p.ec[j];
            v = p.ev[j];
        }
        if (__builtin_amdgcn_readfirstlane(j0 + wu * 64) < e_hi) {  // this wave has entries
            float pv[T];
            c -= k_lo;
            const bool in = valid && c >= 0 && c < krange;
#pragma unroll
            for (int t = 0; t < T; ++t) pv[t] = in ? v * xl[t * krange + c] : 0.0f;
            for (int d = 1; d < 64; d <<= 1) {
                const int rn = __shfl_up(r, d);
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    const float o = __shfl_up(pv[t], d);
                    if (lane >= d && rn == r) pv[t] += o;
                }
            }
            const int rnext = __shfl_down(r, 1);
            if (valid && (lane == 63 || rnext != r)) {
#pragma unroll
                for (int t = 0; t < T; ++t) excw[r * T + t] += pv[t];
            }
        }
    }
    __syncthreads();

    float rs[T];
#pragma unroll
    for (int t = 0; t < T; ++t) rs[t] = 1.0f;
    if (p.lnw && S == 1) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
            float v = 0.0f;
            for (int w = 0; w < W; ++w) v += ssq[w * T + t];
            rs[t] = 1.0f / sqrtf(v / (float)p.K + p.eps);
        }
    }
    for (int idx = threadIdx.x; idx < RB * 16 * T; idx += blockDim.x) {
        const int r = idx % (RB * 16), t = idx / (RB * 16);
        const int b = r >> 4, l16 = r & 15;
        float v = 0.0f;
        for (int w = 0; w < W; ++w) v += red[((w * RB + b) * T + t) * 16 + l16];
        float e = 0.0f;
        for (int w = 0; w < W; ++w) e += exc[(w * RB * 16 + r) * T + t];
        v = ldexpf(v, p.base - 1) + e;
        const int n = n0 + r;
        if (n < p.N) {
            if (S == 1) {
                float* y = p.y + (int64_t)t * p.N + n;
                if (p.lnw) v *= rs[t];
                *y = p.mode == 0 ? v : *y + v;
            } else {
                p.part[((int64_t)sp * T + t) * p.npad + n] = v;
            }
        }
    }
    if (S > 1 && p.lnw && blockIdx.x == 0 && threadIdx.x < T) {
        float v = 0.0f;
        for (int w = 0; w < W; ++w) v += ssq[w * T + threadIdx.x];
        p.ssq[sp * T + threadIdx.x] = v;
    }
}

// second pass of a split linear: sum the partials of each output in split order
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ part, const float* __restrict__ ssq,
                                                       float* __restrict__ y, int N, int npad, int T, int S,
                                                       int mode, int rms, float eps, int K) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)T * N) return;
    const int t = (int)(idx / N), n = (int)(idx % N);
    float v = 0.0f;
    for (int s = 0; s < S; ++s) v += part[((int64_t)s * T + t) * npad + n];
    if (rms) {
        float q = 0.0f;
        for (int s = 0; s < S; ++s) q += ssq[s * T + t];
        v *= 1.0f / sqrtf(q / (float)K + eps);
    }
    float* o = y + (int64_t)t * N + n;
    *o = mode == 0 ? v : *o + v;
}

// ------------------------------------------------------------------ launch
template <int T, int RB>
static void launch_t(const LinearParams& p, dim3 grid, int threads, size_t lds, hipStream_t st) {
    hipLaunchKernelGGL((k_linear<T, RB>), grid, dim3(threads), lds, st, p);
}

template <int RB>
static int launch_rb(const LinearParams& p, int T, dim3 grid, int threads, size_t lds, hipStream_t st) {
    switch (T) {
#define RV12_CASE(TT) \
    case TT: launch_t<TT, RB>(p, grid, threads, lds, st); return 0;
        RV12_CASE(1) RV12_CASE(2) RV12_CASE(3) RV12_CASE(4) RV12_CASE(5) RV12_CASE(6) RV12_CASE(7) RV12_CASE(8)
        RV12_CASE(9) RV12_CASE(10) RV12_CASE(11) RV12_CASE(12) RV12_CASE(13) RV12_CASE(14) RV12_CASE(15)
        RV12_CASE(16)
#undef RV12_CASE
    }
    return -1;
}

int launch_linear(const LinearParams& p, int T, int rb, int waves, int splits, hipStream_t st) {
    const int64_t nblk = (p.N + 15) / 16;
    dim3 grid((unsigned)((nblk + rb - 1) / rb), (unsigned)splits);
    const size_t lds = linear_lds_bytes(p.K, T, rb, waves, splits);
    int rc;
    switch (rb) {
        case 1: rc = launch_rb<1>(p, T, grid, waves * 64, lds, st); break;
        case 2: rc = launch_rb<2>(p, T, grid, waves * 64, lds, st); break;
        case 4: rc = launch_rb<4>(p, T, grid, waves * 64, lds, st); break;
        default: return -1;
    }
    if (rc) return rc;
    if (splits > 1) {
        const int64_t tot = (int64_t)T * p.N;
        hipLaunchKernelGGL(k_splitk_reduce, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st, p.part, p.ssq,
                           p.y, p.N, (int)(nblk * 16), T, splits, p.mode, p.lnw != nullptr, p.eps, p.K);
    }
    return 0;
}

void launch_retile(const uint8_t* m8, const uint8_t* e4, int N, int K, int CH, int base, uint32_t* tiles,
                   hipStream_t st) {
    const int64_t groups = (int64_t)((N + 15) / 16) * (K / 32) * 64;
    hipLaunchKernelGGL(k_retile, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st, m8, e4, N, K, CH, base,
                       tiles, groups);
}

void launch_decode(const rv12_matrix& w, int first, int last, void* out, int out_f32, hipStream_t st,
                   int64_t e0, int64_t e1) {
    const int64_t b0 = first / 16, b1 = (last + 15) / 16;
    const int64_t groups = (b1 - b0) * (w.k / 32) * 64;
    hipLaunchKernelGGL(k_decode, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st, w.tiles, w.k, w.base,
                       first, last, b0, groups, out, out_f32);
    if (e1 > e0)
        hipLaunchKernelGGL(k_decode_exc, dim3((unsigned)((e1 - e0 + 255) / 256)), dim3(256), 0, st, w.er, w.ec, w.ev,
                           e0, e1, w.k, first, last, out, out_f32);
}

void launch_encode_stats(const uint16_t* w, int64_t count, int32_t* hist, hipStream_t st) {
    hipLaunchKernelGGL(k_zero_i32, dim3(1), dim3(256), 0, st, hist, 256);
    int64_t blocks = (count / 8 + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(k_hist, dim3((unsigned)blocks), dim3(256), 0, st, w, count, hist);
}

void launch_encode(const uint16_t* w, int N, int K, int CH, int base, uint8_t* m8, uint8_t* e4, int32_t* row_exc,
                   hipStream_t st) {
    hipLaunchKernelGGL(k_encode_rows, dim3((unsigned)N), dim3(256), 0, st, w, K, CH, base, m8, e4, row_exc);
}

void launch_encode_exc(const uint16_t* w, int N, int K, int base, const int32_t* rp, int32_t* er, int32_t* ec,
                       float* ev, hipStream_t st) {
    hipLaunchKernelGGL(k_encode_exc, dim3((unsigned)N), dim3(256), 0, st, w, K, base, rp, er, ec, ev);
}

}  // namespace rv12
