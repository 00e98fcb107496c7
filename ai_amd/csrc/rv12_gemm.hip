// rv12 fused 12-bit decode + skinny GEMM on bf16 MFMA, 1..16 tokens (gfx950).
//
// y[t] (=|+=) W_dec . x'[t] for t < T <= 16 with W in the Q16 layout
// (rv12_device.h), whose 16 x 32 step tiles are already the A operand of
// v_mfma_f32_16x16x32_bf16: lane l holds row l%16 at k = 8(l/16) + 0..7, and
// the four h-pairs of a 12-byte group are those 8 bf16 values (the weights
// times 2^-sc; MFMA keeps subnormal inputs and products).
//
// The activations keep float32 accuracy the way the reference's bf16 tensor
// path does (ramvi/engine/ramvi_engine/kernels/wcomp.py:130-140): x' is split
// into three bf16 parts hi + mid + lo (hi = bf16(x'), mid = bf16(x' - hi),
// lo = bf16(x' - hi - mid); the sum carries 24 mantissa bits) and each weight
// tile meets each part in its own MFMA, accumulated in float32.
//
// Workgroup = W waves over the K steps [s_lo, s_hi) of split blockIdx.y and
// W * RBW row blocks; wave w owns row blocks w*RBW .. w*RBW + RBW - 1.
//   1. every thread loads the activations of its B-operand groups (one group
//      = one step x one lane: token l%16, k = 8(l/16) + 0..7);
//   2. each wave issues the loads of its first D weight steps (buffer loads;
//      a step past the split's end takes an offset past the descriptor's
//      range, which returns zeros without a memory access);
//   3. x' is formed (MODE / RMS transform), scaled by 2^64 and split into
//      hi/mid/lo, and written to LDS in B-operand lane order (tokens >= T are
//      zeros); barrier.  The scale lifts the products of the Q16 values
//      (h << 16 is below 2^-111) with x' out of the float32 subnormal range
//      that an unscaled x' of moderate size would put them in; where some
//      nonzero |x'| of the split lies outside [2^-64, 2^63) (found by a ballot
//      and an LDS flag per wave), the parts are staged again with x' * 2^P,
//      P = 100 - the exponent of the split's largest |x'| per token;
//   4. main loop: per step each of the wave's row blocks is unpacked once,
//      the load D steps ahead is issued into the same registers (D loads stay
//      in flight across the rounds), three ds_read_b128 fetch the B parts and
//      each row block meets the three parts in three MFMAs into three
//      independent accumulators;
//   5. epilogue per wave: the exceptions of the wave's rows whose column is
//      inside the split are added per (row, token) in list order (the entries
//      found by a ballot, one at a time), x' taken from the LDS parts times
//      2^-P; the sum of the three accumulators is rescaled by 2^(sc - P), the
//      exception sums added, and stored (one split) or written as a partial
//      for k_splitk_reduce.
//      The exception range, the row windows and the old y are loaded right
//      after the weight prefetch, the first 64 exception entries right after
//      the x' staging, so the epilogue waits for no memory in the common case.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rv12_device.h"
#include "rv12_internal.h"

namespace rv12 {


constexpr int kGroupsPerThread = 4;  // B-operand groups a thread loads before the weight prefetch

// an offset past any weight descriptor (<= 2^31 - 1 bytes), which
// wraps no 32-bit sum with a row-block offset
constexpr uint32_t kPastEnd = 0x80000000u;

template <int RBW>
__device__ __forceinline__ void issue_rows(u32x3 (&dst)[RBW], __amdgpu_buffer_rsrc_t rv, const int (&voff)[RBW], int s,
                                           int s_hi) {
    // a step past the end takes an offset beyond every descriptor's range
    // (the range check covers the vector offset, not the scalar one)
    const uint32_t off = s < s_hi ? (uint32_t)s * kStepBytes : kPastEnd;
#pragma unroll
    for (int b = 0; b < RBW; ++b) dst[b] = load_group(rv, (int)((uint32_t)voff[b] + off), 0);
}


// TP: the token columns staged, 4, 8 or 16 (T <= TP); G = 4 TP B-operand
// groups per K step (4 k-groups of 8 x TP tokens).  M2: silu(g) * u prologue
// (MODE 2); LN: RMSNorm weight.  Template arguments, so that the activation
// loads of step 1 are straight-line code that waits for no kernel argument
// test, and the group arithmetic is shifts.
// KS: the waves split the workgroup's K steps instead of its rows: the
// workgroup covers RBW row blocks, wave w takes steps s_lo + w + W i of all of
// them, the waves' sums are joined through LDS in a fixed order and wave b
// < RBW finishes row block b (exceptions, scale, store).  One workgroup then
// needs no K split for as many rows as the LDS holds x' for: at 4 token
// columns (768 B per K step) K up to ~6000, so the split's reduce launch goes.
template <int TP, int RBW, bool M2, bool LN, bool KS>
__global__ __launch_bounds__(kGemmMaxWaves * 64) void k_gemm(LinearParams p, int T) {
    constexpr int G = 4 * TP;
    constexpr int ORB = KS ? 1 : RBW;  // row blocks of this wave's outputs
    extern __shared__ u32x4 lds4[];
    const int W = blockDim.x >> 6;
    const int nthr = blockDim.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wu = __builtin_amdgcn_readfirstlane(wave);
    const int S = gridDim.y, sp = blockIdx.y;
    // the workgroup size, the split count and the exception count in SGPRs
    // now: their loads then join the other kernel arguments' and are waited
    // for with them, not after the first global loads
    asm volatile("" : : "s"(nthr), "s"(S), "s"(p.n_exc));
    const int nsteps = p.K >> 5;
    // split bounds in 32 bits: nsteps <= 2^15 and S <= 64
    int s_lo = 0, s_hi = nsteps;
    if (S > 1) {
        s_lo = (int)((uint32_t)(sp * nsteps) / (uint32_t)S);
        s_hi = (int)((uint32_t)((sp + 1) * nsteps) / (uint32_t)S);
    }
    const int nst = s_hi - s_lo, k_lo = s_lo * 32, krange = nst * 32;
    const int ngr = nst * G;  // B-operand groups of the split
    const int64_t nblk = (p.N + 15) / 16;
    const int64_t blk0 = (int64_t)blockIdx.x * (KS ? 1 : W) * RBW;
    const int n0 = (int)(blk0 * 16);
    const int64_t wblk = KS ? blk0 : blk0 + wu * RBW;  // first row block whose weights this wave loads
    const int nvalid = (int)max((int64_t)0, min((int64_t)RBW, nblk - wblk));
    const int64_t oblk = KS ? blk0 + wu : wblk;  // first row block of this wave's outputs
    const int nw = (int)(oblk * 16);             // first output row of this wave
    const int onvalid = KS ? (wu < RBW && oblk < nblk ? 1 : 0) : nvalid;

    u32x4* xb = lds4;                                                  // [nst][3][G]
    float* exc = reinterpret_cast<float*>(xb + (size_t)nst * 3 * G);  // [W*ORB*16 rows][16 tokens]
    f32x4* red = reinterpret_cast<f32x4*>(exc + W * ORB * 256);       // KS: [W][RBW][64] the waves' sums
    float* ssq = reinterpret_cast<float*>(red + (KS ? W * RBW * 64 : 0));  // [W][16]
    int* wflag = reinterpret_cast<int*>(ssq + W * 16);                 // [W] x' outside the fast path's range
    int* wexp = wflag + W;                                             // [W][16] slow path: largest exponent

    // ---- 1. activations of this thread's B groups g = threadIdx.x + i nthr
    // (step g / G, k-group (g % G) / TP, token g % TP), as straight-line
    // loads: a group past the split reads column k_lo again and a token past
    // T reads token T - 1 (both unused), so no load waits for a branch.
    // Every group of a thread has the same token (nthr is a multiple of TP).
    f32x4 xa[kGroupsPerThread][2], ua[kGroupsPerThread][2];
    u32x4 la[kGroupsPerThread];
    const int tg = threadIdx.x % TP;  // token of this thread's groups
    const bool tgok = tg < T;
    const float* xrow = p.x + (int64_t)min(tg, T - 1) * p.xs;
    auto gcol = [&](int g) { return k_lo + (g < ngr ? (g / G) * 32 + ((g % G) / TP) * 8 : 0); };
#pragma unroll
    for (int i = 0; i < kGroupsPerThread; ++i) {
        const int k = gcol(threadIdx.x + i * nthr);
        xa[i][0] = *reinterpret_cast<const f32x4*>(xrow + k);
        xa[i][1] = *reinterpret_cast<const f32x4*>(xrow + k + 4);
        if constexpr (M2) {
            ua[i][0] = *reinterpret_cast<const f32x4*>(xrow + p.K + k);
            ua[i][1] = *reinterpret_cast<const f32x4*>(xrow + p.K + k + 4);
        }
        if constexpr (LN) la[i] = *reinterpret_cast<const u32x4*>(p.lnw + k);
    }
    // every wave's activation loads enter the memory pipeline before any
    // weight load (a bare barrier: it orders the issue, it waits for no data)
    __builtin_amdgcn_s_barrier();

    // ---- 2. first D weight steps of this wave's row blocks.  D per row
    // blocks of a wave, measured on the Qwen3-14B shapes at 4-16 tokens: 2 row
    // blocks (qkv, o) 4 (qkv M4 17.2 us at 8, 15.8 at 4), one 6, four 3
    constexpr int D = RBW >= 4 ? 3 : (RBW == 2 ? 4 : 6);
    const uint32_t blk_bytes = (uint32_t)nsteps * kStepBytes;
    const char* wbase = reinterpret_cast<const char*>(p.tiles) + wblk * (int64_t)blk_bytes;
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(wbase, (uint32_t)nvalid * blk_bytes);
    int voff[RBW];
#pragma unroll
    for (int b = 0; b < RBW; ++b) voff[b] = (int)(b * blk_bytes) + lane * 12;
    u32x3 buf[D][RBW];
    const int s0 = s_lo + (KS ? wu : 0);  // this wave's first step
    const int stride = KS ? W : 1;        // steps between this wave's consecutive steps
#pragma unroll
    for (int u = 0; u < D; ++u) issue_rows<RBW>(buf[u], rv, voff, s0 + u * stride, s_hi);

    // what the epilogue reads, loaded now so that it arrives during the main
    // loop: the wave's exception range (its first 64 entries are loaded after
    // the x' staging below, so that the wait for these row pointers does not
    // hold up the staging), and per output the row window and, for an
    // accumulating single split, the old y (rows and tokens clamped into
    // range: no branch).  Outputs are in the MFMA result layout: lane l holds
    // token jj = l % 16 and rows 4 (l / 16) + 0..3 of each row block.
    const int q = lane >> 4;
    const int jj = lane & 15;  // token of this lane's outputs
    const bool tok = jj < T;
    const int32_t e_lo = p.rp[min(nw, p.N)], e_hi = p.rp[min(nw + ORB * 16, p.N)];
    // Per row block, lane l's four rows 4(l/16) + 0..3 are consecutive: one
    // 16-byte load of their windows and (one split, accumulating) of their
    // old y.  With N % 4 == 0 each such group lies wholly inside or wholly
    // past the rows, and the descriptors (over rbase and y) read zeros past
    // the end; with N % 4 != 0 the epilogue reads them one by one instead.
    // y is loaded whatever the mode, so every load here is straight-line and
    // the waits of the staging below count exactly; with four row blocks per
    // wave y is read in the epilogue (registers).
    constexpr bool kPreY = ORB <= 2;
    const bool vec = (p.N & 3) == 0;
    const __amdgpu_buffer_rsrc_t r_rb = make_rsrc(p.rbase, (uint32_t)p.N * 4u);
    const __amdgpu_buffer_rsrc_t r_y = make_rsrc(p.y, (uint32_t)((int64_t)T * p.N * 4));
    u32x4 obase[ORB];
    f32x4 oy[ORB];
#pragma unroll
    for (int b = 0; b < ORB; ++b) {
        const int nb = nw + b * 16 + q * 4;
        obase[b] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r_rb, nb * 4, 0, 0));
        if constexpr (kPreY)
            oy[b] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r_y, (min(jj, T - 1) * p.N + nb) * 4, 0, 0));
    }

    // ---- 3. x' * 2^64 split into bf16 parts, in B-operand order (group g at
    // xb[(g / G) 3 G + g % G], parts G apart; tokens past T are zeros); the
    // exponent range of x' is tracked for the fast path's check
    float sq = 0.0f;
    int elo = 0, ehi = 0;
    auto stage = [&](int g, f32x4 x0, f32x4 x1, f32x4 u0, f32x4 u1, u32x4 lw4) {
        u32x4 hi = {0, 0, 0, 0}, mid = {0, 0, 0, 0}, lo = {0, 0, 0, 0};
        if (tgok) {
            float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            if constexpr (LN) {
#pragma unroll
                for (int e = 0; e < 8; ++e) sq += (v[e] * kSsqScale) * (v[e] * kSsqScale);
            }
            if constexpr (M2) {
                const float u[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = silu_mul(v[e], u[e]);
            }
            if constexpr (LN) {
                const uint32_t lw[4] = {lw4.x, lw4.y, lw4.z, lw4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[2 * e] *= __uint_as_float(lw[e] << 16);
                    v[2 * e + 1] *= __uint_as_float(lw[e] & 0xFFFF0000u);
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                track_exp(v[e], elo, ehi);
                v[e] *= kXScale;
            }
            split3(v, hi, mid, lo);
        }
        u32x4* d = xb + (size_t)(g / G) * 3 * G + (g % G);
        d[0] = hi;
        d[G] = mid;
        d[2 * G] = lo;
    };
#pragma unroll
    for (int i = 0; i < kGroupsPerThread; ++i) {
        const int g = threadIdx.x + i * nthr;
        if (g < ngr) stage(g, xa[i][0], xa[i][1], ua[i][0], ua[i][1], la[i]);
    }
    // groups beyond the register-staged ones (long splits at few tokens):
    // loaded here, after the weight prefetch
    for (int g = threadIdx.x + kGroupsPerThread * nthr; g < ngr; g += nthr) {
        const int k = gcol(g);
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(xrow + k), x1 = *reinterpret_cast<const f32x4*>(xrow + k + 4);
        f32x4 u0 = x0, u1 = x1;
        if constexpr (M2) {
            u0 = *reinterpret_cast<const f32x4*>(xrow + p.K + k);
            u1 = *reinterpret_cast<const f32x4*>(xrow + p.K + k + 4);
        }
        u32x4 lw4 = {0, 0, 0, 0};
        if constexpr (LN) lw4 = *reinterpret_cast<const u32x4*>(p.lnw + k);
        stage(g, x0, x1, u0, u1, lw4);
    }
    if constexpr (LN) {
        // lanes tg, tg + TP, ... of the wave hold token tg
#pragma unroll
        for (int o = TP; o < 64; o <<= 1) sq += __shfl_xor(sq, o);
        if (lane < TP) ssq[wave * 16 + lane] = sq;
    }
    {
        const bool bad = elo < kXRangeLo || ehi > kXRangeHi;
        const uint64_t bm = __ballot(bad);
        if (lane == 0) wflag[wave] = bm != 0;
    }
    // this wave's exception sums start at zero
    float* excw = exc + wu * ORB * 256;
#pragma unroll
    for (int i = 0; i < ORB * 4; ++i) excw[i * 64 + lane] = 0.0f;
    // the wave's first 64 exception entries (a descriptor over the list reads
    // zeros past its end)
    const uint32_t exc_bytes = (uint32_t)min(p.n_exc, (int64_t)(1 << 28)) * 4u;
    const __amdgpu_buffer_rsrc_t r_er = make_rsrc(p.er, exc_bytes), r_ec = make_rsrc(p.ec, exc_bytes),
                                 r_ev = make_rsrc(p.ev, exc_bytes);
    const uint32_t e_off = e_lo + lane < e_hi ? (uint32_t)(e_lo + lane) * 4u : 0xFFFFFFF0u;
    const int er0 = (int)__builtin_amdgcn_raw_buffer_load_b32(r_er, (int)e_off, 0, 0);
    const int ec0 = (int)__builtin_amdgcn_raw_buffer_load_b32(r_ec, (int)e_off, 0, 0);
    const float ev0 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r_ev, (int)e_off, 0, 0));
    __syncthreads();

    // ---- 3b. (rare) some nonzero |x'| of the split outside [2^-64, 2^63):
    // per-token scale exponents P from the largest |x'| of the split, and the
    // parts staged again from the inputs with x' * 2^P.  Pj is the exponent of
    // token jj (this lane's outputs and exception sums), Pg that of token tg
    // (this thread's staged groups).
    int Pj = kXScaleExp;
    // the W flags in one LDS read, lane w reading wave w's
    if (__ballot(lane < W && wflag[lane] != 0) != 0) {
        auto xprime = [&](int k, float (&v)[8]) {
            const f32x4 a0 = *reinterpret_cast<const f32x4*>(xrow + k);
            const f32x4 a1 = *reinterpret_cast<const f32x4*>(xrow + k + 4);
            v[0] = a0.x, v[1] = a0.y, v[2] = a0.z, v[3] = a0.w, v[4] = a1.x, v[5] = a1.y, v[6] = a1.z, v[7] = a1.w;
            if constexpr (M2) {
                const f32x4 u0 = *reinterpret_cast<const f32x4*>(xrow + p.K + k);
                const f32x4 u1 = *reinterpret_cast<const f32x4*>(xrow + p.K + k + 4);
                const float u[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = silu_mul(v[e], u[e]);
            }
            if constexpr (LN) {
                const u32x4 l = *reinterpret_cast<const u32x4*>(p.lnw + k);
                const uint32_t lw[4] = {l.x, l.y, l.z, l.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[2 * e] *= __uint_as_float(lw[e] << 16);
                    v[2 * e + 1] *= __uint_as_float(lw[e] & 0xFFFF0000u);
                }
            }
        };
        int em = -1000;
        if (tgok) {
            for (int g = threadIdx.x; g < ngr; g += nthr) {
                float v[8];
                xprime(gcol(g), v);
#pragma unroll
                for (int e = 0; e < 8; ++e) em = max(em, exp_or_min(v[e]));
            }
        }
        // lanes tg, tg + TP, ... hold token tg
#pragma unroll
        for (int o = TP; o < 64; o <<= 1) em = max(em, __shfl_xor(em, o));
        if (lane < TP) wexp[wave * 16 + lane] = em;
        __syncthreads();
        int eg = -1000, ej = -1000;
        for (int w = 0; w < W; ++w) {
            eg = max(eg, wexp[w * 16 + tg]);
            ej = max(ej, wexp[w * 16 + min(jj, TP - 1)]);
        }
        const int Pg = slow_scale_exp(eg);
        Pj = slow_scale_exp(ej);
        if (tgok) {
            for (int g = threadIdx.x; g < ngr; g += nthr) {
                float v[8];
                xprime(gcol(g), v);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = ldexpf(v[e], Pg);
                u32x4 hi, mid, lo;
                split3(v, hi, mid, lo);
                u32x4* d = xb + (size_t)(g / G) * 3 * G + (g % G);
                d[0] = hi;
                d[G] = mid;
                d[2 * G] = lo;
            }
        }
        __syncthreads();
    }

    // ---- 4. main loop: lane l reads the B group of token l % 16 and k-group
    // l / 16; lanes of tokens >= TP take zeros without an LDS read
    const int bl = jj < TP ? q * TP + jj : -1;
    f32x4 acc[RBW][3];
#pragma unroll
    for (int b = 0; b < RBW; ++b)
#pragma unroll
        for (int c = 0; c < 3; ++c) acc[b][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // rounds of D of this wave's steps s0, s0 + stride, ...; a wave stops
    // after its last step (the steps after it are all past s_hi)
    for (int sb = s0; sb < s_hi; sb += D * stride) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            const int s = sb + u * stride;
            const int sr = s - s_lo;  // step within the split
            // the step's words are unpacked before the load D steps ahead
            // reuses their registers: no copy of the loaded registers at the
            // loop's back edge, so no wait there for the loads in flight
            u32x4 a[RBW];
#pragma unroll
            for (int b = 0; b < RBW; ++b) {
                uint32_t pr[4];
                unpack_pairs(buf[u][b].x, buf[u][b].y, buf[u][b].z, pr);
                a[b] = u32x4{pr[0], pr[1], pr[2], pr[3]};
                // (kept ahead of the load by the compiler's scheduler)
                asm volatile("" : "+v"(a[b])::"memory");
            }
            issue_rows<RBW>(buf[u], rv, voff, s + D * stride, s_hi);
            if (s < s_hi) {
                u32x4 b0 = {0, 0, 0, 0}, b1 = {0, 0, 0, 0}, b2 = {0, 0, 0, 0};
                if (TP == 16 || bl >= 0) {
                    const u32x4* bsrc = xb + (size_t)sr * 3 * G + bl;
                    b0 = bsrc[0];
                    b1 = bsrc[G];
                    b2 = bsrc[2 * G];
                }
#pragma unroll
                for (int b = 0; b < RBW; ++b) {
                    acc[b][0] = mfma(a[b], b0, acc[b][0]);
                    acc[b][1] = mfma(a[b], b1, acc[b][1]);
                    acc[b][2] = mfma(a[b], b2, acc[b][2]);
                }
            }
        }
    }

    // ---- 4b. this wave's output sums: KS joins the waves' sums through LDS
    // in wave order, wave b < RBW taking row block b
    f32x4 osum[ORB];
    if constexpr (KS) {
#pragma unroll
        for (int b = 0; b < RBW; ++b) red[(wu * RBW + b) * 64 + lane] = acc[b][0] + acc[b][1] + acc[b][2];
        __syncthreads();
        osum[0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (wu < RBW)
            for (int w = 0; w < W; ++w) osum[0] += red[(w * RBW + wu) * 64 + lane];
    } else {
#pragma unroll
        for (int b = 0; b < ORB; ++b) osum[b] = acc[b][0] + acc[b][1] + acc[b][2];
    }

    // ---- 5. exceptions of this wave's output rows, columns inside the split
    const uint8_t* xbytes = reinterpret_cast<const uint8_t*>(xb);
    if (onvalid > 0) {
        for (int32_t j0 = e_lo; j0 < e_hi; j0 += 64) {
            const int32_t j = j0 + lane;
            const bool valid = j < e_hi;
            int r = 0x7FFFFFFF, c = -1;
            float v = 0.0f;
            if (j0 == e_lo) {  // the first 64 entries were loaded at the start
                if (valid) {
                    r = er0 - nw;
                    c = ec0 - k_lo;
                    v = ev0;
                }
            } else if (valid) {  // rare: more than 64 exceptions in the wave's rows
                r = p.er[j] - nw;
                c = p.ec[j] - k_lo;
                v = p.ev[j];
            }
            const bool in = valid && c >= 0 && c < krange;
            // the entries inside the split, in list order (so each output adds
            // its products in a fixed order): row, column and value made
            // wave-uniform, lanes t < T add ev * x'(t, c) for their token
            uint64_t m = __ballot(in);
            while (m) {
                const int src = __builtin_ctzll(m);
                m &= m - 1;
                const int rr = __builtin_amdgcn_readlane(r, src), cc = __builtin_amdgcn_readlane(c, src);
                const float vv = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), src));
                if (lane < T) {
                    // byte offset of x'(token lane, cc) in part 0: step cc/32,
                    // group ((cc%32)/8) TP + token, element cc%8; parts G 16
                    // bytes apart
                    const int o = ((cc >> 5) * 3 * G + ((cc & 31) >> 3) * TP + lane) * 16 + (cc & 7) * 2;
                    const float xv = bf16_value(*reinterpret_cast<const uint16_t*>(xbytes + o)) +
                                     bf16_value(*reinterpret_cast<const uint16_t*>(xbytes + o + G * 16)) +
                                     bf16_value(*reinterpret_cast<const uint16_t*>(xbytes + o + 2 * G * 16));
                    excw[rr * 16 + lane] += vv * ldexpf(xv, -Pj);
                }
            }
        }
    }

    // ---- 6. outputs: lane l holds token l%16 and rows 4(l/16) + 0..3 of each
    // row block, four consecutive outputs of one token: one 16-byte store
    // where all four rows exist and the token rows of y are 16-byte aligned
    float rs = 1.0f;
    if (LN && S == 1 && tok) {
        float v = 0.0f;
        for (int w = 0; w < W; ++w) v += ssq[w * 16 + jj];
        rs = rms_scale(v, p.K, p.eps);
    }
#pragma unroll
    for (int b = 0; b < ORB; ++b) {
        if (b >= onvalid) break;
        const f32x4 a = osum[b];
        const float av[4] = {a.x, a.y, a.z, a.w};
        const int nb = nw + b * 16 + q * 4;
        int ob[4] = {(int)obase[b].x, (int)obase[b].y, (int)obase[b].z, (int)obase[b].w};
        if (!vec) {
#pragma unroll
            for (int i = 0; i < 4; ++i) ob[i] = p.rbase[min(nb + i, p.N - 1)];
        }
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = ldexpf(av[i], scale_exp(ob[i]) - Pj) + excw[(b * 16 + q * 4 + i) * 16 + jj];
        if (!tok) continue;
        if (S == 1) {
            if constexpr (LN) {
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] *= rs;
            }
            float* yp = p.y + (int64_t)jj * p.N + nb;
            if (vec && nb < p.N) {
                f32x4 o = {v[0], v[1], v[2], v[3]};
                if (p.mode != 0) o = (kPreY ? oy[b] : *reinterpret_cast<const f32x4*>(yp)) + o;
                *reinterpret_cast<f32x4*>(yp) = o;
            } else if (!vec) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (nb + i < p.N) yp[i] = p.mode == 0 ? v[i] : yp[i] + v[i];
            }
        } else {  // partial rows run to npad, a multiple of 16: always four
            *reinterpret_cast<f32x4*>(p.part + ((int64_t)sp * T + jj) * p.npad + nb) = f32x4{v[0], v[1], v[2], v[3]};
        }
    }
    if (LN && S > 1 && blockIdx.x == 0 && threadIdx.x < T) {
        float v = 0.0f;
        for (int w = 0; w < W; ++w) v += ssq[w * 16 + threadIdx.x];
        p.ssq[sp * T + threadIdx.x] = v;
    }
    (void)n0;
}

template <int TP, int RBW, bool M2, bool LN, bool KS>
static void launch_t(const LinearParams& p, int T, dim3 grid, int threads, size_t lds, hipStream_t st) {
    if (lds > kDefaultLds)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm<TP, RBW, M2, LN, KS>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL((k_gemm<TP, RBW, M2, LN, KS>), grid, dim3(threads), lds, st, p, T);
}

template <int TP, int RBW, bool KS>
static void launch_r(const LinearParams& p, int T, dim3 grid, int threads, size_t lds, hipStream_t st) {
    const bool m2 = p.mode == 2, ln = p.lnw != nullptr;
    if (m2 && ln) launch_t<TP, RBW, true, true, KS>(p, T, grid, threads, lds, st);
    else if (m2) launch_t<TP, RBW, true, false, KS>(p, T, grid, threads, lds, st);
    else if (ln) launch_t<TP, RBW, false, true, KS>(p, T, grid, threads, lds, st);
    else launch_t<TP, RBW, false, false, KS>(p, T, grid, threads, lds, st);
}

template <int TP, bool KS>
static int launch_tp(const LinearParams& p, int T, int rbw, dim3 grid, int threads, size_t lds, hipStream_t st) {
    switch (rbw) {
        case 1: launch_r<TP, 1, KS>(p, T, grid, threads, lds, st); return 0;
        case 2: launch_r<TP, 2, KS>(p, T, grid, threads, lds, st); return 0;
        case 4: launch_r<TP, 4, KS>(p, T, grid, threads, lds, st); return 0;
    }
    return -1;
}

// ks: the waves split K (kernel 3): rbw row blocks per workgroup, waves >= rbw
int launch_gemm(const LinearParams& p, int T, int rbw, int waves, int splits, bool ks, hipStream_t st) {
    const int64_t nblk = (p.N + 15) / 16;
    const int64_t per_wg = (int64_t)rbw * (ks ? 1 : waves);
    dim3 grid((unsigned)((nblk + per_wg - 1) / per_wg), (unsigned)splits);
    const int tp = gemm_tokens(T);
    const size_t lds = ks ? gemm_ks_lds_bytes(p.K, rbw, waves, splits, T) : gemm_lds_bytes(p.K, rbw, waves, splits, T);
    if (ks && waves < rbw) return -1;
    int rc;
    switch (tp * 2 + (ks ? 1 : 0)) {
        case 8: rc = launch_tp<4, false>(p, T, rbw, grid, waves * 64, lds, st); break;
        case 9: rc = launch_tp<4, true>(p, T, rbw, grid, waves * 64, lds, st); break;
        case 16: rc = launch_tp<8, false>(p, T, rbw, grid, waves * 64, lds, st); break;
        case 17: rc = launch_tp<8, true>(p, T, rbw, grid, waves * 64, lds, st); break;
        case 32: rc = launch_tp<16, false>(p, T, rbw, grid, waves * 64, lds, st); break;
        case 33: rc = launch_tp<16, true>(p, T, rbw, grid, waves * 64, lds, st); break;
        default: return -1;
    }
    if (rc) return rc;
    if (splits > 1) launch_splitk_reduce(p, T, splits, st);
    return 0;
}

}  // namespace rv12
