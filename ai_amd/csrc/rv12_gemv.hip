// rv12 fused 12-bit decode + linear on the vector ALUs, 1..4 tokens (gfx950).
//
// y[t] (=|+=) W_dec . x'[t] with W in the Q16 layout (rv12_device.h).
//
// Workgroup = W waves over 16*RB rows (RB row blocks) and the K steps
// [s_lo, s_hi) of split blockIdx.y.  Wave w takes the steps s_lo + w + W*i.
// Order of work, so that every long-latency load is in flight before
// anything waits on it:
//   1. every thread loads its share of the activations (x, and u in mode 2,
//      and the RMSNorm weight) for the split's K range, as straight-line code
//      (the prologue variants are template arguments); a bare barrier puts
//      every wave's activation loads ahead of the weight loads;
//   2. each wave issues the loads of its first D weight steps (buffer
//      loads; a step past the split's end takes an offset past the
//      descriptor's range, which returns zeros without a memory access);
//   3. the activation loads are waited for (the weight loads stay in flight)
//      and x' * 2^64 is written to LDS: the MODE / RMS transform, the sum of
//      squares for RMS and the exponent range of x'; one barrier; if any
//      nonzero |x'| lies outside [2^-64, 2^63), x' is staged again with a
//      per-token scale (the activation scaling of rv12_device.h);
//   4. main loop: per step each wave unpacks its 12-byte words, issues the
//      load D steps ahead into the same registers (D: the prefetch depth
//      chosen per variant below) and does 8 FMAs per token and row block into
//      fp32 accumulators; D loads stay in flight across the rounds;
//   5. epilogue: one thread per output sums the lane quarters and waves in a
//      fixed order (no atomics), rescales by 2^(sc - P) of its row, adds the
//      products ev * x' of its row's exceptions whose column lies in the split
//      (staged per round in LDS, added in list order), and stores the result
//      (one split) or writes it as a partial for k_splitk_reduce.  The row's
//      scale, exception range and old y are loaded at the very start, so the
//      epilogue issues no global load.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rv12_device.h"
#include "rv12_internal.h"

namespace rv12 {

// an offset past any weight descriptor (<= 2^31 - 1 bytes), which
// wraps no 32-bit sum with a row-block offset
constexpr uint32_t kPastEnd = 0x80000000u;

template <int RB>
__device__ __forceinline__ void issue_step(u32x3 (&dst)[RB], __amdgpu_buffer_rsrc_t rv, const int (&voff)[RB], int s,
                                           int s_hi) {
    // a step past the end takes an offset beyond every descriptor's range
    // (the range check covers the vector offset, not the scalar one)
    const uint32_t off = s < s_hi ? (uint32_t)s * kStepBytes : kPastEnd;
#pragma unroll
    for (int b = 0; b < RB; ++b) dst[b] = load_group(rv, (int)((uint32_t)voff[b] + off), 0);
}

// NXM = float4 chunks of activations per thread loaded in step 1, before the
// weight prefetch; columns beyond 4 * NXM * blockDim.x are staged after it.
// M2: silu(g) * u prologue (MODE 2); LN: RMSNorm weight.  Both are template
// arguments so that the loads of step 1 are straight-line code, issued without
// waiting for any kernel argument test.  SH: the shallow prefetch (4 steps).
// The host guarantees blockDim.x >= 16 * RB * T (one thread per output).
template <int T, int RB, bool M2, bool LN, bool SH>
__global__ __launch_bounds__(gemv_max_waves(RB) * 64) void k_gemv(LinearParams p) {
    constexpr int NXM = gemv_chunks(T);
    constexpr int NO = RB * 16 * T;  // outputs of the workgroup
    // weight steps in flight per wave
    constexpr int D = gemv_depth(T, RB, M2, LN, SH);
    extern __shared__ float smem[];
    const int W = blockDim.x >> 6;
    const int nthr = blockDim.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, q = lane >> 4;
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
    const int k_lo = s_lo * 32, krange = (s_hi - s_lo) * 32;
    const int64_t blk0 = (int64_t)blockIdx.x * RB;
    const int n0 = (int)(blk0 * 16);
    const int nvalid = min(RB, (int)(((uint32_t)p.N + 15u) >> 4) - (int)blockIdx.x * RB);

    float* xl = smem;                    // [T][krange]  x' * 2^P[t]
    float* red = xl + T * krange;        // [W][RB][T][16]
    float* excv = red + W * RB * T * 16; // [nthr][T] exception products of one round
    float* ssq = excv + nthr * T;        // [W][T]
    int* wflag = reinterpret_cast<int*>(ssq + W * T);  // [W] x' outside the fast path's range
    int* wexp = wflag + W;                               // [W][T] slow path: largest exponent

    // ---- 0. what the epilogue needs, loaded first: thread i < NO owns output
    // (row n0 + i % (16 RB), token i / (16 RB)): its row's scale exponent and
    // exception range, and y for an accumulating single-split launch.  Every
    // thread loads (row and token clamped into range, so the loads need no
    // branch); only the owners' values are used, in the epilogue.
    const bool owner = threadIdx.x < NO;
    const int orow = threadIdx.x % (RB * 16), otok = threadIdx.x / (RB * 16);
    const int on = n0 + orow;
    const bool oval = owner && on < p.N;
    const int onc = min(on, p.N - 1);
    const int obase = p.rbase[onc];  // raw: the scale exponent is formed in the epilogue
    const int32_t oe0 = p.rp[onc], oe1 = p.rp[onc + 1];
    const float oy = p.y[(int64_t)min(otok, T - 1) * p.N + onc];

    // ---- 1. activations of this thread: the chunks j with 4 j nthr < krange
    // hold the split's columns (lanes past its end load its last 4 columns
    // again, unused)
    f32x4 xr[NXM][T], ur[NXM][T];
    uint2 lr[NXM];
#pragma unroll
    for (int j = 0; j < NXM; ++j) {
        if (j * 4 * nthr < krange) {
            const int i = (threadIdx.x + j * nthr) * 4;
            const uint32_t k = (uint32_t)(k_lo + min(i, krange - 4));
            if constexpr (LN) lr[j] = *reinterpret_cast<const uint2*>(p.lnw + k);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const float* xt = p.x + (int64_t)t * p.xs;
                xr[j][t] = *reinterpret_cast<const f32x4*>(xt + k);
                if constexpr (M2) ur[j][t] = *reinterpret_cast<const f32x4*>(xt + p.K + k);
            }
        }
    }
    // every wave's activation loads enter the memory pipeline before any
    // weight load (a bare barrier: it orders the issue, it waits for no data)
    __builtin_amdgcn_s_barrier();

    // ---- 2. first D weight steps of this wave
    const uint32_t blk_bytes = (uint32_t)nsteps * kStepBytes;
    const char* wbase = reinterpret_cast<const char*>(p.tiles) + blk0 * (int64_t)blk_bytes;
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(wbase, (uint32_t)nvalid * blk_bytes);
    int voff[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) voff[b] = (int)(b * blk_bytes) + lane * 12;
    const int s0 = s_lo + wu;
    u32x3 buf[D][RB];
#pragma unroll
    for (int u = 0; u < D; ++u) issue_step<RB>(buf[u], rv, voff, s0 + u * W, s_hi);

    // the workgroup's exception range, from the row pointers of step 0 (vector
    // loads issued before the activations): in every wave lane 0 holds
    // rp[n0] and lane 16 RB - 1 holds rp[min(n0 + 16 RB, N)].  Scalar loads of
    // the same two words would be waited for at the barrier after the
    // staging, and under the weight stream a scalar miss takes about 1 us.
    const int32_t e_lo = __builtin_amdgcn_readlane(oe0, 0);
    const int32_t e_hi = __builtin_amdgcn_readlane(oe1, RB * 16 - 1);

    // ---- 3. x' * 2^64 into LDS (the fast path's scale), with the exponent
    // range of the x' values and, for RMS, the sums of (x 2^-32)^2
    float sq[T];
    int elo = 0, ehi = 0;
#pragma unroll
    for (int t = 0; t < T; ++t) sq[t] = 0.0f;
    auto stage4 = [&](f32x4 v, f32x4 u, f32x4 lw, int t, int i) {
        if constexpr (LN) {
            const f32x4 s = v * kSsqScale;
            sq[t] += s.x * s.x + s.y * s.y + s.z * s.z + s.w * s.w;
        }
        if constexpr (M2) v = f32x4{silu_mul(v.x, u.x), silu_mul(v.y, u.y), silu_mul(v.z, u.z), silu_mul(v.w, u.w)};
        if constexpr (LN) v = lw * v;
        track_exp4(v, elo, ehi);
        *reinterpret_cast<f32x4*>(xl + t * krange + i) = v * kXScale;
    };
#pragma unroll
    for (int j = 0; j < NXM; ++j) {
        if (j * 4 * nthr >= krange) break;  // chunk j was not loaded
        const int i = (threadIdx.x + j * nthr) * 4;
        if (i < krange) {
            f32x4 lw = {1.0f, 1.0f, 1.0f, 1.0f};
            if constexpr (LN) lw = bf16x4_to_f32(lr[j]);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                f32x4 u = xr[j][t];
                if constexpr (M2) u = ur[j][t];
                stage4(xr[j][t], u, lw, t, i);
            }
        }
    }
    // columns beyond the register-staged ones (large K ranges with few
    // threads): loaded here, after the weight prefetch
    for (int i = (threadIdx.x + NXM * nthr) * 4; i < krange; i += nthr * 4) {
        const int k = k_lo + i;
        f32x4 lw = {1.0f, 1.0f, 1.0f, 1.0f};
        if constexpr (LN) lw = bf16x4_to_f32(*reinterpret_cast<const uint2*>(p.lnw + k));
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float* xt = p.x + (int64_t)t * p.xs;
            const f32x4 v = *reinterpret_cast<const f32x4*>(xt + k);
            f32x4 u = v;
            if constexpr (M2) u = *reinterpret_cast<const f32x4*>(xt + p.K + k);
            stage4(v, u, lw, t, i);
        }
    }
    if constexpr (LN) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
            float v = sq[t];
            for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
            if (lane == 0) ssq[wave * T + t] = v;
        }
    }
    {
        const bool bad = elo < kXRangeLo || ehi > kXRangeHi;
        const uint64_t b = __ballot(bad);
        if (lane == 0) wflag[wave] = b != 0;
    }
    // the workgroup's first round of exceptions, one entry per thread; a
    // descriptor over the n_exc entries reads zeros past the list's end
    const uint32_t exc_bytes = (uint32_t)min(p.n_exc, (int64_t)(1 << 28)) * 4u;
    const __amdgpu_buffer_rsrc_t r_ec = make_rsrc(p.ec, exc_bytes), r_ev = make_rsrc(p.ev, exc_bytes);
    const int32_t j_exc = e_lo + (int32_t)threadIdx.x;
    const uint32_t exc_off = j_exc < e_hi ? (uint32_t)j_exc * 4u : 0xFFFFFFF0u;
    const int ec0 = (int)__builtin_amdgcn_raw_buffer_load_b32(r_ec, (int)exc_off, 0, 0);
    const float ev0 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r_ev, (int)exc_off, 0, 0));
    __syncthreads();

    // ---- 3b. (rare) some nonzero |x'| outside [2^-64, 2^63): per-token scale
    // exponents from the largest |x'| of the workgroup's columns, and x'
    // staged again from the inputs with them
    int P[T];
#pragma unroll
    for (int t = 0; t < T; ++t) P[t] = kXScaleExp;
    // the W flags in one LDS read, lane w reading wave w's
    if (__ballot(lane < W && wflag[lane] != 0) != 0) {
        auto xprime = [&](int t, int k) {
            const float* xt = p.x + (int64_t)t * p.xs;
            f32x4 v = *reinterpret_cast<const f32x4*>(xt + k);
            if constexpr (M2) {
                const f32x4 u = *reinterpret_cast<const f32x4*>(xt + p.K + k);
                v = f32x4{silu_mul(v.x, u.x), silu_mul(v.y, u.y), silu_mul(v.z, u.z), silu_mul(v.w, u.w)};
            }
            if constexpr (LN) v = bf16x4_to_f32(*reinterpret_cast<const uint2*>(p.lnw + k)) * v;
            return v;
        };
        int em[T];
#pragma unroll
        for (int t = 0; t < T; ++t) em[t] = -1000;
        for (int i = threadIdx.x * 4; i < krange; i += nthr * 4) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const f32x4 v = xprime(t, k_lo + i);
                em[t] = max(max(max(em[t], exp_or_min(v.x)), max(exp_or_min(v.y), exp_or_min(v.z))),
                            exp_or_min(v.w));
            }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            int e = em[t];
            for (int o = 32; o > 0; o >>= 1) e = max(e, __shfl_xor(e, o));
            if (lane == 0) wexp[wave * T + t] = e;
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < T; ++t) {
            int e = -1000;
            for (int w = 0; w < W; ++w) e = max(e, wexp[w * T + t]);
            P[t] = slow_scale_exp(e);
        }
        for (int i = threadIdx.x * 4; i < krange; i += nthr * 4) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const f32x4 v = xprime(t, k_lo + i);
                *reinterpret_cast<f32x4*>(xl + t * krange + i) =
                    f32x4{ldexpf(v.x, P[t]), ldexpf(v.y, P[t]), ldexpf(v.z, P[t]), ldexpf(v.w, P[t])};
            }
        }
        __syncthreads();
    }

    // ---- 4. main loop
    float acc[RB][T];
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[b][t] = 0.0f;

    // rounds of D of this wave's steps s0, s0 + W, ...; a wave stops after
    // its last step (the steps after it are all past s_hi)
    for (int sr = s0; sr < s_hi; sr += D * W) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            const int s = sr + u * W;
            // the step's words are unpacked before the load D steps ahead
            // reuses their registers: no copy of the loaded registers at the
            // loop's back edge, so no wait there for the loads in flight
            uint32_t pr[RB][4];
#pragma unroll
            for (int b = 0; b < RB; ++b) {
                unpack_pairs(buf[u][b].x, buf[u][b].y, buf[u][b].z, pr[b]);
                // (kept ahead of the load by the compiler's scheduler)
                asm volatile("" : "+v"(pr[b][0]), "+v"(pr[b][1]), "+v"(pr[b][2]), "+v"(pr[b][3])::"memory");
            }
            issue_step<RB>(buf[u], rv, voff, s + D * W, s_hi);
            if (s < s_hi) {
                const float* xs = xl + (s - s_lo) * 32 + q * 8;
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    const f32x4 xa = *reinterpret_cast<const f32x4*>(xs + t * krange);
                    const f32x4 xb = *reinterpret_cast<const f32x4*>(xs + t * krange + 4);
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

    // ---- 5. epilogue: lane quarters to LDS (waves are summed by the owners)
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int t = 0; t < T; ++t) {
            // (q0 + q1) + (q2 + q3) of the four lane quarters, on the VALU
            const float v = rows_and_halves(acc[b][t], [](float x, float y) { return x + y; });
            if (lane < 16) red[((wave * RB + b) * T + t) * 16 + lane] = v;
        }

    // exception products ev * x' of one round of nthr entries of the
    // workgroup's row-major exception list (zero outside the split's columns);
    // each owner adds its row's entries in list order
    auto stage_round = [&](int32_t j0, int c, float v) {
        const int32_t j = j0 + threadIdx.x;
        c -= k_lo;
        const bool in = j < e_hi && c >= 0 && c < krange;
#pragma unroll
        for (int t = 0; t < T; ++t) excv[threadIdx.x * T + t] = in ? v * ldexpf(xl[t * krange + c], -P[t]) : 0.0f;
    };
    float eacc = 0.0f;
    auto add_round = [&](int32_t j0) {
        if (oval) {
            const int32_t a = max(oe0, j0), z = min(oe1, j0 + nthr);
            // four entries per LDS round trip, added in list order
            for (int32_t j = a; j < z; j += 4) {
                float e[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) e[i] = excv[(min(j + i, z - 1) - j0) * T + otok];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (j + i < z) eacc += e[i];
            }
        }
    };
    if (e_lo < e_hi) stage_round(e_lo, ec0, ev0);
    // the owner's RMS scale, from the waves' sums staged before the loop:
    // formed before the barrier, where the waves that end their loop early
    // would only wait
    float rs = 1.0f;
    if constexpr (LN) {
        if (S == 1 && oval) {
            float sqs = 0.0f;
            for (int w = 0; w < W; ++w) sqs += ssq[w * T + otok];
            rs = rms_scale(sqs, p.K, p.eps);
        }
    }
    __syncthreads();
    float v = 0.0f;
    if (owner) {
        const int b = orow >> 4, l16 = orow & 15;
        for (int w = 0; w < W; ++w) v += red[((w * RB + b) * T + otok) * 16 + l16];
    }
    if (e_lo < e_hi) add_round(e_lo);
    for (int32_t j0 = e_lo + nthr; j0 < e_hi; j0 += nthr) {  // rare: more entries than threads
        __syncthreads();
        const int32_t j = j0 + threadIdx.x;
        int c = 0;
        float ev = 0.0f;
        if (j < e_hi) {
            c = p.ec[j];
            ev = p.ev[j];
        }
        stage_round(j0, c, ev);
        __syncthreads();
        add_round(j0);
    }

    float yv = 0.0f;  // the stored output
    if (oval) {
        int Po = P[0];
#pragma unroll
        for (int t = 1; t < T; ++t) Po = otok == t ? P[t] : Po;
        v = ldexpf(v, scale_exp(obase) - Po) + eacc;
        if (S == 1) {
            if constexpr (LN) v *= rs;
            yv = p.mode == 0 ? v : oy + v;
            if (p.store_y) p.y[(int64_t)otok * p.N + on] = yv;
        } else {
            p.part[((int64_t)sp * T + otok) * p.npad + on] = v;
        }
    }
    // ---- 6. fused greedy pick (one split; the host checks): the 16 RB owners
    // of a token are consecutive lanes of one wave, aligned to 16 RB, so an
    // xor butterfly over them leaves their best (output, row) pair in every
    // one; the first writes it for the second pass (launch_pick)
    if (p.amv) {
        float bv = oval ? yv : -__builtin_inff();
        int bi = oval ? on : 0x7FFFFFFF;
#pragma unroll
        for (int o = 1; o < RB * 16; o <<= 1) {
            const float ov = __shfl_xor(bv, o);
            const int oi = __shfl_xor(bi, o);
            if (pick_beats(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if (owner && orow == 0) {
            p.amv[(int64_t)otok * gridDim.x + blockIdx.x] = bv;
            p.ami[(int64_t)otok * gridDim.x + blockIdx.x] = bi;
        }
    }
    if (LN && S > 1 && blockIdx.x == 0 && threadIdx.x < T) {
        float sqs = 0.0f;
        for (int w = 0; w < W; ++w) sqs += ssq[w * T + threadIdx.x];
        p.ssq[sp * T + threadIdx.x] = sqs;
    }
}

// second pass of a split linear: sum the partials of each output in split
// order.  Every split's partial (and, with RMS, sum of squares) is loaded
// before any is added, CB at a time through a descriptor over the partials
// (one memory round trip for up to CB splits, where a load-add loop paid one
// per split); the sum runs in split order.  CB = 8 where the splits fit,
// else 16 (kReduceBatchMax).  Grid (rows / 256, tokens): no index division.
template <int CB, bool RMS>
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ part, const float* __restrict__ ssq,
                                                       float* __restrict__ y, int N, int npad, int T, int S,
                                                       int mode, float eps, int K) {
    const int t = blockIdx.y, n = blockIdx.x * 256 + threadIdx.x;
    if (n >= N) return;
    float* o = y + (int64_t)t * N + n;
    const float old = mode == 0 ? 0.0f : *o;
    // byte offsets in 32 bits: the host rejects (S + 16) T npad 4 >= 2^31
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(part, (uint32_t)((int64_t)S * T * npad * 4));
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(ssq, RMS ? (uint32_t)(S * T * 4) : 0u);
    float v = 0.0f, q = 0.0f;
    for (int s0 = 0; s0 < S; s0 += CB) {
        float a[CB], b[CB];
#pragma unroll
        for (int u = 0; u < CB; ++u) {
            const int sp = s0 + u;  // past S: out of the descriptor's range, reads 0 (not added)
            a[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rp, ((sp * T + t) * npad + n) * 4, 0, 0));
            b[u] = RMS ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rq, (sp * T + t) * 4, 0, 0)) : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < CB; ++u) {
            if (s0 + u < S) {
                v += a[u];
                q += b[u];
            }
        }
    }
    if (RMS) v *= rms_scale(q, K, eps);
    *o = mode == 0 ? v : old + v;
}

// greedy pick over entries [c * len, min(n, (c + 1) * len)) of token
// blockIdx.y, c = blockIdx.x: the best (value, index) pair (pick_beats order,
// which makes the result independent of the order of combination) goes to
// tv / ti [token][chunk], or to ids[token] when ids is given (one chunk)
__global__ __launch_bounds__(kPickThreads) void k_pick(const float* __restrict__ v, const int32_t* __restrict__ ix,
                                                       int64_t n, int64_t stride, int64_t len, float* tv,
                                                       int32_t* ti, int64_t* ids) {
    __shared__ float sv[kPickThreads / 64];
    __shared__ int si[kPickThreads / 64];
    const int t = blockIdx.y;
    const int64_t lo = (int64_t)blockIdx.x * len, hi = min(n, lo + len);
    const float* vt = v + (int64_t)t * stride;
    const int32_t* it = ix ? ix + (int64_t)t * stride : nullptr;
    float bv = -__builtin_inff();
    int bi = 0x7FFFFFFF;
    // eight independent loads per thread in flight per round: a chunk of
    // kPickChunk entries takes one memory round trip
    static_assert(kPickChunk <= 8 * kPickThreads, "one round per chunk");
    for (int64_t i0 = lo + threadIdx.x; i0 < hi; i0 += 8 * (int64_t)kPickThreads) {
        float a[8];
        int ai[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t i = i0 + (int64_t)u * kPickThreads;
            a[u] = i < hi ? vt[i] : -__builtin_inff();
            ai[u] = i < hi ? (it ? it[i] : (int)i) : 0x7FFFFFFF;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (pick_beats(a[u], ai[u], bv, bi)) {
                bv = a[u];
                bi = ai[u];
            }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (pick_beats(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kPickThreads / 64; ++w)
            if (pick_beats(sv[w], si[w], bv, bi)) {
                bv = sv[w];
                bi = si[w];
            }
        if (ids) {
            ids[t] = bi;
        } else {
            tv[(int64_t)t * gridDim.x + blockIdx.x] = bv;
            ti[(int64_t)t * gridDim.x + blockIdx.x] = bi;
        }
    }
}

void launch_pick(const float* v, const int32_t* ix, int64_t n, int64_t stride, int T, float* tv, int32_t* ti,
                 int64_t* ids, hipStream_t st) {
    if (n <= kPickChunk) {
        hipLaunchKernelGGL(k_pick, dim3(1, T), dim3(kPickThreads), 0, st, v, ix, n, stride, n, nullptr, nullptr, ids);
        return;
    }
    const int64_t nc = pick_chunks(n);
    hipLaunchKernelGGL(k_pick, dim3((unsigned)nc, T), dim3(kPickThreads), 0, st, v, ix, n, stride,
                       (int64_t)kPickChunk, tv, ti, nullptr);
    hipLaunchKernelGGL(k_pick, dim3(1, T), dim3(kPickThreads), 0, st, tv, ti, nc, nc, nc, nullptr, nullptr, ids);
}

// the decode step's bookkeeping after its greedy pick: id = ids[0] is recorded
// in out[*steps] (when steps lies in [0, out_len)), becomes the next input
// token (tok, when given) and its embedding row (bf16, converted exactly) the
// next step's activations x; *steps and *pos advance by one.  The id used for
// the row is clamped into [0, vocab).
__global__ __launch_bounds__(256) void k_decode_advance(const int64_t* __restrict__ ids,
                                                        const uint16_t* __restrict__ emb, int64_t vocab, int hidden,
                                                        float* __restrict__ x, int64_t* __restrict__ out,
                                                        int64_t out_len, int64_t* __restrict__ steps,
                                                        int64_t* __restrict__ pos, int64_t* __restrict__ tok) {
    const int64_t id = ids[0];
    const uint16_t* row = emb + min(max(id, (int64_t)0), vocab - 1) * (int64_t)hidden;
    if (((uintptr_t)row & 15u) == 0 && ((uintptr_t)x & 15u) == 0 && hidden % 8 == 0) {
        // 8 values per 16-byte load, four loads per thread in flight before
        // the first store (one memory round trip for hidden <= 8192)
        const int ng = hidden / 8;
        for (int g0 = threadIdx.x; g0 < ng; g0 += 4 * (int)blockDim.x) {
            uint4 w[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int gi = g0 + u * (int)blockDim.x;
                w[u] = gi < ng ? reinterpret_cast<const uint4*>(row)[gi] : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int gi = g0 + u * (int)blockDim.x;
                if (gi < ng) {
                    const uint32_t c[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
                    float4* o = reinterpret_cast<float4*>(x) + 2 * (int64_t)gi;
                    o[0] = make_float4(__uint_as_float(c[0] << 16), __uint_as_float(c[0] & 0xFFFF0000u),
                                       __uint_as_float(c[1] << 16), __uint_as_float(c[1] & 0xFFFF0000u));
                    o[1] = make_float4(__uint_as_float(c[2] << 16), __uint_as_float(c[2] & 0xFFFF0000u),
                                       __uint_as_float(c[3] << 16), __uint_as_float(c[3] & 0xFFFF0000u));
                }
            }
        }
    } else {
        for (int k = threadIdx.x; k < hidden; k += blockDim.x) x[k] = __uint_as_float((uint32_t)row[k] << 16);
    }
    if (threadIdx.x == 0) {
        const int64_t s = *steps;
        if (s >= 0 && s < out_len) out[s] = id;
        *steps = s + 1;
        *pos += 1;
        if (tok) *tok = id;
    }
}

void launch_decode_advance(const int64_t* ids, const uint16_t* emb, int64_t vocab, int hidden, float* x,
                           int64_t* out, int64_t out_len, int64_t* steps, int64_t* pos, int64_t* tok,
                           hipStream_t st) {
    hipLaunchKernelGGL(k_decode_advance, dim3(1), dim3(256), 0, st, ids, emb, vocab, hidden, x, out, out_len, steps,
                       pos, tok);
}

// ------------------------------------------------------------------ launch
template <int T, int RB, bool M2, bool LN, bool SH>
static void launch_t(const LinearParams& p, dim3 grid, int threads, size_t lds, hipStream_t st) {
    if (lds > kDefaultLds)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv<T, RB, M2, LN, SH>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL((k_gemv<T, RB, M2, LN, SH>), grid, dim3(threads), lds, st, p);
}

template <int T, int RB, bool M2, bool LN>
static void launch_depth(const LinearParams& p, dim3 grid, int threads, size_t lds, hipStream_t st) {
    if (gemv_shallow(T, RB, threads / 64, M2, LN)) launch_t<T, RB, M2, LN, true>(p, grid, threads, lds, st);
    else launch_t<T, RB, M2, LN, false>(p, grid, threads, lds, st);
}

template <int T, int RB>
static void launch_pro(const LinearParams& p, dim3 grid, int threads, size_t lds, hipStream_t st) {
    const bool m2 = p.mode == 2, ln = p.lnw != nullptr;
    if (m2 && ln) launch_depth<T, RB, true, true>(p, grid, threads, lds, st);
    else if (m2) launch_depth<T, RB, true, false>(p, grid, threads, lds, st);
    else if (ln) launch_depth<T, RB, false, true>(p, grid, threads, lds, st);
    else launch_depth<T, RB, false, false>(p, grid, threads, lds, st);
}

template <int RB>
static int launch_rb(const LinearParams& p, int T, dim3 grid, int threads, size_t lds, hipStream_t st) {
    switch (T) {
        case 1: launch_pro<1, RB>(p, grid, threads, lds, st); return 0;
        case 2: launch_pro<2, RB>(p, grid, threads, lds, st); return 0;
        case 3: launch_pro<3, RB>(p, grid, threads, lds, st); return 0;
        case 4: launch_pro<4, RB>(p, grid, threads, lds, st); return 0;
    }
    return -1;
}

template <int CB, bool RMS>
static void launch_reduce_t(const LinearParams& p, int T, int splits, hipStream_t st) {
    hipLaunchKernelGGL((k_splitk_reduce<CB, RMS>), dim3((unsigned)((p.N + 255) / 256), (unsigned)T), dim3(256), 0, st, p.part,
                       p.ssq, p.y, p.N, p.npad, T, splits, p.mode, p.eps, p.K);
}

void launch_splitk_reduce(const LinearParams& p, int T, int splits, hipStream_t st) {
    const bool rms = p.lnw != nullptr;
    if (splits <= 8) {
        if (rms) launch_reduce_t<8, true>(p, T, splits, st);
        else launch_reduce_t<8, false>(p, T, splits, st);
    } else {
        if (rms) launch_reduce_t<kReduceBatchMax, true>(p, T, splits, st);
        else launch_reduce_t<kReduceBatchMax, false>(p, T, splits, st);
    }
}

int launch_gemv(const LinearParams& p, int T, int rb, int waves, int splits, hipStream_t st) {
    const int64_t nblk = (p.N + 15) / 16;
    dim3 grid((unsigned)((nblk + rb - 1) / rb), (unsigned)splits);
    const size_t lds = gemv_lds_bytes(p.K, T, rb, waves, splits);
    int rc;
    switch (rb) {
        case 1: rc = launch_rb<1>(p, T, grid, waves * 64, lds, st); break;
        case 2: rc = launch_rb<2>(p, T, grid, waves * 64, lds, st); break;
        case 4: rc = launch_rb<4>(p, T, grid, waves * 64, lds, st); break;
        default: return -1;
    }
    if (rc) return rc;
    if (splits > 1) launch_splitk_reduce(p, T, splits, st);
    return 0;
}

}  // namespace rv12
