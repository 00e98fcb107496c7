// Decode-step attention for one layer (one token), gfx950: the companion of
// the 12-bit linears in a decode step (replaces rope_attn_k,
// ramvi/engine/ramvi_engine/kernels/tkernels.py:164-213).
//
// Grid (KV heads, splits), 320 threads (a short cache: one split, 1024
// threads and one workgroup per q head instead, QH below).  Workgroup (g, sp)
// covers the positions [lo, hi) of 0..pos, at most 80 of them (256 at 1024
// threads):
//   0. first the step's own q/k/v values, then every cache value the
//      workgroup reads are loaded: a quarter key row (HD/4 dims) per thread,
//      4 threads per position, and the values of 16 (8) positions at a dim
//      pair per thread.  The cache loads go through descriptors that end at
//      min(hi, pos), so the positions beyond the split and the step's own slot
//      (written by split 0 in step 1) read as zeros without a memory access;
//   1. q (G heads) and k get their head RMSNorm and the rotate-half RoPE at
//      position pos (angle pos * inv[i], precise sin/cos), one wave per head;
//      k and v are rounded to the cache dtype (as the reference rounds them,
//      tkernels.py:187-190); split 0 writes them into the cache at pos;
//   2. scores s[i][j] = scale * q_i . K[j]: each of the 4 threads of a
//      position sums its quarter of the dims, two lane exchanges add them;
//      j == pos uses the step's own k;
//   3. per head (one wave each, the scores passed through LDS) the split's
//      max m, the weights exp(s - m) and their sum l;
//   4. acc[i][d] = sum_j exp(s[i][j] - m_i) V[j][d]: threads over dim pairs and
//      position groups, the groups added through LDS in a fixed order;
//   5. one split: out = acc / l.  Several: (acc, m, l) partials, combined by
//      k_attn_combine in split order.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "rv12_device.h"
#include "rv12_internal.h"

namespace rv12 {

__device__ __forceinline__ float bf16f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f2bf16(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t attn_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)0x00020000);
}

template <int N>
__device__ __forceinline__ void load_words(__amdgpu_buffer_rsrc_t r, int off, uint32_t (&w)[N][4]) {
#pragma unroll
    for (int c = 0; c < N; ++c) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off + c * 16, 0, 0);
        w[c][0] = v[0];
        w[c][1] = v[1];
        w[c][2] = v[2];
        w[c][3] = v[3];
    }
}

// value i of raw cache words (bf16 pairs or float32)
template <bool BF16, int N>
__device__ __forceinline__ float word_val(const uint32_t (&w)[N][4], int i) {
    if constexpr (BF16) {
        const uint32_t u = w[i >> 3][(i >> 1) & 3];
        return __uint_as_float((i & 1) ? (u & 0xFFFF0000u) : (u << 16));
    } else {
        return __uint_as_float(w[i >> 2][i & 3]);
    }
}

template <bool BF16>
__device__ __forceinline__ float pair_val(const uint32_t (&u)[2], int e) {
    if constexpr (BF16) return __uint_as_float(e ? (u[0] & 0xFFFF0000u) : (u[0] << 16));
    else return __uint_as_float(u[e]);
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    v += dpp<kDppMirror>(v);
    return rows_and_halves(v, [](float x, float y) { return x + y; });
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<kDppXor1>(v));
    v = fmaxf(v, dpp<kDppXor2>(v));
    v = fmaxf(v, dpp<kDppHalfMirror>(v));
    v = fmaxf(v, dpp<kDppMirror>(v));
    return rows_and_halves(v, [](float x, float y) { return fmaxf(x, y); });
}

// RMSNorm (weight pair wa, wb) and rotate-half RoPE (cos c, sin sn) of one
// head held by one wave: lane l < HD/2 holds the pair (a, b) = (x[l], x[l + HD/2])
// (the other lanes hold zeros), so the whole transform needs no barrier.
// BF16: the results are rounded to bf16 (the cache dtype of the step's key);
// a non-null crow (the key's cache row, bf16 or float32) receives them too.
template <int HD, bool BF16 = false>
__device__ __forceinline__ void norm_rope_wave(float a, float b, float wa, float wb, float c, float sn, float eps,
                                               float* dst, int lane, void* crow = nullptr) {
    constexpr int half = HD / 2;
    const float rs = 1.0f / sqrtf(wave_sum(a * a + b * b) / (float)HD + eps);
    if (lane < half) {
        const float x = wa * (a * rs), y = wb * (b * rs);
        float o0 = x * c - y * sn, o1 = y * c + x * sn;
        if constexpr (BF16) {
            const uint16_t b0 = f2bf16(o0), b1 = f2bf16(o1);
            o0 = bf16f(b0);
            o1 = bf16f(b1);
            if (crow) {
                static_cast<uint16_t*>(crow)[lane] = b0;
                static_cast<uint16_t*>(crow)[lane + half] = b1;
            }
        } else if (crow) {
            static_cast<float*>(crow)[lane] = o0;
            static_cast<float*>(crow)[lane + half] = o1;
        }
        dst[lane] = o0;
        dst[lane + half] = o1;
    }
}

// NT threads, 4 per position: a workgroup covers P = NT / 4 positions at
// most (kAttnThreads = 320 over 80 positions; kAttnLongThreads = 1024 over
// 256, one split per kv head for short contexts, so no combine pass).  GK q
// heads share a kv head.  QH (one split only): one workgroup per q head
// instead of per kv head, the grid over the q heads; the first q head of each
// kv head writes the step's key and value into the cache (the others read
// only the positions before it, which the write does not touch).
template <int HD, int GK, bool BF16, int NT, bool QH = false>
__global__ __launch_bounds__(NT) void k_rope_attn(AttnParams p) {
    constexpr int G = QH ? 1 : GK;  // q heads of this workgroup
    extern __shared__ float lds[];
    constexpr int NW = NT / 64;
    constexpr int P = NT / 4;              // positions of one workgroup at most
    constexpr int EB = BF16 ? 2 : 4;       // cache bytes per value
    constexpr int QD = HD / 4;             // dims per thread in the scores
    constexpr int KW = QD * EB / 16;       // 16-byte words of a thread's key quarter
    constexpr int DP = HD / 2;             // dim pairs
    constexpr int PG = NT / DP;            // position groups of the value sums
    constexpr int PPG = P / PG;            // positions per group
    constexpr int half = HD / 2, HPW = (G + NW) / NW;
    const int g = QH ? (int)blockIdx.x / GK : (int)blockIdx.x, sp = blockIdx.y, S = gridDim.y;
    const int qh0 = QH ? (int)blockIdx.x : g * G;            // the workgroup's first q head
    const bool writer = !QH || (int)blockIdx.x == g * GK;  // writes the step's k and v
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wu = __builtin_amdgcn_readfirstlane(wave);
    const int H = p.n_kv * GK;
    // every kernel argument in SGPRs now: their loads then form one batch and
    // one wait, not a chain of them after the position's
    asm volatile("" : : "s"(p.maxt), "s"(p.n_kv), "s"(p.smul), "s"(__float_as_uint(p.eps)),
                 "s"(__float_as_uint(p.scale)));
    // ---- 0. the step's values: wave w the heads w, w + NW, .. of q (0..G-1)
    // and k (G), lane l < HD/2 the pair (l, l + HD/2), thread d < HD v[d]
    const int la = lane < half ? lane : 0;
    const float msk = lane < half ? 1.0f : 0.0f;
    const __amdgpu_buffer_rsrc_t qr = attn_rsrc(p.qkv, (uint32_t)((H + 2 * p.n_kv) * HD * 4));
    float qa[HPW], qb[HPW];
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
        const int i = min(wave + j * NW, G);
        const int off = ((i < G ? qh0 + i : H + g) * HD + la) * 4;
        qa[j] = msk * __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(qr, off, 0, 0));
        qb[j] = msk * __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(qr, off + half * 4, 0, 0));
    }
    const float vown = __uint_as_float(
        __builtin_amdgcn_raw_buffer_load_b32(qr, ((H + p.n_kv + g) * HD + (t < HD ? t : 0)) * 4, 0, 0));
    const float wqa = p.qn[la], wqb = p.qn[la + half], wka = p.kn[la], wkb = p.kn[la + half], iv = p.inv[la];

    // a position outside the cache is computed as position 0 with nothing
    // cached (every cache load reads zeros) and no cache write, and its
    // outputs are zeros (partials that combine to zeros): no branch before
    // the loads, so the position's load and the step's q/k/v loads leave
    // together
    const int64_t pos_in = *p.pos;
    const bool bad = pos_in < 0 || pos_in >= p.maxt;
    const int64_t pos = bad ? 0 : pos_in;
    float* qs = lds;                // [G][HD]
    float* kn = qs + G * HD;        // [HD] step key (normed, roped, rounded)
    float* vn = kn + HD;            // [HD] step value (rounded)
    float* wt = vn + HD;            // [P][G] weights exp(s - m)
    float* ss = wt + P * G;         // [G][P] scaled scores (-inf beyond the span)
    float* stat = ss + G * P;       // [2 G] m, l
    float* wacc = stat + 2 * G;     // [PG][G][HD] value sums of the position groups
    const int n = (int)pos + 1;  // n <= 10240 and S <= 128: 32-bit products below 2^21
    // (selects, not a branch: one split takes all n positions)
    const int lo = S > 1 ? (int)__umulhi((uint32_t)(sp * n), p.smul) : 0;
    const int hi = S > 1 ? (int)__umulhi((uint32_t)((sp + 1) * n), p.smul) : n;
    const int span = hi - lo;  // <= P (host)
    const int64_t row0 = (int64_t)g * p.maxt * HD;

    // the cache values: positions [0, min(hi, pos)) are in range
    const uint32_t cbytes = (uint32_t)min(hi, n - 1) * HD * EB;
    const __amdgpu_buffer_rsrc_t kr = attn_rsrc(reinterpret_cast<const char*>(p.kc) + row0 * EB, cbytes);
    const __amdgpu_buffer_rsrc_t vr = attn_rsrc(reinterpret_cast<const char*>(p.vc) + row0 * EB, cbytes);
    const int pl = t >> 2, qq = t & 3;  // score thread: position lo + pl, dims [qq QD, qq QD + QD)
    uint32_t kw[KW][4];
    load_words<KW>(kr, ((lo + pl) * HD + qq * QD) * EB, kw);
    const int dp = t % DP, pg = t / DP;  // value thread: dims 2 dp, 2 dp + 1 of positions pg PPG ..
    uint32_t vw[PPG][2];
#pragma unroll
    for (int r = 0; r < PPG; ++r) {
        const int off = ((lo + pg * PPG + r) * HD + 2 * dp) * EB;
        if constexpr (BF16) {
            vw[r][0] = __builtin_amdgcn_raw_buffer_load_b32(vr, off, 0, 0);
            vw[r][1] = 0;
        } else {
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(vr, off, 0, 0);
            vw[r][0] = v[0];
            vw[r][1] = v[1];
        }
    }

    // ---- 1. the step's q (G heads) and k, one wave per head; v as read
    float sn, cs;
    sincosf((float)pos * iv, &sn, &cs);
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
        const int i = wave + j * NW;
        if (i < G) {
            norm_rope_wave<HD>(qa[j], qb[j], wqa, wqb, cs, sn, p.eps, qs + i * HD, lane);
        } else if (i == G) {  // k, rounded to the cache dtype; split 0 writes it at pos
            void* krow = sp == 0 && !bad && writer ? static_cast<char*>(p.kc) + (row0 + pos * HD) * EB : nullptr;
            norm_rope_wave<HD, BF16>(qa[j], qb[j], wka, wkb, cs, sn, p.eps, kn, lane, krow);
        }
    }
    if (t < HD) {  // v, rounded to the cache dtype; split 0 writes it at pos
        float v = vown;
        if constexpr (BF16) {
            const uint16_t vb = f2bf16(v);
            v = bf16f(vb);
            if (sp == 0 && !bad && writer) reinterpret_cast<uint16_t*>(p.vc)[row0 + pos * HD + t] = vb;
        } else if (sp == 0 && !bad && writer) {
            reinterpret_cast<float*>(p.vc)[row0 + pos * HD + t] = v;
        }
        vn[t] = v;
    }
    __syncthreads();

    // ---- 2. scores: thread (pl, qq) sums its quarter of the dims.  The key
    // quarter (the step's own key at j == pos, whose cache slot reads as
    // zeros) and the G heads' q quarters are in registers before the first
    // product, so the LDS reads are waited for once
    const bool valid = pl < span;
    const bool own = lo + pl == pos;
    float kf[QD];
#pragma unroll
    for (int d = 0; d < QD; ++d) kf[d] = word_val<BF16>(kw, d);
    if (own) {
#pragma unroll
        for (int d = 0; d < QD; d += 4) {
            const float4 k4 = *reinterpret_cast<const float4*>(kn + qq * QD + d);
            kf[d] = k4.x;
            kf[d + 1] = k4.y;
            kf[d + 2] = k4.z;
            kf[d + 3] = k4.w;
        }
    }
    float4 qv[G][QD / 4];
#pragma unroll
    for (int i = 0; i < G; ++i) {
#pragma unroll
        for (int d = 0; d < QD; d += 4) qv[i][d / 4] = *reinterpret_cast<const float4*>(qs + i * HD + qq * QD + d);
    }
    float sc[G];
#pragma unroll
    for (int i = 0; i < G; ++i) {
        float s = 0.0f;
#pragma unroll
        for (int d = 0; d < QD; d += 4) {
            s = fmaf(qv[i][d / 4].x, kf[d], s);
            s = fmaf(qv[i][d / 4].y, kf[d + 1], s);
            s = fmaf(qv[i][d / 4].z, kf[d + 2], s);
            s = fmaf(qv[i][d / 4].w, kf[d + 3], s);
        }
        sc[i] = s;
    }
#pragma unroll
    for (int i = 0; i < G; ++i) {
        float s = sc[i];
        s += dpp<kDppXor1>(s);
        s += dpp<kDppXor2>(s);
        sc[i] = valid ? s * p.scale : -INFINITY;
    }

    // ---- 3. softmax statistics: the scores go through LDS, then the wave
    // of each head (wave w takes the heads w, w + NW, ..) finds the split's
    // max m, the weights exp(s - m) and their sum l with wave-wide reductions
    // only (lane j holds the positions j, j + 64, ..)
    if (qq == 0) {
#pragma unroll
        for (int i = 0; i < G; ++i) ss[i * P + pl] = sc[i];
    }
    __syncthreads();
    constexpr int PL = (P + 63) / 64;  // positions per lane
    static_assert(P > 64, "every lane holds a position");
    for (int i = wu; i < G; i += NW) {
        float a[PL];
#pragma unroll
        for (int j = 0; j < PL; ++j) a[j] = lane + 64 * j < P ? ss[i * P + lane + 64 * j] : -INFINITY;
        float mx = a[0];
#pragma unroll
        for (int j = 1; j < PL; ++j) mx = fmaxf(mx, a[j]);
        const float m = wave_max(mx);
        float ls = 0.0f;
#pragma unroll
        for (int j = 0; j < PL; ++j) {
            const int jp = lane + 64 * j;
            const float e = jp < span ? expf(a[j] - m) : 0.0f;
            if (jp < P) wt[jp * G + i] = e;
            ls += e;
        }
        const float l = wave_sum(ls);
        if (lane == 0) {
            stat[i] = m;
            stat[G + i] = l;
        }
    }
    __syncthreads();  // the weights of every position

    // ---- 4. weighted values: thread (dp, pg) over its PPG positions
    float acc[G][2];
#pragma unroll
    for (int i = 0; i < G; ++i) acc[i][0] = acc[i][1] = 0.0f;
    const float vn0 = vn[2 * dp], vn1 = vn[2 * dp + 1];
    float w[PPG][G];  // the weights (zero beyond the span), read before the first product
#pragma unroll
    for (int r = 0; r < PPG; ++r) {
        if constexpr (G % 4 == 0) {  // 16-byte reads: wt is 16-byte aligned (offsets G HD + 2 HD floats)
#pragma unroll
            for (int i = 0; i < G; i += 4) {
                const float4 w4 = *reinterpret_cast<const float4*>(wt + (pg * PPG + r) * G + i);
                w[r][i] = w4.x;
                w[r][i + 1] = w4.y;
                w[r][i + 2] = w4.z;
                w[r][i + 3] = w4.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < G; ++i) w[r][i] = wt[(pg * PPG + r) * G + i];
        }
    }
#pragma unroll
    for (int r = 0; r < PPG; ++r) {
        const bool ownj = lo + pg * PPG + r == pos;
        const float v0 = ownj ? vn0 : pair_val<BF16>(vw[r], 0);
        const float v1 = ownj ? vn1 : pair_val<BF16>(vw[r], 1);
#pragma unroll
        for (int i = 0; i < G; ++i) {
            acc[i][0] = fmaf(w[r][i], v0, acc[i][0]);
            acc[i][1] = fmaf(w[r][i], v1, acc[i][1]);
        }
    }
#pragma unroll
    for (int i = 0; i < G; ++i) {
        wacc[(pg * G + i) * HD + 2 * dp] = acc[i][0];
        wacc[(pg * G + i) * HD + 2 * dp + 1] = acc[i][1];
    }
    __syncthreads();

    // ---- 5. output or partials
    // [n_kv][S][G][HD + 2] (S > 1 only, which the one-q-head form never runs with)
    float* part = p.part + ((int64_t)g * S + sp) * G * (HD + 2);
    for (int o = t; o < G * HD; o += NT) {
        const int i = o / HD, d = o % HD;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < PG; ++w) v += wacc[(w * G + i) * HD + d];
        if (S == 1) p.out[((int64_t)qh0 + i) * HD + d] = bad ? 0.0f : v / stat[G + i];
        else part[i * (HD + 2) + d] = bad ? 0.0f : v;
    }
    if (S > 1 && t < G) {  // (a position outside the cache: l = 1 on split 0 only)
        part[t * (HD + 2) + HD] = bad ? (sp == 0 ? 0.0f : -INFINITY) : stat[t];
        part[t * (HD + 2) + HD + 1] = bad ? (sp == 0 ? 1.0f : 0.0f) : stat[G + t];
    }
}

// combine the splits of each head: M = max m_s, w_s = e^(m_s - M),
// out = sum acc_s w_s / sum l_s w_s, the numerator in split order.  One
// workgroup per head, one thread per dim; every load (the split statistics,
// one split per thread, and the thread's value of every split, CB at a time)
// is issued before anything waits, so the combine costs one memory round trip.
// Descriptors over the head's partials read zeros past the last split.
// CB values per thread at a time: the smallest of 16, 32, 64 that holds the
// splits (8B decode at 2k context, 32 splits: 11.49 -> 11.20 us per layer
// with 32 against 64, half of whose loads read past the last split; 0.6B at
// 12 splits: 7.42 -> 7.24 us with 16 against 32).
// R rows per kv head (G at one token, T G for a batch: row i is token i / G,
// head i % G of the group); out is [T][n_heads][HD].
// HD is a template argument, so the loops over the workgroup's waves unroll.
// rmul, gmul: floor(2^32 / R) + 1 and floor(2^32 / G) + 1 (R, G >= 2), so
// that the quotients of the row indexes (below 2^16) are mulhi products.
template <int HD, int CB>
__global__ __launch_bounds__(128) void k_attn_combine(const float* __restrict__ part, float* __restrict__ out, int S,
                                                      int G, int R, int H, uint32_t rmul, uint32_t gmul) {
    constexpr int nw = HD >> 6;
    __shared__ float wts[kAttnMaxSplits];
    __shared__ float red[2][nw];
    const int h = blockIdx.x, d = threadIdx.x, lane = d & 63, wave = d >> 6;
    const int g = R > 1 ? (int)__umulhi((uint32_t)h, rmul) : h, i = h - g * R;
    const int stride = R * (HD + 2) * 4;  // bytes from one split's partial of row i to the next
    const __amdgpu_buffer_rsrc_t r =
        attn_rsrc(part + ((int64_t)g * S * R + i) * (HD + 2), (uint32_t)((S - 1) * stride + (HD + 2) * 4));
    // statistics of splits d, d + HD (HD >= 64 threads, S <= 128)
    float m[2], l[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int s2 = d + u * HD;
        const auto ml = __builtin_amdgcn_raw_buffer_load_b64(r, s2 * stride + HD * 4, 0, 0);
        m[u] = s2 < S ? __uint_as_float(ml[0]) : -INFINITY;
        l[u] = s2 < S ? __uint_as_float(ml[1]) : 0.0f;
    }
    float a[CB];
#pragma unroll
    for (int u = 0; u < CB; ++u)
        a[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, u * stride + d * 4, 0, 0));
    // M over the splits, then the weights and the denominator
    float mx = wave_max(fmaxf(m[0], m[1]));
    if (lane == 0) red[0][wave] = mx;
    __syncthreads();
    mx = red[0][0];
    for (int w = 1; w < nw; ++w) mx = fmaxf(mx, red[0][w]);
    float dn = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int s2 = d + u * HD;
        const float w8 = l[u] > 0.0f ? expf(m[u] - mx) : 0.0f;
        if (s2 < kAttnMaxSplits) wts[s2] = w8;
        dn = fmaf(l[u], w8, dn);
    }
    dn = wave_sum(dn);
    if (lane == 0) red[1][wave] = dn;
    __syncthreads();
    float den = red[1][0];
    for (int w = 1; w < nw; ++w) den += red[1][w];
    float num = 0.0f;
#pragma unroll
    for (int u = 0; u < CB; ++u) num = fmaf(a[u], u < S ? wts[u] : 0.0f, num);
    for (int s0 = CB; s0 < S; s0 += CB) {  // more splits than one batch
#pragma unroll
        for (int u = 0; u < CB; ++u)
            a[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (s0 + u) * stride + d * 4, 0, 0));
#pragma unroll
        for (int u = 0; u < CB; ++u)
            num = fmaf(a[u], s0 + u < S ? wts[min(s0 + u, kAttnMaxSplits - 1)] : 0.0f, num);
    }
    const int tk = G > 1 ? (int)__umulhi((uint32_t)i, gmul) : i;  // token i / G, head g G + i % G
    out[((int64_t)tk * H + g * G + (i - tk * G)) * HD + d] = num / den;
}

// the combine pass over R rows per kv head (nothing to do for one split)
static uint32_t div_mul(int v) { return v > 1 ? (uint32_t)((uint64_t(1) << 32) / (uint64_t)v + 1) : 0u; }

static void launch_combine(const AttnParams& p, int S, int G, int R, hipStream_t st) {
    const dim3 grid((unsigned)(p.n_kv * R)), block((unsigned)p.head_dim);
    if (S <= 1) return;
    const uint32_t rm = div_mul(R), gm = div_mul(G);
    if (p.head_dim == 128) {
        if (S <= 16) hipLaunchKernelGGL((k_attn_combine<128, 16>), grid, block, 0, st, p.part, p.out, S, G, R, p.n_heads, rm, gm);
        else if (S <= 32) hipLaunchKernelGGL((k_attn_combine<128, 32>), grid, block, 0, st, p.part, p.out, S, G, R, p.n_heads, rm, gm);
        else hipLaunchKernelGGL((k_attn_combine<128, 64>), grid, block, 0, st, p.part, p.out, S, G, R, p.n_heads, rm, gm);
    } else {
        if (S <= 16) hipLaunchKernelGGL((k_attn_combine<64, 16>), grid, block, 0, st, p.part, p.out, S, G, R, p.n_heads, rm, gm);
        else if (S <= 32) hipLaunchKernelGGL((k_attn_combine<64, 32>), grid, block, 0, st, p.part, p.out, S, G, R, p.n_heads, rm, gm);
        else hipLaunchKernelGGL((k_attn_combine<64, 64>), grid, block, 0, st, p.part, p.out, S, G, R, p.n_heads, rm, gm);
    }
}

// ---------------------------------------------------------------- batches
// T tokens of one sequence at positions p0 = *pos .. p0 + T - 1 (the
// reference's batched companions qk_rope_cache_k + attn_k,
// ramvi/engine/ramvi_engine/kernels/tkernels.py:82-150).  A batch that does
// not fit the cache (p0 < 0 or p0 + T > maxt) gives zeros and writes no cache.

// 1. one wave per (head, token): q heads get their RMSNorm and RoPE into qo;
// k heads the same, rounded to the cache dtype, into the cache at p0 + t; v
// heads rounded into the cache.
template <int HD, bool BF16>
__global__ __launch_bounds__(64) void k_qk_rope_cache(AttnParams p) {
    constexpr int half = HD / 2;
    const int h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int H = p.n_heads, KV = p.n_kv;
    const int64_t p0 = *p.pos;
    if (p0 < 0 || p0 + p.T > p.maxt) return;
    const int64_t pos = p0 + t;
    const float* row = p.qkv + (int64_t)t * (H + 2 * KV) * HD;
    if (h < H + KV) {
        const int la = lane < half ? lane : 0;
        const float msk = lane < half ? 1.0f : 0.0f;
        const float a = msk * row[h * HD + la], b = msk * row[h * HD + la + half];
        const float* nw = h < H ? p.qn : p.kn;
        float sn, cs;
        sincosf((float)pos * p.inv[la], &sn, &cs);
        const float rs = 1.0f / sqrtf(wave_sum(a * a + b * b) / (float)HD + p.eps);
        if (lane < half) {
            const float x = nw[la] * (a * rs), y = nw[la + half] * (b * rs);
            const float o0 = x * cs - y * sn, o1 = y * cs + x * sn;
            if (h < H) {
                float* dst = p.qo + ((int64_t)t * H + h) * HD;
                dst[la] = o0;
                dst[la + half] = o1;
            } else {
                const int64_t off = ((int64_t)(h - H) * p.maxt + pos) * HD;
                if constexpr (BF16) {
                    reinterpret_cast<uint16_t*>(p.kc)[off + la] = f2bf16(o0);
                    reinterpret_cast<uint16_t*>(p.kc)[off + la + half] = f2bf16(o1);
                } else {
                    reinterpret_cast<float*>(p.kc)[off + la] = o0;
                    reinterpret_cast<float*>(p.kc)[off + la + half] = o1;
                }
            }
        }
    } else {
        const int64_t off = ((int64_t)(h - H - KV) * p.maxt + pos) * HD;
        for (int d = lane; d < HD; d += 64) {
            const float v = row[h * HD + d];
            if constexpr (BF16) reinterpret_cast<uint16_t*>(p.vc)[off + d] = f2bf16(v);
            else reinterpret_cast<float*>(p.vc)[off + d] = v;
        }
    }
}

// 2. the attention itself: k_prefill_attn below over S position splits
// (launch_batch_t), then k_attn_combine.

typedef short s16x4 __attribute__((ext_vector_type(4)));  // four bf16 MFMA operand bits

// ---------------------------------------------------------------------------
// Prompt attention (the blocked prefill's att_k,
// ramvi/engine/ramvi_engine/kernels/prefill_kernels.py:29-54): token r of a
// block of T at positions p0 .. p0 + T - 1 attends over positions
// 0 .. p0 + r with float32 products (the reference's input_precision='ieee')
// on the float32 matrix cores, v_mfma_f32_16x16x4_f32 (lane l: A row l%16,
// B column l%16, k = l/16; result rows 4(l/16) + 0..3, column l%16).
//
// Grid (token tiles of 16, kv heads, position splits), the last tile first
// (it has the most positions); with S > 1 splits (the batched pass: T <= 16,
// one tile) split sp covers blocks [sp nkb / S, (sp + 1) nkb / S) of the
// tile's nkb blocks of 16 positions and writes (sums, m, l) partials for
// k_attn_combine; workgroup = the G query heads of kv head g, one wave per head,
// all reading the same cache rows.  Per block of 16 positions a wave computes
// the scores transposed, S^T = K . Q^T (rows = positions, columns = its 16
// tokens), so each lane holds 4 positions of one token: the online softmax
// (running max m, rescale exp(m_old - m_new), running sum) needs two lane
// exchanges per block and no LDS.  The sums over dims and positions run in
// an order of our choosing, the same for both operands:
//   scores  MFMA t = 8a + b, k slot q: dim 32a + 8q + b, so lane l loads the
//           8 consecutive dims 32a + 8(l/16) .. +7 of its position l%16 (and
//           of its token's q) with one 16-byte (32-byte for float32) load;
//   values  O^T = V^T . P^T over output dim tiles dt: tile row r is dim
//           DT r + dt (DT = HD / 16), k slot q of MFMA j is position 4q + j,
//           so lane l loads the DT consecutive dims DT (l%16) .. of position
//           4(l/16) + j, and P^T's operand is the lane's own probability j.
// The caches are read through descriptors ending at position p0 + T, the q
// rows through one ending at row T: tokens and positions past the block
// read zeros, are masked (-inf scores) and never stored.
template <int HD, bool BF16>
__global__ __launch_bounds__(512) void k_prefill_attn(AttnParams p) {
    constexpr int EB = BF16 ? 2 : 4;    // cache bytes per value
    constexpr int NA = HD / 32;         // 8-dim score chunks per lane
    constexpr int DT = HD / 16;         // output dim tiles = value dims per lane
    constexpr int KWD = 8 * EB / 4;     // words of one 8-dim key chunk
    constexpr int VWD = DT * EB / 4;    // words of one lane's value dims
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int q4 = lane >> 4, c16 = lane & 15;
    const int H = p.n_heads, KV = p.n_kv, G = H / KV;
    const int g = blockIdx.y, h = g * G + wv;
    const int S = gridDim.z, sp = blockIdx.z;  // position splits (S > 1: T <= 16, one token tile)
    const int T = p.T;
    const int ntile = (T + 15) >> 4;
    const int t0 = (ntile - 1 - (int)blockIdx.x) * 16;
    const int tq = t0 + c16;  // this lane's token
    const int64_t p0 = *p.pos;
    float* orow = p.out + (int64_t)min(tq, T - 1) * H * HD + h * HD;
    // split partials [n_kv][S][R][HD + 2], row tq G + (h - g G) of R = T G
    float* prow =
        S > 1 ? p.part + (((int64_t)g * S + sp) * T * G + (int64_t)min(tq, T - 1) * G + wv) * (HD + 2) : nullptr;
    if (p0 < 0 || p0 + T > p.maxt) {  // a block outside the cache: zeros, as the prologue writes nothing
        if (tq < T && q4 == 0) {
            if (S == 1) {
                for (int d = 0; d < HD; ++d) orow[d] = 0.0f;
            } else {  // partials that combine to zeros: acc 0, and l = 1 on split 0 only
                for (int d = 0; d < HD; ++d) prow[d] = 0.0f;
                prow[HD] = sp == 0 ? 0.0f : -INFINITY;
                prow[HD + 1] = sp == 0 ? 1.0f : 0.0f;
            }
        }
        return;
    }
    const int n = (int)p0 + T;  // positions in the cache after the block
    const uint32_t head_bytes = (uint32_t)n * HD * EB;
    const char* kbase = reinterpret_cast<const char*>(p.kc) + (int64_t)g * p.maxt * HD * EB;
    const char* vbase = reinterpret_cast<const char*>(p.vc) + (int64_t)g * p.maxt * HD * EB;
    const __amdgpu_buffer_rsrc_t rk = attn_rsrc(kbase, head_bytes), rv = attn_rsrc(vbase, head_bytes);
    const __amdgpu_buffer_rsrc_t rq = attn_rsrc(p.qo, (uint32_t)T * H * HD * 4);

    // q of (tq, h): the B operand of the score MFMAs
    float qv[NA][8];
    {
        const int qoff = ((tq * H + h) * HD + 8 * q4) * 4;
#pragma unroll
        for (int a = 0; a < NA; ++a) {
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const auto v = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff + a * 128 + c * 16, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; ++e) qv[a][4 * c + e] = __uint_as_float(v[e]);
            }
        }
    }
    // bf16 caches: the keys and values are exact bf16, so the products run on
    // the bf16 matrix cores with q and the probabilities split into three bf16
    // parts (hi + mid + lo = the float32 value to 24 bits; every product of
    // bf16 values is exact in float32): q's parts once per tile here
    u32x4 qp[BF16 ? NA : 1][3];
    if constexpr (BF16) {
#pragma unroll
        for (int a = 0; a < NA; ++a) split3(qv[a], qp[a][0], qp[a][1], qp[a][2]);
    }
    const int last = min((int)p0 + t0 + 15, n - 1);  // last position any token of the tile sees
    // this split's blocks of 16 positions: [kb0, kb1) of the tile's nkb
    const int nkb = last / 16 + 1;
    const int kb0 = (int)((int64_t)sp * nkb / S), kb1 = (int)((int64_t)(sp + 1) * nkb / S);

    uint32_t kw[NA][KWD], vw[4][VWD];
    auto load_block = [&](int kb) {
        const int koff = ((kb * 16 + c16) * HD + 8 * q4) * EB;
#pragma unroll
        for (int a = 0; a < NA; ++a) {
#pragma unroll
            for (int c = 0; c < KWD / 4; ++c) {
                const auto v = __builtin_amdgcn_raw_buffer_load_b128(rk, koff + a * 32 * EB + c * 16, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; ++e) kw[a][4 * c + e] = v[e];
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int voff = ((kb * 16 + 4 * q4 + j) * HD + DT * c16) * EB;
            if constexpr (VWD == 2) {
                const auto v = __builtin_amdgcn_raw_buffer_load_b64(rv, voff, 0, 0);
                vw[j][0] = v[0];
                vw[j][1] = v[1];
            } else {
#pragma unroll
                for (int c = 0; c < VWD / 4; ++c) {
                    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rv, voff + c * 16, 0, 0);
#pragma unroll
                    for (int e = 0; e < 4; ++e) vw[j][4 * c + e] = v[e];
                }
            }
        }
    };
    auto word_f = [](const uint32_t* w, int i) -> float {
        if constexpr (BF16) return __uint_as_float((i & 1) ? (w[i >> 1] & 0xFFFF0000u) : (w[i >> 1] << 16));
        else return __uint_as_float(w[i]);
    };

    f32x4 o[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) o[d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;
    const int qpos = (int)p0 + tq;  // the last position this lane's token sees
    if (kb0 < kb1) load_block(kb0);
    for (int kb = kb0; kb < kb1; ++kb) {
        uint32_t kcur[NA][KWD], vcur[4][VWD];
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int i = 0; i < KWD; ++i) kcur[a][i] = kw[a][i];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < VWD; ++i) vcur[j][i] = vw[j][i];
        if (kb + 1 < kb1) load_block(kb + 1);
        // scores of positions kb 16 + 4 q4 + r for token tq
        f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (BF16) {
            // v_mfma_f32_16x16x32_bf16: A = the lane's 8 key dims 32a + 8 q4 ..
            // of position c16, B = the same dims of its token's q part
#pragma unroll
            for (int a = 0; a < NA; ++a) {
                const u32x4 ka = {kcur[a][0], kcur[a][1], kcur[a][2], kcur[a][3]};
#pragma unroll
                for (int c = 0; c < 3; ++c) s = mfma(ka, qp[a][c], s);
            }
        } else {
#pragma unroll
            for (int a = 0; a < NA; ++a)
#pragma unroll
                for (int b = 0; b < 8; ++b)
                    s = __builtin_amdgcn_mfma_f32_16x16x4f32(word_f(kcur[a], b), qv[a][b], s, 0, 0, 0);
        }
        float sc[4], pr[4];
        float mb = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int pos = kb * 16 + 4 * q4 + r;
            sc[r] = (pos <= qpos && pos < n) ? s[r] * p.scale : -INFINITY;
            mb = fmaxf(mb, sc[r]);
        }
        mb = fmaxf(mb, __shfl_xor(mb, 16));
        mb = fmaxf(mb, __shfl_xor(mb, 32));
        // finite from the first block with a position the token sees (block 0
        // for every token of an unsplit range); before it nothing accumulates
        const float mn = fmaxf(m, mb);
        const bool none = mn == -INFINITY;
        const float alpha = none ? 1.0f : expf(m - mn);
        float ls = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            pr[r] = none ? 0.0f : expf(sc[r] - mn);
            ls += pr[r];
        }
        l = l * alpha + ls;
        m = mn;
        if constexpr (BF16) {
            // v_mfma_f32_16x16x16_bf16 per output dim tile: A = dim DT c16 + d
            // of positions 4 q4 + 0..3 (from the lane's four value rows), B =
            // the lane's own probabilities of those positions, per part
            uint32_t ph[4], pm[4], pl[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                ph[j] = bf16_bits(pr[j]);
                const float r1 = pr[j] - bf16_value(ph[j]);
                pm[j] = bf16_bits(r1);
                pl[j] = bf16_bits(r1 - bf16_value(pm[j]));
            }
            const s16x4 pb[3] = {__builtin_bit_cast(s16x4, uint2{ph[0] | ph[1] << 16, ph[2] | ph[3] << 16}),
                                 __builtin_bit_cast(s16x4, uint2{pm[0] | pm[1] << 16, pm[2] | pm[3] << 16}),
                                 __builtin_bit_cast(s16x4, uint2{pl[0] | pl[1] << 16, pl[2] | pl[3] << 16})};
#pragma unroll
            for (int d = 0; d < DT; ++d) {
                o[d] *= alpha;
                const int w = d >> 1;
                const uint32_t a01 = (d & 1) ? (vcur[0][w] >> 16) | (vcur[1][w] & 0xFFFF0000u)
                                             : (vcur[0][w] & 0xFFFFu) | (vcur[1][w] << 16);
                const uint32_t a23 = (d & 1) ? (vcur[2][w] >> 16) | (vcur[3][w] & 0xFFFF0000u)
                                             : (vcur[2][w] & 0xFFFFu) | (vcur[3][w] << 16);
                const s16x4 va = __builtin_bit_cast(s16x4, uint2{a01, a23});
#pragma unroll
                for (int c = 0; c < 3; ++c) o[d] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pb[c], o[d], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int d = 0; d < DT; ++d) {
                o[d] *= alpha;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(word_f(vcur[j], d), pr[j], o[d], 0, 0, 0);
            }
        }
    }
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (S > 1) {  // the split's partial: unnormalised sums, m, l
        if (tq < T) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float* dst = prow + DT * (4 * q4 + r);
#pragma unroll
                for (int d = 0; d < DT; ++d) dst[d] = o[d][r];
            }
            if (q4 == 0) {
                prow[HD] = m;
                prow[HD + 1] = l;
            }
        }
        return;
    }
    if (tq < T) {
        // lane l holds dims DT (4 q4 + r) + dt of its token
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float* dst = orow + DT * (4 * q4 + r);
#pragma unroll
            for (int d4 = 0; d4 < DT; d4 += 4)
                *reinterpret_cast<f32x4*>(dst + d4) =
                    f32x4{o[d4][r] / l, o[d4 + 1][r] / l, o[d4 + 2][r] / l, o[d4 + 3][r] / l};
        }
    }
}

template <int HD, bool BF16>
static void launch_prefill_t(const AttnParams& p, hipStream_t st) {
    hipLaunchKernelGGL((k_qk_rope_cache<HD, BF16>), dim3(p.n_heads + 2 * p.n_kv, p.T), dim3(64), 0, st, p);
    hipLaunchKernelGGL((k_prefill_attn<HD, BF16>), dim3((p.T + 15) / 16, p.n_kv),
                       dim3(64 * (p.n_heads / p.n_kv)), 0, st, p);
}

int launch_prefill_attn(const AttnParams& p, hipStream_t st) {
    if (p.head_dim == 128) {
        if (p.kv_bf16) launch_prefill_t<128, true>(p, st);
        else launch_prefill_t<128, false>(p, st);
    } else if (p.head_dim == 64) {
        if (p.kv_bf16) launch_prefill_t<64, true>(p, st);
        else launch_prefill_t<64, false>(p, st);
    } else {
        return -1;
    }
    return 0;
}

// the batched pass (T <= 16 tokens): the prologue, then the prompt attention
// kernel over S position splits (one token tile, its G waves per kv head on
// the matrix cores), then the combine of the splits
template <int HD, bool BF16>
static void launch_batch_t(const AttnParams& p, int S, hipStream_t st) {
    hipLaunchKernelGGL((k_qk_rope_cache<HD, BF16>), dim3(p.n_heads + 2 * p.n_kv, p.T), dim3(64), 0, st, p);
    hipLaunchKernelGGL((k_prefill_attn<HD, BF16>), dim3(1, p.n_kv, S), dim3(64 * (p.n_heads / p.n_kv)), 0, st, p);
}

int launch_attn_batch(const AttnParams& p, int S, hipStream_t st) {
    if (p.T < 1 || p.T > 16) return -1;
    if (p.head_dim == 128) {
        if (p.kv_bf16) launch_batch_t<128, true>(p, S, st);
        else launch_batch_t<128, false>(p, S, st);
    } else if (p.head_dim == 64) {
        if (p.kv_bf16) launch_batch_t<64, true>(p, S, st);
        else launch_batch_t<64, false>(p, S, st);
    } else {
        return -1;
    }
    launch_combine(p, S, p.n_heads / p.n_kv, p.T * (p.n_heads / p.n_kv), st);
    return 0;
}

template <int HD, int G, bool BF16, int NT, bool QH>
static void launch_attn_nt(const AttnParams& p, int S, hipStream_t st) {
    const size_t lds = attn_lds_bytes(HD, QH ? 1 : G, NT);
    if (lds > kDefaultLds)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_rope_attn<HD, G, BF16, NT, QH>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL((k_rope_attn<HD, G, BF16, NT, QH>), dim3(QH ? p.n_heads : p.n_kv, S), dim3(NT), lds, st, p);
}

// one split over more than kAttnSpan positions: the long-span workgroup, one
// per q head (Qwen3-0.6B shape, 16 q over 8 kv heads at a 192-position cache:
// 5.10-5.15 us per layer at position 100 against 5.82 with one workgroup per
// kv head, 5.86-5.91 against 5.93-6.04 at 190; the 0.6B decode 1292 -> 1330
// tokens/s)
template <int HD, int G, bool BF16>
static void launch_attn_t(const AttnParams& p, int S, size_t, hipStream_t st) {
    if (S == 1 && p.maxt > kAttnSpan) launch_attn_nt<HD, G, BF16, kAttnLongThreads, true>(p, S, st);
    else launch_attn_nt<HD, G, BF16, kAttnThreads, false>(p, S, st);
}

template <int HD, int G>
static void launch_attn_g(const AttnParams& p, int S, size_t lds, hipStream_t st) {
    if (p.kv_bf16) launch_attn_t<HD, G, true>(p, S, lds, st);
    else launch_attn_t<HD, G, false>(p, S, lds, st);
}

template <int HD>
static int launch_attn_hd(const AttnParams& p, int G, int S, size_t lds, hipStream_t st) {
    switch (G) {
        case 1: launch_attn_g<HD, 1>(p, S, lds, st); return 0;
        case 2: launch_attn_g<HD, 2>(p, S, lds, st); return 0;
        case 4: launch_attn_g<HD, 4>(p, S, lds, st); return 0;
        case 8: launch_attn_g<HD, 8>(p, S, lds, st); return 0;
    }
    return -1;
}

int launch_attn(const AttnParams& pa, int S, hipStream_t st) {
    AttnParams p = pa;
    p.smul = div_mul(S);
    const int G = p.n_heads / p.n_kv;
    const bool longspan = S == 1 && p.maxt > kAttnSpan;  // one workgroup per q head
    const size_t lds = attn_lds_bytes(p.head_dim, longspan ? 1 : G, longspan ? kAttnLongThreads : kAttnThreads);
    int rc = p.head_dim == 128 ? launch_attn_hd<128>(p, G, S, lds, st)
                               : (p.head_dim == 64 ? launch_attn_hd<64>(p, G, S, lds, st) : -1);
    if (rc) return rc;
    launch_combine(p, S, G, G, st);
    return 0;
}

}  // namespace rv12
