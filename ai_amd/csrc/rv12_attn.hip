// Decode-step attention for one layer (one token), gfx950: the companion of
// the 12-bit linears in a decode step (replaces rope_attn_k,
// ramvi/engine/ramvi_engine/kernels/tkernels.py:164-213).
//
// Grid (KV heads, splits), 256 threads.  Workgroup (g, sp):
//   0. first of all the step's own q/k/v values and then every cache value the
//      workgroup reads are loaded: the key row of one position per thread and
//      the values of 32 positions per wave (a split covers at most 128
//      positions), so the kernel waits for memory about once, and the head
//      transforms below run while the cache values are still in flight;
//   1. the G query heads of group g and the step's key and value are read
//      from the qkv linear's output; q and k get their head RMSNorm and the
//      rotate-half RoPE at position pos (angle pos * inv[i], precise sin/cos),
//      one wave per head;
//      k and v are rounded to the cache dtype (as the reference rounds them,
//      tkernels.py:187-190); split 0 writes them into the cache at pos;
//   2. scores s[i][j] = scale * q_i . K[j] for the split's positions
//      j in [lo, hi) of 0..pos, one position per thread; j == pos uses the
//      step's own k (so no workgroup reads the slot split 0 writes);
//   3. per head the split's max m and sum l of exp(s - m);
//   4. acc[i][d] = sum_j exp(s[i][j] - m_i) V[j][d], each wave over its 32
//      positions from registers, the waves added through LDS;
//   5. one split: out = acc / l; several: (acc, m, l) partials, combined by
//      k_attn_combine in split order.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "rv12_internal.h"

namespace rv12 {

constexpr int kAttnThreads = 256;

__device__ __forceinline__ float bf16f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f2bf16(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t attn_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)0x00020000);
}

// Raw cache words one thread keeps between the loads at kernel start and their
// first use (no conversion on load, so no wait): a key row of HD values, and
// DPL = HD / 64 values of one position at a lane's dims.
template <int HD, bool BF16>
struct KRow {
    static constexpr int N = BF16 ? HD / 8 : HD / 4;  // 16-byte words
    uint32_t w[N][4];
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, int off) {
#pragma unroll
        for (int c = 0; c < N; ++c) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off + c * 16, 0, 0);
            w[c][0] = v[0];
            w[c][1] = v[1];
            w[c][2] = v[2];
            w[c][3] = v[3];
        }
    }
    __device__ __forceinline__ float at(int i) const {  // value i of the row
        if constexpr (BF16) {
            const uint32_t u = w[i >> 3][(i >> 1) & 3];
            return __uint_as_float((i & 1) ? (u & 0xFFFF0000u) : (u << 16));
        } else {
            return __uint_as_float(w[i >> 2][i & 3]);
        }
    }
};

template <int HD, bool BF16>
__device__ __forceinline__ void load_vals(__amdgpu_buffer_rsrc_t r, int off, uint32_t (&u)[2]) {
    constexpr int DPL = HD / 64;
    if constexpr (BF16 && DPL == 2) {
        u[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    } else if constexpr (BF16) {
        u[0] = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
    } else if constexpr (DPL == 2) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
        u[0] = v[0];
        u[1] = v[1];
    } else {
        u[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    }
}

template <int HD, bool BF16>
__device__ __forceinline__ float val_at(const uint32_t (&u)[2], int e) {
    if constexpr (BF16) return __uint_as_float(e ? (u[0] & 0xFFFF0000u) : (u[0] << 16));
    else return __uint_as_float(u[e]);
}

__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// RMSNorm (weight pair wa, wb) and rotate-half RoPE (cos c, sin sn) of one
// head held by one wave: lane l < HD/2 holds the pair (a, b) = (x[l], x[l + HD/2])
// (the other lanes hold zeros), so the whole transform needs no barrier.
template <int HD>
__device__ __forceinline__ void norm_rope_wave(float a, float b, float wa, float wb, float c, float sn, float eps,
                                               float* dst, int lane) {
    constexpr int half = HD / 2;
    const float rs = 1.0f / sqrtf(wave_sum(a * a + b * b) / (float)HD + eps);
    if (lane < half) {
        const float x = wa * (a * rs), y = wb * (b * rs);
        dst[lane] = x * c - y * sn;
        dst[lane + half] = y * c + x * sn;
    }
}

template <int HD, int G, bool BF16>
__global__ __launch_bounds__(kAttnThreads) void k_rope_attn(AttnParams p) {
    extern __shared__ float lds[];
    constexpr int NW = kAttnThreads / 64;
    constexpr int PW = kAttnSpan / NW;  // positions per wave in the value sum
    constexpr int DPL = HD / 64;        // value dims per lane
    const int g = blockIdx.x, sp = blockIdx.y, S = gridDim.y;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int H = p.n_kv * G;
    const int64_t pos = *p.pos;
    float* qs = lds;                   // [G][HD]
    float* kn = qs + G * HD;           // [HD] step key (normed, roped, rounded)
    float* vn = kn + HD;               // [HD] step value (rounded)
    float* red = vn + HD;              // [NW][G] per-wave maxima / sums
    float* stat = red + NW * G;        // [2 G] m, l
    float* sc = stat + 2 * G;          // [G][kAttnSpan] scores, then weights
    float* wacc = sc + G * kAttnSpan;  // [NW][G][HD] per-wave value sums
    if (pos < 0 || pos >= p.maxt) {    // a position outside the cache: defined output, no access
        for (int o = t; o < G * HD; o += kAttnThreads) {
            const int i = o / HD, d = o % HD;
            if (S == 1) p.out[(g * G + i) * HD + d] = 0.0f;
            else p.part[(((int64_t)(g * G + i) * S + sp) * (HD + 2)) + d] = 0.0f;
        }
        if (S > 1 && t < G) {
            float* pp = p.part + ((int64_t)(g * G + t) * S + sp) * (HD + 2);
            pp[HD] = sp == 0 ? 0.0f : -INFINITY;
            pp[HD + 1] = sp == 0 ? 1.0f : 0.0f;
        }
        return;
    }
    const int64_t n = pos + 1;
    const int64_t lo = sp * n / S, hi = (sp + 1) * n / S;  // hi - lo <= kAttnSpan (host)
    const int span = (int)(hi - lo);
    const int64_t row0 = (int64_t)g * p.maxt * HD;

    // ---- 0. every cache value this workgroup reads, loaded first: thread t
    // the key row of position lo + t, wave w the values of positions
    // lo + PW w .. lo + PW w + PW - 1 at its lanes' dims.  The loads go through
    // descriptors that end at position pos: the step's own slot (written by
    // split 0, taken from the qkv output instead) and anything beyond read as
    // zeros without a memory access.
    // the step's values: wave w the heads w, w + NW, .. of q (0..G-1) and k (G),
    // lane l < HD/2 the pair (l, l + HD/2), thread d < HD the value v[d]
    constexpr int half = HD / 2, HPW = (G + NW) / NW;
    const int la = lane < half ? lane : 0;
    const __amdgpu_buffer_rsrc_t qr = attn_rsrc(p.qkv, (uint32_t)((H + 2 * p.n_kv) * HD * 4));
    float qa[HPW], qb[HPW];
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
        const int i = min(wave + j * NW, G);
        const int off = ((i < G ? g * G + i : H + g) * HD + la) * 4;
        const float msk = lane < half ? 1.0f : 0.0f;
        qa[j] = msk * __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(qr, off, 0, 0));
        qb[j] = msk * __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(qr, off + half * 4, 0, 0));
    }
    const float vown = __uint_as_float(
        __builtin_amdgcn_raw_buffer_load_b32(qr, ((H + p.n_kv + g) * HD + (t < HD ? t : 0)) * 4, 0, 0));
    const float wqa = p.qn[la], wqb = p.qn[la + half], wka = p.kn[la], wkb = p.kn[la + half], iv = p.inv[la];

    constexpr int EB = BF16 ? 2 : 4;
    const char* kbase = reinterpret_cast<const char*>(p.kc) + row0 * EB;
    const char* vbase = reinterpret_cast<const char*>(p.vc) + row0 * EB;
    const __amdgpu_buffer_rsrc_t kr = attn_rsrc(kbase, (uint32_t)(pos * HD * EB));
    const __amdgpu_buffer_rsrc_t vr = attn_rsrc(vbase, (uint32_t)(pos * HD * EB));
    KRow<HD, BF16> krow;
    krow.load(kr, (int)((lo + t) * HD * EB));
    uint32_t vraw[PW][2];
#pragma unroll
    for (int r = 0; r < PW; ++r) load_vals<HD, BF16>(vr, (int)((lo + wave * PW + r) * HD + lane * DPL) * EB, vraw[r]);

    // ---- 1. the step's q (G heads) and k, one wave per head; v as read
    float sn, cs;
    sincosf((float)pos * iv, &sn, &cs);
#pragma unroll
    for (int j = 0; j < HPW; ++j) {
        const int i = wave + j * NW;
        if (i < G) norm_rope_wave<HD>(qa[j], qb[j], wqa, wqb, cs, sn, p.eps, qs + i * HD, lane);
        else if (i == G) norm_rope_wave<HD>(qa[j], qb[j], wka, wkb, cs, sn, p.eps, kn, lane);
    }
    if (t < HD) vn[t] = vown;
    __syncthreads();
    if (t < HD) {
        if constexpr (BF16) {
            const uint16_t kb = f2bf16(kn[t]), vb = f2bf16(vn[t]);
            kn[t] = bf16f(kb);
            vn[t] = bf16f(vb);
            if (sp == 0) {
                reinterpret_cast<uint16_t*>(p.kc)[row0 + pos * HD + t] = kb;
                reinterpret_cast<uint16_t*>(p.vc)[row0 + pos * HD + t] = vb;
            }
        } else if (sp == 0) {
            reinterpret_cast<float*>(p.kc)[row0 + pos * HD + t] = kn[t];
            reinterpret_cast<float*>(p.vc)[row0 + pos * HD + t] = vn[t];
        }
    }
    __syncthreads();

    // ---- 2. scores, one position per thread
    float mloc[G];
#pragma unroll
    for (int i = 0; i < G; ++i) mloc[i] = -INFINITY;
    if (t < span) {
        const bool own = lo + t == pos;
#pragma unroll
        for (int i = 0; i < G; ++i) {
            float s = 0.0f;
#pragma unroll
            for (int c = 0; c < HD; c += 4) {
                const float4 q = *reinterpret_cast<const float4*>(qs + i * HD + c);
                if (own) {
                    s = fmaf(q.x, kn[c], s);
                    s = fmaf(q.y, kn[c + 1], s);
                    s = fmaf(q.z, kn[c + 2], s);
                    s = fmaf(q.w, kn[c + 3], s);
                } else {
                    s = fmaf(q.x, krow.at(c), s);
                    s = fmaf(q.y, krow.at(c + 1), s);
                    s = fmaf(q.z, krow.at(c + 2), s);
                    s = fmaf(q.w, krow.at(c + 3), s);
                }
            }
            s *= p.scale;
            sc[i * kAttnSpan + t] = s;
            mloc[i] = s;
        }
    }

    // ---- 3. per-head max, then the weights exp(s - m) and their sum
#pragma unroll
    for (int i = 0; i < G; ++i) {
        const float m = wave_max(mloc[i]);
        if (lane == 0) red[wave * G + i] = m;
    }
    __syncthreads();
    if (t < G) {
        float m = red[t];
        for (int w = 1; w < NW; ++w) m = fmaxf(m, red[w * G + t]);
        stat[t] = m;
    }
    __syncthreads();
    float lloc[G];
#pragma unroll
    for (int i = 0; i < G; ++i) {
        float e = 0.0f;
        if (t < span) {
            e = expf(sc[i * kAttnSpan + t] - stat[i]);
            sc[i * kAttnSpan + t] = e;
        }
        lloc[i] = wave_sum(e);
    }
    __syncthreads();  // every thread has read stat[] and red[] of the max step
#pragma unroll
    for (int i = 0; i < G; ++i)
        if (lane == 0) red[wave * G + i] = lloc[i];
    __syncthreads();
    if (t < G) {
        float l = 0.0f;
        for (int w = 0; w < NW; ++w) l += red[w * G + t];
        stat[G + t] = l;
    }

    // ---- 4. weighted values: wave w sums its PW positions from registers
    // for every head at its lanes' dims, then the waves are added
    float acc[G][DPL];
#pragma unroll
    for (int i = 0; i < G; ++i)
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[i][e] = 0.0f;
    const int wv = __builtin_amdgcn_readfirstlane(wave);  // wave-uniform: scalar loop bounds
    float vnl[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) vnl[e] = vn[lane * DPL + e];
#pragma unroll
    for (int r = 0; r < PW; ++r) {
        const int jj = wv * PW + r;
        if (jj >= span) break;
        const bool own = lo + jj == pos;
#pragma unroll
        for (int i = 0; i < G; ++i) {
            const float w8 = sc[i * kAttnSpan + jj];
#pragma unroll
            for (int e = 0; e < DPL; ++e)
                acc[i][e] = fmaf(w8, own ? vnl[e] : val_at<HD, BF16>(vraw[r], e), acc[i][e]);
        }
    }
#pragma unroll
    for (int i = 0; i < G; ++i)
#pragma unroll
        for (int e = 0; e < DPL; ++e) wacc[(wave * G + i) * HD + lane * DPL + e] = acc[i][e];
    __syncthreads();

    // ---- 5. output or partials
    for (int o = t; o < G * HD; o += kAttnThreads) {
        const int i = o / HD, d = o % HD;
        float v = 0.0f;
        for (int w = 0; w < NW; ++w) v += wacc[(w * G + i) * HD + d];
        if (S == 1) p.out[(g * G + i) * HD + d] = v / stat[G + i];
        else p.part[((int64_t)(g * G + i) * S + sp) * (HD + 2) + d] = v;
    }
    if (S > 1 && t < G) {
        float* pp = p.part + ((int64_t)(g * G + t) * S + sp) * (HD + 2);
        pp[HD] = stat[t];
        pp[HD + 1] = stat[G + t];
    }
}

// combine the splits of each head: M = max m_s, out = sum acc_s e^(m_s - M) / sum l_s e^(m_s - M);
// one workgroup per head, every partial loaded at once (a descriptor over the
// head's S partials reads zeros beyond them)
__global__ __launch_bounds__(128) void k_attn_combine(const float* __restrict__ part, float* __restrict__ out, int S, int HD) {
    const int h = blockIdx.x, d = threadIdx.x;
    const int stride = (HD + 2) * 4;
    const __amdgpu_buffer_rsrc_t r = attn_rsrc(part + (int64_t)h * S * (HD + 2), (uint32_t)(S * stride));
    float a[kMaxSplits], m[kMaxSplits], l[kMaxSplits];
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s) {
        a[s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, s * stride + d * 4, 0, 0));
        const auto ml = __builtin_amdgcn_raw_buffer_load_b64(r, s * stride + HD * 4, 0, 0);
        m[s] = __uint_as_float(ml[0]);
        l[s] = __uint_as_float(ml[1]);
    }
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s)
        if (s < S) M = fmaxf(M, m[s]);
    float num = 0.0f, den = 0.0f;
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s) {
        const float w = (s < S && l[s] > 0.0f) ? expf(m[s] - M) : 0.0f;
        num = fmaf(a[s], w, num);
        den = fmaf(l[s], w, den);
    }
    out[h * HD + d] = num / den;
}

template <int HD, int G, bool BF16>
static void launch_attn_t(const AttnParams& p, int S, size_t lds, hipStream_t st) {
    if (lds > kDefaultLds)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_rope_attn<HD, G, BF16>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL((k_rope_attn<HD, G, BF16>), dim3(p.n_kv, S), dim3(kAttnThreads), lds, st, p);
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

int launch_attn(const AttnParams& p, int S, hipStream_t st) {
    const int G = p.n_heads / p.n_kv;
    const size_t lds = attn_lds_bytes(p.head_dim, G);
    int rc = p.head_dim == 128 ? launch_attn_hd<128>(p, G, S, lds, st)
                               : (p.head_dim == 64 ? launch_attn_hd<64>(p, G, S, lds, st) : -1);
    if (rc) return rc;
    if (S > 1) hipLaunchKernelGGL(k_attn_combine, dim3(p.n_heads), dim3(p.head_dim), 0, st, p.part, p.out, S, p.head_dim);
    return 0;
}

}  // namespace rv12
