/* C restatement of the reference 12-bit codec and of the CPU linear paths.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (as a fast checker), by
 * __graft_entry__.smoke() and by bench.py's CPU-baseline leg.  The product
 * path never links it.
 *
 *  rvo_compress      codec encode (ramvi/engine/ramvi_engine/kernels/wcomp.py:13-32)
 *  rvo_decode        codec decode to float32 (wcomp.py:35-44, before .bfloat16())
 *  rvo_gemv_bf16     Y[t] (+)= W X[t] with W in bf16 bits, fp32 sums, one output row
 *                    per task: the reference CPU layer's matmat16
 *                    (ramvi/engine/ramvi_engine/cpu/cpu_layer.py:35-48)
 *  rvo_gemv_12bit    the same product straight from the 12-bit codec: decode one
 *                    CH-chunk of a row to fp32, dot it, then add the row's
 *                    exceptions (the order of wcomp.py:80-108), with the MODE /
 *                    RMS prologue of wcomp.py:57-86 (the block decode + dot of
 *                    the reference's native CPU path, native/qmm.cpp:195-212).
 *  rvo_rms_rows, rvo_qk_rope_attn, rvo_silu_mul
 *                    the reference CPU layer's other steps
 *                    (cpu/cpu_layer.py:51-59, 62-131, 134-140): with
 *                    rvo_gemv_bf16 they make CpuLayer.__call__ (:155-175).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf16f(uint16_t u) {
    uint32_t b = (uint32_t)u << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

int rvo_abi(void) { return 1; }

/* first window start b in [0, 241] maximising #{e in [b, b+14]} */
int rvo_choose_base(const uint16_t* w, int64_t count) {
    int64_t cnt[256] = {0};
    for (int64_t i = 0; i < count; i++) cnt[(w[i] >> 7) & 0xFF]++;
    int64_t best = -1;
    int base = 0;
    for (int b = 0; b <= 241; b++) {
        int64_t s = 0;
        for (int j = 0; j < 15; j++) s += cnt[b + j];
        if (s > best) { best = s; base = b; }
    }
    return base;
}

/* Encode W[N, K] (bf16 bits).  Exceptions are written in row-major order into
 * er/ec/ev (capacity cap); returns the exception count, or -1 on bad shape,
 * -2 when cap is too small (count still computed). */
int64_t rvo_compress(const uint16_t* w, int N, int K, int CH, uint8_t* m8, uint8_t* e4,
                     int32_t* rp, int32_t* er, int32_t* ec, float* ev, int64_t cap, int* base_out) {
    if (N < 1 || K < 1 || CH < 2 || (CH & 1) || K % CH) return -1;
    int base = rvo_choose_base(w, (int64_t)N * K);
    *base_out = base;
    int64_t E = 0;
    int half = CH / 2;
    rp[0] = 0;
    for (int n = 0; n < N; n++) {
        const uint16_t* row = w + (int64_t)n * K;
        for (int k = 0; k < K; k++) {
            uint16_t b = row[k];
            int e = (b >> 7) & 0xFF;
            int code = e - base;
            if (code < 0 || code > 14) {
                code = 15;
                if (E < cap) { er[E] = n; ec[E] = k; ev[E] = bf16f(b); }
                E++;
            }
            m8[(int64_t)n * K + k] = (uint8_t)(((b >> 15) << 7) | (b & 0x7F));
            int c = k / CH, i = k % CH;
            uint8_t* byte = e4 + (int64_t)n * (K / 2) + (int64_t)c * half + (i % half);
            if (i < half) *byte = (uint8_t)((*byte & 0xF0) | code);
            else *byte = (uint8_t)((*byte & 0x0F) | (code << 4));
        }
        rp[n + 1] = (int32_t)E;
    }
    return E > cap ? -2 : E;
}

/* Decode to float32 W[N, K] (exceptions scattered last). */
void rvo_decode(const uint8_t* m8, const uint8_t* e4, int base, const int32_t* er, const int32_t* ec,
                const float* ev, int64_t E, int N, int K, int CH, float* out) {
    int half = CH / 2;
    for (int n = 0; n < N; n++) {
        for (int k = 0; k < K; k++) {
            int c = k / CH, i = k % CH;
            uint8_t byte = e4[(int64_t)n * (K / 2) + (int64_t)c * half + (i % half)];
            int code = i < half ? (byte & 15) : (byte >> 4);
            uint32_t m = m8[(int64_t)n * K + k];
            uint32_t bits = code == 15 ? 0u : (((m >> 7) << 31) | ((uint32_t)(code + base) << 23) | ((m & 0x7F) << 16));
            memcpy(out + (int64_t)n * K + k, &bits, 4);
        }
    }
    for (int64_t j = 0; j < E; j++) out[(int64_t)er[j] * K + ec[j]] = ev[j];
}

/* matmat16: Y[t, n] (+)= sum_k bf(W[n, k]) * X[t, k]  (fp32 sums; X rows K apart) */
void rvo_gemv_bf16(const uint16_t* W, const float* X, float* Y, int N, int K, int T, int add, int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
    for (int n = 0; n < N; n++) {
        const uint16_t* row = W + (int64_t)n * K;
        for (int t = 0; t < T; t++) {
            const float* x = X + (int64_t)t * K;
            float s = 0.0f;
#pragma omp simd reduction(+ : s)
            for (int k = 0; k < K; k++) s += bf16f(row[k]) * x[k];
            if (add) Y[(int64_t)t * N + n] += s;
            else Y[(int64_t)t * N + n] = s;
        }
    }
}

/* x'[t, k] for the MODE / RMS prologue (T rows, X rows xs apart). */
static void prologue(const float* X, int xs, int K, int T, int mode, const uint16_t* lnw, float eps, float* xp) {
    for (int t = 0; t < T; t++) {
        const float* x = X + (int64_t)t * xs;
        float rs = 1.0f;
        if (lnw) {
            float s = 0.0f;
            for (int k = 0; k < K; k++) s += x[k] * x[k];
            rs = 1.0f / sqrtf(s / (float)K + eps);
        }
        for (int k = 0; k < K; k++) {
            float v = mode == 2 ? x[k] / (1.0f + expf(-x[k])) * x[K + k] : x[k];
            if (lnw) v = bf16f(lnw[k]) * (v * rs);
            xp[(int64_t)t * K + k] = v;
        }
    }
}

/* 12-bit decode + product: Y[t] (=|+=) W_dec x'[t]; mode as in the reference. */
int rvo_gemv_12bit(const uint8_t* m8, const uint8_t* e4, int base, const int32_t* rp, const int32_t* ec,
                   const float* ev, const float* X, float* Y, const uint16_t* lnw, float eps, int N, int K,
                   int CH, int T, int mode, int threads) {
    if (N < 1 || K < 1 || CH < 2 || K % CH || T < 1 || T > 16 || mode < 0 || mode > 2) return -1;
    int xs = mode == 2 ? 2 * K : K;
    float* xp = (float*)malloc(sizeof(float) * (size_t)T * K);
    if (!xp) return -3;
    prologue(X, xs, K, T, mode, lnw, eps, xp);
    int half = CH / 2;
    const uint32_t ub = (uint32_t)base;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel
#endif
    {
        /* the decoded chunk as float bits; both loops below vectorise */
        uint32_t* wb = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)CH);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int n = 0; n < N; n++) {
            float acc[16] = {0};
            const uint8_t* mr = m8 + (int64_t)n * K;
            const uint8_t* er = e4 + (int64_t)n * (K / 2);
            for (int c = 0; c < K / CH; c++) {
                const uint8_t* eb = er + (int64_t)c * half;
                const uint8_t* mb = mr + (int64_t)c * CH;
                for (int i = 0; i < half; i++) {
                    const uint32_t byte = eb[i], c0 = byte & 15u, c1 = byte >> 4;
                    const uint32_t m0 = mb[i], m1 = mb[half + i];
                    const uint32_t b0 = ((m0 >> 7) << 31) | ((c0 + ub) << 23) | ((m0 & 0x7Fu) << 16);
                    const uint32_t b1 = ((m1 >> 7) << 31) | ((c1 + ub) << 23) | ((m1 & 0x7Fu) << 16);
                    wb[i] = c0 == 15u ? 0u : b0;
                    wb[half + i] = c1 == 15u ? 0u : b1;
                }
                for (int t = 0; t < T; t++) {
                    const float* x = xp + (int64_t)t * K + (int64_t)c * CH;
                    float s = 0.0f;
#pragma omp simd reduction(+ : s)
                    for (int i = 0; i < CH; i++) {
                        float w;
                        memcpy(&w, wb + i, 4);
                        s += w * x[i];
                    }
                    acc[t] += s;
                }
            }
            for (int j = rp[n]; j < rp[n + 1]; j++)
                for (int t = 0; t < T; t++) acc[t] += ev[j] * xp[(int64_t)t * K + ec[j]];
            for (int t = 0; t < T; t++) {
                if (mode == 0) Y[(int64_t)t * N + n] = acc[t];
                else Y[(int64_t)t * N + n] += acc[t];
            }
        }
        free(wb);
    }
    free(xp);
    return 0;
}

/* rms_rows (cpu_layer.py:51-59): out[t] = w * (X[t] / sqrt(mean(X[t]^2) + eps)),
 * sequential fp32 sums */
void rvo_rms_rows(const float* X, const float* w, float* out, int T, int D, float eps) {
    for (int t = 0; t < T; t++) {
        const float* x = X + (int64_t)t * D;
        float s = 0.0f;
        for (int i = 0; i < D; i++) s += x[i] * x[i];
        const float r = 1.0f / sqrtf(s / (float)D + eps);
        for (int i = 0; i < D; i++) out[(int64_t)t * D + i] = w[i] * (x[i] * r);
    }
}

/* head RMSNorm + rotate-half RoPE at position p of one head (HD values at
 * src, weights nw) into dst (cpu_layer.py:70-83, 95-105) */
static void norm_rope(const float* src, const float* nw, const float* inv, int p, int HD, float eps, float* dst) {
    const int half = HD / 2;
    float s = 0.0f;
    for (int d = 0; d < HD; d++) s += src[d] * src[d];
    const float r = 1.0f / sqrtf(s / (float)HD + eps);
    for (int d = 0; d < half; d++) {
        const float ang = (float)p * inv[d];
        const float c = cosf(ang), sn = sinf(ang);
        const float a = nw[d] * (src[d] * r), b = nw[d + half] * (src[d + half] * r);
        dst[d] = a * c - b * sn;
        dst[d + half] = b * c + a * sn;
    }
}

/* qk_rope_attn (cpu_layer.py:62-131): q/k head norms and RoPE, k and v of the
 * T rows into the float32 caches Kc / Vc [KV][maxt][HD] at positions
 * pos0..pos0+T-1, then per (row, head) the causal softmax attention over
 * positions 0..pos0+t (max-subtracted exponentials, fp32 sums) into out
 * [T][H*HD].  QKV rows hold q (H heads), k (KV), v (KV). */
void rvo_qk_rope_attn(const float* QKV, const float* qn, const float* kn, const float* inv, int pos0, float* Kc,
                      float* Vc, int maxt, float* out, int T, int H, int KV, int HD, float eps, int threads) {
    const int G = H / KV, W = (H + 2 * KV) * HD;
    for (int t = 0; t < T; t++) {
        const int p = pos0 + t;
        const float* row = QKV + (int64_t)t * W;
        for (int g = 0; g < KV; g++) {
            norm_rope(row + (H + g) * HD, kn, inv, p, HD, eps, Kc + ((int64_t)g * maxt + p) * HD);
            memcpy(Vc + ((int64_t)g * maxt + p) * HD, row + (H + KV + g) * HD, sizeof(float) * HD);
        }
    }
    const float scale = 1.0f / sqrtf((float)HD);
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel
#endif
    {
        float* q = (float*)malloc(sizeof(float) * HD);
        float* sc = (float*)malloc(sizeof(float) * (pos0 + T));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int th = 0; th < T * H; th++) {
            const int t = th / H, h = th % H, g = h / G, p = pos0 + t, n = p + 1;
            norm_rope(QKV + (int64_t)t * W + h * HD, qn, inv, p, HD, eps, q);
            float m = -1e30f;
            for (int j = 0; j < n; j++) {
                const float* k = Kc + ((int64_t)g * maxt + j) * HD;
                float s = 0.0f;
                for (int d = 0; d < HD; d++) s += q[d] * k[d];
                s *= scale;
                sc[j] = s;
                if (s > m) m = s;
            }
            float l = 0.0f;
            for (int j = 0; j < n; j++) {
                sc[j] = expf(sc[j] - m);
                l += sc[j];
            }
            float* o = out + (int64_t)t * H * HD + h * HD;
            for (int d = 0; d < HD; d++) o[d] = 0.0f;
            for (int j = 0; j < n; j++) {
                const float w = sc[j] / l;
                const float* v = Vc + ((int64_t)g * maxt + j) * HD;
                for (int d = 0; d < HD; d++) o[d] += w * v[d];
            }
        }
        free(q);
        free(sc);
    }
}

/* silu_mul (cpu_layer.py:134-140): M[t, i] = g / (1 + exp(-g)) * u, g = GU[t, i],
 * u = GU[t, FF + i] */
void rvo_silu_mul(const float* GU, float* M, int T, int FF) {
    for (int t = 0; t < T; t++)
        for (int i = 0; i < FF; i++) {
            const float g = GU[(int64_t)t * 2 * FF + i];
            M[(int64_t)t * FF + i] = g / (1.0f + expf(-g)) * GU[(int64_t)t * 2 * FF + FF + i];
        }
}
