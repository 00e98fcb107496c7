// Shared declarations of the rv12 kernels and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "rv12.h"

namespace rv12 {

struct LinearParams {
    const uint32_t* tiles;
    const int32_t* rp;
    const int32_t* er;
    const int32_t* ec;
    const float* ev;
    const float* x;
    float* y;
    const uint16_t* lnw;
    const int32_t* rbase;  // exponent window start of each row
    float* part;           // split partials [splits][T][npad]
    float* ssq;            // split sums of squares [splits][T]
    float* amv = nullptr;    // fused greedy pick (vector kernel, one split): per token and
    int32_t* ami = nullptr;  // workgroup the largest output and its row, [T][workgroups]
    int N, K, npad, mode, xs;
    int store_y = 1;  // 0: the vector kernel's fused greedy pick without logits (y is then only read)
    int64_t n_exc;
    float eps;
};

// scale exponent of the h values of the Q16 layout: h << 16 read as a float
// is the weight times 2^-sc
__host__ __device__ inline int scale_exp(int base) { return base > 0 ? base - 1 : 0; }

constexpr int kDepth = 8;          // weight steps in flight per wave
constexpr int kMaxThreads = 1024;  // 16 waves
constexpr int kMaxSplits = 64;
constexpr int kReduceBatchMax = 16;  // splits the reduce pass loads at once
constexpr int kMaxWaves = 16;
constexpr size_t kMaxLds = 163840;  // LDS bytes of one gfx950 workgroup (160 KB)
constexpr size_t kDefaultLds = 65536;  // above this a kernel needs hipFuncAttributeMaxDynamicSharedMemorySize
constexpr int kMaxK = 1 << 20;             // keeps every 32-bit buffer offset of a workgroup in range
constexpr int64_t kMaxExc = (int64_t)1 << 28;  // exception entries of one matrix (read through 32-bit buffer ranges)
constexpr int kMaxVectorTokens = 4;  // k_gemv (vector FMA) serves 1..4 tokens

// --- vector-FMA linear (k_gemv), 1..4 tokens
// K steps of the largest split
inline int split_steps(int K, int splits) { return (K / 32 + splits - 1) / splits; }

// float4 activation chunks per thread the kernel keeps in registers (loaded
// before the weight prefetch; the rest of the split's columns are staged
// after it).  Two from 3 tokens on (one before: 8B qkv at 4 tokens 11.41 ->
// 10.21 us, 8B o 8.79 -> 7.94, 14B qkv 14.36 -> 13.43; no spill, the
// one-row-block variants at most 120 VGPRs of their 128); three at 3 tokens
// measured within a few percent either way.
__host__ __device__ constexpr int gemv_chunks(int T) { return T == 1 ? 6 : (T == 2 ? 3 : 2); }

inline size_t gemv_lds_bytes(int K, int T, int rb, int waves, int splits) {
    const size_t krange = (size_t)split_steps(K, splits) * 32;
    return 4 * ((size_t)T * krange + (size_t)waves * rb * T * 16 + (size_t)waves * 64 * T + (size_t)waves * T +
                (size_t)waves + (size_t)waves * T);
}

// waves per workgroup the kernel is built for (its register budget)
__host__ __device__ constexpr int gemv_max_waves(int rb) { return rb == 1 ? 16 : 8; }

// weight steps in flight per wave.  At one token 6, 4 with the 2K
// silu(g)*u activations and 8 for the one-row-block RMS variant (many rounds
// of workgroups per CU), measured per Qwen3-8B shape; at two tokens 6 (it beat
// 8 on every shape: 14B o 12.28 -> 11.93, gate/up 28.7 -> 28.1), above 8.
// The shallow form (4) for workgroups of 8 or more waves, at one token where
// their first weight loads reach kGemvPrefetchMax: the late waves wait at the
// issue of their first loads, behind the CU's misses in flight (8B qkv, 2 row
// blocks x 8 waves: one token 9.63 us at 6, 9.02 at 4; two tokens 9.61 ->
// 8.81; 14B o at three tokens 12.96 -> 11.10, 16 waves at four 20.27 ->
// 17.44; one row block of 8 waves: 14B gate/up at two tokens 27.8 -> 26.0, 8B
// o at three 8.89 -> 7.79, 0.6B qkv with RMS at one 4.79 -> 4.09).  With 4
// waves the deep form stays (2 row blocks at four tokens: 14B o 18.1 us deep,
// 20.2 shallow).
__host__ __device__ constexpr int gemv_depth(int T, int rb, bool m2, bool ln, bool shallow) {
    return shallow ? 4 : (T > 2 ? kDepth : (T == 2 ? 6 : (m2 ? 4 : (ln && rb == 1 ? kDepth : 6))));
}
constexpr size_t kGemvPrefetchMax = 48 * 1024;  // bytes of one workgroup's first weight loads
// (only where it changes the depth, so that a variant whose deep form is
// already 4 steps keeps one instantiation)
inline bool gemv_shallow(int T, int rb, int waves, bool m2, bool ln) {
    const int d = gemv_depth(T, rb, m2, ln, false);
    return d > 4 && waves >= 8 && (T > 1 || (size_t)waves * rb * d * 768 /* one step tile */ >= kGemvPrefetchMax);
}

// launch shape fits the kernel's register budget and LDS
inline bool gemv_fits(int K, int T, int rb, int waves, int splits) {
    return waves <= gemv_max_waves(rb) && waves * 64 >= rb * 16 * T &&
           gemv_lds_bytes(K, T, rb, waves, splits) <= kMaxLds;
}

// every activation column of the split is loaded before the weight prefetch
inline bool gemv_prefetch_all(int K, int T, int waves, int splits) {
    return (size_t)split_steps(K, splits) * 32 <= (size_t)4 * gemv_chunks(T) * waves * 64;
}

// --- MFMA linear (k_gemm), 1..16 tokens
constexpr size_t kGemmMaxLds = kMaxLds;
constexpr int kGemmMaxWaves = 8;
// token columns the kernel stages for T tokens: 4, 8 or 16
__host__ __device__ constexpr int gemm_tokens(int T) { return T <= 4 ? 4 : (T <= 8 ? 8 : 16); }
inline size_t gemm_lds_bytes(int K, int rbw, int waves, int splits, int T) {
    const size_t steps = (size_t)split_steps(K, splits);
    // parts (3 x 4 k-groups x TP tokens x 16 bytes per step), exception sums,
    // sums of squares, range flags, slow-path exponents
    return steps * 3 * 64 * (size_t)gemm_tokens(T) + (size_t)waves * rbw * 16 * 16 * 4 + 16 * 4 * (size_t)waves +
           4 * (size_t)waves + 16 * 4 * (size_t)waves;
}
inline bool gemm_fits(int K, int T, int rbw, int waves, int splits) {
    return waves <= kGemmMaxWaves && gemm_lds_bytes(K, rbw, waves, splits, T) <= kGemmMaxLds;
}
// the waves split K (kernel 3): rbw row blocks per workgroup, every wave's
// output sums (1 KB per row block) joined through LDS; one output row block
// per wave for the exception sums
inline size_t gemm_ks_lds_bytes(int K, int rbw, int waves, int splits, int T) {
    const size_t steps = (size_t)split_steps(K, splits);
    return steps * 3 * 64 * (size_t)gemm_tokens(T) + (size_t)waves * 16 * 16 * 4 + (size_t)waves * rbw * 1024 +
           16 * 4 * (size_t)waves + 4 * (size_t)waves + 16 * 4 * (size_t)waves;
}
inline bool gemm_ks_fits(int K, int T, int rbw, int waves, int splits) {
    return waves <= kGemmMaxWaves && waves >= rbw && gemm_ks_lds_bytes(K, rbw, waves, splits, T) <= kGemmMaxLds;
}

// --- decode-step attention (k_rope_attn)
struct AttnParams {
    const float* qkv;
    const float* qn;
    const float* kn;
    const float* inv;
    const int64_t* pos;
    void* kc;
    void* vc;
    float* out;
    float* part;  // split partials [n_kv][splits][rows][HD + 2]
    int n_heads, n_kv, head_dim, maxt, kv_bf16;
    float eps, scale;
    float* qo = nullptr;  // batch: the T tokens' normed, roped q rows [T][n_heads][HD]
    int T = 1;            // batch: tokens at positions *pos .. *pos + T - 1
    // decode: floor(2^32 / splits) + 1, so that a / splits rounds down to
    // mulhi(a, smul) for every a < 2^32 / splits (the split bounds: a <= 2^21)
    uint32_t smul = 0;
};
constexpr int kAttnThreads = 320;     // 4 per position of the span
constexpr int kAttnSpan = 80;         // positions one attention workgroup covers at most
constexpr int kAttnMaxSplits = 128;   // so the context is at most 10240 positions
// one split per kv head over a short context: a workgroup of 1024 threads
// covers up to 256 positions, with no combine pass
constexpr int kAttnLongThreads = 1024;
constexpr int kAttnLongSpan = kAttnLongThreads / 4;
inline size_t attn_lds_bytes(int hd, int g, int nt = kAttnThreads) {
    const size_t pg = (size_t)nt / (hd / 2);  // position groups of the value sums
    const size_t span = (size_t)nt / 4;
    return 4 * ((size_t)g * hd + 2 * (size_t)hd + span * g + span * g + 2 * (size_t)g + pg * g * hd);
}
inline size_t attn_part_floats(int n_kv, int g, int hd, int splits) {
    return (size_t)n_kv * splits * g * (hd + 2);
}
int launch_attn(const AttnParams& p, int splits, hipStream_t st);
// batch of T <= 16 tokens: rows of one kv head = T * G (the prompt attention
// kernel over position splits, then the combine)
int launch_attn_batch(const AttnParams& p, int splits, hipStream_t st);
// prompt block of T tokens: the q/k/v prologue, then causal attention on the
// float32 matrix cores (one wave per head and 16 tokens)
constexpr int kMaxPrefillAttnTokens = 1 << 15;  // the prologue grid's second dimension stays below 65536
int launch_prefill_attn(const AttnParams& p, hipStream_t st);

int launch_gemv(const LinearParams& p, int T, int rb, int waves, int splits, hipStream_t st);
// ks: the waves of a workgroup split its K steps (kernel 3) instead of its rows (kernel 2)
int launch_gemm(const LinearParams& p, int T, int rbw, int waves, int splits, bool ks, hipStream_t st);
// workspace bytes of the launch rv12_gemm resolves (n, k, t, cfg) to; a
// negative status where it rejects the shape or cfg
int64_t launch_ws_bytes(int n, int k, int t, const rv12_launch* cfg);
void launch_splitk_reduce(const LinearParams& p, int T, int splits, hipStream_t st);

// --- greedy pick: per token the largest value of n entries and its index
// (the smallest index on ties; NaN counts as larger than any number)
constexpr int kPickThreads = 1024;
constexpr int kPickChunk = 8192;  // entries one workgroup of the first stage reduces
inline int64_t pick_chunks(int64_t n) { return (n + kPickChunk - 1) / kPickChunk; }
// the entries of token t are v[t * stride + i] (index ix[t * stride + i], or i
// where ix is NULL), i < n; one stage where n <= kPickChunk, else a first
// stage into tv / ti (T * pick_chunks(n) pairs) and a second into ids
void launch_pick(const float* v, const int32_t* ix, int64_t n, int64_t stride, int T, float* tv, int32_t* ti,
                 int64_t* ids, hipStream_t st);
// --- prefill linear (k_prefill_x + k_prefill_mm), any T
constexpr int kMaxPrefillTokens = 1 << 16;
size_t prefill_ws_bytes(int N, int K, int T);
int prefill_splits(int N, int K, int T);
void launch_decode_advance(const int64_t* ids, const uint16_t* emb, int64_t vocab, int hidden, float* x,
                           int64_t* out, int64_t out_len, int64_t* steps, int64_t* pos, int64_t* tok,
                           hipStream_t st);
void launch_prefill(const rv12_matrix& w, const float* x, float* y, int T, int mode, const uint16_t* lnw, float eps,
                    void* ws, hipStream_t st);
void launch_codec_to_bf16(const rv12_codec& c, uint16_t* w, hipStream_t st);
void launch_pack_plan(const uint16_t* w, int N, int K, int32_t* rbase, int32_t* row_exc, hipStream_t st);
void launch_pack(const uint16_t* w, int N, int K, const int32_t* rbase, const int32_t* rp, uint32_t* tiles,
                 int32_t* er, int32_t* ec, float* ev, int64_t n_exc, hipStream_t st);
void launch_decode(const rv12_matrix& w, int first, int last, void* out, int out_f32, hipStream_t st, int64_t e0,
                   int64_t e1);
void launch_encode_stats(const uint16_t* w, int64_t count, int32_t* hist, hipStream_t st);
void launch_encode(const uint16_t* w, int N, int K, int CH, int base, uint8_t* m8, uint8_t* e4, int32_t* row_exc,
                   hipStream_t st);
void launch_encode_exc(const uint16_t* w, int N, int K, int base, const int32_t* rp, int32_t* er, int32_t* ec,
                       float* ev, hipStream_t st);

}  // namespace rv12
