/* rv12 — MI355X (gfx950) kernels for the 12-bit lossless bf16 decode-linear.
 *
 * C ABI of ai_amd/librv12.so.  Plain pointers and sizes only; every pointer
 * named "device" is HIP device memory, and `stream` is a hipStream_t (NULL =
 * the legacy default stream).  Every entry point validates its arguments on
 * the host and returns a negative status before touching the GPU; a launch
 * failure reported by hipGetLastError() returns RV12_E_LAUNCH.  No entry point
 * allocates device memory or synchronises the stream: the caller owns every
 * buffer (weights, activations, outputs, workspace), so the calls are
 * reentrant and can be captured in a HIP graph.
 *
 * Each entry point replaces one piece of the reference operator API for the
 * path; reference paths are relative to the reference repository root.
 */
#ifndef RV12_H
#define RV12_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RV12_ABI_VERSION 8

enum rv12_status {
    RV12_OK = 0,
    RV12_E_NULL = -1,      /* a required pointer is NULL */
    RV12_E_SHAPE = -2,     /* N < 1, K < 32, K % 32, K > 2^20, n_exc > 2^28, K % CH, CH % 16, or rows outside [0, N] */
    RV12_E_MODE = -3,      /* mode not in {0, 1, 2} */
    RV12_E_TOKENS = -4,    /* T not in [1, 16] */
    RV12_E_WORKSPACE = -5, /* workspace smaller than rv12_workspace_bytes() */
    RV12_E_CONFIG = -6,    /* launch configuration out of range */
    RV12_E_BASE = -7,      /* base outside [0, 241] */
    RV12_E_ALIGN = -8,     /* x, y or tiles not 16-byte aligned */
    RV12_E_SIZE = -9,      /* output buffer smaller than rv12_tiles_bytes() */
    RV12_E_SCRATCH = -10,  /* rv12_gemm_static: workspace beyond RV12_STATIC_SCRATCH_BYTES */
    RV12_E_LAUNCH = -20    /* hipGetLastError() after a launch */
};

/* The reference codec dict of one matrix W[N, K] (device pointers), as built
 * by compress(): ramvi/engine/ramvi_engine/kernels/wcomp.py:13-32. */
typedef struct rv12_codec {
    const uint8_t* m8;  /* [N, K]   sign << 7 | mantissa */
    const uint8_t* e4;  /* [N, K/2] per CH-chunk: byte i = code[i] | code[CH/2 + i] << 4 */
    const int32_t* rp;  /* [N + 1]  exception row pointer */
    const int32_t* er;  /* [E]      exception rows (row-major order) */
    const int32_t* ec;  /* [E]      exception columns */
    const float* ev;    /* [E]      exact exception values */
    int32_t n, k, ch, base;
    int64_t n_exc;
} rv12_codec;

/* A matrix packed for the kernels (device pointers), written by
 * rv12_pack_plan() + rv12_pack().  `tiles` holds the weights in the Q16
 * layout, 12 bytes per 8 weights, with one exponent window per row: row n
 * keeps the weights whose biased exponent lies in [rbase[n], rbase[n] + 14]
 * in the tiles, and every other weight in the exception list rp/er/ec/ev (CSR
 * by row, row-major order, exact float32 values).  The window of each row is
 * chosen by the reference's rule for a whole matrix
 * (ramvi/engine/ramvi_engine/kernels/wcomp.py:19-21), so a row of large
 * weights does not turn into a long exception list. */
typedef struct rv12_matrix {
    const uint32_t* tiles; /* rv12_tiles_bytes(n, k) bytes */
    const int32_t* rbase;  /* [n] window start of each row */
    const int32_t* rp;     /* [n + 1] */
    const int32_t* er;     /* [n_exc] */
    const int32_t* ec;     /* [n_exc] */
    const float* ev;       /* [n_exc] */
    int32_t n, k;
    int64_t n_exc;
} rv12_matrix;

/* Launch shape of a linear.
 *   kernel  0 = built-in (rv12_launch_shape: vector up to T = 2, MFMA
 *           above), 1 = vector-FMA kernel (T <= 4), 2 = bf16-MFMA kernel
 *           (T <= 16), each wave owning its rows, 3 = the bf16-MFMA kernel
 *           with the waves of a workgroup splitting its K steps (T <= 16)
 *   rb      vector kernel: row blocks of 16 rows per workgroup (1, 2, 4);
 *           MFMA kernel 2: row blocks per wave (1, 2, 4); kernel 3: row
 *           blocks per workgroup (1, 2, 4; at most waves)
 *   waves   waves per workgroup (1..16; the MFMA kernels 1..8)
 *   splits  K splits across workgroups (1..64); more than one adds a second,
 *           atomic-free pass that sums the partials in split order
 * A zero field (or a NULL pointer) selects the built-in choice for the shape
 * (rv12_launch_shape). */
typedef struct rv12_launch {
    int32_t kernel, rb, waves, splits;
} rv12_launch;

/* The launch shape a linear of n rows, k columns and t tokens runs with for
 * cfg (NULL or all-zero: the built-in choice — the vector kernel at 1 token,
 * from 2 to 4 tokens where its activations fit the LDS without splitting K,
 * at 3 tokens on up to 512 row blocks or k <= 4096 (below 4096 row blocks)
 * and at 4 tokens on up to 512 row blocks that keep 192 workgroups or split
 * K; the MFMA kernel otherwise, with waves, row blocks and splits from
 * launch-shape sweeps on MI355X; zero fields of a partial cfg are filled in,
 * with K split further where the given fields need it).  Fills *out and
 * returns RV12_OK, or the status rv12_gemm would return for the shape and
 * cfg (RV12_E_NULL, RV12_E_SHAPE, RV12_E_TOKENS, RV12_E_CONFIG).  Size the
 * workspace with out->splits.  The reference's launch defaults and tuning
 * tables, CFG1 / CFGT in ramvi/engine/ramvi_engine/kernels/wcomp.py:115, 222. */
int rv12_launch_shape(int n, int k, int t, const rv12_launch* cfg, rv12_launch* out);

/* ABI version of the library (RV12_ABI_VERSION).  Mirrors the reference's
 * native ABI check, ramvi/engine/ramvi_engine/native/qmm.cpp:24. */
int rv12_abi_version(void);

/* Message for a status code. */
const char* rv12_strerror(int status);

/* Bytes of the Q16 tile layout for W[n, k]: ceil(n/16) * 16 * k * 3 / 2. */
size_t rv12_tiles_bytes(int n, int k);

/* Pack a bf16 matrix w[n, k] (bits, row-major, device) for the kernels, in
 * two device passes with one host step between them:
 *   rv12_pack_plan  rbase[n] = window start of each row,
 *                   row_exc[n] = weights of each row outside its window
 *   (host: rp = [0, cumsum(row_exc)], n_exc = rp[n])
 *   rv12_pack       tiles (Q16 layout) and the exception list er/ec/ev[n_exc]
 * Replaces nothing in the reference, whose kernels read m8/e4 directly; run
 * once per matrix after compress(), ramvi/engine/ramvi_engine/core/engine.py:224. */
int rv12_pack_plan(const uint16_t* w, int n, int k, int32_t* rbase, int32_t* row_exc, void* stream);
int rv12_pack(const uint16_t* w, int n, int k, const int32_t* rbase, const int32_t* rp, int64_t n_exc,
              uint32_t* tiles, size_t tiles_bytes, int32_t* er, int32_t* ec, float* ev, void* stream);

/* The bf16 matrix w[n, k] a codec dict encodes (the inverse of compress(),
 * bit for bit; the reference's decompress, wcomp.py:35-45, ends with a
 * .bfloat16() that would also map every NaN payload to one NaN).  Used to
 * pack a dict that was not built by rv12_encode* (the reference's own
 * compress, a file). */
int rv12_codec_to_bf16(const rv12_codec* in, uint16_t* w, void* stream);

/* Encode a bf16 matrix W[n, k] (bits, row-major, device) into the codec dict
 * in three calls, each a device pass with no host synchronisation:
 *   rv12_encode_stats  hist[256] = exponent histogram (int32, device)
 *   (host: base = first argmax of the 15-wide window sums of hist)
 *   rv12_encode        m8[n, k], e4[n, k/2], row_exc[n] = exceptions per row
 *   (host: rp = [0, cumsum(row_exc)], E = rp[n])
 *   rv12_encode_exc    er/ec/ev[E] in row-major order
 * Together they replace the tensor arithmetic of compress(),
 * ramvi/engine/ramvi_engine/kernels/wcomp.py:13-32. */
int rv12_encode_stats(const uint16_t* w, int n, int k, int32_t* hist, void* stream);
int rv12_encode(const uint16_t* w, int n, int k, int ch, int base, uint8_t* m8, uint8_t* e4,
                int32_t* row_exc, void* stream);
int rv12_encode_exc(const uint16_t* w, int n, int k, int base, const int32_t* rp, int32_t* er, int32_t* ec,
                    float* ev, void* stream);

/* Workspace bytes a linear needs: splits * t * ceil(n/16)*16 partial sums and
 * splits * t sums of squares (0 when splits == 1).  splits == 0 asks for the
 * built-in choice for (n, k, t).  No counterpart in the reference, whose
 * wcomp.py:226-230 allocates the split buffer itself. */
size_t rv12_workspace_bytes(int n, int k, int t, int splits);

/* Workspace bytes of exactly the launch rv12_gemm resolves (n, k, t, cfg) to
 * (cfg NULL: the built-in shape; a cfg with only some fields set has the rest
 * filled in as rv12_launch_shape does); 0 where it needs none or where
 * rv12_gemm would reject the arguments. */
size_t rv12_launch_workspace_bytes(int n, int k, int t, const rv12_launch* cfg);

/* T = 1 fused decode + GEMV:  y (=|+=) W_dec . x'
 *   mode 0: y = W x';  1: y += W x';  2: x' = silu(x[0:K]) * x[K:2K], y += W x'
 *   lnw != NULL: x' = lnw * (x' * rsqrt(mean(x[0:K]^2) + eps))
 * x: float[K] (float[2K] in mode 2), y: float[N], lnw: bf16 bits [K].
 * Replaces gemvc1 / gemvc1_k, ramvi/engine/ramvi_engine/kernels/wcomp.py:67-126. */
int rv12_gemv(const rv12_matrix* w, const float* x, float* y, const uint16_t* lnw, float eps, int mode,
              const rv12_launch* cfg, void* ws, size_t ws_bytes, void* stream);

/* 1 <= T <= 16 tokens:  y[t] (=|+=) W_dec . x'[t], rows of x are K floats apart
 * (2K in mode 2), rows of y N floats apart.  lnw as in rv12_gemv (NULL in the
 * reference's batched path).  Replaces gemvc_tc / gemvc_tc_k,
 * ramvi/engine/ramvi_engine/kernels/wcomp.py:155-242. */
int rv12_gemm(const rv12_matrix* w, const float* x, float* y, int t, const uint16_t* lnw, float eps, int mode,
              const rv12_launch* cfg, void* ws, size_t ws_bytes, void* stream);

/* Greedy next-token ids over the 12-bit lm_head, 1 <= T <= 16 rows:
 * ids[t] = the row n with the largest (W_dec . x'[t])[n], the smallest n on
 * ties, a NaN logit counting as larger than any number (the first NaN wins).
 * x' as rv12_gemm mode 0 (lnw: the final RMSNorm fused).  logits: NULL, or
 * float[T][N] that also receives the logits.  With the vector kernel and no
 * K split (the built-in launch at 1-2 tokens for a vocabulary head) the pick
 * is fused into the linear's epilogue (a (value, row) pair per workgroup and
 * token) and finished by a second small pass, with no atomics and, when
 * logits is NULL, no logits written; other launches write the logits (into
 * the workspace when logits is NULL) and reduce them in two passes.  ws:
 * rv12_head_workspace_bytes(n, k, t, cfg) bytes, 16-byte aligned; ids: 8-byte
 * aligned, written on the device (no host synchronisation).  Replaces the
 * greedy branch of Head.pick (int8 bounds + exact CPU rows, smallest id on
 * ties), ramvi/engine/ramvi_engine/generation/head.py:59-88 (tie rule
 * :76-79) and vocab_a_k, ramvi/engine/ramvi_engine/kernels/vocab8.py:19-44. */
int rv12_head_argmax(const rv12_matrix* w, const float* x, int t, const uint16_t* lnw, float eps, float* logits,
                     int64_t* ids, const rv12_launch* cfg, void* ws, size_t ws_bytes, void* stream);

/* The decode step's bookkeeping after its greedy pick, on the device (one
 * small kernel, no host synchronisation, graph-capturable): id = ids[0] is
 * recorded in out[*steps] (only when 0 <= *steps < out_len), becomes the next
 * input token (*tok, tok may be NULL), and its embedding row
 * emb[id][0:hidden) (bf16, id clamped into [0, vocab)) is written to x as
 * float32, the next step's activations; *steps and *pos are incremented.
 * ids, out, steps, pos, tok: 8-byte aligned; x 4-byte; emb 2-byte.  Replaces
 * the step's embedding lookup and the bookkeeping after the pick (the next
 * token becomes the input, position and step counters advance) that the
 * reference's decode graph does with torch operations,
 * ramvi/engine/ramvi_engine/core/engine.py:432-444. */
int rv12_decode_advance(const int64_t* ids, const uint16_t* emb, int64_t vocab, int hidden, float* x, int64_t* out,
                        int64_t out_len, int64_t* steps, int64_t* pos, int64_t* tok, void* stream);

/* Workspace bytes of rv12_head_argmax for (n, k, t, cfg) (never 0 for valid
 * arguments; 0 where rv12_head_argmax would reject them). */
size_t rv12_head_workspace_bytes(int n, int k, int t, const rv12_launch* cfg);

/* rv12_gemm with the split-K workspace in a scratch array the library holds
 * in device memory (RV12_STATIC_SCRATCH_BYTES on every GPU it runs on, until
 * the process ends) instead of a caller-owned one: no device memory is
 * allocated by the call.  A launch whose workspace (rv12_workspace_bytes for
 * the shape it resolves to) exceeds the scratch returns RV12_E_SCRATCH before
 * any device work.  The first call on a device looks up that device's scratch
 * address (with the device current); every call on one GPU shares its scratch,
 * so calls that overlap on one GPU (other streams, other threads) race.  No
 * counterpart in the reference: it serves callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  Other arguments and statuses as rv12_gemm. */
#define RV12_STATIC_SCRATCH_BYTES (8u << 20)
int rv12_gemm_static(const rv12_matrix* w, const float* x, float* y, int t, const uint16_t* lnw, float eps,
                     int mode, const rv12_launch* cfg, void* stream);

/* The prompt's linear, 1 <= t <= 65536 tokens at once:  y[r] (=|+=) W_dec . x'[r]
 * for every token row r (x rows K floats apart, 2K in mode 2; y rows N apart),
 * mode and lnw / eps (the RMSNorm prologue, modes 0 and 1; 16-byte aligned)
 * as rv12_gemv.  The 12-bit decode is fused into a bf16 MFMA GEMM:
 * x' is split per token into three bf16 parts (24 significand bits, after an
 * exact power-of-two scale), every weight is read once in its 12-bit form,
 * products and sums are fp32, the exceptions are added in list order.  Where
 * the rows and tokens give too few workgroups to fill the GPU (few tokens, or
 * a last round of workgroups mostly empty), K is split and an ordered pass
 * sums the splits.  ws: rv12_prefill_workspace_bytes(n, k, t) bytes (10 bytes
 * per column and padded token: the parts and a transposed fp32 copy of x'
 * for the exception entries; 8 per padded token; with a K split, 4 per split,
 * padded token and row for the partial sums), 16-byte aligned; 0 for
 * arguments rv12_prefill_linear rejects.  Replaces the
 * blocked prefill's rmsg_k + matrix() (decode_rows + the fp32 GEMM mm_k),
 * ramvi/engine/ramvi_engine/kernels/prefill.py:66-78, 94-99,
 * ramvi/engine/ramvi_engine/kernels/prefill_kernels.py:8-26, 58-110. */
size_t rv12_prefill_workspace_bytes(int n, int k, int t);
int rv12_prefill_linear(const rv12_matrix* w, const float* x, float* y, int t, const uint16_t* lnw, float eps,
                        int mode, void* ws, size_t ws_bytes, void* stream);

/* Bit-exact decode of rows [first, last) to bf16 bits (out_f32 == 0, out is
 * uint16[last-first, K]) or to float32 (out_f32 != 0, out is float[last-first, K]).
 * Replaces decode_rows / dequant_k TYPE 0 + exceptions_k,
 * ramvi/engine/ramvi_engine/kernels/prefill_kernels.py:58-110. */
int rv12_decode_rows(const rv12_matrix* w, int first, int last, void* out, int out_f32, void* stream);

/* Decode-step attention of one layer, one token.  The step's q (n_heads
 * heads), k and v (n_kv heads) are read from the qkv linear's output
 * (float[(n_heads + 2 n_kv) * head_dim]); q and k get their head RMSNorm
 * (weights qn, kn: float[head_dim]) and the rotate-half RoPE at position *pos
 * (angle *pos * inv[i], inv: float[head_dim / 2]); k and v, rounded to the cache
 * dtype, go into the caches kc / vc ([n_kv, maxt, head_dim], bf16 bits or
 * float32) at *pos; out (float[n_heads * head_dim]) is the grouped-query
 * attention of each head over positions 0..*pos (softmax(q.K * scale) V).
 * *pos is read on the device, so a captured graph can advance it; a *pos
 * outside [0, maxt) gives zeros and touches no cache.  The positions are spread
 * over `splits` workgroups per kv head, each covering at most 80 of them (so
 * splits >= maxt / 80, at most 128: maxt <= 10240), or, with splits == 1 and
 * maxt <= 256, one workgroup of 1024 threads per kv head covering them all;
 * splits > 1 adds a combine pass over partials in the workspace
 * (rv12_attn_workspace_bytes).  Calls
 * sharing a workspace must be ordered on one stream.  Replaces rope_attn_k,
 * ramvi/engine/ramvi_engine/kernels/tkernels.py:164-213. */
typedef struct rv12_attn {
    int32_t n_heads, n_kv, head_dim, maxt;
    int32_t kv_bf16; /* 1: bf16 cache, 0: float32 cache */
    int32_t splits;  /* 1..128 */
    float eps, scale;
} rv12_attn;

size_t rv12_attn_workspace_bytes(const rv12_attn* a);
int rv12_rope_attn(const rv12_attn* a, const float* qkv, const float* qn, const float* kn, const float* inv,
                   const int64_t* pos, void* kc, void* vc, float* out, void* ws, size_t ws_bytes, void* stream);

/* Attention of a batch of 1 <= t <= 16 tokens of one sequence at positions
 * *pos .. *pos + t - 1 (read on the device): rows r of qkv (t rows of
 * (n_heads + 2 n_kv) * head_dim floats) as in rv12_rope_attn; q and k get the
 * head RMSNorm and RoPE at their position, k and v (rounded to the cache dtype)
 * go into the caches, and token r attends over positions 0..*pos + r (causal)
 * into out[r] (t rows of n_heads * head_dim floats).  Three passes (q/k/v
 * prologue; attention of the batch's 16-token tile over min(a.splits,
 * ceil(256 / n_kv)) position splits, one wave per query head on the matrix
 * cores — float32 products, as rv12_prefill_rope_attn; the ordered combine),
 * no atomics.  A batch
 * outside [0, maxt) gives zeros and leaves the caches untouched.  ws:
 * rv12_attn_batch_workspace_bytes(a, t) bytes (the q rows and the split
 * partials), 16-byte aligned.  Replaces qk_rope_cache_k and attn_k,
 * ramvi/engine/ramvi_engine/kernels/tkernels.py:82-150. */
size_t rv12_attn_batch_workspace_bytes(const rv12_attn* a, int t);
int rv12_rope_attn_batch(const rv12_attn* a, int t, const float* qkv, const float* qn, const float* kn,
                         const float* inv, const int64_t* pos, void* kc, void* vc, float* out, void* ws,
                         size_t ws_bytes, void* stream);

/* Attention of a prompt block of 1 <= t <= 32768 tokens at positions *pos ..
 * *pos + t - 1 (read on the device), the blocked prefill's: the q/k/v
 * prologue of rv12_rope_attn_batch (head RMSNorm, RoPE, k and v rounded into
 * the caches), then token r attends over positions 0..*pos + r with float32
 * products and an online softmax into out[r] (t rows of n_heads * head_dim
 * floats): one wave per (head, 16 tokens) on the float32 matrix cores, the
 * G heads of a kv head in one workgroup.  a->splits is not used.  A block
 * outside [0, maxt) gives zeros and leaves the caches untouched.  ws:
 * rv12_prefill_attn_workspace_bytes(a, t) bytes (the q rows), 16-byte
 * aligned; 0 there means the shape is not supported (maxt * head_dim * cache
 * bytes and t * n_heads * head_dim * 4 must stay below 2^31).  Replaces
 * qk_rope_cache_k + attention / att_k of the blocked prefill,
 * ramvi/engine/ramvi_engine/kernels/prefill.py:100-103 and
 * prefill_kernels.py:29-54. */
size_t rv12_prefill_attn_workspace_bytes(const rv12_attn* a, int t);
int rv12_prefill_rope_attn(const rv12_attn* a, int t, const float* qkv, const float* qn, const float* kn,
                           const float* inv, const int64_t* pos, void* kc, void* vc, float* out, void* ws,
                           size_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* RV12_H */
