// C-ABI layer of librv12: host-side validation, launch-shape choice and
// kernel launches.  Every check runs before any GPU call, so a bad argument
// returns a status without touching the device.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rv12.h"
#include "rv12_internal.h"

#include <algorithm>

using namespace rv12;

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int launch_status() { return hipGetLastError() == hipSuccess ? RV12_OK : RV12_E_LAUNCH; }

int64_t nblocks(int n) { return ((int64_t)n + 15) / 16; }

struct Shape {
    int kernel, rb, waves, splits;
};

bool shape_fits(int K, int T, const Shape& c) {
    if (c.kernel == 1) return T <= kMaxVectorTokens && gemv_fits(K, T, c.rb, c.waves, c.splits);
    // MFMA: the split's staged activations (sized by the token columns) fit the LDS
    if (c.kernel == 3) return gemm_ks_fits(K, T, c.rb, c.waves, c.splits);
    return gemm_fits(K, T, c.rb, c.waves, c.splits);
}

// Built-in launch shapes, from launch-shape sweeps of the Qwen3-8B / 14B
// linear shapes on MI355X.
//   vector kernel: one row block per workgroup and 8 waves (16 for
//     K >= 8192); two row blocks and 4 waves beyond 4096 row blocks; two
//     row blocks and 8 waves for 257-512 row blocks, and from 3 tokens on
//     for more; at one token 4 waves above 512 row blocks for K <= 6144.
//     K is split from 2 tokens on when
//     there are fewer than 128 row blocks, so the grid still covers the 256
//     CUs, and at one token wherever the activations would not fit in
//     registers;
//   MFMA kernel: the shape with the least time in a model of its rounds of
//     workgroups (mfma_model_us).
// Which kernel: the vector kernel at 1 token; from 2 to 4 tokens where its
// activations fit the LDS without a K split (a split adds rounds of
// workgroups and the reduce pass) and, at 3 tokens, on up to 512 row blocks
// or K <= 4096 (below 4096 row blocks), at 4 tokens on up to 512 row blocks
// whose grid keeps at least 192 workgroups (or that split K to fill the CUs):
// there its FMAs still hide behind the weight stream (vector_wins); the MFMA
// kernel elsewhere.
Shape vector_shape(int N, int K, int T) {
    const int64_t nblk = nblocks(N);
    Shape c;
    c.kernel = 1;
    c.rb = 1;
    c.waves = K >= 8192 ? 16 : 8;
    if (nblk >= 4096) {
        c.rb = 2;
        c.waves = 4;
    } else if (nblk > 256 && (nblk <= 512 || T >= 3)) {
        // 257-512 row blocks: two row blocks of 8 waves per workgroup
        // (Qwen3-8B qkv 11.0 -> 10.4 us, 14B o 12.3 -> 11.6, 32B o
        // 17.5 -> 15.6, 14B down 33.1 -> 27.7 with 3 splits; at 2 tokens
        // 14B o 12.9 -> 11.1, 8B qkv 11.2 -> 10.1, 32B o 16.3 -> 14.4); from
        // 3 tokens on also above (8B gate/up 24576x4096 at 3 tokens 32.2 ->
        // 27.7, at 4 36.9 -> 30.6)
        c.rb = 2;
        c.waves = 8;
    } else if (T == 1 && nblk > 512 && K <= 6144) {
        // more row blocks: 4 waves, twice the workgroups resident per CU, so
        // one's prologue overlaps another's stream (with the RMS prologue
        // Qwen3-32B gu 51200x5120 67.6 -> 63.5 us, 8B gu 28.0 -> 26.7)
        c.waves = 4;
    }
    c.splits = 1;
    // below 128 row blocks a K split fills more CUs but costs a reduce
    // launch: at one token the unsplit launch is faster (Qwen3-8B k/v
    // 1024x4096 6.0 vs 7.2 us with 4 splits, 0.6B o 1024x2048 4.6 vs 6.7)
    if (nblk < 128 && T > 1) c.splits = (int)std::min<int64_t>(4, (256 + nblk - 1) / nblk);
    return c;
}

// Time model of the MFMA kernel, in us.  A workgroup stages x' for its K
// split in LDS before streaming, so the launch runs in rounds of one
// workgroup per CU.  Each round costs a fixed part plus the staging of its
// split (per K step, in proportion to the token columns staged) plus its
// weight bytes at the smaller of the HBM rate and a per-CU rate (the bytes
// one CU keeps in flight over the memory latency); a K split adds the reduce
// pass, a launch plus a cost per MB of partials.  The constants are fitted to
// a sweep of the launch shapes the model considers (kernel 2: 1, 2 or 4 row
// blocks per wave, 4 or 8 waves, the first 10 splits that fit; 3284 timed
// launches) on 13 Qwen3-8B/14B/32B shapes at 4, 8 and 16 tokens on MI355X,
// with the kernel's per-row-block prefetch depths: the model's pick lies
// 1.3 % above the measured best on average and 9.5 % at worst (Qwen3-32B o at
// 4 tokens); the per-CU rate depends on the row blocks and waves of a wave's
// workgroup (one row block of 8 waves streams best, four of 4 worst).
constexpr double kModelRoundUs = 1.0;
constexpr double kModelStepUs = 0.2;
constexpr double kModelHbmGBs = 6500.0;
constexpr double kModelCuGBs = 30.0;
constexpr double kModelCuGBs1x8 = 35.0;  // one row block per wave, 8 waves
constexpr double kModelCuGBs4x4 = 10.0;  // four row blocks per wave, 4 waves
// kernel 3 (the waves split K): the per-CU rate fitted to the same sweep with
// its shapes added; it is slower than kernel 2 on all but 2 of the 42 cases
// (Qwen3-8B down and 32B o at 4 tokens, by 1-4 %), so the built-in choice is
// kernel 2 and kernel 3 a candidate of the tuner and of explicit launches
constexpr double kModelKsCuGBs = 10.0;
constexpr double kModelReduceUs = 0.5;
constexpr double kModelReduceUsPerMB = 2.0;
constexpr int kModelCUs = 256;
constexpr double kModelStepBytes = 768.0;  // one (row block, step) tile

// kernel 2: each wave owns rb row blocks (rb x waves per workgroup); kernel
// 3: the waves split K over rb row blocks per workgroup
double mfma_model_us(int64_t nblk, int N, int K, int T, int rb, int waves, int splits, int kernel = 2) {
    const int64_t per_wg = (int64_t)rb * (kernel == 3 ? 1 : waves);
    const int64_t wgs = (nblk + per_wg - 1) / per_wg * splits;
    const int steps = split_steps(K, splits);
    const double wg_bytes = (double)per_wg * steps * kModelStepBytes;
    const double cu_rate = kernel == 3 ? kModelKsCuGBs
                           : rb == 1 && waves == 8 ? kModelCuGBs1x8
                           : rb == 4 && waves == 4 ? kModelCuGBs4x4
                                                   : kModelCuGBs;
    double t = 0.0;
    for (int64_t left = wgs; left > 0;) {
        const int64_t n = std::min<int64_t>(left, (int64_t)kModelCUs);
        t += kModelRoundUs + kModelStepUs * steps * gemm_tokens(T) / 16.0 +
             (double)n * wg_bytes / (std::min(kModelHbmGBs, (double)n * cu_rate) * 1e3);
        left -= n;
    }
    if (splits > 1) t += kModelReduceUs + kModelReduceUsPerMB * (double)(splits + 1) * T * N * 4 / 1e6;
    return t;
}

// candidates of MFMA kernel `kernel` (2, 3, or 0 for both): 1, 2 or 4 row
// blocks per wave (kernel 2) or per workgroup (kernel 3, at most one per
// wave), 4 or 8 waves, the fewest K splits whose staging fits and up to 10
// more
Shape mfma_shape(int N, int K, int T, int kernel = 2) {
    const int64_t nblk = nblocks(N);
    const int nsteps = K / 32;
    Shape best;
    best.kernel = 2;
    best.rb = 1;
    best.waves = 1;
    best.splits = nsteps;
    double best_t = 1e300;
    for (int kn : {2, 3}) {
        if (kernel && kn != kernel) continue;
        for (int rb : {1, 2, 4}) {
            for (int w : {4, 8}) {
                const int wv = std::min(w, nsteps);  // no more waves than K steps
                if (kn == 3 && wv < rb) continue;
                // (shapes whose activation groups do not all fit the four
                // registers per thread stage the rest after the weight
                // prefetch; the sweep the constants are fitted to timed them
                // as fast, and a rule that kept them out doubled the model's
                // mean miss: 2.0 against 1.3 %)
                auto fits = [&](int s) {
                    return kn == 3 ? gemm_ks_fits(K, T, rb, wv, s) : gemm_fits(K, T, rb, wv, s);
                };
                int s0 = 1;
                while (s0 < std::min(kMaxSplits, nsteps) && !fits(s0)) ++s0;
                if (!fits(s0)) continue;
                for (int s = s0; s <= std::min({s0 + 10, kMaxSplits, nsteps}); ++s) {
                    if (!fits(s)) continue;
                    const double t = mfma_model_us(nblk, N, K, T, rb, wv, s, kn);
                    if (t < best_t) {
                        best_t = t;
                        best.kernel = kn;
                        best.rb = rb;
                        best.waves = wv;
                        best.splits = s;
                    }
                }
            }
        }
    }
    return best;
}

// 2 to 4 tokens: the vector kernel against the MFMA kernel's best shape, from
// a sweep of 18 Qwen3-0.6B/8B/14B/32B linear shapes on MI355X (median of
// interleaved timings).  Unsplit activations in LDS at every token count (at
// 2 tokens Qwen3-14B down 5120x17408: 26.5 against 27.6 us; 32B down, whose
// activations need a split, 43.8 against 37.6).  At 3 tokens up to 512 row
// blocks (32B o 5120x8192: 15.9 against 17.1, 8B down 16.6-17.4 against
// 18.3) or K <= 4096 below 4096 row blocks (8B gate/up 27.7 against 31.6;
// the 8B head 151936x4096: 175.9 against 168.0), but not the wide K = 5120
// matrices (14B gate/up 30.0 against 28.6, 32B qkv 20.1 against 18.6; 32B
// gate/up 51200x5120 the exception, 70.7 against 74.5).  At 4 tokens the vector kernel's time grows with the tokens while the
// MFMA kernel's stays: only where the grid keeps 3/4 of the CUs busy (8B qkv
// 11.8 against 12.7, 14B qkv 14.4 against 15.9, 0.6B gate/up 5.7 against 8.4;
// but 14B o, 160 workgroups of two row blocks: 13.4 against 12.8) or K is
// split to fill them (14B k/v 7.2 against 8.1).
bool vector_wins(int N, int K, int T, const Shape& v) {
    if (T <= 1) return true;
    if (T > kMaxVectorTokens || gemv_lds_bytes(K, T, v.rb, v.waves, 1) > kMaxLds) return false;
    const int64_t nblk = nblocks(N);
    if (T == 3) return nblk <= 512 || (K <= 4096 && nblk < 4096);
    if (T == 4) return nblk <= 512 && (v.splits > 1 || (nblk + v.rb - 1) / v.rb >= 192);
    return true;
}

Shape default_shape(int N, int K, int T) {
    const int nsteps = K / 32;
    const Shape v = vector_shape(N, K, T);
    Shape c = vector_wins(N, K, T, v) ? v : mfma_shape(N, K, T);
    // (a former rule, at most one wave per 8 K steps at one token, no longer
    // holds with the 4-step prefetch of 8-wave workgroups: at K = 1024, 8
    // waves beat 4 with every prologue, Qwen3-0.6B qkv 4.12 against 4.53 us,
    // gate/up with two row blocks 5.02 against 5.51, 1024x1024 3.55 against
    // 3.91)
    while (c.kernel != 3 && c.waves > 1 && split_steps(K, c.splits) < c.waves) c.waves >>= 1;
    while (c.splits < kMaxSplits && c.splits < nsteps && !shape_fits(K, T, c)) ++c.splits;
    // at one token the vector kernel streams best with all activations loaded
    // before the weights; from 2 tokens on the unsplit launch that stages the
    // rest after the weight prefetch is faster (32B o at 2 tokens: 14.4 us)
    const int s_fit = c.splits;
    while (c.kernel == 1 && T == 1 && c.splits < kMaxSplits && c.splits < nsteps &&
           !gemv_prefetch_all(K, T, c.waves, c.splits))
        ++c.splits;
    if (c.splits > s_fit) {
        // once K is split anyway, up to two more splits may fill the last
        // round of workgroups better (Qwen3-14B down at one token: 480
        // workgroups in 27.7 us against 320 in 33.8)
        const int s0 = c.splits;
        double best = 0.0;
        for (int s = s0; s <= std::min(s0 + 2, std::min(kMaxSplits, nsteps)); ++s) {
            const int64_t wg = (nblocks(N) + c.rb - 1) / c.rb * s;
            const double fill = (double)wg / (double)(kModelCUs * ((wg + kModelCUs - 1) / kModelCUs));
            if (fill > best + 1e-9 && gemv_prefetch_all(K, T, c.waves, s)) {
                best = fill;
                c.splits = s;
            }
        }
    }
    return c;
}

int resolve_launch(int N, int K, int T, const rv12_launch* cfg, Shape* out) {
    Shape c = default_shape(N, K, T);
    if (cfg) {
        if (cfg->kernel && cfg->kernel != c.kernel)  // that kernel's own defaults first
            c = cfg->kernel >= 2 ? mfma_shape(N, K, T, cfg->kernel == 3 ? 3 : 2) : vector_shape(N, K, T);
        if (cfg->kernel) c.kernel = cfg->kernel;                            // an unknown kernel is rejected below
        if (cfg->rb) c.rb = cfg->rb;
        if (cfg->waves) c.waves = cfg->waves;
        if (cfg->splits) {
            c.splits = cfg->splits;
        } else {
            // keep the staging / LDS bounds when only other fields were given
            while (c.splits < kMaxSplits && c.splits < K / 32 && c.kernel >= 1 && c.kernel <= 3 &&
                   c.rb >= 1 && c.waves >= 1 && c.waves <= kMaxWaves && !shape_fits(K, T, c))
                ++c.splits;
        }
    }
    if (c.kernel < 1 || c.kernel > 3) return RV12_E_CONFIG;
    if (c.kernel == 1 && T > kMaxVectorTokens) return RV12_E_CONFIG;
    if (c.rb != 1 && c.rb != 2 && c.rb != 4) return RV12_E_CONFIG;
    if (c.waves < 1 || c.waves > kMaxWaves) return RV12_E_CONFIG;
    if (c.splits < 1 || c.splits > kMaxSplits || c.splits > K / 32) return RV12_E_CONFIG;
    if (!shape_fits(K, T, c)) return RV12_E_CONFIG;
    *out = c;
    return RV12_OK;
}

size_t ws_bytes_for(int N, int T, int splits) {
    if (splits <= 1) return 0;
    return 4 * ((size_t)splits * T * (size_t)(nblocks(N) * 16) + (size_t)splits * T);
}

int check_matrix(const rv12_matrix* w) {
    if (!w || !w->tiles || !w->rbase || !w->rp) return RV12_E_NULL;
    if (w->n_exc > 0 && (!w->er || !w->ec || !w->ev)) return RV12_E_NULL;
    if (w->n < 1 || w->k < 32 || w->k % 32 || w->k > kMaxK || w->n_exc < 0 || w->n_exc > kMaxExc)
        return RV12_E_SHAPE;
    if (!aligned16(w->tiles)) return RV12_E_ALIGN;
    return RV12_OK;
}

bool shape_ok(int n, int k) { return n >= 1 && k >= 32 && k % 32 == 0 && k <= kMaxK; }

}  // namespace

int64_t rv12::launch_ws_bytes(int n, int k, int t, const rv12_launch* cfg) {
    if (!shape_ok(n, k)) return RV12_E_SHAPE;
    if (t < 1 || t > 16) return RV12_E_TOKENS;
    Shape c;
    const int rc = resolve_launch(n, k, t, cfg, &c);
    if (rc) return rc;
    return (int64_t)ws_bytes_for(n, t, c.splits);
}

namespace {

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// Workspace of a greedy pick (rv12_head_argmax), each part 256-byte aligned:
// the linear's split partials, the logits, the fused pick's per-workgroup
// pairs (vector kernel, one split), then the first pick stage's pairs where
// more than one chunk is reduced.
struct HeadWs {
    bool fused;
    int64_t m;  // entries the pick reduces per token
    size_t pv, pi, logits, tv, ti, total;
};

HeadWs head_ws(int n, int t, const Shape& c) {
    HeadWs h{};
    h.fused = c.kernel == 1 && c.splits == 1;
    size_t o = align256(ws_bytes_for(n, t, c.splits));
    // logits: the output of a launch that is not fused, or, fused, what the
    // vector kernel reads as y (it loads y before it knows the mode)
    h.logits = o;
    o = align256(o + (size_t)t * n * 4);
    if (h.fused) {
        h.m = (nblocks(n) + c.rb - 1) / c.rb;  // workgroups of the vector kernel
        h.pv = o;
        o = align256(o + (size_t)t * h.m * 4);
        h.pi = o;
        o = align256(o + (size_t)t * h.m * 4);
    } else {
        h.m = n;
    }
    const int64_t nc = h.m > kPickChunk ? pick_chunks(h.m) : 0;
    h.tv = o;
    o = align256(o + (size_t)t * nc * 4);
    h.ti = o;
    o = align256(o + (size_t)t * nc * 4);
    h.total = o;
    return h;
}

void fill_params(LinearParams& p, const rv12_matrix* w, const float* x, float* y, int t, const uint16_t* lnw,
                 float eps, int mode, void* ws, int splits, bool split_ws) {
    p.tiles = w->tiles;
    p.rp = w->rp;
    p.er = w->er;
    p.ec = w->ec;
    p.ev = w->ev;
    p.x = x;
    p.y = y;
    p.lnw = lnw;
    p.part = (float*)ws;
    p.ssq = split_ws ? (float*)ws + (size_t)splits * t * (size_t)(nblocks(w->n) * 16) : nullptr;
    p.N = w->n;
    p.K = w->k;
    p.npad = (int)(nblocks(w->n) * 16);
    p.rbase = w->rbase;
    p.mode = mode;
    p.xs = mode == 2 ? 2 * w->k : w->k;
    p.n_exc = w->n_exc;
    p.eps = eps;
}

// the reduce pass addresses the partials with 32-bit byte offsets
bool split_in_range(int n, int t, int splits) {
    return splits <= 1 || (int64_t)(splits + kReduceBatchMax) * t * nblocks(n) * 16 * 4 < ((int64_t)1 << 31);
}

}  // namespace

extern "C" {

int rv12_abi_version(void) { return RV12_ABI_VERSION; }

const char* rv12_strerror(int s) {
    switch (s) {
        case RV12_OK: return "ok";
        case RV12_E_NULL: return "required pointer is NULL";
        case RV12_E_SHAPE: return "bad shape (N >= 1, K >= 32, K % 32 == 0, K % CH == 0, CH % 16 == 0, rows in [0, N])";
        case RV12_E_MODE: return "mode must be 0, 1 or 2";
        case RV12_E_TOKENS: return "T must be in [1, 16]";
        case RV12_E_WORKSPACE: return "workspace smaller than rv12_workspace_bytes()";
        case RV12_E_CONFIG: return "launch configuration out of range";
        case RV12_E_BASE: return "base must be in [0, 241]";
        case RV12_E_ALIGN: return "x, y, lnw or tiles not aligned (16 bytes; lnw 8 bytes)";
        case RV12_E_SIZE: return "tiles buffer smaller than rv12_tiles_bytes()";
        case RV12_E_SCRATCH: return "workspace of the launch exceeds the static scratch (RV12_STATIC_SCRATCH_BYTES, 8 MiB)";
        case RV12_E_LAUNCH: return "kernel launch failed";
    }
    return "unknown rv12 status";
}

size_t rv12_tiles_bytes(int n, int k) {
    if (n < 1 || k < 32 || k % 32 || k > kMaxK) return 0;
    return (size_t)nblocks(n) * 16 * (size_t)k * 3 / 2;
}

int rv12_pack_plan(const uint16_t* w, int n, int k, int32_t* rbase, int32_t* row_exc, void* stream) {
    if (!w || !rbase || !row_exc) return RV12_E_NULL;
    if (!shape_ok(n, k)) return RV12_E_SHAPE;
    if (!aligned16(w)) return RV12_E_ALIGN;
    launch_pack_plan(w, n, k, rbase, row_exc, (hipStream_t)stream);
    return launch_status();
}

int rv12_pack(const uint16_t* w, int n, int k, const int32_t* rbase, const int32_t* rp, int64_t n_exc,
              uint32_t* tiles, size_t tiles_bytes, int32_t* er, int32_t* ec, float* ev, void* stream) {
    if (!w || !rbase || !rp || !tiles) return RV12_E_NULL;
    if (n_exc > 0 && (!er || !ec || !ev)) return RV12_E_NULL;
    if (!shape_ok(n, k) || n_exc < 0) return RV12_E_SHAPE;
    if (!aligned16(w) || !aligned16(tiles)) return RV12_E_ALIGN;
    if (tiles_bytes < rv12_tiles_bytes(n, k)) return RV12_E_SIZE;
    launch_pack(w, n, k, rbase, rp, tiles, er, ec, ev, n_exc, (hipStream_t)stream);
    return launch_status();
}

int rv12_codec_to_bf16(const rv12_codec* in, uint16_t* w, void* stream) {
    if (!in || !w || !in->m8 || !in->e4) return RV12_E_NULL;
    if (in->n_exc > 0 && (!in->er || !in->ec || !in->ev)) return RV12_E_NULL;
    if (!shape_ok(in->n, in->k) || in->ch < 16 || in->ch % 16 || in->k % in->ch || in->n_exc < 0) return RV12_E_SHAPE;
    if (in->base < 0 || in->base > 241) return RV12_E_BASE;
    if (!aligned16(w)) return RV12_E_ALIGN;
    launch_codec_to_bf16(*in, w, (hipStream_t)stream);
    return launch_status();
}

int rv12_encode_stats(const uint16_t* w, int n, int k, int32_t* hist, void* stream) {
    if (!w || !hist) return RV12_E_NULL;
    if (n < 1 || k < 1) return RV12_E_SHAPE;
    if (!aligned16(w)) return RV12_E_ALIGN;
    launch_encode_stats(w, (int64_t)n * k, hist, (hipStream_t)stream);
    return launch_status();
}

int rv12_encode(const uint16_t* w, int n, int k, int ch, int base, uint8_t* m8, uint8_t* e4, int32_t* row_exc,
                void* stream) {
    if (!w || !m8 || !e4 || !row_exc) return RV12_E_NULL;
    if (n < 1 || k < 2 || ch < 2 || ch % 2 || k % ch) return RV12_E_SHAPE;
    if (base < 0 || base > 241) return RV12_E_BASE;
    launch_encode(w, n, k, ch, base, m8, e4, row_exc, (hipStream_t)stream);
    return launch_status();
}

int rv12_encode_exc(const uint16_t* w, int n, int k, int base, const int32_t* rp, int32_t* er, int32_t* ec,
                    float* ev, void* stream) {
    if (!w || !rp || !er || !ec || !ev) return RV12_E_NULL;
    if (n < 1 || k < 1) return RV12_E_SHAPE;
    if (base < 0 || base > 241) return RV12_E_BASE;
    launch_encode_exc(w, n, k, base, rp, er, ec, ev, (hipStream_t)stream);
    return launch_status();
}

int rv12_launch_shape(int n, int k, int t, const rv12_launch* cfg, rv12_launch* out) {
    if (!out) return RV12_E_NULL;
    if (n < 1 || k < 32 || k % 32 || k > kMaxK) return RV12_E_SHAPE;
    if (t < 1 || t > 16) return RV12_E_TOKENS;
    Shape c;
    const int rc = resolve_launch(n, k, t, cfg, &c);
    if (rc) return rc;
    out->kernel = c.kernel;
    out->rb = c.rb;
    out->waves = c.waves;
    out->splits = c.splits;
    return RV12_OK;
}

size_t rv12_workspace_bytes(int n, int k, int t, int splits) {
    if (n < 1 || k < 32 || k % 32 || k > kMaxK || t < 1 || t > 16) return 0;
    if (splits == 0) splits = default_shape(n, k, t).splits;
    return ws_bytes_for(n, t, splits);
}

size_t rv12_launch_workspace_bytes(int n, int k, int t, const rv12_launch* cfg) {
    const int64_t b = launch_ws_bytes(n, k, t, cfg);
    return b < 0 ? 0 : (size_t)b;
}

int rv12_gemm(const rv12_matrix* w, const float* x, float* y, int t, const uint16_t* lnw, float eps, int mode,
              const rv12_launch* cfg, void* ws, size_t ws_bytes, void* stream) {
    int rc = check_matrix(w);
    if (rc) return rc;
    if (!x || !y) return RV12_E_NULL;
    if (mode < 0 || mode > 2) return RV12_E_MODE;
    if (t < 1 || t > 16) return RV12_E_TOKENS;
    if (!aligned16(x) || !aligned16(y) || ((uintptr_t)lnw & 7u)) return RV12_E_ALIGN;
    Shape c;
    rc = resolve_launch(w->n, w->k, t, cfg, &c);
    if (rc) return rc;
    const int splits = c.splits;
    if (!split_in_range(w->n, t, splits)) return RV12_E_CONFIG;
    const size_t need = ws_bytes_for(w->n, t, splits);
    if (need && (!ws || ws_bytes < need)) return RV12_E_WORKSPACE;
    if (need && !aligned16(ws)) return RV12_E_ALIGN;
    LinearParams p;
    fill_params(p, w, x, y, t, lnw, eps, mode, ws, splits, need != 0);
    const int lrc = c.kernel == 1 ? launch_gemv(p, t, c.rb, c.waves, splits, (hipStream_t)stream)
                                  : launch_gemm(p, t, c.rb, c.waves, splits, c.kernel == 3, (hipStream_t)stream);
    if (lrc) return RV12_E_CONFIG;
    return launch_status();
}

size_t rv12_head_workspace_bytes(int n, int k, int t, const rv12_launch* cfg) {
    if (!shape_ok(n, k) || t < 1 || t > 16) return 0;
    Shape c;
    if (resolve_launch(n, k, t, cfg, &c)) return 0;
    return head_ws(n, t, c).total;
}

int rv12_decode_advance(const int64_t* ids, const uint16_t* emb, int64_t vocab, int hidden, float* x, int64_t* out,
                        int64_t out_len, int64_t* steps, int64_t* pos, int64_t* tok, void* stream) {
    if (!ids || !emb || !x || !out || !steps || !pos) return RV12_E_NULL;
    if (vocab < 1 || hidden < 1 || out_len < 0) return RV12_E_SHAPE;
    if (((uintptr_t)ids | (uintptr_t)out | (uintptr_t)steps | (uintptr_t)pos | (uintptr_t)tok) & 7u ||
        ((uintptr_t)x & 3u) || ((uintptr_t)emb & 1u))
        return RV12_E_ALIGN;
    launch_decode_advance(ids, emb, vocab, hidden, x, out, out_len, steps, pos, tok, (hipStream_t)stream);
    return launch_status();
}

int rv12_head_argmax(const rv12_matrix* w, const float* x, int t, const uint16_t* lnw, float eps, float* logits,
                     int64_t* ids, const rv12_launch* cfg, void* ws, size_t ws_bytes, void* stream) {
    int rc = check_matrix(w);
    if (rc) return rc;
    if (!x || !ids) return RV12_E_NULL;
    if (t < 1 || t > 16) return RV12_E_TOKENS;
    if (!aligned16(x) || (logits && !aligned16(logits)) || ((uintptr_t)lnw & 7u) || ((uintptr_t)ids & 7u))
        return RV12_E_ALIGN;
    Shape c;
    rc = resolve_launch(w->n, w->k, t, cfg, &c);
    if (rc) return rc;
    if (!split_in_range(w->n, t, c.splits)) return RV12_E_CONFIG;
    const HeadWs h = head_ws(w->n, t, c);
    if (!ws || ws_bytes < h.total) return RV12_E_WORKSPACE;
    if (!aligned16(ws)) return RV12_E_ALIGN;
    char* b = (char*)ws;
    hipStream_t st = (hipStream_t)stream;
    LinearParams p;
    float* y = logits ? logits : (float*)(b + h.logits);
    fill_params(p, w, x, y, t, lnw, eps, 0, ws, c.splits, c.splits > 1);
    int lrc;
    if (h.fused) {
        p.store_y = logits != nullptr;
        p.amv = (float*)(b + h.pv);
        p.ami = (int32_t*)(b + h.pi);
        lrc = launch_gemv(p, t, c.rb, c.waves, 1, st);
    } else {
        lrc = c.kernel == 1 ? launch_gemv(p, t, c.rb, c.waves, c.splits, st)
                            : launch_gemm(p, t, c.rb, c.waves, c.splits, c.kernel == 3, st);
    }
    if (lrc) return RV12_E_CONFIG;
    if (h.fused)
        launch_pick(p.amv, p.ami, h.m, h.m, t, (float*)(b + h.tv), (int32_t*)(b + h.ti), ids, st);
    else
        launch_pick(y, nullptr, h.m, w->n, t, (float*)(b + h.tv), (int32_t*)(b + h.ti), ids, st);
    return launch_status();
}

size_t rv12_prefill_workspace_bytes(int n, int k, int t) {
    if (n < 1 || k < 32 || k % 32 || k > kMaxK || t < 1 || t > kMaxPrefillTokens) return 0;
    return prefill_ws_bytes(n, k, t);
}

int rv12_prefill_linear(const rv12_matrix* w, const float* x, float* y, int t, const uint16_t* lnw, float eps,
                        int mode, void* ws, size_t ws_bytes, void* stream) {
    int rc = check_matrix(w);
    if (rc) return rc;
    if (!x || !y) return RV12_E_NULL;
    if (mode < 0 || mode > 2) return RV12_E_MODE;
    if (lnw && mode == 2) return RV12_E_MODE;  // the RMS prologue belongs to the plain linear
    if (lnw && (uintptr_t)lnw % 16) return RV12_E_ALIGN;
    if (t < 1 || t > kMaxPrefillTokens) return RV12_E_TOKENS;
    if (!aligned16(x) || !aligned16(y)) return RV12_E_ALIGN;
    const size_t need = prefill_ws_bytes(w->n, w->k, t);
    if (!ws || ws_bytes < need) return RV12_E_WORKSPACE;
    if (!aligned16(ws)) return RV12_E_ALIGN;
    launch_prefill(*w, x, y, t, mode, lnw, eps, ws, (hipStream_t)stream);
    return launch_status();
}

int rv12_gemv(const rv12_matrix* w, const float* x, float* y, const uint16_t* lnw, float eps, int mode,
              const rv12_launch* cfg, void* ws, size_t ws_bytes, void* stream) {
    return rv12_gemm(w, x, y, 1, lnw, eps, mode, cfg, ws, ws_bytes, stream);
}

int rv12_decode_rows(const rv12_matrix* w, int first, int last, void* out, int out_f32, void* stream) {
    int rc = check_matrix(w);
    if (rc) return rc;
    if (first < 0 || last > w->n || first > last) return RV12_E_SHAPE;
    if (first == last) return RV12_OK;  // nothing to write: out may be NULL
    if (!out) return RV12_E_NULL;
    if (!aligned16(out)) return RV12_E_ALIGN;
    launch_decode(*w, first, last, out, out_f32, (hipStream_t)stream, 0, w->n_exc);
    return launch_status();
}

static int check_attn(const rv12_attn* a) {
    if (!a) return RV12_E_NULL;
    if (a->head_dim != 64 && a->head_dim != 128) return RV12_E_SHAPE;
    if (a->n_kv < 1 || a->n_heads < a->n_kv || a->n_heads % a->n_kv) return RV12_E_SHAPE;
    const int g = a->n_heads / a->n_kv;
    if (g != 1 && g != 2 && g != 4 && g != 8) return RV12_E_SHAPE;
    if (a->maxt < 1) return RV12_E_SHAPE;
    if (a->splits < 1 || a->splits > kAttnMaxSplits) return RV12_E_CONFIG;
    // a split covers at most kAttnSpan positions of 0..maxt-1; one split may
    // cover up to kAttnLongSpan (the long-span workgroup, no combine)
    const bool longspan = a->splits == 1 && a->maxt > kAttnSpan;
    if (longspan ? a->maxt > kAttnLongSpan : (a->maxt + a->splits - 1) / a->splits > kAttnSpan)
        return RV12_E_CONFIG;
    // (the long-span workgroup takes one q head)
    if (attn_lds_bytes(a->head_dim, longspan ? 1 : g, longspan ? kAttnLongThreads : kAttnThreads) > kMaxLds)
        return RV12_E_CONFIG;
    return RV12_OK;
}

size_t rv12_attn_workspace_bytes(const rv12_attn* a) {
    if (check_attn(a) || a->splits == 1) return 0;
    return 4 * attn_part_floats(a->n_kv, a->n_heads / a->n_kv, a->head_dim, a->splits);
}

int rv12_rope_attn(const rv12_attn* a, const float* qkv, const float* qn, const float* kn, const float* inv,
                   const int64_t* pos, void* kc, void* vc, float* out, void* ws, size_t ws_bytes, void* stream) {
    int rc = check_attn(a);
    if (rc) return rc;
    if (!qkv || !qn || !kn || !inv || !pos || !kc || !vc || !out) return RV12_E_NULL;
    if (!aligned16(qkv) || !aligned16(kc) || !aligned16(vc) || !aligned16(out)) return RV12_E_ALIGN;
    const size_t need = rv12_attn_workspace_bytes(a);
    if (need && (!ws || ws_bytes < need)) return RV12_E_WORKSPACE;
    AttnParams p;
    p.qkv = qkv;
    p.qn = qn;
    p.kn = kn;
    p.inv = inv;
    p.pos = pos;
    p.kc = kc;
    p.vc = vc;
    p.out = out;
    p.part = (float*)ws;
    p.n_heads = a->n_heads;
    p.n_kv = a->n_kv;
    p.head_dim = a->head_dim;
    p.maxt = a->maxt;
    p.kv_bf16 = a->kv_bf16 ? 1 : 0;
    p.eps = a->eps;
    p.scale = a->scale;
    if (launch_attn(p, a->splits, (hipStream_t)stream)) return RV12_E_CONFIG;
    return launch_status();
}

size_t rv12_attn_batch_workspace_bytes(const rv12_attn* a, int t) {
    if (check_attn(a) || t < 1 || t > 16) return 0;
    const size_t q = align256((size_t)t * a->n_heads * a->head_dim * 4);
    const size_t rows = (size_t)t * (a->n_heads / a->n_kv);
    return q + (a->splits > 1 ? 4 * (size_t)a->n_kv * a->splits * rows * (a->head_dim + 2) : 0);
}

int rv12_rope_attn_batch(const rv12_attn* a, int t, const float* qkv, const float* qn, const float* kn,
                         const float* inv, const int64_t* pos, void* kc, void* vc, float* out, void* ws,
                         size_t ws_bytes, void* stream) {
    int rc = check_attn(a);
    if (rc) return rc;
    if (t < 1 || t > 16) return RV12_E_TOKENS;
    if (!qkv || !qn || !kn || !inv || !pos || !kc || !vc || !out) return RV12_E_NULL;
    if (!aligned16(qkv) || !aligned16(kc) || !aligned16(vc) || !aligned16(out)) return RV12_E_ALIGN;
    const size_t need = rv12_attn_batch_workspace_bytes(a, t);
    if (!need) return RV12_E_CONFIG;
    if (!ws || ws_bytes < need) return RV12_E_WORKSPACE;
    if (!aligned16(ws)) return RV12_E_ALIGN;
    AttnParams p;
    p.qkv = qkv;
    p.qn = qn;
    p.kn = kn;
    p.inv = inv;
    p.pos = pos;
    p.kc = kc;
    p.vc = vc;
    p.out = out;
    p.qo = (float*)ws;
    p.part = (float*)((char*)ws + align256((size_t)t * a->n_heads * a->head_dim * 4));
    p.n_heads = a->n_heads;
    p.n_kv = a->n_kv;
    p.head_dim = a->head_dim;
    p.maxt = a->maxt;
    p.kv_bf16 = a->kv_bf16 ? 1 : 0;
    p.eps = a->eps;
    p.scale = a->scale;
    p.T = t;
    // at most one workgroup per CU: n_kv S <= 256 (Qwen3-32B 8-token pass at
    // 4k positions: 212.6 us per layer with 53 splits, 200.7 with 32, 202.5
    // with 24, 225.9 with 8)
    const int S = std::min(a->splits, std::max(1, (256 + a->n_kv - 1) / a->n_kv));
    if (launch_attn_batch(p, S, (hipStream_t)stream)) return RV12_E_CONFIG;
    return launch_status();
}


// the prompt attention ignores splits: its workgroups cover 16 tokens, not a
// position range; every 32-bit byte offset of its loads stays below 2^31
static int check_prefill_attn(const rv12_attn* a, int t) {
    if (!a) return RV12_E_NULL;
    if (a->head_dim != 64 && a->head_dim != 128) return RV12_E_SHAPE;
    if (a->n_kv < 1 || a->n_heads < a->n_kv || a->n_heads % a->n_kv) return RV12_E_SHAPE;
    const int g = a->n_heads / a->n_kv;
    if (g != 1 && g != 2 && g != 4 && g != 8) return RV12_E_SHAPE;
    if (a->maxt < 1 || (int64_t)a->maxt * a->head_dim * (a->kv_bf16 ? 2 : 4) >= ((int64_t)1 << 31))
        return RV12_E_SHAPE;
    if (t < 1 || t > kMaxPrefillAttnTokens || (int64_t)(t + 15) * a->n_heads * a->head_dim * 4 >= ((int64_t)1 << 31))
        return RV12_E_TOKENS;
    return RV12_OK;
}

size_t rv12_prefill_attn_workspace_bytes(const rv12_attn* a, int t) {
    if (check_prefill_attn(a, t)) return 0;
    return (size_t)t * a->n_heads * a->head_dim * 4;
}

int rv12_prefill_rope_attn(const rv12_attn* a, int t, const float* qkv, const float* qn, const float* kn,
                           const float* inv, const int64_t* pos, void* kc, void* vc, float* out, void* ws,
                           size_t ws_bytes, void* stream) {
    int rc = check_prefill_attn(a, t);
    if (rc) return rc;
    if (!qkv || !qn || !kn || !inv || !pos || !kc || !vc || !out) return RV12_E_NULL;
    if (!aligned16(qkv) || !aligned16(kc) || !aligned16(vc) || !aligned16(out)) return RV12_E_ALIGN;
    const size_t need = rv12_prefill_attn_workspace_bytes(a, t);
    if (!ws || ws_bytes < need) return RV12_E_WORKSPACE;
    if (!aligned16(ws)) return RV12_E_ALIGN;
    AttnParams p;
    p.qkv = qkv;
    p.qn = qn;
    p.kn = kn;
    p.inv = inv;
    p.pos = pos;
    p.kc = kc;
    p.vc = vc;
    p.out = out;
    p.qo = (float*)ws;
    p.part = nullptr;
    p.n_heads = a->n_heads;
    p.n_kv = a->n_kv;
    p.head_dim = a->head_dim;
    p.maxt = a->maxt;
    p.kv_bf16 = a->kv_bf16 ? 1 : 0;
    p.eps = a->eps;
    p.scale = a->scale;
    p.T = t;
    if (launch_prefill_attn(p, (hipStream_t)stream)) return RV12_E_CONFIG;
    return launch_status();
}

}  // extern "C"
