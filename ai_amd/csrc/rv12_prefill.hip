// rv12 prefill linear: the 12-bit decode fused into a bf16x3 MFMA GEMM over
// all the prompt's tokens at once (gfx950).  Replaces the blocked prefill's
// decode_rows + fp32 GEMM (ramvi/engine/ramvi_engine/kernels/prefill.py:66-78,
// prefill_kernels.py:8-26 and 58-110): every weight is read once per prompt
// in its 12-bit form, never written back in a wider format.
//
// y[t] (=|+=) W_dec . x'[t], t < T, with the MODE prologue (2: x' =
// silu(x[0:K]) * x[K:2K]) or the RMSNorm prologue of mode 0 (x' = lnw x,
// the token's rs = 1 / sqrt(mean x^2 + eps) applied to its outputs, as the
// decode kernels apply it).  Three launches:
//   1. k_prefill_stats (one wave per token): each token's exponent scale
//      P_t (64 when its largest |x'| lies in [2^-40, 2^63), else 100 minus
//      the exponent of the largest) and, with RMS, its rs (sum of squares of
//      x 2^-32); k_prefill_parts (32 tokens x 64 columns per workgroup):
//      x' 2^P_t split into bf16 parts
//      hi + mid + lo (24 significand bits, as the reference's _x3 split,
//      wcomp.py:130-140) in B-operand lane order: for token block tb, step
//      s (32 columns) and part, 64 lanes x 8 bf16 (lane l: token l%16,
//      k = 8(l/16) + 0..7), and x' itself in fp32, transposed (column-major
//      over the padded tokens).  Token rows past T are zeros.
//   2. k_prefill_mm: workgroup = 256 rows x 128 tokens, 8 waves of 64 rows x
//      64 tokens.  Per 32-column step the workgroup's 16 row blocks' Q16
//      tiles (the A operand of v_mfma_f32_16x16x32_bf16, the h values
//      w 2^-sc) and the B parts of its 8 token blocks go from memory straight
//      into a ring of four LDS slots (buffer loads with the LDS destination;
//      no register holds them on the way, every wait is explicit), three
//      steps ahead; one wait + barrier per step; each wave reads the next
//      step's fragments while its 48 MFMAs of the current step run; the MFMAs
//      accumulate in 16 independent fp32 accumulators.  Epilogue:
//      v = acc 2^(sc_row - P_t) (exact); the packed form's exception entries
//      of the wave's rows (weights outside a row's window, zeros in the
//      tiles) add ev * x'[t][col] in list order, x' read from the transposed
//      copy (one column of the wave's 64 tokens is 256 contiguous bytes,
//      where the rows of x would take a cache line per token); with RMS v is
//      scaled by rs_t; then y is stored or added; rows past N and tokens past
//      T are skipped.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rv12_device.h"
#include "rv12_internal.h"

namespace rv12 {

constexpr int kPfRowBlocks = 16;  // row blocks (of 16 rows) per workgroup
constexpr int kPfTokBlocks = 8;   // token blocks (of 16 tokens) per workgroup
constexpr int kPfThreads = 512;
// wave tile: kPfWB row blocks x kPfWT token blocks (8 waves: 16 / kPfWB along
// the rows times 8 / kPfWT along the tokens)
constexpr int kPfWB = 4;
constexpr int kPfWR = kPfRowBlocks / kPfWB;                          // waves along the rows
constexpr int kPfWT = kPfTokBlocks / (kPfThreads / 64 / kPfWR);  // token blocks per wave
static_assert(kPfWR * (kPfTokBlocks / kPfWT) == kPfThreads / 64, "8 waves cover the workgroup tile");
constexpr int kPfRing = 4;  // LDS slots: the A tiles and B parts of steps s .. s + 3
// slot layout (u32x4 units): 16 A tiles of 1 KB (a 12-byte-per-lane load with
// the LDS destination writes lane l at 16 l: 768 B of each KB), then the B
// parts (8 token blocks x 3 parts x 64 lanes)
constexpr int kPfSlotA = kPfRowBlocks * 64;
constexpr int kPfSlot = kPfSlotA + kPfTokBlocks * 3 * 64;  // 40 KB
constexpr size_t kPfLds = (size_t)kPfRing * kPfSlot * 16;   // 160 KB
static_assert(kPfLds <= 160 * 1024, "gfx950 LDS per workgroup");
// loads a wave issues per step: 2 A tiles and 3 B chunks, all into LDS
constexpr int kPfOpsPerStep = kPfRowBlocks / (kPfThreads / 64) + 3;
// at the top of step s, the wave's loads of step s + 1 (issued at step
// s + 1 - kPfRing) are followed by those of the kPfRing - 2 steps between
constexpr int kPfWait = kPfOpsPerStep * (kPfRing - 2);
static_assert(kPfWait < 64, "vmcnt holds 6 bits");
// s_waitcnt immediates (gfx9 encoding): vmcnt(n) and lgkmcnt(0), expcnt not
// waited for; vmcnt(n) alone
constexpr int waitcnt_vm_lgkm0(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }
constexpr int waitcnt_vm(int n) { return waitcnt_vm_lgkm0(n) | (15 << 8); }

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

// 1a. k_prefill_stats: one wave per token (4 per workgroup, a grid over the
// padded tokens): the largest exponent of |x'| and, with RMS, the sum of
// squares of x 2^-32, lane l over columns 8 l + 512 i, reduced across the
// wave in a fixed order; writes the token's scale exponent P_t and rs_t.
constexpr int kPsThreads = 256;
__global__ __launch_bounds__(kPsThreads) void k_prefill_stats(const float* __restrict__ x, int T, int K, int xs,
                                                              int m2, const uint16_t* __restrict__ lnw, float eps,
                                                              int* __restrict__ P, float* __restrict__ R) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * (kPsThreads / 64) + (threadIdx.x >> 6);
    int e = -1000;
    float sq = 0.0f;
    if (t < T) {
        const float* xr = x + (int64_t)t * xs;
        for (int k = lane * 8; k < K; k += 512) {
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
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        e = max(e, __shfl_xor(e, o));
        sq += __shfl_xor(sq, o);
    }
    if (lane == 0) {
        P[t] = (e >= -39 && e <= kXRangeHi) ? kXScaleExp : slow_scale_exp(e);
        if (lnw) R[t] = rms_scale(sq, K, eps);
    }
}

// 1b. k_prefill_parts: grid (32-token blocks, 64-column chunks), 256 threads,
// thread (token tok, 8-column group k8): x' (prologue applied) of token t at
// columns kc .. kc + 7 written transposed (per column, 32 consecutive tokens:
// full 128-byte lines), then x' 2^P_t split into the bf16 parts in B-operand
// lane order.  Tokens past T are zeros.
constexpr int kPpThreads = 256;
__global__ __launch_bounds__(kPpThreads) void k_prefill_parts(const float* __restrict__ x, int T, int K, int xs,
                                                              int m2, const uint16_t* __restrict__ lnw,
                                                              const int* __restrict__ P, u32x4* __restrict__ xb,
                                                              float* __restrict__ xt, int tp) {
    const int tok = threadIdx.x & 31, k8 = threadIdx.x >> 5;
    const int t = blockIdx.x * 32 + tok;
    const int kc = blockIdx.y * 64 + k8 * 8;
    if (kc >= K) return;
    const int nsteps = K >> 5;
    float v[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (t < T) prefill_xprime(x + (int64_t)t * xs, K, kc, m2 != 0, lnw, v);
    float* xc = xt + (int64_t)kc * tp + t;
#pragma unroll
    for (int i = 0; i < 8; ++i) xc[(int64_t)i * tp] = v[i];
    u32x4 hi = {0, 0, 0, 0}, mid = {0, 0, 0, 0}, lo = {0, 0, 0, 0};
    if (t < T) {
        const int p = P[t];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = ldexpf(v[i], p);
        split3(v, hi, mid, lo);
    }
    const int s = kc >> 5, g = (kc & 31) >> 3;  // step, 8-column group in the step
    u32x4* d = xb + ((int64_t)(t >> 4) * nsteps + s) * 192 + g * 16 + (t & 15);
    d[0] = hi;
    d[64] = mid;
    d[128] = lo;
}

// Workgroup i -> (row tile, token tile).  Workgroups are dispatched in order,
// round-robin over the 8 XCDs (each with its own L2): i runs on XCD i % 8 as
// its (i / 8)-th.  The virtual index v gives each XCD a contiguous range of
// G / 8 tiles (the remainder past 8 (G / 8) keeps v = i), and v runs over
// groups of kPfGroupRows row tiles x all token tiles, row tile fastest, so the
// ~32 workgroups an XCD holds at once cover 8 row tiles x 4 token tiles: per
// step their L2 misses are 8 A tiles (12 KB each) and 4 B sets (24 KB each),
// 192 KB, where 2 row tiles x 16 token tiles (the Qwen3-8B o and down in
// launch order) would miss 408 KB.  A bijection of [0, G).
constexpr int kPfGroupRows = 8;
__device__ __forceinline__ void prefill_tile(int i, int G, int nx, int ny, int& rt, int& tt) {
    const int g8 = G / 8;
    const int v = i < g8 * 8 ? (i % 8) * g8 + i / 8 : i;
    const int per = kPfGroupRows * ny;
    const int g = v / per, r0 = g * kPfGroupRows;
    const int gr = min(kPfGroupRows, nx - r0);
    const int w = v - g * per;
    tt = w / gr;
    rt = r0 + w % gr;
}

// 2. grid (row tiles of 256 rows x token tiles of 128, in the order above),
// 512 threads.  LN (the RMS prologue: each token's rs applied to its outputs)
// is a template argument; the prologues themselves were applied in the
// pre-pass, to the parts and to the transposed x' (xt, row stride tp).
template <bool LN>
__global__ __launch_bounds__(kPfThreads) void k_prefill_mm(const uint32_t* __restrict__ tiles,
                                                           const int32_t* __restrict__ rbase,
                                                           const u32x4* __restrict__ xb, const int* __restrict__ P,
                                                           const int32_t* __restrict__ rp,
                                                           const int32_t* __restrict__ er,
                                                           const int32_t* __restrict__ ec,
                                                           const float* __restrict__ ev, const float* __restrict__ xt,
                                                           int tp, const float* __restrict__ R, float* __restrict__ y,
                                                           float* __restrict__ part, int N, int K, int T, int add) {
    extern __shared__ u32x4 bs[];  // [kPfRing][kPfSlot]: A tiles and B parts of steps s .. s + 3
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave % kPfWR, wc = wave / kPfWR;
    const int nsteps = K >> 5;
    // K split blockIdx.y of gridDim.y: steps [s_lo, s_hi)
    const int S = gridDim.y, sp = blockIdx.y;
    const int s_lo = (int)((int64_t)sp * nsteps / S), s_hi = (int)((int64_t)(sp + 1) * nsteps / S);
    const int64_t nblk = (N + 15) / 16;
    const int nx = (int)((nblk + kPfRowBlocks - 1) / kPfRowBlocks);
    int rt, tt;
    prefill_tile(blockIdx.x, gridDim.x, nx, gridDim.x / nx, rt, tt);
    const int64_t blk0 = (int64_t)rt * kPfRowBlocks + wr * kPfWB;  // this wave's first row block
    const int tb0 = tt * kPfTokBlocks;                          // the workgroup's first token block
    const uint32_t blk_bytes = (uint32_t)nsteps * kStepBytes;
    typedef __attribute__((address_space(3))) void* lds_ptr;
    // the workgroup's A tiles: wave w loads row blocks 2w and 2w + 1 of the
    // workgroup through a descriptor over its valid row blocks (a row block
    // past N, or a step past the end through the 0-byte descriptor, reads
    // zeros)
    const int64_t wblk0 = (int64_t)rt * kPfRowBlocks;
    const int nvalid_wg = (int)max((int64_t)0, min((int64_t)kPfRowBlocks, nblk - wblk0));
    const char* wgbase = reinterpret_cast<const char*>(tiles) + wblk0 * (int64_t)blk_bytes;
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(wgbase, (uint32_t)nvalid_wg * blk_bytes);
    const __amdgpu_buffer_rsrc_t rnull = make_rsrc(wgbase, 0u);
    constexpr int kAPerWave = kPfRowBlocks / (kPfThreads / 64);
    int aoff[kAPerWave];
#pragma unroll
    for (int i = 0; i < kAPerWave; ++i) aoff[i] = (int)((wave * kAPerWave + i) * blk_bytes) + lane * 12;
    // the B parts of the workgroup's token blocks: 3 chunks of 64 lanes x
    // 16 B per wave, through a descriptor over the workgroup's parts
    const u32x4* xbw = xb + (int64_t)tb0 * nsteps * 192;
    const __amdgpu_buffer_rsrc_t rbx = make_rsrc(xbw, (uint32_t)kPfTokBlocks * nsteps * 192 * 16);
    const __amdgpu_buffer_rsrc_t rbnull = make_rsrc(xbw, 0u);
    int boff[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int idx = tid + j * kPfThreads;  // (token block, part, lane) of the step
        boff[j] = ((idx / 192) * nsteps * 192 + idx % 192) * 16;
    }
    // step s's A tiles and B parts into LDS slot `slot`; a step past the end
    // goes through the 0-byte descriptors, which write zeros, so the loop has
    // no branch around a load
    auto load_step = [&](int slot, int j) {  // step s_lo + j
        const int s = s_lo + j;
        const bool in = s < s_hi;
        const __amdgpu_buffer_rsrc_t ra = in ? rv : rnull, rb = in ? rbx : rbnull;
        const int sa = (in ? s : 0) * kStepBytes, sb = (in ? s : 0) * 192 * 16;
        u32x4* d = bs + slot * kPfSlot;
#pragma unroll
        for (int i = 0; i < kAPerWave; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr)(d + (wave * kAPerWave + i) * 64), 12, aoff[i], sa,
                                                     0, 0);
#pragma unroll
        for (int j = 0; j < 3; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr)(d + kPfSlotA + wave * 64 + j * kPfThreads), 16,
                                                     boff[j], sb, 0, 0);
    };
    // this wave's fragments of the step in slot `slot`: its 4 row blocks' A
    // groups (12 bytes per lane) and 3 parts x 4 token blocks of B,
    // part-major so the first part's MFMAs wait only for its own reads
    auto read_frags = [&](u32x3 (&ra)[kPfWB], u32x4 (&rb)[3][kPfWT], int slot) {
        const u32x4* d = bs + slot * kPfSlot;
#pragma unroll
        for (int b = 0; b < kPfWB; ++b) ra[b] = *reinterpret_cast<const u32x3*>(d + (wr * kPfWB + b) * 64 + lane);
        const u32x4* src = d + kPfSlotA + (wc * kPfWT) * 192 + lane;
#pragma unroll
        for (int q = 0; q < 3; ++q)
#pragma unroll
            for (int c = 0; c < kPfWT; ++c) rb[q][c] = src[c * 192 + q * 64];
    };

    f32x4 acc[kPfWB][kPfWT];
#pragma unroll
    for (int b = 0; b < kPfWB; ++b)
#pragma unroll
        for (int c = 0; c < kPfWT; ++c) acc[b][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // prologue: steps 0-3 into slots 0-3, all landed; step 0's fragments read
#pragma unroll
    for (int i = 0; i < kPfRing; ++i) load_step(i, i);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    u32x3 fa[2][kPfWB];
    u32x4 fb[2][3][kPfWT];
    read_frags(fa[0], fb[0], 0);

    // Step s, software-pipelined: wait for this wave's loads of step s + 1
    // and for its fragment reads of step s; barrier (every wave's loads of
    // step s + 1 have landed, and every wave is done reading slot s % 4);
    // step s + 4 into that slot; the fragments of step s + 1 read while the
    // A groups of step s are unpacked and its 48 MFMAs run.  The loop runs
    // whole rounds of the unroll: steps past the split read zeros (A and B) and
    // add nothing.
    const int nround = (s_hi - s_lo + kPfRing - 1) / kPfRing * kPfRing;
    for (int s0 = 0; s0 < nround; s0 += kPfRing) {
#pragma unroll
        for (int u = 0; u < kPfRing; ++u) {
            const int s = s0 + u;
            // (the empty asm statements keep every LDS access on its side of
            // the wait and the barrier: neither builtin orders memory)
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(kPfWait));
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            load_step(u, s + kPfRing);
            read_frags(fa[(u + 1) & 1], fb[(u + 1) & 1], (u + 1) % kPfRing);
            // the reads are issued here, ahead of the MFMAs they overlap
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            u32x4 a[kPfWB];
#pragma unroll
            for (int b = 0; b < kPfWB; ++b) {
                uint32_t pr[4];
                unpack_pairs(fa[u & 1][b].x, fa[u & 1][b].y, fa[u & 1][b].z, pr);
                a[b] = u32x4{pr[0], pr[1], pr[2], pr[3]};
            }
#pragma unroll
            for (int q = 0; q < 3; ++q)
#pragma unroll
                for (int b = 0; b < kPfWB; ++b)
#pragma unroll
                    for (int c = 0; c < kPfWT; ++c) acc[b][c] = mfma(a[b], fb[u & 1][q][c], acc[b][c]);
        }
    }
    // the last loads (zeros into slots nobody reads) land before the
    // workgroup's LDS can be handed on
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));

    // epilogue: lane l holds token 16 c + l%16 and rows 4(l/16) + 0..3 of each tile
    const int q = lane >> 4, jj = lane & 15;
    // (a) rescale: v = acc 2^(sc_row - P_t), exact
    float v[kPfWB][kPfWT][4];
    int tok[kPfWT];
#pragma unroll
    for (int c = 0; c < kPfWT; ++c) {
        tok[c] = (tb0 + wc * kPfWT + c) * 16 + jj;
        const int pt = tok[c] < T ? P[tok[c]] : 0;
#pragma unroll
        for (int b = 0; b < kPfWB; ++b) {
            const int64_t n = (blk0 + b) * 16 + q * 4;
            const float av[4] = {acc[b][c].x, acc[b][c].y, acc[b][c].z, acc[b][c].w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                v[b][c][i] = ldexpf(av[i], scale_exp(rbase[min(n + i, (int64_t)N - 1)]) - pt);
        }
    }
    // (b) the exceptions of the wave's 64 rows (the tiles hold zeros there), in
    // list order, 8 entries at a time, the next batch's metadata and x'
    // gathers issued before the current one is added: each entry's row,
    // column and value are wave-uniform (scalar loads), x' of the lane's 4
    // tokens at its column comes from the transposed copy (the wave's 64
    // tokens of one column: 256 contiguous bytes), and a switch on the row's
    // (row block, row) slot adds the product to that output only, in the
    // lanes of the row's quarter
    const int64_t rlo = blk0 * 16;
    if (rlo < N) {
        const int32_t e_lo = rp[rlo], e_hi = rp[min(rlo + 16 * kPfWB, (int64_t)N)];
        constexpr int EB = 8;
        const float* xtw = xt + (int64_t)(tb0 + wc * kPfWT) * 16 + jj;  // token block c at + 16 c
        // (with a K split, the entries whose column lies in the split's steps)
        const int c_lo = s_lo * 32, c_hi = s_hi * 32;
        int nr[EB];
        bool nin[EB];
        float nv[EB], ng[EB][kPfWT];
        auto fetch = [&](int32_t e0) {
#pragma unroll
            for (int j = 0; j < EB; ++j) {
                const int32_t e = min(e0 + j, e_hi - 1);
                nr[j] = (int)(er[e] - rlo);
                nv[j] = ev[e];
                const int col = ec[e];
                nin[j] = col >= c_lo && col < c_hi;
                const float* xc = xtw + (int64_t)col * tp;
#pragma unroll
                for (int c = 0; c < kPfWT; ++c) ng[j][c] = xc[c * 16];
            }
        };
        // no entry for these rows (n_exc = 0 included, where er / ec / ev may
        // be null): nothing is fetched, so no index below e_lo is formed
        if (e_lo < e_hi) fetch(e_lo);
        for (int32_t e0 = e_lo; e0 < e_hi; e0 += EB) {
            int rr[EB];
            bool rin[EB];
            float evv[EB], xv[EB][kPfWT];
#pragma unroll
            for (int j = 0; j < EB; ++j) {
                rr[j] = nr[j];
                rin[j] = nin[j];
                evv[j] = nv[j];
#pragma unroll
                for (int c = 0; c < kPfWT; ++c) xv[j][c] = ng[j][c];
            }
            if (e0 + EB < e_hi) fetch(e0 + EB);
#pragma unroll
            for (int j = 0; j < EB; ++j) {
                if (e0 + j >= e_hi) break;
                if (!rin[j]) continue;
                const int r = rr[j];
                const bool mine = q == ((r & 15) >> 2);
#define RV12_EXC_CASE(B, I)                                                                 \
    case (B) * 4 + (I):                                                                     \
        if (mine) {                                                                         \
            _Pragma("unroll") for (int c = 0; c < kPfWT; ++c) v[B][c][I] += evv[j] * xv[j][c]; \
        }                                                                                   \
        break;
                static_assert(kPfWB == 4, "one case per (row block, row) slot of the wave");
                switch (((r >> 4) << 2) | (r & 3)) {
                    RV12_EXC_CASE(0, 0) RV12_EXC_CASE(0, 1) RV12_EXC_CASE(0, 2) RV12_EXC_CASE(0, 3)
                    RV12_EXC_CASE(1, 0) RV12_EXC_CASE(1, 1) RV12_EXC_CASE(1, 2) RV12_EXC_CASE(1, 3)
                    RV12_EXC_CASE(2, 0) RV12_EXC_CASE(2, 1) RV12_EXC_CASE(2, 2) RV12_EXC_CASE(2, 3)
                    RV12_EXC_CASE(3, 0) RV12_EXC_CASE(3, 1) RV12_EXC_CASE(3, 2) RV12_EXC_CASE(3, 3)
                    default: break;
                }
#undef RV12_EXC_CASE
            }
        }
    }
    // (c) with RMS the token's rs; store or add; rows past N and tokens past
    // T are skipped.  With a K split: the split's sums to part[sp][token][row]
    // (rs and the store or add are the reduce pass's)
    if (S > 1) {
        float* ps = part + (int64_t)sp * tp * N;
#pragma unroll
        for (int c = 0; c < kPfWT; ++c) {
            if (tok[c] >= T) continue;
#pragma unroll
            for (int b = 0; b < kPfWB; ++b) {
                const int64_t n = (blk0 + b) * 16 + q * 4;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (n + i < N) ps[(int64_t)tok[c] * N + n + i] = v[b][c][i];
            }
        }
        return;
    }
#pragma unroll
    for (int c = 0; c < kPfWT; ++c) {
        if (tok[c] >= T) continue;
        if constexpr (LN) {
            const float rs = R[tok[c]];
#pragma unroll
            for (int b = 0; b < kPfWB; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i) v[b][c][i] *= rs;
        }
#pragma unroll
        for (int b = 0; b < kPfWB; ++b) {
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

// 3. (K split only) y[t][n] (=|+=) rs_t * sum over the splits, in split order
__global__ __launch_bounds__(256) void k_prefill_reduce(const float* __restrict__ part, const float* __restrict__ R,
                                                        float* __restrict__ y, int64_t N, int T, int tp, int S,
                                                        int add) {
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (n >= N) return;
    for (int t = blockIdx.y; t < T; t += gridDim.y) {
        float v = 0.0f;
        for (int sp = 0; sp < S; ++sp) v += part[((int64_t)sp * tp + t) * N + n];
        if (R) v *= R[t];
        float* yp = y + (int64_t)t * N + n;
        *yp = add ? *yp + v : v;
    }
}

// K splits of the GEMM: the fewest that minimise a model of its rounds of
// workgroups (one per CU) — each round costs the steps of a split at 1.4 us
// plus 10 us — and of the reduce pass over the (S + 1) T N partial floats
// (3 us + bytes at 5 TB/s); no split below 8 steps
int prefill_splits(int N, int K, int T) {
    const int64_t nx = ((int64_t)N + 16 * kPfRowBlocks - 1) / (16 * kPfRowBlocks);
    const int64_t tp = prefill_tokens_padded(T);
    const int64_t G = nx * (tp / (kPfTokBlocks * 16));
    const int nsteps = K / 32;
    int best = 1;
    double best_us = 0.0;
    for (int S = 1; S <= 16; ++S) {
        if (S > 1 && nsteps / S < 8) break;
        const double rounds = (double)((G * S + 255) / 256);
        double us = rounds * ((double)nsteps / S * 1.4 + 10.0);
        if (S > 1) us += 3.0 + (double)(S + 1) * tp * N * 4 / 5e6;
        if (S == 1 || us < best_us) {
            best = S;
            best_us = us;
        }
    }
    return best;
}

size_t prefill_ws_bytes(int N, int K, int T) {
    const size_t tp = (size_t)prefill_tokens_padded(T);
    const int S = prefill_splits(N, K, T);
    // parts, P and R, transposed x', split partials
    return tp * (size_t)K * 10 + tp * 8 + (S > 1 ? (size_t)S * tp * (size_t)N * 4 : 0);
}

void launch_prefill(const rv12_matrix& w, const float* x, float* y, int T, int mode, const uint16_t* lnw, float eps,
                    void* ws, hipStream_t st) {
    const int K = w.k, N = w.n;
    const int tp = prefill_tokens_padded(T);
    u32x4* xb = reinterpret_cast<u32x4*>(ws);
    int* P = reinterpret_cast<int*>(reinterpret_cast<char*>(ws) + (size_t)tp * K * 6);
    float* R = reinterpret_cast<float*>(P + tp);
    float* xt = R + tp;
    float* part = xt + (size_t)tp * K;
    const int xs = mode == 2 ? 2 * K : K;
    const int m2 = mode == 2 ? 1 : 0;
    hipLaunchKernelGGL(k_prefill_stats, dim3(tp / (kPsThreads / 64)), dim3(kPsThreads), 0, st, x, T, K, xs, m2, lnw, eps,
                       P, R);
    hipLaunchKernelGGL(k_prefill_parts, dim3(tp / 32, (K + 63) / 64), dim3(kPpThreads), 0, st, x, T, K, xs, m2, lnw, P,
                       xb, xt, tp);
    const int S = prefill_splits(N, K, T);
    const int64_t nblk = ((int64_t)N + 15) / 16;
    const dim3 grid((unsigned)((nblk + kPfRowBlocks - 1) / kPfRowBlocks * (tp / (kPfTokBlocks * 16))), (unsigned)S);
    const auto kern = lnw ? k_prefill_mm<true> : k_prefill_mm<false>;
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)kPfLds);
    hipLaunchKernelGGL(kern, grid, dim3(kPfThreads), kPfLds, st, reinterpret_cast<const uint32_t*>(w.tiles), w.rbase, xb,
                       P, w.rp, w.er, w.ec, w.ev, xt, tp, R, y, part, N, K, T, mode != 0 ? 1 : 0);
    if (S > 1)
        hipLaunchKernelGGL(k_prefill_reduce, dim3((unsigned)((N + 255) / 256), (unsigned)min(T, 65535)), dim3(256), 0, st, part,
                           lnw ? R : nullptr, y, (int64_t)N, T, tp, S, mode != 0 ? 1 : 0);
}

}  // namespace rv12
