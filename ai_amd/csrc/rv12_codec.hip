// rv12 codec kernels for gfx950.
//   encode   the reference 12-bit codec dict of a bf16 matrix: exponent
//            histogram, m8/e4, row-major exception list (k_hist,
//            k_encode_rows, k_encode_exc)
//   to_bf16  a codec dict back to bf16 bits (k_codec_to_bf16 + k_scatter_exc)
//   pack     bf16 bits -> the Q16 layout with one exponent window per row and
//            that layout's own exception list (k_row_base, k_pack_count,
//            k_pack_tiles, k_encode_exc)
//   decode   Q16 rows back to the exact bf16 / float32 values (k_decode,
//            k_decode_exc)
// The Q16 layout and the h encoding are described in rv12_device.h.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rv12_device.h"
#include "rv12_internal.h"

namespace rv12 {

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
// (base = rbase[n] when rbase is given: the row windows of the packed form)
__global__ __launch_bounds__(256) void k_encode_exc(const uint16_t* __restrict__ w, int K, int base,
                                                    const int32_t* __restrict__ rbase,
                                                    const int32_t* __restrict__ rp, int32_t* __restrict__ er,
                                                    int32_t* __restrict__ ec, float* __restrict__ ev) {
    const int n = blockIdx.x;
    if (rbase) base = rbase[n];
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

// ------------------------------------------------------------------ to_bf16
// one thread per 8 weights of a codec dict: code 15 (an exception) -> 0 bits
__global__ __launch_bounds__(256) void k_codec_to_bf16(const uint8_t* __restrict__ m8, const uint8_t* __restrict__ e4,
                                                       int K, int CH, int base, int64_t groups,
                                                       uint16_t* __restrict__ w) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= groups) return;
    const int64_t i0 = gid * 8;  // K % 8 == 0: the 8 weights share a row and a half-chunk
    const int64_t n = i0 / K;
    const int k0 = (int)(i0 % K);
    const int half = CH / 2;
    const int c = k0 / CH, i = k0 % CH;
    const uint8_t* erow = e4 + n * (K / 2) + (int64_t)c * half + (i % half);
    const int shift = i < half ? 0 : 4;
    uint32_t b[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t m = m8[i0 + j];
        const uint32_t code = (erow[j] >> shift) & 15u;
        b[j] = code == 15u ? 0u : ((m >> 7) << 15) | ((code + (uint32_t)base) << 7) | (m & 0x7Fu);
    }
    *reinterpret_cast<uint4*>(w + i0) = make_uint4(b[0] | b[1] << 16, b[2] | b[3] << 16, b[4] | b[5] << 16,
                                                   b[6] | b[7] << 16);
}

// exact exception values into a bf16 matrix
// (entries outside the matrix are skipped)
__global__ __launch_bounds__(256) void k_scatter_exc(const int32_t* __restrict__ er, const int32_t* __restrict__ ec,
                                                     const float* __restrict__ ev, int64_t E, int N, int K,
                                                     uint16_t* __restrict__ w) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= E) return;
    const int r = er[j], c = ec[j];
    if (r < 0 || r >= N || c < 0 || c >= K) return;
    w[(int64_t)r * K + c] = (uint16_t)(__float_as_uint(ev[j]) >> 16);
}

// ------------------------------------------------------------------ pack
// one workgroup per row: the row's exponent window, chosen by the reference's
// rule for a whole matrix (wcomp.py:19-21): the first start b whose 15-wide
// window [b, b+14] holds the most weights
__global__ __launch_bounds__(256) void k_row_base(const uint16_t* __restrict__ w, int K, int32_t* __restrict__ rbase) {
    __shared__ int32_t h[256];
    __shared__ int32_t win[256];
    const int64_t n = blockIdx.x;
    h[threadIdx.x] = 0;
    __syncthreads();
    const uint16_t* row = w + n * (int64_t)K;
    for (int k = threadIdx.x * 8; k < K; k += blockDim.x * 8) {
        const uint4 v = *reinterpret_cast<const uint4*>(row + k);
        const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            atomicAdd(&h[(d[j] >> 7) & 0xFF], 1);
            atomicAdd(&h[(d[j] >> 23) & 0xFF], 1);
        }
    }
    __syncthreads();
    int sum = 0;
    if (threadIdx.x <= 241)
        for (int j = 0; j < 15; ++j) sum += h[threadIdx.x + j];
    win[threadIdx.x] = threadIdx.x <= 241 ? sum : -1;
    __syncthreads();
    if (threadIdx.x == 0) {
        int best = 0;
        for (int j = 1; j <= 241; ++j)
            if (win[j] > win[best]) best = j;
        rbase[n] = best;
    }
}

// one workgroup per row: weights outside the row's window
__global__ __launch_bounds__(256) void k_pack_count(const uint16_t* __restrict__ w, int K,
                                                    const int32_t* __restrict__ rbase,
                                                    int32_t* __restrict__ row_exc) {
    const int n = blockIdx.x;
    const int base = rbase[n];
    const uint16_t* row = w + (int64_t)n * K;
    int cnt = 0;
    for (int k = threadIdx.x * 8; k < K; k += blockDim.x * 8) {
        const uint4 v = *reinterpret_cast<const uint4*>(row + k);
        const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c0 = (int)((d[j] >> 7) & 0xFF) - base, c1 = (int)((d[j] >> 23) & 0xFF) - base;
            cnt += (c0 < 0 || c0 > 14) + (c1 < 0 || c1 > 14);
        }
    }
    __shared__ int red[4];
    for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = cnt;
    __syncthreads();
    if (threadIdx.x == 0) {
        int t = 0;
        for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += red[i];
        row_exc[n] = t;
    }
}

// one thread per 12-byte group (row block b, step s, lane l): the 8 weights of
// row 16b + l%16 at k = 32s + 8(l/16) + 0..7 as h values of the row's window
__global__ __launch_bounds__(256) void k_pack_tiles(const uint16_t* __restrict__ w, int N, int K,
                                                    const int32_t* __restrict__ rbase, uint32_t* __restrict__ tiles,
                                                    int64_t groups) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
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
        const int base = rbase[n];
        const uint32_t off = (uint32_t)(base - scale_exp(base));  // c = code + off
        const uint4 v = *reinterpret_cast<const uint4*>(w + n * K + k0);
        const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t bits = (d[j >> 1] >> ((j & 1) * 16)) & 0xFFFFu;
            const int code = (int)((bits >> 7) & 0xFF) - base;
            h[j] = (code < 0 || code > 14) ? 0u : (bits & 0x807Fu) | (((uint32_t)code + off) << 7);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = 0u;
    }
    const uint32_t p0 = h[0] | (h[1] << 16), p1 = h[2] | (h[3] << 16), p2 = h[4] | (h[5] << 16),
                   p3 = h[6] | (h[7] << 16);
    uint32_t* o = tiles + gid * 3;
    o[0] = p0 | ((p3 & 0x000F000Fu) << 11);
    o[1] = p1 | ((p3 & 0x00F000F0u) << 7);
    o[2] = p2 | ((p3 & 0x07000700u) << 3) | ((p3 & 0x80008000u) >> 1);
}

// ------------------------------------------------------------------ decode
// one thread per 12-byte group of the row blocks covering [first, last)
__global__ __launch_bounds__(256) void k_decode(const uint32_t* __restrict__ tiles,
                                                const int32_t* __restrict__ rbase, int K, int first, int last,
                                                int64_t b0, int64_t groups, void* __restrict__ out, int out_f32) {
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
    const int sc = scale_exp(rbase[n]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[2 * j] = h_to_bf16(p[j] & 0xFFFFu, sc);
        v[2 * j + 1] = h_to_bf16(p[j] >> 16, sc);
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

// ------------------------------------------------------------------ launch
void launch_codec_to_bf16(const rv12_codec& c, uint16_t* w, hipStream_t st) {
    const int64_t groups = (int64_t)c.n * c.k / 8;
    hipLaunchKernelGGL(k_codec_to_bf16, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st, c.m8, c.e4, c.k,
                       c.ch, c.base, groups, w);
    if (c.n_exc > 0)
        hipLaunchKernelGGL(k_scatter_exc, dim3((unsigned)((c.n_exc + 255) / 256)), dim3(256), 0, st, c.er, c.ec,
                           c.ev, c.n_exc, c.n, c.k, w);
}

void launch_pack_plan(const uint16_t* w, int N, int K, int32_t* rbase, int32_t* row_exc, hipStream_t st) {
    hipLaunchKernelGGL(k_row_base, dim3((unsigned)N), dim3(256), 0, st, w, K, rbase);
    hipLaunchKernelGGL(k_pack_count, dim3((unsigned)N), dim3(256), 0, st, w, K, rbase, row_exc);
}

void launch_pack(const uint16_t* w, int N, int K, const int32_t* rbase, const int32_t* rp, uint32_t* tiles,
                 int32_t* er, int32_t* ec, float* ev, int64_t n_exc, hipStream_t st) {
    const int64_t groups = (int64_t)((N + 15) / 16) * (K / 32) * 64;
    hipLaunchKernelGGL(k_pack_tiles, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st, w, N, K, rbase, tiles,
                       groups);
    if (n_exc > 0)
        hipLaunchKernelGGL(k_encode_exc, dim3((unsigned)N), dim3(256), 0, st, w, K, 0, rbase, rp, er, ec, ev);
}

void launch_decode(const rv12_matrix& w, int first, int last, void* out, int out_f32, hipStream_t st,
                   int64_t e0, int64_t e1) {
    const int64_t b0 = first / 16, b1 = (last + 15) / 16;
    const int64_t groups = (b1 - b0) * (w.k / 32) * 64;
    hipLaunchKernelGGL(k_decode, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st, w.tiles, w.rbase, w.k,
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
    hipLaunchKernelGGL(k_encode_exc, dim3((unsigned)N), dim3(256), 0, st, w, K, base, nullptr, rp, er, ec, ev);
}

}  // namespace rv12
