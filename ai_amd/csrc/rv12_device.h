// Device-side helpers shared by the rv12 kernels (gfx950).
//
// Q16 layout (written by k_retile, read by every other kernel)
// -------------------------------------------------------------
// Rows are grouped in blocks of 16, K in steps of 32.  For row block b, step s
// and lane l (0..63) one 12-byte group holds the 8 weights of row 16b + l%16 at
// k = 32s + 8(l/16) + 0..7.  The groups of one (b, s) are contiguous
// (64 x 12 = 768 bytes, one coalesced buffer_load_dwordx3 per wave), the steps
// of one row block follow each other (K/32 * 768 bytes per row block), and the
// lane -> (row, k) map is the A-operand map of v_mfma_f32_16x16x32_bf16.
//
// Each weight is kept as a 16-bit "h" = sign << 15 | c << 7 | mantissa7 with a
// 4-bit exponent field c in bits 7..10.  With sc = max(base - 1, 0):
//   c = e - sc        weight in the window (e = biased exponent, code = e - base)
//   h = 0             exception (its value is in the codec's ev list)
// For base >= 1 every in-window weight has c = code + 1 >= 1, so h = 0 marks
// exactly the exceptions; for base = 0, c = e and the zero / subnormal weights
// of the window keep their own bits.  Read as the top half of a float32,
// h << 16 is the weight times 2^-sc, exactly, so a dot product can use the raw
// h values and rescale the sum once by 2^sc.
// Weights 0..7 pair up as P0 = h0 | h1 << 16 ... P3 = h6 | h7 << 16.  The pairs
// never use bits 11..14 and 27..30, so three dwords carry four pairs:
//   D0 = P0 | (P3 & 0x000F000F) << 11
//   D1 = P1 | (P3 & 0x00F000F0) << 7
//   D2 = P2 | (P3 & 0x07000700) << 3 | (P3 & 0x80008000) >> 1
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rv12_internal.h"

namespace rv12 {

typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kStepBytes = 768;       // one (row block, step) tile: 16 rows x 32 k x 1.5 bytes
constexpr int kStepWords = 192;
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data format (gfx9 family)
constexpr int kNonTemporal = 2;        // cache policy bits of a streaming load

// the four h-pairs of one 12-byte group
__device__ __forceinline__ void unpack_pairs(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t p[4]) {
    p[0] = d0 & 0x87FF87FFu;
    p[1] = d1 & 0x87FF87FFu;
    p[2] = d2 & 0x87FF87FFu;
    p[3] = ((d0 >> 11) & 0x000F000Fu) | ((d1 >> 7) & 0x00F000F0u) | ((d2 >> 3) & 0x07000700u) |
           ((d2 << 1) & 0x80008000u);
}

__device__ __forceinline__ float lo_f(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float hi_f(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }

// h -> original bf16 bits (exceptions come out as 0 and are scattered later)
__device__ __forceinline__ uint32_t h_to_bf16(uint32_t h, int sc) {
    const uint32_t c = (h >> 7) & 15u;
    return c ? ((h + ((uint32_t)sc << 7)) & 0xFFFFu) : h;
}

// Activation scaling.  The h values sit at the bottom of the float32 range
// (2^-126 <= |h| < 2^-111 for in-window weights), so the kernels multiply them
// by x' * 2^P, an exact power-of-two scaling folded back into the row's final
// 2^(sc - P):
//   fast path  P = 64, taken when every nonzero |x'| of the workgroup (of the
//              wave in the MFMA kernel) lies in [2^-64, 2^63): every product
//              with an in-window weight is a normal float below 2^16 and the
//              bf16 parts of x' * 2^64 stay finite;
//   slow path  otherwise: P = 100 - e, with e the float exponent (frexp) of the
//              largest finite nonzero |x'| of the token, so max |x'| * 2^P is
//              in [2^99, 2^100); values below max |x'| * 2^-225 are lost.
// The exception products ev * x' use x' itself (x' * 2^P * 2^-P is exact).
constexpr int kXScaleExp = 64;
constexpr int kXSlowExp = 100;
constexpr int kXRangeLo = -63;  // frexp exponent of 2^-64
constexpr int kXRangeHi = 63;   // frexp exponent of the largest value below 2^63
constexpr float kXScale = 0x1p64f;
// The RMSNorm sum of squares runs over (x * 2^-32)^2 (exact scaling, the same
// sums where no square under- or overflows), so it stays finite up to
// |x| ~ 2^90; rs = 2^-32 / sqrt(S / K + eps * 2^-64).
constexpr float kSsqScale = 0x1p-32f;
constexpr float kSsqEpsScale = 0x1p-64f;

__device__ __forceinline__ void track_exp(float v, int& lo, int& hi) {
    const int e = __builtin_amdgcn_frexp_expf(v);  // 0 for zero, inf and NaN
    lo = min(lo, e);
    hi = max(hi, e);
}
__device__ __forceinline__ void track_exp4(const f32x4 v, int& lo, int& hi) {
    track_exp(v.x, lo, hi);
    track_exp(v.y, lo, hi);
    track_exp(v.z, lo, hi);
    track_exp(v.w, lo, hi);
}
// exponent of a finite nonzero value, else a value below any exponent
__device__ __forceinline__ int exp_or_min(float v) {
    return (v != 0.0f && __builtin_isfinite(v)) ? __builtin_amdgcn_frexp_expf(v) : -1000;
}
__device__ __forceinline__ int slow_scale_exp(int emax) { return emax < -500 ? kXScaleExp : kXSlowExp - emax; }
__device__ __forceinline__ float rms_scale(float ssq, int K, float eps) {
    return kSsqScale * (1.0f / sqrtf(ssq / (float)K + eps * kSsqEpsScale));
}

// greedy pick order: (av, ai) replaces (bv, bi) when av is larger, or equal
// with a smaller index; NaN counts as larger than any number (the first NaN
// wins), as torch.argmax orders them
__device__ __forceinline__ bool pick_beats(float av, int ai, float bv, int bi) {
    const bool an = av != av, bn = bv != bv;
    if (an || bn) return an && (!bn || ai < bi);
    return av > bv || (av == bv && ai < bi);
}

// a float rounded to bf16 (nearest even), as bits; the value of bf16 bits
__device__ __forceinline__ uint32_t bf16_bits(float v) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v);
}
__device__ __forceinline__ float bf16_value(uint32_t b) { return __uint_as_float(b << 16); }

// split 8 values into three bf16x8 parts (as u32x4) with hi + mid + lo = v to 24 bits
__device__ __forceinline__ void split3(const float (&v)[8], u32x4& hi, u32x4& mid, u32x4& lo) {
    uint32_t h[8], m[8], l[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        h[e] = bf16_bits(v[e]);
        const float r1 = v[e] - bf16_value(h[e]);
        m[e] = bf16_bits(r1);
        const float r2 = r1 - bf16_value(m[e]);
        l[e] = bf16_bits(r2);
    }
    hi = u32x4{h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16};
    mid = u32x4{m[0] | m[1] << 16, m[2] | m[3] << 16, m[4] | m[5] << 16, m[6] | m[7] << 16};
    lo = u32x4{l[0] | l[1] << 16, l[2] | l[3] << 16, l[4] | l[5] << 16, l[6] | l[7] << 16};
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// one v_mfma_f32_16x16x32_bf16: c + a . b, a and b eight bf16 values per lane
__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

// four bf16 values (bits) as floats
__device__ __forceinline__ f32x4 bf16x4_to_f32(uint2 b) {
    return f32x4{__uint_as_float(b.x << 16), __uint_as_float(b.x & 0xFFFF0000u), __uint_as_float(b.y << 16),
                 __uint_as_float(b.y & 0xFFFF0000u)};
}

// silu(g) * u with the hardware exp2 and reciprocal (about 2 ulp each)
__device__ __forceinline__ float silu_mul(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);
    return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// Lane exchanges on the VALU, no LDS round trip: DPP within rows of 16 lanes,
// the gfx950 lane swaps across rows.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7 - i within 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15 - i within 16
// the two 16-lane rows of each 32-lane half, then the two halves, combined
// with op into every lane
template <typename Op>
__device__ __forceinline__ float rows_and_halves(float v, Op op) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return op(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)kRsrcWord3);
}

// one 12-byte group; a load through a descriptor of 0 bytes (or past its
// end) returns zeros without touching memory
__device__ __forceinline__ u32x3 load_group(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_amdgcn_raw_buffer_load_b96(r, voff, soff, kNonTemporal);
}

}  // namespace rv12
