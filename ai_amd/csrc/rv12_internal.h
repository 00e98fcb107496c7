// Shared declarations of the rv12 kernels and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
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
    float* part;  // split partials [splits][T][npad]
    float* ssq;   // split sums of squares [splits][T]
    int N, K, npad, base, mode, xs;
    int64_t n_exc;
    float eps;
};

constexpr int kMaxSplits = 64;
constexpr int kMaxWaves = 16;
constexpr size_t kMaxLds = 65536;

// LDS bytes of k_linear for a launch shape (largest split)
inline size_t linear_lds_bytes(int K, int T, int rb, int waves, int splits) {
    const int nsteps = K / 32;
    const size_t krange = (size_t)((nsteps + splits - 1) / splits) * 32;
    return 4 * ((size_t)T * krange + (size_t)waves * rb * T * 16 + (size_t)waves * rb * 16 * T + (size_t)waves * T);
}

int launch_linear(const LinearParams& p, int T, int rb, int waves, int splits, hipStream_t st);
void launch_retile(const uint8_t* m8, const uint8_t* e4, int N, int K, int CH, int base, uint32_t* tiles,
                   hipStream_t st);
void launch_decode(const rv12_matrix& w, int first, int last, void* out, int out_f32, hipStream_t st, int64_t e0,
                   int64_t e1);
void launch_encode_stats(const uint16_t* w, int64_t count, int32_t* hist, hipStream_t st);
void launch_encode(const uint16_t* w, int N, int K, int CH, int base, uint8_t* m8, uint8_t* e4, int32_t* row_exc,
                   hipStream_t st);
void launch_encode_exc(const uint16_t* w, int N, int K, int base, const int32_t* rp, int32_t* er, int32_t* ec,
                       float* ev, hipStream_t st);

}  // namespace rv12
