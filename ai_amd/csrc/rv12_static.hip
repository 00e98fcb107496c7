// rv12_gemm_static: the linear of rv12_gemm with its split-K partial sums in a
// scratch array the library owns in device memory, so that a caller that
// cannot allocate (code under HIP graph capture, a serving loop, a harness that
// forbids hipMalloc) still gets every launch shape.
//
// The array is a file-scope __device__ variable: every GPU the library runs on
// holds its own copy, from module load until the process ends.  Host code never
// passes the array's name to a kernel (in host code it is a stand-in, not a
// device address): the first call on a device, with that device current, asks
// the runtime for that device's address once (hipGetSymbolAddress) and keeps
// it; every later call uses the kept address.
//
// The partials need no clearing: a split launch writes every partial and sum
// of squares it later reads.  All calls on one GPU share that GPU's array, so
// calls that overlap on one GPU (two streams, two host threads) race on it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "rv12.h"
#include "rv12_internal.h"

static __device__ __align__(256) unsigned char scratch[RV12_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;

std::mutex g_mu;
void* g_ptr[kMaxDevices];  // device address of `scratch` per device, once known

int scratch_ptr(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return RV12_E_LAUNCH;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return RV12_E_LAUNCH;
        g_ptr[dev] = p;
    }
    *out = g_ptr[dev];
    return RV12_OK;
}

}  // namespace

extern "C" int rv12_gemm_static(const rv12_matrix* w, const float* x, float* y, int t, const uint16_t* lnw,
                                float eps, int mode, const rv12_launch* cfg, void* stream) {
    // every argument check of rv12_gemm that needs the launch shape, and the
    // scratch bound, before any device call
    if (!w) return RV12_E_NULL;
    const int64_t need = rv12::launch_ws_bytes(w->n, w->k, t, cfg);
    if (need < 0) return (int)need;
    if (need > (int64_t)RV12_STATIC_SCRATCH_BYTES) return RV12_E_SCRATCH;
    void* ws = nullptr;
    const int sr = scratch_ptr(&ws);
    if (sr) return sr;
    return rv12_gemm(w, x, y, t, lnw, eps, mode, cfg, ws, (size_t)RV12_STATIC_SCRATCH_BYTES, stream);
}
