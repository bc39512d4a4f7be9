// s2x_static.hip -- the drop-in Q8_0 x F32 matmul without any allocation,
// for callers that cannot call hipMalloc (code under HIP graph capture,
// serving loops, harnesses that forbid it): its workspace is one
// file-scope device array, `scratch`, of S2X_STATIC_SCRATCH_BYTES, which
// every GPU the library runs on holds until the process ends.
//
// The host never uses the array's name as an address: the first call on a
// device, with that device current, asks HIP for the device address of
// `scratch` (hipGetSymbolAddress) and keeps it per device; kernels receive
// that address as their workspace argument, exactly as they receive the
// caller's buffer in s2x_mul_mat_q8_0_f32.
//
// Every call on one GPU shares that GPU's array and leaves its contents
// behind.  Nothing in it has to start at zero: each byte a call reads
// (repacked weight planes with their zero padding, the Q8_1 activation) was
// written earlier in that same call, on the same stream.  Calls that
// overlap on one GPU (different streams, or several threads on one device
// without ordering) race on the array.
#include "s2x.h"

#include <hip/hip_runtime.h>

#include <mutex>

#include "s2x_internal.h"

namespace {

constexpr size_t SCRATCH_BYTES = S2X_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void *g_scratch[MAX_DEVICES];  // device address of `scratch`, per device

// Device address of the current device's `scratch` (looked up once per
// device; HIP loads the code object on that device if it has not yet).
int scratch_of_current_device(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return s2x::hip_fail(e, "mul_mat_q8_0_f32_static: hipGetDevice");
    if (dev < 0 || dev >= MAX_DEVICES)
        return s2x::fail(S2X_ERR_UNSUPPORTED, "mul_mat_q8_0_f32_static: device %d >= %d", dev,
                         MAX_DEVICES);
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess)
            return s2x::hip_fail(e, "mul_mat_q8_0_f32_static: hipGetSymbolAddress(scratch)");
        if (!p || !s2x::aligned(p, 256))
            return s2x::fail(S2X_ERR_HIP, "mul_mat_q8_0_f32_static: scratch address %p unusable", p);
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return S2X_OK;
}

}  // namespace

extern "C" int s2x_mul_mat_q8_0_f32_static(const void *w_raw, int64_t K_pad, int64_t N,
                                           const float *x, int64_t K, int64_t ldx, int64_t M,
                                           float *y, void *stream) {
    // shapes the size formula accepts are checked against the array first;
    // every other argument check is the one of s2x_mul_mat_q8_0_f32
    const size_t need = s2x_mul_mat_workspace_size(K_pad, N, M);
    if (need > SCRATCH_BYTES)
        return s2x::fail(S2X_ERR_UNSUPPORTED,
                         "mul_mat_q8_0_f32_static: K_pad=%lld N=%lld M=%lld needs %zu bytes of "
                         "workspace, the static scratch array holds %zu",
                         (long long)K_pad, (long long)N, (long long)M, need, SCRATCH_BYTES);
    void *ws = nullptr;
    const int st = scratch_of_current_device(&ws);
    if (st != S2X_OK) return st;
    return s2x_mul_mat_q8_0_f32(w_raw, K_pad, N, x, K, ldx, M, y, ws, SCRATCH_BYTES, stream);
}
