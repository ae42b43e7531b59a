// Library-wide pieces of the C ABI: version, error strings, the fill smoke kernel.
#include <stdarg.h>
#include <stdio.h>

#include "fx_device.h"

namespace fx {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error((int)e, "%s failed: hipError=%d (%s)", what, (int)e, hipGetErrorString(e));
    return 0;
}

int device_cus() {
    // initialised once, thread-safely (host threads such as autograd's may call first)
    static const int s_cus = [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
            return cus;
        return 256;
    }();
    return s_cus;
}

__global__ void __launch_bounds__(256) fill_f32_kernel(float* __restrict__ p, int64_t n, float value) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = value;
}

}  // namespace fx

extern "C" int fx_abi_version(void) { return FX_ABI_VERSION; }

extern "C" const char* fx_last_error(void) { return fx::g_err; }

extern "C" int fx_fill_f32(float* p, int64_t n, float value, void* stream) {
    FX_REQUIRE(n >= 0, "fx_fill_f32: n=%lld < 0", (long long)n);
    FX_REQUIRE(n == 0 || p != nullptr, "fx_fill_f32: null pointer");
    if (n == 0) return 0;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fx::fill_f32_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, p, n, value);
    return fx::check_launch("fill_f32");
}
