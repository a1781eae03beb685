// Library-wide entry points of libtandem_w4.so: version, architecture, per-thread error text,
// and the one-time device set-up that must run before any graph capture.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "tw4_common.h"

#define TW4_VERSION "0.1.0"

int tw4_gemm_prepare_device(int dev);    // tw4_gemm.hip
int tw4_decode_prepare_device(int dev);  // tw4_decode.hip
int tw4_noalloc_prepare_device(int dev); // tw4_noalloc.hip

namespace tw4host {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
}

int hip_fail(hipError_t e, const char* what) {
    set_error("%s: %s (%s)", what, hipGetErrorString(e), hipGetErrorName(e));
    return TW4_EHIP;
}

}  // namespace tw4host

extern "C" const char* tw4_version(void) { return "tandem_w4 " TW4_VERSION " gfx950"; }

extern "C" const char* tw4_arch(void) { return "gfx950"; }

extern "C" const char* tw4_last_error(void) { return tw4host::g_error; }

extern "C" int tw4_init(int device) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return tw4host::hip_fail(e, "init: hipGetDeviceCount");
    TW4_REQUIRE(device >= 0 && device < count, TW4_EINVAL, "init: device %d of %d", device, count);
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return tw4host::hip_fail(e, "init: hipGetDeviceProperties");
    TW4_REQUIRE(strncmp(prop.gcnArchName, "gfx950", 6) == 0, TW4_EINVAL,
                "init: device %d is %s; this library is built for gfx950 (MI355X) only", device, prop.gcnArchName);
    int current = 0;
    e = hipGetDevice(&current);
    if (e != hipSuccess) return tw4host::hip_fail(e, "init: hipGetDevice");
    if (current != device) {
        e = hipSetDevice(device);
        if (e != hipSuccess) return tw4host::hip_fail(e, "init: hipSetDevice");
    }
    int rc = tw4_gemm_prepare_device(device);
    if (rc == TW4_OK) rc = tw4_decode_prepare_device(device);
    if (rc == TW4_OK) rc = tw4_noalloc_prepare_device(device);
    if (current != device) {
        e = hipSetDevice(current);
        if (e != hipSuccess && rc == TW4_OK) return tw4host::hip_fail(e, "init: restore device");
    }
    return rc;
}
