// Host-side runtime pieces of libmaskahead_hip.so: error strings, launch checks,
// device properties.  No allocation, no synchronisation.
#include <stdarg.h>
#include <stdio.h>

#include "ma_common.h"

static thread_local char g_err[512] = "";

void ma_set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

extern "C" const char *ma_last_error(void) { return g_err; }

extern "C" int ma_version(void) { return 1; }

int ma_check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        ma_set_error("%s: launch failed: %s", what, hipGetErrorString(e));
        return MA_EHIP;
    }
    return MA_OK;
}

int ma_num_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}
