// Host-side helpers of the HIP layer: error reporting, device properties, dim coalescing.
#include "common.hpp"
#include "intdiv.hpp"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

namespace nchip {

static thread_local char g_err[512];

int set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(NC_HIP_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
    return NC_HIP_OK;
}

static int g_grid_cus = -1;  // -1: not read from the environment yet; 0: the device's own count

int num_cus() {
    if (g_grid_cus < 0) {
        const char *env = getenv("NC_HIP_CUS");
        const int v = env ? atoi(env) : 0;
        g_grid_cus = v > 0 ? v : 0;
    }
    if (g_grid_cus > 0) return g_grid_cus;
    static int cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return kPlanCUs;
    if (!cache[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = kPlanCUs;
        cache[dev] = n;
    }
    return cache[dev];
}

hipStream_t as_stream(void *s) { return (hipStream_t)s; }

int coalesce(int nd, int64_t *shape, int nops, int64_t (*st)[NC_HIP_MAX_DIMS]) {
    // drop size-1 dims (their stride never matters)
    int k = 0;
    for (int d = 0; d < nd; d++) {
        if (shape[d] == 1) continue;
        shape[k] = shape[d];
        for (int o = 0; o < nops; o++) st[o][k] = st[o][d];
        k++;
    }
    nd = k;
    if (nd == 0) return 0;
    // merge d-1 into d when, for every operand, stride[d-1] == stride[d] * shape[d]
    int out = 0;
    for (int d = 1; d < nd; d++) {
        bool ok = true;
        for (int o = 0; o < nops && ok; o++) ok = st[o][out] == st[o][d] * shape[d];
        if (ok) {
            shape[out] *= shape[d];
            for (int o = 0; o < nops; o++) st[o][out] = st[o][d];
        } else {
            out++;
            shape[out] = shape[d];
            for (int o = 0; o < nops; o++) st[o][out] = st[o][d];
        }
    }
    return out + 1;
}

}  // namespace nchip

extern "C" NC_HIP_API const char *nc_hip_last_error(void) { return nchip::g_err; }

extern "C" NC_HIP_API int nc_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

extern "C" NC_HIP_API void nc_hip_set_grid_cus(int n) { nchip::g_grid_cus = n > 0 ? n : 0; }

extern "C" NC_HIP_API uint64_t nc_hip_check_intdiv(const uint32_t *divs, int ndivs, const uint32_t *nums, int nnums) {
    uint64_t bad = 0;
    for (int i = 0; i < ndivs; i++) {
        if (divs[i] == 0) continue;
        const nchip::IntDiv d(divs[i]);
        for (int j = 0; j < nnums; j++) {
            bad += d.div(nums[j]) != nums[j] / divs[i];
            if (nums[j] < (1u << 31) && divs[i] <= (1u << 31)) bad += d.div31(nums[j]) != nums[j] / divs[i];
        }
    }
    return bad;
}
