// Library-level entry points of the C ABI: version, status names and device properties.
#include <hip/hip_runtime.h>

#include "../../include/mica_amd.h"

extern "C" int mica_version(void) { return (0 << 16) | 1; }

extern "C" const char *mica_status_name(int rc) {
    switch (rc) {
    case 0: return "ok";
    case MICA_MISS_SHAPE: return "shape";
    case MICA_MISS_DTYPE: return "dtype";
    case MICA_MISS_ALIGN: return "align";
    case MICA_MISS_STRIDE: return "stride";
    case MICA_MISS_RANGE: return "i32_range";
    case MICA_MISS_ARG: return "arg";
    case MICA_MISS_DEVICE: return "device";
    default: break;
    }
    if (rc < 0) return hipGetErrorString((hipError_t)(-rc));
    return "unknown";
}

extern "C" int mica_device_info(int device, int *cu_count, int *clock_khz, int *lds_per_block, int *gfx_arch) {
    hipDeviceProp_t prop;
    const hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return -(int)e;
    if (cu_count) *cu_count = prop.multiProcessorCount;
    if (clock_khz) *clock_khz = prop.clockRate;
    if (lds_per_block) *lds_per_block = (int)prop.sharedMemPerBlock;
    if (gfx_arch) {
        // gcnArchName is e.g. "gfx950:sramecc+:xnack-"
        int v = 0;
        const char *s = prop.gcnArchName;
        if (s[0] == 'g' && s[1] == 'f' && s[2] == 'x') {
            for (const char *c = s + 3; *c >= '0' && *c <= '9'; ++c) v = v * 10 + (*c - '0');
        }
        *gfx_arch = v;
    }
    return 0;
}
