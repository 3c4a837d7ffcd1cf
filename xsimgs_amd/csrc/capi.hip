// C-ABI plumbing: thread-local error messages, version and pack-size queries.
#include <cstdarg>
#include <cstdio>
#include <string>

#include "xsg_common.h"

namespace {
thread_local std::string g_last_error;
}

int xsg_fail(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int xsg_launch_status(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return xsg_fail(XSG_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
    return XSG_OK;
}

extern "C" const char* xsg_last_error(void) { return g_last_error.c_str(); }

extern "C" int xsg_abi_version(void) { return XSG_ABI_VERSION; }

extern "C" int xsg_camera_pack_elements(int kind) {
    switch (kind) {
        case XSG_CAM_PINHOLE:
        case XSG_CAM_SPHERICAL: return 21;
        case XSG_CAM_LIDAR: return 23;
        case XSG_CAM_DISTORTED: return 30;
        case XSG_CAM_FISHEYE: return 25;
        default: return xsg_fail(XSG_ERR_INVALID, "unknown camera kind %d", kind);
    }
}
