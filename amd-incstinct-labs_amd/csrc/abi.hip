// Library-level entry points of libcdna4_attn.so: version, error text, device check.
#include "common.hpp"
#include <atomic>
#include <string.h>

namespace cdna4 {

namespace {
constexpr int kMaxDevices = 64;
// 0 = unknown, 1 = gfx950, 2 = other architecture.
std::atomic<int> g_arch[kMaxDevices];
}  // namespace

int check_device() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return CDNA4_ERR_INVALID_DEVICE_FUNCTION;
    int a = g_arch[dev].load(std::memory_order_relaxed);
    if (a == 0) {
        hipDeviceProp_t prop;
        e = hipGetDeviceProperties(&prop, dev);
        if (e != hipSuccess) return (int)e;
        a = (strncmp(prop.gcnArchName, "gfx950", 6) == 0) ? 1 : 2;
        g_arch[dev].store(a, std::memory_order_relaxed);
    }
    return a == 1 ? 0 : CDNA4_ERR_INVALID_DEVICE_FUNCTION;
}

namespace {
std::atomic<int> g_cus[kMaxDevices];
}

int device_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int n = g_cus[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        g_cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

}  // namespace cdna4

extern "C" int cdna3_abi_version(void) { return CDNA4_ABI_VERSION; }

extern "C" const char* cdna3_error_string(int code) {
    switch (code) {
        case CDNA4_OK: return "success";
        case CDNA4_ERR_INVALID_VALUE: return "invalid value (shape, dtype, op or workspace size)";
        case CDNA4_ERR_SCRATCH_TOO_SMALL:
            return "cdna3_attn_decode_noalloc: the call needs more split-K scratch than the library's static "
                   "array holds (cdna3_attn_decode_noalloc_max_bytes); pass a workspace to cdna3_attn_decode "
                   "instead";
        case CDNA4_ERR_INVALID_DEVICE_FUNCTION: return "current device is not gfx950 (MI355X)";
        default: return hipGetErrorString((hipError_t)code);
    }
}
