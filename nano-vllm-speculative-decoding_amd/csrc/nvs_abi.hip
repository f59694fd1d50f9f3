// ABI version and error reporting of libnvs_amd.
#include "nvs_common.hpp"

namespace nvs {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        set_error("%s: kernel launch failed: %s", what, hipGetErrorString(err));
        return NVS_ERR_HIP;
    }
    return NVS_OK;
}

}  // namespace nvs

extern "C" int nvs_abi_version(void) { return NVS_ABI_VERSION; }

extern "C" const char* nvs_last_error(void) { return nvs::g_last_error.c_str(); }
