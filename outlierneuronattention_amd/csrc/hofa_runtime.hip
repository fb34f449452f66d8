// Library-wide host helpers: error reporting and device queries.
#include "hofa_common.h"

namespace hofa {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error(std::string(what) + ": " + hipGetErrorString(e));
        return HOFA_ELAUNCH;
    }
    return HOFA_OK;
}

int device_cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
    return n;
}

}  // namespace hofa

extern "C" const char *hofa_last_error(void) { return hofa::g_last_error.c_str(); }

extern "C" int hofa_version(void) { return 1; }
