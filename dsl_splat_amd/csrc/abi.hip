// ABI bookkeeping: version and the per-thread last error message.
#include <cstdio>
#include <cstring>

#include "common.hpp"

namespace gs3d {

static thread_local char g_last_error[512] = "";

void set_error(const char* message) {
    std::snprintf(g_last_error, sizeof(g_last_error), "%s", message);
}

int launch_status(const char* where) {
    const hipError_t err = hipGetLastError();
    if (err == hipSuccess) return GS3D_OK;
    std::snprintf(g_last_error, sizeof(g_last_error), "%s: %s", where, hipGetErrorString(err));
    return GS3D_ERR_LAUNCH;
}

}  // namespace gs3d

extern "C" int gs3d_abi_version(void) { return 10; }

extern "C" const char* gs3d_last_error(void) { return gs3d::g_last_error; }
