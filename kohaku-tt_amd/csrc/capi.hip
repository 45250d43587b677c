// C ABI plumbing: the thread_local last-error string and HIP status mapping.
//
// The reference's C ABI keeps a thread_local message read by ktt_last_error() and
// returns NULL / -1 on failure (src/kohakutt_native/csrc/py_bridge/capi.cpp:19,58-79);
// here every entry point returns a kmi_status and sets the same kind of message.
#include "common.hpp"

namespace kmi {

namespace {
thread_local std::string g_last_error;
}

int fail(int status, const std::string& message) {
    g_last_error = message;
    return status;
}

int hip_status(hipError_t err, const char* what) {
    if (err == hipSuccess) return KMI_OK;
    return fail(KMI_EHIP, std::string(what) + ": HIP error " + hipGetErrorName(err) + ": " +
                              hipGetErrorString(err));
}

}  // namespace kmi

extern "C" const char* kmi_last_error(void) { return kmi::g_last_error.c_str(); }

extern "C" int kmi_abi_version(void) { return KMI_ABI_VERSION; }
