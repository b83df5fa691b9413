// Library-wide entry points: version, status strings, thread-local last error.
#include "kvc_common.h"

namespace kvc {

static thread_local std::string g_last_error;

int set_error(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}

}  // namespace kvc

extern "C" {

int kvc_version(void) { return 100; }  // 0.1.0

const char* kvc_status_string(int status) {
  switch (status) {
    case KVC_OK: return "ok";
    case KVC_ERR_INVALID_ARG: return "invalid argument";
    case KVC_ERR_UNSUPPORTED: return "unsupported configuration";
    case KVC_ERR_ALIGNMENT: return "misaligned pointer or stride";
    case KVC_ERR_WORKSPACE: return "workspace or staging buffer too small";
    case KVC_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

const char* kvc_last_error(void) { return kvc::g_last_error.c_str(); }

}  // extern "C"
