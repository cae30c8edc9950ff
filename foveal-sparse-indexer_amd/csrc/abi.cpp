// C-ABI utilities: version, status strings, per-thread last-error message.
#include <stdarg.h>
#include <stdio.h>

#include "fsi_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace fsi_host {
void set_last_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}
}  // namespace fsi_host

extern "C" {

int fsi_abi_version(void) { return 1; }

const char* fsi_last_error(void) { return g_last_error; }

const char* fsi_status_string(int status) {
  switch (status) {
    case FSI_OK: return "ok";
    case FSI_ERR_INVALID_ARG: return "invalid argument";
    case FSI_ERR_SHAPE: return "unsupported or inconsistent shape";
    case FSI_ERR_INDEX_RANGE: return "index out of range";
    case FSI_ERR_CAPACITY: return "capacity exceeded";
    case FSI_ERR_DTYPE: return "unsupported dtype";
    case FSI_ERR_HIP: return "HIP runtime error";
    case FSI_ERR_ALIGN: return "misaligned pointer or leading dimension";
    case FSI_ERR_WORKSPACE: return "workspace missing or too small";
    default: return "unknown status";
  }
}

}  // extern "C"
