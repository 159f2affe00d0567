// C ABI plumbing of libgpa_hip: version, thread-local error text, launch checks.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string>

#include "gpa_hip.h"
#include "gpa_common.h"

namespace {
thread_local std::string g_last_error;
}

int fail(int code, const char* message) {
  g_last_error = message;
  return code;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    char buf[256];
    snprintf(buf, sizeof buf, "%s: kernel launch failed: %s", what, hipGetErrorString(err));
    return fail(GPA_HIP_EHIP, buf);
  }
  return GPA_HIP_OK;
}

extern "C" int gpa_hip_abi_version(void) { return GPA_HIP_ABI_VERSION; }

extern "C" const char* gpa_hip_last_error(void) { return g_last_error.c_str(); }

void mark(gpa_timing* timing, hipStream_t stream) {
  if (!timing || timing->launched > GPA_MAX_TIMED) return;
  (void)hipEventRecord(timing->events[timing->launched], stream);
  timing->launched += 1;
}
