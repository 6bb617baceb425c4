// Status plumbing for the C ABI: per-thread last error, launch checks, and the
// small host helpers (inv_freq, ABI version).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include "nvf_host.hpp"

namespace nvf {

static thread_local char g_last_error[512];

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NVF_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return NVF_OK;
}

void dropin_check(int status, const char* what) {
  if (status == NVF_OK) return;
  fprintf(stderr, "HIP error in %s: %s\n", what, g_last_error);
  exit(1);
}

}  // namespace nvf

extern "C" const char* nvf_last_error(void) { return nvf::g_last_error; }

extern "C" int nvf_abi_version(void) { return 1; }

// src/model.cpp:416-420: computed in double, rounded to float.
extern "C" int nvf_rope_inv_freq(double theta, int head_dim, float* out) {
  if (!out || head_dim <= 0 || (head_dim & 1) || !(theta > 0.0))
    return nvf::fail(NVF_ERR_INVALID, "nvf_rope_inv_freq: bad theta %g or head_dim %d", theta, head_dim);
  for (int i = 0; i < head_dim / 2; ++i) out[i] = (float)(1.0 / pow(theta, (2.0 * i) / head_dim));
  return NVF_OK;
}
