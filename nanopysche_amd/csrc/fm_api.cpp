// Library-level entry points: error reporting, version, host-side e4m3 codec.
#include <stdarg.h>
#include <stdio.h>

#include <hip/hip_runtime.h>

#include "fm_common.h"
#include "../../include/fm_hip.h"

namespace fm {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(err));
    return int(err);
  }
  return 0;
}

}  // namespace fm

extern "C" {

const char* fm_last_error_string(void) { return fm::g_error; }

const char* fm_version(void) { return "fm_hip 0.2 gfx950"; }

#ifndef FM_SOURCE_HASH
#define FM_SOURCE_HASH "unstamped"
#endif
const char* fm_source_hash(void) { return FM_SOURCE_HASH; }

void fm_host_encode_e4m3(const float* in, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = fm::f32_to_e4m3(in[i]);
}

void fm_host_decode_e4m3(const uint8_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = fm::e4m3_to_f32(in[i]);
}

}  // extern "C"
