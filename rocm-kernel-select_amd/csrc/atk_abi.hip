// Library-wide C ABI pieces: version, error text, variant tables.
#include <stdarg.h>
#include <stdio.h>

#include "atk_common.h"

namespace atk {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(ATK_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return ATK_OK;
}

int device_cu_count() {
  // per device, queried once (the host code runs on one device at a time)
  static int cached[64] = {0};
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64 && cached[dev] > 0) return cached[dev];
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) cached[dev] = n;
  return n;
}

int device_wall_clock_khz() {
  static int cached[64] = {0};
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64 && cached[dev] > 0) return cached[dev];
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeWallClockRate, dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64) cached[dev] = n;
  return n;
}

// Variant tables are defined next to their kernels.
int dwconv1d_num_variants();
const char* dwconv1d_variant_name(int v);
int group_norm_num_variants();
const char* group_norm_variant_name(int v);
int conv_num_variants();
const char* conv_variant_name(int v);

}  // namespace atk

extern "C" {

int atk_abi_version(void) { return 1; }

const char* atk_last_error(void) { return atk::g_err; }

int atk_num_variants(int op) {
  switch (op) {
    case ATK_OP_DWCONV1D: return atk::dwconv1d_num_variants();
    case ATK_OP_GROUP_NORM: return atk::group_norm_num_variants();
    case ATK_OP_CONV: return atk::conv_num_variants();
    default: return 0;
  }
}

const char* atk_variant_name(int op, int variant) {
  switch (op) {
    case ATK_OP_DWCONV1D: return atk::dwconv1d_variant_name(variant);
    case ATK_OP_GROUP_NORM: return atk::group_norm_variant_name(variant);
    case ATK_OP_CONV: return atk::conv_variant_name(variant);
    default: return nullptr;
  }
}

}  // extern "C"
