// Error plumbing and device queries of the C ABI (see include/hla_s6.h).
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace hla {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(HLA_S6_ELAUNCH, "%s: %s", what, hipGetErrorString(err));
  return HLA_S6_OK;
}

}  // namespace hla

extern "C" int hla_s6_abi_version(void) { return HLA_S6_ABI_VERSION; }

extern "C" const char* hla_s6_last_error(void) { return hla::g_last_error; }

extern "C" int hla_s6_device_cus(int device, int* cus) {
  HLA_REQUIRE(cus != nullptr, HLA_S6_EINVAL, "device_cus: null output");
  int value = 0;
  hipError_t err = hipDeviceGetAttribute(&value, hipDeviceAttributeMultiprocessorCount, device);
  if (err != hipSuccess) return hla::fail(HLA_S6_EDEVICE, "device_cus: %s", hipGetErrorString(err));
  *cus = value;
  return HLA_S6_OK;
}
