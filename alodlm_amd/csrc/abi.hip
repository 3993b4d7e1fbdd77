// Library identity and error reporting for the C ABI.
#include <cstdarg>
#include <cstdio>

#include "common.h"

static thread_local char g_last_error[512] = "";

int alodlm_set_error(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
  return code;
}

extern "C" int alodlm_abi_version(void) { return ALODLM_ABI_VERSION; }

extern "C" const char* alodlm_last_error(void) { return g_last_error; }

extern "C" int alodlm_device_info(int device, int64_t* compute_units, int64_t* max_clock_khz) {
  int cus = 0, khz = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      hipDeviceGetAttribute(&khz, hipDeviceAttributeClockRate, device) != hipSuccess)
    return alodlm_set_error(ALODLM_EHIP, "device_info: no such device %d", device);
  *compute_units = cus;
  *max_clock_khz = khz;
  return ALODLM_OK;
}
