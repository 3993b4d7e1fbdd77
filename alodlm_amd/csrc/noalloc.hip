// RMSNorm backward that allocates nothing: the partial weight-gradient rows
// and the column reduction's group sums live in a file-scope device array
// instead of a caller-supplied workspace.
//
// Each GPU holds its own copy of `scratch` (ALODLM_NOALLOC_SCRATCH_FLOATS
// floats, 16 MiB) until the process ends.  Its device address is looked up
// once per device, with that device current, and kept in `g_scratch`; host
// code only ever passes that address, never the array's name (which on the
// host is a stand-in symbol, not device memory).
//
// Nothing in the array has to start at zero: the backward writes every
// partial row and every group sum before it reads them.  Every call on one
// GPU shares that GPU's array, so calls that overlap on one GPU (on different
// streams, or from different threads without ordering) race; calls on one
// stream are ordered and safe.
#include <mutex>

#include "norm.h"

#define ALODLM_MAX_DEVICES 64

static __device__ __align__(256) float scratch[ALODLM_NOALLOC_SCRATCH_FLOATS];

static std::mutex g_scratch_lock;
static float* g_scratch[ALODLM_MAX_DEVICES];

// Device address of `scratch` on `device`, looked up on first use.
static int scratch_on(int device, float** out) {
  if (device < 0 || device >= ALODLM_MAX_DEVICES)
    return alodlm_set_error(ALODLM_EINVAL, "rmsnorm_bwd_noalloc: device %d out of range", device);
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch[device] == nullptr) {
    int current = -1;
    if (hipGetDevice(&current) != hipSuccess)
      return alodlm_set_error(ALODLM_EHIP, "rmsnorm_bwd_noalloc: no current device");
    if (current != device && hipSetDevice(device) != hipSuccess)
      return alodlm_set_error(ALODLM_EHIP, "rmsnorm_bwd_noalloc: cannot select device %d", device);
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (current != device) (void)hipSetDevice(current);
    if (e != hipSuccess || ptr == nullptr)
      return alodlm_set_error(ALODLM_EHIP, "rmsnorm_bwd_noalloc: scratch lookup failed: %s",
                              hipGetErrorString(e));
    g_scratch[device] = static_cast<float*>(ptr);
  }
  *out = g_scratch[device];
  return ALODLM_OK;
}

extern "C" int alodlm_rmsnorm_bwd_noalloc(const void* dy, const void* x, const float* rstd,
                                          const void* w, const void* dres, void* dx,
                                          float* dw_accum, int64_t rows, int64_t cols, int dtype,
                                          void* stream) {
  ALODLM_CHECK_ARG(rows >= 0 && cols > 0, "rmsnorm_bwd_noalloc: bad shape");
  const int64_t need = alodlm_rmsnorm_bwd_workspace(rows, cols);
  ALODLM_CHECK_ARG(need <= ALODLM_NOALLOC_SCRATCH_FLOATS,
                   "rmsnorm_bwd_noalloc: %lld rows x %lld cols need %lld scratch floats, more "
                   "than the %d the library holds; use alodlm_rmsnorm_bwd with a workspace",
                   (long long)rows, (long long)cols, (long long)need,
                   (int)ALODLM_NOALLOC_SCRATCH_FLOATS);
  hipStream_t st = as_stream(stream);
  int device = -1;
  if (st != nullptr) {
    if (hipStreamGetDevice(st, &device) != hipSuccess)
      return alodlm_set_error(ALODLM_EHIP, "rmsnorm_bwd_noalloc: cannot query the stream's device");
  } else if (hipGetDevice(&device) != hipSuccess) {
    return alodlm_set_error(ALODLM_EHIP, "rmsnorm_bwd_noalloc: no current device");
  }
  float* ws = nullptr;
  const int rc = scratch_on(device, &ws);
  if (rc) return rc;
  return rmsnorm_bwd_launch(dy, x, rstd, w, dres, dx, dw_accum, ws, rows, cols, dtype, nullptr, 0,
                            st);
}
