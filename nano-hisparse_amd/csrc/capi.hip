// Library-wide C ABI pieces: status messages, the pinned-host device alias
// and the legacy per-head column expansion.
#include <stdarg.h>
#include <stdio.h>

#include "nhs_common.h"

namespace nhs {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

static thread_local LaunchEvents g_launch_events;

LaunchEvents take_launch_events() {
  LaunchEvents ev = g_launch_events;
  g_launch_events = LaunchEvents();
  return ev;
}

int launch_status(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail((int)err, "%s: launch failed: %s", what, hipGetErrorString(err));
  return NHS_OK;
}

__global__ __launch_bounds__(256) void expand_columns_kernel(const int64_t* __restrict__ shared_rows, int64_t n,
                                                             const int64_t* __restrict__ columns, int64_t total,
                                                             int64_t* __restrict__ out) {
  int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= total) return;
  int64_t c = columns[i];
  out[i] = (c >= 0 && c < n) ? shared_rows[c] : -1;
}

}  // namespace nhs

extern "C" {

int nhs_abi_version(void) { return 2; }

const char* nhs_last_error(void) { return nhs::g_last_error; }

int nhs_set_launch_events(void* start_event, void* stop_event) {
  nhs::g_launch_events.start = (hipEvent_t)start_event;
  nhs::g_launch_events.stop = (hipEvent_t)stop_event;
  return NHS_OK;
}

int nhs_host_device_ptr(const void* pinned_host, void** device_alias) {
  if (!pinned_host || !device_alias) return nhs::fail(NHS_ERR_INVALID, "nhs_host_device_ptr: null pointer");
  hipError_t err = hipHostGetDevicePointer(device_alias, const_cast<void*>(pinned_host), 0);
  if (err != hipSuccess)
    return nhs::fail((int)err, "nhs_host_device_ptr: memory is not pinned host memory: %s", hipGetErrorString(err));
  return NHS_OK;
}

int nhs_expand_columns(const int64_t* shared_rows, int64_t n, const int64_t* columns, int64_t heads, int64_t width,
                       int64_t* out, void* stream) {
  const nhs::LaunchEvents ev = nhs::take_launch_events();
  if (n < 1 || heads < 0 || width < 0 || !shared_rows || !columns || !out)
    return nhs::fail(NHS_ERR_INVALID, "nhs_expand_columns: invalid arguments");
  int64_t total = heads * width;
  if (total == 0) return NHS_OK;
  int64_t blocks = (total + 255) / 256;
  nhs::launch(nhs::expand_columns_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, ev.start,
              ev.stop, shared_rows, n, columns, total, out);
  return nhs::launch_status("nhs_expand_columns");
}

}  // extern "C"
