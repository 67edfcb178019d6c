// Library identity and the thread-local error channel of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace cachalot {

static thread_local char g_last_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(CACHALOT_EHIP, "%s: %s", what, hipGetErrorString(e));
  return CACHALOT_OK;
}

}  // namespace cachalot

extern "C" int cachalot_version(void) { return 1; }

extern "C" const char* cachalot_last_error(void) { return cachalot::g_last_error; }

// Bank loading: n experts' bytes of one tensor, [n, tensor_bytes] contiguous at `src`
// (pinned host or device memory), into slot records first_slot .. first_slot + n - 1
// of a pool at offset `offset`: one 2-D copy (destination pitch = the record).
extern "C" int cachalot_copy_records(uint8_t* pool, int64_t record_bytes, int64_t offset, int64_t first_slot,
                                     const void* src, int64_t tensor_bytes, int64_t n, cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(pool && src, "copy_records: null pointer");
  CACHALOT_REQUIRE(record_bytes > 0 && tensor_bytes > 0 && n >= 0 && first_slot >= 0,
                   "copy_records: record_bytes=%lld tensor_bytes=%lld n=%lld first_slot=%lld", (long long)record_bytes,
                   (long long)tensor_bytes, (long long)n, (long long)first_slot);
  CACHALOT_REQUIRE(offset >= 0 && offset + tensor_bytes <= record_bytes,
                   "copy_records: tensor [%lld, %lld) outside the %lld-byte record", (long long)offset,
                   (long long)(offset + tensor_bytes), (long long)record_bytes);
  if (n == 0) return CACHALOT_OK;
  hipError_t e = hipMemcpy2DAsync(pool + first_slot * record_bytes + offset, (size_t)record_bytes, src,
                                  (size_t)tensor_bytes, (size_t)tensor_bytes, (size_t)n, hipMemcpyDefault,
                                  (hipStream_t)stream);
  if (e != hipSuccess) return fail(CACHALOT_EHIP, "copy_records: %s", hipGetErrorString(e));
  return CACHALOT_OK;
}
