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

// Measurement aid: a plain streaming read of `bytes` (a multiple of 16) at `src`,
// 16-byte loads, grid-stride, every lane's XOR of what it read folded into one
// word per workgroup at sink[blockIdx.x] (so the loads cannot be dropped).  Its
// time is the HBM read ceiling the expert kernels are judged against.
namespace {
__global__ void __launch_bounds__(256) stream_read_kernel(const uint4* __restrict__ src, size_t n16,
                                                          uint32_t* __restrict__ sink) {
  uint32_t acc = 0u;
  const size_t stride = (size_t)gridDim.x * 256;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    const uint4 a = src[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t v = 0u;
    for (int t = 0; t < 256; ++t) v ^= red[t];
    sink[blockIdx.x] = v;
  }
}
}  // namespace

extern "C" int cachalot_stream_read(const void* src, size_t bytes, uint32_t* sink, int blocks,
                                    cachalot_stream_t stream) {
  using namespace cachalot;
  CACHALOT_REQUIRE(src && sink, "stream_read: null pointer");
  CACHALOT_REQUIRE(bytes % 16 == 0 && blocks >= 1 && blocks <= 65536, "stream_read: bytes=%zu blocks=%d", bytes,
                   blocks);
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const uint4*>(src), bytes / 16, sink);
  return check_launch("stream_read_kernel");
}
