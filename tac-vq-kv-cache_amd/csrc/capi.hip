// Library-wide entry points: version, thread-local error text, fp16 deploy.
#include <stdarg.h>
#include <stdio.h>

#include "jkv_common.h"

namespace jkv {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

__global__ void f32_to_f16_kernel(const float* __restrict__ src,
                                  _Float16* __restrict__ dst, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) dst[i] = (_Float16)src[i];
}

}  // namespace jkv

extern "C" {

int jkv_version(void) { return 100; }

const char* jkv_last_error(void) { return jkv::g_last_error; }

int jkv_f32_to_f16(const float* src, void* dst, int64_t n, jkv_stream_t stream) {
  JKV_CHECK_ARG(n >= 0, "negative element count");
  if (n == 0) return JKV_OK;
  JKV_CHECK_ARG(src != nullptr && dst != nullptr, "null buffer");
  int64_t blocks = jkv::ceil_div(n, 256);
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(jkv::f32_to_f16_kernel, dim3((uint32_t)blocks), dim3(256), 0,
                     (hipStream_t)stream, src, (_Float16*)dst, n);
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

}  // extern "C"
