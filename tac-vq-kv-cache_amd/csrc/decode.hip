// Codes-to-vector reconstruction with frozen codes.
#include "jkv_common.h"

namespace jkv {

// One thread per (row, group, dimension).  out[b,h,t,g*d+i] =
// dtype( sum_{s<depth} fp32(fp16(C[h*G+g, s, code_s, i])) ), in stage order.
template <int DT>
__global__ __launch_bounds__(256) void rvq_decode_kernel(
    const uint8_t* __restrict__ codes, int64_t cb, int64_t ch, int64_t ct, int64_t B,
    int64_t H, int64_t T, int64_t G, int64_t d, const float* __restrict__ tables, int64_t S,
    int64_t K, int32_t depth, void* __restrict__ out) {
  const int64_t D = G * d;
  const int64_t n = B * H * T * D;
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int64_t col = idx % D;
  const int64_t bht = idx / D;
  const int64_t t = bht % T;
  const int64_t bh = bht / T;
  const int64_t h = bh % H;
  const int64_t b = bh / H;
  const int64_t g = col / d, i = col % d;
  const uint8_t* cp = codes + b * cb + h * ch + t * ct + g * S;
  const int64_t p = h * G + g;
  float acc = 0.f;
  for (int s = 0; s < depth; ++s) {
    int64_t k = cp[s];
    acc += deploy16(tables[((p * S + s) * K + k) * d + i]);
  }
  Elem<DT>::store(out, idx, acc);
}

}  // namespace jkv

extern "C" int jkv_rvq_decode(const uint8_t* codes, int64_t code_stride_b, int64_t code_stride_h,
                              int64_t code_stride_t, int64_t B, int64_t H, int64_t T, int64_t G,
                              int64_t d, const float* tables, int64_t S, int64_t K, int32_t depth,
                              void* out, int32_t out_dtype, jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(B >= 0 && H > 0 && T >= 0 && G > 0 && d > 0 && S > 0 && K > 0 && K <= 256,
                "invalid decode geometry");
  JKV_CHECK_ARG(depth >= 1 && depth <= S, "decode depth outside the ladder");
  const int64_t n = B * H * T * G * d;
  if (n == 0) return JKV_OK;
  JKV_CHECK_ARG(codes && tables && out, "null buffer");
  dim3 grid((uint32_t)ceil_div(n, 256));
  switch (out_dtype) {
    case JKV_F16:
      hipLaunchKernelGGL(rvq_decode_kernel<JKV_F16>, grid, dim3(256), 0, stream, codes,
                         code_stride_b, code_stride_h, code_stride_t, B, H, T, G, d, tables, S, K,
                         depth, out);
      break;
    case JKV_BF16:
      hipLaunchKernelGGL(rvq_decode_kernel<JKV_BF16>, grid, dim3(256), 0, stream, codes,
                         code_stride_b, code_stride_h, code_stride_t, B, H, T, G, d, tables, S, K,
                         depth, out);
      break;
    case JKV_F32:
      hipLaunchKernelGGL(rvq_decode_kernel<JKV_F32>, grid, dim3(256), 0, stream, codes,
                         code_stride_b, code_stride_h, code_stride_t, B, H, T, G, d, tables, S, K,
                         depth, out);
      break;
    default:
      return set_error(JKV_EINVAL, "unknown output dtype %d", out_dtype);
  }
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}
