// Gradient-norm reduction, clip multiply and plain SGD for the fp32
// codebook masters.
#include "jkv_common.h"

namespace jkv {

static const int kMaxTensors = 64;
#ifndef JKV_SUMSQ_EPT
#define JKV_SUMSQ_EPT 64
#endif

struct SumsqArgs {
  const float* buf[kMaxTensors];
  int64_t numel[kMaxTensors];
  double* out;
  int32_t blocks_per_tensor;
};

// grid = n * blocks_per_tensor; fp64 accumulation, one fp64 atomic per block.
__global__ __launch_bounds__(256) void sumsq_kernel(SumsqArgs a) {
  const int tensor = blockIdx.x / a.blocks_per_tensor;
  const int part = blockIdx.x % a.blocks_per_tensor;
  const float* __restrict__ x = a.buf[tensor];
  const int64_t n = a.numel[tensor];
  const int64_t stride = (int64_t)a.blocks_per_tensor * blockDim.x;
  // 16-byte loads over the aligned body, four in flight per thread, two fp64
  // chains; the tail one by one
  const int64_t n4 = ((uintptr_t)x % 16 == 0) ? n / 4 : 0;
  double acc0 = 0.0, acc1 = 0.0;
  for (int64_t i = (int64_t)part * blockDim.x + threadIdx.x; i < n4; i += 4 * stride) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t j = i + u * stride;
      v[u] = j < n4 ? ((const float4*)x)[j] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc0 = fma((double)v[u].x, (double)v[u].x, acc0);
      acc1 = fma((double)v[u].y, (double)v[u].y, acc1);
      acc0 = fma((double)v[u].z, (double)v[u].z, acc0);
      acc1 = fma((double)v[u].w, (double)v[u].w, acc1);
    }
  }
  for (int64_t i = 4 * n4 + (int64_t)part * blockDim.x + threadIdx.x; i < n; i += stride) {
    const double v = x[i];
    acc0 = fma(v, v, acc0);
  }
  double acc = acc0 + acc1;
  // block reduction
  __shared__ double red[4];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) s += red[w];
    atomicAdd(&a.out[tensor], s);
  }
}

__global__ void zero_f64_kernel(double* out, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = 0.0;
}

struct ScaleSgdArgs {
  float* param[kMaxTensors];
  float* grad[kMaxTensors];
  int64_t numel[kMaxTensors];
  float scale[kMaxTensors];
  float lr;
  int32_t blocks_per_tensor;
};

__global__ __launch_bounds__(256) void scale_sgd_kernel(ScaleSgdArgs a) {
  const int tensor = blockIdx.x / a.blocks_per_tensor;
  const int part = blockIdx.x % a.blocks_per_tensor;
  float* __restrict__ g = a.grad[tensor];
  float* __restrict__ p = a.param[tensor];
  const float sc = a.scale[tensor];
  const int64_t n = a.numel[tensor];
  const int64_t stride = (int64_t)a.blocks_per_tensor * blockDim.x;
  // 16-byte accesses over the aligned body (the same per-element arithmetic)
  const bool vec = (uintptr_t)g % 16 == 0 && (a.lr == 0.f || (uintptr_t)p % 16 == 0);
  const int64_t n4 = vec ? n / 4 : 0;
  for (int64_t i = (int64_t)part * blockDim.x + threadIdx.x; i < n4; i += stride) {
    float4 gv = ((const float4*)g)[i];
    gv.x *= sc;
    gv.y *= sc;
    gv.z *= sc;
    gv.w *= sc;
    ((float4*)g)[i] = gv;
    if (a.lr != 0.f) {
      float4 pv = ((const float4*)p)[i];
      pv.x = pv.x + (-a.lr) * gv.x;
      pv.y = pv.y + (-a.lr) * gv.y;
      pv.z = pv.z + (-a.lr) * gv.z;
      pv.w = pv.w + (-a.lr) * gv.w;
      ((float4*)p)[i] = pv;
    }
  }
  for (int64_t i = 4 * n4 + (int64_t)part * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float gv = g[i] * sc;
    g[i] = gv;
    if (a.lr != 0.f) p[i] = p[i] + (-a.lr) * gv;
  }
}

}  // namespace jkv

extern "C" {

int jkv_sumsq(int32_t n, const float* const* buffers, const int64_t* numels, double* out_sumsq,
              jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(n >= 0, "negative tensor count");
  if (n == 0) return JKV_OK;
  JKV_CHECK_ARG(out_sumsq != nullptr && buffers != nullptr && numels != nullptr, "null buffer");
  hipLaunchKernelGGL(zero_f64_kernel, dim3((uint32_t)ceil_div(n, 256)), dim3(256), 0, stream, out_sumsq, n);
  JKV_CHECK_LAUNCH();
  for (int32_t base = 0; base < n; base += kMaxTensors) {
    SumsqArgs a = {};
    const int32_t m = (n - base) < kMaxTensors ? (n - base) : kMaxTensors;
    int64_t maxn = 0;
    for (int32_t i = 0; i < m; ++i) {
      JKV_CHECK_ARG(numels[base + i] >= 0, "negative numel");
      JKV_CHECK_ARG(numels[base + i] == 0 || buffers[base + i] != nullptr, "null tensor");
      a.buf[i] = buffers[base + i];
      a.numel[i] = numels[base + i];
      if (a.numel[i] > maxn) maxn = a.numel[i];
    }
    a.out = out_sumsq + base;
    int64_t bpt = ceil_div(maxn, 256 * JKV_SUMSQ_EPT);  // elements per thread
    if (bpt < 1) bpt = 1;
    if (bpt > 256) bpt = 256;
    a.blocks_per_tensor = (int32_t)bpt;
    hipLaunchKernelGGL(sumsq_kernel, dim3((uint32_t)(m * bpt)), dim3(256), 0, stream, a);
    JKV_CHECK_LAUNCH();
  }
  return JKV_OK;
}

int jkv_scale_sgd(int32_t n, float* const* params, float* const* grads, const int64_t* numels,
                  const float* scales, float lr, jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(n >= 0, "negative tensor count");
  if (n == 0) return JKV_OK;
  JKV_CHECK_ARG(grads && numels && scales, "null argument");
  JKV_CHECK_ARG(lr == 0.f || params != nullptr, "SGD needs parameter buffers");
  for (int32_t base = 0; base < n; base += kMaxTensors) {
    ScaleSgdArgs a = {};
    const int32_t m = (n - base) < kMaxTensors ? (n - base) : kMaxTensors;
    int64_t maxn = 0;
    for (int32_t i = 0; i < m; ++i) {
      a.grad[i] = grads[base + i];
      a.param[i] = params ? params[base + i] : nullptr;
      a.numel[i] = numels[base + i];
      a.scale[i] = scales[base + i];
      JKV_CHECK_ARG(a.numel[i] == 0 || a.grad[i] != nullptr, "null gradient");
      JKV_CHECK_ARG(lr == 0.f || a.numel[i] == 0 || a.param[i] != nullptr, "null parameter");
      if (a.numel[i] > maxn) maxn = a.numel[i];
    }
    a.lr = lr;
    int64_t bpt = ceil_div(maxn, 256 * 8);
    if (bpt < 1) bpt = 1;
    if (bpt > 512) bpt = 512;
    a.blocks_per_tensor = (int32_t)bpt;
    hipLaunchKernelGGL(scale_sgd_kernel, dim3((uint32_t)(m * bpt)), dim3(256), 0, stream, a);
    JKV_CHECK_LAUNCH();
  }
  return JKV_OK;
}

}  // extern "C"
