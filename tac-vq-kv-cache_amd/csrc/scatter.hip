// Straight-through codebook gradient scatter-add (the backward of the
// reference's torch.gather over fp16-deployed fp32 masters).
#include "jkv_common.h"

namespace jkv {

struct ScatterArgs {
  const void* grads[JKV_MAX_EXITS];
  int32_t exit_depth[JKV_MAX_EXITS];
  int32_t n_exits;
  const uint8_t* codes;
  int64_t cb, ch, ct;
  int64_t B, H, T, G, d, S, K;
  float* grad_tables;  // [H*G,S,K,d]
  int64_t rows_per_chunk;
  int64_t n_chunks;
  int32_t groups_per_block;  // privatised groups per block (LDS path)
  float* partials;           // deterministic path workspace
};

template <int DT>
__device__ __forceinline__ float grad_sum(const ScatterArgs& a, int s, int64_t off) {
  float acc = 0.f;
  for (int e = 0; e < a.n_exits; ++e)
    if (a.exit_depth[e] > s) acc += Elem<DT>::load(a.grads[e], off);
  return acc;
}

// LDS-privatised bins for `groups_per_block` groups of one head over a chunk
// of rows; one global fp32 atomic per touched bin element at the end.
template <int DT>
__global__ __launch_bounds__(256) void scatter_lds_kernel(ScatterArgs a) {
  extern __shared__ float bins[];  // [gpb][S][K][d]
  const int gpb = a.groups_per_block;
  const int64_t per_group = a.S * a.K * a.d;
  const int64_t nbins = gpb * per_group;
  for (int64_t i = threadIdx.x; i < nbins; i += blockDim.x) bins[i] = 0.f;
  __syncthreads();

  const int64_t n_quads = ceil_div(a.G, gpb);
  const int64_t chunk = blockIdx.x % a.n_chunks;
  const int64_t hq = blockIdx.x / a.n_chunks;
  const int64_t h = hq / n_quads, q = hq % n_quads;
  const int64_t rows = a.B * a.T;
  const int64_t r0 = chunk * a.rows_per_chunk;
  int64_t r1 = r0 + a.rows_per_chunk;
  if (r1 > rows) r1 = rows;
  const int64_t D = a.G * a.d;
  // work items: (row, local group, dim) with dim fastest -> coalesced reads
  const int64_t items = (r1 - r0) * gpb * a.d;
  for (int64_t it = threadIdx.x; it < items; it += blockDim.x) {
    const int64_t i = it % a.d;
    const int64_t gl = (it / a.d) % gpb;
    const int64_t row = r0 + it / (a.d * gpb);
    const int64_t g = q * gpb + gl;
    if (g >= a.G) continue;
    const int64_t b = row / a.T, t = row % a.T;
    const int64_t off = ((b * a.H + h) * a.T + t) * D + g * a.d + i;
    const uint8_t* cp = a.codes + b * a.cb + h * a.ch + t * a.ct + g * a.S;
    float* gbins = bins + gl * per_group;
    for (int s = 0; s < (int)a.S; ++s) {
      const float v = grad_sum<DT>(a, s, off);
      if (v != 0.f) atomicAdd(&gbins[((int64_t)s * a.K + cp[s]) * a.d + i], v);
    }
  }
  __syncthreads();
  for (int64_t i = threadIdx.x; i < nbins; i += blockDim.x) {
    const float v = bins[i];
    if (v == 0.f) continue;
    const int64_t gl = i / per_group;
    const int64_t g = q * gpb + gl;
    if (g >= a.G) continue;
    const int64_t p = h * a.G + g;
    atomicAdd(&a.grad_tables[p * per_group + (i % per_group)], v);
  }
}

// Direct global atomics (bins too large to privatise, e.g. d = 128).
template <int DT>
__global__ __launch_bounds__(256) void scatter_global_kernel(ScatterArgs a) {
  const int64_t D = a.G * a.d;
  const int64_t n = a.B * a.H * a.T * D;
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int64_t col = idx % D;
  const int64_t bht = idx / D;
  const int64_t t = bht % a.T, bh = bht / a.T;
  const int64_t h = bh % a.H, b = bh / a.H;
  const int64_t g = col / a.d, i = col % a.d;
  const uint8_t* cp = a.codes + b * a.cb + h * a.ch + t * a.ct + g * a.S;
  const int64_t p = h * a.G + g;
  for (int s = 0; s < (int)a.S; ++s) {
    const float v = grad_sum<DT>(a, s, idx);
    if (v != 0.f) atomicAdd(&a.grad_tables[((p * a.S + s) * a.K + cp[s]) * a.d + i], v);
  }
}

// Deterministic path, pass 1: partial[c][p][s][k][i] = ordered sum over the
// rows of chunk c whose stage-s code is k.  One thread per (p, s, k, i).
template <int DT>
__global__ __launch_bounds__(256) void scatter_det_partial_kernel(ScatterArgs a) {
  const int64_t P = a.H * a.G;
  const int64_t per_chunk = P * a.S * a.K * a.d;
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= per_chunk * a.n_chunks) return;
  const int64_t c = idx / per_chunk;
  const int64_t rem = idx % per_chunk;
  const int64_t i = rem % a.d;
  const int64_t k = (rem / a.d) % a.K;
  const int64_t s = (rem / (a.d * a.K)) % a.S;
  const int64_t p = rem / (a.d * a.K * a.S);
  const int64_t h = p / a.G, g = p % a.G;
  const int64_t rows = a.B * a.T;
  const int64_t r0 = c * a.rows_per_chunk;
  int64_t r1 = r0 + a.rows_per_chunk;
  if (r1 > rows) r1 = rows;
  const int64_t D = a.G * a.d;
  float acc = 0.f;
  for (int64_t row = r0; row < r1; ++row) {
    const int64_t b = row / a.T, t = row % a.T;
    if (a.codes[b * a.cb + h * a.ch + t * a.ct + g * a.S + s] != k) continue;
    acc += grad_sum<DT>(a, (int)s, ((b * a.H + h) * a.T + t) * D + g * a.d + i);
  }
  a.partials[idx] = acc;
}

// Deterministic path, pass 2: grad += sum over chunks in chunk order.
__global__ __launch_bounds__(256) void scatter_det_reduce_kernel(ScatterArgs a) {
  const int64_t per_chunk = a.H * a.G * a.S * a.K * a.d;
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= per_chunk) return;
  float acc = 0.f;
  for (int64_t c = 0; c < a.n_chunks; ++c) acc += a.partials[c * per_chunk + idx];
  a.grad_tables[idx] += acc;
}

static const int64_t kDetRowsPerChunk = 256;

template <int DT>
static int launch_scatter(ScatterArgs a, int deterministic, hipStream_t stream) {
  const int64_t rows = a.B * a.T;
  const int64_t P = a.H * a.G;
  if (deterministic) {
    a.rows_per_chunk = kDetRowsPerChunk;
    a.n_chunks = ceil_div(rows, kDetRowsPerChunk);
    const int64_t per_chunk = P * a.S * a.K * a.d;
    hipLaunchKernelGGL(scatter_det_partial_kernel<DT>,
                       dim3((uint32_t)ceil_div(per_chunk * a.n_chunks, 256)), dim3(256), 0,
                       stream, a);
    JKV_CHECK_LAUNCH();
    hipLaunchKernelGGL(scatter_det_reduce_kernel, dim3((uint32_t)ceil_div(per_chunk, 256)),
                       dim3(256), 0, stream, a);
    JKV_CHECK_LAUNCH();
    return JKV_OK;
  }
  const int64_t per_group_bytes = a.S * a.K * a.d * (int64_t)sizeof(float);
  const int64_t lds_budget = 64 * 1024;
  if (per_group_bytes <= lds_budget) {
    int64_t gpb = lds_budget / per_group_bytes;
    if (gpb > a.G) gpb = a.G;
    if (gpb > 16) gpb = 16;
    a.groups_per_block = (int32_t)gpb;
    const int64_t n_quads = ceil_div(a.G, gpb);
    int64_t rpc = 4096;
    while (rpc > 64 && a.H * n_quads * ceil_div(rows, rpc) < 1024) rpc >>= 1;
    a.rows_per_chunk = rpc;
    a.n_chunks = ceil_div(rows, rpc);
    const int64_t blocks = a.H * n_quads * a.n_chunks;
    hipLaunchKernelGGL(scatter_lds_kernel<DT>, dim3((uint32_t)blocks), dim3(256),
                       (size_t)(gpb * per_group_bytes), stream, a);
    JKV_CHECK_LAUNCH();
    return JKV_OK;
  }
  const int64_t n = rows * a.H * a.G * a.d;
  hipLaunchKernelGGL(scatter_global_kernel<DT>, dim3((uint32_t)ceil_div(n, 256)), dim3(256), 0,
                     stream, a);
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

}  // namespace jkv

extern "C" {

int64_t jkv_rvq_scatter_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t G, int64_t d,
                                        int64_t S, int64_t K, int32_t deterministic) {
  if (!deterministic) return 0;
  return jkv::ceil_div(B * T, jkv::kDetRowsPerChunk) * H * G * S * K * d * (int64_t)sizeof(float);
}

int jkv_rvq_scatter_grad(int32_t n_exits, const void* const* grads, int32_t grad_dtype,
                         const int32_t* exit_depths, const uint8_t* codes, int64_t code_stride_b,
                         int64_t code_stride_h, int64_t code_stride_t, int64_t B, int64_t H,
                         int64_t T, int64_t G, int64_t d, int64_t S, int64_t K, float* grad_tables,
                         int32_t deterministic, void* workspace, int64_t workspace_bytes,
                         jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(n_exits >= 1 && n_exits <= JKV_MAX_EXITS, "1..%d exits", JKV_MAX_EXITS);
  JKV_CHECK_ARG(B >= 0 && H > 0 && T >= 0 && G > 0 && d > 0 && S > 0 && K > 0 && K <= 256,
                "invalid scatter geometry");
  if (B * T == 0) return JKV_OK;
  JKV_CHECK_ARG(codes && grad_tables && grads, "null buffer");
  ScatterArgs a = {};
  a.n_exits = n_exits;
  for (int e = 0; e < n_exits; ++e) {
    JKV_CHECK_ARG(grads[e] != nullptr, "null exit gradient");
    JKV_CHECK_ARG(exit_depths[e] >= 1 && exit_depths[e] <= S, "exit depth outside the ladder");
    a.grads[e] = grads[e];
    a.exit_depth[e] = exit_depths[e];
  }
  a.codes = codes;
  a.cb = code_stride_b; a.ch = code_stride_h; a.ct = code_stride_t;
  a.B = B; a.H = H; a.T = T; a.G = G; a.d = d; a.S = S; a.K = K;
  a.grad_tables = grad_tables;
  if (deterministic) {
    const int64_t need = jkv_rvq_scatter_workspace_bytes(B, H, T, G, d, S, K, 1);
    JKV_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                  "deterministic scatter needs %lld bytes of workspace", (long long)need);
    a.partials = (float*)workspace;
  }
  switch (grad_dtype) {
    case JKV_F16: return launch_scatter<JKV_F16>(a, deterministic, stream);
    case JKV_BF16: return launch_scatter<JKV_BF16>(a, deterministic, stream);
    case JKV_F32: return launch_scatter<JKV_F32>(a, deterministic, stream);
    default: return set_error(JKV_EINVAL, "unknown gradient dtype %d", grad_dtype);
  }
}

}  // extern "C"
