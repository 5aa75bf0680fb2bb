// Per-codeword sums and the residual update of the offline gain-shape k-means
// parent fitting (experiments/build_frozen_gsrq_multi_exit.py:400-657,
// `fit_residual_stages`).
//
// Sums.  Each wave owns 8 consecutive codewords of one head and one slice of
// rows.  It walks the slice's codeword indices 64 at a time (the next 64
// load while the current ones are summed); a ballot marks the rows assigned
// to its codewords and the wave takes them lowest lane first, loading up to
// 8 rows at once, so every codeword's sums run in row order.  A crowded
// codeword's rows are summed by one wave per slice, one after another.  Lane l holds
// dimensions l and l + 64 of the row (D <= 128): the row norm is one
// butterfly sum, and the normalised, weighted and plain rows are added to the
// codeword's registers.  Slices write partial sums that a second kernel adds in slice
// order, so the result does not depend on scheduling.
//
// Residual update.  residual[h, n, :] -= tables[h, indices[h, n], :], one
// thread per element.  Indices outside [0, K) match no codeword: the sums
// skip such rows and the update leaves them unchanged.
#include "jkv_common.h"

namespace jkv {

static const int kGsWaveCodes = 8;                                // codewords per wave
static const int kGsThreads = 256;                                // 4 waves
static const int kGsBlockCodes = kGsWaveCodes * (kGsThreads / 64);  // 32
static const int kGsMaxD = 128;
static const int64_t kGsTargetWaves = 4096;  // slices are added until about this many waves run
static const int64_t kGsMinSliceRows = 512;
static const int kGsBatch = 8;  // rows loaded together

struct GsArgs {
  const float* rows;       // [H][N][D]
  const int64_t* indices;  // [H][N]
  const float* weights;    // [H][N] or null (weight 1)
  int64_t H, N, D, K;
  int64_t slice_rows;
  int32_t slices;
  int32_t with_shapes;
  float* shape;  // [slices][H][K][D] (the outputs when slices == 1); null without shapes
  float* raw;    // [slices][H][K][D]
  float* den;    // [slices][H][K]
};

// sum over the 64 lanes; every lane ends with the same bits (a xor butterfly
// adds the same two values in both lanes of each pair)
__device__ __forceinline__ float gs_wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__global__ __launch_bounds__(kGsThreads) void gain_shape_sums_kernel(GsArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t h = blockIdx.z;
  const int64_t c0 = (int64_t)blockIdx.x * kGsBlockCodes + wave * kGsWaveCodes;
  if (c0 >= a.K) return;  // the whole wave
  const int64_t n0 = (int64_t)blockIdx.y * a.slice_rows;
  int64_t n1 = n0 + a.slice_rows;
  if (n1 > a.N) n1 = a.N;
  const float* rows = a.rows + h * a.N * a.D;
  const int64_t* idx = a.indices + h * a.N;
  const float* wts = a.weights ? a.weights + h * a.N : nullptr;
  const bool lo = lane < a.D, hi = lane + 64 < a.D;
  float s0[kGsWaveCodes], s1[kGsWaveCodes], r0[kGsWaveCodes], r1[kGsWaveCodes], dn[kGsWaveCodes];
#pragma unroll
  for (int c = 0; c < kGsWaveCodes; ++c) s0[c] = s1[c] = r0[c] = r1[c] = dn[c] = 0.f;

  // the next chunk's indices are loaded while the current chunk's rows are
  // summed; the rows of a chunk are loaded kGsBatch at a time
  auto rel_of = [&](int64_t base) -> int64_t {
    const int64_t n = base + lane;
    const int64_t v = idx[n < n1 ? n : n0];  // unconditional load of a valid row
    return n < n1 ? v - c0 : (int64_t)-1;
  };
  int64_t rel_next = n0 < n1 ? rel_of(n0) : (int64_t)-1;
  for (int64_t base = n0; base < n1; base += 64) {
    const int64_t rel = rel_next;
    if (base + 64 < n1) rel_next = rel_of(base + 64);
    uint64_t m = __ballot(rel >= 0 && rel < kGsWaveCodes);
    while (m) {
      int jj[kGsBatch];
      int cnt = 0;
#pragma unroll
      for (int q = 0; q < kGsBatch; ++q) {
        jj[q] = m ? __builtin_ctzll(m) : 0;  // lowest rows first
        cnt += m ? 1 : 0;
        m &= m - 1;
      }
      float x0[kGsBatch], x1[kGsBatch], wt[kGsBatch];
#pragma unroll
      for (int q = 0; q < kGsBatch; ++q) {
        // rows past cnt repeat row base and are not summed
        const float* xr = rows + (base + jj[q]) * a.D;
        x0[q] = lo ? xr[lane] : 0.f;
        x1[q] = hi ? xr[lane + 64] : 0.f;
        wt[q] = wts ? wts[base + jj[q]] : 1.f;
      }
#pragma unroll
      for (int q = 0; q < kGsBatch; ++q) {
        if (q >= cnt) break;  // uniform
        const int c = __builtin_amdgcn_readfirstlane(__shfl((int)rel, jj[q]));
        float n0v = 0.f, n1v = 0.f;
        if (a.with_shapes) {
          // x / max(|x|, 1e-8), then times the weight (two roundings, as the
          // normalise-then-weight order does)
          const float nrm =
              fmaxf(sqrtf(gs_wave_sum(__fmul_rn(x0[q], x0[q]) + __fmul_rn(x1[q], x1[q]))), 1e-8f);
          n0v = x0[q] / nrm;
          n1v = x1[q] / nrm;
          if (wts) {
            n0v = __fmul_rn(n0v, wt[q]);
            n1v = __fmul_rn(n1v, wt[q]);
          }
        }
        const float w0 = wts ? __fmul_rn(x0[q], wt[q]) : x0[q], w1 = wts ? __fmul_rn(x1[q], wt[q]) : x1[q];
#pragma unroll
        for (int k = 0; k < kGsWaveCodes; ++k) {
          if (c == k) {  // uniform
            s0[k] += n0v;
            s1[k] += n1v;
            r0[k] += w0;
            r1[k] += w1;
            dn[k] += wt[q];
          }
        }
      }
    }
  }

  const int64_t slab = ((int64_t)blockIdx.y * a.H + h) * a.K;
#pragma unroll
  for (int k = 0; k < kGsWaveCodes; ++k) {
    const int64_t c = c0 + k;
    if (c >= a.K) break;
    const int64_t o = (slab + c) * a.D;
    if (lo) a.raw[o + lane] = r0[k];
    if (hi) a.raw[o + lane + 64] = r1[k];
    if (a.with_shapes) {
      if (lo) a.shape[o + lane] = s0[k];
      if (hi) a.shape[o + lane + 64] = s1[k];
    }
    if (lane == 0) a.den[slab + c] = dn[k];
  }
}

// out[i] = sum over slices, in slice order, of part[s][i]
__global__ __launch_bounds__(256) void gain_shape_reduce_kernel(const float* __restrict__ part, int32_t slices,
                                                                int64_t n, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float acc = part[i];
  for (int s = 1; s < slices; ++s) acc += part[(int64_t)s * n + i];
  out[i] = acc;
}

__global__ __launch_bounds__(256) void subtract_codewords_kernel(float* __restrict__ residual,
                                                                 const float* __restrict__ tables,
                                                                 const int64_t* __restrict__ indices, int64_t N,
                                                                 int32_t D, int64_t K) {
  const uint32_t e = blockIdx.x * 256u + threadIdx.x;
  const int64_t h = blockIdx.y;
  if ((int64_t)e >= N * D) return;
  const uint32_t n = e / (uint32_t)D, d = e % (uint32_t)D;
  const int64_t k = indices[h * N + n];
  if (k < 0 || k >= K) return;  // not a codeword: the row is left as it is
  residual[h * N * D + e] -= tables[(h * K + k) * D + d];
}

static int64_t gs_slices(int64_t H, int64_t N, int64_t K) {
  const int64_t waves = H * ceil_div(K, kGsWaveCodes);
  int64_t s = ceil_div(kGsTargetWaves, waves);
  const int64_t cap = ceil_div(N, kGsMinSliceRows);
  if (s > cap) s = cap;
  if (s > 65535) s = 65535;
  return s < 1 ? 1 : s;
}

}  // namespace jkv

extern "C" {

int64_t jkv_gain_shape_sums_workspace_bytes(int64_t H, int64_t N, int64_t D, int64_t K, int32_t with_shapes) {
  using namespace jkv;
  if (H <= 0 || N <= 0 || D <= 0 || K <= 0) return 0;
  const int64_t slices = gs_slices(H, N, K);
  if (slices == 1) return 0;
  return slices * (H * K * D * (with_shapes ? 2 : 1) + H * K) * (int64_t)sizeof(float);
}

int jkv_gain_shape_sums(const float* rows, int64_t H, int64_t N, int64_t D, const int64_t* indices,
                        const float* weights, int64_t K, int32_t with_shapes, float* shape_sums, float* raw_sums,
                        float* denominators, void* workspace, int64_t workspace_bytes, jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(H > 0 && N >= 0 && K > 0, "invalid gain-shape geometry");
  JKV_CHECK_ARG(D > 0 && D <= kGsMaxD, "gain-shape dimension must lie in 1..%d (got %lld)", kGsMaxD,
                (long long)D);
  JKV_CHECK_ARG(H <= 65535 && K < ((int64_t)1 << 31), "gain-shape geometry too large");
  JKV_CHECK_ARG(raw_sums && denominators && (!with_shapes || shape_sums), "null buffer");
  const int64_t hk = H * K, hkd = hk * D;
  if (N == 0) {
    JKV_CHECK_HIP(hipMemsetAsync(raw_sums, 0, hkd * sizeof(float), stream));
    if (with_shapes) JKV_CHECK_HIP(hipMemsetAsync(shape_sums, 0, hkd * sizeof(float), stream));
    JKV_CHECK_HIP(hipMemsetAsync(denominators, 0, hk * sizeof(float), stream));
    return JKV_OK;
  }
  JKV_CHECK_ARG(rows && indices, "null buffer");
  const int64_t slices = gs_slices(H, N, K);
  const int64_t need = jkv_gain_shape_sums_workspace_bytes(H, N, D, K, with_shapes);
  JKV_CHECK_ARG(workspace_bytes >= need && (need == 0 || workspace),
                "gain-shape workspace too small (%lld < %lld bytes)", (long long)workspace_bytes,
                (long long)need);
  GsArgs a;
  a.rows = rows; a.indices = indices; a.weights = weights;
  a.H = H; a.N = N; a.D = D; a.K = K;
  a.slices = (int32_t)slices;
  a.slice_rows = ceil_div(N, slices);
  a.with_shapes = with_shapes ? 1 : 0;
  if (slices == 1) {
    a.shape = shape_sums; a.raw = raw_sums; a.den = denominators;
  } else {
    float* ws = (float*)workspace;
    a.raw = ws;
    a.shape = with_shapes ? ws + slices * hkd : nullptr;
    a.den = ws + slices * hkd * (with_shapes ? 2 : 1);
  }
  const dim3 grid((uint32_t)ceil_div(K, kGsBlockCodes), (uint32_t)slices, (uint32_t)H);
  hipLaunchKernelGGL(gain_shape_sums_kernel, grid, dim3(kGsThreads), 0, stream, a);
  JKV_CHECK_LAUNCH();
  if (slices > 1) {
    hipLaunchKernelGGL(gain_shape_reduce_kernel, dim3((uint32_t)ceil_div(hkd, 256)), dim3(256), 0, stream, a.raw,
                       a.slices, hkd, raw_sums);
    if (with_shapes)
      hipLaunchKernelGGL(gain_shape_reduce_kernel, dim3((uint32_t)ceil_div(hkd, 256)), dim3(256), 0, stream,
                         a.shape, a.slices, hkd, shape_sums);
    hipLaunchKernelGGL(gain_shape_reduce_kernel, dim3((uint32_t)ceil_div(hk, 256)), dim3(256), 0, stream, a.den,
                       a.slices, hk, denominators);
    JKV_CHECK_LAUNCH();
  }
  return JKV_OK;
}

int jkv_subtract_codewords(float* residual, int64_t H, int64_t N, int64_t D, const float* tables, int64_t K,
                           const int64_t* indices, jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(H > 0 && N >= 0 && D > 0 && K > 0, "invalid residual geometry");
  JKV_CHECK_ARG(H <= 65535 && N * D < ((int64_t)1 << 31), "residual slice too large");
  if (N == 0) return JKV_OK;
  JKV_CHECK_ARG(residual && tables && indices, "null buffer");
  const dim3 grid((uint32_t)ceil_div(N * D, 256), (uint32_t)H);
  hipLaunchKernelGGL(subtract_codewords_kernel, grid, dim3(256), 0, stream, residual, tables, indices, N,
                     (int32_t)D, K);
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

}  // extern "C"
