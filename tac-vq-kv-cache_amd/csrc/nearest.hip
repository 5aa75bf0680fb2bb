// fp32 nearest codeword per row, for the offline multi-exit additive
// coordinate refinement (src/jointkv/nested_vq.py:178-215 `_nearest_indices`
// as called at nested_vq.py:690-692): states [H,N,D], tables [H,K,D], both
// fp32 and not deployed to fp16, distance (|x|^2 + |c|^2) - 2 x.c, the lowest
// index on ties (torch.argmin's rule).
//
// One 256-thread block takes 64 rows of one head and walks the head's table
// in 64-codeword tiles.  Rows and codewords are staged in LDS with a row
// pitch of D rounded up to 4 plus 4 floats, so the 16 codeword rows a wave
// reads at one k fall in distinct banks.  Thread (r, c) of the 16 x 16 grid
// accumulates x.c for rows 4r..4r+3 and codewords 4c..4c+3 of the tile with
// float4 LDS reads and keeps each row's best (distance, index); the 16
// threads that share a row then reduce over lane shuffles.
#include "jkv_common.h"

namespace jkv {

static const int kNrRows = 64;
static const int kNrCodes = 64;
static const int kNrMaxD = 128;
static const int kNrPitch = kNrMaxD + 4;

struct NearestArgs {
  const float* states;  // [H][N][D]
  const float* tables;  // [H][K][D]
  int64_t* indices;     // [H][N]
  int64_t H, N, D, K;
};

__global__ __launch_bounds__(256) void nearest_f32_kernel(NearestArgs a) {
  __shared__ __align__(16) float xs[kNrRows * kNrPitch];
  __shared__ __align__(16) float cs[kNrCodes * kNrPitch];
  __shared__ float s_xx[kNrRows];
  __shared__ float s_cc[kNrCodes];

  const int tid = threadIdx.x;
  const int64_t h = blockIdx.y;
  const int64_t row0 = (int64_t)blockIdx.x * kNrRows;
  const int D = (int)a.D;
  const int DP = (D + 3) & ~3;
  const int64_t nrows = min((int64_t)kNrRows, a.N - row0);

  // rows of this block, zero padded to DP and to 64 rows
  const float* xsrc = a.states + (h * a.N + row0) * a.D;
  for (int i = tid; i < kNrRows * DP; i += 256) {
    const int r = i / DP, k = i - r * DP;
    xs[r * kNrPitch + k] = (r < nrows && k < D) ? xsrc[(int64_t)r * D + k] : 0.f;
  }
  __syncthreads();
  if (tid < kNrRows) {
    // |x|^2 in dimension order
    float acc = 0.f;
    for (int k = 0; k < D; ++k) acc = fmaf(xs[tid * kNrPitch + k], xs[tid * kNrPitch + k], acc);
    s_xx[tid] = acc;
  }

  const int tr = tid >> 4;  // rows 4tr..4tr+3
  const int tc = tid & 15;  // codewords 4tc..4tc+3 of a tile
  float best[4];
  int bidx[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    best[i] = __builtin_huge_valf();
    bidx[i] = 0;
  }
  const float* csrc_head = a.tables + h * a.K * a.D;
  for (int64_t c0 = 0; c0 < a.K; c0 += kNrCodes) {
    const int64_t ncodes = min((int64_t)kNrCodes, a.K - c0);
    __syncthreads();  // the previous tile's readers are done
    const float* csrc = csrc_head + c0 * a.D;
    for (int i = tid; i < kNrCodes * DP; i += 256) {
      const int r = i / DP, k = i - r * DP;
      cs[r * kNrPitch + k] = (r < ncodes && k < D) ? csrc[(int64_t)r * D + k] : 0.f;
    }
    __syncthreads();
    if (tid < kNrCodes) {
      float acc = 0.f;
      for (int k = 0; k < D; ++k) acc = fmaf(cs[tid * kNrPitch + k], cs[tid * kNrPitch + k], acc);
      s_cc[tid] = acc;
    }
    float dot[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) dot[i][j] = 0.f;
    const float* xrow = &xs[(4 * tr) * kNrPitch];
    const float* crow = &cs[(4 * tc) * kNrPitch];
    for (int k = 0; k < DP; k += 4) {
      float4 xv[4], cv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xv[i] = *(const float4*)(xrow + i * kNrPitch + k);
        cv[i] = *(const float4*)(crow + i * kNrPitch + k);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float t = dot[i][j];
          t = fmaf(xv[i].x, cv[j].x, t);
          t = fmaf(xv[i].y, cv[j].y, t);
          t = fmaf(xv[i].z, cv[j].z, t);
          t = fmaf(xv[i].w, cv[j].w, t);
          dot[i][j] = t;
        }
    }
    __syncthreads();  // s_cc of this tile is written
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = 4 * tc + j;
      if (c < ncodes) {
        const float cc = s_cc[c];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float dist = (s_xx[4 * tr + i] + cc) - 2.f * dot[i][j];
          // codewords arrive in increasing index order per thread: strict <
          // keeps the first of equal distances
          if (dist < best[i]) {
            best[i] = dist;
            bidx[i] = (int)(c0 + c);
          }
        }
      }
    }
  }
  // the 16 lanes of one row group hold disjoint codeword sets: reduce with
  // the lower index winning ties
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ob = __shfl_xor(best[i], off, 16);
      const int oi = __shfl_xor(bidx[i], off, 16);
      if (ob < best[i] || (ob == best[i] && oi < bidx[i])) {
        best[i] = ob;
        bidx[i] = oi;
      }
    }
  }
  if (tc == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * tr + i;
      if (r < nrows) a.indices[h * a.N + row0 + r] = bidx[i];
    }
  }
}


// The M nearest codewords of every row, nearest first (equal distances in
// index order), optionally skipping one index per row (`excluded`, [H][N]):
// `_nearest_topk_indices` (nested_vq.py:218-260), the shortlist search of the
// block refinement.  Same tiles as above; each thread keeps a sorted list of
// M per row, and one thread per row merges the 16 lists from LDS.
template <int M>
__global__ __launch_bounds__(256) void nearest_topk_f32_kernel(NearestArgs a, const int64_t* excluded) {
  __shared__ __align__(16) float xs[kNrRows * kNrPitch];
  __shared__ __align__(16) float cs[kNrCodes * kNrPitch];
  __shared__ float s_xx[kNrRows];
  __shared__ float s_cc[kNrCodes];
  __shared__ float cand_d[kNrRows][16 * M];
  __shared__ int cand_i[kNrRows][16 * M];

  const int tid = threadIdx.x;
  const int64_t h = blockIdx.y;
  const int64_t row0 = (int64_t)blockIdx.x * kNrRows;
  const int D = (int)a.D;
  const int DP = (D + 3) & ~3;
  const int64_t nrows = min((int64_t)kNrRows, a.N - row0);

  const float* xsrc = a.states + (h * a.N + row0) * a.D;
  for (int i = tid; i < kNrRows * DP; i += 256) {
    const int r = i / DP, k = i - r * DP;
    xs[r * kNrPitch + k] = (r < nrows && k < D) ? xsrc[(int64_t)r * D + k] : 0.f;
  }
  __syncthreads();
  if (tid < kNrRows) {
    float acc = 0.f;
    for (int k = 0; k < D; ++k) acc = fmaf(xs[tid * kNrPitch + k], xs[tid * kNrPitch + k], acc);
    s_xx[tid] = acc;
  }

  const int tr = tid >> 4;
  const int tc = tid & 15;
  int ex[4];
  float bd[4][M];
  int bi[4][M];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * tr + i;
    ex[i] = (excluded != nullptr && r < nrows) ? (int)excluded[h * a.N + row0 + r] : -1;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      bd[i][m] = __builtin_huge_valf();
      bi[i][m] = -1;
    }
  }
  const float* csrc_head = a.tables + h * a.K * a.D;
  for (int64_t c0 = 0; c0 < a.K; c0 += kNrCodes) {
    const int64_t ncodes = min((int64_t)kNrCodes, a.K - c0);
    __syncthreads();
    const float* csrc = csrc_head + c0 * a.D;
    for (int i = tid; i < kNrCodes * DP; i += 256) {
      const int r = i / DP, k = i - r * DP;
      cs[r * kNrPitch + k] = (r < ncodes && k < D) ? csrc[(int64_t)r * D + k] : 0.f;
    }
    __syncthreads();
    if (tid < kNrCodes) {
      float acc = 0.f;
      for (int k = 0; k < D; ++k) acc = fmaf(cs[tid * kNrPitch + k], cs[tid * kNrPitch + k], acc);
      s_cc[tid] = acc;
    }
    float dot[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) dot[i][j] = 0.f;
    const float* xrow = &xs[(4 * tr) * kNrPitch];
    const float* crow = &cs[(4 * tc) * kNrPitch];
    for (int k = 0; k < DP; k += 4) {
      float4 xv[4], cv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xv[i] = *(const float4*)(xrow + i * kNrPitch + k);
        cv[i] = *(const float4*)(crow + i * kNrPitch + k);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float t = dot[i][j];
          t = fmaf(xv[i].x, cv[j].x, t);
          t = fmaf(xv[i].y, cv[j].y, t);
          t = fmaf(xv[i].z, cv[j].z, t);
          t = fmaf(xv[i].w, cv[j].w, t);
          dot[i][j] = t;
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = 4 * tc + j;
      if (c < ncodes) {
        const float cc = s_cc[c];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float dd = (s_xx[4 * tr + i] + cc) - 2.f * dot[i][j];
          int ii = (int)(c0 + c);
          if (ii != ex[i] && dd < bd[i][M - 1]) {
            // insertion into the sorted list: strict < keeps equal
            // distances in arrival (index) order
#pragma unroll
            for (int m = 0; m < M; ++m) {
              if (dd < bd[i][m]) {
                const float td = bd[i][m];
                const int ti = bi[i][m];
                bd[i][m] = dd;
                bi[i][m] = ii;
                dd = td;
                ii = ti;
              }
            }
          }
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      cand_d[4 * tr + i][tc * M + m] = bd[i][m];
      cand_i[4 * tr + i][tc * M + m] = bi[i][m];
    }
  __syncthreads();
  if (tid < nrows) {
    int64_t* out = a.indices + (h * a.N + row0 + tid) * M;
    for (int m = 0; m < M; ++m) {
      float best = __builtin_huge_valf();
      int bidx = 0x7fffffff, pos = -1;
      for (int q = 0; q < 16 * M; ++q) {
        const int id = cand_i[tid][q];
        const float d = cand_d[tid][q];
        if (id >= 0 && (pos < 0 || d < best || (d == best && id < bidx))) {
          best = d;
          bidx = id;
          pos = q;
        }
      }
      out[m] = pos >= 0 ? bidx : 0;
      if (pos >= 0) cand_i[tid][pos] = -1;
    }
  }
}

}  // namespace jkv

extern "C" int jkv_nearest_f32(const float* states, int64_t H, int64_t N, int64_t D,
                               const float* tables, int64_t K, int64_t* indices,
                               jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(H > 0 && N >= 0 && K > 0, "invalid nearest-codeword geometry");
  JKV_CHECK_ARG(D > 0 && D <= kNrMaxD, "nearest-codeword dimension must lie in 1..%d (got %lld)",
                kNrMaxD, (long long)D);
  JKV_CHECK_ARG(H <= 65535, "at most 65535 heads per call (got %lld)", (long long)H);
  JKV_CHECK_ARG(K < ((int64_t)1 << 31), "nearest-codeword size too large");
  // one 256-thread block per 64 rows: the grid's x extent counts work items
  JKV_CHECK_ARG(ceil_div(N, (int64_t)kNrRows) * 256 < ((int64_t)1 << 32),
                "at most %lld rows per head (got %lld)", (long long)(kNrRows * ((((int64_t)1 << 32) - 1) / 256)),
                (long long)N);
  if (N == 0) return JKV_OK;
  JKV_CHECK_ARG(states && tables && indices, "null buffer");
  NearestArgs a = {states, tables, indices, H, N, D, K};
  dim3 grid((uint32_t)ceil_div(N, (int64_t)kNrRows), (uint32_t)H);
  hipLaunchKernelGGL(nearest_f32_kernel, grid, dim3(256), 0, stream, a);
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

extern "C" int jkv_nearest_topk_f32(const float* states, int64_t H, int64_t N, int64_t D,
                                    const float* tables, int64_t K, int64_t M,
                                    const int64_t* excluded, int64_t* indices,
                                    jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(H > 0 && N >= 0 && K > 0, "invalid nearest-codeword geometry");
  JKV_CHECK_ARG(D > 0 && D <= kNrMaxD, "nearest-codeword dimension must lie in 1..%d (got %lld)",
                kNrMaxD, (long long)D);
  JKV_CHECK_ARG(M >= 1 && M <= 8, "top-k candidate count must lie in 1..8 (got %lld)", (long long)M);
  JKV_CHECK_ARG(M < K, "top-k candidate count must lie in [1, cardinality)");
  JKV_CHECK_ARG(H <= 65535, "at most 65535 heads per call (got %lld)", (long long)H);
  JKV_CHECK_ARG(K < ((int64_t)1 << 31), "nearest-codeword size too large");
  // one 256-thread block per 64 rows: the grid's x extent counts work items
  JKV_CHECK_ARG(ceil_div(N, (int64_t)kNrRows) * 256 < ((int64_t)1 << 32),
                "at most %lld rows per head (got %lld)", (long long)(kNrRows * ((((int64_t)1 << 32) - 1) / 256)),
                (long long)N);
  if (N == 0) return JKV_OK;
  JKV_CHECK_ARG(states && tables && indices, "null buffer");
  NearestArgs a = {states, tables, indices, H, N, D, K};
  dim3 grid((uint32_t)ceil_div(N, (int64_t)kNrRows), (uint32_t)H);
  switch (M) {
#define JKV_TOPK_CASE(m) \
  case m: hipLaunchKernelGGL(nearest_topk_f32_kernel<m>, grid, dim3(256), 0, stream, a, excluded); break;
    JKV_TOPK_CASE(1) JKV_TOPK_CASE(2) JKV_TOPK_CASE(3) JKV_TOPK_CASE(4)
    JKV_TOPK_CASE(5) JKV_TOPK_CASE(6) JKV_TOPK_CASE(7) JKV_TOPK_CASE(8)
#undef JKV_TOPK_CASE
  }
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}
