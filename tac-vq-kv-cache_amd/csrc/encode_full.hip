// Full-vector greedy residual VQ for gfx950: d = 128, K = 256, S <= 32
// stages, fp16 states, no whitener (the reference's R16/R32 geometry,
// closed_loop_vq.py:235-410 with G = 1, and the literal two-stage reading of
// the C2 configuration).
//
// full_tables_kernel deploys the fp32 masters once per call into the
// workspace: fp16 tables [P][S][256][128], a bias plane [P][S][256] of
// (n_hi, n_lo, 2^12, 2^12, 0, 0, 0, 0) with n = |c|^2/2 in two fp16 halves,
// and 16 partial maxima of |c|^2 per (problem, stage).
//
// rvq_encode_full_kernel: one workgroup of up to 8 waves per (problem, block
// of 16 rows per wave).  Stage tables stream through LDS with direct
// global->LDS loads, double-buffered: stage s+1 lands while stage s runs.
// Codeword rows are stored with their 16-byte chunks XOR-swizzled by the row
// index (chunk q of row r at r*256 + 16*(q ^ (r & 15))), so the MFMA's A reads
// of 16 consecutive codewords hit 16 distinct bank groups.
//
// Each wave keeps its 16 rows in registers in the B-operand layout of
// v_mfma_f32_16x16x32_f16 (lane (lg, j) holds dims [32kk + 8lg, +8) of row j
// for kk = 0..3): the input x (fp16) and the running reconstruction `dec`
// (fp32, the reference's `decoded` buffer, summed in stage order).  Stage s
// searches with the fp32 residual r = x - dec, carried as r_hi + r_lo (two
// fp16 words, |r - r_hi - r_lo| <= 2^-22 |r|):
//   D[i][j] = c_i.r_hi + c_i.r_lo - |c_i|^2/2 - (|r|^2 + delta)/2
// over 4 + 4 K-steps of 32 dims plus one bias step (stage 1: r = x, 4 + 1).
// Near-ties are far more common at d = 128 than at d = 8, so the key keeps the
// whole mantissa: the row bias also carries a power of two M >= 2 (|r|^2 +
// max|c|^2 + delta) > 4 max_i (|r - c_i|^2 + delta)/2, which puts every D'' =
// D - M of the row in the one binade [-2M, -M).  Sign and exponent are then
// common to the row and key = (bits(D'') << 9) | index orders by distance at
// 2^-23 M, ties to the lowest index.  delta = 2^-8 (|r|^2 + max|c|^2) keeps
// every D below zero; M is a per-row constant and never changes the order.
#include "encode_args.h"

namespace jkv {

static const int kFullD = 128;
static const int kFullK = 256;
static const int kFullMaxS = 32;
static const int kFullTabHalves = kFullK * kFullD;         // one stage table
static const int kFullTabBytes = kFullTabHalves * 2;      // 64 KiB
static const int kFullBufBytes = kFullTabBytes + kFullK * 16;  // + bias plane
static const int kFullMaxWaves = 8;

int64_t full_workspace_bytes(int64_t P, int64_t S) {
  return P * S * ((int64_t)kFullTabBytes + kFullK * 16 + 16 * 4);
}

// One block per (problem, stage, 16 codewords): lane (codeword ci, chunk q)
// converts 8 dims, the 16 lanes of a codeword sum its norm, and the block
// writes the largest |c|^2 of its 16 codewords (the main kernel folds the 16
// partial maxima of a stage).
__global__ __launch_bounds__(256) void full_tables_kernel(const float* __restrict__ masters,
                                                          _Float16* __restrict__ tab16,
                                                          half8* __restrict__ bias_plane,
                                                          float* __restrict__ ncmax_part) {
  const int64_t ps = blockIdx.x >> 4;  // (problem, stage)
  const int part = blockIdx.x & 15;
  const int tid = threadIdx.x;
  const int k = part * 16 + (tid >> 4), q = tid & 15;
  const int64_t row = (ps * kFullK + k) * kFullD + 8 * q;
  const float4 v0 = *(const float4*)(masters + row);
  const float4 v1 = *(const float4*)(masters + row + 4);
  const half8 w = {(half_t)v0.x, (half_t)v0.y, (half_t)v0.z, (half_t)v0.w,
                   (half_t)v1.x, (half_t)v1.y, (half_t)v1.z, (half_t)v1.w};
  *(half8*)(tab16 + row) = w;
  float nc = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) nc = fmaf((float)w[e], (float)w[e], nc);
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) nc += __shfl_xor(nc, off, 16);
  if (q == 0) {
    const float halfn = 0.5f * nc;
    const half_t nhi = (half_t)halfn;
    const half_t nlo = (half_t)(halfn - (float)nhi);
    bias_plane[ps * kFullK + k] =
        half8{nhi, nlo, (half_t)4096.f, (half_t)4096.f, (half_t)0.f, (half_t)0.f, (half_t)0.f, (half_t)0.f};
  }
  __shared__ float red[4];
  float mx = nc;
#pragma unroll
  for (int off = 32; off >= 16; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  if (tid == 0) ncmax_part[ps * 16 + part] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

struct FullArgs {
  EncodeArgs e;
  const _Float16* tab16;
  const half8* bias_plane;
  const float* ncmax;
  int64_t row_blocks;  // row blocks per problem
};

__device__ __forceinline__ uint32_t umin3_f(uint32_t a, uint32_t b, uint32_t c) {
  return min(min(a, b), c);
}

// sum / min over lanes {j, j+16, j+32, j+48}
__device__ __forceinline__ float lane_group_sum_f(float v) {
  auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float a = __uint_as_float((uint32_t)s16[0]) + __uint_as_float((uint32_t)s16[1]);
  auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a), false, false);
  return __uint_as_float((uint32_t)s32[0]) + __uint_as_float((uint32_t)s32[1]);
}
__device__ __forceinline__ uint32_t lane_group_min_u(uint32_t v) {
  auto s16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  const uint32_t m = min((uint32_t)s16[0], (uint32_t)s16[1]);
  auto s32 = __builtin_amdgcn_permlane32_swap(m, m, false, false);
  return min((uint32_t)s32[0], (uint32_t)s32[1]);
}

__global__ __launch_bounds__(512) void rvq_encode_full_kernel(FullArgs f) {
  const EncodeArgs& a = f.e;
  extern __shared__ __align__(16) unsigned char lds[];  // 2 x (table + bias plane)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = (int)(blockDim.x >> 6);
  const int lg = lane >> 4, j = lane & 15;

  // logical block: row blocks of one problem are consecutive (one table set
  // per XCD's L2)
  const uint32_t L = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t P = a.H * a.G;
  if ((int64_t)L >= P * f.row_blocks) return;
  const int64_t p = (int64_t)L / f.row_blocks;
  const int64_t blk = (int64_t)L % f.row_blocks;
  const int64_t h = p / a.G, g = p % a.G;
  const int S = (int)a.S;
  const int64_t rows = a.B * a.T;
  const int64_t row = blk * (16 * nw) + wave * 16 + j;
  const bool valid = row < rows;
  const int64_t rw = valid ? row : 0;
  const int64_t b = rw / a.T, t = rw - (rw / a.T) * a.T;
  const _Float16* xrow = (const _Float16*)a.states + b * a.sb + h * a.sh + t * a.st + g * kFullD;

  // stage tables: 64 direct loads of 1 KiB (4 codeword rows) plus 4 of the
  // bias plane, spread over the waves
  auto dma_stage = [&](int s, int buf) {
    unsigned char* base = lds + buf * kFullBufBytes;
    const _Float16* src_tab = f.tab16 + ((int64_t)p * S + s) * kFullTabHalves;
    for (int k = wave; k < 64; k += nw) {
      const int r = 4 * k + (lane >> 4), q = lane & 15;
      __builtin_amdgcn_global_load_lds(
          (const void __attribute__((address_space(1)))*)(src_tab + r * kFullD + 8 * (q ^ (r & 15))),
          (void __attribute__((address_space(3)))*)(base + k * 1024), 16, 0, 0);
    }
    const half8* src_bias = f.bias_plane + ((int64_t)p * S + s) * kFullK;
    for (int k = wave; k < 4; k += nw) {
      __builtin_amdgcn_global_load_lds(
          (const void __attribute__((address_space(1)))*)(src_bias + 64 * k + lane),
          (void __attribute__((address_space(3)))*)(base + kFullTabBytes + k * 1024), 16, 0, 0);
    }
  };

  dma_stage(0, 0);
  half8 x[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) x[kk] = *(const half8*)(xrow + 32 * kk + 8 * lg);
  float dec[4][8];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
#pragma unroll
    for (int e = 0; e < 8; ++e) dec[kk][e] = 0.f;
  uint8_t* const code_row = a.codes + b * a.cb + h * a.ch + t * a.ct + g * S;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const uint32_t lg4 = (uint32_t)lg << 2;
  const half8 zero8 = {};
  const float4v zero4 = {0.f, 0.f, 0.f, 0.f};
  const int64_t Dfull = a.G * kFullD;
  const int64_t out_off = ((b * a.H + h) * a.T + t) * Dfull + g * kFullD;

  for (int s = 0; s < S; ++s) {
    const int buf = s & 1;
    if (s + 1 < S) dma_stage(s + 1, buf ^ 1);
    const half8* tabA = (const half8*)(lds + buf * kFullBufBytes);
    const half8* biasA = (const half8*)(lds + buf * kFullBufBytes + kFullTabBytes);

    // ---- B operands of this stage: r = x - dec as r_hi + r_lo, |r|^2 ----
    half8 bh[4], bl[4];
    float rr = 0.f;
    if (s == 0) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        bh[kk] = x[kk];
        bl[kk] = zero8;
#pragma unroll
        for (int e = 0; e < 8; ++e) rr = fmaf((float)x[kk][e], (float)x[kk][e], rr);
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float r = (float)x[kk][e] - dec[kk][e];
          const half_t hi = (half_t)r;
          bh[kk][e] = hi;
          bl[kk][e] = (half_t)(r - (float)hi);
          rr = fmaf(r, r, rr);
        }
      }
    }
    rr = lane_group_sum_f(rr);
    float ncm = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) ncm = fmaxf(ncm, f.ncmax[((int64_t)p * S + s) * 16 + i]);
    const float delta = (rr + ncm) * 0x1p-8f;
    // M = 2^(e+2) for rr + ncm + delta in [2^e, 2^(e+1))
    const float M = __uint_as_float((__float_as_uint(rr + ncm + delta) & 0x7F800000u) + (2u << 23));
    const float beta_s = ((rr + delta) * 0.5f + M) * 0x1p-12f;
    const half_t bhi = (half_t)beta_s;
    const half_t blo = (half_t)(beta_s - (float)bhi);
    const half8 bbias = lg == 0 ? half8{(half_t)-1.f, (half_t)-1.f, -bhi, -blo, (half_t)0.f, (half_t)0.f,
                                        (half_t)0.f, (half_t)0.f}
                                : zero8;

    // ---- distances to the 256 codewords, two 16-codeword chunks at a time ----
    uint32_t best = 0xFFFFFFFFu;
    auto keys = [&](const float4v& v, int c) {
      const uint32_t k0 = (__float_as_uint(v[0]) << 9) | (uint32_t)(16 * c + 0);
      const uint32_t k1 = (__float_as_uint(v[1]) << 9) | (uint32_t)(16 * c + 1);
      const uint32_t k2 = (__float_as_uint(v[2]) << 9) | (uint32_t)(16 * c + 2);
      const uint32_t k3 = (__float_as_uint(v[3]) << 9) | (uint32_t)(16 * c + 3);
      best = umin3_f(umin3_f(k0, k1, k2), k3, best);
    };
    const bool lo = s > 0;
    // four independent 16-codeword chunks per pass (a rolled loop: unrolled,
    // the compiler hoists every chunk's A loads)
#pragma unroll 1
    for (int c = 0; c < 16; c += 4) {
      float4v acc[4];
      int w[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        acc[u] = zero4;
        w[u] = 16 * (c + u) + j;
      }
      // A operands of K-step kk+1 load while kk's MFMAs run
      half8 A[2][4];
#pragma unroll
      for (int u = 0; u < 4; ++u) A[0][u] = tabA[w[u] * 16 + (lg ^ (w[u] & 15))];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if (kk + 1 < 4) {
#pragma unroll
          for (int u = 0; u < 4; ++u) A[(kk + 1) & 1][u] = tabA[w[u] * 16 + ((4 * (kk + 1) + lg) ^ (w[u] & 15))];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
          acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[kk & 1][u], bh[kk], acc[u], 0, 0, 0);
        if (lo) {
#pragma unroll
          for (int u = 0; u < 4; ++u)
            acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[kk & 1][u], bl[kk], acc[u], 0, 0, 0);
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(lg == 0 ? biasA[w[u]] : zero8, bbias, acc[u], 0, 0, 0);
        keys(acc[u], c + u);
      }
    }
    // the row's winner over the four lane groups (lanes j + 16 lg hold row j)
    const uint32_t idx = lane_group_min_u(best | lg4) & 255u;
    if (valid && lg == 0) code_row[s] = (uint8_t)idx;

    // ---- dec += C[idx] (fp32, stage order) and the exits at depth s+1 ----
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const half8 cw = tabA[idx * 16 + ((4 * kk + lg) ^ (idx & 15))];
#pragma unroll
      for (int e = 0; e < 8; ++e) dec[kk][e] += (float)cw[e];
    }
    if (valid) {
      for (int ex = 0; ex < a.n_exits; ++ex) {
        if (a.exit_depth[ex] != s + 1 || a.recon[ex] == nullptr) continue;
        _Float16* op = (_Float16*)a.recon[ex] + out_off;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          half8 o;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = (half_t)dec[kk][e];
          *(half8*)(op + 32 * kk + 8 * lg) = o;
        }
      }
    }
    // stage s+1's table has landed and every wave is done with stage s's
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
}

int launch_full(const EncodeArgs& a, void* workspace, hipStream_t stream) {
  const int64_t P = a.H * a.G;
  const int64_t S = a.S;
  unsigned char* ws = (unsigned char*)workspace;
  _Float16* tab16 = (_Float16*)ws;
  half8* bias_plane = (half8*)(ws + P * S * (int64_t)kFullTabBytes);
  float* ncmax = (float*)(ws + P * S * ((int64_t)kFullTabBytes + kFullK * 16));
  JKV_CHECK_ARG(P * S * 16 < ((int64_t)1 << 31), "too many (problem, stage) tables");
  hipLaunchKernelGGL(full_tables_kernel, dim3((uint32_t)(P * S * 16)), dim3(256), 0, stream, a.tables,
                     tab16, bias_plane, ncmax);
  JKV_CHECK_LAUNCH();

  FullArgs f = {};
  f.e = a;
  f.tab16 = tab16;
  f.bias_plane = bias_plane;
  f.ncmax = ncmax;
  // waves per workgroup: 8 (128 rows) unless that leaves the chip short of
  // workgroups; each workgroup holds most of a CU's LDS
  const int64_t rows = a.B * a.T;
  int nw = kFullMaxWaves;
  while (nw > 2 && P * ceil_div(rows, 16 * nw) < 256) nw >>= 1;
  f.row_blocks = ceil_div(rows, 16 * nw);
  int64_t nblocks = P * f.row_blocks;
  if (nblocks > 8) nblocks = ceil_div(nblocks, 8) * 8;  // xcd_remap needs a multiple of 8
  JKV_CHECK_ARG(nblocks < ((int64_t)1 << 31), "grid too large");
  hipLaunchKernelGGL(rvq_encode_full_kernel, dim3((uint32_t)nblocks), dim3(64 * nw), 2 * kFullBufBytes,
                     stream, f);
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

}  // namespace jkv
