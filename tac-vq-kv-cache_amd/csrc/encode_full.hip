// Full-vector greedy residual VQ for gfx950: d = 128, K = 256, S <= 32
// stages, fp16 states, no whitener (the reference's R16/R32 geometry,
// closed_loop_vq.py:235-410 with G = 1, and the literal two-stage reading of
// the C2 configuration).
//
// full_tables_kernel deploys the fp32 masters once per call into the
// workspace: fp16 tables [P][S][256][128], the fp32 plane -|c|^2/2 [P][S][256]
// (from the fp16 codewords the search multiplies) and 16 partial maxima of
// |c|^2 per (problem, stage).
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
// fp16 words, |r - r_hi - r_lo| <= 2^-22 |r|).  The accumulator starts at
// -|c_i|^2/2 and gathers c_i.r_hi + c_i.r_lo over 4 + 4 K-steps of 32 dims
// (stage 1: r = x, 4 steps); one fp32 subtraction then gives
//   D''[i][j] = c_i.r - |c_i|^2/2 - (|r|^2 + delta)/2 - M = -(|r - c_i|^2 + delta)/2 - M.
// Near-ties are far more common at d = 128 than at d = 8, so the key keeps the
// whole mantissa: M is a power of two >= 2 (|r|^2 + max|c|^2 + delta) > 2 max_i
// (|r - c_i|^2 + delta)/2, which puts every D'' of the row in the one binade
// (-2M, -M).  Sign and exponent are then common to the row and key =
// (bits(D'') << 9) | index orders by distance at 2^-23 M, ties to the lowest
// index.  delta = 2^-8 (|r|^2 + max|c|^2) keeps every D'' below -M; M is a
// per-row constant and never changes the order.
#include "encode_args.h"

namespace jkv {

static const int kFullD = 128;
static const int kFullK = 256;
static const int kFullMaxS = 32;
static const int kFullTabHalves = kFullK * kFullD;         // one stage table
static const int kFullTabBytes = kFullTabHalves * 2;      // 64 KiB
static const int kFullBufBytes = kFullTabBytes + kFullK * 4;  // + -|c|^2/2 plane
static const int kFullMaxWaves = 8;

int64_t full_workspace_bytes(int64_t P, int64_t S) {
  return P * S * ((int64_t)kFullTabBytes + kFullK * 4 + 16 * 4);
}

// One block per (problem, stage, 16 codewords): lane (codeword ci, chunk q)
// converts 8 dims, the 16 lanes of a codeword sum its norm, and the block
// writes the largest |c|^2 of its 16 codewords (the main kernel folds the 16
// partial maxima of a stage).
__global__ __launch_bounds__(256) void full_tables_kernel(const float* __restrict__ masters,
                                                          _Float16* __restrict__ tab16,
                                                          float* __restrict__ nhalf,
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
  if (q == 0) nhalf[ps * kFullK + k] = -0.5f * nc;
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
  const float* nhalf;
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

// Distances of a wave's 16 rows to the stage's 256 codewords: 16 steps (four
// passes of four K-steps over four 16-codeword chunks); returns the lane's
// smallest key.  A operands run two steps ahead through a three-slot ring; a
// pass's accumulator seeds (-|c|^2/2) load at the start of the pass before,
// alternating between two seed sets so each pass accumulates in place; the
// caller's `dma(step)` issues a sixteenth of the next stage's table loads in
// each step.  Everything is unrolled, so LDS addresses are a per-lane base
// plus an immediate offset; scheduling barriers keep the order as written.
template <bool LO, typename Dma>
__device__ __forceinline__ uint32_t full_search(const half8* __restrict__ tabA, const float* __restrict__ nhA,
                                                const half8 (&bh)[4], const half8 (&bl)[4], float bm, int lg,
                                                int j, Dma&& dma) {
  // chunk (4kk + lg) of codeword 16m + j sits at tabA[(16m + j) * 16 + ((4kk + lg) ^ j)]
  const half8* ak[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) ak[kk] = tabA + j * 16 + ((4 * kk + lg) ^ j);
  const float* nl = nhA + 4 * lg;
  uint32_t best = 0xFFFFFFFFu;
  half8 ring[3][4];
  float4v seed[2][4];
  auto load_step = [&](int i) {
    const int c = 4 * (i >> 2), kk = i & 3;
#pragma unroll
    for (int u = 0; u < 4; ++u) ring[i % 3][u] = ak[kk][(c + u) * 256];
  };
  auto load_seeds = [&](int pass) {
#pragma unroll
    for (int u = 0; u < 4; ++u) seed[pass & 1][u] = *(const float4v*)(nl + 16 * (4 * pass + u));
  };
  load_seeds(0);
  load_step(0);
  load_step(1);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int pass = i >> 2, kk = i & 3;
    if (i + 2 < 16) load_step(i + 2);
    if (kk == 0 && pass + 1 < 4) load_seeds(pass + 1);
    dma(i);
    float4v (&acc)[4] = seed[pass & 1];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ring[i % 3][u], bh[kk], acc[u], 0, 0, 0);
      if (LO) acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ring[i % 3][u], bl[kk], acc[u], 0, 0, 0);
    }
    if (kk == 3) {
      // key = mantissa of D'' above the index: lanes add the low bits v (0..3)
      // per value and the chunk bits 16 (c + u) per chunk after its minimum
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t k0 = (__float_as_uint(acc[u][0] - bm) << 9) | 0u;
        const uint32_t k1 = (__float_as_uint(acc[u][1] - bm) << 9) | 1u;
        const uint32_t k2 = (__float_as_uint(acc[u][2] - bm) << 9) | 2u;
        const uint32_t k3 = (__float_as_uint(acc[u][3] - bm) << 9) | 3u;
        const uint32_t m = min(umin3_f(k0, k1, k2), k3) | (uint32_t)(16 * (4 * pass + u));
        best = min(best, m);
      }
      // the pass's keys are final here (left to itself the compiler sinks them
      // to the end, keeping all 16 accumulators live); emits nothing
      asm volatile("" : "+v"(best));
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  return best;
}

template <int NW>
__global__ __launch_bounds__(64 * NW) void rvq_encode_full_kernel(FullArgs f) {
  const EncodeArgs& a = f.e;
  extern __shared__ __align__(16) unsigned char lds[];  // 2 x (table + -|c|^2/2 plane)
  __shared__ float ncm_s[kFullMaxS];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int nw = NW;  // 4 or 8 waves
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

  // stage tables: 64 direct buffer->LDS loads of 1 KiB (4 codeword rows) plus
  // one of the -|c|^2/2 plane.  Wave w issues loads k = w + nw*i, i < 64/nw;
  // load k carries codeword rows 4k..4k+3, lane (lg, q) chunk q of row 4k + lg
  // into swizzled slot q ^ ((4k + lg) & 15).  With nw a multiple of 4 that slot
  // is the same for every i, so each load is one per-lane 32-bit offset plus a
  // uniform one.  (MUBUF rather than global_load_lds: the compiler's wait
  // counting treats the latter as a flat access to both memories and then
  // drains every LDS read to zero, which undoes the search's prefetching.)
  constexpr int per_wave = 64 / nw;
  const int rlane = 4 * wave + lg;  // row 4k + lg for i = 0
  const uint32_t lane_off = (uint32_t)(rlane * kFullD + 8 * ((lane & 15) ^ (rlane & 15))) * 2u;
  const __amdgpu_buffer_rsrc_t tab_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(f.tab16 + (int64_t)p * S * kFullTabHalves), (short)0, S * kFullTabBytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t plane_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(f.nhalf + (int64_t)p * S * kFullK), (short)0, S * kFullK * 4, 0x00020000);
  auto dma_load = [&](int s, int buf, int i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        tab_rsrc, (__attribute__((address_space(3))) void*)(lds + buf * kFullBufBytes + (wave + nw * i) * 1024), 16,
        lane_off, (uint32_t)(s * kFullTabBytes + i * nw * 1024), 0, 0);
  };
  auto dma_plane = [&](int s, int buf) {
    if (wave == nw - 1) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          plane_rsrc, (__attribute__((address_space(3))) void*)(lds + buf * kFullBufBytes + kFullTabBytes), 16,
          (uint32_t)lane * 16u, (uint32_t)(s * kFullK * 4), 0, 0);
    }
  };
  // step t of 16 issues this wave's loads [t * per_wave / 16, (t + 1) * per_wave / 16)
  auto dma_step = [&](int s, int buf, int t) {
#pragma unroll
    for (int i = (t * per_wave) >> 4; i < ((t + 1) * per_wave) >> 4; ++i) dma_load(s, buf, i);
    if (t == 0) dma_plane(s, buf);
  };
  auto dma_stage = [&](int s, int buf) {
    for (int t = 0; t < 16; ++t) dma_step(s, buf, t);
  };

  dma_stage(0, 0);
  if (tid < S) {
    const float* part = f.ncmax + ((int64_t)p * S + tid) * 16;
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) m = fmaxf(m, part[i]);
    ncm_s[tid] = m;
  }
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
  // 1.0 the compiler cannot see: fma(fp16 -> fp32 operand, one, c) then stays
  // one v_fma_mix (convert and add in one instruction; fma(a, 1, c) rounds
  // once, exactly like a + c) instead of a conversion plus an add
  float one = 1.0f;
  asm volatile("" : "+v"(one));
  const int64_t Dfull = a.G * kFullD;
  const int64_t out_off = ((b * a.H + h) * a.T + t) * Dfull + g * kFullD;

  for (int s = 0; s < S; ++s) {
    const int buf = s & 1;
    const bool next = s + 1 < S;
    auto dma = [&](int t) {
      if (next) dma_step(s + 1, buf ^ 1, t);
    };
    const half8* tabA = (const half8*)(lds + buf * kFullBufBytes);
    const float* nhA = (const float*)(lds + buf * kFullBufBytes + kFullTabBytes);

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
          const float r = fmaf((float)x[kk][e], one, -dec[kk][e]);
          const half_t hi = (half_t)r;
          bh[kk][e] = hi;
          bl[kk][e] = (half_t)fmaf((float)hi, -one, r);
          rr = fmaf(r, r, rr);
        }
      }
    }
    rr = lane_group_sum_f(rr);
    const float ncm = ncm_s[s];
    const float delta = (rr + ncm) * 0x1p-8f;
    // M = 2^(e+2) for rr + ncm + delta in [2^e, 2^(e+1))
    const float M = __uint_as_float((__float_as_uint(rr + ncm + delta) & 0x7F800000u) + (2u << 23));
    const float bm = (rr + delta) * 0.5f + M;

    const uint32_t best = s == 0 ? full_search<false>(tabA, nhA, bh, bl, bm, lg, j, dma)
                                 : full_search<true>(tabA, nhA, bh, bl, bm, lg, j, dma);
    // the row's winner over the four lane groups (lanes j + 16 lg hold row j)
    const uint32_t idx = lane_group_min_u(best | lg4) & 255u;
    if (valid && lg == 0) code_row[s] = (uint8_t)idx;

    // ---- dec += C[idx] (fp32, stage order) and the exits at depth s+1 ----
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const half8 cw = tabA[idx * 16 + ((4 * kk + lg) ^ (idx & 15))];
#pragma unroll
      for (int e = 0; e < 8; ++e) dec[kk][e] = fmaf((float)cw[e], one, dec[kk][e]);
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
  float* nhalf = (float*)(ws + P * S * (int64_t)kFullTabBytes);
  float* ncmax = (float*)(ws + P * S * ((int64_t)kFullTabBytes + kFullK * 4));
  JKV_CHECK_ARG(P * S * 16 < ((int64_t)1 << 31), "too many (problem, stage) tables");
  hipLaunchKernelGGL(full_tables_kernel, dim3((uint32_t)(P * S * 16)), dim3(256), 0, stream, a.tables,
                     tab16, nhalf, ncmax);
  JKV_CHECK_LAUNCH();

  FullArgs f = {};
  f.e = a;
  f.tab16 = tab16;
  f.nhalf = nhalf;
  f.ncmax = ncmax;
  // waves per workgroup: 8 (128 rows) unless that leaves the chip short of
  // workgroups; each workgroup holds most of a CU's LDS
  const int64_t rows = a.B * a.T;
  int nw = kFullMaxWaves;
  while (nw > 4 && P * ceil_div(rows, 16 * nw) < 256) nw >>= 1;  // nw in {4, 8}
  f.row_blocks = ceil_div(rows, 16 * nw);
  int64_t nblocks = P * f.row_blocks;
  if (nblocks > 8) nblocks = ceil_div(nblocks, 8) * 8;  // xcd_remap needs a multiple of 8
  JKV_CHECK_ARG(nblocks < ((int64_t)1 << 31), "grid too large");
  if (nw == 8)
    hipLaunchKernelGGL(rvq_encode_full_kernel<8>, dim3((uint32_t)nblocks), dim3(64 * 8), 2 * kFullBufBytes,
                       stream, f);
  else
    hipLaunchKernelGGL(rvq_encode_full_kernel<4>, dim3((uint32_t)nblocks), dim3(64 * 4), 2 * kFullBufBytes,
                       stream, f);
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

}  // namespace jkv
