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
// (stage 1: r = x, 4 steps) into a_i = c_i.r - |c_i|^2/2, and the distance
// is |r|^2 - 2 a_i.  Near-ties are far more common at d = 128 than at d = 8,
// so the key keeps the whole mantissa: with A >= |c||r| + |c|^2/2 >= |a_i|
// for every codeword of the stage (max |c|^2 per stage, a 2^-8 margin for
// rounding) and M a power of two in (2A, 4A], one fp32 subtraction gives
//   D''[i][j] = a_i - 1.5 M  in the one binade (-2M, -M).
// Sign and exponent are then common to the row and key = (bits(D'') << 9) |
// index orders by distance at 2^-23 M, ties to the lowest index.  M is a
// per-row constant and never changes the order; bounding by |c||r| rather
// than by |r|^2 keeps the step small where codewords are small next to the
// residual (the deep stages of a long residual chain).
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

// Whitened search (selector whitener W per problem, M = W^T W): the same
// tables plus M c per codeword (fp32, the u update), M in fp32 and M's rows,
// permuted into the B-operand order, as hi and lo fp16 planes.
static const int64_t kWhMcBytes = (int64_t)kFullK * kFullD * 4;  // per (problem, stage)
static const int64_t kWhMBytes = (int64_t)kFullD * kFullD * 4;   // per problem
static const int64_t kWhPermBytes = kFullTabBytes;               // hi + lo planes per problem

int64_t full_wh_workspace_bytes(int64_t P, int64_t S) {
  return full_workspace_bytes(P, S) + P * S * kWhMcBytes + P * (kWhMBytes + kWhPermBytes);
}

// One block per (problem, stage, 16 codewords): lane (codeword ci, chunk q)
// converts 8 dims, the 16 lanes of a codeword sum its norm, and the block
// writes the largest |c|^2 of its 16 codewords (the main kernel folds the 16
// partial maxima of a stage).
__device__ __forceinline__ void full_tables_block(const float* __restrict__ masters, _Float16* __restrict__ tab16,
                                                  float* __restrict__ nhalf, float* __restrict__ ncmax_part,
                                                  uint32_t bid) {
  const int64_t ps = bid >> 4;  // (problem, stage)
  const int part = bid & 15;
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

__global__ __launch_bounds__(256) void full_tables_kernel(const float* __restrict__ masters,
                                                          _Float16* __restrict__ tab16,
                                                          float* __restrict__ nhalf,
                                                          float* __restrict__ ncmax_part) {
  full_tables_block(masters, tab16, nhalf, ncmax_part, blockIdx.x);
}

// Many encodes of one geometry: job j's tables land in workspace region j
// (full_workspace_bytes(P, S) each); its blocks are [j P S 16, (j + 1) P S 16).
static const int kFullMaxJobs = 64;
struct FullPrepMany {
  const float* masters[kFullMaxJobs];
  unsigned char* ws;
  int64_t ws_stride;
  int64_t P, S;
};

// the workspace regions of one job: fp16 tables, -|c|^2/2, partial maxima
struct FullTables {
  _Float16* tab16;
  float* nhalf;
  float* ncmax;
};
__host__ __device__ __forceinline__ FullTables full_tables_at(unsigned char* ws, int64_t P, int64_t S) {
  FullTables t;
  t.tab16 = (_Float16*)ws;
  t.nhalf = (float*)(ws + P * S * (int64_t)kFullTabBytes);
  t.ncmax = (float*)(ws + P * S * ((int64_t)kFullTabBytes + kFullK * 4));
  return t;
}

__global__ __launch_bounds__(256) void full_tables_many_kernel(FullPrepMany m) {
  const uint32_t per = (uint32_t)(m.P * m.S * 16);
  const uint32_t job = blockIdx.x / per;
  const FullTables t = full_tables_at(m.ws + (int64_t)job * m.ws_stride, m.P, m.S);
  full_tables_block(m.masters[job], t.tab16, t.nhalf, t.ncmax, blockIdx.x - job * per);
}

// M = W^T W per problem, and M's rows as hi/lo fp16 planes in the order the
// mat-vec u = M x leaves in the search's B-operand layout: plane row 16c + i
// holds M row 32(c/2) + 8(i/4) + 4(c%2) + i%4, so output chunk c, lane group
// lg, element v of the mat-vec is dim 32(c/2) + 8lg + 4(c%2) + v (chunk c/2,
// word 4(c%2) + v of the lane's B operand).  Hi plane rows 0..127, lo plane
// rows 128..255.  One 256-thread block per (problem, 8 plane rows), W in LDS;
// each block writes the M rows its plane rows come from.
__global__ __launch_bounds__(256) void full_whiten_m_kernel(const float* __restrict__ whiteners,
                                                            float* __restrict__ m_out,
                                                            _Float16* __restrict__ perm) {
  extern __shared__ __align__(16) float wsh[];  // W [e][i]
  const int64_t p = blockIdx.x >> 4;
  const int r0 = (blockIdx.x & 15) * 8;
  const float* w = whiteners + p * kFullD * kFullD;
  for (int idx = threadIdx.x; idx < kFullD * kFullD / 4; idx += 256)
    *(float4*)(wsh + 4 * idx) = *(const float4*)(w + 4 * idx);
  __syncthreads();
  float* mp = m_out + p * kFullD * kFullD;
  _Float16* hi = perm + p * 2 * kFullD * kFullD;
  _Float16* lo = hi + kFullD * kFullD;
  for (int idx = threadIdx.x; idx < 8 * kFullD; idx += 256) {
    const int r = r0 + idx / kFullD, col = idx % kFullD;
    const int c = r >> 4, i = r & 15;
    const int src = 32 * (c >> 1) + 8 * (i >> 2) + 4 * (c & 1) + (i & 3);
    float v = 0.f;
    for (int e = 0; e < kFullD; ++e) v = fmaf(wsh[e * kFullD + src], wsh[e * kFullD + col], v);
    mp[src * kFullD + col] = v;
    const half_t h = (half_t)v;
    hi[r * kFullD + col] = h;
    lo[r * kFullD + col] = (half_t)(v - (float)h);
  }
}

// M c for every codeword (fp32, tiled like selector_tables128_kernel: one
// 256-thread block per (problem, stage, 64 codewords), M^T = M in LDS and the
// fp16 codewords beside it, so two blocks share a CU), the
// selector norms |W c|^2 = c . M c as the -|c'|^2/2 plane, and four partial
// maxima of |c'|^2 (the other twelve partial slots are zero).
__global__ __launch_bounds__(256) void full_whiten_tables_kernel(const _Float16* __restrict__ tab16,
                                                                 const float* __restrict__ m_all,
                                                                 float* __restrict__ mc, float* __restrict__ nhalf,
                                                                 float* __restrict__ ncmax_part, int64_t S) {
  constexpr int kKTile = 64;
  extern __shared__ __align__(16) float sm[];
  float* mt = sm;                                  // [e][i] = M[i][e] = M[e][i]
  _Float16* ct = (_Float16*)(sm + kFullD * kFullD);  // [e][k], fp16 codewords (exact)
  __shared__ float red[4];
  const int64_t ps = blockIdx.x >> 2;
  const int part = blockIdx.x & 3;
  const int k0 = part * kKTile;
  const int64_t p = ps / S;
  const int tid = threadIdx.x;
  const float* msrc = m_all + p * kFullD * kFullD;
  for (int idx = tid; idx < kFullD * kFullD / 4; idx += 256)
    *(float4*)(mt + 4 * idx) = *(const float4*)(msrc + 4 * idx);
  const _Float16* csrc = tab16 + (ps * kFullK + k0) * kFullD;
  for (int idx = tid; idx < kKTile * kFullD; idx += 256) {
    const int k = idx / kFullD, e = idx % kFullD;
    ct[e * kKTile + k] = csrc[k * kFullD + e];
  }
  __syncthreads();
  const int tx = tid & 15, ty = tid >> 4;
  float acc[4][8];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj)
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[jj][u] = 0.f;
  for (int e = 0; e < kFullD; ++e) {
    const half4 c4 = *(const half4*)(ct + e * kKTile + 4 * ty);
    const float4 m0 = *(const float4*)(mt + e * kFullD + 8 * tx);
    const float4 m1 = *(const float4*)(mt + e * kFullD + 8 * tx + 4);
    const float cv[4] = {(float)c4[0], (float)c4[1], (float)c4[2], (float)c4[3]};
    const float mv[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
      for (int u = 0; u < 8; ++u) acc[jj][u] = fmaf(cv[jj], mv[u], acc[jj][u]);
  }
  float mx = 0.f;
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int k = k0 + 4 * ty + jj;
    float* dst = mc + (ps * kFullK + k) * kFullD + 8 * tx;
    *(float4*)dst = float4{acc[jj][0], acc[jj][1], acc[jj][2], acc[jj][3]};
    *(float4*)(dst + 4) = float4{acc[jj][4], acc[jj][5], acc[jj][6], acc[jj][7]};
    // |c'|^2 = c . (M c) over this thread's 8 dims, summed over the 16 tx lanes
    float nc = 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) nc = fmaf((float)ct[(8 * tx + u) * kKTile + 4 * ty + jj], acc[jj][u], nc);
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) nc += __shfl_xor(nc, off, 16);
    if (tx == 0) nhalf[ps * kFullK + k] = -0.5f * nc;
    mx = fmaxf(mx, nc);
  }
#pragma unroll
  for (int off = 32; off >= 16; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  if (tid < 4) {
    ncmax_part[ps * 16 + 4 * part + tid] = tid == 0 ? fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) : 0.f;
  }
}

struct FullArgs {
  EncodeArgs e;
  const _Float16* tab16;
  const float* nhalf;
  const float* ncmax;
  const float* mc;          // whitened: M c per codeword [P][S][256][128]
  const _Float16* mperm;    // whitened: M's permuted rows, hi and lo planes [P][256][128]
  int64_t row_blocks;  // row blocks per problem
  int64_t blocks_per_wg;  // consecutive row blocks of one problem per workgroup (1 when whitened)
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

// WH: assignment in selector space (whitener W, M = W^T W).  Scores use the
// raw fp16 codewords against u = W^T r' (r' the selector residual), since
// c' . r' = (W c) . r' = c . u:
//   u starts at M x, and each stage subtracts M c of its winner;
//   |r'|^2 starts at x . u and each stage subtracts 2 c . u and adds |c'|^2
//   (this only sets the row's binade, never the order within the row).
// MANY: up to kFullMaxJobs encodes of one geometry (no whitener, at most two
// exits) in one launch: job j takes logical workgroups [j W, (j + 1) W) and
// its tables from workspace region j.
struct FullJobBuffers {
  const void* states;
  uint8_t* codes;
  void* recon[2];  // exits 0 and 1 of the shared exit list
};
struct FullManyArgs {
  FullArgs shape;  // geometry, exits, row blocks and runs (buffers unused)
  int64_t wgs_per_job;
  int32_t n_jobs;
  unsigned char* ws;
  int64_t ws_stride;
  FullJobBuffers buf[kFullMaxJobs];
};
template <bool MANY> struct FullArgsOf { using type = FullArgs; };
template <> struct FullArgsOf<true> { using type = FullManyArgs; };

template <int NW, bool WH, bool MANY>
__global__ __launch_bounds__(64 * NW) void rvq_encode_full_kernel(typename FullArgsOf<MANY>::type m) {
  static_assert(!(WH && MANY), "many-job launches carry no whitener");
  uint32_t L = xcd_remap(blockIdx.x, gridDim.x);
  const FullArgs* fp;
  const void* states_v;
  uint8_t* codes_p;
  const _Float16* tab16_p;
  const float* nhalf_p;
  const float* ncmax_p;
  void* rec01[2] = {nullptr, nullptr};
  if constexpr (MANY) {
    const uint32_t per = (uint32_t)m.wgs_per_job;
    const uint32_t job = L / per;
    if (job >= (uint32_t)m.n_jobs) return;  // grid padding (before any barrier)
    L -= job * per;
    fp = &m.shape;
    states_v = m.buf[job].states;
    codes_p = m.buf[job].codes;
    rec01[0] = m.buf[job].recon[0];
    rec01[1] = m.buf[job].recon[1];
    const FullTables tb = full_tables_at(m.ws + (int64_t)job * m.ws_stride, m.shape.e.H * m.shape.e.G,
                                         m.shape.e.S);
    tab16_p = tb.tab16;
    nhalf_p = tb.nhalf;
    ncmax_p = tb.ncmax;
  } else {
    fp = &m;
    states_v = m.e.states;
    codes_p = m.e.codes;
    tab16_p = m.tab16;
    nhalf_p = m.nhalf;
    ncmax_p = m.ncmax;
  }
  const FullArgs& f = *fp;
  const EncodeArgs& a = f.e;
  auto recon_of = [&](int ex) -> void* {
    if constexpr (MANY) {
      return ex == 0 ? rec01[0] : rec01[1];
    } else {
      return a.recon[ex];
    }
  };
  extern __shared__ __align__(16) unsigned char lds[];  // 2 x (table + -|c|^2/2 plane)
  __shared__ float ncm_s[kFullMaxS];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int nw = NW;  // 4 or 8 waves
  const int lg = lane >> 4, j = lane & 15;

  // logical workgroup: a run of consecutive row blocks of one problem (one
  // table set per XCD's L2); with S <= 2 both stage tables stay in LDS for
  // the whole run
  const int64_t P = a.H * a.G;
  const int64_t wgs_per_p = (f.row_blocks + f.blocks_per_wg - 1) / f.blocks_per_wg;
  if ((int64_t)L >= P * wgs_per_p) return;
  const int64_t p = (int64_t)L / wgs_per_p;
  const int64_t blk0 = ((int64_t)L % wgs_per_p) * f.blocks_per_wg;
  const int64_t nblk = min(f.blocks_per_wg, f.row_blocks - blk0);
  const int64_t h = p / a.G, g = p % a.G;
  const int S = (int)a.S;
  const bool resident = !WH && S <= 2;  // both tables loaded once per run
  const int64_t rows = a.B * a.T;
  // this lane's row of block blk0 + bi (rows past the end read row 0)
  struct RowAt {
    bool valid;
    int64_t b, t;
  };
  auto row_at = [&](int64_t bi) {
    const int64_t row = (blk0 + bi) * (16 * nw) + wave * 16 + j;
    RowAt r;
    r.valid = row < rows;
    const int64_t rw = r.valid ? row : 0;
    r.b = rw / a.T;
    r.t = rw - r.b * a.T;
    return r;
  };
  auto load_x = [&](const RowAt& r, half8 (&x)[4]) {
    const _Float16* xrow = (const _Float16*)states_v + r.b * a.sb + h * a.sh + r.t * a.st + g * kFullD;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) x[kk] = *(const half8*)(xrow + 32 * kk + 8 * lg);
  };

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
      (void*)(tab16_p + (int64_t)p * S * kFullTabHalves), (short)0, S * kFullTabBytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t plane_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(nhalf_p + (int64_t)p * S * kFullK), (short)0, S * kFullK * 4, 0x00020000);
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
  if constexpr (WH) {
    // M's permuted hi/lo rows (256 rows, like a stage table) into buffer 1
    const __amdgpu_buffer_rsrc_t perm_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(f.mperm + (int64_t)p * kFullTabHalves), (short)0, kFullTabBytes, 0x00020000);
#pragma unroll
    for (int i = 0; i < per_wave; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          perm_rsrc, (__attribute__((address_space(3))) void*)(lds + kFullBufBytes + (wave + nw * i) * 1024), 16,
          lane_off, (uint32_t)(i * nw * 1024), 0, 0);
  }
  if (tid < S) {
    const float* part = ncmax_p + ((int64_t)p * S + tid) * 16;
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) m = fmaxf(m, part[i]);
    ncm_s[tid] = m;
  }
  RowAt ra = row_at(0);
  half8 x[4];
  load_x(ra, x);
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

  for (int64_t bi = 0; bi < nblk; ++bi) {
  const bool valid = ra.valid;
  const int64_t b = ra.b, t = ra.t;
  float dec[4][8];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
#pragma unroll
    for (int e = 0; e < 8; ++e) dec[kk][e] = 0.f;
  uint8_t* const code_row = codes_p + b * a.cb + h * a.ch + t * a.ct + g * S;
  const int64_t out_off = ((b * a.H + h) * a.T + t) * Dfull + g * kFullD;

  // whitened state: u in the B-operand layout (dims 32kk + 8lg + e) and |r'|^2
  float u[4][8];
  float rr_sel = 0.f, rr0 = 0.f;
  if constexpr (WH) {
    // u = M x: output chunk c of 16 permuted rows, lane (lg, i) reads plane
    // row 16c + i (hi) and 128 + 16c + i (lo); element v lands on dim
    // 32(c/2) + 8lg + 4(c%2) + v
    const half8* tabM = (const half8*)(lds + kFullBufBytes);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int q = (4 * kk + lg) ^ j;
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(tabM[(16 * c + j) * 16 + q], x[kk], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(tabM[(128 + 16 * c + j) * 16 + q], x[kk], acc, 0, 0, 0);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) u[c >> 1][4 * (c & 1) + v] = acc[v];
    }
    float xu = 0.f;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) xu = fmaf((float)x[kk][e], u[kk][e], xu);
    rr_sel = lane_group_sum_f(xu);
    rr0 = fmaxf(rr_sel, 0.f);
    __syncthreads();  // every wave is done with M before stage 1's table lands there
  }

  for (int s = 0; s < S; ++s) {
    // streamed tables alternate buffers over the whole run (stage s of block
    // bi is the run's (bi S + s)-th table); resident ones sit in buffer s
    const int buf = resident ? s : (int)((bi * S + s) & 1);
    // the table this stage's search loads into the other buffer: the next
    // stage's, or the next block's first when the run goes on; resident
    // tables load only during the run's first block
    const bool next_stage = s + 1 < S && (!resident || bi == 0);
    const bool next_block = !resident && s + 1 == S && bi + 1 < nblk;
    const bool next = next_stage || next_block;
    const int next_s = next_stage ? s + 1 : 0;
    auto dma = [&](int t) {
      if (next) dma_step(next_s, buf ^ 1, t);
    };
    const half8* tabA = (const half8*)(lds + buf * kFullBufBytes);
    const float* nhA = (const float*)(lds + buf * kFullBufBytes + kFullTabBytes);

    // ---- B operands of this stage: r = x - dec as r_hi + r_lo, |r|^2 ----
    half8 bh[4], bl[4];
    float rr = 0.f;
    if constexpr (WH) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const half_t hi = (half_t)u[kk][e];
          bh[kk][e] = hi;
          bl[kk][e] = (half_t)fmaf((float)hi, -one, u[kk][e]);
        }
      }
    } else if (s == 0) {
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
    if constexpr (WH) {
      // the tracked |r'|^2 drifts by a few fp32 roundings of |x'|^2 per stage:
      // the bound below takes that much on top
      rr = fmaxf(rr_sel, 0.f) + rr0 * 0x1p-14f;
    } else {
      rr = lane_group_sum_f(rr);
    }
    // acc = c . r - |c|^2/2 and |acc| <= |c||r| + |c|^2/2 <= A for every
    // codeword of the stage.  With M = 2^(e+2) for A (1 + 2^-8) in
    // [2^e, 2^(e+1)), acc - 1.5 M lies in (-2M, -M), one binade whose
    // mantissa orders the distances |r|^2 - 2 acc.  Leaving |r|^2 out of the
    // bound keeps the step at 2^-21 A: at deep stages, where the codewords are
    // small next to the residual, far finer than 2^-21 |r|^2.
    const float ncm = ncm_s[s];
    const float A = (sqrtf(rr * ncm) + 0.5f * ncm) * (1.f + 0x1p-8f);
    const float M = __uint_as_float((__float_as_uint(A) & 0x7F800000u) + (2u << 23));
    const float bm = 1.5f * M;

    // x is spent for this block: the next block's rows load during the
    // last stage's search
    if (s + 1 == S && bi + 1 < nblk) {
      ra = row_at(bi + 1);
      load_x(ra, x);
    }
    const uint32_t best = (s == 0 && !WH) ? full_search<false>(tabA, nhA, bh, bl, bm, lg, j, dma)
                                          : full_search<true>(tabA, nhA, bh, bl, bm, lg, j, dma);
    // the row's winner over the four lane groups (lanes j + 16 lg hold row j)
    const uint32_t idx = lane_group_min_u(best | lg4) & 255u;
    if (valid && lg == 0) code_row[s] = (uint8_t)idx;

    // ---- dec += C[idx] (fp32, stage order) and the exits at depth s+1 ----
    float4 mcw[4][2];
    if constexpr (WH) {
      // the winner's M c row (dims 32kk + 8lg .. +8), in flight during the rest
      const float* mrow = f.mc + (((int64_t)p * S + s) * kFullK + idx) * kFullD + 8 * lg;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        mcw[kk][0] = *(const float4*)(mrow + 32 * kk);
        mcw[kk][1] = *(const float4*)(mrow + 32 * kk + 4);
      }
    }
    float cu = 0.f;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const half8 cw = tabA[idx * 16 + ((4 * kk + lg) ^ (idx & 15))];
#pragma unroll
      for (int e = 0; e < 8; ++e) dec[kk][e] = fmaf((float)cw[e], one, dec[kk][e]);
      if constexpr (WH) {
#pragma unroll
        for (int e = 0; e < 8; ++e) cu = fmaf((float)cw[e], u[kk][e], cu);
      }
    }
    if constexpr (WH) {
      // |r' - c'|^2 = |r'|^2 - 2 c . u + |c'|^2, then u -= M c
      rr_sel = rr_sel - 2.f * lane_group_sum_f(cu) - 2.f * nhA[idx];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const float mv[8] = {mcw[kk][0].x, mcw[kk][0].y, mcw[kk][0].z, mcw[kk][0].w,
                             mcw[kk][1].x, mcw[kk][1].y, mcw[kk][1].z, mcw[kk][1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) u[kk][e] -= mv[e];
      }
    }
    if (valid) {
      for (int ex = 0; ex < a.n_exits; ++ex) {
        if (a.exit_depth[ex] != s + 1 || recon_of(ex) == nullptr) continue;
        _Float16* op = (_Float16*)recon_of(ex) + out_off;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          half8 o;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = (half_t)dec[kk][e];
          *(half8*)(op + 32 * kk + 8 * lg) = o;
        }
      }
    }
    // the table loaded during this stage has landed and every wave is done
    // with this stage's (the next stage's load goes into its buffer)
    if (next) {
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
  }
  }  // row blocks of the run
}

int launch_full(const EncodeArgs& a, void* workspace, hipStream_t stream) {
  const int64_t P = a.H * a.G;
  const int64_t S = a.S;
  const bool wh = a.whiteners != nullptr;
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
  if (wh) {
    unsigned char* rest = ws + full_workspace_bytes(P, S);
    float* mc = (float*)rest;
    float* m_all = (float*)(rest + P * S * kWhMcBytes);
    _Float16* mperm = (_Float16*)(rest + P * S * kWhMcBytes + P * kWhMBytes);
    hipLaunchKernelGGL(full_whiten_m_kernel, dim3((uint32_t)(P * 16)), dim3(256), kFullD * kFullD * sizeof(float),
                       stream, a.whiteners, m_all, mperm);
    JKV_CHECK_LAUNCH();
    // the whitened norms overwrite the raw ones in the plane and the maxima
    hipLaunchKernelGGL(full_whiten_tables_kernel, dim3((uint32_t)(P * S * 4)), dim3(256),
                       kFullD * kFullD * sizeof(float) + kFullD * 64 * sizeof(_Float16), stream, tab16, m_all, mc,
                       nhalf, ncmax, S);
    JKV_CHECK_LAUNCH();
    f.mc = mc;
    f.mperm = mperm;
  }
  // waves per workgroup: 8 (128 rows) unless that leaves the chip short of
  // workgroups; each workgroup holds most of a CU's LDS
  const int64_t rows = a.B * a.T;
  int nw = kFullMaxWaves;
  while (nw > 4 && P * ceil_div(rows, 16 * nw) < 256) nw >>= 1;  // nw in {4, 8}
  if (wh) nw = 4;  // the whitened state (u) needs the registers of one wave per SIMD
  f.row_blocks = ceil_div(rows, 16 * nw);
  // runs of row blocks per workgroup: one workgroup per CU's worth of the
  // problem's blocks (tables loaded once per run; the whitened state keeps
  // one block per workgroup)
  f.blocks_per_wg = wh ? 1 : std::max<int64_t>(1, (P * f.row_blocks) / 256);
  const int64_t wgs_per_p = ceil_div(f.row_blocks, f.blocks_per_wg);
  int64_t nblocks = P * wgs_per_p;
  if (nblocks > 8) nblocks = ceil_div(nblocks, 8) * 8;  // xcd_remap needs a multiple of 8
  JKV_CHECK_ARG(nblocks < ((int64_t)1 << 31), "grid too large");
  if (wh)
    hipLaunchKernelGGL((rvq_encode_full_kernel<4, true, false>), dim3((uint32_t)nblocks), dim3(64 * 4),
                       2 * kFullBufBytes, stream, f);
  else if (nw == 8)
    hipLaunchKernelGGL((rvq_encode_full_kernel<8, false, false>), dim3((uint32_t)nblocks), dim3(64 * 8),
                       2 * kFullBufBytes, stream, f);
  else
    hipLaunchKernelGGL((rvq_encode_full_kernel<4, false, false>), dim3((uint32_t)nblocks), dim3(64 * 4),
                       2 * kFullBufBytes, stream, f);
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

// Many full-vector encodes of one geometry in two launches (every job's
// tables, then every job's search): jobs share everything but their
// buffers; no whitener; at most two exits; `workspace` holds n regions of
// full_workspace_bytes(P, S).
int launch_full_many(const EncodeArgs* jobs, int n, void* workspace, hipStream_t stream) {
  JKV_CHECK_ARG(n >= 1 && n <= kFullMaxJobs, "1 to %d jobs per launch", kFullMaxJobs);
  const EncodeArgs& a = jobs[0];
  JKV_CHECK_ARG(a.n_exits <= 2 && a.whiteners == nullptr, "many-job full-vector launches take at most two exits");
  const int64_t P = a.H * a.G;
  const int64_t S = a.S;
  const int64_t stride = full_workspace_bytes(P, S);
  unsigned char* ws = (unsigned char*)workspace;
  FullPrepMany pm = {};
  for (int j = 0; j < n; ++j) pm.masters[j] = jobs[j].tables;
  pm.ws = ws;
  pm.ws_stride = stride;
  pm.P = P;
  pm.S = S;
  JKV_CHECK_ARG(n * P * S * 16 < ((int64_t)1 << 31), "too many (problem, stage) tables");
  hipLaunchKernelGGL(full_tables_many_kernel, dim3((uint32_t)(n * P * S * 16)), dim3(256), 0, stream, pm);
  JKV_CHECK_LAUNCH();

  FullManyArgs m = {};
  m.shape.e = a;
  const int64_t rows = a.B * a.T;
  int nw = kFullMaxWaves;
  while (nw > 4 && n * P * ceil_div(rows, 16 * nw) < 256) nw >>= 1;  // nw in {4, 8}
  m.shape.row_blocks = ceil_div(rows, 16 * nw);
  // runs as long as the jobs leave two rounds of workgroups, within a problem
  m.shape.blocks_per_wg =
      std::min<int64_t>(m.shape.row_blocks, std::max<int64_t>(1, (n * P * m.shape.row_blocks) / 512));
  m.wgs_per_job = P * ceil_div(m.shape.row_blocks, m.shape.blocks_per_wg);
  m.n_jobs = n;
  m.ws = ws;
  m.ws_stride = stride;
  for (int j = 0; j < n; ++j) {
    m.buf[j].states = jobs[j].states;
    m.buf[j].codes = jobs[j].codes;
    for (int e = 0; e < a.n_exits; ++e) m.buf[j].recon[e] = jobs[j].recon[e];
  }
  int64_t nblocks = n * m.wgs_per_job;
  if (nblocks > 8) nblocks = ceil_div(nblocks, 8) * 8;  // xcd_remap needs a multiple of 8
  JKV_CHECK_ARG(nblocks < ((int64_t)1 << 31), "grid too large");
  if (nw == 8)
    hipLaunchKernelGGL((rvq_encode_full_kernel<8, false, true>), dim3((uint32_t)nblocks), dim3(64 * 8),
                       2 * kFullBufBytes, stream, m);
  else
    hipLaunchKernelGGL((rvq_encode_full_kernel<4, false, true>), dim3((uint32_t)nblocks), dim3(64 * 4),
                       2 * kFullBufBytes, stream, m);
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

}  // namespace jkv
