// Hard greedy residual-VQ / grouped-CQ encode for gfx950.
//
// Two kernels share one argument block:
//  * rvq_encode_mfma<D,S>: fp16 states, d in {4,8}, K=256, S<=2, no whitener.
//    A workgroup owns one (head, group) problem and a chunk of rows; the
//    problem's codebooks are staged in LDS and feed the A operand of the
//    MFMAs (codewords x contraction slots; 32x32x16 in stage 1, 16x16x32 in
//    stage 2); row tiles are the B operand.  The contraction packs
//    [x | -c_prev | norm] so one MFMA yields -(|r - c|^2 + delta)/2 for a
//    tile of codewords x rows with exact products and fp32 accumulation; the
//    argmin is a min over keys that carry the codeword index in their low
//    bits.
//  * rvq_encode_generic<DT,DMAX>: any dtype, d<=128, K<=256, any S, optional
//    whitener; one thread per row, fp32 distances in the reference's
//    |r|^2 + |c|^2 - 2 r.c form.
#include "encode_args.h"

namespace jkv {

// ---------------------------------------------------------------------------
// Whitened selector tables: sel[p,s,k,i] = sum_e fp16(C[p,s,k,e]) * W[p,i,e]
// (einsum "hrke,hde->hrkd", closed_loop_vq.py:324; bmm(C, F^T), cq_tac.py:84)
__global__ void selector_tables_kernel(const float* __restrict__ tables,
                                       const float* __restrict__ whiteners,
                                       float* __restrict__ sel, int64_t P,
                                       int64_t S, int64_t K, int64_t d) {
  int64_t n = P * S * K * d;
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  int64_t i = idx % d;
  int64_t row = idx / d;  // (p,s,k)
  int64_t p = row / (S * K);
  const float* c = tables + row * d;
  const float* w = whiteners + (p * d + i) * d;
  float acc = 0.f;
  for (int64_t e = 0; e < d; ++e) acc = fmaf(deploy16(c[e]), w[e], acc);
  sel[idx] = acc;
}

// The same tables for d = 128, tiled: one 256-thread block per (p, s, 64
// codewords) holds W^T (64 KiB) and the codewords transposed (32 KiB) in LDS;
// thread (tx, ty) accumulates outputs i = 8tx..8tx+7 of codewords
// k = 4ty..4ty+3 over e in order, so every value equals the one-thread-per-
// output kernel's bit for bit.
__global__ __launch_bounds__(256) void selector_tables128_kernel(const float* __restrict__ tables,
                                                                 const float* __restrict__ whiteners,
                                                                 float* __restrict__ sel, int64_t S) {
  constexpr int kD = 128, kKTile = 64;
  extern __shared__ __align__(16) float sm[];
  float* wt = sm;              // [e][i]
  float* ct = sm + kD * kD;    // [e][k]
  const int64_t blk = blockIdx.x;
  const int64_t ps = blk / (256 / kKTile);  // (p, s)
  const int k0 = (int)(blk % (256 / kKTile)) * kKTile;
  const int64_t p = ps / S;
  const int tid = threadIdx.x;
  const float* wsrc = whiteners + p * kD * kD;
  for (int idx = tid; idx < kD * kD / 4; idx += 256) {
    const int i = idx / (kD / 4), e4 = (idx % (kD / 4)) * 4;
    const float4 v = *(const float4*)(wsrc + i * kD + e4);
    wt[(e4 + 0) * kD + i] = v.x;
    wt[(e4 + 1) * kD + i] = v.y;
    wt[(e4 + 2) * kD + i] = v.z;
    wt[(e4 + 3) * kD + i] = v.w;
  }
  const float* csrc = tables + (ps * 256 + k0) * kD;
  for (int idx = tid; idx < kKTile * kD / 4; idx += 256) {
    const int k = idx / (kD / 4), e4 = (idx % (kD / 4)) * 4;
    const float4 v = *(const float4*)(csrc + k * kD + e4);
    ct[(e4 + 0) * kKTile + k] = deploy16(v.x);
    ct[(e4 + 1) * kKTile + k] = deploy16(v.y);
    ct[(e4 + 2) * kKTile + k] = deploy16(v.z);
    ct[(e4 + 3) * kKTile + k] = deploy16(v.w);
  }
  __syncthreads();
  const int tx = tid & 15, ty = tid >> 4;
  float acc[4][8];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[j][u] = 0.f;
  for (int e = 0; e < kD; ++e) {
    const float4 c4 = *(const float4*)(ct + e * kKTile + 4 * ty);
    const float4 w0 = *(const float4*)(wt + e * kD + 8 * tx);
    const float4 w1 = *(const float4*)(wt + e * kD + 8 * tx + 4);
    const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int u = 0; u < 8; ++u) acc[j][u] = fmaf(cv[j], wv[u], acc[j][u]);
  }
  float* dst = sel + (ps * 256 + k0 + 4 * ty) * kD + 8 * tx;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    *(float4*)(dst + j * kD) = float4{acc[j][0], acc[j][1], acc[j][2], acc[j][3]};
    *(float4*)(dst + j * kD + 4) = float4{acc[j][4], acc[j][5], acc[j][6], acc[j][7]};
  }
}

// ---------------------------------------------------------------------------
// Generic fp32 kernel.
template <int DT, int DMAX>
__global__ __launch_bounds__(256) void rvq_encode_generic(EncodeArgs a) {
  const int64_t rows = a.B * a.T;
  const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t p = blockIdx.y;
  if (row >= rows) return;
  const int d = (int)a.d;
  const int64_t h = p / a.G, g = p % a.G;
  const int64_t b = row / a.T, t = row % a.T;
  const int64_t base = b * a.sb + h * a.sh + t * a.st + g * a.d;
  uint8_t* code_row = a.codes + b * a.cb + h * a.ch + t * a.ct + g * a.S;
  const int64_t D = a.G * a.d;
  const int64_t out_base = (b * a.H + h) * a.T * D + t * D + g * a.d;

  float r[DMAX];
#pragma unroll
  for (int i = 0; i < DMAX; ++i) r[i] = (i < d) ? Elem<DT>::load(a.states, base + i) : 0.f;
  if (a.whiteners != nullptr) {
    float x[DMAX];
#pragma unroll
    for (int i = 0; i < DMAX; ++i) x[i] = r[i];
    const float* w = a.whiteners + p * a.d * a.d;
#pragma unroll
    for (int i = 0; i < DMAX; ++i) {
      if (i < d) {
        float acc = 0.f;
        for (int e = 0; e < d; ++e) acc = fmaf(w[i * a.d + e], x[e], acc);
        r[i] = acc;
      }
    }
  }
  const float* sel = a.sel_tables;
  for (int64_t s = 0; s < a.S; ++s) {
    float rr = 0.f;
#pragma unroll
    for (int i = 0; i < DMAX; ++i)
      if (i < d) rr = fmaf(r[i], r[i], rr);
    const int64_t tab0 = (p * a.S + s) * a.K * a.d;
    float best = __builtin_inff();
    int bk = 0;
    for (int k = 0; k < (int)a.K; ++k) {
      const int64_t off = tab0 + (int64_t)k * a.d;
      float cc = 0.f, dot = 0.f;
#pragma unroll
      for (int i = 0; i < DMAX; ++i) {
        if (i < d) {
          float c = sel ? sel[off + i] : deploy16(a.tables[off + i]);
          cc = fmaf(c, c, cc);
          dot = fmaf(r[i], c, dot);
        }
      }
      float dist = (rr + cc) - 2.0f * dot;
      if (dist < best) {
        best = dist;
        bk = k;
      }
    }
    const int64_t off = tab0 + (int64_t)bk * a.d;
#pragma unroll
    for (int i = 0; i < DMAX; ++i)
      if (i < d) r[i] -= sel ? sel[off + i] : deploy16(a.tables[off + i]);
    code_row[s] = (uint8_t)bk;
    // Exits at depth s+1: decoded = sum_{j<=s} fp32(fp16(C[p,j,code_j])),
    // accumulated in stage order exactly like the reference's fp32 buffer.
    for (int e = 0; e < a.n_exits; ++e) {
      if (a.exit_depth[e] != s + 1 || a.recon[e] == nullptr) continue;
      float dec[DMAX];
#pragma unroll
      for (int i = 0; i < DMAX; ++i) dec[i] = 0.f;
      for (int64_t j = 0; j <= s; ++j) {
        const int64_t o = ((p * a.S + j) * a.K + code_row[j]) * a.d;
#pragma unroll
        for (int i = 0; i < DMAX; ++i)
          if (i < d) dec[i] += deploy16(a.tables[o + i]);
      }
#pragma unroll
      for (int i = 0; i < DMAX; ++i)
        if (i < d) Elem<DT>::store(a.recon[e], out_base + i, dec[i]);
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA kernel for d in {4, 8}, K = 256, S in {1, 2}, fp16 states.
//
// Workgroup = 4 waves on one (head, group) problem; the problem's S
// codebooks are staged once in LDS: plane lo[s][k] = c_k (d=4: [c_k, c_k])
// and plane hi[k] = [n_hi, n_lo, 16, 16] of stage 1 then of stage 2, with
// n = |c_k|^2/2 split into two fp16 halves.  A wave encodes 64 rows per
// iteration; lane L owns row L of the 64 for everything that is per row
// (bias, winner, outputs).
//
// Stage 1 runs on v_mfma_f32_32x32x16_f16 (two 32-row tiles, 32-codeword
// chunks), stage 2 on v_mfma_f32_16x16x32_f16 (four 16-row tiles, 16-codeword
// chunks); i = codeword in chunk, j = row in tile, slot group sg = k/8:
//   stage 1 (K = 16): sg0  x . c  (d=4: [x,0] . [c,c])   sg1  bias . hi
//   stage 2 (K = 32): d=8: sg0  x . c   sg1  (-c_1) . c   sg2  bias . hi
//                     d=4: sg0  [x,-c_1] . [c,c]          sg1  bias . hi
// where bias = (-1,-1,-b_hi,-b_lo, 0,0,0,0) in stage 1 and
// (0,0,0,0, -1,-1,-b_hi,-b_lo) in stage 2 picks that stage's half of hi.
// Other slot groups are zero.  A 32x32 product costs half as much per
// distance as a 16x16 one, but stage 2's 20 slots need K = 32.  Each row
// owner writes its row's B slots into a per-wave LDS image [slot group][row];
// a lane then reads its tile's operand as one 16-byte word.  hi carries
// (16, 16) against the row's -(beta/16) in two fp16 halves,
// beta = (|r|^2 + delta)/2, so with C = 0
//   D[i][j] = c_i.(x - c_prev) - |c_i|^2/2 - (|r|^2 + delta)/2
//           = -(|r - c_i|^2 + delta)/2  < 0,
// exact in the products (fp16 x fp16) and fp32 in the sum.  As unsigned bit
// patterns negative floats order by magnitude, so the row's nearest codeword
// is the min over keys (bits & ~255) | index: in-lane keys carry the index
// bits a lane's accumulator element fixes (stage 1: 32*chunk + 8*(i/8) + i%4,
// stage 2: 16*chunk + i%4) and the lane's bits of the index (4*(i/4)%2 resp.
// 4*(i/4)) are added before the cross-lane step (ties -> lowest index,
// torch.argmin's rule).
// delta = 2^-8 (|r|^2 + max|c|^2) keeps every key negative despite fp32
// rounding and the approximate |r|^2; it is common to all codewords of the
// row, so it never changes the order.  Stage 1 takes |r|^2 = |x|^2 from a
// dot product; stage 2 reads |x - c_1|^2 off stage 1's winning key
// (-2 D_min - delta_1, its magnitude rounded down by the cleared index
// bits, under 2^-15 relative) and widens delta_2 by 2^-10 delta_1 to cover
// that and the |x|^2-scaled rounding of D_min.

__device__ __forceinline__ uint32_t umin3(uint32_t a, uint32_t b, uint32_t c) {
  return min(min(a, b), c);
}

// Min over the four lane groups of tile lg's key: after the call lane
// (lg, j) holds the minimum of b[lg] over lanes {j, j+16, j+32, j+48}.
// Lane rows are 16 lanes; permlane32_swap exchanges rows {2,3} of its first
// operand with rows {0,1} of its second, permlane16_swap rows {1,3} of its
// first with rows {0,2} of its second.
__device__ __forceinline__ uint32_t tile_row_min(uint32_t b0, uint32_t b1, uint32_t b2,
                                                 uint32_t b3) {
  auto p02 = __builtin_amdgcn_permlane32_swap(b0, b2, false, false);
  const uint32_t t02 = min((uint32_t)p02[0], (uint32_t)p02[1]);  // rows 0-1: tile 0, 2-3: tile 2
  auto p13 = __builtin_amdgcn_permlane32_swap(b1, b3, false, false);
  const uint32_t t13 = min((uint32_t)p13[0], (uint32_t)p13[1]);  // rows 0-1: tile 1, 2-3: tile 3
  auto q = __builtin_amdgcn_permlane16_swap(t02, t13, false, false);
  return min((uint32_t)q[0], (uint32_t)q[1]);
}

__device__ __forceinline__ float dot2_acc(half8 a, half8 b) {
  float acc = 0.f;
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    half2v x = {a[e], a[e + 1]};
    half2v y = {b[e], b[e + 1]};
    acc = __builtin_amdgcn_fdot2(x, y, acc, false);
  }
  return acc;
}

// LDS writes of one wave become visible to the wave's other lanes
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

static const int kTiles = 4;                      // 16-row tiles per wave iteration
static const int kRowsPerWave = kTiles * 16;      // rows per wave iteration
static const int kRowsPerIter = 4 * kRowsPerWave; // rows per workgroup iteration


// PAIR: two jobs in the launch (a single-job launch keeps every argument at
// a fixed kernarg offset).  WH (d = 4, one stage): a selector whitener F per
// problem.  The search distance |F x - F c|^2 = x.Mx - 2 x.Mc + c.Mc with
// M = F^T F (cq_tac.py:81-95), so the codeword plane holds M c as two fp16
// words [Mc_hi | Mc_lo] against B slots [x | x] (x.Mc to 2^-22), the norm
// plane holds c.Mc / 2, the row bias x.Mx, and the raw codeword rides in the
// norm plane's upper half (its B slots are zero) for the reconstruction.
// At d = 8 the stage's [x | x | bias] takes 20 slots, so it runs on the
// 16x16x32 layout of the later stages: planes Mc_hi, Mc_lo and the raw
// codeword, M in LDS.
template <int D, int S, bool PAIR, bool WH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
void rvq_encode_mfma(MfmaArgs m) {
  const uint32_t L0 = xcd_remap(blockIdx.x, gridDim.x);
  const int jb = PAIR && (int64_t)L0 >= m.split ? 1 : 0;
  const MfmaJob& mj = m.job[jb];
  const EncodeArgs& a = mj.e;
  // slot groups with data (bias sits where the lanes read plane hi):
  // stage 1 [x, bias]; stage 2 d=8 [x, -c_1, bias], d=4 [[x,-c_1], bias]
  constexpr int kSgX = 0;
  constexpr int kSgC = (D == 8 && S > 1) ? 1 : 0;  // d=4: upper half of sg0
  // whitened d=8: stage 1 on K = 32 with slot groups [x, x, bias]
  constexpr bool kWh8 = WH && D == 8;
  static_assert(!WH || S == 1, "whitened search runs one stage");
  constexpr int kSgBias1 = kWh8 ? 2 : 1;            // stage 1 (K = 16)
  constexpr int kSgBias = (D == 8) ? 2 : 1;         // later stages (K = 32)
  constexpr int kSlotGroups = ((D == 8 && S > 1) || kWh8) ? 3 : 2;
  constexpr int kPlanes = kWh8 ? 3 : S;             // Mc_hi, Mc_lo, raw codeword
  __shared__ half8 tab_lo[kPlanes][256];
  __shared__ float s_M[kWh8 ? 64 : 1];
  __shared__ half8 tab_hi[256];
  // per-wave B images [slot group][tile][row] plus one shared zero plane
  __shared__ half8 bimg[4][kSlotGroups][kTiles][16];
  __shared__ half8 bzero[kTiles][16];
  __shared__ float s_ncmax[S][4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform, so row planning and addressing stay in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lg = lane >> 4;
  const int ln = lane & 15;

  // logical block: group fastest, then head, then row chunk
  const uint32_t L = jb ? L0 - (uint32_t)m.split : L0;
  const int64_t P = a.H * a.G;
  const bool active = (int64_t)L < P * mj.n_chunks;
  const int64_t g = active ? (int64_t)L % a.G : 0;
  const int64_t h = active ? ((int64_t)L / a.G) % a.H : 0;
  const int64_t chunk = active ? (int64_t)L / P : 0;
  const int64_t p = h * a.G + g;

  // WH: M = F^T F of this problem, in every lane (the row norm x.Mx uses it)
  float Mw[4][4];
  if constexpr (kWh8) {
    // M = F^T F, one entry per thread of the first wave
    if (tid < 64) {
      const float* F = a.whiteners + p * 64;
      const int i = tid >> 3, j = tid & 7;
      float acc = 0.f;
#pragma unroll
      for (int r = 0; r < 8; ++r) acc = fmaf(F[r * 8 + i], F[r * 8 + j], acc);
      s_M[tid] = acc;
    }
    __syncthreads();
  } else if constexpr (WH) {
    const float* F = a.whiteners + p * 16;
    float f[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) f[i] = F[i];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float acc = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) acc = fmaf(f[r * 4 + i], f[r * 4 + j], acc);
        Mw[i][j] = acc;
      }
  }
  // ---- stage the fp16-deployed codebooks (one codeword per thread) ----
  half8 hi = half8{};
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const float* src = a.tables + ((p * S + s) * 256 + tid) * D;
    half_t cw[D];
    if (D == 8) {
      const float4 v0 = ((const float4*)src)[0];
      const float4 v1 = ((const float4*)src)[1];
      const float f[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) cw[i] = (half_t)f[i];
    } else {
      const float4 v0 = ((const float4*)src)[0];
      const float f[4] = {v0.x, v0.y, v0.z, v0.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) cw[i] = (half_t)f[i];
    }
    float nc = 0.f;
    half8 lo;
    if constexpr (kWh8) {
      float mc[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = fmaf(s_M[i * 8 + j], (float)cw[j], acc);
        mc[i] = acc;
      }
      half8 mlo, raw;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        nc = fmaf((float)cw[i], mc[i], nc);
        const half_t mh = (half_t)mc[i];
        lo[i] = mh;
        mlo[i] = (half_t)(mc[i] - (float)mh);
        raw[i] = cw[i];
      }
      tab_lo[1][tid] = mlo;
      tab_lo[2][tid] = raw;
    } else if constexpr (WH) {
      float mc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = fmaf(Mw[i][j], (float)cw[j], acc);
        mc[i] = acc;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        nc = fmaf((float)cw[i], mc[i], nc);
        const half_t mh = (half_t)mc[i];
        lo[i] = mh;
        lo[4 + i] = (half_t)(mc[i] - (float)mh);
        hi[4 + i] = cw[i];  // the raw codeword (zero B slots)
      }
    } else {
#pragma unroll
      for (int i = 0; i < D; ++i) nc = fmaf((float)cw[i], (float)cw[i], nc);
#pragma unroll
      for (int e = 0; e < 8; ++e) lo[e] = cw[e % D];
    }
    const float halfn = 0.5f * nc;
    const half_t nhi = (half_t)halfn;
    const half_t nlo = (half_t)(halfn - (float)nhi);
    hi[4 * s + 0] = nhi;
    hi[4 * s + 1] = nlo;
    hi[4 * s + 2] = (half_t)16.f;  // bias slots: 16 * (beta/16)_hi + 16 * (beta/16)_lo
    hi[4 * s + 3] = (half_t)16.f;
    tab_lo[s][tid] = lo;
    float mx = nc;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if (lane == 0) s_ncmax[s][wave] = mx;
  }
  tab_hi[tid] = hi;
  // this lane's B rows start as zero
#pragma unroll
  for (int sg = 0; sg < kSlotGroups; ++sg) bimg[wave][sg][lg][ln] = half8{};
  bzero[tid >> 4 & 3][tid & 15] = half8{};
  __syncthreads();
  if (!active) return;
  float ncmax[S];
#pragma unroll
  for (int s = 0; s < S; ++s)
    ncmax[s] = fmaxf(fmaxf(s_ncmax[s][0], s_ncmax[s][1]), fmaxf(s_ncmax[s][2], s_ncmax[s][3]));

  // this lane's A plane: d=8 lanes 0-31 read c, 32-63 the norm plane;
  // d=4 lanes 0-15 read [c,c], 16-63 the norm plane (B is zero past slot 15)
  const bool a_hi = (D == 8) ? (lg >= 2) : (lg >= 1);
  const half8* plane_lo = &tab_lo[0][0];
  // this lane's B operand words: slot group lg of tile i, or zeros
  const half8* bsrc = (lg < kSlotGroups) ? &bimg[wave][lg][0][ln] : &bzero[0][ln];
  // the words this lane writes for its own row: slot group sg, tile lg, row ln
  half8* bdst = &bimg[wave][0][lg][ln];
  constexpr int kSgStride = kTiles * 16;  // half8 words between slot groups

  const int64_t rows = a.B * a.T;
  const int64_t r_begin = chunk * mj.rows_per_wg;
  int64_t r_end = r_begin + mj.rows_per_wg;
  if (r_end > rows) r_end = rows;
  const _Float16* states = (const _Float16*)a.states;
  const int64_t Dfull = a.G * D;
  const int64_t head_x = h * a.sh + g * D;             // states offset of (h, g)
  const int64_t head_c = h * a.ch + g * S;             // codes offset of (h, g)
  const int64_t out_bstride = a.H * a.T * Dfull;       // recon is contiguous
  const int64_t head_o = h * a.T * Dfull + g * D;

  int64_t base = r_begin + wave * kRowsPerWave;  // the wave's first row

  // Wave-uniform description of one iteration (64 rows starting at row
  // `at`).  In the common case all rows sit in one batch entry and every
  // address is a uniform base plus (row in iteration) * stride; otherwise
  // rows are located one by one.  Rows fit in 32 bits (host-checked).
  struct Iter {
    int64_t at, xb, cb, ob;
    bool fast;
  };
  const uint32_t T32 = (uint32_t)a.T;
  auto plan = [&](int64_t at) {
    Iter it;
    it.at = at;
    const uint32_t b0 = (uint32_t)at / T32;
    const uint32_t t0 = (uint32_t)at - b0 * T32;
    it.fast = t0 + kRowsPerWave <= T32 && at + kRowsPerWave <= r_end;
    it.xb = (int64_t)b0 * a.sb + head_x + (int64_t)t0 * a.st;
    it.cb = (int64_t)b0 * a.cb + head_c + (int64_t)t0 * a.ct;
    it.ob = (int64_t)b0 * out_bstride + head_o + (int64_t)t0 * Dfull;
    return it;
  };
  // offsets of this lane's row (valid, states, codes, reconstruction).  The
  // row strides are below 2^24 (host-checked), so the full-rate 24-bit
  // multiply replaces the quarter-rate 32-bit one.
  auto locate = [&](const Iter& it, uint32_t* xo, uint32_t* co, uint32_t* oo) -> bool {
    const uint32_t rr = (uint32_t)lane;
    if (it.fast) {
      *xo = (uint32_t)it.xb + __umul24(rr, (uint32_t)a.st);
      *co = (uint32_t)it.cb + __umul24(rr, (uint32_t)a.ct);
      *oo = (uint32_t)it.ob + __umul24(rr, (uint32_t)Dfull);
      return true;
    }
    // rows, strides and offsets fit in 32 bits on this path (host-checked)
    const uint32_t row = (uint32_t)it.at + rr;
    const bool valid = row < (uint32_t)r_end;
    const uint32_t rw = valid ? row : (uint32_t)r_begin;
    const uint32_t rb = rw / T32, rt = rw - rb * T32;
    *xo = rb * (uint32_t)a.sb + (uint32_t)head_x + rt * (uint32_t)a.st;
    *co = rb * (uint32_t)a.cb + (uint32_t)head_c + rt * (uint32_t)a.ct;
    *oo = rb * (uint32_t)out_bstride + (uint32_t)head_o + rt * (uint32_t)Dfull;
    return valid;
  };
  auto load_x = [&](const Iter& it) -> half8 {
    uint32_t xo, co, oo;
    locate(it, &xo, &co, &oo);
    if (D == 8) return *(const half8*)(states + xo);
    const half4 v = *(const half4*)(states + xo);
    if constexpr (WH) return half8{v[0], v[1], v[2], v[3], v[0], v[1], v[2], v[3]};  // [x | x]
    return half8{v[0], v[1], v[2], v[3], (half_t)0.f, (half_t)0.f, (half_t)0.f, (half_t)0.f};
  };
  // stage s's bias slots (-1, -1, -(beta/16) in two fp16 halves) in half s
  // of the word, zeros in the other half
  auto bias_slots = [&](int s, float rr, float delta) -> half8 {
    const float beta16 = (rr + delta) * (0.5f / 16.f) + 0x1p-60f;
    const half_t bh = (half_t)beta16;
    const half_t bl = (half_t)(beta16 - (float)bh);
    half8 w = half8{};
    w[4 * s + 0] = (half_t)-1.f;
    w[4 * s + 1] = (half_t)-1.f;
    w[4 * s + 2] = -bh;
    w[4 * s + 3] = -bl;
    return w;
  };

  const uint32_t lg4 = (uint32_t)lg << 2;
  // the key mask lives in a VGPR so that each key is one v_and_or_b32 with
  // its index tag (not an inline constant) in a scalar register
  uint32_t kmask = ~255u;
  asm volatile("" : "+v"(kmask));

  // Stage 1 on v_mfma_f32_32x32x16_f16: its 12 slots [x | bias] fit K = 16,
  // and a 32x32 product costs half as much per distance as a 16x16 one.
  //   A[i][k]: lane i + 32*(k/8)   B[k][j]: lane j + 32*(k/8)
  //   D[i][j]: lane j + 32*((i/4)%2), element 4*(i/8) + i%4
  // Two 32-row tiles per wave, eight 32-codeword chunks; lane (h, j) reads
  // slot group h of row 32t + j and, as A, codeword i = j of plane lo or hi.
  const int h32 = lane >> 5, j32 = lane & 31;
  const uint32_t h4 = (uint32_t)h32 << 2;
  const half8* b32src = &bimg[wave][h32][0][0] + j32;
  const half8* a32src = (h32 ? &tab_hi[0] : plane_lo) + j32;
  auto stage_first = [&]() -> uint32_t {
    half8 bop[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) bop[t] = b32src[32 * t];
    const float16v zero16 = {};
    uint32_t best[2] = {0xFFFFFFFFu, 0xFFFFFFFFu};
    half8 af_next = a32src[0];
    float16v acc[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
      acc[0][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af_next, bop[t], zero16, 0, 0, 0);
    af_next = a32src[32];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int cur_b = c & 1;
      const half8 af = af_next;
      if (c + 2 < 8) af_next = a32src[(c + 2) * 32];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (c + 1 < 8)
          acc[cur_b ^ 1][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bop[t], zero16, 0, 0, 0);
        const float16v v = acc[cur_b][t];
        uint32_t k[16];
#pragma unroll
        for (int el = 0; el < 16; ++el)
          k[el] = (__float_as_uint(v[el]) & kmask) | (uint32_t)(32 * c + 8 * (el >> 2) + (el & 3));
        uint32_t m = best[t];
#pragma unroll
        for (int el = 0; el < 16; el += 2) m = umin3(k[el], k[el + 1], m);
        best[t] = m;
        asm volatile("" : "+v"(best[t]));
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (c + 1 < 8) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 24, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // this lane's row L: tile L/32, the minimum over both lane halves
    auto p = __builtin_amdgcn_permlane32_swap(best[0] | h4, best[1] | h4, false, false);
    return min((uint32_t)p[0], (uint32_t)p[1]);
  };

  // Later stages on v_mfma_f32_16x16x32_f16 (20 slots): four 16-row tiles,
  // sixteen 16-codeword chunks.
  auto stage_next = [&](const half8* pl) -> uint32_t {
    half8 bop[kTiles];
#pragma unroll
    for (int i = 0; i < kTiles; ++i) bop[i] = bsrc[i * 16];

    const float4v zero4 = {0.f, 0.f, 0.f, 0.f};
    uint32_t best[kTiles];
#pragma unroll
    for (int i = 0; i < kTiles; ++i) best[i] = 0xFFFFFFFFu;
    // software pipeline: the MFMAs of chunk c+1 run while the keys of
    // chunk c are reduced
    half8 af_next = pl[0];
    float4v acc[2][kTiles];
#pragma unroll
    for (int i = 0; i < kTiles; ++i)
      acc[0][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af_next, bop[i], zero4, 0, 0, 0);
    af_next = pl[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const int cur_b = c & 1;
      const half8 af = af_next;
      if (c + 2 < 16) af_next = pl[(c + 2) * 16];
#pragma unroll
      for (int i = 0; i < kTiles; ++i) {
        if (c + 1 < 16)
          acc[cur_b ^ 1][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bop[i], zero4, 0, 0, 0);
        const float4v v = acc[cur_b][i];
        const uint32_t k0 = (__float_as_uint(v[0]) & kmask) | (uint32_t)(c * 16 + 0);
        const uint32_t k1 = (__float_as_uint(v[1]) & kmask) | (uint32_t)(c * 16 + 1);
        const uint32_t k2 = (__float_as_uint(v[2]) & kmask) | (uint32_t)(c * 16 + 2);
        const uint32_t k3 = (__float_as_uint(v[3]) & kmask) | (uint32_t)(c * 16 + 3);
        best[i] = umin3(umin3(k0, k1, k2), k3, best[i]);
        // pin the running minimum here: without it the compiler sinks the
        // key reduction of later tiles past the stage epilogue and keeps
        // every MFMA result of the stage live
        asm volatile("" : "+v"(best[i]));
      }
      // issue order per chunk: one MFMA of chunk c+1, then the six key
      // operations of one tile of chunk c, four times
#pragma unroll
      for (int i = 0; i < kTiles; ++i) {
        if (c + 1 < 16) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // this lane's row: the winner over all four lane groups
    return tile_row_min(best[0] | lg4, best[1] | lg4, best[2] | lg4, best[3] | lg4);
  };
  half8 x = half8{};
  Iter cur = plan(base);
  if (base < r_end) x = load_x(cur);

  for (; base < r_end; base += kRowsPerIter) {
    const bool more = base + kRowsPerIter < r_end;
    const Iter nxt = plan(base + kRowsPerIter);
    uint32_t xo, co, oo;
    const bool valid = locate(cur, &xo, &co, &oo);

    // stage-1 B rows of this lane's row: x, no previous codeword, bias
    float rr1;
    if constexpr (kWh8) {
      rr1 = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float mx = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) mx = fmaf(s_M[i * 8 + j], (float)x[j], mx);
        rr1 = fmaf((float)x[i], mx, rr1);
      }
    } else if constexpr (WH) {
      // |F x|^2 = x.Mx
      rr1 = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float mx = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) mx = fmaf(Mw[i][j], (float)x[j], mx);
        rr1 = fmaf((float)x[i], mx, rr1);
      }
    } else {
      rr1 = dot2_acc(x, x);
    }
    const float delta1 = (rr1 + ncmax[0]) * 0x1p-8f;
    bdst[kSgX * kSgStride] = x;  // d=4: [x, 0]
    if constexpr (kWh8) bdst[1 * kSgStride] = x;
    bdst[kSgBias1 * kSgStride] = bias_slots(0, rr1, delta1);
    // x is consumed: the next iteration's row loads during this one
    if (more) x = load_x(nxt);

    uint32_t code = 0u;
    half8 negc1 = half8{};  // -c_1 of this lane's row
#pragma unroll
    for (int s = 0; s < S; ++s) {
      wave_lds_sync();
      uint32_t kmin;
      if (s == 0 && !kWh8) {
        kmin = stage_first();
      } else {
        // lane group lg reads plane lg (whitened d=8) or the stage's plane
        kmin = stage_next((a_hi ? &tab_hi[0] : plane_lo + (kWh8 ? lg : s) * 256) + ln);
      }
      const uint32_t kstar = kmin & 255u;
      code |= kstar << (8 * s);
      half8 cw = tab_lo[s][kstar];
      if constexpr (kWh8) {
        cw = tab_lo[2][kstar];
      } else if constexpr (WH) {
        const half8 t = tab_hi[kstar];
        cw = half8{t[4], t[5], t[6], t[7], t[4], t[5], t[6], t[7]};
      }
      if (s + 1 < S) {
        // stage-2 B rows: -c_1 and the bias from |x - c_1|^2
        negc1 = -cw;
        const float rr2 = fmaxf(-2.f * __uint_as_float(kmin & ~255u) - delta1, 0.f);
        const float delta2 = (rr2 + ncmax[s + 1]) * 0x1p-8f + delta1 * 0x1p-10f;
        if (D == 8) {
          bdst[kSgC * kSgStride] = negc1;
        } else {
          ((half4*)&bdst[kSgX * kSgStride])[1] = half4{negc1[0], negc1[1], negc1[2], negc1[3]};
        }
        bdst[kSgBias * kSgStride] = bias_slots(s + 1, rr2, delta2);
      }
      // depth-(s+1) reconstruction fp16(fp32(c1) + fp32(c2)): the sum of two
      // fp16 words is exact in fp32 or, when it is not, too small to move the
      // fp16 rounding, so one fp16 add gives the same bits.
      void* out = mj.recon_depth[s];
      if (out != nullptr && valid) {
        const half8 dec = (s > 0) ? sub_h8(cw, negc1) : cw;
        _Float16* op = (_Float16*)out + oo;
        if (D == 8) {
          *(half8*)op = dec;
        } else {
          *(half4*)op = half4{dec[0], dec[1], dec[2], dec[3]};
        }
      }
    }
    if (valid) {
      uint8_t* cp = a.codes + co;
      if (S == 1) {
        cp[0] = (uint8_t)code;
      } else {
        *(uint16_t*)cp = (uint16_t)code;
      }
    }
    cur = nxt;
  }
}
// ---------------------------------------------------------------------------
template <int DT>
static int launch_generic(const EncodeArgs& a, hipStream_t stream) {
  const int64_t rows = a.B * a.T;
  dim3 grid((uint32_t)ceil_div(rows, 256), (uint32_t)(a.H * a.G));
  if (a.d <= 8) {
    hipLaunchKernelGGL((rvq_encode_generic<DT, 8>), grid, dim3(256), 0, stream, a);
  } else if (a.d <= 32) {
    hipLaunchKernelGGL((rvq_encode_generic<DT, 32>), grid, dim3(256), 0, stream, a);
  } else {
    hipLaunchKernelGGL((rvq_encode_generic<DT, 128>), grid, dim3(256), 0, stream, a);
  }
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

static MfmaJob mfma_job(const EncodeArgs& e) {
  MfmaJob j = {};
  j.e = e;
  for (int i = 0; i < e.n_exits; ++i) j.recon_depth[e.exit_depth[i] - 1] = e.recon[i];
  const int64_t rows = e.B * e.T;
  const int64_t P = e.H * e.G;
  // rows per workgroup: amortise the codebook staging, fill 256 CUs x 4 WGs
  int64_t rpw = 4096;
  while (rpw > kRowsPerIter && P * ceil_div(rows, rpw) < 256 * 4) rpw >>= 1;
  j.rows_per_wg = rpw;
  j.n_chunks = ceil_div(rows, rpw);
  return j;
}

// one job, or two of the same geometry (second non-null) in one launch
template <int D, int S>
static int launch_mfma(const EncodeArgs& e, const EncodeArgs* e2, hipStream_t stream) {
  MfmaArgs m = {};
  m.job[0] = mfma_job(e);
  const int64_t per_job = e.H * e.G * m.job[0].n_chunks;
  int64_t nblocks = per_job;
  m.split = per_job;
  if (e2 != nullptr) {
    m.job[1] = mfma_job(*e2);
    nblocks += per_job;
  } else {
    m.job[1] = m.job[0];
  }
  if (nblocks > 8) nblocks = ceil_div(nblocks, 8) * 8;  // xcd_remap needs a multiple of 8
  JKV_CHECK_ARG(nblocks < (int64_t)1 << 31, "grid too large");
  if (e2 == nullptr) {
    m.split = nblocks;
    if constexpr (S == 1) {
      if (e.whiteners != nullptr) {
        hipLaunchKernelGGL((rvq_encode_mfma<D, 1, false, true>), dim3((uint32_t)nblocks), dim3(256), 0, stream, m);
        JKV_CHECK_LAUNCH();
        return JKV_OK;
      }
    }
    hipLaunchKernelGGL((rvq_encode_mfma<D, S, false, false>), dim3((uint32_t)nblocks), dim3(256), 0, stream, m);
  } else {
    hipLaunchKernelGGL((rvq_encode_mfma<D, S, true, false>), dim3((uint32_t)nblocks), dim3(256), 0, stream, m);
  }
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

template <int D, int S>
static int launch_mfma(const EncodeArgs& e, hipStream_t stream) {
  return launch_mfma<D, S>(e, nullptr, stream);
}

// Whether rvq_encode_mfma takes these arguments: fp16 states, d in {4, 8},
// K = 256, S <= 2, no whitener, 16-byte aligned states and reconstructions,
// and offsets that fit the kernel's 32-bit (24-bit for token strides)
// arithmetic.
static bool mfma_eligible(const EncodeArgs& a, int32_t states_dtype) {
  const int64_t B = a.B, H = a.H, T = a.T, G = a.G, d = a.d, S = a.S;
  const bool aligned16 = (((uintptr_t)a.states) % 16 == 0) && a.sb % 8 == 0 && a.sh % 8 == 0 && a.st % 8 == 0;
  const bool codes_aligned =
      (S == 1) || ((((uintptr_t)a.codes) % 2 == 0) && a.cb % 2 == 0 && a.ch % 2 == 0 && a.ct % 2 == 0);
  bool recon_aligned = true, distinct_exits = true;
  for (int e = 0; e < a.n_exits; ++e) {
    if (a.recon[e] && ((uintptr_t)a.recon[e]) % 16 != 0) recon_aligned = false;
    for (int f = 0; f < e; ++f)
      if (a.exit_depth[e] == a.exit_depth[f]) distinct_exits = false;
  }
  const int64_t x_span = (B - 1) * a.sb + (H - 1) * a.sh + (T - 1) * a.st + G * d;
  const int64_t c_span = (B - 1) * a.cb + (H - 1) * a.ch + (T - 1) * a.ct + G * S;
  const bool offsets32 = a.sb >= 0 && a.sh >= 0 && a.st >= 0 && a.cb >= 0 && a.ch >= 0 && a.ct >= 0 &&
                         x_span < ((int64_t)1 << 31) && c_span < ((int64_t)1 << 31) &&
                         B * H * T * G * d < ((int64_t)1 << 31) && a.st < ((int64_t)1 << 24) &&
                         a.ct < ((int64_t)1 << 24) && G * d < ((int64_t)1 << 24);
  return offsets32 && states_dtype == JKV_F16 && a.whiteners == nullptr && a.K == 256 &&
         (d == 8 || d == 4) && (S == 1 || S == 2) && aligned16 && codes_aligned && recon_aligned &&
         distinct_exits && B * T < ((int64_t)1 << 31) && T < ((int64_t)1 << 31);
}

}  // namespace jkv

extern "C" {

int64_t jkv_rvq_encode_workspace_bytes(int64_t H, int64_t G, int64_t S, int64_t K,
                                       int64_t d, int32_t has_whitener) {
  const bool full = d == 128 && K == 256 && S >= 1 && S <= 32;
  if (has_whitener) return full ? jkv::full_wh_workspace_bytes(H * G, S) : H * G * S * K * d * (int64_t)sizeof(float);
  if (full) return jkv::full_workspace_bytes(H * G, S);
  return 0;
}

int64_t jkv_rvq_encode_many_workspace_bytes(int32_t n_jobs, int64_t H, int64_t G, int64_t S, int64_t K,
                                            int64_t d) {
  const bool full = d == 128 && K == 256 && S >= 1 && S <= 32;
  if (full && n_jobs > 1) return std::min<int64_t>(n_jobs, jkv::kMaxManyJobs) * jkv::full_workspace_bytes(H * G, S);
  return jkv_rvq_encode_workspace_bytes(H, G, S, K, d, 0);
}

int jkv_rvq_encode(const void* states, int32_t states_dtype, int64_t B, int64_t H,
                   int64_t T, int64_t G, int64_t d, int64_t stride_b, int64_t stride_h,
                   int64_t stride_t, const float* tables, int64_t S, int64_t K,
                   const float* whiteners, uint8_t* codes, int64_t code_stride_b,
                   int64_t code_stride_h, int64_t code_stride_t, int32_t n_exits,
                   const int32_t* exit_depths, void* const* recon, void* workspace,
                   int64_t workspace_bytes, jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(B >= 0 && H > 0 && T >= 0 && G > 0 && d > 0, "invalid states geometry");
  JKV_CHECK_ARG(S > 0 && K > 0, "invalid table geometry");
  JKV_CHECK_ARG(K <= 256, "codes are uint8: at most 256 codewords per stage (got %lld)",
                (long long)K);
  JKV_CHECK_ARG(d <= 128, "group dimension above 128 is not supported (got %lld)",
                (long long)d);
  JKV_CHECK_ARG(states_dtype == JKV_F16 || states_dtype == JKV_BF16 || states_dtype == JKV_F32,
                "unknown states dtype %d", states_dtype);
  JKV_CHECK_ARG(n_exits >= 0 && n_exits <= JKV_MAX_EXITS, "at most %d exits", JKV_MAX_EXITS);
  if (B * T == 0) return JKV_OK;
  JKV_CHECK_ARG(states && tables && codes, "null buffer");

  EncodeArgs a = {};
  a.states = states;
  a.sb = stride_b; a.sh = stride_h; a.st = stride_t;
  a.B = B; a.H = H; a.T = T; a.G = G; a.d = d; a.S = S; a.K = K;
  a.tables = tables;
  a.whiteners = whiteners;
  a.codes = codes;
  a.cb = code_stride_b; a.ch = code_stride_h; a.ct = code_stride_t;
  a.n_exits = n_exits;
  for (int e = 0; e < n_exits; ++e) {
    JKV_CHECK_ARG(exit_depths[e] >= 1 && exit_depths[e] <= S, "exit depth outside the ladder");
    a.exit_depth[e] = exit_depths[e];
    a.recon[e] = recon ? recon[e] : nullptr;
  }

  const bool aligned16 = (((uintptr_t)states) % 16 == 0) && stride_b % 8 == 0 &&
                         stride_h % 8 == 0 && stride_t % 8 == 0;
  bool recon_aligned = true;
  for (int e = 0; e < n_exits; ++e)
    if (a.recon[e] && ((uintptr_t)a.recon[e]) % 16 != 0) recon_aligned = false;
  bool distinct_exits = true;
  for (int i = 0; i < n_exits; ++i)
    for (int j = 0; j < i; ++j)
      if (exit_depths[i] == exit_depths[j]) distinct_exits = false;
  const bool fast = mfma_eligible(a, states_dtype);
  // whitened grouped CQ at d = 4 (one stage): the same kernel with M = F^T F
  EncodeArgs plain = a;
  plain.whiteners = nullptr;
  if (whiteners != nullptr && (d == 4 || d == 8) && S == 1 && ((uintptr_t)whiteners) % 4 == 0 &&
      mfma_eligible(plain, states_dtype))
    return d == 4 ? launch_mfma<4, 1>(a, stream) : launch_mfma<8, 1>(a, stream);
  if (fast) return launch_grouped(a, nullptr, stream);
  // full-vector codebooks on MFMA (fp16-deployed tables in the workspace),
  // plain or whitened
  const bool full = states_dtype == JKV_F16 && d == 128 && K == 256 && S <= 32 && aligned16 &&
                    recon_aligned && distinct_exits && workspace != nullptr &&
                    ((uintptr_t)workspace) % 16 == 0 &&
                    (whiteners == nullptr
                         ? workspace_bytes >= full_workspace_bytes(H * G, S)
                         : workspace_bytes >= full_wh_workspace_bytes(H * G, S) && ((uintptr_t)whiteners) % 16 == 0);
  if (full) return launch_full(a, workspace, stream);
  if (whiteners != nullptr) {
    int64_t need = jkv_rvq_encode_workspace_bytes(H, G, S, K, d, 1);
    JKV_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                  "whitened encode needs %lld bytes of workspace", (long long)need);
    float* sel = (float*)workspace;
    int64_t n = H * G * S * K * d;
    if (d == 128 && K == 256 && ((uintptr_t)tables) % 16 == 0 && ((uintptr_t)whiteners) % 16 == 0 &&
        ((uintptr_t)sel) % 16 == 0) {
      hipLaunchKernelGGL(selector_tables128_kernel, dim3((uint32_t)(H * G * S * 4)), dim3(256),
                         (128 * 128 + 128 * 64) * sizeof(float), stream, tables, whiteners, sel, S);
    } else {
      hipLaunchKernelGGL(selector_tables_kernel, dim3((uint32_t)ceil_div(n, 256)), dim3(256), 0,
                         stream, tables, whiteners, sel, H * G, S, K, d);
    }
    JKV_CHECK_LAUNCH();
    a.sel_tables = sel;
  }


  switch (states_dtype) {
    case JKV_F16: return launch_generic<JKV_F16>(a, stream);
    case JKV_BF16: return launch_generic<JKV_BF16>(a, stream);
    default: return launch_generic<JKV_F32>(a, stream);
  }
}

int jkv_rvq_encode_kv(const void* key_states, const void* value_states, int32_t states_dtype, int64_t B,
                      int64_t H, int64_t T, int64_t G, int64_t d, int64_t stride_b, int64_t stride_h,
                      int64_t stride_t, const float* key_tables, const float* value_tables, int64_t S,
                      int64_t K, uint8_t* key_codes, uint8_t* value_codes, int64_t code_stride_b,
                      int64_t code_stride_h, int64_t code_stride_t, int32_t n_exits,
                      const int32_t* exit_depths, void* const* key_recon, void* const* value_recon,
                      void* workspace, int64_t workspace_bytes, jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(B >= 0 && H > 0 && T >= 0 && G > 0 && d > 0 && S > 0 && K > 0, "invalid geometry");
  JKV_CHECK_ARG(n_exits >= 0 && n_exits <= JKV_MAX_EXITS, "at most %d exits", JKV_MAX_EXITS);
  if (B * T == 0) return JKV_OK;
  JKV_CHECK_ARG(key_states && value_states && key_tables && value_tables && key_codes && value_codes,
                "null buffer");
  EncodeArgs ak = {};
  ak.states = key_states;
  ak.sb = stride_b; ak.sh = stride_h; ak.st = stride_t;
  ak.B = B; ak.H = H; ak.T = T; ak.G = G; ak.d = d; ak.S = S; ak.K = K;
  ak.tables = key_tables;
  ak.codes = key_codes;
  ak.cb = code_stride_b; ak.ch = code_stride_h; ak.ct = code_stride_t;
  ak.n_exits = n_exits;
  for (int e = 0; e < n_exits; ++e) {
    JKV_CHECK_ARG(exit_depths[e] >= 1 && exit_depths[e] <= S, "exit depth outside the ladder");
    ak.exit_depth[e] = exit_depths[e];
    ak.recon[e] = key_recon ? key_recon[e] : nullptr;
  }
  EncodeArgs av = ak;
  av.states = value_states;
  av.tables = value_tables;
  av.codes = value_codes;
  for (int e = 0; e < n_exits; ++e) av.recon[e] = value_recon ? value_recon[e] : nullptr;
  if (mfma_eligible(ak, states_dtype) && mfma_eligible(av, states_dtype)) return launch_grouped(ak, &av, stream);
  // other geometries: the two encodes one after the other on the stream
  // (they may share the workspace: the second starts after the first)
  const int rc = jkv_rvq_encode(key_states, states_dtype, B, H, T, G, d, stride_b, stride_h, stride_t,
                                key_tables, S, K, nullptr, key_codes, code_stride_b, code_stride_h,
                                code_stride_t, n_exits, exit_depths, key_recon, workspace, workspace_bytes,
                                stream_);
  if (rc != JKV_OK) return rc;
  return jkv_rvq_encode(value_states, states_dtype, B, H, T, G, d, stride_b, stride_h, stride_t,
                        value_tables, S, K, nullptr, value_codes, code_stride_b, code_stride_h, code_stride_t,
                        n_exits, exit_depths, value_recon, workspace, workspace_bytes, stream_);
}

int jkv_rvq_encode_many(int32_t n_jobs, const void* const* states, int32_t states_dtype, int64_t B,
                        int64_t H, int64_t T, int64_t G, int64_t d, int64_t stride_b, int64_t stride_h,
                        int64_t stride_t, const float* const* tables, int64_t S, int64_t K,
                        uint8_t* const* codes, int64_t code_stride_b, int64_t code_stride_h,
                        int64_t code_stride_t, int32_t n_exits, const int32_t* exit_depths,
                        void* const* recon, void* workspace, int64_t workspace_bytes,
                        jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(n_jobs >= 0, "negative job count");
  JKV_CHECK_ARG(B >= 0 && H > 0 && T >= 0 && G > 0 && d > 0 && S > 0 && K > 0, "invalid geometry");
  JKV_CHECK_ARG(n_exits >= 0 && n_exits <= JKV_MAX_EXITS, "at most %d exits", JKV_MAX_EXITS);
  if (n_jobs == 0 || B * T == 0) return JKV_OK;
  JKV_CHECK_ARG(states && tables && codes, "null job array");
  EncodeArgs batch[kMaxManyJobs];
  for (int32_t j0 = 0; j0 < n_jobs; j0 += kMaxManyJobs) {
    const int n = (int)std::min<int64_t>(kMaxManyJobs, n_jobs - j0);
    bool grouped = true;
    for (int i = 0; i < n; ++i) {
      const int32_t j = j0 + i;
      JKV_CHECK_ARG(states[j] && tables[j] && codes[j], "null buffer in job %d", j);
      EncodeArgs& a = batch[i];
      a = EncodeArgs{};
      a.states = states[j];
      a.sb = stride_b; a.sh = stride_h; a.st = stride_t;
      a.B = B; a.H = H; a.T = T; a.G = G; a.d = d; a.S = S; a.K = K;
      a.tables = tables[j];
      a.codes = codes[j];
      a.cb = code_stride_b; a.ch = code_stride_h; a.ct = code_stride_t;
      a.n_exits = n_exits;
      for (int e = 0; e < n_exits; ++e) {
        JKV_CHECK_ARG(exit_depths[e] >= 1 && exit_depths[e] <= S, "exit depth outside the ladder");
        a.exit_depth[e] = exit_depths[e];
        a.recon[e] = recon ? recon[(int64_t)j * n_exits + e] : nullptr;
      }
      if (!mfma_eligible(a, states_dtype)) grouped = false;
    }
    if (grouped) {
      const int rc = launch_grouped_many(batch, n, stream);
      if (rc != JKV_OK) return rc;
      continue;
    }
    // full-vector codebooks with a workspace region per job: every job's
    // tables in one launch, every job's search in another
    bool full = n > 1 && states_dtype == JKV_F16 && d == 128 && K == 256 && S <= 32 && n_exits <= 2 &&
                workspace != nullptr && ((uintptr_t)workspace) % 16 == 0 &&
                workspace_bytes >= n * full_workspace_bytes(H * G, S) && stride_b % 8 == 0 && stride_h % 8 == 0 &&
                stride_t % 8 == 0 && !(n_exits == 2 && exit_depths[0] == exit_depths[1]);
    for (int i = 0; i < n && full; ++i) {
      if (((uintptr_t)batch[i].states) % 16 != 0) full = false;
      for (int e = 0; e < n_exits; ++e)
        if (batch[i].recon[e] && ((uintptr_t)batch[i].recon[e]) % 16 != 0) full = false;
    }
    if (full) {
      const int rc = launch_full_many(batch, n, workspace, stream);
      if (rc != JKV_OK) return rc;
      continue;
    }
    // other geometries: the encodes one after the other on the stream
    // (they may share the workspace: each starts after the one before)
    for (int i = 0; i < n; ++i) {
      const int32_t j = j0 + i;
      const int rc = jkv_rvq_encode(states[j], states_dtype, B, H, T, G, d, stride_b, stride_h, stride_t,
                                    tables[j], S, K, nullptr, codes[j], code_stride_b, code_stride_h,
                                    code_stride_t, n_exits, exit_depths,
                                    recon ? recon + (int64_t)j * n_exits : nullptr, workspace,
                                    workspace_bytes, stream_);
      if (rc != JKV_OK) return rc;
    }
  }
  return JKV_OK;
}

}  // extern "C"
