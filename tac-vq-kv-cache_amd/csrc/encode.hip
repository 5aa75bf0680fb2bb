// Hard greedy residual-VQ / grouped-CQ encode for gfx950.
//
// Two kernels share one argument block:
//  * rvq_encode_mfma<D,S>: fp16 states, d in {4,8}, K=256, S<=2, no whitener.
//    A workgroup owns one (head, group) problem and a chunk of rows; the
//    problem's codebooks are staged in LDS and feed the A operand of
//    v_mfma_f32_16x16x32_f16 (codewords x contraction slots); 16-row tiles
//    are the B operand.  The contraction packs [x | -c_prev | norm] so one
//    MFMA yields -(|r - c|^2 + delta)/2 for 16 codewords x 16 rows with exact
//    products and fp32 accumulation; the argmin is a min over keys that
//    carry the codeword index in their low bits.
//  * rvq_encode_generic<DT,DMAX>: any dtype, d<=128, K<=256, any S, optional
//    whitener; one thread per row, fp32 distances in the reference's
//    |r|^2 + |c|^2 - 2 r.c form.
#include "jkv_common.h"

namespace jkv {

struct EncodeArgs {
  const void* states;
  int64_t sb, sh, st;  // element strides of the B, H, T axes
  int64_t B, H, T, G, d, S, K;
  const float* tables;      // fp32 masters [P,S,K,d]
  const float* sel_tables;  // whitened selector tables [P,S,K,d] or null
  const float* whiteners;   // [P,d,d] or null
  uint8_t* codes;
  int64_t cb, ch, ct;  // byte strides of the B, H, T axes
  int32_t n_exits;
  int32_t exit_depth[JKV_MAX_EXITS];
  void* recon[JKV_MAX_EXITS];
};

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
// codebooks are staged once in LDS as two planes, c (fp16) and
// [n_hi, n_lo] with n = |c|^2/2 split into two fp16 halves.  Each wave
// encodes 4 tiles of 16 rows per iteration (independent MFMA chains).
//
// v_mfma_f32_16x16x32_f16 (wave64), i = codeword in chunk, j = row in tile:
//   A[i][k]: lane = i + 16*(k/8), element k%8
//   B[k][j]: lane = j + 16*(k/8), element k%8
//   D[i][j]: lane = j + 16*(i/4), element i%4
// Contraction slots (lane group lg = lane/16 owns slots 8lg..8lg+7):
//   d=8: lg0  x . c   lg1  (-c_prev) . c   lg2  (-1,-1,-b_hi,-b_lo) . (n_hi,n_lo,16,16)
//   d=4: lg0  [x,-c_prev] . [c,c]          lg1  (-1,-1,-b_hi,-b_lo) . (n_hi,n_lo,16,16)
// Remaining lane groups carry B = 0 (their A entries are finite LDS data).
// The norm plane also carries (16, 16) against the row's -(beta/16) in two
// fp16 halves, beta = (|r|^2 + delta)/2, so with C = 0
//   D[i][j] = c_i.(x - c_prev) - |c_i|^2/2 - (|r|^2 + delta)/2
//           = -(|r - c_i|^2 + delta)/2  < 0,
// exact in the products (fp16 x fp16) and fp32 in the sum.  As unsigned bit
// patterns negative floats order by magnitude, so the row's nearest codeword
// is the min over keys (bits & ~63) | (chunk<<2 | i%4); the lane group adds
// the last two index bits in the cross-lane step (ties -> lowest index).
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

__device__ __forceinline__ uint32_t lane_group_min(uint32_t v) {
  // min over lanes {j, j+16, j+32, j+48}
  auto s16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  uint32_t m = min((uint32_t)s16[0], (uint32_t)s16[1]);
  auto s32 = __builtin_amdgcn_permlane32_swap(m, m, false, false);
  return min((uint32_t)s32[0], (uint32_t)s32[1]);
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

static const int kTiles = 4;                      // 16-row tiles per wave iteration
static const int kRowsPerWave = kTiles * 16;      // rows per wave iteration
static const int kRowsPerIter = 4 * kRowsPerWave; // rows per workgroup iteration

struct MfmaArgs {
  EncodeArgs e;
  void* recon_depth[2];  // reconstruction at depth 1 / 2 (or null)
  int64_t rows_per_wg;
  int64_t n_chunks;      // row chunks per problem
};

template <int D, int S>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
void rvq_encode_mfma(MfmaArgs m) {
  const EncodeArgs& a = m.e;
  // LDS codebook image, two contiguous 16-byte planes per stage so that 16
  // consecutive codewords are one conflict-free 256-byte row:
  //   lo[s][k] = c_k          (d=4: [c_k, c_k])
  //   hi[s][k] = [n_hi, n_lo, 16, 16, 0, 0, 0, 0],  n = |c_k|^2 / 2
  //   neg[k]   = -c_k of stage 1 (d=4: [-c_k, -c_k]), the stage-2 B slots
  __shared__ half8 tab_lo[S][256];
  __shared__ half8 tab_hi[S][256];
  __shared__ half8 tab_neg[S > 1 ? 256 : 1];
  __shared__ float s_ncmax[S][4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform, so row planning and addressing stay in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lg = lane >> 4;
  const int ln = lane & 15;

  // logical block: group fastest, then head, then row chunk
  const uint32_t L = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t P = a.H * a.G;
  const bool active = (int64_t)L < P * m.n_chunks;
  const int64_t g = active ? (int64_t)L % a.G : 0;
  const int64_t h = active ? ((int64_t)L / a.G) % a.H : 0;
  const int64_t chunk = active ? (int64_t)L / P : 0;
  const int64_t p = h * a.G + g;

  // ---- stage the fp16-deployed codebooks (one codeword per thread) ----
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
#pragma unroll
    for (int i = 0; i < D; ++i) nc = fmaf((float)cw[i], (float)cw[i], nc);
    const float halfn = 0.5f * nc;
    const half_t nhi = (half_t)halfn;
    const half_t nlo = (half_t)(halfn - (float)nhi);
    half8 lo, hi;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      lo[e] = cw[e % D];
      hi[e] = (half_t)0.f;
    }
    hi[0] = nhi;
    hi[1] = nlo;
    hi[2] = (half_t)16.f;  // row-bias slots: 16 * (beta/16)_hi + 16 * (beta/16)_lo
    hi[3] = (half_t)16.f;
    tab_lo[s][tid] = lo;
    tab_hi[s][tid] = hi;
    if (S > 1 && s == 0) tab_neg[tid] = -lo;
    float mx = nc;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if (lane == 0) s_ncmax[s][wave] = mx;
  }
  __syncthreads();
  if (!active) return;
  float ncmax[S];
#pragma unroll
  for (int s = 0; s < S; ++s)
    ncmax[s] = fmaxf(fmaxf(s_ncmax[s][0], s_ncmax[s][1]), fmaxf(s_ncmax[s][2], s_ncmax[s][3]));

  // this lane's A plane: d=8 lanes 0-31 read c, 32-63 the norm plane;
  // d=4 lanes 0-15 read [c,c], 16-63 the norm plane (B is zero past slot 9)
  const bool a_hi = (D == 8) ? (lg >= 2) : (lg >= 1);
  const half8* plane = a_hi ? &tab_hi[0][0] : &tab_lo[0][0];

  const int64_t rows = a.B * a.T;
  const int64_t r_begin = chunk * m.rows_per_wg;
  int64_t r_end = r_begin + m.rows_per_wg;
  if (r_end > rows) r_end = rows;
  const _Float16* states = (const _Float16*)a.states;
  const int64_t Dfull = a.G * D;
  const int64_t head_x = h * a.sh + g * D;             // states offset of (h, g)
  const int64_t head_c = h * a.ch + g * S;             // codes offset of (h, g)
  const int64_t out_bstride = a.H * a.T * Dfull;       // recon is contiguous
  const int64_t head_o = h * a.T * Dfull + g * D;

  half8 neg_one_slot;
#pragma unroll
  for (int e = 0; e < 8; ++e) neg_one_slot[e] = (half_t)0.f;
  neg_one_slot[0] = (half_t)-1.f;
  neg_one_slot[1] = (half_t)-1.f;

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
  // per-lane offsets of tile i: (valid, states, codes, reconstruction).  The
  // row strides are below 2^24 (host-checked), so the full-rate 24-bit
  // multiply replaces the quarter-rate 32-bit one.
  auto locate = [&](const Iter& it, int i, uint32_t* xo, uint32_t* co, uint32_t* oo) -> bool {
    const uint32_t rr = (uint32_t)(i * 16 + ln);
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
  auto load_x = [&](const Iter& it, half8* dst) {
#pragma unroll
    for (int i = 0; i < kTiles; ++i) {
      uint32_t xo, co, oo;
      locate(it, i, &xo, &co, &oo);
      if (D == 8) {
        dst[i] = *(const half8*)(states + xo);
      } else {
        const half4 v = *(const half4*)(states + xo);
        dst[i] = half8{v[0], v[1], v[2], v[3], (half_t)0.f, (half_t)0.f, (half_t)0.f, (half_t)0.f};
      }
    }
  };

  half8 x[kTiles];
  Iter cur = plan(base);
  if (base < r_end) load_x(cur, x);

  for (; base < r_end; base += kRowsPerIter) {
    const bool more = base + kRowsPerIter < r_end;
    const Iter nxt = plan(base + kRowsPerIter);
    uint32_t code_bytes[kTiles];
    // stage 1's winning D (negative) and delta_1 per row, for stage 2's bias
    float dwin[kTiles], delta1[kTiles];
#pragma unroll
    for (int i = 0; i < kTiles; ++i) {
      code_bytes[i] = 0u;
      dwin[i] = 0.f;
      delta1[i] = 0.f;
    }

#pragma unroll
    for (int s = 0; s < S; ++s) {
      half8 bop[kTiles];
#pragma unroll
      for (int i = 0; i < kTiles; ++i) {
        // row bias beta = (|r|^2 + delta)/2 enters through the norm plane's
        // (16, 16) slots as -(beta/16) split into two fp16 halves
        float rr, delta;
        half8 negc = half8{};
        if (s == 0) {
          rr = dot2_acc(x[i], x[i]);
          delta = (rr + ncmax[0]) * 0x1p-8f;
          delta1[i] = delta;
        } else {
          negc = tab_neg[code_bytes[i] & 255u];  // -c_1 (d=4: [-c_1, -c_1])
          rr = fmaxf(-2.f * dwin[i] - delta1[i], 0.f);
          delta = (rr + ncmax[s]) * 0x1p-8f + delta1[i] * 0x1p-10f;
        }
        const float beta16 = (rr + delta) * (0.5f / 16.f) + 0x1p-60f;
        const half_t bh = (half_t)beta16;
        const half_t bl = (half_t)(beta16 - (float)bh);
        half8 normb = neg_one_slot;
        normb[2] = -bh;
        normb[3] = -bl;
        half8 b;
        if (D == 8) {
          b = (lg == 0) ? x[i] : (lg == 1) ? negc : (lg == 2) ? normb : half8{};
        } else {
          const half8 xc = half8{x[i][0], x[i][1], x[i][2], x[i][3], negc[4], negc[5], negc[6], negc[7]};
          b = (lg == 0) ? xc : (lg == 1) ? normb : half8{};
        }
        bop[i] = b;
      }
      // the rows are consumed: load the next iteration's into the same
      // registers, in flight during this stage's MFMA loop
      if (s == S - 1 && more) load_x(nxt, x);
      const float4v zero4 = {0.f, 0.f, 0.f, 0.f};
      uint32_t best[kTiles];
#pragma unroll
      for (int i = 0; i < kTiles; ++i) best[i] = 0xFFFFFFFFu;
      const half8* pl = plane + s * 256 + ln;
      // software pipeline: the MFMAs of chunk c+1 run while the keys of
      // chunk c are reduced (scheduling barriers keep ~2 chunks in flight)
      half8 af_next = pl[0];
      float4v acc[2][kTiles];
#pragma unroll
      for (int i = 0; i < kTiles; ++i)
        acc[0][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af_next, bop[i], zero4, 0, 0, 0);
      af_next = pl[16];
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const int cur = c & 1;
        const half8 af = af_next;
        if (c + 2 < 16) af_next = pl[(c + 2) * 16];
#pragma unroll
        for (int i = 0; i < kTiles; ++i) {
          if (c + 1 < 16)
            acc[cur ^ 1][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bop[i], zero4, 0, 0, 0);
          const float4v v = acc[cur][i];
          const uint32_t k0 = (__float_as_uint(v[0]) & ~63u) | (uint32_t)(c * 4 + 0);
          const uint32_t k1 = (__float_as_uint(v[1]) & ~63u) | (uint32_t)(c * 4 + 1);
          const uint32_t k2 = (__float_as_uint(v[2]) & ~63u) | (uint32_t)(c * 4 + 2);
          const uint32_t k3 = (__float_as_uint(v[3]) & ~63u) | (uint32_t)(c * 4 + 3);
          best[i] = umin3(umin3(k0, k1, k2), k3, best[i]);
          // pin the running minimum here: without it the compiler sinks the
          // key reduction of later tiles past the stage epilogue and keeps
          // every MFMA result of the stage live
          asm volatile("" : "+v"(best[i]));
        }
        // issue order per chunk: one MFMA of chunk c+1, then the six key
        // operations of one tile of chunk c, four times, so both the MFMA and
        // the VALU pipe always have work from this wave
#pragma unroll
        for (int i = 0; i < kTiles; ++i) {
          if (c + 1 < 16) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int i = 0; i < kTiles; ++i) {
        const uint32_t tag = best[i] & 63u;
        const uint32_t kidx = ((tag >> 2) << 4) | ((uint32_t)lg << 2) | (tag & 3u);
        const uint32_t kfull = lane_group_min((best[i] & ~255u) | kidx);
        const uint32_t kstar = kfull & 255u;
        if (s + 1 < S) dwin[i] = __uint_as_float(kfull & ~255u);
        code_bytes[i] |= kstar << (8 * s);
        half8 cw = tab_lo[s][kstar];
        if (D == 4) cw = half8{cw[0], cw[1], cw[2], cw[3], (half_t)0.f, (half_t)0.f, (half_t)0.f, (half_t)0.f};
        // depth-2 reconstruction fp16(fp32(c1) + fp32(c2)): the sum of two fp16
        // words is exact in fp32 or, when it is not, too small to move the
        // fp16 rounding, so one fp16 add gives the same bits.
        half8 dec = cw;
        if (s > 0) {
          half8 c1 = tab_lo[0][code_bytes[i] & 255u];
          if (D == 4) c1 = half8{c1[0], c1[1], c1[2], c1[3], (half_t)0.f, (half_t)0.f, (half_t)0.f, (half_t)0.f};
          dec = c1 + cw;
        }
        void* out = m.recon_depth[s];
        uint32_t xo, co, oo;
        const bool valid = locate(cur, i, &xo, &co, &oo);
        if (out != nullptr && lg == 0 && valid) {
          _Float16* op = (_Float16*)out + oo;
          if (D == 8) {
            *(half8*)op = dec;
          } else {
            *(half4*)op = half4{dec[0], dec[1], dec[2], dec[3]};
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kTiles; ++i) {
      uint32_t xo, co, oo;
      const bool valid = locate(cur, i, &xo, &co, &oo);
      if (lg == 0 && valid) {
        uint8_t* cp = a.codes + co;
        if (S == 1) {
          cp[0] = (uint8_t)code_bytes[i];
        } else {
          *(uint16_t*)cp = (uint16_t)code_bytes[i];
        }
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

template <int D, int S>
static int launch_mfma(const EncodeArgs& e, hipStream_t stream) {
  MfmaArgs m = {};
  m.e = e;
  for (int i = 0; i < e.n_exits; ++i) m.recon_depth[e.exit_depth[i] - 1] = e.recon[i];
  const int64_t rows = e.B * e.T;
  const int64_t P = e.H * e.G;
  // rows per workgroup: amortise the codebook staging, fill 256 CUs x 4 WGs
  int64_t rpw = 4096;
  while (rpw > kRowsPerIter && P * ceil_div(rows, rpw) < 256 * 4) rpw >>= 1;
  m.rows_per_wg = rpw;
  m.n_chunks = ceil_div(rows, rpw);
  int64_t nblocks = P * m.n_chunks;
  if (nblocks > 8) nblocks = ceil_div(nblocks, 8) * 8;  // xcd_remap needs a multiple of 8
  JKV_CHECK_ARG(nblocks < (int64_t)1 << 31, "grid too large");
  hipLaunchKernelGGL((rvq_encode_mfma<D, S>), dim3((uint32_t)nblocks), dim3(256), 0, stream, m);
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

}  // namespace jkv

extern "C" {

int64_t jkv_rvq_encode_workspace_bytes(int64_t H, int64_t G, int64_t S, int64_t K,
                                       int64_t d, int32_t has_whitener) {
  if (!has_whitener) return 0;
  return H * G * S * K * d * (int64_t)sizeof(float);
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

  if (whiteners != nullptr) {
    int64_t need = jkv_rvq_encode_workspace_bytes(H, G, S, K, d, 1);
    JKV_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                  "whitened encode needs %lld bytes of workspace", (long long)need);
    float* sel = (float*)workspace;
    int64_t n = H * G * S * K * d;
    hipLaunchKernelGGL(selector_tables_kernel, dim3((uint32_t)ceil_div(n, 256)), dim3(256), 0,
                       stream, tables, whiteners, sel, H * G, S, K, d);
    JKV_CHECK_LAUNCH();
    a.sel_tables = sel;
  }

  const bool aligned16 = (((uintptr_t)states) % 16 == 0) && stride_b % 8 == 0 &&
                         stride_h % 8 == 0 && stride_t % 8 == 0;
  const bool codes_aligned = (S == 1) || ((((uintptr_t)codes) % 2 == 0) && code_stride_b % 2 == 0 &&
                                          code_stride_h % 2 == 0 && code_stride_t % 2 == 0);
  bool recon_aligned = true;
  for (int e = 0; e < n_exits; ++e)
    if (a.recon[e] && ((uintptr_t)a.recon[e]) % 16 != 0) recon_aligned = false;
  bool distinct_exits = true;
  for (int i = 0; i < n_exits; ++i)
    for (int j = 0; j < i; ++j)
      if (exit_depths[i] == exit_depths[j]) distinct_exits = false;
  // the MFMA path addresses states, codes and reconstructions with 32-bit
  // element offsets
  const int64_t x_span = (B - 1) * stride_b + (H - 1) * stride_h + (T - 1) * stride_t + G * d;
  const int64_t c_span = (B - 1) * code_stride_b + (H - 1) * code_stride_h + (T - 1) * code_stride_t + G * S;
  // (and token strides below 2^24, for 24-bit multiplies)
  const bool offsets32 = stride_b >= 0 && stride_h >= 0 && stride_t >= 0 && code_stride_b >= 0 &&
                         code_stride_h >= 0 && code_stride_t >= 0 && x_span < ((int64_t)1 << 31) &&
                         c_span < ((int64_t)1 << 31) && B * H * T * G * d < ((int64_t)1 << 31) &&
                         stride_t < ((int64_t)1 << 24) && code_stride_t < ((int64_t)1 << 24) &&
                         G * d < ((int64_t)1 << 24);
  const bool fast = offsets32 && states_dtype == JKV_F16 && whiteners == nullptr && K == 256 &&
                    (d == 8 || d == 4) && (S == 1 || S == 2) && aligned16 && codes_aligned &&
                    recon_aligned && distinct_exits && B * T < ((int64_t)1 << 31) &&
                    T < ((int64_t)1 << 31);
  if (fast) {
    if (d == 8) return S == 1 ? launch_mfma<8, 1>(a, stream) : launch_mfma<8, 2>(a, stream);
    return S == 1 ? launch_mfma<4, 1>(a, stream) : launch_mfma<4, 2>(a, stream);
  }
  switch (states_dtype) {
    case JKV_F16: return launch_generic<JKV_F16>(a, stream);
    case JKV_BF16: return launch_generic<JKV_BF16>(a, stream);
    default: return launch_generic<JKV_F32>(a, stream);
  }
}

}  // extern "C"
