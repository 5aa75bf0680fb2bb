// Hard greedy residual-VQ / grouped-CQ encode for gfx950.
//
// Two kernels share one argument block:
//  * rvq_encode_mfma<D,S>: fp16 states, d in {4,8}, K=256, S<=2, no whitener.
//    One wave owns one (head, group) problem and a range of rows.  The
//    problem's codebooks live in VGPRs as the A operand of
//    v_mfma_f32_16x16x32_f16 (codewords x contraction slots); a tile of 16
//    rows is the B operand.  The contraction packs [r_hi | r_lo | norm]
//    so one MFMA yields -(|r|^2 + |c|^2 - 2 r.c + delta)/2 for 16 codewords
//    x 16 rows with fp32 accumulation; the argmin is a min over keys that
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
  int64_t rows_per_unit;  // rows handled by one wave (mfma kernel)
  int64_t n_units;
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
// v_mfma_f32_16x16x32_f16 operand layout (wave64):
//   A[i][k]: lane = i + 16*(k/8), element k%8      (i = codeword in chunk)
//   B[k][j]: lane = j + 16*(k/8), element k%8      (j = row in tile)
//   D[i][j]: lane = j + 16*(i/4), element i%4
// Contraction slots (k):
//   d=8: [ 0.. 7] r_hi . c   [ 8..15] r_lo . c   [16,17] (-1).(|c|^2/2 hi,lo)
//   d=4: [ 0.. 3] r_hi . c   [ 4.. 7] r_lo . c   [ 8, 9] (-1).(|c|^2/2 hi,lo)
// C input: -(|r|^2 + delta)/2 for every codeword of the row.
// Result: D = -(dist + delta)/2 < 0; as unsigned bit patterns negative
// floats order by magnitude, so min over bits = min distance.  The low 6
// bits are replaced by (chunk<<2 | i%4) before the min; the lane group adds
// the remaining 2 index bits in the cross-lane step (8 bits total).

template <int D>
struct MfmaGeom {
  // lanes holding the residual-hi/lo slots and the norm slot
  static constexpr int kNormLaneGroup = (D == 8) ? 2 : 1;
};

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

template <int D, int S>
__global__ __launch_bounds__(256) void rvq_encode_mfma(EncodeArgs a) {
  __shared__ half_t lds_tab[4][S][256][D];  // per-wave fp16 codebook copy

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lg = lane >> 4;  // lane group
  const int ln = lane & 15;

  const uint32_t nblocks = gridDim.x;
  const int64_t unit = (int64_t)xcd_remap(blockIdx.x, nblocks) * 4 + wave;
  const int64_t P = a.H * a.G;
  const bool active = unit < a.n_units;
  const int64_t p = active ? unit % P : 0;
  const int64_t range = active ? unit / P : 0;
  const int64_t h = p / a.G, g = p % a.G;

  // ---- A operand image and LDS codebook copy ----------------------------
  half8 aimg[S][16];
  float delta_scale[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    float ncmax = 0.f;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const int kidx = c * 16 + ln;
      const float* src = a.tables + ((p * S + s) * 256 + kidx) * D;
      half_t cw[D];
      float nc = 0.f;
#pragma unroll
      for (int i = 0; i < D; ++i) {
        cw[i] = (half_t)src[i];
        float f = (float)cw[i];
        nc = fmaf(f, f, nc);
      }
      ncmax = fmaxf(ncmax, nc);
      const float halfn = 0.5f * nc;
      const half_t nhi = (half_t)halfn;
      const half_t nlo = (half_t)(halfn - (float)nhi);
      half8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (half_t)0.f;
      if (D == 8) {
        if (lg <= 1) {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = cw[e % D];
        } else if (lg == 2) {
          v[0] = nhi;
          v[1] = nlo;
        }
      } else {
        if (lg == 0) {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = cw[e % D];
        } else if (lg == 1) {
          v[0] = nhi;
          v[1] = nlo;
        }
      }
      aimg[s][c] = v;
      if (lg == 0) {
#pragma unroll
        for (int i = 0; i < D; ++i) lds_tab[wave][s][kidx][i] = cw[i];
      }
    }
    // max |c|^2 over the codebook (wave reduction)
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
      ncmax = fmaxf(ncmax, __shfl_xor(ncmax, off, 64));
    delta_scale[s] = ncmax;
  }
  __syncthreads();
  if (!active) return;

  // ---- B operand constants ------------------------------------------------
  const int norm_lg = MfmaGeom<D>::kNormLaneGroup;
  const int64_t rows = a.B * a.T;
  const int64_t row_begin = range * a.rows_per_unit;
  int64_t row_end = row_begin + a.rows_per_unit;
  if (row_end > rows) row_end = rows;
  const int64_t Dfull = a.G * D;
  const _Float16* states = (const _Float16*)a.states;

  for (int64_t tile = row_begin; tile < row_end; tile += 16) {
    const int64_t row = tile + ln;
    const bool valid = row < row_end;
    const int64_t rb = valid ? row / a.T : 0;
    const int64_t rt = valid ? row % a.T : 0;
    // every lane holds the 16-row tile's residual for its row (lane & 15)
    float r[D];
    {
      const _Float16* xp = states + rb * a.sb + h * a.sh + rt * a.st + g * D;
      if (D == 8) {
        half8 xv = valid ? *(const half8*)xp : half8{};
#pragma unroll
        for (int i = 0; i < D; ++i) r[i] = (float)xv[i];
      } else {
        half4 xv = valid ? *(const half4*)xp : half4{};
#pragma unroll
        for (int i = 0; i < D; ++i) r[i] = (float)xv[i];
      }
    }
    float dec[D];
#pragma unroll
    for (int i = 0; i < D; ++i) dec[i] = 0.f;
    uint32_t code_bytes = 0;

#pragma unroll
    for (int s = 0; s < S; ++s) {
      // hi/lo split of the fp32 residual (exact for s == 0: fp16 inputs)
      half_t rhi[D], rlo[D];
      float rr = 0.f;
#pragma unroll
      for (int i = 0; i < D; ++i) {
        rhi[i] = (half_t)r[i];
        rlo[i] = (half_t)(r[i] - (float)rhi[i]);
        rr = fmaf(r[i], r[i], rr);
      }
      half8 bop;
#pragma unroll
      for (int e = 0; e < 8; ++e) bop[e] = (half_t)0.f;
      if (D == 8) {
        if (lg == 0) {
#pragma unroll
          for (int e = 0; e < 8; ++e) bop[e] = rhi[e % D];
        } else if (lg == 1) {
#pragma unroll
          for (int e = 0; e < 8; ++e) bop[e] = rlo[e % D];
        }
      } else {
        if (lg == 0) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            bop[e] = rhi[e];
            bop[e + 4] = rlo[e];
          }
        }
      }
      if (lg == norm_lg) {
        bop[0] = (half_t)-1.f;
        bop[1] = (half_t)-1.f;
      }
      // delta dominates the fp32 rounding of the accumulation so every key
      // stays strictly negative; it is common to all codewords of the row.
      const float delta = (rr + delta_scale[s]) * 0x1p-16f + 0x1p-100f;
      const float cval = -0.5f * (rr + delta);
      const float4v cin = {cval, cval, cval, cval};

      uint32_t best = 0xFFFFFFFFu;
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        float4v acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(aimg[s][c], bop, cin, 0, 0, 0);
        uint32_t k0 = (__float_as_uint(acc[0]) & ~63u) | (uint32_t)(c * 4 + 0);
        uint32_t k1 = (__float_as_uint(acc[1]) & ~63u) | (uint32_t)(c * 4 + 1);
        uint32_t k2 = (__float_as_uint(acc[2]) & ~63u) | (uint32_t)(c * 4 + 2);
        uint32_t k3 = (__float_as_uint(acc[3]) & ~63u) | (uint32_t)(c * 4 + 3);
        best = umin3(umin3(k0, k1, k2), k3, best);
      }
      // codeword index = chunk*16 + lane_group*4 + i%4
      const uint32_t tag = best & 63u;
      const uint32_t kidx = ((tag >> 2) << 4) | ((uint32_t)lg << 2) | (tag & 3u);
      const uint32_t key = lane_group_min((best & ~255u) | kidx);
      const uint32_t kstar = key & 255u;
      code_bytes |= kstar << (8 * s);
      // residual / decoded update with the fp16-deployed codeword
      const half_t* cw = &lds_tab[wave][s][kstar][0];
      float cf[D];
      if (D == 8) {
        half8 cv = *(const half8*)cw;
#pragma unroll
        for (int i = 0; i < D; ++i) cf[i] = (float)cv[i];
      } else {
        half4 cv = *(const half4*)cw;
#pragma unroll
        for (int i = 0; i < D; ++i) cf[i] = (float)cv[i];
      }
#pragma unroll
      for (int i = 0; i < D; ++i) {
        r[i] -= cf[i];
        dec[i] += cf[i];
      }
      // exits at depth s+1
      if (lg == 0 && valid) {
        for (int e = 0; e < a.n_exits; ++e) {
          if (a.exit_depth[e] != s + 1 || a.recon[e] == nullptr) continue;
          _Float16* op = (_Float16*)a.recon[e] + (rb * a.H + h) * a.T * Dfull + rt * Dfull + g * D;
          if (D == 8) {
            half8 o;
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = (half_t)dec[i];
            *(half8*)op = o;
          } else {
            half4 o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = (half_t)dec[i];
            *(half4*)op = o;
          }
        }
      }
    }
    if (lg == 0 && valid) {
      uint8_t* cp = a.codes + rb * a.cb + h * a.ch + rt * a.ct + g * S;
      if (S == 1) {
        cp[0] = (uint8_t)code_bytes;
      } else {
        *(uint16_t*)cp = (uint16_t)code_bytes;
      }
    }
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
static int launch_mfma(EncodeArgs a, hipStream_t stream) {
  const int64_t rows = a.B * a.T;
  const int64_t P = a.H * a.G;
  // rows per wave: enough to amortise the codebook load, enough waves to
  // fill 256 CUs x 8 waves.
  int64_t rpu = 1024;
  while (rpu > 64 && P * ceil_div(rows, rpu) < 256 * 8) rpu >>= 1;
  a.rows_per_unit = rpu;
  a.n_units = P * ceil_div(rows, rpu);
  int64_t nblocks = ceil_div(a.n_units, 4);
  if (nblocks > 8) nblocks = ceil_div(nblocks, 8) * 8;  // xcd_remap needs a multiple of 8
  JKV_CHECK_ARG(nblocks < (int64_t)1 << 31, "grid too large");
  hipLaunchKernelGGL((rvq_encode_mfma<D, S>), dim3((uint32_t)nblocks), dim3(256), 0, stream, a);
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
  const bool fast = states_dtype == JKV_F16 && whiteners == nullptr && K == 256 &&
                    (d == 8 || d == 4) && (S == 1 || S == 2) && aligned16 && codes_aligned &&
                    recon_aligned;
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
