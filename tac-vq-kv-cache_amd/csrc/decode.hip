// Codes-to-vector reconstruction with frozen codes.
#include "jkv_common.h"

namespace jkv {

struct RvqDecodeArgs {
  const uint8_t* codes;
  int64_t cb, ch, ct;  // code byte strides (b, h, t); the (G,S) block contiguous
  int64_t BH, H;
  int32_t T, G, d, S, K, depth;
  int32_t run_tokens;   // rvq_decode_lds_kernel: tokens per workgroup
  const void* tables;   // [H*G][S][K][d]: fp32 masters, or their fp16 deployed words
  void* out;            // [B,H,T,G*d] contiguous
};

// CW consecutive outputs from fp32 sums
template <int DT, int CW>
__device__ __forceinline__ void store_chunk(void* out, int64_t i, const float* v) {
  if constexpr (CW == 1) {
    Elem<DT>::store(out, i, v[0]);
  } else if constexpr (DT == JKV_F16) {
    typedef _Float16 hv __attribute__((ext_vector_type(CW)));
    hv h;
#pragma unroll
    for (int e = 0; e < CW; ++e) h[e] = (_Float16)v[e];
    *(hv*)((_Float16*)out + i) = h;
  } else if constexpr (DT == JKV_F32) {
#pragma unroll
    for (int e = 0; e < CW; e += 4) *(float4*)((float*)out + i + e) = float4{v[e], v[e + 1], v[e + 2], v[e + 3]};
  } else {
#pragma unroll
    for (int e = 0; e < CW; ++e) Elem<DT>::store(out, i + e, v[e]);
  }
}

// One thread per (row, group): the group's code bytes, then per chunk of CW
// dimensions each stage's codeword read as fp32 (16-byte loads for CW >= 4),
// rounded to fp16 and back (the deployed table), summed in fp32 in stage
// order and stored as CW consecutive outputs:
//   out[b,h,t,g*d+i] = dtype( sum_{s<depth} fp32(fp16(C[h*G+g, s, code_s, i])) ).
// Grid: x over the (row, group) items of one (batch, head) slice, y over the
// slices.  F16: the tables are already the fp16 deployed words (half the
// bytes per codeword read; the same sums).
template <int DT, int CW, bool F16>
__global__ __launch_bounds__(256) void rvq_decode_kernel(RvqDecodeArgs a) {
  const uint32_t item = blockIdx.x * 256u + threadIdx.x;
  const uint32_t n = (uint32_t)a.T * (uint32_t)a.G;
  if (item >= n) return;
  const uint32_t t = item / (uint32_t)a.G, g = item % (uint32_t)a.G;
  const int64_t D = (int64_t)a.G * a.d;
  for (int64_t bh = blockIdx.y; bh < a.BH; bh += gridDim.y) {
    const int64_t b = bh / a.H, h = bh % a.H;
    const uint8_t* cp = a.codes + b * a.cb + h * a.ch + t * a.ct + g * a.S;
    const int64_t tab0 = (h * a.G + g) * (int64_t)a.S * a.K * a.d;
    const int64_t o = (bh * a.T + t) * D + (int64_t)g * a.d;
    const int depth = a.depth;
    for (int i = 0; i < a.d; i += CW) {
      float acc[CW];
#pragma unroll
      for (int e = 0; e < CW; ++e) acc[e] = 0.f;
      for (int s = 0; s < depth; ++s) {
        const int64_t wo = tab0 + ((int64_t)s * a.K + cp[s]) * a.d + i;
        if constexpr (F16) {
          typedef _Float16 hv __attribute__((ext_vector_type(CW)));
          const hv w = *((const hv*)((const _Float16*)a.tables + wo));
#pragma unroll
          for (int e = 0; e < CW; ++e) acc[e] += (float)w[e];
          continue;
        }
        const float* w = (const float*)a.tables + wo;
        if constexpr (CW == 1) {
          acc[0] += deploy16(w[0]);
        } else {
#pragma unroll
          for (int e = 0; e < CW; e += 4) {
            const float4 x = *(const float4*)(w + e);
            acc[e] += deploy16(x.x);
            acc[e + 1] += deploy16(x.y);
            acc[e + 2] += deploy16(x.z);
            acc[e + 3] += deploy16(x.w);
          }
        }
      }
      store_chunk<DT, CW>(a.out, o + i, acc);
    }
  }
}

// 8-dim groups and 256 codewords with every (group, stage) table of a head
// fitting 128 KiB of LDS (G S <= 32): one 512-thread workgroup per (batch,
// head, run of tokens; one round of workgroups over the CUs where the
// tokens allow) stages the head's tables as fp16
// words (converted from the fp32 masters when those are given), then
// rebuilds its (token, group) items from LDS gathers instead of one random
// 16-byte read per stage from L2.  Thread i takes group i % G of tokens
// i / G, i / G + 512 / G, ...: the 16 or 32 threads of a token write its row
// in one contiguous run.  The same sums in the same order as
// rvq_decode_kernel.
static const int kLdsDecodeTokens = 512;  // shortest run
template <int DT, bool F16>
__global__ __launch_bounds__(512) void rvq_decode_lds_kernel(RvqDecodeArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  half8* tab = (half8*)lds_raw;  // [G * S][256] codeword words
  const int G = a.G, S = a.S;
  const int64_t n_runs = ((int64_t)a.T + a.run_tokens - 1) / a.run_tokens;
  const int64_t run = (int64_t)blockIdx.x % n_runs;
  const int64_t bh = (int64_t)blockIdx.x / n_runs;
  const int64_t b = bh / a.H, h = bh % a.H;
  const int n_words = G * S * 256;
  const int64_t src0 = h * (int64_t)n_words;  // the head's tables are contiguous
  for (int i = threadIdx.x; i < n_words; i += 512) {
    half8 w;
    if constexpr (F16) {
      w = ((const half8*)a.tables)[src0 + i];
    } else {
      const float4 x0 = ((const float4*)a.tables)[2 * (src0 + i)];
      const float4 x1 = ((const float4*)a.tables)[2 * (src0 + i) + 1];
      w = half8{(_Float16)x0.x, (_Float16)x0.y, (_Float16)x0.z, (_Float16)x0.w,
                (_Float16)x1.x, (_Float16)x1.y, (_Float16)x1.z, (_Float16)x1.w};
    }
    tab[i] = w;
  }
  __syncthreads();
  const int g = (int)threadIdx.x % G;
  const int tstep = 512 / G;
  const int64_t t_end = min((int64_t)a.T, (run + 1) * (int64_t)a.run_tokens);
  const int64_t D = (int64_t)G * 8;
  const uint8_t* cbase = a.codes + b * a.cb + h * a.ch + g * S;
  // eight tokens at a time: their code bytes are all requested before the
  // first gather, so the loads' latency is paid once per eight items
  constexpr int kU = 8;
  const int depth = a.depth;
  for (int64_t t0 = run * (int64_t)a.run_tokens + (int)threadIdx.x / G; t0 < t_end; t0 += kU * tstep) {
    uint32_t code[kU][2];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t t = t0 + (int64_t)u * tstep;
      const uint8_t* cp = cbase + (t < t_end ? t : t0) * a.ct;
      code[u][0] = cp[0];
      code[u][1] = depth > 1 ? cp[1] : 0u;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t t = t0 + (int64_t)u * tstep;
      if (t >= t_end) break;
      float acc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (s >= depth) break;
        const half8 w = tab[(g * S + s) * 256 + code[u][s]];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += (float)w[e];
      }
      store_chunk<DT, 8>(a.out, (bh * a.T + t) * D + (int64_t)g * 8, acc);
    }
  }
}

template <int DT, bool F16>
static void launch_decode_lds(const RvqDecodeArgs& a, hipStream_t stream) {
  const int64_t n_runs = ((int64_t)a.T + a.run_tokens - 1) / a.run_tokens;
  hipLaunchKernelGGL((rvq_decode_lds_kernel<DT, F16>), dim3((uint32_t)(a.BH * n_runs)), dim3(512),
                     (size_t)a.G * a.S * 256 * 16, stream, a);
}

template <int DT, bool F16>
static void launch_decode(const RvqDecodeArgs& a, int cw, dim3 grid, hipStream_t stream) {
  if (cw == 8) {
    hipLaunchKernelGGL((rvq_decode_kernel<DT, 8, F16>), grid, dim3(256), 0, stream, a);
  } else if (cw == 4) {
    hipLaunchKernelGGL((rvq_decode_kernel<DT, 4, F16>), grid, dim3(256), 0, stream, a);
  } else {
    hipLaunchKernelGGL((rvq_decode_kernel<DT, 1, F16>), grid, dim3(256), 0, stream, a);
  }
}

static int rvq_decode_impl(const uint8_t* codes, int64_t code_stride_b, int64_t code_stride_h,
                           int64_t code_stride_t, int64_t B, int64_t H, int64_t T, int64_t G, int64_t d,
                           const void* tables, bool tables_f16, int64_t S, int64_t K, int32_t depth, void* out,
                           int32_t out_dtype, jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(B >= 0 && H > 0 && T >= 0 && G > 0 && d > 0 && S > 0 && K > 0 && K <= 256,
                "invalid decode geometry");
  JKV_CHECK_ARG(depth >= 1 && depth <= S, "decode depth outside the ladder");
  JKV_CHECK_ARG(T * G < ((int64_t)1 << 31) && S <= 65536 && d <= 65536, "decode slice too large");
  const int64_t n = B * H * T * G * d;
  if (n == 0) return JKV_OK;
  JKV_CHECK_ARG(codes && tables && out, "null buffer");
  if (out_dtype != JKV_F16 && out_dtype != JKV_BF16 && out_dtype != JKV_F32)
    return set_error(JKV_EINVAL, "unknown output dtype %d", out_dtype);
  RvqDecodeArgs a;
  a.codes = codes; a.cb = code_stride_b; a.ch = code_stride_h; a.ct = code_stride_t;
  a.BH = B * H; a.H = H;
  a.T = (int32_t)T; a.G = (int32_t)G; a.d = (int32_t)d; a.S = (int32_t)S; a.K = (int32_t)K; a.depth = depth;
  a.tables = tables;
  a.out = out;
  // vector chunks when every table row and output chunk is 16-byte aligned
  // (fp32 rows) and the output chunk is aligned to its own width
  const size_t esize = out_dtype == JKV_F32 ? 4 : 2;
  auto aligned = [&](int cw) {
    const uintptr_t tab_align = tables_f16 ? (uintptr_t)(cw * 2) : 16u;
    return d % cw == 0 && (uintptr_t)tables % tab_align == 0 && (uintptr_t)out % (cw * esize) == 0;
  };
  const int cw = aligned(8) ? 8 : aligned(4) ? 4 : 1;
  // 8-dim groups whose head tables fit 128 KiB of LDS: gathers from LDS
  const bool lds = d == 8 && K == 256 && G * S <= 32 && 512 % G == 0 && cw == 8 && depth <= 2 &&
                   (uintptr_t)tables % 16 == 0 && B * H * ceil_div(T, kLdsDecodeTokens) < ((int64_t)1 << 31);
  if (lds) {
    // runs long enough for one round of workgroups over 256 CUs (each holds
    // one: 128 KiB of tables), so each CU stages its tables once
    const int64_t runs_per_slice = std::max<int64_t>(1, 256 / (B * H));
    a.run_tokens = (int32_t)std::max<int64_t>(kLdsDecodeTokens, ceil_div(T, runs_per_slice));
    switch (out_dtype) {
      case JKV_F16:
        tables_f16 ? launch_decode_lds<JKV_F16, true>(a, stream) : launch_decode_lds<JKV_F16, false>(a, stream);
        break;
      case JKV_BF16:
        tables_f16 ? launch_decode_lds<JKV_BF16, true>(a, stream) : launch_decode_lds<JKV_BF16, false>(a, stream);
        break;
      default:
        tables_f16 ? launch_decode_lds<JKV_F32, true>(a, stream) : launch_decode_lds<JKV_F32, false>(a, stream);
        break;
    }
    JKV_CHECK_LAUNCH();
    return JKV_OK;
  }
  const int64_t slices = B * H;
  const dim3 grid((uint32_t)ceil_div(T * G, 256), (uint32_t)(slices < 65535 ? slices : 65535));
  switch (out_dtype) {
    case JKV_F16:
      tables_f16 ? launch_decode<JKV_F16, true>(a, cw, grid, stream) : launch_decode<JKV_F16, false>(a, cw, grid, stream);
      break;
    case JKV_BF16:
      tables_f16 ? launch_decode<JKV_BF16, true>(a, cw, grid, stream) : launch_decode<JKV_BF16, false>(a, cw, grid, stream);
      break;
    default:
      tables_f16 ? launch_decode<JKV_F32, true>(a, cw, grid, stream) : launch_decode<JKV_F32, false>(a, cw, grid, stream);
      break;
  }
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

}  // namespace jkv

extern "C" int jkv_rvq_decode(const uint8_t* codes, int64_t code_stride_b, int64_t code_stride_h,
                              int64_t code_stride_t, int64_t B, int64_t H, int64_t T, int64_t G,
                              int64_t d, const float* tables, int64_t S, int64_t K, int32_t depth,
                              void* out, int32_t out_dtype, jkv_stream_t stream) {
  return jkv::rvq_decode_impl(codes, code_stride_b, code_stride_h, code_stride_t, B, H, T, G, d, tables, false, S,
                              K, depth, out, out_dtype, stream);
}

extern "C" int jkv_rvq_decode_f16(const uint8_t* codes, int64_t code_stride_b, int64_t code_stride_h,
                                  int64_t code_stride_t, int64_t B, int64_t H, int64_t T, int64_t G,
                                  int64_t d, const void* tables16, int64_t S, int64_t K, int32_t depth,
                                  void* out, int32_t out_dtype, jkv_stream_t stream) {
  return jkv::rvq_decode_impl(codes, code_stride_b, code_stride_h, code_stride_t, B, H, T, G, d, tables16, true,
                              S, K, depth, out, out_dtype, stream);
}
