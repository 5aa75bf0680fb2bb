// Fused decode attention over a packed uint8 GSRQ/CQ code cache.
//
// One workgroup per (batch, kv head, split of the visible window).  K̂ and V̂
// are rebuilt from fp16 codewords on the fly (never written to memory):
//  * scores: each lane rebuilds 32 dims (4 channel groups, both stages) of one
//    key, rotates it at its absolute position with the reference's fp16
//    rotary sequence (cos/sin from a table built with the reference's fp32
//    angle arithmetic), and four v_mfma_f32_16x16x32_f16 per 16-key tile
//    produce the scores of all query heads of the GQA group;
//  * softmax over the split in fp32; P.V̂ accumulates in fp32 on the VALU;
//  * the split's unnormalised (max, sum, out) go to a workspace that
//    decode_combine folds into fp16 outputs.
#include "jkv_common.h"
#include "rotary.h"

namespace jkv {

static const int kHeadDim = 128;
static const int kSplitTokens = 256;  // tokens per split (workgroup)
static const int kMaxCodeBytes = 64;  // code records staged in LDS up to this size

struct DecodeArgs {
  const _Float16* q;
  int64_t qsb, qsh;
  const uint8_t* kc;
  const uint8_t* vc;
  int64_t csb, csh, cap;
  const _Float16* kt;  // [KVH*G,S,K,d] fp16
  const _Float16* vt;
  int64_t B, QH, KVH, G, d, S, K;
  const int32_t* lengths;
  int64_t window;
  const half2v* rope;  // [rope_len][64] (cos, sin) fp16
  int64_t rope_len;
  int32_t n_splits;
  float* ws_o;   // [B,QH,n_splits,D]
  float* ws_ml;  // [B,QH,n_splits,2]
  _Float16* out;
};


// fp16 words of dims [8*c8, 8*c8+8) of one token: fp16(sum_s fp32(word_s)).
// The sum of two fp16 words is exact in fp32 or too small to move the fp16
// rounding, so for S = 2 one fp16 add gives the same bits; S > 2 sums in fp32.
template <int D>
__device__ __forceinline__ half8 rebuild8(const uint8_t* codes_tok, const _Float16* tab,
                                          int64_t kvh, int64_t G, int S, int c8) {
  if (D == 8) {
    const int g = c8;
    const _Float16* base = tab + ((kvh * G + g) * S) * 256 * 8;
    if (S == 2) {
      const half8 w0 = *(const half8*)(base + codes_tok[g * 2] * 8);
      const half8 w1 = *(const half8*)(base + 256 * 8 + codes_tok[g * 2 + 1] * 8);
      return w0 + w1;
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < S; ++s) {
      const half8 w = *(const half8*)(base + (s * 256 + codes_tok[g * S + s]) * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += (float)w[e];
    }
    half8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (_Float16)acc[e];
    return r;
  } else {  // D == 4: two groups per 8-dim chunk
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int g = 2 * c8 + half;
      const _Float16* base = tab + ((kvh * G + g) * S) * 256 * 4;
      for (int s = 0; s < S; ++s) {
        const half4 w = *(const half4*)(base + (s * 256 + codes_tok[g * S + s]) * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[half * 4 + e] += (float)w[e];
      }
    }
    half8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (_Float16)acc[e];
    return r;
  }
}

template <int D, int NQ>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeArgs a) {
  __shared__ _Float16 q_lds[NQ][kHeadDim];
  __shared__ float s_lds[NQ][kSplitTokens];
  __shared__ float red[NQ][4][2];
  __shared__ float o_red[4][NQ][kHeadDim];
  // the split's K and V code records (up to 64 bytes per token), fetched once
  __shared__ __align__(16) uint8_t kc_lds[kSplitTokens * kMaxCodeBytes];
  __shared__ __align__(16) uint8_t vc_lds[kSplitTokens * kMaxCodeBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int lg = lane >> 4, ln = lane & 15;
  const int64_t split = blockIdx.x % a.n_splits;
  const int64_t bk = blockIdx.x / a.n_splits;
  const int64_t kvh = bk % a.KVH;
  const int64_t b = bk / a.KVH;
  const int64_t L = a.lengths[b];
  const int64_t n_vis = L < a.window ? L : a.window;
  const int64_t start = L - n_vis;
  const int64_t t0 = start + split * kSplitTokens;
  int64_t t1 = t0 + kSplitTokens;
  if (t1 > L) t1 = L;
  const int ntok = t1 > t0 ? (int)(t1 - t0) : 0;
  const float scale = 1.0f / sqrtf((float)kHeadDim);
  const int S = (int)a.S;
  const int64_t code_bytes = a.G * a.S;

  // ---- rotated queries (fp16 rotary at position L-1) ----
  if (L > 0) {
    const half2v* qrow = a.rope + ((L - 1) < a.rope_len ? (L - 1) : a.rope_len - 1) * 64;
    for (int idx = tid; idx < NQ * 8; idx += blockDim.x) {
      const int h = idx / 8, c8 = idx % 8;  // dims [8c8, 8c8+8) and +64
      const _Float16* qp = a.q + b * a.qsb + (kvh * NQ + h) * a.qsh;
      half8 qa, qb, c, s, ra, rb;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qa[e] = qp[8 * c8 + e];
        qb[e] = qp[8 * c8 + 64 + e];
      }
      load_trig8(qrow, 8 * c8, &c, &s);
      rope16(qa, qb, c, s, &ra, &rb);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        q_lds[h][8 * c8 + e] = ra[e];
        q_lds[h][8 * c8 + 64 + e] = rb[e];
      }
    }
  }
  // ---- the split's code records into LDS, 16-byte chunks, one pass ----
  const bool codes_in_lds = code_bytes <= kMaxCodeBytes && (code_bytes % 16) == 0;
  if (codes_in_lds) {
    const int per_tok = (int)(code_bytes / 16);
    const int64_t kbase = b * a.csb + kvh * a.csh;
    for (int idx = tid; idx < ntok * per_tok; idx += blockDim.x) {
      const int j = idx / per_tok, part = idx % per_tok;
      const int64_t off = kbase + ((t0 + j) % a.cap) * code_bytes + part * 16;
      *(uint4*)(kc_lds + j * code_bytes + part * 16) = *(const uint4*)(a.kc + off);
      *(uint4*)(vc_lds + j * code_bytes + part * 16) = *(const uint4*)(a.vc + off);
    }
  }
  __syncthreads();
  auto key_codes = [&](int j) -> const uint8_t* {
    return codes_in_lds ? kc_lds + j * code_bytes
                        : a.kc + b * a.csb + kvh * a.csh + ((t0 + j) % a.cap) * code_bytes;
  };
  auto value_codes = [&](int j) -> const uint8_t* {
    return codes_in_lds ? vc_lds + j * code_bytes
                        : a.vc + b * a.csb + kvh * a.csh + ((t0 + j) % a.cap) * code_bytes;
  };

  // ---- pass A: scores on MFMA.  Lane (token ln, lane group lg) owns the
  // 8-dim chunks {lg, lg+4} and their rotary partners {lg+8, lg+12}; slice m
  // of the contraction is chunk 4m+lg, so chunk m*4+lg <-> MFMA m.
  {
    half8 qb[4];  // B operand: Q^T slices, column = head
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        qb[m][e] = (ln < NQ) ? q_lds[ln < NQ ? ln : 0][(4 * m + lg) * 8 + e] : (_Float16)0.f;
    }
    const int ntiles = (ntok + 15) / 16;
    for (int tile = wave; tile < ntiles; tile += 4) {
      const int tt = tile * 16 + ln;
      const bool valid = tt < ntok;
      const int64_t pos = valid ? t0 + tt : t0;
      const uint8_t* ct = key_codes(valid ? tt : 0);
      half8 k0 = rebuild8<D>(ct, a.kt, kvh, a.G, S, lg);
      half8 k1 = rebuild8<D>(ct, a.kt, kvh, a.G, S, lg + 4);
      half8 k2 = rebuild8<D>(ct, a.kt, kvh, a.G, S, lg + 8);
      half8 k3 = rebuild8<D>(ct, a.kt, kvh, a.G, S, lg + 12);
      // the host sizes the table past every length; the clamp only keeps a
      // misuse from reading out of bounds
      const half2v* trow = a.rope + (pos < a.rope_len ? pos : a.rope_len - 1) * 64;
      half8 c, s, r0, r1, r2, r3;
      load_trig8(trow, 8 * lg, &c, &s);
      rope16(k0, k2, c, s, &r0, &r2);
      load_trig8(trow, 8 * (lg + 4), &c, &s);
      rope16(k1, k3, c, s, &r1, &r3);
      if (!valid) {
        r0 = half8{}; r1 = half8{}; r2 = half8{}; r3 = half8{};
      }
      float4v acc = {0.f, 0.f, 0.f, 0.f};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(r0, qb[0], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(r1, qb[1], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(r2, qb[2], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(r3, qb[3], acc, 0, 0, 0);
      // D[token 4lg+r][head ln]
      if (ln < NQ) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = tile * 16 + 4 * lg + r;
          if (tok < ntok) s_lds[ln][tok] = acc[r] * scale;
        }
      }
    }
  }
  __syncthreads();

  // ---- pass B: split max and exp-sum per head ----
  float mh[NQ], lh[NQ];
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    float m = -__builtin_inff();
    for (int j = tid; j < ntok; j += blockDim.x) m = fmaxf(m, s_lds[h][j]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if (lane == 0) red[h][wave][0] = m;
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < NQ; ++h)
    mh[h] = fmaxf(fmaxf(red[h][0][0], red[h][1][0]), fmaxf(red[h][2][0], red[h][3][0]));
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    float l = 0.f;
    for (int j = tid; j < ntok; j += blockDim.x) {
      const float p = __expf(s_lds[h][j] - mh[h]);
      s_lds[h][j] = p;
      l += p;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) l += __shfl_xor(l, off, 64);
    if (lane == 0) red[h][wave][1] = l;
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < NQ; ++h) lh[h] = red[h][0][1] + red[h][1][1] + red[h][2][1] + red[h][3][1];

  // ---- pass C: P.V.  thread = (8-dim chunk ch, token lane tl) ----
  {
    const int ch = tid & 15, tl = tid >> 4;
    float o[NQ][8];
#pragma unroll
    for (int h = 0; h < NQ; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[h][e] = 0.f;
    // four tokens per step so their codeword gathers are in flight together
    for (int j0 = tl; j0 < ntok; j0 += 64) {
      half8 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = j0 + 16 * u;
        v[u] = rebuild8<D>(value_codes(j < ntok ? j : j0), a.vt, kvh, a.G, S, ch);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = j0 + 16 * u;
        if (j >= ntok) break;
#pragma unroll
        for (int h = 0; h < NQ; ++h) {
          const float p = s_lds[h][j];
#pragma unroll
          for (int e = 0; e < 8; ++e) o[h][e] = fmaf(p, (float)v[u][e], o[h][e]);
        }
      }
    }
#pragma unroll
    for (int h = 0; h < NQ; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float x = o[h][e];
        x += __shfl_xor(x, 16, 64);
        x += __shfl_xor(x, 32, 64);
        o[h][e] = x;
      }
    if ((lane >> 4) == 0) {
#pragma unroll
      for (int h = 0; h < NQ; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) o_red[wave][h][ch * 8 + e] = o[h][e];
    }
  }
  __syncthreads();
  for (int idx = tid; idx < NQ * kHeadDim; idx += blockDim.x) {
    const int h = idx / kHeadDim, i = idx % kHeadDim;
    const float v = o_red[0][h][i] + o_red[1][h][i] + o_red[2][h][i] + o_red[3][h][i];
    const int64_t qh = kvh * NQ + h;
    a.ws_o[((b * a.QH + qh) * a.n_splits + split) * kHeadDim + i] = v;
    if (i == 0) {
      float* ml = a.ws_ml + ((b * a.QH + qh) * a.n_splits + split) * 2;
      ml[0] = ntok > 0 ? mh[h] : -__builtin_inff();
      ml[1] = ntok > 0 ? lh[h] : 0.f;
    }
  }
}

// out[b,qh,:] = sum_s o_s e^{m_s-M} / sum_s l_s e^{m_s-M}
__global__ __launch_bounds__(128) void decode_combine_kernel(DecodeArgs a) {
  const int64_t bq = blockIdx.x;  // b*QH + qh
  const int i = threadIdx.x;
  const float* ml = a.ws_ml + bq * a.n_splits * 2;
  float M = -__builtin_inff();
  for (int s = 0; s < a.n_splits; ++s) M = fmaxf(M, ml[2 * s]);
  float Lsum = 0.f, acc = 0.f;
  for (int s = 0; s < a.n_splits; ++s) {
    const float m = ml[2 * s];
    if (m == -__builtin_inff()) continue;
    const float w = __expf(m - M);
    Lsum += ml[2 * s + 1] * w;
    acc += a.ws_o[(bq * a.n_splits + s) * kHeadDim + i] * w;
  }
  a.out[bq * kHeadDim + i] = (_Float16)(Lsum > 0.f ? acc / Lsum : 0.f);
}

// Rotary table: (cos, sin) of position p and frequency i as the reference's
// rotary module computes them: angle = fp32(p) * inv_freq[i] in fp32,
// cos/sin in fp32, then rounded to fp16.  inv_freq comes from the host.
__global__ void rope_table_kernel(const float* __restrict__ inv_freq, int64_t n_pos,
                                  half2v* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n_pos * 64) return;
  const int64_t p = idx / 64;
  const int i = (int)(idx % 64);
  const float ang = (float)p * inv_freq[i];
  out[idx] = half2v{(_Float16)cosf(ang), (_Float16)sinf(ang)};
}

template <int D, int NQ>
static int launch_decode(const DecodeArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((decode_split_kernel<D, NQ>), dim3((uint32_t)(a.B * a.KVH * a.n_splits)),
                     dim3(256), 0, stream, a);
  JKV_CHECK_LAUNCH();
  hipLaunchKernelGGL(decode_combine_kernel, dim3((uint32_t)(a.B * a.QH)), dim3(kHeadDim), 0,
                     stream, a);
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

}  // namespace jkv

extern "C" {

int jkv_rope_table(const float* inv_freq, int64_t n_pos, void* out, jkv_stream_t stream_) {
  using namespace jkv;
  JKV_CHECK_ARG(n_pos >= 0, "negative position count");
  if (n_pos == 0) return JKV_OK;
  JKV_CHECK_ARG(inv_freq != nullptr && out != nullptr, "null buffer");
  hipLaunchKernelGGL(rope_table_kernel, dim3((uint32_t)ceil_div(n_pos * 64, 256)), dim3(256), 0,
                     (hipStream_t)stream_, inv_freq, n_pos, (half2v*)out);
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

int64_t jkv_decode_workspace_bytes(int64_t B, int64_t QH, int64_t D, int64_t window) {
  const int64_t ns = jkv::ceil_div(window, jkv::kSplitTokens);
  return B * QH * ns * (D + 2) * (int64_t)sizeof(float);
}

int jkv_decode_attention(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                         const uint8_t* k_codes, const uint8_t* v_codes, int64_t code_stride_b,
                         int64_t code_stride_h, int64_t cap, const void* k_tables,
                         const void* v_tables, int64_t B, int64_t QH, int64_t KVH, int64_t G,
                         int64_t d, int64_t S, int64_t K, const int32_t* lengths, int64_t window,
                         const void* rope_table, int64_t rope_len, void* out, void* workspace,
                         int64_t workspace_bytes, jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(B >= 0 && QH > 0 && KVH > 0 && QH % KVH == 0, "invalid head geometry");
  JKV_CHECK_ARG(G * d == kHeadDim, "decode attention supports head_dim 128 (got %lld)",
                (long long)(G * d));
  JKV_CHECK_ARG(K == 256, "decode attention expects 256-entry codebooks");
  JKV_CHECK_ARG(d == 8 || d == 4, "decode attention supports group dims 4 and 8 (got %lld)",
                (long long)d);
  JKV_CHECK_ARG(S >= 1 && S <= 8, "decode attention supports 1..8 stages");
  JKV_CHECK_ARG(window > 0 && cap > 0, "window and cache capacity must be positive");
  JKV_CHECK_ARG(cap >= window, "cache capacity below the attention window");
  JKV_CHECK_ARG(rope_len > 0, "rotary table is empty");
  const int64_t nq = QH / KVH;
  JKV_CHECK_ARG(nq == 1 || nq == 2 || nq == 4 || nq == 8, "GQA group of %lld query heads",
                (long long)nq);
  if (B == 0) return JKV_OK;
  JKV_CHECK_ARG(q && k_codes && v_codes && k_tables && v_tables && lengths && out && rope_table,
                "null buffer");
  const int64_t need = jkv_decode_workspace_bytes(B, QH, kHeadDim, window);
  JKV_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                "decode attention needs %lld bytes of workspace", (long long)need);
  DecodeArgs a = {};
  a.q = (const _Float16*)q;
  a.qsb = q_stride_b; a.qsh = q_stride_h;
  a.kc = k_codes; a.vc = v_codes;
  a.csb = code_stride_b; a.csh = code_stride_h; a.cap = cap;
  a.kt = (const _Float16*)k_tables; a.vt = (const _Float16*)v_tables;
  a.B = B; a.QH = QH; a.KVH = KVH; a.G = G; a.d = d; a.S = S; a.K = K;
  a.lengths = lengths;
  a.window = window;
  a.rope = (const half2v*)rope_table;
  a.rope_len = rope_len;
  a.n_splits = (int32_t)ceil_div(window, kSplitTokens);
  a.ws_o = (float*)workspace;
  a.ws_ml = a.ws_o + B * QH * a.n_splits * kHeadDim;
  a.out = (_Float16*)out;
#define JKV_DEC(DD, NN) \
  if (d == DD && nq == NN) return launch_decode<DD, NN>(a, stream);
  JKV_DEC(8, 1) JKV_DEC(8, 2) JKV_DEC(8, 4) JKV_DEC(8, 8)
  JKV_DEC(4, 1) JKV_DEC(4, 2) JKV_DEC(4, 4) JKV_DEC(4, 8)
#undef JKV_DEC
  return set_error(JKV_ENOTSUP, "unsupported decode geometry");
}

}  // extern "C"
