// Fused decode attention over a packed uint8 GSRQ/CQ code cache.
//
// One workgroup per (batch, kv head, split of the visible window).  K̂ and V̂
// are rebuilt from fp16 codewords on the fly (never written to memory),
// K̂ is rotated at its absolute position with the reference's fp16 RoPE
// sequence, scores for the NQ query heads of the GQA group are reduced
// across the workgroup, and the split's unnormalised (max, sum, out) go to a
// workspace that decode_combine folds into fp16 outputs.
#include "jkv_common.h"

namespace jkv {

static const int kHeadDim = 128;
static const int kSplitTokens = 256;  // tokens per split (workgroup)
static const int kMaxNQ = 8;           // query heads per kv head

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
  float theta;
  int32_t n_splits;
  float* ws_o;   // [B,QH,n_splits,D]
  float* ws_ml;  // [B,QH,n_splits,2]
  _Float16* out;
};

__device__ __forceinline__ float r16(float x) { return (float)(_Float16)x; }

// HF rotary sequence in fp16: (x * cos) + (rotate_half(x) * sin), each
// operation rounded to fp16, with cos/sin rounded to fp16.
__device__ __forceinline__ void rope_pair16(float a, float b, float c16, float s16, float* ra,
                                            float* rb) {
  *ra = r16(r16(a * c16) + r16(-b * s16));
  *rb = r16(r16(b * c16) + r16(a * s16));
}

// inv_freq_i = 1 / theta^(2i/D) computed the way the reference's rotary
// module does (fp32 pow of an fp32 exponent), then the angle p*inv_freq in
// fp32, then cos/sin in fp32 rounded to fp16.
__device__ __forceinline__ float inv_freq(float theta, int i) {
  float e = (float)(2 * i) / (float)kHeadDim;
  return 1.0f / powf(theta, e);
}

// Reconstruct dims [c*8, c*8+8) of one token from its codes (fp32 stage sum,
// one fp16 rounding).
template <int D>
__device__ __forceinline__ void rebuild_chunk(const uint8_t* codes_tok, const _Float16* tab,
                                              int64_t kvh, int64_t G, int64_t S, int c,
                                              float* v) {
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  if (D == 8) {
    const int g = c;
    for (int s = 0; s < (int)S; ++s) {
      const int k = codes_tok[g * S + s];
      const half8 w = *(const half8*)(tab + (((kvh * G + g) * S + s) * 256 + k) * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += (float)w[e];
    }
  } else {  // D == 4: two groups per 8-dim chunk
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int g = 2 * c + half;
      for (int s = 0; s < (int)S; ++s) {
        const int k = codes_tok[g * S + s];
        const half4 w = *(const half4*)(tab + (((kvh * G + g) * S + s) * 256 + k) * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[half * 4 + e] += (float)w[e];
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = r16(acc[e]);
}

template <int D, int NQ>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeArgs a) {
  __shared__ float q_lds[NQ][kHeadDim];
  __shared__ float s_lds[NQ][kSplitTokens];
  __shared__ float red[NQ][4][2];
  __shared__ float o_red[4][NQ][kHeadDim];

  const int tid = threadIdx.x;
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

  // ---- rotated, scaled queries (HF fp16 rope at position L-1) ----
  const float qpos = (float)(L - 1);
  for (int idx = tid; idx < NQ * (kHeadDim / 2); idx += blockDim.x) {
    const int h = idx / (kHeadDim / 2), i = idx % (kHeadDim / 2);
    const int64_t qh = kvh * NQ + h;
    const _Float16* qp = a.q + b * a.qsb + qh * a.qsh;
    const float ang = qpos * inv_freq(a.theta, i);
    const float c16 = r16(cosf(ang)), s16 = r16(sinf(ang));
    float ra, rb;
    rope_pair16((float)qp[i], (float)qp[i + 64], c16, s16, &ra, &rb);
    q_lds[h][i] = ra * scale;
    q_lds[h][i + 64] = rb * scale;
  }
  __syncthreads();

  // ---- pass A: scores.  thread = (token slot ts, quarter qd); the quarter
  // owns 8-dim chunks {qd, qd+4} of the first half and their rotary partners
  // {qd+8, qd+12}.
  {
    const int ts = tid >> 2, qd = tid & 3;
    float qreg[NQ][32];
#pragma unroll
    for (int h = 0; h < NQ; ++h)
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
#pragma unroll
        for (int e = 0; e < 8; ++e) qreg[h][cc * 8 + e] = q_lds[h][(qd + 4 * cc) * 8 + e];
    float ifreq[16];
#pragma unroll
    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
      for (int e = 0; e < 8; ++e) ifreq[cc * 8 + e] = inv_freq(a.theta, (qd + 4 * cc) * 8 + e);
    for (int j = ts; j < ntok; j += 64) {
      const int64_t pos = t0 + j;
      const uint8_t* ct = a.kc + b * a.csb + kvh * a.csh + (pos % a.cap) * a.G * a.S;
      float kv[4][8];
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) rebuild_chunk<D>(ct, a.kt, kvh, a.G, a.S, qd + 4 * cc, kv[cc]);
      float kr[4][8];
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float ang = (float)pos * ifreq[cc * 8 + e];
          const float c16 = r16(cosf(ang)), s16 = r16(sinf(ang));
          rope_pair16(kv[cc][e], kv[cc + 2][e], c16, s16, &kr[cc][e], &kr[cc + 2][e]);
        }
      }
      float sc[NQ];
#pragma unroll
      for (int h = 0; h < NQ; ++h) {
        float acc = 0.f;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc = fmaf(qreg[h][cc * 8 + e], kr[cc][e], acc);
        acc += __shfl_xor(acc, 1, 64);
        acc += __shfl_xor(acc, 2, 64);
        sc[h] = acc;
      }
      if (qd == 0) {
#pragma unroll
        for (int h = 0; h < NQ; ++h) s_lds[h][j] = sc[h];
      }
    }
  }
  __syncthreads();

  // ---- pass B: split max and exp-sum per head ----
  const int wave = tid >> 6, lane = tid & 63;
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
    for (int j = tl; j < ntok; j += 16) {
      const int64_t pos = t0 + j;
      const uint8_t* ct = a.vc + b * a.csb + kvh * a.csh + (pos % a.cap) * a.G * a.S;
      float v[8];
      rebuild_chunk<D>(ct, a.vt, kvh, a.G, a.S, ch, v);
#pragma unroll
      for (int h = 0; h < NQ; ++h) {
        const float p = s_lds[h][j];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] = fmaf(p, v[e], o[h][e]);
      }
    }
    // reduce over token lanes: within the wave over lane bits 4,5, then waves
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

int64_t jkv_decode_workspace_bytes(int64_t B, int64_t QH, int64_t D, int64_t window) {
  const int64_t ns = jkv::ceil_div(window, jkv::kSplitTokens);
  return B * QH * ns * (D + 2) * (int64_t)sizeof(float);
}

int jkv_decode_attention(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                         const uint8_t* k_codes, const uint8_t* v_codes, int64_t code_stride_b,
                         int64_t code_stride_h, int64_t cap, const void* k_tables,
                         const void* v_tables, int64_t B, int64_t QH, int64_t KVH, int64_t G,
                         int64_t d, int64_t S, int64_t K, const int32_t* lengths, int64_t window,
                         float rope_theta, void* out, void* workspace, int64_t workspace_bytes,
                         jkv_stream_t stream_) {
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
  JKV_CHECK_ARG(rope_theta > 0.f, "rope theta must be positive");
  const int64_t nq = QH / KVH;
  JKV_CHECK_ARG(nq == 1 || nq == 2 || nq == 4 || nq == 8, "GQA group of %lld query heads",
                (long long)nq);
  if (B == 0) return JKV_OK;
  JKV_CHECK_ARG(q && k_codes && v_codes && k_tables && v_tables && lengths && out,
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
  a.theta = rope_theta;
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
