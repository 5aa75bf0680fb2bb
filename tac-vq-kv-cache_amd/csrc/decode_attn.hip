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
#include <mutex>

#include "jkv_common.h"
#include "rotary.h"

namespace jkv {

static const int kHeadDim = 128;
static const int kSplitTokens = 256;  // tokens per split (workgroup)
static const int kWinSplitTokens = 512;  // tokens per split over a decoded window (streamed rows)
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
  const _Float16* rope;  // [rope_len][2][64]: cos row, sin row (fp16)
  int64_t rope_len;
  int32_t n_splits;
  int32_t split_tokens;  // tokens per split
  float* ws_o;   // [B,QH,n_splits,D]
  float* ws_ml;  // [B,QH,n_splits,2]
  _Float16* out;
  // decode with append (decode_g8_kernel<..., true>): the raw fp16 K/V of
  // the token at position lengths[b]-1, [B][KVH][128] with element strides,
  // encoded into slot (lengths[b]-1) % cap of kc_out/vc_out (= kc/vc)
  const _Float16* knew;
  const _Float16* vnew;
  int64_t nsb, nsh;
  uint8_t* kc_out;
  uint8_t* vc_out;
};


// fp16 words of dims [8*c8, 8*c8+8) of one token: fp16(sum_s fp32(word_s)).
// The sum of two fp16 words is exact in fp32 or too small to move the fp16
// rounding, so for S = 2 one fp16 add gives the same bits; S > 2 sums in fp32.
// D = 128 is one full-vector group (G = 1): the chunk is the 16-byte slice
// c8 of every stage's 256-byte codeword, read from L2.  D = 0 reads a decoded
// fp16 window instead of codes (the 256-byte row is the token's record).
template <int D>
__device__ __forceinline__ half8 rebuild8(const uint8_t* codes_tok, const _Float16* tab,
                                          int64_t kvh, int64_t G, int S, int c8) {
  if (D == 0) {
    // decoded window: the token's "record" is its fp16 row of 128 values
    return *(const half8*)(codes_tok + 16 * c8);
  } else if (D == 128) {
    const _Float16* base = tab + kvh * S * 256 * 128 + 8 * c8;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < S; ++s) {
      const half8 w = *(const half8*)(base + (s * 256 + codes_tok[s]) * 128);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += (float)w[e];
    }
    half8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (_Float16)acc[e];
    return r;
  } else if (D == 8) {
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

// Full-vector codebooks (one 128-dim group) with SS stages known at compile
// time.  gather_sum adds up N items of SS 16-byte codeword slices each (8
// dims of one token) and hands item i to done(i, acc) with acc = the fp32
// sum over stages s of slice(i, s), in stage order.  The slices stream in
// groups of kGatherStages, one group ahead of the group being summed, so two
// groups are in flight per lane.  Each add is one v_fma_mix_f32 taking the
// fp16 word as it is: x * 1 + acc rounds once, exactly as the fp32 add of the
// converted word.
constexpr int kGatherStages = 4;

template <int N, int SS, typename Slice, typename Done>
__device__ __forceinline__ void gather_sum(Slice slice, Done done) {
  constexpr int GS = kGatherStages;
  static_assert(SS % GS == 0, "whole groups of stages");
  constexpr int G = SS / GS, T = N * G;
  _Float16 one = (_Float16)1.f;
  asm volatile("" : "+v"(one));  // an opaque 1, so the fma is not folded back into cvt + add
  float acc[8];
  half8 buf[2][GS];
  auto issue = [&](int t, half8 (&b)[GS]) {
#pragma unroll
    for (int u = 0; u < GS; ++u) b[u] = slice(t / G, GS * (t % G) + u);
  };
  issue(0, buf[0]);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if (t + 1 < T) issue(t + 1, buf[(t + 1) & 1]);
    __builtin_amdgcn_sched_barrier(0);
    if (t % G == 0)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
    for (int u = 0; u < GS; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf((float)buf[t & 1][u][e], (float)one, acc[e]);
    if (t % G == G - 1) done(t / G, acc);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// one 16-byte codeword slice of a stage table (SS x 256 x 128 fp16, 64 KiB a
// stage) held in a buffer resource: the stage offset is uniform (scalar), the
// code and chunk a 32-bit lane offset, and a read past the resource's size
// returns zeros
__device__ __forceinline__ half8 table_slice(__amdgpu_buffer_rsrc_t tab, int stage, uint32_t code, int c8) {
  const auto w = __builtin_amdgcn_raw_buffer_load_b128(tab, (int)(code * 256u + 16u * (uint32_t)c8), stage * 65536, 0);
  return __builtin_bit_cast(half8, w);
}

// the stage-s code of a token whose SS code bytes are held as dwords
template <int SS>
__device__ __forceinline__ uint32_t stage_code(const uint32_t (&cw)[SS / 4], int s) {
  return __builtin_amdgcn_ubfe(cw[s >> 2], 8u * (uint32_t)(s & 3), 8u);
}

// SS: the stage count of full-vector codebooks (D = 128) when it is 16 or
// 32, else 0 (a.S at run time).
template <int D, int NQ, int SS>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeArgs a) {
  __shared__ _Float16 q_lds[NQ][kHeadDim];
  constexpr int kTok = D == 0 ? kWinSplitTokens : kSplitTokens;
  __shared__ float s_lds[NQ][kTok];
  __shared__ float red[NQ][4][2];
  __shared__ float o_red[4][NQ][kHeadDim];
  // the split's K and V code records (up to 64 bytes per token), fetched once
  // (a decoded window, D = 0, reads its rows from global memory instead)
  constexpr int kRecLds = D == 0 ? 16 : kTok * (SS != 0 ? SS : kMaxCodeBytes);
  __shared__ __align__(16) uint8_t kc_lds[kRecLds];
  __shared__ __align__(16) uint8_t vc_lds[kRecLds];
  // SS != 0 and the decoded window (D = 0): each wave's rotated 16-key K
  // tile, built in the line layout and read back in the MFMA layout (rows
  // padded to 272 bytes)
  constexpr bool kLineK = SS != 0 || D == 0;
  constexpr int kKRow = kHeadDim + 8;
  __shared__ __align__(16) _Float16 kt_lds[kLineK ? 4 : 1][kLineK ? 16 * kKRow : 8];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int lg = lane >> 4, ln = lane & 15;
  // logical block: split fastest, then batch row, then kv head, so that the
  // blocks of one kv head (its codebooks) sit on one XCD and share its L2
  const uint32_t bid = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t split = bid % (uint32_t)a.n_splits;
  const int64_t b = (bid / (uint32_t)a.n_splits) % (uint32_t)a.B;
  const int64_t kvh = bid / ((uint32_t)a.n_splits * (uint32_t)a.B);
  const int64_t L = a.lengths[b];
  const int64_t n_vis = L < a.window ? L : a.window;
  const int64_t start = L - n_vis;
  const int64_t t0 = start + split * kTok;
  int64_t t1 = t0 + kTok;
  if (t1 > L) t1 = L;
  const int ntok = t1 > t0 ? (int)(t1 - t0) : 0;
  const float scale = 1.0f / sqrtf((float)kHeadDim);
  const int S = (int)a.S;
  const int64_t code_bytes = a.G * a.S;

  // ---- rotated queries (fp16 rotary at position L-1) ----
  if (L > 0) {
    const _Float16* qrow = a.rope + ((L - 1) < a.rope_len ? (L - 1) : a.rope_len - 1) * kRopeRow;
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
  const bool codes_in_lds = D != 0 && code_bytes <= kMaxCodeBytes && (code_bytes % 16) == 0 &&
                            code_bytes * kTok <= kRecLds;
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
    // a tile's key rows and rotary rows, loaded one tile ahead of their use
    struct KTile {
      half8 k[4], c0, s0, c1, s1;
    };
    auto load_ktile = [&](int tile, KTile& kt) {
      const int tt = tile * 16 + ln;
      const bool valid = tt < ntok;
      const int64_t pos = valid ? t0 + tt : t0;
      const uint8_t* ct = key_codes(valid ? tt : 0);
#pragma unroll
      for (int q = 0; q < 4; ++q) kt.k[q] = rebuild8<D>(ct, a.kt, kvh, a.G, S, lg + 4 * q);
      // the host sizes the table past every length; the clamp only keeps a
      // misuse from reading out of bounds
      const _Float16* trow = a.rope + (pos < a.rope_len ? pos : a.rope_len - 1) * kRopeRow;
      load_trig8(trow, 8 * lg, &kt.c0, &kt.s0);
      load_trig8(trow, 8 * (lg + 4), &kt.c1, &kt.s1);
    };
    if constexpr (kLineK) {
      // The line layout: lane (t8, c8) = (lane / 8, lane % 8) holds dims
      // [8c8, 8c8 + 8) and their rotary partners [64 + 8c8, ..) of keys t8
      // and 8 + t8 of a 16-key tile, so each 16-byte load covers whole
      // 128-byte lines of eight rows (codeword rows, or the decoded window's
      // K rows): half the lines per load of the MFMA layout, and the vector
      // memory path pays per line.  The rotated rows pass through a per-wave
      // LDS tile into the MFMA layout, so the products are those of the
      // path below.
      const int t8 = lane >> 3, c8 = lane & 7;
      _Float16* const ktile = kt_lds[kLineK ? wave : 0];
      struct LineTile {
        half8 k[2][2], cs[2], sn[2];  // [key half][dims 8c8.. | 64 + 8c8..]
        bool valid[2];
      };
      // the tile's rotary rows and validity; key records for the gather
      auto tile_keys = [&](int tile, LineTile& w, const uint8_t* (&ct)[2]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int tt = tile * 16 + 8 * h + t8;
          w.valid[h] = tt < ntok;
          const int64_t pos = w.valid[h] ? t0 + tt : t0;
          ct[h] = key_codes(w.valid[h] ? tt : 0);
          const _Float16* trow = a.rope + (pos < a.rope_len ? pos : a.rope_len - 1) * kRopeRow;
          load_trig8(trow, 8 * c8, &w.cs[h], &w.sn[h]);
        }
      };
      auto tile_scores = [&](int tile, const LineTile& w) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          half8 r0, r1;
          rope16(w.k[h][0], w.k[h][1], w.cs[h], w.sn[h], &r0, &r1);
          if (!w.valid[h]) {
            r0 = half8{}; r1 = half8{};
          }
          _Float16* row = ktile + (8 * h + t8) * kKRow;
          *(half8*)(row + 8 * c8) = r0;
          *(half8*)(row + 64 + 8 * c8) = r1;
        }
        // MFMA layout: lane (ln, lg) holds chunk lg + 4m of key ln for MFMA m
        half8 r[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) r[m] = *(const half8*)(ktile + ln * kKRow + 8 * (lg + 4 * m));
        float4v acc = {0.f, 0.f, 0.f, 0.f};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(r[0], qb[0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(r[1], qb[1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(r[2], qb[2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(r[3], qb[3], acc, 0, 0, 0);
        if (ln < NQ) {
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const int tok = tile * 16 + 4 * lg + rr;
            if (tok < ntok) s_lds[ln][tok] = acc[rr] * scale;
          }
        }
      };
      if constexpr (D == 0) {
        // decoded window: the rows stream from HBM, one tile ahead
        auto load_rows = [&](int tile, LineTile& w) {
          const uint8_t* ct[2];
          tile_keys(tile, w, ct);
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            w.k[h][0] = *(const half8*)(ct[h] + 16 * c8);
            w.k[h][1] = *(const half8*)(ct[h] + 16 * (c8 + 8));
          }
        };
        LineTile nxt;
        if (wave < ntiles) load_rows(wave, nxt);
        for (int tile = wave; tile < ntiles; tile += 4) {
          const LineTile cur = nxt;
          if (tile + 4 < ntiles) load_rows(tile + 4, nxt);
          tile_scores(tile, cur);
        }
      } else {
        // full-vector codebooks with 16 or 32 stages: each chunk is the fp32
        // stage sum in stage order rounded to fp16; no tile runs ahead (the
        // slice loads in flight fill the register budget)
        const __amdgpu_buffer_rsrc_t krsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(a.kt + kvh * SS * 256 * 128), (short)0, SS * 65536, 0x00020000);
        for (int tile = wave; tile < ntiles; tile += 4) {
          LineTile w;
          const uint8_t* ct[2];
          tile_keys(tile, w, ct);
          uint32_t cw[2][SS != 0 ? SS / 4 : 1];
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < SS / 4; ++i) cw[h][i] = ((const uint32_t*)ct[h])[i];
          gather_sum<4, SS>([&](int i, int st) {
            return table_slice(krsrc, st, stage_code<SS>(cw[i >> 1], st), c8 + 8 * (i & 1));
          }, [&](int i, const float (&acc)[8]) {
#pragma unroll
            for (int e = 0; e < 8; ++e) w.k[i >> 1][i & 1][e] = (_Float16)acc[e];
          });
          tile_scores(tile, w);
        }
      }
    }
    KTile nxt;
    if (!kLineK && wave < ntiles) load_ktile(wave, nxt);
    for (int tile = wave; !kLineK && tile < ntiles; tile += 4) {
      const KTile cur = nxt;
      if (tile + 4 < ntiles) load_ktile(tile + 4, nxt);
      const bool valid = tile * 16 + ln < ntok;
      half8 r0, r1, r2, r3;
      rope16(cur.k[0], cur.k[2], cur.c0, cur.s0, &r0, &r2);
      rope16(cur.k[1], cur.k[3], cur.c1, cur.s1, &r1, &r3);
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
    // four tokens per step so their loads are in flight together, and the
    // next step's four go out before this step's products
    half8 vn[4];
    auto load_v = [&](int j0, half8 (&v)[4]) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = j0 + 16 * u;
        v[u] = rebuild8<D>(value_codes(j < ntok ? j : j0), a.vt, kvh, a.G, S, ch);
      }
    };
    if constexpr (SS != 0) {
      // full-vector codebooks with 16 or 32 stages: two tokens per gather_sum
      // (the slice loads in flight fill the register budget), the products in
      // token order as below
      const __amdgpu_buffer_rsrc_t vrsrc = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(a.vt + kvh * SS * 256 * 128), (short)0, SS * 65536, 0x00020000);
      for (int j = tl; j < ntok; j += 32) {
        // tokens j and j + 16 (the second past the split reads the first's
        // codes and is not used)
        const int j2 = j + 16 < ntok ? j + 16 : j;
        uint32_t cw[2][SS / 4];
#pragma unroll
        for (int i = 0; i < SS / 4; ++i) {
          cw[0][i] = ((const uint32_t*)value_codes(j))[i];
          cw[1][i] = ((const uint32_t*)value_codes(j2))[i];
        }
        gather_sum<2, SS>([&](int u, int st) {
          return table_slice(vrsrc, st, stage_code<SS>(cw[u], st), ch);
        }, [&](int u, const float (&acc)[8]) {
          if (u == 1 && j + 16 >= ntok) return;
          const int jj = j + 16 * u;
          half8 v;
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = (_Float16)acc[e];
#pragma unroll
          for (int h = 0; h < NQ; ++h) {
            const float p = s_lds[h][jj];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[h][e] = fmaf(p, (float)v[e], o[h][e]);
          }
        });
      }
    }
    if (SS == 0 && tl < ntok) load_v(tl, vn);
    for (int j0 = tl; SS == 0 && j0 < ntok; j0 += 64) {
      half8 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = vn[u];
      if (j0 + 64 < ntok) load_v(j0 + 64, vn);
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

// ---------------------------------------------------------------------------
// LDS-table decode: one 512-thread workgroup (8 waves) per (kv head, batch
// row, split of up to 2048 visible tokens).  The kv head's fp16 tables
// ([G][S][K][d], 128 KiB at G2) are staged in LDS so every codeword gather is
// an LDS read, and the split's code records stream through LDS in coalesced,
// double-buffered 256-token chunks.  Wave w owns 32-key block w of every chunk
// in both phases, so its scores never leave registers:
//   K phase  K tables in LDS; per 16-key tile a lane rebuilds 32 dims of one
//            key (four 8-dim chunks), rotates them with the reference's fp16
//            rotary, and four v_mfma_f32_16x16x32_f16 give the tile's scores
//            for every query head of the GQA group (Sᵀ = K̂ Qᵀ);
//   softmax  split max and exp-sum per head; fp16 P in B-operand order;
//   V phase  V tables in LDS; per 16-dim slice the wave rebuilds V̂ of its
//            32 keys, transposes it through a small per-wave LDS tile, and one
//            MFMA accumulates Oᵀ += V̂ᵀ Pᵀ (contraction slots of the two 16-key
//            tiles interleaved to match the Sᵀ accumulator layout).
// The split's (max, sum, out) go to decode_combine_kernel.

static const int kLdsThreads = 512;
static const int kLdsWaves = kLdsThreads / 64;
static const int kLdsMaxSplit = 2048;      // 8 chunks: one register slot per chunk
static const int kLdsChunk = 256;          // tokens per chunk: one 32-key block per wave
static const int kLdsCodeBytes = 32;       // code-record bytes per token the buffer holds
static const int kLdsK = 256;              // codewords per stage
static const int kStgRows = 32;            // V̂ᵀ staging: 32 dims (two 16-dim slices) ...
static const int kStgStride = 36;          // ... x 32 keys, row stride 72 B (conflict-free b32 writes)

// Code bytes of 8-dim chunk c8 of one token record (the chunk's 8/DG groups
// x S stages are contiguous and aligned to their size).
template <int DG, int S>
__device__ __forceinline__ uint32_t chunk_codes(const uint8_t* rec, int c8) {
  constexpr int n = (8 / DG) * S;
  const uint8_t* p = rec + c8 * n;
  if constexpr (n == 4) return *(const uint32_t*)p;
  if constexpr (n == 2) return *(const uint16_t*)p;
  return *p;
}

// fp16 words of dims [8*c8, 8*c8+8) of one token from LDS tables [G][S][256][DG]
// (S <= 2): fp16(fp32(c1) + fp32(c2)) equals the fp16 add of the two words.
template <int DG, int S>
__device__ __forceinline__ half8 rebuild8_lds(const _Float16* tab, uint32_t codes, int c8) {
  if constexpr (DG == 8) {
    const _Float16* base = tab + c8 * (S * kLdsK * 8);
    const half8 w0 = *(const half8*)(base + (codes & 0xffu) * 8);
    if constexpr (S == 1) return w0;
    const half8 w1 = *(const half8*)(base + kLdsK * 8 + ((codes >> 8) & 0xffu) * 8);
    return w0 + w1;
  } else {
    half4 r[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const _Float16* base = tab + (2 * c8 + h) * (S * kLdsK * 4);
      const uint32_t c = codes >> (8 * h * S);
      const half4 w0 = *(const half4*)(base + (c & 0xffu) * 4);
      if constexpr (S == 1) {
        r[h] = w0;
      } else {
        const half4 w1 = *(const half4*)(base + kLdsK * 4 + ((c >> 8) & 0xffu) * 4);
        r[h] = w0 + w1;
      }
    }
    return half8{r[0][0], r[0][1], r[0][2], r[0][3], r[1][0], r[1][1], r[1][2], r[1][3]};
  }
}

// Codes of the four 8-dim chunks 4q + sel (q = 0..3) of one token, from its
// whole code record held as dwords w[].  A chunk has n = (8/DG)*S code bytes
// (1, 2 or 4) at byte (4q + sel)*n = 4*(q*n) + sel*n of the record.
template <int DG, int S>
__device__ __forceinline__ void record_codes(const uint32_t* w, int sel, uint32_t (&out)[4]) {
  constexpr int n = (8 / DG) * S;
  // v_perm_b32 picks bytes of the 8-byte pair (hi:lo) by a per-lane selector
  // (selector byte 0x0c yields zero), so no lane indexes an array
  const uint32_t off = (uint32_t)(sel * n) & 7u;  // first code byte within its dword pair
  const uint32_t pick = n == 1   ? (off | 0x0c0c0c00u)
                        : n == 2 ? (off | ((off + 1) << 8) | 0x0c0c0000u)
                                 : (off | ((off + 1) << 8) | ((off + 2) << 16) | ((off + 3) << 24));
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if constexpr (n == 4) {
      // dword 4q + sel: pair (4q, 4q+1) or (4q+2, 4q+3), then the pair's half
      const uint32_t p01 = __builtin_amdgcn_perm(w[4 * q + 1], w[4 * q], pick);
      const uint32_t p23 = __builtin_amdgcn_perm(w[4 * q + 3], w[4 * q + 2], pick);
      const uint32_t m = 0u - (((uint32_t)sel >> 1) & 1u);
      out[q] = (p01 & ~m) | (p23 & m);
    } else if constexpr (n == 2) {
      // bytes 2 sel, 2 sel + 1 of the pair (w[2q], w[2q+1])
      out[q] = __builtin_amdgcn_perm(w[2 * q + 1], w[2 * q], pick);
    } else {
      // byte sel of w[q] (sel < 4)
      out[q] = __builtin_amdgcn_perm(w[q], w[q], pick);
    }
  }
}

// a token's whole code record (kCb a multiple of 16 bytes, 16-byte aligned in LDS)
template <int kCb>
__device__ __forceinline__ void read_record(const uint8_t* rec, uint32_t (&w)[kCb / 4]) {
#pragma unroll
  for (int i = 0; i < kCb / 16; ++i) {
    const uint4 v = *(const uint4*)(rec + 16 * i);
    w[4 * i] = v.x;
    w[4 * i + 1] = v.y;
    w[4 * i + 2] = v.z;
    w[4 * i + 3] = v.w;
  }
}

// (a[e], b[e]) as one 32-bit word, e = 0..7
__device__ __forceinline__ uint32_t pair_halves(half8 a, half8 b, int e) {
  const half2v h = {a[e], b[e]};
  return __builtin_bit_cast(uint32_t, h);
}

template <int DG, int NQ, int S>
__global__ __launch_bounds__(kLdsThreads) void decode_lds_kernel(DecodeArgs a) {
  extern __shared__ __align__(16) unsigned char dyn[];
  constexpr int tab_halves = kHeadDim * S * kLdsK;  // G * S * K * DG with G * DG = 128
  constexpr int kSlots = kLdsMaxSplit / kLdsChunk;
  constexpr int kCb = (kHeadDim / DG) * S;  // code bytes per token (16 or 32)
  const int cb = kCb;
  _Float16* tab = (_Float16*)dyn;
  uint8_t* cbuf = dyn + (size_t)tab_halves * 2;                           // [chunk][32]
  _Float16* stg_all = (_Float16*)(cbuf + kLdsChunk * kLdsCodeBytes);      // [waves][32][36]
  float* red = (float*)(stg_all + kLdsWaves * kStgRows * kStgStride);     // [2][waves][NQ]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  _Float16* stg = stg_all + wave * kStgRows * kStgStride;
  // logical block: split fastest, then batch row, then kv head (one kv head's
  // tables stay in one XCD's L2)
  const uint32_t bid = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t split = bid % (uint32_t)a.n_splits;
  const int64_t b = (bid / (uint32_t)a.n_splits) % (uint32_t)a.B;
  const int64_t kvh = bid / ((uint32_t)a.n_splits * (uint32_t)a.B);
  const int64_t L = a.lengths[b];
  const int64_t n_vis = L < a.window ? L : a.window;
  const int64_t t0 = L - n_vis + split * a.split_tokens;
  int64_t t1 = t0 + a.split_tokens;
  if (t1 > L) t1 = L;
  const int ntok = t1 > t0 ? (int)(t1 - t0) : 0;
  const int nchunks = (ntok + kLdsChunk - 1) / kLdsChunk;
  const int64_t cbase = b * a.csb + kvh * a.csh;
  const uint32_t cap = (uint32_t)a.cap;
  const uint32_t slot0 = (uint32_t)(t0 % a.cap);  // ring slot of the split's first token
  const float scale2 = 1.4426950408889634f / sqrtf((float)kHeadDim);  // log2(e)/sqrt(D)
  const int64_t rope_last = a.rope_len - 1;
  auto rope_row = [&](int64_t pos) -> const _Float16* {
    return a.rope + (pos < rope_last ? pos : rope_last) * kRopeRow;
  };
  // one 16-byte piece of chunk c's code records: token i = tid*16/cb
  const int pieces = kLdsChunk * cb / 16;
  auto fetch_codes = [&](const uint8_t* codes, int c) -> uint4 {
    uint4 v = {0u, 0u, 0u, 0u};
    if (tid < pieces) {
      const int i = tid * 16 / cb, part = tid * 16 % cb;
      const int t = c * kLdsChunk + i;
      if (t < ntok) {
        uint32_t slot = slot0 + (uint32_t)t;
        if (slot >= cap) slot -= cap;
        v = *(const uint4*)(codes + cbase + (int64_t)slot * cb + part);
      }
    }
    return v;
  };
  auto store_codes = [&](uint4 v) {
    if (tid < pieces) {
      const int i = tid * 16 / cb, part = tid * 16 % cb;
      *(uint4*)(cbuf + i * cb + part) = v;
    }
  };
  // Tables go global -> LDS directly (global_load_lds_dwordx4: lane i of a
  // wave lands at the wave's LDS base + 16 i), 8 KiB per workgroup-wide
  // step.  The workgroups of one kv head (one XCD) copy the same tables at the
  // same time; each starts at a different slice so the reads spread over the
  // L2 channels.  The caller waits (vmcnt) and synchronises before use.
  const int rot = (int)(bid % ((uint32_t)a.n_splits * (uint32_t)a.B));
  auto load_tables = [&](const _Float16* src_tab) {
    const uint4* src = (const uint4*)(src_tab + kvh * (int64_t)tab_halves);
    uint4* dst = (uint4*)tab;
    constexpr int n = tab_halves / 8;
    static_assert(n % kLdsThreads == 0, "tables are whole 8 KiB slices");
    constexpr int per = n / kLdsThreads;
#pragma unroll
    for (int u = 0; u < per; ++u) {
      const int uu = (u + rot) % per;
      __builtin_amdgcn_global_load_lds(
          (const void __attribute__((address_space(1)))*)(src + tid + uu * kLdsThreads),
          (void __attribute__((address_space(3)))*)(dst + uu * kLdsThreads + wave * 64), 16, 0, 0);
    }
  };
  // rotary rows of the two 16-key tiles of the wave's block in chunk c
  auto fetch_trig = [&](int c, half8 (&tg)[2][4]) {
#pragma unroll
    for (int tl = 0; tl < 2; ++tl) {
      const int tk = c * kLdsChunk + 32 * wave + 16 * tl + ln;
      const _Float16* tr = rope_row(t0 + (tk < ntok ? tk : 0));
      load_trig8(tr, 8 * lg, &tg[tl][0], &tg[tl][1]);
      load_trig8(tr, 32 + 8 * lg, &tg[tl][2], &tg[tl][3]);
    }
  };

  // ---- the K tables and the first chunk's code records into LDS; the other
  // chunks' records (one 16-byte piece per thread per chunk) load into
  // registers once the K phase has started ----
  uint4 kcodes[kSlots];
  load_tables(a.kt);
  kcodes[0] = nchunks > 0 ? fetch_codes(a.kc, 0) : uint4{0u, 0u, 0u, 0u};
  if (nchunks > 0) store_codes(kcodes[0]);
  // ---- rotated queries at position L-1: B operand, column ln = head ----
  const half8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
  half8 qb[4];
  {
    const int64_t head = kvh * NQ + (ln < NQ ? ln : 0);
    const _Float16* qp = a.q + b * a.qsb + head * a.qsh;
    const _Float16* tr = rope_row(L > 0 ? L - 1 : 0);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int d0 = 32 * c + 8 * lg;
      half8 x0, x1, cs, sn, r0, r1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x0[e] = qp[d0 + e];
        x1[e] = qp[d0 + 64 + e];
      }
      load_trig8(tr, d0, &cs, &sn);
      rope16(x0, x1, cs, sn, &r0, &r1);
      qb[c] = ln < NQ ? r0 : zero8;
      qb[c + 2] = ln < NQ ? r1 : zero8;
    }
  }
  half8 trig[2][4];
  if (nchunks > 0) fetch_trig(0, trig);
  __builtin_amdgcn_s_waitcnt(0);  // the tables' direct-to-LDS loads have landed
  __syncthreads();
#pragma unroll
  for (int c = 1; c < kSlots; ++c)
    kcodes[c] = c < nchunks ? fetch_codes(a.kc, c) : uint4{0u, 0u, 0u, 0u};

  // ---- K phase.  Lane (key ln of a 16-key tile, lane group lg) owns 8-dim
  // chunks 4q+lg (q = 0..3) = MFMA contraction slice q; chunks lg/lg+8 and
  // lg+4/lg+12 are rotary partners.  sc[c][tl][e]: score of key 4lg+e of tile
  // tl of the wave's block in chunk c, for head ln ----
  float4v sc[kSlots][2];
#pragma unroll
  for (int c = 0; c < kSlots; ++c) {
    sc[c][0] = float4v{-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
    sc[c][1] = sc[c][0];
    if (c >= nchunks) continue;
    const bool more = c + 1 < nchunks;
    half8 tnext[2][4];
    if (more) fetch_trig(c + 1, tnext);
    // both tiles' key records (the four lanes of a key read the same bytes),
    // so tile 1's gathers can go out while tile 0 computes
    uint32_t wrec[2][kCb / 4];
#pragma unroll
    for (int tl = 0; tl < 2; ++tl) read_record<kCb>(cbuf + (32 * wave + 16 * tl + ln) * kCb, wrec[tl]);
#pragma unroll
    for (int tl = 0; tl < 2; ++tl) {
      const int kb = 32 * wave + 16 * tl;  // first key of the tile in the chunk
      // all eight gathers of the lane's four chunks at once
      uint32_t cc[4];
      record_codes<DG, S>(wrec[tl], lg, cc);
      half8 k[4];
      if constexpr (DG == 8) {
        // every stage word of the four chunks first, then the sums (left to
        // itself the scheduler waits for each pair before issuing the next)
        half8 g[4][S];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const _Float16* base = tab + (4 * q + lg) * (S * kLdsK * 8);
#pragma unroll
          for (int st = 0; st < S; ++st)
            g[q][st] = *(const half8*)(base + st * kLdsK * 8 + ((cc[q] >> (8 * st)) & 0xffu) * 8);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < 4; ++q) k[q] = S == 2 ? g[q][0] + g[q][S - 1] : g[q][0];
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) k[q] = rebuild8_lds<DG, S>(tab, cc[q], 4 * q + lg);
      }
      half8 r[4];
      rope16(k[0], k[2], trig[tl][0], trig[tl][1], &r[0], &r[2]);
      rope16(k[1], k[3], trig[tl][2], trig[tl][3], &r[1], &r[3]);
      float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(r[q], qb[q], acc, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = c * kLdsChunk + kb + 4 * lg + e;
        sc[c][tl][e] = (ln < NQ && key < ntok) ? acc[e] * scale2 : -__builtin_inff();
      }
    }
    __syncthreads();  // chunk c's records are consumed
    if (more) {
      store_codes(kcodes[c + 1 < kSlots ? c + 1 : c]);
#pragma unroll
      for (int tl = 0; tl < 2; ++tl)
#pragma unroll
        for (int u = 0; u < 4; ++u) trig[tl][u] = tnext[tl][u];
    }
    __syncthreads();
  }

  // the K phase's last barrier has passed: every wave is done with the K
  // tables, so the V tables and the first chunk of V records load while the
  // softmax runs
  load_tables(a.vt);
  uint4 vcodes[kSlots];
  vcodes[0] = nchunks > 0 ? fetch_codes(a.vc, 0) : uint4{0u, 0u, 0u, 0u};

  // ---- split max and exp-sum per head (lanes ln < NQ carry head ln) ----
  float mx = -__builtin_inff();
#pragma unroll
  for (int c = 0; c < kSlots; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) mx = fmaxf(mx, fmaxf(sc[c][0][e], sc[c][1][e]));
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (lg == 0 && ln < NQ) red[wave * NQ + ln] = mx;
  __syncthreads();
  float mh[NQ];
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    float m = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < kLdsWaves; ++w) m = fmaxf(m, red[w * NQ + h]);
    mh[h] = m;
  }
  float m_lane = 0.f;
#pragma unroll
  for (int h = 0; h < NQ; ++h) m_lane = ln == h ? mh[h] : m_lane;
  const float m_use = m_lane == -__builtin_inff() ? 0.f : m_lane;
  half8 pf[kSlots];
  float lsum = 0.f;
#pragma unroll
  for (int c = 0; c < kSlots; ++c) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float pa = __builtin_amdgcn_exp2f(sc[c][0][e] - m_use);
      const float pb = __builtin_amdgcn_exp2f(sc[c][1][e] - m_use);
      lsum += pa + pb;
      pf[c][e] = (_Float16)pa;
      pf[c][e + 4] = (_Float16)pb;
    }
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  if (lg == 0 && ln < NQ) red[kLdsWaves * NQ + wave * NQ + ln] = lsum;
  __syncthreads();
  float lh[NQ];
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < kLdsWaves; ++w) l += red[kLdsWaves * NQ + w * NQ + h];
    lh[h] = l;
  }

  // ---- the V tables have landed; the first chunk of V codes into LDS, the
  // other chunks' records into registers behind the V phase ----
  if (nchunks > 0) store_codes(vcodes[0]);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
#pragma unroll
  for (int c = 1; c < kSlots; ++c)
    vcodes[c] = c < nchunks ? fetch_codes(a.vc, c) : uint4{0u, 0u, 0u, 0u};

  // ---- V phase, two 16-dim slices (4 chunks of 8 dims) at a time: lane
  // (chunk 4dp + (lane>>4), keys 2kp and 2kp+1 of the block, kp = lane&15)
  // rebuilds 16 values, writes them transposed as (key pair) words into the
  // wave's staging tile, and lane (dim ln, lg) of slice dt reads keys
  // {4lg..4lg+3} and {16+4lg..16+4lg+3} of its dim as the A operand ----
  float4v o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = float4v{0.f, 0.f, 0.f, 0.f};
  const int vq = lane >> 4, kp = lane & 15;
#pragma unroll
  for (int c = 0; c < kSlots; ++c) {
    if (c >= nchunks) continue;
    const bool more = c + 1 < nchunks;
    const int kb0 = 32 * wave + 2 * kp;
    const bool ok0 = c * kLdsChunk + kb0 < ntok, ok1 = c * kLdsChunk + kb0 + 1 < ntok;
    // both keys' records once per chunk; slice dp+1's gathers go out before
    // slice dp's transpose
    uint32_t w0[kCb / 4], w1[kCb / 4];
    read_record<kCb>(cbuf + kb0 * kCb, w0);
    read_record<kCb>(cbuf + (kb0 + 1) * kCb, w1);
    uint32_t cc0[4], cc1[4];
    record_codes<DG, S>(w0, vq, cc0);
    record_codes<DG, S>(w1, vq, cc1);
    // gathers run for every key (a record past the split's tokens still holds
    // code bytes, so the reads stay inside the tables) and the sums of keys
    // past it are then zeroed: selects, not branches around the reads
    half8 vn0 = rebuild8_lds<DG, S>(tab, cc0[0], vq);
    half8 vn1 = rebuild8_lds<DG, S>(tab, cc1[0], vq);
#pragma unroll
    for (int dp = 0; dp < 4; ++dp) {
      const half8 v0 = ok0 ? vn0 : zero8, v1 = ok1 ? vn1 : zero8;
      if (dp + 1 < 4) {
        const int c8n = 4 * (dp + 1) + vq;
        vn0 = rebuild8_lds<DG, S>(tab, cc0[dp + 1], c8n);
        vn1 = rebuild8_lds<DG, S>(tab, cc1[dp + 1], c8n);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
        *(uint32_t*)(stg + (8 * vq + e) * kStgStride + 2 * kp) = pair_halves(v0, v1, e);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const _Float16* row = stg + (16 * h + ln) * kStgStride;
        const half4 lo = *(const half4*)(row + 4 * lg);
        const half4 hi = *(const half4*)(row + 16 + 4 * lg);
        const half8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[2 * dp + h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pf[c], o[2 * dp + h], 0, 0, 0);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    __syncthreads();  // chunk c's records are consumed
    if (more) store_codes(vcodes[c + 1 < kSlots ? c + 1 : c]);
    __syncthreads();
  }

  // ---- workgroup sum of the waves' Oᵀ (lane (head ln, lg) holds dims
  // 16dt + 4lg + e) and the split's partial ----
  float* o_red = (float*)dyn;  // [waves][NQ][128], in the table area
  if (ln < NQ) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int e = 0; e < 4; ++e) o_red[(wave * NQ + ln) * kHeadDim + 16 * dt + 4 * lg + e] = o[dt][e];
  }
  __syncthreads();
  for (int idx = tid; idx < NQ * kHeadDim; idx += kLdsThreads) {
    const int h = idx / kHeadDim, i = idx % kHeadDim;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kLdsWaves; ++w) v += o_red[(w * NQ + h) * kHeadDim + i];
    const int64_t qh = kvh * NQ + h;
    a.ws_o[((b * a.QH + qh) * a.n_splits + split) * kHeadDim + i] = v;
    if (i == 0) {
      float* ml = a.ws_ml + ((b * a.QH + qh) * a.n_splits + split) * 2;
      // the combine works in natural-exponent units: m * ln 2
      ml[0] = ntok > 0 ? mh[h] * 0.6931471805599453f : -__builtin_inff();
      ml[1] = ntok > 0 ? lh[h] : 0.f;
    }
  }
}

// ---------------------------------------------------------------------------
// LDS-table decode at group dim 8 (GSRQ / grouped CQ, S <= 2): one
// 512-thread workgroup (8 waves) per (kv head, batch row, split of up to
// 2048 visible tokens).  The kv head's fp16 tables ([16][S][256][8],
// 128 KiB at G2) sit in LDS; the split's code records stream through LDS in
// 256-token chunks, one 32-key block per wave.
//   K phase  as decode_lds_kernel: per 16-key tile a lane rebuilds 32 dims of
//            one key from 16-byte codeword gathers, rotates them with the
//            reference's fp16 rotary, and four v_mfma_f32_16x16x32_f16 give
//            Sᵀ = K̂ Qᵀ for the GQA group;
//   V phase  the MFMA A operand V̂ᵀ (16 dims x 32 keys) is gathered straight
//            from the codeword tables with ds_read_b64_tr_b16: in each 16-lane
//            block, lane 4j + e receives element e of the 8-byte pieces that
//            the block's lanes j, j+4, j+8, j+12 address, so when lane
//            4i + j of block b addresses dims 16t + 4j..+3 of key 4b + i (and
//            then of key 16 + 4b + i), lane w of block b holds dim 16t + w of
//            the keys the P operand of block b carries.  The stage words are
//            added in fp16 after the read (one rounding, as the reference's
//            fp16(c1 + c2)); no staging tile, no per-key transposes.
// The split's (max, sum, out) go to decode_combine_kernel.

static const int kG8Threads = 512;
static const int kG8Waves = kG8Threads / 64;
static const int kG8Chunk = 256;       // tokens per chunk: one 32-key block per wave
static const int kG8MaxSplit = 2048;   // eight chunks
static const int kG8Plane = kLdsK * 16;  // bytes of one (group, stage) table: 256 words x 8 fp16

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4v;

// transposing LDS read of the 8-byte piece at LDS byte address addr (see above)
__device__ __forceinline__ half4 lds_read_tr(uint32_t addr) {
  return __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(size_t)addr));
}

// rope16 on packed pairs: (x * cos) + (rotate_half(x) * sin), every
// operation rounded to fp16, written pair by pair so that the subtraction
// becomes a v_pk_mul_f16 with a negated operand plus a v_pk_add_f16
// (fp16(b * -s) = -fp16(b * s)), with no separate sign flips
#pragma clang fp contract(off)
__device__ __forceinline__ void rope16_pk(half8 a, half8 b, half8 c, half8 s, half8* ra, half8* rb) {
  const uint4 A = __builtin_bit_cast(uint4, a), B = __builtin_bit_cast(uint4, b);
  const uint4 C = __builtin_bit_cast(uint4, c), Sn = __builtin_bit_cast(uint4, s);
  const uint32_t av[4] = {A.x, A.y, A.z, A.w}, bv[4] = {B.x, B.y, B.z, B.w};
  const uint32_t cv[4] = {C.x, C.y, C.z, C.w}, sv[4] = {Sn.x, Sn.y, Sn.z, Sn.w};
  uint32_t x[4], y[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const half2v ap = __builtin_bit_cast(half2v, av[p]), bp = __builtin_bit_cast(half2v, bv[p]);
    const half2v cp = __builtin_bit_cast(half2v, cv[p]), sp = __builtin_bit_cast(half2v, sv[p]);
    x[p] = __builtin_bit_cast(uint32_t, ap * cp - bp * sp);
    y[p] = __builtin_bit_cast(uint32_t, bp * cp + ap * sp);
  }
  *ra = __builtin_bit_cast(half8, uint4{x[0], x[1], x[2], x[3]});
  *rb = __builtin_bit_cast(half8, uint4{y[0], y[1], y[2], y[3]});
}
#pragma clang fp contract(on)

// Minimum of v over the wave, wave-uniform: within each 16-lane row by DPP
// (quad swaps, half-row and row mirrors), then across the four rows through
// lane reads; no LDS round trips.
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));  // row_half_mirror
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));  // row_mirror
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return min(min(r0, r1), min(r2, r3));
}

// What lane l of wave w needs to encode the appended token x: its groups
// 2w and 2w + 1 of x and their codewords l, l + 64, l + 128, l + 192 of
// every stage, from the kv head's fp16 tables ([16][S][256][8], 4 KiB per
// (group, stage)) in global memory or LDS.  The K search reads them from
// global memory before the tables' direct-to-LDS copy is issued, so that it
// runs while the copy is in flight (a load issued after the copy would wait
// for all of it).
template <int S>
__device__ __forceinline__ void fetch_new_token_words(const unsigned char* gtab, const _Float16* x, int wave,
                                                      int lane, half8 (&xv)[2], half8 (&cw)[S][2][4]) {
  xv[0] = *(const half8*)(x + 16 * wave);
  xv[1] = *(const half8*)(x + 16 * wave + 8);
#pragma unroll
  for (int st = 0; st < S; ++st)
#pragma unroll
    for (int gi = 0; gi < 2; ++gi)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        cw[st][gi][j] = *(const half8*)(gtab + ((2 * wave + gi) * S + st) * kG8Plane + (lane + 64 * j) * 16);
}

// Greedy residual search of one raw fp16 head vector over those codewords.
// Stage s scores ||c||^2 - 2 r.c, the reference's expanded distance
// ||r||^2 + ||c||^2 - 2 r.c less the row's constant ||r||^2, with r the
// residual x - c_1 - ... taken in its exact split x.c - c_1.c - ...: every
// product is fp16 x fp16 into an fp32 v_dot2 sum.  Keys keep the score's
// order-preserving bits with the index in the low byte, so the lowest score
// wins and, within 2^-16 of it, the lowest index.  The chosen codeword of a
// stage comes from the lane that holds it.  The code record [16][S] goes to
// rec (LDS) and out (global).
template <int S>
__device__ __forceinline__ void encode_new_token(const half8 (&xv)[2], const half8 (&cw)[S][2][4], uint8_t* rec,
                                                 uint8_t* out, int wave, int lane) {
  auto dot8 = [](half8 p, half8 q, float acc) {
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const half2v u = {p[e], p[e + 1]}, v = {q[e], q[e + 1]};
      acc = __builtin_amdgcn_fdot2(u, v, acc, false);
    }
    return acc;
  };
  half8 negc[2][S];  // negated words of the stages chosen so far
#pragma unroll
  for (int st = 0; st < S; ++st) {
    uint32_t best[2] = {~0u, ~0u};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = lane + 64 * j;
#pragma unroll
      for (int gi = 0; gi < 2; ++gi) {
        const half8 c = cw[st][gi][j];
        float rc = dot8(xv[gi], c, 0.f);
#pragma unroll
        for (int p = 0; p < st; ++p) rc = dot8(negc[gi][p], c, rc);
        const float score = fmaf(-2.f, rc, dot8(c, c, 0.f));
        const uint32_t u = __float_as_uint(score);
        const uint32_t ord = u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);  // monotonic in the score
        const uint32_t key = (ord & ~0xffu) | (uint32_t)k;
        best[gi] = key < best[gi] ? key : best[gi];
      }
    }
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) best[gi] = wave_min_u32(best[gi]);
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      const int g = 2 * wave + gi;
      const int code = (int)(best[gi] & 0xffu);  // wave-uniform
      if (st + 1 < S) {
        // codeword `code` is slot code >> 6 of lane code & 63: read every
        // slot of that lane, then pick (register arrays stay static-indexed)
        const int jj = code >> 6, src = code & 63;
        uint4 w = uint4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint4 m = __builtin_bit_cast(uint4, cw[st][gi][j]);
          const uint4 r = uint4{(uint32_t)__builtin_amdgcn_readlane((int)m.x, src),
                                (uint32_t)__builtin_amdgcn_readlane((int)m.y, src),
                                (uint32_t)__builtin_amdgcn_readlane((int)m.z, src),
                                (uint32_t)__builtin_amdgcn_readlane((int)m.w, src)};
          if (jj == j) w = r;
        }
        negc[gi][st] = __builtin_bit_cast(half8, uint4{w.x ^ 0x80008000u, w.y ^ 0x80008000u, w.z ^ 0x80008000u,
                                                       w.w ^ 0x80008000u});
      }
      if (lane == 0) {
        rec[g * S + st] = (uint8_t)code;
        out[g * S + st] = (uint8_t)code;
      }
    }
  }
}

template <int NQ, int S, bool APPEND>
__global__ __launch_bounds__(kG8Threads) void decode_g8_kernel(DecodeArgs a) {
  extern __shared__ __align__(16) unsigned char dyn[];
  constexpr int tab_bytes = 16 * S * kG8Plane;
  constexpr int kSlots = kG8MaxSplit / kG8Chunk;
  constexpr int kCb = 16 * S;    // code bytes per token
  constexpr int kCw = kCb / 4;   // as dwords
  unsigned char* tab = dyn;
  float* red = (float*)(dyn + tab_bytes);                 // [2][waves][NQ]
  uint8_t* newrec = (uint8_t*)(red + 2 * kG8Waves * NQ);  // [kCb] code record of the appended token

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  // logical block: split fastest, then batch row, then kv head
  const uint32_t bid = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t split = bid % (uint32_t)a.n_splits;
  const int64_t b = (bid / (uint32_t)a.n_splits) % (uint32_t)a.B;
  const int64_t kvh = bid / ((uint32_t)a.n_splits * (uint32_t)a.B);
  const int64_t L = a.lengths[b];
  const int64_t n_vis = L < a.window ? L : a.window;
  const int64_t t0 = L - n_vis + split * a.split_tokens;
  int64_t t1 = t0 + a.split_tokens;
  if (t1 > L) t1 = L;
  const int ntok = t1 > t0 ? (int)(t1 - t0) : 0;
  const int nchunks = (ntok + kG8Chunk - 1) / kG8Chunk;
  const int64_t cbase = b * a.csb + kvh * a.csh;
  const uint32_t cap = (uint32_t)a.cap;
  const uint32_t slot0 = (uint32_t)(t0 % a.cap);
  const float scale2 = 1.4426950408889634f / sqrtf((float)kHeadDim);  // log2(e)/sqrt(D)
  const int64_t rope_last = a.rope_len - 1;
  // the split holding position L-1 encodes the appended token; its record
  // takes the place of the ring slot's old bytes when its key is rebuilt
  const bool owner = APPEND && ntok > 0 && t1 == L;
  const int new_i = ntok - 1;  // its index in the split
  const int new_c = new_i / kG8Chunk;
  const int64_t new_slot = cbase + ((L - 1) % a.cap) * kCb;
  auto rope_row = [&](int64_t pos) -> const _Float16* {
    return a.rope + (pos < rope_last ? pos : rope_last) * kRopeRow;
  };
  // The code record of key k of the split, straight from the ring (each lane
  // loads the record of the key it rebuilds; the four lanes of a key share
  // the cache line).  Keys past the split read the split's first record, so
  // every rebuilt vector is one the reference also forms (its score is masked
  // and its weight is 0).
  auto load_rec = [&](const uint8_t* codes, int k, uint32_t (&w)[kCw]) {
    uint32_t slot = slot0 + (uint32_t)(k < ntok ? k : 0);
    if (slot >= cap) slot -= cap;
    const uint4* p = (const uint4*)(codes + cbase + (int64_t)slot * kCb);
#pragma unroll
    for (int i = 0; i < kCb / 16; ++i) {
      const uint4 v = p[i];
      w[4 * i] = v.x;
      w[4 * i + 1] = v.y;
      w[4 * i + 2] = v.z;
      w[4 * i + 3] = v.w;
    }
  };
  // the appended token's record (LDS) for the lane whose key it is
  auto splice_new = [&](int k, uint32_t (&w)[kCw]) {
    uint32_t nw[kCw];
    read_record<kCb>(newrec, nw);
    const bool mine = k == new_i;
#pragma unroll
    for (int i = 0; i < kCw; ++i) w[i] = mine ? nw[i] : w[i];
  };
  // tables global -> LDS directly, 8 KiB per workgroup-wide step; the
  // workgroups of one kv head start at different slices
  const int rot = (int)(bid % ((uint32_t)a.n_splits * (uint32_t)a.B));
  auto load_tables = [&](const _Float16* src_tab) {
    const uint4* src = (const uint4*)((const unsigned char*)src_tab + kvh * (int64_t)tab_bytes);
    uint4* dst = (uint4*)tab;
    constexpr int n = tab_bytes / 16;
    static_assert(n % kG8Threads == 0, "tables are whole 8 KiB slices");
    constexpr int per = n / kG8Threads;
#pragma unroll
    for (int u = 0; u < per; ++u) {
      const int uu = (u + rot) % per;
      __builtin_amdgcn_global_load_lds(
          (const void __attribute__((address_space(1)))*)(src + tid + uu * kG8Threads),
          (void __attribute__((address_space(3)))*)(dst + uu * kG8Threads + wave * 64), 16, 0, 0);
    }
  };
  // rotary rows of one 16-key tile (key positions past the split clamp to a
  // real row; their scores are masked).  Positions and row offsets fit 32
  // bits (the table has rope_len < 2^24 rows of 128 halves: host-checked).
  const uint32_t pos0 = (uint32_t)t0, rlast = (uint32_t)rope_last;
  auto fetch_trig = [&](int c, int tl, half8 (&tg)[4]) {
    const int tk = c * kG8Chunk + 32 * wave + 16 * tl + ln;
    uint32_t pos = pos0 + (uint32_t)(tk < ntok ? tk : 0);
    pos = pos < rlast ? pos : rlast;
    const _Float16* tr = a.rope + pos * (uint32_t)kRopeRow;
    load_trig8(tr, 8 * lg, &tg[0], &tg[1]);
    load_trig8(tr, 32 + 8 * lg, &tg[2], &tg[3]);
  };

  // ---- K tables into LDS; the first chunk's records and rotary rows load
  // beside them ----
  if constexpr (APPEND) {
    if (owner) {
      half8 xv[2], cw[S][2][4];
      fetch_new_token_words<S>((const unsigned char*)a.kt + kvh * (int64_t)tab_bytes, a.knew + b * a.nsb + kvh * a.nsh,
                               wave, lane, xv, cw);
      __builtin_amdgcn_sched_barrier(0);  // keep those loads ahead of the copy
      load_tables(a.kt);
      encode_new_token<S>(xv, cw, newrec, a.kc_out + new_slot, wave, lane);
    } else {
      load_tables(a.kt);
    }
  } else {
    load_tables(a.kt);
  }
  uint32_t rk[2][kCw];  // the records of the wave's two tiles in the current chunk
#pragma unroll
  for (int tl = 0; tl < 2; ++tl) load_rec(a.kc, 32 * wave + 16 * tl + ln, rk[tl]);
  // ---- rotated queries at position L-1: B operand, column ln = head ----
  const half8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
  half8 qb[4];
  {
    const int64_t head = kvh * NQ + (ln < NQ ? ln : 0);
    const _Float16* qp = a.q + b * a.qsb + head * a.qsh;
    const _Float16* tr = rope_row(L > 0 ? L - 1 : 0);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int d0 = 32 * c + 8 * lg;
      half8 x0, x1, cs, sn, r0, r1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x0[e] = qp[d0 + e];
        x1[e] = qp[d0 + 64 + e];
      }
      load_trig8(tr, d0, &cs, &sn);
      rope16_pk(x0, x1, cs, sn, &r0, &r1);
      qb[c] = ln < NQ ? r0 : zero8;
      qb[c + 2] = ln < NQ ? r1 : zero8;
    }
  }
  half8 trig[4];
  fetch_trig(0, 0, trig);
  __builtin_amdgcn_s_waitcnt(0);  // the tables' direct-to-LDS loads have landed
  __syncthreads();                 // (and the appended K record is in LDS)

  // ---- K phase, no barriers: each wave streams its own keys' records.
  // Lane (key ln of a 16-key tile, lane group lg) owns 8-dim chunks 4q+lg
  // (q = 0..3) = MFMA contraction slice q; chunks lg/lg+8 and lg+4/lg+12 are
  // rotary partners.  sc[c][tl][e]: score of key 4lg+e of tile tl of the
  // wave's block in chunk c, for head ln ----
  // byte offsets of chunk lg's tables (chunks 8 + lg .. through a second base,
  // so that every gather's constant part fits the instruction's offset)
  const uint32_t kgrp = (uint32_t)lg * S * kG8Plane;
  const uint32_t kgrp_hi = kgrp + 8u * S * kG8Plane;
  float4v sc[kSlots][2];
#pragma unroll
  for (int c = 0; c < kSlots; ++c) {
    sc[c][0] = float4v{-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
    sc[c][1] = sc[c][0];
    if (c >= nchunks) continue;
    // the next chunk's records go out now
    uint32_t rn[2][kCw];
    const int cn = c + 1 < kSlots ? c + 1 : c;
#pragma unroll
    for (int tl = 0; tl < 2; ++tl) load_rec(a.kc, cn * kG8Chunk + 32 * wave + 16 * tl + ln, rn[tl]);
    if constexpr (APPEND) {
      if (owner && c == new_c) {
#pragma unroll
        for (int tl = 0; tl < 2; ++tl) splice_new(c * kG8Chunk + 32 * wave + 16 * tl + ln, rk[tl]);
      }
    }
#pragma unroll
    for (int tl = 0; tl < 2; ++tl) {
      // the next tile's rotary rows go out now
      half8 tnext[4];
      if (tl == 0) {
        fetch_trig(c, 1, tnext);
      } else {
        fetch_trig(cn, 0, tnext);
      }
      uint32_t cc[4];
      record_codes<8, S>(rk[tl], lg, cc);
      half8 g[4][S];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int st = 0; st < S; ++st)
          g[q][st] = *(const half8*)(tab + (q < 2 ? kgrp : kgrp_hi) + (uint32_t)(4 * (q & 1) * S + st) * kG8Plane +
                                     (__builtin_amdgcn_ubfe(cc[q], 8u * st, 8u) << 4));
      // every gather of the tile is in flight before the first sum (left to
      // itself the scheduler interleaves the tiles and waits more)
      __builtin_amdgcn_sched_barrier(0);
      half8 k[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) k[q] = S == 2 ? g[q][0] + g[q][S - 1] : g[q][0];
      half8 r[4];
      rope16_pk(k[0], k[2], trig[0], trig[1], &r[0], &r[2]);
      rope16_pk(k[1], k[3], trig[2], trig[3], &r[1], &r[3]);
      float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(r[q], qb[q], acc, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = c * kG8Chunk + 32 * wave + 16 * tl + 4 * lg + e;
        sc[c][tl][e] = (ln < NQ && key < ntok) ? acc[e] * scale2 : -__builtin_inff();
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) trig[u] = tnext[u];
    }
#pragma unroll
    for (int tl = 0; tl < 2; ++tl)
#pragma unroll
      for (int i = 0; i < kCw; ++i) rk[tl][i] = rn[tl][i];
  }

  // every wave is done with the K tables (and the appended K record): the V
  // tables and the first chunk's V records load while the softmax runs
  __syncthreads();
  load_tables(a.vt);
  // the lane's two V keys of each chunk (as a source of the transposing
  // reads): 4lg + si and 16 + 4lg + si of the wave's block
  const int si = ln >> 2, sj = ln & 3;
  const int vkey = 32 * wave + 4 * lg + si;
  uint32_t rva[kCw], rvb[kCw];
  load_rec(a.vc, vkey, rva);
  load_rec(a.vc, vkey + 16, rvb);

  // ---- split max and exp-sum per head (lanes ln < NQ carry head ln) ----
  float mx = -__builtin_inff();
#pragma unroll
  for (int c = 0; c < kSlots; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) mx = fmaxf(mx, fmaxf(sc[c][0][e], sc[c][1][e]));
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (lg == 0 && ln < NQ) red[wave * NQ + ln] = mx;
  __syncthreads();
  float mh[NQ];
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    float m = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < kG8Waves; ++w) m = fmaxf(m, red[w * NQ + h]);
    mh[h] = m;
  }
  float m_lane = 0.f;
#pragma unroll
  for (int h = 0; h < NQ; ++h) m_lane = ln == h ? mh[h] : m_lane;
  const float m_use = m_lane == -__builtin_inff() ? 0.f : m_lane;
  half8 pf[kSlots];
  float lsum = 0.f;
#pragma unroll
  for (int c = 0; c < kSlots; ++c) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float pa = __builtin_amdgcn_exp2f(sc[c][0][e] - m_use);
      const float pb = __builtin_amdgcn_exp2f(sc[c][1][e] - m_use);
      lsum += pa + pb;
      pf[c][e] = (_Float16)pa;
      pf[c][e + 4] = (_Float16)pb;
    }
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  if (lg == 0 && ln < NQ) red[kG8Waves * NQ + wave * NQ + ln] = lsum;
  __syncthreads();
  float lh[NQ];
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < kG8Waves; ++w) l += red[kG8Waves * NQ + w * NQ + h];
    lh[h] = l;
  }

  // ---- the V tables have landed ----
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if constexpr (APPEND) {
    // the V search reads the landed tables (the softmax above already
    // covers the copy's flight time)
    if (owner) {
      half8 xv[2], cw[S][2][4];
      fetch_new_token_words<S>(tab, a.vnew + b * a.nsb + kvh * a.nsh, wave, lane, xv, cw);
      encode_new_token<S>(xv, cw, newrec, a.vc_out + new_slot, wave, lane);
      __syncthreads();
    }
  }

  // ---- V phase, no barriers.  As a source of the transposing reads, lane
  // 4i + j of lane group lg addresses, for keys 4lg + i and 16 + 4lg + i of
  // the wave's block, dims 4j..4j+3 of each 16-dim slice t: group 2t + (j >> 1),
  // half j & 1.  As an MFMA A lane (dim ln of slice t, keys of lane group lg)
  // it receives what the P operand of the same lane group weights ----
  // LDS byte addresses (the table area starts the dynamic allocation)
  const uint32_t vlane = (uint32_t)(size_t)(const void __attribute__((address_space(3)))*)tab +
                         (uint32_t)(sj >> 1) * S * kG8Plane + (uint32_t)(sj & 1) * 8u;
  const uint32_t vlane_hi = vlane + 8u * S * kG8Plane;  // slices 4..7 (groups 8..15)
  // record bits of this lane's group parity: S = 2: group 2t + jh sits at
  // bits 16 jh + 8 s of dword t; S = 1: bits 8 (2 (t & 1) + jh) of dword t / 2
  const uint32_t jsh = (uint32_t)(sj >> 1) * (S == 2 ? 16u : 8u);
  float4v o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < kSlots; ++c) {
    if (c >= nchunks) continue;
    uint32_t na[kCw], nb[kCw];
    const int cn = c + 1 < kSlots ? c + 1 : c;
    load_rec(a.vc, cn * kG8Chunk + vkey, na);
    load_rec(a.vc, cn * kG8Chunk + vkey + 16, nb);
    if constexpr (APPEND) {
      if (owner && c == new_c) {
        splice_new(c * kG8Chunk + vkey, rva);
        splice_new(c * kG8Chunk + vkey + 16, rvb);
      }
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      // the lane's codes of group 2dt + (sj >> 1), stage st, as byte offsets
      // of their words (code * 16) plus the lane's piece
      uint32_t ra[S], rb[S];
#pragma unroll
      for (int st = 0; st < S; ++st) {
        const uint32_t wa_ = S == 2 ? rva[dt] : rva[dt >> 1];
        const uint32_t wb_ = S == 2 ? rvb[dt] : rvb[dt >> 1];
        const uint32_t off = jsh + (S == 2 ? 8u * st : 16u * (dt & 1));
        const uint32_t base = dt < 4 ? vlane : vlane_hi;
        ra[st] = (__builtin_amdgcn_ubfe(wa_, off, 8u) << 4) + base;
        rb[st] = (__builtin_amdgcn_ubfe(wb_, off, 8u) << 4) + base;
      }
      const uint32_t plane = (uint32_t)(2 * (dt & 3) * S) * kG8Plane;
      half4 va = lds_read_tr(ra[0] + plane);
      half4 vb = lds_read_tr(rb[0] + plane);
      if constexpr (S == 2) {
        va = va + lds_read_tr(ra[1] + plane + kG8Plane);
        vb = vb + lds_read_tr(rb[1] + plane + kG8Plane);
      }
      const uint4 w = uint4{__builtin_bit_cast(uint2, va).x, __builtin_bit_cast(uint2, va).y,
                            __builtin_bit_cast(uint2, vb).x, __builtin_bit_cast(uint2, vb).y};
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, w), pf[c], o[dt], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kCw; ++i) {
      rva[i] = na[i];
      rvb[i] = nb[i];
    }
  }

  // ---- workgroup sum of the waves' Oᵀ (lane (head ln, lg) holds dims
  // 16dt + 4lg + e) and the split's partial ----
  __syncthreads();  // every wave is done with the V tables
  float* o_red = (float*)dyn;  // [waves][NQ][128], in the table area
  if (ln < NQ) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int e = 0; e < 4; ++e) o_red[(wave * NQ + ln) * kHeadDim + 16 * dt + 4 * lg + e] = o[dt][e];
  }
  __syncthreads();
  for (int idx = tid; idx < NQ * kHeadDim; idx += kG8Threads) {
    const int h = idx / kHeadDim, i = idx % kHeadDim;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kG8Waves; ++w) v += o_red[(w * NQ + h) * kHeadDim + i];
    const int64_t qh = kvh * NQ + h;
    a.ws_o[((b * a.QH + qh) * a.n_splits + split) * kHeadDim + i] = v;
    if (i == 0) {
      float* ml = a.ws_ml + ((b * a.QH + qh) * a.n_splits + split) * 2;
      ml[0] = ntok > 0 ? mh[h] * 0.6931471805599453f : -__builtin_inff();
      ml[1] = ntok > 0 ? lh[h] : 0.f;
    }
  }
}

// out[b,qh,:] = sum_s o_s e^{m_s-M} / sum_s l_s e^{m_s-M}
__global__ __launch_bounds__(128) void decode_combine_kernel(DecodeArgs a) {
  const int64_t bq = blockIdx.x;  // b*QH + qh
  const int i = threadIdx.x;
  const float* ml = a.ws_ml + bq * a.n_splits * 2;
  constexpr int kFew = 4;
  if (a.n_splits <= kFew) {
    // every split's (max, sum) and output element in flight together
    float mv[kFew], lv[kFew], ov[kFew];
#pragma unroll
    for (int s = 0; s < kFew; ++s) {
      if (s < a.n_splits) {
        mv[s] = ml[2 * s];
        lv[s] = ml[2 * s + 1];
        ov[s] = a.ws_o[(bq * a.n_splits + s) * kHeadDim + i];
      }
    }
    float M = -__builtin_inff();
#pragma unroll
    for (int s = 0; s < kFew; ++s)
      if (s < a.n_splits) M = fmaxf(M, mv[s]);
    float Lsum = 0.f, acc = 0.f;
#pragma unroll
    for (int s = 0; s < kFew; ++s) {
      if (s >= a.n_splits || mv[s] == -__builtin_inff()) continue;
      const float w = __expf(mv[s] - M);
      Lsum += lv[s] * w;
      acc += ov[s] * w;
    }
    a.out[bq * kHeadDim + i] = (_Float16)(Lsum > 0.f ? acc / Lsum : 0.f);
    return;
  }
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

// Rotary table: cos and sin of position p and frequency i as the reference's
// rotary module computes them: angle = fp32(p) * inv_freq[i] in fp32,
// cos/sin in fp32, then rounded to fp16.  inv_freq comes from the host.
// Row p = [cos of the 64 frequencies | sin of the 64 frequencies].
__global__ void rope_table_kernel(const float* __restrict__ inv_freq, int64_t n_pos,
                                  _Float16* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n_pos * 64) return;
  const int64_t p = idx / 64;
  const int i = (int)(idx % 64);
  const float ang = (float)p * inv_freq[i];
  out[p * kRopeRow + i] = (_Float16)cosf(ang);
  out[p * kRopeRow + 64 + i] = (_Float16)sinf(ang);
}

static const int64_t kMaxLds = 160 * 1024;

// Dynamic LDS of decode_lds_kernel: tables, one code-record chunk, the
// waves' staging tiles and the reductions.
static int64_t lds_bytes(int64_t S, int64_t nq) {
  return kHeadDim * S * kLdsK * 2 + kLdsChunk * kLdsCodeBytes +
         kLdsWaves * kStgRows * kStgStride * 2 + 2 * kLdsWaves * nq * 4;
}

// Tokens per split of decode_lds_kernel (0: the geometry does not fit).
static int64_t lds_split_tokens(int64_t G, int64_t S, int64_t K, int64_t nq, int64_t window) {
  if (S > 2 || K != kLdsK || G * S > kLdsCodeBytes || (G * S) % 16 != 0) return 0;
  if (lds_bytes(S, nq) > kMaxLds) return 0;
  if (kLdsWaves * nq * kHeadDim * 4 > kHeadDim * S * K * 2) return 0;  // partials fit the table area
  const int64_t w = ceil_div(window, kLdsChunk) * kLdsChunk;
  return w < kLdsMaxSplit ? w : kLdsMaxSplit;
}

// Dynamic LDS of decode_g8_kernel: tables, one chunk of code records, the
// reductions.
static int64_t g8_lds_bytes(int64_t S, int64_t nq) {
  return 16 * S * kG8Plane + 2 * kG8Waves * nq * 4 + 32;
}

// Tokens per split of decode_g8_kernel (0: the geometry does not fit).
static int64_t g8_split_tokens(int64_t G, int64_t S, int64_t K, int64_t nq, int64_t window) {
  if (G != 16 || S < 1 || S > 2 || K != kLdsK) return 0;
  if (g8_lds_bytes(S, nq) > kMaxLds) return 0;
  if (kG8Waves * nq * kHeadDim * 4 > 16 * S * kG8Plane) return 0;  // partials fit the table area
  const int64_t w = ceil_div(window, kG8Chunk) * kG8Chunk;
  return w < kG8MaxSplit ? w : kG8MaxSplit;
}

// Tokens per split of the kernel launch_decode picks for a packed-code
// geometry (the LDS-table kernels take up to 2048-token splits, the L2
// split kernel kSplitTokens), so callers can size the partials exactly.
static int64_t packed_split_tokens(int64_t G, int64_t d, int64_t S, int64_t K, int64_t nq, int64_t window,
                                   bool lds_ok) {
  if (lds_ok && d == 8) {
    const int64_t g8 = g8_split_tokens(G, S, K, nq, window);
    if (g8 > 0) return g8;
  }
  if (lds_ok && (d == 8 || d == 4)) {
    const int64_t lds = lds_split_tokens(G, S, K, nq, window);
    if (lds > 0) return lds;
  }
  return kSplitTokens;
}

// Bytes of split partials ([B,QH,n_splits] x (128 + 2) fp32) that launch.
static int64_t packed_partial_bytes(int64_t B, int64_t QH, int64_t G, int64_t d, int64_t S, int64_t K, int64_t nq,
                                    int64_t window, bool lds_ok) {
  const int64_t ns = ceil_div(window, packed_split_tokens(G, d, S, K, nq, window, lds_ok));
  return B * QH * ns * (kHeadDim + 2) * (int64_t)sizeof(float);
}

// The LDS-table kernels copy code records and tables in 16-byte pieces.
static bool packed_lds_ok(const void* k_codes, const void* v_codes, int64_t code_stride_b, int64_t code_stride_h,
                          const void* k_tables, const void* v_tables) {
  return ((uintptr_t)k_codes % 16 == 0) && ((uintptr_t)v_codes % 16 == 0) && code_stride_b % 16 == 0 &&
         code_stride_h % 16 == 0 && ((uintptr_t)k_tables % 16 == 0) && ((uintptr_t)v_tables % 16 == 0);
}

// The L2 split kernel, with the full-vector stage count as a template
// argument where it is 16 or 32 (R16 / R32 codecs).
template <int D, int NQ>
static void launch_split(const DecodeArgs& a, hipStream_t stream) {
  const dim3 grid((uint32_t)(a.B * a.KVH * a.n_splits));
  if constexpr (D == 128) {
    if (a.S == 16) {
      hipLaunchKernelGGL((decode_split_kernel<D, NQ, 16>), grid, dim3(256), 0, stream, a);
      return;
    }
    if (a.S == 32) {
      hipLaunchKernelGGL((decode_split_kernel<D, NQ, 32>), grid, dim3(256), 0, stream, a);
      return;
    }
  }
  hipLaunchKernelGGL((decode_split_kernel<D, NQ, 0>), grid, dim3(256), 0, stream, a);
}

template <int D, int NQ>
static int launch_decode(DecodeArgs a, bool lds_ok, hipStream_t stream, bool append = false) {
  const int64_t split = lds_ok && D != 128 && D != 0 ? lds_split_tokens(a.G, a.S, a.K, NQ, a.window) : 0;
  const int64_t g8_split = lds_ok && D == 8 ? g8_split_tokens(a.G, a.S, a.K, NQ, a.window) : 0;
  if constexpr (D == 128 || D == 0) {
    launch_split<D, NQ>(a, stream);
  } else if (D == 8 && g8_split > 0) {
    a.split_tokens = (int32_t)g8_split;
    a.n_splits = (int32_t)ceil_div(a.window, g8_split);
    a.ws_ml = a.ws_o + a.B * a.QH * a.n_splits * kHeadDim;
    const size_t lds = (size_t)g8_lds_bytes(a.S, NQ);
    const dim3 grid((uint32_t)(a.KVH * a.B * a.n_splits));
    if (a.S == 2) {
      if (append) {
        hipLaunchKernelGGL((decode_g8_kernel<NQ, 2, true>), grid, dim3(kG8Threads), lds, stream, a);
      } else {
        hipLaunchKernelGGL((decode_g8_kernel<NQ, 2, false>), grid, dim3(kG8Threads), lds, stream, a);
      }
    } else {
      if (append) {
        hipLaunchKernelGGL((decode_g8_kernel<NQ, 1, true>), grid, dim3(kG8Threads), lds, stream, a);
      } else {
        hipLaunchKernelGGL((decode_g8_kernel<NQ, 1, false>), grid, dim3(kG8Threads), lds, stream, a);
      }
    }
  } else if (append) {
    return set_error(JKV_ENOTSUP, "decode with append needs group dim 8, 16 groups, 1-2 stages, 256 codewords "
                                  "and 16-byte aligned codes and tables");
  } else if (split > 0) {
    a.split_tokens = (int32_t)split;
    a.n_splits = (int32_t)ceil_div(a.window, split);
    a.ws_ml = a.ws_o + a.B * a.QH * a.n_splits * kHeadDim;
    const size_t lds = (size_t)lds_bytes(a.S, NQ);
    const dim3 grid((uint32_t)(a.KVH * a.B * a.n_splits));
    if (a.S == 2) {
      hipLaunchKernelGGL((decode_lds_kernel<D, NQ, 2>), grid, dim3(kLdsThreads), lds, stream, a);
    } else {
      hipLaunchKernelGGL((decode_lds_kernel<D, NQ, 1>), grid, dim3(kLdsThreads), lds, stream, a);
    }
  } else {
    launch_split<D, NQ>(a, stream);
  }
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
                     (hipStream_t)stream_, inv_freq, n_pos, (_Float16*)out);
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

int64_t jkv_decode_workspace_bytes(int64_t B, int64_t QH, int64_t D, int64_t window) {
  const int64_t ns = jkv::ceil_div(window, jkv::kSplitTokens);
  return B * QH * ns * (D + 2) * (int64_t)sizeof(float);
}

}  // extern "C"

namespace jkv {

// Packed-code decode with the split partials in `workspace`; the C entry
// points below pass the caller's buffer or the library's static scratch.
static int decode_packed(const void* q, int64_t q_stride_b, int64_t q_stride_h, const uint8_t* k_codes,
                         const uint8_t* v_codes, int64_t code_stride_b, int64_t code_stride_h, int64_t cap,
                         const void* k_tables, const void* v_tables, int64_t B, int64_t QH, int64_t KVH,
                         int64_t G, int64_t d, int64_t S, int64_t K, const int32_t* lengths, int64_t window,
                         const void* rope_table, int64_t rope_len, void* out, void* workspace,
                         int64_t workspace_bytes, hipStream_t stream, const void* k_new = nullptr,
                         const void* v_new = nullptr, int64_t new_stride_b = 0, int64_t new_stride_h = 0) {
  const bool append = k_new != nullptr || v_new != nullptr;
  JKV_CHECK_ARG(!append || (k_new != nullptr && v_new != nullptr), "append needs both the new K and the new V");
  JKV_CHECK_ARG(B >= 0 && QH > 0 && KVH > 0 && QH % KVH == 0, "invalid head geometry");
  JKV_CHECK_ARG(G * d == kHeadDim, "decode attention supports head_dim 128 (got %lld)",
                (long long)(G * d));
  JKV_CHECK_ARG(K == 256, "decode attention expects 256-entry codebooks");
  JKV_CHECK_ARG(d == 8 || d == 4 || d == 128,
                "decode attention supports group dims 4, 8 and 128 (got %lld)", (long long)d);
  JKV_CHECK_ARG(S >= 1 && S <= (d == 128 ? 32 : 8), "decode attention supports 1..%d stages for group dim %lld",
                d == 128 ? 32 : 8, (long long)d);
  JKV_CHECK_ARG(window > 0 && cap > 0, "window and cache capacity must be positive");
  JKV_CHECK_ARG(cap >= window, "cache capacity below the attention window");
  JKV_CHECK_ARG(rope_len > 0, "rotary table is empty");
  const int64_t nq = QH / KVH;
  JKV_CHECK_ARG(nq == 1 || nq == 2 || nq == 4 || nq == 8, "GQA group of %lld query heads",
                (long long)nq);
  if (B == 0) return JKV_OK;
  JKV_CHECK_ARG(q && k_codes && v_codes && k_tables && v_tables && lengths && out && rope_table,
                "null buffer");
  const bool lds_ok = packed_lds_ok(k_codes, v_codes, code_stride_b, code_stride_h, k_tables, v_tables);
  // what the chosen kernel writes; jkv_decode_workspace_bytes() is an upper
  // bound of it for every packed geometry
  const int64_t need = packed_partial_bytes(B, QH, G, d, S, K, nq, window, lds_ok);
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
  a.rope = (const _Float16*)rope_table;
  a.rope_len = rope_len;
  a.n_splits = (int32_t)ceil_div(window, kSplitTokens);
  a.split_tokens = kSplitTokens;
  a.ws_o = (float*)workspace;
  a.ws_ml = a.ws_o + B * QH * a.n_splits * kHeadDim;
  a.out = (_Float16*)out;
  if (append) {
    JKV_CHECK_ARG(((uintptr_t)k_new % 16 == 0) && ((uintptr_t)v_new % 16 == 0) && new_stride_b % 8 == 0 &&
                      new_stride_h % 8 == 0,
                  "appended K/V rows must be 16-byte aligned");
    a.knew = (const _Float16*)k_new;
    a.vnew = (const _Float16*)v_new;
    a.nsb = new_stride_b;
    a.nsh = new_stride_h;
    a.kc_out = const_cast<uint8_t*>(k_codes);
    a.vc_out = const_cast<uint8_t*>(v_codes);
  }
#define JKV_DEC(DD, NN) \
  if (d == DD && nq == NN) return launch_decode<DD, NN>(a, lds_ok, stream, append);
  JKV_DEC(8, 1) JKV_DEC(8, 2) JKV_DEC(8, 4) JKV_DEC(8, 8)
  JKV_DEC(4, 1) JKV_DEC(4, 2) JKV_DEC(4, 4) JKV_DEC(4, 8)
  JKV_DEC(128, 1) JKV_DEC(128, 2) JKV_DEC(128, 4) JKV_DEC(128, 8)
#undef JKV_DEC
  return set_error(JKV_ENOTSUP, "unsupported decode geometry");
}

// Allocation-free decode (jkv_decode_attention_noalloc): the split partials
// live in this file-scope array, one copy per GPU, held until the process
// ends.  Host code never passes the array's name to a kernel (on the host it
// is a stand-in, not a device address): the device address comes from
// hipGetSymbolAddress, once per device with that device current, and is kept
// in g_scratch_ptr.
static const int64_t kNoAllocScratchBytes = (int64_t)16 << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

static const int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch (looked up on first use).
static int current_scratch(void** ptr) {
  int dev = -1;
  JKV_CHECK_HIP(hipGetDevice(&dev));
  JKV_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "device ordinal %d outside 0..%d", dev, kMaxDevices - 1);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    JKV_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    JKV_CHECK_ARG(p != nullptr, "scratch symbol has no device address");
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return JKV_OK;
}

}  // namespace jkv

extern "C" {

int jkv_decode_attention(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                         const uint8_t* k_codes, const uint8_t* v_codes, int64_t code_stride_b,
                         int64_t code_stride_h, int64_t cap, const void* k_tables,
                         const void* v_tables, int64_t B, int64_t QH, int64_t KVH, int64_t G,
                         int64_t d, int64_t S, int64_t K, const int32_t* lengths, int64_t window,
                         const void* rope_table, int64_t rope_len, void* out, void* workspace,
                         int64_t workspace_bytes, jkv_stream_t stream) {
  return jkv::decode_packed(q, q_stride_b, q_stride_h, k_codes, v_codes, code_stride_b, code_stride_h, cap,
                            k_tables, v_tables, B, QH, KVH, G, d, S, K, lengths, window, rope_table, rope_len,
                            out, workspace, workspace_bytes, (hipStream_t)stream);
}

int jkv_decode_attention_append(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_new,
                                const void* v_new, int64_t new_stride_b, int64_t new_stride_h, uint8_t* k_codes,
                                uint8_t* v_codes, int64_t code_stride_b, int64_t code_stride_h, int64_t cap,
                                const void* k_tables, const void* v_tables, int64_t B, int64_t QH, int64_t KVH,
                                int64_t G, int64_t d, int64_t S, int64_t K, const int32_t* lengths,
                                int64_t window, const void* rope_table, int64_t rope_len, void* out,
                                void* workspace, int64_t workspace_bytes, jkv_stream_t stream) {
  if (B > 0) JKV_CHECK_ARG(k_new != nullptr && v_new != nullptr, "null buffer");
  return jkv::decode_packed(q, q_stride_b, q_stride_h, k_codes, v_codes, code_stride_b, code_stride_h, cap,
                            k_tables, v_tables, B, QH, KVH, G, d, S, K, lengths, window, rope_table, rope_len,
                            out, workspace, workspace_bytes, (hipStream_t)stream, B > 0 ? k_new : nullptr,
                            B > 0 ? v_new : nullptr, new_stride_b, new_stride_h);
}

int64_t jkv_decode_noalloc_max_workspace_bytes(void) { return jkv::kNoAllocScratchBytes; }

int jkv_decode_attention_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                 const uint8_t* k_codes, const uint8_t* v_codes, int64_t code_stride_b,
                                 int64_t code_stride_h, int64_t cap, const void* k_tables,
                                 const void* v_tables, int64_t B, int64_t QH, int64_t KVH, int64_t G,
                                 int64_t d, int64_t S, int64_t K, const int32_t* lengths, int64_t window,
                                 const void* rope_table, int64_t rope_len, void* out,
                                 jkv_stream_t stream) {
  using namespace jkv;
  JKV_CHECK_ARG(B >= 0 && QH > 0 && KVH > 0 && QH % KVH == 0 && window > 0, "invalid head geometry");
  // the partials of the kernel this call will run: 2048-token splits on the
  // LDS-table kernels (group dims 4 and 8), 256-token splits otherwise
  const bool lds_ok = packed_lds_ok(k_codes, v_codes, code_stride_b, code_stride_h, k_tables, v_tables);
  const int64_t need = packed_partial_bytes(B, QH, G, d, S, K, QH / KVH, window, lds_ok);
  JKV_CHECK_ARG(need <= kNoAllocScratchBytes,
                "allocation-free decode attention holds at most %lld bytes of split partials; "
                "B=%lld, QH=%lld, window=%lld need %lld (use jkv_decode_attention with a workspace)",
                (long long)kNoAllocScratchBytes, (long long)B, (long long)QH, (long long)window, (long long)need);
  if (B == 0) return JKV_OK;
  void* ws = nullptr;
  const int rc = current_scratch(&ws);
  if (rc != JKV_OK) return rc;
  return decode_packed(q, q_stride_b, q_stride_h, k_codes, v_codes, code_stride_b, code_stride_h, cap, k_tables,
                       v_tables, B, QH, KVH, G, d, S, K, lengths, window, rope_table, rope_len, out, ws,
                       kNoAllocScratchBytes, (hipStream_t)stream);
}

int jkv_decode_attention_window(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                const void* k_window, const void* v_window, int64_t kv_stride_b,
                                int64_t kv_stride_h, int64_t cap, int64_t B, int64_t QH, int64_t KVH,
                                const int32_t* lengths, int64_t window, const void* rope_table,
                                int64_t rope_len, void* out, void* workspace, int64_t workspace_bytes,
                                jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(B >= 0 && QH > 0 && KVH > 0 && QH % KVH == 0, "invalid head geometry");
  JKV_CHECK_ARG(window > 0 && cap > 0, "window and cache capacity must be positive");
  JKV_CHECK_ARG(cap >= window, "cache capacity below the attention window");
  JKV_CHECK_ARG(rope_len > 0, "rotary table is empty");
  const int64_t nq = QH / KVH;
  JKV_CHECK_ARG(nq == 1 || nq == 2 || nq == 4 || nq == 8, "GQA group of %lld query heads",
                (long long)nq);
  if (B == 0) return JKV_OK;
  JKV_CHECK_ARG(q && k_window && v_window && lengths && out && rope_table, "null buffer");
  JKV_CHECK_ARG(((uintptr_t)k_window % 16 == 0) && ((uintptr_t)v_window % 16 == 0) && kv_stride_b % 8 == 0 &&
                    kv_stride_h % 8 == 0,
                "decoded windows need 16-byte aligned rows");
  const int64_t need = jkv_decode_workspace_bytes(B, QH, kHeadDim, window);
  JKV_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                "decode attention needs %lld bytes of workspace", (long long)need);
  DecodeArgs a = {};
  a.q = (const _Float16*)q;
  a.qsb = q_stride_b; a.qsh = q_stride_h;
  // each token's record is its 256-byte fp16 row
  a.kc = (const uint8_t*)k_window; a.vc = (const uint8_t*)v_window;
  a.csb = kv_stride_b * 2; a.csh = kv_stride_h * 2; a.cap = cap;
  a.kt = nullptr; a.vt = nullptr;
  a.B = B; a.QH = QH; a.KVH = KVH; a.G = kHeadDim * 2; a.d = 0; a.S = 1; a.K = 0;
  a.lengths = lengths;
  a.window = window;
  a.rope = (const _Float16*)rope_table;
  a.rope_len = rope_len;
  a.n_splits = (int32_t)ceil_div(window, kWinSplitTokens);  // within the queried workspace
  a.split_tokens = kWinSplitTokens;
  a.ws_o = (float*)workspace;
  a.ws_ml = a.ws_o + B * QH * a.n_splits * kHeadDim;
  a.out = (_Float16*)out;
  switch (nq) {
    case 1: return launch_decode<0, 1>(a, false, stream);
    case 2: return launch_decode<0, 2>(a, false, stream);
    case 4: return launch_decode<0, 4>(a, false, stream);
    default: return launch_decode<0, 8>(a, false, stream);
  }
}

}  // extern "C"
