// Value gradient of the causal sliding-window GQA prefill attention:
//   dV̂[b, kvh, s, :] = sum over the group's query heads h and rows t of
//                       P[b, h, t, s] * dO[b, h, t, :]
// with P recomputed from the rotated q and K̂ and the forward's per-row
// log-sum-exp (P = exp(q.k / sqrt(D) - lse), zero where the mask hides s).
// This is the value leg of the SDPA backward that the reference's V-only step
// runs under loss.backward() (experiments/train_full_model_closed_loop_vq.py:
// 277-304 forward; experiments_followup_mistral/train_mistral_v_only.py:
// 142-150 step): the K tables and the backbone are frozen there, so the query
// and key gradients are not needed for the value tables.
//
// One workgroup of NQ waves per (batch row, kv head, block of 32 keys); wave
// h is query head h of the group.  The block's rotated K̂ stays in registers
// as MFMA B operands.  Per 32-row query tile, on v_mfma_f32_16x16x32_f16:
//   S[row][key]    = Q K̂ᵀ          A = the wave's rotated q rows, B = K̂
//   P              = exp2(S log2e/sqrt(D) - lse log2e), masked, fp16
//   dO in B order  = dO I           A = dO rows, B = identity columns: the
//                                  MFMA output layout is the transpose of its
//                                  A layout, so lane (dim j) ends up holding
//                                  rows of dim j; exact, since every product
//                                  is one fp16 value times 1
//   dV̂[key][dim] += Pᵀ dO          A = P read straight off the S accumulators
//                                  (two 16-row tiles interleaved into the 32
//                                  contraction slots), B = the transposed dO
// The heads' partial sums meet in LDS and are added in head order.
#include <math.h>

#include "jkv_common.h"
#include "rotary.h"

namespace jkv {

static const int kBD = 128;      // head dim
static const int kBKeys = 32;    // keys per workgroup
static const int kBRows = 32;    // query rows per tile

struct ValueGradArgs {
  const _Float16* q;
  int64_t qsb, qsh, qst;
  const _Float16* k;
  int64_t ksb, ksh, kst;
  const _Float16* dout;
  int64_t dsb, dsh, dst;
  const float* lse;  // [B,QH,T]
  int64_t B, QH, KVH, T;
  const int32_t* start;
  int64_t window;
  const _Float16* rope;
  int64_t rope_len;
  float* dv;  // [B,KVH,T,D] fp32 contiguous
};

template <int NQ>
__global__ __launch_bounds__(64 * NQ) void prefill_value_grad_kernel(ValueGradArgs a) {
  // partial sums of heads 1..NQ-1: [head-1][key][dim] fp32
  extern __shared__ __align__(16) float part[];
  const int tid = threadIdx.x, lane = tid & 63, h = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int64_t nkb = ceil_div(a.T, kBKeys);
  // key blocks fastest: the blocks of one (batch row, kv head) share its q and
  // dO rows in one XCD's L2
  const uint32_t bid = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t kb = bid % (uint32_t)nkb;
  const int64_t kvh = (bid / (uint32_t)nkb) % (uint32_t)a.KVH;
  const int64_t b = bid / ((uint32_t)nkb * (uint32_t)a.KVH);
  const int64_t head = kvh * NQ + h;
  const int64_t key0 = kb * kBKeys;
  const int64_t p0 = a.start[b];
  const float scale2 = 1.4426950408889634f / sqrtf((float)kBD);
  const int64_t rope_last = a.rope_len - 1;
  auto rope_row = [&](int64_t pos) -> const _Float16* {
    return a.rope + (pos < 0 ? 0 : (pos < rope_last ? pos : rope_last)) * kRopeRow;
  };
  const half8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};

  // ---- the block's rotated keys as B operands: kb_[kt][c] = dims
  // [32c + 8lg, +8) of key 16kt + ln (chunks c and c+2 are rotary partners) ----
  half8 kop[2][4];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    const int64_t key = key0 + 16 * kt + ln;
    const bool ok = key < a.T;
    const _Float16* kp = a.k + b * a.ksb + kvh * a.ksh + (ok ? key : 0) * a.kst;
    const _Float16* tr = rope_row(p0 + (ok ? key : 0));
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int d0 = 32 * c + 8 * lg;
      half8 cs, sn, r0, r1;
      load_trig8(tr, d0, &cs, &sn);
      rope16(*(const half8*)(kp + d0), *(const half8*)(kp + d0 + 64), cs, sn, &r0, &r1);
      kop[kt][c] = ok ? r0 : zero8;
      kop[kt][c + 2] = ok ? r1 : zero8;
    }
  }
  // identity columns: B operand lane (column ln, lg) holds contraction slots
  // 8lg..8lg+7; ident[half] selects column ln of dims 16 half .. 16 half + 15
  half8 ident[2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int e = 0; e < 8; ++e) ident[hf][e] = (_Float16)(8 * lg + e == 16 * hf + ln ? 1.f : 0.f);

  float4v acc[2][8];  // dV̂[key 16kt + 4lg + e][dim 16dt + ln]
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[kt][dt] = float4v{0.f, 0.f, 0.f, 0.f};

  // query rows that see some key of the block: [key0, key0 + 31 + window)
  int64_t rend = key0 + kBKeys - 1 + a.window;
  if (rend > a.T || rend < 0) rend = a.T;
  const _Float16* qbase = a.q + b * a.qsb + head * a.qsh;
  const _Float16* dbase = a.dout + b * a.dsb + head * a.dsh;
  const float* lbase = a.lse + (b * a.QH + head) * a.T;

  for (int64_t r0 = key0; r0 < rend; r0 += kBRows) {
    // ---- the tile's rotated q rows (A operands) and dO rows ----
    half8 qa[2][4], da[2][4];
#pragma unroll
    for (int rg = 0; rg < 2; ++rg) {
      const int64_t row = r0 + 16 * rg + ln;
      const bool ok = row < a.T;
      const _Float16* qp = qbase + (ok ? row : 0) * a.qst;
      const _Float16* dp = dbase + (ok ? row : 0) * a.dst;
      const _Float16* tr = rope_row(p0 + (ok ? row : 0));
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int d0 = 32 * c + 8 * lg;
        half8 cs, sn, r0h, r1h;
        load_trig8(tr, d0, &cs, &sn);
        rope16(*(const half8*)(qp + d0), *(const half8*)(qp + d0 + 64), cs, sn, &r0h, &r1h);
        qa[rg][c] = ok ? r0h : zero8;
        qa[rg][c + 2] = ok ? r1h : zero8;
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) da[rg][c] = ok ? *(const half8*)(dp + 32 * c + 8 * lg) : zero8;
    }
    // lse (base 2) of the rows this lane's S elements belong to: 4lg + e, 16 + 4lg + e
    float l2[2][4];
#pragma unroll
    for (int rg = 0; rg < 2; ++rg)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t row = r0 + 16 * rg + 4 * lg + e;
        l2[rg][e] = row < a.T ? lbase[row] * 1.4426950408889634f : 0.f;
      }

    // ---- S[row][key] for 2 row tiles x 2 key tiles ----
    float4v s[2][2];
#pragma unroll
    for (int rg = 0; rg < 2; ++rg)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        s[rg][kt] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c)
          s[rg][kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[rg][c], kop[kt][c], s[rg][kt], 0, 0, 0);
      }
    // ---- P, masked: element (rg, kt, e) is row r0 + 16rg + 4lg + e, key
    // key0 + 16kt + ln.  pa[kt]: A operand of key 16kt + ln, contraction slot
    // 8lg + e <-> row 4lg + e (e < 4), 16 + 4lg + e - 4 (e >= 4) ----
    const bool full = r0 >= key0 + kBKeys - 1 && r0 + kBRows - 1 - key0 < a.window && r0 + kBRows <= a.T;
    // masks in 32-bit offsets from the tile: row - key = base + 16rg + e - 16kt
    const int base = (int)(r0 - key0) + 4 * lg - ln;
    const int rows_left = (int)(a.T - r0 < kBRows ? a.T - r0 : kBRows);  // valid rows of the tile
    const int keys_left = (int)(a.T - key0 < kBKeys ? a.T - key0 : kBKeys);
    const int win = a.window < 0x40000000 ? (int)a.window : 0x40000000;
    half8 pa[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int rg = 0; rg < 2; ++rg)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float p = __builtin_amdgcn_exp2f(fmaf(s[rg][kt][e], scale2, -l2[rg][e]));
          if (!full) {
            const int diff = base + 16 * rg + e - 16 * kt;
            const bool vis = diff >= 0 && diff < win && 16 * rg + 4 * lg + e < rows_left && 16 * kt + ln < keys_left;
            p = vis ? p : 0.f;
          }
          pa[kt][4 * rg + e] = (_Float16)p;
        }
    // ---- per 16-dim slice: dO in B order (db = rows {4lg+e, 16+4lg+e} of
    // dim 16dt + ln), then dV̂ += Pᵀ dO for both key tiles ----
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      half8 db;
#pragma unroll
      for (int rg = 0; rg < 2; ++rg) {
        const float4v t = __builtin_amdgcn_mfma_f32_16x16x32_f16(da[rg][dt >> 1], ident[dt & 1],
                                                               float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) db[4 * rg + e] = (_Float16)t[e];
      }
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
        acc[kt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[kt], db, acc[kt][dt], 0, 0, 0);
    }
  }

  // ---- sum the heads in order (head 0 + head 1 + ...) and store ----
  if (NQ > 1) {
    if (h > 0) {
      float* mine = part + (size_t)(h - 1) * kBKeys * kBD;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
          for (int e = 0; e < 4; ++e) mine[(16 * kt + 4 * lg + e) * kBD + 16 * dt + ln] = acc[kt][dt][e];
    }
    __syncthreads();
    if (h > 0) return;
#pragma unroll 1
    for (int o = 1; o < NQ; ++o) {
      const float* other = part + (size_t)(o - 1) * kBKeys * kBD;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[kt][dt][e] += other[(16 * kt + 4 * lg + e) * kBD + 16 * dt + ln];
    }
  }
  float* out = a.dv + ((b * a.KVH + kvh) * a.T) * kBD;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t key = key0 + 16 * kt + 4 * lg + e;
      if (key >= a.T) continue;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) out[key * kBD + 16 * dt + ln] = acc[kt][dt][e];
    }
}

template <int NQ>
static void launch_value_grad(const ValueGradArgs& a, int64_t blocks, hipStream_t stream) {
  const size_t lds = (size_t)(NQ - 1) * kBKeys * kBD * sizeof(float);
  hipLaunchKernelGGL(prefill_value_grad_kernel<NQ>, dim3((uint32_t)blocks), dim3(64 * NQ), lds, stream, a);
}

}  // namespace jkv

extern "C" {

int jkv_prefill_attention_value_grad(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                     int64_t q_stride_t, const void* k, int64_t k_stride_b,
                                     int64_t k_stride_h, int64_t k_stride_t, const void* d_out,
                                     int64_t d_stride_b, int64_t d_stride_h, int64_t d_stride_t,
                                     const float* lse, int64_t B, int64_t QH, int64_t KVH, int64_t T,
                                     int64_t D, const int32_t* start_positions, int64_t window,
                                     const void* rope_table, int64_t rope_len, float* d_value,
                                     jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(D == kBD, "prefill value gradient supports head_dim 128, got %lld", (long long)D);
  JKV_CHECK_ARG(B >= 0 && QH > 0 && KVH > 0 && T >= 0 && QH % KVH == 0, "invalid prefill geometry");
  const int64_t NQ = QH / KVH;
  JKV_CHECK_ARG(NQ == 1 || NQ == 2 || NQ == 4 || NQ == 8,
                "query heads per kv head must be 1, 2, 4 or 8, got %lld", (long long)NQ);
  JKV_CHECK_ARG(window >= 1, "window must be positive");
  if (B == 0 || T == 0) return JKV_OK;
  JKV_CHECK_ARG(q && k && d_out && lse && d_value && start_positions && rope_table, "null buffer");
  JKV_CHECK_ARG(rope_len >= 1, "rotary table is empty");
  const int64_t strides[9] = {q_stride_b, q_stride_h, q_stride_t, k_stride_b, k_stride_h,
                              k_stride_t, d_stride_b, d_stride_h, d_stride_t};
  for (int i = 0; i < 9; ++i)
    JKV_CHECK_ARG(strides[i] % 8 == 0, "prefill strides must be multiples of 8 elements");
  JKV_CHECK_ARG(((uintptr_t)q | (uintptr_t)k | (uintptr_t)d_out | (uintptr_t)d_value) % 16 == 0,
                "prefill buffers must be 16-byte aligned");
  ValueGradArgs a = {};
  a.q = (const _Float16*)q; a.qsb = q_stride_b; a.qsh = q_stride_h; a.qst = q_stride_t;
  a.k = (const _Float16*)k; a.ksb = k_stride_b; a.ksh = k_stride_h; a.kst = k_stride_t;
  a.dout = (const _Float16*)d_out; a.dsb = d_stride_b; a.dsh = d_stride_h; a.dst = d_stride_t;
  a.lse = lse;
  a.B = B; a.QH = QH; a.KVH = KVH; a.T = T;
  a.start = start_positions;
  a.window = window;
  a.rope = (const _Float16*)rope_table;
  a.rope_len = rope_len;
  a.dv = d_value;
  const int64_t blocks = ceil_div(T, kBKeys) * KVH * B;
  JKV_CHECK_ARG(blocks < ((int64_t)1 << 31), "prefill grid too large");
  switch (NQ) {
    case 1: launch_value_grad<1>(a, blocks, stream); break;
    case 2: launch_value_grad<2>(a, blocks, stream); break;
    case 4: launch_value_grad<4>(a, blocks, stream); break;
    default: launch_value_grad<8>(a, blocks, stream); break;
  }
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

}  // extern "C"
