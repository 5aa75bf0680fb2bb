// One sliding-pair step of the offline multi-exit additive block refinement
// (src/jointkv/nested_vq.py:757-1001): score every (first, second) pair of
// two shortlists by the weighted squared error of the exits that contain the
// block, keep the lowest (the old pair on ties) and move those exits'
// residuals by the change.
//
// With the exits' reconstructions r_m ([E][H][N][D] fp32) and the row x, a
// block's cost for shortlist entries (i, j) is
//   sum_m w_m |(x - r_m) + c1[old1] + s_m c2[old2] - c1[i] - s_m c2[j]|^2,
// s_m = 1 when exit m also contains the second stage.  One wave takes one row:
// lane k scores pairs k and k + 64 (L <= 9, so L^2 <= 81), streaming the
// row's vectors in float4 pieces (x, r_m and the old words are the same
// address in every lane: one broadcast fetch), then a wave-wide minimum of
// (cost bits << 32 | pair) picks the winner, the lowest pair on equal cost.
// Finally the lanes split the D dimensions to add the winner's changes to
// the reconstructions, first stage then second.
#include "jkv_common.h"

namespace jkv {

static const int kPairMaxExits = 32;
static const int kPairMaxShort = 9;

struct PairArgs {
  const float* x;  // [H][N][D]
  float* recon;    // [E][H][N][D]
  int64_t H, N, D;
  int32_t n_exits;  // exits that contain the first stage and carry weight
  int32_t slot[kPairMaxExits];
  float weight[kPairMaxExits];
  int32_t second[kPairMaxExits];
  const float* t1;  // [H][K1][D]
  const float* t2;  // [H][K2][D]
  int64_t K1, K2;
  const int64_t* sl1;  // [H][N][L], entry 0 = the current index
  const int64_t* sl2;
  int32_t L;
  int64_t* out1;  // [H][N]
  int64_t* out2;
};

template <bool VEC4>
__global__ __launch_bounds__(256) void pair_block_kernel(PairArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (h, n)
  if (row >= a.H * a.N) return;
  const int64_t h = row / a.N;
  const int64_t D = a.D;
  const int L = a.L;
  const int64_t* s1 = a.sl1 + row * L;
  const int64_t* s2 = a.sl2 + row * L;
  // shortlist entries lie in [0, K) by contract; clamped so that no input can
  // address outside the tables
  auto in1 = [&](int64_t k) { return k < 0 ? (int64_t)0 : (k >= a.K1 ? a.K1 - 1 : k); };
  auto in2 = [&](int64_t k) { return k < 0 ? (int64_t)0 : (k >= a.K2 ? a.K2 - 1 : k); };
  const float* o1 = a.t1 + (h * a.K1 + in1(s1[0])) * D;
  const float* o2 = a.t2 + (h * a.K2 + in2(s2[0])) * D;
  const int64_t rstride = a.H * a.N * D;
  const float* xrow = a.x + row * D;
  const float* rrow = a.recon + row * D;

  float cost[2] = {0.f, 0.f};
  const float* c1[2];
  const float* c2[2];
  bool live[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int p = lane + 64 * u;
    live[u] = p < L * L;
    const int i = live[u] ? p / L : 0, j = live[u] ? p % L : 0;
    c1[u] = a.t1 + (h * a.K1 + in1(s1[i])) * D;
    c2[u] = a.t2 + (h * a.K2 + in2(s2[j])) * D;
  }
  for (int m = 0; m < a.n_exits; ++m) {
    const float* r = rrow + (int64_t)a.slot[m] * rstride;
    const bool sec = a.second[m] != 0;
    float acc[2] = {0.f, 0.f};
    if constexpr (VEC4) {
      for (int64_t d = 0; d < D; d += 4) {
        const float4 xv = *(const float4*)(xrow + d);
        const float4 rv = *(const float4*)(r + d);
        const float4 w1 = *(const float4*)(o1 + d);
        float4 base = make_float4((xv.x - rv.x) + w1.x, (xv.y - rv.y) + w1.y, (xv.z - rv.z) + w1.z,
                                  (xv.w - rv.w) + w1.w);
        if (sec) {
          const float4 w2 = *(const float4*)(o2 + d);
          base = make_float4(base.x + w2.x, base.y + w2.y, base.z + w2.z, base.w + w2.w);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          float4 cand = *(const float4*)(c1[u] + d);
          if (sec) {
            const float4 v = *(const float4*)(c2[u] + d);
            cand = make_float4(cand.x + v.x, cand.y + v.y, cand.z + v.z, cand.w + v.w);
          }
          const float dx = base.x - cand.x, dy = base.y - cand.y, dz = base.z - cand.z, dw = base.w - cand.w;
          acc[u] = fmaf(dx, dx, acc[u]);
          acc[u] = fmaf(dy, dy, acc[u]);
          acc[u] = fmaf(dz, dz, acc[u]);
          acc[u] = fmaf(dw, dw, acc[u]);
        }
      }
    } else {
      for (int64_t d = 0; d < D; ++d) {
        float base = (xrow[d] - r[d]) + o1[d];
        if (sec) base += o2[d];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          float cand = c1[u][d];
          if (sec) cand += c2[u][d];
          const float dx = base - cand;
          acc[u] = fmaf(dx, dx, acc[u]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) cost[u] = fmaf(a.weight[m], acc[u], cost[u]);
  }
  // winner: lowest cost, lowest pair index on equal cost (costs are >= 0, so
  // their bit patterns order like their values)
  uint64_t key = ~0ull;
#pragma unroll
  for (int u = 0; u < 2; ++u)
    if (live[u]) {
      const uint64_t k = ((uint64_t)__float_as_uint(cost[u]) << 32) | (uint32_t)(lane + 64 * u);
      key = k < key ? k : key;
    }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)key, off, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(key >> 32), off, 64);
    const uint64_t other = ((uint64_t)hi << 32) | lo;
    key = other < key ? other : key;
  }
  const int p = (int)(uint32_t)key;
  const int64_t n1 = in1(s1[p / L]), n2 = in2(s2[p % L]);
  if (lane == 0) {
    a.out1[row] = n1;
    a.out2[row] = n2;
  }
  // reconstructions move by the changes: r_m += c1[n1] - c1[old1], then,
  // for exits holding the second stage, r_m += c2[n2] - c2[old2]
  const float* w1n = a.t1 + (h * a.K1 + n1) * D;
  const float* w2n = a.t2 + (h * a.K2 + n2) * D;
  for (int64_t d = lane; d < D; d += 64) {
    const float d1 = w1n[d] - o1[d];
    const float d2 = w2n[d] - o2[d];
    for (int m = 0; m < a.n_exits; ++m) {
      float* r = a.recon + (int64_t)a.slot[m] * rstride + row * D;
      float v = r[d] + d1;
      if (a.second[m]) v += d2;
      r[d] = v;
    }
  }
}

}  // namespace jkv

extern "C" int jkv_pair_block_select(const float* states, float* recon, int64_t n_recon, int64_t H, int64_t N,
                                     int64_t D,
                                     int32_t n_exits, const int32_t* exit_slots, const float* exit_weights,
                                     const int32_t* exit_has_second, const float* first_table,
                                     const float* second_table, int64_t K1, int64_t K2,
                                     const int64_t* first_shortlist, const int64_t* second_shortlist,
                                     int64_t L, int64_t* first_out, int64_t* second_out,
                                     jkv_stream_t stream) {
  using namespace jkv;
  JKV_CHECK_ARG(H > 0 && N >= 0 && D > 0 && K1 > 0 && K2 > 0, "invalid block-refinement geometry");
  JKV_CHECK_ARG(L >= 1 && L <= kPairMaxShort && L <= K1 && L <= K2, "shortlist size must lie in 1..%d",
                kPairMaxShort);
  JKV_CHECK_ARG(n_exits >= 1 && n_exits <= kPairMaxExits && n_exits <= n_recon,
                "1..%d weighted exits per block", kPairMaxExits);
  JKV_CHECK_ARG(exit_slots && exit_weights && exit_has_second, "null exit description");
  JKV_CHECK_ARG(H * N < ((int64_t)1 << 33), "block-refinement rows too many");
  if (N == 0) return JKV_OK;
  JKV_CHECK_ARG(states && recon && first_table && second_table && first_shortlist && second_shortlist && first_out &&
                    second_out,
                "null buffer");
  PairArgs a = {};
  a.x = states;
  a.recon = recon;
  a.H = H; a.N = N; a.D = D;
  a.n_exits = n_exits;
  for (int m = 0; m < n_exits; ++m) {
    JKV_CHECK_ARG(exit_slots[m] >= 0 && exit_slots[m] < n_recon, "exit slot outside the reconstruction stack");
    JKV_CHECK_ARG(exit_weights[m] >= 0.f, "exit weights must be non-negative");
    a.slot[m] = exit_slots[m];
    a.weight[m] = exit_weights[m];
    a.second[m] = exit_has_second[m] != 0;
  }
  a.t1 = first_table; a.t2 = second_table;
  a.K1 = K1; a.K2 = K2;
  a.sl1 = first_shortlist; a.sl2 = second_shortlist;
  a.L = (int32_t)L;
  a.out1 = first_out; a.out2 = second_out;
  const bool vec4 = D % 4 == 0 && ((uintptr_t)states % 16 == 0) && ((uintptr_t)recon % 16 == 0) && ((uintptr_t)first_table % 16 == 0) &&
                    ((uintptr_t)second_table % 16 == 0);
  const dim3 grid((uint32_t)ceil_div(H * N, 4));
  if (vec4) {
    hipLaunchKernelGGL(pair_block_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, a);
  } else {
    hipLaunchKernelGGL(pair_block_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, a);
  }
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}
