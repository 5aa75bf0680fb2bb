// Grouped residual-VQ / grouped-CQ encode on MFMA for gfx950: fp16 states,
// group dimension d in {4, 8}, K = 256 codewords, S in {1, 2} stages, no
// whitener (closed_loop_vq.py:52-76,343-409; cq_tac.py:64-113).
//
// Distances.  A workgroup of 4 waves owns one (head, group) problem and a
// range of rows.  Every stage runs on v_mfma_f32_32x32x16_f16: 32 codewords
// (A rows i) against 32 rows (B columns j), two row tiles per wave.  The
// contraction packs the codeword c, its split norm |c|^2/2 and the row's
// bias beta = (|r|^2 + delta)/2, so that with C = 0
//     D[i][j] = c_i.r_j - |c_i|^2/2 - beta_j = -(|r_j - c_i|^2 + delta_j)/2 < 0
// exactly in the products and in fp32 in the sum.  A lane reads A slots
// 0-7 (lanes 0-31: the codeword plane) or 8-15 (lanes 32-63: the norm plane
// [n1_hi, n1_lo, 16, 16, n2_hi, n2_lo, 16, 16]); B slot group 0 is x (d=4:
// [x, 0]; stage 2 at d=4: [x, -c1]) and group 1 the stage's bias words
// (-1, -1, -beta_hi/16, -beta_lo/16) in half s of the word.  Stage 2 at
// d = 8 needs x and -c1 in 16 slots besides the bias, so it adds a second
// MFMA with B = [-c1 | 0] into the first one's accumulator.
//
// Argmin without a tag per distance.  Negative floats order like their
// unsigned bit patterns, smallest distance = smallest pattern.  The output
// layout of the 32x32 product gives lane (h, j) elements el = 0..15 of row j
// for A rows i = 8(el/4) + 4h + el%4.  The planes are stored in "MFMA
// order": slot 32c + i of chunk c holds codeword 128h(i) + 16c + el(i), so a
// lane half h sees codewords 128h..128h+127 and, within a lane, element el
// of chunk c is codeword 128h + 16c + el.  Per chunk and tile a lane folds
// each run of 8 elements (one "octet", codewords 128h + 8o .. +7, o = 2c +
// {0,1}) with three v_min3 and one v_min, tags the octet minimum with o in
// its low 5 bits (h joins as bit 4 before the cross-lane step) and keeps the
// running minimum: 11 VALU operations per 16 distances, against 24 for a
// tag per distance.  The row's winning octet is then re-scored exactly on
// VALU (8 codewords, fp32 dot products from LDS) and its lowest-distance
// codeword taken, ties to the lowest index.  Keys keep 27 bits of the
// distance (2^-18 relative); the re-scored distances are full fp32.
//
// Launch forms: one encode, a token's K and V, or up to 64 encodes of one
// geometry (a whole cache) whose workgroups run back to back in one grid,
// so the table staging of one job's first workgroups overlaps the last
// workgroups of the job before.
//
// delta = 2^-8 (|r|^2 + max|c|^2) keeps every D negative despite fp32
// rounding; it is common to all codewords of a row, so it never changes
// their order.  Stage 2's |x - c1|^2 is read off stage 1's re-scored
// distance (-2 D - delta_1) and its delta widened by 2^-10 delta_1.
#include "encode_args.h"

namespace jkv {

namespace {

__device__ __forceinline__ uint32_t umin3(uint32_t a, uint32_t b, uint32_t c) {
  return min(min(a, b), c);
}

// codeword index -> its slot in the MFMA-ordered planes
__device__ __forceinline__ int mfma_slot(int k) {
  const int h = k >> 7, c = (k >> 4) & 7, el = k & 15;
  return 32 * c + 8 * (el >> 2) + 4 * h + (el & 3);
}

// sum_e a[e] b[e] over the first 2*PAIRS fp16 lanes, added to acc in fp32
template <int PAIRS>
__device__ __forceinline__ float dot_f16(half8 a, half8 b, float acc) {
#pragma unroll
  for (int e = 0; e < 2 * PAIRS; e += 2) {
    half2v x = {a[e], a[e + 1]};
    half2v y = {b[e], b[e + 1]};
    acc = __builtin_amdgcn_fdot2(x, y, acc, false);
  }
  return acc;
}

// lanes 32-63 of p trade places with lanes 0-31 of q, dword by dword:
// afterwards p = [p_0..31 | q_0..31] and q = [p_32..63 | q_32..63]
__device__ __forceinline__ void swap_halves(half8& p, half8& q) {
  uint4 a = __builtin_bit_cast(uint4, p);
  uint4 b = __builtin_bit_cast(uint4, q);
  auto r0 = __builtin_amdgcn_permlane32_swap(a.x, b.x, false, false);
  auto r1 = __builtin_amdgcn_permlane32_swap(a.y, b.y, false, false);
  auto r2 = __builtin_amdgcn_permlane32_swap(a.z, b.z, false, false);
  auto r3 = __builtin_amdgcn_permlane32_swap(a.w, b.w, false, false);
  a = uint4{(uint32_t)r0[0], (uint32_t)r1[0], (uint32_t)r2[0], (uint32_t)r3[0]};
  b = uint4{(uint32_t)r0[1], (uint32_t)r1[1], (uint32_t)r2[1], (uint32_t)r3[1]};
  p = __builtin_bit_cast(half8, a);
  q = __builtin_bit_cast(half8, b);
}

__device__ __forceinline__ half8 neg_h8(half8 v) {
  uint4 y = __builtin_bit_cast(uint4, v);
  y.x ^= 0x80008000u;
  y.y ^= 0x80008000u;
  y.z ^= 0x80008000u;
  y.w ^= 0x80008000u;
  return __builtin_bit_cast(half8, y);
}

// maximum of v over this lane's 16-lane row, in every lane of the row
// (quad swaps, then half-row and row mirrors: VALU with DPP, no LDS trip)
__device__ __forceinline__ uint32_t row_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));  // row_half_mirror
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));  // row_mirror
  return v;
}

static const int kRowsPerWave = 64;
// largest row range per workgroup
static const int64_t kMaxRowsPerWg = 4096;

}  // namespace

// launch forms: one job, a pair of jobs (a token's K and V), or many jobs of
// one geometry (the layers of a cache)
enum GroupedMode { kOneJob = 0, kPairJobs = 1, kManyJobs = 2 };
template <int MODE> struct GroupedArgsOf { using type = MfmaArgs; };
template <> struct GroupedArgsOf<kManyJobs> { using type = MfmaManyArgs; };

template <int D, int S, int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
void rvq_encode_grouped(typename GroupedArgsOf<MODE>::type m) {
  static_assert(D == 4 || D == 8, "group dimension 4 or 8");
  static_assert(S == 1 || S == 2, "one or two stages");
  const uint32_t L0 = xcd_remap(blockIdx.x, gridDim.x);
  // this block's job: its geometry, its logical block L within the job and
  // its buffers (all wave-uniform)
  uint32_t L;
  const MfmaJob* mjp;
  const void* states_v;
  const float* tables;
  uint8_t* codes_out;
  void* recon1;
  void* recon2;
  if constexpr (MODE == kManyJobs) {
    const uint32_t per = (uint32_t)m.per_job;
    uint32_t jb = L0 / per;
    L = L0 - jb * per;
    if (jb >= (uint32_t)m.n_jobs) {  // grid padding: stages the last job's tables, then leaves
      jb = (uint32_t)m.n_jobs - 1u;
      L = 0xFFFFFFFFu;
    }
    mjp = &m.shape;
    const MfmaJobBuffers& bf = m.buf[jb];
    states_v = bf.states;
    tables = bf.tables;
    codes_out = bf.codes;
    recon1 = bf.recon_depth[0];
    recon2 = bf.recon_depth[1];
  } else {
    const int jb = MODE == kPairJobs && (int64_t)L0 >= m.split ? 1 : 0;
    L = jb ? L0 - (uint32_t)m.split : L0;
    mjp = &m.job[jb];
    states_v = mjp->e.states;
    tables = mjp->e.tables;
    codes_out = mjp->e.codes;
    recon1 = mjp->recon_depth[0];
    recon2 = mjp->recon_depth[1];
  }
  const MfmaJob& mj = *mjp;
  const EncodeArgs& a = mj.e;

  __shared__ half8 tab_lo[S][256];  // codeword planes, MFMA order (d=4: [c, c])
  __shared__ half8 tab_hi[256];     // norm planes of both stages, MFMA order
  __shared__ __align__(16) float nrm[S][256];  // |c|^2/2 in fp32, index order
  __shared__ __align__(16) uint32_t s_rowmax[S][16];  // max |c|^2 per 16-lane row of the staging threads

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h32 = lane >> 5, j32 = lane & 31;

  // logical block: group fastest, then row chunk, then head, so that the
  // groups of one row range share its 256-byte rows and the blocks of one
  // head (its tables and rows) sit on one XCD
  // (block counts, problems and chunks fit 32 bits: host-checked)
  const uint32_t G32 = (uint32_t)a.G, nch = (uint32_t)mj.n_chunks;
  const bool active = L < (uint32_t)(a.H * a.G) * nch;
  const uint32_t Lg = active ? L / G32 : 0u;
  const uint32_t g = active ? L - Lg * G32 : 0u;
  const uint32_t h = Lg / nch;
  const uint32_t chunk = Lg - h * nch;
  const uint32_t p = h * G32 + g;

  // ---- row addressing (as the one-job kernels: 32-bit offsets, host-checked) ----
  // rows, strides and element offsets fit 32 bits (host-checked)
  const uint32_t rows = (uint32_t)(a.B * a.T);
  const uint32_t r_begin = chunk * (uint32_t)mj.rows_per_wg;
  const uint32_t r_end = min(r_begin + (uint32_t)mj.rows_per_wg, rows);
  const _Float16* states = (const _Float16*)states_v;
  const uint32_t Dfull = G32 * D;
  const uint32_t T32 = (uint32_t)a.T;
  const uint32_t head_x = h * (uint32_t)a.sh + g * D;
  const uint32_t head_c = h * (uint32_t)a.ch + g * S;
  const uint32_t out_bstride = (uint32_t)a.H * T32 * Dfull;  // reconstructions are contiguous
  const uint32_t head_o = h * T32 * Dfull + g * D;

  // a wave's 64-row slab: first row `at` = (batch b0, token t0), wave-uniform
  struct Iter {
    uint32_t at, b0, t0, xb, cb, ob;
    bool fast;
  };
  auto finish = [&](Iter& it) {
    it.fast = it.t0 + kRowsPerWave <= T32 && it.at + kRowsPerWave <= r_end;
    it.xb = it.b0 * (uint32_t)a.sb + head_x + it.t0 * (uint32_t)a.st;
    it.cb = it.b0 * (uint32_t)a.cb + head_c + it.t0 * (uint32_t)a.ct;
    it.ob = it.b0 * out_bstride + head_o + it.t0 * Dfull;
  };
  auto plan = [&](uint32_t at) {
    Iter it;
    it.at = at;
    it.b0 = at / T32;
    it.t0 = at - it.b0 * T32;
    finish(it);
    return it;
  };
  // the slab kGroupedRowsPerIter rows on, without a division
  auto advance = [&](const Iter& c) {
    Iter it;
    it.at = c.at + kGroupedRowsPerIter;
    it.b0 = c.b0;
    it.t0 = c.t0 + kGroupedRowsPerIter;
    while (it.t0 >= T32) {
      it.t0 -= T32;
      ++it.b0;
    }
    finish(it);
    return it;
  };
  // offsets of this lane's row; false for a row past the range (its offsets
  // then point at the range's first row, so every load stays in bounds)
  auto locate = [&](const Iter& it, uint32_t* xo, uint32_t* co, uint32_t* oo) -> bool {
    const uint32_t rr = (uint32_t)lane;
    if (it.fast) {
      *xo = it.xb + __umul24(rr, (uint32_t)a.st);
      *co = it.cb + __umul24(rr, (uint32_t)a.ct);
      *oo = it.ob + __umul24(rr, Dfull);
      return true;
    }
    const uint32_t row = it.at + rr;
    const bool valid = row < r_end;
    const uint32_t rw = valid ? row : r_begin;
    const uint32_t rb = rw / T32, rt = rw - rb * T32;
    *xo = rb * (uint32_t)a.sb + head_x + rt * (uint32_t)a.st;
    *co = rb * (uint32_t)a.cb + head_c + rt * (uint32_t)a.ct;
    *oo = rb * out_bstride + head_o + rt * Dfull;
    return valid;
  };
  auto load_x = [&](const Iter& it) -> half8 {
    uint32_t xo, co, oo;
    locate(it, &xo, &co, &oo);
    if constexpr (D == 8) return *(const half8*)(states + xo);
    const half4 v = *(const half4*)(states + xo);
    return half8{v[0], v[1], v[2], v[3], (half_t)0.f, (half_t)0.f, (half_t)0.f, (half_t)0.f};
  };
  // stage s's bias words (-1, -1, -(beta/16) in two fp16 halves) in half s
  auto bias_slots = [&](int s, float beta) -> half8 {
    const float beta16 = beta * (1.f / 16.f) + 0x1p-60f;
    const half_t bh = (half_t)beta16;
    const half_t bl = (half_t)(beta16 - (float)bh);
    half8 w = half8{};
    w[4 * s + 0] = (half_t)-1.f;
    w[4 * s + 1] = (half_t)-1.f;
    w[4 * s + 2] = -bh;
    w[4 * s + 3] = -bl;
    return w;
  };

  // the key mask lives in a VGPR so that each octet key is one v_and_or_b32
  // with its tag as an inline constant
  uint32_t kmask = ~31u;
  asm volatile("" : "+v"(kmask));
  const uint32_t hbit = (uint32_t)h32 << 4;

  // One stage's search: 8 chunks of 32 codewords x 2 row tiles.  b[part][t]
  // are the B operands of tile t (after swap_halves); NP = 2 adds the second
  // product.  Returns this lane's row key: distance bits | (h << 4 | octet).
  auto search = [&](int s, auto np_tag, const half8 (&b)[2][2]) -> uint32_t {
    constexpr int NP = decltype(np_tag)::value;
    const half8* ap = (h32 ? &tab_hi[0] : &tab_lo[s][0]) + j32;
    const float16v zero16 = {};
    uint32_t best[2] = {0xFFFFFFFFu, 0xFFFFFFFFu};
    float16v acc[2][2];
    half8 af = ap[0];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      acc[0][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, b[0][t], zero16, 0, 0, 0);
      if constexpr (NP == 2) acc[0][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, b[1][t], acc[0][t], 0, 0, 0);
    }
    af = ap[32];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int cur = c & 1;
      const half8 an = (c + 2 < 8) ? ap[(c + 2) * 32] : af;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (c + 1 < 8) {
          acc[cur ^ 1][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, b[0][t], zero16, 0, 0, 0);
          if constexpr (NP == 2)
            acc[cur ^ 1][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, b[1][t], acc[cur ^ 1][t], 0, 0, 0);
        }
        const float16v v = acc[cur][t];
        uint32_t e[16];
#pragma unroll
        for (int el = 0; el < 16; ++el) e[el] = __float_as_uint(v[el]);
        uint32_t m0 = umin3(e[0], e[1], e[2]);
        m0 = umin3(m0, e[3], e[4]);
        m0 = umin3(m0, e[5], e[6]);
        m0 = min(m0, e[7]);
        uint32_t m1 = umin3(e[8], e[9], e[10]);
        m1 = umin3(m1, e[11], e[12]);
        m1 = umin3(m1, e[13], e[14]);
        m1 = min(m1, e[15]);
        const uint32_t k0 = (m0 & kmask) | (uint32_t)(2 * c);
        const uint32_t k1 = (m1 & kmask) | (uint32_t)(2 * c + 1);
        best[t] = umin3(k0, k1, best[t]);
        // pin the running minimum here, so the compiler does not keep every
        // accumulator of the stage live
        asm volatile("" : "+v"(best[t]));
      }
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (c + 1 < 8) __builtin_amdgcn_sched_group_barrier(0x008, NP, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 11, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      af = an;
    }
    // row `lane`: tile lane/32; the minimum over both lane halves
    auto pr = __builtin_amdgcn_permlane32_swap(best[0] | hbit, best[1] | hbit, false, false);
    return min((uint32_t)pr[0], (uint32_t)pr[1]);
  };

  // Exact re-scoring of the row's winning octet of stage s.  u and w are the
  // row's B words of the codeword plane (w: second product, stage 2 at
  // d = 8); the score is u.c [+ w.c] - |c|^2/2 - beta, negative.  Returns the
  // winning key (score bits | octet position) and sets the code and the
  // codeword plane word.
  auto rescore = [&](int s, uint32_t key, half8 u, half8 w, bool two, float beta, int* code,
                     half8* cw) -> uint32_t {
    const int tag = (int)(key & 31u);
    const int hs = tag >> 4, oc = tag & 15;
    const int cs = oc >> 1, q = oc & 1;
    const int pbase = 32 * cs + 16 * q + 4 * hs;  // slots of codewords 4k..4k+3: pbase + 8k + 0..3
    const int ibase = 128 * hs + 8 * oc;
    const float4 n0 = *(const float4*)&nrm[s][ibase];
    const float4 n1 = *(const float4*)&nrm[s][ibase + 4];
    const float nv[8] = {n0.x, n0.y, n0.z, n0.w, n1.x, n1.y, n1.z, n1.w};
    const float nbeta = -beta;
    half8 cand[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) cand[e] = tab_lo[s][pbase + 8 * (e >> 2) + (e & 3)];
    uint32_t kk[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = nbeta - nv[e];
      if (D == 8 || s > 0) {
        acc = dot_f16<4>(u, cand[e], acc);  // d=4 stage 2: [x, -c1] . [c, c]
      } else {
        acc = dot_f16<2>(u, cand[e], acc);
      }
      if (D == 8 && two) acc = dot_f16<4>(w, cand[e], acc);
      kk[e] = (__float_as_uint(acc) & ~7u) | (uint32_t)e;
    }
    uint32_t km = umin3(kk[0], kk[1], kk[2]);
    km = umin3(km, kk[3], kk[4]);
    km = umin3(km, kk[5], kk[6]);
    km = min(km, kk[7]);
    const int e = (int)(km & 7u);
    *code = ibase + e;
    *cw = tab_lo[s][pbase + 8 * (e >> 2) + (e & 3)];
    return km;
  };

  uint32_t base = r_begin + (uint32_t)wave * kRowsPerWave;
  half8 x = half8{};
  Iter cur = plan(base);
  if (base < r_end) x = load_x(cur);
  // the first rows load while the codebooks stage
  // ---- stage the fp16-deployed codebooks: thread tid takes codeword tid ----
  {
    half8 hi = half8{};
    const int slot = mfma_slot(tid);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const float* src = tables + ((p * S + s) * 256 + tid) * D;
      half_t cw[D];
      const float4 v0 = ((const float4*)src)[0];
      cw[0] = (half_t)v0.x; cw[1] = (half_t)v0.y; cw[2] = (half_t)v0.z; cw[3] = (half_t)v0.w;
      if constexpr (D == 8) {
        const float4 v1 = ((const float4*)src)[1];
        cw[4] = (half_t)v1.x; cw[5] = (half_t)v1.y; cw[6] = (half_t)v1.z; cw[7] = (half_t)v1.w;
      }
      float nc = 0.f;
#pragma unroll
      for (int i = 0; i < D; ++i) nc = fmaf((float)cw[i], (float)cw[i], nc);
      half8 lo;
#pragma unroll
      for (int e = 0; e < 8; ++e) lo[e] = cw[e % D];
      const float halfn = 0.5f * nc;
      const half_t nhi = (half_t)halfn;
      const half_t nlo = (half_t)(halfn - (float)nhi);
      hi[4 * s + 0] = nhi;
      hi[4 * s + 1] = nlo;
      hi[4 * s + 2] = (half_t)16.f;  // against -(beta/16) in two fp16 halves
      hi[4 * s + 3] = (half_t)16.f;
      tab_lo[s][slot] = lo;
      nrm[s][tid] = halfn;
      // |c|^2 >= 0, so its bit pattern orders like the value
      const uint32_t mx = row_max_u32(__float_as_uint(nc));
      if ((tid & 15) == 0) s_rowmax[s][tid >> 4] = mx;
    }
    tab_hi[slot] = hi;
  }
  __syncthreads();
  if (!active) return;
  float ncmax[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    uint32_t mx = 0u;
#pragma unroll
    for (int q = 0; q < 16; q += 4) {
      const uint4 v = *(const uint4*)&s_rowmax[s][q];
      mx = max(max(mx, max(v.x, v.y)), max(v.z, v.w));
    }
    ncmax[s] = __uint_as_float(mx);
  }


  for (; base < r_end; base += kGroupedRowsPerIter) {
    const bool more = base + kGroupedRowsPerIter < r_end;
    const Iter nxt = advance(cur);
    uint32_t xo, co, oo;
    const bool valid = locate(cur, &xo, &co, &oo);

    // stage 1: B = [x | bias_1]
    const float rr1 = dot_f16<D / 2>(x, x, 0.f);
    const float delta1 = (rr1 + ncmax[0]) * 0x1p-8f;
    const float beta1 = (rr1 + delta1) * 0.5f;
    const half8 xs = x;
    half8 b1[2][2];
    b1[0][0] = x;
    b1[0][1] = bias_slots(0, beta1);
    swap_halves(b1[0][0], b1[0][1]);
    b1[1][0] = b1[1][1] = half8{};
    // x is consumed: the next iteration's row loads during this one
    if (more) x = load_x(nxt);

    uint32_t key1 = search(0, std::integral_constant<int, 1>{}, b1);
    int code1;
    half8 c1;
    const uint32_t win1 = rescore(0, key1, xs, half8{}, false, beta1, &code1, &c1);
    uint32_t code = (uint32_t)code1;
    if (recon1 != nullptr && valid) {
      _Float16* op = (_Float16*)recon1 + oo;
      if constexpr (D == 8) {
        *(half8*)op = c1;
      } else {
        *(half4*)op = half4{c1[0], c1[1], c1[2], c1[3]};
      }
    }
    if constexpr (S == 2) {
      // stage 2 on the residual x - c1: |x - c1|^2 from stage 1's score
      const float rr2 = fmaxf(-2.f * __uint_as_float(win1 & ~7u) - delta1, 0.f);
      const float delta2 = (rr2 + ncmax[1]) * 0x1p-8f + delta1 * 0x1p-10f;
      const float beta2 = (rr2 + delta2) * 0.5f;
      const half8 negc1 = neg_h8(c1);
      half8 u2 = xs, w2 = half8{};
      half8 b2[2][2];
      if constexpr (D == 8) {
        w2 = negc1;
        b2[0][0] = xs;
        b2[0][1] = bias_slots(1, beta2);
        swap_halves(b2[0][0], b2[0][1]);
        b2[1][0] = negc1;
        b2[1][1] = half8{};
        swap_halves(b2[1][0], b2[1][1]);
      } else {
        u2 = half8{xs[0], xs[1], xs[2], xs[3], negc1[0], negc1[1], negc1[2], negc1[3]};
        b2[0][0] = u2;
        b2[0][1] = bias_slots(1, beta2);
        swap_halves(b2[0][0], b2[0][1]);
        b2[1][0] = b2[1][1] = half8{};
      }
      uint32_t key2;
      if constexpr (D == 8) {
        key2 = search(1, std::integral_constant<int, 2>{}, b2);
      } else {
        key2 = search(1, std::integral_constant<int, 1>{}, b2);
      }
      int code2;
      half8 c2;
      rescore(1, key2, u2, w2, D == 8, beta2, &code2, &c2);
      code |= (uint32_t)code2 << 8;
      // depth-2 reconstruction fp16(fp32(c1) + fp32(c2)): the sum of two fp16
      // words is exact in fp32 or, when it is not, too small to move the fp16
      // rounding, so one fp16 add gives the same bits
      if (recon2 != nullptr && valid) {
        const half8 dec = c1 + c2;
        _Float16* op = (_Float16*)recon2 + oo;
        if constexpr (D == 8) {
          *(half8*)op = dec;
        } else {
          *(half4*)op = half4{dec[0], dec[1], dec[2], dec[3]};
        }
      }
    }
    if (valid) {
      uint8_t* cp = codes_out + co;
      if constexpr (S == 1) {
        cp[0] = (uint8_t)code;
      } else {
        *(uint16_t*)cp = (uint16_t)code;
      }
    }
    cur = nxt;
  }
}

// ---------------------------------------------------------------------------
// rows per workgroup: amortise the codebook staging while the launch still
// has `min_blocks` workgroups
static MfmaJob grouped_job(const EncodeArgs& e, int64_t min_blocks) {
  MfmaJob j = {};
  j.e = e;
  for (int i = 0; i < e.n_exits; ++i) j.recon_depth[e.exit_depth[i] - 1] = e.recon[i];
  const int64_t rows = e.B * e.T;
  const int64_t P = e.H * e.G;
  int64_t rpw = kMaxRowsPerWg;
  while (rpw > kGroupedRowsPerIter && P * ceil_div(rows, rpw) < min_blocks) rpw >>= 1;
  j.rows_per_wg = rpw;
  j.n_chunks = ceil_div(rows, rpw);
  return j;
}

template <int D, int S>
static int launch_grouped_t(const EncodeArgs& e, const EncodeArgs* e2, hipStream_t stream) {
  MfmaArgs m = {};
  // one job fills 256 CUs x 4 workgroups by itself
  m.job[0] = grouped_job(e, 256 * 4);
  const int64_t per_job = e.H * e.G * m.job[0].n_chunks;
  int64_t nblocks = per_job;
  m.split = per_job;
  if (e2 != nullptr) {
    m.job[1] = grouped_job(*e2, 256 * 4);
    nblocks += per_job;
  } else {
    m.job[1] = m.job[0];
  }
  if (nblocks > 8) nblocks = ceil_div(nblocks, 8) * 8;  // xcd_remap needs a multiple of 8
  JKV_CHECK_ARG(nblocks < (int64_t)1 << 31, "grid too large");
  if (e2 == nullptr) {
    m.split = nblocks;
    hipLaunchKernelGGL((rvq_encode_grouped<D, S, kOneJob>), dim3((uint32_t)nblocks), dim3(256), 0, stream, m);
  } else {
    hipLaunchKernelGGL((rvq_encode_grouped<D, S, kPairJobs>), dim3((uint32_t)nblocks), dim3(256), 0, stream, m);
  }
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

template <int D, int S>
static int launch_grouped_many_t(const EncodeArgs* jobs, int n, hipStream_t stream) {
  MfmaManyArgs m = {};
  // the jobs together fill the chip: rows per workgroup only need to leave
  // every CU several workgroups' worth
  m.shape = grouped_job(jobs[0], (256 * 4 * 4 + n - 1) / n);
  m.n_jobs = n;
  m.per_job = jobs[0].H * jobs[0].G * m.shape.n_chunks;
  for (int j = 0; j < n; ++j) {
    const MfmaJob one = grouped_job(jobs[j], (256 * 4 * 4 + n - 1) / n);
    m.buf[j].states = jobs[j].states;
    m.buf[j].tables = jobs[j].tables;
    m.buf[j].codes = jobs[j].codes;
    m.buf[j].recon_depth[0] = one.recon_depth[0];
    m.buf[j].recon_depth[1] = one.recon_depth[1];
  }
  int64_t nblocks = m.per_job * n;
  if (nblocks > 8) nblocks = ceil_div(nblocks, 8) * 8;  // xcd_remap needs a multiple of 8
  JKV_CHECK_ARG(nblocks < (int64_t)1 << 31, "grid too large");
  hipLaunchKernelGGL((rvq_encode_grouped<D, S, kManyJobs>), dim3((uint32_t)nblocks), dim3(256), 0, stream, m);
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

int launch_grouped(const EncodeArgs& e, const EncodeArgs* e2, hipStream_t stream) {
  if (e.d == 8) return e.S == 1 ? launch_grouped_t<8, 1>(e, e2, stream) : launch_grouped_t<8, 2>(e, e2, stream);
  return e.S == 1 ? launch_grouped_t<4, 1>(e, e2, stream) : launch_grouped_t<4, 2>(e, e2, stream);
}

int launch_grouped_many(const EncodeArgs* jobs, int n, hipStream_t stream) {
  JKV_CHECK_ARG(n >= 1 && n <= kMaxManyJobs, "1 to %d jobs per launch", kMaxManyJobs);
  const EncodeArgs& e = jobs[0];
  if (e.d == 8) return e.S == 1 ? launch_grouped_many_t<8, 1>(jobs, n, stream) : launch_grouped_many_t<8, 2>(jobs, n, stream);
  return e.S == 1 ? launch_grouped_many_t<4, 1>(jobs, n, stream) : launch_grouped_many_t<4, 2>(jobs, n, stream);
}

}  // namespace jkv
