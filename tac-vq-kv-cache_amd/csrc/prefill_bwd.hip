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
// The entry point first writes the rotated queries q_rot (the reference's
// fp16 rotary at each row's position) into its workspace, once for all key
// blocks.  Then one workgroup of 4 waves per (batch row, kv head, block of
// 128 keys) and run of query tiles; wave w owns keys 32w..32w+31 of the block
// and keeps their rotated K̂ in registers as MFMA B operands and their dV̂ in
// accumulators.  The workgroup walks (32-row query tile, query head of the
// group) steps; each step's q_rot and dO rows go straight from global memory
// into LDS (buffer loads with the LDS destination, two steps ahead into
// three buffers, 16-byte chunks XOR-swizzled per row) and serve all four
// waves; its lse goes through a register.  Per step and wave, on
// v_mfma_f32_16x16x32_f16:
//   S[row][key]    = Q K̂ᵀ      A = q_rot rows from LDS, B = the wave's K̂
//   P              = exp2(S log2e/sqrt(D) - lse log2e), masked, fp16
//   dV̂[key][dim] += Pᵀ dO      A = P read straight off the S accumulators
//                              (two 16-row tiles interleaved into the 32
//                              contraction slots), B = dOᵀ read from the
//                              row-major dO tile with ds_read_b64_tr_b16, in
//                              the same slot order
// Steps where none of a wave's keys is visible skip its arithmetic.  168
// registers: three workgroups per CU.
#include <math.h>

#include <type_traits>

#include "jkv_common.h"
#include "rotary.h"

namespace jkv {

static const int kBD = 128;            // head dim
static const int kBKeys = 128;         // keys per workgroup (32 per wave)
static const int kBRows = 32;          // query rows per step
static const int kBThreads = 256;      // 4 waves

struct ValueGradArgs {
  const _Float16* q;  // pre-RoPE q; for the value kernel the rotated q_rot, contiguous [B,QH,T,128]
  int64_t qsb, qsh, qst;
  const _Float16* k;
  int64_t ksb, ksh, kst;
  const _Float16* dout;
  int64_t dsb, dsh, dst;
  const _Float16* v;  // key gradient only: V̂ [B,KVH,T,D]
  int64_t vsb, vsh, vst;
  const float* lse;    // [B,QH,T]
  const float* delta;  // key gradient only: rowsum(dO * O) [B,QH,T]
  int64_t B, QH, KVH, T;
  const int32_t* start;
  int64_t window;
  const _Float16* rope;
  int64_t rope_len;
  float* dv;  // [B,KVH,T,D] fp32 contiguous, or the chunk's partial slot
  float* dk;  // the same for dK̂ when the walk forms both gradients
  int32_t nq;
  int32_t chunk_tiles;  // query tiles per chunk (the query rows are split in chunks of tiles)
  int64_t slot_stride;  // elements between the chunks' partial slots (0: one chunk)
  int32_t slots;        // partial slots (grid rows) of the key-block kernels
};

// The 32-row query tiles (absolute: tile t holds rows 32t..32t+31) that the
// workgroup of key block key0 in grid row y walks, top tile first.  The rows
// that see some key of the block are [key0, key0 + 127 + window) within
// [0, T): tiles [tf, tl].  The query rows are split in absolute chunks of
// `per` tiles; a block meets at most `slots` consecutive chunks, and chunk c
// runs in grid row c mod slots, so the workgroups that walk one chunk for the
// blocks of a (batch row, kv head) sit side by side in the grid and read each
// q/dO tile at about the same time.
struct TileRun {
  int64_t top, n;
};
__host__ __device__ inline void block_tiles(int64_t key0, int64_t T, int64_t window, int keys, int64_t* tf,
                                            int64_t* tl) {
  int64_t rend = key0 + keys - 1 + window;
  if (rend > T || rend < 0) rend = T;
  *tf = key0 / kBRows;
  *tl = (rend - 1) / kBRows;
}
__device__ inline TileRun tile_run(int64_t key0, int64_t T, int64_t window, int keys, int64_t per, int slots,
                                  int y) {
  int64_t tf, tl;
  block_tiles(key0, T, window, keys, &tf, &tl);
  const int64_t c_lo = tf / per;
  const int64_t c = c_lo + ((int64_t)y - c_lo % slots + slots) % slots;
  const int64_t lo = tf > c * per ? tf : c * per;
  const int64_t hi = tl < c * per + per - 1 ? tl : c * per + per - 1;
  return TileRun{hi, hi >= lo ? hi - lo + 1 : 0};
}

// Rotated rows for the gradient kernels: out[b,h,t,:] = the reference's fp16
// rotary of q[b,h,t,:] (queries, or keys) at position start[b] + t (clamped
// to the table), contiguous [B,H,T,128].  One thread per (row, rotary chunk
// pair p): dims [8p, +8) and their partners [64 + 8p, +8).  Grid
// (ceil(8T/256), H, B).
__global__ __launch_bounds__(256) void rotate_rows_kernel(const _Float16* __restrict__ q, int64_t qsb,
                                                                int64_t qsh, int64_t qst, int64_t T,
                                                                const int32_t* __restrict__ start,
                                                                const _Float16* __restrict__ rope,
                                                                int64_t rope_len, _Float16* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t t = i >> 3;
  if (t >= T) return;
  const int p = (int)(i & 7);
  const int64_t h = blockIdx.y, b = blockIdx.z;
  int64_t pos = (int64_t)start[b] + t;
  pos = pos < 0 ? 0 : (pos < rope_len - 1 ? pos : rope_len - 1);
  const _Float16* src = q + b * qsb + h * qsh + t * qst + 8 * p;
  half8 cs, sn, r0, r1;
  load_trig8(rope + pos * kRopeRow, 8 * p, &cs, &sn);
  rope16(*(const half8*)src, *(const half8*)(src + 64), cs, sn, &r0, &r1);
  _Float16* dst = out + ((b * gridDim.y + h) * T + t) * kBD + 8 * p;
  *(half8*)dst = r0;
  *(half8*)(dst + 64) = r1;
}

// transposing LDS read of the 8-byte piece at LDS byte address addr: in each
// 16-lane block, lane 4j + e receives element e of the pieces that the
// block's lanes j, j+4, j+8, j+12 address (ds_read_b64_tr_b16)
typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4v;
__device__ __forceinline__ half4 lds_read_tr16(uint32_t addr) {
  return __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(size_t)addr));
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(size_t)(const void __attribute__((address_space(3)))*)p;
}

// Staged rows (q_rot, dO, K̂_rot and V̂ tiles, 32 rows x 256 bytes) hold their
// 16-byte chunks XOR-swizzled: chunk j of row r sits in slot j ^ f(r), with f
// chosen by how the tile is read.  An A-operand read (ds_read_b128) takes 16
// consecutive rows at one chunk: f = r & 15.  A transposing read
// (ds_read_b64_tr_b16) takes chunks 2t, 2t + 1 of 8 consecutive rows: f =
// 2 (r & 7).  A tile read both ways takes f = 2 (r & 7) + ((r >> 3) & 1).
// Each keeps a read's lanes on distinct banks, or nearly (measured: the
// both-ways form costs the value kernel ~3 % when used for its tiles).
enum Swz { kSwzA, kSwzT, kSwzAT };
template <Swz W>
__device__ __forceinline__ uint32_t row_slot(int r, int j) {
  const int f = W == kSwzA ? (r & 15) : W == kSwzT ? 2 * (r & 7) : ((r & 7) << 1) | ((r >> 3) & 1);
  return (uint32_t)(j ^ f);
}

// The key-block walk of the value gradient (MODE kWalkV), of the key gradient
// (kWalkK) and of both at once (kWalkKV):
//   V   dV̂ += Pᵀ dO
//   K   dP = dO V̂ᵀ, dS = P (dP - delta_row), dK̂_rot += dSᵀ Q_rot / sqrt(D),
//       then the rotary's transpose at the key's position
//   KV  both, from one S and one dP per step
// (delta = rowsum(dO * O) from the query kernel).  For the key gradient the
// wave's V̂ rows join its K̂ as B operands, the staged dO rows are the A
// operand of dP, and Q_rotᵀ for the last product comes off the staged q
// rows with the same transposing reads that give dOᵀ to the value gradient.
// Each wave owns KT 16-key tiles (a workgroup 64 KT keys): KT = 2 for one
// gradient, KT = 1 for both, which keeps both sets of accumulators within
// three waves per SIMD.
enum WalkMode { kWalkV, kWalkK, kWalkKV };
template <int MODE, int KT>
__device__ __forceinline__ void kv_grad_walk(const ValueGradArgs& a) {
  constexpr bool kV = MODE != kWalkK, DK = MODE != kWalkV;  // forms dV̂ / dK̂
  constexpr int kKeys = 64 * KT;                           // keys per workgroup
  constexpr int NA = (kV ? 1 : 0) + (DK ? 1 : 0);          // accumulator sets
  constexpr int iV = 0, iK = kV ? 1 : 0;
  __shared__ __align__(1024) _Float16 q_lds[3][kBRows * kBD];
  __shared__ __align__(1024) _Float16 d_lds[3][kBRows * kBD];
  __shared__ __align__(16) float l_lds[2][kBRows];
  __shared__ __align__(16) float x_lds[DK ? 2 : 1][kBRows];  // delta (DK)
  // q rows: A operand of S (and, DK, transposed for dK); dO rows: transposed
  // for dV and (DK) the A operand of dP
  constexpr Swz kQSwz = DK ? kSwzAT : kSwzA, kDSwz = DK ? (kV ? kSwzAT : kSwzA) : kSwzT;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the step tests below branch on it
  const int ln = lane & 15, lg = lane >> 4;
  const int NQ = a.nq;
  const int64_t nkb = ceil_div(a.T, kKeys);
  // key blocks fastest: the blocks of one (batch row, kv head) share its q and
  // dO rows in one XCD's L2
  const uint32_t bid = xcd_remap(blockIdx.x, gridDim.x);
  const int chunk = blockIdx.y;  // grid row: the chunk of query tiles (chunk index mod slots)
  const int64_t kb = bid % (uint32_t)nkb;
  const int64_t kvh = (bid / (uint32_t)nkb) % (uint32_t)a.KVH;
  const int64_t b = bid / ((uint32_t)nkb * (uint32_t)a.KVH);
  const int64_t key0 = kb * kKeys;
  const int64_t kw0 = key0 + 16 * KT * wave;  // this wave's first key
  const int64_t p0 = a.start[b];
  const float scale2 = 1.4426950408889634f / sqrtf((float)kBD);
  const int64_t rope_last = a.rope_len - 1;
  auto rope_row = [&](int64_t pos) -> const _Float16* {
    return a.rope + (pos < 0 ? 0 : (pos < rope_last ? pos : rope_last)) * kRopeRow;
  };
  const half8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};

  // ---- the wave's rotated keys as B operands: kop[kt][c] = dims
  // [32c + 8lg, +8) of key kw0 + 16kt + ln (chunks c and c+2 are rotary
  // partners); DK: its V̂ rows the same way (no rotary) ----
  half8 kop[KT][4], vop[KT][4];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
    const int64_t key = kw0 + 16 * kt + ln;
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
    if constexpr (DK) {
      const _Float16* vp = a.v + b * a.vsb + kvh * a.vsh + (ok ? key : 0) * a.vst;
#pragma unroll
      for (int c = 0; c < 4; ++c) vop[kt][c] = ok ? *(const half8*)(vp + 32 * c + 8 * lg) : zero8;
    }
  }
  float4v acc[NA][KT][8];  // dV̂ (set iV) and dK̂ (set iK)[key kw0 + 16kt + 4lg + e][dim 16dt + ln]
#pragma unroll
  for (int i = 0; i < NA; ++i)
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[i][kt][dt] = float4v{0.f, 0.f, 0.f, 0.f};

  // this workgroup's query tiles, top first (none: no slot to write)
  const TileRun run = tile_run(key0, a.T, a.window, kKeys, a.chunk_tiles, a.slots, chunk);
  if (run.n == 0) return;
  const int64_t t_top = run.top;
  const int32_t nsteps = (int32_t)run.n * NQ;

  // ---- staging.  A step's q_rot and dO rows go global -> LDS directly
  // (buffer_load_dwordx4 ... lds: lane i of an instruction lands at its LDS
  // base + 16 i, so an instruction fills 4 rows), two steps ahead into three
  // buffers: wave w fills rows 8w..8w+7 with two instructions per tensor,
  // lane -> row 8w + 4i + lane/16, slot lane%16, loading the chunk that
  // belongs in that slot.  (The MUBUF form: the compiler's wait counting
  // takes global_load_lds for an access to both memories and drains every
  // LDS read behind it.)  The step's lse (and delta) go through registers
  // one step ahead, loaded before the step-ahead copies so that one wait
  // (vmcnt 4) covers the next step's copies, lse and delta.  A load's
  // address is the (batch row, kv head)'s buffer, a uniform tile offset and
  // a per-thread offset that also carries the head (one add per step); they
  // fit 31 bits (host-checked).  Rows past T read the step's first row
  // (every step's first row is in range; only the top tile has rows past T)
  // and are staged with lse = +inf, which gives them weight exactly 0 ----
  const int srow = 8 * wave + (lane >> 4), slot = lane & 15;
  const int32_t T32 = (int32_t)a.T;
  // q_rot is contiguous [B,QH,T,128]
  const uint32_t q_head = (uint32_t)a.T * (2u * kBD), d_head = (uint32_t)a.dsh * 2u, l_head = (uint32_t)a.T * 4u;
  const __amdgpu_buffer_rsrc_t q_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.q + ((b * a.QH + kvh * NQ) * a.T) * kBD), (short)0, (int)(NQ * a.T * 2 * kBD), 0x00020000);
  const __amdgpu_buffer_rsrc_t d_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.dout + b * a.dsb + kvh * NQ * a.dsh), (short)0,
      (int)(((NQ - 1) * a.dsh + (a.T - 1) * a.dst + kBD) * 2), 0x00020000);
  const int64_t lrow0 = (b * a.QH + kvh * NQ) * a.T;
  const char* l_b = (const char*)(a.lse + lrow0);
  const char* x_b = DK ? (const char*)(a.delta + lrow0) : nullptr;
  // copies: the next step to copy
  int fh = 0;
  int32_t fr0 = (int32_t)(t_top * kBRows);  // first row of its tile
  uint32_t q_tile, d_tile;                  // the tile's byte offsets (uniform)
  uint32_t qo[2], dof[2];
  auto aim = [&]() {
    q_tile = (uint32_t)fr0 * (2u * kBD);
    d_tile = (uint32_t)fr0 * (uint32_t)a.dst * 2u;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = srow + 4 * i;
      const uint32_t rr = fr0 + r < T32 ? (uint32_t)r : 0u;
      qo[i] = rr * (2u * kBD) + 16u * row_slot<kQSwz>(r, slot);
      dof[i] = rr * (uint32_t)a.dst * 2u + 16u * row_slot<kDSwz>(r, slot);
    }
  };
  aim();
  auto copy = [&](int buf) {
    char* qd = (char*)q_lds[buf] + 2048 * wave;
    char* dd = (char*)d_lds[buf] + 2048 * wave;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(q_rsrc, (void __attribute__((address_space(3)))*)(qd + 1024 * i), 16,
                                               qo[i], q_tile, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(d_rsrc, (void __attribute__((address_space(3)))*)(dd + 1024 * i), 16,
                                               dof[i], d_tile, 0, 0);
    }
    if (++fh == NQ) {
      fh = 0;
      fr0 -= kBRows;
      aim();
    } else {
      qo[0] += q_head;
      qo[1] += q_head;
      dof[0] += d_head;
      dof[1] += d_head;
    }
  };
  // lse (and delta): the next step to load, in every wave (uniform wait
  // counts); the first kBRows threads keep theirs
  int lh = 0;
  int32_t lr0 = (int32_t)(t_top * kBRows);
  uint32_t l_tile, l_off;
  auto aim_l = [&]() {
    l_tile = (uint32_t)lr0 * 4u;
    l_off = tid < kBRows && lr0 + tid < T32 ? 4u * tid : 0u;
  };
  aim_l();
  float lreg = 0.f, xreg = 0.f;
  auto load_lse = [&]() {
    lreg = *(const float*)(l_b + l_tile + l_off);
    if constexpr (DK) xreg = *(const float*)(x_b + l_tile + l_off);
    if (++lh == NQ) {
      lh = 0;
      lr0 -= kBRows;
      aim_l();
    } else {
      l_off += l_head;
    }
  };
  // after the wait: the staged step's lse (log2 units; +inf past T) and delta
  auto put_lse = [&](int buf, int32_t srow0) {
    if (tid < kBRows) {
      l_lds[buf][tid] = srow0 + tid < T32 ? lreg * 1.4426950408889634f : __builtin_inff();
      if constexpr (DK) x_lds[buf][tid] = xreg;
    }
  };
  // s_waitcnt vmcnt(4), leaving the other counters alone (gfx9 encoding:
  // vmcnt [3:0], expcnt [6:4] = 7, lgkmcnt [11:8] = 15)
  constexpr int kWaitVm4 = 4 | (7 << 4) | (15 << 8);

  load_lse();
  copy(0);
  if (nsteps > 1) {
    copy(1);
    __builtin_amdgcn_s_waitcnt(kWaitVm4);  // step 0's copies and lse have landed
  } else {
    __builtin_amdgcn_s_waitcnt(0);
  }
  put_lse(0, (int32_t)(t_top * kBRows));
  __syncthreads();

  int ch = 0;                               // head of the step being computed
  int32_t r0 = (int32_t)(t_top * kBRows);   // and its first row
  const int32_t kw32 = (int32_t)kw0;
  const int32_t win = a.window < 0x40000000 ? (int32_t)a.window : 0x40000000;
  // per-lane LDS byte offsets of the transposing reads: rows 4lg + ln/4
  // (+16), dims 16dt + 4(ln%4), 8 bytes
  const int tr_row = 4 * lg + (ln >> 2);
  const uint32_t tr_off = (uint32_t)tr_row * 256u + 8u * (ln & 1);
  int buf = 0, buf2 = 2;  // buffers of this step and of step + 2
  // one step; MORE: a step follows, MORE2: two follow (the steady state, with
  // no tests of its own; the last two steps are peeled)
  for (int32_t step = 0; step < nsteps; ++step) {
    const bool more = step + 1 < nsteps, more2 = step + 2 < nsteps;
    // the lse of step + 1, then step + 2's copies into the buffer that step
    // - 1 used (freed by the last barrier)
    if (more) load_lse();
    if (more2) copy(buf2);
    // does any row of the step see any of this wave's keys?
    const bool any = r0 + kBRows - 1 >= kw32 && r0 - (kw32 + 16 * KT - 1) < win && kw32 < T32;
    if (any) {
      const char* ql = (const char*)q_lds[buf];
      const char* dl = (const char*)d_lds[buf];
      // ---- S[row][key] (and DK: dP[row][key] = dO V̂ᵀ): 2 row tiles x KT
      // key tiles; A = the staged rows (row 16rg + ln, chunk 4c + lg) ----
      float4v sacc[2][KT], dpacc[2][KT];
#pragma unroll
      for (int rg = 0; rg < 2; ++rg) {
        half8 qa[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
          qa[c] = *(const half8*)(ql + (16 * rg + ln) * 256 + 16 * row_slot<kQSwz>(ln, 4 * c + lg));
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
          sacc[rg][kt] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < 4; ++c)
            sacc[rg][kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[c], kop[kt][c], sacc[rg][kt], 0, 0, 0);
        }
      }
      if constexpr (DK) {
#pragma unroll
        for (int rg = 0; rg < 2; ++rg) {
          half8 da[4];
#pragma unroll
          for (int c = 0; c < 4; ++c)
            da[c] = *(const half8*)(dl + (16 * rg + ln) * 256 + 16 * row_slot<kDSwz>(ln, 4 * c + lg));
#pragma unroll
          for (int kt = 0; kt < KT; ++kt) {
            dpacc[rg][kt] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 4; ++c)
              dpacc[rg][kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(da[c], vop[kt][c], dpacc[rg][kt], 0, 0, 0);
          }
        }
      }
      // ---- P, masked: element (rg, kt, e) is row r0 + 16rg + 4lg + e, key
      // kw0 + 16kt + ln; pa[kt] contraction slot 4rg + e (of lane group lg)
      // <-> row 16rg + 4lg + e ----
      const bool full = r0 >= kw32 + 16 * KT - 1 && r0 + kBRows - 1 - kw32 < win && r0 + kBRows <= T32;
      const int base = r0 - kw32 + 4 * lg - ln;  // row - key = base + 16rg + e - 16kt
      // (rows past T hold the step's first row and lse +inf, keys past T
      // zeros: their scores are finite and their weights 0, rows by the
      // lse and keys by the mask, since a visible key is at most the row)
      // P (for dV̂) and dS (for dK̂) in A order
      half8 pa[KT], dsa[KT];
      auto make_p = [&](auto masked_tag) {
        constexpr bool masked = decltype(masked_tag)::value;
#pragma unroll
        for (int rg = 0; rg < 2; ++rg) {
          const float4 l4 = *(const float4*)(&l_lds[step & 1][16 * rg + 4 * lg]);
          const float l2[4] = {l4.x, l4.y, l4.z, l4.w};
          float x4[4] = {0.f, 0.f, 0.f, 0.f};
          if constexpr (DK) {
            const float4 d4 = *(const float4*)(&x_lds[step & 1][16 * rg + 4 * lg]);
            x4[0] = d4.x;
            x4[1] = d4.y;
            x4[2] = d4.z;
            x4[3] = d4.w;
          }
#pragma unroll
          for (int kt = 0; kt < KT; ++kt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              // hidden elements take exponent -inf (weight exactly 0); the
              // selection goes before the exponential, which every lane
              // then runs (a selection after it becomes a branch round it).
              // Visible: 0 <= row - key < window, one unsigned compare
              float x = fmaf(sacc[rg][kt][e], scale2, -l2[e]);
              if constexpr (masked) {
                const uint32_t diff = (uint32_t)(base + 16 * rg + e - 16 * kt);
                x = diff < (uint32_t)win ? x : -__builtin_inff();
              }
              const float p = __builtin_amdgcn_exp2f(x);
              if constexpr (kV) pa[kt][4 * rg + e] = (_Float16)p;
              // DK: dS = P (dP - delta_row), rounded to fp32 and then to
              // fp16 in every element (the empty asm keeps the compiler from
              // fusing the product into the conversion, v_fma_mixlo_f16, in
              // some elements and not in others)
              if constexpr (DK) {
                float ds = p * (dpacc[rg][kt][e] - x4[e]);
                asm volatile("" : "+v"(ds));
                dsa[kt][4 * rg + e] = (_Float16)ds;
              }
            }
        }
      };
      // a uniform branch: the steps away from the diagonal and the ends pay
      // for no mask
      if (full) {
        make_p(std::false_type{});
      } else {
        make_p(std::true_type{});
      }
      // ---- dV̂ += Pᵀ dO and dK̂ += dSᵀ Q_rot: B = the staged rows' dim
      // 16dt + ln at slots {4lg..4lg+3} = rows 4lg..4lg+3 and {16+4lg..} =
      // rows 16+4lg.., two transposing reads of dO (for dV̂) or q_rot (dK̂) ----
      const uint32_t tld = lds_addr(dl) + tr_off, tlq = lds_addr(ql) + tr_off;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const int ch2 = 2 * dt + ((ln & 3) >> 1);
        if constexpr (kV) {
          const uint32_t at = tld + 16u * row_slot<kDSwz>(tr_row, ch2);
          const half4 lo = lds_read_tr16(at);
          const half4 hi = lds_read_tr16(at + 16u * 256u);
          const half8 db = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
          for (int kt = 0; kt < KT; ++kt)
            acc[iV][kt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[kt], db, acc[iV][kt][dt], 0, 0, 0);
        }
        if constexpr (DK) {
          const uint32_t at = tlq + 16u * row_slot<kQSwz>(tr_row, ch2);
          const half4 lo = lds_read_tr16(at);
          const half4 hi = lds_read_tr16(at + 16u * 256u);
          const half8 qb = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
          for (int kt = 0; kt < KT; ++kt)
            acc[iK][kt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(dsa[kt], qb, acc[iK][kt][dt], 0, 0, 0);
        }
      }
    }
    if (++ch == NQ) {
      ch = 0;
      r0 -= kBRows;
    }
    // step + 1's copies and lse have landed (this wave's part; the barrier
    // covers the rest)
    if (more2) {
      __builtin_amdgcn_s_waitcnt(kWaitVm4);
    } else {
      __builtin_amdgcn_s_waitcnt(0);
    }
    if (more) put_lse((step + 1) & 1, r0);
    __syncthreads();
    buf = buf == 2 ? 0 : buf + 1;
    buf2 = buf2 == 2 ? 0 : buf2 + 1;
  }

  // ---- store the wave's keys: lane holds dims 16dt + ln of keys kw0 + 16kt
  // + 4lg + e.  dV̂ goes to a.dv; dK̂ (1/sqrt(D), then the rotary's transpose
  // at the key's position: dims f and f + 64, slices dt and dt + 4, are one
  // rotation pair) to a.dv when it is the only gradient, else to a.dk ----
  const int64_t orow = (int64_t)chunk * a.slot_stride + ((b * a.KVH + kvh) * a.T) * kBD;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t key = kw0 + 16 * kt + 4 * lg + e;
      if (key >= a.T) continue;
      if constexpr (kV) {
        float* out = a.dv + orow;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) out[key * kBD + 16 * dt + ln] = acc[iV][kt][dt][e];
      }
      if constexpr (DK) {
        float* out = (kV ? a.dk : a.dv) + orow;
        const _Float16* tr = rope_row(p0 + key);
        const float inv = 1.0f / sqrtf((float)kBD);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const int f = 16 * dt + ln;
          const float c = (float)tr[f], sn = (float)tr[64 + f];
          const float lo = acc[iK][kt][dt][e] * inv, hi = acc[iK][kt][dt + 4][e] * inv;
          out[key * kBD + f] = lo * c + hi * sn;
          out[key * kBD + 64 + f] = hi * c - lo * sn;
        }
      }
    }
}

// 168 registers: three workgroups per CU
__global__ __launch_bounds__(kBThreads) __attribute__((amdgpu_waves_per_eu(3)))
void prefill_value_grad_kernel(ValueGradArgs a) {
  kv_grad_walk<kWalkV, 2>(a);
}
__global__ __launch_bounds__(kBThreads) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_key_grad_kernel(ValueGradArgs a) {
  kv_grad_walk<kWalkK, 2>(a);
}
__global__ __launch_bounds__(kBThreads) __attribute__((amdgpu_waves_per_eu(3)))
void prefill_kv_grad_kernel(ValueGradArgs a) {
  kv_grad_walk<kWalkKV, 1>(a);
}

// Query gradient of the same attention, and delta = rowsum(dO * O) that the
// key gradient needs:
//   dSᵀ = Pᵀ (dPᵀ - delta_row),  dPᵀ = V̂ dOᵀ,  dQ_rot += dS K̂_rot / sqrt(D),
// then the rotary's transpose at the row's position.  One workgroup of 4
// waves per (batch row, kv head, head group, block of query rows) and run of
// 32-key tiles; wave w is query head w % HW of the group on rows
// 32 (w / HW) .. + 31 of the block.  Its rotated q and its dO rows stay in
// registers as B operands; each key tile's rotated K̂ rows (rotated once by
// the entry point) and V̂ rows go straight into LDS once for the four waves.
// Per tile and wave, on v_mfma_f32_16x16x32_f16:
//   Sᵀ[key][row] = K̂ Qᵀ and dPᵀ[key][row] = V̂ dOᵀ   (A = K̂ / V̂ rows from LDS)
//   dS in A order read straight off the Sᵀ/dPᵀ accumulators (two 16-key
//   tiles interleaved into the contraction slots)
//   K̂ in B order by transposing reads of the staged K̂ rows
//   dQ[row][dim] += dS K̂
static const int kQKeys = 32;  // keys per tile

struct QGradArgs {
  ValueGradArgs g;
  const _Float16* o;  // forward output [B,QH,T,D] fp16
  int64_t osb, osh, ost;
  float* delta;       // [B,QH,T] written
  float* dq;          // [B,QH,T,D] fp32, or the run's partial slot
  _Float16* q_rot;    // [B,QH,T,D] fp16 contiguous: the rotated queries, written for the key and value legs (or null)
  int32_t heads_per_wg, row_sets, head_groups;
};

__global__ __launch_bounds__(kBThreads) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_q_grad_kernel(QGradArgs qa_) {
  const ValueGradArgs& a = qa_.g;  // a.k: the rotated K̂_rot, contiguous [B,KVH,T,128]
  __shared__ __align__(1024) _Float16 k_lds[3][kQKeys * kBD];
  __shared__ __align__(1024) _Float16 v_lds[3][kQKeys * kBD];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the tile tests below branch on it
  const int ln = lane & 15, lg = lane >> 4;
  const int HW = qa_.heads_per_wg, RS = qa_.row_sets;
  const int NQ = a.nq;
  const int64_t block_rows = 32 * (int64_t)RS;
  const int64_t nqb = ceil_div(a.T, block_rows);
  const uint32_t bid = xcd_remap(blockIdx.x, gridDim.x);
  const int chunk = blockIdx.y;
  // longest key ranges first (later row blocks see more keys)
  const int64_t qblk = nqb - 1 - (int64_t)(bid % (uint32_t)nqb);
  const int64_t yz = bid / (uint32_t)nqb;
  const int64_t gy = a.KVH * qa_.head_groups;
  const int64_t kvh = (yz % gy) / qa_.head_groups;
  const int64_t hg = (yz % gy) % qa_.head_groups;
  const int64_t b = yz / gy;
  const int64_t head = kvh * NQ + hg * HW + wave % HW;
  const int64_t wg_row0 = qblk * block_rows;
  const int64_t row0 = wg_row0 + (wave / HW) * 32;  // the wave's first row
  const int64_t p0 = a.start[b];
  const float scale2 = 1.4426950408889634f / sqrtf((float)kBD);
  const int64_t rope_last = a.rope_len - 1;
  auto rope_row = [&](int64_t pos) -> const _Float16* {
    return a.rope + (pos < 0 ? 0 : (pos < rope_last ? pos : rope_last)) * kRopeRow;
  };
  const half8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};

  // ---- the wave's rotated q and dO rows as B operands (lane (row ln, lg):
  // dims [32c + 8lg, +8)), its rows' lse (base 2) and delta ----
  half8 qop[2][4], dop[2][4];
  float l2[2], dl[2];
#pragma unroll
  for (int rg = 0; rg < 2; ++rg) {
    const int64_t row = row0 + 16 * rg + ln;
    const bool ok = row < a.T;
    const _Float16* qp = a.q + b * a.qsb + head * a.qsh + (ok ? row : 0) * a.qst;
    const _Float16* dp = a.dout + b * a.dsb + head * a.dsh + (ok ? row : 0) * a.dst;
    const _Float16* op = qa_.o + b * qa_.osb + head * qa_.osh + (ok ? row : 0) * qa_.ost;
    const _Float16* tr = rope_row(p0 + (ok ? row : 0));
    float dsum = 0.f;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int d0 = 32 * c + 8 * lg;
      half8 cs, sn, r0, r1;
      load_trig8(tr, d0, &cs, &sn);
      rope16(*(const half8*)(qp + d0), *(const half8*)(qp + d0 + 64), cs, sn, &r0, &r1);
      qop[rg][c] = ok ? r0 : zero8;
      qop[rg][c + 2] = ok ? r1 : zero8;
      // every (head, row) has one wave (one run per row block): it also
      // writes the row's q_rot for the key and value legs
      if (qa_.q_rot != nullptr && ok) {
        _Float16* qr = qa_.q_rot + ((b * a.QH + head) * a.T + row) * kBD + d0;
        *(half8*)qr = r0;
        *(half8*)(qr + 64) = r1;
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const half8 dv = *(const half8*)(dp + 32 * c + 8 * lg);
      const half8 ov = *(const half8*)(op + 32 * c + 8 * lg);
      dop[rg][c] = ok ? dv : zero8;
#pragma unroll
      for (int e = 0; e < 8; ++e) dsum = fmaf((float)dv[e], (float)ov[e], dsum);
    }
    dsum += __shfl_xor(dsum, 16);
    dsum += __shfl_xor(dsum, 32);
    dl[rg] = ok ? dsum : 0.f;
    l2[rg] = ok ? a.lse[(b * a.QH + head) * a.T + row] * 1.4426950408889634f : 0.f;
    if (ok && lg == 0 && chunk == 0) qa_.delta[(b * a.QH + head) * a.T + row] = dsum;
  }
  float4v acc[2][8];  // dQ_rot[row 16rg + 4lg + e][dim 16dt + ln]
#pragma unroll
  for (int rg = 0; rg < 2; ++rg)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[rg][dt] = float4v{0.f, 0.f, 0.f, 0.f};

  // ---- the key tiles the block's rows see: [wg_row0 - window + 1, wg_row1) ----
  int64_t wg_row1 = wg_row0 + block_rows;
  if (wg_row1 > a.T) wg_row1 = a.T;
  int64_t kmin = wg_row0 - a.window + 1;
  if (kmin < 0) kmin = 0;
  const int64_t t_first = kmin / kQKeys;
  const int64_t all_tiles = ceil_div(wg_row1, kQKeys) - t_first;
  const int64_t tile_lo = (int64_t)chunk * a.chunk_tiles;
  int64_t ntiles = all_tiles - tile_lo;
  if (ntiles > a.chunk_tiles) ntiles = a.chunk_tiles;
  if (ntiles < 0) ntiles = 0;

  // ---- tile staging: a tile's K̂_rot rows (rotated by the entry point,
  // contiguous [B,KVH,T,128]) and V̂ rows go global -> LDS directly, as in
  // the key-block walk: two tiles ahead into three buffers, wave w filling
  // key rows 8w..8w+7 of both with two instructions each, chunks swizzled
  // by row_slot (K̂ rows read both ways, V̂ rows as A operands).  Keys past
  // T read the tile's first key (always in range; causality masks them for
  // every row) ----
  const int srow = 8 * wave + (lane >> 4), slot = lane & 15;
  const int32_t T32 = (int32_t)a.T;
  const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.k + (b * a.KVH + kvh) * a.T * kBD), (short)0, (int)(a.T * 2 * kBD), 0x00020000);
  const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.v + b * a.vsb + kvh * a.vsh), (short)0, (int)(((a.T - 1) * a.vst + kBD) * 2), 0x00020000);
  const int32_t key_first = (int32_t)((t_first + tile_lo) * kQKeys);
  const int32_t nt = (int32_t)ntiles;
  auto copy = [&](int32_t tile, int buf) {
    const int32_t first = key_first + tile * kQKeys;
    char* kd = (char*)k_lds[buf] + 2048 * wave;
    char* vd = (char*)v_lds[buf] + 2048 * wave;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = srow + 4 * i;
      const uint32_t rr = first + r < T32 ? (uint32_t)r : 0u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(k_rsrc, (void __attribute__((address_space(3)))*)(kd + 1024 * i), 16,
                                               rr * (2u * kBD) + 16u * row_slot<kSwzAT>(r, slot),
                                               (uint32_t)first * (2u * kBD), 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(v_rsrc, (void __attribute__((address_space(3)))*)(vd + 1024 * i), 16,
                                               rr * (uint32_t)a.vst * 2u + 16u * row_slot<kSwzA>(r, slot),
                                               (uint32_t)first * (uint32_t)a.vst * 2u, 0, 0);
    }
  };
  // s_waitcnt vmcnt(4), leaving the other counters alone (gfx9 encoding)
  constexpr int kWaitVm4 = 4 | (7 << 4) | (15 << 8);
  if (nt > 0) {
    copy(0, 0);
    if (nt > 1) {
      copy(1, 1);
      __builtin_amdgcn_s_waitcnt(kWaitVm4);  // tile 0 has landed
    } else {
      __builtin_amdgcn_s_waitcnt(0);
    }
  }
  __syncthreads();
  const int32_t win = a.window < 0x40000000 ? (int32_t)a.window : 0x40000000;
  const int32_t r32 = (int32_t)row0;
  // per-lane LDS byte offsets of the transposing reads: key rows 4lg + ln/4
  // (+16), dims 16dt + 4(ln%4), 8 bytes
  const int tr_row = 4 * lg + (ln >> 2);
  const uint32_t tr_off = (uint32_t)tr_row * 256u + 8u * (ln & 1);

  int buf = 0, buf2 = 2;  // buffers of this tile and of tile + 2
  // one tile; MORE2: two follow (the steady state; the last two are peeled)
  for (int32_t tile = 0; tile < nt; ++tile) {
    const bool more2 = tile + 2 < nt;
    if (more2) copy(tile + 2, buf2);
    const int32_t key0 = key_first + tile * kQKeys;
    const bool any = key0 <= r32 + 31 && r32 - (key0 + kQKeys - 1) < win;
    if (any) {
      const char* kl = (const char*)k_lds[buf];
      const char* vl = (const char*)v_lds[buf];
      // ---- Sᵀ and dPᵀ [key][row]: 2 key tiles x 2 row tiles; A = the staged
      // rows (key 16kt + ln, chunk 4c + lg) ----
      float4v st[2][2], dpt[2][2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        half8 ka[4], va[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          ka[c] = *(const half8*)(kl + (16 * kt + ln) * 256 + 16 * row_slot<kSwzAT>(ln, 4 * c + lg));
          va[c] = *(const half8*)(vl + (16 * kt + ln) * 256 + 16 * row_slot<kSwzA>(ln, 4 * c + lg));
        }
#pragma unroll
        for (int rg = 0; rg < 2; ++rg) {
          st[kt][rg] = float4v{0.f, 0.f, 0.f, 0.f};
          dpt[kt][rg] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            st[kt][rg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[c], qop[rg][c], st[kt][rg], 0, 0, 0);
            dpt[kt][rg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[c], dop[rg][c], dpt[kt][rg], 0, 0, 0);
          }
        }
      }
      // ---- dS, masked: element (kt, rg, e) is key key0 + 16kt + 4lg + e of
      // row row0 + 16rg + ln; dsa[rg] contraction slot 4kt + e (of lane group
      // lg) <-> key 16kt + 4lg + e.  Rows past T need no mask: a row's dQ
      // depends on its own dS only, and those rows are never stored ----
      const bool full = key0 + kQKeys - 1 <= r32 && r32 + 31 - key0 < win;
      const int base = r32 - key0 + ln - 4 * lg;  // row - key = base + 16rg - 16kt - e
      half8 dsa[2];
      auto make_ds = [&](auto masked_tag) {
        constexpr bool masked = decltype(masked_tag)::value;
#pragma unroll
        for (int rg = 0; rg < 2; ++rg)
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              // hidden elements take exponent -inf (weight exactly 0),
              // selected before the exponential; visible: 0 <= row - key <
              // window, one unsigned compare
              float x = fmaf(st[kt][rg][e], scale2, -l2[rg]);
              if constexpr (masked) {
                const uint32_t diff = (uint32_t)(base + 16 * rg - 16 * kt - e);
                x = diff < (uint32_t)win ? x : -__builtin_inff();
              }
              // dS = fp16(fp32(P (dP - delta))) in every element (the empty
              // asm keeps the product out of the conversion, v_fma_mixlo_f16)
              float ds = __builtin_amdgcn_exp2f(x) * (dpt[kt][rg][e] - dl[rg]);
              asm volatile("" : "+v"(ds));
              dsa[rg][4 * kt + e] = (_Float16)ds;
            }
      };
      // a uniform branch: the tiles away from the diagonal and the ends pay
      // for no mask
      if (full) {
        make_ds(std::false_type{});
      } else {
        make_ds(std::true_type{});
      }
      // ---- dQ += dS K̂: B = K̂ in B order (keys {4lg+e, 16+4lg+e} of dim
      // 16dt + ln), two transposing reads of the staged K̂ rows ----
      const uint32_t tl = lds_addr(kl) + tr_off;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const uint32_t at = tl + 16u * row_slot<kSwzAT>(tr_row, 2 * dt + ((ln & 3) >> 1));
        const half4 lo = lds_read_tr16(at);
        const half4 hi = lds_read_tr16(at + 16u * 256u);
        const half8 kbo = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
        for (int rg = 0; rg < 2; ++rg)
          acc[rg][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(dsa[rg], kbo, acc[rg][dt], 0, 0, 0);
      }
    }
    // tile + 1 has landed (this wave's part; the barrier covers the rest)
    if (more2) {
      __builtin_amdgcn_s_waitcnt(kWaitVm4);
    } else {
      __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();
    buf = buf == 2 ? 0 : buf + 1;
    buf2 = buf2 == 2 ? 0 : buf2 + 1;
  }

  // ---- 1/sqrt(D), the rotary's transpose at the row's position, store:
  // lane holds dims 16dt + ln of rows row0 + 16rg + 4lg + e ----
  float* out = qa_.dq + (int64_t)chunk * a.slot_stride + ((b * a.QH + head) * a.T) * kBD;
  const float inv = 1.0f / sqrtf((float)kBD);
#pragma unroll
  for (int rg = 0; rg < 2; ++rg)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t row = row0 + 16 * rg + 4 * lg + e;
      if (row >= a.T) continue;
      const _Float16* tr = rope_row(p0 + row);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const int f = 16 * dt + ln;
        const float c = (float)tr[f], sn = (float)tr[64 + f];
        const float lo = acc[rg][dt][e] * inv, hi = acc[rg][dt + 4][e] * inv;
        out[row * kBD + f] = lo * c + hi * sn;
        out[row * kBD + 64 + f] = hi * c - lo * sn;
      }
    }
}

// dV̂ (or dK̂) = the sum of the partial slots of the chunks that the key's
// block meets, in chunk order.  Rows [*, T, 128] fp32, as float4.
__global__ __launch_bounds__(256) void value_grad_reduce_kernel(const float* __restrict__ part,
                                                                float* __restrict__ dv, int64_t n4,
                                                                int64_t slot4, int slots, int64_t T,
                                                                int64_t window, int keys, int64_t per) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  const int64_t key = (i / (kBD / 4)) % T;
  int64_t tf, tl;
  block_tiles(key - key % keys, T, window, keys, &tf, &tl);
  const int64_t c_lo = tf / per, c_hi = tl / per;
  float4 acc = ((const float4*)part)[i + (c_lo % slots) * slot4];
  for (int64_t c = c_lo + 1; c <= c_hi; ++c) {
    const float4 v = ((const float4*)part)[i + (c % slots) * slot4];
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  }
  ((float4*)dv)[i] = acc;
}

// Tiles per chunk and partial slots of the key-block kernels (blocks of
// `keys` keys): chunks of 16 tiles, or of an eighth of the longest block's
// rows when that is more; the slots are the most chunks one block meets.
static void value_grad_chunks(int64_t T, int64_t window, int keys, int* chunk_tiles, int* slots);

// bytes of the value gradient's workspace: the chunks' partial slots (when
// there are several), then the rotated queries [B,QH,T,128] fp16 at a
// 256-byte boundary
static int64_t value_grad_workspace(int64_t B, int64_t QH, int64_t KVH, int64_t T, int64_t window) {
  int chunk_tiles, chunks;
  value_grad_chunks(T, window, kBKeys, &chunk_tiles, &chunks);
  const int64_t slots = chunks > 1 ? (int64_t)chunks * B * KVH * T * kBD * (int64_t)sizeof(float) : 0;
  return ceil_div(slots, 256) * 256 + B * QH * T * kBD * 2;
}

static void value_grad_chunks(int64_t T, int64_t window, int keys, int* chunk_tiles, int* slots) {
  int64_t rows = (int64_t)keys - 1 + window;
  if (rows > T || rows < 0) rows = T;
  const int64_t span = ceil_div(rows, kBRows);  // tiles of the longest block (blocks start on a tile)
  int64_t per = 16;
  if (ceil_div(span, per) > 8) per = ceil_div(span, 8);
  const int64_t all = ceil_div(ceil_div(T, kBRows), per);
  const int64_t most = ceil_div(span - 1, per) + 1;
  *chunk_tiles = (int)per;
  *slots = (int)(all < most ? all : most);
}

}  // namespace jkv

extern "C" {

int64_t jkv_prefill_value_grad_workspace_bytes(int64_t B, int64_t QH, int64_t KVH, int64_t T, int64_t window) {
  if (B <= 0 || QH <= 0 || KVH <= 0 || T <= 0 || window < 1) return 0;
  return jkv::value_grad_workspace(B, QH, KVH, T, window);
}

}  // extern "C"

namespace jkv {

// shared by the value and key gradients and the walk that forms both:
// checks, the rotated queries (into the workspace, unless the caller hands
// them in), the row runs, the launch and the reduction of the runs' partial
// slots.  d_out_buf is dV̂ (kWalkV, kWalkKV) or dK̂ (kWalkK); d_key_buf dK̂
// for kWalkKV.
template <int MODE>
static int launch_kv_grad(ValueGradArgs a, int64_t D, const int64_t (&strides)[12], int nstrides,
                          const void* rope_table, float* d_out_buf, void* workspace, int64_t workspace_bytes,
                          hipStream_t stream, const _Float16* q_rot_given = nullptr, float* d_key_buf = nullptr) {
  constexpr bool DK = MODE != kWalkV;
  constexpr int keys = MODE == kWalkKV ? 64 : kBKeys;
  constexpr int nout = MODE == kWalkKV ? 2 : 1;
  const int64_t B = a.B, QH = a.QH, KVH = a.KVH, T = a.T;
  JKV_CHECK_ARG(D == kBD, "prefill gradients support head_dim 128, got %lld", (long long)D);
  JKV_CHECK_ARG(B >= 0 && QH > 0 && KVH > 0 && T >= 0 && QH % KVH == 0, "invalid prefill geometry");
  const int64_t NQ = QH / KVH;
  JKV_CHECK_ARG(NQ <= 64, "at most 64 query heads per kv head, got %lld", (long long)NQ);
  JKV_CHECK_ARG(a.window >= 1, "window must be positive");
  if (B == 0 || T == 0) return JKV_OK;
  JKV_CHECK_ARG(a.q && a.k && a.dout && a.lse && d_out_buf && a.start && rope_table, "null buffer");
  JKV_CHECK_ARG(!DK || (a.v && a.delta), "null buffer");
  JKV_CHECK_ARG(MODE != kWalkKV || (d_key_buf && q_rot_given && (uintptr_t)d_key_buf % 16 == 0),
                "null or misaligned buffer");
  JKV_CHECK_ARG(a.rope_len >= 1, "rotary table is empty");
  JKV_CHECK_ARG(B < 65536 && QH < 65536, "prefill gradients: batch and query heads must be below 65536");
  {
    // the walk's 32-bit offsets: positions, rotary rows, and the bytes of
    // one (batch row, kv head)'s rotated queries, output gradient and lse
    const int64_t nq1 = NQ - 1, lim = (int64_t)1 << 31;
    JKV_CHECK_ARG(T < ((int64_t)1 << 30) && a.rope_len < ((int64_t)1 << 23),
                  "prefill gradients support at most 2^30 tokens and 2^23 rotary positions");
    JKV_CHECK_ARG(a.dst >= 0 && a.dsh >= 0 && NQ * T * kBD * 2 < lim &&
                      (nq1 * a.dsh + (T - 1) * a.dst + kBD) * 2 < lim && (nq1 * T + kBRows) * 4 < lim,
                  "prefill gradients: the query heads of one kv head must span under 2^31 bytes "
                  "of q, d_out and lse");
  }
  for (int i = 0; i < nstrides; ++i)
    JKV_CHECK_ARG(strides[i] % 8 == 0, "prefill strides must be multiples of 8 elements");
  JKV_CHECK_ARG(((uintptr_t)a.q | (uintptr_t)a.k | (uintptr_t)a.dout | (uintptr_t)d_out_buf |
                 (uintptr_t)(DK ? a.v : a.q)) % 16 == 0,
                "prefill buffers must be 16-byte aligned");
  a.rope = (const _Float16*)rope_table;
  a.nq = (int32_t)NQ;
  int chunk_tiles, chunks;
  value_grad_chunks(T, a.window, keys, &chunk_tiles, &chunks);
  a.chunk_tiles = chunk_tiles;
  a.slots = chunks;
  const int64_t n = B * KVH * T * kBD;
  // workspace: the chunks' partial slots (of each output), then the rotated
  // queries (unless the caller hands them in)
  const int64_t slot_bytes = chunks > 1 ? (int64_t)chunks * n * (int64_t)sizeof(float) : 0;
  const int64_t need =
      q_rot_given != nullptr ? nout * slot_bytes : value_grad_workspace(B, QH, KVH, T, a.window);
  if (need > 0) {
    JKV_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                  "prefill gradient workspace too small: %lld bytes, need %lld", (long long)workspace_bytes,
                  (long long)need);
    JKV_CHECK_ARG(((uintptr_t)workspace) % 16 == 0, "workspace must be 16-byte aligned");
  }
  if (chunks > 1) {
    a.dv = (float*)workspace;
    a.dk = (float*)((unsigned char*)workspace + slot_bytes);
    a.slot_stride = n;
  } else {
    a.dv = d_out_buf;
    a.dk = d_key_buf;
    a.slot_stride = 0;
  }
  const int64_t blocks = ceil_div(T, keys) * KVH * B;
  JKV_CHECK_ARG(blocks < ((int64_t)1 << 31), "prefill grid too large");
  const _Float16* q_rot = q_rot_given;
  if (q_rot == nullptr) {
    _Float16* qr = (_Float16*)((unsigned char*)workspace + ceil_div(slot_bytes, 256) * 256);
    hipLaunchKernelGGL(rotate_rows_kernel, dim3((uint32_t)ceil_div(8 * T, 256), (uint32_t)QH, (uint32_t)B),
                       dim3(256), 0, stream, a.q, a.qsb, a.qsh, a.qst, T, a.start, a.rope, a.rope_len, qr);
    JKV_CHECK_LAUNCH();
    q_rot = qr;
  }
  a.q = q_rot;  // contiguous [B,QH,T,128]
  if constexpr (MODE == kWalkK) {
    hipLaunchKernelGGL(prefill_key_grad_kernel, dim3((uint32_t)blocks, (uint32_t)chunks), dim3(kBThreads), 0,
                       stream, a);
  } else if constexpr (MODE == kWalkKV) {
    hipLaunchKernelGGL(prefill_kv_grad_kernel, dim3((uint32_t)blocks, (uint32_t)chunks), dim3(kBThreads), 0,
                       stream, a);
  } else {
    hipLaunchKernelGGL(prefill_value_grad_kernel, dim3((uint32_t)blocks, (uint32_t)chunks), dim3(kBThreads), 0,
                       stream, a);
  }
  JKV_CHECK_LAUNCH();
  if (chunks > 1) {
    const int64_t n4 = n / 4;
    for (int o = 0; o < nout; ++o) {
      hipLaunchKernelGGL(value_grad_reduce_kernel, dim3((uint32_t)ceil_div(n4, 256)), dim3(256), 0, stream,
                         (const float*)((unsigned char*)workspace + o * slot_bytes), o == 0 ? d_out_buf : d_key_buf,
                         n4, n4, chunks, T, a.window, keys, (int64_t)chunk_tiles);
      JKV_CHECK_LAUNCH();
    }
  }
  return JKV_OK;
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
                                     void* workspace, int64_t workspace_bytes, jkv_stream_t stream_) {
  using namespace jkv;
  ValueGradArgs a = {};
  a.q = (const _Float16*)q; a.qsb = q_stride_b; a.qsh = q_stride_h; a.qst = q_stride_t;
  a.k = (const _Float16*)k; a.ksb = k_stride_b; a.ksh = k_stride_h; a.kst = k_stride_t;
  a.dout = (const _Float16*)d_out; a.dsb = d_stride_b; a.dsh = d_stride_h; a.dst = d_stride_t;
  a.lse = lse;
  a.B = B; a.QH = QH; a.KVH = KVH; a.T = T;
  a.start = start_positions;
  a.window = window;
  a.rope_len = rope_len;
  const int64_t strides[12] = {q_stride_b, q_stride_h, q_stride_t, k_stride_b, k_stride_h, k_stride_t,
                               d_stride_b, d_stride_h, d_stride_t, 0, 0, 0};
  return launch_kv_grad<kWalkV>(a, D, strides, 9, rope_table, d_value, workspace, workspace_bytes,
                                (hipStream_t)stream_);
}

int jkv_prefill_attention_key_grad(const void* q, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t,
                                   const void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                                   const void* v, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_t,
                                   const void* d_out, int64_t d_stride_b, int64_t d_stride_h,
                                   int64_t d_stride_t, const float* lse, const float* delta, int64_t B,
                                   int64_t QH, int64_t KVH, int64_t T, int64_t D,
                                   const int32_t* start_positions, int64_t window, const void* rope_table,
                                   int64_t rope_len, float* d_key, void* workspace, int64_t workspace_bytes,
                                   jkv_stream_t stream_) {
  using namespace jkv;
  ValueGradArgs a = {};
  a.q = (const _Float16*)q; a.qsb = q_stride_b; a.qsh = q_stride_h; a.qst = q_stride_t;
  a.k = (const _Float16*)k; a.ksb = k_stride_b; a.ksh = k_stride_h; a.kst = k_stride_t;
  a.v = (const _Float16*)v; a.vsb = v_stride_b; a.vsh = v_stride_h; a.vst = v_stride_t;
  a.dout = (const _Float16*)d_out; a.dsb = d_stride_b; a.dsh = d_stride_h; a.dst = d_stride_t;
  a.lse = lse;
  a.delta = delta;
  a.B = B; a.QH = QH; a.KVH = KVH; a.T = T;
  a.start = start_positions;
  a.window = window;
  a.rope_len = rope_len;
  const int64_t strides[12] = {q_stride_b, q_stride_h, q_stride_t, k_stride_b, k_stride_h, k_stride_t,
                               v_stride_b, v_stride_h, v_stride_t, d_stride_b, d_stride_h, d_stride_t};
  return launch_kv_grad<kWalkK>(a, D, strides, 12, rope_table, d_key, workspace, workspace_bytes,
                                (hipStream_t)stream_);
}

int64_t jkv_prefill_backward_workspace_bytes(int64_t B, int64_t QH, int64_t KVH, int64_t T, int64_t window) {
  using namespace jkv;
  if (B <= 0 || QH <= 0 || KVH <= 0 || T <= 0 || window < 1) return 0;
  int chunk_tiles, chunks, chunks64;
  value_grad_chunks(T, window, kBKeys, &chunk_tiles, &chunks);
  value_grad_chunks(T, window, 64, &chunk_tiles, &chunks64);
  const int64_t delta = ceil_div(B * QH * T * (int64_t)sizeof(float), 256) * 256;
  const int64_t k_rot = ceil_div(B * KVH * T * kBD * 2, 256) * 256;
  const int64_t q_rot = ceil_div(B * QH * T * kBD * 2, 256) * 256;
  // the slot area serves the query leg (delta only), then the key leg's
  // slots, the value leg's slots (and rotated queries, when it runs alone) or
  // the slots of both from the walk that forms both
  const int64_t qk = (int64_t)chunks * B * QH * T * kBD * (int64_t)sizeof(float);
  const int64_t v = value_grad_workspace(B, QH, KVH, T, window);
  const int64_t kv = chunks64 > 1 ? 2 * (int64_t)chunks64 * B * KVH * T * kBD * (int64_t)sizeof(float) : 0;
  const int64_t area = qk > v ? (qk > kv ? qk : kv) : (v > kv ? v : kv);
  return delta + k_rot + q_rot + area;
}

int jkv_prefill_attention_backward(const void* q, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t,
                                   const void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
                                   const void* v, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_t,
                                   const void* out, int64_t o_stride_b, int64_t o_stride_h, int64_t o_stride_t,
                                   const void* d_out, int64_t d_stride_b, int64_t d_stride_h,
                                   int64_t d_stride_t, const float* lse, int64_t B, int64_t QH, int64_t KVH,
                                   int64_t T, int64_t D, const int32_t* start_positions, int64_t window,
                                   const void* rope_table, int64_t rope_len, float* d_query, float* d_key,
                                   float* d_value, void* workspace, int64_t workspace_bytes,
                                   jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(D == kBD, "prefill gradients support head_dim 128, got %lld", (long long)D);
  JKV_CHECK_ARG(B >= 0 && QH > 0 && KVH > 0 && T >= 0 && QH % KVH == 0, "invalid prefill geometry");
  JKV_CHECK_ARG(window >= 1, "window must be positive");
  if (B == 0 || T == 0 || (!d_query && !d_key && !d_value)) return JKV_OK;
  const int64_t need = jkv_prefill_backward_workspace_bytes(B, QH, KVH, T, window);
  JKV_CHECK_ARG(workspace != nullptr && workspace_bytes >= need && ((uintptr_t)workspace) % 16 == 0,
                "prefill backward needs %lld bytes of 16-byte aligned workspace", (long long)need);
  const int64_t NQ = QH / KVH;
  // workspace: delta, the rotated keys of the query leg, the rotated
  // queries it writes for the key and value legs, the slot area
  float* delta = (float*)workspace;
  _Float16* k_rot = (_Float16*)((unsigned char*)workspace + ceil_div(B * QH * T * (int64_t)sizeof(float), 256) * 256);
  _Float16* q_rot = (_Float16*)((unsigned char*)k_rot + ceil_div(B * KVH * T * kBD * 2, 256) * 256);
  unsigned char* slots = (unsigned char*)q_rot + ceil_div(B * QH * T * kBD * 2, 256) * 256;
  const int64_t slot_bytes = workspace_bytes - (slots - (unsigned char*)workspace);
  ValueGradArgs g = {};
  g.q = (const _Float16*)q; g.qsb = q_stride_b; g.qsh = q_stride_h; g.qst = q_stride_t;
  g.k = (const _Float16*)k; g.ksb = k_stride_b; g.ksh = k_stride_h; g.kst = k_stride_t;
  g.v = (const _Float16*)v; g.vsb = v_stride_b; g.vsh = v_stride_h; g.vst = v_stride_t;
  g.dout = (const _Float16*)d_out; g.dsb = d_stride_b; g.dsh = d_stride_h; g.dst = d_stride_t;
  g.lse = lse;
  g.delta = delta;
  g.B = B; g.QH = QH; g.KVH = KVH; g.T = T;
  g.start = start_positions;
  g.window = window;
  g.rope_len = rope_len;
  const int64_t strides[12] = {q_stride_b, q_stride_h, q_stride_t, k_stride_b, k_stride_h, k_stride_t,
                               v_stride_b, v_stride_h, v_stride_t, d_stride_b, d_stride_h, d_stride_t};
  // ---- dQ and delta: the query kernel; its runs are summed into d_query
  // (they stay in the slots when only delta is wanted) ----
  if (d_query || d_key) {
    JKV_CHECK_ARG(q && k && v && out && d_out && lse && start_positions && rope_table && rope_len >= 1,
                  "null buffer");
    for (int i = 0; i < 12; ++i)
      JKV_CHECK_ARG(strides[i] % 8 == 0, "prefill strides must be multiples of 8 elements");
    JKV_CHECK_ARG(o_stride_b % 8 == 0 && o_stride_h % 8 == 0 && o_stride_t % 8 == 0,
                  "prefill strides must be multiples of 8 elements");
    JKV_CHECK_ARG(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out | (uintptr_t)d_out |
                   (uintptr_t)(d_query ? d_query : (float*)slots)) % 16 == 0,
                  "prefill buffers must be 16-byte aligned");
    // four waves: head w % HW on rows 32 (w / HW) of the block
    JKV_CHECK_ARG(NQ < 4 || NQ % 4 == 0, "query heads per kv head must be 1, 2 or a multiple of 4");
    // the query kernel's 32-bit offsets into one (batch row, kv head)'s K̂_rot and V̂
    JKV_CHECK_ARG(B < 65536 && KVH < 65536 && T < ((int64_t)1 << 30) && rope_len < ((int64_t)1 << 23) &&
                      v_stride_t >= 0 && T * kBD * 2 < ((int64_t)1 << 31) &&
                      ((T - 1) * v_stride_t + kBD) * 2 < ((int64_t)1 << 31),
                  "prefill backward: one (batch row, kv head) must span under 2^31 bytes of K and V");
    hipLaunchKernelGGL(rotate_rows_kernel, dim3((uint32_t)ceil_div(8 * T, 256), (uint32_t)KVH, (uint32_t)B),
                       dim3(256), 0, stream, (const _Float16*)k, k_stride_b, k_stride_h, k_stride_t, T,
                       start_positions, (const _Float16*)rope_table, rope_len, k_rot);
    JKV_CHECK_LAUNCH();
    QGradArgs qa = {};
    qa.g = g;
    qa.g.k = k_rot;  // contiguous [B,KVH,T,128]
    qa.g.rope = (const _Float16*)rope_table;
    qa.g.nq = (int32_t)NQ;
    qa.o = (const _Float16*)out; qa.osb = o_stride_b; qa.osh = o_stride_h; qa.ost = o_stride_t;
    qa.delta = delta;
    qa.q_rot = (d_key || d_value) ? q_rot : nullptr;
    qa.heads_per_wg = (int32_t)(NQ < 4 ? NQ : 4);
    qa.row_sets = 4 / qa.heads_per_wg;
    qa.head_groups = (int32_t)(NQ / qa.heads_per_wg);
    // one run per row block (32-row blocks are many, and the longest go
    // first), written straight to d_query, or to the slot area when only
    // delta is wanted
    qa.g.chunk_tiles = 0x7fffffff;
    const int64_t n = B * QH * T * kBD;
    JKV_CHECK_ARG(d_query != nullptr || slot_bytes >= n * (int64_t)sizeof(float), "workspace too small");
    qa.dq = d_query != nullptr ? d_query : (float*)slots;
    qa.g.slot_stride = 0;
    const int64_t nqb = ceil_div(T, 32 * (int64_t)qa.row_sets);
    const int64_t blocks = nqb * KVH * qa.head_groups * B;
    JKV_CHECK_ARG(blocks < ((int64_t)1 << 31), "prefill grid too large");
    hipLaunchKernelGGL(prefill_q_grad_kernel, dim3((uint32_t)blocks), dim3(kBThreads), 0, stream, qa);
    JKV_CHECK_LAUNCH();
  }
  // the key and value legs read the rotated queries the query leg wrote;
  // without it (d_value alone) the value leg rotates them itself.  Both
  // gradients come from one walk (one S and one dP per step)
  const bool q_leg = d_query || d_key;
  if (d_key && d_value) {
    const int rc = launch_kv_grad<kWalkKV>(g, D, strides, 12, rope_table, d_value, slots, slot_bytes, stream,
                                           q_rot, d_key);
    if (rc != JKV_OK) return rc;
  } else if (d_key) {
    const int rc = launch_kv_grad<kWalkK>(g, D, strides, 12, rope_table, d_key, slots, slot_bytes, stream, q_rot);
    if (rc != JKV_OK) return rc;
  } else if (d_value) {
    const int rc = launch_kv_grad<kWalkV>(g, D, strides, 12, rope_table, d_value, slots, slot_bytes, stream,
                                          q_leg ? q_rot : nullptr);
    if (rc != JKV_OK) return rc;
  }
  return JKV_OK;
}

}  // extern "C"
