// Causal sliding-window GQA prefill attention over the chunk's quantized
// fp16 K̂/V̂ (pre-RoPE), with the reference model's fp16 rotary applied to
// q and K̂ at absolute positions start[b] + t.
//
// One workgroup of 8 waves per (batch, kv head, head group, block of query
// rows).  Each wave owns one query head and 32 query rows (two 16-row
// groups); the workgroup
// shares 64-key tiles of rotated K̂ ([key][dim]) and V̂ᵀ ([dim][key]) in LDS,
// double-buffered: the next tile's global loads are issued before the
// current tile's MFMAs and land in the other buffer afterwards.  Per tile and
// wave, on v_mfma_f32_16x16x32_f16:
//   Sᵀ[key][row] = K̂ Qᵀ     A = K̂ rows from LDS, B = the wave's rotated q
//   Oᵀ[dim][row] += V̂ᵀ Pᵀ   A = V̂ᵀ rows from LDS, B = fp16 P straight from
//                           the Sᵀ accumulators (the contraction slots of
//                           two 16-key groups are interleaved so that no
//                           cross-lane move is needed)
// with an online softmax in fp32 (base-2 exponent, scale folded in).
#include <math.h>

#include <type_traits>

#include "jkv_common.h"
#include "rotary.h"

namespace jkv {

static const int kPD = 128;            // head dim
static const int kPKT = 64;            // keys per tile
static const int kPThreads = 512;      // 8 waves
static const int kKStride = kPD + 8;   // K̂ tile row stride (halves): 272 B spreads keys over banks
static const int kVStride = kPKT + 4;  // V̂ᵀ tile row stride (halves): 136 B, conflict-free b64 reads and pair writes
static const int kKTile = kPKT * kKStride;
static const int kVTile = kPD * kVStride;

struct PrefillArgs {
  const _Float16* q;
  int64_t qsb, qsh, qst;
  const _Float16* k;
  int64_t ksb, ksh, kst;
  const _Float16* v;
  int64_t vsb, vsh, vst;
  int64_t B, QH, KVH, T;
  const int32_t* start;  // [B] position of the chunk's first token
  int64_t window;
  const _Float16* rope;  // [rope_len][2][64]: cos row, sin row
  int64_t rope_len;
  _Float16* out;  // [B,QH,T,D] contiguous
  float* lse;     // [B,QH,T] natural-log row normaliser, or null
  int32_t heads_per_wg;  // HW: query heads per workgroup (min(NQ, 4))
  int32_t row_sets;      // 8 / HW: 32-row sets per head in a workgroup
  int32_t head_groups;   // NQ / HW
  // codes instead of K̂/V̂ rows (prefill_attn_kernel<CS>, CS = stages): uint8
  // records [B,KVH,T,16,CS] with byte strides and the fp16 deployed tables
  // [KVH*16][CS][256][8]
  const uint8_t* kc;
  const uint8_t* vc;
  int64_t csb, csh, cst;
  const _Float16* kt16;
  const _Float16* vt16;
};

static const int kPCodeGroups = 16;  // codes path: 16 groups of 8 dims, 256 codewords
static const int kPCodewords = 256;

// max / sum of v over lanes l, l^16, l^32, l^48 (the four lane groups of one
// MFMA row) with the gfx950 row-swap permutes: VALU only, no LDS round trip.
// permlane16_swap(v, v) gives (v of the even row, v of the odd row) of each
// row pair in every lane; permlane32_swap(v, v) the same for the two halves.
__device__ __forceinline__ float lane_group_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float lane_group_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// max(a, b, c); the compiler forms v_max3_f32 from it
__device__ __forceinline__ float max3_f32(float a, float b, float c) { return fmaxf(fmaxf(a, b), c); }

// (a[e], b[e]) as one 32-bit word
__device__ __forceinline__ uint32_t pair16(half8 a, half8 b, int e) {
  const half2v h = {a[e], b[e]};
  return __builtin_bit_cast(uint32_t, h);
}

// transposing LDS read of the 8-byte piece at LDS byte address addr: in each
// 16-lane block, lane 4j + e receives element e of the pieces that the
// block's lanes j, j+4, j+8, j+12 address (ds_read_b64_tr_b16)
typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4v;
__device__ __forceinline__ half4 lds_read_tr16(uint32_t addr) {
  return __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(size_t)addr));
}

// CS = 0: the chunk's fp16 K̂/V̂ rows.  CS = 1, 2: K̂/V̂ rebuilt from uint8
// codes while each tile loads (codes -> 16-byte codeword gathers from the
// L2-resident fp16 tables -> fp16 stage sum, the codec's reconstruction), so
// K̂ and V̂ are never written to memory.
template <int CS>
__global__ __launch_bounds__(kPThreads) void prefill_attn_kernel(PrefillArgs a) {
  __shared__ __align__(16) _Float16 k_lds[2][kKTile];
  __shared__ __align__(16) _Float16 v_lds[2][kVTile];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the tile tests below branch on it
  const int ln = lane & 15, lg = lane >> 4;
  const int HW = a.heads_per_wg, RS = a.row_sets;
  const int64_t block_rows = 32 * (int64_t)RS;
  const int64_t nqb = ceil_div(a.T, block_rows);
  // logical block: query blocks fastest, then (kv head, head group), then
  // batch row.  xcd_remap keeps the query blocks of one (batch, kv head) on
  // one XCD, so its K/V tiles are fetched into one L2; longest key ranges go
  // first within each.
  const uint32_t bid = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t gy = a.KVH * a.head_groups;
  const int64_t qblk = nqb - 1 - (int64_t)(bid % (uint32_t)nqb);
  const int64_t yz = bid / (uint32_t)nqb;
  const int64_t kvh = (yz % gy) / a.head_groups;
  const int64_t hg = (yz % gy) % a.head_groups;
  const int64_t b = yz / gy;
  const int64_t NQ = a.QH / a.KVH;
  const int64_t head = kvh * NQ + hg * HW + wave % HW;
  const int64_t wg_row0 = qblk * block_rows;
  int64_t wg_row1 = wg_row0 + block_rows;
  if (wg_row1 > a.T) wg_row1 = a.T;
  const int64_t row0 = wg_row0 + (wave / HW) * 32;  // this wave's first query row
  const int64_t p0 = a.start[b];
  const float scale2 = 1.4426950408889634f / sqrtf((float)kPD);  // log2(e)/sqrt(D)

  auto rope_row = [&](int64_t pos) -> const _Float16* {
    int64_t r = pos < 0 ? 0 : pos;
    if (r >= a.rope_len) r = a.rope_len - 1;
    return a.rope + r * kRopeRow;
  };

  // ---- the wave's rotated queries: B operand (8 dims of row ln per lane) ----
  half8 qf[2][4];
#pragma unroll
  for (int rg = 0; rg < 2; ++rg) {
    const int64_t row = row0 + 16 * rg + ln;
    const bool ok = row < a.T;
    const _Float16* qp = a.q + b * a.qsb + head * a.qsh + (ok ? row : 0) * a.qst;
    const _Float16* tr = rope_row(p0 + (ok ? row : 0));
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int d0 = 32 * c + 8 * lg;  // < 64; partner d0 + 64
      half8 x0 = *(const half8*)(qp + d0);
      half8 x1 = *(const half8*)(qp + d0 + 64);
      half8 cs, sn, r0, r1;
      load_trig8(tr, d0, &cs, &sn);
      rope16(x0, x1, cs, sn, &r0, &r1);
      const half8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
      qf[rg][c] = ok ? r0 : zero;
      qf[rg][c + 2] = ok ? r1 : zero;
    }
  }

  float4v o[2][8];
#pragma unroll
  for (int rg = 0; rg < 2; ++rg)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[rg][dt] = float4v{0.f, 0.f, 0.f, 0.f};
  float m[2] = {-INFINITY, -INFINITY};
  float l[2] = {0.f, 0.f};

  int64_t kmin = wg_row0 - a.window + 1;
  if (kmin < 0) kmin = 0;
  const int64_t tile0 = kmin / kPKT;
  const int64_t tile1 = ceil_div(wg_row1, kPKT);
  const _Float16* kbase = CS == 0 ? a.k + b * a.ksb + kvh * a.ksh : nullptr;
  const _Float16* vbase = CS == 0 ? a.v + b * a.vsb + kvh * a.vsh : nullptr;

  // Tile loaders.  K̂: thread -> key tid/8, 8-dim chunk pair (p, p+8), p =
  // tid%8, rotated before it is stored.  V̂: thread -> key pair tid%32, dims
  // [8*(tid/32), +8), stored transposed as (key, key+1) words.  Every load
  // (the rotary rows too) is unconditional and its result untouched until
  // store(), so the wave waits for a tile's loads only after the current
  // tile's products: keys past T read a valid key of the tile (K̂ its last,
  // V̂ its first) and the mask gives them weight 0.
  const int kk = tid >> 3, kpart = tid & 7;
  const int vkp = tid & 31, vdb = tid >> 5;
  // rows: K̂ pair (p, p+8) and V̂ of two keys; codes: the stage words of the
  // same dims (groups p and p + 8 for K̂, group tid/32 of both keys for V̂)
  constexpr int NW = CS > 0 ? CS : 1;
  struct TileRegs {
    half8 k[2][NW], v[2][NW], cs, sn;
  };
  // the code bytes of one tile's K̂ pair and V̂ keys (CS > 0): dword 0 holds
  // groups p and p + 8 of key tid/8 (CS bytes each, at bytes 0 and 2), dword 1
  // group tid/32 of keys 2(tid%32) and 2(tid%32) + 1
  struct CodeRegs {
    uint32_t kw, vw;
  };
  // A tile's loads are a uniform base plus per-thread 32-bit offsets fixed
  // for the whole walk (offsets within one (batch row, kv head) slice fit 32
  // bits: host-checked); a key past T, or past the rotary table, takes the
  // offset of a valid one.
  const int64_t rstride_k = CS > 0 ? a.cst : a.kst, rstride_v = CS > 0 ? a.cst : a.vst;
  const uint32_t k_row = (uint32_t)(kk * rstride_k), v_row0 = (uint32_t)(2 * vkp * rstride_v),
                 v_row1 = v_row0 + (uint32_t)rstride_v;
  const uint32_t t_off = (uint32_t)(kk * kRopeRow + 8 * kpart);
  struct TileBase {
    int64_t first;
    uint32_t ko, vo0, vo1, to;  // row offsets (elements or bytes) of this thread's keys; rotary offset
    const _Float16* tt;
  };
  auto tile_base = [&](int64_t tile) {
    TileBase t;
    t.first = tile * kPKT;               // < T for every tile walked
    int64_t last = a.T - 1 - t.first;    // the tile's last valid key, relative
    if (last > kPKT - 1) last = kPKT - 1;
    int64_t pos = p0 + t.first;          // rotary row of the tile's first key
    if (pos > a.rope_len - 1) pos = a.rope_len - 1;
    if (pos < 0) pos = 0;
    int64_t tlast = a.rope_len - 1 - pos;  // keys past it use the table's last row
    if (tlast > last) tlast = last;
    const uint32_t lk = (uint32_t)last, lt = (uint32_t)tlast;
    t.ko = (uint32_t)kk <= lk ? k_row : (uint32_t)(last * rstride_k);
    t.vo0 = (uint32_t)(2 * vkp) <= lk ? v_row0 : 0u;
    t.vo1 = (uint32_t)(2 * vkp + 1) <= lk ? v_row1 : 0u;
    t.to = (uint32_t)kk <= lt ? t_off : (uint32_t)(tlast * kRopeRow + 8 * kpart);
    t.tt = a.rope + pos * kRopeRow;
    return t;
  };
  // CS > 0: the code bytes of a tile (loaded a tile before its gathers)
  const uint8_t* kcbase = CS > 0 ? a.kc + b * a.csb + kvh * a.csh : nullptr;
  const uint8_t* vcbase = CS > 0 ? a.vc + b * a.csb + kvh * a.csh : nullptr;
  auto load_codes = [&](int64_t tile, CodeRegs& c) {
    if constexpr (CS > 0) {
      const TileBase t = tile_base(tile);
      const uint8_t* kr = kcbase + t.first * a.cst + t.ko;
      const uint8_t* v0 = vcbase + t.first * a.cst + t.vo0 + vdb * CS;
      const uint8_t* v1 = vcbase + t.first * a.cst + t.vo1 + vdb * CS;
      if constexpr (CS == 2) {
        c.kw = (uint32_t)*(const uint16_t*)(kr + 2 * kpart) | ((uint32_t)*(const uint16_t*)(kr + 2 * (kpart + 8)) << 16);
        c.vw = (uint32_t)*(const uint16_t*)v0 | ((uint32_t)*(const uint16_t*)v1 << 16);
      } else {
        c.kw = (uint32_t)kr[kpart] | ((uint32_t)kr[kpart + 8] << 16);
        c.vw = (uint32_t)*v0 | ((uint32_t)*v1 << 16);
      }
    }
  };
  const _Float16* ktab = CS > 0 ? a.kt16 + kvh * (int64_t)kPCodeGroups * NW * kPCodewords * 8 : nullptr;
  const _Float16* vtab = CS > 0 ? a.vt16 + kvh * (int64_t)kPCodeGroups * NW * kPCodewords * 8 : nullptr;
  auto word = [&](const _Float16* tab, int g, int st, uint32_t code) -> half8 {
    return *(const half8*)(tab + ((g * NW + st) * kPCodewords + (int)code) * 8);
  };
  // CS = 0: K̂ rows and rotary rows through buffer loads: a per-thread 32-bit
  // offset and the tile's uniform one, with int32 row arithmetic (keys past T
  // read the tile's first key; positions clamp to the table)
  const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)kbase, (short)0, CS == 0 ? (int)(((a.T - 1) * a.kst + kPD) * 2) : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t t_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.rope, (short)0, (int)(a.rope_len * kRopeRow * 2), 0x00020000);
  const int32_t p32 = (int32_t)p0, rlast32 = (int32_t)(a.rope_len - 1), T32 = (int32_t)a.T;
  auto fetch = [&](int64_t tile, const CodeRegs& c, TileRegs& r) {
    if constexpr (CS == 0) {
      const int32_t first = (int32_t)(tile * kPKT);
      const uint32_t kr = first + kk < T32 ? (uint32_t)kk : 0u;
      int32_t pos = p32 >= rlast32 ? rlast32 : p32 + first + (int32_t)kr;  // (no int32 overflow)
      pos = pos < 0 ? 0 : (pos < rlast32 ? pos : rlast32);
      const uint32_t ko = kr * (uint32_t)a.kst * 2u + 16u * kpart, to = (uint32_t)pos * (2u * kRopeRow) + 16u * kpart;
      const int ks = (int)((uint32_t)first * (uint32_t)a.kst * 2u);
      r.k[0][0] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(k_rsrc, (int)ko, ks, 0));
      r.k[1][0] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(k_rsrc, (int)(ko + 128u), ks, 0));
      r.cs = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(t_rsrc, (int)to, 0, 0));
      r.sn = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(t_rsrc, (int)(to + 128u), 0, 0));
    } else {
      const TileBase t = tile_base(tile);
      r.cs = *(const half8*)(t.tt + t.to);
      r.sn = *(const half8*)(t.tt + t.to + 64);
#pragma unroll
      for (int st = 0; st < CS; ++st) {
        r.k[0][st] = word(ktab, kpart, st, (c.kw >> (8 * st)) & 0xffu);
        r.k[1][st] = word(ktab, kpart + 8, st, (c.kw >> (16 + 8 * st)) & 0xffu);
        r.v[0][st] = word(vtab, vdb, st, (c.vw >> (8 * st)) & 0xffu);
        r.v[1][st] = word(vtab, vdb, st, (c.vw >> (16 + 8 * st)) & 0xffu);
      }
    }
  };
  auto store = [&](const TileRegs& r, int buf) {
    // the codec's reconstruction: fp16 of the fp32 stage sum, which one fp16
    // add gives for two stages
    half8 k0 = r.k[0][0], k1 = r.k[1][0];
    if constexpr (CS == 2) {
      k0 = k0 + r.k[0][1];
      k1 = k1 + r.k[1][1];
    }
    half8 r0, r1;
    rope16(k0, k1, r.cs, r.sn, &r0, &r1);
    _Float16* kd = k_lds[buf] + kk * kKStride + 8 * kpart;
    *(half8*)kd = r0;
    *(half8*)(kd + 64) = r1;
    if constexpr (CS > 0) {
      half8 v0 = r.v[0][0], v1 = r.v[1][0];
      if constexpr (CS == 2) {
        v0 = v0 + r.v[0][1];
        v1 = v1 + r.v[1][1];
      }
      _Float16* vd = v_lds[buf] + (8 * vdb) * kVStride + 2 * vkp;
#pragma unroll
      for (int e = 0; e < 8; ++e) *(uint32_t*)(vd + e * kVStride) = pair16(v0, v1, e);
    }
  };
  // CS = 0: a tile's V̂ rows go global -> LDS directly (buffer_load_dwordx4
  // ... lds: lane i of an instruction lands at its LDS base + 16 i), row-major
  // [key][dim] with 16-byte chunk j of key r in slot j ^ 2 (r & 7), so that
  // the transposing reads of the product below (32 bytes of 8 keys) hit
  // distinct banks.  Wave w fills keys 8w..8w+7 with two instructions; keys
  // past T read the tile's first key (their weights are 0).  Offsets fit 32
  // bits (host-checked).
  const int vrow = 8 * wave + (lane >> 4), vslot = lane & 15;
  const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)vbase, (short)0, CS == 0 ? (int)(((a.T - 1) * a.vst + kPD) * 2) : 0, 0x00020000);
  auto copy_v = [&](int64_t tile, int buf) {
    if constexpr (CS == 0) {
      const int32_t first = (int32_t)(tile * kPKT), T32 = (int32_t)a.T;
      char* vd = (char*)v_lds[buf] + 2048 * wave;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = vrow + 4 * i;
        const uint32_t rr = first + r < T32 ? (uint32_t)r : 0u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            v_rsrc, (void __attribute__((address_space(3)))*)(vd + 1024 * i), 16,
            rr * (uint32_t)a.vst * 2u + 16u * (uint32_t)(vslot ^ (2 * (r & 7))), (uint32_t)first * (uint32_t)a.vst * 2u,
            0, 0);
      }
    }
  };

  // codes two tiles ahead, rows (or gathered words) one tile ahead
  CodeRegs cn = {0u, 0u};
  if (tile0 < tile1) {
    CodeRegs c0 = {0u, 0u};
    load_codes(tile0, c0);
    TileRegs r;
    fetch(tile0, c0, r);
    copy_v(tile0, 0);
    if (tile0 + 1 < tile1) load_codes(tile0 + 1, cn);
    store(r, 0);
    if constexpr (CS == 0) __builtin_amdgcn_s_waitcnt(0);  // the V̂ copies have landed
  }
  __syncthreads();

  for (int64_t tile = tile0; tile < tile1; ++tile) {
    const int buf = (int)((tile - tile0) & 1);
    const int64_t key0 = tile * kPKT;
    const bool more = tile + 1 < tile1;
    TileRegs nxt;
    if (more) {
      fetch(tile + 1, cn, nxt);
      copy_v(tile + 1, buf ^ 1);  // (the other buffer was freed by the last barrier)
    }
    if (tile + 2 < tile1) load_codes(tile + 2, cn);
    const _Float16* kl = k_lds[buf];
    const _Float16* vl = v_lds[buf];

    // ---- Sᵀ for the wave's 32 rows: 4 key groups x 2 row groups ----
    float4v s[4][2];
#pragma unroll
    for (int kg = 0; kg < 4; ++kg) {
      s[kg][0] = float4v{0.f, 0.f, 0.f, 0.f};
      s[kg][1] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const half8 ka = *(const half8*)(kl + (16 * kg + ln) * kKStride + 32 * c + 8 * lg);
        s[kg][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qf[0][c], s[kg][0], 0, 0, 0);
        s[kg][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qf[1][c], s[kg][1], 0, 0, 0);
      }
    }
    // ---- mask, online softmax, fp16 P in B-operand order.  Tiles wholly
    // inside every row's causal window need no mask (wave-uniform test); the
    // scale enters the exponent through one fma; the running output is only
    // rescaled when some row's reference maximum moves ----
    const bool full = key0 + kPKT - 1 <= row0 && row0 + 31 - key0 < a.window && key0 + kPKT <= a.T;
    half8 pf[2][2];
    float alpha[2];
    // the whole softmax in two versions under one uniform branch, so that the
    // unmasked tiles carry none of the mask's work or register copies
    auto softmax = [&](auto masked_tag) {
      constexpr bool masked = decltype(masked_tag)::value;
#pragma unroll
      for (int rg = 0; rg < 2; ++rg) {
        float mx = -INFINITY;
        if constexpr (!masked) {
          // two new scores per v_max3_f32
#pragma unroll
          for (int kg = 0; kg < 4; ++kg) {
            mx = max3_f32(mx, s[kg][rg][0], s[kg][rg][1]);
            mx = max3_f32(mx, s[kg][rg][2], s[kg][rg][3]);
          }
        } else {
          // row - key of element (kg, e) = d0 - 16 kg - e; key - key0 < keys_left
          // (rows and keys < T < 2^31: host-checked)
          const int d0 = (int)(row0 + 16 * rg + ln - key0) - 4 * lg;
          const int keys_left = (int)(a.T - key0 < kPKT ? a.T - key0 : kPKT);
          const int win = a.window < 0x40000000 ? (int)a.window : 0x40000000;
#pragma unroll
          for (int kg = 0; kg < 4; ++kg)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int diff = d0 - 16 * kg - e;
              const bool vis = diff >= 0 && diff < win && 16 * kg + 4 * lg + e < keys_left;
              const float v = vis ? s[kg][rg][e] : -INFINITY;
              s[kg][rg][e] = v;
              mx = fmaxf(mx, v);
            }
        }
        mx = lane_group_max(mx) * scale2;
        // the reference maximum only moves when the row maximum passes it by
        // more than 8 (so p < 2^8 and the output rescale is rare); o and l
        // share it, so o / l is unchanged
        const float m_new = mx > m[rg] + 8.f ? mx : m[rg];
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        alpha[rg] = __builtin_amdgcn_exp2f(m[rg] - m_use);
        m[rg] = m_new;
        float pr[16];
#pragma unroll
        for (int kg = 0; kg < 4; ++kg)
#pragma unroll
          for (int e = 0; e < 4; ++e) pr[4 * kg + e] = __builtin_amdgcn_exp2f(fmaf(s[kg][rg][e], scale2, -m_use));
        // the tile's row sum as a tree (four adds deep, not sixteen)
        float t8[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t8[i] = pr[2 * i] + pr[2 * i + 1];
        const float psum = ((t8[0] + t8[1]) + (t8[2] + t8[3])) + ((t8[4] + t8[5]) + (t8[6] + t8[7]));
        l[rg] = l[rg] * alpha[rg] + psum;
#pragma unroll
        for (int kp = 0; kp < 2; ++kp)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pf[rg][kp][e] = (_Float16)pr[4 * (2 * kp) + e];
            pf[rg][kp][e + 4] = (_Float16)pr[4 * (2 * kp + 1) + e];
          }
      }
    };
    if (full) {
      softmax(std::false_type{});
    } else {
      softmax(std::true_type{});
    }
#pragma unroll
    for (int rg = 0; rg < 2; ++rg)
      if (__any(alpha[rg] != 1.f)) {
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[rg][dt] *= alpha[rg];
      }
    // ---- Oᵀ += V̂ᵀ Pᵀ: contraction slot 8lg+e <-> key 32kp + 4lg + e (e < 4),
    //      32kp + 16 + 4lg + e - 4 (e >= 4) ----
    // (CS = 0: V̂ᵀ by two transposing reads of the row-major tile, keys
    // 32kp + 4lg + ln/4 and 16 further, dims 16dt + 4(ln%4))
    const int tr_row = 4 * lg + (ln >> 2);
    const uint32_t vtr = (uint32_t)(size_t)(const void __attribute__((address_space(3)))*)vl + (uint32_t)tr_row * 256u +
                         8u * (ln & 1);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) {
        half4 lo, hi;
        if constexpr (CS == 0) {
          const uint32_t at = vtr + 32u * 256u * kp + 16u * (uint32_t)((2 * dt + ((ln & 3) >> 1)) ^ (2 * (tr_row & 7)));
          lo = lds_read_tr16(at);
          hi = lds_read_tr16(at + 16u * 256u);
        } else {
          const _Float16* vr = vl + (16 * dt + ln) * kVStride + 32 * kp + 4 * lg;
          lo = *(const half4*)vr;
          hi = *(const half4*)(vr + 16);
        }
        const half8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[0][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pf[0][kp], o[0][dt], 0, 0, 0);
        o[1][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pf[1][kp], o[1][dt], 0, 0, 0);
      }
    }
    // ---- the next tile into the other buffer ----
    if (more) store(nxt, buf ^ 1);
    if constexpr (CS == 0) __builtin_amdgcn_s_waitcnt(0);  // the next tile's V̂ copies have landed
    __syncthreads();
  }

  // ---- normalise and store: lane holds dims 16dt + 4lg + e of row ln ----
#pragma unroll
  for (int rg = 0; rg < 2; ++rg) {
    const int64_t row = row0 + 16 * rg + ln;
    const float lt = lane_group_sum(l[rg]);
    if (row >= a.T) continue;
    if (a.lse != nullptr && lg == 0) {
      // log sum_s exp(q.k_s / sqrt(D)) = ln2 (m + log2 l), m in base-2 units
      const float mu = m[rg] == -INFINITY ? 0.f : m[rg];
      a.lse[(b * a.QH + head) * a.T + row] = (mu + log2f(lt)) * 0.6931471805599453f;
    }
    const float inv = 1.0f / lt;
    _Float16* op = a.out + ((b * a.QH + head) * a.T + row) * kPD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      half4 h;
#pragma unroll
      for (int e = 0; e < 4; ++e) h[e] = (_Float16)(o[rg][dt][e] * inv);
      *(half4*)(op + 16 * dt + 4 * lg) = h;
    }
  }
}

// the fields and grid both entry points share; launches CS's kernel
static int launch_prefill(PrefillArgs& a, int cs, const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                          int64_t B, int64_t QH, int64_t KVH, int64_t T, const int32_t* start, int64_t window,
                          const void* rope_table, int64_t rope_len, void* out, float* lse, hipStream_t stream) {
  a.q = (const _Float16*)q; a.qsb = q_sb; a.qsh = q_sh; a.qst = q_st;
  a.B = B; a.QH = QH; a.KVH = KVH; a.T = T;
  a.start = start;
  a.window = window;
  a.rope = (const _Float16*)rope_table;
  a.rope_len = rope_len;
  a.out = (_Float16*)out;
  a.lse = lse;
  const int64_t NQ = QH / KVH;
  a.heads_per_wg = (int32_t)(NQ < 4 ? NQ : 4);
  a.row_sets = 8 / a.heads_per_wg;
  a.head_groups = (int32_t)(NQ / a.heads_per_wg);
  const int64_t nqb = ceil_div(T, 32 * (int64_t)a.row_sets);
  const int64_t blocks = nqb * KVH * a.head_groups * B;
  JKV_CHECK_ARG(blocks < ((int64_t)1 << 31), "prefill grid too large");
  const dim3 grid((uint32_t)blocks), block(kPThreads);
  if (cs == 2) {
    hipLaunchKernelGGL(prefill_attn_kernel<2>, grid, block, 0, stream, a);
  } else if (cs == 1) {
    hipLaunchKernelGGL(prefill_attn_kernel<1>, grid, block, 0, stream, a);
  } else {
    hipLaunchKernelGGL(prefill_attn_kernel<0>, grid, block, 0, stream, a);
  }
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

}  // namespace jkv

extern "C" {

int jkv_prefill_attention(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st, const void* k,
                          int64_t k_sb, int64_t k_sh, int64_t k_st, const void* v, int64_t v_sb,
                          int64_t v_sh, int64_t v_st, int64_t B, int64_t QH, int64_t KVH,
                          int64_t T, int64_t D, const int32_t* start_positions, int64_t window,
                          const void* rope_table, int64_t rope_len, void* out, float* lse,
                          jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(D == kPD, "prefill attention supports head_dim 128, got %lld", (long long)D);
  JKV_CHECK_ARG(B >= 0 && QH > 0 && KVH > 0 && T >= 0 && QH % KVH == 0,
                "invalid prefill geometry");
  const int64_t NQ = QH / KVH;
  JKV_CHECK_ARG((NQ & (NQ - 1)) == 0, "query heads per kv head must be a power of two");
  JKV_CHECK_ARG(window >= 1, "window must be positive");
  JKV_CHECK_ARG(T < ((int64_t)1 << 31), "prefill chunk too long");
  JKV_CHECK_ARG(T * (k_st > v_st ? k_st : v_st) < ((int64_t)1 << 30), "prefill K/V rows too far apart");
  if (B == 0 || T == 0) return JKV_OK;
  JKV_CHECK_ARG(q && k && v && out && start_positions && rope_table, "null buffer");
  JKV_CHECK_ARG(rope_len >= 1 && rope_len < ((int64_t)1 << 23), "rotary table must have 1 to 2^23 - 1 rows");
  const int64_t strides[9] = {q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st};
  for (int i = 0; i < 9; ++i)
    JKV_CHECK_ARG(strides[i] % 8 == 0, "prefill strides must be multiples of 8 elements");
  JKV_CHECK_ARG(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) % 16 == 0,
                "prefill buffers must be 16-byte aligned");
  PrefillArgs a = {};
  a.k = (const _Float16*)k; a.ksb = k_sb; a.ksh = k_sh; a.kst = k_st;
  a.v = (const _Float16*)v; a.vsb = v_sb; a.vsh = v_sh; a.vst = v_st;
  return launch_prefill(a, 0, q, q_sb, q_sh, q_st, B, QH, KVH, T, start_positions, window, rope_table, rope_len,
                        out, lse, stream);
}

int jkv_prefill_attention_codes(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st, const uint8_t* k_codes,
                                const uint8_t* v_codes, int64_t code_sb, int64_t code_sh, int64_t code_st,
                                const void* k_tables, const void* v_tables, int64_t B, int64_t QH, int64_t KVH,
                                int64_t T, int64_t G, int64_t d, int64_t S, int64_t K,
                                const int32_t* start_positions, int64_t window, const void* rope_table,
                                int64_t rope_len, void* out, float* lse, jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(B >= 0 && QH > 0 && KVH > 0 && T >= 0 && QH % KVH == 0, "invalid prefill geometry");
  if (G != kPCodeGroups || d != 8 || (S != 1 && S != 2) || K != kPCodewords)
    return set_error(JKV_ENOTSUP, "prefill from codes needs 16 groups of 8 dims, 1-2 stages and 256 codewords");
  const int64_t NQ = QH / KVH;
  JKV_CHECK_ARG((NQ & (NQ - 1)) == 0, "query heads per kv head must be a power of two");
  JKV_CHECK_ARG(window >= 1, "window must be positive");
  JKV_CHECK_ARG(T < ((int64_t)1 << 31), "prefill chunk too long");
  JKV_CHECK_ARG(code_st >= G * S && T * code_st < ((int64_t)1 << 31), "code records overlap or lie too far apart");
  if (B == 0 || T == 0) return JKV_OK;
  JKV_CHECK_ARG(q && k_codes && v_codes && k_tables && v_tables && out && start_positions && rope_table,
                "null buffer");
  JKV_CHECK_ARG(rope_len >= 1, "rotary table is empty");
  JKV_CHECK_ARG(q_sb % 8 == 0 && q_sh % 8 == 0 && q_st % 8 == 0, "prefill strides must be multiples of 8 elements");
  JKV_CHECK_ARG(code_sb % 2 == 0 && code_sh % 2 == 0 && code_st % 2 == 0 && ((uintptr_t)k_codes % 2 == 0) &&
                    ((uintptr_t)v_codes % 2 == 0),
                "code records must be 2-byte aligned");
  JKV_CHECK_ARG(((uintptr_t)q | (uintptr_t)out | (uintptr_t)k_tables | (uintptr_t)v_tables) % 16 == 0,
                "prefill buffers must be 16-byte aligned");
  PrefillArgs a = {};
  a.kc = k_codes; a.vc = v_codes; a.csb = code_sb; a.csh = code_sh; a.cst = code_st;
  a.kt16 = (const _Float16*)k_tables; a.vt16 = (const _Float16*)v_tables;
  return launch_prefill(a, (int)S, q, q_sb, q_sh, q_st, B, QH, KVH, T, start_positions, window, rope_table,
                        rope_len, out, lse, stream);
}

}  // extern "C"
