// Straight-through codebook gradient scatter-add (the backward of the
// reference's torch.gather over fp16-deployed fp32 masters).
//
// grad_tables[h*G+g, s, k, :] += sum over rows whose stage-s code is k of the
// exit-summed upstream slice g*d:(g+1)*d.  Three kernels:
//   scatter_bins_kernel    LDS-privatised bins of one (head, group, stage,
//                          slice of 4 or 8 dims) over a chunk of rows (any d
//                          that is a multiple of 4).  fp16 gradients
//                          accumulate in exact 64-bit fixed point (every fp16
//                          value is an integer multiple of 2^-24), so the sum
//                          is exact, rounded to fp32 once, and bit-identical
//                          from run to run; bf16/fp32 gradients use fp32 LDS
//                          atomics.
//   scatter_global_kernel  global fp32 atomics (misaligned gradients, or d not
//                          a multiple of 4).
//   scatter_det_*          fixed-order fp32 sums for bf16/fp32 gradients when
//                          a deterministic result is asked for.
// scatter_group8_kernel (below) serves fp16 8-dim groups with every stage's
// bins in one block.  The bins and group8 kernels also run many scatters of
// one geometry (a calibration step's layers) in one launch, one job per
// range of blocks, storing or adding their sums.
#include <type_traits>

#include "jkv_common.h"

namespace jkv {

struct ScatterArgs {
  const void* grads[JKV_MAX_EXITS];
  int32_t exit_depth[JKV_MAX_EXITS];
  int32_t n_exits;
  const uint8_t* codes;
  int64_t cb, ch, ct;
  int64_t B, H, T, G, d, S, K;
  float* grad_tables;  // [H*G,S,K,d]
  int64_t rows_per_chunk;
  int64_t n_chunks;
  void* partials;            // per-chunk partial bins (workspace)
};

// Many scatters of one geometry in one launch (every layer's value tables):
// the geometry and exits once, then each job's buffers.  One row chunk per
// job, so no partial bins.  Job j takes logical blocks [j * per_job,
// (j + 1) * per_job).  overwrite != 0 stores the sums instead of adding them
// (the gradient tables need not be initialised).
static const int kMaxScatterJobs = 64;
static const int kMaxScatterJobExits = 1;
struct ScatterJobBuffers {
  const void* grads[kMaxScatterJobExits];
  const uint8_t* codes;
  float* grad_tables;
};
struct ScatterManyArgs {
  ScatterArgs shape;  // geometry, strides, exits (its buffers unused)
  int64_t per_job;
  int32_t n_jobs;
  int32_t overwrite;
  ScatterJobBuffers buf[kMaxScatterJobs];
};
template <bool MANY> struct ScatterArgsOf { using type = ScatterArgs; };
template <> struct ScatterArgsOf<true> { using type = ScatterManyArgs; };

template <int DT>
__device__ __forceinline__ float grad_sum(const ScatterArgs& a, int s, int64_t off) {
  float acc = 0.f;
  for (int e = 0; e < a.n_exits; ++e)
    if (a.exit_depth[e] > s) acc += Elem<DT>::load(a.grads[e], off);
  return acc;
}

// fp16 value times 2^24 as an exact integer (|result| < 2^40), in four
// instructions: f * 2^24 + 1.5 * 2^52 is an integer in [2^52, 2^53), exact in
// fp64, whose bit pattern is that of 1.5 * 2^52 plus the integer; the low word
// of 1.5 * 2^52 is zero, so subtracting its high word gives the int64.  The
// high word of a finite value lies in [0x4337FF00, 0x433800FF]; inf and nan
// give 0x7FF00000 or more, which `hmax` (the largest high word seen) reveals.
__device__ __forceinline__ long long fp16_fixed(uint16_t bits, uint32_t& hmax) {
  const float f = (float)__builtin_bit_cast(_Float16, bits);
  const double y = __builtin_fma((double)f, 16777216.0, 6755399441055744.0);
  const unsigned long long w = __builtin_bit_cast(unsigned long long, y);
  const uint32_t hi = (uint32_t)(w >> 32);
  hmax = max(hmax, hi);
  return (long long)(((unsigned long long)(hi - 0x43380000u) << 32) | (uint32_t)w);
}
__device__ __forceinline__ bool fixed_nonfinite(uint32_t hmax) { return hmax > 0x433800FFu; }

__device__ __forceinline__ float fixed_to_float(long long v) {
  return (float)v * 5.9604644775390625e-8f;  // 2^-24: exact scaling
}

// D gradient elements at element offset `off` (a multiple of D, base
// aligned to D elements) with one vector load, as the accumulator type:
// exact fixed point for fp16 (Acc = long long, `bad` flags inf/nan) or fp32.
template <int DT, int D, typename Acc>
__device__ __forceinline__ void load_slice(const void* base, int64_t off, Acc (&v)[D],
                                           uint32_t& bad) {
  typedef typename Elem<DT>::T T;
  typedef T TV __attribute__((ext_vector_type(D)));
  if constexpr (std::is_same<Acc, long long>::value) {
    typedef uint16_t UV __attribute__((ext_vector_type(D)));
    const UV x = *(const UV*)((const uint16_t*)base + off);
    uint32_t hmax = 0u;
#pragma unroll
    for (int i = 0; i < D; ++i) v[i] = fp16_fixed(x[i], hmax);
    bad |= fixed_nonfinite(hmax) ? 1u : 0u;
  } else {
    const TV x = *(const TV*)((const T*)base + off);
#pragma unroll
    for (int i = 0; i < D; ++i) {
      if constexpr (DT == JKV_BF16) {
        v[i] = __uint_as_float((uint32_t)x[i] << 16);
      } else {
        v[i] = (float)x[i];
      }
    }
  }
}

__device__ __forceinline__ void lds_add(long long* p, long long v) {
  atomicAdd((unsigned long long*)p, (unsigned long long)v);  // ds_add_u64
}
__device__ __forceinline__ void lds_add(float* p, float v) { atomicAdd(p, v); }

// One block per (head h, group g, stage s, slice j of D dims of the group)
// over a chunk of rows: the block owns bins grad[h*G+g, s, :, j*D:(j+1)*D],
// held in LDS ([K][D+1]; the pad element spreads consecutive codewords over
// the banks), and every row adds its exit-summed D-dim slice to the bin of its
// stage-s code with an LDS atomic.  Splitting by bins rather than by rows
// means no block's bins overlap another's when the rows are not chunked: the
// block adds them straight into the gradient.  With several row chunks each
// block stores its bins as the chunk's partial and a reduce kernel sums them.
// Logical blocks run slice, stage, group, head, chunk from fastest to
// slowest; xcd_remap keeps consecutive logical blocks on one XCD, so the
// blocks that read the same rows (one head) share an L2.
//
// Fixed-point mode (fp16): if a slice holds inf or nan the block discards its
// bins and adds every slice of its chunk with global fp32 atomics instead,
// which gives the IEEE inf/nan outcome of a floating-point sum.
//
// MANY: one launch for many jobs of one geometry (ScatterManyArgs), one row
// chunk each; with `overwrite` the block stores its bins (zeros for a stage
// no exit reaches) instead of adding them.
template <int DT, int D, bool MANY>
__global__ __launch_bounds__(1024) void scatter_bins_kernel(typename ScatterArgsOf<MANY>::type m) {
  constexpr bool kFixed = DT == JKV_F16;
  constexpr int U = 4;  // rows per thread with their loads in flight together
  typedef typename std::conditional<kFixed, long long, float>::type Acc;
  extern __shared__ __align__(16) unsigned char lds_raw[];
  Acc* bins = (Acc*)lds_raw;
  __shared__ uint32_t nonfinite;

  uint32_t bid = xcd_remap(blockIdx.x, gridDim.x);
  const ScatterArgs* ap;
  const void* grad0 = nullptr;  // a many-job launch's one exit gradient
  const uint8_t* codes;
  float* grad_tables;
  bool overwrite = false;
  if constexpr (MANY) {
    const uint32_t per = (uint32_t)m.per_job;
    const uint32_t job = bid / per;
    if (job >= (uint32_t)m.n_jobs) return;  // grid padding (before any barrier)
    bid -= job * per;
    ap = &m.shape;
    grad0 = m.buf[job].grads[0];
    codes = m.buf[job].codes;
    grad_tables = m.buf[job].grad_tables;
    overwrite = m.overwrite != 0;
  } else {
    ap = &m;
    codes = m.codes;
    grad_tables = m.grad_tables;
  }
  const ScatterArgs& a = *ap;
  auto grads = [&](int e) -> const void* {
    if constexpr (MANY) {
      return grad0;
    } else {
      return a.grads[e];
    }
  };
  const int S = (int)a.S, K = (int)a.K, d = (int)a.d;
  const uint32_t n_slices = (uint32_t)(d / D);
  const uint32_t j = bid % n_slices;
  const uint32_t s = (bid / n_slices) % (uint32_t)S;
  const uint32_t p = (bid / (n_slices * S)) % (uint32_t)(a.H * a.G);
  const uint32_t chunk = bid / (n_slices * S * (uint32_t)(a.H * a.G));
  const uint32_t h = p / (uint32_t)a.G, g = p % (uint32_t)a.G;
  const int per_out = K * D;
  float* const out_base = grad_tables + (((int64_t)p * S + s) * K) * d + (int64_t)j * D;
  Acc* const part_base =
      (Acc*)a.partials + ((((int64_t)chunk * a.H * a.G + p) * S + s) * K) * d + (int64_t)j * D;

  bool active = false;  // some exit reaches stage s
  for (int e = 0; e < a.n_exits; ++e) active = active || a.exit_depth[e] > (int)s;
  if (!active) {
    if (a.n_chunks > 1)
      for (int i = threadIdx.x; i < per_out; i += blockDim.x)
        part_base[(int64_t)(i / D) * d + i % D] = (Acc)0;
    if (overwrite)
      for (int i = threadIdx.x; i < per_out; i += blockDim.x) out_base[(int64_t)(i / D) * d + i % D] = 0.f;
    return;
  }
  for (int i = threadIdx.x; i < K * (D + 1); i += blockDim.x) bins[i] = (Acc)0;
  if (threadIdx.x == 0) nonfinite = 0u;
  __syncthreads();

  const int64_t rows = a.B * a.T;
  const int64_t r0 = (int64_t)chunk * a.rows_per_chunk;
  int64_t r1 = r0 + a.rows_per_chunk;
  if (r1 > rows) r1 = rows;
  const int64_t Dfull = a.G * d;
  const int64_t col = (int64_t)g * d + (int64_t)j * D;
  const uint32_t T32 = (uint32_t)a.T;
  uint32_t bad = 0u;

  // Visits the rows of the chunk U at a time: row_fn(offsets, codes, valid).
  auto for_rows = [&](auto&& row_fn) {
    for (int64_t row0 = r0 + threadIdx.x; row0 < r1; row0 += (int64_t)U * blockDim.x) {
      int64_t offs[U];
      uint32_t cv[U];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t row = row0 + (int64_t)u * blockDim.x;
        ok[u] = row < r1;
        const uint32_t rw = (uint32_t)(ok[u] ? row : r0);
        const uint32_t b = rw / T32, t = rw - b * T32;
        offs[u] = (((int64_t)b * a.H + h) * a.T + t) * Dfull + col;
        cv[u] = codes[(int64_t)b * a.cb + (int64_t)h * a.ch + (int64_t)t * a.ct +
                      (int64_t)g * S + s];
      }
      row_fn(offs, cv, ok);
    }
  };

  for_rows([&](const int64_t(&offs)[U], const uint32_t(&cv)[U], const bool(&ok)[U]) {
    Acc v[U][D];
    if (MANY || a.n_exits == 1) {  // a many-job launch takes one exit
#pragma unroll
      for (int u = 0; u < U; ++u) load_slice<DT, D>(grads(0), offs[u], v[u], bad);
    } else {
      // stage s takes the sum of the exits deeper than s
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < D; ++i) v[u][i] = (Acc)0;
      for (int e = 0; e < a.n_exits; ++e) {
        if (a.exit_depth[e] <= (int)s) continue;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          Acc x[D];
          load_slice<DT, D>(grads(e), offs[u], x, bad);
#pragma unroll
          for (int i = 0; i < D; ++i) v[u][i] += x[i];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!ok[u]) continue;
      Acc* bin = bins + cv[u] * (D + 1);
#pragma unroll
      for (int i = 0; i < D; ++i) lds_add(&bin[i], v[u][i]);
    }
  });
  if constexpr (kFixed) {
    if (bad) atomicOr(&nonfinite, 1u);
  }
  __syncthreads();

  if (kFixed && nonfinite) {
    // fp32 sums with global atomics (exit sums in exit order, as grad_sum)
    if (overwrite) {
      // this block owns its part of the table: clear it, and make the stores
      // reach memory before any atomic adds to it
      for (int i = threadIdx.x; i < per_out; i += blockDim.x) out_base[(int64_t)(i / D) * d + i % D] = 0.f;
      __threadfence();
      __syncthreads();
    }
    for_rows([&](const int64_t(&offs)[U], const uint32_t(&cv)[U], const bool(&ok)[U]) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (!ok[u]) continue;
        float* dst = out_base + (int64_t)cv[u] * d;
#pragma unroll
        for (int i = 0; i < D; ++i) {
          float acc = 0.f;
          for (int e = 0; e < a.n_exits; ++e)
            if (a.exit_depth[e] > (int)s) acc += Elem<DT>::load(grads(e), offs[u] + i);
          if (acc != 0.f || acc != acc) atomicAdd(&dst[i], acc);
        }
      }
    });
    if (a.n_chunks > 1)
      for (int i = threadIdx.x; i < per_out; i += blockDim.x)
        part_base[(int64_t)(i / D) * d + i % D] = (Acc)0;
    return;
  }
  for (int i = threadIdx.x; i < per_out; i += blockDim.x) {
    const int k = i / D, c = i - k * D;
    const Acc v = bins[k * (D + 1) + c];
    if (a.n_chunks == 1) {
      float x;
      if constexpr (kFixed) {
        x = fixed_to_float(v);
      } else {
        x = v;
      }
      if (overwrite) {
        out_base[(int64_t)k * d + c] = x;
      } else {
        out_base[(int64_t)k * d + c] += x;
      }
    } else {
      part_base[(int64_t)k * d + c] = v;
    }
  }
}

// fp16 gradients with 8-dim groups (the G2 / cq1 geometry): one block of
// 1024 threads owns every stage's bins of one (head, group) over a chunk of
// rows, so each row's 16-byte gradient slice is read once and feeds all
// stages (bins [S][K][9] of exact 64-bit fixed point in LDS).  Row
// addresses advance by the block stride without a division per row.
// Logical blocks run group, chunk, head from fastest to slowest: the groups
// of one row range share its 256-byte rows in one XCD's L2.
//
// MANY: one launch for many jobs of one geometry and one exit
// (ScatterManyArgs), one row chunk each; with `overwrite` the block stores
// its bins instead of adding them.
template <int S, bool MANY>
__global__ __launch_bounds__(1024) void scatter_group8_kernel(typename ScatterArgsOf<MANY>::type m) {
  constexpr int D = 8, U = 4, kPad = D + 1;
  extern __shared__ __align__(16) unsigned char lds_raw[];
  long long* bins = (long long*)lds_raw;  // [S][K][kPad]
  __shared__ uint32_t nonfinite;
  uint32_t bid = xcd_remap(blockIdx.x, gridDim.x);
  const ScatterArgs* ap;
  const void* grad0 = nullptr;
  const uint8_t* codes;
  float* grad_tables;
  bool overwrite = false;
  if constexpr (MANY) {
    const uint32_t per = (uint32_t)m.per_job;
    const uint32_t job = bid / per;
    if (job >= (uint32_t)m.n_jobs) return;  // grid padding (before any barrier)
    bid -= job * per;
    ap = &m.shape;
    grad0 = m.buf[job].grads[0];
    codes = m.buf[job].codes;
    grad_tables = m.buf[job].grad_tables;
    overwrite = m.overwrite != 0;
  } else {
    ap = &m;
    codes = m.codes;
    grad_tables = m.grad_tables;
  }
  const ScatterArgs& a = *ap;
  auto grads = [&](int e) -> const void* {
    if constexpr (MANY) {
      return grad0;
    } else {
      return a.grads[e];
    }
  };
  const int K = (int)a.K;
  const uint32_t G = (uint32_t)a.G;
  const uint32_t g = bid % G;
  const uint32_t chunk = (bid / G) % (uint32_t)a.n_chunks;
  const uint32_t h = bid / (G * (uint32_t)a.n_chunks);
  const uint32_t p = h * G + g;
  for (int i = threadIdx.x; i < S * K * kPad; i += blockDim.x) bins[i] = 0;
  if (threadIdx.x == 0) nonfinite = 0u;
  __syncthreads();

  // rows [r0, r1) of this chunk; offsets fit 32 bits (host-checked)
  const uint32_t rows = (uint32_t)(a.B * a.T), T32 = (uint32_t)a.T;
  const uint32_t r0 = chunk * (uint32_t)a.rows_per_chunk;
  const uint32_t r1 = min(r0 + (uint32_t)a.rows_per_chunk, rows);
  const uint32_t Dfull = G * D;
  const uint32_t gstride_t = Dfull, gstride_b = (uint32_t)a.H * T32 * Dfull;
  const uint32_t gbase = h * T32 * Dfull + g * D;
  const int64_t cbase = (int64_t)h * a.ch + (int64_t)g * S;
  const uint32_t step = blockDim.x;
  // this thread's first row as (b, t); later rows advance by `step`
  uint32_t row = r0 + threadIdx.x;
  uint32_t b = row / T32, t = row - b * T32;
  auto advance = [&]() {
    row += step;
    if (T32 >= step) {
      t += step;
      if (t >= T32) { t -= T32; ++b; }
    } else {
      b = row / T32;
      t = row - b * T32;
    }
  };
  uint32_t bad = 0u;
  while (row < r1) {
    uint32_t goff[U];
    int64_t coff[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ok[u] = row < r1;
      goff[u] = ok[u] ? b * gstride_b + gbase + t * gstride_t : gbase;
      coff[u] = ok[u] ? (int64_t)b * a.cb + cbase + (int64_t)t * a.ct : cbase;
      advance();
    }
    uint32_t code[U][S];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int s = 0; s < S; ++s) code[u][s] = codes[coff[u] + s];
    // each exit's slice goes straight into the bins of the stages it covers
    // (exact integer sums, so the order of the additions does not matter)
    const int n_exits = MANY ? 1 : a.n_exits;
    for (int e = 0; e < n_exits; ++e) {
      long long x[U][D];
#pragma unroll
      for (int u = 0; u < U; ++u) load_slice<JKV_F16, D>(grads(e), goff[u], x[u], bad);
      const int depth = a.exit_depth[e];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (!ok[u]) continue;
#pragma unroll
        for (int s = 0; s < S; ++s) {
          if (s >= depth) continue;
          long long* bin = bins + (s * K + (int)code[u][s]) * kPad;
#pragma unroll
          for (int i = 0; i < D; ++i) lds_add(&bin[i], x[u][i]);
        }
      }
    }
  }
  if (bad) atomicOr(&nonfinite, 1u);
  __syncthreads();

  const int64_t d = a.d;
  if (nonfinite) {
    // a slice holds inf or nan: fp32 sums with global atomics give the IEEE
    // outcome (exit sums in exit order, as grad_sum)
    if (overwrite) {
      // this block owns its (head, group) of the table: clear it, and make
      // the stores reach memory before any atomic adds to it
      float* own = grad_tables + (int64_t)p * S * K * d;
      for (int i = threadIdx.x; i < S * K * D; i += blockDim.x) own[i] = 0.f;
      __threadfence();
      __syncthreads();
    }
    for (uint32_t rr = r0 + threadIdx.x; rr < r1; rr += step) {
      const uint32_t bb = rr / T32, tt = rr - bb * T32;
      const int64_t off = (int64_t)bb * gstride_b + gbase + (int64_t)tt * gstride_t;
      const int64_t co = (int64_t)bb * a.cb + cbase + (int64_t)tt * a.ct;
      for (int s = 0; s < S; ++s) {
        float* dst = grad_tables + (((int64_t)p * S + s) * K + codes[co + s]) * d;
        for (int i = 0; i < D; ++i) {
          float acc = 0.f;
          for (int e = 0; e < a.n_exits; ++e)
            if (a.exit_depth[e] > s) acc += Elem<JKV_F16>::load(grads(e), off + i);
          if (acc != 0.f || acc != acc) atomicAdd(&dst[i], acc);
        }
      }
    }
    if (a.n_chunks > 1) {
      long long* part = (long long*)a.partials + (((int64_t)chunk * a.H * a.G + p) * S) * K * d;
      for (int i = threadIdx.x; i < S * K * D; i += blockDim.x) part[i] = 0;
    }
    return;
  }
  // element i = 8k + c of stage s's bins (d = D here)
  const int64_t pbase = (int64_t)p * S * K * D;
  long long* part = a.n_chunks > 1 ? (long long*)a.partials + (int64_t)chunk * a.H * a.G * S * K * D + pbase
                                   : nullptr;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    for (int i = threadIdx.x; i < K * D; i += blockDim.x) {
      const long long v = bins[(s * K + (i >> 3)) * kPad + (i & 7)];
      const int64_t o = (int64_t)s * K * D + i;
      if (a.n_chunks == 1) {
        if (overwrite) {
          grad_tables[pbase + o] = fixed_to_float(v);
        } else {
          grad_tables[pbase + o] += fixed_to_float(v);
        }
      } else {
        part[o] = v;
      }
    }
  }
}

// grad[p, ...] += sum over chunks of the per-chunk partials: an exact integer
// sum for fixed-point partials, else an fp32 sum in chunk order.
template <typename Acc>
__global__ __launch_bounds__(256) void scatter_chunk_reduce_kernel(ScatterArgs a,
                                                                   int64_t per_chunk) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= per_chunk) return;
  const Acc* part = (const Acc*)a.partials;
  Acc acc = (Acc)0;
  for (int64_t c = 0; c < a.n_chunks; ++c) acc += part[c * per_chunk + idx];
  if constexpr (std::is_same<Acc, long long>::value) {
    a.grad_tables[idx] += fixed_to_float(acc);
  } else {
    a.grad_tables[idx] += acc;
  }
}

// Direct global atomics, one thread per gradient element.
template <int DT>
__global__ __launch_bounds__(256) void scatter_global_kernel(ScatterArgs a) {
  const int64_t D = a.G * a.d;
  const int64_t n = a.B * a.H * a.T * D;
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int64_t col = idx % D;
  const int64_t bht = idx / D;
  const int64_t t = bht % a.T, bh = bht / a.T;
  const int64_t h = bh % a.H, b = bh / a.H;
  const int64_t g = col / a.d, i = col % a.d;
  const uint8_t* cp = a.codes + b * a.cb + h * a.ch + t * a.ct + g * a.S;
  const int64_t p = h * a.G + g;
  for (int s = 0; s < (int)a.S; ++s) {
    const float v = grad_sum<DT>(a, s, idx);
    if (v != 0.f || v != v)
      atomicAdd(&a.grad_tables[((p * a.S + s) * a.K + cp[s]) * a.d + i], v);
  }
}

// Deterministic path, pass 1: partial[c][p][s][k][i] = ordered sum over the
// rows of chunk c whose stage-s code is k.  One thread per (p, s, k, i).
template <int DT>
__global__ __launch_bounds__(256) void scatter_det_partial_kernel(ScatterArgs a) {
  const int64_t P = a.H * a.G;
  const int64_t per_chunk = P * a.S * a.K * a.d;
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= per_chunk * a.n_chunks) return;
  const int64_t c = idx / per_chunk;
  const int64_t rem = idx % per_chunk;
  const int64_t i = rem % a.d;
  const int64_t k = (rem / a.d) % a.K;
  const int64_t s = (rem / (a.d * a.K)) % a.S;
  const int64_t p = rem / (a.d * a.K * a.S);
  const int64_t h = p / a.G, g = p % a.G;
  const int64_t rows = a.B * a.T;
  const int64_t r0 = c * a.rows_per_chunk;
  int64_t r1 = r0 + a.rows_per_chunk;
  if (r1 > rows) r1 = rows;
  const int64_t D = a.G * a.d;
  float acc = 0.f;
  for (int64_t row = r0; row < r1; ++row) {
    const int64_t b = row / a.T, t = row % a.T;
    if (a.codes[b * a.cb + h * a.ch + t * a.ct + g * a.S + s] != k) continue;
    acc += grad_sum<DT>(a, (int)s, ((b * a.H + h) * a.T + t) * D + g * a.d + i);
  }
  ((float*)a.partials)[idx] = acc;
}

static const int64_t kDetRowsPerChunk = 256;

// Plan of scatter_bins_kernel.  Tuning knobs: the block count to reach and
// the minimum rows per chunk (a chunk's partial is as large as its bins).
#ifndef JKV_SCATTER_TARGET_BLOCKS
#define JKV_SCATTER_TARGET_BLOCKS 256
#endif
#ifndef JKV_SCATTER_MIN_ROWS
#define JKV_SCATTER_MIN_ROWS 2048
#endif

struct BinsPlan {
  bool ok;
  bool fixed;      // exact 64-bit fixed-point bins (fp16 gradients)
  bool group8;     // scatter_group8_kernel: every stage of an 8-dim group per block
  int32_t slice;   // dims per block (D): 8 or 4, dividing d
  int64_t chunks;  // row chunks (power of two)
  size_t lds;      // dynamic LDS bytes per block
  int64_t workspace;
};

static BinsPlan bins_plan(int64_t B, int64_t T, int64_t H, int64_t G, int64_t d, int64_t S,
                          int64_t K, int32_t grad_dtype) {
  BinsPlan r = {false, false, false, 0, 1, 0, 0};
  const int64_t rows = B * T;
  if (d % 4 != 0 || rows >= ((int64_t)1 << 31)) return r;
  r.slice = d % 8 == 0 ? 8 : 4;
  // fixed point: |bin| < rows * 8 exits * 2^40 must stay below 2^63
  r.fixed = grad_dtype == JKV_F16 && rows <= ((int64_t)1 << 20);
  const int64_t acc_bytes = r.fixed ? 8 : 4;
  // every stage of an 8-dim group in one block (32-bit offsets over the
  // gradient rows, B*H*T*G*8 elements, and the code records), unless one
  // block per stage already fills the chip: then there are no row chunks, no
  // partial bins and no reduce launch, which costs less than reading each
  // slice once per stage (17.0 against 19.6 us at 128 groups x 2 stages)
  const bool stages_fill = H * G * S * (d / r.slice) >= JKV_SCATTER_TARGET_BLOCKS;
  r.group8 = r.fixed && d == 8 && S <= 4 && K <= 256 && B * H * T * G * d < ((int64_t)1 << 31) &&
             !stages_fill;
  if (r.group8) {
    const int64_t blocks = H * G;
    int64_t chunks = 1;
    while (blocks * chunks < JKV_SCATTER_TARGET_BLOCKS &&
           ceil_div(rows, chunks * 2) >= JKV_SCATTER_MIN_ROWS)
      chunks *= 2;
    r.ok = true;
    r.chunks = chunks;
    r.lds = (size_t)(S * K * (d + 1) * acc_bytes);
    r.workspace = chunks > 1 ? chunks * H * G * S * K * d * acc_bytes : 0;
    return r;
  }
  const int64_t blocks = H * G * S * (d / r.slice);
  if (blocks >= ((int64_t)1 << 24)) return r;
  int64_t chunks = 1;
  while (blocks * chunks < JKV_SCATTER_TARGET_BLOCKS &&
         ceil_div(rows, chunks * 2) >= JKV_SCATTER_MIN_ROWS)
    chunks *= 2;
  r.ok = true;
  r.chunks = chunks;
  r.lds = (size_t)(K * (r.slice + 1) * acc_bytes);
  r.workspace = chunks > 1 ? chunks * H * G * S * K * d * acc_bytes : 0;
  return r;
}

// The deterministic request is met by the fixed-point bins (exact sums);
// otherwise it takes the ordered two-pass kernels.
static bool use_ordered(const BinsPlan& plan, int32_t deterministic) {
  return deterministic && !(plan.ok && plan.fixed);
}

static int64_t scatter_workspace(int64_t B, int64_t H, int64_t T, int64_t G, int64_t d, int64_t S,
                                 int64_t K, int32_t grad_dtype, int32_t deterministic) {
  const BinsPlan plan = bins_plan(B, T, H, G, d, S, K, grad_dtype);
  if (use_ordered(plan, deterministic))
    return ceil_div(B * T, kDetRowsPerChunk) * H * G * S * K * d * (int64_t)sizeof(float);
  return plan.ok ? plan.workspace : 0;
}

template <int DT>
static int launch_scatter(ScatterArgs a, int deterministic, hipStream_t stream) {
  const int64_t rows = a.B * a.T;
  const int64_t P = a.H * a.G;
  const BinsPlan plan = bins_plan(a.B, a.T, a.H, a.G, a.d, a.S, a.K, DT);
  if (use_ordered(plan, deterministic)) {
    a.rows_per_chunk = kDetRowsPerChunk;
    a.n_chunks = ceil_div(rows, kDetRowsPerChunk);
    const int64_t per_chunk = P * a.S * a.K * a.d;
    hipLaunchKernelGGL(scatter_det_partial_kernel<DT>,
                       dim3((uint32_t)ceil_div(per_chunk * a.n_chunks, 256)), dim3(256), 0,
                       stream, a);
    JKV_CHECK_LAUNCH();
    hipLaunchKernelGGL(scatter_chunk_reduce_kernel<float>,
                       dim3((uint32_t)ceil_div(per_chunk, 256)), dim3(256), 0, stream, a,
                       per_chunk);
    JKV_CHECK_LAUNCH();
    return JKV_OK;
  }
  bool aligned = true;
  const uintptr_t align = (uintptr_t)(plan.ok ? plan.slice * sizeof(typename Elem<DT>::T) : 1);
  for (int e = 0; e < a.n_exits; ++e) aligned = aligned && ((uintptr_t)a.grads[e] % align == 0);
  JKV_CHECK_ARG(aligned || !deterministic,
                "deterministic scatter needs gradient buffers aligned to 8 (or 4) elements");
  if (plan.ok && aligned && plan.group8) {
    a.n_chunks = plan.chunks;
    a.rows_per_chunk = ceil_div(rows, plan.chunks);
    int64_t nblocks = P * plan.chunks;
    const dim3 grid((uint32_t)nblocks);
    switch (a.S) {
      case 1: hipLaunchKernelGGL((scatter_group8_kernel<1, false>), grid, dim3(1024), plan.lds, stream, a); break;
      case 2: hipLaunchKernelGGL((scatter_group8_kernel<2, false>), grid, dim3(1024), plan.lds, stream, a); break;
      case 3: hipLaunchKernelGGL((scatter_group8_kernel<3, false>), grid, dim3(1024), plan.lds, stream, a); break;
      default: hipLaunchKernelGGL((scatter_group8_kernel<4, false>), grid, dim3(1024), plan.lds, stream, a); break;
    }
    JKV_CHECK_LAUNCH();
    if (a.n_chunks > 1) {
      const int64_t per_chunk = P * a.S * a.K * a.d;
      hipLaunchKernelGGL(scatter_chunk_reduce_kernel<long long>, dim3((uint32_t)ceil_div(per_chunk, 256)),
                         dim3(256), 0, stream, a, per_chunk);
      JKV_CHECK_LAUNCH();
    }
    return JKV_OK;
  }
  if (plan.ok && aligned && !plan.group8) {
    a.n_chunks = plan.chunks;
    a.rows_per_chunk = ceil_div(rows, plan.chunks);
    const dim3 grid((uint32_t)(P * a.S * (a.d / plan.slice) * plan.chunks));
    if (plan.slice == 8) {
      hipLaunchKernelGGL((scatter_bins_kernel<DT, 8, false>), grid, dim3(1024), plan.lds, stream, a);
    } else {
      hipLaunchKernelGGL((scatter_bins_kernel<DT, 4, false>), grid, dim3(1024), plan.lds, stream, a);
    }
    JKV_CHECK_LAUNCH();
    if (a.n_chunks > 1) {
      const int64_t per_chunk = P * a.S * a.K * a.d;
      const dim3 rgrid((uint32_t)ceil_div(per_chunk, 256));
      if (plan.fixed) {
        hipLaunchKernelGGL(scatter_chunk_reduce_kernel<long long>, rgrid, dim3(256), 0, stream,
                           a, per_chunk);
      } else {
        hipLaunchKernelGGL(scatter_chunk_reduce_kernel<float>, rgrid, dim3(256), 0, stream, a,
                           per_chunk);
      }
      JKV_CHECK_LAUNCH();
    }
    return JKV_OK;
  }
  // misaligned gradients or d not a multiple of 4: global atomics
  const int64_t n = rows * a.H * a.G * a.d;
  hipLaunchKernelGGL(scatter_global_kernel<DT>, dim3((uint32_t)ceil_div(n, 256)), dim3(256), 0,
                     stream, a);
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

// Many fp16 scatters in one launch (scatter_bins_kernel<F16, D, true>): up to
// kMaxScatterJobs jobs of one geometry, one row chunk each.  Returns
// JKV_ENOTSUP when the geometry or the buffers do not fit that path.
static int launch_scatter_many(const ScatterArgs& shape, const ScatterJobBuffers* buf, int n,
                               bool overwrite, hipStream_t stream) {
  const BinsPlan plan = bins_plan(shape.B, shape.T, shape.H, shape.G, shape.d, shape.S, shape.K, JKV_F16);
  if (!plan.ok || !plan.fixed || shape.n_exits > kMaxScatterJobExits) return JKV_ENOTSUP;
  const uintptr_t align = (uintptr_t)(plan.slice * sizeof(uint16_t));
  for (int j = 0; j < n; ++j)
    for (int e = 0; e < shape.n_exits; ++e)
      if ((uintptr_t)buf[j].grads[e] % align != 0) return JKV_ENOTSUP;
  ScatterManyArgs m = {};
  m.shape = shape;
  m.shape.n_chunks = 1;
  m.shape.rows_per_chunk = shape.B * shape.T;
  m.shape.partials = nullptr;
  m.n_jobs = n;
  m.overwrite = overwrite ? 1 : 0;
  for (int j = 0; j < n; ++j) m.buf[j] = buf[j];
  // 8-dim groups: one block per (job, head, group) takes every stage, so
  // each row's 16-byte slice is read once (the jobs fill the chip without
  // row chunks)
  const bool group8 = shape.d == 8 && shape.S <= 4 && shape.K <= 256 &&
                      shape.B * shape.H * shape.T * shape.G * shape.d < ((int64_t)1 << 31);
  m.per_job = group8 ? shape.H * shape.G : shape.H * shape.G * shape.S * (shape.d / plan.slice);
  int64_t nblocks = m.per_job * n;
  if (nblocks > 8) nblocks = ceil_div(nblocks, 8) * 8;  // xcd_remap needs a multiple of 8
  JKV_CHECK_ARG(nblocks < ((int64_t)1 << 31), "grid too large");
  if (group8) {
    const size_t lds8 = (size_t)(shape.S * shape.K * 9 * 8);
    const dim3 grid((uint32_t)nblocks);
    switch (shape.S) {
      case 1: hipLaunchKernelGGL((scatter_group8_kernel<1, true>), grid, dim3(1024), lds8, stream, m); break;
      case 2: hipLaunchKernelGGL((scatter_group8_kernel<2, true>), grid, dim3(1024), lds8, stream, m); break;
      case 3: hipLaunchKernelGGL((scatter_group8_kernel<3, true>), grid, dim3(1024), lds8, stream, m); break;
      default: hipLaunchKernelGGL((scatter_group8_kernel<4, true>), grid, dim3(1024), lds8, stream, m); break;
    }
    JKV_CHECK_LAUNCH();
    return JKV_OK;
  }
  const size_t lds = (size_t)(shape.K * (plan.slice + 1) * 8);
  if (plan.slice == 8) {
    hipLaunchKernelGGL((scatter_bins_kernel<JKV_F16, 8, true>), dim3((uint32_t)nblocks), dim3(1024), lds, stream, m);
  } else {
    hipLaunchKernelGGL((scatter_bins_kernel<JKV_F16, 4, true>), dim3((uint32_t)nblocks), dim3(1024), lds, stream, m);
  }
  JKV_CHECK_LAUNCH();
  return JKV_OK;
}

__global__ __launch_bounds__(256) void zero_f32_kernel(float* out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = 0.f;
}

}  // namespace jkv

extern "C" {

int64_t jkv_rvq_scatter_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t G, int64_t d,
                                        int64_t S, int64_t K, int32_t grad_dtype,
                                        int32_t deterministic) {
  return jkv::scatter_workspace(B, H, T, G, d, S, K, grad_dtype, deterministic);
}

int jkv_rvq_scatter_grad(int32_t n_exits, const void* const* grads, int32_t grad_dtype,
                         const int32_t* exit_depths, const uint8_t* codes, int64_t code_stride_b,
                         int64_t code_stride_h, int64_t code_stride_t, int64_t B, int64_t H,
                         int64_t T, int64_t G, int64_t d, int64_t S, int64_t K, float* grad_tables,
                         int32_t deterministic, void* workspace, int64_t workspace_bytes,
                         jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(n_exits >= 1 && n_exits <= JKV_MAX_EXITS, "1..%d exits", JKV_MAX_EXITS);
  JKV_CHECK_ARG(B >= 0 && H > 0 && T >= 0 && G > 0 && d > 0 && S > 0 && K > 0 && K <= 256,
                "invalid scatter geometry");
  JKV_CHECK_ARG(grad_dtype == JKV_F16 || grad_dtype == JKV_BF16 || grad_dtype == JKV_F32,
                "unknown gradient dtype %d", grad_dtype);
  if (B * T == 0) return JKV_OK;
  JKV_CHECK_ARG(codes && grad_tables && grads, "null buffer");
  ScatterArgs a = {};
  a.n_exits = n_exits;
  for (int e = 0; e < n_exits; ++e) {
    JKV_CHECK_ARG(grads[e] != nullptr, "null exit gradient");
    JKV_CHECK_ARG(exit_depths[e] >= 1 && exit_depths[e] <= S, "exit depth outside the ladder");
    a.grads[e] = grads[e];
    a.exit_depth[e] = exit_depths[e];
  }
  a.codes = codes;
  a.cb = code_stride_b; a.ch = code_stride_h; a.ct = code_stride_t;
  a.B = B; a.H = H; a.T = T; a.G = G; a.d = d; a.S = S; a.K = K;
  a.grad_tables = grad_tables;
  const int64_t need = scatter_workspace(B, H, T, G, d, S, K, grad_dtype, deterministic);
  if (need > 0) {
    JKV_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                  "scatter needs %lld bytes of workspace", (long long)need);
    a.partials = workspace;
  }
  switch (grad_dtype) {
    case JKV_F16: return launch_scatter<JKV_F16>(a, deterministic, stream);
    case JKV_BF16: return launch_scatter<JKV_BF16>(a, deterministic, stream);
    default: return launch_scatter<JKV_F32>(a, deterministic, stream);
  }
}

int jkv_rvq_scatter_grad_many(int32_t n_jobs, int32_t n_exits, const void* const* grads,
                              int32_t grad_dtype, const int32_t* exit_depths,
                              const uint8_t* const* codes, int64_t code_stride_b,
                              int64_t code_stride_h, int64_t code_stride_t, int64_t B, int64_t H,
                              int64_t T, int64_t G, int64_t d, int64_t S, int64_t K,
                              float* const* grad_tables, int32_t accumulate, int32_t deterministic,
                              void* workspace, int64_t workspace_bytes, jkv_stream_t stream_) {
  using namespace jkv;
  hipStream_t stream = (hipStream_t)stream_;
  JKV_CHECK_ARG(n_jobs >= 0, "negative job count");
  JKV_CHECK_ARG(n_exits >= 1 && n_exits <= JKV_MAX_EXITS, "1..%d exits", JKV_MAX_EXITS);
  JKV_CHECK_ARG(B >= 0 && H > 0 && T >= 0 && G > 0 && d > 0 && S > 0 && K > 0 && K <= 256,
                "invalid scatter geometry");
  JKV_CHECK_ARG(grad_dtype == JKV_F16 || grad_dtype == JKV_BF16 || grad_dtype == JKV_F32,
                "unknown gradient dtype %d", grad_dtype);
  if (n_jobs == 0) return JKV_OK;
  JKV_CHECK_ARG(grads && codes && grad_tables && exit_depths, "null job array");
  for (int32_t j = 0; j < n_jobs; ++j) {
    JKV_CHECK_ARG(codes[j] && grad_tables[j], "null buffer in job %d", j);
    for (int e = 0; e < n_exits; ++e)
      JKV_CHECK_ARG(grads[(int64_t)j * n_exits + e] != nullptr, "null exit gradient in job %d", j);
  }
  for (int e = 0; e < n_exits; ++e)
    JKV_CHECK_ARG(exit_depths[e] >= 1 && exit_depths[e] <= S, "exit depth outside the ladder");
  const int64_t table_elems = H * G * S * K * d;
  if (B * T == 0) {
    if (!accumulate)
      for (int32_t j = 0; j < n_jobs; ++j) {
        hipLaunchKernelGGL(zero_f32_kernel, dim3((uint32_t)ceil_div(table_elems, 256)), dim3(256), 0, stream,
                           grad_tables[j], table_elems);
        JKV_CHECK_LAUNCH();
      }
    return JKV_OK;
  }
  // fp16 gradients: up to kMaxScatterJobs jobs per launch; jobs that path
  // does not take (other dtypes, more exits, misaligned gradients) run one
  // scatter each
  int32_t first_single = 0;
  if (grad_dtype == JKV_F16 && n_exits <= kMaxScatterJobExits) {
    ScatterArgs shape = {};
    shape.n_exits = n_exits;
    for (int e = 0; e < n_exits; ++e) shape.exit_depth[e] = exit_depths[e];
    shape.cb = code_stride_b; shape.ch = code_stride_h; shape.ct = code_stride_t;
    shape.B = B; shape.H = H; shape.T = T; shape.G = G; shape.d = d; shape.S = S; shape.K = K;
    ScatterJobBuffers buf[kMaxScatterJobs];
    for (int32_t j0 = 0; j0 < n_jobs; j0 += kMaxScatterJobs) {
      const int n = (int)std::min<int64_t>(kMaxScatterJobs, n_jobs - j0);
      for (int i = 0; i < n; ++i) {
        const int64_t j = j0 + i;
        buf[i] = ScatterJobBuffers{};
        for (int e = 0; e < n_exits; ++e) buf[i].grads[e] = grads[j * n_exits + e];
        buf[i].codes = codes[j];
        buf[i].grad_tables = grad_tables[j];
      }
      const int rc = launch_scatter_many(shape, buf, n, !accumulate, stream);
      if (rc == JKV_ENOTSUP) break;
      if (rc != JKV_OK) return rc;
      first_single = j0 + n;
    }
  }
  for (int32_t j = first_single; j < n_jobs; ++j) {
    if (!accumulate) {
      hipLaunchKernelGGL(zero_f32_kernel, dim3((uint32_t)ceil_div(table_elems, 256)), dim3(256), 0, stream,
                         grad_tables[j], table_elems);
      JKV_CHECK_LAUNCH();
    }
    const int rc = jkv_rvq_scatter_grad(n_exits, grads + (int64_t)j * n_exits, grad_dtype, exit_depths, codes[j],
                                        code_stride_b, code_stride_h, code_stride_t, B, H, T, G, d, S, K,
                                        grad_tables[j], deterministic, workspace, workspace_bytes, stream_);
    if (rc != JKV_OK) return rc;
  }
  return JKV_OK;
}

}  // extern "C"
