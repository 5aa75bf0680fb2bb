// fp16 rotary embedding with the arithmetic of the reference's model code
// (HF transformers apply_rotary_pos_emb on fp16 tensors).
#pragma once

#include "jkv_common.h"

namespace jkv {

// (x * cos) + (rotate_half(x) * sin) in fp16, every operation rounded to
// fp16 (no contraction).  a = dims [i, i+8) of the first half of the head,
// b = the partner dims [i+64, i+72); c, s = cos/sin of those 8 frequencies.
#pragma clang fp contract(off)
__device__ __forceinline__ void rope16(half8 a, half8 b, half8 c, half8 s, half8* ra, half8* rb) {
  const half8 ac = a * c;
  const half8 bs = b * s;
  const half8 bc = b * c;
  const half8 as = a * s;
  *ra = sub_h8(ac, bs);
  *rb = bc + as;
}
#pragma clang fp contract(on)

// Rotary table row of one position: [2][64] fp16, cos of the 64 frequencies
// then their sin.
static const int kRopeRow = 128;

// cos/sin of 8 consecutive frequencies starting at i0 of one table row.
__device__ __forceinline__ void load_trig8(const _Float16* row, int i0, half8* c, half8* s) {
  *c = *(const half8*)(row + i0);
  *s = *(const half8*)(row + 64 + i0);
}

}  // namespace jkv
