// Device-side building blocks shared by the gfx950 W4A16 kernels.
//
// Storage format (reference w4a16-kernel/src/w4a16/quant.py:1-30, W4A16_SPEC.md:109-171):
//   qweight int32 [K/8, N]: word (i, n) holds codes for rows k = 8i + j, j = 0..7,
//                           code j in bits [4j, 4j+4), unsigned.
//   scales  fp16  [K/G, N], zeros fp16 [K/G, N] (integer zero-points).
//   W_dq[k, n] = fp16((fp16(q) - z) * s)  (quant.py:173-177).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a16 {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f16x2 as_h2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }
__device__ __forceinline__ uint32_t as_u32(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ f16 as_h(uint16_t u) { return __builtin_bit_cast(f16, u); }
__device__ __forceinline__ uint16_t as_u16(f16 h) { return __builtin_bit_cast(uint16_t, h); }

// Per-column dequant constants for one quantisation group.
//   s  = (scale, scale)
//   z0 = (1024 + zero, 1024 + zero)   pairs built from nibbles at bits [0,4) of a half
//   z1 = (  64 + zero,   64 + zero)   pairs built from nibbles at bits [4,8) of a half
// OR-ing a nibble q into the mantissa of fp16 1024 (0x6400) gives exactly 1024 + q;
// OR-ing q << 4 into fp16 64 (0x5400) gives exactly 64 + q.  Subtracting 1024 + z
// (or 64 + z) is then exact for integer zero-points in [-63, 63], so
// (p - z0) * s == fp16(q - z) * s with a single RNE rounding, as in the reference.
struct ColQ {
  f16x2 s, z0, z1;
};

__device__ __forceinline__ ColQ make_colq(uint16_t sbits, uint16_t zbits) {
  const f16 s = as_h(sbits), z = as_h(zbits);
  const f16 a = (f16)1024.0f + z;
  const f16 b = (f16)64.0f + z;
  ColQ c;
  c.s = f16x2{s, s};
  c.z0 = f16x2{a, a};
  c.z1 = f16x2{b, b};
  return c;
}

// Dequantise one packed word into four fp16 pairs in "pair order":
//   d[0] = (w0, w4), d[1] = (w1, w5), d[2] = (w2, w6), d[3] = (w3, w7)
// where w_j is the weight of row 8i + j.  Consumers permute the activations the
// same way, so the dot products see matching k.
__device__ __forceinline__ void dq_word(uint32_t w, const ColQ& c, f16x2 d[4]) {
  const uint32_t t = w >> 8;
  const uint32_t p0 = (w & 0x000F000Fu) | 0x64006400u;
  const uint32_t p1 = (w & 0x00F000F0u) | 0x54005400u;
  const uint32_t p2 = (t & 0x000F000Fu) | 0x64006400u;
  const uint32_t p3 = (t & 0x00F000F0u) | 0x54005400u;
  d[0] = (as_h2(p0) - c.z0) * c.s;
  d[1] = (as_h2(p1) - c.z1) * c.s;
  d[2] = (as_h2(p2) - c.z0) * c.s;
  d[3] = (as_h2(p3) - c.z1) * c.s;
}

// Permute eight consecutive fp16 activations x0..x7 (four dwords, natural order)
// into pair order (x0,x4) (x1,x5) (x2,x6) (x3,x7).
__device__ __forceinline__ uint4 perm_pairs(uint4 v) {
  uint4 r;
  r.x = (v.x & 0xFFFFu) | (v.z << 16);
  r.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
  r.z = (v.y & 0xFFFFu) | (v.w << 16);
  r.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
  return r;
}

__device__ __forceinline__ f16 f32_to_f16(float x) { return (f16)x; }  // v_cvt_f16_f32, RNE

}  // namespace w4a16
