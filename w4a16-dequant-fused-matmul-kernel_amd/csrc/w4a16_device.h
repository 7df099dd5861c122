// Device-side building blocks shared by the gfx950 W4A16 kernels.
//
// Storage format (reference w4a16-kernel/src/w4a16/quant.py:1-30, W4A16_SPEC.md:109-171):
//   qweight int32 [K/8, N]: word (i, n) holds codes for rows k = 8i + j, j = 0..7,
//                           code j in bits [4j, 4j+4), unsigned.
//   scales  fp16  [K/G, N], zeros fp16 [K/G, N].
//   W_dq[k, n] = fp16(fp16(fp16(q) - z) * s)  (quant.py:173-177).
//
// Zero-points.  The fused kernels are instantiated twice over a template flag
// AZ ("any zero"):
//   AZ = false: every zero is an integer with |z| <= 1024 (quantize_weight
//     makes 0..15).  Then 1024 + z and 64 + z are fp16 numbers, so one
//     subtract of the magic-biased zero from the magic-biased code gives q - z
//     exactly and one multiply rounds once, as the reference's two roundings
//     do when q - z is exact.
//   AZ = true: any fp16 zero.  The magic is subtracted first (exact: the code
//     q as fp16), then z with the reference's own RNE rounding of fp16(q) - z,
//     then the multiply: one more packed subtract per pair of weights.
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
//   (AZ: z0 = z1 = (zero, zero))
// OR-ing a nibble q into the mantissa of fp16 1024 (0x6400) gives exactly 1024 + q;
// OR-ing q << 4 into fp16 64 (0x5400) gives exactly 64 + q.  Subtracting 1024 + z
// (or 64 + z) is then exact for integer zero-points with |z| <= 1024, so
// (p - z0) * s == fp16(q - z) * s with a single RNE rounding, as in the reference.
struct ColQ {
  f16x2 s, z0, z1;
};

template <bool AZ = false>
__device__ __forceinline__ ColQ make_colq(uint16_t sbits, uint16_t zbits) {
  const f16 s = as_h(sbits), z = as_h(zbits);
  const f16 a = AZ ? z : (f16)1024.0f + z;
  const f16 b = AZ ? z : (f16)64.0f + z;
  ColQ c;
  c.s = f16x2{s, s};
  c.z0 = f16x2{a, a};
  c.z1 = f16x2{b, b};
  return c;
}

// Two columns' scale/zero state, packed: lane c of each pair is column c.
// Used through colq_of<c>(), whose broadcasts fold into the packed ops' op_sel.
struct ColQ2 {
  f16x2 s, za, zb;   // scales, 1024 + zeros, 64 + zeros (AZ: zeros, zeros)
};

template <bool AZ = false>
__device__ __forceinline__ ColQ2 make_colq2(uint32_t sbits2, uint32_t zbits2) {
  const f16x2 z = as_h2(zbits2);
  ColQ2 q;
  q.s = as_h2(sbits2);
  if constexpr (AZ) {
    q.za = z;
    q.zb = z;
  } else {
    q.za = z + f16x2{(f16)1024.0f, (f16)1024.0f};
    q.zb = z + f16x2{(f16)64.0f, (f16)64.0f};
  }
  return q;
}

template <int C>
__device__ __forceinline__ ColQ colq_of(const ColQ2& q) {
  ColQ c;
  c.s = __builtin_shufflevector(q.s, q.s, C, C);
  c.z0 = __builtin_shufflevector(q.za, q.za, C, C);
  c.z1 = __builtin_shufflevector(q.zb, q.zb, C, C);
  return c;
}

// (w & mask) | magic in one v_and_or_b32.  gfx9 VOP3 encodings take no literal
// constants and read at most one SGPR, so the mask rides in an SGPR and the
// magic in a VGPR that the caller materialises once (MagicRegs).
__device__ __forceinline__ uint32_t and_or(uint32_t w, uint32_t mask, uint32_t magic_vgpr) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(w), "s"(mask), "v"(magic_vgpr));
  return r;
}

// The two magic words in VGPRs.  Loaded through an opaque move so the compiler
// keeps them live instead of re-materialising a constant for every use.
struct MagicRegs {
  uint32_t m1024, m64;
};
__device__ __forceinline__ MagicRegs make_magic() {
  MagicRegs m;
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(m.m1024));
  asm volatile("v_mov_b32 %0, 0x54005400" : "=v"(m.m64));
  return m;
}

// Dequantise one packed word into four fp16 pairs in "pair order":
//   d[0] = (w0, w4), d[1] = (w1, w5), d[2] = (w2, w6), d[3] = (w3, w7)
// where w_j is the weight of row 8i + j.  Consumers permute the activations the
// same way, so the dot products see matching k.  The unpack takes five
// instructions (one shift, four v_and_or_b32); the magic words are also the
// fp16 pairs (1024, 1024) and (64, 64) that AZ subtracts first.
template <bool AZ = false>
__device__ __forceinline__ void dq_word_fast(uint32_t w, const ColQ& c, const MagicRegs& mg,
                                             f16x2 d[4]) {
  const uint32_t t = w >> 8;
  if constexpr (AZ) {
    const f16x2 a = as_h2(mg.m1024), b = as_h2(mg.m64);
    d[0] = ((as_h2(and_or(w, 0x000F000Fu, mg.m1024)) - a) - c.z0) * c.s;
    d[1] = ((as_h2(and_or(w, 0x00F000F0u, mg.m64)) - b) - c.z1) * c.s;
    d[2] = ((as_h2(and_or(t, 0x000F000Fu, mg.m1024)) - a) - c.z0) * c.s;
    d[3] = ((as_h2(and_or(t, 0x00F000F0u, mg.m64)) - b) - c.z1) * c.s;
  } else {
    d[0] = (as_h2(and_or(w, 0x000F000Fu, mg.m1024)) - c.z0) * c.s;
    d[1] = (as_h2(and_or(w, 0x00F000F0u, mg.m64)) - c.z1) * c.s;
    d[2] = (as_h2(and_or(t, 0x000F000Fu, mg.m1024)) - c.z0) * c.s;
    d[3] = (as_h2(and_or(t, 0x00F000F0u, mg.m64)) - c.z1) * c.s;
  }
}

// Permute eight consecutive fp16 activations x0..x7 (four dwords, natural order)
// into pair order (x0,x4) (x1,x5) (x2,x6) (x3,x7).
__device__ __forceinline__ uint4 perm_pairs(uint4 v) {
  // each output dword takes two 16-bit halves of two input dwords: one
  // v_perm_b32 each (selector bytes index {v.z, v.x} / {v.w, v.y} as 7..0)
  uint4 r;
  r.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);   // x.lo, z.lo
  r.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);   // x.hi, z.hi
  r.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);   // y.lo, w.lo
  r.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);   // y.hi, w.hi
  return r;
}

// v <- v from lane (l - N) mod 16 of the same 16-lane DPP row (row_ror:N).
template <int kN>
__device__ __forceinline__ float dpp_row_ror(float v) {
  static_assert(kN >= 1 && kN <= 15, "row rotation is 1..15 lanes");
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x120 + kN, 0xF, 0xF, false));
}

// Row exchanges between two registers (16-lane rows r0..r3 of a wave):
// v_permlane16_swap swaps the odd rows of `a` with the even rows of `b`,
// v_permlane32_swap the upper 32 lanes of `a` with the lower 32 lanes of `b`.
// Inline asm: the compiler's builtins for these instructions hand back the
// first register for both results.  The s_nops give the VALU -> permlane and
// permlane -> DPP wait states the compiler cannot see through the asm.
__device__ __forceinline__ void permlane16_swap(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane32_swap(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

// Transpose-reduce of four values over the four 16-lane rows: on return, row c
// of the result holds v_c summed over the rows, (r0 + r1) + (r2 + r3), at the
// same position within the row.
//   swap16(v0, v1), swap16(v2, v3); s01 = v0 + v1, s23 = v2 + v3:
//     s01 rows = (v0 r0+r1, v1 r0+r1, v0 r2+r3, v1 r2+r3), s23 likewise;
//   swap32(s01, s23); s01 + s23: row c = v_c (r0+r1) + v_c (r2+r3).
__device__ __forceinline__ float fold_rows4(float v0, float v1, float v2, float v3) {
  permlane16_swap(v0, v1);
  permlane16_swap(v2, v3);
  float s01 = v0 + v1, s23 = v2 + v3;
  permlane32_swap(s01, s23);
  return s01 + s23;
}

// k / G for 0 <= k < 2^31 from the host's group_div(G) constants.
__device__ __forceinline__ uint32_t div_group(uint32_t k, uint32_t magic, int shift) {
  return (__umulhi(k, magic) + k) >> shift;
}

__device__ __forceinline__ f16 f32_to_f16(float x) { return (f16)x; }  // v_cvt_f16_f32, RNE

// Buffer resource over [p, p + bytes): raw buffer loads outside the range return
// zero (gfx9-family descriptor word 3 = 0x00020000).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
// Byte offset that no buffer range contains: loads from it return zero.
constexpr uint32_t kOobOffset = 0x80000000u;

// LDS destination of the buffer loads' LDS-direct form (address space 3).
typedef __attribute__((address_space(3))) void lds_void;

// Wave-uniform value promised to the compiler (keeps buffer SGPR offsets scalar).
__device__ __forceinline__ uint32_t uniform(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// `soff` must be wave-uniform (it is an SGPR operand).
template <int kPolicy = 0>
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  typedef int v4i __attribute__((ext_vector_type(4)));
  const v4i v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, kPolicy);
  return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}
__device__ __forceinline__ uint2 buf_load8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  typedef int v2i __attribute__((ext_vector_type(2)));
  const v2i v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0);
  return make_uint2((uint32_t)v.x, (uint32_t)v.y);
}

}  // namespace w4a16
