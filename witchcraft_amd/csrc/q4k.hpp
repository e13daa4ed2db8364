// q4k.hpp -- Q4_K nibble unpacking shared by the GEMM and GEMV kernels.
//
// GGML Q4_K super-block (256 values, 144 bytes): f16 d, f16 dmin, 12 bytes of packed 6-bit
// (scale, min) pairs for 8 sub-blocks of 32, 128 bytes of nibbles.  Chunk c (values
// 64c..64c+63) = sub-block 2c (low nibbles of qs[32c..32c+31]) and sub-block 2c+1 (high
// nibbles of the same bytes).  value = (d * sc) * q - dmin * m; both products are exact in
// f32, so one fused multiply-add gives the bit-exact f32 value, rounded once to f16 here.
//
// Nibble -> float: a byte holding a nibble q (0..15) reads as OCP fp8 e4m3 q * 2^-9 exactly
// (codes 0-7 are the subnormals m * 2^-9, codes 8-15 are (8 + m) * 2^-9), so
// v_cvt_pk_f32_fp8 converts two nibbles per instruction; the sub-block scale carries the
// compensating 2^9 (exact: a power of two), leaving (d*sc)*q - dmin*m and its single rounding
// unchanged.
#pragma once
#include "common.hpp"

namespace {

__device__ __forceinline__ int sbyte(const uint4& hd, int i) {
  // byte i (0..11) of the 12 packed scale bytes = header bytes 4..15
  const uint32_t w = i < 4 ? hd.y : (i < 8 ? hd.z : hd.w);
  return (int)((w >> (8 * (i & 3))) & 0xff);
}

// GGML get_scale_min_k4 for the sub-block pair (2c, 2c+1); c is wave-uniform.  Returns the
// scales times 2^9 (s0 = d*sc0*512, ...) for deq4's fp8 reading of the nibbles, and the mins
// dmin*m unscaled.
__device__ __forceinline__ void chunk_scales(const uint4& hd, int c, float& s0, float& o0, float& s1,
                                             float& o1) {
  const float d = f16_bits_to_f32(hd.x & 0xffff) * 512.0f, dmin = f16_bits_to_f32(hd.x >> 16);
  int sc0, m0, sc1, m1;
  const int j0 = 2 * c, j1 = 2 * c + 1;
  if (c < 2) {
    sc0 = sbyte(hd, j0) & 63;
    m0 = sbyte(hd, j0 + 4) & 63;
    sc1 = sbyte(hd, j1) & 63;
    m1 = sbyte(hd, j1 + 4) & 63;
  } else {
    sc0 = (sbyte(hd, j0 + 4) & 15) | ((sbyte(hd, j0 - 4) >> 6) << 4);
    m0 = (sbyte(hd, j0 + 4) >> 4) | ((sbyte(hd, j0) >> 6) << 4);
    sc1 = (sbyte(hd, j1 + 4) & 15) | ((sbyte(hd, j1 - 4) >> 6) << 4);
    m1 = (sbyte(hd, j1 + 4) >> 4) | ((sbyte(hd, j1) >> 6) << 4);
  }
  s0 = d * (float)sc0;
  o0 = dmin * (float)m0;
  s1 = d * (float)sc1;
  o1 = dmin * (float)m1;
}

// 4 packed bytes (8 nibbles) -> 4 low-nibble (sub-block 2c) and 4 high-nibble (2c+1) f16:
// mask the nibbles into byte lanes once, convert two bytes per instruction (fp8 reading,
// q * 2^-9), then one fused multiply-add per value with the 2^9-scaled scale (s0, s1 from
// chunk_scales), rounded once to f16.
__device__ __forceinline__ void deq4(uint32_t v, float s0, float o0, float s1, float o1, h4& lo, h4& hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  const uint32_t l = v & 0x0f0f0f0fu, h = (v >> 4) & 0x0f0f0f0fu;
  const f2 l01 = __builtin_amdgcn_cvt_pk_f32_fp8(l, false), l23 = __builtin_amdgcn_cvt_pk_f32_fp8(l, true);
  const f2 h01 = __builtin_amdgcn_cvt_pk_f32_fp8(h, false), h23 = __builtin_amdgcn_cvt_pk_f32_fp8(h, true);
  lo = h4{(_Float16)__builtin_fmaf(s0, l01[0], -o0), (_Float16)__builtin_fmaf(s0, l01[1], -o0),
          (_Float16)__builtin_fmaf(s0, l23[0], -o0), (_Float16)__builtin_fmaf(s0, l23[1], -o0)};
  hi = h4{(_Float16)__builtin_fmaf(s1, h01[0], -o1), (_Float16)__builtin_fmaf(s1, h01[1], -o1),
          (_Float16)__builtin_fmaf(s1, h23[0], -o1), (_Float16)__builtin_fmaf(s1, h23[1], -o1)};
}

}  // namespace
