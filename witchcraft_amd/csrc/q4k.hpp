// q4k.hpp -- Q4_K nibble unpacking shared by the GEMM and GEMV kernels.
//
// GGML Q4_K super-block (256 values, 144 bytes): f16 d, f16 dmin, 12 bytes of packed 6-bit
// (scale, min) pairs for 8 sub-blocks of 32, 128 bytes of nibbles.  Chunk c (values
// 64c..64c+63) = sub-block 2c (low nibbles of qs[32c..32c+31]) and sub-block 2c+1 (high
// nibbles of the same bytes).  value = (d * sc) * q - dmin * m; both products are exact in
// f32, so one fused multiply-add gives the bit-exact f32 value, rounded once to f16 here.
#pragma once
#include "common.hpp"

namespace {

__device__ __forceinline__ int sbyte(const uint4& hd, int i) {
  // byte i (0..11) of the 12 packed scale bytes = header bytes 4..15
  const uint32_t w = i < 4 ? hd.y : (i < 8 ? hd.z : hd.w);
  return (int)((w >> (8 * (i & 3))) & 0xff);
}

// GGML get_scale_min_k4 for the sub-block pair (2c, 2c+1); c is wave-uniform.
__device__ __forceinline__ void chunk_scales(const uint4& hd, int c, float& s0, float& o0, float& s1,
                                             float& o1) {
  const float d = f16_bits_to_f32(hd.x & 0xffff), dmin = f16_bits_to_f32(hd.x >> 16);
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

// Byte i of v as f32 (v_cvt_f32_ubyte{0..3}: extraction and conversion in one instruction).
template <int I>
__device__ __forceinline__ float ubyte(uint32_t v) {
  float r;
  if constexpr (I == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
  else if constexpr (I == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
  else if constexpr (I == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
  return r;
}

// 4 packed bytes (8 nibbles) -> 4 low-nibble (sub-block 2c) and 4 high-nibble (2c+1) f16:
// mask the nibbles into byte lanes once, convert each byte with one instruction, then one
// fused multiply-add per value rounded once to f16.
__device__ __forceinline__ void deq4(uint32_t v, float s0, float o0, float s1, float o1, h4& lo, h4& hi) {
  const uint32_t l = v & 0x0f0f0f0fu, h = (v >> 4) & 0x0f0f0f0fu;
  lo = h4{(_Float16)__builtin_fmaf(s0, ubyte<0>(l), -o0), (_Float16)__builtin_fmaf(s0, ubyte<1>(l), -o0),
          (_Float16)__builtin_fmaf(s0, ubyte<2>(l), -o0), (_Float16)__builtin_fmaf(s0, ubyte<3>(l), -o0)};
  hi = h4{(_Float16)__builtin_fmaf(s1, ubyte<0>(h), -o1), (_Float16)__builtin_fmaf(s1, ubyte<1>(h), -o1),
          (_Float16)__builtin_fmaf(s1, ubyte<2>(h), -o1), (_Float16)__builtin_fmaf(s1, ubyte<3>(h), -o1)};
}

}  // namespace
