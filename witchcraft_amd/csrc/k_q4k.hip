// k_q4k.hip -- bit-exact Q4_K -> f32 dequantization (candle BlockQ4K::to_float semantics).
//
// Reference call sites: src/quantized_t5.rs:44 (CPU default: every weight dequantized at
// load), :60, :154, :326-334.  Per sub-block j the value is (d*sc_j)*q - (dmin*m_j); both
// products are exact in f32, so the one rounding is the final subtraction and the result
// is independent of evaluation order (FMA included).
#include "common.hpp"

namespace {

__device__ __forceinline__ void scale_min(const uint8_t* s, int j, int& sc, int& m) {
  if (j < 4) {
    sc = s[j] & 63;
    m = s[j + 4] & 63;
  } else {
    sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

// One wavefront per 144-byte block; lane l covers bytes 2(l%16), 2(l%16)+1 of chunk l/16
// and writes their low-nibble values (sub-block 2c) and high-nibble values (2c+1).
__global__ __launch_bounds__(256) void q4k_dequant_f32_kernel(const uint8_t* __restrict__ blocks,
                                                              size_t nblk, float* __restrict__ out) {
  const size_t blk = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= nblk) return;
  const int lane = threadIdx.x & 63;
  const uint8_t* b = blocks + blk * Q4K_BYTES;
  const uint16_t dh = (uint16_t)b[0] | ((uint16_t)b[1] << 8);
  const uint16_t mh = (uint16_t)b[2] | ((uint16_t)b[3] << 8);
  const float d = f16_bits_to_f32(dh), dmin = f16_bits_to_f32(mh);
  const int c = lane >> 4, i0 = (lane & 15) * 2;
  int sc0, m0, sc1, m1;
  scale_min(b + 4, 2 * c, sc0, m0);
  scale_min(b + 4, 2 * c + 1, sc1, m1);
  const float d0 = d * (float)sc0, mm0 = dmin * (float)m0;
  const float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
  const uint8_t q0 = b[16 + 32 * c + i0], q1 = b[16 + 32 * c + i0 + 1];
  float* y = out + blk * QK_K + 64 * c;
  float2 lo, hi;
  lo.x = d0 * (float)(q0 & 15) - mm0;
  lo.y = d0 * (float)(q1 & 15) - mm0;
  hi.x = d1 * (float)(q0 >> 4) - mm1;
  hi.y = d1 * (float)(q1 >> 4) - mm1;
  *reinterpret_cast<float2*>(y + i0) = lo;
  *reinterpret_cast<float2*>(y + 32 + i0) = hi;
}

// The hybrid-dequant + fbgemm build's dense weights (src/quantized_t5.rs:57-62 dequantizes them
// to f32 at load, fbgemm-rs/src/bf16.rs:21-25 truncates them to bf16) as the f16 operand of the
// dense GEMMs: the exact f32 value above, its low 16 bits cleared, converted to f16 (exact for
// |w| >= 2^-17, where 8 significant bits fit f16; rounded to the f16 subnormal grid below).
// Same block/lane mapping as q4k_dequant_f32_kernel; out is [nblk * 256] f16 in block order.
__device__ __forceinline__ _Float16 bf16_trunc_f16(float v) {
  return (_Float16)__uint_as_float(__float_as_uint(v) & 0xffff0000u);
}

__global__ __launch_bounds__(256) void q4k_dequant_bf16_f16_kernel(const uint8_t* __restrict__ blocks,
                                                                   size_t nblk, _Float16* __restrict__ out) {
  const size_t blk = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= nblk) return;
  const int lane = threadIdx.x & 63;
  const uint8_t* b = blocks + blk * Q4K_BYTES;
  const uint16_t dh = (uint16_t)b[0] | ((uint16_t)b[1] << 8);
  const uint16_t mh = (uint16_t)b[2] | ((uint16_t)b[3] << 8);
  const float d = f16_bits_to_f32(dh), dmin = f16_bits_to_f32(mh);
  const int c = lane >> 4, i0 = (lane & 15) * 2;
  int sc0, m0, sc1, m1;
  scale_min(b + 4, 2 * c, sc0, m0);
  scale_min(b + 4, 2 * c + 1, sc1, m1);
  const float d0 = d * (float)sc0, mm0 = dmin * (float)m0;
  const float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
  const uint8_t q0 = b[16 + 32 * c + i0], q1 = b[16 + 32 * c + i0 + 1];
  _Float16* y = out + blk * QK_K + 64 * c;
  y[i0] = bf16_trunc_f16(d0 * (float)(q0 & 15) - mm0);
  y[i0 + 1] = bf16_trunc_f16(d0 * (float)(q1 & 15) - mm0);
  y[32 + i0] = bf16_trunc_f16(d1 * (float)(q0 >> 4) - mm1);
  y[32 + i0 + 1] = bf16_trunc_f16(d1 * (float)(q1 >> 4) - mm1);
}

}  // namespace

namespace t5k {
hipError_t launch_q4k_dequant(const void* blocks, size_t nblk, float* out, hipStream_t s) {
  if (nblk == 0) return hipSuccess;
  const size_t grid = (nblk + 3) / 4;
  hipLaunchKernelGGL(q4k_dequant_f32_kernel, dim3((unsigned)grid), dim3(256), 0, s,
                     (const uint8_t*)blocks, nblk, out);
  return hipGetLastError();
}

hipError_t launch_q4k_dequant_bf16_f16(const void* blocks, size_t nblk, _Float16* out, hipStream_t s) {
  if (nblk == 0) return hipSuccess;
  const size_t grid = (nblk + 3) / 4;
  hipLaunchKernelGGL(q4k_dequant_bf16_f16_kernel, dim3((unsigned)grid), dim3(256), 0, s,
                     (const uint8_t*)blocks, nblk, out);
  return hipGetLastError();
}
}  // namespace t5k
