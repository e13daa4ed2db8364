// k_q8k.hip -- the reference's hybrid-dequant FFN numerics: f32 activations quantized to GGML
// Q8_K blocks, for Q4_K x Q8_K integer dot products on the matrix cores (launch_gemm_hybrid in
// k_gemm.hip).
//
// Reference: with the `hybrid-dequant` feature (src/quantized_t5.rs:18-21,233-244) the gated
// FFN's wi_0 / wi_1 run through fused_gated_gelu_inner (src/fused_matmul.rs:138-177) and the
// final projection through QTiledOp (tiled_matmul_inner, :27-59).  Both quantize every f32
// activation row with candle's BlockQ8K::from_float and take GGML's Q4_K x Q8_K vec_dot per
// (row, token); the gate goes through a Pade tanh gelu (:128-133,168-170).  This is the
// numerics of the reference's x86 default build.
//
//  * q8k_quantize_kernel: one wave per token, four tokens per workgroup (D <= 1024).
//    Optional T5LayerNorm first (x / sqrt(mean(x^2) + eps) * w in f32, src/quantized_t5.rs:
//    162-173).  Q8_K: the value of largest magnitude (the first one on ties) sets
//    iscale = -128 / v, q = min(127, round(iscale * x)) with halves away from zero, d = 1 / iscale,
//    bsums = sums of 16 consecutive q; an all-zero block gives d = 0 and q = 0.  Bit-exact with
//    BlockQ8K::from_float on the same f32 input.  Writes the Q8_K blocks and/or the operands of
//    the matrix-core product: q as the int8 operand of v_mfma_i32_16x16x64_i8, d per block, and
//    the bsums as the B operand of the min-term MFMA.
//  * q8k_operands_kernel: Q8_K blocks -> the same operands (the standalone matmul entry point).
#include "common.hpp"

#pragma clang fp contract(off)

namespace {

constexpr int Q8K_BYTES = 292;  // {f32 d, i8 qs[256], i16 bsums[16]}

// wave64 arg-max of |v| with the smallest index on ties; every lane gets the winner's value.
__device__ __forceinline__ void wave_absmax_first(float& a, int& idx, float& v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float oa = __shfl_xor(a, o);
    const int oi = __shfl_xor(idx, o);
    const float ov = __shfl_xor(v, o);
    if (oa > a || (oa == a && oi < idx)) {
      a = oa;
      idx = oi;
      v = ov;
    }
  }
}

// The matrix-core operands of one lane's four values q[0..3] (values 4 lane .. 4 lane + 3 of block
// b of token t), the block scale d (lane 0) and the 16-value group sum s of lane 4g (the bsum of
// group g = lane / 4): q into the int8 operand xq (4 bytes; blocks of 16 tokens x 64 K, lane l of
// a block holding token l % 16, K 16 (l / 16) .. +15), d into d8, bsum g into its slot of the
// (t / 16, b) bsum operand block, and lanes 4g + 1 zero the slot of lane group 2 + g / 8 (K slots
// 16..31 of the min-term MFMA, which have no bsum).
__device__ __forceinline__ void q8k_store_operands(const int (&q)[4], float d, int s, int t, int b, int nb, int D,
                                                   int lane, int8_t* xq, float* d8, _Float16* bsop) {
  const int k = 256 * b + 4 * lane;
  const uint32_t packed = (uint32_t)(q[0] & 255) | ((uint32_t)(q[1] & 255) << 8) | ((uint32_t)(q[2] & 255) << 16) |
                          ((uint32_t)(q[3] & 255) << 24);
  *reinterpret_cast<uint32_t*>(xq + ((size_t)(t >> 4) * (D / 64) + (k >> 6)) * 1024 +
                               (((k & 63) >> 4) * 16 + (t & 15)) * 16 + (k & 15)) = packed;
  if (lane == 0) d8[(size_t)t * nb + b] = d;
  const int g = lane >> 2;
  _Float16* blk = bsop + ((size_t)(t >> 4) * nb + b) * 512;
  if ((lane & 3) == 0) blk[((g >> 3) * 16 + (t & 15)) * 8 + (g & 7)] = (_Float16)s;
  if ((lane & 3) == 1) blk[((2 + (g >> 3)) * 16 + (t & 15)) * 8 + (g & 7)] = (_Float16)0.f;
}

// One wave per token (four tokens per workgroup), all of the token's blocks in registers: lane l
// holds values 4 l .. 4 l + 3 of every block, so the norm's and each block's reductions are wave
// shuffles only.  The norm's sum of squares is added in the order of the one-wave-per-block form
// (per block: lane pairs, then lanes by xor; then blocks (0 + 1) + (2 + 3)).
__global__ __launch_bounds__(256) void q8k_quantize_kernel(const float* __restrict__ x, const float* __restrict__ gamma,
                                                           float eps, int T, int D, uint8_t* __restrict__ out,
                                                           int8_t* __restrict__ xq, float* __restrict__ d8,
                                                           _Float16* __restrict__ bsop) {
  const int lane = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int nb = D / 256;
  float v[4][4];
#pragma unroll
  for (int b = 0; b < 4; b++) {
    float4 u = make_float4(0.f, 0.f, 0.f, 0.f);
    if (b < nb) u = *reinterpret_cast<const float4*>(x + (size_t)t * D + 256 * b + 4 * lane);
    v[b][0] = u.x, v[b][1] = u.y, v[b][2] = u.z, v[b][3] = u.w;
  }
  if (gamma) {  // T5LayerNorm in f32
    float part[4];
#pragma unroll
    for (int b = 0; b < 4; b++) {
      float ss = (v[b][0] * v[b][0] + v[b][1] * v[b][1]) + (v[b][2] * v[b][2] + v[b][3] * v[b][3]);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
      part[b] = ss;
    }
    const float tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float den = sqrtf(tot / (float)D + eps);
#pragma unroll
    for (int b = 0; b < 4; b++)
      if (b < nb) {
        const float4 g = *reinterpret_cast<const float4*>(gamma + 256 * b + 4 * lane);
        v[b][0] = (v[b][0] / den) * g.x;
        v[b][1] = (v[b][1] / den) * g.y;
        v[b][2] = (v[b][2] / den) * g.z;
        v[b][3] = (v[b][3] / den) * g.w;
      }
  }
#pragma unroll
  for (int b = 0; b < 4; b++) {
    if (b >= nb) break;
    // largest magnitude, first index on ties (the block's values in index order 4 * lane + i)
    float a = fabsf(v[b][0]), mv = v[b][0];
    int idx = 4 * lane;
#pragma unroll
    for (int i = 1; i < 4; i++)
      if (fabsf(v[b][i]) > a) {
        a = fabsf(v[b][i]);
        mv = v[b][i];
        idx = 4 * lane + i;
      }
    wave_absmax_first(a, idx, mv);
    int q[4] = {0, 0, 0, 0};
    float d = 0.f;
    if (a != 0.f) {
      const float iscale = -128.f / mv;
#pragma unroll
      for (int i = 0; i < 4; i++) q[i] = min(127, (int)roundf(iscale * v[b][i]));
      d = 1.f / iscale;
    }
    int s = (q[0] + q[1]) + (q[2] + q[3]);  // 16-value group g = lanes 4g .. 4g+3
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    if (out) {
      uint8_t* blk = out + ((size_t)t * nb + b) * Q8K_BYTES;
      const uint32_t packed = (uint32_t)(q[0] & 255) | ((uint32_t)(q[1] & 255) << 8) |
                              ((uint32_t)(q[2] & 255) << 16) | ((uint32_t)(q[3] & 255) << 24);
      *reinterpret_cast<uint32_t*>(blk + 4 + 4 * lane) = packed;
      if ((lane & 3) == 0) *reinterpret_cast<int16_t*>(blk + 260 + 2 * (lane >> 2)) = (int16_t)s;
      if (lane == 0) *reinterpret_cast<float*>(blk) = d;
    }
    if (xq) q8k_store_operands(q, d, s, t, b, nb, D, lane, xq, d8, bsop);
  }
}

// Q8_K blocks [T][D/256] -> the matrix-core operands: one workgroup per token, one wave per block.
__global__ __launch_bounds__(256) void q8k_operands_kernel(const uint8_t* __restrict__ blocks, int D,
                                                           int8_t* __restrict__ xq, float* __restrict__ d8,
                                                           _Float16* __restrict__ bsop) {
  const int t = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nb = D / QK_K;
  if (wave >= nb) return;
  const uint8_t* blk = blocks + ((size_t)t * nb + wave) * Q8K_BYTES;
  const uint32_t packed = *reinterpret_cast<const uint32_t*>(blk + 4 + 4 * lane);
  const int q[4] = {(int)(int8_t)(packed & 255), (int)(int8_t)((packed >> 8) & 255),
                    (int)(int8_t)((packed >> 16) & 255), (int)(int8_t)(packed >> 24)};
  const int s = *reinterpret_cast<const int16_t*>(blk + 260 + 2 * (lane >> 2));
  q8k_store_operands(q, *reinterpret_cast<const float*>(blk), s, t, wave, nb, D, lane, xq, d8, bsop);
}

}  // namespace

namespace t5k {
int q8k_bytes_per_row(int D) { return D / QK_K * Q8K_BYTES; }

hipError_t launch_q8k_quantize(const float* x, const float* gamma, float eps, int T, int D, uint8_t* out,
                               hipStream_t s, int8_t* xq, float* d8, _Float16* bsop) {
  if (T <= 0) return hipSuccess;
  if (D <= 0 || D % QK_K || D > 1024 || (!out && !xq) || (xq && (!d8 || !bsop))) return hipErrorInvalidValue;
  T5K_LAUNCH(q8k_quantize_kernel, dim3((T + 3) / 4), dim3(256), 0, s, x, gamma, eps, T, D, out, xq, d8, bsop);
  return hipGetLastError();
}

hipError_t launch_q8k_operands(const uint8_t* blocks, int T, int D, int8_t* xq, float* d8, _Float16* bsop,
                               hipStream_t s) {
  if (T <= 0) return hipSuccess;
  if (D <= 0 || D % QK_K || D > 1024 || !blocks || !xq || !d8 || !bsop) return hipErrorInvalidValue;
  T5K_LAUNCH(q8k_operands_kernel, dim3(T), dim3(256), 0, s, blocks, D, xq, d8, bsop);
  return hipGetLastError();
}
}  // namespace t5k
