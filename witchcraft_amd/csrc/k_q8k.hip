// k_q8k.hip -- the reference's hybrid-dequant FFN numerics: f32 activations quantized to GGML
// Q8_K blocks and multiplied against Q4_K weights with integer dot products.
//
// Reference: with the `hybrid-dequant` feature (src/quantized_t5.rs:18-21,233-244) the gated
// FFN's wi_0 / wi_1 run through fused_gated_gelu_inner (src/fused_matmul.rs:138-177) and the
// final projection through QTiledOp (tiled_matmul_inner, :27-59).  Both quantize every f32
// activation row with candle's BlockQ8K::from_float and take GGML's Q4_K x Q8_K vec_dot per
// (row, token); the gate goes through a Pade tanh gelu (:128-133,168-170).  This is the
// numerics of the reference's x86 default build.
//
//  * q8k_quantize_kernel: one workgroup per token, one wave per 256-value block (D <= 1024).
//    Optional T5LayerNorm first (x / sqrt(mean(x^2) + eps) * w in f32, src/quantized_t5.rs:
//    162-173).  Q8_K: the value of largest magnitude (the first one on ties) sets
//    iscale = -128 / v, q = min(127, round(iscale * x)) with halves away from zero, d = 1 / iscale,
//    bsums = sums of 16 consecutive q; an all-zero block gives d = 0 and q = 0.  Bit-exact with
//    BlockQ8K::from_float on the same f32 input.
//  * q4k_q8k_kernel: tile of 64 weight rows x 16 tokens per 256-thread workgroup; the Q4_K
//    rows and Q8_K token blocks of each 256-wide K block are staged in LDS; each thread forms
//    the integer sums of 32-value sub-blocks with v_dot4_i32_i8 (exact), weights them with the
//    6-bit scales in int32 (exact), and combines per block in f32 as vec_dot does:
//    + f16(d) * d8 * sum_j sc_j (q4 . q8)_j  - f16(dmin) * d8 * sum_j m_j (bsum_2j + bsum_2j+1).
//    GGML's generic C code keeps eight lane partials of the first term and x86 builds use AVX2
//    lanes: the float combination order is implementation-defined in the reference too.
//    Epilogues: f32 rows (projection) or gelu_pade(gate) * up stored as the f16 operand of
//    the wo GEMM (operand order).
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

__global__ __launch_bounds__(256) void q8k_quantize_kernel(const float* __restrict__ x, const float* __restrict__ gamma,
                                                           float eps, int T, int D, uint8_t* __restrict__ out) {
  const int t = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int nb = D / 256;
  __shared__ float part[4];
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (wave < nb) {
    const float4 u = *reinterpret_cast<const float4*>(x + (size_t)t * D + 4 * tid);
    v[0] = u.x, v[1] = u.y, v[2] = u.z, v[3] = u.w;
  }
  if (gamma) {  // T5LayerNorm in f32
    float ss = (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if (lane == 0) part[wave] = ss;
    __syncthreads();
    const float tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float den = sqrtf(tot / (float)D + eps);
    if (wave < nb) {
      const float4 g = *reinterpret_cast<const float4*>(gamma + 4 * tid);
      v[0] = (v[0] / den) * g.x;
      v[1] = (v[1] / den) * g.y;
      v[2] = (v[2] / den) * g.z;
      v[3] = (v[3] / den) * g.w;
    }
  }
  if (wave >= nb) return;
  // largest magnitude, first index on ties (the block's values in index order 4 * lane + i)
  float a = fabsf(v[0]), mv = v[0];
  int idx = 4 * lane;
#pragma unroll
  for (int i = 1; i < 4; i++)
    if (fabsf(v[i]) > a) {
      a = fabsf(v[i]);
      mv = v[i];
      idx = 4 * lane + i;
    }
  wave_absmax_first(a, idx, mv);
  uint8_t* blk = out + ((size_t)t * nb + wave) * Q8K_BYTES;
  int q[4] = {0, 0, 0, 0};
  float d = 0.f;
  if (a != 0.f) {
    const float iscale = -128.f / mv;
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = min(127, (int)roundf(iscale * v[i]));
    d = 1.f / iscale;
  }
  const uint32_t packed = (uint32_t)(q[0] & 255) | ((uint32_t)(q[1] & 255) << 8) | ((uint32_t)(q[2] & 255) << 16) |
                          ((uint32_t)(q[3] & 255) << 24);
  *reinterpret_cast<uint32_t*>(blk + 4 + 4 * lane) = packed;
  int s = (q[0] + q[1]) + (q[2] + q[3]);  // 16-value group g = lanes 4g .. 4g+3
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  if ((lane & 3) == 0) *reinterpret_cast<int16_t*>(blk + 260 + 2 * (lane >> 2)) = (int16_t)s;
  if (lane == 0) *reinterpret_cast<float*>(blk) = d;
}

// candle's Pade tanh (src/fused_matmul.rs:128-133) and the gate of the fused FFN (:168-170).
__device__ __forceinline__ float fast_tanh_pade(float x) {
  x = x < -4.97f ? -4.97f : (x > 4.97f ? 4.97f : x);
  const float x2 = x * x;
  return x * (135135.0f + x2 * (17325.0f + x2 * (378.0f + x2))) /
         (135135.0f + x2 * (62370.0f + x2 * (3150.0f + 28.0f * x2)));
}
__device__ __forceinline__ float gelu_pade(float g) {
  return 0.5f * g * (1.0f + fast_tanh_pade(0.7978845608f * g * (1.0f + 0.044715f * g * g)));
}

constexpr int QR = 64, QT = 16;  // weight rows x tokens per workgroup

template <int G>  // 1: plain, 2: gated (W0 gate, W1 up)
__global__ __launch_bounds__(256) void q4k_q8k_kernel(const uint8_t* __restrict__ W0, const uint8_t* __restrict__ W1,
                                                      const uint8_t* __restrict__ X8, int T, int N, int K,
                                                      float* __restrict__ outf, int ldo, _Float16* __restrict__ outh) {
  __shared__ uint32_t wsh[G][QR * Q4K_BYTES / 4];
  __shared__ uint32_t xsh[QT * Q8K_BYTES / 4];
  const int tid = threadIdx.x, r = tid >> 2, tq = tid & 3;
  const int n0 = blockIdx.x * QR, t0 = blockIdx.y * QT;
  const int kb_n = K / QK_K;
  float accd[G][4], accm[G][4];
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int j = 0; j < 4; j++) accd[g][j] = accm[g][j] = 0.f;
  const uint8_t* Wg[2] = {W0, W1};

  for (int kb = 0; kb < kb_n; kb++) {
    // stage the 64 rows' Q4_K blocks and the 16 tokens' Q8_K blocks of this K block
#pragma unroll
    for (int g = 0; g < G; g++)
      for (int i = tid; i < QR * Q4K_BYTES / 4; i += 256) {
        const int row = i / (Q4K_BYTES / 4), w = i % (Q4K_BYTES / 4);
        wsh[g][i] = reinterpret_cast<const uint32_t*>(Wg[g] + ((size_t)(n0 + row) * kb_n + kb) * Q4K_BYTES)[w];
      }
    for (int i = tid; i < QT * Q8K_BYTES / 4; i += 256) {
      const int tok = i / (Q8K_BYTES / 4), w = i % (Q8K_BYTES / 4);
      xsh[i] = t0 + tok < T ? reinterpret_cast<const uint32_t*>(X8 + ((size_t)(t0 + tok) * kb_n + kb) * Q8K_BYTES)[w]
                            : 0u;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) {
      const uint32_t* blk = &wsh[g][r * (Q4K_BYTES / 4)];
      const float d4 = f16_bits_to_f32(blk[0] & 0xffff), dmin4 = f16_bits_to_f32(blk[0] >> 16);
      // get_scale_min_k4 over the 12 scale bytes (words 1..3)
      const uint8_t* sb = reinterpret_cast<const uint8_t*>(blk + 1);
      int sc[8], mn[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        if (j < 4) {
          sc[j] = sb[j] & 63;
          mn[j] = sb[j + 4] & 63;
        } else {
          sc[j] = (sb[j + 4] & 15) | ((sb[j - 4] >> 6) << 4);
          mn[j] = (sb[j + 4] >> 4) | ((sb[j] >> 6) << 4);
        }
      }
      int aux[4] = {0, 0, 0, 0};
#pragma unroll
      for (int sbk = 0; sbk < 8; sbk++) {
        const int c = sbk >> 1;
        uint32_t q4[8];
#pragma unroll
        for (int w = 0; w < 8; w++) {
          const uint32_t b = blk[4 + 8 * c + w];  // nibble bytes qs[32c .. 32c + 31]
          q4[w] = (sbk & 1) ? (b >> 4) & 0x0f0f0f0fu : b & 0x0f0f0f0fu;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const uint32_t* q8 = &xsh[(4 * tq + j) * (Q8K_BYTES / 4) + 1 + 8 * sbk];
          int isum = 0;
#pragma unroll
          for (int w = 0; w < 8; w++) isum = __builtin_amdgcn_sdot4((int)q4[w], (int)q8[w], isum, false);
          aux[j] += sc[sbk] * isum;
        }
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t* xb = &xsh[(4 * tq + j) * (Q8K_BYTES / 4)];
        const float d8 = __uint_as_float(xb[0]);
        const int16_t* bs = reinterpret_cast<const int16_t*>(xb + 65);
        int sumi = 0;
#pragma unroll
        for (int k = 0; k < 16; k++) sumi += bs[k] * mn[k / 2];
        accd[g][j] += (d4 * d8) * (float)aux[j];
        accm[g][j] -= (dmin4 * d8) * (float)sumi;
      }
    }
    __syncthreads();
  }
  const int n = n0 + r;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int t = t0 + 4 * tq + j;
    if (t >= T) continue;
    if constexpr (G == 1) {
      outf[(size_t)t * ldo + n] = accm[0][j] + accd[0][j];
    } else {
      const float gate = accm[0][j] + accd[0][j], up = accm[1][j] + accd[1][j];
      outh[tiled_index(t, n, N)] = (_Float16)(gelu_pade(gate) * up);
    }
  }
}

}  // namespace

namespace t5k {
int q8k_bytes_per_row(int D) { return D / QK_K * Q8K_BYTES; }

hipError_t launch_q8k_quantize(const float* x, const float* gamma, float eps, int T, int D, uint8_t* out,
                               hipStream_t s) {
  if (T <= 0) return hipSuccess;
  if (D <= 0 || D % QK_K || D > 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(q8k_quantize_kernel, dim3(T), dim3(256), 0, s, x, gamma, eps, T, D, out);
  return hipGetLastError();
}

hipError_t launch_q4k_q8k(const uint8_t* W0, const uint8_t* W1, const uint8_t* X8, int T, int N, int K, float* outf,
                          int ldo, _Float16* outh, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  if (N % QR || K % QK_K || K <= 0) return hipErrorInvalidValue;
  const dim3 grid(N / QR, (T + QT - 1) / QT);
  if (W1) {
    if (!outh) return hipErrorInvalidValue;
    hipLaunchKernelGGL(q4k_q8k_kernel<2>, grid, dim3(256), 0, s, W0, W1, X8, T, N, K, nullptr, 0, outh);
  } else {
    if (!outf) return hipErrorInvalidValue;
    hipLaunchKernelGGL(q4k_q8k_kernel<1>, grid, dim3(256), 0, s, W0, nullptr, X8, T, N, K, outf, ldo, nullptr);
  }
  return hipGetLastError();
}
}  // namespace t5k
