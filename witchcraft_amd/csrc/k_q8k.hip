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
//  * q4k_q8k_kernel: tile of 128 weight rows x 32 tokens per 256-thread workgroup (4 rows x 4
//    tokens per thread); the Q4_K rows and Q8_K token blocks of each 256-wide K block are
//    staged in LDS; each thread forms the integer sums of 32-value sub-blocks with
//    v_dot4_i32_i8 (exact), weights them with the 6-bit scales in int32 (exact), and combines
//    per block in f32 as vec_dot does:
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

constexpr int QR = 128, QT = 32;  // weight rows x tokens per workgroup

// Workgroup of 256 threads: thread (rg = tid / 8, tg = tid % 8) owns weight rows 4 rg .. 4 rg + 3
// and tokens 4 tg .. 4 tg + 3 (16 outputs per weight matrix).  Per 256-wide K block the rows'
// Q4_K blocks and the tokens' Q8_K blocks are staged in LDS; per pair of 32-value sub-blocks a
// thread reads each of its rows' 32 nibble bytes and each of its tokens' 64 q8 bytes once
// (16-byte reads) and issues 16 v_dot4_i32_i8 per (row, token).
template <int G>  // 1: plain, 2: gated (W0 gate, W1 up)
__global__ __launch_bounds__(256) void q4k_q8k_kernel(const uint8_t* __restrict__ W0, const uint8_t* __restrict__ W1,
                                                      const uint8_t* __restrict__ X8, int T, int N, int K,
                                                      float* __restrict__ outf, int ldo, _Float16* __restrict__ outh) {
  __shared__ __attribute__((aligned(16))) uint32_t wsh[G][QR * Q4K_BYTES / 4];
  // Q8_K blocks in LDS padded to 76 words so the q8 bytes start 16-byte aligned: d at word 0,
  // q8 at words 4 .. 67, bsums at words 68 .. 75
  constexpr int XW = 76;
  __shared__ __attribute__((aligned(16))) uint32_t xsh[QT * XW];
  const int tid = threadIdx.x, rg = tid >> 3, tg = tid & 7;
  const int n0 = blockIdx.x * QR, t0 = blockIdx.y * QT;
  const int kb_n = K / QK_K;
  float accd[G][4][4], accm[G][4][4];
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
      for (int j = 0; j < 4; j++) accd[g][r][j] = accm[g][r][j] = 0.f;
  const uint8_t* Wg[2] = {W0, W1};

  for (int kb = 0; kb < kb_n; kb++) {
#pragma unroll
    for (int g = 0; g < G; g++)
      for (int i = tid; i < QR * Q4K_BYTES / 4; i += 256) {
        const int row = i / (Q4K_BYTES / 4), w = i % (Q4K_BYTES / 4);
        wsh[g][i] = n0 + row < N
                        ? reinterpret_cast<const uint32_t*>(Wg[g] + ((size_t)(n0 + row) * kb_n + kb) * Q4K_BYTES)[w]
                        : 0u;
      }
    for (int i = tid; i < QT * Q8K_BYTES / 4; i += 256) {
      const int tok = i / (Q8K_BYTES / 4), w = i % (Q8K_BYTES / 4);
      xsh[tok * XW + (w ? w + 3 : 0)] =
          t0 + tok < T ? reinterpret_cast<const uint32_t*>(X8 + ((size_t)(t0 + tok) * kb_n + kb) * Q8K_BYTES)[w] : 0u;
    }
    __syncthreads();
    // per token: d8 and the 16 bsums of this block
    float d8[4];
    int bsp[4][8];  // bsum_2j + bsum_2j+1
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t* xb = &xsh[(4 * tg + j) * XW];
      d8[j] = __uint_as_float(xb[0]);
      const int16_t* bs = reinterpret_cast<const int16_t*>(xb + 68);
#pragma unroll
      for (int k = 0; k < 8; k++) bsp[j][k] = bs[2 * k] + bs[2 * k + 1];
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
      int aux[4][4];
#pragma unroll
      for (int r = 0; r < 4; r++)
#pragma unroll
        for (int j = 0; j < 4; j++) aux[r][j] = 0;
#pragma unroll
      for (int c = 0; c < 4; c++) {  // sub-blocks 2c (low nibbles) and 2c + 1 (high nibbles)
        uint4 q8[4][4];             // token j: q8 bytes 64c .. 64c + 63
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
          for (int v = 0; v < 4; v++)
            q8[j][v] = *reinterpret_cast<const uint4*>(&xsh[(4 * tg + j) * XW + 4 + 16 * c + 4 * v]);
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const uint32_t* blk = &wsh[g][(4 * rg + r) * (Q4K_BYTES / 4)];
          const uint8_t* sb = reinterpret_cast<const uint8_t*>(blk + 1);
          int sc0, sc1;
          if (c < 2) {
            sc0 = sb[2 * c] & 63;
            sc1 = sb[2 * c + 1] & 63;
          } else {
            sc0 = (sb[2 * c + 4] & 15) | ((sb[2 * c - 4] >> 6) << 4);
            sc1 = (sb[2 * c + 5] & 15) | ((sb[2 * c - 3] >> 6) << 4);
          }
          const uint4 qa = *reinterpret_cast<const uint4*>(blk + 4 + 8 * c);
          const uint4 qb = *reinterpret_cast<const uint4*>(blk + 8 + 8 * c);
          const uint32_t qw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const uint32_t q8w[16] = {q8[j][0].x, q8[j][0].y, q8[j][0].z, q8[j][0].w, q8[j][1].x, q8[j][1].y,
                                      q8[j][1].z, q8[j][1].w, q8[j][2].x, q8[j][2].y, q8[j][2].z, q8[j][2].w,
                                      q8[j][3].x, q8[j][3].y, q8[j][3].z, q8[j][3].w};
            int lo = 0, hi = 0;
#pragma unroll
            for (int w = 0; w < 8; w++) {
              lo = __builtin_amdgcn_sdot4((int)(qw[w] & 0x0f0f0f0fu), (int)q8w[w], lo, false);
              hi = __builtin_amdgcn_sdot4((int)((qw[w] >> 4) & 0x0f0f0f0fu), (int)q8w[8 + w], hi, false);
            }
            aux[r][j] += sc0 * lo + sc1 * hi;
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t* blk = &wsh[g][(4 * rg + r) * (Q4K_BYTES / 4)];
        const float d4 = f16_bits_to_f32(blk[0] & 0xffff), dmin4 = f16_bits_to_f32(blk[0] >> 16);
        const uint8_t* sb = reinterpret_cast<const uint8_t*>(blk + 1);
        int mn[8];
#pragma unroll
        for (int k = 0; k < 8; k++) mn[k] = k < 4 ? sb[k + 4] & 63 : (sb[k + 4] >> 4) | ((sb[k] >> 6) << 4);
#pragma unroll
        for (int j = 0; j < 4; j++) {
          int sumi = 0;
#pragma unroll
          for (int k = 0; k < 8; k++) sumi += bsp[j][k] * mn[k];
          accd[g][r][j] += (d4 * d8[j]) * (float)aux[r][j];
          accm[g][r][j] -= (dmin4 * d8[j]) * (float)sumi;
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int n = n0 + 4 * rg + r;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int t = t0 + 4 * tg + j;
      if (t >= T || n >= N) continue;
      if constexpr (G == 1) {
        outf[(size_t)t * ldo + n] = accm[0][r][j] + accd[0][r][j];
      } else {
        const float gate = accm[0][r][j] + accd[0][r][j], up = accm[1][r][j] + accd[1][r][j];
        outh[tiled_index(t, n, N)] = (_Float16)(gelu_pade(gate) * up);
      }
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
  if (N <= 0 || N % 4 || K % QK_K || K <= 0) return hipErrorInvalidValue;
  const dim3 grid((N + QR - 1) / QR, (T + QT - 1) / QT);
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
