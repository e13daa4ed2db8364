// epilogue.hpp -- output stores shared by the GEMM and GEMV kernels.
//
// Both kernels run v_mfma_f32_16x16x32_f16 with the weight fragment as the A operand
// (D^T = W . X^T), so a lane ends with 4 consecutive output columns n..n+3 of one token m.
// These helpers write such a quad for every epilogue kind (Epilogue in common.hpp).
#pragma once
#include "common.hpp"

template <int EPI>
__device__ __forceinline__ void store_quad(const GemmArgs& p, int m, int n, f4 v) {
  if constexpr (EPI == EPI_RESID) {  // residual stream x += acc (f32)
    float4* x = reinterpret_cast<float4*>((float*)p.out + (size_t)m * p.ldo + n);
    float4 r = *x;
    r.x += v[0];
    r.y += v[1];
    r.z += v[2];
    r.w += v[3];
    *x = r;
  } else if constexpr (EPI == EPI_F32) {
    *reinterpret_cast<float4*>((float*)p.out + (size_t)m * p.ldo + n) = make_float4(v[0], v[1], v[2], v[3]);
  } else if constexpr (EPI == EPI_F16 || EPI == EPI_RELU) {  // operand order for the next GEMM
    if (EPI == EPI_RELU) v = f4{fmaxf(v[0], 0.f), fmaxf(v[1], 0.f), fmaxf(v[2], 0.f), fmaxf(v[3], 0.f)};
    *reinterpret_cast<h4*>((_Float16*)p.out + tiled_index(m, n, p.ldo)) =
        h4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
  } else if constexpr (EPI == EPI_QKV) {  // 4 consecutive columns stay inside one head (dkv % 4 == 0)
    const int inner = p.heads * p.dkv;
    const int nn = n + p.n_off;
    const int which = nn / inner, rem = nn % inner;
    const int h = rem / p.dkv, d = rem % p.dkv;
    _Float16* dst = (_Float16*)p.out + (((size_t)which * p.heads + h) * p.tpad + m) * p.dkv + d;
    *reinterpret_cast<h4*>(dst) = h4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
  }
}

// Gated FFN hidden state gelu_tanh(x W0^T) * (x W1^T), in operand order for the wo GEMM.
__device__ __forceinline__ void store_quad_gated(const GemmArgs& p, int m, int n, f4 g, f4 u) {
  *reinterpret_cast<h4*>((_Float16*)p.out + tiled_index(m, n, p.ldo)) =
      h4{(_Float16)(gelu_tanh_dev(g[0]) * u[0]), (_Float16)(gelu_tanh_dev(g[1]) * u[1]),
         (_Float16)(gelu_tanh_dev(g[2]) * u[2]), (_Float16)(gelu_tanh_dev(g[3]) * u[3])};
}

// Consumer side of a folded T5LayerNorm (GemmArgs::rec).  Lane l serves token
// mrow0 + 16 * (l / 16) + l % 16 (lanes whose row block lies past MB read block 0 instead):
// norm_rec_load fetches its record before the K loop's first loads, norm_factor turns it
// into rsqrt(mean(x^2) + eps) / s once those have landed.  The sums run in a fixed order, so
// every tile of every launch (and the one-launch FFN of k_ffn.hip) gets the same bits.  Tiles
// at n0 = 0 also store the next producer's operand scale.
template <int MB>
__device__ __forceinline__ int norm_row(int mrow0) {
  const int lane = threadIdx.x & 63, mb = lane >> 4;
  return mrow0 + 16 * (mb < MB ? mb : 0) + (lane & 15);
}
template <int MB>
__device__ __forceinline__ void norm_rec_load(const GemmArgs& p, int mrow0, float4 (&r)[4]) {
  const float4* src = reinterpret_cast<const float4*>(p.rec + (size_t)norm_row<MB>(mrow0) * 16);
#pragma unroll
  for (int i = 0; i < 4; i++) r[i] = src[i];
}
// rsqrt(mean(x^2) + eps) of a token of K features from its norm record r (slot 15 unused here).
__device__ __forceinline__ float norm_inv(const float4 (&r)[4], int K, float eps) {
  // slots past K / 64 are masked: the record array may hold another layout's data there
  const int ns = K / 64;
  float v[15];
#pragma unroll
  for (int i = 0; i < 15; i++) {
    const float4 q = r[i / 4];
    const float x = (i & 3) == 0 ? q.x : (i & 3) == 1 ? q.y : (i & 3) == 2 ? q.z : q.w;
    v[i] = i < ns ? x : 0.f;
  }
  const float tot = (((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]))) +
                    (((v[8] + v[9]) + (v[10] + v[11])) + ((v[12] + v[13]) + v[14]));
  return 1.0f / sqrtf(tot / (float)K + eps);
}
template <int MB>
__device__ __forceinline__ float norm_factor(const GemmArgs& p, int mrow0, int n0, const float4 (&r)[4]) {
  const float inv = norm_inv(r, p.K, p.eps);
  const int m = norm_row<MB>(mrow0);
  if (p.rec_next && n0 == 0 && (threadIdx.x & 63) < 16 * MB && m < p.M)
    p.rec_next[(size_t)m * 16 + 15] = norm_operand_scale(inv);
  return inv / r[3].w;
}

// A quad's sum of squares, as the residual epilogues add it into a norm record slot.
__device__ __forceinline__ float quad_sq(float4 r) { return (r.x * r.x + r.y * r.y) + (r.z * r.z + r.w * r.w); }
