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
