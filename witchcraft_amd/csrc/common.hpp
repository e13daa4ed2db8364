// common.hpp -- shared types and helpers for the t5-hip kernels (gfx950 / CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

// GGML Q4_K super-block: {f16 d, f16 dmin, u8 scales[12], u8 qs[128]} = 144 bytes, 256 values.
constexpr int QK_K = 256;
constexpr int Q4K_BYTES = 144;

// Weight storage formats on the device.
enum WeightFmt : int { WF_Q4K = 0, WF_F16 = 1 };
// Embedding table formats.
enum EmbFmt : int { EMB_F32 = 0, EMB_Q4K = 1 };

// GEMM epilogues.
enum Epilogue : int {
  EPI_F16 = 0,    // out f16 [M][ldo]
  EPI_RESID = 1,  // resid f32 [M][ldo] += acc
  EPI_GATED = 2,  // out f16 = gelu_tanh(acc(W0)) * acc(W1)
  EPI_F32 = 3,    // out f32 [M][ldo]
  EPI_QKV = 4,    // q/k/v f16 head-major [3][H][tpad][dkv]
  EPI_RELU = 5    // out f16 = max(acc, 0) (non-gated T5DenseActDense)
};

struct GemmArgs {
  const _Float16* A;  // [Mpad][lda] f16, Mpad >= roundup(M, 128)
  int lda;
  const void* W0;  // [N][K] weights (Q4_K blocks row-major along K, or f16)
  const void* W1;  // second weight for EPI_GATED
  int M, N, K;     // N counts output columns (per weight for EPI_GATED)
  void* out;
  int ldo;
  int n_off;  // column offset added before the QKV scatter
  int heads, dkv, tpad;
};

struct AttnArgs {
  const _Float16* qkv;  // [3][H][tpad][dkv]
  _Float16* out;        // [T][H*dkv]
  const int* cu;        // [B+1] device
  const int2* work;     // (seq, q_tile) pairs
  const float* lut;     // [H][2*maxl-1] relative bias by (j - i)
  int heads, tpad, maxl;
};

// Device-side helpers ---------------------------------------------------------

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  _Float16 h;
  uint16_t b = (uint16_t)bits16;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;
}

// candle Tensor::gelu (tanh form) with tanh(u) = 1 - 2/(exp(2u)+1).
__device__ __forceinline__ float gelu_tanh_dev(float x) {
  const float u = 0.7978845608028654f * x * (1.0f + 0.044715f * x * x);
  const float e = __expf(2.0f * u);
  const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
  return 0.5f * x * (1.0f + t);
}

// Host-side launchers (defined in the .hip files) --------------------------------
namespace t5k {
hipError_t launch_q4k_dequant(const void* blocks, size_t nblk, float* out, hipStream_t s);
hipError_t launch_gemm(int epi, int wfmt, int mw, int bn, const GemmArgs& a, hipStream_t s);
void gemm_pick_tile(int M, int n_rows, int cus, int& mw, int& bn);
hipError_t launch_attention(const AttnArgs& a, int n_work, int dkv, hipStream_t s);
hipError_t launch_embed(const uint32_t* ids, int T, const void* table, int fmt, int vocab, int D,
                        float* x, unsigned* err_flag, hipStream_t s);
hipError_t launch_rmsnorm(const float* x, const float* w, _Float16* out, int T, int D, float eps,
                          hipStream_t s);
hipError_t launch_rownorm(float* y, float* norm, int T, int P, int normalize, hipStream_t s);
hipError_t launch_f32_to_f16(const float* x, _Float16* y, size_t n, hipStream_t s);
hipError_t launch_window_sum(const float* win_out, const int* src_rows, int n_tokens, int max_windows,
                             int P, float* sum, float* norm, float* normalized, hipStream_t s);
}  // namespace t5k
