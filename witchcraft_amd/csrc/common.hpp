// common.hpp -- shared types and helpers for the t5-hip kernels (gfx950 / CDNA4).
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace t5k {
// Kernel-time events of a profiled forward (host, per thread).  While `stop` is set, the encoder's
// launches go through hipExtLaunchKernelGGL with these events, which the runtime binds to the
// kernel dispatch itself: start is the first such kernel's start, stop the last one's end, so
// their elapsed time is kernel execution time inside the forward, without the gaps between
// launches.  The launch takes `start` (once) and leaves `stop` for later launches of the class.
struct LaunchTiming {
  hipEvent_t start = nullptr, stop = nullptr;
};
extern thread_local LaunchTiming tl_launch_timing;
}  // namespace t5k

// hipLaunchKernelGGL, or its timed form while a profiled forward has set t5k::tl_launch_timing.
#define T5K_LAUNCH(kernel, grid, block, shmem, stream, ...)                                          \
  do {                                                                                             \
    t5k::LaunchTiming& lt_ = t5k::tl_launch_timing;                                                \
    if (lt_.stop) {                                                                                \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, lt_.start, lt_.stop, 0, __VA_ARGS__); \
      lt_.start = nullptr;                                                                         \
    } else {                                                                                       \
      hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                        \
    }                                                                                              \
  } while (0)

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
  EPI_F16 = 0,    // out f16 [M][ldo] in operand order (tiled_index)
  EPI_RESID = 1,  // resid f32 [M][ldo] += acc; the batched GEMM reads (not writes) rows up to Mpad
  EPI_GATED = 2,  // out f16 = gelu_tanh(acc(W0)) * acc(W1), operand order
  EPI_F32 = 3,    // out f32 [M][ldo]
  EPI_QKV = 4,    // q/k/v f16 head-major [3][H][tpad][dkv]
  EPI_RELU = 5    // out f16 = max(acc, 0), operand order (non-gated T5DenseActDense)
};

// Activations that feed a GEMM (RMSNorm output, attention output, gated hidden state) are
// stored in "MFMA operand order": the [M][K] f16 matrix is cut into 16-row x 32-column
// blocks of 1 KiB, blocks row-major ([M/16][K/32]), and inside a block lane l of a wave64
// owns the 16 bytes at l*16 = row (l % 16), columns 8*(l / 16) .. +7 -- exactly the
// register layout of a v_mfma_f32_16x16x32_f16 operand.  A wave loads one operand with one
// fully contiguous 1 KiB dwordx4 load.  M must be padded to a multiple of 16, K % 32 == 0.
__host__ __device__ __forceinline__ size_t tiled_index(size_t m, size_t k, size_t K) {
  return ((m >> 4) * (K >> 5) + (k >> 5)) * 512 + ((((k & 31) >> 3) << 4) + (m & 15)) * 8 + (k & 7);
}

struct GemmArgs {
  const _Float16* A;  // [Mpad][K] f16 in operand order (tiled_index), Mpad >= roundup(M, 512)
  int lda;            // unused (A's row length is K)
  const void* W0;  // [N][K] weights (Q4_K blocks row-major along K, or f16)
  const void* W1;  // second weight for EPI_GATED
  int M, N, K;     // N counts output columns (per weight for EPI_GATED)
  void* out;
  int ldo;
  int n_off;  // column offset added before the QKV scatter
  int heads, dkv, tpad;
  // GEMV only: when xf is set, the operand is T5LayerNorm(xf) computed in the kernel
  // (xf f32 [M][K] row-major, gamma [K]) instead of A.
  const float* xf;
  const float* gamma;
  float eps;
  // Batched GEMM only: T5LayerNorm folded into the GEMMs on either side of it.  Each token
  // has a 64-byte record rec[16m .. 16m+15]: slots t < 15 hold sums of x^2 over the columns
  // [64t, 64t + 64) (slots past D/64 are ignored), slot 15 the power of two s with which the
  // f16 operand of that token was stored.
  //  * producer (EPI_RESID with nx set): x += acc as usual; then nx = f16(x * ngamma * s) in
  //    operand order with s = rec[16m + 15], and each tile's sums of x^2 into rec.
  //  * consumer (any other epilogue with rec set): the operand is f16(x * gamma * s), so acc
  //    is scaled by rsqrt(mean(x^2) + eps) / s; the tile at n0 = 0 writes the s of the next
  //    producer, a power of two near 1/16 of that inverse RMS, into rec_next[16m + 15].
  float* rec;
  float* rec_next;
  _Float16* nx;
  const float* ngamma;
  // GEMV only: compute units of the device, for the grid shape (0: 256).
  int cus;
  // Hybrid numerics (launch_gemm_hybrid): A holds the Q8_K integers q8 of every token as int8
  // (blocks of 16 tokens x 64 K, 1 KiB, [Mpad/16][K/64]; lane l of a block: token l % 16, K
  // 16 (l / 16) .. +15), d8 [Mpad][K/256] their block scales, bsop the blocks' 16 bsums as the
  // B operand of one 16x16x32 MFMA per (16-token row block, K block) -- 1 KiB blocks [Mpad/16][K/256], lane l
  // = (token l % 16, K slots 8 (l / 16) .. +7): bsum 8 (l / 16) + e for l < 32, zero for l >= 32.
  const float* d8;
  const _Float16* bsop;
};

// Largest row length (d_model) whose sums of squares fit a norm record (15 slots of 64).
constexpr int NORM_REC_MAX_D = 15 * 64;
// The GEMV kernels (M <= GEMV_MAX_M) fold the norm the same way with 64-float records: a
// GEMV workgroup owns 16 columns, so slot t < 63 holds the sum of x^2 over [16t, 16t + 16)
// and slot 63 the operand scale s.
constexpr int NORM_REC_GEMV = 64;

// The operand scale that follows an inverse RMS: the power of two at or below inv, / 16.
// Stored values then have an RMS near |gamma| / 16, leaving room for the residual stream to
// grow before the next norm; 1 when inv is 0, subnormal, infinite or NaN.
__host__ __device__ __forceinline__ float norm_operand_scale(float inv) {
  uint32_t b;
  __builtin_memcpy(&b, &inv, 4);
  const uint32_t e = b & 0x7f800000u;
  uint32_t r = 0x3f800000u;
  if (e > (4u << 23) && e < 0x7f800000u) r = e - (4u << 23);
  float s;
  __builtin_memcpy(&s, &r, 4);
  return s;
}

// Queries per attention work list item (one workgroup): 4 waves x 32 for sequences longer than
// ATTN_SMALL_L tokens, 4 waves x 16 up to that length.  The split depends on the sequence's own
// length only.
constexpr int ATTN_QT = 128;
constexpr int ATTN_SMALL_L = 128;
__host__ __device__ __forceinline__ int attn_item_queries(int L) { return L <= ATTN_SMALL_L ? 64 : ATTN_QT; }
__host__ __device__ __forceinline__ int attn_items(int L) {
  const int q = attn_item_queries(L);
  return (L + q - 1) / q;
}

struct AttnArgs {
  const _Float16* qkv;  // [3][H][tpad][dkv]
  _Float16* out;        // [T][H*dkv] in operand order (tiled_index)
  const int4* work;     // (sequence start, length, first query, head) per workgroup; length 0: empty
  const float* lut;     // [H][2*lutw+1] relative bias by (j - i), centred at lutw
  int heads, tpad, lutw;
};

// Device-side helpers ---------------------------------------------------------

// LDS tiles of f16 with 64-half rows, unpadded, where 16-byte chunk c of row r is stored at
// chunk c ^ (r & 7): a read of 16 rows x one chunk (ds_read_b128) and a transposed read of 16
// rows x 32 bytes (ds_read_b64_tr_b16) each hit every bank once (measured with probe kernels).
__device__ __forceinline__ int swz64(int row, int col) {
  return row * 64 + ((((col >> 3) ^ row) & 7) << 3) + (col & 7);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  _Float16 h;
  uint16_t b = (uint16_t)bits16;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;
}

// Cross-lane pairs without LDS (gfx950 v_permlane16_swap / v_permlane32_swap with the same
// register as both operands): every lane l receives its own value and that of lane l ^ 16
// (l ^ 32), in an order that differs between the two lanes of a pair -- so only commutative
// combinations (+, max) are taken, and both lanes of a pair get identical bits.
__device__ __forceinline__ float sum_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// candle Tensor::gelu (tanh form): 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3),
// evaluated as the identical x * sigmoid(2u) = x / (1 + 2^(-2u log2 e)).
__device__ __forceinline__ float gelu_tanh_dev(float x) {
  // -2 log2(e) * u = x * (-2.302208198 - 0.102943497 x^2)
  const float t = x * __builtin_fmaf(-0.10294324148f * x, x, -2.3022081983f);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

// candle's Pade tanh (src/fused_matmul.rs:128-133) and the gelu of the hybrid-dequant gated FFN
// (:168-170), in f32 with no contraction, as the reference's scalar code rounds it.
__device__ __forceinline__ float fast_tanh_pade(float x) {
#pragma clang fp contract(off)
  x = x < -4.97f ? -4.97f : (x > 4.97f ? 4.97f : x);
  const float x2 = x * x;
  return x * (135135.0f + x2 * (17325.0f + x2 * (378.0f + x2))) /
         (135135.0f + x2 * (62370.0f + x2 * (3150.0f + 28.0f * x2)));
}
__device__ __forceinline__ float gelu_pade(float g) {
#pragma clang fp contract(off)
  return 0.5f * g * (1.0f + fast_tanh_pade(0.7978845608f * g * (1.0f + 0.044715f * g * g)));
}

// Host-side launchers (defined in the .hip files) --------------------------------
namespace t5k {
hipError_t launch_q4k_dequant(const void* blocks, size_t nblk, float* out, hipStream_t s);
// Q4_K -> f32 (exact) -> bf16 truncation -> f16, [nblk * 256] in block order.
hipError_t launch_q4k_dequant_bf16_f16(const void* blocks, size_t nblk, _Float16* out, hipStream_t s);
// Tile plan of one batched GEMM launch: full tiles of 64*mw token rows x bn weight rows
// cover rows [0, m_main); thin tiles of 16*tail_mb rows per math wave cover [m_main, M)
// (tail_mb = 0: full tiles everywhere).
// mb: 16-token row blocks per math wave in the full tiles (4, or 3 with mw = 4).
struct GemmPlan {
  int mw = 4, bn = 128, m_main = 0, tail_mb = 0, mb = 4;
};
GemmPlan gemm_plan(int M, int n_rows, int cus, int mw_override, int bn_override, int tail_override,
                   int mb_override = 0);
hipError_t launch_gemm(int epi, int wfmt, const GemmPlan& plan, const GemmArgs& a, hipStream_t s);
// Small-M variant (M <= GEMV_MAX_M tokens), same arguments and results.
constexpr int GEMV_MAX_M = 64;
hipError_t launch_gemv(int epi, int wfmt, const GemmArgs& a, hipStream_t s);
void gemm_pick_tile(int M, int n_rows, int cus, int& mw, int& bn);
hipError_t launch_attention(const AttnArgs& a, int n_work, int dkv, hipStream_t s);
// With rec set, also the first block's T5LayerNorm (weight gamma) in record mode into xn / rec,
// as launch_rmsnorm's record mode (D <= 1024); rec_stride 16 (batched GEMMs) or 64 (GEMV).
hipError_t launch_embed(const uint32_t* ids, int T, const void* table, int fmt, int vocab, int D,
                        float* x, unsigned* err_flag, hipStream_t s, const float* gamma = nullptr,
                        float eps = 0.f, _Float16* xn = nullptr, float* rec = nullptr, int rec_stride = 16);
// rec: when set, record mode for a consuming GEMM that folds the norm (GemmArgs::rec).
hipError_t launch_rmsnorm(const float* x, const float* w, _Float16* out, int T, int D, float eps,
                          hipStream_t s, float* rec = nullptr, int rec_stride = 16);
// err (may be null): set to 1 when a row's norm is not finite.
hipError_t launch_rownorm(float* y, float* norm, int T, int P, int normalize, hipStream_t s,
                          unsigned* err = nullptr);
hipError_t launch_f32_to_f16(const float* x, _Float16* y, size_t n, int K, hipStream_t s);
// Query-side scoring: C = A . B^T (f32) and its per-row argmax (k_score.hip).
hipError_t launch_matmul_t(const float* A, const float* B, float* C, int M, int N, int D, bool bf16_b,
                           hipStream_t s);
hipError_t launch_matmul_argmax(const float* A, const float* B, uint32_t* out, int M, int N, int D, bool bf16_b,
                                hipStream_t s);
// The gated FFN of one block in one launch (k_ffn.hip): x += (gelu(xn' W0^T) * (xn' W1^T)) Wo^T,
// xn' the T5LayerNorm of x folded as for the batched GEMMs, the same bits as the EPI_GATED and
// EPI_RESID launches with their NormLinks.  D must be 768 and F % 256 == 0.
struct FfnArgs {
  const _Float16* xn;     // [Mpad][D] f16(x * gamma * s), operand order (the gate|up GEMM's A)
  const void* W0;         // [F][D] Q4_K
  const void* W1;         // [F][D] Q4_K
  const void* Wo;         // [D][F] Q4_K or f16
  float* x;               // [Mpad][D] residual stream, += the FFN output
  const float* rec;       // norm records of x (the gate|up GEMM's rec)
  float* rec_out;         // slot 15 <- the next operand scale; slots < D/64 <- sums of x^2 of the new x
  _Float16* nx;           // the next norm's operand (may be xn), or null: no records, no operand
  const float* ngamma;    // the next norm's weight
  float eps;
  int M, D, F;
};
hipError_t launch_ffn_fused(const FfnArgs& a, int wo_fmt, hipStream_t s);
// Attention work items written from kernel arguments: CAP sequences per launch.
// Attention work list entries passed by value: item q of entry i is written at
// work[pos + 8 q] as (start, len, 64 q, head); an entry of length 0 writes `start` empty items.
struct WorkChunk {
  static constexpr int CAP = 96;
  int n;
  int start[CAP], len[CAP], head[CAP], pos[CAP];
};
hipError_t launch_work_list(const WorkChunk& c, int4* work, hipStream_t s);
// Embedder post-processing over a batch of documents (k_embed.hip): win = packed window outputs,
// docs[d] = (first token, tokens, first window row, windows), tok_doc[t] = document of token t.
hipError_t launch_embed_batch(const float* win, const int4* docs, const int* tok_doc, int N, int max_len, int stride,
                              int P, float* norms, uint8_t* flags, int* block_counts, int* block_offsets, float* out,
                              int* kept_index, int* kept_offsets, hipStream_t s);
// Blocks of tokens the embed kernels use for N tokens (block_counts / block_offsets need one more).
int embed_batch_blocks(int N);
// Hybrid-dequant numerics (k_q8k.hip): f32 rows [T][D] (T5LayerNorm with gamma first, unless
// gamma is null) quantized to GGML Q8_K; the result as Q8_K blocks [T][D/256] (out, may be
// null) and/or as the operands of launch_gemm_hybrid (xq, d8, bsop as GemmArgs describes them;
// xq null: not written).  launch_q8k_operands converts Q8_K blocks to those operands.
int q8k_bytes_per_row(int D);
hipError_t launch_q8k_quantize(const float* x, const float* gamma, float eps, int T, int D, uint8_t* out,
                               hipStream_t s, int8_t* xq = nullptr, float* d8 = nullptr, _Float16* bsop = nullptr);
hipError_t launch_q8k_operands(const uint8_t* blocks, int T, int D, int8_t* xq, float* d8, _Float16* bsop,
                               hipStream_t s);
// Q4_K weights x Q8_K activations on the matrix cores (k_gemm.hip): per K block of 256, the int8
// planes (sc >> 3) q4 and (sc & 7) q4 against int8 q8 sum the block's integers exactly in int32
// (8 hi + lo); the block then adds d4 d8 * sum - dmin4 d8 * (mins . bsums) in f32.  epi:
// EPI_GATED (gelu_pade(W0) * W1 into the f16 operand, operand order) or EPI_F32.  Q4_K weights, bn = 64, K <= 1024.
GemmPlan gemm_plan_hybrid(int M, int n_rows, int cus);
// Rows of the A operand, d8 and bsop a hybrid launch over M tokens may read (its full tiles
// round M up to the tile height): the buffers must hold at least this many.
int gemm_hybrid_rows(int M);
hipError_t launch_gemm_hybrid(int epi, const GemmPlan& plan, const GemmArgs& a, hipStream_t s);
}  // namespace t5k
