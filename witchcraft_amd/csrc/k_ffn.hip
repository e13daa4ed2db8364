// k_ffn.hip -- the gated-GELU FFN of one T5 block in one launch, its d_ff intermediate kept in LDS.
//
// Reference: T5DenseGatedActDense::forward, src/quantized_t5.rs:231-252 (h = gelu_tanh(x W0^T) *
// (x W1^T), y = h Wo^T), with the T5LayerNorm in front of it and the residual add after it
// (T5LayerFF, :284-293).  Per token this computes what the two batched launches of k_gemm.hip
// compute -- gate|up with the folded norm and the gelu * up epilogue, then wo with the residual
// epilogue that prepares the next norm -- with the same bits: every product runs on
// v_mfma_f32_16x16x32_f16 with the weight fragment as the A operand and the same values in the
// same lanes, every output keeps its K order, and the epilogues share their arithmetic.  What
// differs is where the hidden state h lives: never in memory.
//
// Workgroup: 64 tokens (4 row blocks of 16), 8 wave64s (two per SIMD), one workgroup per CU.
//  * The tile's f16 operand xn [64][D] (operand order, 1 KiB per 16 x 32 block) is copied
//    global -> LDS once, and its norm records give each token's factor rsqrt(mean(x^2)+eps)/s.
//  * d_ff is walked in slices of SL = 256 columns.  Phase 1: wave w computes gate and up for
//    slice columns 32w .. 32w+31 over all 64 tokens.  It unpacks its own 2 + 2 Q4_K weight row
//    blocks (the nibble arithmetic of the GEMM producers) straight into MFMA A operands and
//    reads the token operands from LDS, each one feeding 4 MFMAs.  The norm factor and
//    gelu(gate) * up give its 32 columns of h, stored in LDS in operand order.  Phase 2: wave w
//    accumulates output columns 96w .. 96w+95 (6 row blocks of Wo) over the slice's 256 K, its
//    A operands again unpacked in registers and h read from LDS.  The 6 x 4 output
//    accumulators stay in registers across all slices.
//  * Epilogue: x += acc, the next norm's f16 operand (into xn, whose rows this tile has
//    already read), and each token's sums of x^2 per 64 columns.  A 64-column group spans two
//    waves, so the per-lane partial sums go through an LDS table and are added in the order of
//    the batched epilogue.
// The weights are read from L2 by every workgroup (2.65 MB per layer, resident in each XCD's L2);
// nothing is written but x, the operand and the records.
#include "common.hpp"
#include "epilogue.hpp"
#include "q4k.hpp"

namespace {

constexpr int FD = 768;            // d_model (D); the host checks it
constexpr int KD = FD / 32;        // 32-wide K blocks of the token operand
constexpr int TM = 64, TB = TM / 16;
constexpr int NW = 8;
constexpr int SL = 256;            // d_ff columns per slice (one Q4_K block of each Wo row)
constexpr int RB2 = FD / 16 / NW;  // Wo row blocks per wave in phase 2 (6)
constexpr int GROUPS = FD / 64;    // norm record slots per token (12)
static_assert(SL == 32 * NW && SL == QK_K && FD % (16 * NW) == 0 && FD % QK_K == 0, "tile shape");
// Buffer resource word 3 of a raw byte buffer on gfx9 (no format conversion, offsets in bytes).
constexpr int BUF_DW3 = 0x00020000;

// One MFMA A operand from 8 packed nibble bytes: the low nibbles (hi = 0, sub-block 2c of the
// chunk) or the high nibbles (hi = 1, sub-block 2c + 1), with deq4's arithmetic per value (fp8
// reading of the nibble, one fused multiply-add with the 2^9-scaled scale, one rounding to f16).
__device__ __forceinline__ h8 deq8(uint2 v, float s, float o, int hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  const uint32_t a = (hi ? v.x >> 4 : v.x) & 0x0f0f0f0fu, b = (hi ? v.y >> 4 : v.y) & 0x0f0f0f0fu;
  const f2 a01 = __builtin_amdgcn_cvt_pk_f32_fp8(a, false), a23 = __builtin_amdgcn_cvt_pk_f32_fp8(a, true);
  const f2 b01 = __builtin_amdgcn_cvt_pk_f32_fp8(b, false), b23 = __builtin_amdgcn_cvt_pk_f32_fp8(b, true);
  return h8{(_Float16)__builtin_fmaf(s, a01[0], -o), (_Float16)__builtin_fmaf(s, a01[1], -o),
            (_Float16)__builtin_fmaf(s, a23[0], -o), (_Float16)__builtin_fmaf(s, a23[1], -o),
            (_Float16)__builtin_fmaf(s, b01[0], -o), (_Float16)__builtin_fmaf(s, b01[1], -o),
            (_Float16)__builtin_fmaf(s, b23[0], -o), (_Float16)__builtin_fmaf(s, b23[1], -o)};
}

// Hidden-state operand position of (token t of a row block, slice column k in [0, 32) of one
// 32-wide K block): lane t + 16 (k / 8) holds columns 8 (k / 8) .. +7.
__device__ __forceinline__ int hpos(int t, int k) { return ((k >> 3) * 16 + t) * 8 + (k & 7); }

template <bool WO_F16>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2)))
void ffn_fused_kernel(t5k::FfnArgs p) {
  // token operand [TB][KD] blocks, then (after the last slice) the epilogue's record table
  __shared__ __attribute__((aligned(16))) _Float16 Xs[TB * KD * 512];
  __shared__ __attribute__((aligned(16))) _Float16 Hs[TB * (SL / 32) * 512];  // h of one slice
  // per token: the folded norm's factor rsqrt(mean(x^2) + eps) / s and the next operand scale
  __shared__ float Fs[TM], Sn[TM];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = blockIdx.x * TM;

  // ---- token operand into LDS: the tile's TB x KD blocks are contiguous in operand order ----
  {
    const _Float16* src = p.xn + (size_t)(m0 >> 4) * KD * 512;
#pragma unroll
    for (int i = 0; i < TB * KD / NW; i++) {
      const int ch = i * NW + wave;
      __builtin_amdgcn_global_load_lds(src + (size_t)ch * 512 + lane * 8, Xs + ch * 512, 16, 0, 0);
    }
  }
  // ---- the folded norm: lane l serves token m0 + l ----
  if (wave == 0) {
    float4 r[4];
    const float4* rs = reinterpret_cast<const float4*>(p.rec + (size_t)(m0 + lane) * 16);
#pragma unroll
    for (int i = 0; i < 4; i++) r[i] = rs[i];
    const float inv = norm_inv(r, FD, p.eps);
    const float snext = norm_operand_scale(inv);
    Fs[lane] = inv / r[3].w;
    Sn[lane] = snext;
    // the next producer's operand scale (the batched gate|up's tiles at column 0 store it)
    if (m0 + lane < p.M) p.rec_out[(size_t)(m0 + lane) * 16 + 15] = snext;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // Weights through buffer resources: the lane's part of an address (its row within a row block,
  // its 8 bytes of nibbles) is one VGPR offset for the whole kernel, the rest a scalar offset.
  constexpr int rowb1 = (FD / QK_K) * Q4K_BYTES;  // bytes per W0 / W1 row
  const int rowbo = WO_F16 ? 2 * p.F : (p.F / QK_K) * Q4K_BYTES;  // bytes per Wo row
  const __amdgpu_buffer_rsrc_t rw0 = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.W0), (short)0, p.F * rowb1, BUF_DW3);
  const __amdgpu_buffer_rsrc_t rw1 = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.W1), (short)0, p.F * rowb1, BUF_DW3);
  const __amdgpu_buffer_rsrc_t rwo = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.Wo), (short)0, FD * rowbo, BUF_DW3);
  const int vh1 = lr * rowb1, vq1 = vh1 + 16 + 8 * lg;                       // W0 / W1: header, nibbles
  const int vho = lr * rowbo, vqo = vho + (WO_F16 ? 16 * lg : 16 + 8 * lg);  // Wo
  f4 o[RB2][TB];
#pragma unroll
  for (int r = 0; r < RB2; r++)
#pragma unroll
    for (int t = 0; t < TB; t++) o[r][t] = f4{0.f, 0.f, 0.f, 0.f};

  const int nslice = p.F / SL;
  for (int sl = 0; sl < nslice; sl++) {
    // ------------------------------ phase 1: gate | up ------------------------------
    // row blocks 0, 1: W0 rows n0 + 16 j + lr; 2, 3: the same rows of W1
    const int n0 = sl * SL + 32 * wave;
    f4 acc[4][TB];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int t = 0; t < TB; t++) acc[j][t] = f4{0.f, 0.f, 0.f, 0.f};
    // Raw weights of step ks + 1 are loaded while step ks is unpacked and multiplied.
    auto load_step = [&](int ks, uint4 (&hd)[4], uint2 (&q)[4]) {
      const int kb = ks >> 2, c = ks & 3;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int so = (n0 + 16 * (j & 1)) * rowb1 + kb * Q4K_BYTES;
        hd[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(j < 2 ? rw0 : rw1, vh1, so, 0));
        const auto qv = __builtin_amdgcn_raw_buffer_load_b64(j < 2 ? rw0 : rw1, vq1, so + 32 * c, 0);
        q[j] = make_uint2(qv[0], qv[1]);
      }
    };
    uint4 hd[4];
    uint2 q[4];
    load_step(0, hd, q);
    for (int ks = 0; ks < FD / 64; ks++) {
      const int c = ks & 3;
      float sc[4][4];  // per row block: the chunk's two (scale, min) pairs
      uint2 qc[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        chunk_scales(hd[j], c, sc[j][0], sc[j][1], sc[j][2], sc[j][3]);
        qc[j] = q[j];
      }
      if (ks + 1 < FD / 64) load_step(ks + 1, hd, q);
#pragma unroll
      for (int s = 0; s < 2; s++) {
        h8 a[4];
#pragma unroll
        for (int j = 0; j < 4; j++) a[j] = deq8(qc[j], sc[j][2 * s], sc[j][2 * s + 1], s);
#pragma unroll
        for (int t = 0; t < TB; t++) {
          const h8 b = *reinterpret_cast<const h8*>(Xs + (t * KD + 2 * ks + s) * 512 + lane * 8);
#pragma unroll
          for (int j = 0; j < 4; j++) acc[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j], b, acc[j][t], 0, 0, 0);
        }
      }
    }
    // every wave has finished reading the previous slice's h
    __syncthreads();
    // folded norm factor, gelu(gate) * up -> h columns 32 wave + 16 j + 4 lg .. +3 of the slice
#pragma unroll
    for (int t = 0; t < TB; t++) {
      const float f = Fs[16 * t + lr];
#pragma unroll
      for (int j = 0; j < 4; j++) acc[j][t] *= f;
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const f4 g = acc[j][t], u = acc[j + 2][t];
        *reinterpret_cast<h4*>(Hs + (t * (SL / 32) + wave) * 512 + hpos(lr, 16 * j + 4 * lg)) =
            h4{(_Float16)(gelu_tanh_dev(g[0]) * u[0]), (_Float16)(gelu_tanh_dev(g[1]) * u[1]),
               (_Float16)(gelu_tanh_dev(g[2]) * u[2]), (_Float16)(gelu_tanh_dev(g[3]) * u[3])};
      }
    }
    __syncthreads();

    // --------------------------- phase 2: wo over this slice ---------------------------
    // row blocks r: Wo rows (output columns) 96 wave + 16 r + lr; K = the slice's 256 columns
    // (one Q4_K block per row)
#pragma unroll
    for (int ks = 0; ks < SL / 64; ks++) {
      h8 b[2][TB];
#pragma unroll
      for (int s = 0; s < 2; s++)
#pragma unroll
        for (int t = 0; t < TB; t++)
          b[s][t] = *reinterpret_cast<const h8*>(Hs + (t * (SL / 32) + 2 * ks + s) * 512 + lane * 8);
#pragma unroll
      for (int r = 0; r < RB2; r++) {
        const int nb = RB2 * 16 * wave + 16 * r;  // the row block's first row
        h8 a[2];
        if constexpr (WO_F16) {
          const int so = nb * rowbo + 2 * (sl * SL + 64 * ks);
          a[0] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rwo, vqo, so, 0));
          a[1] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rwo, vqo, so + 64, 0));
        } else {
          const int so = nb * rowbo + sl * Q4K_BYTES;
          const uint4 hv = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rwo, vho, so, 0));
          const auto qv = __builtin_amdgcn_raw_buffer_load_b64(rwo, vqo, so + 32 * ks, 0);
          float s0, o0, s1, o1;
          chunk_scales(hv, ks, s0, o0, s1, o1);
          a[0] = deq8(make_uint2(qv[0], qv[1]), s0, o0, 0);
          a[1] = deq8(make_uint2(qv[0], qv[1]), s1, o1, 1);
        }
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
          for (int t = 0; t < TB; t++) o[r][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[s], b[s][t], o[r][t], 0, 0, 0);
      }
    }
  }

  // ---------------------------------- epilogue ----------------------------------
  // lane (lr, lg) of block (r, t): token m0 + 16 t + lr, columns 96 wave + 16 r + 4 lg .. +3
  float* Qt = reinterpret_cast<float*>(Xs);  // [TM][FD / 16][4] quad sums of x^2
  const bool fold = p.nx != nullptr;
  __syncthreads();  // Xs is free: every wave is past its last phase-1 read
#pragma unroll
  for (int t = 0; t < TB; t++) {
    const int m = m0 + 16 * t + lr;
    const float s = Sn[16 * t + lr];
#pragma unroll
    for (int r = 0; r < RB2; r++) {
      const int n = RB2 * 16 * wave + 16 * r + 4 * lg;
      float4 xv = *reinterpret_cast<const float4*>(p.x + (size_t)m * FD + n);
      xv.x += o[r][t][0];
      xv.y += o[r][t][1];
      xv.z += o[r][t][2];
      xv.w += o[r][t][3];
      if (fold) Qt[((16 * t + lr) * (FD / 16) + RB2 * wave + r) * 4 + lg] = quad_sq(xv);
      if (m < p.M) {
        *reinterpret_cast<float4*>(p.x + (size_t)m * FD + n) = xv;
        if (fold) {
          const float4 g = *reinterpret_cast<const float4*>(p.ngamma + n);
          *reinterpret_cast<h4*>(p.nx + tiled_index(m, n, FD)) =
              h4{(_Float16)((xv.x * g.x) * s), (_Float16)((xv.y * g.y) * s), (_Float16)((xv.z * g.z) * s),
                 (_Float16)((xv.w * g.w) * s)};
        }
      }
    }
  }
  if (!fold) return;
  __syncthreads();
  // record slot G of token t: per lane group the 4 row blocks of the group in order, then the
  // lane groups as (0 + 1) + (2 + 3) -- the batched epilogue's sums and cross-lane adds
  for (int i = tid; i < TM * GROUPS; i += 64 * NW) {
    const int t = i / GROUPS, G = i % GROUPS, m = m0 + t;
    float sg[4];
#pragma unroll
    for (int l = 0; l < 4; l++) {
      const float* q = Qt + ((size_t)t * (FD / 16) + 4 * G) * 4 + l;
      sg[l] = ((q[0] + q[4]) + q[8]) + q[12];
    }
    if (m < p.M) p.rec_out[(size_t)m * 16 + G] = (sg[0] + sg[1]) + (sg[2] + sg[3]);
  }
}

}  // namespace

namespace t5k {
hipError_t launch_ffn_fused(const FfnArgs& a, int wo_fmt, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (a.D != FD || a.F <= 0 || a.F % SL || !a.xn || !a.W0 || !a.W1 || !a.Wo || !a.x || !a.rec || !a.rec_out)
    return hipErrorInvalidValue;
  if (a.nx && !a.ngamma) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((a.M + TM - 1) / TM));
  if (wo_fmt == WF_F16) T5K_LAUNCH(ffn_fused_kernel<true>, grid, dim3(64 * NW), 0, s, a);
  else if (wo_fmt == WF_Q4K) T5K_LAUNCH(ffn_fused_kernel<false>, grid, dim3(64 * NW), 0, s, a);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}
}  // namespace t5k
