// k_gemm.hip -- Q4_K dequant-GEMM on CDNA4 MFMA (v_mfma_f32_16x16x32_f16).
//
// C[M,N] = A[M,K] . W[N,K]^T, A = f16 activations (tokens x features), W = Q4_K
// super-blocks (or f16).  Reference: every linear of the encoder, candle QMatMul /
// f32 matmul (src/quantized_t5.rs:383-424 QKV, :501 O, :231-252 FFN, :700 projection).
//
// Workgroup: 256 threads = 4 wave64s in a 2x2 grid, tile BM=128 x BN=128 x BK=64.
// Each wave owns a 64x64 sub-tile = 4x4 MFMA 16x16 blocks (64 f32 accumulators/lane).
// Per K step of 64 the workgroup:
//   - reads the A tile (128 rows x 128 B f16) with 16-byte coalesced loads,
//   - reads for each of its 128 weight rows the 16-byte Q4_K header (d, dmin, scales)
//     and 32 bytes of packed nibbles (one 64-value chunk = sub-blocks 2c and 2c+1),
//   - dequantizes nibbles to f16 (f32 scale/min math, then one rounding) into LDS,
//   - runs 2 x 16 MFMAs per wave out of LDS.
// Global loads for step k+1 are issued before the MFMAs of step k (register double
// buffer) and the LDS tiles are double-buffered, so one barrier per step suffices.
#include "common.hpp"

namespace {

constexpr int BM = 128, BN = 128, BK = 64, LDSK = BK + 8;  // +16 B row pad vs bank conflicts

__device__ __forceinline__ void scale_min_u32(uint32_t s0, uint32_t s1, uint32_t s2, int j, int& sc,
                                              int& m) {
  // scales[12] packed in three little-endian dwords s0 (bytes 0-3), s1 (4-7), s2 (8-11).
  auto byte = [&](int i) -> int {
    const uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
    return (int)((w >> (8 * (i & 3))) & 0xff);
  };
  if (j < 4) {
    sc = byte(j) & 63;
    m = byte(j + 4) & 63;
  } else {
    sc = (byte(j + 4) & 15) | ((byte(j - 4) >> 6) << 4);
    m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
  }
}

// Map a B-tile row to (weight matrix, output column).  For the gated epilogue the
// 128 tile rows interleave W0 and W1 so that each wave holds the gate and the up
// projection of the same 32 columns: wave column wn covers tile rows [64wn, 64wn+64),
// MFMA blocks ni=0,1 are W0 columns and ni=2,3 the same W1 columns.
template <int EPI>
__device__ __forceinline__ void brow_map(int r, int n0, int& mat, int& n) {
  if (EPI == EPI_GATED) {
    const int wn = r >> 6, ni = (r >> 4) & 3, c = r & 15;
    mat = ni >> 1;
    n = n0 + wn * 32 + (ni & 1) * 16 + c;
  } else {
    mat = 0;
    n = n0 + r;
  }
}

template <int EPI, int WF>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * LDSK];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN * LDSK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * (EPI == EPI_GATED ? BN / 2 : BN);
  const int K = p.K;
  const int nkt = K / BK;

  // ---- A tile loader: 4 x 16 B per thread ----
  const _Float16* Ag = p.A + (size_t)m0 * p.lda;
  uint4 areg[4];
  auto load_a = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = i * 32 + (tid >> 3), c = (tid & 7) * 8;
      areg[i] = *reinterpret_cast<const uint4*>(Ag + (size_t)r * p.lda + kt * BK + c);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = i * 32 + (tid >> 3), c = (tid & 7) * 8;
      *reinterpret_cast<uint4*>(&As[buf][r * LDSK + c]) = areg[i];
    }
  };

  // ---- B tile loader ----
  // Q4_K: thread -> (row r = tid/2, half h = tid%2): header 16 B + 16 B of nibbles.
  // f16:  same pattern as A (4 x 16 B per thread).
  uint4 breg[4];
  const int kblocks = K / QK_K;
  auto load_b = [&](int kt) {
    if (WF == WF_Q4K) {
      const int r = tid >> 1, h = tid & 1;
      int mat, n;
      brow_map<EPI>(r, n0, mat, n);
      const uint8_t* W = (const uint8_t*)(mat ? p.W1 : p.W0);
      const int kb = (kt * BK) / QK_K, chunk = ((kt * BK) % QK_K) / 64;
      const uint8_t* blk = W + ((size_t)n * kblocks + kb) * Q4K_BYTES;
      breg[0] = *reinterpret_cast<const uint4*>(blk);
      breg[1] = *reinterpret_cast<const uint4*>(blk + 16 + 32 * chunk + 16 * h);
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = i * 32 + (tid >> 3), c = (tid & 7) * 8;
        int mat, n;
        brow_map<EPI>(r, n0, mat, n);
        const _Float16* W = (const _Float16*)(mat ? p.W1 : p.W0);
        breg[i] = *reinterpret_cast<const uint4*>(W + (size_t)n * K + kt * BK + c);
      }
    }
  };
  auto store_b = [&](int buf, int kt) {
    if (WF == WF_Q4K) {
      const int r = tid >> 1, h = tid & 1;
      const int chunk = ((kt * BK) % QK_K) / 64;
      const uint4 hd = breg[0];
      const float d = f16_bits_to_f32(hd.x & 0xffff), dmin = f16_bits_to_f32(hd.x >> 16);
      int sc0, mn0, sc1, mn1;
      scale_min_u32(hd.y, hd.z, hd.w, 2 * chunk, sc0, mn0);
      scale_min_u32(hd.y, hd.z, hd.w, 2 * chunk + 1, sc1, mn1);
      const float s0 = d * (float)sc0, o0 = dmin * (float)mn0;
      const float s1 = d * (float)sc1, o1 = dmin * (float)mn1;
      const uint32_t q[4] = {breg[1].x, breg[1].y, breg[1].z, breg[1].w};
      h8 lo[2], hi[2];
#pragma unroll
      for (int w = 0; w < 4; w++) {
#pragma unroll
        for (int bb = 0; bb < 4; bb++) {
          const uint32_t byte = (q[w] >> (8 * bb)) & 0xff;
          const int e = w * 4 + bb;  // 0..15
          lo[e >> 3][e & 7] = (_Float16)(s0 * (float)(byte & 15) - o0);
          hi[e >> 3][e & 7] = (_Float16)(s1 * (float)(byte >> 4) - o1);
        }
      }
      _Float16* row = &Bs[buf][r * LDSK];
      *reinterpret_cast<h8*>(row + 16 * h) = lo[0];
      *reinterpret_cast<h8*>(row + 16 * h + 8) = lo[1];
      *reinterpret_cast<h8*>(row + 32 + 16 * h) = hi[0];
      *reinterpret_cast<h8*>(row + 32 + 16 * h + 8) = hi[1];
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = i * 32 + (tid >> 3), c = (tid & 7) * 8;
        *reinterpret_cast<uint4*>(&Bs[buf][r * LDSK + c]) = breg[i];
      }
    }
  };

  f4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  load_a(0);
  load_b(0);
  store_a(0);
  store_b(0, 0);
  __syncthreads();

  const int lr = lane & 15, lk = (lane >> 4) * 8;
  for (int kt = 0; kt < nkt; kt++) {
    const int buf = kt & 1;
    if (kt + 1 < nkt) {
      load_a(kt + 1);
      load_b(kt + 1);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      h8 a[4], b[4];
#pragma unroll
      for (int mi = 0; mi < 4; mi++)
        a[mi] = *reinterpret_cast<const h8*>(&As[buf][(wm * 64 + mi * 16 + lr) * LDSK + ks * 32 + lk]);
#pragma unroll
      for (int ni = 0; ni < 4; ni++)
        b[ni] = *reinterpret_cast<const h8*>(&Bs[buf][(wn * 64 + ni * 16 + lr) * LDSK + ks * 32 + lk]);
#pragma unroll
      for (int mi = 0; mi < 4; mi++)
#pragma unroll
        for (int ni = 0; ni < 4; ni++)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mi], b[ni], acc[mi][ni], 0, 0, 0);
    }
    if (kt + 1 < nkt) {
      store_a(buf ^ 1);
      store_b(buf ^ 1, kt + 1);
    }
    __syncthreads();
  }

  // ---- epilogue: lane holds D[row 4*(lane/16)+i][col lane%16] of each 16x16 block ----
  const int rbase = m0 + wm * 64 + (lane >> 4) * 4;
  if (EPI == EPI_GATED) {
    _Float16* out = (_Float16*)p.out;
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
      for (int ni = 0; ni < 2; ni++) {
        const int n = n0 + wn * 32 + ni * 16 + lr;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int m = rbase + mi * 16 + i;
          if (m < p.M) {
            const float g = acc[mi][ni][i], u = acc[mi][ni + 2][i];
            out[(size_t)m * p.ldo + n] = (_Float16)(gelu_tanh_dev(g) * u);
          }
        }
      }
  } else {
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
      for (int ni = 0; ni < 4; ni++) {
        const int n = n0 + wn * 64 + ni * 16 + lr;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int m = rbase + mi * 16 + i;
          if (m >= p.M) continue;
          const float v = acc[mi][ni][i];
          if (EPI == EPI_F16) {
            ((_Float16*)p.out)[(size_t)m * p.ldo + n] = (_Float16)v;
          } else if (EPI == EPI_RELU) {
            ((_Float16*)p.out)[(size_t)m * p.ldo + n] = (_Float16)(v > 0.f ? v : 0.f);
          } else if (EPI == EPI_F32) {
            ((float*)p.out)[(size_t)m * p.ldo + n] = v;
          } else if (EPI == EPI_RESID) {
            float* x = (float*)p.out + (size_t)m * p.ldo + n;
            *x = *x + v;
          } else {  // EPI_QKV
            const int nn = n + p.n_off, inner = p.heads * p.dkv;
            const int which = nn / inner, rem = nn % inner;
            const int h = rem / p.dkv, d = rem % p.dkv;
            ((_Float16*)p.out)[(((size_t)which * p.heads + h) * p.tpad + m) * p.dkv + d] = (_Float16)v;
          }
        }
      }
  }
}

template <int EPI>
hipError_t launch_epi(int wfmt, const GemmArgs& a, hipStream_t s) {
  const int bn = EPI == EPI_GATED ? BN / 2 : BN;
  dim3 grid(a.N / bn, (a.M + BM - 1) / BM);
  if (wfmt == WF_Q4K)
    hipLaunchKernelGGL((gemm_kernel<EPI, WF_Q4K>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((gemm_kernel<EPI, WF_F16>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace

namespace t5k {
// Shapes are validated by the caller: N % 128 == 0 (N % 64 for gated), K % 256 == 0,
// A allocated with at least roundup(M, 128) rows.
hipError_t launch_gemm(int epi, int wfmt, const GemmArgs& a, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  switch (epi) {
    case EPI_F16: return launch_epi<EPI_F16>(wfmt, a, s);
    case EPI_RESID: return launch_epi<EPI_RESID>(wfmt, a, s);
    case EPI_GATED: return launch_epi<EPI_GATED>(wfmt, a, s);
    case EPI_F32: return launch_epi<EPI_F32>(wfmt, a, s);
    case EPI_QKV: return launch_epi<EPI_QKV>(wfmt, a, s);
    case EPI_RELU: return launch_epi<EPI_RELU>(wfmt, a, s);
  }
  return hipErrorInvalidValue;
}
}  // namespace t5k
