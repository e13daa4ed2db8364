// k_gemm.hip -- Q4_K dequant-GEMM on CDNA4 MFMA (v_mfma_f32_16x16x32_f16).
//
// C[M,N] = A[M,K] . W[N,K]^T, A = f16 activations (tokens x features), W = Q4_K
// super-blocks (or f16).  Reference: every linear of the encoder, candle QMatMul /
// f32 matmul (src/quantized_t5.rs:383-424 QKV, :501 O, :231-252 FFN, :700 projection).
//
// Workgroup = MW wave64s stacked along M; tile BM = 64*MW tokens x BN = 128 or 64 weight rows,
// K stepped by 64 (one Q4_K chunk: sub-blocks 2c and 2c+1 of every row).
//  * B (weights): each K step the workgroup reads, per weight row, the 16-byte Q4_K header
//    (d, dmin, 12 scale bytes) and 32 bytes of packed nibbles, dequantizes them with f32
//    scale/min math (one rounding to f16 per value) and stores the 128x64 f16 tile in LDS,
//    double-buffered.  Every wave consumes the whole tile, so the dequantization is
//    amortised over BM tokens.
//  * A (activations): each wave owns 64 rows and streams them straight from global memory
//    into VGPRs -- no LDS round trip.  A lane of lane-group g reads 32 contiguous bytes
//    (K = 16g .. 16g+15) of its row, so the 4 lane groups cover one 128-byte line per row.
//    MFMA step s (of 2) uses K = 16g + 8s + 0..7; the B fragments are read from LDS with
//    the same K order, so the product is the plain dot product.
//  * Each wave holds 64 x BN f32 accumulators (4 x BN/16 blocks of 16x16).
//  * Tiles are ordered so that each XCD (8 per device, workgroups dealt round-robin) works
//    on a contiguous band of M tiles: its L2 holds the A rows it streams plus the weights.
#include "common.hpp"

namespace {

constexpr int BK = 64, LDSK = BK + 8;  // +16 B row pad: conflict-free b128 reads

__device__ __forceinline__ int sbyte(const uint4& hd, int i) {
  // byte i (0..11) of the 12 packed scale bytes = header bytes 4..15
  const uint32_t w = i < 4 ? hd.y : (i < 8 ? hd.z : hd.w);
  return (int)((w >> (8 * (i & 3))) & 0xff);
}

// GGML get_scale_min_k4 for the chunk pair (2c, 2c+1); c is wave-uniform.
__device__ __forceinline__ void chunk_scales(const uint4& hd, int c, float& s0, float& o0, float& s1,
                                             float& o1) {
  const float d = f16_bits_to_f32(hd.x & 0xffff), dmin = f16_bits_to_f32(hd.x >> 16);
  int sc0, m0, sc1, m1;
  const int j0 = 2 * c, j1 = 2 * c + 1;
  if (c < 2) {
    sc0 = sbyte(hd, j0) & 63;
    m0 = sbyte(hd, j0 + 4) & 63;
    sc1 = sbyte(hd, j1) & 63;
    m1 = sbyte(hd, j1 + 4) & 63;
  } else {
    sc0 = (sbyte(hd, j0 + 4) & 15) | ((sbyte(hd, j0 - 4) >> 6) << 4);
    m0 = (sbyte(hd, j0 + 4) >> 4) | ((sbyte(hd, j0) >> 6) << 4);
    sc1 = (sbyte(hd, j1 + 4) & 15) | ((sbyte(hd, j1 - 4) >> 6) << 4);
    m1 = (sbyte(hd, j1 + 4) >> 4) | ((sbyte(hd, j1) >> 6) << 4);
  }
  s0 = d * (float)sc0;
  o0 = dmin * (float)m0;
  s1 = d * (float)sc1;
  o1 = dmin * (float)m1;
}

// Dequantize 4 packed bytes (8 nibbles) -> 4 low-nibble and 4 high-nibble f16 values.
__device__ __forceinline__ void deq4(uint32_t v, float s0, float o0, float s1, float o1, h4& lo, h4& hi) {
  const uint32_t l = v & 0x0f0f0f0fu, h = (v >> 4) & 0x0f0f0f0fu;
  lo = h4{(_Float16)(s0 * (float)(l & 0xff) - o0), (_Float16)(s0 * (float)((l >> 8) & 0xff) - o0),
          (_Float16)(s0 * (float)((l >> 16) & 0xff) - o0), (_Float16)(s0 * (float)(l >> 24) - o0)};
  hi = h4{(_Float16)(s1 * (float)(h & 0xff) - o1), (_Float16)(s1 * (float)((h >> 8) & 0xff) - o1),
          (_Float16)(s1 * (float)((h >> 16) & 0xff) - o1), (_Float16)(s1 * (float)(h >> 24) - o1)};
}

template <int EPI, int BN>
__device__ __forceinline__ void brow(int r, int n0, const GemmArgs& p, const void*& W, int& n) {
  if (EPI == EPI_GATED) {  // rows [0,BN/2): W0 columns n0.., rows [BN/2,BN): W1 same columns
    W = r < BN / 2 ? p.W0 : p.W1;
    n = n0 + (r & (BN / 2 - 1));
  } else {
    W = p.W0;
    n = n0 + r;
  }
}

// Raw B data of one K step held in registers between the global load and the LDS store.
template <int WF, int NT, int BN>
struct BRaw {
  static constexpr int TPR = NT / BN;           // threads per weight row (Q4_K)
  static constexpr int BPT = 32 / TPR;          // nibble bytes per thread
  static constexpr int F16_LOADS = BN * BK * 2 / 16 / NT;
  uint4 hd;
  uint32_t q[BPT / 4];
  uint4 f[WF == WF_F16 ? F16_LOADS : 1];
};

template <int EPI, int WF, int NT, int BN>
__device__ __forceinline__ void load_b(BRaw<WF, NT, BN>& br, const GemmArgs& p, int n0, int kt, int tid) {
  using R = BRaw<WF, NT, BN>;
  if (WF == WF_Q4K) {
    const int r = tid / R::TPR, part = tid % R::TPR;
    const void* W;
    int n;
    brow<EPI, BN>(r, n0, p, W, n);
    const int kb = (kt * BK) / QK_K, c = ((kt * BK) % QK_K) / 64;
    const uint8_t* blk = (const uint8_t*)W + ((size_t)n * (p.K / QK_K) + kb) * Q4K_BYTES;
    br.hd = *reinterpret_cast<const uint4*>(blk);
    const uint8_t* qs = blk + 16 + 32 * c + part * R::BPT;
    if constexpr (R::BPT == 32) {
      const uint4 a = *reinterpret_cast<const uint4*>(qs), b = *reinterpret_cast<const uint4*>(qs + 16);
      br.q[0] = a.x; br.q[1] = a.y; br.q[2] = a.z; br.q[3] = a.w;
      br.q[4] = b.x; br.q[5] = b.y; br.q[6] = b.z; br.q[7] = b.w;
    } else if constexpr (R::BPT == 16) {
      const uint4 a = *reinterpret_cast<const uint4*>(qs);
      br.q[0] = a.x; br.q[1] = a.y; br.q[2] = a.z; br.q[3] = a.w;
    } else {
      const uint2 a = *reinterpret_cast<const uint2*>(qs);
      br.q[0] = a.x; br.q[1] = a.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < R::F16_LOADS; i++) {
      const int idx = i * NT + tid, r = idx >> 3, c8 = (idx & 7) * 8;
      const void* W;
      int n;
      brow<EPI, BN>(r, n0, p, W, n);
      br.f[i] = *reinterpret_cast<const uint4*>((const _Float16*)W + (size_t)n * p.K + kt * BK + c8);
    }
  }
}

template <int WF, int NT, int BN>
__device__ __forceinline__ void store_b(const BRaw<WF, NT, BN>& br, _Float16* Bs, int kt, int tid) {
  using R = BRaw<WF, NT, BN>;
  if (WF == WF_Q4K) {
    const int r = tid / R::TPR, part = tid % R::TPR;
    const int c = ((kt * BK) % QK_K) / 64;
    float s0, o0, s1, o1;
    chunk_scales(br.hd, c, s0, o0, s1, o1);
    _Float16* row = Bs + r * LDSK;
#pragma unroll
    for (int w = 0; w < R::BPT / 4; w++) {
      h4 lo, hi;
      deq4(br.q[w], s0, o0, s1, o1, lo, hi);
      *reinterpret_cast<h4*>(row + part * R::BPT + 4 * w) = lo;
      *reinterpret_cast<h4*>(row + 32 + part * R::BPT + 4 * w) = hi;
    }
  } else {
#pragma unroll
    for (int i = 0; i < R::F16_LOADS; i++) {
      const int idx = i * NT + tid, r = idx >> 3, c8 = (idx & 7) * 8;
      *reinterpret_cast<uint4*>(Bs + r * LDSK + c8) = br.f[i];
    }
  }
}

template <int EPI, int WF, int MW, int BN>
__global__ __launch_bounds__(64 * MW) __attribute__((amdgpu_waves_per_eu(2))) void gemm_kernel(GemmArgs p, int tiles_m, int tiles_n) {
  constexpr int NT = 64 * MW, BM = 64 * MW, NB = BN / 16;
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN * LDSK];

  // XCD-aware tile order: block b runs on XCD b % 8; give each XCD a contiguous tile range.
  const int per_xcd = gridDim.x / 8;
  const int tile = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (tile >= tiles_m * tiles_n) return;
  const int tm = tile / tiles_n, tn = tile % tiles_n;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int m0 = tm * BM;
  const int n0 = tn * (EPI == EPI_GATED ? BN / 2 : BN);
  const int nkt = p.K / BK;

  const _Float16* arow[4];
#pragma unroll
  for (int mb = 0; mb < 4; mb++) arow[mb] = p.A + (size_t)(m0 + wave * 64 + mb * 16 + lr) * p.lda + 16 * lg;

  f4 acc[4][NB];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < NB; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  uint4 a0[4][2], a1[4][2];
  BRaw<WF, NT, BN> br;

#define LOAD_A(dst, kt)                                                                     \
  _Pragma("unroll") for (int mb = 0; mb < 4; mb++) {                                        \
    dst[mb][0] = *reinterpret_cast<const uint4*>(arow[mb] + (kt) * BK);                     \
    dst[mb][1] = *reinterpret_cast<const uint4*>(arow[mb] + (kt) * BK + 8);                 \
  }
#define COMPUTE(areg, buf)                                                                  \
  _Pragma("unroll") for (int s = 0; s < 2; s++) {                                           \
    h8 bf[NB];                                                                              \
    _Pragma("unroll") for (int nb = 0; nb < NB; nb++) bf[nb] =                              \
        *reinterpret_cast<const h8*>(&Bs[buf][(nb * 16 + lr) * LDSK + 16 * lg + 8 * s]);    \
    _Pragma("unroll") for (int mb = 0; mb < 4; mb++) {                                      \
      const h8 af = __builtin_bit_cast(h8, areg[mb][s]);                                    \
      _Pragma("unroll") for (int nb = 0; nb < NB; nb++) acc[mb][nb] =                       \
          __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[nb], acc[mb][nb], 0, 0, 0);         \
    }                                                                                       \
  }

  load_b<EPI, WF, NT, BN>(br, p, n0, 0, tid);
  LOAD_A(a0, 0);
  store_b<WF, NT, BN>(br, Bs[0], 0, tid);
  __syncthreads();
  // Drain every counter once here: otherwise the prologue's A loads are still pending at
  // the loop header, and the wait that covers them lands inside the loop body, where in
  // steady state it would stall each step on the *next* step's prefetch.
  __builtin_amdgcn_s_waitcnt(0);

  // One MFMA site per iteration keeps the accumulators in place (no AGPR<->VGPR copies);
  // the next step's A and B are in flight while this step's MFMAs run.
  for (int kt = 0; kt < nkt; kt++) {
    const int buf = kt & 1;
    const bool more = kt + 1 < nkt;
    if (more) {  // B first: store_b below then waits only for the B loads
      load_b<EPI, WF, NT, BN>(br, p, n0, kt + 1, tid);
      LOAD_A(a1, kt + 1);
    }
    COMPUTE(a0, buf);
    if (more) store_b<WF, NT, BN>(br, Bs[buf ^ 1], kt + 1, tid);
    __syncthreads();
#pragma unroll
    for (int mb = 0; mb < 4; mb++) {
      a0[mb][0] = a1[mb][0];
      a0[mb][1] = a1[mb][1];
    }
  }
#undef LOAD_A
#undef COMPUTE

  // ---- epilogue: lane holds D[row 4*lg+i][col lr] of each 16x16 block ----
  const int rbase = m0 + wave * 64 + lg * 4;
  if (EPI == EPI_GATED) {
    _Float16* out = (_Float16*)p.out;
#pragma unroll
    for (int mb = 0; mb < 4; mb++)
#pragma unroll
      for (int nb = 0; nb < NB / 2; nb++) {
        const int n = n0 + nb * 16 + lr;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int m = rbase + mb * 16 + i;
          if (m < p.M) out[(size_t)m * p.ldo + n] = (_Float16)(gelu_tanh_dev(acc[mb][nb][i]) * acc[mb][nb + NB / 2][i]);
        }
      }
  } else {
#pragma unroll
    for (int mb = 0; mb < 4; mb++)
#pragma unroll
      for (int nb = 0; nb < NB; nb++) {
        const int n = n0 + nb * 16 + lr;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int m = rbase + mb * 16 + i;
          if (m >= p.M) continue;
          const float v = acc[mb][nb][i];
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

template <int EPI, int WF, int BN>
hipError_t launch_cfg(int mw, const GemmArgs& a, hipStream_t s) {
  const int cols = EPI == EPI_GATED ? BN / 2 : BN;
  const int tiles_n = a.N / cols, tiles_m = (a.M + 64 * mw - 1) / (64 * mw);
  const int grid = (tiles_m * tiles_n + 7) / 8 * 8;
  switch (mw) {
    case 2: hipLaunchKernelGGL((gemm_kernel<EPI, WF, 2, BN>), dim3(grid), dim3(128), 0, s, a, tiles_m, tiles_n); break;
    case 4: hipLaunchKernelGGL((gemm_kernel<EPI, WF, 4, BN>), dim3(grid), dim3(256), 0, s, a, tiles_m, tiles_n); break;
    default: hipLaunchKernelGGL((gemm_kernel<EPI, WF, 8, BN>), dim3(grid), dim3(512), 0, s, a, tiles_m, tiles_n); break;
  }
  return hipGetLastError();
}

template <int EPI>
hipError_t launch_epi(int wfmt, int mw, int bn, const GemmArgs& a, hipStream_t s) {
  if (wfmt == WF_Q4K)
    return bn == 64 ? launch_cfg<EPI, WF_Q4K, 64>(mw, a, s) : launch_cfg<EPI, WF_Q4K, 128>(mw, a, s);
  return bn == 64 ? launch_cfg<EPI, WF_F16, 64>(mw, a, s) : launch_cfg<EPI, WF_F16, 128>(mw, a, s);
}

}  // namespace

namespace t5k {
// Tile choice for C[M, N]: rows 64*mw (mw in {2, 4, 8}) x bn weight rows (64 or 128).
// Measured on MI355X for every encoder GEMM (N = 128..4096, K = 768/2048, M = 32..73728):
// the 4-wave x 128-row tile is fastest once it yields >= 1.4 tiles per CU; below that the
// 4-wave x 64-row tile while it still covers >= 0.75 of the CUs; otherwise 2-wave x 64-row
// tiles (small token counts, where latency dominates).  n_rows = weight rows of the launch
// (both matrices for the gated FFN).
void gemm_pick_tile(int M, int n_rows, int cus, int& mw, int& bn) {
  auto tiles = [&](int w, int b) { return (double)((M + 64 * w - 1) / (64 * w)) * (n_rows / b); };
  if (n_rows % 128 == 0 && tiles(4, 128) >= 1.4 * cus) {
    mw = 4;
    bn = 128;
  } else if (tiles(4, 64) >= 0.75 * cus) {
    mw = 4;
    bn = 64;
  } else {
    mw = 2;
    bn = 64;
  }
}

hipError_t launch_gemm(int epi, int wfmt, int mw, int bn, const GemmArgs& a, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  switch (epi) {
    case EPI_F16: return launch_epi<EPI_F16>(wfmt, mw, bn, a, s);
    case EPI_RESID: return launch_epi<EPI_RESID>(wfmt, mw, bn, a, s);
    case EPI_GATED: return launch_epi<EPI_GATED>(wfmt, mw, bn, a, s);
    case EPI_F32: return launch_epi<EPI_F32>(wfmt, mw, bn, a, s);
    case EPI_QKV: return launch_epi<EPI_QKV>(wfmt, mw, bn, a, s);
    case EPI_RELU: return launch_epi<EPI_RELU>(wfmt, mw, bn, a, s);
  }
  return hipErrorInvalidValue;
}
}  // namespace t5k
