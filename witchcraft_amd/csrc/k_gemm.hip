// k_gemm.hip -- Q4_K dequant-GEMM on CDNA4 MFMA (v_mfma_f32_16x16x32_f16).
//
// C[M,N] = A[M,K] . W[N,K]^T, A = f16 activations (tokens x features), W = Q4_K
// super-blocks (or f16).  Reference: every linear of the encoder, candle QMatMul /
// f32 matmul (src/quantized_t5.rs:383-424 QKV, :501 O, :231-252 FFN, :700 projection).
//
// Warp-specialised workgroup: MW "math" wave64s + MW "producer" wave64s.  Waves are dealt
// to the CU's four SIMDs round-robin, so with MW = 4 every SIMD runs one math wave and one
// producer wave: the producer's global loads and nibble unpacking (VALU) issue while the
// math wave's MFMAs occupy the matrix core.
//  * Tile: BM = 64*MW tokens x BN weight rows (BN = 128 or 64), K stepped by 64 (one Q4_K
//    chunk = sub-blocks 2c and 2c+1 of each weight row).
//  * Producers: per K step, read each weight row's 16-byte Q4_K header (d, dmin, 12 scale
//    bytes) and 32 bytes of nibbles, dequantize with f32 scale/min math (one rounding to
//    f16 per value) and write the BN x 64 f16 stage into LDS (double-buffered).  The raw
//    bytes of step k+2 are in flight while step k+1 is unpacked.
//  * Math waves: each owns 64 token rows, streams them straight from global memory into
//    VGPRs one step ahead.  Activations are stored in MFMA operand order (tiled_index), so
//    each 16-row x 32-column operand is one contiguous 1 KiB dwordx4 load per wave.  They
//    run 4 x BN/16 MFMAs per 32-wide K slice with the weight fragment as the A operand:
//    D^T = W . X^T, so each lane ends up with 4 consecutive output columns of one token and
//    the epilogue stores 8-16 bytes at a time (f16 outputs that feed the next GEMM are
//    written in operand order too).
//  * One barrier per K step hands the LDS stage from producers to math waves.
//  * Tiles are ordered so that each XCD (8 per device, workgroups dealt round-robin) works
//    on a contiguous band of M tiles: its L2 holds the A rows it streams plus the weights.
#include "common.hpp"
#include "epilogue.hpp"
#include "q4k.hpp"

namespace {

// Weight stage rows of 64 halves in the swz64 layout, so the math waves' fragment reads (16 rows
// x 4 chunks per instruction) hit every bank once.
constexpr int BK = 64, LDSK = BK;
__device__ __forceinline__ int bswz(int r, int c) { return swz64(r, c); }

// B-tile row r -> (weight matrix, output column).  Gated: rows [0, BN/2) are W0 columns
// n0.., rows [BN/2, BN) the same W1 columns, so a math wave's N blocks nb < NB/2 (gate)
// and nb + NB/2 (up) hold the same output columns in the same lanes.
template <int EPI, int BN>
__device__ __forceinline__ void brow(int r, int n0, const GemmArgs& p, const void*& W, int& n) {
  if (EPI == EPI_GATED) {
    W = r < BN / 2 ? p.W0 : p.W1;
    n = n0 + (r & (BN / 2 - 1));
  } else {
    W = p.W0;
    n = n0 + r;
  }
}

// Raw weights of one K step held by a producer thread between load and unpack.  The f16
// chunks use a native vector type: arrays of HIP's uint4 (a union) in this ring are not
// promoted to registers and end up in scratch memory.
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
template <int WF, int NP, int BN>
struct BRaw {
  static constexpr int TPR = NP / BN;   // producer threads per weight row (Q4_K)
  static constexpr int BPT = 32 / TPR;  // nibble bytes per thread: 32, 16 or 8
  static constexpr int NQ = BPT / 4;
  static constexpr int F16_LOADS = BN * BK * 2 / 16 / NP;
  uint4 hd;
  uint32_t q[NQ];
  u4v f[WF == WF_F16 ? F16_LOADS : 1];
};

template <int EPI, int WF, int NP, int BN>
__device__ __forceinline__ void load_b(BRaw<WF, NP, BN>& br, const GemmArgs& p, int n0, int kt, int pt) {
  using R = BRaw<WF, NP, BN>;
  if constexpr (WF == WF_Q4K) {
    const int r = pt / R::TPR, part = pt % R::TPR;
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
      const int idx = i * NP + pt, r = idx >> 3, c8 = (idx & 7) * 8;
      const void* W;
      int n;
      brow<EPI, BN>(r, n0, p, W, n);
      br.f[i] = *reinterpret_cast<const u4v*>((const _Float16*)W + (size_t)n * p.K + kt * BK + c8);
    }
  }
}

template <int WF, int NP, int BN>
__device__ __forceinline__ void store_b(const BRaw<WF, NP, BN>& br, _Float16* Bs, int kt, int pt) {
  using R = BRaw<WF, NP, BN>;
  if constexpr (WF == WF_Q4K) {
    const int r = pt / R::TPR, part = pt % R::TPR;
    const int c = ((kt * BK) % QK_K) / 64;
    float s0, o0, s1, o1;
    chunk_scales(br.hd, c, s0, o0, s1, o1);
#pragma unroll
    for (int w = 0; w < R::NQ; w += 2) {
      h4 lo0, hi0, lo1, hi1;
      deq4(br.q[w], s0, o0, s1, o1, lo0, hi0);
      deq4(br.q[w + 1], s0, o0, s1, o1, lo1, hi1);
      *reinterpret_cast<h8*>(Bs + bswz(r, part * R::BPT + 4 * w)) =
          h8{lo0[0], lo0[1], lo0[2], lo0[3], lo1[0], lo1[1], lo1[2], lo1[3]};
      *reinterpret_cast<h8*>(Bs + bswz(r, 32 + part * R::BPT + 4 * w)) =
          h8{hi0[0], hi0[1], hi0[2], hi0[3], hi1[0], hi1[1], hi1[2], hi1[3]};
    }
  } else {
#pragma unroll
    for (int i = 0; i < R::F16_LOADS; i++) {
      const int idx = i * NP + pt, r = idx >> 3, c8 = (idx & 7) * 8;
      *reinterpret_cast<u4v*>(Bs + bswz(r, c8)) = br.f[i];
    }
  }
}

// Hybrid numerics (launch_gemm_hybrid): the stage holds the nibbles times their sub-block scale
// as two int8 planes.  A 6-bit scale splits as sc = 8 sh + sl (sh, sl <= 7), so sh q and sl q are
// at most 105 and fit int8: the hi plane holds sh q, the lo plane sl q, and a K block's integer
// sum is 8 (hi . q8) + (lo . q8), exact in int32.  Four nibbles masked into the bytes of a word
// times a scale <= 7 give all four products with one multiply (no byte carries into the next).
// Plane rows are 64 bytes (one K step); 16-byte chunk j of row r sits at chunk j ^ ((r >> 2) & 3),
// so the math waves' fragment reads (16 rows x one chunk) hit every bank once.  At the first K
// step of a 256-wide block the row's first producer thread also writes the block's d and dmin
// (Md) and its eight 6-bit mins as the A operand of the min-term MFMA (Mm: m0 m0 m1 m1 .. m7 m7,
// one per bsum).
// 16-token row blocks per math wave in a full hybrid tile (the tile is 16 HYB_MB MW tokens).
constexpr int HYB_MB = 3;
__device__ __forceinline__ int hyb_off(int r, int k) {  // byte offset of (row r, K index k) in a plane
  return r * 64 + ((((k >> 4) ^ (r >> 2)) & 3) << 4) + (k & 15);
}
template <int NP, int BN>
__device__ __forceinline__ void store_b_hybrid(const BRaw<WF_Q4K, NP, BN>& br, _Float16* Bs, float2* Md, h8* Mm,
                                               int kt, int pt) {
  using R = BRaw<WF_Q4K, NP, BN>;
  static_assert(R::BPT == 8 || R::BPT == 16 || R::BPT == 32, "nibble bytes per thread");
  const int r = pt / R::TPR, part = pt % R::TPR;
  const int c = ((kt * BK) % QK_K) / 64;
  const uint4 hd = br.hd;
  // get_scale_min_k4 on the 12 scale bytes (header words y, z, w); sub-blocks 2c, 2c + 1
  auto byte = [&](int i) -> int {
    const uint32_t w = i < 4 ? hd.y : (i < 8 ? hd.z : hd.w);
    return (int)((w >> (8 * (i & 3))) & 0xff);
  };
  auto scale_min = [&](int j, int& sc, int& m) {
    if (j < 4) {
      sc = byte(j) & 63;
      m = byte(j + 4) & 63;
    } else {
      sc = (byte(j + 4) & 15) | ((byte(j - 4) >> 6) << 4);
      m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
  };
  int sc0, m0, sc1, m1;
  scale_min(2 * c, sc0, m0);
  scale_min(2 * c + 1, sc1, m1);
  uint8_t* hi = reinterpret_cast<uint8_t*>(Bs);
  uint8_t* lo = hi + BN * 64;
  // nibble word w holds values k0 + 4w .. +3 of sub-block 2c (low nibbles) and of 2c + 1 (high)
  const int k0 = part * R::BPT;
#pragma unroll
  for (int w = 0; w < R::NQ; w += 2) {
    const uint32_t l0 = br.q[w] & 0x0f0f0f0fu, l1 = br.q[w + 1] & 0x0f0f0f0fu;
    const uint32_t h0 = (br.q[w] >> 4) & 0x0f0f0f0fu, h1 = (br.q[w + 1] >> 4) & 0x0f0f0f0fu;
    const int k = k0 + 4 * w;
    *reinterpret_cast<uint2*>(hi + hyb_off(r, k)) = make_uint2(l0 * (uint32_t)(sc0 >> 3), l1 * (uint32_t)(sc0 >> 3));
    *reinterpret_cast<uint2*>(lo + hyb_off(r, k)) = make_uint2(l0 * (uint32_t)(sc0 & 7), l1 * (uint32_t)(sc0 & 7));
    *reinterpret_cast<uint2*>(hi + hyb_off(r, 32 + k)) =
        make_uint2(h0 * (uint32_t)(sc1 >> 3), h1 * (uint32_t)(sc1 >> 3));
    *reinterpret_cast<uint2*>(lo + hyb_off(r, 32 + k)) =
        make_uint2(h0 * (uint32_t)(sc1 & 7), h1 * (uint32_t)(sc1 & 7));
  }
  if (c == 0 && part == 0) {
    Md[r] = make_float2(f16_bits_to_f32(hd.x & 0xffff), f16_bits_to_f32(hd.x >> 16));
    _Float16 mh[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      int sc, m;
      scale_min(j, sc, m);
      mh[j] = (_Float16)m;
    }
    Mm[2 * r] = h8{mh[0], mh[0], mh[1], mh[1], mh[2], mh[2], mh[3], mh[3]};
    Mm[2 * r + 1] = h8{mh[4], mh[4], mh[5], mh[5], mh[6], mh[6], mh[7], mh[7]};
  }
}

// QKV epilogue through LDS (d_kv = 64).  The accumulators give each lane 4 columns of one
// token, so direct stores into the head-major [3][H][tpad][64] layout write 16 x 32-byte
// pieces per instruction.  Instead each 16-token block is staged in this wave's LDS region
// (the weight stage, idle once the K loop has ended) and copied out as whole 128-byte head
// rows, 16 bytes per lane.  `stage` holds 16 rows of BN + 8 halves.  No wait is needed between
// the staging writes and reads: a wave's LDS instructions execute in order, and the compiler
// keeps the order of these possibly aliasing accesses.
template <int BN, int MB>
__device__ __forceinline__ void qkv_store_staged(const GemmArgs& p, int mrow0, int n0, const f4 (&acc)[MB][BN / 16],
                                                 _Float16* stage) {
  constexpr int NB = BN / 16, RS = BN + 8;
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
  const int inner = p.heads * 64;
#pragma unroll
  for (int mb = 0; mb < MB; mb++) {
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
      *reinterpret_cast<h4*>(stage + lr * RS + 16 * nb + 4 * lg) =
          h4{(_Float16)acc[mb][nb][0], (_Float16)acc[mb][nb][1], (_Float16)acc[mb][nb][2], (_Float16)acc[mb][nb][3]};
#pragma unroll
    for (int g = 0; g < BN / 64; g++) {
      const int nn = n0 + 64 * g + p.n_off, which = nn / inner, h = (nn % inner) / 64;
      _Float16* dst = (_Float16*)p.out + ((size_t)which * p.heads + h) * p.tpad * 64;
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int c = lane + 64 * j, tok = c >> 3, part = c & 7;
        const int m = mrow0 + 16 * mb + tok;
        const uint4 v = *reinterpret_cast<const uint4*>(stage + tok * RS + 64 * g + 8 * part);
        if (m < p.M) *reinterpret_cast<uint4*>(dst + (size_t)m * 64 + 8 * part) = v;
      }
    }
  }
}

// Residual epilogue x += acc; with GemmArgs::nx set it also prepares the next T5LayerNorm:
// the f16 operand f16(x * gamma * s) in operand order and the tile's sums of x^2 per 64-column
// group in the token's norm record.  Lane (lr, lg) holds columns n0 + 16nb + 4lg .. +3 of token
// mrow0 + 16mb + lr, so a group's sum is the lane's 16 squares plus those of the lanes lr + 16,
// lr + 32, lr + 48 (xor 16, xor 32).  Every load is unconditional -- x and the records have
// Mpad rows, so rows past M read padding -- and the x reads of CH row blocks are issued
// together: a guarded load per quad would cost one memory round trip each.  Only the stores
// are guarded; rows past M take part in the sums but store nothing.
template <int BN, int MB>
__device__ __forceinline__ void resid_store_tile(const GemmArgs& p, int mrow0, int n0, const f4 (&acc)[MB][BN / 16]) {
  constexpr int NB = BN / 16, G = BN / 64;
  constexpr int CH = BN == 64 ? MB : (MB % 2 == 0 ? 2 : 1);  // row blocks whose x is read at once
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
  const bool fold = p.nx != nullptr;
  float* x = (float*)p.out;
  float4 g[NB];
  float s[MB], ss[MB][G];
#pragma unroll
  for (int mb = 0; mb < MB; mb++) {
#pragma unroll
    for (int j = 0; j < G; j++) ss[mb][j] = 0.f;
    s[mb] = 0.f;
  }
  if (fold) {
#pragma unroll
    for (int nb = 0; nb < NB; nb++) g[nb] = *reinterpret_cast<const float4*>(p.ngamma + n0 + 16 * nb + 4 * lg);
#pragma unroll
    for (int mb = 0; mb < MB; mb++) s[mb] = p.rec[(size_t)(mrow0 + 16 * mb + lr) * 16 + 15];
  }
#pragma unroll
  for (int c0 = 0; c0 < MB; c0 += CH) {
    float4 xv[CH][NB];
#pragma unroll
    for (int j = 0; j < CH; j++)
#pragma unroll
      for (int nb = 0; nb < NB; nb++)
        xv[j][nb] = *reinterpret_cast<const float4*>(x + (size_t)(mrow0 + 16 * (c0 + j) + lr) * p.ldo + n0 +
                                                     16 * nb + 4 * lg);
#pragma unroll
    for (int j = 0; j < CH; j++) {
      const int mb = c0 + j, m = mrow0 + 16 * mb + lr;
#pragma unroll
      for (int nb = 0; nb < NB; nb++) {
        float4& r = xv[j][nb];
        r.x += acc[mb][nb][0];
        r.y += acc[mb][nb][1];
        r.z += acc[mb][nb][2];
        r.w += acc[mb][nb][3];
        ss[mb][nb / 4] += quad_sq(r);
      }
      if (m < p.M) {
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
          const int n = n0 + 16 * nb + 4 * lg;
          const float4 r = xv[j][nb];
          *reinterpret_cast<float4*>(x + (size_t)m * p.ldo + n) = r;
          if (fold)
            *reinterpret_cast<h4*>(p.nx + tiled_index(m, n, p.ldo)) =
                h4{(_Float16)((r.x * g[nb].x) * s[mb]), (_Float16)((r.y * g[nb].y) * s[mb]),
                   (_Float16)((r.z * g[nb].z) * s[mb]), (_Float16)((r.w * g[nb].w) * s[mb])};
        }
      }
    }
  }
  if (fold) {
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
      const int m = mrow0 + 16 * mb + lr;
#pragma unroll
      for (int j = 0; j < G; j++) {
        const float t = sum_xor32(sum_xor16(ss[mb][j]));
        if (m < p.M && lg == 0) p.rec[(size_t)m * 16 + n0 / 64 + j] = t;
      }
    }
  }
}


// Hybrid-numerics tile (launch_gemm_hybrid).  The stage holds sc q4 as the int8 planes
// hi = (sc >> 3) q4 and lo = (sc & 7) q4 (store_b_hybrid) and the A operand the Q8_K integers q8
// as int8, so v_mfma_i32_16x16x64_i8 sums each plane against q8 exactly in int32, and a 256-wide
// K block's integer sum is S = 8 hi + lo.  The block is then folded into the f32 output:
//   out += d8 * (d4 * float(S) - dmin4 * (mins . bsums)),
// the min term from one f16 MFMA of the row's mins (Mm) against the tokens' bsums (bsop, exact:
// <= 16 * 63 * 2048).  This is vec_dot's d * d8 * sum_j sc_j (q4 . q8)_j - dmin * d8 *
// sum_j m_j (bsum_2j + bsum_2j+1) per block (src/fused_matmul.rs:36-41,147-172): the integer
// sum is exact and converted to f32 once, as there.
// The math waves only run the integer MFMAs: at a block's last K step each writes its S tiles to
// the exchange buffer Sx, and producer wave MW + w folds math wave w's block during the next
// block's first K step (HybFold), so the fold's VALU work overlaps the next block's MFMAs on the
// same SIMD instead of stalling them.  Sx is read three barriers before it is written again.
// A operand (p.A as bytes): blocks of 16 tokens x 64 K (1 KiB) [Mpad/16][K/64], lane l holding
// token l % 16, K 16 (l / 16) .. +15; the weight fragment of lane l is row l % 16 of its row
// block, the same 16 K values.  Sx: [MW][MB][NB][64 lanes] int4, the lane's four outputs.
typedef int v4i __attribute__((ext_vector_type(4)));
template <int EPI, int MW, int BN, int S, int MB>
__device__ __forceinline__ void math_hybrid(const GemmArgs& p, int m0, _Float16 (*Bs)[BN * LDSK], int4* Sx) {
  constexpr int NB = BN / 16;
  static_assert(S == 2, "the hybrid loop unrolls a K block as two A stages");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, lr = lane & 15, lg = lane >> 4;
  const int nkt = p.K / BK, nblk = p.K / QK_K;
  const int mrow0 = m0 + wave * 16 * MB;
  const size_t kch = p.K / 64;  // 1 KiB operand blocks per 16-token row block
  const uint8_t* ablk[MB];
#pragma unroll
  for (int mb = 0; mb < MB; mb++)
    ablk[mb] = reinterpret_cast<const uint8_t*>(p.A) + (size_t)(mrow0 / 16 + mb) * kch * 1024 + lane * 16;
  int4* sx = Sx + (size_t)wave * MB * NB * 64 + lane;

  v4i acc_hi[MB][NB], acc_lo[MB][NB];
  uint4 a[S][MB];
#define LOAD_A(st, kt) \
  _Pragma("unroll") for (int mb = 0; mb < MB; mb++) a[st][mb] = *reinterpret_cast<const uint4*>(ablk[mb] + (size_t)(kt) * 1024);
  LOAD_A(0, 0);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();

  // this lane's fragment of row block nb: row 16 nb + lr, K chunk lg
  int foff[NB];
#pragma unroll
  for (int nb = 0; nb < NB; nb++) foff[nb] = hyb_off(16 * nb + lr, 16 * lg);
  const v4i izero = {0, 0, 0, 0};
  for (int b = 0; b < nblk; b++) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int kt = 4 * b + u;
      LOAD_A((u + 1) % S, min(kt + 1, nkt - 1));
      __builtin_amdgcn_sched_barrier(0);
      const uint8_t* hi = reinterpret_cast<const uint8_t*>(Bs[kt & 1]);
      const uint8_t* lo = hi + BN * 64;
      // every fragment of the step is requested before the first MFMA, so the LDS latency is
      // paid once per step rather than once per row block
      v4i wh[NB], wl[NB];
#pragma unroll
      for (int nb = 0; nb < NB; nb++) {
        wh[nb] = *reinterpret_cast<const v4i*>(hi + foff[nb]);
        wl[nb] = *reinterpret_cast<const v4i*>(lo + foff[nb]);
      }
#pragma unroll
      for (int nb = 0; nb < NB; nb++) {
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
          const v4i x = __builtin_bit_cast(v4i, a[u % S][mb]);
          acc_hi[mb][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wh[nb], x, u == 0 ? izero : acc_hi[mb][nb], 0, 0, 0);
          acc_lo[mb][nb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wl[nb], x, u == 0 ? izero : acc_lo[mb][nb], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (u == 3) {
        // block b's sums for the fold waves: lane holds rows 16nb + 4lg + i of token 16mb + lr
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
          for (int nb = 0; nb < NB; nb++) {
            const v4i sum = (acc_hi[mb][nb] << 3) + acc_lo[mb][nb];
            sx[(mb * NB + nb) * 64] = make_int4(sum[0], sum[1], sum[2], sum[3]);
          }
      }
      __syncthreads();
    }
  }
#undef LOAD_A
}

// Producer wave MW + w's share of a hybrid tile: the f32 outputs of math wave w, folded block by
// block from Sx, and the epilogue.
template <int EPI, int MW, int BN, int MB>
struct HybFold {
  static constexpr int NB = BN / 16;
  f4 out[MB][NB];
  float d8v[MB];  // the next block's d8 and bsum operand, requested a block ahead
  uint4 bsf[MB];
  int mrow0, lane, lr, lg, nblk;
  const int4* sx;

  __device__ __forceinline__ void load_meta(const GemmArgs& p, int b) {
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
      d8v[mb] = p.d8[(size_t)(mrow0 + 16 * mb + lr) * nblk + b];
      bsf[mb] = *reinterpret_cast<const uint4*>(p.bsop + ((size_t)(mrow0 / 16 + mb) * nblk + b) * 512 + lane * 8);
    }
  }
  __device__ __forceinline__ void init(const GemmArgs& p, int m0, const int4* Sx) {
    const int w = (threadIdx.x >> 6) - MW;
    lane = threadIdx.x & 63;
    lr = lane & 15;
    lg = lane >> 4;
    nblk = p.K / QK_K;
    mrow0 = m0 + w * 16 * MB;
    sx = Sx + (size_t)w * MB * NB * 64 + lane;
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
      for (int j = 0; j < NB; j++) out[i][j] = f4{0.f, 0.f, 0.f, 0.f};
    load_meta(p, 0);
  }
  // block b: its sums in Sx, its row metadata in Md / Mm [b % 2], its d8 / bsums in d8v / bsf
  __device__ __forceinline__ void fold(const GemmArgs& p, int b, const float2 (*Md)[BN], const h8 (*Mm)[2 * BN]) {
    const int bp = b & 1;
    const f4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
      const float4 q0 = *reinterpret_cast<const float4*>(&Md[bp][16 * nb + 4 * lg]);
      const float4 q1 = *reinterpret_cast<const float4*>(&Md[bp][16 * nb + 4 * lg + 2]);
      const float dd[4] = {q0.x, q0.z, q1.x, q1.z}, dm[4] = {q0.y, q0.w, q1.y, q1.w};
      const h8 mf = lg < 2 ? Mm[bp][2 * (16 * nb + lr) + lg] : h8{};
#pragma unroll
      for (int mb = 0; mb < MB; mb++) {
        const f4 cm = __builtin_amdgcn_mfma_f32_16x16x32_f16(mf, __builtin_bit_cast(h8, bsf[mb]), zero, 0, 0, 0);
        const int4 sv = sx[(mb * NB + nb) * 64];
        const int si[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          // d8 (d S - dmin M): the block's row scales first, the token's scale once
          const float t = __builtin_fmaf(-dm[i], cm[i], dd[i] * (float)si[i]);
          out[mb][nb][i] = __builtin_fmaf(d8v[mb], t, out[mb][nb][i]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // one row block at a time: bounded live registers
    }
    if (b + 1 < nblk) load_meta(p, b + 1);
  }
  __device__ __forceinline__ void epilogue(const GemmArgs& p, int n0) {
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
      const int m = mrow0 + mb * 16 + lr;
      if (m >= p.M) continue;
      if constexpr (EPI == EPI_GATED) {
#pragma unroll
        for (int nb = 0; nb < NB / 2; nb++) {
          const f4 g = out[mb][nb], v = out[mb][nb + NB / 2];
          *reinterpret_cast<h4*>((_Float16*)p.out + tiled_index(m, n0 + nb * 16 + 4 * lg, p.ldo)) =
              h4{(_Float16)(gelu_pade(g[0]) * v[0]), (_Float16)(gelu_pade(g[1]) * v[1]),
                 (_Float16)(gelu_pade(g[2]) * v[2]), (_Float16)(gelu_pade(g[3]) * v[3])};
        }
      } else {
#pragma unroll
        for (int nb = 0; nb < NB; nb++) store_quad<EPI_F32>(p, m, n0 + nb * 16 + 4 * lg, out[mb][nb]);
      }
    }
  }
};

// One output tile: tokens [m0, m0 + 16*MB*MW) x weight rows from n0.  MB = 16-row operand
// blocks per math wave: 4 for full tiles, 1 or 2 for the thin tiles that spread the last,
// partial round of a launch over every CU (the weight stage per K step is the same).
template <int EPI, int WF, int MW, int BN, int S, int MB, bool HY = false>
__device__ __forceinline__ void gemm_tile(const GemmArgs& p, int m0, int n0, _Float16 (*Bs)[BN * LDSK],
                                          float2 (*Md)[BN] = nullptr, h8 (*Mm)[2 * BN] = nullptr,
                                          int4* Sx = nullptr) {
  constexpr int NP = 64 * MW, NB = BN / 16;
  // S register stages of A (math waves) and PB of raw weights (producers): the loads of a
  // step are issued S-1 (PB-1) steps before it is consumed, covering L2/MALL latency.
  // K / 64 is a multiple of S and of PB.
  constexpr int PB = 4;
  using R = BRaw<WF, NP, BN>;
  const int nkt = p.K / BK;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  // waves [0, MW) compute, waves [MW, 2MW) produce; wave w runs on SIMD w % 4

  if (wave >= MW) {
    // ------------------------------ producer waves ------------------------------
    // Raw bytes of step j live in ring slot j % PB; step kt+1 is unpacked into LDS while
    // steps kt+2 .. kt+PB are in flight.  One barrier per step, as in the math waves.
    const int pt = tid - NP;
    R br[PB];
    // step kt's weights into stage kt % 2 (hybrid numerics: the block's metadata into kt / 4 % 2)
    auto store = [&](const R& r, int kt) {
      if constexpr (HY) store_b_hybrid<NP, BN>(r, Bs[kt & 1], Md[(kt >> 2) & 1], Mm[(kt >> 2) & 1], kt, pt);
      else store_b<WF, NP, BN>(r, Bs[kt & 1], kt, pt);
    };
    load_b<EPI, WF, NP, BN>(br[0], p, n0, 0, pt);
    store(br[0], 0);
#pragma unroll
    for (int i = 1; i < PB; i++) load_b<EPI, WF, NP, BN>(br[i], p, n0, i, pt);
    // hybrid numerics: these waves also fold the math waves' block sums (PB steps = one block)
    HybFold<EPI, MW, BN, MB> hf;
    if constexpr (HY) {
      static_assert(PB * BK == QK_K, "one producer ring turn per Q4_K block");
      hf.init(p, m0, Sx);
    }
    __syncthreads();
    // nkt % PB == 0 (K % 256 == 0); loads past the last step re-read it (in bounds, unused)
    // so that every load is unconditional and the compiler's wait counts stay exact.
    for (int kt0 = 0; kt0 < nkt; kt0 += PB) {
#pragma unroll
      for (int u = 0; u < PB; u++) {
        const int kt = kt0 + u;
        if (kt + 1 < nkt) store(br[(u + 1) % PB], kt + 1);
        load_b<EPI, WF, NP, BN>(br[u], p, n0, min(kt + PB, nkt - 1), pt);
        if constexpr (HY)
          if (u == 0 && kt0 > 0) hf.fold(p, kt0 / PB - 1, Md, Mm);
        __syncthreads();
      }
    }
    if constexpr (HY) {
      hf.fold(p, nkt / PB - 1, Md, Mm);
      hf.epilogue(p, n0);
    }
    return;
  }

  // -------------------------------- math waves ---------------------------------
  if constexpr (HY) {
    math_hybrid<EPI, MW, BN, S, MB>(p, m0, Bs, Sx);
    return;
  }
  const int lr = lane & 15, lg = lane >> 4;
  // operand blocks of this wave's MB row groups: block (rb, kb) at ((rb * K/32) + kb) * 512
  const size_t kblk = p.K / 32;
  // wave-uniform block bases plus the lane's 16 bytes: the loads take the base from SGPRs
  const _Float16* ablk[MB];
#pragma unroll
  for (int mb = 0; mb < MB; mb++) ablk[mb] = p.A + ((size_t)((m0 + wave * 16 * MB) / 16 + mb) * kblk) * 512;
  uint32_t alane = 16u * lane;

  f4 acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; i++)
#pragma unroll
    for (int j = 0; j < NB; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  // folded T5LayerNorm: the records are requested ahead of the first A loads
  const bool fold = EPI != EPI_RESID && p.rec != nullptr;
  float4 nrec[4];
  if (fold) norm_rec_load<MB>(p, m0 + wave * 16 * MB, nrec);
  __builtin_amdgcn_sched_barrier(0);

  // A ring: step j in register stage j % S, loaded S-1 steps before it is used.
  uint4 a[S][MB][2];
#define LOAD_A(st, kt)                                                                      \
  asm volatile("" : "+v"(alane));                                                            \
  _Pragma("unroll") for (int mb = 0; mb < MB; mb++) {                                        \
    a[st][mb][0] = *reinterpret_cast<const uint4*>(                                          \
        reinterpret_cast<const char*>(ablk[mb] + (size_t)(2 * (kt)) * 512) + alane);           \
    a[st][mb][1] = *reinterpret_cast<const uint4*>(                                          \
        reinterpret_cast<const char*>(ablk[mb] + (size_t)(2 * (kt) + 1) * 512) + alane);       \
  }
#pragma unroll
  for (int i = 0; i < S - 1; i++) {
    LOAD_A(i, i);
    __builtin_amdgcn_sched_barrier(0);  // stages issued in order
  }
  const float fs = fold ? norm_factor<MB>(p, m0 + wave * 16 * MB, n0, nrec) : 1.f;
  __syncthreads();

  // nkt % S == 0 (K % 256 == 0); as in the producers, loads past the end are clamped
  // fragment (nb, s) of this lane: row 16 nb + lr, columns 32 s + 8 lg .. +7 (row & 7 = lr & 7)
  const _Float16* bbase0 = &Bs[0][bswz(lr, 8 * lg)];
  const _Float16* bbase1 = &Bs[0][bswz(lr, 32 + 8 * lg)];
  for (int kt0 = 0; kt0 < nkt; kt0 += S) {
#pragma unroll
    for (int u = 0; u < S; u++) {
      const int kt = kt0 + u;
      {
        LOAD_A((u + S - 1) % S, min(kt + S - 1, nkt - 1));
        __builtin_amdgcn_sched_barrier(0);  // issue the prefetch before this step's MFMAs
        const _Float16* bsrc0 = bbase0 + (kt & 1) * (BN * LDSK);
        const _Float16* bsrc1 = bbase1 + (kt & 1) * (BN * LDSK);
        // Weight fragments j = s * NB + nb in order, each read FD fragments ahead of its MFMAs
        // so that the LDS latency hides behind the MFMAs of the fragments before it; the
        // scheduling barriers keep the compiler from regrouping the reads.
        constexpr int NF = 2 * NB, FD = 2;
        h8 wf[FD + 1];
#pragma unroll
        for (int j = 0; j < FD; j++)
          wf[j] = *reinterpret_cast<const h8*>((j / NB ? bsrc1 : bsrc0) + (j % NB) * 16 * LDSK);
#pragma unroll
        for (int j = 0; j < NF; j++) {
          if (j + FD < NF)
            wf[(j + FD) % (FD + 1)] =
                *reinterpret_cast<const h8*>(((j + FD) / NB ? bsrc1 : bsrc0) + ((j + FD) % NB) * 16 * LDSK);
          const int s = j / NB, nb = j % NB;
#pragma unroll
          for (int mb = 0; mb < MB; mb++)
            acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[j % (FD + 1)], __builtin_bit_cast(h8, a[u][mb][s]),
                                                                  acc[mb][nb], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();
      }
    }
  }
#undef LOAD_A

  // ---- epilogue: lane holds C[token m0+16MB*w+16mb+lr][columns n0+16nb+4lg+0..3] ----
  if constexpr (EPI == EPI_RESID) {
    resid_store_tile<BN, MB>(p, m0 + wave * 16 * MB, n0, acc);
    return;
  } else if (fold) {
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
      const float f = __shfl(fs, mb * 16 + lr);
#pragma unroll
      for (int nb = 0; nb < NB; nb++) acc[mb][nb] *= f;
    }
  }
  if constexpr (EPI == EPI_QKV) {
    if (p.dkv == 64) {  // every 64-column group of the tile is one head: full-row stores
      qkv_store_staged<BN, MB>(p, m0 + wave * 16 * MB, n0, acc, &Bs[0][0] + wave * (16 * (BN + 8)));
      return;
    }
  }
#pragma unroll
  for (int mb = 0; mb < MB; mb++) {
    const int m = m0 + wave * 16 * MB + mb * 16 + lr;
    if (m >= p.M) continue;
    if constexpr (EPI == EPI_GATED) {
#pragma unroll
      for (int nb = 0; nb < NB / 2; nb++)
        store_quad_gated(p, m, n0 + nb * 16 + 4 * lg, acc[mb][nb], acc[mb][nb + NB / 2]);
    } else {
#pragma unroll
      for (int nb = 0; nb < NB; nb++) store_quad<EPI>(p, m, n0 + nb * 16 + 4 * lg, acc[mb][nb]);
    }
  }
}

// Grid of one launch: blocks [0, main_blocks) run the full tiles of rows [0, m_main), the
// rest the thin tiles (TMB row blocks per math wave) of rows [m_main, M).  Within each part,
// block b runs on XCD b % 8 (workgroups are dealt round-robin), and each XCD gets a
// contiguous range of tiles, so its L2 holds the A rows it streams plus the weights.
struct GemmGrid {
  int tiles_n, main_tiles, main_blocks, m_main, tail_tiles;
};

template <int EPI, int WF, int MW, int BN, int S, int TMB, bool HY = false, int FMB = 4>
__global__ __launch_bounds__(128 * MW) __attribute__((amdgpu_waves_per_eu(MW == 8 ? 4 : 2)))
void gemm_kernel(GemmArgs p, GemmGrid g) {
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN * LDSK];
  // hybrid numerics: per-row block metadata (d, dmin; mins as an MFMA operand), two blocks deep
  __shared__ __attribute__((aligned(16))) float2 Md[HY ? 2 : 1][HY ? BN : 1];
  __shared__ __attribute__((aligned(16))) h8 Mm[HY ? 2 : 1][HY ? 2 * BN : 1];
  // hybrid numerics: the math waves' block sums for the fold waves
  __shared__ int4 Sx[HY ? MW * HYB_MB * (BN / 16) * 64 : 1];
  constexpr int cols = EPI == EPI_GATED ? BN / 2 : BN;  // output columns per tile
  // Full tiles: FMB (4 or 3) row blocks per math wave; HYB_MB with hybrid numerics, whose math
  // waves hold two int32 accumulator sets (the planes' block sums).
  constexpr int MBM = HY ? HYB_MB : FMB;
  int b = blockIdx.x;
  if (TMB == 0 || b < g.main_blocks) {
    const int tile = (b % 8) * (g.main_blocks / 8) + b / 8;
    if (tile >= g.main_tiles) return;
    if constexpr (HY)
      gemm_tile<EPI, WF, MW, BN, S, MBM, true>(p, (tile / g.tiles_n) * 16 * MBM * MW, (tile % g.tiles_n) * cols, Bs,
                                               Md, Mm, Sx);
    else
      gemm_tile<EPI, WF, MW, BN, S, MBM>(p, (tile / g.tiles_n) * 16 * MBM * MW, (tile % g.tiles_n) * cols, Bs);
  } else {
    constexpr int MBT = TMB == 0 ? 1 : TMB;
    b -= g.main_blocks;
    const int tile = (b % 8) * (((int)gridDim.x - g.main_blocks) / 8) + b / 8;
    if (tile >= g.tail_tiles) return;
    if constexpr (HY)
      gemm_tile<EPI, WF, MW, BN, S, MBT, true>(p, g.m_main + (tile / g.tiles_n) * 16 * MBT * MW,
                                               (tile % g.tiles_n) * cols, Bs, Md, Mm, Sx);
    else
      gemm_tile<EPI, WF, MW, BN, S, MBT>(p, g.m_main + (tile / g.tiles_n) * 16 * MBT * MW,
                                          (tile % g.tiles_n) * cols, Bs);
  }
}

template <int EPI, int WF, int BN, int S, int MW, int TMB, bool HY = false, int FMB = 4>
hipError_t launch_plan(const t5k::GemmPlan& pl, const GemmArgs& a, hipStream_t s) {
  constexpr int cols = EPI == EPI_GATED ? BN / 2 : BN, bm = 16 * (HY ? HYB_MB : FMB) * MW;
  GemmGrid g;
  g.tiles_n = a.N / cols;
  g.m_main = TMB ? pl.m_main : a.M;
  g.main_tiles = (g.m_main + bm - 1) / bm * g.tiles_n;
  g.main_blocks = (g.main_tiles + 7) / 8 * 8;
  const int bmt = 16 * (TMB ? TMB : 1) * MW;
  g.tail_tiles = TMB ? (a.M - g.m_main + bmt - 1) / bmt * g.tiles_n : 0;
  const int grid = g.main_blocks + (g.tail_tiles + 7) / 8 * 8;
  if (grid == 0) return hipSuccess;
  T5K_LAUNCH((gemm_kernel<EPI, WF, MW, BN, S, TMB, HY, FMB>), dim3(grid), dim3(128 * MW), 0, s, a, g);
  return hipGetLastError();
}

// A prefetch depth 2 (one step ahead): deeper rings measured slower -- the A stream is
// bound by L1/TA bandwidth, not latency, and more requests in flight only add contention.
template <int EPI, int WF, int BN>
hipError_t launch_cfg(const t5k::GemmPlan& pl, const GemmArgs& a, hipStream_t s) {
  // 8 math waves of 32 tokens (two per SIMD, 128 registers each): a measurement variant of the
  // gated FFN (T5H_GATED_MW8), same bits, not faster
  if constexpr (EPI == EPI_GATED && WF == WF_Q4K && BN == 128)
    if (pl.mw == 8) return launch_plan<EPI, WF, BN, 2, 8, 0, false, 2>(pl, a, s);
  if (pl.mw == 2) return launch_plan<EPI, WF, BN, 2, 2, 0>(pl, a, s);
  if (pl.mb == 3) switch (pl.tail_mb) {
      case 1: return launch_plan<EPI, WF, BN, 2, 4, 1, false, 3>(pl, a, s);
      case 2: return launch_plan<EPI, WF, BN, 2, 4, 2, false, 3>(pl, a, s);
      default: return launch_plan<EPI, WF, BN, 2, 4, 0, false, 3>(pl, a, s);
    }
  switch (pl.tail_mb) {
    case 1: return launch_plan<EPI, WF, BN, 2, 4, 1>(pl, a, s);
    case 2: return launch_plan<EPI, WF, BN, 2, 4, 2>(pl, a, s);
    default: return launch_plan<EPI, WF, BN, 2, 4, 0>(pl, a, s);
  }
}

template <int EPI>
hipError_t launch_epi(int wfmt, const t5k::GemmPlan& pl, const GemmArgs& a, hipStream_t s) {
  if (wfmt == WF_Q4K)
    return pl.bn == 64 ? launch_cfg<EPI, WF_Q4K, 64>(pl, a, s) : launch_cfg<EPI, WF_Q4K, 128>(pl, a, s);
  return pl.bn == 64 ? launch_cfg<EPI, WF_F16, 64>(pl, a, s) : launch_cfg<EPI, WF_F16, 128>(pl, a, s);
}

// Run time of the last tile when `tail` tiles of cost c follow `main` tiles of cost 1 on
// `slots` workgroup slots, each tile taking the earliest free slot (the dispatcher's order).
// After the main tiles, slots free up at r (slots - k of them) and r + 1 (k of them); the
// tail tiles start at r + i*c and r + 1 + j*c, earliest first.
double list_makespan(int main, int tail, double c, int slots) {
  const int r = main / slots, k = main % slots;
  double end = k ? r + 1 : r;
  if (tail <= 0) return end;
  const int n1 = slots - k, n2 = k;
  int i = 0, j = 0, left = tail;
  double start = r;
  while (left > 0) {
    const double t1 = r + i * c, t2 = n2 ? r + 1 + j * c : 1e30;
    if (t1 <= t2) {
      start = t1;
      left -= n1;
      i++;
    } else {
      start = t2;
      left -= n2;
      j++;
    }
  }
  return start + c > end ? start + c : end;
}

}  // namespace

namespace t5k {
// Tile choice for C[M, N]: 64*mw token rows (mw in {2, 4}) x bn weight rows (64 or 128).
// Prefer the 4-math-wave x 128-row tile once it fills at least one round of the CUs (the
// thin tail tiles of gemm_plan spread a partial last round; cfg2 QKV, 324 tiles: 26.0 -> 24.7
// us against 64-row tiles); then the 4 x 64 tile while it still covers >= 0.75 of the CUs;
// otherwise 2 x 64 (small token counts, where latency dominates).  n_rows = weight rows of
// the launch (both matrices for the gated FFN).
void gemm_pick_tile(int M, int n_rows, int cus, int& mw, int& bn) {
  auto tiles = [&](int w, int b) { return (double)((M + 64 * w - 1) / (64 * w)) * (n_rows / b); };
  if (n_rows % 128 == 0 && tiles(4, 128) >= cus) {
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

// Relative run time of a thin tile (16 or 32 token rows per math wave) against a full tile
// of the same weight rows: the producers' weight unpacking per K step is the same, only the
// MFMA work and the activation stream shrink.  Measured on MI355X as one round of 252 thin
// tiles against one round of 252 full tiles, over the encoder's four weight shapes:
// bn = 128: 0.45-0.55 (16 rows), 0.64-0.69 (32 rows); bn = 64: 0.50-0.61, 0.65-0.73.
static double thin_tile_cost(int bn, int mb) {
  if (bn == 128) return mb == 1 ? 0.53 : 0.68;
  return mb == 1 ? 0.56 : 0.70;
}

// Full tiles for rows [0, m_main), thin tiles for the rest, where that shortens the launch:
// with one workgroup per CU a launch of T full tiles takes ceil(T / CUs) rounds, and a last
// round that is mostly empty costs as much as a full one.  Every split at a multiple of the
// full tile height and both thin heights is evaluated with list_makespan, for full tiles of 64
// and of 48 tokens per math wave: the shorter tile costs 0.82 of the longer one (cfg4's M =
// 70,983, where rounds do not quantize: gate|up 561 vs 612 us, QKV 316 vs 343 us for 4/3 as
// many tiles) and wins where it fills the last round better (cfg2 gate|up 36.9 -> 33.7 us, QKV
// 23.5 -> 22.4 us; O and wo stay on one round of 64-token tiles).
// tail_override: -1 = choose, 0 = full tiles only, 1 / 2 = thin tiles of that height for the
// last row of full tiles, 3 / 4 = thin tiles of height 1 / 2 for every row (tests, tuning); a
// tail override keeps 64-token full tiles unless mb_override (3 or 4) sets their height.
static double full_tile_cost(int mb) { return mb == 3 ? 0.82 : 1.0; }

GemmPlan gemm_plan(int M, int n_rows, int cus, int mw_override, int bn_override, int tail_override,
                   int mb_override) {
  GemmPlan pl;
  gemm_pick_tile(M, n_rows, cus, pl.mw, pl.bn);
  if (mw_override == 2 || mw_override == 4) pl.mw = mw_override;
  if (bn_override == 64 || bn_override == 128) pl.bn = bn_override;
  pl.mb = pl.mw == 4 && mb_override == 3 ? 3 : 4;
  pl.m_main = M;
  pl.tail_mb = 0;
  if (pl.mw != 4 || M <= 0) return pl;
  const int tiles_n = n_rows / pl.bn;
  if (tail_override >= 0) {
    const int bm = 64 * pl.mb, full = (M + bm - 1) / bm;
    if (tail_override >= 1 && tail_override <= 4) {  // 3, 4: every row in thin tiles of height 1, 2
      pl.tail_mb = tail_override > 2 ? tail_override - 2 : tail_override;
      pl.m_main = tail_override > 2 ? 0 : (full - 1) * bm;
    }
    return pl;
  }
  double best = 1e30;
  for (int mb = 4; mb >= 3; mb--) {
    if (mb_override && mb != pl.mb) continue;
    const int bm = 64 * mb, full = (M + bm - 1) / bm;
    const double cf = full_tile_cost(mb);
    auto consider = [&](double t, int m_main, int tail_mb) {
      if (t < best - 1e-9) {
        best = t;
        pl.mb = mb;
        pl.m_main = m_main;
        pl.tail_mb = tail_mb;
      }
    };
    consider(list_makespan(full * tiles_n, 0, 1.0, cus) * cf, M, 0);
    for (int j = full - 1; j >= 0; j--)
      for (int tmb = 1; tmb <= 2; tmb++) {
        const int bmt = 64 * tmb, tail = (M - j * bm + bmt - 1) / bmt * tiles_n;
        consider(list_makespan(j * tiles_n, tail, thin_tile_cost(pl.bn, tmb) / cf, cus) * cf, j * bm, tmb);
      }
  }
  return pl;
}

// Hybrid plans: full tiles of 32 mw tokens (two row blocks per math wave) x 64 weight rows, or
// with tail_mb = 1 thin tiles of one row block per math wave for rows [m_main, M).
int gemm_hybrid_rows(int M) { return (M + 64 * HYB_MB - 1) / (64 * HYB_MB) * (64 * HYB_MB); }

GemmPlan gemm_plan_hybrid(int M, int n_rows, int cus) {
  GemmPlan pl;
  pl.bn = 64;
  pl.mw = 4;
  pl.m_main = M;
  pl.tail_mb = 0;
  const int bm = 64 * HYB_MB, tiles_n = n_rows / 64, full = (M + bm - 1) / bm;
  double best = list_makespan(full * tiles_n, 0, 1.0, cus);
  for (int j = full - 1; j >= 0; j--) {
    const int tail = (M - j * bm + 63) / 64 * tiles_n;
    const double t = list_makespan(j * tiles_n, tail, 0.6, cus);
    if (t < best - 1e-9) {
      best = t;
      pl.m_main = j * bm;
      pl.tail_mb = 1;
    }
  }
  return pl;
}

hipError_t launch_gemm_hybrid(int epi, const GemmPlan& pl, const GemmArgs& a, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (pl.bn != 64 || pl.mw != 4 || a.K % 256 || !a.A || !a.d8 || !a.bsop) return hipErrorInvalidValue;
  if (pl.tail_mb && (pl.tail_mb != 1 || pl.m_main < 0 || pl.m_main % (64 * HYB_MB) || pl.m_main >= a.M))
    return hipErrorInvalidValue;
  if (epi == EPI_GATED) {
    if (a.N % 32 || !a.W1) return hipErrorInvalidValue;
    return pl.tail_mb ? launch_plan<EPI_GATED, WF_Q4K, 64, 2, 4, 1, true>(pl, a, s)
                      : launch_plan<EPI_GATED, WF_Q4K, 64, 2, 4, 0, true>(pl, a, s);
  }
  if (epi != EPI_F32 || a.N % 64) return hipErrorInvalidValue;
  return pl.tail_mb ? launch_plan<EPI_F32, WF_Q4K, 64, 2, 4, 1, true>(pl, a, s)
                    : launch_plan<EPI_F32, WF_Q4K, 64, 2, 4, 0, true>(pl, a, s);
}

hipError_t launch_gemm(int epi, int wfmt, const GemmPlan& pl, const GemmArgs& a, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (pl.mw == 8) {  // 8 math waves of 32 tokens: gated FFN, Q4_K, 128-row tiles, full tiles only
    if (epi != EPI_GATED || wfmt != WF_Q4K || pl.bn != 128 || pl.mb != 2 || pl.tail_mb) return hipErrorInvalidValue;
  } else {
    if (pl.mw != 2 && pl.mw != 4) return hipErrorInvalidValue;
    if (pl.mb != 4 && !(pl.mb == 3 && pl.mw == 4)) return hipErrorInvalidValue;
  }
  if (pl.tail_mb && (pl.mw != 4 || pl.m_main < 0 || pl.m_main % (64 * pl.mb) || pl.m_main >= a.M))
    return hipErrorInvalidValue;
  if (pl.bn != 64 && pl.bn != 128) return hipErrorInvalidValue;
  // whole tiles along N and whole 4-step rings of 64-wide K steps
  if (a.N % (epi == EPI_GATED ? pl.bn / 2 : pl.bn) || a.K % 256) return hipErrorInvalidValue;
  // folded T5LayerNorm: the normalised row must fit one norm record
  if (epi == EPI_RESID && a.nx && (!a.rec || !a.ngamma || a.N != a.ldo || a.N > NORM_REC_MAX_D))
    return hipErrorInvalidValue;
  if (epi != EPI_RESID && a.rec && a.K > NORM_REC_MAX_D) return hipErrorInvalidValue;
  switch (epi) {
    case EPI_F16: return launch_epi<EPI_F16>(wfmt, pl, a, s);
    case EPI_RESID: return launch_epi<EPI_RESID>(wfmt, pl, a, s);
    case EPI_GATED: return launch_epi<EPI_GATED>(wfmt, pl, a, s);
    case EPI_F32: return launch_epi<EPI_F32>(wfmt, pl, a, s);
    case EPI_QKV: return launch_epi<EPI_QKV>(wfmt, pl, a, s);
    case EPI_RELU: return launch_epi<EPI_RELU>(wfmt, pl, a, s);
  }
  return hipErrorInvalidValue;
}
}  // namespace t5k
