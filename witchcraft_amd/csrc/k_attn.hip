// k_attn.hip -- varlen self-attention with T5 relative-position bias, no 1/sqrt(d) scale.
//
// Reference: T5Attention::forward, src/quantized_t5.rs:426-500: scores = Q K^T (:426, no
// scaling), + position bias (:441,490), softmax_last_dim (:496), . V (:497).  The reference
// runs one [1, L] sequence at a time with no mask (src/embedder.rs:40-41); here sequences
// are packed back to back (cu_seqlens) and a query only sees keys of its own sequence,
// which reproduces the per-sequence result.  The bias depends only on j - i
// (:452-483), so it is read from a per-head LUT indexed by the signed distance instead of
// materialising [H, L, L].
//
// Workgroup = 4 wave64s = 64 queries of one (sequence, head); each wave owns 16 queries.
// Keys are streamed in tiles of 64 through double-buffered LDS with an online softmax; the
// next tile's global loads are issued before the current tile is computed, so one barrier
// per tile remains and load latency overlaps the MFMA/softmax work.  The score block is
// computed transposed, S^T = K . Q^T, so that the accumulator layout (lane = query column,
// 4 consecutive keys per lane group) is exactly the B-operand layout the P.V MFMA needs:
// P never leaves registers.  V is transposed on its way into LDS (4x4 register blocks, 8-byte
// stores) with the keys of each 32-key group permuted so that a lane's 8 P.V operand keys are
// one contiguous 16-byte read.  The 127 bias values a tile needs (by j - i) are staged in LDS
// with the tile.
#include "common.hpp"

namespace {

constexpr int QT = 64;   // queries per workgroup
constexpr int KT = 64;   // keys per tile
constexpr int DK = 64;   // head dim (d_kv)
constexpr int KPAD = DK + 8;
constexpr int VPAD = KT + 8;
constexpr float LOG2E = 1.4426950408889634f;
constexpr float RESCALE = 5.5f;  // P <= e^5.5 < 256, far inside f16

// Slot of key `key` (a multiple of 4) inside a tile row of Vt: key 16h + 4g + i of a 32-key
// group sits at 8g + 4h + i, so keys {4g..4g+3, 16+4g..16+4g+3} -- the K-slots 8g..8g+7 of
// the P^T operand built from the S^T accumulators -- are contiguous.
__device__ __forceinline__ int vslot(int key) {
  const int kk = key & 31;
  return (key & ~31) + 8 * ((kk >> 2) & 3) + 4 * (kk >> 4);
}

// One key tile of one wave's 16 queries: S^T = K . Q^T, bias, online softmax, O^T += V^T . P^T.
// NKB = 16-key blocks of the tile that hold keys < L (the rest are skipped: their P is 0);
// MASK: the tile holds keys >= L, which get score -inf (only a sequence's last tile).
template <int NKB, bool MASK>
__device__ __forceinline__ void attn_tile(const _Float16* Ksb, const _Float16* Vtb, const float* Bsb, int bofs,
                                          const h8 (&qf)[2], int k0, int L, float& m_run, float& l_run,
                                          f4 (&o)[4]) {
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
  // S^T[key][query] + bias for the valid key blocks of 16: the accumulators start from the
  // bias, so the matrix core does the add
  f4 s[4];
#pragma unroll
  for (int kb = 0; kb < 4; kb++) {
    s[kb] = f4{0.f, 0.f, 0.f, 0.f};
    if (kb >= NKB) continue;
#pragma unroll
    for (int i = 0; i < 4; i++) s[kb][i] = Bsb[bofs + kb * 16 + i];
#pragma unroll
    for (int ds = 0; ds < 2; ds++) {
      const h8 a = *reinterpret_cast<const h8*>(&Ksb[(kb * 16 + lr) * KPAD + ds * 32 + lg * 8]);
      s[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[ds], s[kb], 0, 0, 0);
    }
  }
  // mask, running max
  float mx = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < NKB; kb++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      if (MASK && k0 + kb * 16 + lg * 4 + i >= L) s[kb][i] = -INFINITY;
      mx = fmaxf(mx, s[kb][i]);
    }
  mx = max_xor32(max_xor16(mx));
  // The reference max moves only when a score exceeds it by more than RESCALE (or on the
  // first tile, where m_run = -inf), so P <= e^RESCALE and the rescaling of O and l below
  // is skipped for a whole wave on most tiles.  Same result up to rounding: P and l carry
  // the same factor, divided out at the end.  mx is finite: key k0 < L is always valid.
  const float m_new = mx > m_run + RESCALE ? mx : m_run;
  // e^(v - m) = 2^(v log2e - m log2e): one FMA and one v_exp_f32 per score
  const float mb = -m_new * LOG2E;
  float rs = 0.f;
#pragma unroll
  for (int kb = 0; kb < NKB; kb++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][i], LOG2E, mb));
      s[kb][i] = e;
      rs += e;
    }
  rs = sum_xor32(sum_xor16(rs));
  if (__any(m_new != m_run)) {
    // exactly 1 for lanes whose max did not move (the wave-wide test also sees padding
    // queries, which must not perturb real ones); 0 on the first tile (m_run = -inf)
    const float corr = __builtin_amdgcn_exp2f((m_run - m_new) * LOG2E);
    l_run *= corr;
#pragma unroll
    for (int db = 0; db < 4; db++) o[db] *= corr;
  }
  l_run += rs;
  m_run = m_new;

  // O^T[d][query] += V^T[d][keys] . P^T[keys][query]; K-slots 8lg..8lg+7 of step ks are
  // keys {32ks + 4lg + 0..3, 32ks + 16 + 4lg + 0..3} in both operands.  A step whose 32 keys
  // are all past L adds nothing and is skipped.
  constexpr int NKS = (NKB + 1) / 2;
  h8 pb[2];
#pragma unroll
  for (int ks = 0; ks < NKS; ks++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      pb[ks][i] = (_Float16)s[2 * ks][i];
      pb[ks][4 + i] = (_Float16)s[2 * ks + 1][i];
    }
#pragma unroll
  for (int db = 0; db < 4; db++)
#pragma unroll
    for (int ks = 0; ks < NKS; ks++) {
      const h8 a = *reinterpret_cast<const h8*>(&Vtb[(db * 16 + lr) * VPAD + ks * 32 + lg * 8]);
      o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb[ks], o[db], 0, 0, 0);
    }
}

__global__ __launch_bounds__(256) void attn_relbias_kernel(AttnArgs p) {
  __shared__ __attribute__((aligned(16))) _Float16 Ks[2][KT * KPAD];
  __shared__ __attribute__((aligned(16))) _Float16 Vt[2][DK * VPAD];
  __shared__ float Bs[2][2 * KT];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int4 wk = p.work[blockIdx.x / p.heads];
  const int s0 = wk.x, L = wk.y, q0 = wk.z, h = blockIdx.x % p.heads;
  const int lr = lane & 15, lg = lane >> 4;

  const size_t head_stride = (size_t)p.tpad * DK;
  const _Float16* Q = p.qkv + ((size_t)0 * p.heads + h) * head_stride + (size_t)s0 * DK;
  const _Float16* Kg = p.qkv + ((size_t)1 * p.heads + h) * head_stride + (size_t)s0 * DK;
  const _Float16* Vg = p.qkv + ((size_t)2 * p.heads + h) * head_stride + (size_t)s0 * DK;
  // bias of distance d = j - i at lut[d], |d| <= lutw (lutw >= padded sequence length + 1)
  const float* lut = p.lut + (size_t)h * (2 * p.lutw + 1) + p.lutw;

  // This lane's query (relative to the sequence start).  Queries past L compute on
  // in-bounds padding rows and are never stored.
  const int qi = q0 + wave * 16 + lr;
  h8 qf[2];
  qf[0] = *reinterpret_cast<const h8*>(Q + (size_t)qi * DK + lg * 8);
  qf[1] = *reinterpret_cast<const h8*>(Q + (size_t)qi * DK + 32 + lg * 8);

  // tile staging: K copied row-major (rows kr, kr + 32; 8 dims at kc); V as a 4x4 block
  // (keys vk..vk+3, dims vd..vd+3), zeroed past L so padding rows cannot inject NaN into P.V.
  const int kr = tid >> 3, kc = (tid & 7) * 8;
  const int vk = (tid & 15) * 4, vd = (tid >> 4) * 4;
  uint4 kreg0, kreg1;
  h4 vreg[4];
  float breg = 0.f;
  auto gload = [&](int k0) {
    kreg0 = *reinterpret_cast<const uint4*>(Kg + (size_t)(k0 + kr) * DK + kc);
    kreg1 = *reinterpret_cast<const uint4*>(Kg + (size_t)(k0 + kr + 32) * DK + kc);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const h4 v = *reinterpret_cast<const h4*>(Vg + (size_t)(k0 + vk + j) * DK + vd);
      vreg[j] = (k0 + vk + j < L) ? v : h4{0, 0, 0, 0};
    }
    if (tid < 2 * KT) breg = lut[k0 - q0 - (QT - 1) + tid];
  };
  auto lstore = [&](int buf) {
    *reinterpret_cast<uint4*>(&Ks[buf][kr * KPAD + kc]) = kreg0;
    *reinterpret_cast<uint4*>(&Ks[buf][(kr + 32) * KPAD + kc]) = kreg1;
    const int slot = vslot(vk);
#pragma unroll
    for (int i = 0; i < 4; i++)
      *reinterpret_cast<h4*>(&Vt[buf][(vd + i) * VPAD + slot]) =
          h4{vreg[0][i], vreg[1][i], vreg[2][i], vreg[3][i]};
    if (tid < 2 * KT) Bs[buf][tid] = breg;
  };

  float m_run = -INFINITY, l_run = 0.f;
  f4 o[4];
#pragma unroll
  for (int i = 0; i < 4; i++) o[i] = f4{0.f, 0.f, 0.f, 0.f};

  const int ntile = (L + KT - 1) / KT;
  gload(0);
  lstore(0);
  __syncthreads();
  // Bs index of this lane's (key 4lg + i of key block 0, query qi): (j - qi) - (k0 - q0 - 63)
  const int bofs = (QT - 1) - wave * 16 - lr + 4 * lg;
  // Waves whose 16 queries all lie past L (in a sequence's last query tile) only help stage
  // the tiles.  The test is wave-uniform.
  const bool active = __builtin_amdgcn_readfirstlane(q0 + wave * 16) < L;
  for (int t = 0; t < ntile; ++t) {
    const int k0 = t * KT, buf = t & 1;
    if (t + 1 < ntile) gload(k0 + KT);
    if (active) {
      const _Float16* Ksb = Ks[buf];
      const _Float16* Vtb = Vt[buf];
      const float* Bsb = Bs[buf];
      if (k0 + KT <= L) {
        attn_tile<4, false>(Ksb, Vtb, Bsb, bofs, qf, k0, L, m_run, l_run, o);
      } else {  // the last tile: only its key blocks below L
        switch ((L - k0 + 15) >> 4) {
          case 1: attn_tile<1, true>(Ksb, Vtb, Bsb, bofs, qf, k0, L, m_run, l_run, o); break;
          case 2: attn_tile<2, true>(Ksb, Vtb, Bsb, bofs, qf, k0, L, m_run, l_run, o); break;
          case 3: attn_tile<3, true>(Ksb, Vtb, Bsb, bofs, qf, k0, L, m_run, l_run, o); break;
          default: attn_tile<4, true>(Ksb, Vtb, Bsb, bofs, qf, k0, L, m_run, l_run, o); break;
        }
      }
    }
    if (t + 1 < ntile) lstore(buf ^ 1);
    __syncthreads();
  }

  if (qi < L) {  // written in operand order for the O GEMM
    const float inv = 1.0f / l_run;
    const int inner = p.heads * DK;
#pragma unroll
    for (int db = 0; db < 4; db++) {
      const h4 v = {(_Float16)(o[db][0] * inv), (_Float16)(o[db][1] * inv), (_Float16)(o[db][2] * inv),
                    (_Float16)(o[db][3] * inv)};
      *reinterpret_cast<h4*>(p.out + tiled_index(s0 + qi, h * DK + db * 16 + lg * 4, inner)) = v;
    }
  }
}

}  // namespace

namespace t5k {
hipError_t launch_attention(const AttnArgs& a, int n_work, int dkv, hipStream_t s) {
  if (dkv != DK) return hipErrorInvalidValue;
  if (n_work <= 0) return hipSuccess;
  // heads fastest: the work list is ordered longest sequence first, so the costliest
  // workgroups start first on every head.
  hipLaunchKernelGGL(attn_relbias_kernel, dim3((unsigned)n_work * a.heads), dim3(256), 0, s, a);
  return hipGetLastError();
}
}  // namespace t5k
