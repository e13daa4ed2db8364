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
// Keys are streamed in tiles of 64 through LDS (K row-major, V transposed) with an
// online softmax.  The score block is computed transposed, S^T = K . Q^T, so that the
// accumulator layout (lane = query column, 4 consecutive keys per lane group) is exactly
// the B-operand layout the P.V MFMA needs: P never leaves registers.
#include "common.hpp"

namespace {

constexpr int QT = 64;   // queries per workgroup
constexpr int KT = 64;   // keys per tile
constexpr int DK = 64;   // head dim (d_kv)
constexpr int KPAD = DK + 8;
constexpr int VPAD = KT + 8;

__global__ __launch_bounds__(256) void attn_relbias_kernel(AttnArgs p) {
  __shared__ __attribute__((aligned(16))) _Float16 Ks[KT * KPAD];
  __shared__ __attribute__((aligned(16))) _Float16 Vt[DK * VPAD];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int2 wk = p.work[blockIdx.x];
  const int seq = wk.x, qtile = wk.y, h = blockIdx.y;
  const int s0 = p.cu[seq], L = p.cu[seq + 1] - s0;
  const int lr = lane & 15, lg = lane >> 4;

  const size_t head_stride = (size_t)p.tpad * DK;
  const _Float16* Q = p.qkv + ((size_t)0 * p.heads + h) * head_stride;
  const _Float16* Kg = p.qkv + ((size_t)1 * p.heads + h) * head_stride;
  const _Float16* Vg = p.qkv + ((size_t)2 * p.heads + h) * head_stride;
  const float* lut = p.lut + (size_t)h * (2 * p.maxl - 1) + (p.maxl - 1);

  // This lane's query (relative to the sequence start).  Queries past L compute on
  // in-bounds padding rows and are never stored.
  const int qi = qtile * QT + wave * 16 + lr;
  h8 qf[2];
  {
    const _Float16* qrow = Q + (size_t)(s0 + qi) * DK;
    qf[0] = *reinterpret_cast<const h8*>(qrow + lg * 8);
    qf[1] = *reinterpret_cast<const h8*>(qrow + 32 + lg * 8);
  }

  float m_run = -INFINITY, l_run = 0.f;
  f4 o[4];
#pragma unroll
  for (int i = 0; i < 4; i++) o[i] = f4{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < L; k0 += KT) {
    // cooperative tile load: 64 keys x 64 dims of K (row-major) and V (transposed)
#pragma unroll
    for (int it = 0; it < 2; it++) {
      const int r = it * 32 + (tid >> 3), c = (tid & 7) * 8;
      const size_t g = (size_t)(s0 + k0 + r) * DK + c;
      *reinterpret_cast<uint4*>(&Ks[r * KPAD + c]) = *reinterpret_cast<const uint4*>(Kg + g);
      const h8 v = *reinterpret_cast<const h8*>(Vg + g);
#pragma unroll
      for (int e = 0; e < 8; e++) Vt[(c + e) * VPAD + r] = v[e];
    }
    __syncthreads();

    // S^T[key][query] for 4 key blocks of 16
    f4 s[4];
#pragma unroll
    for (int kb = 0; kb < 4; kb++) {
      s[kb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < 2; ds++) {
        const h8 a = *reinterpret_cast<const h8*>(&Ks[(kb * 16 + lr) * KPAD + ds * 32 + lg * 8]);
        s[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[ds], s[kb], 0, 0, 0);
      }
    }
    // bias + mask, running max
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; kb++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int j = k0 + kb * 16 + lg * 4 + i;
        const int dlt = min(max(j - qi, 1 - p.maxl), p.maxl - 1);  // clamp: padded rows only
        float v = s[kb][i] + lut[dlt];
        v = j < L ? v : -INFINITY;
        s[kb][i] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);  // finite: key k0 < L is always valid
    const float corr = __expf(m_run - m_new);
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < 4; kb++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float e = __expf(s[kb][i] - m_new);
        s[kb][i] = e;
        rs += e;
      }
    rs += __shfl_xor(rs, 16);
    rs += __shfl_xor(rs, 32);
    l_run = l_run * corr + rs;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < 4; db++) o[db] *= corr;

    // O^T[d][query] += V^T[d][keys] . P^T[keys][query]; K-slot order = keys
    // {16(2ks)+4lg+0..3, 16(2ks+1)+4lg+0..3} in both operands.
    h8 pb[2];
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        pb[ks][i] = (_Float16)s[2 * ks][i];
        pb[ks][4 + i] = (_Float16)s[2 * ks + 1][i];
      }
#pragma unroll
    for (int db = 0; db < 4; db++) {
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        const _Float16* vrow = &Vt[(db * 16 + lr) * VPAD];
        const h4 v0 = *reinterpret_cast<const h4*>(vrow + (2 * ks) * 16 + lg * 4);
        const h4 v1 = *reinterpret_cast<const h4*>(vrow + (2 * ks + 1) * 16 + lg * 4);
        const h8 a = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb[ks], o[db], 0, 0, 0);
      }
    }
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
  hipLaunchKernelGGL(attn_relbias_kernel, dim3(n_work, a.heads), dim3(256), 0, s, a);
  return hipGetLastError();
}
}  // namespace t5k
