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
// Keys are streamed in tiles of 64 through double-buffered LDS with an online softmax.  The
// tiles travel global -> LDS without registers (global_load_lds_dwordx4): K and V rows as
// they lie in memory, 128 B per key, and the bias values a tile needs (by j - i).  The next
// tile's loads are issued before the current tile is computed; one barrier per tile.
//
// The score block is computed transposed, S^T = K . Q^T, so that the accumulator layout
// (lane = query column, 4 consecutive keys per lane group) is exactly the B-operand layout of
// O^T = V^T . P^T: P never leaves registers.  The V^T operand (8 keys of one dim per lane) is
// read from the row-major V tile with ds_read_b64_tr_b16, which hands lane n of each 16-lane
// group column n of a 4-row block, so V needs no transpose on its way in.
#include "common.hpp"

namespace {

constexpr int QT = ATTN_QT;  // queries per workgroup
constexpr int KT = 64;   // keys per tile
constexpr int DK = 64;   // head dim (d_kv)
constexpr float LOG2E = 1.4426950408889634f;

typedef short s4v __attribute__((ext_vector_type(4)));

// LDS tiles are 64 keys x 64 dims of f16 in the swz64 layout (128 B rows, XOR-swizzled
// 16-byte chunks): the K operand reads and the transposed V reads are conflict-free.
__device__ __forceinline__ int swz(int row, int col) { return swz64(row, col); }

// Global -> LDS copy of one 64-row tile by this wave's 16 rows: LDS slot l of an instruction
// (16 B, consecutive by lane) holds row 16 wave + 8 j + l / 8, chunk (l % 8) ^ (row % 8), so
// each group of 8 lanes still reads one 128-byte row.  Rows at or past `nrows` repeat the last
// row of the sequence: finite values, which the masked scores (P = 0) then ignore.
__device__ __forceinline__ void dma_tile(const _Float16* src, int nrows, _Float16* dst, int wave, int lane) {
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int row = 16 * wave + 8 * j + (lane >> 3);
    const int chunk = (lane ^ row) & 7;
    const int srow = row < nrows ? row : nrows - 1;
    __builtin_amdgcn_global_load_lds(src + (size_t)srow * DK + chunk * 8, dst + (16 * wave + 8 * j) * DK, 16, 0, 0);
  }
}

// The V^T operand of P.V step ks for dims 16 db..16 db+15: lane (n, g) = (lane % 16, lane / 16)
// gets V[32 ks + 4 g + r][16 db + n] and V[32 ks + 16 + 4 g + r][16 db + n], r = 0..3 -- the
// keys of K-slots 8g..8g+7 of the P^T operand.  Lane i of a 16-lane group addresses row
// base + i / 4, dims 16 db + 4 (i % 4): the transposing read returns column n of those 4 rows.
__device__ __forceinline__ h8 v_operand(const _Float16* Vb, int ks, int db, int lane) {
  const int i = lane & 15, g = lane >> 4;
  const int row = 32 * ks + 4 * g + (i >> 2), col = 16 * db + 4 * (i & 3);
  typedef __attribute__((address_space(3))) s4v lds_s4;
  const s4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(Vb + swz(row, col)));
  const s4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(Vb + swz(row + 16, col)));
  h8 r;
  __builtin_memcpy(&r, &lo, 8);
  __builtin_memcpy(reinterpret_cast<char*>(&r) + 8, &hi, 8);
  return r;
}

// P = 2^(S log2e + mb) of this tile's valid key blocks into the f16 P^T operand; returns this
// lane's sum of P.  K-slots 8lg..8lg+7 of step ks are keys {32ks + 4lg + 0..3, 32ks + 16 + 4lg + 0..3}.
template <int NKB>
__device__ __forceinline__ float tile_exp(const f4 (&s)[4], float mb, h8 (&pb)[2]) {
  float rs = 0.f;
#pragma unroll
  for (int kb = 0; kb < 4; kb++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float e = 0.f;
      if (kb < NKB) {
        e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][i], LOG2E, mb));
        rs += e;
      }
      pb[kb >> 1][(kb & 1) * 4 + i] = (_Float16)e;
    }
  return rs;
}

// One key tile of one wave's 16 queries: S^T = K . Q^T, bias, softmax against the running
// reference max m_run, O^T += V^T . P^T.
// NKB = 16-key blocks of the tile that hold keys < L (the rest are skipped: their P is 0);
// MASK: the tile holds keys >= L, which get score -inf (only a sequence's last tile);
// FIRST: the sequence's first tile, which sets the reference max.
//
// The reference max moves only when needed: P is first taken against the current m_run, and
// only if some lane's sum of P exceeds 2^14 (so that a P could leave the f16 range, and on the
// first tile, where m_run = -inf gives inf) is the tile's true max taken, O and l rescaled and P
// recomputed.  Same result up to rounding: P and l carry the same factor 2^((m - m_run) log2e),
// divided out at the end, and m_run is a score already seen, so l >= 1.  l is kept per lane
// (this lane's keys) and reduced across the four lanes of a query only at the end.
//
// FAR: every (query, key) distance of the tile lies where the bias buckets have saturated, so
// the bias is the single value cb: it joins the exponent's constant instead of the scores.
template <int NKB, bool MASK, bool FIRST, bool FAR>
__device__ __forceinline__ void attn_tile(const _Float16* Ksb, const _Float16* Vb, const float* Bsb, int bofs,
                                          float cb, const h8 (&qf)[2], int k0, int L, float& m_run,
                                          float& l_run, f4 (&o)[4]) {
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
  if (!FAR) cb = 0.f;
  // S^T[key][query] (+ bias for the valid key blocks of 16 unless FAR): the accumulators start
  // from the bias, so the matrix core does the add.  Independent accumulators back to back: no
  // MFMA waits on the one before it.
  f4 s[4];
#pragma unroll
  for (int kb = 0; kb < 4; kb++) {
    s[kb] = f4{0.f, 0.f, 0.f, 0.f};
    if (!FAR && kb < NKB)
#pragma unroll
      for (int i = 0; i < 4; i++) s[kb][i] = Bsb[bofs + kb * 16 + i];
  }
#pragma unroll
  for (int ds = 0; ds < 2; ds++)
#pragma unroll
    for (int kb = 0; kb < NKB; kb++) {
      const h8 a = *reinterpret_cast<const h8*>(&Ksb[swz(kb * 16 + lr, ds * 32 + lg * 8)]);
      s[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[ds], s[kb], 0, 0, 0);
    }
  if (MASK) {
#pragma unroll
    for (int kb = 0; kb < NKB; kb++)
#pragma unroll
      for (int i = 0; i < 4; i++)
        if (k0 + kb * 16 + lg * 4 + i >= L) s[kb][i] = -INFINITY;
  }
  h8 pb[2];
  float rs = 0.f, corr = 1.f;
  if (!FIRST) rs = tile_exp<NKB>(s, (cb - m_run) * LOG2E, pb);
  // !(rs <= 2^14) also catches NaN
  const bool remax = FIRST || __any(!(rs <= 16384.f));
  if (remax) {
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < NKB; kb++)
#pragma unroll
      for (int i = 0; i < 4; i++) mx = fmaxf(mx, s[kb][i]);
    mx = max_xor32(max_xor16(mx)) + cb;  // finite: key k0 < L is valid
    const float m_new = fmaxf(m_run, mx);
    if (!FIRST) corr = __builtin_amdgcn_exp2f((m_run - m_new) * LOG2E);  // 1 where the max did not move
    m_run = m_new;
    rs = tile_exp<NKB>(s, (cb - m_new) * LOG2E, pb);
  }
  // the rescale of O sits in a branch of its own, so the accumulators keep their registers
  if (!FIRST && remax) {
    l_run *= corr;
#pragma unroll
    for (int db = 0; db < 4; db++) o[db] *= corr;
  }
  l_run += rs;

  // O^T[d][query] += V^T[d][keys] . P^T[keys][query]; a step whose 32 keys are all past L adds
  // nothing and is skipped.
  constexpr int NKS = (NKB + 1) / 2;
#pragma unroll
  for (int ks = 0; ks < NKS; ks++)
#pragma unroll
    for (int db = 0; db < 4; db++)
      o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(v_operand(Vb, ks, db, lane), pb[ks], o[db], 0, 0, 0);
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void attn_relbias_kernel(AttnArgs p) {
  // double-buffered tiles as separate objects, so that the loads into one buffer are not
  // waited on by the reads of the other
  __shared__ __attribute__((aligned(16))) _Float16 Ks0[KT * DK], Ks1[KT * DK];
  __shared__ __attribute__((aligned(16))) _Float16 Vs0[KT * DK], Vs1[KT * DK];
  __shared__ __attribute__((aligned(16))) float Bs0[2 * KT], Bs1[2 * KT];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int4 wk = p.work[blockIdx.x];
  const int s0 = wk.x, L = wk.y, q0 = wk.z, h = wk.w;
  if (L == 0) return;  // an empty slot of the work list (the whole workgroup)
  const int lr = lane & 15, lg = lane >> 4;

  const size_t head_stride = (size_t)p.tpad * DK;
  const _Float16* Q = p.qkv + ((size_t)0 * p.heads + h) * head_stride + (size_t)s0 * DK;
  const _Float16* Kg = p.qkv + ((size_t)1 * p.heads + h) * head_stride + (size_t)s0 * DK;
  const _Float16* Vg = p.qkv + ((size_t)2 * p.heads + h) * head_stride + (size_t)s0 * DK;
  // bias of distance d = j - i at lut[d], |d| <= lutw (lutw >= padded sequence length + 1)
  const float* lut = p.lut + (size_t)h * (2 * p.lutw + 1) + p.lutw;
  // the bias of every distance <= -sat and of every distance >= sat
  const float bias_far[2] = {lut[-p.lutw], lut[p.lutw]};
  // A middle tile (not the first or the last, which always read the staged bias) whose
  // distances to every query of the workgroup are that far needs no bias values.
  auto stage_bias = [&](int k0) {
    return k0 == 0 || k0 + KT >= L || !(k0 - q0 - (QT - 1) >= p.sat || k0 + KT - 1 - q0 <= -p.sat);
  };

  // This lane's query (relative to the sequence start).  Queries past L compute on
  // in-bounds padding rows and are never stored.
  const int qi = q0 + wave * 16 + lr;
  h8 qf[2];
  qf[0] = *reinterpret_cast<const h8*>(Q + (size_t)qi * DK + lg * 8);
  qf[1] = *reinterpret_cast<const h8*>(Q + (size_t)qi * DK + 32 + lg * 8);

  // tile loads straight into LDS: K and V rows k0.. (clamped to the sequence), and the 128 bias
  // values of distances k0 - q0 - 63 .. k0 - q0 + 64 by waves 0 and 1
  auto load_tile = [&](int k0, _Float16* Kd, _Float16* Vd, float* Bd) {
    dma_tile(Kg + (size_t)k0 * DK, L - k0, Kd, wave, lane);
    dma_tile(Vg + (size_t)k0 * DK, L - k0, Vd, wave, lane);
    if (wave < 2 && stage_bias(k0))
      __builtin_amdgcn_global_load_lds(lut + (k0 - q0 - (QT - 1) + 64 * wave + lane), Bd + 64 * wave, 4, 0, 0);
  };

  float m_run = -INFINITY, l_run = 0.f;
  f4 o[4];
#pragma unroll
  for (int i = 0; i < 4; i++) o[i] = f4{0.f, 0.f, 0.f, 0.f};

  const int ntile = (L + KT - 1) / KT;
  // Bs index of this lane's (key 4lg + i of key block 0, query qi): (j - qi) - (k0 - q0 - 63)
  const int bofs = (QT - 1) - wave * 16 - lr + 4 * lg;
  // Waves whose 16 queries all lie past L (in a sequence's last query tile) only help load
  // the tiles.  The test is wave-uniform.
  const bool active = q0 + wave * 16 < L;
  // The first tile sets the reference max; the middle tiles are full; the last one holds keys
  // past L unless L is a multiple of 64 (rem = 0).  A single tile is both first and last.
  const int rem = L & (KT - 1);
  // one tile: issue the next tile's loads into the other buffer, compute this one, wait for
  // this wave's loads and meet the other waves
  auto step = [&](int t, const _Float16* Kc, const _Float16* Vc, const float* Bc, _Float16* Kn, _Float16* Vn,
                  float* Bn, auto&& compute) {
    if (t + 1 < ntile) load_tile((t + 1) * KT, Kn, Vn, Bn);
    if (active) compute(Kc, Vc, Bc, t * KT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };
  auto middle = [&](const _Float16* Kc, const _Float16* Vc, const float* Bc, int k0) {
    const int qa = q0 + wave * 16;  // this wave's distances j - i span [k0 - qa - 15, k0 + 63 - qa]
    if (k0 - qa - 15 >= p.sat || k0 + KT - 1 - qa <= -p.sat)
      attn_tile<4, false, false, true>(Kc, Vc, Bc, bofs, k0 > qa ? bias_far[1] : bias_far[0], qf, k0, L, m_run,
                                       l_run, o);
    else
      attn_tile<4, false, false, false>(Kc, Vc, Bc, bofs, 0.f, qf, k0, L, m_run, l_run, o);
  };
  auto last = [&](const _Float16* Kc, const _Float16* Vc, const float* Bc, int k0) {
    if (rem == 0) {
      attn_tile<4, false, false, false>(Kc, Vc, Bc, bofs, 0.f, qf, k0, L, m_run, l_run, o);
    } else {
      switch ((rem + 15) >> 4) {
        case 1: attn_tile<1, true, false, false>(Kc, Vc, Bc, bofs, 0.f, qf, k0, L, m_run, l_run, o); break;
        case 2: attn_tile<2, true, false, false>(Kc, Vc, Bc, bofs, 0.f, qf, k0, L, m_run, l_run, o); break;
        case 3: attn_tile<3, true, false, false>(Kc, Vc, Bc, bofs, 0.f, qf, k0, L, m_run, l_run, o); break;
        default: attn_tile<4, true, false, false>(Kc, Vc, Bc, bofs, 0.f, qf, k0, L, m_run, l_run, o); break;
      }
    }
  };

  load_tile(0, Ks0, Vs0, Bs0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  step(0, Ks0, Vs0, Bs0, Ks1, Vs1, Bs1, [&](const _Float16* Kc, const _Float16* Vc, const float* Bc, int k0) {
    if (ntile > 1 || rem == 0) {
      attn_tile<4, false, true, false>(Kc, Vc, Bc, bofs, 0.f, qf, k0, L, m_run, l_run, o);
    } else {
      switch ((rem + 15) >> 4) {
        case 1: attn_tile<1, true, true, false>(Kc, Vc, Bc, bofs, 0.f, qf, k0, L, m_run, l_run, o); break;
        case 2: attn_tile<2, true, true, false>(Kc, Vc, Bc, bofs, 0.f, qf, k0, L, m_run, l_run, o); break;
        case 3: attn_tile<3, true, true, false>(Kc, Vc, Bc, bofs, 0.f, qf, k0, L, m_run, l_run, o); break;
        default: attn_tile<4, true, true, false>(Kc, Vc, Bc, bofs, 0.f, qf, k0, L, m_run, l_run, o); break;
      }
    }
  });
  // middle tiles in pairs (odd tiles in buffer 1, even ones in buffer 0), then the last tile
  int t = 1;
  for (; t + 2 < ntile; t += 2) {
    step(t, Ks1, Vs1, Bs1, Ks0, Vs0, Bs0, middle);
    step(t + 1, Ks0, Vs0, Bs0, Ks1, Vs1, Bs1, middle);
  }
  if (t + 1 < ntile) {
    step(t, Ks1, Vs1, Bs1, Ks0, Vs0, Bs0, middle);
    t++;
  }
  if (t < ntile) {
    if (t & 1) step(t, Ks1, Vs1, Bs1, Ks0, Vs0, Bs0, last);
    else step(t, Ks0, Vs0, Bs0, Ks1, Vs1, Bs1, last);
  }
  l_run = sum_xor32(sum_xor16(l_run));

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
  // one workgroup per work item; item b runs on XCD b % 8, and the list keeps all query tiles of
  // a (sequence, head) on one XCD so that its keys and values stay in that XCD's L2
  T5K_LAUNCH(attn_relbias_kernel, dim3((unsigned)n_work), dim3(256), 0, s, a);
  return hipGetLastError();
}
}  // namespace t5k
