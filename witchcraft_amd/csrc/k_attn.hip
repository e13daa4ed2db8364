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
// Workgroup = 4 wave64s = 128 queries of one (sequence, head); each wave owns 32 queries and
// runs v_mfma_f32_32x32x16_f16, so every K and V operand it reads from LDS feeds 32 queries.
// Keys are streamed in tiles of 64 through a three-deep LDS ring with an online softmax.  The
// tiles travel global -> LDS without registers (global_load_lds_dwordx4): K and V rows as they
// lie in memory, 128 B per key, and the bias values a tile needs (by j - i).  A tile's loads
// are issued two tiles ahead; one barrier per tile.  A sequence of at most 128 tokens takes a
// path with 64-query work items and 16-query waves instead (small_sequence).
//
// The score block is computed transposed, S^T = K . Q^T (32 keys x 32 queries per MFMA), so
// that the accumulator layout (lane = query column; lane half h holds keys 8a + 4h + b) is, four
// registers at a time, the B operand of O^T = V^T . P^T with the keys of each 16-key step taken
// in the order {4h .. 4h+3, 8+4h .. 8+4h+3}: P never leaves registers.  The V^T operand (32 dims
// x those 8 keys per lane) is read from the row-major V tile with ds_read_b64_tr_b16, which
// hands lane n of each 16-lane group column n of a 4-row block, so V needs no transpose on its
// way in.
#include <type_traits>

#include "common.hpp"

namespace {

constexpr int QT = ATTN_QT;     // queries per workgroup
constexpr int QW = 32;          // queries per wave
constexpr int NWV = QT / QW;    // waves per workgroup
constexpr int KT = 64;          // keys per tile
constexpr int DK = 64;          // head dim (d_kv)
constexpr int BSN = 64 * NWV;   // bias values staged per tile (QT + KT - 1 of them are read)
constexpr int LOADS = 5;        // global -> LDS loads per wave per tile: 2 K, 2 V, 1 bias
constexpr float LOG2E = 1.4426950408889634f;
static_assert(NWV == 4 && 16 * NWV == KT && BSN >= QT + KT && BSN >= 256 && ATTN_SMALL_L == 2 * KT, "tile shape");

typedef short s4v __attribute__((ext_vector_type(4)));

// One slot of the LDS ring: a key tile's K and V rows and its bias values.
struct __attribute__((aligned(16))) Slot {
  _Float16 k[KT * DK], v[KT * DK];
  float b[BSN];
};
typedef float f16v __attribute__((ext_vector_type(16)));

// LDS tiles are 64 keys x 64 dims of f16, 128 B rows of eight 16-byte chunks; chunk c of row r
// sits at position c ^ rot(r).  Each rotation is a bijection on each 8 consecutive rows.  The V
// tile uses ROT_V(r) = r's low three bits with bits 1 and 2 swapped, the K tile ROT_K(r) =
// (r ^ (r >> 2)) % 8: with them the transposed V reads and the K operand reads of the 32-query
// waves are free of bank conflicts (SQ_LDS_BANK_CONFLICT reads 0 for each pattern alone on
// gfx950), where the plain ROT_8(r) = r % 8 costs 2-way conflicts on both.  The 16-query waves
// of a short sequence read 16 rows per K operand and 4 rows x 2 chunks per 16 lanes of V, which
// ROT_8 serves without conflicts.  ROT_K(r + 32) = ROT_K(r), and none depends on higher row
// bits than that, so key offsets of 8, 16 and 32 rows fold into immediates.
enum { ROT_V = 0, ROT_K = 1, ROT_8 = 2 };
template <int R>
__device__ __forceinline__ int rot(int row) {
  return R == ROT_V ? ((row & 1) | ((row & 2) << 1) | ((row & 4) >> 1)) : R == ROT_K ? ((row ^ (row >> 2)) & 7) : (row & 7);
}
template <int R>
__device__ __forceinline__ int swz(int row, int col) {
  return row * DK + ((((col >> 3) ^ rot<R>(row)) & 7) << 3) + (col & 7);
}

// Global -> LDS loads (global_load_lds), written as inline asm so that the compiler does not
// track them: its tracking waits for every outstanding one before a read of one of the ring
// slots (it cannot tell the slots apart there), which would stall on the tile just issued.
// The kernel orders them itself: a wave issues exactly LOADS of them per tile and waits with
// vmcnt before the barrier that publishes the tile; the "memory" clobbers keep every LDS
// access on its side of these statements.  M0 holds the wave's LDS destination; the 16-byte
// form writes lane l's 16 bytes at M0 + 16 l, the 4-byte form lane l's 4 bytes at M0 + 4 l.
// The source address is a wave-uniform base (an SGPR pair) plus the lane's 32-bit byte offset,
// so a tile's loads cost no 64-bit address arithmetic per lane.
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void lds_load16(const void* base, uint32_t voff, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(m0)
               : "memory", "m0");
}
__device__ __forceinline__ void lds_load4(const void* base, uint32_t voff, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "s"(m0)
               : "memory", "m0");
}

// Global -> LDS copy of one 64-row tile by this wave's 16 rows: LDS slot l of an instruction
// (16 B, consecutive by lane) holds row 16 wave + 8 j + l / 8, chunk (l % 8) ^ rot<R>(row), so
// each group of 8 lanes still reads one 128-byte row.  Rows at or past
// `nrows` repeat the last row of the sequence: finite values, which the masked scores (P = 0)
// then ignore.
template <int R>
__device__ __forceinline__ void dma_tile(const _Float16* src, int nrows, _Float16* dst, int wave, int lane) {
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int row = 16 * wave + 8 * j + (lane >> 3);
    const int chunk = (lane ^ rot<R>(row)) & 7;
    const int srow = row < nrows ? row : nrows - 1;
    lds_load16(src, (uint32_t)(srow * (DK * 2) + chunk * 16), lds_offset(dst + (16 * wave + 8 * j) * DK));
  }
}

// Per-lane LDS offsets (f16 elements from a tile's base) of the operand reads.
// k[ds]: the K operand of dims 16 ds .. +15 for key half 0 (key row l % 32, dims + 8 (l / 32));
// half kb adds 32 rows.  v[db]: the V^T operand of dims 32 db .. +31 for key step 0 (below);
// step c adds 16 rows, its second 8 keys another 8.  Rows that differ by a multiple of 8 share
// their rotation, so those additions are constants that fold into the reads' immediate offsets.
struct LaneOfs {
  int k[4], v[2];
};
__device__ __forceinline__ LaneOfs lane_offsets(int lane) {
  const int l32 = lane & 31, h = lane >> 5, i = lane & 15, g = lane >> 4;
  LaneOfs o;
#pragma unroll
  for (int ds = 0; ds < 4; ds++) o.k[ds] = swz<ROT_K>(l32, 16 * ds + 8 * h);
#pragma unroll
  for (int db = 0; db < 2; db++) o.v[db] = swz<ROT_V>(4 * h + (i >> 2), 32 * db + 16 * (g & 1) + 4 * (i & 3));
  return o;
}

// The V^T operand of P.V key step c (keys 16c .. 16c+15 of the tile) for dims 32 db .. +31 (vo =
// LaneOfs::v[db]): lane l gets dim 32 db + l % 32 of the keys 16c + 4h + r and 16c + 8 + 4h + r,
// r = 0..3, h = l / 32 -- the order in which the lane's P^T operand holds them.  Within a
// 16-lane group, lane i addresses row 16c + 4h + i / 4, dims c0 + 4 (i % 4); the transposing
// read returns column c0 + n of those 4 rows to lane n.
__device__ __forceinline__ h8 v_operand(const _Float16* Vb, int c, int vo) {
  typedef __attribute__((address_space(3))) s4v lds_s4;
  const s4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(Vb + vo + 16 * c * DK));
  const s4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(Vb + vo + (16 * c + 8) * DK));
  h8 r;
  __builtin_memcpy(&r, &lo, 8);
  __builtin_memcpy(reinterpret_cast<char*>(&r) + 8, &hi, 8);
  return r;
}

// One key tile of one wave's 32 queries: S^T = K . Q^T + bias, softmax against the running
// reference max m_run, O^T += V^T . P^T.
// FULL: both 32-key halves of the tile hold keys < L; otherwise only the first does, and the
// second is skipped (its P is 0).  MASK: the tile holds keys >= L, which get score -inf (a
// sequence's last tile).
//
// The reference max moves only when needed.  A query's scores lie in two lanes (the two key
// halves of each 8-key group), so its tile max is one permlane32 swap away; the reference
// m_run is moved to the running max, and O and l rescaled, only when some query's tile max
// exceeds m_run by more than 14 / log2(e) (always on the first tile, where m_run = -inf), so
// every P = 2^((s - m_run) log2e) stays at most 2^14, well inside f16.  Same result up to
// rounding: P and l carry the same factor, divided out at the end, and m_run is a score
// already seen, so l >= 1.  A rescale on every tile measured slower.  l sums the f16 P that the
// P.V product uses; it is kept per lane (this lane's keys) and reduced across the two lanes of
// a query only at the end.
template <bool FULL, bool MASK>
__device__ __forceinline__ void attn_tile(const _Float16* Ksb, const _Float16* Vb, const float* Bsb, int bofs,
                                          LaneOfs lo, const h8 (&qf)[4], bool qv, int k0, int L, float& m_run,
                                          float& l_run, f16v (&o)[2]) {
  constexpr int NS = FULL ? 2 : 1;  // 32-key halves with keys < L
  const int h = (threadIdx.x >> 5) & 1;
  // The offsets pass through an empty asm, so the compiler keeps these eight lane values and
  // folds each ring slot's base into the reads' immediate offsets, rather than holding a
  // precomputed address per slot.
  asm volatile("" : "+v"(bofs), "+v"(lo.k[0]), "+v"(lo.k[1]), "+v"(lo.k[2]), "+v"(lo.k[3]), "+v"(lo.v[0]),
               "+v"(lo.v[1]));
  // S^T[key][query] + bias: register r of half kb holds key 32 kb + 8 (r / 4) + 4 h + r % 4.
  // The accumulators start from the bias, so the matrix core does the add.  The lane's bias
  // address is formed once per tile and kept opaque, so its 32 reads (all within 60 floats)
  // pair up as ds_read2_b32 with immediate offsets from that one register; a slot base too large
  // for those offsets would otherwise be added per pair.
  typedef const __attribute__((address_space(3))) float lds_f;
  uint32_t baddr = lds_offset(Bsb) + 4u * (uint32_t)bofs;
  asm volatile("" : "+v"(baddr));
  lds_f* bsrc = (lds_f*)(uintptr_t)baddr;
  f16v s[NS];
#pragma unroll
  for (int kb = 0; kb < NS; kb++)
#pragma unroll
    for (int r = 0; r < 16; r++) s[kb][r] = bsrc[32 * kb + 8 * (r >> 2) + (r & 3)];
  // every LDS operand of the tile is read before the products that use it: the K operands
  // ahead of the score products, the V^T operands ahead of the softmax, whose VALU work covers
  // their latency
  h8 ka[4][NS];
#pragma unroll
  for (int ds = 0; ds < 4; ds++)
#pragma unroll
    for (int kb = 0; kb < NS; kb++) ka[ds][kb] = *reinterpret_cast<const h8*>(&Ksb[lo.k[ds] + 32 * kb * DK]);
#pragma unroll
  for (int ds = 0; ds < 4; ds++)
#pragma unroll
    for (int kb = 0; kb < NS; kb++) s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[ds][kb], qf[ds], s[kb], 0, 0, 0);
  h8 va[2 * NS][2];
#pragma unroll
  for (int c = 0; c < 2 * NS; c++)
#pragma unroll
    for (int db = 0; db < 2; db++) va[c][db] = v_operand(Vb, c, lo.v[db]);
  if (MASK) {
    const int lim = L - k0 - 4 * h;  // key 32 kb + 8 (r / 4) + 4 h + r % 4 >= L - k0
#pragma unroll
    for (int kb = 0; kb < NS; kb++)
#pragma unroll
      for (int r = 0; r < 16; r++)
        if (32 * kb + 8 * (r >> 2) + (r & 3) >= lim) s[kb][r] = -INFINITY;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < NS; kb++)
#pragma unroll
    for (int r = 0; r < 16; r++) mx = fmaxf(mx, s[kb][r]);
  mx = max_xor32(mx);  // finite: key k0 < L is valid
  // Only lanes of queries below L take part (qv), so that whatever the rows past L hold cannot
  // change when the valid queries rescale: the result stays independent of the batch around
  // the sequence.  !(x <= 14) also catches NaN.
  if (__any(qv && !((mx - m_run) * LOG2E <= 14.f))) {
    // the rescale of O sits in a branch of its own, so the accumulators keep their registers
    const float m_new = fmaxf(m_run, mx);
    // 1 where the max did not move, 0 on the first tile (O and l are still 0 there)
    const float corr = __builtin_amdgcn_exp2f((m_run - m_new) * LOG2E);
    m_run = m_new;
    l_run *= corr;
#pragma unroll
    for (int db = 0; db < 2; db++) o[db] *= corr;
  }
  const float mb = -m_run * LOG2E;

  // P = 2^(S log2e - m_run log2e) in f16; O^T[d][query] += V^T[d][keys] . P^T[keys][query] over
  // the 16-key steps of the valid halves, the P^T operand of step c being registers
  // 8 (c % 2) .. +7 of half c / 2; l += the f16 P, two at a time (v_dot2 with (1, 1))
  const h2 ones = {(_Float16)1.f, (_Float16)1.f};
#pragma unroll
  for (int c = 0; c < 2 * NS; c++) {
    h8 pb;
#pragma unroll
    for (int j = 0; j < 8; j++)
      pb[j] = (_Float16)__builtin_amdgcn_exp2f(__builtin_fmaf(s[c >> 1][8 * (c & 1) + j], LOG2E, mb));
#pragma unroll
    for (int j = 0; j < 8; j += 2) l_run = __builtin_amdgcn_fdot2(h2{pb[j], pb[j + 1]}, ones, l_run, false);
#pragma unroll
    for (int db = 0; db < 2; db++) o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[c][db], pb, o[db], 0, 0, 0);
  }
}

// A sequence of at most 128 tokens: one or two key tiles, whose work items hold 64 queries
// (attn_item_queries), taken by the four waves as 16 queries each on v_mfma_f32_16x16x32_f16 --
// half the chain of dependent work per wave of the 32-query path, which is what bounds such
// short launches -- and with no running max: the scores of every key are taken before the
// softmax, whose reference is their max.  Whether a sequence takes this path depends on its
// length only, so its result does not depend on the batch around it.
//
// Layouts of the 16x16x32 product: A lane l = row l % 16, K 8 (l / 16) .. +7; B lane l = column
// l % 16, the same K; D lane l register i = row 4 (l / 16) + i, column l % 16.  S^T = K . Q^T in
// key blocks of 16, so lane (lr, lg) = (l % 16, l / 16) holds query lr against keys
// 16 kb + 4 lg + i; the P^T operand of key step ks (32 keys) is then registers 0..3 of blocks
// 2 ks and 2 ks + 1, keys {32 ks + 4 lg + i, 32 ks + 16 + 4 lg + i}, and the V^T operand is read
// in that key order.  Key block kb lies in tile kb / 4 (Ks[kb / 4], Vs[kb / 4]).
template <int NKB>
__device__ __forceinline__ void small_tiles(const Slot& S0, const Slot& S1, const float* Bs, const h8 (&qf)[2], int L, int q0, int s0, int hd,
                                            int qi, const AttnArgs& p) {
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4, wave = threadIdx.x >> 6;
  constexpr int NKS = (NKB + 1) / 2;  // 32-key P.V steps holding keys < L
  // bias of (key j, query i) staged at j - i + 127
  const int bofs = 127 - q0 - 16 * wave - lr + 4 * lg;
  f4 s[2 * NKS];
#pragma unroll
  for (int kb = 0; kb < 2 * NKS; kb++)
#pragma unroll
    for (int i = 0; i < 4; i++) s[kb][i] = kb < NKB ? Bs[bofs + 16 * kb + i] : 0.f;
#pragma unroll
  for (int ds = 0; ds < 2; ds++)
#pragma unroll
    for (int kb = 0; kb < NKB; kb++) {
      const h8 a = *reinterpret_cast<const h8*>(&(kb >> 2 ? S1 : S0).k[swz<ROT_8>(16 * (kb & 3) + lr, 32 * ds + 8 * lg)]);
      s[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[ds], s[kb], 0, 0, 0);
    }
  float mx = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < 2 * NKS; kb++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      if (kb >= NKB || 16 * kb + 4 * lg + i >= L) s[kb][i] = -INFINITY;  // keys past L
      mx = fmaxf(mx, s[kb][i]);
    }
  mx = max_xor32(max_xor16(mx));  // finite: key 0 < L
  const float mb = -mx * LOG2E;
  const h2 ones = {(_Float16)1.f, (_Float16)1.f};
  float l = 0.f;
  h8 pb[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ks++) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      pb[ks][i] = (_Float16)__builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * ks][i], LOG2E, mb));
      pb[ks][4 + i] = (_Float16)__builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * ks + 1][i], LOG2E, mb));
    }
#pragma unroll
    for (int j = 0; j < 8; j += 2) l = __builtin_amdgcn_fdot2(h2{pb[ks][j], pb[ks][j + 1]}, ones, l, false);
  }
  l = sum_xor32(sum_xor16(l));
  // O^T[d][query] = V^T[d][keys] . P^T[keys][query]: lane (n, g) = (l % 16, l / 16) of 16-lane group g
  // reads rows 32 ks + 4 g + i / 4 (+ 16) of the step's tile, dims 16 db + 4 (i % 4); the
  // transposing read returns V[32 ks + 4 g + r][16 db + n] (and 16 rows on), the keys of its
  // P^T slots.
  typedef __attribute__((address_space(3))) s4v lds_s4;
  f4 o[4];
#pragma unroll
  for (int db = 0; db < 4; db++) {
    o[db] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < NKS; ks++) {
      const _Float16* Vt = (ks >> 1 ? S1 : S0).v;
      const int row = 32 * (ks & 1) + 4 * lg + (lr >> 2), col = 16 * db + 4 * (lr & 3);
      const s4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(Vt + swz<ROT_8>(row, col)));
      const s4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(Vt + swz<ROT_8>(row + 16, col)));
      h8 v;
      __builtin_memcpy(&v, &lo, 8);
      __builtin_memcpy(reinterpret_cast<char*>(&v) + 8, &hi, 8);
      o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(v, pb[ks], o[db], 0, 0, 0);
    }
  }
  if (qi < L) {  // written in operand order for the O GEMM
    const float inv = 1.0f / l;
    const int inner = p.heads * DK;
#pragma unroll
    for (int db = 0; db < 4; db++)
      *reinterpret_cast<h4*>(p.out + tiled_index(s0 + qi, hd * DK + 16 * db + 4 * lg, inner)) =
          h4{(_Float16)(o[db][0] * inv), (_Float16)(o[db][1] * inv), (_Float16)(o[db][2] * inv),
             (_Float16)(o[db][3] * inv)};
  }
}

// The loads of a sequence of at most 128 tokens: its one or two K and V tiles (rows past L
// repeat the last row) and the bias of distances -127 .. 128, all in one round trip, then the
// 64 queries from q0 (0 or 64).
__device__ __forceinline__ void small_sequence(const AttnArgs& p, Slot& S0, Slot& S1, int s0, int L, int q0, int hd, int wave, int lane) {
  const size_t head_stride = (size_t)p.tpad * DK;
  const _Float16* Q = p.qkv + ((size_t)0 * p.heads + hd) * head_stride + (size_t)s0 * DK;
  const _Float16* Kg = p.qkv + ((size_t)1 * p.heads + hd) * head_stride + (size_t)s0 * DK;
  const _Float16* Vg = p.qkv + ((size_t)2 * p.heads + hd) * head_stride + (size_t)s0 * DK;
  const float* lut = p.lut + (size_t)hd * (2 * p.lutw + 1) + p.lutw;
  const int ntile = (L + KT - 1) / KT;  // 1 or 2
  for (int t = 0; t < ntile; t++) {
    Slot& d = t ? S1 : S0;
    dma_tile<ROT_8>(Kg + (size_t)t * KT * DK, L - t * KT, d.k, wave, lane);
    dma_tile<ROT_8>(Vg + (size_t)t * KT * DK, L - t * KT, d.v, wave, lane);
  }
  lds_load4(lut + (64 * wave - 127), 4u * lane, lds_offset(S0.b + 64 * wave));
  const int lr = lane & 15, lg = lane >> 4, qi = q0 + 16 * wave + lr;
  const bool active = q0 + 16 * wave < L;  // wave-uniform
  h8 qf[2];
  if (active) {
    qf[0] = *reinterpret_cast<const h8*>(Q + (size_t)qi * DK + 8 * lg);
    qf[1] = *reinterpret_cast<const h8*>(Q + (size_t)qi * DK + 32 + 8 * lg);
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (!active) return;
  switch ((L + 15) >> 4) {
    case 1: small_tiles<1>(S0, S1, S0.b, qf, L, q0, s0, hd, qi, p); break;
    case 2: small_tiles<2>(S0, S1, S0.b, qf, L, q0, s0, hd, qi, p); break;
    case 3: small_tiles<3>(S0, S1, S0.b, qf, L, q0, s0, hd, qi, p); break;
    case 4: small_tiles<4>(S0, S1, S0.b, qf, L, q0, s0, hd, qi, p); break;
    case 5: small_tiles<5>(S0, S1, S0.b, qf, L, q0, s0, hd, qi, p); break;
    case 6: small_tiles<6>(S0, S1, S0.b, qf, L, q0, s0, hd, qi, p); break;
    case 7: small_tiles<7>(S0, S1, S0.b, qf, L, q0, s0, hd, qi, p); break;
    default: small_tiles<8>(S0, S1, S0.b, qf, L, q0, s0, hd, qi, p); break;
  }
}

__global__ __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(3))) void attn_relbias_kernel(AttnArgs p) {
  __shared__ Slot S0, S1, S2;  // the ring; tile t lives in slot t % 3

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int4 wk = p.work[blockIdx.x];
  const int s0 = wk.x, L = wk.y, q0 = wk.z, hd = wk.w;
  if (L == 0) return;  // an empty slot of the work list (the whole workgroup)
  if (L <= ATTN_SMALL_L) {  // one or two key tiles, 64-query items (uniform across the workgroup)
    small_sequence(p, S0, S1, s0, L, q0, hd, wave, lane);
    return;
  }
  const int l32 = lane & 31, h = lane >> 5;

  const size_t head_stride = (size_t)p.tpad * DK;
  const _Float16* Q = p.qkv + ((size_t)0 * p.heads + hd) * head_stride + (size_t)s0 * DK;
  const _Float16* Kg = p.qkv + ((size_t)1 * p.heads + hd) * head_stride + (size_t)s0 * DK;
  const _Float16* Vg = p.qkv + ((size_t)2 * p.heads + hd) * head_stride + (size_t)s0 * DK;
  // bias of distance d = j - i at lut[d], |d| <= lutw (lutw >= padded sequence length + QT)
  const float* lut = p.lut + (size_t)hd * (2 * p.lutw + 1) + p.lutw;

  // This lane's query (relative to the sequence start).  Queries past L compute on in-bounds
  // padding rows and are never stored.
  const int qi = q0 + wave * QW + l32;
  h8 qf[4];

  // A tile's loads, the same five per wave for every tile: K and V rows k0.. (clamped to the
  // sequence) and 64 of the bias values of distances k0 - q0 - (QT - 1) .. (QT + KT - 1 of the
  // 256 staged are read).
  auto load_tile = [&](int k0, _Float16* Kd, _Float16* Vd, float* Bd) __attribute__((always_inline)) {
    dma_tile<ROT_K>(Kg + (size_t)k0 * DK, L - k0, Kd, wave, lane);
    dma_tile<ROT_V>(Vg + (size_t)k0 * DK, L - k0, Vd, wave, lane);
    lds_load4(lut + (k0 - q0 - (QT - 1) + 64 * wave), 4u * lane, lds_offset(Bd + 64 * wave));
  };
  static_assert(LOADS == 5, "the wait below counts five loads per tile");

  float m_run = -INFINITY, l_run = 0.f;
  f16v o[2];
#pragma unroll
  for (int db = 0; db < 2; db++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[db][r] = 0.f;

  const int ntile = (L + KT - 1) / KT;
  // Bs index of this lane's (key 4h + r of the tile, query qi): (j - qi) - (k0 - q0 - (QT - 1))
  const int bofs = (QT - 1) - wave * QW - l32 + 4 * h;
  const LaneOfs lofs = lane_offsets(lane);
  // Tile t lives in slot t % 3.  Step t waits for this wave's loads of tile t (those of t + 1
  // may still be in flight), meets the other waves (every wave's part of tile t has landed, and
  // every wave is done with tile t - 1), issues tile t + 2 into the slot tile t - 1 used, then
  // computes tile t.  Every tile but the last is full; the last one holds keys past L unless L
  // is a multiple of 64, and its second half holds none below L when L - k0 <= 32.
  // act: whether this wave computes (below); tail: whether t may be the last tile.
  auto step = [&](auto act, auto tail, int t, const Slot& cur, Slot& next) __attribute__((always_inline)) {
    const bool last = decltype(tail)::value && t + 1 == ntile;
    // lgkmcnt(0): this wave's LDS reads of tile t - 1 have completed before any wave may refill
    // that slot (the compiler may have sunk their products past this point)
    if (!last) asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (t + 2 < ntile) load_tile((t + 2) * KT, next.k, next.v, next.b);
    if (!decltype(act)::value) return;
    const int k0 = t * KT;
    if (!last) attn_tile<true, false>(cur.k, cur.v, cur.b, bofs, lofs, qf, qi < L, k0, L, m_run, l_run, o);
    else if (L - k0 > 32) attn_tile<true, true>(cur.k, cur.v, cur.b, bofs, lofs, qf, qi < L, k0, L, m_run, l_run, o);
    else attn_tile<false, true>(cur.k, cur.v, cur.b, bofs, lofs, qf, qi < L, k0, L, m_run, l_run, o);
  };
  // The Q loads complete before tile 0, which is peeled off the loop, so that the loop body (whose
  // steps are never the last tile) carries a single tile variant and no wait on them.
  auto run = [&](auto act) __attribute__((always_inline)) {
    constexpr std::false_type body{};
    constexpr std::true_type tail{};
    load_tile(0, S0.k, S0.v, S0.b);
    if (ntile > 1) load_tile(KT, S1.k, S1.v, S1.b);
    if (decltype(act)::value) {
#pragma unroll
      for (int ds = 0; ds < 4; ds++) qf[ds] = *reinterpret_cast<const h8*>(Q + (size_t)qi * DK + 16 * ds + 8 * h);
      // The empty asm reads and redefines qf, so the compiler completes the Q loads here (its
      // wait also covers the first two tiles, issued just before) and no step waits on them.
      asm volatile("" : "+v"(qf[0]), "+v"(qf[1]), "+v"(qf[2]), "+v"(qf[3]));
    }
    step(act, tail, 0, S0, S2);
    int t = 1;
    for (; t + 3 < ntile; t += 3) {
      step(act, body, t, S1, S0);
      step(act, body, t + 1, S2, S1);
      step(act, body, t + 2, S0, S2);
    }
    if (t < ntile) step(act, tail, t, S1, S0);
    if (t + 1 < ntile) step(act, tail, t + 1, S2, S1);
    if (t + 2 < ntile) step(act, tail, t + 2, S0, S2);
  };
  // Waves whose 32 queries all lie past L (in a sequence's last query tile) only help load the
  // tiles, through the same waits and barriers.  The test is wave-uniform.
  const bool active = q0 + wave * QW < L;
  if (active) run(std::true_type{});
  else run(std::false_type{});
  l_run = sum_xor32(l_run);

  if (active && qi < L) {  // written in operand order for the O GEMM
    const float inv = 1.0f / l_run;
    const int inner = p.heads * DK;
#pragma unroll
    for (int db = 0; db < 2; db++)
#pragma unroll
      for (int a = 0; a < 4; a++) {
        const h4 v = {(_Float16)(o[db][4 * a] * inv), (_Float16)(o[db][4 * a + 1] * inv),
                      (_Float16)(o[db][4 * a + 2] * inv), (_Float16)(o[db][4 * a + 3] * inv)};
        *reinterpret_cast<h4*>(p.out + tiled_index(s0 + qi, hd * DK + 32 * db + 8 * a + 4 * h, inner)) = v;
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
  T5K_LAUNCH(attn_relbias_kernel, dim3((unsigned)n_work), dim3(64 * NWV), 0, s, a);
  return hipGetLastError();
}
}  // namespace t5k
