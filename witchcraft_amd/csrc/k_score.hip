// k_score.hip -- query-side scoring next to the encoder: C = A . B^T in f32 and its per-row
// argmax (k-means assignment).
//
// Reference: fast_ops::matmul_t (src/fast_ops.rs:98-116) and PackedRight::matmul
// (:65-95), used for query x centroid / residual scores (src/lib.rs:637,735,759,1646), and
// matmul_argmax_batched (src/lib.rs:187-208, called at :235,1330).  The default build
// multiplies f32 x f32 (candle); the fbgemm build first truncates B to bf16
// (PackedMatrixBf16, fbgemm-rs/src/bf16.rs:21-31) and accumulates in f32 -- bf16_b selects it.
//
// f32 MFMA (v_mfma_f32_16x16x4_f32): products are exact f32 as on the CPU.  A lane holds 4
// consecutive K values of one row (one float4 load from global) and feeds them to 4
// consecutive MFMAs, each of which sums its K-lane group g = lane / 16 over k = 16 kb + 4 g + j;
// A and B use the same assignment, so every product a[k] b[k] is summed once.
//   * matmul_t: wave tile = 16 MB rows x 64 columns, MB = ceil(M / 16) up to 4, so query-sized
//     M (32 query tokens against many residuals, HBM-bound on B) pads to 16 rows at most.
//     Workgroup = 4 waves side by side along N (or along M when N <= 64).
//   * argmax:   workgroup = 4 waves on 64 rows, looping over N in 256-column chunks; the
//     running (max, index) per row lives in registers, the 4 waves' results meet in LDS.
//     Ties resolve to the smallest column index (candle's argmax keeps the first maximum).
#include "common.hpp"

#include <algorithm>
#include <atomic>

namespace {

typedef float f4v __attribute__((ext_vector_type(4)));

// Word 3 of a raw (stride 0) buffer descriptor on gfx9-family GPUs: 32-bit data format, so
// an access beyond num_records returns zero (loads) or is dropped (stores).
constexpr int kBufDword3 = 0x00020000;

__device__ __forceinline__ float4 ldg4(const float* p) { return *reinterpret_cast<const float4*>(p); }

__device__ __forceinline__ float4 trunc_bf16(float4 v) {
  auto t = [](float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x) & 0xffff0000u;
    return __builtin_bit_cast(float, u);
  };
  return make_float4(t(v.x), t(v.y), t(v.z), t(v.w));
}

// p[0..3] of one row (zero if !ok).  VEC: rows are 16-byte aligned (D % 4 == 0 and aligned
// bases), so one float4 load; otherwise 4 scalar loads.
template <bool VEC>
__device__ __forceinline__ float4 ld4(const float* p, bool ok) {
  if (VEC) return ok ? ldg4(p) : make_float4(0.f, 0.f, 0.f, 0.f);
  return ok ? make_float4(p[0], p[1], p[2], p[3]) : make_float4(0.f, 0.f, 0.f, 0.f);
}

// p[j] for j < n (zero past it, or everywhere if !ok): the last, partial K block.
__device__ __forceinline__ float4 ld4_tail(const float* p, int n, bool ok) {
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; j++) v[j] = (ok && j < n) ? p[j] : 0.f;
  return make_float4(v[0], v[1], v[2], v[3]);
}

template <int MB>
__device__ __forceinline__ void mfma_4x4(const float4 (&a)[4], const float4 (&b)[4], f4v (&acc)[4][4]) {
#pragma unroll
  for (int mb = 0; mb < MB; mb++)
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
      // B as the MFMA A operand: lane ends with 4 consecutive columns of one row
      acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(b[nb].x, a[mb].x, acc[mb][nb], 0, 0, 0);
      acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(b[nb].y, a[mb].y, acc[mb][nb], 0, 0, 0);
      acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(b[nb].z, a[mb].z, acc[mb][nb], 0, 0, 0);
      acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(b[nb].w, a[mb].w, acc[mb][nb], 0, 0, 0);
    }
}

// acc[mb][nb] += A[rows 16mb..] . B[cols 16nb..]^T over all of K for a 16 MB x 64 wave tile;
// rows / columns outside the matrices and K past D read as zero.  Full 16-wide K blocks run
// unguarded; the last partial block (D % 16 != 0) masks per element.
template <int MB, bool BF16B, bool VEC>
__device__ __forceinline__ void wave_tile(const float* __restrict__ A, const float* __restrict__ B, int M,
                                           int N, int D, int r0, int c0, int lane, f4v (&acc)[4][4]) {
  const int lr = lane & 15, lg = lane >> 4;
  const float* ar[4];
  const float* br[4];
  bool av[4], bv[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = r0 + 16 * i + lr, c = c0 + 16 * i + lr;
    av[i] = r < M;
    bv[i] = c < N;
    ar[i] = A + (size_t)(av[i] ? r : 0) * D + 4 * lg;
    br[i] = B + (size_t)(bv[i] ? c : 0) * D + 4 * lg;
  }
  const int dfull = D & ~15;
  for (int kb = 0; kb < dfull; kb += 16) {
    float4 a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      a[i] = i < MB ? ld4<VEC>(ar[i] + kb, av[i]) : make_float4(0.f, 0.f, 0.f, 0.f);
      b[i] = ld4<VEC>(br[i] + kb, bv[i]);
      if (BF16B) b[i] = trunc_bf16(b[i]);
    }
    mfma_4x4<MB>(a, b, acc);
  }
  if (dfull < D) {
    // this lane's 4 values are k = dfull + 4 lg + j, of which the first D - dfull - 4 lg exist
    const int n = D - dfull - 4 * lg;
    float4 a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      a[i] = i < MB ? ld4_tail(ar[i] + dfull, n, av[i]) : make_float4(0.f, 0.f, 0.f, 0.f);
      b[i] = ld4_tail(br[i] + dfull, n, bv[i]);
      if (BF16B) b[i] = trunc_bf16(b[i]);
    }
    mfma_4x4<MB>(a, b, acc);
  }
}

// With B as the MFMA A operand (16 columns) and A as the B operand (16 rows), lane l holds
// C[row 16mb + (l % 16)][cols 16nb + 4(l / 16) + 0..3].  wn = waves of the workgroup along N
// (4, or 1 when N <= 64, then the 4 waves stack along M).
template <int MB, bool BF16B, bool VEC>
__global__ __launch_bounds__(256) void matmul_t_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                       float* __restrict__ C, int M, int N, int D, int wn,
                                                       int tiles_n) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = 4 / wn;
  // 1-D grid, column tiles fastest: workgroups in flight share rows of A and walk B in order
  const int bm = blockIdx.x / tiles_n, bn = blockIdx.x - bm * tiles_n;
  const int r0 = (bm * wm + wave / wn) * 16 * MB, c0 = (bn * wn + wave % wn) * 64;
  if (r0 >= M || c0 >= N) return;  // wave-uniform; no workgroup barrier follows
  f4v acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f4v{0.f, 0.f, 0.f, 0.f};
  wave_tile<MB, BF16B, VEC>(A, B, M, N, D, r0, c0, lane, acc);
  const int lr = lane & 15, lg = lane >> 4;
  const bool vec_out = (N & 3) == 0 && VEC;
#pragma unroll
  for (int mb = 0; mb < MB; mb++) {
    const int r = r0 + 16 * mb + lr;
    if (r >= M) continue;
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
      const int c = c0 + 16 * nb + 4 * lg;
      float* out = C + (size_t)r * N + c;
      if (vec_out && c + 3 < N) {
        *reinterpret_cast<float4*>(out) = make_float4(acc[mb][nb][0], acc[mb][nb][1], acc[mb][nb][2], acc[mb][nb][3]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (c + i < N) out[i] = acc[mb][nb][i];
      }
    }
  }
}

// Query-sized A (M <= 16 MB <= 32) against a long B of 128-d rows, N % 4 == 0
// (src/lib.rs:734-735): a stream over B.  Persistent waves; wave w takes 32-column tiles
// w, w + W, w + 2W, ... (W = all waves of the grid, so the waves in flight cover one
// contiguous stretch of B).  A sits in LDS for the whole run, and the next tile's B loads
// are issued before the current tile's MFMAs and stores, so HBM streams while the f32
// MFMAs run.
template <int MB, bool BF16B>
__global__ __launch_bounds__(256, 2) void matmul_t_stream_kernel(const float* __restrict__ A,
                                                                 const float* __restrict__ B,
                                                                 float* __restrict__ C, int M, int N) {
  constexpr int D = 128, KB = D / 16, AS = D / 4 + 1;  // A row stride in LDS: 33 float4
  __shared__ float4 As[16 * MB * AS];
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
  // wave index made visibly uniform, so tile bases and descriptors live in scalar registers
  const int w0 = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = gridDim.x * 4;
  const int ntiles = (N + 31) / 32, nfull = N / 32, tail_bytes = (N % 32) * D * 4;
  // A (16 MB rows, rows past M repeat row M - 1) into LDS once; no barrier after this one
  for (int e = threadIdx.x; e < 16 * MB * (D / 4); e += 256) {
    const int r = e / (D / 4), q = e - r * (D / 4);
    As[r * AS + q] = ldg4(A + (size_t)min(r, M - 1) * D + 4 * q);
  }
  __syncthreads();
  // B tile t through a buffer descriptor whose range ends at column N: columns past N (the
  // last tile's tail, and the prefetch past the last tile) read as zero without touching
  // memory.  Lane offsets are loop-invariant, so no address registers live across the loop.
  const int voff[2] = {(lr * D + 4 * lg) * 4, ((16 + lr) * D + 4 * lg) * 4};
  auto load = [&](int t, float4 (&b)[KB][2]) {
    // (selected on the tile index rather than clamped: a clamp becomes a vector med3, whose
    // result register the allocator may take from a load still in flight)
    const int bytes = t < nfull ? 32 * D * 4 : (t == nfull ? tail_bytes : 0);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(B + (size_t)t * 32 * D), (short)0, bytes, kBufDword3);
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
      for (int kb = 0; kb < KB; kb++) {
        const f4v v = __builtin_amdgcn_raw_buffer_load_b128(rs, voff[nb] + 64 * kb, 0, 0);
        b[kb][nb] = make_float4(v[0], v[1], v[2], v[3]);
      }
  };
  auto compute = [&](const float4 (&b)[KB][2], f4v (&acc)[MB][2]) {
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
      for (int nb = 0; nb < 2; nb++) acc[i][nb] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < KB; kb++)
#pragma unroll
      for (int nb = 0; nb < 2; nb++) {
        const float4 bb = BF16B ? trunc_bf16(b[kb][nb]) : b[kb][nb];
#pragma unroll
        for (int i = 0; i < MB; i++) {
          const float4 a = As[(16 * i + lr) * AS + 4 * kb + lg];
          acc[i][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(bb.x, a.x, acc[i][nb], 0, 0, 0);
          acc[i][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(bb.y, a.y, acc[i][nb], 0, 0, 0);
          acc[i][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(bb.z, a.z, acc[i][nb], 0, 0, 0);
          acc[i][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(bb.w, a.w, acc[i][nb], 0, 0, 0);
        }
      }
  };
  // lane holds C[16 i + lr][32 t + 16 nb + 4 lg + 0..3]; N % 4 == 0, so a lane's 4 columns
  // are all inside or all outside [0, N)
  // (stores through a descriptor based at column 32 t; row offsets r N 4 < 2^31 is a launch
  // condition)
  int soff[MB];
#pragma unroll
  for (int i = 0; i < MB; i++) soff[i] = ((16 * i + lr) * N + 4 * lg) * 4;
  auto store = [&](int t, const f4v (&acc)[MB][2]) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(C + (size_t)t * 32), (short)0, 0x7fffffff, kBufDword3);
#pragma unroll
    for (int i = 0; i < MB; i++) {
      const bool row_ok = 16 * i + lr < M;
#pragma unroll
      for (int nb = 0; nb < 2; nb++)
        if (row_ok && 32 * t + 16 * nb + 4 * lg < N)
          __builtin_amdgcn_raw_buffer_store_b128(acc[i][nb], rs, soff[i] + 64 * nb, 0, 0);
    }
  };
  // Per tile: issue the next tile's loads, then the previous tile's stores, then this tile's
  // MFMAs.  Loads and stores share one in-order counter, so stores issued after the next
  // loads never hold up the wait for this tile's data.  Two tiles per trip let the B and
  // accumulator buffers alternate without copies; every bound is wave-uniform.  (The
  // scheduling barriers keep that issue order.)
  float4 b0[KB][2], b1[KB][2];
  f4v acc0[MB][2], acc1[MB][2];
  int t = w0, t1 = -1;  // t1: tile whose results wait in acc1
  load(t, b0);
  while (t < ntiles) {
    load(t + nw, b1);
    __builtin_amdgcn_sched_barrier(0);
    if (t1 >= 0) store(t1, acc1);
    __builtin_amdgcn_sched_barrier(0);
    compute(b0, acc0);
    const int t0 = t;
    t += nw;
    t1 = -1;
    if (t >= ntiles) {
      store(t0, acc0);
      break;
    }
    load(t + nw, b0);
    __builtin_amdgcn_sched_barrier(0);
    store(t0, acc0);
    __builtin_amdgcn_sched_barrier(0);
    compute(b1, acc1);
    t1 = t;
    t += nw;
  }
  if (t1 >= 0) store(t1, acc1);
}

// (v, i) beats (w, j) if v > w, or v == w and i < j (first maximum wins).
__device__ __forceinline__ void amax_merge(float& v, int& i, float w, int j) {
  if (w > v || (w == v && j < i)) {
    v = w;
    i = j;
  }
}

template <bool BF16B, bool VEC>
__global__ __launch_bounds__(256) void matmul_argmax_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                            uint32_t* __restrict__ out, int M, int N, int D) {
  __shared__ float sv[4][64];
  __shared__ int si[4][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int lr = lane & 15, lg = lane >> 4;
  const int r0 = blockIdx.x * 64;
  // running maximum of row 16mb + lr (identical in the 4 lanes of that row); starting from
  // (-inf, 0) keeps the result in range when no score exceeds -inf (NaN or -inf rows give 0)
  float bv[4];
  int bi[4];
#pragma unroll
  for (int mb = 0; mb < 4; mb++) {
    bv[mb] = -INFINITY;
    bi[mb] = 0;
  }
  for (int n0 = 0; n0 < N; n0 += 256) {
    const int c0 = n0 + wave * 64;
    if (c0 >= N) break;  // wave-uniform
    f4v acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[i][j] = f4v{0.f, 0.f, 0.f, 0.f};
    wave_tile<4, BF16B, VEC>(A, B, M, N, D, r0, c0, lane, acc);
#pragma unroll
    for (int mb = 0; mb < 4; mb++) {
      float v = -INFINITY;
      int ix = 0x7fffffff;
#pragma unroll
      for (int nb = 0; nb < 4; nb++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int c = c0 + 16 * nb + 4 * lg + i;
          if (c < N) amax_merge(v, ix, acc[mb][nb][i], c);
        }
      // combine the 4 lanes (lg = 0..3) holding this row: lanes l ^ 16, l ^ 32
#pragma unroll
      for (int o = 16; o <= 32; o <<= 1) {
        const float w = __shfl_xor(v, o);
        const int j = __shfl_xor(ix, o);
        amax_merge(v, ix, w, j);
      }
      amax_merge(bv[mb], bi[mb], v, ix);
    }
  }
  if (lg == 0)
#pragma unroll
    for (int mb = 0; mb < 4; mb++) {
      sv[wave][16 * mb + lr] = bv[mb];
      si[wave][16 * mb + lr] = bi[mb];
    }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int t = threadIdx.x, r = r0 + t;
    float v = sv[0][t];
    int ix = si[0][t];
    for (int w = 1; w < 4; w++) amax_merge(v, ix, sv[w][t], si[w][t]);
    if (r < M) out[r] = (uint32_t)ix;
  }
}

// k-means assignment (src/lib.rs:233-236, 1330) at D = 128 and large M: MFMA-bound.  Each
// wave owns 32 rows of A, held in registers for the whole run (16 float4 per lane); the 4
// waves of a workgroup share each 64-column chunk of B through LDS (double-buffered: the
// next chunk's global loads are issued before this chunk's MFMAs, one barrier per chunk).
// Global traffic per MFMA is a quarter of the per-wave tile above, which was bound by
// L2 -> CU bandwidth.  Per row: running (max, first index), as in matmul_argmax_kernel.
template <bool BF16B>
__global__ __launch_bounds__(256, 2) void matmul_argmax_rows_kernel(const float* __restrict__ A,
                                                                    const float* __restrict__ B,
                                                                    uint32_t* __restrict__ out, int M, int N) {
  constexpr int D = 128, KB = D / 16, BS = D / 4 + 1, RB = 2;  // LDS row stride: 33 float4
  __shared__ float4 Bs[2][64 * BS];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  const int r0 = blockIdx.x * (64 * RB) + wave * (16 * RB);
  // A fragments: row r0 + 16 mb + lr, K slice 16 kb + 4 lg; rows past M repeat row M - 1
  // (their results are not stored)
  float4 a[KB][4];
#pragma unroll
  for (int mb = 0; mb < RB; mb++) {
    const float* p = A + (size_t)min(r0 + 16 * mb + lr, M - 1) * D + 4 * lg;
#pragma unroll
    for (int kb = 0; kb < KB; kb++) a[kb][mb] = ldg4(p + 16 * kb);
  }
  // chunk loader: thread tid moves float4 q = tid + 256 j (j < 8) of the 64 x 32 float4 chunk;
  // columns past N repeat column N - 1 (masked out of the argmax)
  float4 st[8];
  auto gload = [&](int n0) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int q = tid + 256 * j, c = q >> 5, k4 = q & 31;
      st[j] = ldg4(B + (size_t)min(n0 + c, N - 1) * D + 4 * k4);
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int q = tid + 256 * j, c = q >> 5, k4 = q & 31;
      Bs[buf][c * BS + k4] = BF16B ? trunc_bf16(st[j]) : st[j];
    }
  };
  float bv[RB];
  int bi[RB];
#pragma unroll
  for (int mb = 0; mb < RB; mb++) {
    bv[mb] = -INFINITY;
    bi[mb] = 0;
  }
  const int nchunks = (N + 63) / 64;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int ch = 0; ch < nchunks; ch++) {
    const int buf = ch & 1, n0 = ch * 64;
    if (ch + 1 < nchunks) gload(n0 + 64);
    f4v acc[4][4];
#pragma unroll
    for (int i = 0; i < RB; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[i][j] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
      float4 b[4];
#pragma unroll
      for (int nb = 0; nb < 4; nb++) b[nb] = Bs[buf][(16 * nb + lr) * BS + 4 * kb + lg];
      mfma_4x4<RB>(a[kb], b, acc);
    }
#pragma unroll
    for (int mb = 0; mb < RB; mb++) {
      float v = -INFINITY;
      int ix = 0x7fffffff;
#pragma unroll
      for (int nb = 0; nb < 4; nb++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int c = n0 + 16 * nb + 4 * lg + i;
          if (c < N) amax_merge(v, ix, acc[mb][nb][i], c);
        }
#pragma unroll
      for (int o = 16; o <= 32; o <<= 1) {
        const float w = __shfl_xor(v, o);
        const int j = __shfl_xor(ix, o);
        amax_merge(v, ix, w, j);
      }
      amax_merge(bv[mb], bi[mb], v, ix);
    }
    if (ch + 1 < nchunks) {
      lstore(buf ^ 1);
      __syncthreads();
    }
  }
  if (lg == 0)
#pragma unroll
    for (int mb = 0; mb < RB; mb++) {
      const int r = r0 + 16 * mb + lr;
      if (r < M) out[r] = (uint32_t)bi[mb];
    }
}

}  // namespace

namespace t5k {
namespace {
bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// compute units of the current device (cached per device; 256 if the query fails)
int num_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v <= 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}
}  // namespace

hipError_t launch_matmul_t(const float* A, const float* B, float* C, int M, int N, int D, bool bf16_b,
                           hipStream_t s) {
  if (M <= 0 || N <= 0) return hipSuccess;
  if (D < 0) return hipErrorInvalidValue;
  const int mb = M >= 64 ? 4 : (M + 15) / 16;
  const int wn = N <= 64 ? 1 : 4, wm = 4 / wn;
  const long tiles_n = (N + 64L * wn - 1) / (64L * wn), tiles_m = (M + 16L * mb * wm - 1) / (16L * mb * wm);
  if (tiles_n * tiles_m > 0x7fffffffL) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(tiles_n * tiles_m));
  const bool vec = D % 4 == 0 && aligned16(A) && aligned16(B) && aligned16(C);
  if (vec && D == 128 && M <= 32 && N >= 4096 && N % 4 == 0 && 32L * N * 4 < (1L << 31)) {
    // query x residuals: persistent streaming kernel, 2 workgroups per CU
    const int wgs = (int)std::min<long>(2L * num_cus(), (N + 127) / 128);
    if (mb == 1) {
      if (bf16_b) hipLaunchKernelGGL((matmul_t_stream_kernel<1, true>), dim3(wgs), dim3(256), 0, s, A, B, C, M, N);
      else hipLaunchKernelGGL((matmul_t_stream_kernel<1, false>), dim3(wgs), dim3(256), 0, s, A, B, C, M, N);
    } else {
      if (bf16_b) hipLaunchKernelGGL((matmul_t_stream_kernel<2, true>), dim3(wgs), dim3(256), 0, s, A, B, C, M, N);
      else hipLaunchKernelGGL((matmul_t_stream_kernel<2, false>), dim3(wgs), dim3(256), 0, s, A, B, C, M, N);
    }
    return hipGetLastError();
  }
#define T5K_MMT(MBV, BF, VEC) \
  hipLaunchKernelGGL((matmul_t_kernel<MBV, BF, VEC>), grid, dim3(256), 0, s, A, B, C, M, N, D, wn, (int)tiles_n)
#define T5K_MMT_MB(BF, VEC)      \
  switch (mb) {                  \
    case 1: T5K_MMT(1, BF, VEC); break; \
    case 2: T5K_MMT(2, BF, VEC); break; \
    case 3: T5K_MMT(3, BF, VEC); break; \
    default: T5K_MMT(4, BF, VEC); break; \
  }
  if (bf16_b) {
    if (vec) { T5K_MMT_MB(true, true) } else { T5K_MMT_MB(true, false) }
  } else {
    if (vec) { T5K_MMT_MB(false, true) } else { T5K_MMT_MB(false, false) }
  }
#undef T5K_MMT_MB
#undef T5K_MMT
  return hipGetLastError();
}

hipError_t launch_matmul_argmax(const float* A, const float* B, uint32_t* out, int M, int N, int D, bool bf16_b,
                                hipStream_t s) {
  if (M <= 0) return hipSuccess;
  if (N <= 0 || D < 0) return hipErrorInvalidValue;
  const bool vec = D % 4 == 0 && aligned16(A) && aligned16(B);
  if (vec && D == 128 && M >= 256L * num_cus()) {
    // enough rows for two 128-row workgroups per CU: the register-A / LDS-B kernel
    const dim3 g((M + 127) / 128);
    if (bf16_b)
      hipLaunchKernelGGL((matmul_argmax_rows_kernel<true>), g, dim3(256), 0, s, A, B, out, M, N);
    else
      hipLaunchKernelGGL((matmul_argmax_rows_kernel<false>), g, dim3(256), 0, s, A, B, out, M, N);
    return hipGetLastError();
  }
  const dim3 grid((M + 63) / 64);
  if (bf16_b) {
    if (vec)
      hipLaunchKernelGGL((matmul_argmax_kernel<true, true>), grid, dim3(256), 0, s, A, B, out, M, N, D);
    else
      hipLaunchKernelGGL((matmul_argmax_kernel<true, false>), grid, dim3(256), 0, s, A, B, out, M, N, D);
  } else {
    if (vec)
      hipLaunchKernelGGL((matmul_argmax_kernel<false, true>), grid, dim3(256), 0, s, A, B, out, M, N, D);
    else
      hipLaunchKernelGGL((matmul_argmax_kernel<false, false>), grid, dim3(256), 0, s, A, B, out, M, N, D);
  }
  return hipGetLastError();
}
}  // namespace t5k
