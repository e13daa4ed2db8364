// k_misc.hip -- memory-bound kernels around the GEMMs: embedding gather, T5 RMSNorm,
// row norms / L2 normalisation.
#include "common.hpp"

namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Embedding gather (candle quantized_nn::Embedding, src/quantized_t5.rs:659,687):
// x[t] = table[ids[t]].  The table is f32 or Q4_K (dequantized on the fly, bit-exact).
// One wave per token.  Ids outside the vocabulary yield a zero row and set *err.
// With rec set (D <= EMB_NORM_MAX_D) the wave also emits the first block's T5LayerNorm in
// record mode, as rmsnorm_kernel does: the operand f16(x * gamma * s) and the token's record of
// rs floats (whole sum of squares in slot 0, s in slot rs - 1) for a GEMM that folds the norm.
constexpr int EMB_NORM_MAX_D = 1024;

__global__ __launch_bounds__(256) void embed_kernel(const uint32_t* __restrict__ ids, int T,
                                                    const void* __restrict__ table, int fmt, int vocab,
                                                    int D, float* __restrict__ x, unsigned* err,
                                                    const float* __restrict__ gamma, float eps,
                                                    _Float16* __restrict__ xn, float* __restrict__ rec,
                                                    int rs) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int lane = threadIdx.x & 63;
  const uint32_t id = ids[t];
  float* xr = x + (size_t)t * D;
  const bool bad = id >= (uint32_t)vocab;
  if (bad && lane == 0) *(volatile unsigned*)err = 1u;  // host-mapped flag; every writer stores 1
  if (fmt == EMB_F32 || bad) {
    // lane holds columns 4i .. 4i+3, i = lane + 64j
    const float4* src = reinterpret_cast<const float4*>((const float*)table + (size_t)(bad ? 0 : id) * D);
    float4 v[EMB_NORM_MAX_D / 256], g[EMB_NORM_MAX_D / 256];
    float ss = 0.f;
    if (rec) {
      // the row and gamma are requested together: one memory round trip before the sum
#pragma unroll
      for (int j = 0; j < EMB_NORM_MAX_D / 256; j++) {
        const int i = lane + 64 * j;
        v[j] = g[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < D / 4 && !bad) v[j] = src[i];
        if (i < D / 4) g[j] = reinterpret_cast<const float4*>(gamma)[i];
      }
#pragma unroll
      for (int j = 0; j < EMB_NORM_MAX_D / 256; j++) {
        const int i = lane + 64 * j;
        if (i < D / 4) reinterpret_cast<float4*>(xr)[i] = v[j];
        ss += (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
      }
      const float tot = wave_sum(ss);
      const float inv = 1.0f / sqrtf(tot / (float)D + eps);
      const float sc = norm_operand_scale(inv);
#pragma unroll
      for (int j = 0; j < EMB_NORM_MAX_D / 256; j++) {
        const int i = lane + 64 * j;
        if (i >= D / 4) continue;
        *reinterpret_cast<h4*>(xn + tiled_index(t, 4 * i, D)) =
            h4{(_Float16)((v[j].x * g[j].x) * sc), (_Float16)((v[j].y * g[j].y) * sc),
               (_Float16)((v[j].z * g[j].z) * sc), (_Float16)((v[j].w * g[j].w) * sc)};
      }
      if (lane < rs / 4) {
        float4* d = reinterpret_cast<float4*>(rec + (size_t)t * rs) + lane;
        *d = lane == 0 ? make_float4(tot, 0.f, 0.f, 0.f)
                       : (lane == rs / 4 - 1 ? make_float4(0.f, 0.f, 0.f, sc) : make_float4(0.f, 0.f, 0.f, 0.f));
      }
      return;
    }
    for (int i = lane; i < D / 4; i += 64)
      reinterpret_cast<float4*>(xr)[i] = bad ? make_float4(0.f, 0.f, 0.f, 0.f) : src[i];
    return;
  }
  // Q4_K table: D/256 blocks per row
  const uint8_t* row = (const uint8_t*)table + (size_t)id * (D / QK_K) * Q4K_BYTES;
  auto deq = [&](int e) {
    const uint8_t* b = row + (e / QK_K) * Q4K_BYTES;
    const int k = e % QK_K, c = k / 64, w = k % 64, hi = w >= 32, l = w & 31;
    const int jj = 2 * c + hi;
    const uint8_t* sb = b + 4;
    int sc, m;
    if (jj < 4) {
      sc = sb[jj] & 63;
      m = sb[jj + 4] & 63;
    } else {
      sc = (sb[jj + 4] & 15) | ((sb[jj - 4] >> 6) << 4);
      m = (sb[jj + 4] >> 4) | ((sb[jj] >> 6) << 4);
    }
    const float d = f16_bits_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    const float dmin = f16_bits_to_f32((uint32_t)b[2] | ((uint32_t)b[3] << 8));
    const uint8_t q = b[16 + 32 * c + l];
    const float ds = d * (float)sc, mm = dmin * (float)m;
    return ds * (float)(hi ? (q >> 4) : (q & 15)) - mm;
  };
  if (!rec) {
    for (int e = lane; e < D; e += 64) xr[e] = deq(e);
    return;
  }
  // lane holds columns lane + 64j; gamma is requested with the table bytes
  float v[EMB_NORM_MAX_D / 64], g[EMB_NORM_MAX_D / 64];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < EMB_NORM_MAX_D / 64; j++) {
    const int e = lane + 64 * j;
    g[j] = e < D ? gamma[e] : 0.f;
  }
#pragma unroll
  for (int j = 0; j < EMB_NORM_MAX_D / 64; j++) {
    const int e = lane + 64 * j;
    v[j] = 0.f;
    if (e >= D) continue;
    v[j] = deq(e);
    xr[e] = v[j];
    ss += v[j] * v[j];
  }
  const float tot = wave_sum(ss);
  const float inv = 1.0f / sqrtf(tot / (float)D + eps);
  const float sc = norm_operand_scale(inv);
#pragma unroll
  for (int j = 0; j < EMB_NORM_MAX_D / 64; j++) {
    const int e = lane + 64 * j;
    if (e < D) xn[tiled_index(t, e, D)] = (_Float16)((v[j] * g[j]) * sc);
  }
  if (lane < rs / 4) {
    float4* d = reinterpret_cast<float4*>(rec + (size_t)t * rs) + lane;
    *d = lane == 0 ? make_float4(tot, 0.f, 0.f, 0.f)
                   : (lane == rs / 4 - 1 ? make_float4(0.f, 0.f, 0.f, sc) : make_float4(0.f, 0.f, 0.f, 0.f));
  }
}

// T5LayerNorm (src/quantized_t5.rs:162-173): x / sqrt(mean(x^2) + eps) * w, emitted as the
// f16 GEMM operand (operand order, see tiled_index).  One workgroup per 16-row band: wave w
// owns the 16x32 operand blocks w, w+4, ... of the band, so each lane reads 32 contiguous bytes
// of its row per block and each block leaves as one contiguous 1 KiB store.  Up to RN_KEEP
// blocks per wave stay in registers between the sum of squares and the store (D <= 1024 reads x
// once).  Rows >= T of the last band are written as zeros.
constexpr int RN_KEEP = 8;

__device__ __forceinline__ float sq4(float4 v) { return v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w; }

__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ w,
                                                      _Float16* __restrict__ out, int T, int D,
                                                      float eps, float* __restrict__ rec, int rs) {
  __shared__ float part[4][16];
  // gamma of the kept blocks, staged once per workgroup: the per-lane gamma reads come from
  // LDS instead of adding as many global loads as the x reads themselves
  __shared__ __attribute__((aligned(16))) float gs[RN_KEEP * 4 * 32];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 15, c8 = (lane >> 4) * 8;
  const int t = blockIdx.x * 16 + r;
  const bool live = t < T;
  const int nblk = D >> 5;
  const int dk = D < RN_KEEP * 4 * 32 ? D : RN_KEEP * 4 * 32;  // gamma values staged
  const float* xr = x + (size_t)(live ? t : 0) * D + c8;
  // x of the kept blocks is requested at once: one memory round trip
  float4 keep[RN_KEEP][2];
#pragma unroll
  for (int j = 0; j < RN_KEEP; ++j) {
    const int kb = wave + 4 * j;
    keep[j][0] = keep[j][1] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (kb < nblk && live) {
      keep[j][0] = *reinterpret_cast<const float4*>(xr + kb * 32);
      keep[j][1] = *reinterpret_cast<const float4*>(xr + kb * 32 + 4);
    }
  }
  for (int i = threadIdx.x * 4; i < dk; i += 256 * 4)
    *reinterpret_cast<float4*>(gs + i) = *reinterpret_cast<const float4*>(w + i);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < RN_KEEP; ++j) ss += sq4(keep[j][0]) + sq4(keep[j][1]);
  for (int kb = wave + 4 * RN_KEEP; live && kb < nblk; kb += 4)
    ss += sq4(*reinterpret_cast<const float4*>(xr + kb * 32)) +
          sq4(*reinterpret_cast<const float4*>(xr + kb * 32 + 4));
  ss = sum_xor32(sum_xor16(ss));
  if (lane < 16) part[wave][lane] = ss;
  __syncthreads();  // also publishes gs
  const float tot = (part[0][r] + part[1][r]) + (part[2][r] + part[3][r]);
  const float inv = 1.0f / sqrtf(tot / (float)D + eps);
  _Float16* ob = out + (size_t)blockIdx.x * nblk * 512 + lane * 8;
  auto emit_n = [&](int kb, float4 a, float4 b, float4 ga, float4 gb) {
    h8 o = h8{(_Float16)((a.x * inv) * ga.x), (_Float16)((a.y * inv) * ga.y),
              (_Float16)((a.z * inv) * ga.z), (_Float16)((a.w * inv) * ga.w),
              (_Float16)((b.x * inv) * gb.x), (_Float16)((b.y * inv) * gb.y),
              (_Float16)((b.z * inv) * gb.z), (_Float16)((b.w * inv) * gb.w)};
    *reinterpret_cast<h8*>(ob + (size_t)kb * 512) = o;
  };
  // Record mode (the batched GEMMs fold the norm, see GemmArgs::rec): the operand is
  // f16(x * gamma * s) with the power of two s = norm_operand_scale(inv), and the token's
  // record of rs floats carries the whole sum of squares in slot 0 and s in its last slot, so the consuming
  // GEMM recomputes this same inv and scales its result by inv / s.
  const float sc = rec ? norm_operand_scale(inv) : 0.f;
  auto emit_s = [&](int kb, float4 a, float4 b, float4 ga, float4 gb) {
    h8 o = h8{(_Float16)((a.x * ga.x) * sc), (_Float16)((a.y * ga.y) * sc),
              (_Float16)((a.z * ga.z) * sc), (_Float16)((a.w * ga.w) * sc),
              (_Float16)((b.x * gb.x) * sc), (_Float16)((b.y * gb.y) * sc),
              (_Float16)((b.z * gb.z) * sc), (_Float16)((b.w * gb.w) * sc)};
    *reinterpret_cast<h8*>(ob + (size_t)kb * 512) = o;
  };
  auto emit = [&](int kb, float4 a, float4 b, float4 ga, float4 gb) {
    if (rec)
      emit_s(kb, a, b, ga, gb);
    else
      emit_n(kb, a, b, ga, gb);
  };
  if (rec && wave == 0 && lane < 16 && live) {
    float4* d = reinterpret_cast<float4*>(rec + (size_t)t * rs);
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    d[0] = make_float4(tot, 0.f, 0.f, 0.f);
    for (int i = 1; i < rs / 4 - 1; i++) d[i] = z;
    d[rs / 4 - 1] = make_float4(0.f, 0.f, 0.f, sc);
  }
#pragma unroll
  for (int j = 0; j < RN_KEEP; ++j) {
    const int kb = wave + 4 * j;
    if (kb < nblk)
      emit(kb, keep[j][0], keep[j][1], *reinterpret_cast<const float4*>(gs + kb * 32 + c8),
           *reinterpret_cast<const float4*>(gs + kb * 32 + c8 + 4));
  }
  for (int kb = wave + 4 * RN_KEEP; kb < nblk; kb += 4) {
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
    if (live) {
      a = *reinterpret_cast<const float4*>(xr + kb * 32);
      b = *reinterpret_cast<const float4*>(xr + kb * 32 + 4);
    }
    emit(kb, a, b, *reinterpret_cast<const float4*>(w + kb * 32 + c8),
         *reinterpret_cast<const float4*>(w + kb * 32 + c8 + 4));
  }
}

// L2 norm of each output row (src/embedder.rs:83) and optional normalisation (:7-9).
// A row whose norm is not finite sets *err: an f16 operand of some GEMM overflowed (a
// T5LayerNorm output |x * gamma| beyond the f16 range) or the weights hold non-finite values.
__global__ __launch_bounds__(256) void rownorm_kernel(float* __restrict__ y, float* __restrict__ norm,
                                                      int T, int P, int normalize, unsigned* err) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int lane = threadIdx.x & 63;
  float* r = y + (size_t)t * P;
  float ss = 0.f;
  for (int i = lane; i < P; i += 64) ss += r[i] * r[i];
  ss = wave_sum(ss);
  const float n = sqrtf(ss);
  if (lane == 0 && norm) norm[t] = n;
  if (lane == 0 && err && !__builtin_isfinite(n)) *(volatile unsigned*)err = 1u;  // every writer stores 1
  if (normalize)
    for (int i = lane; i < P; i += 64) r[i] = r[i] / n;
}

// f32 [T][K] row-major -> f16 GEMM operand (operand order).
__global__ void f32_to_f16_kernel(const float* __restrict__ x, _Float16* __restrict__ y, size_t n, int K) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[tiled_index(i / K, i % K, K)] = (_Float16)x[i];
}

// Attention work list from by-value arguments (no host staging buffer), the layout
// upload_batch writes: item q of entry i at work[pos[i] + 8 q] (its XCD's list), empty items
// for an entry of length 0.
__global__ __launch_bounds__(256) void work_list_kernel(t5k::WorkChunk c, int4* __restrict__ work) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= c.n) return;
  const int L = c.len[i], n = L ? attn_items(L) : c.start[i];
  for (int q = 0; q < n; q++)
    work[c.pos[i] + 8 * q] = L ? make_int4(c.start[i], L, q * attn_item_queries(L), c.head[i]) : make_int4(0, 0, 0, 0);
}

}  // namespace

namespace t5k {
hipError_t launch_embed(const uint32_t* ids, int T, const void* table, int fmt, int vocab, int D,
                        float* x, unsigned* err, hipStream_t s, const float* gamma, float eps, _Float16* xn,
                        float* rec, int rec_stride) {
  if (T <= 0) return hipSuccess;
  if (rec && (D > EMB_NORM_MAX_D || D % 32 || !gamma || !xn || (rec_stride != 16 && rec_stride != 64)))
    return hipErrorInvalidValue;
  T5K_LAUNCH(embed_kernel, dim3((T + 3) / 4), dim3(256), 0, s, ids, T, table, fmt, vocab, D, x, err,
                     gamma, eps, xn, rec, rec_stride);
  return hipGetLastError();
}
hipError_t launch_rmsnorm(const float* x, const float* w, _Float16* out, int T, int D, float eps,
                          hipStream_t s, float* rec, int rec_stride) {
  if (T <= 0) return hipSuccess;
  if (rec && rec_stride != 16 && rec_stride != 64) return hipErrorInvalidValue;
  T5K_LAUNCH(rmsnorm_kernel, dim3((T + 15) / 16), dim3(256), 0, s, x, w, out, T, D, eps, rec, rec_stride);
  return hipGetLastError();
}
hipError_t launch_rownorm(float* y, float* norm, int T, int P, int normalize, hipStream_t s, unsigned* err) {
  if (T <= 0) return hipSuccess;
  T5K_LAUNCH(rownorm_kernel, dim3((T + 3) / 4), dim3(256), 0, s, y, norm, T, P, normalize, err);
  return hipGetLastError();
}
hipError_t launch_f32_to_f16(const float* x, _Float16* y, size_t n, int K, hipStream_t s) {
  if (n == 0) return hipSuccess;
  T5K_LAUNCH(f32_to_f16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n, K);
  return hipGetLastError();
}
hipError_t launch_work_list(const WorkChunk& c, int4* work, hipStream_t s) {
  if (c.n <= 0) return hipSuccess;
  if (c.n > WorkChunk::CAP) return hipErrorInvalidValue;
  T5K_LAUNCH(work_list_kernel, dim3((c.n + 255) / 256), dim3(256), 0, s, c, work);
  return hipGetLastError();
}
}  // namespace t5k
