// k_gemv.hip -- dequant-GEMM for small token counts (M <= 64): the query path.
//
// Same product and epilogues as k_gemm.hip (C[M,N] = A[M,K] . W[N,K]^T, W Q4_K or f16,
// A f16 in operand order), shaped for the regime where the weights are read once and the
// launch is bound by HBM latency/bandwidth rather than by the matrix cores
// (reference: the query-side forward of T5EncoderModel, src/quantized_t5.rs:698-701, one
// [1, L] sequence at a time, L ~ 32).
//
//  * One workgroup owns 16 weight rows (one MFMA A operand) and MT blocks of 16 tokens (one, or
//    two where one would overflow the CUs, launch_wf); up to 16 wave64s split K into equal
//    ranges of one or two 64-wide chunks (K = 768: 12 waves; K = 2048: 16 waves), so every
//    weight byte of a token slice is read by exactly one lane.
//  * Each wave issues the raw loads of its chunks (Q4_K header + 8 nibble bytes per lane,
//    plus the activation operands) before unpacking any of them: one memory round trip.
//  * The partial accumulators meet in LDS and are summed in wave order (results do not
//    depend on timing); wave w then runs the epilogue of token block w.
//  * Optional fused T5LayerNorm: with GemmArgs::xf set, a prologue computes each token's
//    1/rms from the f32 residual stream and the operand is built as f16((x * inv) * gamma)
//    while loading -- the standalone RMSNorm launch and its round trip disappear.
//  * The residual epilogue fetches its x quad at kernel start.
//  * Folded T5LayerNorm (GemmArgs::rec, 64-float records): the residual GEMV stores the next
//    norm's operand f16(x * gamma * s) and its 16 columns' sum of x^2; the GEMV that consumes
//    it loads the f16 operand like any other and scales its sums by rsqrt(mean(x^2) + eps) / s
//    in the epilogue, so nothing waits on the norm before the dot products start.
#include "common.hpp"
#include "epilogue.hpp"
#include "q4k.hpp"

namespace {

// Raw bytes of one 64-wide K chunk of weight row n0 + lr for MFMA A-operand lane group lg:
// Q4_K: r0 = block header (d, dmin, scales), r1.xy = nibble bytes qs[32c + 8lg .. +7];
// f16: r0 = W[n][k + 8lg .. +7], r1 = W[n][k + 32 + 8lg .. +7].  n0 and k are wave-uniform, so
// each load is an SGPR base plus the lane's 32-bit byte offset (no per-lane 64-bit address math
// ahead of the launch's one memory round trip).
template <int WF>
__device__ __forceinline__ void wload(const void* W, int K, int n0, int lr, int k, int lg, uint4& r0, uint4& r1) {
  if constexpr (WF == WF_Q4K) {
    const uint8_t* blk = (const uint8_t*)W + ((size_t)n0 * (K / QK_K) + k / QK_K) * Q4K_BYTES;
    uint32_t ro = (uint32_t)(lr * (K / QK_K) * Q4K_BYTES);
    asm volatile("" : "+v"(ro));  // an opaque 32-bit lane offset: the saddr form, not a 64-bit VGPR address
    r0 = *reinterpret_cast<const uint4*>(blk + ro);
    const uint2 q = *reinterpret_cast<const uint2*>(blk + 16 + 32 * ((k % QK_K) / 64) + ro + 8u * lg);
    r1 = make_uint4(q.x, q.y, 0u, 0u);
  } else {
    const char* row = (const char*)((const _Float16*)W + (size_t)n0 * K + k);
    uint32_t ro = (uint32_t)(lr * K * 2 + 16 * lg);
    asm volatile("" : "+v"(ro));
    r0 = *reinterpret_cast<const uint4*>(row + ro);
    r1 = *reinterpret_cast<const uint4*>(row + 64 + ro);
  }
}

// A-operand fragments of the chunk: f0 = K slice k..k+31, f1 = k+32..k+63.
template <int WF>
__device__ __forceinline__ void wfrag(const uint4& r0, const uint4& r1, int k, h8& f0, h8& f1) {
  if constexpr (WF == WF_Q4K) {
    float s0, o0, s1, o1;
    chunk_scales(r0, (k % QK_K) / 64, s0, o0, s1, o1);
    h4 lo0, hi0, lo1, hi1;
    deq4(r1.x, s0, o0, s1, o1, lo0, hi0);
    deq4(r1.y, s0, o0, s1, o1, lo1, hi1);
    f0 = h8{lo0[0], lo0[1], lo0[2], lo0[3], lo1[0], lo1[1], lo1[2], lo1[3]};
    f1 = h8{hi0[0], hi0[1], hi0[2], hi0[3], hi1[0], hi1[1], hi1[2], hi1[3]};
  } else {
    f0 = __builtin_bit_cast(h8, r0);
    f1 = __builtin_bit_cast(h8, r1);
  }
}

// K chunks a wave loads per round: as many as fit the register budget of the launch bound
// (1024 threads -> 128 registers per lane, 512 -> 256), at most 4.
template <int G, int MT, bool NORM, int LB>
constexpr int gemv_group() {
  const int budget = LB == 1024 ? 112 : 224;  // headroom for addresses and conversions
  const int fixed = 4 * G * MT + 40;
  const int per_chunk = 8 * G + (NORM ? 16 * MT + 16 : 8 * MT);
  const int g = (budget - fixed) / per_chunk;
  return g >= 4 ? 4 : (g >= 2 ? 2 : 1);
}

// Workgroup = blockDim.x / 64 waves splitting K evenly (each owns K / 64 / waves chunks);
// dynamic LDS holds the waves' partial accumulators [waves][G][MT][64] f4.
template <int EPI, int WF, int MT, bool NORM, int LB>
__global__ __launch_bounds__(LB) void gemv_kernel(GemmArgs p) {
  constexpr int G = EPI == EPI_GATED ? 2 : 1;  // weight matrices (gate, up)
  constexpr int GROUP = gemv_group<G, MT, NORM, LB>();
  extern __shared__ f4 red[];
  __shared__ float rinv[NORM ? MT * 16 : 1];

  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int nw = blockDim.x >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int tb0 = blockIdx.y * MT;  // first 16-token block of this workgroup
  const int kw = p.K / nw, kbeg = wave * kw, nch = kw / 64;
  const size_t kblk = p.K / 32;
  // operand block (mt, kb) at (mt * K/32 + kb) * 512 halves; lane l reads its 16 bytes at 16 l
  const _Float16* xa = p.A;
  uint32_t xl = 16u * lane;
  asm volatile("" : "+v"(xl));
  const void* Wg[2] = {p.W0, p.W1};

  uint4 raw[GROUP][G][2];
  uint4 xr[NORM ? 1 : GROUP][2][MT];      // f16 operand blocks
  float4 xv[NORM ? GROUP : 1][2][MT][2];  // f32 rows for the fused norm
  float4 gv[NORM ? GROUP : 1][2][2];
  // Loads of chunks c0 .. c0+GROUP-1: weights (LOAD_W) and operands (LOAD_X), all issued
  // before any is used.
#define GEMV_LOAD_W(c0)                                                                          \
  _Pragma("unroll") for (int c = 0; c < GROUP; c++) {                                          \
    if ((c0) + c < nch) {                                                                      \
      const int k = kbeg + 64 * ((c0) + c);                                                    \
      _Pragma("unroll") for (int g = 0; g < G; g++)                                            \
          wload<WF>(Wg[g], p.K, n0, lr, k, lg, raw[c][g][0], raw[c][g][1]);                   \
    }                                                                                          \
  }
#define GEMV_LOAD_X(c0)                                                                          \
  _Pragma("unroll") for (int c = 0; c < GROUP; c++) {                                          \
    if ((c0) + c < nch) {                                                                      \
      const int k = kbeg + 64 * ((c0) + c);                                                    \
      _Pragma("unroll") for (int s = 0; s < 2; s++) {                                          \
        if constexpr (NORM) {                                                                  \
          const int kk = k + 32 * s + 8 * lg;                                                  \
          gv[c][s][0] = *reinterpret_cast<const float4*>(p.gamma + kk);                        \
          gv[c][s][1] = *reinterpret_cast<const float4*>(p.gamma + kk + 4);                    \
          _Pragma("unroll") for (int mt = 0; mt < MT; mt++) {                                  \
            const int t = (tb0 + mt) * 16 + lr;                                                \
            xv[c][s][mt][0] = xv[c][s][mt][1] = make_float4(0.f, 0.f, 0.f, 0.f);               \
            if (t < p.M) {                                                                     \
              xv[c][s][mt][0] = *reinterpret_cast<const float4*>(p.xf + (size_t)t * p.K + kk);     \
              xv[c][s][mt][1] = *reinterpret_cast<const float4*>(p.xf + (size_t)t * p.K + kk + 4); \
            }                                                                                  \
          }                                                                                    \
        } else {                                                                               \
          _Pragma("unroll") for (int mt = 0; mt < MT; mt++)                                    \
              xr[c][s][mt] = *reinterpret_cast<const uint4*>(                                  \
                  reinterpret_cast<const char*>(xa + ((size_t)(tb0 + mt) * kblk + k / 32 + s) * 512) + xl); \
        }                                                                                      \
      }                                                                                        \
    }                                                                                          \
  }
  GEMV_LOAD_W(0);
  GEMV_LOAD_X(0);

  // Residual epilogue: fetch this lane's x quad now, so the add does not wait on memory.
  float4 xres = make_float4(0.f, 0.f, 0.f, 0.f);
  if constexpr (EPI == EPI_RESID) {
    if (wave < MT && (tb0 + wave) * 16 + lr < p.M)
      xres = *reinterpret_cast<const float4*>((const float*)p.out + (size_t)((tb0 + wave) * 16 + lr) * p.ldo + n0 + 4 * lg);
  }

  // Fused T5LayerNorm (src/quantized_t5.rs:162-173): 1 / sqrt(mean(x^2) + eps) per token.
  // Each wave sums x^2 over its own K range from the operand values it holds anyway (the
  // lanes of one token then combine by shuffles), the waves' partials meet in LDS and are
  // added in wave order.  Only when a wave's chunks arrive in several rounds does it read
  // its K range once more for the sums.
  if constexpr (NORM) {
    constexpr int NT = MT * 16;
    __shared__ float part[16][NT];
    float ssl[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) ssl[mt] = 0.f;
    auto sq = [](float4 u) { return u.x * u.x + u.y * u.y + u.z * u.z + u.w * u.w; };
    if (nch <= GROUP) {
#pragma unroll
      for (int c = 0; c < GROUP; c++)
        if (c < nch)
#pragma unroll
          for (int s = 0; s < 2; s++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) ssl[mt] += sq(xv[c][s][mt][0]) + sq(xv[c][s][mt][1]);
    } else {
      for (int c = 0; c < nch; c++)
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
          for (int mt = 0; mt < MT; mt++) {
            const int t = (tb0 + mt) * 16 + lr;
            if (t < p.M) {
              const float* xp = p.xf + (size_t)t * p.K + kbeg + 64 * c + 32 * s + 8 * lg;
              ssl[mt] += sq(*reinterpret_cast<const float4*>(xp)) + sq(*reinterpret_cast<const float4*>(xp + 4));
            }
          }
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      ssl[mt] = sum_xor32(sum_xor16(ssl[mt]));
      if (lg == 0) part[wave][mt * 16 + lr] = ssl[mt];
    }
    __syncthreads();
    if (tid < NT) {
      float tot = 0.f;
      for (int w = 0; w < nw; w++) tot += part[w][tid];
      rinv[tid] = 1.0f / sqrtf(tot / (float)p.K + p.eps);
    }
    __syncthreads();
  }

  f4 acc[G][MT];
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[g][mt] = f4{0.f, 0.f, 0.f, 0.f};

  for (int c0 = 0; c0 < nch; c0 += GROUP) {
    if (c0) {
      GEMV_LOAD_W(c0);
      GEMV_LOAD_X(c0);
    }
#pragma unroll
    for (int c = 0; c < GROUP; c++) {
      if (c0 + c < nch) {
        const int k = kbeg + 64 * (c0 + c);
        h8 wf[G][2];
#pragma unroll
        for (int g = 0; g < G; g++) wfrag<WF>(raw[c][g][0], raw[c][g][1], k, wf[g][0], wf[g][1]);
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
          for (int mt = 0; mt < MT; mt++) {
            h8 xf;
            if constexpr (NORM) {  // same expression as the standalone RMSNorm kernel
              const float inv = rinv[mt * 16 + lr];
              const float4 a = xv[c][s][mt][0], b = xv[c][s][mt][1];
              const float4 ga = gv[c][s][0], gb = gv[c][s][1];
              xf = h8{(_Float16)((a.x * inv) * ga.x), (_Float16)((a.y * inv) * ga.y),
                      (_Float16)((a.z * inv) * ga.z), (_Float16)((a.w * inv) * ga.w),
                      (_Float16)((b.x * inv) * gb.x), (_Float16)((b.y * inv) * gb.y),
                      (_Float16)((b.z * inv) * gb.z), (_Float16)((b.w * inv) * gb.w)};
            } else {
              xf = __builtin_bit_cast(h8, xr[c][s][mt]);
            }
#pragma unroll
            for (int g = 0; g < G; g++)
              acc[g][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[g][s], xf, acc[g][mt], 0, 0, 0);
          }
      }
    }
  }
#undef GEMV_LOAD_W
#undef GEMV_LOAD_X

  // Folded T5LayerNorm (GemmArgs::rec, 64-float records): the epilogue wave of token block
  // mt = wave fetches its token's record while the partial sums meet in LDS -- as a consumer
  // the 63 partial sums (lane group lg holds slots 16lg .. 16lg + 15) and the operand scale,
  // as a producer that scale and gamma.  (Fetched before the K loop they would stay live
  // through it and spill at the 1024-thread register budget.)
  float4 nrec[4];
  float nsc = 1.f;
  float4 ngam = make_float4(0.f, 0.f, 0.f, 0.f);
  if (p.rec && wave < MT) {
    const float* r = p.rec + (size_t)((tb0 + wave) * 16 + lr) * NORM_REC_GEMV;
    nsc = r[NORM_REC_GEMV - 1];
    if constexpr (EPI == EPI_RESID) {
      ngam = *reinterpret_cast<const float4*>(p.ngamma + n0 + 4 * lg);
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) nrec[i] = reinterpret_cast<const float4*>(r + 16 * lg)[i];
    }
  }

#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++) red[((wave * G + g) * MT + mt) * 64 + lane] = acc[g][mt];
  __syncthreads();

  // lane holds C[token 16mt + lr][columns n0 + 4lg .. +3]; partials summed in wave order
  for (int mt = wave; mt < MT; mt += nw) {
    f4 v[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
      v[g] = red[(g * MT + mt) * 64 + lane];
      for (int w = 1; w < nw; w++) v[g] += red[((w * G + g) * MT + mt) * 64 + lane];
    }
    const int m = (tb0 + mt) * 16 + lr;
    const bool live = m < p.M;
    const float* rrow = p.rec ? p.rec + (size_t)m * NORM_REC_GEMV : nullptr;
    if constexpr (EPI == EPI_RESID) {  // x quad prefetched above for mt == wave
      float4* xp = reinterpret_cast<float4*>((float*)p.out + (size_t)m * p.ldo + n0 + 4 * lg);
      float4 r = mt == wave ? xres : (live ? *xp : make_float4(0.f, 0.f, 0.f, 0.f));
      r = make_float4(r.x + v[0][0], r.y + v[0][1], r.z + v[0][2], r.w + v[0][3]);
      if (live) *xp = r;
      if (p.nx) {  // next norm: f16(x * gamma * s) and the sum of x^2 over these 16 columns
        const float sc = mt == wave ? nsc : rrow[NORM_REC_GEMV - 1];
        const float4 g = mt == wave ? ngam : *reinterpret_cast<const float4*>(p.ngamma + n0 + 4 * lg);
        const float ss = sum_xor32(sum_xor16((r.x * r.x + r.y * r.y) + (r.z * r.z + r.w * r.w)));
        if (live) {
          *reinterpret_cast<h4*>(p.nx + tiled_index(m, n0 + 4 * lg, p.ldo)) =
              h4{(_Float16)((r.x * g.x) * sc), (_Float16)((r.y * g.y) * sc), (_Float16)((r.z * g.z) * sc),
                 (_Float16)((r.w * g.w) * sc)};
          if (lg == 0) p.rec[(size_t)m * NORM_REC_GEMV + n0 / 16] = ss;
        }
      }
      continue;
    } else {
      if (p.rec) {  // folded norm: scale by rsqrt(mean(x^2) + eps) / s
        float4 q[4];
        float sc;
        if (mt == wave) {
#pragma unroll
          for (int i = 0; i < 4; i++) q[i] = nrec[i];
          sc = nsc;
        } else {
#pragma unroll
          for (int i = 0; i < 4; i++) q[i] = reinterpret_cast<const float4*>(rrow + 16 * lg)[i];
          sc = rrow[NORM_REC_GEMV - 1];
        }
        // slots 16lg + 4i + j; those past K / 16 (and slot 63, the scale) are masked: the
        // record array may hold another layout's data there
        const int ns = p.K / 16;
        float part = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int t = 16 * lg + 4 * i;
          part += ((t < ns ? q[i].x : 0.f) + (t + 1 < ns ? q[i].y : 0.f)) +
                  ((t + 2 < ns ? q[i].z : 0.f) + (t + 3 < ns ? q[i].w : 0.f));
        }
        const float tot = sum_xor32(sum_xor16(part));
        const float inv = 1.0f / sqrtf(tot / (float)p.K + p.eps);
        const float f = inv / sc;
#pragma unroll
        for (int g = 0; g < G; g++) v[g] *= f;
        if (p.rec_next && blockIdx.x == 0 && lg == 0 && live)
          p.rec_next[(size_t)m * NORM_REC_GEMV + NORM_REC_GEMV - 1] = norm_operand_scale(inv);
      }
      if (!live) continue;
      if constexpr (EPI == EPI_GATED) {
        store_quad_gated(p, m, n0 + 4 * lg, v[0], v[G - 1]);
      } else {
        store_quad<EPI>(p, m, n0 + 4 * lg, v[0]);
      }
    }
  }
}

// Waves per workgroup: the most (<= cap) that divide the K/64 chunks evenly while the
// partial accumulators fit 64 KiB of LDS.
int gemv_waves(int K, int G, int MT, int cap) {
  const int nch = K / 64;
  for (int w : {16, 12, 8, 6, 4, 3, 2})
    if (w <= cap && nch % w == 0 && w * G * MT <= 64) return w;
  return 1;
}

template <int EPI, int WF, int MT, bool NORM>
hipError_t launch_mt(const GemmArgs& a, hipStream_t s) {
  constexpr int G = EPI == EPI_GATED ? 2 : 1;
  // 12-16 waves (128 registers each) only where a chunk's operands fit that budget
  constexpr bool WIDE = G * MT * 12 <= 64 && !(NORM && MT == 4);
  const int nw = gemv_waves(a.K, G, MT, WIDE ? 16 : 8);
  const size_t lds = (size_t)nw * G * MT * 64 * sizeof(f4);
  const dim3 grid(a.N / 16, (a.M + 16 * MT - 1) / (16 * MT));
  if constexpr (WIDE) {
    if (nw > 8) {
      T5K_LAUNCH((gemv_kernel<EPI, WF, MT, NORM, 1024>), grid, dim3(64 * nw), lds, s, a);
      return hipGetLastError();
    }
  }
  T5K_LAUNCH((gemv_kernel<EPI, WF, MT, NORM, 512>), grid, dim3(64 * nw), lds, s, a);
  return hipGetLastError();
}

// Token blocks per workgroup.  Each workgroup streams the activations of its own tokens, which
// is what bounds these launches (each CU receives activation bytes at a fixed rate), while the
// weight rows are re-read per token block from L2.  So one 16-token block per workgroup, unless
// that overflows the CUs into a second, mostly empty round of workgroups: then all tokens of a
// 32-token block pair (QKV, N = 2304 at 32 tokens: 288 -> 144 workgroups, 5.1 -> 4.2 us).  Both
// give the same bits: an output's K order is fixed by the waves' K split alone.  (Half blocks of
// 8 tokens for the N = 768 launches, 192 workgroups, measured slower: wo 5.4 -> 6.1 us.)
template <int EPI, int WF, bool NORM>
hipError_t launch_wf(const GemmArgs& a, hipStream_t s) {
  const int cus = a.cus > 0 ? a.cus : 256, cols = a.N / 16;
  const int b16 = (a.M + 15) / 16, b32 = (a.M + 31) / 32;
  if (cols * b16 > cus && b32 < b16) return launch_mt<EPI, WF, 2, NORM>(a, s);
  return launch_mt<EPI, WF, 1, NORM>(a, s);
}

template <int EPI>
hipError_t launch_epi(int wfmt, const GemmArgs& a, hipStream_t s) {
  // the residual update never takes a normalised operand (its input is attention or FFN output)
  constexpr bool CAN_NORM = EPI != EPI_RESID;
  if (a.xf) {
    if (!CAN_NORM) return hipErrorInvalidValue;
    return wfmt == WF_Q4K ? launch_wf<EPI, WF_Q4K, CAN_NORM>(a, s) : launch_wf<EPI, WF_F16, CAN_NORM>(a, s);
  }
  return wfmt == WF_Q4K ? launch_wf<EPI, WF_Q4K, false>(a, s) : launch_wf<EPI, WF_F16, false>(a, s);
}

}  // namespace

namespace t5k {
hipError_t launch_gemv(int epi, int wfmt, const GemmArgs& a, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (a.M > GEMV_MAX_M || a.N % 16 || a.K % 256 || (a.xf && !a.gamma)) return hipErrorInvalidValue;
  // folded T5LayerNorm: the row must fit one 64-float record
  if (a.rec && a.xf) return hipErrorInvalidValue;
  if (epi == EPI_RESID && a.nx && (!a.rec || !a.ngamma || a.N != a.ldo || a.N > 16 * (NORM_REC_GEMV - 1)))
    return hipErrorInvalidValue;
  if (epi != EPI_RESID && a.rec && a.K > 16 * (NORM_REC_GEMV - 1)) return hipErrorInvalidValue;
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
