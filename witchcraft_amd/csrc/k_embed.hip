// k_embed.hip -- Embedder::embed post-processing for a batch of documents, on the device.
//
// Reference: src/embedder.rs:22-103, called once per document by Gatherer::next
// (src/lib.rs:930-934).  Each document is cut into windows of max_len tokens overlapping by
// `stride` (:38-63); every window is encoded as its own [1, L] sequence; a token's row is the
// sum, in window order, of its rows in the windows that cover it; tokens whose summed row has
// norm < MIN_NORM = 1.0 are dropped (:79-91); the kept rows are L2-normalised (:7-9,94).
//
// All windows of all documents are encoded as one packed batch (the caller), then three
// kernels over the documents' concatenated tokens produce the kept rows in document order:
//  1. embed_flags_kernel: summed row -> norm and keep flag per token, kept count per block;
//  2. embed_scan_kernel: exclusive prefix of the block counts (one workgroup);
//  3. embed_scatter_kernel: local prefix of the flags, summed row recomputed and normalised
//     into its compacted position, with the token's position in its document and, for the
//     first token of a document, the document's first output row.
#include "common.hpp"

namespace {

constexpr int EB_TOK = 64;  // tokens per workgroup (16 per wave)

// Summed row of token p of document d: windows k with k*step <= p < k*step + max_len, k < nwin.
// Lane holds columns lane + 64 i, i < P / 64 (<= 4).
__device__ __forceinline__ void window_row(const float* __restrict__ win, int4 doc, int p, int max_len, int step,
                                           int P, int lane, float (&v)[4]) {
  const int nwin = doc.w, row_base = doc.z;
  int k0 = p >= max_len ? (p - max_len) / step + 1 : 0;  // first k with k*step + max_len > p
  const int k1 = min(p / step, nwin - 1);
#pragma unroll
  for (int i = 0; i < 4; i++) v[i] = 0.f;
  for (int k = k0; k <= k1; k++) {
    const float* r = win + (size_t)(row_base + k * max_len + (p - k * step)) * P;
#pragma unroll
    for (int i = 0; i < 4; i++)
      if (lane + 64 * i < P) v[i] = k == k0 ? r[lane + 64 * i] : v[i] + r[lane + 64 * i];
  }
}

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// docs[d] = (first token of d in the concatenated token space, n tokens, first packed window row,
// number of windows); tok_doc[t] = document of token t.
__global__ __launch_bounds__(256) void embed_flags_kernel(const float* __restrict__ win, const int4* __restrict__ docs,
                                                          const int* __restrict__ tok_doc, int N, int max_len, int step,
                                                          int P, float* __restrict__ norms, uint8_t* __restrict__ flags,
                                                          int* __restrict__ block_counts) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __shared__ int cnt[4];
  int kept = 0;
  for (int j = 0; j < EB_TOK / 4; j++) {
    const int t = blockIdx.x * EB_TOK + wave * (EB_TOK / 4) + j;
    if (t >= N) break;
    const int4 doc = docs[tok_doc[t]];
    float v[4];
    window_row(win, doc, t - doc.x, max_len, step, P, lane, v);
    const float nrm = sqrtf(wave_sum64((v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3])));
    const bool keep = nrm >= 1.0f;  // MIN_NORM, src/embedder.rs:79-88
    if (lane == 0) {
      norms[t] = nrm;
      flags[t] = keep;
    }
    kept += keep;
  }
  if (lane == 0) cnt[wave] = kept;
  __syncthreads();
  if (threadIdx.x == 0) block_counts[blockIdx.x] = (cnt[0] + cnt[1]) + (cnt[2] + cnt[3]);
}

// Exclusive prefix of n block counts into offsets[0..n); offsets[n] = total.
__global__ __launch_bounds__(1024) void embed_scan_kernel(const int* __restrict__ counts, int n, int* __restrict__ offsets) {
  __shared__ int part[1024];
  __shared__ int carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int base = 0; base < n; base += 1024) {
    const int i = base + threadIdx.x;
    const int c = i < n ? counts[i] : 0;
    part[threadIdx.x] = c;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {  // inclusive scan (Hillis-Steele)
      const int add = threadIdx.x >= o ? part[threadIdx.x - o] : 0;
      __syncthreads();
      part[threadIdx.x] += add;
      __syncthreads();
    }
    if (i < n) offsets[i] = carry + part[threadIdx.x] - c;
    __syncthreads();
    if (threadIdx.x == 1023) carry += part[1023];
    __syncthreads();
  }
  if (threadIdx.x == 0) offsets[n] = carry;
}

__global__ __launch_bounds__(256) void embed_scatter_kernel(const float* __restrict__ win, const int4* __restrict__ docs,
                                                            const int* __restrict__ tok_doc, int N, int max_len, int step,
                                                            int P, const float* __restrict__ norms,
                                                            const uint8_t* __restrict__ flags,
                                                            const int* __restrict__ block_offsets, float* __restrict__ out,
                                                            int* __restrict__ kept_index, int* __restrict__ kept_offsets) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __shared__ int pos[EB_TOK];
  // exclusive prefix of the block's flags (block order = token order)
  if (threadIdx.x < EB_TOK) {
    const int t = blockIdx.x * EB_TOK + threadIdx.x;
    const uint64_t m = __ballot(t < N && flags[t]);
    pos[threadIdx.x] = block_offsets[blockIdx.x] + __popcll(m & ((1ull << threadIdx.x) - 1ull));
  }
  __syncthreads();
  for (int j = 0; j < EB_TOK / 4; j++) {
    const int lt = wave * (EB_TOK / 4) + j, t = blockIdx.x * EB_TOK + lt;
    if (t >= N) break;
    const int d = tok_doc[t];
    const int4 doc = docs[d];
    const int p = t - doc.x;
    if (p == 0 && lane == 0) kept_offsets[d] = pos[lt];  // the document's first output row
    if (!flags[t]) continue;
    float v[4];
    window_row(win, doc, p, max_len, step, P, lane, v);
    const float nrm = norms[t];
    float* o = out + (size_t)pos[lt] * P;
#pragma unroll
    for (int i = 0; i < 4; i++)
      if (lane + 64 * i < P) o[lane + 64 * i] = v[i] / nrm;  // normalize_l2, src/embedder.rs:7-9
    if (lane == 0) kept_index[pos[lt]] = p;
  }
}

}  // namespace

namespace t5k {
hipError_t launch_embed_batch(const float* win, const int4* docs, const int* tok_doc, int N, int max_len, int stride,
                              int P, float* norms, uint8_t* flags, int* block_counts, int* block_offsets, float* out,
                              int* kept_index, int* kept_offsets, hipStream_t s) {
  if (N <= 0) return hipSuccess;
  if (P <= 0 || P > 256 || P % 64 || stride < 0 || stride >= max_len) return hipErrorInvalidValue;
  const int nb = (N + EB_TOK - 1) / EB_TOK, step = max_len - stride;
  T5K_LAUNCH(embed_flags_kernel, dim3(nb), dim3(256), 0, s, win, docs, tok_doc, N, max_len, step, P, norms,
                     flags, block_counts);
  T5K_LAUNCH(embed_scan_kernel, dim3(1), dim3(1024), 0, s, block_counts, nb, block_offsets);
  T5K_LAUNCH(embed_scatter_kernel, dim3(nb), dim3(256), 0, s, win, docs, tok_doc, N, max_len, step, P, norms,
                     flags, block_offsets, out, kept_index, kept_offsets);
  return hipGetLastError();
}
int embed_batch_blocks(int N) { return (N + EB_TOK - 1) / EB_TOK; }
}  // namespace t5k
