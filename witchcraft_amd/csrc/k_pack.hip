// k_pack.hip -- Witchcraft's packed chunk-embedding codec on the GPU, byte-exact with the
// reference: embeddings_to_packed / embeddings_from_packed (src/packops.rs:172-301, :303-438),
// haar_forward/inverse_mirror_edge (src/haarops.rs:4-70), rANS64 (src/rans64.rs, ryg_rans).
//
// A batch holds many matrices ([rows][cols] f32, cols <= 255); each is cut into windows of at
// most 1024 rows.  The host builds one PkWin per window (offsets only); every transform, the
// entropy coder and the assembly of the output bytes run here:
//   encode: pk_colsort (column sums in row order, stable rank sort, inverse permutation bytes)
//           -> pk_haar_rows (permute + row transform, one wave per row)
//           -> pk_haar_cols (column transform in LDS, 8 columns per workgroup)
//           -> pk_quant (max |x| < 1, symbols round(29 x) folded to unsigned, histogram over
//              the used symbol range in 8192-bin LDS passes, scale_histogram)
//           -> pk_rans_enc (one workgroup per window: per-position coder parameters staged in
//              LDS in parallel, then the wave-uniform state loop writes 32-bit words backwards)
//           -> pk_assemble (header pieces and stream copied to host-computed offsets).
//   decode: pk_rans_dec (decode table in LDS, wave-uniform state loop, values in reverse)
//           -> pk_haar_rows<inverse> -> pk_haar_cols<inverse> -> pk_unpermute_norm.
// rANS64 has one state per window and the format fixes one stream per window, so the coder
// runs one stream per workgroup; windows run in parallel.
//
// Float arithmetic follows the reference operation by operation (two roundings for a*b + c,
// sequential sums in the reference's order, correctly rounded division and square root), so
// the bytes match exactly.
#include "common.hpp"

#pragma clang fp contract(off)

namespace t5k {
// One window of one matrix.  Host-filled: row0 (first row in the batch's row space), rows,
// cols (all windows share it), hdr (byte offset of the window's header scratch slot), data
// (byte offset of its rANS scratch, capacity 2 * rows * cols + 16), plus the decoder's input
// offsets.  Kernel-filled: m (histogram size), dlen (stream bytes), err.
struct PkWin {
  int row0, rows;
  long long hdr, data;    // scratch offsets (encode) / input offsets of perm+pairs, stream (decode)
  int m, dlen, err, pad;  // filled by pk_quant / pk_rans_enc; decode: m and dlen are inputs
};
}  // namespace t5k

namespace {

using t5k::PkWin;

constexpr float INV_SQRT2 = 0.7071067811865475f;
constexpr int RANS_BITS = 12, RANS_TOTAL = 1 << RANS_BITS;
constexpr unsigned long long RANS_L = 1ull << 31;

enum PkErr : int { PK_OK = 0, PK_NAN = 1, PK_HIST = 2, PK_OVERFLOW = 3, PK_CORRUPT = 4 };

// ---- encode 1: column sums (each column summed in row order, as the reference's r-outer
// loop does), stable rank by sum, inverse permutation bytes.  One workgroup per window. ----
__global__ __launch_bounds__(256) void pk_colsort(const float* __restrict__ x, PkWin* __restrict__ win, int cols,
                                                   uint8_t* __restrict__ hdr_scratch, int* __restrict__ perm_out) {
  __shared__ float sums[256];
  PkWin& w = win[blockIdx.x];
  const int c = threadIdx.x;
  // identity first: with a NaN sum the ranks below may collide (the window then fails), and
  // every slot must still hold a valid column for the row pass
  perm_out[(size_t)blockIdx.x * 256 + c] = c < cols ? c : 0;
  if (c < cols) {
    const float* p = x + (size_t)w.row0 * cols + c;
    float s = 0.f;
    for (int r = 0; r < w.rows; r++) s += p[(size_t)r * cols];
    sums[c] = s;
  }
  __syncthreads();  // also orders the identity fill before the ranked writes
  if (c < cols) {
    const float s = sums[c];
    if (s != s) atomicMax(&w.err, (int)PK_NAN);  // partial_cmp().unwrap() panics on NaN
    int rank = 0;
    for (int j = 0; j < cols; j++) {
      const float t = sums[j];
      rank += (t < s || (t == s && j < c)) ? 1 : 0;
    }
    hdr_scratch[w.hdr + c] = (uint8_t)rank;          // inv_perm[c] = new position of column c
    perm_out[(size_t)blockIdx.x * 256 + rank] = c;   // perm[new] = original column
  }
}

// Haar forward / inverse of one length-n vector held in LDS (v, scratch t), by one wave.
template <bool INV>
__device__ void haar_wave(float* v, float* t, int n, int lane) {
  if (!INV) {
    int m = n;
    while (m > 1) {
      const int pairs = m / 2, odd = m & 1, nc = pairs + odd;
      for (int i = lane; i < pairs; i += 64) {
        const float a = v[2 * i], b = v[2 * i + 1];
        t[i] = (a + b) * INV_SQRT2;
        t[nc + i] = (a - b) * INV_SQRT2;
      }
      if (odd && lane == 0) {
        const float a = v[m - 1];
        t[pairs] = (a + a) * INV_SQRT2;
      }
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      for (int i = lane; i < m; i += 64) v[i] = t[i];
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      m = nc;
    }
  } else {
    int levels[12], nl = 0, m = n;
    levels[nl++] = m;
    while (m > 1) {
      m = m / 2 + (m & 1);
      levels[nl++] = m;
    }
    for (int l = nl - 1; l >= 1; l--) {
      const int np = levels[l - 1], odd = np & 1, pairs = np / 2, nc = pairs + odd;
      for (int i = lane; i < pairs; i += 64) {
        const float sum = v[i], diff = v[nc + i];
        t[2 * i] = (sum + diff) * INV_SQRT2;
        t[2 * i + 1] = (sum - diff) * INV_SQRT2;
      }
      if (odd && lane == 0) t[np - 1] = v[nc - 1] * INV_SQRT2;
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      for (int i = lane; i < np; i += 64) v[i] = t[i];
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
  }
}

// ---- encode 2 / decode 3: rows.  One wave per row (4 rows per workgroup).  Encode gathers
// the row through the column permutation first. ----
template <bool INV>
__global__ __launch_bounds__(256) void pk_haar_rows(const float* __restrict__ src, float* __restrict__ dst,
                                                     int total_rows, int cols, const int* __restrict__ row_win,
                                                     const int* __restrict__ perm) {
  __shared__ float buf[4][2][256];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + wv;
  if (row >= total_rows) return;  // wave-uniform; only wave barriers follow
  float* v = buf[wv][0];
  float* t = buf[wv][1];
  const float* s = src + (size_t)row * cols;
  const int* pm = INV ? nullptr : perm + (size_t)row_win[row] * 256;
  for (int c = lane; c < cols; c += 64) {
    int sc = c;
    if (!INV) {
      sc = pm[c];
      sc = (unsigned)sc < (unsigned)cols ? sc : 0;
    }
    v[c] = s[sc];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  haar_wave<INV>(v, t, cols, lane);
  for (int c = lane; c < cols; c += 64) dst[(size_t)row * cols + c] = v[c];
}

// ---- encode 3 / decode 4: columns, in place.  Workgroup = (window, 8 columns); one wave per
// column pair; columns of up to 1024 rows in LDS. ----
template <bool INV>
__global__ __launch_bounds__(256) void pk_haar_cols(float* __restrict__ x, const PkWin* __restrict__ win, int cols) {
  __shared__ float buf[8][2][1024];
  const PkWin& w = win[blockIdx.x];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = w.rows;
  for (int k = 0; k < 2; k++) {
    const int c = blockIdx.y * 8 + wv * 2 + k;
    if (c >= cols) break;  // wave-uniform
    float* v = buf[wv * 2 + k][0];
    float* t = buf[wv * 2 + k][1];
    float* col = x + (size_t)w.row0 * cols + c;
    for (int r = lane; r < n; r += 64) v[r] = col[(size_t)r * cols];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    haar_wave<INV>(v, t, n, lane);
    for (int r = lane; r < n; r += 64) col[(size_t)r * cols] = v[r];
  }
}

// f32 -> unsigned symbol exactly as packops.rs does it (round(29 x) folded; Rust's saturating
// float -> usize cast, then the wrapping cast to u16).
__device__ __forceinline__ uint32_t pk_symbol(float v) {
  const float q = roundf(29.0f * v);
  const float sf = 2.0f * fabsf(q) + (q < 0.0f ? 1.0f : 0.0f);
  unsigned long long s;
  if (!(sf >= 1.0f)) s = 0;
  else if (sf >= 18446744073709551616.0f) s = ~0ull;
  else s = (unsigned long long)sf;
  return (uint32_t)(uint16_t)(s > 0 ? s - 1 : 0);
}

// ---- encode 4: scaling, symbols, histogram, scale_histogram.  One 1024-thread workgroup per
// window. ----
constexpr int HBINS = 8192;
__global__ __launch_bounds__(1024) void pk_quant(const float* __restrict__ x, PkWin* __restrict__ win, int cols,
                                                  uint16_t* __restrict__ syms, uint8_t* __restrict__ hdr_scratch,
                                                  uint32_t* __restrict__ pairs_scratch) {
  __shared__ uint32_t hist[HBINS];
  __shared__ float red[32];
  __shared__ uint32_t ured[32];
  __shared__ uint32_t cnt_m;
  PkWin& w = win[blockIdx.x];
  const int n = w.rows * cols, tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
  const float* v = x + (size_t)w.row0 * cols;
  uint16_t* sy = syms + (size_t)w.row0 * cols;
  // max over |x| < 1 (exact in any order), floor 1e-5
  float am = 0.00001f;
  for (int i = tid; i < n; i += 1024) {
    const float a = fabsf(v[i]);
    if (a < 1.0f && a > am) am = a;
  }
  for (int o = 32; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
  if (lane == 0) red[wid] = am;
  __syncthreads();
  if (tid == 0) {
    float m = red[0];
    for (int i = 1; i < 16; i++) m = fmaxf(m, red[i]);
    red[16] = __fdiv_rn(1.0f, m);
  }
  __syncthreads();
  const float inv = red[16];
  uint32_t ms = 0;
  for (int i = tid; i < n; i += 1024) {
    const uint32_t s = pk_symbol(v[i] * inv);
    sy[i] = (uint16_t)s;
    ms = ms > s ? ms : s;
  }
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t t = __shfl_xor(ms, o);
    ms = ms > t ? ms : t;
  }
  if (lane == 0) ured[wid] = ms;
  if (tid == 0) cnt_m = 0;
  __syncthreads();
  uint32_t max_sym = ured[0];
  for (int i = 1; i < 16; i++) max_sym = max_sym > ured[i] ? max_sym : ured[i];
  // histogram in passes of HBINS symbols; the used symbols, in increasing order, with counts
  uint32_t* pairs = pairs_scratch + (size_t)blockIdx.x * 4096 * 2;  // (symbol, count) then freq
  for (uint32_t base = 0; base <= max_sym; base += HBINS) {
    for (int i = tid; i < HBINS; i += 1024) hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < n; i += 1024) {
      const uint32_t s = sy[i];
      if (s >= base && s < base + HBINS) atomicAdd(&hist[s - base], 1u);
    }
    __syncthreads();
    // compact the non-zero bins in order: per-thread chunks of 8 bins, exclusive scan of counts
    const int b0 = tid * 8;
    int nz = 0;
    for (int b = b0; b < b0 + 8; b++) nz += hist[b] != 0;
    // block-wide exclusive scan of nz
    int incl = nz;
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(incl, o);
      if (lane >= o) incl += t;
    }
    if (lane == 63) ured[wid] = incl;
    __syncthreads();
    int before = cnt_m;
    for (int i = 0; i < wid; i++) before += ured[i];
    int pos = before + incl - nz;
    for (int b = b0; b < b0 + 8; b++)
      if (hist[b] && pos < 4096) {
        pairs[2 * pos] = base + b;
        pairs[2 * pos + 1] = hist[b];
        pos++;
      }
    __syncthreads();
    if (tid == 0) {
      int tot = 0;
      for (int i = 0; i < 16; i++) tot += ured[i];
      cnt_m += tot;
    }
    __syncthreads();
  }
  const int m = cnt_m;
  if (tid == 0) w.m = m;
  if (m > RANS_TOTAL) {  // scale_histogram asserts: more symbols than frequency slots
    if (tid == 0) atomicMax(&w.err, (int)PK_HIST);
    return;
  }
  // scale_histogram (packops.rs:31-103): 1 + floor(count * (4096 - m) / n) each, the deficit to
  // the largest remainders (stable: lower index first on ties), residue to the last maximum.
  const uint64_t total = (uint64_t)n, rest = (uint64_t)(RANS_TOTAL - m);
  __syncthreads();
  uint32_t* rem_rank = hist;  // reuse: rank of each symbol by remainder
  for (int i = tid; i < m; i += 1024) {
    const uint64_t ri = ((uint64_t)pairs[2 * i + 1] * rest) % total;
    int rank = 0;
    for (int j = 0; j < m; j++) {
      const uint64_t rj = ((uint64_t)pairs[2 * j + 1] * rest) % total;
      rank += (rj > ri || (rj == ri && j < i)) ? 1 : 0;
    }
    rem_rank[i] = rank;
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t acc = 0;
    for (int i = 0; i < m; i++) acc += (uint32_t)(((uint64_t)pairs[2 * i + 1] * rest) / total);
    ured[0] = (uint32_t)rest - acc;  // deficit
  }
  __syncthreads();
  const uint32_t deficit = ured[0];
  for (int i = tid; i < m; i += 1024) {
    const uint32_t q = (uint32_t)(((uint64_t)pairs[2 * i + 1] * rest) / total);
    hist[4096 + i] = 1 + q + (rem_rank[i] < deficit ? 1u : 0u);
  }
  __syncthreads();
  uint8_t* hdr = hdr_scratch + w.hdr;
  if (tid == 0) {
    int64_t tot = 0;
    int mi = 0;
    for (int i = 0; i < m; i++) {
      tot += hist[4096 + i];
      if (hist[4096 + i] >= hist[4096 + mi]) mi = i;
    }
    while (tot < RANS_TOTAL) {
      hist[4096 + mi]++;
      tot++;
    }
    while (tot > RANS_TOTAL && hist[4096 + mi] > 1) {
      hist[4096 + mi]--;
      tot--;
    }
  }
  __syncthreads();
  // header bytes after the permutation: u16 m, then (u16 symbol, u16 freq) pairs
  if (tid == 0) {
    hdr[256] = (uint8_t)m;
    hdr[257] = (uint8_t)(m >> 8);
  }
  for (int i = tid; i < m; i += 1024) {
    const uint32_t s = pairs[2 * i], f = hist[4096 + i];
    uint8_t* p = hdr + 258 + 4 * i;
    p[0] = (uint8_t)s;
    p[1] = (uint8_t)(s >> 8);
    p[2] = (uint8_t)f;
    p[3] = (uint8_t)(f >> 8);
    pairs[2 * i + 1] = f;  // now (symbol, freq)
  }
}

// rANS64 encoder symbol (rans64.rs:41-87): reciprocal of freq with ceil(log2 freq) shift.
struct EncSym {
  unsigned long long rcp;
  uint32_t bias, freq_shift;  // freq | (rcp_shift << 16)
};

__device__ __forceinline__ EncSym enc_sym(uint32_t cum, uint32_t freq) {
  EncSym e;
  if (freq < 2) {
    e.rcp = ~0ull;
    e.bias = cum + (RANS_TOTAL - 1);
    e.freq_shift = freq;
  } else {
    uint32_t shift = 0;
    while (freq > (1u << shift)) shift++;
    // ceil(2^(shift + 63) / freq) in 128-bit arithmetic: 2^(shift+63) = hi * 2^64 with hi = 2^(shift-1)
    const unsigned long long hi = 1ull << (shift - 1);
    const unsigned long long q_hi = hi / freq, r_hi = hi % freq;  // (r_hi * 2^64) / freq next
    // long division of r_hi * 2^64 by freq (freq < 2^13): 4 steps of 16 bits
    unsigned long long q_lo = 0, r = r_hi;
    for (int k = 0; k < 4; k++) {
      r = (r << 16);
      q_lo = (q_lo << 16) | (r / freq);
      r = r % freq;
    }
    (void)q_hi;  // 2^(shift+63) / freq < 2^64 since freq > 2^(shift-1): q_hi == 0
    e.rcp = q_lo + (r != 0 ? 1ull : 0ull);
    e.bias = cum;
    e.freq_shift = freq | ((shift - 1) << 16);
  }
  return e;
}

// ---- encode 5: rANS64, one workgroup per window.  Encoder parameters of the window's m
// symbols go to LDS; chunks of per-position parameters are staged in LDS by all threads; wave 0
// runs the (wave-uniform) state loop and writes each 32-bit word with lane 0. ----
constexpr int ENC_CHUNK = 2048;
__global__ __launch_bounds__(256) void pk_rans_enc(const uint16_t* __restrict__ syms, PkWin* __restrict__ win,
                                                    int cols, const uint32_t* __restrict__ pairs_scratch,
                                                    uint8_t* __restrict__ data_scratch) {
  __shared__ EncSym table[4096];
  __shared__ uint16_t sym2idx[HBINS];
  __shared__ EncSym stage[ENC_CHUNK];
  __shared__ int fail;
  PkWin& w = win[blockIdx.x];
  if (w.err) return;  // uniform
  const int m = w.m, n = w.rows * cols, tid = threadIdx.x;
  const uint32_t* pairs = pairs_scratch + (size_t)blockIdx.x * 4096 * 2;
  if (tid == 0) {
    uint32_t cum = 0;
    for (int i = 0; i < m; i++) {
      table[i].bias = cum;  // cumulative start, turned into EncSym below
      cum += pairs[2 * i + 1];
    }
    fail = 0;
  }
  __syncthreads();
  for (int i = tid; i < m; i += 256) {
    const uint32_t sym = pairs[2 * i], cum = table[i].bias;
    table[i] = enc_sym(cum, pairs[2 * i + 1]);
    if (sym < HBINS) sym2idx[sym] = (uint16_t)i;
  }
  __syncthreads();
  // The encoder pushes symbols 0..n-1 in order.  The reference writes them backwards into a
  // buffer of 2n bytes (renormalisation needs 4 free bytes, the final flush 8, else it
  // panics); here word j (the j-th emitted) goes to out_words[cap_w - 1 - j] and the state
  // just before the last word, so the stream is contiguous: state, words k-1 .. 0.
  uint32_t* out_words = reinterpret_cast<uint32_t*>(data_scratch + w.data);
  const long long cap_w = n / 2 + 4;
  long long k = 0;               // words emitted
  const long long cap_b = 2LL * n;  // the reference's buffer size in bytes
  unsigned long long x = RANS_L;
  for (int c0 = 0; c0 < n; c0 += ENC_CHUNK) {
    const int cn = min(ENC_CHUNK, n - c0);
    for (int i = tid; i < cn; i += 256) {
      const uint32_t s = syms[(size_t)w.row0 * cols + c0 + i];
      int kk;
      if (s < HBINS) {
        kk = sym2idx[s];
      } else {  // rare large symbols: binary search in the sorted symbol list
        int lo = 0, hi = m - 1;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (pairs[2 * mid] < s) lo = mid + 1;
          else hi = mid;
        }
        kk = lo;
      }
      stage[i] = table[kk];
    }
    __syncthreads();
    if (__builtin_amdgcn_readfirstlane(tid >> 6) == 0 && !fail) {
      // Wave 0 runs the coder; every value below is wave-uniform (parameters pass through
      // readfirstlane), so the state lives in scalar registers and the loop branches on the
      // scalar unit.  Parameters of the next 4 positions are read from LDS one group ahead.
      EncSym nx[4];
#pragma unroll
      for (int j = 0; j < 4; j++) nx[j] = stage[min(j, cn - 1)];
      bool ok = true;
      for (int i = 0; i < cn && ok; i += 4) {
        EncSym cu[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          cu[j] = nx[j];
          nx[j] = stage[min(i + 4 + j, cn - 1)];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
          if (i + j >= cn || !ok) break;
          const uint32_t fs = __builtin_amdgcn_readfirstlane(cu[j].freq_shift);
          const uint32_t bias = __builtin_amdgcn_readfirstlane(cu[j].bias);
          const uint32_t rlo = __builtin_amdgcn_readfirstlane((uint32_t)cu[j].rcp);
          const uint32_t rhi = __builtin_amdgcn_readfirstlane((uint32_t)(cu[j].rcp >> 32));
          const uint32_t freq = fs & 0xffffu, shift = fs >> 16;
          const unsigned long long rcp = ((unsigned long long)rhi << 32) | rlo;
          const unsigned long long x_max = (1ull << 51) * freq;  // ((L >> 12) << 32) * freq
          while (x >= x_max) {
            if (cap_b - 4 * k < 4) {
              ok = false;
              break;
            }
            if (tid == 0) out_words[cap_w - 1 - k] = (uint32_t)x;
            k++;
            x >>= 32;
          }
          const unsigned long long q = __umul64hi(x, rcp) >> shift;
          x = x + bias + q * (unsigned long long)(RANS_TOTAL - freq);
        }
      }
      if (!ok && tid == 0) fail = 1;
    }
    __syncthreads();
  }
  if (tid == 0) {
    if (fail || cap_b - 4 * k < 8) {
      atomicMax(&w.err, (int)PK_OVERFLOW);
    } else {
      out_words[cap_w - 2 - k] = (uint32_t)x;
      out_words[cap_w - 1 - k] = (uint32_t)(x >> 32);
      w.dlen = (int)(8 + 4 * k);
      w.pad = (int)((cap_w - 2 - k) * 4);  // stream start within the slot
    }
  }
}

// ---- encode 6: assemble.  out_off[window] = output byte offset of the window's pieces:
// perm bytes, u16 m + pairs, u16 dlen, stream.  One workgroup per window. ----
__global__ __launch_bounds__(256) void pk_assemble(const PkWin* __restrict__ win, int cols,
                                                    const uint8_t* __restrict__ hdr_scratch,
                                                    const uint8_t* __restrict__ data_scratch,
                                                    const long long* __restrict__ out_off, uint8_t* __restrict__ out) {
  const PkWin& w = win[blockIdx.x];
  uint8_t* o = out + out_off[blockIdx.x];
  const uint8_t* h = hdr_scratch + w.hdr;
  const int tid = threadIdx.x;
  for (int i = tid; i < cols; i += 256) o[i] = h[i];
  const int hb = 2 + 4 * w.m;
  for (int i = tid; i < hb; i += 256) o[cols + i] = h[256 + i];
  if (tid == 0) {
    o[cols + hb] = (uint8_t)w.dlen;  // `data.len() as u16`, as the reference writes it
    o[cols + hb + 1] = (uint8_t)(w.dlen >> 8);
  }
  const uint8_t* d = data_scratch + w.data + w.pad;
  for (int i = tid; i < w.dlen; i += 256) o[cols + hb + 2 + i] = d[i];
}

// The u32 row count that opens each packed matrix (native-endian, as `to_ne_bytes`).
__global__ void pk_headers(const long long* __restrict__ off, const int* __restrict__ rows, int B,
                           uint8_t* __restrict__ out) {
  const int b = blockIdx.x * 256 + threadIdx.x;
  if (b >= B) return;
  const uint32_t r = (uint32_t)rows[b];
  uint8_t* o = out + off[b];
  o[0] = (uint8_t)r;
  o[1] = (uint8_t)(r >> 8);
  o[2] = (uint8_t)(r >> 16);
  o[3] = (uint8_t)(r >> 24);
}

// ---- decode 2: rANS64, one workgroup per window.  cum -> (start, freq, value) in LDS; wave 0
// runs the state loop from the last value to the first, staging values in LDS chunks that the
// workgroup then writes out. ----
constexpr int DEC_CHUNK = 4096;
__global__ __launch_bounds__(256) void pk_rans_dec(const uint8_t* __restrict__ in, PkWin* __restrict__ win, int cols,
                                                    float* __restrict__ out) {
  __shared__ uint32_t cum_sf[RANS_TOTAL];  // start | freq << 16
  __shared__ float cum_v[RANS_TOTAL];
  __shared__ float stage[DEC_CHUNK];
  __shared__ int st_err;
  PkWin& w = win[blockIdx.x];
  const int tid = threadIdx.x, n = w.rows * cols, m = w.m;
  // freq 4096 (a single symbol) needs 13 bits next to the 16-bit start: start | freq << 16
  const uint8_t* pairs = in + w.hdr + cols + 2;  // after perm bytes and u16 m
  __shared__ uint32_t run_start[4097];
  for (int c = tid; c < RANS_TOTAL; c += 256) {
    cum_sf[c] = 1u << 16;  // slots no symbol covers keep RansDecSymbol::new(0, 1) and 0.0
    cum_v[c] = 0.f;
  }
  if (tid == 0) {
    st_err = 0;
    uint32_t cum = 0;
    for (int i = 0; i < m && i < RANS_TOTAL; i++) {
      run_start[i] = cum;
      cum += pairs[4 * i + 2] | (pairs[4 * i + 3] << 8);
      if (cum > (uint32_t)RANS_TOTAL) st_err = PK_CORRUPT;  // the reference indexes past its tables
    }
    if (m > RANS_TOTAL) st_err = PK_CORRUPT;
  }
  __syncthreads();
  if (st_err) {
    if (tid == 0) atomicMax(&w.err, st_err);
    return;  // uniform
  }
  for (int i = tid; i < m; i += 256) {
    const uint32_t sym = pairs[4 * i] | (pairs[4 * i + 1] << 8), f = pairs[4 * i + 2] | (pairs[4 * i + 3] << 8);
    float v = 0.f;
    if (sym != 0) {
      const uint32_t q = sym + 1;
      v = (1.0f / 29.0f) * ((q & 1) ? -1.0f : 1.0f) * (float)(q >> 1);
    }
    const uint32_t start = run_start[i];
    for (uint32_t c = start; c < start + f; c++) {
      cum_sf[c] = start | (f << 16);
      cum_v[c] = v;
    }
  }
  __syncthreads();
  // The stream, read 4 bytes at a time from any byte offset: two aligned dwords funnel-
  // shifted (the input buffer carries 16 bytes of padding).  Addresses are wave-uniform.
  const uint8_t* d = in + w.data;
  const int clen = w.dlen;
  auto word_at = [&](int p) -> uint32_t {
    const uintptr_t a = (uintptr_t)(d + p);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(a & ~(uintptr_t)3);
    const unsigned long long two = ((unsigned long long)q[1] << 32) | q[0];
    return (uint32_t)(two >> (8 * (a & 3)));
  };
  float* dst = out + (size_t)w.row0 * cols;
  unsigned long long x = ((unsigned long long)word_at(4) << 32) | word_at(0);
  int pos = 8;
  bool bad = false;
  uint32_t next = word_at(min(pos, clen - 4));  // prefetched renormalisation word
  // decode positions n-1 .. 0 in chunks of DEC_CHUNK (chunk j covers [hi - cn, hi))
  for (int hi = n; hi > 0; hi -= DEC_CHUNK) {
    const int cn = min(DEC_CHUNK, hi);
    if (__builtin_amdgcn_readfirstlane(tid >> 6) == 0 && !bad) {
      // wave 0, wave-uniform state in scalar registers (table entries pass through readfirstlane)
      for (int i = cn - 1; i >= 0; i--) {
        const uint32_t c = (uint32_t)(x & (RANS_TOTAL - 1));
        const uint32_t sf = __builtin_amdgcn_readfirstlane(cum_sf[c]);
        stage[i] = cum_v[c];
        x = (unsigned long long)(sf >> 16) * (x >> RANS_BITS) + c - (sf & 0xffffu);
        if (x < RANS_L) {
          if (pos + 4 > clen) {
            bad = true;
            break;
          }
          x = (x << 32) | next;
          pos += 4;
          next = word_at(min(pos, clen - 4));
          if (x < RANS_L) {
            bad = true;
            break;
          }
        }
      }
    }
    if (tid == 0 && bad) st_err = PK_CORRUPT;
    __syncthreads();
    for (int i = tid; i < cn; i += 256) dst[hi - cn + i] = stage[i];
    __syncthreads();
  }
  if (tid == 0) {
    if (st_err) atomicMax(&w.err, st_err);
    w.pad = pos;  // bytes consumed
  }
}

// Correctly rounded f32 square root (Rust's f32::sqrt): the hardware estimate (within 1 ulp)
// moved to the neighbour on the right side of the true root, decided by the exact residual
// x - s' s of each neighbour s' (one fused multiply-add each).  Inputs below 2^-96 are scaled
// by 2^32 first (the root by 2^-16 after; both exact) so the residuals stay normal.
__device__ __forceinline__ float sqrt_rn(float x) {
  if (!(x > 0.f) || x == __builtin_inff()) return __builtin_sqrtf(x);  // 0, inf, NaN, < 0
  const bool small = x < 0x1p-96f;
  const float xs = small ? x * 0x1p32f : x;
  float s = __builtin_amdgcn_sqrtf(xs);
  const float sd = __uint_as_float(__float_as_uint(s) - 1u), su = __uint_as_float(__float_as_uint(s) + 1u);
  const float rd = __builtin_fmaf(-sd, s, xs), ru = __builtin_fmaf(-su, s, xs);
  s = rd <= 0.f ? sd : s;
  s = ru > 0.f ? su : s;
  return small ? s * 0x1p-16f : s;
}

// ---- decode 5: undo the column permutation and L2-normalise each row (row norms summed
// sequentially in column order, as the reference's iterator sum).  One wave per row. ----
__global__ __launch_bounds__(256) void pk_unpermute_norm(float* __restrict__ x, int total_rows, int cols,
                                                          const int* __restrict__ row_win,
                                                          const uint8_t* __restrict__ in,
                                                          const PkWin* __restrict__ win) {
  __shared__ float buf[4][256];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + wv;
  if (row >= total_rows) return;  // wave-uniform
  const uint8_t* idxs = in + win[row_win[row]].hdr;
  float* r = x + (size_t)row * cols;
  float* v = buf[wv];
  for (int c = lane; c < cols; c += 64) v[c] = r[idxs[c]];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float ss = 0.f;
  if (lane == 0)
    for (int c = 0; c < cols; c++) ss += v[c] * v[c];
  ss = __shfl(ss, 0);
  const float inv = __fdiv_rn(1.0f, sqrt_rn(ss));
  for (int c = lane; c < cols; c += 64) r[c] = v[c] * inv;
}

}  // namespace

namespace t5k {

hipError_t pk_encode(const float* x, int total_rows, int cols, PkWin* win, int nwin, const int* row_win,
                     float* work, uint16_t* syms, int* perm, uint8_t* hdr, uint32_t* pairs, uint8_t* data,
                     hipStream_t s) {
  if (nwin == 0) return hipSuccess;
  hipLaunchKernelGGL(pk_colsort, dim3(nwin), dim3(256), 0, s, x, win, cols, hdr, perm);
  hipLaunchKernelGGL((pk_haar_rows<false>), dim3((total_rows + 3) / 4), dim3(256), 0, s, x, work, total_rows, cols,
                     row_win, perm);
  hipLaunchKernelGGL((pk_haar_cols<false>), dim3(nwin, (cols + 7) / 8), dim3(256), 0, s, work, win, cols);
  hipLaunchKernelGGL(pk_quant, dim3(nwin), dim3(1024), 0, s, work, win, cols, syms, hdr, pairs);
  hipLaunchKernelGGL(pk_rans_enc, dim3(nwin), dim3(256), 0, s, syms, win, cols, pairs, data);
  return hipGetLastError();
}

hipError_t pk_assemble_out(const PkWin* win, int nwin, int cols, const uint8_t* hdr, const uint8_t* data,
                           const long long* out_off, const long long* mat_off, const int* mat_rows, int B,
                           uint8_t* out, hipStream_t s) {
  if (B > 0) hipLaunchKernelGGL(pk_headers, dim3((B + 255) / 256), dim3(256), 0, s, mat_off, mat_rows, B, out);
  if (nwin > 0) hipLaunchKernelGGL(pk_assemble, dim3(nwin), dim3(256), 0, s, win, cols, hdr, data, out_off, out);
  return hipGetLastError();
}

hipError_t pk_decode(const uint8_t* in, int total_rows, int cols, PkWin* win, int nwin, const int* row_win,
                     float* out, float* work, hipStream_t s) {
  if (nwin == 0) return hipSuccess;
  hipLaunchKernelGGL(pk_rans_dec, dim3(nwin), dim3(256), 0, s, in, win, cols, work);
  hipLaunchKernelGGL((pk_haar_rows<true>), dim3((total_rows + 3) / 4), dim3(256), 0, s, work, out, total_rows, cols,
                     row_win, nullptr);
  hipLaunchKernelGGL((pk_haar_cols<true>), dim3(nwin, (cols + 7) / 8), dim3(256), 0, s, out, win, cols);
  hipLaunchKernelGGL(pk_unpermute_norm, dim3((total_rows + 3) / 4), dim3(256), 0, s, out, total_rows, cols, row_win,
                     in, win);
  return hipGetLastError();
}

}  // namespace t5k
