/*
 * codec_oracle.c -- CPU restatement of Witchcraft's embedding codecs (packops.rs,
 * haarops.rs, rans64.rs).
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP codecs in witchcraft_amd/.
 * Only tests/ and bench.py's cpu_baseline leg load it; the product never links it.
 *
 * Two codecs:
 *  1. Residual codec.  Index build: residual = embedding - assigned centre, then
 *     compand() (mu-law, packops.rs:136-142), quantize(4) (:156-162) and to_q4_bytes
 *     (:440-462), called at src/lib.rs:1375-1376.  Search: from_companded_q4_bytes
 *     (packops.rs:491-513) with make_q4_dequant_table (:14-25), called at src/lib.rs:626,676.
 *  2. Packed chunk embeddings: embeddings_to_packed (packops.rs:172-301) and
 *     embeddings_from_packed (:303-438): per window of <= 1024 rows, columns sorted by their
 *     sum, 2-D Haar transform with mirror edges (haarops.rs), max-abs scaling, symbols
 *     round(29 x) folded to unsigned, a histogram scaled to 2^12 (scale_histogram,
 *     packops.rs:31-103) and one rANS64 stream (rans64.rs, ryg_rans' rans64.h).
 *
 * Scalar semantics follow candle's CPU ops as the reference calls them: `tensor * f64`,
 * `tensor + f64` and `tensor - f64` are affine(mul, add) = v * (f32)mul + (f32)add with two
 * roundings; log/exp are the platform libm's logf/expf (Rust's f32::ln / f32::exp);
 * Tensor::pow(rhs) = exp(rhs * ln(self)); round() rounds half away from zero.  Rust's
 * float -> integer `as` casts saturate (NaN -> 0) and integer `as u16` casts wrap.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "t5_oracle.h"

/* ------------------------------------------------------------------------------------ */
/* 1. residual codec                                                                      */

static float affine(float v, double mul, double add) { return v * (float)mul + (float)add; }

static float sign_f(float v) { return v > 0.f ? 1.f : (v < 0.f ? -1.f : 0.f); }

/* compand() then quantize(4) of one value: the 4-bit code as packops.rs computes it. */
uint8_t orc_compand_q4(float v) {
  /* compand (packops.rs:136-142) */
  const double inv_denominator = 1.0 / log(1.0 + 255.0);
  const float x = affine(v, 4.0, 0.0);
  float t = affine(fabsf(x), 255.0, 0.0);
  t = affine(t, 1.0, 1.0);
  const float c = sign_f(x) * affine(logf(t), inv_denominator, 0.0);
  /* quantize(4) (packops.rs:156-162): qmax = 15, scale1 = zp = 7.5 */
  float y = affine(c, 7.5, 0.0);
  y = affine(y, 1.0, 7.5);
  y = roundf(y);
  /* clamp(0, 15) = maximum(0) then minimum(15); NaN compares false and yields the bound */
  y = y > 0.f ? y : 0.f;
  y = y < 15.f ? y : 15.f;
  return (uint8_t)y;
}

/* make_q4_dequant_table (packops.rs:14-25): arange(0,16).dequantize(4).inv_compand(). */
void orc_q4_dequant_table(float table[16]) {
  const float ln256 = logf(affine(1.0f, 1.0, 255.0)); /* (ones + 255).pow(abs) = exp(abs ln 256) */
  for (int i = 0; i < 16; i++) {
    /* dequantize(4) (packops.rs:164-170): (x - 7.5) * (2 / 15) */
    float x = affine((float)i, 1.0, -7.5);
    x = affine(x, 2.0 / 15.0, 0.0);
    /* inv_compand (packops.rs:144-154) */
    const float p = expf(fabsf(x) * ln256);
    float s = affine(p, 1.0, -1.0);
    s = affine(s, 1.0 / 255.0, 0.0);
    s = sign_f(x) * s;
    table[i] = affine(s, 0.25, 0.0);
  }
}

/* residual = emb[i] - centers[assign[i]]; compand().quantize(4).to_q4_bytes(): value 2j of a
 * row in the high nibble of byte j, value 2j + 1 in the low nibble (src/lib.rs:1375-1376). */
void orc_residual_encode(const float* emb, const float* centers, const uint32_t* assign, int N, int D,
                         uint8_t* out) {
#pragma omp parallel for schedule(static)
  for (int i = 0; i < N; i++) {
    const float* e = emb + (size_t)i * D;
    const float* c = centers + (size_t)assign[i] * D;
    for (int j = 0; j < D; j += 2) {
      const uint8_t hi = orc_compand_q4(e[j] - c[j]), lo = orc_compand_q4(e[j + 1] - c[j + 1]);
      out[(size_t)i * (D / 2) + j / 2] = (uint8_t)((hi << 4) | lo);
    }
  }
}

/* from_companded_q4_bytes (packops.rs:491-513). */
void orc_residual_decode(const uint8_t* bytes, int N, int D, const float table[16], float* out) {
  for (size_t b = 0; b < (size_t)N * D / 2; b++) {
    out[2 * b] = table[bytes[b] >> 4];
    out[2 * b + 1] = table[bytes[b] & 15];
  }
}

/* Checks a 15-entry threshold ladder (q(x) = #{j : x >= t[j]}) against orc_compand_q4 on every
 * one of the 2^32 f32 bit patterns.  Returns the mismatch count, first_bad = the first bits. */
uint64_t orc_ladder_mismatches(const float t[15], uint32_t* first_bad) {
  uint64_t bad = 0;
  uint32_t first = 0xffffffffu;
#pragma omp parallel for schedule(static) reduction(+ : bad) reduction(min : first)
  for (int64_t hi = 0; hi < 65536; hi++) {
    for (uint32_t lo = 0; lo < 65536; lo++) {
      const uint32_t bits = ((uint32_t)hi << 16) | lo;
      float x;
      memcpy(&x, &bits, 4);
      uint8_t q = 0;
      for (int j = 0; j < 15; j++) q += x >= t[j];
      if (q != orc_compand_q4(x)) {
        bad++;
        if (bits < first) first = bits;
      }
    }
  }
  if (first_bad) *first_bad = first;
  return bad;
}

/* ------------------------------------------------------------------------------------ */
/* 2. packed chunk embeddings                                                              */

#define PK_MAX_WINDOW_ROWS 1024 /* packops.rs:8 */
#define PK_RANS_BITS 12         /* packops.rs:9 */
#define PK_RANGE 29.0f          /* packops.rs:10 */
#define PK_INV_SQRT2 0.7071067811865475f /* haarops.rs:1 */
#define RANS64_L (1ull << 31)

/* haar_forward_mirror_edge (haarops.rs:4-31) */
void orc_haar_forward(float* x, int n0) {
  float* tmp = (float*)calloc((size_t)n0 + 1, sizeof(float));
  int n = n0;
  while (n > 1) {
    const int pairs = n / 2, odd = n & 1, nc = pairs + odd;
    for (int i = 0; i < pairs; i++) {
      const float a = x[2 * i], b = x[2 * i + 1];
      tmp[i] = (a + b) * PK_INV_SQRT2;
      tmp[nc + i] = (a - b) * PK_INV_SQRT2;
    }
    if (odd) {
      const float a = x[n - 1];
      tmp[pairs] = (a + a) * PK_INV_SQRT2;
    }
    memcpy(x, tmp, (size_t)n * sizeof(float));
    n = nc;
  }
  free(tmp);
}

/* haar_inverse_mirror_edge (haarops.rs:34-70) */
void orc_haar_inverse(float* x, int n0) {
  float* tmp = (float*)calloc((size_t)n0 + 1, sizeof(float));
  int levels[40], nl = 0, n = n0;
  levels[nl++] = n;
  while (n > 1) {
    n = n / 2 + (n & 1);
    levels[nl++] = n;
  }
  for (int w = nl - 1; w >= 1; w--) {
    const int np = levels[w - 1], odd = np & 1, pairs = np / 2, nc = pairs + odd;
    for (int i = 0; i < pairs; i++) {
      const float sum = x[i], diff = x[nc + i];
      tmp[2 * i] = (sum + diff) * PK_INV_SQRT2;
      tmp[2 * i + 1] = (sum - diff) * PK_INV_SQRT2;
    }
    if (odd) tmp[np - 1] = x[nc - 1] * PK_INV_SQRT2;
    memcpy(x, tmp, (size_t)np * sizeof(float));
  }
  free(tmp);
}

/* scale_histogram (packops.rs:31-103): counts of m symbols (in symbol order) -> frequencies
 * summing to 2^log2_scale, each >= 1.  Returns 0, or -1 where the reference asserts. */
int orc_scale_histogram(const uint32_t* counts, int m, int log2_scale, uint16_t* freq) {
  if (m <= 0 || log2_scale > 16) return -1;
  const uint32_t target = 1u << log2_scale;
  if ((uint32_t)m > target) return -1;
  const uint32_t remaining = target - (uint32_t)m;
  uint64_t sum = 0;
  for (int i = 0; i < m; i++) sum += counts[i];
  uint32_t* scaled = (uint32_t*)malloc(sizeof(uint32_t) * m);
  uint64_t* rem = (uint64_t*)malloc(sizeof(uint64_t) * m);
  int* order = (int*)malloc(sizeof(int) * m);
  uint32_t acc = 0;
  for (int i = 0; i < m; i++) {
    const uint64_t num = (uint64_t)counts[i] * remaining;
    const uint32_t q = (uint32_t)(num / sum);
    rem[i] = num % sum;
    scaled[i] = 1 + q;
    acc += q;
    order[i] = i;
  }
  const uint32_t deficit = remaining - acc;
  if (deficit > 0) {
    /* stable sort by remainder, descending (insertion sort keeps equal keys in index order) */
    for (int i = 1; i < m; i++) {
      const int o = order[i];
      int j = i - 1;
      while (j >= 0 && rem[order[j]] < rem[o]) {
        order[j + 1] = order[j];
        j--;
      }
      order[j + 1] = o;
    }
    for (uint32_t k = 0; k < deficit && (int)k < m; k++) scaled[order[k]] += 1;
  }
  int64_t total = 0;
  for (int i = 0; i < m; i++) total += scaled[i];
  if (total != (int64_t)target) {
    /* max_by_key keeps the LAST of equal maxima */
    int mi = 0;
    for (int i = 1; i < m; i++)
      if (scaled[i] >= scaled[mi]) mi = i;
    while (total < (int64_t)target) {
      scaled[mi]++;
      total++;
    }
    while (total > (int64_t)target && scaled[mi] > 1) {
      scaled[mi]--;
      total--;
    }
  }
  for (int i = 0; i < m; i++) freq[i] = (uint16_t)scaled[i];
  free(scaled);
  free(rem);
  free(order);
  return 0;
}

/* rANS64 encoder symbol (RansEncSymbol::new, rans64.rs:41-87) */
typedef struct {
  uint64_t x_max, rcp_freq, bias;
  uint32_t cmpl_freq, rcp_shift;
} enc_sym;

static enc_sym enc_sym_new(uint32_t cum, uint32_t freq, uint32_t scale_bits) {
  enc_sym s;
  s.x_max = ((RANS64_L >> scale_bits) << 32) * (uint64_t)freq;
  s.cmpl_freq = (1u << scale_bits) - freq;
  if (freq < 2) {
    s.rcp_freq = ~0ull;
    s.rcp_shift = 0;
    s.bias = (uint64_t)cum + ((1ull << scale_bits) - 1);
  } else {
    uint32_t shift = 0;
    while (freq > (1u << shift)) shift++;
    const unsigned __int128 num = (unsigned __int128)1 << (shift + 63);
    s.rcp_freq = (uint64_t)((num + freq - 1) / freq);
    s.rcp_shift = shift - 1;
    s.bias = cum;
  }
  return s;
}

static uint16_t f32_to_symbol(float v) {
  const float q = roundf(PK_RANGE * v);
  const float sf = 2.0f * fabsf(q) + (q < 0.0f ? 1.0f : 0.0f);
  uint64_t s; /* Rust `as usize`: saturating, NaN -> 0 */
  if (!(sf >= 1.0f)) s = 0;
  else if (sf >= 18446744073709551616.0f) s = UINT64_MAX;
  else s = (uint64_t)sf;
  return (uint16_t)(s > 0 ? s - 1 : 0);
}

static void put_u16(uint8_t* p, uint16_t v) { memcpy(p, &v, 2); }

/* embeddings_to_packed (packops.rs:172-301) of x[rows][cols].  Writes at most cap bytes;
 * returns the packed size, -2 if cap is too small, -1 where the reference errors or panics
 * (cols > 255, a NaN column sum). */
long orc_embeddings_to_packed(const float* x, int rows, int cols, uint8_t* out, size_t cap) {
  if (cols > 255 || cols <= 0 || rows < 0) return -1;
  size_t pos = 0;
#define NEED(n)                           \
  do {                                    \
    if (pos + (size_t)(n) > cap) goto small; \
  } while (0)
  float* raw = (float*)malloc(sizeof(float) * (size_t)PK_MAX_WINDOW_ROWS * cols);
  float* col = (float*)malloc(sizeof(float) * PK_MAX_WINDOW_ROWS);
  float* sums = (float*)malloc(sizeof(float) * cols);
  float* rowbuf = (float*)malloc(sizeof(float) * cols);
  int* perm = (int*)malloc(sizeof(int) * cols);
  uint16_t* qs = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)PK_MAX_WINDOW_ROWS * cols);
  uint32_t* hist = (uint32_t*)malloc(sizeof(uint32_t) * 65536);
  uint32_t* counts = (uint32_t*)malloc(sizeof(uint32_t) * 65536);
  uint16_t* syms = (uint16_t*)malloc(sizeof(uint16_t) * 65536);
  uint16_t* freqs = (uint16_t*)malloc(sizeof(uint16_t) * 65536);
  enc_sym* q2sym = (enc_sym*)malloc(sizeof(enc_sym) * 65536);
  uint8_t* enc = (uint8_t*)malloc((size_t)2 * PK_MAX_WINDOW_ROWS * cols + 16);
  long result = -1;
  NEED(4);
  const uint32_t r32 = (uint32_t)rows;
  memcpy(out, &r32, 4);
  pos = 4;
  for (int off = 0; off < rows; off += PK_MAX_WINDOW_ROWS) {
    const int wr = rows - off < PK_MAX_WINDOW_ROWS ? rows - off : PK_MAX_WINDOW_ROWS;
    const size_t n = (size_t)wr * cols;
    memcpy(raw, x + (size_t)off * cols, n * sizeof(float));
    /* column sums in row order; stable sort of the columns by sum */
    for (int c = 0; c < cols; c++) sums[c] = 0.f;
    for (int r = 0; r < wr; r++)
      for (int c = 0; c < cols; c++) sums[c] += raw[(size_t)r * cols + c];
    for (int c = 0; c < cols; c++)
      if (isnan(sums[c])) goto fail; /* partial_cmp().unwrap() panics */
    for (int c = 0; c < cols; c++) perm[c] = c;
    for (int i = 1; i < cols; i++) {
      const int p = perm[i];
      int j = i - 1;
      while (j >= 0 && sums[perm[j]] > sums[p]) {
        perm[j + 1] = perm[j];
        j--;
      }
      perm[j + 1] = p;
    }
    NEED(cols);
    for (int newp = 0; newp < cols; newp++) out[pos + perm[newp]] = (uint8_t)newp; /* inv_perm */
    pos += cols;
    for (int r = 0; r < wr; r++) {
      float* row = raw + (size_t)r * cols;
      for (int c = 0; c < cols; c++) rowbuf[c] = row[perm[c]];
      memcpy(row, rowbuf, sizeof(float) * cols);
      orc_haar_forward(row, cols);
    }
    for (int c = 0; c < cols; c++) {
      for (int r = 0; r < wr; r++) col[r] = raw[(size_t)r * cols + c];
      orc_haar_forward(col, wr);
      for (int r = 0; r < wr; r++) raw[(size_t)r * cols + c] = col[r];
    }
    float abs_max = 0.00001f;
    for (size_t i = 0; i < n; i++) {
      const float a = fabsf(raw[i]);
      if (a < 1.0f && a > abs_max) abs_max = a;
    }
    const float inv = 1.0f / abs_max;
    uint16_t max_sym = 0;
    for (size_t i = 0; i < n; i++) {
      qs[i] = f32_to_symbol(raw[i] * inv);
      if (qs[i] > max_sym) max_sym = qs[i];
    }
    memset(hist, 0, sizeof(uint32_t) * ((size_t)max_sym + 1));
    for (size_t i = 0; i < n; i++) hist[qs[i]]++;
    int m = 0;
    for (uint32_t s = 0; s <= max_sym; s++)
      if (hist[s]) {
        syms[m] = (uint16_t)s;
        counts[m] = hist[s];
        m++;
      }
    if (orc_scale_histogram(counts, m, PK_RANS_BITS, freqs)) goto fail;
    NEED(2 + 4 * (size_t)m);
    put_u16(out + pos, (uint16_t)m);
    pos += 2;
    uint32_t cum = 0;
    for (int i = 0; i < m; i++) {
      q2sym[syms[i]] = enc_sym_new(cum, freqs[i], PK_RANS_BITS);
      put_u16(out + pos, syms[i]);
      put_u16(out + pos + 2, freqs[i]);
      pos += 4;
      cum += freqs[i];
    }
    /* rANS64 put/renorm/flush (rans64.rs:111-166): symbols in order, written backwards,
     * state flushed last */
    const size_t encap = 2 * n;
    size_t idx = encap;
    uint64_t st = RANS64_L;
    for (size_t i = 0; i < n; i++) {
      const enc_sym* s = &q2sym[qs[i]];
      while (st >= s->x_max) {
        if (idx < 4) goto fail; /* the reference panics */
        idx -= 4;
        const uint32_t v = (uint32_t)st;
        memcpy(enc + idx, &v, 4);
        st >>= 32;
      }
      const uint64_t q = (uint64_t)(((unsigned __int128)st * s->rcp_freq) >> 64) >> s->rcp_shift;
      st = st + s->bias + q * s->cmpl_freq;
    }
    if (idx < 8) goto fail;
    idx -= 8;
    memcpy(enc + idx, &st, 8);
    const size_t dlen = encap - idx;
    NEED(2 + dlen);
    put_u16(out + pos, (uint16_t)dlen); /* `data.len() as u16`, as the reference writes it */
    pos += 2;
    memcpy(out + pos, enc + idx, dlen);
    pos += dlen;
  }
  result = (long)pos;
  goto done;
small:
  result = -2;
  goto done;
fail:
  result = -1;
done:
  free(raw);
  free(col);
  free(sums);
  free(rowbuf);
  free(perm);
  free(qs);
  free(hist);
  free(counts);
  free(syms);
  free(freqs);
  free(q2sym);
  free(enc);
#undef NEED
  return result;
}

/* embeddings_from_packed (packops.rs:303-438): decodes into out[rows][cols] (cap_rows rows of
 * room) with every row L2-normalised.  Returns rows, or -1 on a malformed buffer. */
long orc_embeddings_from_packed(const uint8_t* buf, size_t len, int cols, float* out, size_t cap_rows) {
  if (len < 4 || cols <= 0) return -1;
  uint32_t rows;
  memcpy(&rows, buf, 4);
  if (rows > cap_rows) return -1;
  size_t pos = 4;
  const float scale = 1.0f / PK_RANGE;
  float* cum2float = (float*)malloc(sizeof(float) << PK_RANS_BITS);
  uint32_t* cum_start = (uint32_t*)malloc(sizeof(uint32_t) << PK_RANS_BITS);
  uint32_t* cum_freq = (uint32_t*)malloc(sizeof(uint32_t) << PK_RANS_BITS);
  float* col = (float*)malloc(sizeof(float) * PK_MAX_WINDOW_ROWS);
  float* rowbuf = (float*)malloc(sizeof(float) * cols);
  int* idxs = (int*)malloc(sizeof(int) * cols);
  long result = -1;
  size_t done_rows = 0;
  for (uint32_t off = 0; off < rows; off += PK_MAX_WINDOW_ROWS) {
    const int wr = rows - off < PK_MAX_WINDOW_ROWS ? (int)(rows - off) : PK_MAX_WINDOW_ROWS;
    if (pos + cols + 2 > len) goto fail;
    for (int c = 0; c < cols; c++) idxs[c] = buf[pos + c];
    pos += cols;
    uint16_t m;
    memcpy(&m, buf + pos, 2);
    pos += 2;
    if (pos + 4 * (size_t)m > len) goto fail;
    for (int c = 0; c < (1 << PK_RANS_BITS); c++) {
      cum2float[c] = 0.f;
      cum_start[c] = 0;
      cum_freq[c] = 1;
    }
    uint32_t cum = 0;
    for (int i = 0; i < m; i++) {
      uint16_t sym, fr;
      memcpy(&sym, buf + pos + 4 * i, 2);
      memcpy(&fr, buf + pos + 4 * i + 2, 2);
      float v = 0.f;
      if (sym != 0) {
        const uint32_t q = (uint32_t)sym + 1;
        const float sg = (q & 1) ? -1.0f : 1.0f;
        v = scale * sg * (float)(q >> 1);
      }
      /* RansDecSymbol::new bounds (rans64.rs:220-229); the cum tables hold 2^12 entries */
      if (cum + fr > (1u << PK_RANS_BITS)) goto fail;
      for (uint32_t c = cum; c < cum + fr; c++) {
        cum2float[c] = v;
        cum_start[c] = cum;
        cum_freq[c] = fr;
      }
      cum += fr;
    }
    pos += 4 * (size_t)m;
    if (pos + 2 > len) goto fail;
    uint16_t clen;
    memcpy(&clen, buf + pos, 2);
    pos += 2;
    if (pos + clen > len || clen < 8) goto fail;
    const uint8_t* d = buf + pos;
    size_t di = 8;
    uint64_t st;
    memcpy(&st, d, 8);
    float* t = out + done_rows * cols;
    const size_t n = (size_t)wr * cols;
    for (size_t i = n; i-- > 0;) {
      const uint32_t c = (uint32_t)(st & ((1u << PK_RANS_BITS) - 1));
      t[i] = cum2float[c];
      st = (uint64_t)cum_freq[c] * (st >> PK_RANS_BITS) + (st & ((1u << PK_RANS_BITS) - 1)) - cum_start[c];
      if (st < RANS64_L) {
        if (di + 4 > clen) goto fail;
        uint32_t v;
        memcpy(&v, d + di, 4);
        di += 4;
        st = (st << 32) | v;
        if (st < RANS64_L) goto fail;
      }
    }
    pos += clen;
    for (int r = 0; r < wr; r++) orc_haar_inverse(t + (size_t)r * cols, cols);
    for (int c = 0; c < cols; c++) {
      for (int r = 0; r < wr; r++) col[r] = t[(size_t)r * cols + c];
      orc_haar_inverse(col, wr);
      for (int r = 0; r < wr; r++) t[(size_t)r * cols + c] = col[r];
    }
    for (int r = 0; r < wr; r++) {
      float* row = t + (size_t)r * cols;
      for (int c = 0; c < cols; c++) rowbuf[c] = row[idxs[c]];
      memcpy(row, rowbuf, sizeof(float) * cols);
    }
    done_rows += wr;
  }
  if (pos != len) goto fail; /* leftover bytes: the reference bails */
  for (size_t r = 0; r < rows; r++) {
    float* row = out + r * cols;
    float ss = 0.f;
    for (int c = 0; c < cols; c++) ss += row[c] * row[c];
    const float inv = 1.0f / sqrtf(ss);
    for (int c = 0; c < cols; c++) row[c] *= inv;
  }
  result = (long)rows;
fail:
  free(cum2float);
  free(cum_start);
  free(cum_freq);
  free(col);
  free(rowbuf);
  free(idxs);
  return result;
}
