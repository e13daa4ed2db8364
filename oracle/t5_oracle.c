/*
 * t5_oracle.c -- CPU restatement of the reference XTR-T5 encoder numerics.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker; see t5_oracle.h).  Every function
 * cites the reference file:line it restates.  Paths are relative to the reference
 * checkout (dropbox/witchcraft).
 *
 * Pinning (how each part is checked independently of this file):
 *   - orc_q4k_dequant: closed form of the GGML Q4_K block (exact arithmetic), swept
 *     exhaustively over scale/min byte patterns in tests/test_oracle_codecs.py and
 *     against tests/golden/q4k_blocks.npz.
 *   - orc_rel_bucket: the integer thresholds of the log-bucket map, enumerated for
 *     every distance < 2048 (tests/golden/rel_buckets.npz) and against closed forms.
 *   - encoder forward: against HuggingFace transformers' T5EncoderModel built from a
 *     local T5Config with the same (dequantized) weights, fixtures written by
 *     tests/golden/make_hf_golden.py; plus brute-force invariants.
 *   - Q8_K quantizer / Q4_K.Q8_K vec_dot: integer parts checked exactly against a
 *     direct double-precision dot over dequantized operands; float combination order
 *     is candle's and tolerance-level only ("parity unpinned" bitwise).
 */
#include "t5_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>

void orc_set_threads(int n) {
  if (n > 0) omp_set_num_threads(n);
}
int orc_max_threads(void) { return omp_get_max_threads(); }
#endif

#define QK_K 256
#define Q4K_BYTES 144
#define Q8K_BYTES 292

/* ------------------------------------------------------------------------- */
/* Block codecs                                                               */
/* ------------------------------------------------------------------------- */

/* IEEE binary16 -> binary32, exact (candle's f16::to_f32, used by BlockQ4K). */
float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do {
        e++;
        man <<= 1;
      } while ((man & 0x400) == 0);
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ff) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* GGML get_scale_min_k4: 8 six-bit (scale, min) pairs packed into 12 bytes.
 * candle k_quants (via BlockQ4K::to_float, reached from src/quantized_t5.rs:44,60,154). */
void orc_get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* BlockQ4K::to_float -- 144-byte block {f16 d, f16 dmin, u8 scales[12], u8 qs[128]}
 * -> 256 f32.  Chunk c (64 values) uses sub-blocks 2c (low nibbles of qs[32c..32c+32])
 * and 2c+1 (high nibbles).  y = (d*sc)*q - (dmin*m): the products are exact in f32, so
 * the final subtraction is the only rounding.
 * Call sites: src/quantized_t5.rs:44 (CPU default dequantize), :60, :154, :326-334. */
void orc_q4k_dequant(const uint8_t* blocks, size_t nblk, float* out) {
  for (size_t b = 0; b < nblk; b++) {
    const uint8_t* blk = blocks + b * Q4K_BYTES;
    uint16_t dh, mh;
    memcpy(&dh, blk, 2);
    memcpy(&mh, blk + 2, 2);
    const float d = orc_f16_to_f32(dh), dmin = orc_f16_to_f32(mh);
    const uint8_t* scales = blk + 4;
    const uint8_t* qs = blk + 16;
    float* y = out + b * QK_K;
    for (int c = 0; c < 4; c++) {
      uint8_t sc, m;
      orc_get_scale_min_k4(2 * c, scales, &sc, &m);
      const float d1 = d * sc, m1 = dmin * m;
      orc_get_scale_min_k4(2 * c + 1, scales, &sc, &m);
      const float d2 = d * sc, m2 = dmin * m;
      for (int l = 0; l < 32; l++) y[64 * c + l] = d1 * (float)(qs[32 * c + l] & 0xf) - m1;
      for (int l = 0; l < 32; l++) y[64 * c + 32 + l] = d2 * (float)(qs[32 * c + l] >> 4) - m2;
    }
  }
}

/* Rust f32::round: half away from zero (candle k_quants nearest_int). */
static int orc_nearest_int(float v) { return (int)roundf(v); }

/* BlockQ8K::from_float (src/fused_matmul.rs:36-41,147-152 call it per activation row).
 * Block {f32 d, i8 qs[256], i16 bsums[16]}: iscale = -128/x_at_max|x|, q = min(127, round(iscale*x)),
 * d = 1/iscale, bsums = sums of 16-value groups. */
void orc_q8k_quantize(const float* x, size_t n, uint8_t* blocks) {
  for (size_t b = 0; b < n / QK_K; b++) {
    const float* xb = x + b * QK_K;
    uint8_t* blk = blocks + b * Q8K_BYTES;
    float maxv = 0.f, amax = 0.f;
    for (int j = 0; j < QK_K; j++) {
      float ax = fabsf(xb[j]);
      if (ax > amax) {
        amax = ax;
        maxv = xb[j];
      }
    }
    int8_t qs[QK_K];
    int16_t bsums[16];
    float d;
    if (amax == 0.f) {
      d = 0.f;
      memset(qs, 0, sizeof qs);
    } else {
      const float iscale = -128.f / maxv;
      for (int j = 0; j < QK_K; j++) {
        int v = orc_nearest_int(iscale * xb[j]);
        qs[j] = (int8_t)(v < 127 ? v : 127);
      }
      d = 1.f / iscale;
    }
    for (int j = 0; j < 16; j++) {
      int s = 0;
      for (int i = 0; i < 16; i++) s += qs[16 * j + i];
      bsums[j] = (int16_t)s;
    }
    memcpy(blk, &d, 4);
    memcpy(blk + 4, qs, QK_K);
    memcpy(blk + 4 + QK_K, bsums, 32);
  }
}

/* BlockQ4K::vec_dot with a Q8K right-hand side (src/fused_matmul.rs:55,166-167).
 * Integer sub-block sums are exact; the float combination follows GGML's generic
 * reference (8 lane partial sums, then -dmin*d8*sum(bsums*mins)). */
float orc_q4k_q8k_vec_dot(size_t n, const uint8_t* q4k, const uint8_t* q8k) {
  float sums[8] = {0};
  float sumf = 0.f;
  for (size_t b = 0; b < n / QK_K; b++) {
    const uint8_t* x = q4k + b * Q4K_BYTES;
    const uint8_t* y = q8k + b * Q8K_BYTES;
    uint16_t dh, mh;
    memcpy(&dh, x, 2);
    memcpy(&mh, x + 2, 2);
    float yd;
    memcpy(&yd, y, 4);
    const int8_t* q8 = (const int8_t*)(y + 4);
    int16_t bsums[16];
    memcpy(bsums, y + 4 + QK_K, 32);
    const uint8_t* scales = x + 4;
    const uint8_t* q4 = x + 16;
    int8_t aux8[QK_K];
    for (int c = 0; c < 4; c++) {
      for (int l = 0; l < 32; l++) aux8[64 * c + l] = (int8_t)(q4[32 * c + l] & 0xf);
      for (int l = 0; l < 32; l++) aux8[64 * c + 32 + l] = (int8_t)(q4[32 * c + l] >> 4);
    }
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; j++) orc_get_scale_min_k4(j, scales, &sc[j], &mn[j]);
    int sumi = 0;
    for (int j = 0; j < 16; j++) sumi += bsums[j] * mn[j / 2];
    int32_t aux32[8] = {0};
    for (int j = 0; j < 8; j++) {
      const int scale = sc[j];
      for (int g = 0; g < 4; g++) {
        for (int l = 0; l < 8; l++) aux32[l] += scale * (q8[32 * j + 8 * g + l] * aux8[32 * j + 8 * g + l]);
      }
    }
    const float d = orc_f16_to_f32(dh) * yd;
    for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
    const float dmin = orc_f16_to_f32(mh) * yd;
    sumf -= dmin * (float)sumi;
  }
  for (int l = 0; l < 8; l++) sumf += sums[l];
  return sumf;
}

/* fbgemm-rs/src/bf16.rs:21-25: f32 -> bf16 by truncation (bits >> 16), widened back. */
float orc_bf16_trunc(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  u &= 0xffff0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

/* ------------------------------------------------------------------------- */
/* Scalar ops                                                                 */
/* ------------------------------------------------------------------------- */

/* Bidirectional relative-position bucket, src/quantized_t5.rs:444-483.
 * Rust f32::log(x, base) = ln(x)/ln(base) with the platform logf. */
uint32_t orc_rel_bucket(uint32_t i, uint32_t j, uint32_t num_buckets_total, uint32_t max_distance) {
  const uint32_t num_buckets = num_buckets_total / 2;
  const uint32_t max_exact = num_buckets / 2;
  if (i < j) {
    if (j - i < max_exact) return j - i + num_buckets;
    float b = logf((float)(j - i) / (float)max_exact) /
              logf((float)max_distance / (float)max_exact) * (float)(num_buckets - max_exact);
    uint32_t v = max_exact + num_buckets + (uint32_t)b;
    return v < num_buckets_total - 1 ? v : num_buckets_total - 1;
  } else if (i - j < max_exact) {
    return i - j;
  } else {
    float b = logf((float)(i - j) / (float)max_exact) /
              logf((float)max_distance / (float)max_exact) * (float)(num_buckets - max_exact);
    uint32_t v = max_exact + (uint32_t)b;
    return v < num_buckets - 1 ? v : num_buckets - 1;
  }
}

/* candle Tensor::gelu (Activation::NewGelu, src/quantized_t5.rs:105-106,246): tanh form. */
float orc_gelu_tanh(float x) {
  const float k = 0.79788456080286535587989211986876373f; /* sqrt(2/pi) */
  return 0.5f * x * (1.0f + tanhf(k * x * (1.0f + 0.044715f * x * x)));
}

/* Pade [3,3] tanh, src/fused_matmul.rs:129-134. */
float orc_fast_tanh(float x) {
  x = x < -4.97f ? -4.97f : (x > 4.97f ? 4.97f : x);
  const float x2 = x * x;
  return x * (135135.0f + x2 * (17325.0f + x2 * (378.0f + x2))) /
         (135135.0f + x2 * (62370.0f + x2 * (3150.0f + 28.0f * x2)));
}

/* Gate activation of the hybrid fused FFN, src/fused_matmul.rs:168-170. */
float orc_gelu_pade(float g) {
  return 0.5f * g * (1.0f + orc_fast_tanh(0.7978845608f * g * (1.0f + 0.044715f * g * g)));
}

/* T5LayerNorm::forward, src/quantized_t5.rs:162-173: x / sqrt(mean(x^2) + eps) * w. */
void orc_rmsnorm(const float* x, const float* w, int rows, int d, float eps, float* out, int acc64) {
  for (int r = 0; r < rows; r++) {
    const float* xr = x + (size_t)r * d;
    float var;
    if (acc64) {
      double s = 0;
      for (int i = 0; i < d; i++) s += (double)xr[i] * xr[i];
      var = (float)(s / d);
    } else {
      float s = 0.f;
      for (int i = 0; i < d; i++) s += xr[i] * xr[i];
      var = s / (float)d;
    }
    const float den = sqrtf(var + eps);
    for (int i = 0; i < d; i++) out[(size_t)r * d + i] = (xr[i] / den) * w[i];
  }
}

/* candle_nn::ops::softmax_last_dim (src/quantized_t5.rs:496): max, exp(x-max), sum, divide. */
void orc_softmax_rows(float* s, int rows, int cols) {
  for (int r = 0; r < rows; r++) {
    float* row = s + (size_t)r * cols;
    float mx = -INFINITY;
    for (int j = 0; j < cols; j++) mx = row[j] > mx ? row[j] : mx;
    float sum = 0.f;
    for (int j = 0; j < cols; j++) {
      row[j] = expf(row[j] - mx);
      sum += row[j];
    }
    for (int j = 0; j < cols; j++) row[j] /= sum;
  }
}

/* Linear layer y = x W^T with W given transposed (wt[K][N]), the layout both
 * candle's f32 matmul (src/fused_matmul.rs:376-383, default path) and this loop
 * stream well.  Each dot is accumulated sequentially in k. */
static void linear_t(const float* x, const float* wt, int T, int N, int K, float* y, int acc64) {
  enum { TB = 16, NB = 256 };
  const int ntb = (T + TB - 1) / TB, nnb = (N + NB - 1) / NB;
#pragma omp parallel for collapse(2) schedule(static)
  for (int tb = 0; tb < ntb; tb++) {
    for (int nb = 0; nb < nnb; nb++) {
      const int t0 = tb * TB, t1 = t0 + TB < T ? t0 + TB : T;
      const int n0 = nb * NB, n1 = n0 + NB < N ? n0 + NB : N;
      const int nn = n1 - n0;
      if (acc64) {
        double acc[TB][NB];
        for (int t = t0; t < t1; t++)
          for (int n = 0; n < nn; n++) acc[t - t0][n] = 0.0;
        for (int k = 0; k < K; k++) {
          const float* wr = wt + (size_t)k * N + n0;
          for (int t = t0; t < t1; t++) {
            const double xv = x[(size_t)t * K + k];
            double* a = acc[t - t0];
            for (int n = 0; n < nn; n++) a[n] += xv * (double)wr[n];
          }
        }
        for (int t = t0; t < t1; t++)
          for (int n = 0; n < nn; n++) y[(size_t)t * N + n0 + n] = (float)acc[t - t0][n];
      } else {
        float acc[TB][NB];
        for (int t = t0; t < t1; t++)
          for (int n = 0; n < nn; n++) acc[t - t0][n] = 0.f;
        for (int k = 0; k < K; k++) {
          const float* wr = wt + (size_t)k * N + n0;
          for (int t = t0; t < t1; t++) {
            const float xv = x[(size_t)t * K + k];
            float* a = acc[t - t0];
            for (int n = 0; n < nn; n++) a[n] += xv * wr[n];
          }
        }
        for (int t = t0; t < t1; t++)
          for (int n = 0; n < nn; n++) y[(size_t)t * N + n0 + n] = acc[t - t0][n];
      }
    }
  }
}

static float* transpose_alloc(const float* w, int N, int K) {
  float* wt = (float*)malloc((size_t)N * K * sizeof(float));
  if (!wt) return NULL;
  for (int n = 0; n < N; n++)
    for (int k = 0; k < K; k++) wt[(size_t)k * N + n] = w[(size_t)n * K + k];
  return wt;
}

void orc_linear(const float* x, const float* w, int T, int N, int K, float* y, int acc64) {
  float* wt = transpose_alloc(w, N, K);
  if (!wt) return;
  linear_t(x, wt, T, N, K, y, acc64);
  free(wt);
}

/* ------------------------------------------------------------------------- */
/* Query-side scoring next to the encoder.                                     */
/* ------------------------------------------------------------------------- */

/* fast_ops::matmul_t (src/fast_ops.rs:98-116) / PackedRight::matmul (:65-95): C[M,N] =
 * A[M,D] . B[N,D]^T.  bf16_b: B truncated to bf16 first (the fbgemm build's
 * PackedMatrixBf16::from_transposed, fbgemm-rs/src/bf16.rs:21-31), A kept f32.  acc64
 * accumulates each dot product in double (the reference order is unknown; tests use it). */
void orc_matmul_t(const float* a, int M, const float* b, int N, int D, int bf16_b, float* c, int acc64) {
#pragma omp parallel for schedule(static)
  for (int i = 0; i < M; i++) {
    const float* ar = a + (size_t)i * D;
    for (int j = 0; j < N; j++) {
      const float* br = b + (size_t)j * D;
      if (acc64) {
        double s = 0.0;
        for (int k = 0; k < D; k++) s += (double)ar[k] * (double)(bf16_b ? orc_bf16_trunc(br[k]) : br[k]);
        c[(size_t)i * N + j] = (float)s;
      } else {
        float s = 0.f;
        for (int k = 0; k < D; k++) s += ar[k] * (bf16_b ? orc_bf16_trunc(br[k]) : br[k]);
        c[(size_t)i * N + j] = s;
      }
    }
  }
}

/* matmul_argmax_batched (src/lib.rs:187-208): per row of A, the index of the largest
 * A[i] . B[j]; candle's argmax keeps the first maximum, so ties go to the smallest j. */
void orc_matmul_argmax(const float* a, int M, const float* b, int N, int D, int bf16_b, uint32_t* out, int acc64) {
#pragma omp parallel for schedule(static)
  for (int i = 0; i < M; i++) {
    const float* ar = a + (size_t)i * D;
    double best = -INFINITY;
    uint32_t bi = 0;
    for (int j = 0; j < N; j++) {
      const float* br = b + (size_t)j * D;
      double s = 0.0;
      if (acc64) {
        for (int k = 0; k < D; k++) s += (double)ar[k] * (double)(bf16_b ? orc_bf16_trunc(br[k]) : br[k]);
      } else {
        float f = 0.f;
        for (int k = 0; k < D; k++) f += ar[k] * (bf16_b ? orc_bf16_trunc(br[k]) : br[k]);
        s = f;
      }
      if (j == 0 || s > best) {
        best = s;
        bi = (uint32_t)j;
      }
    }
    out[i] = bi;
  }
}

/* ------------------------------------------------------------------------- */
/* GGUF reader (format written by tools/quantize-tool/src/main.rs:33-35 via    */
/* candle gguf_file::write, read by VarBuilder::from_gguf_buffer at            */
/* src/quantized_t5.rs:740-743).  Independent of the product's reader.         */
/* ------------------------------------------------------------------------- */

enum { GGML_F32 = 0, GGML_F16 = 1, GGML_Q4K = 12 };

typedef struct {
  char name[160];
  int ndims;
  uint64_t dims[4]; /* GGUF order: dims[0] innermost */
  uint32_t type;
  uint64_t offset;
  const uint8_t* data;
} gguf_tensor;

typedef struct {
  const uint8_t* p;
  size_t len, pos;
  int bad;
} rd;

static uint64_t rd_u(rd* r, int nbytes) {
  if (r->pos + nbytes > r->len) {
    r->bad = 1;
    return 0;
  }
  uint64_t v = 0;
  memcpy(&v, r->p + r->pos, nbytes);
  r->pos += nbytes;
  return v;
}

static void rd_skip_value(rd* r, uint32_t type);

static void rd_skip_string(rd* r) {
  uint64_t n = rd_u(r, 8);
  if (r->pos + n > r->len) {
    r->bad = 1;
    return;
  }
  r->pos += n;
}

static void rd_skip_value(rd* r, uint32_t type) {
  static const int sz[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
  if (type == 8) {
    rd_skip_string(r);
  } else if (type == 9) {
    uint32_t et = (uint32_t)rd_u(r, 4);
    uint64_t n = rd_u(r, 8);
    for (uint64_t i = 0; i < n && !r->bad; i++) rd_skip_value(r, et);
  } else if (type < 13) {
    rd_u(r, sz[type]);
  } else {
    r->bad = 1;
  }
}

static int gguf_parse(const uint8_t* buf, size_t len, gguf_tensor** out, int* nout, char* err,
                      size_t errlen) {
  rd r = {buf, len, 0, 0};
  uint32_t magic = (uint32_t)rd_u(&r, 4);
  if (magic != 0x46554747u) {
    snprintf(err, errlen, "not a GGUF buffer");
    return -1;
  }
  uint32_t version = (uint32_t)rd_u(&r, 4);
  if (version < 2 || version > 3) {
    snprintf(err, errlen, "unsupported GGUF version %u", version);
    return -1;
  }
  uint64_t nt = rd_u(&r, 8), nkv = rd_u(&r, 8);
  uint64_t alignment = 32;
  for (uint64_t i = 0; i < nkv && !r.bad; i++) {
    uint64_t klen = rd_u(&r, 8);
    int is_align = (klen == 17 && r.pos + 17 <= len && memcmp(buf + r.pos, "general.alignment", 17) == 0);
    r.pos += klen;
    uint32_t vt = (uint32_t)rd_u(&r, 4);
    if (is_align && vt == 4)
      alignment = rd_u(&r, 4);
    else
      rd_skip_value(&r, vt);
  }
  if (r.bad || nt > 100000) {
    snprintf(err, errlen, "truncated GGUF header");
    return -1;
  }
  gguf_tensor* ts = (gguf_tensor*)calloc(nt ? nt : 1, sizeof(gguf_tensor));
  for (uint64_t i = 0; i < nt && !r.bad; i++) {
    uint64_t nlen = rd_u(&r, 8);
    if (nlen >= sizeof(ts[i].name) || r.pos + nlen > len) {
      r.bad = 1;
      break;
    }
    memcpy(ts[i].name, buf + r.pos, nlen);
    ts[i].name[nlen] = 0;
    r.pos += nlen;
    ts[i].ndims = (int)rd_u(&r, 4);
    if (ts[i].ndims < 1 || ts[i].ndims > 4) {
      r.bad = 1;
      break;
    }
    for (int d = 0; d < ts[i].ndims; d++) ts[i].dims[d] = rd_u(&r, 8);
    ts[i].type = (uint32_t)rd_u(&r, 4);
    ts[i].offset = rd_u(&r, 8);
  }
  if (r.bad) {
    free(ts);
    snprintf(err, errlen, "truncated GGUF tensor table");
    return -1;
  }
  size_t data0 = (r.pos + alignment - 1) / alignment * alignment;
  for (uint64_t i = 0; i < nt; i++) {
    uint64_t ne = 1;
    for (int d = 0; d < ts[i].ndims; d++) ne *= ts[i].dims[d];
    uint64_t nbytes = ts[i].type == GGML_F32 ? ne * 4
                      : ts[i].type == GGML_F16 ? ne * 2
                      : ts[i].type == GGML_Q4K ? ne / QK_K * Q4K_BYTES
                                               : 0;
    if (nbytes == 0 || data0 + ts[i].offset + nbytes > len) {
      free(ts);
      snprintf(err, errlen, "tensor %s: unsupported type %u or out of range", ts[i].name, ts[i].type);
      return -1;
    }
    ts[i].data = buf + data0 + ts[i].offset;
  }
  *out = ts;
  *nout = (int)nt;
  return 0;
}

static const gguf_tensor* find_t(const gguf_tensor* ts, int n, const char* name) {
  for (int i = 0; i < n; i++)
    if (strcmp(ts[i].name, name) == 0) return &ts[i];
  return NULL;
}

/* QTensor::dequantize for the three tensor types the XTR GGUF holds. */
static float* dequant_tensor(const gguf_tensor* t, size_t expect_rows, size_t expect_cols) {
  size_t cols = t->dims[0], rows = 1;
  for (int d = 1; d < t->ndims; d++) rows *= t->dims[d];
  if (rows != expect_rows || cols != expect_cols) return NULL;
  size_t ne = rows * cols;
  float* out = (float*)malloc(ne * sizeof(float));
  if (!out) return NULL;
  if (t->type == GGML_F32) {
    memcpy(out, t->data, ne * 4);
  } else if (t->type == GGML_F16) {
    for (size_t i = 0; i < ne; i++) {
      uint16_t h;
      memcpy(&h, t->data + 2 * i, 2);
      out[i] = orc_f16_to_f32(h);
    }
  } else {
    orc_q4k_dequant(t->data, ne / QK_K, out);
  }
  return out;
}

/* ------------------------------------------------------------------------- */
/* Model                                                                      */
/* ------------------------------------------------------------------------- */

typedef struct {
  float *ln0, *ln1;
  float *wq_t, *wk_t, *wv_t, *wo_t;    /* transposed [K][N] */
  float *wi0_t, *wi1_t, *wff_t;        /* transposed */
  float *wi0, *wi1;                    /* row-major [F][D], for orc_ffn_dense checks */
  uint8_t *wi0_q, *wi1_q;              /* Q4_K bytes (hybrid variants) */
} orc_layer;

struct orc_model {
  orc_config cfg;
  int variant;
  float* emb;   /* [V, D] */
  float* relb;  /* [num_buckets, H] */
  orc_layer* layers;
  float* final_ln;
  float* proj_t; /* [D][P] */
  uint8_t* proj_q;
};

void orc_model_free(orc_model* m) {
  if (!m) return;
  free(m->emb);
  free(m->relb);
  if (m->layers) {
    for (int l = 0; l < m->cfg.num_layers; l++) {
      orc_layer* L = &m->layers[l];
      free(L->ln0); free(L->ln1);
      free(L->wq_t); free(L->wk_t); free(L->wv_t); free(L->wo_t);
      free(L->wi0_t); free(L->wi1_t); free(L->wff_t);
      free(L->wi0); free(L->wi1);
      free(L->wi0_q); free(L->wi1_q);
    }
    free(m->layers);
  }
  free(m->final_ln);
  free(m->proj_t);
  free(m->proj_q);
  free(m);
}

static void bf16_inplace(float* w, size_t n) {
  for (size_t i = 0; i < n; i++) w[i] = orc_bf16_trunc(w[i]);
}

static uint8_t* copy_q4k(const gguf_tensor* t) {
  if (t->type != GGML_Q4K) return NULL;
  size_t ne = t->dims[0] * (t->ndims > 1 ? t->dims[1] : 1);
  size_t nb = ne / QK_K * Q4K_BYTES;
  uint8_t* q = (uint8_t*)malloc(nb);
  if (q) memcpy(q, t->data, nb);
  return q;
}

/* T5EncoderModel::load (src/quantized_t5.rs:681-696) + new_qmm / new_qmm_dequant
 * (:39-62) for the chosen variant. */
orc_model* orc_model_from_gguf(const uint8_t* buf, size_t len, const orc_config* cfg, int variant,
                               char* err, size_t errlen) {
  gguf_tensor* ts = NULL;
  int nt = 0;
  if (gguf_parse(buf, len, &ts, &nt, err, errlen)) return NULL;
  orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
  m->cfg = *cfg;
  m->variant = variant;
  const int D = cfg->d_model, H = cfg->num_heads, inner = cfg->num_heads * cfg->d_kv;
  const int F = cfg->d_ff, P = cfg->proj_dim;
  char name[200];
#define NEED(ptr, nm, rows, cols)                                                      \
  do {                                                                                 \
    const gguf_tensor* t_ = find_t(ts, nt, nm);                                         \
    if (!t_) {                                                                         \
      snprintf(err, errlen, "missing tensor %s", nm);                                  \
      goto fail;                                                                       \
    }                                                                                  \
    ptr = dequant_tensor(t_, rows, cols);                                              \
    if (!ptr) {                                                                        \
      snprintf(err, errlen, "tensor %s: bad shape", nm);                               \
      goto fail;                                                                       \
    }                                                                                  \
  } while (0)
  {
    const char* embn = find_t(ts, nt, "shared.weight") ? "shared.weight" : "encoder.embed_tokens.weight";
    NEED(m->emb, embn, (size_t)cfg->vocab_size, (size_t)D);
  }
  NEED(m->relb, "encoder.block.0.layer.0.SelfAttention.relative_attention_bias.weight",
       (size_t)cfg->num_buckets, (size_t)H);
  m->layers = (orc_layer*)calloc(cfg->num_layers, sizeof(orc_layer));
  for (int l = 0; l < cfg->num_layers; l++) {
    orc_layer* L = &m->layers[l];
    float* w;
    const int bf = (variant == ORC_VARIANT_HYBRID_BF16);
#define DENSE_T(dst, suffix, rows, cols)                                                 \
  do {                                                                                 \
    snprintf(name, sizeof name, "encoder.block.%d.layer.%s", l, suffix);               \
    NEED(w, name, rows, cols);                                                         \
    if (bf) bf16_inplace(w, (size_t)(rows) * (cols));                                  \
    dst = transpose_alloc(w, rows, cols);                                              \
    free(w);                                                                           \
  } while (0)
    snprintf(name, sizeof name, "encoder.block.%d.layer.0.layer_norm.weight", l);
    NEED(L->ln0, name, 1, (size_t)D);
    snprintf(name, sizeof name, "encoder.block.%d.layer.1.layer_norm.weight", l);
    NEED(L->ln1, name, 1, (size_t)D);
    DENSE_T(L->wq_t, "0.SelfAttention.q.weight", inner, D);
    DENSE_T(L->wk_t, "0.SelfAttention.k.weight", inner, D);
    DENSE_T(L->wv_t, "0.SelfAttention.v.weight", inner, D);
    DENSE_T(L->wo_t, "0.SelfAttention.o.weight", D, inner);
    if (cfg->gated) {
      /* wi_0 / wi_1 are never bf16-truncated: hybrid keeps them Q4_K (:216-217,51-55). */
      snprintf(name, sizeof name, "encoder.block.%d.layer.1.DenseReluDense.wi_0.weight", l);
      NEED(L->wi0, name, F, D);
      L->wi0_t = transpose_alloc(L->wi0, F, D);
      if (variant != ORC_VARIANT_DEFAULT) L->wi0_q = copy_q4k(find_t(ts, nt, name));
      snprintf(name, sizeof name, "encoder.block.%d.layer.1.DenseReluDense.wi_1.weight", l);
      NEED(L->wi1, name, F, D);
      L->wi1_t = transpose_alloc(L->wi1, F, D);
      if (variant != ORC_VARIANT_DEFAULT) L->wi1_q = copy_q4k(find_t(ts, nt, name));
      if (variant != ORC_VARIANT_DEFAULT && (!L->wi0_q || !L->wi1_q)) {
        snprintf(err, errlen, "hybrid variant needs Q4_K wi_0/wi_1 (QGatedMatMul)");
        goto fail;
      }
    } else {
      snprintf(name, sizeof name, "encoder.block.%d.layer.1.DenseReluDense.wi.weight", l);
      NEED(L->wi0, name, F, D);
      L->wi0_t = transpose_alloc(L->wi0, F, D);
    }
    DENSE_T(L->wff_t, "1.DenseReluDense.wo.weight", D, F);
#undef DENSE_T
  }
  NEED(m->final_ln, "encoder.final_layer_norm.weight", 1, (size_t)D);
  {
    float* w;
    NEED(w, "linear.weight", (size_t)P, (size_t)D);
    m->proj_t = transpose_alloc(w, P, D);
    free(w);
    if (variant != ORC_VARIANT_DEFAULT) {
      m->proj_q = copy_q4k(find_t(ts, nt, "linear.weight"));
      if (!m->proj_q) {
        snprintf(err, errlen, "hybrid variant needs Q4_K linear.weight (QTiledOp)");
        goto fail;
      }
    }
  }
#undef NEED
  free(ts);
  return m;
fail:
  free(ts);
  orc_model_free(m);
  return NULL;
}

int orc_model_dims(const orc_model* m, orc_config* cfg) {
  *cfg = m->cfg;
  return 0;
}

/* QTiledOp / tiled_matmul_inner (src/fused_matmul.rs:28-60): Q8_K activations . Q4_K rows. */
static void q4k_q8k_linear(const float* x, const uint8_t* wq, int T, int N, int K, float* y) {
  const size_t q8row = (size_t)(K / QK_K) * Q8K_BYTES, q4row = (size_t)(K / QK_K) * Q4K_BYTES;
  uint8_t* xq = (uint8_t*)malloc((size_t)T * q8row);
  for (int t = 0; t < T; t++) orc_q8k_quantize(x + (size_t)t * K, K, xq + t * q8row);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; n++)
    for (int t = 0; t < T; t++) y[(size_t)t * N + n] = orc_q4k_q8k_vec_dot(K, wq + n * q4row, xq + t * q8row);
  free(xq);
}

/* fused_gated_gelu_inner (src/fused_matmul.rs:138-177). */
static void q4k_gated_gelu(const float* x, const uint8_t* w0, const uint8_t* w1, int T, int N, int K,
                           float* h) {
  const size_t q8row = (size_t)(K / QK_K) * Q8K_BYTES, q4row = (size_t)(K / QK_K) * Q4K_BYTES;
  uint8_t* xq = (uint8_t*)malloc((size_t)T * q8row);
  for (int t = 0; t < T; t++) orc_q8k_quantize(x + (size_t)t * K, K, xq + t * q8row);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; n++) {
    for (int t = 0; t < T; t++) {
      const float g = orc_q4k_q8k_vec_dot(K, w0 + n * q4row, xq + t * q8row);
      const float u = orc_q4k_q8k_vec_dot(K, w1 + n * q4row, xq + t * q8row);
      h[(size_t)t * N + n] = orc_gelu_pade(g) * u;
    }
  }
  free(xq);
}

/* Position-bias lookup by signed distance: bias only depends on (j - i)
 * (src/quantized_t5.rs:452-490 builds it for every (i, j); values are identical). */
static float* rel_bias_lut(const orc_model* m, int L) {
  const int H = m->cfg.num_heads;
  float* lut = (float*)malloc((size_t)H * (2 * L - 1) * sizeof(float));
  for (int delta = -(L - 1); delta <= L - 1; delta++) {
    uint32_t i = delta < 0 ? (uint32_t)(-delta) : 0, j = delta < 0 ? 0 : (uint32_t)delta;
    uint32_t b = orc_rel_bucket(i, j, (uint32_t)m->cfg.num_buckets, (uint32_t)m->cfg.max_distance);
    for (int h = 0; h < H; h++) lut[(size_t)h * (2 * L - 1) + delta + L - 1] = m->relb[b * H + h];
  }
  return lut;
}

int orc_position_bias(const orc_model* m, int L, float* bias) {
  const int H = m->cfg.num_heads;
  float* lut = rel_bias_lut(m, L);
  for (int h = 0; h < H; h++)
    for (int i = 0; i < L; i++)
      for (int j = 0; j < L; j++)
        bias[((size_t)h * L + i) * L + j] = lut[(size_t)h * (2 * L - 1) + (j - i) + L - 1];
  free(lut);
  return 0;
}

/* T5Attention::forward core, src/quantized_t5.rs:426-500 (no 1/sqrt(d_kv) scaling). */
static void attention(const orc_model* m, const float* q, const float* k, const float* v, int L,
                      const float* lut, float* o, int acc64) {
  const int H = m->cfg.num_heads, dk = m->cfg.d_kv, inner = H * dk;
#pragma omp parallel for schedule(static)
  for (int hi = 0; hi < H * L; hi++) {
    const int h = hi / L, i = hi % L;
    float* s = (float*)malloc((size_t)L * sizeof(float));
    for (int j = 0; j < L; j++) {
      const float* qi = q + (size_t)i * inner + h * dk;
      const float* kj = k + (size_t)j * inner + h * dk;
      float dot;
      if (acc64) {
        double a = 0;
        for (int d = 0; d < dk; d++) a += (double)qi[d] * kj[d];
        dot = (float)a;
      } else {
        float a = 0.f;
        for (int d = 0; d < dk; d++) a += qi[d] * kj[d];
        dot = a;
      }
      s[j] = dot + lut[(size_t)h * (2 * L - 1) + (j - i) + L - 1]; /* fast_add :441,490 */
    }
    orc_softmax_rows(s, 1, L);
    for (int d = 0; d < dk; d++) {
      if (acc64) {
        double a = 0;
        for (int j = 0; j < L; j++) a += (double)s[j] * v[(size_t)j * inner + h * dk + d];
        o[(size_t)i * inner + h * dk + d] = (float)a;
      } else {
        float a = 0.f;
        for (int j = 0; j < L; j++) a += s[j] * v[(size_t)j * inner + h * dk + d];
        o[(size_t)i * inner + h * dk + d] = a;
      }
    }
    free(s);
  }
}

/* T5DenseGatedActDense / T5DenseActDense forward on normalised input (src/quantized_t5.rs:197-252). */
static void ffn(const orc_model* m, const orc_layer* Ly, const float* xn, int T, float* y, int acc64) {
  const int D = m->cfg.d_model, F = m->cfg.d_ff;
  float* hbuf = (float*)malloc((size_t)T * F * sizeof(float));
  if (m->cfg.gated) {
    if (m->variant != ORC_VARIANT_DEFAULT) {
      q4k_gated_gelu(xn, Ly->wi0_q, Ly->wi1_q, T, F, D, hbuf);
    } else {
      float* u = (float*)malloc((size_t)T * F * sizeof(float));
      linear_t(xn, Ly->wi0_t, T, F, D, hbuf, acc64);
      linear_t(xn, Ly->wi1_t, T, F, D, u, acc64);
      for (size_t i = 0; i < (size_t)T * F; i++) hbuf[i] = orc_gelu_tanh(hbuf[i]) * u[i];
      free(u);
    }
  } else {
    linear_t(xn, Ly->wi0_t, T, F, D, hbuf, acc64);
    for (size_t i = 0; i < (size_t)T * F; i++) hbuf[i] = hbuf[i] > 0.f ? hbuf[i] : 0.f;
  }
  linear_t(hbuf, Ly->wff_t, T, D, F, y, acc64);
  free(hbuf);
}

/* T5Block::forward (src/quantized_t5.rs:598-627) with the bias LUT for length L. */
static void block_forward(const orc_model* m, int layer, const float* x_in, int L, const float* lut,
                          float* x_out, int acc64) {
  const int D = m->cfg.d_model, inner = m->cfg.num_heads * m->cfg.d_kv;
  const orc_layer* Ly = &m->layers[layer];
  float* xn = (float*)malloc((size_t)L * D * sizeof(float));
  float* q = (float*)malloc((size_t)L * inner * sizeof(float));
  float* k = (float*)malloc((size_t)L * inner * sizeof(float));
  float* v = (float*)malloc((size_t)L * inner * sizeof(float));
  float* o = (float*)malloc((size_t)L * inner * sizeof(float));
  float* y = (float*)malloc((size_t)L * D * sizeof(float));
  /* T5LayerSelfAttention::forward :523-535 */
  orc_rmsnorm(x_in, Ly->ln0, L, D, m->cfg.eps, xn, acc64);
  linear_t(xn, Ly->wq_t, L, inner, D, q, acc64);
  linear_t(xn, Ly->wk_t, L, inner, D, k, acc64);
  linear_t(xn, Ly->wv_t, L, inner, D, v, acc64);
  attention(m, q, k, v, L, lut, o, acc64);
  linear_t(o, Ly->wo_t, L, D, inner, y, acc64);
  for (size_t i = 0; i < (size_t)L * D; i++) x_out[i] = x_in[i] + y[i]; /* fast_add :533 */
  /* T5LayerFF::forward :284-293 */
  orc_rmsnorm(x_out, Ly->ln1, L, D, m->cfg.eps, xn, acc64);
  ffn(m, Ly, xn, L, y, acc64);
  for (size_t i = 0; i < (size_t)L * D; i++) x_out[i] += y[i]; /* fast_add :291 */
  free(xn); free(q); free(k); free(v); free(o); free(y);
}

int orc_layer_forward(const orc_model* m, int layer, const float* x_in, int L, float* x_out, int acc64) {
  if (layer < 0 || layer >= m->cfg.num_layers || L <= 0) return -1;
  float* lut = rel_bias_lut(m, L);
  block_forward(m, layer, x_in, L, lut, x_out, acc64);
  free(lut);
  return 0;
}

int orc_ffn_dense(const orc_model* m, int layer, const float* x, int T, float* y, int acc64) {
  if (layer < 0 || layer >= m->cfg.num_layers || T <= 0) return -1;
  ffn(m, &m->layers[layer], x, T, y, acc64);
  return 0;
}

/* T5Stack::forward (src/quantized_t5.rs:654-670) up to `upto` blocks, before the final norm. */
int orc_encoder_hidden(const orc_model* m, const uint32_t* ids, int L, int upto, float* x, int acc64) {
  const int D = m->cfg.d_model;
  if (L <= 0 || upto < 0 || upto > m->cfg.num_layers) return -1;
  for (int t = 0; t < L; t++) {
    if (ids[t] >= (uint32_t)m->cfg.vocab_size) return -2;
    memcpy(x + (size_t)t * D, m->emb + (size_t)ids[t] * D, D * sizeof(float)); /* Embedding :659 */
  }
  float* lut = rel_bias_lut(m, L);
  float* tmp = (float*)malloc((size_t)L * D * sizeof(float));
  for (int l = 0; l < upto; l++) {
    block_forward(m, l, x, L, lut, tmp, acc64);
    memcpy(x, tmp, (size_t)L * D * sizeof(float));
  }
  free(tmp);
  free(lut);
  return 0;
}

/* final_layer_norm (:669) + final_projection (:700). */
int orc_final(const orc_model* m, const float* x, int L, float* out, int acc64) {
  const int D = m->cfg.d_model, P = m->cfg.proj_dim;
  float* xn = (float*)malloc((size_t)L * D * sizeof(float));
  orc_rmsnorm(x, m->final_ln, L, D, m->cfg.eps, xn, acc64);
  if (m->variant != ORC_VARIANT_DEFAULT)
    q4k_q8k_linear(xn, m->proj_q, L, P, D, out);
  else
    linear_t(xn, m->proj_t, L, P, D, out, acc64);
  free(xn);
  return 0;
}

/* T5EncoderModel::forward (src/quantized_t5.rs:698-701). */
int orc_encoder_forward(const orc_model* m, const uint32_t* ids, int L, float* out, int acc64) {
  const int D = m->cfg.d_model;
  float* x = (float*)malloc((size_t)L * D * sizeof(float));
  int rc = orc_encoder_hidden(m, ids, L, m->cfg.num_layers, x, acc64);
  if (rc == 0) rc = orc_final(m, x, L, out, acc64);
  free(x);
  return rc;
}

/* Embedder::embed after tokenisation (src/embedder.rs:27-101). */
int orc_embed_ids(const orc_model* m, const uint32_t* ids, int n, int max_len, int stride, float* out,
                  int32_t* kept, int acc64) {
  const int P = m->cfg.proj_dim;
  if (n <= 0) return -1;
  float* accum = (float*)calloc((size_t)n * P, sizeof(float));
  float* chunk = (float*)malloc((size_t)(max_len < n ? max_len : n) * P * sizeof(float));
  int start = 0;
  for (;;) {
    int end = start + max_len < n ? start + max_len : n;
    if (orc_encoder_forward(m, ids + start, end - start, chunk, acc64)) {
      free(accum);
      free(chunk);
      return -2;
    }
    for (int i = 0; i < end - start; i++)
      for (int c = 0; c < P; c++) accum[(size_t)(start + i) * P + c] += chunk[(size_t)i * P + c];
    if (end == n) break;
    start = end > stride ? end - stride : 0; /* saturating_sub :62 */
  }
  int nk = 0;
  for (int t = 0; t < n; t++) {
    const float* v = accum + (size_t)t * P;
    float ss = 0.f;
    for (int c = 0; c < P; c++) ss += v[c] * v[c];
    const float norm = sqrtf(ss);
    if (norm >= 1.0f) { /* MIN_NORM :79-88 */
      for (int c = 0; c < P; c++) out[(size_t)nk * P + c] = v[c] / norm; /* normalize_l2 :7-9 */
      kept[nk++] = t;
    }
  }
  free(accum);
  free(chunk);
  return nk > 0 ? nk : -1;
}
