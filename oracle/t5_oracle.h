/*
 * t5_oracle.h -- CPU restatement of Witchcraft's quantized XTR-T5 encoder numerics.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * implementation in witchcraft_amd/.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it.  The product never links it.
 *
 * Reference (read-only, /root/reference):
 *   src/quantized_t5.rs   encoder forward, variant selection (new_qmm*)
 *   src/fused_matmul.rs   hybrid-dequant numerics (Q8_K activations, Pade tanh)
 *   src/fast_ops.rs       elementwise adds
 *   src/embedder.rs       windowing, MIN_NORM filter, L2 normalisation
 *   fbgemm-rs/src/bf16.rs bf16 truncation of pre-dequantized weights
 * The Q4_K / Q8_K block codecs are candle-core's (git rev 5bd5618, not vendored);
 * they restate the public GGML k-quants block design.
 */
#ifndef T5_ORACLE_H
#define T5_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Numerics variant (src/quantized_t5.rs:39-62, src/fused_matmul.rs). */
enum {
  ORC_VARIANT_DEFAULT = 0, /* t5-quantized on CPU: every Q4_K weight dequantized to f32 */
  ORC_VARIANT_HYBRID = 1,  /* hybrid-dequant: wi_0/wi_1/linear Q4_K x Q8_K, Pade gelu */
  ORC_VARIANT_HYBRID_BF16 = 2 /* hybrid-dequant+fbgemm: f32 weights truncated to bf16 */
};

typedef struct {
  int32_t vocab_size, d_model, d_kv, d_ff, num_layers, num_heads;
  int32_t num_buckets, max_distance;
  float eps;
  int32_t gated; /* 1 = gated-gelu (T5DenseGatedActDense), 0 = relu (T5DenseActDense) */
  int32_t proj_dim; /* 128 for XTR (linear.weight) */
} orc_config;

typedef struct orc_model orc_model;

/* ---- block codecs ---- */
/* OpenMP threads of the oracle's parallel loops: set, and read back what they will use. */
void orc_set_threads(int n);
int orc_max_threads(void);
float orc_f16_to_f32(uint16_t h);
void orc_get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m);
void orc_q4k_dequant(const uint8_t* blocks, size_t nblk, float* out);
void orc_q8k_quantize(const float* x, size_t n, uint8_t* blocks /* n/256 * 292 B */);
float orc_q4k_q8k_vec_dot(size_t n, const uint8_t* q4k, const uint8_t* q8k);
float orc_bf16_trunc(float x);

/* ---- scalar ops ---- */
uint32_t orc_rel_bucket(uint32_t i, uint32_t j, uint32_t num_buckets, uint32_t max_distance);
float orc_gelu_tanh(float x);
float orc_fast_tanh(float x);
float orc_gelu_pade(float x);
void orc_rmsnorm(const float* x, const float* w, int rows, int d, float eps, float* out, int acc64);
void orc_softmax_rows(float* s, int rows, int cols);
/* y[T,N] = x[T,K] . W[N,K]^T  (f32 math; acc64 = accumulate each dot in double) */
void orc_linear(const float* x, const float* w, int T, int N, int K, float* y, int acc64);

/* ---- query-side scoring ---- */
/* c[M,N] = a[M,D] . b[N,D]^T (bf16_b: b truncated to bf16 first) */
void orc_matmul_t(const float* a, int M, const float* b, int N, int D, int bf16_b, float* c, int acc64);
/* out[i] = first argmax_j a[i] . b[j] */
void orc_matmul_argmax(const float* a, int M, const float* b, int N, int D, int bf16_b, uint32_t* out, int acc64);

/* ---- GGUF + model ---- */
orc_model* orc_model_from_gguf(const uint8_t* buf, size_t len, const orc_config* cfg, int variant,
                               char* err, size_t errlen);
void orc_model_free(orc_model* m);
/* Full encoder for one sequence of length L (batch 1, as Embedder::embed does):
 * out[L, proj_dim] un-normalised (src/quantized_t5.rs:698-701). */
int orc_encoder_forward(const orc_model* m, const uint32_t* ids, int L, float* out, int acc64);
/* Hidden state after embedding + `upto_layer` blocks (0 = embeddings only), pre final norm. */
int orc_encoder_hidden(const orc_model* m, const uint32_t* ids, int L, int upto_layer, float* x,
                       int acc64);
/* One T5Block on one sequence: x_out = block[layer](x_in) (src/quantized_t5.rs:598-627). */
int orc_layer_forward(const orc_model* m, int layer, const float* x_in, int L, float* x_out,
                      int acc64);
/* T5DenseGatedActDense alone (src/quantized_t5.rs:231-252): y = wo(gelu(x wi_0^T) * (x wi_1^T)). */
int orc_ffn_dense(const orc_model* m, int layer, const float* x, int T, float* y, int acc64);
/* Final RMSNorm + projection on hidden states x[L, d_model]. */
int orc_final(const orc_model* m, const float* x, int L, float* out, int acc64);
/* Relative bias for an L x L sequence: bias[h][i][j] (src/quantized_t5.rs:444-491). */
int orc_position_bias(const orc_model* m, int L, float* bias);

/* Embedder::embed post-processing on token ids (src/embedder.rs:22-103):
 * windows of max_len with overlap `stride`, summed; MIN_NORM filter; L2 normalise.
 * out: [n_tokens, proj_dim] normalised rows of the kept tokens, kept[n] token indices.
 * Returns number of kept tokens, or -1 on error (all filtered). */
int orc_embed_ids(const orc_model* m, const uint32_t* ids, int n_tokens, int max_len, int stride,
                  float* out, int32_t* kept, int acc64);

int orc_model_dims(const orc_model* m, orc_config* cfg);

/* ---- embedding codecs (codec_oracle.c: packops.rs, haarops.rs, rans64.rs) ---- */
uint8_t orc_compand_q4(float v);          /* compand().quantize(4) of one value */
void orc_q4_dequant_table(float table[16]); /* make_q4_dequant_table */
void orc_residual_encode(const float* emb, const float* centers, const uint32_t* assign, int N, int D,
                         uint8_t* out);
void orc_residual_decode(const uint8_t* bytes, int N, int D, const float table[16], float* out);
uint64_t orc_ladder_mismatches(const float t[15], uint32_t* first_bad);
void orc_haar_forward(float* x, int n);
void orc_haar_inverse(float* x, int n);
int orc_scale_histogram(const uint32_t* counts, int m, int log2_scale, uint16_t* freq);
long orc_embeddings_to_packed(const float* x, int rows, int cols, uint8_t* out, size_t cap);
long orc_embeddings_from_packed(const uint8_t* buf, size_t len, int cols, float* out, size_t cap_rows);

#ifdef __cplusplus
}
#endif
#endif
