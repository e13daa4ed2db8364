/*
 * t5hip.h -- C ABI of the MI355X-native quantized XTR-T5 encoder (`t5-hip` backend).
 *
 * This is the drop-in boundary for Witchcraft's `t5_encoder` module alias
 * (reference src/lib.rs:10-21).  Plain pointers and sizes only; every entry point
 * returns 0 on success and a negative T5H_ERR_* code on failure, with a
 * thread-local message from t5h_last_error().  Nothing here aborts or exits.
 *
 * Threading: a model handle is used by one thread at a time (the reference moves
 * one T5EncoderModel into the napi indexer thread and guards another with a Mutex,
 * src/napi.rs:293-304,483-551).  Handles share no mutable state; each owns its
 * device buffers and its own HIP stream, so two handles may run concurrently.
 */
#ifndef T5HIP_H
#define T5HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define T5H_OK 0
#define T5H_ERR_INVALID (-1)   /* bad argument (shape, id out of vocabulary, ...) */
#define T5H_ERR_FORMAT (-2)    /* malformed GGUF / missing or mis-shaped tensor */
#define T5H_ERR_HIP (-3)       /* HIP runtime failure */
#define T5H_ERR_NOMEM (-4)     /* device or host allocation failed */
#define T5H_ERR_NODEVICE (-5)  /* no usable gfx950 device */

typedef struct t5h_model t5h_model;

/* Model hyper-parameters.  Mirrors the fields of the reference `Config`
 * (src/quantized_t5.rs:90-115) that the encoder reads; the host parses
 * config.json into this struct (the reference does it with serde at :713-719). */
typedef struct t5h_config {
  int32_t vocab_size;                      /* Config::vocab_size */
  int32_t d_model;                         /* Config::d_model (768) */
  int32_t d_kv;                            /* Config::d_kv (64) */
  int32_t d_ff;                            /* Config::d_ff (2048) */
  int32_t num_layers;                      /* Config::num_layers (12) */
  int32_t num_heads;                       /* Config::num_heads (12) */
  int32_t relative_attention_num_buckets;  /* 32 */
  int32_t relative_attention_max_distance; /* 128 (default, :64-66) */
  float layer_norm_epsilon;                /* 1e-6 */
  int32_t feed_forward_gated;              /* 1: "gated-gelu" (NewGelu), 0: "relu" */
  int32_t proj_dim;                        /* rows of linear.weight (128, :690) */
  int32_t max_seq_len;                     /* longest sequence accepted (embedder window 2048) */
} t5h_config;

/* Message of the last failure on the calling thread ("" if none). */
const char* t5h_last_error(void);

/* Fill `cfg` with XTR-base (T5-v1.1-base) values. */
int t5h_config_xtr_base(t5h_config* cfg);

/* Load an encoder from GGUF bytes (borrowed for the duration of the call).
 * Replaces T5ModelBuilder::build_encoder + T5EncoderModel::load
 * (src/quantized_t5.rs:681-696,731-749).  Linear weights may be Q4_K, F16 or F32
 * (F16/F32 are kept as f16 on the device); the embedding table may be F32 or Q4_K.
 * hip_device < 0 selects device 0. */
int t5h_create(const void* gguf, size_t len, const t5h_config* cfg, int hip_device,
               t5h_model** out);
void t5h_destroy(t5h_model* model);

/* Encode B packed sequences.  ids[T] holds the concatenated token ids of the
 * sequences, cu_seqlens[B+1] their offsets (cu_seqlens[0] = 0, T = cu_seqlens[B]).
 * Each sequence is encoded exactly as the reference encodes a [1, L] input
 * (T5EncoderModel::forward, src/quantized_t5.rs:698-701): no token of one
 * sequence attends to another.  out[T, proj_dim] receives the UN-normalised
 * projections (host memory); out_norm[T] (optional, may be NULL) their L2 norms.
 * Synchronous: returns after the results are in host memory, like the
 * `.to_device(&Device::Cpu)` at src/embedder.rs:41. */
int t5h_encode(t5h_model* model, const uint32_t* ids, const int32_t* cu_seqlens, int32_t B,
               float* out, float* out_norm);

/* As t5h_encode, but rows are L2-normalised (src/embedder.rs:7-9,94); norms are
 * still reported pre-normalisation in out_norm when non-NULL. */
int t5h_encode_normalized(t5h_model* model, const uint32_t* ids, const int32_t* cu_seqlens,
                          int32_t B, float* out, float* out_norm);

/* Device-resident variant for callers that keep ids and outputs in HBM.
 * d_ids / d_out / d_norm are device pointers; cu_seqlens is a HOST array.
 * Enqueued on the model's stream; returns without waiting (t5h_synchronize).
 * Token ids >= vocab_size produce zero embeddings and raise the device error flag
 * reported by t5h_synchronize. */
int t5h_encode_device(t5h_model* model, const uint32_t* d_ids, const int32_t* cu_seqlens,
                      int32_t B, float* d_out, float* d_norm);

/* No counterpart in the reference.  For callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): t5h_encode_device with the
 * same arguments, ordering and results (bit-identical), but it allocates nothing -- no
 * device, pinned or event allocation, per call or on first use.  Its workspace is a fixed
 * array of T5H_NOALLOC_SCRATCH_BYTES per GPU, mapped by t5h_create and held by every GPU the
 * library runs on until the process ends (about 2,000 tokens of XTR-base per call).  Inputs
 * whose workspace does not fit return T5H_ERR_INVALID before anything is enqueued.  All calls
 * on one GPU share that GPU's array, so the library orders them: each call's stream first waits
 * for a per-GPU event (created by t5h_create) that the previous no-alloc call on that GPU
 * recorded after its launches, whichever handle or thread made it.  A call enqueued while the
 * handle's stream is being captured into a graph is not ordered that way (its launches run at
 * replay time): replays of such graphs must not overlap each other or other no-alloc calls on
 * the same GPU.  No per-kernel event timing is recorded for these calls. */
#define T5H_NOALLOC_SCRATCH_BYTES (40u << 20)
int t5h_encode_device_noalloc(t5h_model* model, const uint32_t* d_ids, const int32_t* cu_seqlens,
                              int32_t B, float* d_out, float* d_norm);
int t5h_synchronize(t5h_model* model);
/* The model's hipStream_t (as void*), for event timing by the caller. */
void* t5h_stream(t5h_model* model);

/* Embedder::embed after tokenisation (src/embedder.rs:22-103): windows of
 * max_len tokens overlapping by `stride`, summed; tokens whose pre-normalisation
 * norm is < 1.0 dropped; rows L2-normalised.  out[n_tokens, proj_dim] receives the
 * kept rows, kept_index[n_tokens] their token positions; *n_kept their count.
 * Returns T5H_ERR_INVALID if every token is filtered (the reference bails). */
int t5h_embed_ids(t5h_model* model, const uint32_t* ids, int32_t n_tokens, int32_t max_len,
                  int32_t stride, float* out, int32_t* kept_index, int32_t* n_kept);
/* Embedder::embed for n_docs documents at once (src/embedder.rs:22-103, called per document
 * by Gatherer::next, src/lib.rs:930-934).  Document d is ids[doc_offsets[d] .. doc_offsets[d+1])
 * (doc_offsets[0] = 0, no empty document).  Every window of every document is encoded as one
 * packed batch; window sums, the norm filter, compaction and normalisation run on the device.
 * Document d's kept rows are out[kept_offsets[d] .. kept_offsets[d+1]) (out has room for
 * doc_offsets[n_docs] rows of proj_dim), kept_index[] their positions within the document,
 * kept_offsets[n_docs + 1].  If a document keeps no token, returns T5H_ERR_INVALID naming it
 * (the reference's embed bails, :89-91); the outputs of all documents are still written.
 * Device buffers are grown on demand per handle and reused, not allocated per call. */
int t5h_embed_batch(t5h_model* model, const uint32_t* ids, const int32_t* doc_offsets, int32_t n_docs,
                    int32_t max_len, int32_t stride, float* out, int32_t* kept_index,
                    int32_t* kept_offsets);

/* ---- numerics of the FFN and the projection ----
 * T5H_NUMERICS_DEFAULT: the `t5-quantized` numerics -- Q4_K weights dequantized exactly,
 *   activations and weights rounded to f16 for the MFMAs (f32 accumulation), tanh gelu.
 * T5H_NUMERICS_HYBRID: the `hybrid-dequant` feature's (src/quantized_t5.rs:18-21,233-244) --
 *   wi_0 / wi_1 and the final projection take f32 T5LayerNorm outputs quantized to Q8_K
 *   (candle BlockQ8K::from_float) times Q4_K weights by GGML's integer vec_dot
 *   (src/fused_matmul.rs:27-59 QTiledOp, :138-177 fused gated gelu with the Pade tanh of
 *   :128-133); the other linears keep the default numerics.  Needs Q4_K wi_0, wi_1 and
 *   linear.weight and a gated FFN.  Default: T5H_NUMERICS_DEFAULT.
 * T5H_NUMERICS_HYBRID_BF16: the `hybrid-dequant` + `fbgemm` build, which `make` selects on
 *   x86 Linux without nvcc (Makefile:26-30) -- T5H_NUMERICS_HYBRID, with the q/k/v/o/wo weights
 *   (dequantized to f32 at load, src/quantized_t5.rs:57-62,218-219) truncated to bf16
 *   (bits & 0xffff0000, fbgemm-rs/src/bf16.rs:21-25) before the f16 MFMAs: exact for |w| >= 2^-17,
 *   the f16 subnormal grid below.  Q4_K dense weights are expanded on the device on the first
 *   switch to this mode (2 bytes per weight, kept by the handle). */
#define T5H_NUMERICS_DEFAULT 0
#define T5H_NUMERICS_HYBRID 1
#define T5H_NUMERICS_HYBRID_BF16 2
int t5h_set_numerics(t5h_model* model, int32_t mode);

/* ---- offline weight quantization (host only, no device needed) ---- */

/* f32 values -> GGML Q4_K super-blocks (144 bytes per 256 values): the quantize tool's
 * QTensor::quantize(_, Q4K) (tools/quantize-tool/src/main.rs:12-24), i.e. candle's
 * BlockQ4K::from_float with GGML's make_qkx1_quants scale/min search.  n_values % 256 == 0;
 * out receives n_values / 256 * 144 bytes.  threads <= 0: up to 16 host threads. */
int t5h_quantize_q4k(const float* x, int64_t n_values, uint8_t* out, int32_t threads);

/* ---- test hooks (teacher-forced parity checks) ---- */

/* BlockQ8K::from_float on the device (src/fused_matmul.rs:36-41): x[rows][cols] f32 (cols % 256
 * == 0, <= 1024) -> rows * cols / 256 blocks of 292 bytes {f32 d, i8 qs[256], i16 bsums[16]}.
 * Host buffers. */
int t5h_q8k_quantize(int32_t hip_device, const float* x, int32_t rows, int32_t cols, uint8_t* blocks);
/* out[T][N] = vec_dot(w row n, x8 row t) for Q4_K rows w[N][K] and Q8_K rows x8[T][K]
 * (BlockQ4K::vec_dot, src/fused_matmul.rs:55), through the same matrix-core kernel as the hybrid
 * numerics of the forward (N % 64 == 0, K % 256 == 0, K <= 1024).  Host buffers. */
int t5h_q4k_q8k_matmul(int32_t hip_device, const uint8_t* w, int32_t N, const uint8_t* x8, int32_t T,
                       int32_t K, float* out);

/* The attention work list the encoder uploads for a batch (cu_seqlens[batch + 1]) of `heads`
 * heads: items of 4 int32 (sequence start, length, first query, head), one per workgroup of
 * 64 queries (sequences of at most 128 tokens) or 128 queries (longer ones) of one (sequence,
 * head), length 0 for the empty slots that pad the 8 per-XCD lists
 * (item i runs on XCD i % 8).  *n_items receives the item count; T5H_ERR_INVALID when it
 * exceeds cap.  Host only, no device needed. */
int t5h_attention_work(const int32_t* cu_seqlens, int32_t batch, int32_t heads, int32_t* items, int32_t cap,
                       int32_t* n_items);

/* Q4_K -> f32, bit-exact with candle BlockQ4K::to_float (reached from
 * src/quantized_t5.rs:44).  blocks/out are HOST buffers. */
int t5h_q4k_dequant_f32(const void* blocks, size_t nblk, float* out, int hip_device);

/* ---- Query-side scoring, next to the encoder ----
 * C[M][N] = A[M][D] . B[N][D]^T in f32: fast_ops::matmul_t (src/fast_ops.rs:98-116) and
 * PackedRight::matmul (:65-95), as used for query x centroid / residual scores
 * (src/lib.rs:637,735,759,1646).  bf16_b != 0 truncates B to bf16 first, as the fbgemm build
 * packs it (fbgemm-rs/src/bf16.rs:21-31); A stays f32 and sums are f32.  Any M, N, D >= 0
 * (M == 0 or N == 0: nothing to do).  Host buffers, synchronous, on HIP device hip_device. */
int t5h_matmul_t(int32_t hip_device, const float* a, int32_t M, const float* b, int32_t N, int32_t D,
                 int32_t bf16_b, float* c);
/* matmul_argmax_batched (src/lib.rs:187-208, k-means assignment at :235,1330):
 * out[i] = argmax_j A[i] . B[j], the first (smallest) j on ties as candle's argmax (0 when no
 * score exceeds -inf).  N > 0.  Same buffers and numerics as t5h_matmul_t, no [M][N]
 * intermediate. */
int t5h_matmul_argmax(int32_t hip_device, const float* a, int32_t M, const float* b, int32_t N,
                      int32_t D, int32_t bf16_b, uint32_t* out);
/* The same on device buffers of the current device, enqueued on `stream` (a hipStream_t;
 * NULL = the default stream); they return without waiting. */
int t5h_matmul_t_device(const float* d_a, int32_t M, const float* d_b, int32_t N, int32_t D,
                        int32_t bf16_b, float* d_c, void* stream);
int t5h_matmul_argmax_device(const float* d_a, int32_t M, const float* d_b, int32_t N, int32_t D,
                             int32_t bf16_b, uint32_t* d_out, void* stream);

/* ---- The residual codec of the index, next to the encoder (src/packops.rs) ----
 * A residual (token embedding minus its k-means centre) is stored as 4-bit codes,
 * compand().quantize(4).to_q4_bytes() (packops.rs:136-142,156-162,440-462): two codes per
 * byte, value 2j of a row in the high nibble of byte j.  Search decodes them through
 * make_q4_dequant_table (packops.rs:14-25) in from_companded_q4_bytes (:491-513). */

/* make_q4_dequant_table (src/packops.rs:14-25): the f32 value of each 4-bit code. */
int t5h_q4_dequant_table(float table[16]);
/* The 15 decision thresholds of compand().quantize(4): code(x) = number of thresholds <= x
 * (NaN -> 0).  No counterpart in the reference; exposed so callers and tests can check the
 * exact encoding the GPU applies. */
int t5h_q4_compand_thresholds(float thresholds[15]);
/* Index build (src/lib.rs:1375-1376): codes[i] = to_q4_bytes(compand(emb[i] -
 * centers[assign[i]]).quantize(4)); emb[N][D], centers[K][D], codes[N][D/2], D % 8 == 0.
 * Host buffers, synchronous.  An assignment >= K is an error. */
int t5h_residual_encode(int32_t hip_device, const float* emb, int32_t N, const float* centers, int32_t K,
                        const uint32_t* assign, int32_t D, uint8_t* codes);
/* Device-buffer form on `stream`; rows whose assignment is >= K get zero bytes and set *d_bad
 * (a device word the caller zeroes). */
int t5h_residual_encode_device(const float* d_emb, int32_t N, const float* d_centers, int32_t K,
                               const uint32_t* d_assign, int32_t D, uint8_t* d_codes, uint32_t* d_bad, void* stream);
/* from_companded_q4_bytes (src/packops.rs:491-513): codes[N][D/2] -> out[N][D] f32, D even. */
int t5h_residual_decode(int32_t hip_device, const uint8_t* codes, int32_t N, int32_t D, float* out);
int t5h_residual_decode_device(const uint8_t* d_codes, int32_t N, int32_t D, float* d_out, void* stream);
/* Search-time residual scores without materialising the residuals (src/lib.rs:676-680,734-735):
 * C[M][N] = A[M][D] . from_companded_q4_bytes(codes)[N][D]^T, D % 4 == 0, within the f32
 * summation bound D * 2^-23 * sum |a||r| of the f32 product (query-sized A against many rows
 * runs on bf16 MFMAs with both operands split in three parts; non-finite queries on f32). */
int t5h_matmul_t_q4(int32_t hip_device, const float* a, int32_t M, const uint8_t* codes, int32_t N, int32_t D,
                    float* c);
int t5h_matmul_t_q4_device(const float* d_a, int32_t M, const uint8_t* d_codes, int32_t N, int32_t D, float* d_c,
                           void* stream);

/* ---- Packed chunk embeddings (src/packops.rs:172-438) ----
 * embeddings_to_packed / embeddings_from_packed over a batch of B matrices of `cols` columns
 * (1..255; Witchcraft stores each chunk's [L', 128] token embeddings this way, src/lib.rs:1091,
 * decoded at :712,1178,1296).  Per matrix: u32 rows, then per window of <= 1024 rows the column
 * permutation, the rANS frequency table and one rANS64 stream (2-D Haar coefficients, columns
 * sorted by sum, quantised to round(29 x / max|x|<1)).  Bytes equal the reference's.
 * Host buffers, synchronous; gpu_ms (may be NULL) receives the device time of the call's
 * kernels.  Errors: T5H_ERR_INVALID where the reference panics or asserts (NaN column sum,
 * > 4096 distinct symbols, stream overflow) or buffers are too small; T5H_ERR_FORMAT for a
 * malformed packed buffer (truncated, leftover bytes, corrupt stream, column index >= cols). */

/* x: the matrices' rows back to back, [row_offsets[B]][cols] f32; row_offsets[B+1] with
 * row_offsets[0] = 0.  out (out_cap bytes) receives the packed matrices back to back;
 * out_offsets[B+1] their byte offsets (out_offsets[B] = total, also set when out_cap is too
 * small, so a caller can size the buffer and call again). */
int t5h_embeddings_to_packed(int32_t hip_device, const float* x, const int32_t* row_offsets, int32_t B,
                             int32_t cols, uint8_t* out, size_t out_cap, size_t* out_offsets, double* gpu_ms);
/* buf: B packed matrices back to back, buf_offsets[B+1] their byte offsets.  out receives
 * the decoded rows (each L2-normalised, as the reference returns them) back to back,
 * out_cap_rows rows of room; row_offsets[B+1] the row offset of each matrix. */
int t5h_embeddings_from_packed(int32_t hip_device, const uint8_t* buf, const size_t* buf_offsets, int32_t B,
                               int32_t cols, float* out, size_t out_cap_rows, int32_t* row_offsets,
                               double* gpu_ms);

/* One T5Block (src/quantized_t5.rs:598-627) on packed sequences: x_in/x_out are
 * host [T, d_model] f32. */
int t5h_layer_forward(t5h_model* model, int32_t layer, const float* x_in,
                      const int32_t* cu_seqlens, int32_t B, float* x_out);

/* T5DenseGatedActDense::forward alone (src/quantized_t5.rs:231-252) on host x[T, d_model]:
 * y = wo(gelu(x wi_0^T) * (x wi_1^T)).  Both modes run gate and up as one dequant-GEMM whose
 * epilogue applies gelu(gate) * up (the [T, d_ff] pre-activations never reach memory), then wo.
 * mode 0: the production kernels (the small-token GEMV kernels for T <= 64, the batched
 * MFMA GEMM above); mode 1: the batched GEMM at every T. */
int t5h_ffn_block(t5h_model* model, int32_t layer, const float* x, int32_t T, float* y,
                  int32_t mode);

/* Per-kernel timing with HIP events on the model stream (0 = off, 1 = on).
 * t5h_kernel_stats fills up to `cap` records and returns the number of kernel
 * classes; names are static strings. */
typedef struct t5h_kernel_stat {
  const char* name;
  int64_t launches;
  double total_ms;
  double flops;  /* algorithmic FLOPs summed over launches (true tokens only) */
  double bytes;  /* algorithmic HBM bytes summed over launches */
} t5h_kernel_stat;
int t5h_set_profiling(t5h_model* model, int32_t on);
int t5h_kernel_stats(t5h_model* model, t5h_kernel_stat* stats, int32_t cap);
/* Measurement hook (no reference counterpart): relaunches the last launch of kernel class
 * `kind` (the index of its t5h_kernel_stats record) from the most recent forward run with
 * profiling on, `reps` times back to back between two HIP events on the model's stream, and
 * returns the average duration in microseconds.  Per-kernel events inside a forward add the
 * dispatch and completion latency of every launch; back-to-back relaunches do not, so these
 * averages are comparable with profiler per-dispatch durations.  The relaunches overwrite the
 * workspace (a residual class adds into the residual stream again); the next forward
 * recomputes it.  They never touch the profiled call's own buffers (d_ids, d_out, d_norm): the
 * records use the handle's workspace copies of those instead, so the caller may free them.  A
 * workspace that grows drops every record (T5H_ERR_INVALID until the next profiled forward). */
int t5h_replay_kernel(t5h_model* model, int32_t kind, int32_t reps, double* avg_us);

#ifdef __cplusplus
}
#endif
#endif
