// t5hip_api.cpp -- the C ABI of include/t5hip.h: model load (GGUF -> HBM), workspace,
// and the per-call launch sequence of the encoder on one HIP stream.
//
// Reference flow being replaced (src/quantized_t5.rs):
//   T5EncoderModel::load :681-696   -> t5h_create
//   T5Stack::forward     :654-670   -> enqueue_forward (embed, 12 blocks, final norm)
//   T5EncoderModel::forward :698-701 -> + projection 768->128
#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include <algorithm>
#include <memory>
#include <mutex>
#include <stdlib.h>
#include <string>
#include <vector>

#include "../../include/t5hip.h"
#include "common.hpp"
#include "gguf.hpp"

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}
}  // namespace

// The workspace of t5h_encode_device_noalloc: one fixed array per GPU the library runs on,
// held until the process ends.  In host code `scratch` names only a host-side stand-in for
// the symbol; each device's own address comes from hipGetSymbolAddress (scratch_init) and
// is the only address that reaches kernels or copies.
static __device__ __align__(256) uint8_t scratch[T5H_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};
// Per device: the event recorded after the last no-alloc call's launches (on that call's
// stream), which the next no-alloc call's stream waits for before it touches the array, so
// calls from different handles and threads run one after another on the GPU.  g_noalloc_mu[dev]
// makes wait + enqueue + record one step for concurrent host threads.  Created with the
// scratch mapping (at t5h_create), so the entry point itself creates nothing.
hipEvent_t g_noalloc_ev[kMaxDevices] = {};
std::mutex g_noalloc_mu[kMaxDevices];

// Maps the scratch array on device `dev` (which must be current) once per process, and creates
// that device's ordering event.
int scratch_init(int dev, void** out) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  *out = nullptr;
  if (dev < 0 || dev >= kMaxDevices) return fail(T5H_ERR_NODEVICE, "device index beyond the scratch table");
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(T5H_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_dev[dev] = p;
  }
  if (!g_noalloc_ev[dev]) {
    hipEvent_t ev = nullptr;
    const hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) return fail(T5H_ERR_HIP, std::string("hipEventCreate(no-alloc order): ") + hipGetErrorString(e));
    g_noalloc_ev[dev] = ev;
  }
  *out = g_scratch_dev[dev];
  return T5H_OK;
}
}  // namespace

namespace t5k {
thread_local LaunchTiming tl_launch_timing;
}

namespace t5h_detail {
// The same thread-local message for the entry points defined in other files (codec.cpp).
int fail(int code, const std::string& msg) { return ::fail(code, msg); }
}  // namespace t5h_detail

namespace {

#define HIP_OK(expr)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess)                                                              \
      return fail(T5H_ERR_HIP, std::string(#expr ": ") + hipGetErrorString(e_));       \
  } while (0)

struct Linear {
  int N = 0, K = 0;
  int fmt = WF_Q4K;
  size_t off = 0;         // byte offset in the weight arena
  const void* w = nullptr;  // device pointer (set after upload)
  // F32/F16 dense weights also keep f16(bf16_trunc(w)) [N][K] for T5H_NUMERICS_HYBRID_BF16
  // (the source values are only borrowed during t5h_create): arena offset, device pointer.
  bool has_bf = false;
  size_t bf_off = 0;
  const void* bf = nullptr;
  size_t bytes() const { return fmt == WF_Q4K ? (size_t)N * K / QK_K * Q4K_BYTES : (size_t)N * K * 2; }
};

struct Layer {
  Linear qkv;           // fused [3*inner][D] when q, k, v share a format
  Linear q, k, v;       // used when they do not
  bool fused_qkv = true;
  Linear o, wi0, wi1, wo;
  size_t ln0_off = 0, ln1_off = 0;
  const float *ln0 = nullptr, *ln1 = nullptr;
};

struct PendingTiming {
  int kind;
  hipEvent_t a, b;
  double flops, bytes;
};

enum KernelKind {
  K_EMBED, K_RMSNORM, K_GEMM_QKV, K_ATTN, K_GEMM_O, K_GEMM_GATE_UP, K_GEMM_WO, K_GEMM_PROJ,
  K_ROWNORM, K_FFN, K_COUNT
};
const char* const kKernelNames[K_COUNT] = {
    "embed_gather", "rmsnorm", "gemm_qkv", "attention", "gemm_o", "gemm_ffn_gate_up",
    "gemm_ffn_wo", "gemm_proj", "rownorm", "ffn_fused"};

// Per-forward device buffers, rows padded to tpad = roundup(T, 512) + 128.
struct Workspace {
  int tpad = 0;
  float* x = nullptr;      // residual stream f32 [tpad][d_model]
  _Float16* xn = nullptr;  // GEMM operand f16 [tpad][max(d_model, inner)], operand order
  // Norm records of the folded T5LayerNorm (GemmArgs::rec), [tpad][16] f32 each on the batched
  // path and [tpad][64] on the GEMV path: rec0 for the norm before attention and the final
  // one, rec1 for the norm before the FFN.
  float* rec0 = nullptr;
  float* rec1 = nullptr;
  _Float16* qkvb = nullptr;  // q/k/v f16 head-major [3][H][tpad][d_kv]
  _Float16* ao = nullptr;    // attention output f16 [tpad][inner], operand order
  _Float16* hb = nullptr;    // gated hidden state f16 [tpad][d_ff], operand order
  float* out = nullptr;      // projections f32 [tpad][proj_dim]
  float* norm = nullptr;     // their norms f32 [tpad]
  uint32_t* ids = nullptr;   // token ids [tpad]
  int4* work = nullptr;      // attention work list [cap_work]
};

// The arguments of the last launch of each kernel class in a profiled forward, so that
// t5h_replay_kernel can relaunch it back to back between two events.
struct ReplayRec {
  enum Type { NONE, GEMM, GEMV, ATTN, EMBED, ROWNORM, RMSNORM, HYBRID, FFN } type = NONE;
  int epi = 0, wfmt = 0, n = 0;
  GemmArgs ga{};
  t5k::GemmPlan plan{};
  AttnArgs aa{};
  // embed / rownorm / rmsnorm
  const uint32_t* ids = nullptr;
  const void* table = nullptr;
  int fmt = 0, vocab = 0, D = 0, P = 0, normalize = 0, rec_stride = 16;
  float* x = nullptr;
  float* y = nullptr;
  float* norm = nullptr;
  const float* gamma = nullptr;
  float eps = 0.f;
  _Float16* xn = nullptr;
  float* rec = nullptr;
  // hybrid linear (Q8_K quantize into the matrix-core operands + Q4_K x Q8_K GEMM): x, gamma,
  // eps, n (tokens), D for the quantizer; ga / plan for the GEMM (epi: EPI_GATED or EPI_F32)
  float* hd8 = nullptr;
  _Float16* hbs = nullptr;
  // one-launch FFN (wfmt: Wo's format)
  t5k::FfnArgs fa{};
};

struct StagingSlot {
  void* host = nullptr;  // pinned
  size_t cap = 0;
  hipEvent_t done = nullptr;
  bool used = false;
};

// A further execution lane of a handle: its own stream, workspace, attention work-list cache and
// staging slots.  enqueue_forward runs a part of a large batch on it (swap_lane puts these
// fields in place of the handle's own for the duration of that part).
struct ExecLane {
  hipStream_t stream = nullptr;
  void* ws = nullptr;
  size_t ws_bytes = 0;
  int cap_tokens = 0, cap_seqs = 0, cap_work = 0;
  Workspace w;
  std::vector<int> order;
  std::vector<int32_t> last_cu;
  int last_B = -1, last_nwork = 0;
  double attn_flops = 0;
  StagingSlot slots[4];
  int next_slot = 0;
};

}  // namespace

// One (sequence, head) of the attention work list: its query tiles go to XCD `xcd`, slots
// slot0, slot0 + 1, ... of that XCD's list.
struct AttnGroup {
  int start, len, head, xcd, slot0;
};

struct t5h_model {
  t5h_config cfg{};
  int device = 0;
  hipStream_t stream = nullptr;
  int inner = 0;
  int cus = 256;          // compute units of the device
  int gemm_mw_override = 0;  // T5H_GEMM_MW / T5H_GEMM_BN tuning knobs (0 = heuristic)
  bool batched_only = false;  // route every linear through the batched GEMM (t5h_ffn_block mode 1)
  int gemm_bn_override = 0;
  int gemm_mb_override = 0;  // T5H_GEMM_MB: 3 / 4 row blocks per math wave in full tiles (0 = choose)
  int gemm_tail_override = -1;  // T5H_GEMM_TAIL: -1 = choose, 0 = full tiles only, 1 / 2 = thin tail, 3 / 4 = all thin
  bool fold_norm_off = false;   // T5H_FOLD_NORM=0: standalone RMSNorm launches on the batched path
  int ffn_chunk = 0;            // T5H_FFN_CHUNK=<tokens, multiple of 512>: FFN in token chunks
  bool gated_mw8 = false;       // T5H_GATED_MW8=1: gated FFN on 8 math waves of 32 tokens
  // T5H_FFN_FUSED=<tokens>: batches (lane parts) of at least that many tokens run the gated FFN
  // as one launch (k_ffn.hip), bit-identical to the two launches and measured slower; 0 = off.
  int ffn_fused_min = 0;
  int numerics = T5H_NUMERICS_DEFAULT;  // t5h_set_numerics

  // ---- weights (one device arena) ----
  void* arena = nullptr;
  size_t arena_bytes = 0;
  const void* emb = nullptr;
  int emb_fmt = EMB_F32;
  const float* rel_lut = nullptr;  // [H][2*lutw+1], bias of distance j - i at lutw + j - i
  int lutw = 0;
  std::vector<int> order;  // host scratch: sequence order of the attention work list
  std::vector<int32_t> last_cu;  // cu_seqlens of the batch whose cu / work list are on the device
  int last_B = -1, last_nwork = 0;
  double attn_flops = 0;   // QK^T + PV flops of one attention launch on the current batch, true tokens
  const float* final_ln = nullptr;
  std::vector<Layer> layers;
  // The layers as T5H_NUMERICS_HYBRID_BF16 runs them: q/k/v/o/wo replaced by their f16 copies of
  // the bf16-truncated weights (from the arena, or expanded from Q4_K into bfw), built on the
  // first switch to that mode.
  std::vector<Layer> layers_bf;
  void* bfw = nullptr;
  Linear proj;

  // ---- workspace ----
  void* ws = nullptr;
  size_t ws_bytes = 0;
  int cap_tokens = 0, cap_seqs = 0, cap_work = 0;
  // The buffers every launch of a forward reads and writes: carved from `ws`, or from the
  // library's fixed per-device array for t5h_encode_device_noalloc (swapped in for that call).
  Workspace w;
  // Error flags in mapped pinned host memory, written by kernels through err_flag (its device
  // address) and read by the host after the stream is synchronised: word 0 out-of-vocabulary
  // ids (embed kernel), word 1 a non-finite output row (row-norm kernel).
  unsigned* err_host = nullptr;
  unsigned* err_flag = nullptr;
  void* scratch = nullptr;  // this device's address of the no-alloc scratch array

  // ---- embedder post-processing (t5h_embed_batch), grown on demand ----
  void* ew = nullptr;
  size_t ew_bytes = 0;

  // ---- host staging ----
  StagingSlot slots[4];
  int next_slot = 0;
  void* io = nullptr;  // pinned buffer for synchronous calls
  size_t io_cap = 0;

  // ---- profiling ----
  bool prof = false;
  std::vector<PendingTiming> pending;
  std::vector<hipEvent_t> event_pool;
  t5h_kernel_stat stats[K_COUNT]{};
  ReplayRec replay[K_COUNT];

  // ---- further lanes for large batches (enqueue_forward) ----
  static constexpr int MAX_LANES = 4;
  bool split_off = false;  // T5H_SPLIT=0: one lane for every batch
  int split_min = 0;       // T5H_SPLIT=<tokens> (> 1): lanes from that many tokens (0: SPLIT_MIN_TOKENS)
  int lanes = 2;           // T5H_LANES: lanes of a large batch (2..MAX_LANES)
  ExecLane extra[MAX_LANES - 1];
  hipEvent_t ev_fork = nullptr, ev_join[MAX_LANES - 1] = {};

  ~t5h_model() {
    for (auto& l : extra) {
      if (l.stream) {
        (void)hipStreamSynchronize(l.stream);
        (void)hipStreamDestroy(l.stream);
      }
      for (auto& s : l.slots) {
        if (s.host) (void)hipHostFree(s.host);
        if (s.done) (void)hipEventDestroy(s.done);
      }
      if (l.ws) (void)hipFree(l.ws);
    }
    if (ev_fork) (void)hipEventDestroy(ev_fork);
    for (auto e : ev_join)
      if (e) (void)hipEventDestroy(e);
    if (stream) (void)hipStreamSynchronize(stream);
    for (auto& s : slots) {
      if (s.host) (void)hipHostFree(s.host);
      if (s.done) (void)hipEventDestroy(s.done);
    }
    if (io) (void)hipHostFree(io);
    if (err_host) (void)hipHostFree(err_host);
    for (auto& p : pending) {
      (void)hipEventDestroy(p.a);
      (void)hipEventDestroy(p.b);
    }
    for (auto e : event_pool) (void)hipEventDestroy(e);
    if (ws) (void)hipFree(ws);
    if (ew) (void)hipFree(ew);
    if (bfw) (void)hipFree(bfw);
    if (arena) (void)hipFree(arena);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

namespace {

// ---------------------------------------------------------------------------------
// Relative-position buckets (src/quantized_t5.rs:444-483).  Rust's f32::log(x, base) is
// ln(x)/ln(base) on the platform logf; the table is built once on the host with the
// same arithmetic and indexed on the device by the signed distance j - i.
uint32_t rel_bucket(uint32_t i, uint32_t j, uint32_t nb_total, uint32_t max_distance) {
  const uint32_t nb = nb_total / 2, max_exact = nb / 2;
  if (i < j) {
    if (j - i < max_exact) return j - i + nb;
    const float b = logf((float)(j - i) / (float)max_exact) /
                    logf((float)max_distance / (float)max_exact) * (float)(nb - max_exact);
    return std::min(max_exact + nb + (uint32_t)b, nb_total - 1);
  } else if (i - j < max_exact) {
    return i - j;
  } else {
    const float b = logf((float)(i - j) / (float)max_exact) /
                    logf((float)max_distance / (float)max_exact) * (float)(nb - max_exact);
    return std::min(max_exact + (uint32_t)b, nb - 1);
  }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int check_config(const t5h_config* c) {
  if (!c) return fail(T5H_ERR_INVALID, "config is NULL");
  if (c->vocab_size <= 0 || c->num_layers <= 0 || c->num_heads <= 0 || c->proj_dim <= 0 ||
      c->max_seq_len <= 0 || c->relative_attention_num_buckets < 4 ||
      c->relative_attention_max_distance <= 0)
    return fail(T5H_ERR_INVALID, "config has non-positive dimensions");
  if (c->d_kv != 64) return fail(T5H_ERR_INVALID, "d_kv must be 64 (attention kernel tile)");
  const int inner = c->num_heads * c->d_kv;
  if (c->d_model % 256 || c->d_ff % 256 || inner % 256)
    return fail(T5H_ERR_INVALID, "d_model, d_ff and num_heads*d_kv must be multiples of 256");
  if (c->proj_dim % 128) return fail(T5H_ERR_INVALID, "proj_dim must be a multiple of 128");
  if (c->max_seq_len > 65536) return fail(T5H_ERR_INVALID, "max_seq_len too large");
  return T5H_OK;
}

// Host-side weight collection before upload.
struct HostArena {
  std::vector<uint8_t> bytes;
  size_t add(const void* src, size_t n) {
    const size_t off = align256(bytes.size());
    bytes.resize(off + n);
    if (src) memcpy(bytes.data() + off, src, n);
    return off;
  }
};

// Adds a linear weight W[N][K]: Q4_K stays as raw blocks; F32/F16 become f16.
int add_linear(HostArena& ha, const t5h::GgufFile& g, const std::string& name, int N, int K,
               Linear& L) {
  const t5h::GgufTensor* t = g.find(name);
  if (!t) return fail(T5H_ERR_FORMAT, "missing tensor " + name);
  if (t->shape.size() != 2 || (int)t->rows() != N || (int)t->cols() != K)
    return fail(T5H_ERR_FORMAT, "tensor " + name + ": expected shape [" + std::to_string(N) + ", " +
                                    std::to_string(K) + "]");
  L.N = N;
  L.K = K;
  if (t->type == t5h::GGML_Q4_K) {
    L.fmt = WF_Q4K;
    L.off = ha.add(t->data, t->nbytes);
  } else {
    L.fmt = WF_F16;
    L.off = ha.add(nullptr, (size_t)N * K * 2);
    _Float16* dst = reinterpret_cast<_Float16*>(ha.bytes.data() + L.off);
    const size_t ne = (size_t)N * K;
    if (t->type == t5h::GGML_F32) {
      const float* s = reinterpret_cast<const float*>(t->data);
      for (size_t i = 0; i < ne; i++) dst[i] = (_Float16)s[i];
    } else {
      memcpy(dst, t->data, ne * 2);
    }
  }
  return T5H_OK;
}

// For an F32/F16 dense linear L (its source tensors `parts`, concatenated along N): a second
// f16 copy of the weights truncated to bf16 first (bits & 0xffff0000, fbgemm-rs/src/bf16.rs:21-25),
// which T5H_NUMERICS_HYBRID_BF16 uses in place of the round-to-nearest f16 copy.
void add_bf16_copy(HostArena& ha, const std::vector<const t5h::GgufTensor*>& parts, Linear& L) {
  if (L.fmt == WF_Q4K) return;
  L.bf_off = ha.add(nullptr, (size_t)L.N * L.K * 2);
  L.has_bf = true;
  _Float16* dst = reinterpret_cast<_Float16*>(ha.bytes.data() + L.bf_off);
  for (const t5h::GgufTensor* t : parts) {
    const size_t ne = t->rows() * t->cols();
    for (size_t i = 0; i < ne; i++) {
      const float v = t->type == t5h::GGML_F32 ? reinterpret_cast<const float*>(t->data)[i]
                                               : (float)reinterpret_cast<const _Float16*>(t->data)[i];
      uint32_t u;
      memcpy(&u, &v, 4);
      u &= 0xffff0000u;
      float tv;
      memcpy(&tv, &u, 4);
      dst[i] = (_Float16)tv;
    }
    dst += ne;
  }
}

int add_f32_vector(HostArena& ha, const t5h::GgufFile& g, const std::string& name, size_t n,
                   size_t& off) {
  const t5h::GgufTensor* t = g.find(name);
  if (!t) return fail(T5H_ERR_FORMAT, "missing tensor " + name);
  uint64_t ne = 1;
  for (auto d : t->shape) ne *= d;
  if (ne != n) return fail(T5H_ERR_FORMAT, "tensor " + name + ": expected " + std::to_string(n) + " values");
  off = ha.add(nullptr, n * 4);
  float* dst = reinterpret_cast<float*>(ha.bytes.data() + off);
  if (t->type == t5h::GGML_F32) {
    memcpy(dst, t->data, n * 4);
  } else if (t->type == t5h::GGML_F16) {
    const _Float16* s = reinterpret_cast<const _Float16*>(t->data);
    for (size_t i = 0; i < n; i++) dst[i] = (float)s[i];
  } else {
    return fail(T5H_ERR_FORMAT, "tensor " + name + ": expected F32 or F16");
  }
  return T5H_OK;
}

// Rows every workspace buffer holds for T tokens: GEMM tiles read A rows up to
// roundup(T, 512); attention reads up to T + ATTN_QT - 1.
int workspace_tpad(int T) { return (T + 511) / 512 * 512 + 128; }

// Lays the workspace of tpad rows and capW attention work items out from `base` (nullptr:
// only measure) and returns its size in bytes.
size_t carve_workspace(const t5h_model* m, int tpad, int capW, uint8_t* base, Workspace& w) {
  const t5h_config& c = m->cfg;
  size_t off = 0;
  auto take = [&](size_t n) {
    const size_t o = off;
    off = align256(off + n);
    return o;
  };
  const size_t o_x = take((size_t)tpad * c.d_model * 4);
  const size_t o_xn = take((size_t)tpad * std::max(c.d_model, m->inner) * 2);
  const size_t o_qkv = take((size_t)3 * tpad * m->inner * 2);
  const size_t o_ao = take((size_t)tpad * m->inner * 2);
  const size_t o_hb = take((size_t)tpad * c.d_ff * 2);
  const size_t o_out = take((size_t)tpad * c.proj_dim * 4);
  const size_t o_norm = take((size_t)tpad * 4);
  const size_t o_ids = take((size_t)tpad * 4);
  const size_t o_work = take((size_t)capW * sizeof(int4));
  const size_t o_rec = take((size_t)2 * tpad * NORM_REC_GEMV * 4);
  if (base) {
    w.tpad = tpad;
    w.x = (float*)(base + o_x);
    w.xn = (_Float16*)(base + o_xn);
    w.qkvb = (_Float16*)(base + o_qkv);
    w.ao = (_Float16*)(base + o_ao);
    w.hb = (_Float16*)(base + o_hb);
    w.out = (float*)(base + o_out);
    w.norm = (float*)(base + o_norm);
    w.ids = (uint32_t*)(base + o_ids);
    w.work = (int4*)(base + o_work);
    w.rec0 = (float*)(base + o_rec);
    w.rec1 = w.rec0 + (size_t)tpad * NORM_REC_GEMV;
  }
  return off;
}

int ensure_workspace(t5h_model* m, int T, int B, int nwork) {
  if (T <= m->cap_tokens && B <= m->cap_seqs && nwork <= m->cap_work) return T5H_OK;
  const int capT = std::max(T, m->cap_tokens), capB = std::max(B, m->cap_seqs);
  const int capW = std::max(nwork, m->cap_work);
  const int tpad = workspace_tpad(capT);
  Workspace w;
  const size_t off = carve_workspace(m, tpad, capW, nullptr, w);
  if (m->ws) {
    HIP_OK(hipStreamSynchronize(m->stream));
    HIP_OK(hipFree(m->ws));
    m->last_B = -1;  // the device work list is gone
    m->ws = nullptr;
    for (auto& r : m->replay) r = ReplayRec{};  // they point into the freed workspace
  }
  if (hipMalloc(&m->ws, off) != hipSuccess) {
    m->cap_tokens = m->cap_seqs = m->cap_work = 0;
    return fail(T5H_ERR_NOMEM, "workspace allocation of " + std::to_string(off) + " bytes failed");
  }
  // On the handle's own stream: hipMemset runs on the null stream, which a non-blocking stream
  // does not wait for, so the clear could land after the uploads that follow on m->stream.
  HIP_OK(hipMemsetAsync(m->ws, 0, off, m->stream));
  m->ws_bytes = off;
  carve_workspace(m, tpad, capW, (uint8_t*)m->ws, m->w);
  m->cap_tokens = tpad - 128;
  m->cap_seqs = capB;
  m->cap_work = capW;
  return T5H_OK;
}

int ensure_io(t5h_model* m, size_t bytes) {
  if (bytes <= m->io_cap) return T5H_OK;
  if (m->io) {
    HIP_OK(hipStreamSynchronize(m->stream));
    (void)hipHostFree(m->io);
    m->io = nullptr;
    m->io_cap = 0;
  }
  const size_t cap = std::max(bytes, (size_t)1 << 20);
  if (hipHostMalloc(&m->io, cap, hipHostMallocDefault) != hipSuccess)
    return fail(T5H_ERR_NOMEM, "pinned host allocation failed");
  m->io_cap = cap;
  return T5H_OK;
}

// Profiling brackets ----------------------------------------------------------------
hipEvent_t take_event(t5h_model* m) {
  if (!m->event_pool.empty()) {
    hipEvent_t e = m->event_pool.back();
    m->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  (void)hipEventCreate(&e);
  return e;
}

// One kernel class's launches in a profiled forward, timed by the kernels' own start/stop
// events (t5k::tl_launch_timing, hipExtLaunchKernelGGL): from the first launch's start to the last
// one's end, so dispatch gaps before and after are not counted and the duration is comparable
// with a profiler's per-dispatch time of the same kernel inside the forward.
struct Timed {
  t5h_model* m;
  int kind;
  double flops, bytes;
  hipEvent_t a = nullptr, b = nullptr;
  Timed(t5h_model* m_, int k, double f, double by) : m(m_), kind(k), flops(f), bytes(by) {
    if (m->prof) {
      a = take_event(m);
      b = take_event(m);
      t5k::tl_launch_timing = {a, b};
    }
  }
  ~Timed() {
    if (!a) return;
    const bool launched = t5k::tl_launch_timing.start == nullptr;  // a launch took the start event
    t5k::tl_launch_timing = {};
    if (launched) {
      m->pending.push_back({kind, a, b, flops, bytes});
    } else {
      m->event_pool.push_back(a);
      m->event_pool.push_back(b);
    }
  }
};

void resolve_timings(t5h_model* m) {
  for (auto& p : m->pending) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
      t5h_kernel_stat& s = m->stats[p.kind];
      s.launches++;
      s.total_ms += ms;
      s.flops += p.flops;
      s.bytes += p.bytes;
    }
    m->event_pool.push_back(p.a);
    m->event_pool.push_back(p.b);
  }
  m->pending.clear();
}

// Launch sequence -----------------------------------------------------------------
// Small token counts run the GEMV kernels (unless a tuning override or t5h_ffn_block mode 1
// forces the batched GEMM).
bool use_gemv(const t5h_model* m, int M) {
  return M <= t5k::GEMV_MAX_M && !m->gemm_mw_override && !m->batched_only;
}

// A T5LayerNorm folded into the batched GEMMs around it (GemmArgs::rec): a consumer passes
// rec (and rec_next, where the next producer's operand scale goes); a residual producer
// passes rec, nx (the operand buffer) and ngamma (the weight of the norm that follows).
struct NormLink {
  float* rec = nullptr;
  float* rec_next = nullptr;
  _Float16* nx = nullptr;
  const float* ngamma = nullptr;
};

// True when this forward's GEMMs fold the norms (the row fits one norm record).
// The block's first T5LayerNorm (before QKV) is folded into the GEMM that produces its input
// (the embedding gather, the previous block's wo) and into the QKV GEMM.
bool fold_attn_norm(const t5h_model* m, int T) {
  (void)T;
  const int D = m->cfg.d_model;
  return !m->fold_norm_off && D % 64 == 0 && D <= NORM_REC_MAX_D;
}

// Both hybrid modes: Q8_K x Q4_K FFN gate|up and projection (T5H_NUMERICS_HYBRID_BF16 also runs
// the dense linears on bf16-truncated weights, through layer_w).
bool hybrid_numerics(const t5h_model* m) { return m->numerics != T5H_NUMERICS_DEFAULT; }

// The weights block l runs with under the current numerics.
const Layer& layer_w(const t5h_model* m, int l) {
  return m->numerics == T5H_NUMERICS_HYBRID_BF16 ? m->layers_bf[l] : m->layers[l];
}

// The one-launch gated FFN (k_ffn.hip) for this layer and batch: batched path, default numerics,
// d_model 768, Q4_K wi_0 / wi_1 and a Q4_K or f16 wo, at least ffn_fused_min tokens.
bool use_ffn_fused(const t5h_model* m, const Layer& Ly, int T) {
  const t5h_config& c = m->cfg;
  return m->ffn_fused_min > 0 && T >= m->ffn_fused_min && m->ffn_chunk == 0 && !use_gemv(m, T) &&
         m->numerics == T5H_NUMERICS_DEFAULT && c.d_model == 768 && c.d_ff % 256 == 0 && Ly.wi0.fmt == WF_Q4K &&
         Ly.wi1.fmt == WF_Q4K && (Ly.wo.fmt == WF_Q4K || Ly.wo.fmt == WF_F16);
}

// Every norm folded.  With hybrid numerics the FFN's and the projection's Q8_K quantizer
// normalises its own f32 input, so only the attention norm is folded there.
bool fold_norm(const t5h_model* m, int T) {
  return fold_attn_norm(m, T) && m->numerics == T5H_NUMERICS_DEFAULT;
}

// Hybrid numerics (t5h_set_numerics): the FFN's gate|up and the projection quantize their f32
// input to Q8_K and take Q4_K x Q8_K integer dot products on the matrix cores.  The quantizer
// writes the integers as the int8 GEMM operand into the operand buffer `xn` (free after the QKV
// GEMM) and the block scales and bsum operand into the attention output buffer `ao` (free once
// the O GEMM has consumed it; checked to fit at t5h_set_numerics).  ln: the T5LayerNorm weight
// applied first (f32, from the residual x).
int hybrid_linear(t5h_model* m, int kind, const float* ln, const Linear& W0, const Linear* W1, int T, float* outf,
                  int ldo) {
  const t5h_config& c = m->cfg;
  const int nblk = c.d_model / QK_K;
  if (t5k::gemm_hybrid_rows(T) > m->w.tpad)  // roundup(T, 512) + 128 covers every tile height used
    return fail(T5H_ERR_INVALID, "internal: hybrid GEMM tiles exceed the workspace rows");
  float* d8 = (float*)m->w.ao;
  _Float16* bs = (_Float16*)((uint8_t*)m->w.ao + align256((size_t)m->w.tpad * nblk * 4));
  Timed t(m, kind, 2.0 * T * W0.N * W0.K * (W1 ? 2 : 1), 0);
  HIP_OK(t5k::launch_q8k_quantize(m->w.x, ln, c.layer_norm_epsilon, T, c.d_model, nullptr, m->stream,
                                  reinterpret_cast<int8_t*>(m->w.xn), d8, bs));
  GemmArgs a{};
  a.A = m->w.xn;  // the int8 operand blocks (GemmArgs::A, hybrid)
  a.W0 = W0.w;
  a.W1 = W1 ? W1->w : nullptr;
  a.M = T;
  a.N = W0.N;
  a.K = W0.K;
  a.out = W1 ? (void*)m->w.hb : (void*)outf;
  a.ldo = W1 ? W0.N : ldo;
  a.tpad = m->w.tpad;
  a.d8 = d8;
  a.bsop = bs;
  const int epi = W1 ? EPI_GATED : EPI_F32;
  const t5k::GemmPlan plan = t5k::gemm_plan_hybrid(T, W0.N * (W1 ? 2 : 1), m->cus);
  HIP_OK(t5k::launch_gemm_hybrid(epi, plan, a, m->stream));
  if (m->prof) {
    ReplayRec& r = m->replay[kind];
    r.type = ReplayRec::HYBRID;
    r.x = m->w.x;
    r.gamma = ln;
    r.eps = c.layer_norm_epsilon;
    r.n = T;
    r.D = c.d_model;
    r.xn = m->w.xn;
    r.hd8 = d8;
    r.hbs = bs;
    r.epi = epi;
    r.ga = a;
    r.plan = plan;
  }
  return T5H_OK;
}
// Floats per norm record: the GEMV kernels keep one partial sum per 16 columns.
int rec_stride(const t5h_model* m, int T) { return use_gemv(m, T) ? NORM_REC_GEMV : 16; }

// C = A . W^T (+ epilogue).  norm_w: on the GEMV path the operand is T5LayerNorm(m->w.x) with
// this weight, computed inside the kernel (A is then unused); callers pass it only when
// use_gemv() holds.  nl: folded norm (fold_norm() holds), on either path.
int gemm(t5h_model* m, int kind, int epi, const Linear& W, const Linear* W1, const _Float16* A, int lda,
         int M, void* out, int ldo, int n_off = 0, const float* norm_w = nullptr, const NormLink* nl = nullptr) {
  GemmArgs a{};
  a.A = A;
  a.lda = lda;
  a.W0 = W.w;
  a.W1 = W1 ? W1->w : nullptr;
  a.M = M;
  a.N = W.N;
  a.K = W.K;
  a.out = out;
  a.ldo = ldo;
  a.n_off = n_off;
  a.heads = m->cfg.num_heads;
  a.dkv = m->cfg.d_kv;
  a.tpad = m->w.tpad;
  a.cus = m->cus;
  const double mats = W1 ? 2.0 : 1.0;
  const double flops = 2.0 * M * W.N * W.K * mats;
  const double out_bytes = (epi == EPI_F32 || epi == EPI_RESID ? 4.0 : 2.0) * M * W.N *
                           (epi == EPI_RESID ? 2.0 : 1.0);
  const double bytes = W.bytes() * mats + 2.0 * M * W.K + out_bytes;
  Timed t(m, kind, flops, bytes);
  if (nl) {
    if (norm_w) return fail(T5H_ERR_INVALID, "internal: fused and folded norm requested together");
    a.rec = nl->rec;
    a.rec_next = nl->rec_next;
    a.nx = nl->nx;
    a.ngamma = nl->ngamma;
    a.eps = m->cfg.layer_norm_epsilon;
  }
  if (use_gemv(m, M)) {
    if (norm_w) {
      a.xf = m->w.x;
      a.gamma = norm_w;
      a.eps = m->cfg.layer_norm_epsilon;
    }
    HIP_OK(t5k::launch_gemv(epi, W.fmt, a, m->stream));
    if (m->prof) {
      ReplayRec& r = m->replay[kind];
      r.type = ReplayRec::GEMV;
      r.epi = epi;
      r.wfmt = W.fmt;
      r.ga = a;
    }
    return T5H_OK;
  }
  if (norm_w) return fail(T5H_ERR_INVALID, "internal: fused norm requested on the batched GEMM path");
  t5k::GemmPlan plan = t5k::gemm_plan(M, W.N * (W1 ? 2 : 1), m->cus, m->gemm_mw_override, m->gemm_bn_override,
                                      m->gemm_tail_override, m->gemm_mb_override);
  if (epi == EPI_GATED && m->gated_mw8 && W.fmt == WF_Q4K && W.N % 64 == 0) {
    plan.mw = 8;  // 256-token tiles of 8 math waves x 32 tokens, 128 weight rows
    plan.mb = 2;
    plan.bn = 128;
    plan.m_main = M;
    plan.tail_mb = 0;
  }
  HIP_OK(t5k::launch_gemm(epi, W.fmt, plan, a, m->stream));
  if (m->prof) {
    ReplayRec& r = m->replay[kind];
    r.type = ReplayRec::GEMM;
    r.epi = epi;
    r.wfmt = W.fmt;
    r.ga = a;
    r.plan = plan;
  }
  return T5H_OK;
}

// Attention work plan.  One workgroup per (sequence, head, attn_item_queries(L) queries: 64 up
// to ATTN_SMALL_L tokens, ATTN_QT above); workgroup b runs on
// XCD b % 8 (workgroups are dealt round-robin), so the list is laid out as 8 interleaved
// per-XCD lists.  All query tiles of one (sequence, head) go to one XCD, one after another, so
// that XCD's L2 holds the group's keys and values while its query tiles stream them (2048
// tokens: 512 KB per group, read by 16 workgroups).  Groups are taken longest sequence first
// and each goes to the XCD with the least work (query tiles x key tiles) among those whose
// list stays within ceil(items / 8) + the longest group, which bounds the padding: the lists
// are padded to the longest one with empty items (length 0), which exit at once.
int attn_tiles(int L) { return attn_items(L); }

// Upper bound of the work list length (items incl. padding) for T tokens in B sequences of at
// most max_len tokens.
int attn_work_cap(int heads, int max_seq_len, int T, int B) {
  // items of at least 64 queries: ceil(L / 64) <= L / 64 + 1 per sequence; at most 2 for
  // L <= ATTN_SMALL_L, ceil(L / ATTN_QT) above
  return heads * ((T + 63) / 64 + B) + 8 * (std::max(2, attn_tiles(max_seq_len)) + 1);
}
int attn_work_cap(const t5h_model* m, int T, int B) { return attn_work_cap(m->cfg.num_heads, m->cfg.max_seq_len, T, B); }

// Calls emit(group) for every (sequence, head) in `order`; returns the slots per XCD.
template <class Emit>
int plan_attention(int H, const int32_t* cu, const std::vector<int>& order, int (&xlen)[8], Emit&& emit) {
  long long items = 0, load[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int maxq = 0;
  for (int b : order) {
    items += (long long)H * attn_tiles(cu[b + 1] - cu[b]);
    maxq = std::max(maxq, attn_tiles(cu[b + 1] - cu[b]));
  }
  const long long cap = (items + 7) / 8 + maxq;
  for (int x = 0; x < 8; x++) xlen[x] = 0;
  for (int b : order) {
    const int L = cu[b + 1] - cu[b], nq = attn_tiles(L);
    if (!nq) continue;
    for (int h = 0; h < H; h++) {
      int best = -1;
      for (int x = 0; x < 8; x++)
        if (xlen[x] + nq <= cap && (best < 0 || load[x] < load[best])) best = x;
      emit(AttnGroup{cu[b], L, h, best, xlen[best]});
      xlen[best] += nq;
      load[best] += (long long)nq * nq;
    }
  }
  int slots = 0;
  for (int x = 0; x < 8; x++) slots = std::max(slots, xlen[x]);
  return slots;
}

// Longest sequences first (order is host scratch, reused across calls).
void order_by_length(std::vector<int>& order, const int32_t* cu, int B) {
  order.resize(B);
  for (int b = 0; b < B; b++) order[b] = b;
  std::stable_sort(order.begin(), order.end(), [cu](int x, int y) { return cu[x + 1] - cu[x] > cu[y + 1] - cu[y]; });
}

// The work list upload_batch writes: item (slot q of XCD x) at index 8 q + x.
int write_attention_work(int H, const int32_t* cu, const std::vector<int>& order, int4* out, size_t cap) {
  int xlen[8];
  const int slots = plan_attention(H, cu, order, xlen, [](const AttnGroup&) {});
  if ((size_t)8 * slots > cap) return -1;
  plan_attention(H, cu, order, xlen, [&](const AttnGroup& g) {
    for (int q = 0; q < attn_tiles(g.len); q++)
      out[(size_t)(g.slot0 + q) * 8 + g.xcd] = make_int4(g.start, g.len, q * attn_item_queries(g.len), g.head);
  });
  for (int x = 0; x < 8; x++)
    for (int q = xlen[x]; q < slots; q++) out[(size_t)q * 8 + x] = make_int4(0, 0, 0, 0);
  return 8 * slots;
}

// Uploads the attention work list through a pinned staging slot: one (start, length, first
// query, head) item per workgroup, so the kernel needs no further lookup.
int upload_batch(t5h_model* m, const int32_t* cu, int B, int& nwork) {
  // The same batch layout as the previous upload (e.g. a stream of equal-length queries):
  // the device copy of the work list is still current.
  if (B == m->last_B && std::equal(cu, cu + B + 1, m->last_cu.begin())) {
    nwork = m->last_nwork;
    return T5H_OK;
  }
  m->last_B = -1;
  order_by_length(m->order, cu, B);
  int xlen[8];
  nwork = 8 * plan_attention(m->cfg.num_heads, cu, m->order, xlen, [](const AttnGroup&) {});
  if (nwork > m->cap_work) return fail(T5H_ERR_INVALID, "internal: attention work list exceeds its capacity");
  StagingSlot& s = m->slots[m->next_slot];
  m->next_slot = (m->next_slot + 1) % 4;
  if (s.used) HIP_OK(hipEventSynchronize(s.done));
  const size_t need = (size_t)nwork * sizeof(int4);
  if (need > s.cap) {
    if (s.host) (void)hipHostFree(s.host);
    s.host = nullptr;
    s.cap = 0;
    if (hipHostMalloc(&s.host, std::max(need, (size_t)4096), hipHostMallocDefault) != hipSuccess)
      return fail(T5H_ERR_NOMEM, "pinned staging allocation failed");
    s.cap = std::max(need, (size_t)4096);
  }
  if (!s.done) HIP_OK(hipEventCreateWithFlags(&s.done, hipEventDisableTiming));
  int4* hw = (int4*)s.host;
  if (write_attention_work(m->cfg.num_heads, cu, m->order, hw, (size_t)nwork) != nwork)
    return fail(T5H_ERR_INVALID, "internal: attention work plan changed between passes");
  m->attn_flops = 0;
  for (int b = 0; b < B; b++)
    m->attn_flops += 4.0 * (double)(cu[b + 1] - cu[b]) * (cu[b + 1] - cu[b]) * m->cfg.d_kv * m->cfg.num_heads;
  if (nwork) HIP_OK(hipMemcpyAsync(m->w.work, hw, (size_t)nwork * sizeof(int4), hipMemcpyHostToDevice, m->stream));
  HIP_OK(hipEventRecord(s.done, m->stream));
  s.used = true;
  m->last_cu.assign(cu, cu + B + 1);
  m->last_B = B;
  m->last_nwork = nwork;
  return T5H_OK;
}

int validate_cu(const t5h_model* m, const int32_t* cu, int B, int& T) {
  if (B < 0 || (B > 0 && !cu)) return fail(T5H_ERR_INVALID, "bad batch description");
  if (B == 0) {
    T = 0;
    return T5H_OK;
  }
  if (cu[0] != 0) return fail(T5H_ERR_INVALID, "cu_seqlens[0] must be 0");
  for (int b = 0; b < B; b++) {
    const int L = cu[b + 1] - cu[b];
    if (L < 0) return fail(T5H_ERR_INVALID, "cu_seqlens must be non-decreasing");
    if (L > m->cfg.max_seq_len)
      return fail(T5H_ERR_INVALID, "sequence " + std::to_string(b) + " longer than max_seq_len");
  }
  T = cu[B];
  return T5H_OK;
}

void record_rmsnorm(t5h_model* m, const float* w, int T, float* rec, int stride) {
  if (!m->prof) return;
  ReplayRec& r = m->replay[K_RMSNORM];
  r.type = ReplayRec::RMSNORM;
  r.x = m->w.x;
  r.gamma = w;
  r.xn = m->w.xn;
  r.n = T;
  r.D = m->cfg.d_model;
  r.eps = m->cfg.layer_norm_epsilon;
  r.rec = rec;
  r.rec_stride = stride;
}

// T5LayerNorm of the residual stream into the f16 operand buffer, unless the consuming GEMV
// fuses it (returns the weight to pass to gemm() then, else nullptr).
const float* prenorm(t5h_model* m, const float* w, int T, int& rc) {
  rc = T5H_OK;
  if (use_gemv(m, T)) return w;
  Timed t(m, K_RMSNORM, 0, (double)T * m->cfg.d_model * 6);
  const hipError_t e = t5k::launch_rmsnorm(m->w.x, w, m->w.xn, T, m->cfg.d_model, m->cfg.layer_norm_epsilon, m->stream);
  if (e != hipSuccess) rc = fail(T5H_ERR_HIP, std::string("rmsnorm launch: ") + hipGetErrorString(e));
  record_rmsnorm(m, w, T, nullptr, 16);
  return nullptr;
}

// T5LayerNorm of the residual stream in record mode, for GEMMs that fold the norm.
int prenorm_rec(t5h_model* m, const float* w, int T, float* rec) {
  Timed t(m, K_RMSNORM, 0, (double)T * m->cfg.d_model * 6);
  const hipError_t e = t5k::launch_rmsnorm(m->w.x, w, m->w.xn, T, m->cfg.d_model, m->cfg.layer_norm_epsilon,
                                           m->stream, rec, rec_stride(m, T));
  if (e != hipSuccess) return fail(T5H_ERR_HIP, std::string("rmsnorm launch: ") + hipGetErrorString(e));
  record_rmsnorm(m, w, T, rec, rec_stride(m, T));
  return T5H_OK;
}

// One encoder block.  When the GEMMs fold the norms (fold_norm), the operand of the
// block's first norm is either made here (operand_ready false) or was left in m->w.xn / rec0 by
// the previous block's wo GEMM; with next_gamma set, this block's wo GEMM in turn prepares the
// operand of the norm that follows (next block's first norm or the final one).  With hybrid
// numerics only the first norm is folded (fold_attn_norm): QKV passes its operand scale on to
// wo, whose records the next block's QKV reads, so the two record buffers swap roles from one
// block to the next (even blocks read rec0).
int run_block(t5h_model* m, int l, int T, int nwork, bool operand_ready = false,
              const float* next_gamma = nullptr) {
  const t5h_config& c = m->cfg;
  const Layer& Ly = layer_w(m, l);
  const int D = c.d_model, inner = m->inner;
  const bool hybrid = hybrid_numerics(m);
  const bool fold = fold_norm(m, T), fold0 = fold_attn_norm(m, T);
  int rc;
  const float* nw0 = nullptr;
  NormLink qn, on, fn, wn;  // QKV consumer, O producer, FFN consumer, wo producer
  const NormLink* qkv_nl = nullptr;
  if (hybrid && fold0) {
    float* ra = (l & 1) ? m->w.rec1 : m->w.rec0;
    float* rb = (l & 1) ? m->w.rec0 : m->w.rec1;
    if (!operand_ready && (rc = prenorm_rec(m, Ly.ln0, T, ra))) return rc;
    qn.rec = ra;
    qn.rec_next = rb;
    wn.rec = rb;
    wn.nx = m->w.xn;
    wn.ngamma = next_gamma;
    qkv_nl = &qn;
  } else if (fold) {
    if (!operand_ready && (rc = prenorm_rec(m, Ly.ln0, T, m->w.rec0))) return rc;
    qn.rec = m->w.rec0;
    qn.rec_next = m->w.rec1;
    on.rec = m->w.rec1;
    on.nx = m->w.xn;
    on.ngamma = Ly.ln1;
    fn.rec = m->w.rec1;
    fn.rec_next = m->w.rec0;
    wn.rec = m->w.rec0;
    wn.nx = m->w.xn;
    wn.ngamma = next_gamma;
    qkv_nl = &qn;
  } else {
    nw0 = prenorm(m, Ly.ln0, T, rc);
    if (rc) return rc;
  }
  if (Ly.fused_qkv) {
    if ((rc = gemm(m, K_GEMM_QKV, EPI_QKV, Ly.qkv, nullptr, m->w.xn, D, T, m->w.qkvb, 0, 0, nw0, qkv_nl))) return rc;
  } else {
    if ((rc = gemm(m, K_GEMM_QKV, EPI_QKV, Ly.q, nullptr, m->w.xn, D, T, m->w.qkvb, 0, 0, nw0, qkv_nl))) return rc;
    if ((rc = gemm(m, K_GEMM_QKV, EPI_QKV, Ly.k, nullptr, m->w.xn, D, T, m->w.qkvb, 0, inner, nw0, qkv_nl))) return rc;
    if ((rc = gemm(m, K_GEMM_QKV, EPI_QKV, Ly.v, nullptr, m->w.xn, D, T, m->w.qkvb, 0, 2 * inner, nw0, qkv_nl)))
      return rc;
  }
  {
    AttnArgs a{};
    a.qkv = m->w.qkvb;
    a.out = m->w.ao;
    a.work = m->w.work;
    a.lut = m->rel_lut;
    a.heads = c.num_heads;
    a.tpad = m->w.tpad;
    a.lutw = m->lutw;
    Timed t(m, K_ATTN, m->attn_flops, 0);
    HIP_OK(t5k::launch_attention(a, nwork, c.d_kv, m->stream));
    if (m->prof) {
      ReplayRec& r = m->replay[K_ATTN];
      r.type = ReplayRec::ATTN;
      r.aa = a;
      r.n = nwork;
      r.D = c.d_kv;
    }
  }
  if ((rc = gemm(m, K_GEMM_O, EPI_RESID, Ly.o, nullptr, m->w.ao, inner, T, m->w.x, D, 0, nullptr, fold ? &on : nullptr)))
    return rc;
  const float* nw1 = nullptr;
  if (hybrid) {
    if ((rc = hybrid_linear(m, K_GEMM_GATE_UP, Ly.ln1, Ly.wi0, &Ly.wi1, T, nullptr, 0))) return rc;
    return gemm(m, K_GEMM_WO, EPI_RESID, Ly.wo, nullptr, m->w.hb, c.d_ff, T, m->w.x, D, 0, nullptr,
                fold0 && next_gamma ? &wn : nullptr);
  }
  if (!fold) {
    nw1 = prenorm(m, Ly.ln1, T, rc);
    if (rc) return rc;
  }
  const NormLink* ffn_nl = fold ? &fn : nullptr;
  if (c.feed_forward_gated && fold && use_ffn_fused(m, Ly, T)) {
    // gate|up, gelu * up and wo in one launch, h never leaving the CU (k_ffn.hip); the same bits
    // as the two launches below
    if (fn.rec_next != wn.rec) return fail(T5H_ERR_INVALID, "internal: FFN norm records out of step");
    t5k::FfnArgs fa{};
    fa.xn = m->w.xn;
    fa.W0 = Ly.wi0.w;
    fa.W1 = Ly.wi1.w;
    fa.Wo = Ly.wo.w;
    fa.x = m->w.x;
    fa.rec = fn.rec;
    fa.rec_out = fn.rec_next;
    fa.nx = next_gamma ? wn.nx : nullptr;
    fa.ngamma = next_gamma;
    fa.eps = c.layer_norm_epsilon;
    fa.M = T;
    fa.D = D;
    fa.F = c.d_ff;
    const double flops = 6.0 * T * D * c.d_ff;
    const double bytes = (double)(Ly.wi0.bytes() + Ly.wi1.bytes() + Ly.wo.bytes()) + 2.0 * T * D + 8.0 * T * D;
    Timed t(m, K_FFN, flops, bytes);
    HIP_OK(t5k::launch_ffn_fused(fa, Ly.wo.fmt, m->stream));
    if (m->prof) {
      ReplayRec& r = m->replay[K_FFN];
      r.type = ReplayRec::FFN;
      r.fa = fa;
      r.wfmt = Ly.wo.fmt;
    }
    return T5H_OK;
  }
  if (c.feed_forward_gated && fold && m->ffn_chunk > 0 && T > m->ffn_chunk && !use_gemv(m, T)) {
    // The FFN in token chunks (T5H_FFN_CHUNK): each chunk's d_ff intermediate, rows [0, n) of hb,
    // is read back by its wo launch right after gate|up wrote it, so at large batches it can stay
    // in the MALL.  Every row is computed as in the two launches over the whole batch (bit-
    // identical); measured no faster at cfg4.
    for (int t0 = 0; t0 < T; t0 += m->ffn_chunk) {
      const int n = std::min(m->ffn_chunk, T - t0);
      NormLink f2 = fn, w2 = wn;
      f2.rec += (size_t)t0 * 16;
      f2.rec_next += (size_t)t0 * 16;
      w2.rec += (size_t)t0 * 16;
      w2.nx += tiled_index(t0, 0, D);
      if ((rc = gemm(m, K_GEMM_GATE_UP, EPI_GATED, Ly.wi0, &Ly.wi1, m->w.xn + tiled_index(t0, 0, D), D, n, m->w.hb,
                     c.d_ff, 0, nullptr, &f2)))
        return rc;
      if ((rc = gemm(m, K_GEMM_WO, EPI_RESID, Ly.wo, nullptr, m->w.hb, c.d_ff, n, m->w.x + (size_t)t0 * D, D, 0,
                     nullptr, next_gamma ? &w2 : nullptr)))
        return rc;
    }
    return T5H_OK;
  }
  if (c.feed_forward_gated) {
    if ((rc = gemm(m, K_GEMM_GATE_UP, EPI_GATED, Ly.wi0, &Ly.wi1, m->w.xn, D, T, m->w.hb, c.d_ff, 0, nw1, ffn_nl)))
      return rc;
  } else {
    if ((rc = gemm(m, K_GEMM_GATE_UP, EPI_RELU, Ly.wi0, nullptr, m->w.xn, D, T, m->w.hb, c.d_ff, 0, nw1, ffn_nl)))
      return rc;
  }
  if ((rc = gemm(m, K_GEMM_WO, EPI_RESID, Ly.wo, nullptr, m->w.hb, c.d_ff, T, m->w.x, D, 0, nullptr,
                 fold && next_gamma ? &wn : nullptr)))
    return rc;
  return T5H_OK;
}

// Full forward from device ids; results in m->w.out / m->w.norm (or the given pointers).
int enqueue_stack(t5h_model* m, const uint32_t* d_ids, int T, int nwork, float* d_out, float* d_norm,
                  int normalize);

int enqueue_lane(t5h_model* m, const uint32_t* d_ids, const int32_t* cu, int B, int T, float* d_out, float* d_norm,
                 int normalize) {
  int nwork = 0, rc;
  if ((rc = ensure_workspace(m, T, B, attn_work_cap(m, T, B)))) return rc;
  if ((rc = upload_batch(m, cu, B, nwork))) return rc;
  return enqueue_stack(m, d_ids, T, nwork, d_out, d_norm, normalize);
}

void swap_lane(t5h_model* m, ExecLane& l) {
  std::swap(m->stream, l.stream);
  std::swap(m->ws, l.ws);
  std::swap(m->ws_bytes, l.ws_bytes);
  std::swap(m->cap_tokens, l.cap_tokens);
  std::swap(m->cap_seqs, l.cap_seqs);
  std::swap(m->cap_work, l.cap_work);
  std::swap(m->w, l.w);
  std::swap(m->order, l.order);
  std::swap(m->last_cu, l.last_cu);
  std::swap(m->last_B, l.last_B);
  std::swap(m->last_nwork, l.last_nwork);
  std::swap(m->attn_flops, l.attn_flops);
  for (int i = 0; i < 4; i++) std::swap(m->slots[i], l.slots[i]);
  std::swap(m->next_slot, l.next_slot);
}

// Batches of at least this many tokens (and two or more sequences) run as two halves, split at
// the sequence boundary nearest T / 2, on two streams: one half's launches fill the CUs the
// other's leave idle (tails of GEMM rounds, attention).  Measured per step, one lane vs two:
// 71 k tokens (cfg4) 18.7 vs 17.5 ms, 16.8 k (cfg5) 4.29 vs 4.22 ms and 5.57 vs 5.35 ms with
// hybrid numerics; 9.2 k and 4.4 k tokens are slower on two (2.48 vs 2.58 ms, 1.38 vs 1.42 ms).
// Outputs are bit-identical (every output row is computed the same way: the GEMMs keep one K
// order per output at any tile plan, attention is per sequence).
constexpr int SPLIT_MIN_TOKENS = 16384;

int enqueue_forward(t5h_model* m, const uint32_t* d_ids, const int32_t* cu, int B, int T, float* d_out,
                    float* d_norm, int normalize) {
  const int tmin = m->split_min > 0 ? m->split_min : SPLIT_MIN_TOKENS;
  if (m->split_off || m->prof || B < 2 || T < tmin)
    return enqueue_lane(m, d_ids, cu, B, T, d_out, d_norm, normalize);
  // parts: cut at the sequence boundaries nearest k T / n; a part without tokens (empty
  // sequences at a cut) ends the split there
  const int n = std::min(m->lanes, B);
  int cut[t5h_model::MAX_LANES + 1];
  int parts = 1;
  cut[0] = 0;
  for (int k = 1; k < n; k++) {
    int s = cut[parts - 1] + 1;
    for (int b = s + 1; b < B; b++)
      if (std::abs(n * cu[b] - k * T) < std::abs(n * cu[s] - k * T)) s = b;
    if (s >= B || cu[s] <= cu[cut[parts - 1]] || cu[s] >= T) break;
    cut[parts++] = s;
  }
  cut[parts] = B;
  // A part small enough for the GEMV kernels would round differently from the batched GEMM the
  // whole batch takes: keep one lane then, so results stay those of one lane.
  for (int i = 0; i < parts && parts > 1; i++)
    if (use_gemv(m, cu[cut[i + 1]] - cu[cut[i]])) parts = 1;
  if (parts == 1) return enqueue_lane(m, d_ids, cu, B, T, d_out, d_norm, normalize);
  const int P = m->cfg.proj_dim;
  if (!m->ev_fork) HIP_OK(hipEventCreateWithFlags(&m->ev_fork, hipEventDisableTiming));
  for (int i = 0; i + 1 < parts; i++) {
    if (!m->extra[i].stream) HIP_OK(hipStreamCreateWithFlags(&m->extra[i].stream, hipStreamNonBlocking));
    if (!m->ev_join[i]) HIP_OK(hipEventCreateWithFlags(&m->ev_join[i], hipEventDisableTiming));
  }
  // the other lanes start after everything enqueued on the handle's stream so far (the inputs)
  HIP_OK(hipEventRecord(m->ev_fork, m->stream));
  int rc = enqueue_lane(m, d_ids, cu, cut[1], cu[cut[1]], d_out, d_norm, normalize);
  if (rc) return rc;
  std::vector<int32_t> cub;
  for (int i = 1; i < parts; i++) {
    const int b0 = cut[i], nb = cut[i + 1] - b0, t0 = cu[b0];
    cub.assign(cu + b0, cu + b0 + nb + 1);
    for (auto& c : cub) c -= t0;
    ExecLane& l = m->extra[i - 1];
    HIP_OK(hipStreamWaitEvent(l.stream, m->ev_fork, 0));
    swap_lane(m, l);
    rc = enqueue_lane(m, d_ids + t0, cub.data(), nb, cub[nb], d_out + (size_t)t0 * P, d_norm ? d_norm + t0 : nullptr,
                      normalize);
    const hipError_t e = rc ? hipSuccess : hipEventRecord(m->ev_join[i - 1], m->stream);
    swap_lane(m, l);
    if (rc) return rc;
    HIP_OK(e);
    // the handle's stream (what callers synchronise or order after) waits for this lane
    HIP_OK(hipStreamWaitEvent(m->stream, m->ev_join[i - 1], 0));
  }
  return T5H_OK;
}

// The replay records of a profiled forward must not keep the caller's buffers (ids, outputs,
// norms of t5h_encode_device or the embedder's buffers): the caller may free or reuse them before
// t5h_replay_kernel runs.  Records that name them are pointed at the workspace's own buffers of
// the same shape instead (ids copied there, so a replayed gather reads the same rows).
int replay_own_buffers(t5h_model* m, const uint32_t* d_ids, int T, float* d_out, float* d_norm) {
  if (d_ids != m->w.ids)
    HIP_OK(hipMemcpyAsync(m->w.ids, d_ids, (size_t)T * 4, hipMemcpyDeviceToDevice, m->stream));
  for (auto& r : m->replay) {
    if (r.ids == d_ids) r.ids = m->w.ids;
    if (d_out && r.ga.out == (void*)d_out) r.ga.out = m->w.out;
    if (d_out && r.y == d_out) r.y = m->w.out;
    if (d_norm && r.norm == d_norm) r.norm = m->w.norm;
  }
  return T5H_OK;
}

// The launches of one forward on the workspace m->w, whose attention work list (nwork items)
// is in place.
int enqueue_stack(t5h_model* m, const uint32_t* d_ids, int T, int nwork, float* d_out, float* d_norm,
                  int normalize) {
  int rc;
  const t5h_config& c = m->cfg;
  // With folded norms the embedding gather also emits the first norm's operand and records
  // (hybrid numerics: when there is a block, whose QKV folds it; the projection's quantizer
  // normalises its own input).
  const bool hybrid = hybrid_numerics(m);
  const bool fold = fold_norm(m, T) || (fold_attn_norm(m, T) && c.num_layers > 0);
  {
    // algorithmic bytes: the table rows read (f32, or 144 B per 256 values of a Q4_K table), x
    // written (f32), and with the folded norm the f16 operand and the 64-byte record per token
    const double row_in = m->emb_fmt == EMB_F32 ? c.d_model * 4.0 : c.d_model / 256.0 * 144.0;
    const double row_out = c.d_model * 4.0 + (fold ? c.d_model * 2.0 + 64.0 : 0.0);
    Timed t(m, K_EMBED, 0, (double)T * (row_in + row_out));
    const float* g0 = c.num_layers > 0 ? m->layers[0].ln0 : m->final_ln;
    HIP_OK(t5k::launch_embed(d_ids, T, m->emb, m->emb_fmt, c.vocab_size, c.d_model, m->w.x, m->err_flag, m->stream,
                             g0, c.layer_norm_epsilon, fold ? m->w.xn : nullptr, fold ? m->w.rec0 : nullptr,
                             rec_stride(m, T)));
    if (m->prof) {
      ReplayRec& r = m->replay[K_EMBED];
      r.type = ReplayRec::EMBED;
      r.ids = d_ids;
      r.n = T;
      r.table = m->emb;
      r.fmt = m->emb_fmt;
      r.vocab = c.vocab_size;
      r.D = c.d_model;
      r.x = m->w.x;
      r.gamma = g0;
      r.eps = c.layer_norm_epsilon;
      r.xn = fold ? m->w.xn : nullptr;
      r.rec = fold ? m->w.rec0 : nullptr;
      r.rec_stride = rec_stride(m, T);
    }
  }
  for (int l = 0; l < c.num_layers; l++) {
    const float* next = l + 1 < c.num_layers ? m->layers[l + 1].ln0 : (hybrid ? nullptr : m->final_ln);
    if ((rc = run_block(m, l, T, nwork, fold, next))) return rc;
  }
  const float* nwf = nullptr;
  NormLink pn;
  if (hybrid) {
    if ((rc = hybrid_linear(m, K_GEMM_PROJ, m->final_ln, m->proj, nullptr, T, d_out, c.proj_dim))) return rc;
  } else {
    if (fold) {
      pn.rec = m->w.rec0;
    } else {
      nwf = prenorm(m, m->final_ln, T, rc);
      if (rc) return rc;
    }
    if ((rc = gemm(m, K_GEMM_PROJ, EPI_F32, m->proj, nullptr, m->w.xn, c.d_model, T, d_out, c.proj_dim, 0, nwf,
                   fold ? &pn : nullptr)))
      return rc;
  }
  {
    Timed t(m, K_ROWNORM, 0, (double)T * c.proj_dim * 8);
    HIP_OK(t5k::launch_rownorm(d_out, d_norm, T, c.proj_dim, normalize, m->stream, m->err_flag + 1));
    if (m->prof) {
      ReplayRec& r = m->replay[K_ROWNORM];
      r.type = ReplayRec::ROWNORM;
      r.y = d_out;
      r.norm = d_norm;
      r.n = T;
      r.P = c.proj_dim;
      r.normalize = normalize;
    }
  }
  if (m->prof) return replay_own_buffers(m, d_ids, T, d_out, d_norm);
  return T5H_OK;
}

int check_model(t5h_model* m) {
  if (!m) return fail(T5H_ERR_INVALID, "model handle is NULL");
  HIP_OK(hipSetDevice(m->device));
  return T5H_OK;
}

// t5h_encode_device on the device's fixed scratch array: no device or host allocation.  The
// workspace is carved from the array and the attention work list is written by a kernel from
// its arguments.  Nothing needs clearing between calls: every buffer is written before it is
// read, except rows past the last token, which only feed outputs that are never stored (the
// attention kernel zeroes value rows past a sequence's end as it loads them).
int encode_device_noalloc(t5h_model* m, const uint32_t* d_ids, const int32_t* cu, int B, float* d_out,
                          float* d_norm) {
  int rc, T = 0;
  if ((rc = check_model(m))) return rc;
  if ((rc = validate_cu(m, cu, B, T))) return rc;
  if (T == 0) return T5H_OK;
  if (!d_ids || !d_out) return fail(T5H_ERR_INVALID, "d_ids/d_out must not be NULL");
  if (!m->scratch) return fail(T5H_ERR_HIP, "no-alloc scratch array is not mapped on this device");
  order_by_length(m->order, cu, B);
  int xlen[8];
  const int nwork = 8 * plan_attention(m->cfg.num_heads, cu, m->order, xlen, [](const AttnGroup&) {});
  const int tpad = workspace_tpad(T);
  Workspace w;
  const size_t need = carve_workspace(m, tpad, nwork, nullptr, w);
  if (need > (size_t)T5H_NOALLOC_SCRATCH_BYTES)
    return fail(T5H_ERR_INVALID, "no-alloc encode of " + std::to_string(T) + " tokens needs " +
                                     std::to_string(need) + " bytes of workspace; the fixed scratch array holds " +
                                     std::to_string((size_t)T5H_NOALLOC_SCRATCH_BYTES));
  carve_workspace(m, tpad, nwork, (uint8_t*)m->scratch, w);
  // The work list of upload_batch, written by kernels from by-value chunks of groups and of
  // padding runs (length 0, `start` = number of empty slots).
  t5k::WorkChunk ch;
  ch.n = 0;
  hipError_t herr = hipSuccess;
  auto add = [&](int start, int len, int head, int pos) {
    ch.start[ch.n] = start;
    ch.len[ch.n] = len;
    ch.head[ch.n] = head;
    ch.pos[ch.n] = pos;
    if (++ch.n == t5k::WorkChunk::CAP) {
      if (herr == hipSuccess) herr = t5k::launch_work_list(ch, w.work, m->stream);
      ch.n = 0;
    }
  };
  plan_attention(m->cfg.num_heads, cu, m->order, xlen,
                 [&](const AttnGroup& g) { add(g.start, g.len, g.head, g.slot0 * 8 + g.xcd); });
  for (int x = 0; x < 8; x++)
    if (xlen[x] < nwork / 8) add(nwork / 8 - xlen[x], 0, 0, xlen[x] * 8 + x);
  if (herr == hipSuccess) herr = t5k::launch_work_list(ch, w.work, m->stream);
  HIP_OK(herr);
  // Run the stack on the scratch workspace without event timing (events would be created).
  const Workspace saved = m->w;
  const bool prof = m->prof;
  m->w = w;
  m->prof = false;
  rc = enqueue_stack(m, d_ids, T, nwork, d_out, d_norm, 0);
  m->w = saved;
  m->prof = prof;
  return rc;
}

// encode_device_noalloc ordered after every earlier no-alloc call on the same GPU (any handle,
// any thread): the array's users form one chain through the device's event.  A stream under
// graph capture is not chained (its launches run when the graph is replayed, not now): the
// caller orders replays against other no-alloc work on that GPU.
int encode_device_noalloc_ordered(t5h_model* m, const uint32_t* d_ids, const int32_t* cu, int B, float* d_out,
                                  float* d_norm) {
  int rc;
  if ((rc = check_model(m))) return rc;
  const int dev = m->device;
  if (dev < 0 || dev >= kMaxDevices || !g_noalloc_ev[dev])
    return fail(T5H_ERR_HIP, "no-alloc ordering event is not created on this device");
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HIP_OK(hipStreamIsCapturing(m->stream, &cap));
  if (cap != hipStreamCaptureStatusNone) return encode_device_noalloc(m, d_ids, cu, B, d_out, d_norm);
  std::lock_guard<std::mutex> lk(g_noalloc_mu[dev]);
  HIP_OK(hipStreamWaitEvent(m->stream, g_noalloc_ev[dev], 0));
  rc = encode_device_noalloc(m, d_ids, cu, B, d_out, d_norm);
  // recorded after a failed call too: whatever it enqueued stays ahead of the next user
  const hipError_t e = hipEventRecord(g_noalloc_ev[dev], m->stream);
  if (rc) return rc;
  HIP_OK(e);
  return T5H_OK;
}

int finish_sync(t5h_model* m) {
  HIP_OK(hipStreamSynchronize(m->stream));
  if (m->prof) resolve_timings(m);
  volatile unsigned* err = m->err_host;
  if (err[0]) {
    err[0] = 0;
    err[1] = 0;
    return fail(T5H_ERR_INVALID, "token id outside the vocabulary");
  }
  if (err[1]) {
    err[1] = 0;
    return fail(T5H_ERR_INVALID,
                "non-finite embedding: an f16 GEMM operand overflowed (a T5LayerNorm output |x * gamma| "
                "beyond the f16 range) or the weights hold non-finite values");
  }
  return T5H_OK;
}

int encode_host(t5h_model* m, const uint32_t* ids, const int32_t* cu, int32_t B, float* out,
                float* out_norm, int normalize) {
  int rc, T = 0;
  if ((rc = check_model(m))) return rc;
  if ((rc = validate_cu(m, cu, B, T))) return rc;
  if (T == 0) return T5H_OK;
  if (!ids || !out) return fail(T5H_ERR_INVALID, "ids/out must not be NULL");
  for (int t = 0; t < T; t++)
    if (ids[t] >= (uint32_t)m->cfg.vocab_size)
      return fail(T5H_ERR_INVALID, "token id " + std::to_string(ids[t]) + " at position " +
                                       std::to_string(t) + " outside the vocabulary");
  const int P = m->cfg.proj_dim;
  if ((rc = ensure_workspace(m, T, B, attn_work_cap(m, T, B)))) return rc;
  const size_t ids_b = align256((size_t)T * 4), out_b = (size_t)T * P * 4, norm_b = (size_t)T * 4;
  if ((rc = ensure_io(m, ids_b + out_b + norm_b))) return rc;
  uint8_t* io = (uint8_t*)m->io;
  memcpy(io, ids, (size_t)T * 4);
  HIP_OK(hipMemcpyAsync(m->w.ids, io, (size_t)T * 4, hipMemcpyHostToDevice, m->stream));
  if ((rc = enqueue_forward(m, m->w.ids, cu, B, T, m->w.out, m->w.norm, normalize))) return rc;
  HIP_OK(hipMemcpyAsync(io + ids_b, m->w.out, out_b, hipMemcpyDeviceToHost, m->stream));
  HIP_OK(hipMemcpyAsync(io + ids_b + out_b, m->w.norm, norm_b, hipMemcpyDeviceToHost, m->stream));
  if ((rc = finish_sync(m))) return rc;
  memcpy(out, io + ids_b, out_b);
  if (out_norm) memcpy(out_norm, io + ids_b + out_b, norm_b);
  return T5H_OK;
}

// Embedder::embed for a batch of documents (src/embedder.rs:22-103, once per document from
// src/lib.rs:930-934): every window of every document encoded as one packed batch, then the
// window sums, MIN_NORM filter, compaction and L2 normalisation on the device (k_embed.hip).
// Host buffers; out / kept_index have room for every token, kept_offsets[n_docs + 1].
int embed_batch_impl(t5h_model* m, const uint32_t* ids, const int32_t* doc_off, int n_docs, int max_len, int stride,
                     float* out, int32_t* kept_index, int32_t* kept_offsets) {
  int rc;
  if ((rc = check_model(m))) return rc;
  if (!ids || !doc_off || !out || !kept_index || !kept_offsets || n_docs <= 0)
    return fail(T5H_ERR_INVALID, "embed: bad arguments");
  if (max_len <= 0 || max_len > m->cfg.max_seq_len || stride < 0 || stride >= max_len)
    return fail(T5H_ERR_INVALID, "embed: need 0 < max_len <= max_seq_len and 0 <= stride < max_len");
  if (doc_off[0] != 0) return fail(T5H_ERR_INVALID, "embed: doc_offsets[0] must be 0");
  for (int d = 0; d < n_docs; d++)
    if (doc_off[d + 1] <= doc_off[d])
      return fail(T5H_ERR_INVALID, "embed: document " + std::to_string(d) + " is empty");
  const int N = doc_off[n_docs], P = m->cfg.proj_dim, step = max_len - stride;
  for (int t = 0; t < N; t++)
    if (ids[t] >= (uint32_t)m->cfg.vocab_size)
      return fail(T5H_ERR_INVALID, "token id " + std::to_string(ids[t]) + " at position " + std::to_string(t) +
                                       " outside the vocabulary");
  // Windows of src/embedder.rs:38-63: start_k = k * (max_len - stride) until a window reaches the
  // end; every window but a document's last holds max_len tokens.
  std::vector<int32_t> cu{0};
  std::vector<int4> docs(n_docs);
  for (int d = 0; d < n_docs; d++) {
    const int n = doc_off[d + 1] - doc_off[d];
    const int nwin = n <= max_len ? 1 : (n - max_len + step - 1) / step + 1;
    docs[d] = make_int4(doc_off[d], n, cu.back(), nwin);
    for (int k = 0; k < nwin; k++) cu.push_back(cu.back() + std::min(max_len, n - k * step));
  }
  const int W = n_docs ? (int)cu.size() - 1 : 0, T = cu.back();
  if ((rc = ensure_workspace(m, T, W, attn_work_cap(m, T, W)))) return rc;
  // device buffers of the post-processing
  const int nb = t5k::embed_batch_blocks(N);
  size_t off = 0;
  auto take = [&](size_t n) {
    const size_t o = off;
    off = align256(off + n);
    return o;
  };
  const size_t o_doc = take((size_t)n_docs * sizeof(int4)), o_tdoc = take((size_t)N * 4), o_nrm = take((size_t)N * 4),
               o_flag = take(N), o_cnt = take((size_t)(nb + 1) * 4), o_boff = take((size_t)(nb + 1) * 4),
               o_out = take((size_t)N * P * 4), o_kidx = take((size_t)N * 4), o_koff = take((size_t)(n_docs + 1) * 4);
  if (off > m->ew_bytes) {
    if (m->ew) {
      HIP_OK(hipStreamSynchronize(m->stream));
      HIP_OK(hipFree(m->ew));
      m->ew = nullptr;
      m->ew_bytes = 0;
    }
    if (hipMalloc(&m->ew, off) != hipSuccess) return fail(T5H_ERR_NOMEM, "embed workspace allocation failed");
    m->ew_bytes = off;
  }
  uint8_t* e = (uint8_t*)m->ew;
  // uploads through the pinned staging buffer: window ids, documents, token -> document
  const size_t h_ids = 0, h_doc = align256((size_t)T * 4), h_tdoc = h_doc + align256((size_t)n_docs * sizeof(int4));
  const size_t h_end = h_tdoc + align256((size_t)N * 4);
  const size_t h_dl = align256((size_t)(n_docs + 1) * 4) + (size_t)N * 4 + (size_t)N * P * 4;  // downloads
  if ((rc = ensure_io(m, std::max(h_end, h_dl)))) return rc;
  uint8_t* io = (uint8_t*)m->io;
  {
    uint32_t* wid = (uint32_t*)(io + h_ids);
    int* tdoc = (int*)(io + h_tdoc);
    for (int d = 0, w = 0; d < n_docs; d++) {
      for (int k = 0; k < docs[d].w; k++, w++)
        memcpy(wid + cu[w], ids + doc_off[d] + k * step, (size_t)(cu[w + 1] - cu[w]) * 4);
      for (int t = doc_off[d]; t < doc_off[d + 1]; t++) tdoc[t] = d;
    }
    memcpy(io + h_doc, docs.data(), (size_t)n_docs * sizeof(int4));
  }
  HIP_OK(hipMemcpyAsync(m->w.ids, io + h_ids, (size_t)T * 4, hipMemcpyHostToDevice, m->stream));
  HIP_OK(hipMemcpyAsync(e + o_doc, io + h_doc, (size_t)n_docs * sizeof(int4), hipMemcpyHostToDevice, m->stream));
  HIP_OK(hipMemcpyAsync(e + o_tdoc, io + h_tdoc, (size_t)N * 4, hipMemcpyHostToDevice, m->stream));
  if ((rc = enqueue_forward(m, m->w.ids, cu.data(), W, T, m->w.out, nullptr, 0))) return rc;
  HIP_OK(t5k::launch_embed_batch(m->w.out, (const int4*)(e + o_doc), (const int*)(e + o_tdoc), N, max_len, stride, P,
                                 (float*)(e + o_nrm), e + o_flag, (int*)(e + o_cnt), (int*)(e + o_boff),
                                 (float*)(e + o_out), (int*)(e + o_kidx), (int*)(e + o_koff), m->stream));
  // first the offsets and the total, then exactly the kept rows
  int32_t* h_koff = (int32_t*)io;
  HIP_OK(hipMemcpyAsync(h_koff, e + o_koff, (size_t)n_docs * 4, hipMemcpyDeviceToHost, m->stream));
  HIP_OK(hipMemcpyAsync(h_koff + n_docs, e + o_boff + (size_t)nb * 4, 4, hipMemcpyDeviceToHost, m->stream));
  if ((rc = finish_sync(m))) return rc;
  const int total = h_koff[n_docs];
  memcpy(kept_offsets, h_koff, (size_t)(n_docs + 1) * 4);
  uint8_t* dl = io + align256((size_t)(n_docs + 1) * 4);
  HIP_OK(hipMemcpyAsync(dl, e + o_out, (size_t)total * P * 4, hipMemcpyDeviceToHost, m->stream));
  HIP_OK(hipMemcpyAsync(dl + (size_t)total * P * 4, e + o_kidx, (size_t)total * 4, hipMemcpyDeviceToHost, m->stream));
  HIP_OK(hipStreamSynchronize(m->stream));
  memcpy(out, dl, (size_t)total * P * 4);
  memcpy(kept_index, dl + (size_t)total * P * 4, (size_t)total * 4);
  for (int d = 0; d < n_docs; d++)
    if (kept_offsets[d + 1] == kept_offsets[d])  // Embedder::embed bails for such a document (:89-91)
      return fail(T5H_ERR_INVALID, "document " + std::to_string(d) + ": all token embeddings below minimum norm threshold");
  return T5H_OK;
}

int create_impl(const void* gguf, size_t len, const t5h_config* cfg, int hip_device, t5h_model** out) {
  if (!out) return fail(T5H_ERR_INVALID, "out is NULL");
  *out = nullptr;
  int rc;
  if ((rc = check_config(cfg))) return rc;
  if (!gguf || len == 0) return fail(T5H_ERR_FORMAT, "model GGUF bytes are missing");
  t5h::GgufFile g;
  std::string perr;
  if (!t5h::parse_gguf((const uint8_t*)gguf, len, g, perr)) return fail(T5H_ERR_FORMAT, perr);

  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return fail(T5H_ERR_NODEVICE, "no HIP device");
  const int dev = hip_device < 0 ? 0 : hip_device;
  if (dev >= ndev) return fail(T5H_ERR_NODEVICE, "HIP device index out of range");
  hipDeviceProp_t prop;
  HIP_OK(hipGetDeviceProperties(&prop, dev));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(T5H_ERR_NODEVICE, std::string("t5-hip kernels target gfx950, device is ") + prop.gcnArchName);
  HIP_OK(hipSetDevice(dev));
  void* scratch_dev = nullptr;
  if ((rc = scratch_init(dev, &scratch_dev))) return rc;

  std::unique_ptr<t5h_model> m(new t5h_model());
  m->scratch = scratch_dev;
  m->cfg = *cfg;
  m->device = dev;
  m->inner = cfg->num_heads * cfg->d_kv;
  m->cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
  if (const char* e = getenv("T5H_GEMM_MW")) {
    const int v = atoi(e);
    if (v == 2 || v == 4 || v == 8) m->gemm_mw_override = v;
  }
  if (const char* e = getenv("T5H_GEMM_BN")) {
    const int v = atoi(e);
    if (v == 64 || v == 128) m->gemm_bn_override = v;
  }
  if (const char* e = getenv("T5H_GEMM_MB")) {
    const int v = atoi(e);
    if (v == 3 || v == 4) m->gemm_mb_override = v;
  }
  if (const char* e = getenv("T5H_GEMM_TAIL")) {
    const int v = atoi(e);
    if (v >= 0 && v <= 4) m->gemm_tail_override = v;
  }
  if (const char* e = getenv("T5H_FOLD_NORM")) m->fold_norm_off = atoi(e) == 0;
  if (const char* e = getenv("T5H_GATED_MW8")) m->gated_mw8 = atoi(e) != 0;
  if (const char* e = getenv("T5H_FFN_FUSED")) {
    const int v = atoi(e);
    m->ffn_fused_min = v > 0 ? v : 0;
  }
  if (const char* e = getenv("T5H_FFN_CHUNK")) {
    const int v = atoi(e);
    if (v > 0 && v % 512 == 0) m->ffn_chunk = v;
  }
  if (const char* e = getenv("T5H_LANES")) {
    const int v = atoi(e);
    if (v >= 2 && v <= t5h_model::MAX_LANES) m->lanes = v;
  }
  if (const char* e = getenv("T5H_SPLIT")) {
    const int v = atoi(e);
    m->split_off = v == 0;
    if (v > 1) m->split_min = v;
  }
  const int D = cfg->d_model, F = cfg->d_ff, inner = m->inner, H = cfg->num_heads;

  HostArena ha;
  // Embedding table: encoder.embed_tokens or shared (src/quantized_t5.rs:682-687).
  const char* emb_name = g.find("shared.weight") ? "shared.weight" : "encoder.embed_tokens.weight";
  const t5h::GgufTensor* et = g.find(emb_name);
  if (!et) return fail(T5H_ERR_FORMAT, "missing tensor encoder.embed_tokens.weight");
  if (et->shape.size() != 2 || (int)et->rows() != cfg->vocab_size || (int)et->cols() != D)
    return fail(T5H_ERR_FORMAT, std::string("tensor ") + emb_name + ": expected [vocab_size, d_model]");
  size_t emb_off;
  if (et->type == t5h::GGML_Q4_K) {
    m->emb_fmt = EMB_Q4K;
    emb_off = ha.add(et->data, et->nbytes);
  } else {
    m->emb_fmt = EMB_F32;
    emb_off = ha.add(nullptr, (size_t)cfg->vocab_size * D * 4);
    float* dst = reinterpret_cast<float*>(ha.bytes.data() + emb_off);
    if (et->type == t5h::GGML_F32)
      memcpy(dst, et->data, et->nbytes);
    else
      for (size_t i = 0; i < (size_t)cfg->vocab_size * D; i++) dst[i] = (float)((const _Float16*)et->data)[i];
  }
  // Relative attention bias of block 0 (src/quantized_t5.rs:351-360,640) -> LUT by j - i.
  const std::string rb_name = "encoder.block.0.layer.0.SelfAttention.relative_attention_bias.weight";
  const t5h::GgufTensor* rb = g.find(rb_name);
  if (!rb) return fail(T5H_ERR_FORMAT, "missing tensor " + rb_name);
  if (rb->type != t5h::GGML_F32 || rb->shape.size() != 2 ||
      (int)rb->rows() != cfg->relative_attention_num_buckets || (int)rb->cols() != H)
    return fail(T5H_ERR_FORMAT, "tensor " + rb_name + ": expected F32 [num_buckets, num_heads]");
  // The attention kernel stages the bias of distances k0 - q0 - (ATTN_QT - 1) .. k0 - q0 + 128
  // for a 64-key tile and an ATTN_QT-query workgroup (256 values, 4 waves x 64), so the LUT
  // covers |j - i| <= roundup(max_seq_len, 64) + ATTN_QT.
  const int lutw = (cfg->max_seq_len + 63) / 64 * 64 + ATTN_QT, span = 2 * lutw + 1;
  const size_t lut_off = ha.add(nullptr, (size_t)H * span * 4);
  {
    float* lut = reinterpret_cast<float*>(ha.bytes.data() + lut_off);
    const float* tab = reinterpret_cast<const float*>(rb->data);
    for (int dlt = -lutw; dlt <= lutw; dlt++) {
      const uint32_t i = dlt < 0 ? (uint32_t)(-dlt) : 0u, j = dlt < 0 ? 0u : (uint32_t)dlt;
      const uint32_t b = rel_bucket(i, j, cfg->relative_attention_num_buckets,
                                    cfg->relative_attention_max_distance);
      for (int h = 0; h < H; h++) lut[(size_t)h * span + dlt + lutw] = tab[b * H + h];
    }
  }
  m->layers.resize(cfg->num_layers);
  for (int l = 0; l < cfg->num_layers; l++) {
    Layer& Ly = m->layers[l];
    const std::string p = "encoder.block." + std::to_string(l) + ".layer.";
    if ((rc = add_f32_vector(ha, g, p + "0.layer_norm.weight", D, Ly.ln0_off))) return rc;
    if ((rc = add_f32_vector(ha, g, p + "1.layer_norm.weight", D, Ly.ln1_off))) return rc;
    // q, k, v: fused into one [3*inner, D] operand when they share a storage format
    // (the hybrid path fuses them the same way, src/quantized_t5.rs:321-339).
    const t5h::GgufTensor* tq = g.find(p + "0.SelfAttention.q.weight");
    const t5h::GgufTensor* tk = g.find(p + "0.SelfAttention.k.weight");
    const t5h::GgufTensor* tv = g.find(p + "0.SelfAttention.v.weight");
    if (!tq || !tk || !tv) return fail(T5H_ERR_FORMAT, "missing q/k/v weights in block " + std::to_string(l));
    auto kind = [](const t5h::GgufTensor* t) { return t->type == t5h::GGML_Q4_K ? 0 : 1; };
    Ly.fused_qkv = kind(tq) == kind(tk) && kind(tk) == kind(tv);
    if ((rc = add_linear(ha, g, p + "0.SelfAttention.q.weight", inner, D, Ly.q))) return rc;
    if ((rc = add_linear(ha, g, p + "0.SelfAttention.k.weight", inner, D, Ly.k))) return rc;
    if ((rc = add_linear(ha, g, p + "0.SelfAttention.v.weight", inner, D, Ly.v))) return rc;
    if (Ly.fused_qkv) {
      // the three regions are consecutive: re-pack them contiguously
      Ly.qkv.N = 3 * inner;
      Ly.qkv.K = D;
      Ly.qkv.fmt = Ly.q.fmt;
      const size_t one = Ly.q.bytes();
      std::vector<uint8_t> tmp(3 * one);
      memcpy(tmp.data(), ha.bytes.data() + Ly.q.off, one);
      memcpy(tmp.data() + one, ha.bytes.data() + Ly.k.off, one);
      memcpy(tmp.data() + 2 * one, ha.bytes.data() + Ly.v.off, one);
      Ly.qkv.off = ha.add(tmp.data(), tmp.size());
      add_bf16_copy(ha, {tq, tk, tv}, Ly.qkv);
    } else {
      add_bf16_copy(ha, {tq}, Ly.q);
      add_bf16_copy(ha, {tk}, Ly.k);
      add_bf16_copy(ha, {tv}, Ly.v);
    }
    if ((rc = add_linear(ha, g, p + "0.SelfAttention.o.weight", D, inner, Ly.o))) return rc;
    add_bf16_copy(ha, {g.find(p + "0.SelfAttention.o.weight")}, Ly.o);
    if (cfg->feed_forward_gated) {
      if ((rc = add_linear(ha, g, p + "1.DenseReluDense.wi_0.weight", F, D, Ly.wi0))) return rc;
      if ((rc = add_linear(ha, g, p + "1.DenseReluDense.wi_1.weight", F, D, Ly.wi1))) return rc;
      if (Ly.wi0.fmt != Ly.wi1.fmt) return fail(T5H_ERR_FORMAT, "wi_0 and wi_1 must share a storage format");
    } else {
      if ((rc = add_linear(ha, g, p + "1.DenseReluDense.wi.weight", F, D, Ly.wi0))) return rc;
    }
    if ((rc = add_linear(ha, g, p + "1.DenseReluDense.wo.weight", D, F, Ly.wo))) return rc;
    add_bf16_copy(ha, {g.find(p + "1.DenseReluDense.wo.weight")}, Ly.wo);
  }
  size_t fln_off;
  if ((rc = add_f32_vector(ha, g, "encoder.final_layer_norm.weight", D, fln_off))) return rc;
  if ((rc = add_linear(ha, g, "linear.weight", cfg->proj_dim, D, m->proj))) return rc;

  // ---- upload ----
  m->arena_bytes = align256(ha.bytes.size());
  if (hipMalloc(&m->arena, m->arena_bytes) != hipSuccess)
    return fail(T5H_ERR_NOMEM, "weight allocation of " + std::to_string(m->arena_bytes) + " bytes failed");
  HIP_OK(hipMemcpy(m->arena, ha.bytes.data(), ha.bytes.size(), hipMemcpyHostToDevice));
  uint8_t* base = (uint8_t*)m->arena;
  auto bind = [&](Linear& L) {
    L.w = base + L.off;
    if (L.has_bf) L.bf = base + L.bf_off;
  };
  m->emb = base + emb_off;
  m->rel_lut = (const float*)(base + lut_off);
  m->lutw = lutw;
  m->final_ln = (const float*)(base + fln_off);
  for (auto& Ly : m->layers) {
    Ly.ln0 = (const float*)(base + Ly.ln0_off);
    Ly.ln1 = (const float*)(base + Ly.ln1_off);
    bind(Ly.q); bind(Ly.k); bind(Ly.v); bind(Ly.o); bind(Ly.wi0); bind(Ly.wo);
    if (cfg->feed_forward_gated) bind(Ly.wi1);
    if (Ly.fused_qkv) bind(Ly.qkv);
  }
  bind(m->proj);
  HIP_OK(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
  if (hipHostMalloc((void**)&m->err_host, 256, hipHostMallocMapped) != hipSuccess)
    return fail(T5H_ERR_NOMEM, "pinned flag allocation failed");
  memset(m->err_host, 0, 256);
  HIP_OK(hipHostGetDevicePointer((void**)&m->err_flag, m->err_host, 0));
  for (int k = 0; k < K_COUNT; k++) m->stats[k].name = kKernelNames[k];
  *out = m.release();
  g_err.clear();
  return T5H_OK;
}

}  // namespace

// =================================================================================
namespace {
// argmax needs N > 0 (an argmax over no columns is undefined); matmul_t allows N == 0.
int check_score_args(const void* a, int32_t M, const void* b, int32_t N, int32_t D, const void* out, bool argmax) {
  if (M < 0 || N < 0 || D < 0) return fail(T5H_ERR_INVALID, "scoring needs M, N, D >= 0");
  if (argmax && N == 0 && M > 0) return fail(T5H_ERR_INVALID, "argmax over N == 0 columns");
  if (M > 0 && N > 0 && (!a || !b || !out)) return fail(T5H_ERR_INVALID, "NULL buffer");
  return T5H_OK;
}

// Host-buffer scoring call: upload A and B, run `launch` (which writes out_bytes at d_out),
// download.  All device memory is released on every path.
template <typename Launch>
int score_host(int32_t hip_device, const float* a, int32_t M, const float* b, int32_t N, int32_t D, void* out,
               size_t out_bytes, Launch launch) {
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return fail(T5H_ERR_NODEVICE, "no HIP device");
  HIP_OK(hipSetDevice(hip_device < 0 ? 0 : hip_device));
  // sub-buffers on 256-byte boundaries so the kernels' 16-byte vector loads stay available
  const size_t a_bytes = ((size_t)M * D * 4 + 255) & ~(size_t)255, b_bytes = ((size_t)N * D * 4 + 255) & ~(size_t)255;
  char* d = nullptr;
  if (hipMalloc((void**)&d, a_bytes + b_bytes + out_bytes) != hipSuccess)
    return fail(T5H_ERR_NOMEM, "scoring buffers");
  std::unique_ptr<void, void (*)(void*)> g(d, [](void* p) { (void)hipFree(p); });
  HIP_OK(hipMemcpy(d, a, (size_t)M * D * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d + a_bytes, b, (size_t)N * D * 4, hipMemcpyHostToDevice));
  HIP_OK(launch((const float*)d, (const float*)(d + a_bytes), (void*)(d + a_bytes + b_bytes)));
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(out, d + a_bytes + b_bytes, out_bytes, hipMemcpyDeviceToHost));
  return T5H_OK;
}
}  // namespace

extern "C" {

const char* t5h_last_error(void) { return g_err.c_str(); }

int t5h_config_xtr_base(t5h_config* c) {
  if (!c) return fail(T5H_ERR_INVALID, "config is NULL");
  c->vocab_size = 32128;
  c->d_model = 768;
  c->d_kv = 64;
  c->d_ff = 2048;
  c->num_layers = 12;
  c->num_heads = 12;
  c->relative_attention_num_buckets = 32;
  c->relative_attention_max_distance = 128;
  c->layer_norm_epsilon = 1e-6f;
  c->feed_forward_gated = 1;
  c->proj_dim = 128;
  c->max_seq_len = 2048;
  return T5H_OK;
}

int t5h_create(const void* gguf, size_t len, const t5h_config* cfg, int hip_device, t5h_model** out) {
  try {
    return create_impl(gguf, len, cfg, hip_device, out);
  } catch (const std::bad_alloc&) {
    return fail(T5H_ERR_NOMEM, "host allocation failed while loading the model");
  }
}

void t5h_destroy(t5h_model* model) {
  if (!model) return;
  (void)hipSetDevice(model->device);
  delete model;
}

int t5h_encode(t5h_model* m, const uint32_t* ids, const int32_t* cu, int32_t B, float* out, float* out_norm) {
  return encode_host(m, ids, cu, B, out, out_norm, 0);
}

int t5h_encode_normalized(t5h_model* m, const uint32_t* ids, const int32_t* cu, int32_t B, float* out,
                          float* out_norm) {
  return encode_host(m, ids, cu, B, out, out_norm, 1);
}

int t5h_encode_device(t5h_model* m, const uint32_t* d_ids, const int32_t* cu, int32_t B, float* d_out,
                      float* d_norm) {
  int rc, T = 0;
  if ((rc = check_model(m))) return rc;
  if ((rc = validate_cu(m, cu, B, T))) return rc;
  if (T == 0) return T5H_OK;
  if (!d_ids || !d_out) return fail(T5H_ERR_INVALID, "d_ids/d_out must not be NULL");
  return enqueue_forward(m, d_ids, cu, B, T, d_out, d_norm, 0);
}

int t5h_encode_device_noalloc(t5h_model* m, const uint32_t* d_ids, const int32_t* cu, int32_t B, float* d_out,
                              float* d_norm) {
  return encode_device_noalloc_ordered(m, d_ids, cu, B, d_out, d_norm);
}

int t5h_synchronize(t5h_model* m) {
  int rc;
  if ((rc = check_model(m))) return rc;
  return finish_sync(m);
}

void* t5h_stream(t5h_model* m) { return m ? (void*)m->stream : nullptr; }

int t5h_embed_ids(t5h_model* m, const uint32_t* ids, int32_t n, int32_t max_len, int32_t stride,
                  float* out, int32_t* kept_index, int32_t* n_kept) {
  if (!n_kept || n <= 0) return fail(T5H_ERR_INVALID, "embed_ids: bad arguments");
  const int32_t doc[2] = {0, n};
  int32_t kept_off[2] = {0, 0};
  const int rc = embed_batch_impl(m, ids, doc, 1, max_len, stride, out, kept_index, kept_off);
  *n_kept = kept_off[1];
  return rc;
}

int t5h_embed_batch(t5h_model* m, const uint32_t* ids, const int32_t* doc_offsets, int32_t n_docs, int32_t max_len,
                    int32_t stride, float* out, int32_t* kept_index, int32_t* kept_offsets) {
  return embed_batch_impl(m, ids, doc_offsets, n_docs, max_len, stride, out, kept_index, kept_offsets);
}

int t5h_q4k_dequant_f32(const void* blocks, size_t nblk, float* out, int hip_device) {
  if (nblk == 0) return T5H_OK;
  if (!blocks || !out) return fail(T5H_ERR_INVALID, "NULL buffer");
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return fail(T5H_ERR_NODEVICE, "no HIP device");
  HIP_OK(hipSetDevice(hip_device < 0 ? 0 : hip_device));
  void* d_in = nullptr;
  float* d_out = nullptr;
  HIP_OK(hipMalloc(&d_in, nblk * Q4K_BYTES));
  std::unique_ptr<void, void (*)(void*)> g1(d_in, [](void* p) { (void)hipFree(p); });
  HIP_OK(hipMalloc((void**)&d_out, nblk * QK_K * 4));
  std::unique_ptr<void, void (*)(void*)> g2(d_out, [](void* p) { (void)hipFree(p); });
  HIP_OK(hipMemcpy(d_in, blocks, nblk * Q4K_BYTES, hipMemcpyHostToDevice));
  HIP_OK(t5k::launch_q4k_dequant(d_in, nblk, d_out, nullptr));
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(out, d_out, nblk * QK_K * 4, hipMemcpyDeviceToHost));
  return T5H_OK;
}

int t5h_matmul_t(int32_t hip_device, const float* a, int32_t M, const float* b, int32_t N, int32_t D, int32_t bf16_b,
                 float* c) {
  int rc;
  if ((rc = check_score_args(a, M, b, N, D, c, false))) return rc;
  if (M == 0 || N == 0) return T5H_OK;
  return score_host(hip_device, a, M, b, N, D, c, (size_t)M * N * 4, [&](const float* da, const float* db, void* dc) {
    return t5k::launch_matmul_t(da, db, (float*)dc, M, N, D, bf16_b != 0, nullptr);
  });
}

int t5h_matmul_argmax(int32_t hip_device, const float* a, int32_t M, const float* b, int32_t N, int32_t D,
                      int32_t bf16_b, uint32_t* out) {
  int rc;
  if ((rc = check_score_args(a, M, b, N, D, out, true))) return rc;
  if (M == 0) return T5H_OK;
  return score_host(hip_device, a, M, b, N, D, out, (size_t)M * 4, [&](const float* da, const float* db, void* dout) {
    return t5k::launch_matmul_argmax(da, db, (uint32_t*)dout, M, N, D, bf16_b != 0, nullptr);
  });
}

int t5h_matmul_t_device(const float* d_a, int32_t M, const float* d_b, int32_t N, int32_t D, int32_t bf16_b,
                        float* d_c, void* stream) {
  int rc;
  if ((rc = check_score_args(d_a, M, d_b, N, D, d_c, false))) return rc;
  HIP_OK(t5k::launch_matmul_t(d_a, d_b, d_c, M, N, D, bf16_b != 0, (hipStream_t)stream));
  return T5H_OK;
}

int t5h_matmul_argmax_device(const float* d_a, int32_t M, const float* d_b, int32_t N, int32_t D, int32_t bf16_b,
                             uint32_t* d_out, void* stream) {
  int rc;
  if ((rc = check_score_args(d_a, M, d_b, N, D, d_out, true))) return rc;
  HIP_OK(t5k::launch_matmul_argmax(d_a, d_b, d_out, M, N, D, bf16_b != 0, (hipStream_t)stream));
  return T5H_OK;
}

int t5h_layer_forward(t5h_model* m, int32_t layer, const float* x_in, const int32_t* cu, int32_t B,
                      float* x_out) {
  int rc, T = 0;
  if ((rc = check_model(m))) return rc;
  if (layer < 0 || layer >= m->cfg.num_layers) return fail(T5H_ERR_INVALID, "layer index out of range");
  if ((rc = validate_cu(m, cu, B, T))) return rc;
  if (T == 0) return T5H_OK;
  if (!x_in || !x_out) return fail(T5H_ERR_INVALID, "NULL buffer");
  if ((rc = ensure_workspace(m, T, B, attn_work_cap(m, T, B)))) return rc;
  int nwork = 0;
  if ((rc = upload_batch(m, cu, B, nwork))) return rc;
  const size_t bytes = (size_t)T * m->cfg.d_model * 4;
  HIP_OK(hipMemcpyAsync(m->w.x, x_in, bytes, hipMemcpyHostToDevice, m->stream));
  if ((rc = run_block(m, layer, T, nwork))) return rc;
  HIP_OK(hipMemcpyAsync(x_out, m->w.x, bytes, hipMemcpyDeviceToHost, m->stream));
  return finish_sync(m);
}

int t5h_ffn_block(t5h_model* m, int32_t layer, const float* x, int32_t T, float* y, int32_t mode) {
  int rc;
  if ((rc = check_model(m))) return rc;
  if (layer < 0 || layer >= m->cfg.num_layers) return fail(T5H_ERR_INVALID, "layer index out of range");
  if (T <= 0 || !x || !y) return fail(T5H_ERR_INVALID, "bad FFN block arguments");
  if (mode != 0 && mode != 1) return fail(T5H_ERR_INVALID, "mode must be 0 or 1");
  if (!m->cfg.feed_forward_gated) return fail(T5H_ERR_INVALID, "model FFN is not gated");
  if ((rc = ensure_workspace(m, T, 1, attn_work_cap(m, T, 1)))) return rc;
  const t5h_config& c = m->cfg;
  const Layer& Ly = layer_w(m, layer);
  const size_t bytes = (size_t)T * c.d_model * 4;
  HIP_OK(hipMemcpyAsync(m->w.x, x, bytes, hipMemcpyHostToDevice, m->stream));
  m->batched_only = mode == 1;
  if (hybrid_numerics(m)) {
    rc = hybrid_linear(m, K_GEMM_GATE_UP, nullptr, Ly.wi0, &Ly.wi1, T, nullptr, 0);
  } else {
    HIP_OK(t5k::launch_f32_to_f16(m->w.x, m->w.xn, (size_t)T * c.d_model, c.d_model, m->stream));
    rc = gemm(m, K_GEMM_GATE_UP, EPI_GATED, Ly.wi0, &Ly.wi1, m->w.xn, c.d_model, T, m->w.hb, c.d_ff);
  }
  if (!rc) rc = gemm(m, K_GEMM_WO, EPI_F32, Ly.wo, nullptr, m->w.hb, c.d_ff, T, m->w.x, c.d_model);
  m->batched_only = false;
  if (rc) return rc;
  HIP_OK(hipMemcpyAsync(y, m->w.x, bytes, hipMemcpyDeviceToHost, m->stream));
  return finish_sync(m);
}

namespace {
// The dense linears of T5H_NUMERICS_HYBRID_BF16 (q/k/v or the fused qkv, o, wo): F32/F16 ones
// point at their arena copy of the truncated weights; Q4_K ones are expanded once into bfw
// (dequantized exactly, truncated to bf16, stored as f16 [N][K]).  Synchronous.
int build_bf16_layers(t5h_model* m) {
  if (!m->layers_bf.empty()) return T5H_OK;
  std::vector<Layer> lb = m->layers;
  std::vector<Linear*> dense;
  for (Layer& Ly : lb) {
    if (Ly.fused_qkv) {
      dense.push_back(&Ly.qkv);
    } else {
      dense.push_back(&Ly.q);
      dense.push_back(&Ly.k);
      dense.push_back(&Ly.v);
    }
    dense.push_back(&Ly.o);
    dense.push_back(&Ly.wo);
  }
  size_t need = 0;
  for (const Linear* L : dense)
    if (L->fmt == WF_Q4K) need += align256((size_t)L->N * L->K * 2);
  if (need && hipMalloc(&m->bfw, need) != hipSuccess) {
    m->bfw = nullptr;
    return fail(T5H_ERR_NOMEM, "bf16 weight allocation of " + std::to_string(need) + " bytes failed");
  }
  size_t off = 0;
  for (Linear* L : dense) {
    if (L->fmt == WF_Q4K) {
      _Float16* dst = (_Float16*)((uint8_t*)m->bfw + off);
      HIP_OK(t5k::launch_q4k_dequant_bf16_f16(L->w, (size_t)L->N * L->K / QK_K, dst, m->stream));
      off += align256((size_t)L->N * L->K * 2);
      L->w = dst;
    } else {
      if (!L->has_bf) return fail(T5H_ERR_INVALID, "internal: dense linear without its bf16 copy");
      L->w = L->bf;
    }
    L->fmt = WF_F16;
  }
  HIP_OK(hipStreamSynchronize(m->stream));
  m->layers_bf = std::move(lb);
  return T5H_OK;
}
}  // namespace

int t5h_set_numerics(t5h_model* m, int32_t mode) {
  int rc;
  if ((rc = check_model(m))) return rc;
  if (mode == T5H_NUMERICS_DEFAULT) {
    HIP_OK(hipStreamSynchronize(m->stream));
    m->numerics = mode;
    return T5H_OK;
  }
  if (mode != T5H_NUMERICS_HYBRID && mode != T5H_NUMERICS_HYBRID_BF16)
    return fail(T5H_ERR_INVALID, "unknown numerics mode");
  const t5h_config& c = m->cfg;
  if (!c.feed_forward_gated) return fail(T5H_ERR_INVALID, "hybrid numerics: the FFN must be gated-gelu");
  for (const Layer& Ly : m->layers)
    if (Ly.wi0.fmt != WF_Q4K || Ly.wi1.fmt != WF_Q4K)
      return fail(T5H_ERR_INVALID, "hybrid numerics: wi_0 / wi_1 must be Q4_K (QGatedMatMul)");
  if (m->proj.fmt != WF_Q4K) return fail(T5H_ERR_INVALID, "hybrid numerics: linear.weight must be Q4_K (QTiledOp)");
  if (c.d_model % QK_K || c.d_model > 1024 || c.d_ff % 64 || c.proj_dim % 64)
    return fail(T5H_ERR_INVALID, "hybrid numerics: needs d_model % 256 == 0 (<= 1024), d_ff and proj_dim % 64 == 0");
  // block scales (4 B) and bsum operand (64 B) per token and K block in the attention output buffer
  // (inner f16 per token; 2 B per token cover the alignment between the two, as tpad >= 128)
  if ((size_t)(c.d_model / QK_K) * 68 + 2 > (size_t)m->inner * 2)
    return fail(T5H_ERR_INVALID, "hybrid numerics: the Q8_K scales do not fit the attention output buffer");
  HIP_OK(hipStreamSynchronize(m->stream));
  if (mode == T5H_NUMERICS_HYBRID_BF16 && (rc = build_bf16_layers(m))) return rc;
  m->numerics = mode;
  return T5H_OK;
}

int t5h_attention_work(const int32_t* cu, int32_t B, int32_t heads, int32_t* items, int32_t cap, int32_t* n_items) {
  if (!cu || !items || !n_items || B < 0 || heads < 1 || cap < 0) return fail(T5H_ERR_INVALID, "bad arguments");
  if (cu[0] != 0) return fail(T5H_ERR_INVALID, "cu_seqlens[0] must be 0");
  for (int b = 0; b < B; b++)
    if (cu[b + 1] < cu[b]) return fail(T5H_ERR_INVALID, "cu_seqlens must be non-decreasing");
  std::vector<int> order;
  order_by_length(order, cu, B);
  const int n = write_attention_work(heads, cu, order, reinterpret_cast<int4*>(items), (size_t)cap);
  if (n < 0) return fail(T5H_ERR_INVALID, "attention work list longer than cap");
  *n_items = n;
  return T5H_OK;
}

int t5h_q8k_quantize(int32_t hip_device, const float* x, int32_t rows, int32_t cols, uint8_t* blocks) {
  if (rows < 0 || cols <= 0 || cols % QK_K || cols > 1024) return fail(T5H_ERR_INVALID, "q8k_quantize: bad shape");
  if (rows == 0) return T5H_OK;
  if (!x || !blocks) return fail(T5H_ERR_INVALID, "q8k_quantize: NULL buffer");
  HIP_OK(hipSetDevice(hip_device));
  const size_t xb = (size_t)rows * cols * 4, ob = (size_t)rows * t5k::q8k_bytes_per_row(cols);
  void* d = nullptr;
  if (hipMalloc(&d, align256(xb) + ob) != hipSuccess) return fail(T5H_ERR_NOMEM, "q8k_quantize buffers");
  uint8_t* dx = (uint8_t*)d;
  hipError_t e = hipMemcpy(dx, x, xb, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = t5k::launch_q8k_quantize((const float*)dx, nullptr, 0.f, rows, cols, dx + align256(xb), nullptr);
  if (e == hipSuccess) e = hipMemcpy(blocks, dx + align256(xb), ob, hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) return fail(T5H_ERR_HIP, std::string("q8k_quantize: ") + hipGetErrorString(e));
  return T5H_OK;
}

int t5h_q4k_q8k_matmul(int32_t hip_device, const uint8_t* w, int32_t N, const uint8_t* x8, int32_t T, int32_t K,
                       float* out) {
  if (N < 0 || T < 0 || K <= 0 || K % QK_K || K > 1024 || N % 64)
    return fail(T5H_ERR_INVALID, "q4k_q8k_matmul: bad shape (K % 256 == 0, K <= 1024, N % 64 == 0)");
  if (N == 0 || T == 0) return T5H_OK;
  if (!w || !x8 || !out) return fail(T5H_ERR_INVALID, "q4k_q8k_matmul: NULL buffer");
  HIP_OK(hipSetDevice(hip_device));
  int cus = 256;
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, hip_device);
  // the GEMM's tiles read operand rows up to a whole tile past T
  const int tpad = t5k::gemm_hybrid_rows(T), nblk = K / QK_K;
  const size_t wb = (size_t)N * K / QK_K * Q4K_BYTES, x8b = (size_t)T * t5k::q8k_bytes_per_row(K),
               xqb = (size_t)tpad * K, d8b = (size_t)tpad * nblk * 4, bsb = (size_t)tpad * nblk * 64,
               ob = (size_t)T * N * 4;
  void* d = nullptr;
  const size_t total = align256(wb) + align256(x8b) + align256(xqb) + align256(d8b) + align256(bsb) + ob;
  if (hipMalloc(&d, total) != hipSuccess) return fail(T5H_ERR_NOMEM, "q4k_q8k_matmul buffers");
  uint8_t* dw = (uint8_t*)d;
  uint8_t* dx = dw + align256(wb);
  int8_t* xq = (int8_t*)(dx + align256(x8b));
  float* d8 = (float*)((uint8_t*)xq + align256(xqb));
  _Float16* bs = (_Float16*)((uint8_t*)d8 + align256(d8b));
  float* dout = (float*)((uint8_t*)bs + align256(bsb));
  hipError_t e = hipMemset(d, 0, total);  // padding rows of the operands: zeros
  if (e == hipSuccess) e = hipMemcpy(dw, w, wb, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(dx, x8, x8b, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = t5k::launch_q8k_operands(dx, T, K, xq, d8, bs, nullptr);
  if (e == hipSuccess) {
    GemmArgs a{};
    a.A = reinterpret_cast<const _Float16*>(xq);  // int8 operand blocks (GemmArgs::A, hybrid)
    a.W0 = dw;
    a.M = T;
    a.N = N;
    a.K = K;
    a.out = dout;
    a.ldo = N;
    a.d8 = d8;
    a.bsop = bs;
    e = t5k::launch_gemm_hybrid(EPI_F32, t5k::gemm_plan_hybrid(T, N, cus), a, nullptr);
  }
  if (e == hipSuccess) e = hipMemcpy(out, dout, ob, hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) return fail(T5H_ERR_HIP, std::string("q4k_q8k_matmul: ") + hipGetErrorString(e));
  return T5H_OK;
}

int t5h_set_profiling(t5h_model* m, int32_t on) {
  int rc;
  if ((rc = check_model(m))) return rc;
  HIP_OK(hipStreamSynchronize(m->stream));
  resolve_timings(m);
  m->prof = on != 0;
  for (int k = 0; k < K_COUNT; k++) m->replay[k] = ReplayRec{};
  for (int k = 0; k < K_COUNT; k++) {
    m->stats[k].launches = 0;
    m->stats[k].total_ms = m->stats[k].flops = m->stats[k].bytes = 0;
  }
  return T5H_OK;
}

int t5h_replay_kernel(t5h_model* m, int32_t kind, int32_t reps, double* avg_us) {
  int rc;
  if ((rc = check_model(m))) return rc;
  if (kind < 0 || kind >= K_COUNT || reps <= 0 || !avg_us) return fail(T5H_ERR_INVALID, "replay: bad arguments");
  const ReplayRec& r = m->replay[kind];
  if (r.type == ReplayRec::NONE)
    return fail(T5H_ERR_INVALID, std::string("replay: no profiled forward launched ") + kKernelNames[kind]);
  auto launch = [&]() -> hipError_t {
    switch (r.type) {
      case ReplayRec::GEMM: return t5k::launch_gemm(r.epi, r.wfmt, r.plan, r.ga, m->stream);
      case ReplayRec::GEMV: return t5k::launch_gemv(r.epi, r.wfmt, r.ga, m->stream);
      case ReplayRec::ATTN: return t5k::launch_attention(r.aa, r.n, r.D, m->stream);
      case ReplayRec::FFN: return t5k::launch_ffn_fused(r.fa, r.wfmt, m->stream);
      case ReplayRec::EMBED:
        return t5k::launch_embed(r.ids, r.n, r.table, r.fmt, r.vocab, r.D, r.x, m->err_flag, m->stream, r.gamma,
                                 r.eps, r.xn, r.rec, r.rec_stride);
      case ReplayRec::ROWNORM:
        return t5k::launch_rownorm(r.y, r.norm, r.n, r.P, r.normalize, m->stream, m->err_flag + 1);
      case ReplayRec::RMSNORM:
        return t5k::launch_rmsnorm(r.x, r.gamma, r.xn, r.n, r.D, r.eps, m->stream, r.rec, r.rec_stride);
      case ReplayRec::HYBRID: {
        const hipError_t e =
            t5k::launch_q8k_quantize(r.x, r.gamma, r.eps, r.n, r.D, nullptr, m->stream,
                                     reinterpret_cast<int8_t*>(r.xn), r.hd8, r.hbs);
        if (e != hipSuccess) return e;
        return t5k::launch_gemm_hybrid(r.epi, r.plan, r.ga, m->stream);
      }
      default: return hipErrorInvalidValue;
    }
  };
  hipEvent_t e0 = take_event(m), e1 = take_event(m);
  if (!e0 || !e1) return fail(T5H_ERR_HIP, "replay: event creation failed");
  HIP_OK(launch());  // warm
  HIP_OK(hipEventRecord(e0, m->stream));
  for (int i = 0; i < reps; i++) HIP_OK(launch());
  HIP_OK(hipEventRecord(e1, m->stream));
  HIP_OK(hipEventSynchronize(e1));
  float ms = 0.f;
  HIP_OK(hipEventElapsedTime(&ms, e0, e1));
  m->event_pool.push_back(e0);
  m->event_pool.push_back(e1);
  *avg_us = (double)ms * 1e3 / reps;
  return T5H_OK;
}

int t5h_kernel_stats(t5h_model* m, t5h_kernel_stat* stats, int32_t cap) {
  int rc;
  if ((rc = check_model(m))) return rc;
  HIP_OK(hipStreamSynchronize(m->stream));
  resolve_timings(m);
  for (int k = 0; k < K_COUNT && k < cap; k++) stats[k] = m->stats[k];
  return K_COUNT;
}

}  // extern "C"
