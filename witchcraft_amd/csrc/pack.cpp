// pack.cpp -- host side of the packed chunk-embedding codec (k_pack.hip) and its C ABI.
//
// embeddings_to_packed (src/packops.rs:172-301) / embeddings_from_packed (:303-438) over a
// batch of matrices.  The host only lays out windows (<= 1024 rows each), walks headers and
// sums byte counts; every transform, the rANS64 coder and the output assembly run on the GPU.
// Packed format per matrix (native-endian, as the reference writes it): u32 rows, then per
// window: cols bytes of inverse column permutation, u16 m, m x (u16 symbol, u16 freq),
// u16 stream bytes, the rANS64 stream.
#include <hip/hip_runtime.h>
#include <string.h>

#include <string>
#include <vector>

#include "../../include/t5hip.h"
#include "common.hpp"

namespace t5k {
struct PkWin {
  int row0, rows;
  long long hdr, data;
  int m, dlen, err, pad;
};
constexpr int PK_HDR_BYTES = 256 + 2 + 4 * 4096 + 254;
hipError_t pk_encode(const float* x, int total_rows, int cols, PkWin* win, int nwin, const int* row_win, float* work,
                     uint16_t* syms, int* perm, uint8_t* hdr, uint32_t* pairs, uint8_t* data, hipStream_t s);
hipError_t pk_assemble_out(const PkWin* win, int nwin, int cols, const uint8_t* hdr, const uint8_t* data,
                           const long long* out_off, const long long* mat_off, const int* mat_rows, int B,
                           uint8_t* out, hipStream_t s);
hipError_t pk_decode(const uint8_t* in, int total_rows, int cols, PkWin* win, int nwin, const int* row_win,
                     float* out, float* work, hipStream_t s);
}  // namespace t5k

namespace t5h_detail {
int fail(int code, const std::string& msg);
}

namespace {

using t5h_detail::fail;
using t5k::PkWin;

#define HIP_OK(expr)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess)                                                              \
      return fail(T5H_ERR_HIP, std::string(#expr ": ") + hipGetErrorString(e_));       \
  } while (0)

constexpr int WINDOW_ROWS = 1024;  // MAX_WINDOW_ROWS, packops.rs:8

size_t a256(size_t n) { return (n + 255) & ~(size_t)255; }

// One device allocation carved into aligned pieces; freed on every path.
struct Arena {
  char* base = nullptr;
  ~Arena() {
    if (base) (void)hipFree(base);
  }
};

int set_device(int32_t dev) {
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return fail(T5H_ERR_NODEVICE, "no HIP device");
  HIP_OK(hipSetDevice(dev < 0 ? 0 : dev));
  return T5H_OK;
}

const char* pk_err_text(int e) {
  switch (e) {
    case 1: return "a column sum is NaN (the reference's sort panics)";
    case 2: return "more than 4096 distinct symbols in a window (scale_histogram asserts)";
    case 3: return "rANS stream overflows 2 bytes per value (the reference's encoder panics)";
    case 4: return "corrupt rANS stream";
  }
  return "codec error";
}

struct Timer {
  hipEvent_t a = nullptr, b = nullptr;
  ~Timer() {
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
  }
};

}  // namespace

extern "C" {

int t5h_embeddings_to_packed(int32_t hip_device, const float* x, const int32_t* row_offsets, int32_t B, int32_t cols,
                             uint8_t* out, size_t out_cap, size_t* out_offsets, double* gpu_ms) {
  if (B < 0 || !row_offsets || !out_offsets) return fail(T5H_ERR_INVALID, "bad batch description");
  if (cols <= 0 || cols > 255) return fail(T5H_ERR_INVALID, "column count must fit in u8 (1..255)");
  if (row_offsets[0] != 0) return fail(T5H_ERR_INVALID, "row_offsets[0] must be 0");
  for (int b = 0; b < B; b++)
    if (row_offsets[b + 1] < row_offsets[b]) return fail(T5H_ERR_INVALID, "row_offsets must be non-decreasing");
  const int total = row_offsets[B];
  if (total > 0 && !x) return fail(T5H_ERR_INVALID, "x is NULL");
  // windows
  std::vector<PkWin> win;
  std::vector<int> row_win(total), mat_rows(B);
  long long data_bytes = 0;
  for (int b = 0; b < B; b++) {
    const int rows = row_offsets[b + 1] - row_offsets[b];
    mat_rows[b] = rows;
    for (int off = 0; off < rows; off += WINDOW_ROWS) {
      PkWin w{};
      w.row0 = row_offsets[b] + off;
      w.rows = std::min(WINDOW_ROWS, rows - off);
      w.hdr = (long long)win.size() * t5k::PK_HDR_BYTES;
      w.data = data_bytes;
      data_bytes += (long long)a256((size_t)2 * w.rows * cols + 16);
      for (int r = 0; r < w.rows; r++) row_win[w.row0 + r] = (int)win.size();
      win.push_back(w);
    }
  }
  const int nwin = (int)win.size();
  int rc;
  if ((rc = set_device(hip_device))) return rc;
  // device layout
  const size_t x_b = a256((size_t)total * cols * 4), s_b = a256((size_t)total * cols * 2);
  const size_t w_b = a256(sizeof(PkWin) * (nwin + 1)), rw_b = a256((size_t)total * 4 + 4);
  const size_t p_b = a256((size_t)nwin * 256 * 4 + 4), h_b = a256((size_t)nwin * t5k::PK_HDR_BYTES + 4);
  const size_t pr_b = a256((size_t)nwin * 4096 * 2 * 4 + 4), d_b = a256((size_t)data_bytes + 4);
  const size_t o_b = a256((size_t)(nwin + 1) * 8), mo_b = a256((size_t)(B + 1) * 8), mr_b = a256((size_t)(B + 1) * 4);
  Arena ar;
  const size_t fixed = 2 * x_b + s_b + w_b + rw_b + p_b + h_b + pr_b + d_b + o_b + mo_b + mr_b;
  if (hipMalloc((void**)&ar.base, fixed) != hipSuccess) return fail(T5H_ERR_NOMEM, "codec workspace");
  char* p = ar.base;
  float* d_x = (float*)p;
  p += x_b;
  float* d_work = (float*)p;
  p += x_b;
  uint16_t* d_syms = (uint16_t*)p;
  p += s_b;
  PkWin* d_win = (PkWin*)p;
  p += w_b;
  int* d_rw = (int*)p;
  p += rw_b;
  int* d_perm = (int*)p;
  p += p_b;
  uint8_t* d_hdr = (uint8_t*)p;
  p += h_b;
  uint32_t* d_pairs = (uint32_t*)p;
  p += pr_b;
  uint8_t* d_data = (uint8_t*)p;
  p += d_b;
  long long* d_off = (long long*)p;
  p += o_b;
  long long* d_moff = (long long*)p;
  p += mo_b;
  int* d_mrows = (int*)p;
  if (total > 0) HIP_OK(hipMemcpy(d_x, x, (size_t)total * cols * 4, hipMemcpyHostToDevice));
  if (nwin > 0) {
    HIP_OK(hipMemcpy(d_win, win.data(), sizeof(PkWin) * nwin, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_rw, row_win.data(), (size_t)total * 4, hipMemcpyHostToDevice));
  }
  Timer tm;
  if (gpu_ms) {
    HIP_OK(hipEventCreate(&tm.a));
    HIP_OK(hipEventCreate(&tm.b));
    HIP_OK(hipEventRecord(tm.a, nullptr));
  }
  HIP_OK(t5k::pk_encode(d_x, total, cols, d_win, nwin, d_rw, d_work, d_syms, d_perm, d_hdr, d_pairs, d_data, nullptr));
  if (nwin > 0) HIP_OK(hipMemcpy(win.data(), d_win, sizeof(PkWin) * nwin, hipMemcpyDeviceToHost));
  for (const PkWin& w : win)
    if (w.err) return fail(T5H_ERR_INVALID, std::string("embeddings_to_packed: ") + pk_err_text(w.err));
  // byte offsets: per matrix u32 rows, per window cols + 2 + 4m + 2 + dlen
  std::vector<long long> off(nwin), moff(B);
  size_t pos = 0;
  int wi = 0;
  for (int b = 0; b < B; b++) {
    out_offsets[b] = pos;
    moff[b] = (long long)pos;
    pos += 4;
    for (int off_r = 0; off_r < mat_rows[b]; off_r += WINDOW_ROWS, wi++) {
      off[wi] = (long long)pos;
      pos += (size_t)cols + 2 + 4 * (size_t)win[wi].m + 2 + (size_t)win[wi].dlen;
    }
  }
  out_offsets[B] = pos;
  if (pos > out_cap || (pos > 0 && !out))
    return fail(T5H_ERR_INVALID, "output buffer of " + std::to_string(out_cap) + " bytes; " + std::to_string(pos) +
                                     " needed (out_offsets[B])");
  uint8_t* d_out = nullptr;
  if (hipMalloc((void**)&d_out, pos + 16) != hipSuccess) return fail(T5H_ERR_NOMEM, "codec output");
  struct Free {
    void* p;
    ~Free() { (void)hipFree(p); }
  } f{d_out};
  if (nwin > 0) HIP_OK(hipMemcpy(d_off, off.data(), sizeof(long long) * nwin, hipMemcpyHostToDevice));
  if (B > 0) {
    HIP_OK(hipMemcpy(d_moff, moff.data(), sizeof(long long) * B, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_mrows, mat_rows.data(), sizeof(int) * B, hipMemcpyHostToDevice));
  }
  HIP_OK(t5k::pk_assemble_out(d_win, nwin, cols, d_hdr, d_data, d_off, d_moff, d_mrows, B, d_out, nullptr));
  if (gpu_ms) {
    HIP_OK(hipEventRecord(tm.b, nullptr));
    HIP_OK(hipEventSynchronize(tm.b));
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, tm.a, tm.b));
    *gpu_ms = ms;
  }
  HIP_OK(hipDeviceSynchronize());
  if (pos > 0) HIP_OK(hipMemcpy(out, d_out, pos, hipMemcpyDeviceToHost));
  return T5H_OK;
}

int t5h_embeddings_from_packed(int32_t hip_device, const uint8_t* buf, const size_t* buf_offsets, int32_t B,
                               int32_t cols, float* out, size_t out_cap_rows, int32_t* row_offsets, double* gpu_ms) {
  if (B < 0 || !buf_offsets || !row_offsets) return fail(T5H_ERR_INVALID, "bad batch description");
  if (cols <= 0 || cols > 255) return fail(T5H_ERR_INVALID, "column count must fit in u8 (1..255)");
  if (buf_offsets[0] != 0) return fail(T5H_ERR_INVALID, "buf_offsets[0] must be 0");
  const size_t len = buf_offsets[B];
  if (len > 0 && !buf) return fail(T5H_ERR_INVALID, "buf is NULL");
  // walk the headers (packops.rs:303-350): bounds-checked like the reference's split_at calls
  std::vector<PkWin> win;
  std::vector<int> row_win;
  long long total = 0;
  row_offsets[0] = 0;
  for (int b = 0; b < B; b++) {
    size_t pos = buf_offsets[b];
    const size_t end = buf_offsets[b + 1];
    if (end < pos || end > len) return fail(T5H_ERR_INVALID, "buf_offsets must be non-decreasing");
    const std::string where = "packed matrix " + std::to_string(b) + ": ";
    if (end - pos < 4) return fail(T5H_ERR_FORMAT, where + "shorter than its row count");
    uint32_t rows;
    memcpy(&rows, buf + pos, 4);
    pos += 4;
    if (total + rows > (long long)out_cap_rows || total + rows > 0x7fffffffLL)
      return fail(T5H_ERR_INVALID, where + "more rows than the output holds");
    for (uint32_t off = 0; off < rows; off += WINDOW_ROWS) {
      PkWin w{};
      w.row0 = (int)(total + off);
      w.rows = (int)std::min<uint32_t>(WINDOW_ROWS, rows - off);
      if (end - pos < (size_t)cols + 2) return fail(T5H_ERR_FORMAT, where + "truncated window header");
      w.hdr = (long long)pos;
      for (int c = 0; c < cols; c++)
        if (buf[pos + c] >= cols) return fail(T5H_ERR_FORMAT, where + "column index out of range");
      pos += cols;
      uint16_t m;
      memcpy(&m, buf + pos, 2);
      pos += 2;
      if (end - pos < 4 * (size_t)m + 2) return fail(T5H_ERR_FORMAT, where + "truncated histogram");
      w.m = m;
      pos += 4 * (size_t)m;
      uint16_t clen;
      memcpy(&clen, buf + pos, 2);
      pos += 2;
      if (end - pos < clen) return fail(T5H_ERR_FORMAT, where + "truncated rANS stream");
      if (clen < 8) return fail(T5H_ERR_FORMAT, where + "rANS stream shorter than its state");
      w.data = (long long)pos;
      w.dlen = clen;
      pos += clen;
      for (int r = 0; r < w.rows; r++) row_win.push_back((int)win.size());
      win.push_back(w);
    }
    if (pos != end)
      return fail(T5H_ERR_FORMAT, where + "leftover " + std::to_string(end - pos) + " bytes after decoding " +
                                      std::to_string(rows) + " rows x " + std::to_string(cols) + " cols");
    total += rows;
    row_offsets[b + 1] = (int32_t)total;
  }
  if (total > 0 && !out) return fail(T5H_ERR_INVALID, "out is NULL");
  const int nwin = (int)win.size();
  int rc;
  if ((rc = set_device(hip_device))) return rc;
  const size_t in_b = a256(len + 16), x_b = a256((size_t)total * cols * 4 + 4), w_b = a256(sizeof(PkWin) * (nwin + 1));
  const size_t rw_b = a256((size_t)total * 4 + 4);
  Arena ar;
  if (hipMalloc((void**)&ar.base, in_b + 2 * x_b + w_b + rw_b) != hipSuccess) return fail(T5H_ERR_NOMEM, "codec workspace");
  uint8_t* d_in = (uint8_t*)ar.base;
  float* d_out = (float*)(ar.base + in_b);
  float* d_work = (float*)(ar.base + in_b + x_b);
  PkWin* d_win = (PkWin*)(ar.base + in_b + 2 * x_b);
  int* d_rw = (int*)(ar.base + in_b + 2 * x_b + w_b);
  if (len > 0) HIP_OK(hipMemcpy(d_in, buf, len, hipMemcpyHostToDevice));
  if (nwin > 0) {
    HIP_OK(hipMemcpy(d_win, win.data(), sizeof(PkWin) * nwin, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_rw, row_win.data(), (size_t)total * 4, hipMemcpyHostToDevice));
  }
  Timer tm;
  if (gpu_ms) {
    HIP_OK(hipEventCreate(&tm.a));
    HIP_OK(hipEventCreate(&tm.b));
    HIP_OK(hipEventRecord(tm.a, nullptr));
  }
  HIP_OK(t5k::pk_decode(d_in, (int)total, cols, d_win, nwin, d_rw, d_out, d_work, nullptr));
  if (gpu_ms) {
    HIP_OK(hipEventRecord(tm.b, nullptr));
    HIP_OK(hipEventSynchronize(tm.b));
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, tm.a, tm.b));
    *gpu_ms = ms;
  }
  HIP_OK(hipDeviceSynchronize());
  if (nwin > 0) HIP_OK(hipMemcpy(win.data(), d_win, sizeof(PkWin) * nwin, hipMemcpyDeviceToHost));
  for (const PkWin& w : win)
    if (w.err) return fail(T5H_ERR_FORMAT, std::string("embeddings_from_packed: ") + pk_err_text(w.err));
  if (total > 0) HIP_OK(hipMemcpy(out, d_out, (size_t)total * cols * 4, hipMemcpyDeviceToHost));
  return T5H_OK;
}

}  // extern "C"
