// codec.cpp -- host side of the residual codec (src/packops.rs) and its C ABI entry points.
//
// The 4-bit residual code is compand().quantize(4) (packops.rs:136-142, 156-162) of the f32
// residual; its decode value is make_q4_dequant_table (packops.rs:14-25).  Both are computed
// here once per process with the reference's scalar op sequence (candle's affine ops are
// v * (f32)mul + (f32)add; log/exp are the C library's logf/expf, which Rust's f32::ln/exp
// call), so the table is the reference's table and the thresholds are exact:
//   code(x) = number of thresholds t_j <= x, t_j = the least f32 x with code(x) >= j,
// found by bisection over the ordered f32 values.  The kernels (k_codec.hip) only compare
// against the thresholds and look up the table.
#include <hip/hip_runtime.h>
#include <math.h>
#include <string.h>

#include <memory>
#include <string>

#include "../../include/t5hip.h"
#include "common.hpp"

// Two roundings per candle affine op, as the reference: never fuse them.
#pragma clang fp contract(off)

namespace t5k {
struct Q4Table {
  float v[16];
};
struct Q4Ladder {
  float t[15];
};
hipError_t launch_residual_encode(const float* emb, const float* centers, const uint32_t* assign, int N, int D,
                                  int K, const Q4Ladder& lad, uint8_t* out, unsigned* bad, hipStream_t s);
hipError_t launch_residual_decode(const uint8_t* codes, size_t nbytes, const Q4Table& tab, float* out,
                                  hipStream_t s);
hipError_t launch_matmul_t_q4(const float* A, const uint8_t* codes, const Q4Table& tab, float* C, int M, int N,
                              int D, hipStream_t s);
}  // namespace t5k

namespace t5h_detail {
int fail(int code, const std::string& msg);
}

namespace {

using t5h_detail::fail;

#define HIP_OK(expr)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess)                                                              \
      return fail(T5H_ERR_HIP, std::string(#expr ": ") + hipGetErrorString(e_));       \
  } while (0)

float affine(float v, double mul, double add) { return v * (float)mul + (float)add; }
float sgn(float v) { return v > 0.f ? 1.f : (v < 0.f ? -1.f : 0.f); }

// compand() (mu-law with scale 4 and mu = 255) then quantize(4) (zero point and scale 7.5,
// round half away from zero, clamp to [0, 15]; a NaN lands on the lower bound).
uint32_t compand_q4(float v) {
  const float x = affine(v, 4.0, 0.0);
  const float t = affine(affine(fabsf(x), 255.0, 0.0), 1.0, 1.0);
  const float c = sgn(x) * affine(logf(t), 1.0 / log(256.0), 0.0);
  float y = roundf(affine(affine(c, 7.5, 0.0), 1.0, 7.5));
  y = y > 0.f ? y : 0.f;
  y = y < 15.f ? y : 15.f;
  return (uint32_t)y;
}

// Monotone map of the non-NaN f32 values (-0 just below +0) onto uint32.
uint32_t f32_key(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
float key_f32(uint32_t k) {
  const uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  float f;
  memcpy(&f, &b, 4);
  return f;
}

struct Codec {
  t5k::Q4Table table;
  t5k::Q4Ladder ladder;
  Codec() {
    // make_q4_dequant_table: arange(0, 16).dequantize(4).inv_compand(), inv_compand's pow as
    // candle computes it, exp(|x| ln(1 + 255))
    const float ln256 = logf(affine(1.0f, 1.0, 255.0));
    for (int i = 0; i < 16; i++) {
      const float x = affine(affine((float)i, 1.0, -7.5), 2.0 / 15.0, 0.0);
      const float p = expf(fabsf(x) * ln256);
      const float s = sgn(x) * affine(affine(p, 1.0, -1.0), 1.0 / 255.0, 0.0);
      table.v[i] = affine(s, 0.25, 0.0);
    }
    const uint32_t lo0 = f32_key(-INFINITY), hi0 = f32_key(INFINITY);
    for (int j = 1; j <= 15; j++) {
      uint32_t lo = lo0, hi = hi0;  // code(lo) < j <= code(hi)
      while (hi - lo > 1) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (compand_q4(key_f32(mid)) >= (uint32_t)j) hi = mid;
        else lo = mid;
      }
      ladder.t[j - 1] = key_f32(hi);
    }
  }
};

const Codec& codec() {
  static const Codec c;
  return c;
}

int set_device(int32_t hip_device) {
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return fail(T5H_ERR_NODEVICE, "no HIP device");
  HIP_OK(hipSetDevice(hip_device < 0 ? 0 : hip_device));
  return T5H_OK;
}

struct DevBuf {
  char* p = nullptr;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
};

size_t pad256(size_t n) { return (n + 255) & ~(size_t)255; }

int check_codes(int32_t N, int32_t D, int multiple) {
  if (N < 0 || D <= 0 || D % multiple) return fail(T5H_ERR_INVALID, "need N >= 0 and D > 0, D % " +
                                                                        std::to_string(multiple) + " == 0");
  return T5H_OK;
}

}  // namespace

extern "C" {

int t5h_q4_dequant_table(float table[16]) {
  if (!table) return fail(T5H_ERR_INVALID, "table is NULL");
  memcpy(table, codec().table.v, sizeof(float) * 16);
  return T5H_OK;
}

int t5h_q4_compand_thresholds(float thresholds[15]) {
  if (!thresholds) return fail(T5H_ERR_INVALID, "thresholds is NULL");
  memcpy(thresholds, codec().ladder.t, sizeof(float) * 15);
  return T5H_OK;
}

int t5h_residual_encode_device(const float* d_emb, int32_t N, const float* d_centers, int32_t K,
                               const uint32_t* d_assign, int32_t D, uint8_t* d_codes, uint32_t* d_bad, void* stream) {
  int rc;
  if ((rc = check_codes(N, D, 8))) return rc;
  if (K <= 0 && N > 0) return fail(T5H_ERR_INVALID, "no centres");
  if (N > 0 && (!d_emb || !d_centers || !d_assign || !d_codes || !d_bad)) return fail(T5H_ERR_INVALID, "NULL buffer");
  HIP_OK(t5k::launch_residual_encode(d_emb, d_centers, d_assign, N, D, K, codec().ladder, d_codes, d_bad,
                                     (hipStream_t)stream));
  return T5H_OK;
}

int t5h_residual_encode(int32_t hip_device, const float* emb, int32_t N, const float* centers, int32_t K,
                        const uint32_t* assign, int32_t D, uint8_t* codes) {
  int rc;
  if ((rc = check_codes(N, D, 8))) return rc;
  if (N == 0) return T5H_OK;
  if (K <= 0) return fail(T5H_ERR_INVALID, "no centres");
  if (!emb || !centers || !assign || !codes) return fail(T5H_ERR_INVALID, "NULL buffer");
  for (int32_t i = 0; i < N; i++)
    if (assign[i] >= (uint32_t)K)
      return fail(T5H_ERR_INVALID, "assignment " + std::to_string(assign[i]) + " of row " + std::to_string(i) +
                                       " is not a centre index");
  if ((rc = set_device(hip_device))) return rc;
  const size_t e_b = pad256((size_t)N * D * 4), c_b = pad256((size_t)K * D * 4), a_b = pad256((size_t)N * 4);
  const size_t o_b = pad256((size_t)N * D / 2);
  DevBuf d;
  if (hipMalloc((void**)&d.p, e_b + c_b + a_b + o_b + 256) != hipSuccess) return fail(T5H_ERR_NOMEM, "codec buffers");
  char *de = d.p, *dc = de + e_b, *da = dc + c_b, *dout = da + a_b, *dbad = dout + o_b;
  HIP_OK(hipMemcpy(de, emb, (size_t)N * D * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dc, centers, (size_t)K * D * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(da, assign, (size_t)N * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemset(dbad, 0, 4));
  HIP_OK(t5k::launch_residual_encode((const float*)de, (const float*)dc, (const uint32_t*)da, N, D, K, codec().ladder,
                                     (uint8_t*)dout, (unsigned*)dbad, nullptr));
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(codes, dout, (size_t)N * D / 2, hipMemcpyDeviceToHost));
  return T5H_OK;
}

int t5h_residual_decode_device(const uint8_t* d_codes, int32_t N, int32_t D, float* d_out, void* stream) {
  int rc;
  if ((rc = check_codes(N, D, 2))) return rc;
  if (N > 0 && (!d_codes || !d_out)) return fail(T5H_ERR_INVALID, "NULL buffer");
  HIP_OK(t5k::launch_residual_decode(d_codes, (size_t)N * D / 2, codec().table, d_out, (hipStream_t)stream));
  return T5H_OK;
}

int t5h_residual_decode(int32_t hip_device, const uint8_t* codes, int32_t N, int32_t D, float* out) {
  int rc;
  if ((rc = check_codes(N, D, 2))) return rc;
  if (N == 0) return T5H_OK;
  if (!codes || !out) return fail(T5H_ERR_INVALID, "NULL buffer");
  if ((rc = set_device(hip_device))) return rc;
  const size_t c_b = pad256((size_t)N * D / 2), o_b = (size_t)N * D * 4;
  DevBuf d;
  if (hipMalloc((void**)&d.p, c_b + o_b) != hipSuccess) return fail(T5H_ERR_NOMEM, "codec buffers");
  HIP_OK(hipMemcpy(d.p, codes, (size_t)N * D / 2, hipMemcpyHostToDevice));
  HIP_OK(t5k::launch_residual_decode((const uint8_t*)d.p, (size_t)N * D / 2, codec().table, (float*)(d.p + c_b),
                                     nullptr));
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(out, d.p + c_b, o_b, hipMemcpyDeviceToHost));
  return T5H_OK;
}

int t5h_matmul_t_q4_device(const float* d_a, int32_t M, const uint8_t* d_codes, int32_t N, int32_t D, float* d_c,
                           void* stream) {
  int rc;
  if (M < 0 || (rc = check_codes(N, D, 4))) return M < 0 ? fail(T5H_ERR_INVALID, "M < 0") : rc;
  if (M > 0 && N > 0 && (!d_a || !d_codes || !d_c)) return fail(T5H_ERR_INVALID, "NULL buffer");
  HIP_OK(t5k::launch_matmul_t_q4(d_a, d_codes, codec().table, d_c, M, N, D, (hipStream_t)stream));
  return T5H_OK;
}

int t5h_matmul_t_q4(int32_t hip_device, const float* a, int32_t M, const uint8_t* codes, int32_t N, int32_t D,
                    float* c) {
  int rc;
  if (M < 0 || (rc = check_codes(N, D, 4))) return M < 0 ? fail(T5H_ERR_INVALID, "M < 0") : rc;
  if (M == 0 || N == 0) return T5H_OK;
  if (!a || !codes || !c) return fail(T5H_ERR_INVALID, "NULL buffer");
  if ((rc = set_device(hip_device))) return rc;
  const size_t a_b = pad256((size_t)M * D * 4), k_b = pad256((size_t)N * D / 2), c_b = (size_t)M * N * 4;
  DevBuf d;
  if (hipMalloc((void**)&d.p, a_b + k_b + c_b) != hipSuccess) return fail(T5H_ERR_NOMEM, "scoring buffers");
  HIP_OK(hipMemcpy(d.p, a, (size_t)M * D * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d.p + a_b, codes, (size_t)N * D / 2, hipMemcpyHostToDevice));
  HIP_OK(t5k::launch_matmul_t_q4((const float*)d.p, (const uint8_t*)(d.p + a_b), codec().table,
                                 (float*)(d.p + a_b + k_b), M, N, D, nullptr));
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(c, d.p + a_b + k_b, c_b, hipMemcpyDeviceToHost));
  return T5H_OK;
}

}  // extern "C"
