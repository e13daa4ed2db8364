// quantize.cpp -- f32 rows -> GGML Q4_K super-blocks on the host: the weight-quantization step
// of the reference's quantize tool.
//
// Reference: tools/quantize-tool/src/main.rs:12-24 quantizes every rank-2 tensor whose second
// dimension is a multiple of 256 with candle's `QTensor::quantize(_, GgmlDType::Q4K)` (candle-core
// at git rev 0.9.2-alpha.2, a third-party dependency absent from the reference tree).  That
// is `BlockQ4K::from_float`, candle's port of GGML's `quantize_row_q4_K_reference` as published
// with `make_qkx1_quants` (k_quants.c), restated here:
//
//   per 32-value sub-block j: (scale_j, min_j) from an alternating least-squares search,
//     min0 = min(x, 0), iscale = 15 / (max - min0); up to 5 rounds of
//       l_i = clamp(round(iscale (x_i - min)), 0, 15)
//       scale = sum (x_i - min) l_i / sum l_i^2        (f32 running sum, integer sum l^2)
//       min = min(sum (x_i - scale l_i) / 32, 0)       (f32 running sum)
//       iscale = 1 / scale
//     stopping after the round in which no l_i changed; a constant sub-block gives (0, 0);
//   d = f16(max_j scale_j / 63), dmin = f16(max_j (-min_j) / 63);
//   6-bit sc_j = min(round(63 / max_scale * scale_j), 63), m_j likewise from the mins,
//     packed as get_scale_min_k4 unpacks them;
//   q_i = clamp(round((x_i + dmin m_j) / (d sc_j)), 0, 15) (0 when d sc_j == 0),
//     qs[32 c + l] = q[64 c + l] | q[64 c + 32 + l] << 4.
//
// round() is candle's nearest_int, f32::round: halves away from zero (GGML's C version rounds
// halves to even; the two differ only on exact ties).  All arithmetic is f32 in the order
// written, without contraction into fused multiply-adds, as the Rust code evaluates it.
#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "../../include/t5hip.h"

#pragma clang fp contract(off)

namespace t5h_detail {
int fail(int code, const std::string& msg);
}

namespace {

constexpr int QK = 256, BLK = 144;

// f32::round() as i32: halves away from zero, saturating at the i32 range (NaN -> 0).
inline int nearest_int(float v) {
  const float r = std::round(v);
  if (!(r == r)) return 0;
  if (r >= 2147483648.0f) return INT_MAX;
  if (r <= -2147483648.0f) return INT_MIN;
  return (int)r;
}

// make_qkx1_quants(nmax = 15, ntry = 5) over 32 values -> (scale, -min).
void qkx1(const float* x, float& scale_out, float& min_out) {
  float mn = x[0], mx = x[0];
  for (int i = 1; i < 32; i++) {
    mn = std::min(mn, x[i]);
    mx = std::max(mx, x[i]);
  }
  if (mx == mn) {
    scale_out = 0.f;
    min_out = 0.f;
    return;
  }
  if (mn > 0.f) mn = 0.f;
  float iscale = 15.f / (mx - mn);
  float scale = 1.f / iscale;
  unsigned char L[32] = {};
  for (int it = 0; it < 5; it++) {
    float sumlx = 0.f;
    int suml2 = 0;
    bool changed = false;
    for (int i = 0; i < 32; i++) {
      const int l = std::min(15, std::max(0, nearest_int(iscale * (x[i] - mn))));
      if (l != L[i]) {
        L[i] = (unsigned char)l;
        changed = true;
      }
      sumlx += (x[i] - mn) * (float)l;
      suml2 += l * l;
    }
    scale = sumlx / (float)suml2;
    float sum = 0.f;
    for (int i = 0; i < 32; i++) sum += x[i] - scale * (float)L[i];
    mn = sum / 32.f;
    if (mn > 0.f) mn = 0.f;
    iscale = 1.f / scale;
    if (!changed) break;
  }
  scale_out = scale;
  min_out = -mn;
}

inline void store_f16(uint8_t* p, float v) {
  const _Float16 h = (_Float16)v;  // round to nearest even
  memcpy(p, &h, 2);
}
inline float load_f16(const uint8_t* p) {
  _Float16 h;
  memcpy(&h, p, 2);
  return (float)h;
}

void quantize_block(const float* x, uint8_t* b) {
  float scales[8], mins[8];
  for (int j = 0; j < 8; j++) qkx1(x + 32 * j, scales[j], mins[j]);
  float max_scale = 0.f, max_min = 0.f;
  for (int j = 0; j < 8; j++) {
    max_scale = std::max(scales[j], max_scale);
    max_min = std::max(mins[j], max_min);
  }
  const float inv_scale = max_scale > 0.f ? 63.f / max_scale : 0.f;
  const float inv_min = max_min > 0.f ? 63.f / max_min : 0.f;
  uint8_t* sc = b + 4;
  memset(sc, 0, 12);
  int ls[8], lm[8];
  for (int j = 0; j < 8; j++) {
    ls[j] = std::min(nearest_int(inv_scale * scales[j]), 63) & 63;
    lm[j] = std::min(nearest_int(inv_min * mins[j]), 63) & 63;
  }
  // get_scale_min_k4 layout: bytes 0-3 sc_0..3 (+ high bits of sc_4..7), 4-7 m_0..3 (+ high
  // bits of m_4..7), 8-11 low nibbles of sc_4..7 | m_4..7 << 4.
  for (int j = 0; j < 4; j++) {
    sc[j] = (uint8_t)(ls[j] | ((ls[j + 4] >> 4) << 6));
    sc[j + 4] = (uint8_t)(lm[j] | ((lm[j + 4] >> 4) << 6));
    sc[j + 8] = (uint8_t)((ls[j + 4] & 15) | ((lm[j + 4] & 15) << 4));
  }
  store_f16(b, max_scale / 63.f);
  store_f16(b + 2, max_min / 63.f);
  const float d = load_f16(b), dmin = load_f16(b + 2);
  uint8_t q[QK] = {};
  for (int j = 0; j < 8; j++) {
    const float dj = d * (float)ls[j];
    if (dj == 0.f) continue;
    const float dm = dmin * (float)lm[j];
    for (int i = 0; i < 32; i++) q[32 * j + i] = (uint8_t)std::min(15, std::max(0, nearest_int((x[32 * j + i] + dm) / dj)));
  }
  uint8_t* qs = b + 16;
  for (int c = 0; c < 4; c++)
    for (int l = 0; l < 32; l++) qs[32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
}

}  // namespace

extern "C" int t5h_quantize_q4k(const float* x, int64_t n_values, uint8_t* out, int32_t threads) {
  if (n_values < 0 || n_values % QK)
    return t5h_detail::fail(T5H_ERR_INVALID, "quantize_q4k: the value count must be a multiple of 256");
  if (n_values == 0) return T5H_OK;
  if (!x || !out) return t5h_detail::fail(T5H_ERR_INVALID, "quantize_q4k: NULL buffer");
  const int64_t nblk = n_values / QK;
  int nt = threads > 0 ? threads : (int)std::min(16u, std::max(1u, std::thread::hardware_concurrency()));
  nt = (int)std::min<int64_t>(nt, (nblk + 1023) / 1024);
  auto run = [&](int64_t b0, int64_t b1) {
    for (int64_t b = b0; b < b1; b++) quantize_block(x + b * QK, out + b * BLK);
  };
  if (nt <= 1) {
    run(0, nblk);
    return T5H_OK;
  }
  std::vector<std::thread> pool;
  const int64_t per = (nblk + nt - 1) / nt;
  for (int t = 0; t < nt; t++) {
    const int64_t b0 = t * per, b1 = std::min(nblk, b0 + per);
    if (b0 < b1) pool.emplace_back(run, b0, b1);
  }
  for (auto& th : pool) th.join();
  return T5H_OK;
}
