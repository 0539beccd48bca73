// Host-side weight quantizers of the .ill converter (CPU code, no GPU needed).
//
// q4: affine 4-bit per 64 columns, w ~ s * q + b with q in 0..15 and (s, b) stored as f16.
// Per group the quantizer tries clipped ranges [mn + a * range, mx - c * range] for a, c in
// {0, 0.03, 0.06, 0.1, 0.15}, refits (s, b) once by least squares on the codes of the
// clipped fit, rounds both to f16, re-derives the codes with the stored values, and keeps
// the candidate with the lowest squared error (the first one on ties). A group whose range
// is below 1e-12 stores zero codes, s = 0 and b = f16(mn). Semantics of quantGroup /
// quantizeQ4Raw, Sources/Engine/Convert.swift:286-370: float32 arithmetic in the same
// order, codes rounded half away from zero, f16 by round-to-nearest-even.
//
// q8: symmetric 8-bit per `group` columns (32 in the reference converter, 64 in BASELINE
// config 4), w ~ s * q with q in -127..127; s = f16(amax / 127), one f16 ulp larger when
// that would leave a code out of range (Convert.swift:252-282).
#pragma once
#include <stdint.h>

#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

namespace illq {

inline uint16_t f16_bits(float v) {
  const _Float16 h = (_Float16)v;
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}
inline float f16_value(uint16_t b) {
  _Float16 h;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;
}
// Codes of one value under (s, b) as stored: min(15, max(0, round((w - b) * inv))).
inline float q4_code(float w, float b, float inv) {
  return std::min(15.0f, std::max(0.0f, std::round((w - b) * inv)));
}

// One group of 64 weights -> 64 codes and the f16 bits of (scale, bias).
inline void quant_group_q4(const float* w, uint8_t* q_out, uint16_t* s_out, uint16_t* b_out) {
  static const float clips[5] = {0.0f, 0.03f, 0.06f, 0.1f, 0.15f};
  float mn = w[0], mx = w[0];
  for (int i = 1; i < 64; i++) {
    mn = std::min(mn, w[i]);
    mx = std::max(mx, w[i]);
  }
  if (mx - mn < 1e-12f) {
    for (int i = 0; i < 64; i++) q_out[i] = 0;
    *s_out = f16_bits(0.0f);
    *b_out = f16_bits(mn);
    return;
  }
  float best_err = INFINITY;
  uint16_t best_s = 0, best_b = 0;
  uint8_t q[64];
  const float range = mx - mn;
  for (float a : clips) {
    for (float c : clips) {
      const float lo = mn + a * range, hi = mx - c * range;
      if (hi <= lo) continue;
      float s = (hi - lo) / 15.0f, b = lo;
      for (int iter = 0; iter < 2; iter++) {
        const float inv = 1.0f / s;
        float sq = 0.f, sw = 0.f, sqq = 0.f, sqw = 0.f;
        for (int i = 0; i < 64; i++) {
          const float v = q4_code(w[i], b, inv);
          q[i] = (uint8_t)v;
          sq += v;
          sw += w[i];
          sqq += v * v;
          sqw += v * w[i];
        }
        if (iter == 1) break;
        const float den = 64.0f * sqq - sq * sq;
        if (den <= 0.f) break;
        const float s2 = (64.0f * sqw - sq * sw) / den;
        if (s2 <= 0.f) break;
        s = s2;
        b = (sw - s2 * sq) / 64.0f;
      }
      const uint16_t sh = f16_bits(s), bh = f16_bits(b);
      const float sf = f16_value(sh), bf = f16_value(bh);
      if (sf <= 0.f) continue;
      const float inv = 1.0f / sf;
      float err = 0.f;
      for (int i = 0; i < 64; i++) {
        const float v = q4_code(w[i], bf, inv);
        q[i] = (uint8_t)v;
        const float d = sf * v + bf - w[i];
        err += d * d;
      }
      if (err < best_err) {
        best_err = err;
        best_s = sh;
        best_b = bh;
        for (int i = 0; i < 64; i++) q_out[i] = q[i];
      }
    }
  }
  *s_out = best_s;
  *b_out = best_b;
}

// Rows [r0, r1) of a [rows][cols] matrix: packed codes [rows][cols / 2] (column 2j in the
// low nibble of byte j) and (scale, bias) f16 pairs [rows][cols / 64][2]. The code buffer
// lives per block of 64 rows, as in quantizeQ4Raw: a group for which no candidate has a
// positive f16 scale (ranges of about 1e-12 .. 5e-7) keeps the codes of the group before it
// in the block (s = b = 0 then, so they do not contribute).
inline void quant_rows_q4(const float* w, int64_t r0, int64_t r1, int cols, uint8_t* packed, uint16_t* sb) {
  const int groups = cols / 64;
  uint8_t q[64] = {};
  for (int64_t r = r0; r < r1; r++)
    for (int g = 0; g < groups; g++) {
      const int64_t base = r * cols + (int64_t)g * 64;
      uint16_t s, b;
      if (g == 0 && r % 64 == 0)
        for (int i = 0; i < 64; i++) q[i] = 0;
      quant_group_q4(w + base, q, &s, &b);
      sb[(r * groups + g) * 2] = s;
      sb[(r * groups + g) * 2 + 1] = b;
      for (int j = 0; j < 32; j++) packed[base / 2 + j] = (uint8_t)(q[2 * j] | (q[2 * j + 1] << 4));
    }
}

inline void quant_rows_q8(const float* w, int64_t r0, int64_t r1, int cols, int group, int8_t* codes, uint16_t* scales) {
  const int groups = cols / group;
  for (int64_t r = r0; r < r1; r++)
    for (int g = 0; g < groups; g++) {
      const int64_t base = r * cols + (int64_t)g * group;
      float amax = 0.f;
      for (int i = 0; i < group; i++) amax = std::max(amax, std::fabs(w[base + i]));
      uint16_t sh = f16_bits(amax / 127.0f);
      if (f16_value(sh) * 127.0f < amax) sh = (uint16_t)(sh + 1);
      const float s = f16_value(sh);
      scales[r * groups + g] = sh;
      const float inv = s > 0.f ? 1.0f / s : 0.f;
      for (int i = 0; i < group; i++)
        codes[base + i] = (int8_t)std::max(-127.0f, std::min(127.0f, std::round(w[base + i] * inv)));
    }
}

// Rows split over `threads` workers in blocks of whole 64-row units (the result does not
// depend on the split).
template <class F>
inline void parallel_rows(int64_t rows, int threads, F&& f) {
  threads = std::max(1, std::min<int>(threads, (int)std::min<int64_t>((rows + 63) / 64, 256)));
  if (threads == 1) {
    f(0, rows);
    return;
  }
  std::vector<std::thread> pool;
  const int64_t per = ((rows + threads - 1) / threads + 63) / 64 * 64;
  for (int t = 0; t < threads; t++) {
    const int64_t a = t * per, b = std::min(rows, a + per);
    if (a < b) pool.emplace_back([&f, a, b] { f(a, b); });
  }
  for (auto& th : pool) th.join();
}

}  // namespace illq
