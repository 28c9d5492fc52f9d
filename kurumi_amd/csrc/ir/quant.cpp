// Host weight quantizer (kurumi_core/src/quant.rs:43-91): the f16 rounding of scales and mins
// is part of the format, so the quantized values are computed against the rounded scale.
#include "quant.h"

#include <cmath>

#include "dtype.h"
#include "graph.h"

namespace ku {

namespace {
void put_field(std::vector<uint8_t>& packed, size_t row_bytes, size_t r, size_t c, int bits, uint32_t v) {
  const size_t per = 8 / bits;
  const size_t i = r * row_bytes + c / per;
  const int shift = (int)(c % per) * bits;
  const uint32_t mask = (1u << bits) - 1;
  packed[i] = (uint8_t)((packed[i] & ~(mask << shift)) | ((v & mask) << shift));
}
float f16_value(uint16_t h) { return (float)f16_to_f64(h); }
}  // namespace

Quantized quantize(const float* w, size_t rows, size_t cols, int bits, size_t group_size, bool symmetric) {
  if (!(bits == 2 || bits == 4 || bits == 8)) throw Error("quantize: bits must be 2, 4, or 8");
  if (group_size == 0 || cols % group_size != 0) throw Error("quantize: cols must be a multiple of group_size");
  const size_t ng = cols / group_size, rb = cols * bits / 8;
  Quantized q;
  q.packed.assign(rows * rb, 0);
  q.scales.assign(rows * ng, 0);
  if (!symmetric) q.mins.assign(rows * ng, 0);
  for (size_t r = 0; r < rows; ++r)
    for (size_t g = 0; g < ng; ++g) {
      const float* grp = w + r * cols + g * group_size;
      const size_t si = r * ng + g;
      if (symmetric) {
        // signed range [-2^(bits-1), 2^(bits-1) - 1]; NaN-ignoring max like f32::max
        float amax = 0.f;
        for (size_t i = 0; i < group_size; ++i) amax = std::fmax(amax, std::fabs(grp[i]));
        const int qlo = -(1 << (bits - 1)), qhi = (1 << (bits - 1)) - 1;
        const uint16_t s = f64_to_f16(amax > 0.f ? (double)(amax / (float)qhi) : 1.0);
        q.scales[si] = s;
        const float sv = f16_value(s);
        for (size_t i = 0; i < group_size; ++i) {
          // round half away from zero (f32::round), clamp, then to i32 (a NaN stays NaN through
          // the clamp and converts to 0)
          const float t = std::round(grp[i] / sv);
          const int qv = t != t ? 0 : (int)std::fmin(std::fmax(t, (float)qlo), (float)qhi);
          put_field(q.packed, rb, r, g * group_size + i, bits, (uint32_t)qv);
        }
      } else {
        float mn = INFINITY, mx = -INFINITY;
        for (size_t i = 0; i < group_size; ++i) {
          mn = std::fmin(mn, grp[i]);
          mx = std::fmax(mx, grp[i]);
        }
        const float qmax = (float)((1u << bits) - 1);
        const uint16_t s = f64_to_f16(mx > mn ? (double)((mx - mn) / qmax) : 1.0);
        const uint16_t m = f64_to_f16((double)mn);
        q.scales[si] = s;
        q.mins[si] = m;
        const float sv = f16_value(s), mv = f16_value(m);
        for (size_t i = 0; i < group_size; ++i) {
          const float t = std::round((grp[i] - mv) / sv);
          const uint32_t qv = t != t ? 0u : (uint32_t)std::fmin(std::fmax(t, 0.f), qmax);
          put_field(q.packed, rb, r, g * group_size + i, bits, qv);
        }
      }
    }
  return q;
}

}  // namespace ku
