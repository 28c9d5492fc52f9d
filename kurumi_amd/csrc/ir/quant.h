// Weight-only quantization on the host: an f32 [rows, cols] matrix to 2/4/8-bit fields along
// cols with one f16 scale (symmetric) or scale + min (asymmetric) per group of `group_size`
// columns, round to nearest. The layout ku_quant_matmul consumes: `packed` row-major with
// 8/bits fields per byte, low field first. Restates kurumi_core/src/quant.rs:43-91.
#pragma once
#include <cstddef>
#include <cstdint>
#include <vector>

namespace ku {

struct Quantized {
  std::vector<uint8_t> packed;    // rows * cols * bits / 8
  std::vector<uint16_t> scales;   // f16 bits, rows * cols / group_size
  std::vector<uint16_t> mins;     // f16 bits, empty when symmetric
};

// Throws ku::Error on bits not in {2, 4, 8} or cols not a multiple of group_size.
Quantized quantize(const float* w, size_t rows, size_t cols, int bits, size_t group_size, bool symmetric);

}  // namespace ku
