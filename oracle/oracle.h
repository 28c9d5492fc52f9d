// TEST INFRASTRUCTURE — not part of the product.
//
// CPU restatement of kurumi's reference interpreter (the oracle every backend is checked
// against, kurumi_core/src/interp.rs:23-112) and of its view-fused CPU evaluator
// (kurumi_core/src/realize*.rs), for the ops on the kurumi_hip hot path. Only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg load it, and only to check or to
// time a CPU baseline; libkurumi_hip never links it.
//
// Pinning (each restated function is checked by something a plausible mistake would fail):
//   - threefry2x32 / uniform: the reference KATs (rng.rs:67-74) + the Random123 vector.
//   - bf16 / f16 rounding: half-crate cases from tests/dtype.rs:102-127 and exhaustive
//     round trips; f16 also against numpy's float16 casts.
//   - e4m3 / e5m2 rounding: the reference's representable round trips
//     (tests/cpu_completeness.rs:60-85); general values are checked against an independent
//     brute-force nearest-value search (the float8 crate's tie/overflow behaviour is not in
//     the container: parity unpinned beyond OCP OFP8 RNE + saturate).
//   - elementwise/reduce/argmax/softmax/sdpa/dot: known answers from tests/engine.rs and
//     tests/ops.rs, numpy on small inputs, brute-force argmax, closed forms.
//   - f32 2D GEMM summation order (gemm 0.19 crate): parity unpinned, tolerance only.
#pragma once
#include <cstddef>
#include <cstdint>

#include "../kurumi_amd/csrc/capi/handles.h"

namespace kuo {

// conversions (oracle-owned implementations)
uint16_t f32_to_bf16(float f);
float bf16_to_f32(uint16_t h);
uint16_t f64_to_f16(double x);
double f16_to_f64(uint16_t h);
uint16_t f64_to_bf16(double x);
uint8_t f32_to_e4m3(float x);
double e4m3_to_f64(uint8_t b);
uint8_t f32_to_e5m2(float x);
double e5m2_to_f64(uint8_t b);

uint64_t threefry2x32(uint64_t key, uint64_t counter);
float uniform_f32(uint64_t bits);

ku::Tensor cast(const ku::Tensor& t, ku::DType to);
std::vector<ku::Tensor> interpret(const ku::Graph& g, const std::vector<ku::NodeId>& roots, const ku::Feeds& feeds);
// view-fused f32 evaluator; returns false (and leaves `out` untouched) when the graph leaves
// the f32 fused path, like realize::force's fallback gate (realize/eval.rs:62-103).
bool realize(const ku::Graph& g, ku::NodeId root, const ku::Feeds& feeds, ku::Tensor* out, int* passes);

}  // namespace kuo
