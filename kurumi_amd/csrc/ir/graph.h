// The kurumi primitive IR, restated in C++: an append-only arena of nodes, each an
// `Op` over earlier nodes with its dtype and shape inferred and stored at record time.
//
// Follows kurumi_core/src/graph.rs:29-112 (arena, process-unique graph id),
// graph/op.rs:12-127 (the closed op set), graph/infer.rs:10-134 (dtype/shape
// inference) and graph/check.rs:8-59 (record-time guards). Builders throw
// `ku::Error` on a record-time error; the C ABI turns that into KU_ERR + last error.
#pragma once
#include <atomic>
#include <cstdint>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "dtype.h"

namespace ku {

using NodeId = uint32_t;
using Shape = std::vector<size_t>;

struct Error : std::runtime_error {
  explicit Error(const std::string& m) : std::runtime_error(m) {}
};

// Closed primitive set (graph/op.rs:12-100). Ops outside the device backend's scope
// are still recordable so that a graph built elsewhere can be inspected; the device
// backend rejects them with an error at eval.
enum class OpKind : uint32_t {
  Const, Input, Iota, RandUniform, Cast, Bitcast, Detach,
  Add, Mul, Max, Neg, IDiv, And, Or, Xor, Shl, Shr, CmpLt, CmpEq, Where,
  Recip, Sqrt, Exp2, Log2, Sin, Floor,
  Sum, Prod, ReduceMax, ArgReduce,
  Softmax, RmsNorm, Sdpa,
  Reshape, Permute, Expand, Slice, Flip, Pad,
  DotGeneral,
  QuantMatmul,
  NumKinds
};
const char* op_name(OpKind k);

enum class ArgKind : uint32_t { Max = 0, Min = 1 };

struct SliceRange { size_t start, end, step; };
struct PadRange { size_t lo, hi; };

struct Op {
  OpKind kind = OpKind::Const;
  DType to = DType::F32;          // Cast/Bitcast target; Input/Iota dtype
  Shape shape;                    // Const/Input/Iota/RandUniform/Reshape/Expand
  std::vector<size_t> perm;       // Permute
  std::vector<size_t> axes;       // Flip
  size_t axis = 0;                // reductions, Softmax, RmsNorm, Iota
  ArgKind arg = ArgKind::Max;     // ArgReduce
  bool causal = false;            // Sdpa
  float eps = 0.f;                // RmsNorm
  std::vector<SliceRange> ranges; // Slice
  std::vector<PadRange> pads;     // Pad
  std::vector<size_t> lc, rc, lb, rb;  // DotGeneral: lhs/rhs contract, lhs/rhs batch
  int qbits = 0;                  // QuantMatmul: 2, 4 or 8
  size_t qgroup = 0;              // QuantMatmul: K columns per scale group
  bool qsym = true;               // QuantMatmul: no per-group min
  std::shared_ptr<const std::vector<uint8_t>> data;  // Const payload, little-endian
  DType data_dtype = DType::F32;                     // Const payload dtype
};

struct Node {
  Op op;
  DType dtype;
  std::vector<NodeId> src;
  Shape shape;
};

inline size_t numel(const Shape& s) {
  size_t n = 1;
  for (size_t d : s) n *= d;
  return n;
}
std::vector<size_t> row_major_strides(const Shape& s);
std::vector<size_t> free_axes(size_t rank, const std::vector<size_t>& batch, const std::vector<size_t>& contract);
std::string shape_str(const Shape& s);

class Graph {
 public:
  Graph();
  uint64_t id() const { return id_; }
  size_t size() const { return nodes_.size(); }
  const Node& node(NodeId i) const;
  DType dtype(NodeId i) const { return node(i).dtype; }
  const Shape& shape(NodeId i) const { return node(i).shape; }

  // leaves (graph.rs:74-100)
  NodeId constant_bytes(DType dt, const uint8_t* bytes, size_t nbytes, const Shape& shape);
  NodeId constant_f32(const std::vector<float>& v, const Shape& shape);
  NodeId input(const Shape& shape, DType dt);
  NodeId iota(const Shape& shape, size_t axis, DType dt);
  NodeId rand_uniform(const Shape& shape, uint64_t seed);
  NodeId rand_uniform_seeded(const Shape& shape, NodeId seed);  // seed: any one-element node
  NodeId cast(NodeId a, DType to);
  NodeId bitcast(NodeId a, DType to);
  NodeId detach(NodeId a);
  NodeId scalar(NodeId like, float v);  // elementwise.rs:83-94

  // elementwise primitives (elementwise.rs:9-80)
  NodeId add(NodeId a, NodeId b);
  NodeId mul(NodeId a, NodeId b);
  NodeId max(NodeId a, NodeId b);
  NodeId neg(NodeId a);
  NodeId recip(NodeId a);
  NodeId sqrt(NodeId a);
  NodeId exp2(NodeId a);
  NodeId log2(NodeId a);
  NodeId sin(NodeId a);
  NodeId floor(NodeId a);
  NodeId idiv(NodeId a, NodeId b);
  NodeId bit_and(NodeId a, NodeId b);
  NodeId bit_or(NodeId a, NodeId b);
  NodeId bit_xor(NodeId a, NodeId b);
  NodeId shl(NodeId a, NodeId b);
  NodeId shr(NodeId a, NodeId b);
  NodeId cmp_lt(NodeId a, NodeId b);
  NodeId cmp_eq(NodeId a, NodeId b);
  NodeId where(NodeId c, NodeId a, NodeId b);

  // decompositions used by the hot-path graphs
  NodeId sub(NodeId a, NodeId b);   // elementwise.rs:104-107
  NodeId div(NodeId a, NodeId b);   // elementwise.rs:109-112
  NodeId exp(NodeId a);             // explog.rs:9-13
  NodeId ln(NodeId a);              // explog.rs:16-20
  NodeId relu(NodeId a);            // activation.rs:17-20
  NodeId sign(NodeId a);            // elementwise.rs:126-135
  NodeId ceil(NodeId a);            // elementwise.rs:164-168
  NodeId round(NodeId a);           // elementwise.rs:171-175 (floor(x + 0.5))
  NodeId square(NodeId a);
  NodeId cos(NodeId a);             // trig.rs: sin(x + pi/2)
  NodeId tanh(NodeId a);            // trig.rs:50-58: 2*sigmoid(2x) - 1
  NodeId sigmoid(NodeId a);         // activation.rs:8-14
  NodeId silu(NodeId a);            // activation.rs:23-26
  NodeId gelu(NodeId a);            // activation.rs:29-44 (tanh form)
  NodeId rope(NodeId a);            // attention.rs:9-36 (NeoX rotate-half, base 10000)
  NodeId randn(const Shape& shape, uint64_t seed);                    // random.rs:28-40
  NodeId rand_range(const Shape& shape, uint64_t seed, float lo, float hi);  // random.rs:43-49
  NodeId mean(NodeId a, size_t axis);
  NodeId reduce_min(NodeId a, size_t axis);   // reduce.rs:54-58
  NodeId logsumexp(NodeId a, size_t axis);    // reduce.rs:115-124
  NodeId log_softmax(NodeId a, size_t axis);  // activation.rs:132-137

  // reductions (reduce.rs:8-43)
  NodeId sum(NodeId a, size_t axis);
  NodeId prod(NodeId a, size_t axis);
  NodeId reduce_max(NodeId a, size_t axis);
  NodeId argreduce(NodeId a, size_t axis, ArgKind k);
  NodeId broadcast_back(NodeId reduced, const Shape& full, size_t axis);

  // nn (activation.rs:122-129, attention.rs:78-153)
  NodeId softmax(NodeId a, size_t axis);
  NodeId rmsnorm(NodeId a, size_t axis, float eps);
  NodeId sdpa(NodeId q, NodeId k, NodeId v, bool causal);
  NodeId sdpa_decomposed(NodeId q, NodeId k, NodeId v, bool causal);
  NodeId sdpa_fused(NodeId q, NodeId k, NodeId v, bool causal);

  // movement (movement/view.rs:9-114)
  NodeId reshape(NodeId a, const Shape& s);
  NodeId permute(NodeId a, const std::vector<size_t>& perm);
  NodeId expand(NodeId a, const Shape& s);
  NodeId broadcast_to(NodeId a, const Shape& s);
  NodeId transpose(NodeId a, size_t i, size_t j);
  NodeId slice(NodeId a, const std::vector<SliceRange>& r);
  NodeId flip(NodeId a, const std::vector<size_t>& axes);
  NodeId pad(NodeId a, const std::vector<PadRange>& p);

  // contraction (contract.rs:13-46)
  NodeId dot_general(NodeId a, NodeId b, const std::vector<size_t>& lc, const std::vector<size_t>& rc,
                     const std::vector<size_t>& lb, const std::vector<size_t>& rb);
  NodeId matmul(NodeId a, NodeId b);
  // weight-only quantized matmul (graph/ops/core/contract.rs:49-115): act [M, K] float x
  // dequant(qweight [N, K*bits/8] U8)^T -> [M, N] in act's dtype; scales / mins F16 [N, K/group].
  // `mins` = KU_ERR-like `kNoNode` for the symmetric form.
  NodeId quant_matmul(NodeId act, NodeId qweight, NodeId scales, NodeId mins, int bits, size_t group_size);
  static constexpr NodeId kNoNode = 0xFFFFFFFFu;

  // raw append with inference (used by passes)
  NodeId push(Op op, std::vector<NodeId> src);

 private:
  void check_id(const char* op, NodeId a) const;
  void same_shape(const char* op, NodeId a, NodeId b) const;
  void same_dtype(const char* op, NodeId a, NodeId b) const;
  void require(const char* op, NodeId a, bool ok, const char* want) const;
  void reduce_axis_ok(const char* op, NodeId a, size_t axis) const;
  DType infer_dtype(const Op& op, const std::vector<NodeId>& src) const;
  Shape derive_shape(const Op& op, const std::vector<NodeId>& src) const;
  NodeId causal_bias(size_t s, const Shape& out_shape);
  NodeId concat_last(NodeId a, NodeId b, size_t alen);
  NodeId slice_last(NodeId a, size_t start, size_t end);
  NodeId broadcast_2d_to(NodeId t, const Shape& target);

  std::vector<Node> nodes_;
  uint64_t id_;
};

// inspection (graph/inspect.rs:10-55)
std::vector<NodeId> reachable_multi(const Graph& g, const std::vector<NodeId>& roots);
std::string dump(const Graph& g, NodeId root);

// The reference's mixed-precision pass (graph/pass/amp.rs:16-40): f32 DotGenerals run in f16
// (operands cast down, result cast back up). Returns the new root.
NodeId amp(Graph& g, NodeId root);

// The build's fp8 mixed-precision pass: rewrites an f32/bf16 `DotGeneral` whose rhs is a
// constant weight into an e4m3 contraction with a per-row weight scale and a per-tensor
// activation scale. Returns the new root. (The reference's `amp` pass, graph/pass/amp.rs:16-40,
// only knows f16; this is the e4m3 policy for the quantized-linear workload.)
NodeId amp_fp8(Graph& g, NodeId root);

}  // namespace ku
