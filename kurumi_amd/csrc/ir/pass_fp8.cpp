// fp8 (OCP e4m3) mixed-precision pass for linear layers.
//
// The reference's mixed-precision pass (kurumi_core/src/graph/pass/amp.rs:16-40) rewrites
// f32 matmuls to f16 only; an f8 `DotGeneral` in the reference would round its *output*
// to f8 (interp/contract.rs:57-64). This pass is the e4m3 policy of the quantized-linear
// workload: a `DotGeneral(x, w; lc=[1], rc=[1])` with a 2-D floating x and weight w becomes
//
//   sx = reduce_max(reduce_max(|x|, 1), 0) * (1/448)        (per-tensor, in-graph)
//   xq = cast_e4m3(x * (1/sx))       (1/1 when sx = 0: an all-zero x gives xq = 0 and y = 0)
//   sw[n] = max_k |w[n,k]| / 448, wq = cast_e4m3(w / sw[n])  (per row; host-side when w is a Const,
//                                                            from the stored f32 weight)
//   y  = cast_out( dot(cast_f32(xq), cast_f32(wq)) * sx * sw[n] )
//
// whose device lowering is one fp8 MFMA GEMM with the scales in its epilogue. The
// dequantised value of every product is exact in f32, so the oracle interprets the
// rewritten graph with plain f32 arithmetic.
#include <cmath>
#include <cstring>
#include <unordered_map>

#include "graph.h"

namespace {
// a / 448 in the graph's terms: div(a, b) is mul(a, recip(b)), and recip of the constant 448 is
// the correctly rounded f32 1/448, so multiplying by this constant is the same value bit for bit
// (and needs no device work to divide a constant)
constexpr float kInv448 = 1.0f / 448.0f;
}  // namespace

namespace ku {

namespace {

// 1 / s where s > 0, else 1 / 1: an all-zero tensor (scale 0) then quantises to zeros, and its
// product to zeros, instead of 0 * (1/0) = NaN.
NodeId guarded_recip(Graph& g, NodeId s) {
  NodeId pos = g.cmp_lt(g.scalar(s, 0.f), s);
  return g.recip(g.where(pos, s, g.scalar(s, 1.f)));
}

double load_as_f64(DType dt, const uint8_t* p) {
  switch (dt) {
    case DType::F32: { float f; std::memcpy(&f, p, 4); return f; }
    case DType::F64: { double d; std::memcpy(&d, p, 8); return d; }
    case DType::BF16: { uint16_t h; std::memcpy(&h, p, 2); return bf16_to_f32(h); }
    case DType::F16: { uint16_t h; std::memcpy(&h, p, 2); return f16_to_f64(h); }
    default: throw Error("amp_fp8: weight dtype must be a float");
  }
}

bool is_linear(const Graph& g, NodeId id) {
  const Node& n = g.node(id);
  if (n.op.kind != OpKind::DotGeneral) return false;
  if (n.op.lc != std::vector<size_t>{1} || n.op.rc != std::vector<size_t>{1} || !n.op.lb.empty()) return false;
  if (g.shape(n.src[0]).size() != 2 || g.shape(n.src[1]).size() != 2) return false;
  DType d = n.dtype;
  return d == DType::F32 || d == DType::BF16 || d == DType::F16;
}

}  // namespace

// Host values of a constant weight: a float Const, or a Cast{f32|bf16|f16} of one. A narrowing
// cast is looked through: the e4m3 policy quantizes the stored weight itself (one rounding,
// straight to e4m3 with its per-row scale) rather than a 16-bit rounding of it, which would
// round twice. False for anything else.
bool const_weight_f32(const Graph& g, NodeId w, std::vector<float>* out) {
  const Node& n = g.node(w);
  const Node* c = &n;
  if (n.op.kind == OpKind::Cast) {
    DType to = n.op.to;
    if (to != DType::F32 && to != DType::BF16 && to != DType::F16) return false;
    c = &g.node(n.src[0]);
  }
  if (c->op.kind != OpKind::Const) return false;
  DType dt = c->op.data_dtype;
  if (!(dt == DType::F32 || dt == DType::F64 || dt == DType::BF16 || dt == DType::F16)) return false;
  size_t cnt = numel(c->op.shape), wd = dt_width(dt);
  const uint8_t* p = c->op.data->data();
  out->resize(cnt);
  for (size_t i = 0; i < cnt; ++i) (*out)[i] = static_cast<float>(load_as_f64(dt, p + i * wd));
  return true;
}

// Quantize a row-major [rows, cols] weight per row: sw[r] = max|w[r,:]| / 448 (f32),
// wq = e4m3(w / sw[r]) with round-to-nearest-even. Rows of zeros get sw = 1.
void quantize_rows_e4m3(const std::vector<float>& w, size_t rows, size_t cols, std::vector<uint8_t>* wq,
                        std::vector<float>* sw) {
  wq->resize(rows * cols);
  sw->resize(rows);
  for (size_t r = 0; r < rows; ++r) {
    float mx = 0.f;
    for (size_t c = 0; c < cols; ++c) mx = std::fmax(mx, std::fabs(w[r * cols + c]));
    float s = mx / 448.0f;
    if (!(s > 0.f) || !std::isfinite(s)) s = 1.0f;
    (*sw)[r] = s;
    for (size_t c = 0; c < cols; ++c) (*wq)[r * cols + c] = f32_to_f8e4m3(w[r * cols + c] / s);
  }
}

NodeId amp_fp8(Graph& g, NodeId root) {
  std::vector<NodeId> order = reachable_multi(g, {root});
  std::unordered_map<NodeId, NodeId> remap;
  auto R = [&](NodeId x) {
    auto it = remap.find(x);
    return it == remap.end() ? x : it->second;
  };
  for (NodeId id : order) {
    Node n = g.node(id);  // copy: g grows below
    bool changed = false;
    for (NodeId& s : n.src)
      if (R(s) != s) { s = R(s); changed = true; }
    if (is_linear(g, id)) {
      NodeId x = n.src[0], w = n.src[1];
      const Shape xs = g.shape(x), ws = g.shape(w);
      size_t M = xs[0], K = xs[1], N = ws[0];
      DType out = n.dtype;
      // weight: host quantization for constants, in-graph otherwise
      NodeId wq_node, sw_node;
      std::vector<float> wv;
      if (const_weight_f32(g, w, &wv)) {
        std::vector<uint8_t> wq;
        std::vector<float> sw;
        quantize_rows_e4m3(wv, N, K, &wq, &sw);
        wq_node = g.constant_bytes(DType::F8E4M3, wq.data(), wq.size(), {N, K});
        sw_node = g.constant_f32(sw, {N});
      } else {
        NodeId wf = g.dtype(w) == DType::F32 ? w : g.cast(w, DType::F32);
        NodeId wa = g.max(wf, g.neg(wf));
        NodeId wm = g.reduce_max(wa, 1);
        sw_node = g.mul(wm, g.scalar(wm, kInv448));
        NodeId inv = guarded_recip(g, sw_node);
        NodeId invb = g.broadcast_back(inv, {N, K}, 1);
        wq_node = g.cast(g.mul(wf, invb), DType::F8E4M3);
      }
      // activation: per-tensor absmax scale, in-graph
      NodeId xf = g.dtype(x) == DType::F32 ? x : g.cast(x, DType::F32);
      NodeId xa = g.max(xf, g.neg(xf));
      NodeId rm = g.reduce_max(xa, 1);
      NodeId am = g.reduce_max(rm, 0);
      NodeId sx = g.mul(am, g.scalar(am, kInv448));
      NodeId inv = guarded_recip(g, sx);
      NodeId invb = g.expand(g.reshape(inv, {1, 1}), {M, K});
      // The quantisation gets its own cast of x: the absmax pass and the quantise pass then each
      // read x in its own (16-bit) storage, instead of sharing an f32 copy written to HBM.
      NodeId xf2 = g.dtype(x) == DType::F32 ? x : g.cast(x, DType::F32);
      NodeId xq = g.cast(g.mul(xf2, invb), DType::F8E4M3);
      NodeId d = g.dot_general(g.cast(xq, DType::F32), g.cast(wq_node, DType::F32), {1}, {1}, {}, {});
      NodeId y1 = g.mul(d, g.expand(g.reshape(sx, {1, 1}), {M, N}));
      NodeId y2 = g.mul(y1, g.expand(g.reshape(sw_node, {1, N}), {M, N}));
      NodeId y = g.cast(y2, out);
      remap[id] = y;
      continue;
    }
    if (changed) remap[id] = g.push(n.op, n.src);
  }
  return R(root);
}

}  // namespace ku
