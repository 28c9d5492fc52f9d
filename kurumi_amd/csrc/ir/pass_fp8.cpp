// fp8 (OCP e4m3) mixed-precision pass for linear layers.
//
// The reference's mixed-precision pass (kurumi_core/src/graph/pass/amp.rs:16-40) rewrites
// f32 matmuls to f16 only; an f8 `DotGeneral` in the reference would round its *output*
// to f8 (interp/contract.rs:57-64). This pass is the e4m3 policy of the quantized-linear
// workload: a `DotGeneral(x, w; lc=[1], rc=[1])` with a 2-D floating x and weight w becomes
//
//   sx = reduce_max(reduce_max(|x|, 1), 0) / 448            (per-tensor, in-graph)
//   xq = cast_e4m3(x * (1/sx))
//   sw[n] = max_k |w[n,k]| / 448, wq = cast_e4m3(w / sw[n])  (per row; host-side when w is a Const)
//   y  = cast_out( dot(cast_f32(xq), cast_f32(wq)) * sx * sw[n] )
//
// whose device lowering is one fp8 MFMA GEMM with the scales in its epilogue. The
// dequantised value of every product is exact in f32, so the oracle interprets the
// rewritten graph with plain f32 arithmetic.
#include <cmath>
#include <cstring>
#include <unordered_map>

#include "graph.h"

namespace ku {

namespace {

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

// Quantize a row-major [rows, cols] weight per row: sw[r] = max|w[r,:]| / 448 (f32),
// wq = e4m3(w / sw[r]) with round-to-nearest-even. Rows of zeros get sw = 1.
void quantize_rows_e4m3(const Graph& g, NodeId w, std::vector<uint8_t>* wq, std::vector<float>* sw) {
  const Node& n = g.node(w);
  size_t rows = n.shape[0], cols = n.shape[1];
  size_t wd = dt_width(n.op.data_dtype);
  const uint8_t* p = n.op.data->data();
  wq->resize(rows * cols);
  sw->resize(rows);
  for (size_t r = 0; r < rows; ++r) {
    float mx = 0.f;
    for (size_t c = 0; c < cols; ++c) mx = std::fmax(mx, std::fabs((float)load_as_f64(n.op.data_dtype, p + (r * cols + c) * wd)));
    float s = mx / 448.0f;
    if (!(s > 0.f) || !std::isfinite(s)) s = 1.0f;
    (*sw)[r] = s;
    for (size_t c = 0; c < cols; ++c) {
      float v = (float)load_as_f64(n.op.data_dtype, p + (r * cols + c) * wd);
      (*wq)[r * cols + c] = f32_to_f8e4m3(v / s);
    }
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
      const Node& wn = g.node(w);
      bool host_quant = wn.op.kind == OpKind::Const &&
                        (wn.op.data_dtype == DType::F32 || wn.op.data_dtype == DType::F64 ||
                         wn.op.data_dtype == DType::BF16 || wn.op.data_dtype == DType::F16);
      if (host_quant) {
        std::vector<uint8_t> wq;
        std::vector<float> sw;
        quantize_rows_e4m3(g, w, &wq, &sw);
        wq_node = g.constant_bytes(DType::F8E4M3, wq.data(), wq.size(), {N, K});
        sw_node = g.constant_f32(sw, {N});
      } else {
        NodeId wf = g.dtype(w) == DType::F32 ? w : g.cast(w, DType::F32);
        NodeId wa = g.max(wf, g.neg(wf));
        NodeId wm = g.reduce_max(wa, 1);
        NodeId c448 = g.scalar(wm, 448.0f);
        sw_node = g.div(wm, c448);
        NodeId inv = g.recip(sw_node);
        NodeId invb = g.broadcast_back(inv, {N, K}, 1);
        wq_node = g.cast(g.mul(wf, invb), DType::F8E4M3);
      }
      // activation: per-tensor absmax scale, in-graph
      NodeId xf = g.dtype(x) == DType::F32 ? x : g.cast(x, DType::F32);
      NodeId xa = g.max(xf, g.neg(xf));
      NodeId rm = g.reduce_max(xa, 1);
      NodeId am = g.reduce_max(rm, 0);
      NodeId c448 = g.scalar(am, 448.0f);
      NodeId sx = g.div(am, c448);
      NodeId inv = g.recip(sx);
      NodeId invb = g.expand(g.reshape(inv, {1, 1}), {M, K});
      NodeId xq = g.cast(g.mul(xf, invb), DType::F8E4M3);
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
