// The reference's mixed-precision pass, matmul-in-f16 (kurumi_core/src/graph/pass/amp.rs:16-40):
// every f32 DotGeneral reachable from `root` takes f16 casts of its operands, contracts in f16
// and is cast back to f32; every other node keeps its dtype. The walk is the reference's
// (post-order over the reachable set, kurumi_core/src/graph/inspect.rs:17-39) and each rewrite
// appends the same nodes in the same order (cast a, cast b, dot, cast back), so the rewritten
// graph is node for node the one kurumi builds. On the device the f16 contraction and its cast
// back to f32 become one f16 MFMA GEMM whose epilogue rounds to f16 and stores f32.
#include <unordered_map>

#include "graph.h"

namespace ku {

NodeId amp(Graph& g, NodeId root) {
  std::unordered_map<NodeId, NodeId> to;  // old node -> its rewritten value
  for (NodeId id : reachable_multi(g, {root})) {
    const Node n = g.node(id);  // copy: the arena grows below
    if (n.src.empty()) {
      to[id] = id;
      continue;
    }
    std::vector<NodeId> src;
    src.reserve(n.src.size());
    bool moved = false;
    for (NodeId s : n.src) {
      src.push_back(to.at(s));
      moved |= src.back() != s;
    }
    if (n.op.kind == OpKind::DotGeneral && n.dtype == DType::F32) {
      const NodeId a = g.cast(src[0], DType::F16);
      const NodeId b = g.cast(src[1], DType::F16);
      const NodeId d = g.push(n.op, {a, b});
      to[id] = g.cast(d, DType::F32);
    } else {
      to[id] = moved ? g.push(n.op, src) : id;
    }
  }
  return to.at(root);
}

}  // namespace ku
