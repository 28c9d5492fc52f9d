// TEST INFRASTRUCTURE / CPU BASELINE. Restatement of kurumi's view-fused CPU evaluator
// (kurumi_core/src/realize/sched.rs:32-104, realize/eval.rs:22-103, realize/tape/run.rs:23-117,
// lower/index/movement.rs:10-117): movement rewrites an index view over a shared source buffer
// (no copy), elementwise ops accrete into one lazy expression, and a boundary (reduce,
// contraction, movement of a fused value, a multi-consumer fused node) materialises it once,
// row by row. f32 only; any other dtype or op leaves the fused path (returns false) exactly
// like `fused_supported`. Per element it performs the same f32 operations as the interpreter,
// so results are bit-identical to `interpret`.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <deque>
#include <functional>
#include <map>
#include <memory>
#include <stdexcept>

#include "oracle.h"

namespace kuo {

using ku::DType;
using ku::NodeId;
using ku::Op;
using ku::OpKind;
using ku::Shape;
using ku::Tensor;

namespace {

struct View {
  Shape shape;
  std::vector<int64_t> strides;
  int64_t offset = 0;
  std::vector<int64_t> plo;  // padding (empty = none)
  Shape src;
};

View source_view(const Shape& s) {
  View v;
  v.shape = s;
  auto st = ku::row_major_strides(s);
  v.strides.assign(st.begin(), st.end());
  return v;
}

bool reshape_view(const View& v, const Shape& to, View* out) {
  if (!v.plo.empty()) return false;
  std::vector<size_t> os;
  std::vector<int64_t> ost;
  for (size_t i = 0; i < v.shape.size(); ++i)
    if (v.shape[i] != 1) os.push_back(v.shape[i]), ost.push_back(v.strides[i]);
  View r;
  r.shape = to;
  r.strides.assign(to.size(), 0);
  r.offset = v.offset;
  if (ku::numel(to) == 0) return false;
  size_t oi = 0, ni = 0;
  while (ni < to.size() || oi < os.size()) {
    if (ni < to.size() && to[ni] == 1) { ++ni; continue; }
    if (ni >= to.size() || oi >= os.size()) return false;
    size_t o0 = oi, n0 = ni;
    size_t po = os[oi++], pn = to[ni++];
    while (po != pn) {
      if (po < pn) { if (oi >= os.size()) return false; po *= os[oi++]; }
      else { while (ni < to.size() && to[ni] == 1) ++ni; if (ni >= to.size()) return false; pn *= to[ni++]; }
    }
    for (size_t t = o0; t + 1 < oi; ++t)
      if (ost[t] != ost[t + 1] * (int64_t)os[t + 1]) return false;
    int64_t st = ost[oi - 1];
    for (size_t t = ni; t-- > n0;) {
      if (to[t] == 1) continue;
      r.strides[t] = st;
      st *= (int64_t)to[t];
    }
  }
  *out = r;
  return true;
}

enum class E { Leaf, Add, Mul, Max, Neg, Recip, Sqrt, Exp2, Log2, Sin };

struct Expr {
  E kind;
  std::shared_ptr<const std::vector<float>> buf;
  View view;
  std::shared_ptr<Expr> a, b;
};

struct Realized {
  bool fused = false;
  Shape shape;
  std::shared_ptr<Expr> expr;  // Leaf or op tree
};

int g_passes = 0;

void read_row(const Expr& e, const std::vector<size_t>& coord, size_t n, float* out) {
  const View& v = e.view;
  size_t r = v.shape.size();
  const float* data = e.buf->data();
  if (!v.plo.empty()) {
    for (size_t j = 0; j < n; ++j) {
      bool ok = true;
      int64_t off = v.offset;
      for (size_t d = 0; d < r; ++d) {
        int64_t c = (int64_t)(d + 1 == r ? j : coord[d]) - v.plo[d];
        if (c < 0 || c >= (int64_t)v.src[d]) { ok = false; break; }
        off += c * v.strides[d];
      }
      out[j] = ok ? data[off] : 0.f;
    }
    return;
  }
  int64_t base = v.offset;
  for (size_t d = 0; d + 1 < r; ++d) base += (int64_t)coord[d] * v.strides[d];
  int64_t s = r ? v.strides[r - 1] : 0;
  if (s == 1) std::memcpy(out, data + base, n * 4);
  else if (s == 0) std::fill(out, out + n, data[base]);
  else for (size_t j = 0; j < n; ++j) out[j] = data[base + (int64_t)j * s];
}

// tape: evaluate an expression tree over one row (realize/tape/run.rs: one row kernel per op)
void eval_row(const Expr& e, const std::vector<size_t>& coord, size_t n, float* out, std::deque<std::vector<float>>& scratch, size_t depth) {
  if (e.kind == E::Leaf) { read_row(e, coord, n, out); return; }
  if (scratch.size() <= depth) scratch.emplace_back();
  std::vector<float>& t = scratch[depth];
  t.resize(n);
  eval_row(*e.a, coord, n, out, scratch, depth + 1);
  if (e.b) eval_row(*e.b, coord, n, t.data(), scratch, depth + 1);
  switch (e.kind) {
    case E::Add: for (size_t j = 0; j < n; ++j) out[j] = out[j] + t[j]; break;
    case E::Mul: for (size_t j = 0; j < n; ++j) out[j] = out[j] * t[j]; break;
    case E::Max: for (size_t j = 0; j < n; ++j) out[j] = std::fmax(out[j], t[j]); break;
    case E::Neg: for (size_t j = 0; j < n; ++j) out[j] = -out[j]; break;
    case E::Recip: for (size_t j = 0; j < n; ++j) out[j] = 1.0f / out[j]; break;
    case E::Sqrt: for (size_t j = 0; j < n; ++j) out[j] = std::sqrt(out[j]); break;
    case E::Exp2: for (size_t j = 0; j < n; ++j) out[j] = exp2f(out[j]); break;
    case E::Log2: for (size_t j = 0; j < n; ++j) out[j] = log2f(out[j]); break;
    case E::Sin: for (size_t j = 0; j < n; ++j) out[j] = sinf(out[j]); break;
    default: break;
  }
}

std::shared_ptr<std::vector<float>> force_contig(const Realized& r) {
  const Shape& s = r.shape;
  size_t n = ku::numel(s);
  auto out = std::make_shared<std::vector<float>>(n);
  if (!r.fused && r.expr->view.plo.empty()) {
    // contiguous source view: share nothing, copy once (a gather if strided)
  }
  size_t rank = s.size();
  size_t row = rank ? s[rank - 1] : 1;
  size_t rows = row ? n / row : 0;
  std::vector<size_t> coord(rank ? rank - 1 : 0, 0);
  Shape lead(s.begin(), rank ? s.end() - 1 : s.end());
  std::deque<std::vector<float>> scratch;
  Expr leaf0;
  const Expr& e = *r.expr;
  for (size_t i = 0; i < rows; ++i) {
    std::vector<size_t> c = coord;
    c.push_back(0);
    eval_row(e, c, row, out->data() + i * row, scratch, 0);
    for (size_t d = coord.size(); d-- > 0;) {
      if (++coord[d] < lead[d]) break;
      coord[d] = 0;
    }
  }
  g_passes++;
  return out;
}

Realized leaf_of(std::shared_ptr<const std::vector<float>> buf, const Shape& s) {
  Realized r;
  r.shape = s;
  r.expr = std::make_shared<Expr>();
  r.expr->kind = E::Leaf;
  r.expr->buf = std::move(buf);
  r.expr->view = source_view(s);
  return r;
}

Realized materialize(const Realized& r) { return leaf_of(force_contig(r), r.shape); }

Realized movement(const Realized& in, const std::function<bool(const View&, View*)>& f, const Shape& out_shape) {
  Realized src = in.fused ? materialize(in) : in;
  View v;
  if (!f(src.expr->view, &v)) {
    src = materialize(src);
    if (!f(src.expr->view, &v)) throw std::runtime_error("realize: movement not representable");
  }
  Realized r;
  r.shape = out_shape;
  r.expr = std::make_shared<Expr>(*src.expr);
  r.expr->view = v;
  return r;
}

bool op_fused(OpKind k) {
  switch (k) {
    case OpKind::Const: case OpKind::Input: case OpKind::Cast: case OpKind::Add: case OpKind::Mul: case OpKind::Max:
    case OpKind::Neg: case OpKind::Recip: case OpKind::Sqrt: case OpKind::Exp2: case OpKind::Log2: case OpKind::Sin:
    case OpKind::Sum: case OpKind::ReduceMax: case OpKind::Reshape: case OpKind::Permute: case OpKind::Expand:
    case OpKind::Slice: case OpKind::Flip: case OpKind::Pad: case OpKind::DotGeneral:
      return true;
    default:
      return false;
  }
}

}  // namespace

bool realize(const ku::Graph& g, NodeId root, const ku::Feeds& feeds, Tensor* out, int* passes) {
  auto order = ku::reachable_multi(g, {root});
  for (NodeId id : order)
    if (g.dtype(id) != DType::F32 || !op_fused(g.node(id).op.kind)) return false;
  std::sort(order.begin(), order.end());
  std::map<NodeId, int> counts;
  for (NodeId id : order)
    for (NodeId s : g.node(id).src) counts[s]++;
  g_passes = 0;
  std::map<NodeId, Realized> memo;
  for (NodeId id : order) {
    const auto& n = g.node(id);
    const Op& op = n.op;
    Realized r;
    auto in = [&](int i) -> const Realized& { return memo.at(n.src[i]); };
    auto un = [&](E k) {
      Realized x;
      x.fused = true;
      x.shape = n.shape;
      x.expr = std::make_shared<Expr>();
      x.expr->kind = k;
      x.expr->a = in(0).expr;
      if (n.src.size() > 1) x.expr->b = in(1).expr;
      return x;
    };
    switch (op.kind) {
      case OpKind::Const: {
        auto b = std::make_shared<std::vector<float>>(ku::numel(op.shape));
        if (!b->empty()) std::memcpy(b->data(), op.data->data(), b->size() * 4);
        r = leaf_of(b, op.shape);
      } break;
      case OpKind::Input: {
        auto it = feeds.find(id);
        if (it == feeds.end()) throw std::runtime_error("realize: missing feed for an Input node");
        auto b = std::make_shared<std::vector<float>>(ku::numel(n.shape));
        if (!b->empty()) std::memcpy(b->data(), it->second->bytes.data(), b->size() * 4);
        r = leaf_of(b, n.shape);
      } break;
      case OpKind::Cast: r = in(0); break;
      case OpKind::Add: r = un(E::Add); break;
      case OpKind::Mul: r = un(E::Mul); break;
      case OpKind::Max: r = un(E::Max); break;
      case OpKind::Neg: r = un(E::Neg); break;
      case OpKind::Recip: r = un(E::Recip); break;
      case OpKind::Sqrt: r = un(E::Sqrt); break;
      case OpKind::Exp2: r = un(E::Exp2); break;
      case OpKind::Log2: r = un(E::Log2); break;
      case OpKind::Sin: r = un(E::Sin); break;
      case OpKind::Reshape:
        r = movement(in(0), [&](const View& v, View* o) { return reshape_view(v, op.shape, o); }, n.shape);
        break;
      case OpKind::Expand:
        r = movement(in(0), [&](const View& v, View* o) {
          if (!v.plo.empty()) return false;
          *o = v;
          o->shape = op.shape;
          for (size_t d = 0; d < op.shape.size(); ++d)
            if (v.shape[d] == 1 && op.shape[d] != 1) o->strides[d] = 0;
          return true;
        }, n.shape);
        break;
      case OpKind::Permute:
        r = movement(in(0), [&](const View& v, View* o) {
          if (!v.plo.empty()) return false;
          View p;
          p.offset = v.offset;
          for (size_t q : op.perm) p.shape.push_back(v.shape[q]), p.strides.push_back(v.strides[q]);
          *o = p;
          return true;
        }, n.shape);
        break;
      case OpKind::Slice:
        r = movement(in(0), [&](const View& v, View* o) {
          if (!v.plo.empty()) return false;
          *o = v;
          for (size_t d = 0; d < op.ranges.size(); ++d) {
            o->offset += (int64_t)op.ranges[d].start * v.strides[d];
            o->strides[d] *= (int64_t)op.ranges[d].step;
            o->shape[d] = n.shape[d];
          }
          return true;
        }, n.shape);
        break;
      case OpKind::Flip:
        r = movement(in(0), [&](const View& v, View* o) {
          if (!v.plo.empty()) return false;
          *o = v;
          for (size_t a : op.axes) {
            o->offset += (int64_t)(v.shape[a] - 1) * v.strides[a];
            o->strides[a] = -o->strides[a];
          }
          return true;
        }, n.shape);
        break;
      case OpKind::Pad:
        r = movement(in(0), [&](const View& v, View* o) {
          if (!v.plo.empty()) return false;
          *o = v;
          o->src = v.shape;
          o->shape = n.shape;
          for (auto& p : op.pads) o->plo.push_back((int64_t)p.lo);
          return true;
        }, n.shape);
        break;
      case OpKind::Sum: case OpKind::ReduceMax: {
        // force_contig then reduce_v (sched.rs:74-83)
        auto d = force_contig(in(0));
        const Shape& s = in(0).shape;
        size_t outer = 1, len = s[op.axis], inner = 1;
        for (size_t q = 0; q < op.axis; ++q) outer *= s[q];
        for (size_t q = op.axis + 1; q < s.size(); ++q) inner *= s[q];
        auto b = std::make_shared<std::vector<float>>(outer * inner);
        bool sum = op.kind == OpKind::Sum;
        const float* x = d->data();
        // reduce_v (interp/reduce.rs:67-84): sequential fold along the axis
        for (size_t p = 0; p < outer; ++p)
          for (size_t q = 0; q < inner; ++q) {
            const float* line = x + p * len * inner + q;
            float acc = sum ? 0.f : -INFINITY;
            if (sum) for (size_t k = 0; k < len; ++k) acc = acc + line[k * inner];
            else for (size_t k = 0; k < len; ++k) acc = std::fmax(acc, line[k * inner]);
            (*b)[p * inner + q] = acc;
          }
        r = leaf_of(b, n.shape);
        g_passes++;
      } break;
      case OpKind::DotGeneral: {
        auto da = force_contig(in(0)), db = force_contig(in(1));
        ku::Graph tmp;
        NodeId a = tmp.input(in(0).shape, DType::F32), b = tmp.input(in(1).shape, DType::F32);
        NodeId y = tmp.dot_general(a, b, op.lc, op.rc, op.lb, op.rb);
        ku::Feeds f;
        auto mk = [](const std::vector<float>& v, const Shape& s) {
          auto t = std::make_shared<Tensor>();
          t->dtype = DType::F32;
          t->shape = s;
          t->bytes.resize(v.size() * 4);
          if (!v.empty()) std::memcpy(t->bytes.data(), v.data(), v.size() * 4);
          return t;
        };
        f[a] = mk(*da, in(0).shape);
        f[b] = mk(*db, in(1).shape);
        Tensor res = interpret(tmp, {y}, f)[0];
        auto buf = std::make_shared<std::vector<float>>(ku::numel(res.shape));
        if (!buf->empty()) std::memcpy(buf->data(), res.bytes.data(), buf->size() * 4);
        r = leaf_of(buf, res.shape);
        g_passes++;
      } break;
      default:
        return false;
    }
    // a multi-consumer fused node materialises once (sched.rs:94-101)
    if (r.fused && counts[id] > 1) r = materialize(r);
    memo[id] = r;
  }
  const Realized& res = memo.at(root);
  auto d = force_contig(res);
  if (!res.fused) g_passes--;  // a plain view read is a copy, not a compute pass
  out->dtype = DType::F32;
  out->shape = res.shape;
  out->bytes.resize(d->size() * 4);
  if (!d->empty()) std::memcpy(out->bytes.data(), d->data(), d->size() * 4);
  if (passes) *passes = g_passes;
  return true;
}

}  // namespace kuo
