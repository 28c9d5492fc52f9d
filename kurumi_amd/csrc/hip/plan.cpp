// Fusion planner + plan executor for the HIP backend (see plan.h).
#include "plan.h"

#include "../ir/hostcopy.h"
#include "fingerprint.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <limits>
#include <sstream>
#include <unordered_map>

#include "kernels/kernels.h"

namespace ku::hipbk {

// ======================= views =======================

View View::contiguous(const Shape& s) {
  View v;
  v.shape = s;
  auto st = row_major_strides(s);
  v.strides.assign(st.begin(), st.end());
  return v;
}

bool View::is_contiguous() const {
  if (padded() || offset != 0) return false;
  auto st = row_major_strides(shape);
  for (size_t i = 0; i < shape.size(); ++i)
    if (shape[i] != 1 && strides[i] != (int64_t)st[i]) return false;
  return true;
}

// A padded view reshapes without a copy only when the reshape inserts or drops unit axes
// (every windowed axis keeps its extent and window).
static bool view_reshape_padded(const View& v, const Shape& to, View* out) {
  View r;
  r.shape = to;
  r.offset = v.offset;
  size_t oi = 0;
  for (size_t ni = 0; ni < to.size(); ++ni) {
    while (oi < v.shape.size() && v.shape[oi] == 1) {  // dropped unit axis: must be inside its window
      if (!(v.wlo[oi] <= 0 && 0 < v.whi[oi])) return false;
      ++oi;
    }
    if (to[ni] == 1) {
      r.strides.push_back(0);
      r.wlo.push_back(0);
      r.whi.push_back(1);
      continue;
    }
    if (oi >= v.shape.size() || v.shape[oi] != to[ni]) return false;
    r.strides.push_back(v.strides[oi]);
    r.wlo.push_back(v.wlo[oi]);
    r.whi.push_back(v.whi[oi]);
    ++oi;
  }
  for (; oi < v.shape.size(); ++oi)
    if (v.shape[oi] != 1 || !(v.wlo[oi] <= 0 && 0 < v.whi[oi])) return false;
  *out = r;
  return true;
}

// No-copy reshape (dims grouped by equal products; each old group must be dense).
bool view_reshape(const View& v, const Shape& to, View* out) {
  if (v.padded()) return view_reshape_padded(v, to, out);
  if (numel(v.shape) == 0) {
    *out = View::contiguous(to);
    out->offset = v.offset;
    return true;
  }
  std::vector<size_t> os;
  std::vector<int64_t> ost;
  for (size_t i = 0; i < v.shape.size(); ++i)
    if (v.shape[i] != 1) os.push_back(v.shape[i]), ost.push_back(v.strides[i]);
  View r;
  r.shape = to;
  r.strides.assign(to.size(), 0);
  r.offset = v.offset;
  size_t oi = 0, ni = 0;
  while (ni < to.size() || oi < os.size()) {
    if (ni < to.size() && to[ni] == 1) { r.strides[ni] = 0; ++ni; continue; }
    if (ni >= to.size() || oi >= os.size()) return false;
    size_t o0 = oi, n0 = ni;
    size_t po = os[oi++], pn = to[ni++];
    while (po != pn) {
      if (po < pn) {
        if (oi >= os.size()) return false;
        po *= os[oi++];
      } else {
        while (ni < to.size() && to[ni] == 1) r.strides[ni++] = 0;
        if (ni >= to.size()) return false;
        pn *= to[ni++];
      }
    }
    for (size_t t = o0; t + 1 < oi; ++t)
      if (ost[t] != ost[t + 1] * (int64_t)os[t + 1]) return false;
    int64_t stride = ost[oi - 1];
    for (size_t t = ni; t-- > n0;) {
      if (to[t] == 1) { r.strides[t] = 0; continue; }
      r.strides[t] = stride;
      stride *= (int64_t)to[t];
    }
  }
  *out = r;
  return true;
}

View view_expand(const View& v, const Shape& to) {
  View r = v;
  r.shape = to;
  for (size_t i = 0; i < to.size(); ++i)
    if (v.shape[i] == 1 && to[i] != 1) {
      r.strides[i] = 0;
      if (v.padded()) {  // the one source element is either inside its window or not
        bool in = v.wlo[i] <= 0 && 0 < v.whi[i];
        r.wlo[i] = 0;
        r.whi[i] = in ? (int64_t)to[i] : 0;
      }
    }
  return r;
}

View view_permute(const View& v, const std::vector<size_t>& perm) {
  View r;
  r.offset = v.offset;
  for (size_t p : perm) {
    r.shape.push_back(v.shape[p]);
    r.strides.push_back(v.strides[p]);
    if (v.padded()) {
      r.wlo.push_back(v.wlo[p]);
      r.whi.push_back(v.whi[p]);
    }
  }
  return r;
}

static int64_t ceil_div(int64_t a, int64_t b) {  // b > 0
  return a >= 0 ? (a + b - 1) / b : -((-a) / b);
}

View view_slice(const View& v, const std::vector<SliceRange>& rg) {
  View r = v;
  for (size_t i = 0; i < rg.size(); ++i) {
    int64_t start = (int64_t)rg[i].start, step = (int64_t)rg[i].step;
    r.offset += start * v.strides[i];
    r.strides[i] = v.strides[i] * step;
    r.shape[i] = (rg[i].end - rg[i].start + rg[i].step - 1) / rg[i].step;
    if (v.padded()) {  // new c valid iff wlo <= start + c*step < whi
      int64_t n = (int64_t)r.shape[i];
      r.wlo[i] = std::min(std::max<int64_t>(ceil_div(v.wlo[i] - start, step), 0), n);
      r.whi[i] = std::min(std::max<int64_t>(ceil_div(v.whi[i] - start, step), 0), n);
    }
  }
  return r;
}

View view_flip(const View& v, const std::vector<size_t>& axes) {
  View r = v;
  for (size_t a : axes) {
    if (r.shape[a] == 0) continue;
    int64_t n = (int64_t)r.shape[a];
    r.offset += (n - 1) * r.strides[a];
    r.strides[a] = -r.strides[a];
    if (r.padded()) {  // c' = n-1-c: valid iff n - whi <= c' < n - wlo
      int64_t lo = n - r.whi[a], hi = n - r.wlo[a];
      r.wlo[a] = lo;
      r.whi[a] = hi;
    }
  }
  return r;
}

View view_pad(const View& v, const std::vector<PadRange>& p) {
  View r = v;
  if (!r.padded()) {
    r.wlo.assign(v.shape.size(), 0);
    r.whi.assign(v.shape.begin(), v.shape.end());
  }
  for (size_t i = 0; i < p.size(); ++i) {
    int64_t lo = (int64_t)p[i].lo;
    r.offset -= lo * v.strides[i];
    r.wlo[i] += lo;
    r.whi[i] += lo;
    r.shape[i] = p[i].lo + v.shape[i] + p[i].hi;
  }
  return r;
}

static bool view_eq(const View& a, const View& b) {
  return a.shape == b.shape && a.strides == b.strides && a.offset == b.offset && a.wlo == b.wlo && a.whi == b.whi;
}

// ======================= const cache =======================

ConstCache::ConstCache(Context* ctx) : ctx_(ctx) {
  const char* e = std::getenv("KURUMI_HIP_CONST_CACHE_MB");
  budget_ = (size_t)(e && *e ? std::strtoull(e, nullptr, 10) : 2048) << 20;
  ctx_->pool().add_reclaimer([this] { return reclaim(); });
}

std::shared_ptr<ConstEntry> ConstCache::get(const Graph& g, NodeId id) {
  const Node& n = g.node(id);
  auto fast = by_node_.find({g.id(), id});
  if (fast != by_node_.end()) {
    auto it = by_content_.find(fast->second);
    if (it != by_content_.end()) {
      it->second->last_use = ++clock_;
      return it->second;
    }
    by_node_.erase(fast);
  }
  Hash128 h = payload_hash(n.op.data);
  const size_t nb = n.op.data ? n.op.data->size() : 0;
  Key key{h.lo, h.hi, nb, (uint32_t)n.op.data_dtype, n.op.shape};
  if (by_node_.size() > (1u << 16)) by_node_.clear();  // stale fast-path records of freed graphs
  by_node_[{g.id(), id}] = key;
  auto it = by_content_.find(key);
  if (it != by_content_.end()) {
    it->second->last_use = ++clock_;
    return it->second;
  }
  auto e = std::make_shared<ConstEntry>();
  e->buf = ctx_->pool().alloc(std::max<size_t>(nb, 1));
  e->pool = &ctx_->pool();
  e->nbytes = e->buf.bytes;
  e->last_use = ++clock_;
  if (nb) ctx_->upload(e->buf.ptr, n.op.data->data(), nb);
  uploads_++;
  by_content_[key] = e;
  enforce_budget();
  return e;
}

void ConstCache::enforce_budget() {
  size_t idle = 0;
  for (auto& kv : by_content_)
    if (kv.second.use_count() == 1) idle += kv.second->nbytes;
  while (idle > budget_) {
    auto victim = by_content_.end();
    for (auto it = by_content_.begin(); it != by_content_.end(); ++it)
      if (it->second.use_count() == 1 && (victim == by_content_.end() || it->second->last_use < victim->second->last_use))
        victim = it;
    if (victim == by_content_.end()) break;
    idle -= victim->second->nbytes;
    by_content_.erase(victim);
  }
}

size_t ConstCache::reclaim() {
  size_t freed = 0;
  for (auto it = by_content_.begin(); it != by_content_.end();) {
    if (it->second.use_count() == 1) {
      freed += it->second->nbytes;
      it = by_content_.erase(it);
    } else {
      ++it;
    }
  }
  return freed;
}

ConstCache::~ConstCache() {
  ctx_->pool().clear_reclaimers();
  by_content_.clear();
}

// ======================= planner =======================

namespace {

constexpr size_t kEmpty = std::numeric_limits<size_t>::max();

struct Val {
  enum K { None, Dev, LFull, LLine, LKeep, LBcast } k = None;
  int slot = -1;
  View view;
  int region = -1;
  int rn = -1;
};

bool is_elementwise(OpKind k) {
  switch (k) {
    case OpKind::Cast: case OpKind::Bitcast: case OpKind::Add: case OpKind::Mul: case OpKind::Max:
    case OpKind::Neg: case OpKind::IDiv: case OpKind::And: case OpKind::Or: case OpKind::Xor: case OpKind::Shl:
    case OpKind::Shr: case OpKind::CmpLt: case OpKind::CmpEq: case OpKind::Where: case OpKind::Recip:
    case OpKind::Sqrt: case OpKind::Exp2: case OpKind::Log2: case OpKind::Sin: case OpKind::Floor:
      return true;
    default:
      return false;
  }
}
bool is_reduce(OpKind k) {
  return k == OpKind::Sum || k == OpKind::Prod || k == OpKind::ReduceMax || k == OpKind::ArgReduce;
}

Shape drop_axis(const Shape& s, int a) {
  Shape r = s;
  r.erase(r.begin() + a);
  return r;
}
Shape keep_axis(const Shape& s, int a) {
  Shape r = s;
  r[a] = 1;
  return r;
}

// value of a scalar constant (all elements equal) or NaN when not uniform
bool const_uniform_value(const Node& n, double* out) {
  if (n.op.kind != OpKind::Const || !n.op.data) return false;
  size_t cnt = numel(n.op.shape);
  if (cnt == 0) return false;
  size_t w = dt_width(n.op.data_dtype);
  const uint8_t* p = n.op.data->data();
  for (size_t i = 1; i < cnt; ++i)
    if (std::memcmp(p, p + i * w, w) != 0) return false;
  double v;
  switch (n.op.data_dtype) {
    case DType::F32: { float f; std::memcpy(&f, p, 4); v = f; } break;
    case DType::F64: std::memcpy(&v, p, 8); break;
    case DType::BF16: { uint16_t h; std::memcpy(&h, p, 2); v = bf16_to_f32(h); } break;
    case DType::F16: { uint16_t h; std::memcpy(&h, p, 2); v = f16_to_f64(h); } break;
    default: return false;
  }
  *out = v;
  return true;
}

}  // namespace

class Planner {
 public:
  Planner(Plan& P, ConstCache* consts) : P_(P), g_(*P.bg_), consts_(consts) {}
  void run();

 private:
  // slots / steps
  int new_slot(SlotKind k, DType dt, size_t bytes, NodeId node) {
    Slot s;
    s.kind = k;
    s.dtype = dt;
    s.bytes = bytes;
    s.node = node;
    P_.slots_.push_back(s);
    slot_producer_.push_back(-1);
    return (int)P_.slots_.size() - 1;
  }
  int new_step(Step::Type t, int index, const std::string& label) {
    Step s;
    s.type = t;
    s.index = index;
    s.label = label;
    P_.steps_.push_back(s);
    step_alive_.push_back(true);
    return (int)P_.steps_.size() - 1;
  }
  int new_region(const Shape& S) {
    Region r;
    r.S = S;
    if (r.S.empty()) r.S = {1};
    P_.regions_.push_back(r);
    int id = (int)P_.regions_.size() - 1;
    region_step_.push_back(new_step(Step::REGION, id, "fused"));
    return id;
  }
  void depend(int step, int slot) {
    int p = slot_producer_[slot];
    if (p >= 0 && p != step) P_.steps_[step].deps.insert(p);
  }

  // region building
  int add_leaf(int rid, int slot, const View& v, DType dt);
  int add_node(int rid, RNode n);
  void set_level(Region& R, RNode& n);
  void materialize(NodeId x);
  int output_slot(int rid, int rn);
  View dev_view_of(NodeId x);
  int region_operand(int rid, NodeId x, bool line_pos);
  bool try_join(NodeId id, int* rid_out, bool* line_pos);
  void merge_regions(int into, int from);
  void close_region(int rid) { P_.regions_[rid].closed = true; }

  void visit(NodeId id);
  void visit_elementwise(NodeId id);
  void visit_movement(NodeId id);
  bool clone_through_movement(NodeId id);
  void visit_reduce(NodeId id);
  void visit_rowop(NodeId id);
  void visit_dot(NodeId id);
  void visit_sdpa(NodeId id);
  void visit_quant(NodeId id);
  int copy_view_to_slot(const View& v, int slot_src, DType dt, NodeId node);

  // pattern pre-pass
  void find_patterns();
  bool match_attention(NodeId d2);
  bool match_fp8_epilogue(NodeId castn);
  bool match_cast_epilogue(NodeId castn);
  bool match_actq(NodeId xq, NodeId sx);
  void visit_actq(NodeId sx);

  struct AttnPattern { NodeId q, k, v; float scale; bool causal; };
  struct Fp8Pattern { NodeId dot, xq, wq, sx, sw; };
  struct ActqPattern { NodeId x, xq; };

  Plan& P_;
  const Graph& g_;
  ConstCache* consts_;
  std::vector<Val> vals_;
  std::vector<int> consumers_;
  std::vector<bool> absorbed_;
  std::map<NodeId, AttnPattern> attn_pat_;
  std::map<NodeId, Fp8Pattern> fp8_pat_;
  std::map<NodeId, NodeId> cast_pat_;  // dot -> the cast its GEMM epilogue performs
  std::map<NodeId, ActqPattern> actq_pat_;  // sx -> the activation quantisation producing it
  std::vector<std::vector<NodeId>> users_;
  std::vector<int> region_step_;
  std::vector<int> slot_producer_;
  std::vector<bool> step_alive_;
  std::map<std::pair<int, int>, int> rn_slot_;
  std::set<NodeId> root_set_;
};

int Planner::add_leaf(int rid, int slot, const View& v, DType dt) {
  Region& R = P_.regions_[rid];
  for (size_t i = 0; i < R.leaves.size(); ++i)
    if (R.leaves[i].slot == slot && R.leaves[i].dtype == dt && view_eq(R.leaves[i].view, v)) {
      for (size_t j = 0; j < R.nodes.size(); ++j)
        if (R.nodes[j].kind == RK_LEAF && R.nodes[j].leaf == (int)i) return (int)j;
    }
  Leaf L;
  L.slot = slot;
  L.view = v;
  L.dtype = dt;
  if (P_.slots_[slot].kind == SlotKind::Const && !v.padded()) {
    bool uniform = true;
    for (size_t d = 0; d < v.shape.size(); ++d)
      if (v.strides[d] != 0 && v.shape[d] > 1) uniform = false;
    const Node& cn = g_.node(P_.slots_[slot].node);
    size_t w = dt_width(dt);
    if (uniform && cn.op.data && v.offset >= 0 && (size_t)(v.offset + 1) * w <= cn.op.data->size() && w <= 8) {
      L.imm = true;
      std::memcpy(L.imm_bits, cn.op.data->data() + (size_t)v.offset * w, w);
    }
  }
  R.leaves.push_back(L);
  depend(region_step_[rid], slot);
  RNode n;
  n.kind = RK_LEAF;
  n.leaf = (int)R.leaves.size() - 1;
  n.dtype = dt;
  // a leaf that is constant along the axis is a LINE value
  n.space = (R.axis >= 0 && v.strides[R.axis] == 0 && !v.padded()) ? Space::Line : Space::Full;
  if (R.axis < 0) n.space = Space::Full;
  return add_node(rid, n);
}

void Planner::set_level(Region& R, RNode& n) {
  int lv = 0;
  for (int i : n.in) lv = std::max(lv, R.nodes[i].level);
  if (is_reduce((OpKind)n.kind)) lv += 1;
  n.level = lv;
}

int Planner::add_node(int rid, RNode n) {
  Region& R = P_.regions_[rid];
  set_level(R, n);
  R.nodes.push_back(n);
  return (int)R.nodes.size() - 1;
}

int Planner::output_slot(int rid, int rn) {
  auto key = std::make_pair(rid, rn);
  auto it = rn_slot_.find(key);
  if (it != rn_slot_.end()) return it->second;
  Region& R = P_.regions_[rid];
  const RNode& n = R.nodes[rn];
  Shape sh = n.space == Space::Full ? R.S : drop_axis(R.S, R.axis);
  int slot = new_slot(SlotKind::Temp, n.dtype, numel(sh) * dt_width(n.dtype), 0);
  slot_producer_[slot] = region_step_[rid];
  R.outputs.push_back({rn, slot});
  rn_slot_[key] = slot;
  return slot;
}

// Turn a lazy value into a device buffer (its region gains an output and is closed:
// whatever reads the buffer runs after the region's kernel).
void Planner::materialize(NodeId x) {
  Val& v = vals_[x];
  if (v.k == Val::Dev) return;
  if (v.k == Val::None) throw Error("kurumi_hip planner: node " + std::to_string(x) + " has no value");
  int rid = v.region;
  Region& R = P_.regions_[rid];
  int slot = output_slot(rid, v.rn);
  close_region(rid);
  const Shape& gs = g_.shape(x);
  View view;
  if (v.k == Val::LFull) {
    view = View::contiguous(R.S);
    if (!view_reshape(view, gs, &view)) throw Error("planner: bad full view");
  } else if (v.k == Val::LLine || v.k == Val::LKeep) {
    view = View::contiguous(drop_axis(R.S, R.axis));
    if (!view_reshape(view, gs, &view)) throw Error("planner: bad line view");
  } else {  // LBcast: the line buffer broadcast along the axis
    View lk = View::contiguous(drop_axis(R.S, R.axis));
    View kd;
    if (!view_reshape(lk, keep_axis(R.S, R.axis), &kd)) throw Error("planner: bad keepdim view");
    view = view_expand(kd, R.S);
    if (gs != R.S && !view_reshape(view, gs, &view)) throw Error("planner: bad bcast view");
  }
  // every graph node sharing this lazy value becomes the same device view
  for (size_t i = 0; i < vals_.size(); ++i) {
    Val& o = vals_[i];
    if (o.k != Val::Dev && o.k != Val::None && o.region == rid && o.rn == v.rn && o.k == v.k &&
        g_.shape((NodeId)i) == gs) {
      o.k = Val::Dev;
      o.slot = slot;
      o.view = view;
    }
  }
}

View Planner::dev_view_of(NodeId x) {
  materialize(x);
  return vals_[x].view;
}

// Operand of a region node: a lazy member or a device leaf viewed over R.S.
int Planner::region_operand(int rid, NodeId x, bool line_pos) {
  Val& v = vals_[x];
  Region& R = P_.regions_[rid];
  if (v.k != Val::Dev) return v.rn;  // caller checked compatibility
  View view = v.view;
  if (line_pos) {
    // x has the line shape (S without the axis): insert a stride-0 axis
    View kd;
    if (!view_reshape(view, keep_axis(R.S, R.axis), &kd)) {
      // not representable (padded view): copy first
      int s = copy_view_to_slot(view, v.slot, g_.dtype(x), x);
      View c = View::contiguous(g_.shape(x));
      view_reshape(c, keep_axis(R.S, R.axis), &kd);
      v.slot = s;
      v.view = c;
    }
    view = view_expand(kd, R.S);
  } else if (g_.shape(x) != R.S) {
    View r;
    if (!view_reshape(view, R.S, &r)) throw Error("planner: operand shape mismatch");
    view = r;
  }
  return add_leaf(rid, v.slot, view, g_.dtype(x));
}

void Planner::merge_regions(int into, int from) {
  Region& A = P_.regions_[into];
  Region& B = P_.regions_[from];
  if (A.axis < 0) A.axis = B.axis;
  int base = (int)A.nodes.size();
  int lbase = (int)A.leaves.size();
  for (auto& L : B.leaves) A.leaves.push_back(L);
  for (RNode n : B.nodes) {
    for (int& i : n.in) i += base;
    if (n.kind == RK_LEAF) n.leaf += lbase;
    A.nodes.push_back(n);
  }
  for (auto& o : B.outputs) {
    A.outputs.push_back({o.first + base, o.second});
    slot_producer_[o.second] = region_step_[into];
  }
  for (auto it = rn_slot_.begin(); it != rn_slot_.end();) {
    if (it->first.first == from) {
      rn_slot_[{into, it->first.second + base}] = it->second;
      it = rn_slot_.erase(it);
    } else {
      ++it;
    }
  }
  for (auto& v : vals_)
    if (v.k != Val::Dev && v.k != Val::None && v.region == from) {
      v.region = into;
      v.rn += base;
    }
  Step& sa = P_.steps_[region_step_[into]];
  for (int d : P_.steps_[region_step_[from]].deps) sa.deps.insert(d);
  step_alive_[region_step_[from]] = false;
  B.nodes.clear();
  B.leaves.clear();
  B.outputs.clear();
  B.closed = true;
  // re-derive leaf spaces for the (possibly new) axis
  for (auto& n : A.nodes)
    if (n.kind == RK_LEAF && A.axis >= 0) {
      const View& lv = A.leaves[n.leaf].view;
      n.space = (lv.strides[A.axis] == 0 && !lv.padded()) ? Space::Line : Space::Full;
    }
}

// Decide whether elementwise node `id` can be evaluated inside an existing open region.
bool Planner::try_join(NodeId id, int* rid_out, bool* line_pos) {
  const Node& n = g_.node(id);
  int rid = -1;
  // position of node n in region R: FULL (shape S), LINE (S without the axis) or neither
  auto full_pos = [&](const Region& R) {
    return n.shape == R.S || (n.shape.empty() && R.S == Shape{1} && R.axis < 0);
  };
  auto line_pos_of = [&](const Region& R) {
    return !full_pos(R) && R.axis >= 0 && n.shape == drop_axis(R.S, R.axis);
  };
  for (NodeId s : n.src) {
    Val& v = vals_[s];
    if (v.k == Val::Dev) continue;
    Region& R = P_.regions_[v.region];
    bool ok = !R.closed;
    if (ok) {
      if (full_pos(R)) ok = (v.k == Val::LFull || v.k == Val::LBcast);
      else if (line_pos_of(R)) ok = (v.k == Val::LLine);
      else ok = false;
    }
    if (!ok) {
      materialize(s);
      continue;
    }
    if (rid < 0) {
      rid = v.region;
    } else if (rid != v.region) {
      Region& A = P_.regions_[rid];
      Region& B = P_.regions_[v.region];
      bool compat = A.S == B.S && (A.axis < 0 || B.axis < 0 || A.axis == B.axis);
      if (compat) merge_regions(rid, v.region);
      else materialize(s);
    }
  }
  if (rid < 0) return false;
  Region& R = P_.regions_[rid];
  *line_pos = line_pos_of(R);
  *rid_out = rid;
  return true;
}

int Planner::copy_view_to_slot(const View& v, int slot_src, DType dt, NodeId node) {
  int rid = new_region(v.shape);
  Region& R = P_.regions_[rid];
  R.name = "copy";
  View vv = v;
  if (vv.shape.empty()) { vv.shape = {1}; vv.strides = {0}; }
  int ln = add_leaf(rid, slot_src, vv, dt);
  (void)node;
  int slot = output_slot(rid, ln);
  close_region(rid);
  return slot;
}

void Planner::visit_elementwise(NodeId id) {
  const Node& n = g_.node(id);
  int rid;
  bool line_pos = false;
  if (!try_join(id, &rid, &line_pos)) {
    rid = new_region(n.shape);
    line_pos = false;
  }
  RNode rn;
  rn.kind = (int)n.op.kind;
  rn.dtype = n.dtype;
  rn.to = n.op.to;
  rn.space = line_pos ? Space::Line : Space::Full;
  for (NodeId s : n.src) rn.in.push_back(region_operand(rid, s, line_pos));
  // A FULL-position op whose operands are all line values is itself a line value
  // broadcast along the axis: compute it once per line instead of per element.
  bool hoist = false;
  if (!line_pos && P_.regions_[rid].axis >= 0) {
    hoist = true;
    for (int i : rn.in)
      if (P_.regions_[rid].nodes[i].space != Space::Line) hoist = false;
    if (hoist) rn.space = Space::Line;
  }
  int r = add_node(rid, rn);
  Val v;
  v.region = rid;
  v.rn = r;
  v.k = line_pos ? Val::LLine : (hoist ? Val::LBcast : Val::LFull);
  vals_[id] = v;
}

// The moved view of `v` for movement node `n` (false when a reshape needs a copy).
static bool move_view(const Node& n, const View& v, View* out) {
  switch (n.op.kind) {
    case OpKind::Reshape: return view_reshape(v, n.shape, out);
    case OpKind::Expand: *out = view_expand(v, n.shape); return true;
    case OpKind::Permute: *out = view_permute(v, n.op.perm); return true;
    case OpKind::Slice: *out = view_slice(v, n.op.ranges); return true;
    case OpKind::Flip: *out = view_flip(v, n.op.axes); return true;
    case OpKind::Pad: *out = view_pad(v, n.op.pads); return true;
    default: return false;
  }
}

// A movement of a lazy elementwise value becomes the same expression evaluated in the moved
// coordinates: its nodes are cloned into a region of the output shape with every leaf view
// (and every pad window) moved the same way, so no buffer and no kernel boundary appear. A
// Pad adds a select that zeroes the new border. Not done when the expression depends on its
// own coordinates (iota, rand), lives in a reduction region, or when a broadcast would
// repeat real work per output element (that value is computed once instead).
bool Planner::clone_through_movement(NodeId id) {
  const Node& n = g_.node(id);
  NodeId s = n.src[0];
  const Val a = vals_[s];
  if (a.k != Val::LFull) return false;
  const int srid = a.region;
  if (P_.regions_[srid].axis >= 0 || P_.regions_[srid].S != g_.shape(s)) return false;
  std::vector<RNode> nodes = P_.regions_[srid].nodes;
  std::vector<Leaf> leaves = P_.regions_[srid].leaves;
  std::vector<int> order;
  std::vector<char> seen(nodes.size(), 0);
  std::function<void(int)> walk = [&](int i) {
    if (seen[i]) return;
    seen[i] = 1;
    for (int j : nodes[i].in) walk(j);
    order.push_back(i);
  };
  walk(a.rn);
  int heavy = 0;
  for (int i : order) {
    const RNode& rn = nodes[i];
    if (rn.kind == RK_LEAF || rn.kind == RK_PADSEL) continue;
    if (rn.kind >= RK_LEAF || !is_elementwise((OpKind)rn.kind)) return false;
    switch ((OpKind)rn.kind) {
      case OpKind::Exp2: case OpKind::Log2: case OpKind::Sin: case OpKind::Sqrt: case OpKind::Recip:
      case OpKind::IDiv:
        ++heavy;
        break;
      default: break;
    }
  }
  if (n.op.kind == OpKind::Expand && numel(n.shape) > numel(g_.shape(s)) && (heavy > 0 || order.size() > 12))
    return false;
  std::vector<View> moved(nodes.size());
  for (int i : order) {
    const RNode& rn = nodes[i];
    if (rn.kind == RK_LEAF && !move_view(n, leaves[rn.leaf].view, &moved[i])) return false;
    if (rn.kind == RK_PADSEL && !move_view(n, rn.win, &moved[i])) return false;
  }
  int rid = new_region(n.shape);
  std::vector<int> map(nodes.size(), -1);
  for (int i : order) {
    const RNode& rn = nodes[i];
    if (rn.kind == RK_LEAF) {
      map[i] = add_leaf(rid, leaves[rn.leaf].slot, moved[i], leaves[rn.leaf].dtype);
      continue;
    }
    RNode c = rn;
    c.space = Space::Full;
    for (int& j : c.in) j = map[j];
    if (rn.kind == RK_PADSEL) c.win = moved[i];
    map[i] = add_node(rid, c);
  }
  int root = map[a.rn];
  if (n.op.kind == OpKind::Pad) {
    RNode ps;
    ps.kind = RK_PADSEL;
    ps.dtype = nodes[a.rn].dtype;
    ps.space = Space::Full;
    ps.in = {root};
    ps.win = view_pad(View::contiguous(g_.shape(s)), n.op.pads);
    root = add_node(rid, ps);
  }
  Val v;
  v.k = Val::LFull;
  v.region = rid;
  v.rn = root;
  vals_[id] = v;
  return true;
}

void Planner::visit_movement(NodeId id) {
  const Node& n = g_.node(id);
  NodeId s = n.src[0];
  if (vals_[s].k == Val::LFull && clone_through_movement(id)) return;
  Val& a = vals_[s];
  if (a.k != Val::Dev) {
    Region& R = P_.regions_[a.region];
    const Shape& is = g_.shape(s);
    if ((n.op.kind == OpKind::Reshape || n.op.kind == OpKind::Expand) && n.shape == is) {
      vals_[id] = a;
      return;
    }
    if (!R.closed && R.axis >= 0) {
      if (n.op.kind == OpKind::Reshape && a.k == Val::LLine && n.shape == keep_axis(R.S, R.axis)) {
        vals_[id] = a;
        vals_[id].k = Val::LKeep;
        return;
      }
      if (n.op.kind == OpKind::Reshape && a.k == Val::LKeep && n.shape == drop_axis(R.S, R.axis)) {
        vals_[id] = a;
        vals_[id].k = Val::LLine;
        return;
      }
      if (n.op.kind == OpKind::Expand && a.k == Val::LKeep && n.shape == R.S) {
        vals_[id] = a;
        vals_[id].k = Val::LBcast;
        return;
      }
    }
    materialize(s);
  }
  Val& d = vals_[s];
  View v = d.view;
  int slot = d.slot;
  View r;
  switch (n.op.kind) {
    case OpKind::Reshape:
      if (!view_reshape(v, n.shape, &r)) {
        slot = copy_view_to_slot(v, slot, n.dtype, s);
        r = View::contiguous(n.shape);
      }
      break;
    case OpKind::Expand: r = view_expand(v, n.shape); break;
    case OpKind::Permute: r = view_permute(v, n.op.perm); break;
    case OpKind::Slice: r = view_slice(v, n.op.ranges); break;
    case OpKind::Flip: r = view_flip(v, n.op.axes); break;
    case OpKind::Pad: r = view_pad(v, n.op.pads); break;
    default: throw Error("planner: not a movement op");
  }
  Val out;
  out.k = Val::Dev;
  out.slot = slot;
  out.view = r;
  vals_[id] = out;
}

void Planner::visit_reduce(NodeId id) {
  const Node& n = g_.node(id);
  NodeId s = n.src[0];
  int axis = (int)n.op.axis;
  Val& a = vals_[s];
  int rid = -1;
  if (a.k == Val::LFull) {
    Region& R = P_.regions_[a.region];
    if (!R.closed && R.S == g_.shape(s) && (R.axis < 0 || R.axis == axis)) rid = a.region;
    else materialize(s);
  } else if (a.k != Val::Dev) {
    materialize(s);
  }
  if (rid < 0) {
    rid = new_region(g_.shape(s));
  }
  Region& R = P_.regions_[rid];
  if (R.axis < 0) {
    R.axis = axis;
    for (auto& nn : R.nodes)
      if (nn.kind == RK_LEAF) {
        const View& lv = R.leaves[nn.leaf].view;
        nn.space = (lv.strides[axis] == 0 && !lv.padded()) ? Space::Line : Space::Full;
      }
  }
  int in = region_operand(rid, s, false);
  RNode rn;
  rn.kind = (int)n.op.kind;
  rn.dtype = n.dtype;
  rn.space = Space::Line;
  rn.arg = n.op.arg;
  rn.in = {in};
  int r = add_node(rid, rn);
  Val v;
  v.k = Val::LLine;
  v.region = rid;
  v.rn = r;
  vals_[id] = v;
}

// Softmax / RmsNorm: a row program inside a line region (interp/nn.rs:18-120).
void Planner::visit_rowop(NodeId id) {
  const Node& n = g_.node(id);
  NodeId s = n.src[0];
  int axis = (int)n.op.axis;
  Val& a = vals_[s];
  int rid = -1;
  if (a.k == Val::LFull) {
    Region& R = P_.regions_[a.region];
    if (!R.closed && R.S == g_.shape(s) && (R.axis < 0 || R.axis == axis)) rid = a.region;
    else materialize(s);
  } else if (a.k != Val::Dev) {
    materialize(s);
  }
  if (rid < 0) rid = new_region(g_.shape(s));
  {
    Region& R = P_.regions_[rid];
    if (R.axis < 0) {
      R.axis = axis;
      for (auto& nn : R.nodes)
        if (nn.kind == RK_LEAF) {
          const View& lv = R.leaves[nn.leaf].view;
          nn.space = (lv.strides[axis] == 0 && !lv.padded()) ? Space::Line : Space::Full;
        }
    }
  }
  DType dt = n.dtype;
  DType acc = dt == DType::F64 ? DType::F64 : DType::F32;
  int x = region_operand(rid, s, false);
  auto mk = [&](int kind, DType d, Space sp, std::vector<int> in) {
    RNode r;
    r.kind = kind;
    r.dtype = d;
    r.space = sp;
    r.to = d;
    r.in = std::move(in);
    return add_node(rid, r);
  };
  int xf = (dt == acc) ? x : mk((int)OpKind::Cast, acc, Space::Full, {x});
  int y;
  if (n.op.kind == OpKind::Softmax) {
    int m = mk((int)OpKind::ReduceMax, acc, Space::Line, {xf});
    int nm = mk((int)OpKind::Neg, acc, Space::Line, {m});
    int d = mk((int)OpKind::Add, acc, Space::Full, {xf, nm});
    int e = mk(RK_EXP, acc, Space::Full, {d});
    int sm = mk((int)OpKind::Sum, acc, Space::Line, {e});
    y = mk(RK_DIV, acc, Space::Full, {e, sm});
  } else {
    int sq = mk((int)OpKind::Mul, acc, Space::Full, {xf, xf});
    int ss = mk((int)OpKind::Sum, acc, Space::Line, {sq});
    RNode rr;
    rr.kind = RK_SQRT_ADD_EPS;
    rr.dtype = acc;
    rr.space = Space::Line;
    rr.in = {ss};
    rr.eps = n.op.eps;
    rr.axis = g_.shape(s)[axis];
    int rms = add_node(rid, rr);
    y = mk(RK_DIV, acc, Space::Full, {xf, rms});
  }
  int out = (dt == acc) ? y : mk((int)OpKind::Cast, dt, Space::Full, {y});
  Val v;
  v.k = Val::LFull;
  v.region = rid;
  v.rn = out;
  vals_[id] = v;
}

// ---------------- contraction ----------------

namespace {
// Merge `axes` (in the given order) of a view into one (stride, size). False if not dense.
bool merge_axes(const View& v, const std::vector<size_t>& axes, int64_t* stride, int64_t* size) {
  int64_t sz = 1, st = 0;
  bool have = false;
  for (size_t i = axes.size(); i-- > 0;) {
    size_t a = axes[i];
    if (v.shape[a] == 1) continue;
    if (!have) {
      st = v.strides[a];
      have = true;
    } else if (v.strides[a] != st * sz) {
      return false;
    }
    sz *= (int64_t)v.shape[a];
  }
  *stride = have ? st : 0;
  *size = sz;
  if (!have) {
    for (size_t a : axes) sz *= (int64_t)v.shape[a];
    *size = sz;
  }
  return true;
}
}  // namespace

void Planner::visit_dot(NodeId id) {
  const Node& n = g_.node(id);
  NodeId an = n.src[0], bn = n.src[1];
  GemmStep G;
  auto fp8 = fp8_pat_.find(id);
  NodeId out_node = id;
  if (fp8 != fp8_pat_.end()) {
    an = fp8->second.xq;
    bn = fp8->second.wq;
  }
  View av = dev_view_of(an), bv = dev_view_of(bn);
  int aslot = vals_[an].slot, bslot = vals_[bn].slot;
  // the GEMM kernels read plain strided operands: zero-padded views are copied out first
  if (av.padded()) {
    aslot = copy_view_to_slot(av, aslot, g_.dtype(an), an);
    av = View::contiguous(av.shape);
  }
  if (bv.padded()) {
    bslot = copy_view_to_slot(bv, bslot, g_.dtype(bn), bn);
    bv = View::contiguous(bv.shape);
  }
  DType in_dt = g_.dtype(an);
  const Op& op = n.op;
  std::vector<size_t> afree = free_axes(av.shape.size(), op.lb, op.lc);
  std::vector<size_t> bfree = free_axes(bv.shape.size(), op.rb, op.rc);
  int64_t sab, bsz, sam, m, sak, k, sbb, bsz2, sbn, nn, sbk, k2;
  bool ok = merge_axes(av, op.lb, &sab, &bsz) && merge_axes(av, afree, &sam, &m) && merge_axes(av, op.lc, &sak, &k);
  bool okb = merge_axes(bv, op.rb, &sbb, &bsz2) && merge_axes(bv, bfree, &sbn, &nn) && merge_axes(bv, op.rc, &sbk, &k2);
  auto canon = [&](NodeId x, View& v, int& slot, const std::vector<size_t>& order) {
    View p = view_permute(v, order);
    slot = copy_view_to_slot(p, slot, g_.dtype(x), x);
    v = View::contiguous(p.shape);
  };
  // A must be k-contiguous (or trivially so) for every kernel family; canonicalise otherwise.
  if (!ok || (k > 1 && sak != 1)) {
    std::vector<size_t> order(op.lb);
    order.insert(order.end(), afree.begin(), afree.end());
    order.insert(order.end(), op.lc.begin(), op.lc.end());
    canon(an, av, aslot, order);
    std::vector<size_t> b0, f0, c0;
    size_t t = 0;
    for (size_t i = 0; i < op.lb.size(); ++i) b0.push_back(t++);
    for (size_t i = 0; i < afree.size(); ++i) f0.push_back(t++);
    for (size_t i = 0; i < op.lc.size(); ++i) c0.push_back(t++);
    merge_axes(av, b0, &sab, &bsz);
    merge_axes(av, f0, &sam, &m);
    merge_axes(av, c0, &sak, &k);
  }
  // B: k-contiguous ([n][k]) or n-contiguous ([k][n]) are native; else make it [b][n][k].
  if (!okb || !((k2 <= 1 || sbk == 1) || (nn <= 1 || sbn == 1))) {
    std::vector<size_t> order(op.rb);
    order.insert(order.end(), bfree.begin(), bfree.end());
    order.insert(order.end(), op.rc.begin(), op.rc.end());
    canon(bn, bv, bslot, order);
    std::vector<size_t> b0, f0, c0;
    size_t t = 0;
    for (size_t i = 0; i < op.rb.size(); ++i) b0.push_back(t++);
    for (size_t i = 0; i < bfree.size(); ++i) f0.push_back(t++);
    for (size_t i = 0; i < op.rc.size(); ++i) c0.push_back(t++);
    merge_axes(bv, b0, &sbb, &bsz2);
    merge_axes(bv, f0, &sbn, &nn);
    merge_axes(bv, c0, &sbk, &k2);
  }
  G.a_slot = aslot;
  G.b_slot = bslot;
  G.a_off = av.offset;
  G.b_off = bv.offset;
  G.sab = sab; G.sam = sam; G.sak = (k <= 1 ? 1 : sak);
  G.sbb = sbb; G.sbk = sbk; G.sbn = sbn;
  if (k2 <= 1) G.sbk = 1;
  if (nn <= 1 && G.sbk != 1) G.sbn = 1;
  G.batch = (size_t)bsz;
  G.m = (size_t)m;
  G.n = (size_t)nn;
  G.k = (size_t)k;
  G.in_dtype = in_dt;
  G.out_dtype = n.dtype;
  DType out_dt = n.dtype;
  if (fp8 != fp8_pat_.end()) {
    out_node = fp8->first == id ? id : id;
    // epilogue scales
    View sxv = dev_view_of(fp8->second.sx);
    View swv = dev_view_of(fp8->second.sw);
    if (vals_[fp8->second.sx].view.padded() || swv.padded()) throw Error("planner: padded fp8 scales");
    G.alpha_slot = vals_[fp8->second.sx].slot;
    G.alpha_off = sxv.offset;
    G.col_scale_slot = vals_[fp8->second.sw].slot;
    G.col_scale_off = swv.offset;
    G.col_scale_stride = swv.strides.empty() ? 1 : swv.strides.back();
    G.out_dtype = g_.dtype(fp8->second.dot);  // final cast dtype recorded as dot key
    out_dt = G.out_dtype;
  }
  auto cp = cast_pat_.find(id);
  if (cp != cast_pat_.end()) {
    out_dt = G.out_dtype = g_.node(cp->second).op.to;
    if (n.dtype != DType::F32) G.round_dtype = n.dtype;  // the dot's own rounding, then the cast's
  }
  int cslot = new_slot(SlotKind::Temp, out_dt, G.batch * G.m * G.n * dt_width(out_dt), id);
  G.c_slot = cslot;
  P_.gemms_.push_back(G);
  int step = new_step(Step::GEMM, (int)P_.gemms_.size() - 1, "gemm");
  depend(step, G.a_slot);
  depend(step, G.b_slot);
  if (G.alpha_slot >= 0) depend(step, G.alpha_slot);
  if (G.col_scale_slot >= 0) depend(step, G.col_scale_slot);
  slot_producer_[cslot] = step;
  Val v;
  v.k = Val::Dev;
  v.slot = cslot;
  v.view = View::contiguous(n.shape);
  NodeId target = id;
  if (fp8 != fp8_pat_.end()) target = fp8->second.dot;  // the pattern's final node
  if (cp != cast_pat_.end()) target = cp->second;
  vals_[target] = v;
  if (target != id) vals_[target].view = View::contiguous(g_.shape(target));
}

// Op::QuantMatmul (graph/ops/core/contract.rs:49-115): every operand as a contiguous device
// buffer; the output [M, N] in act's dtype.
void Planner::visit_quant(NodeId id) {
  const Node& n = g_.node(id);
  QuantStep Q;
  const DType at = g_.dtype(n.src[0]);
  if (!(at == DType::F32 || at == DType::BF16 || at == DType::F16))
    throw Error(std::string("kurumi_hip: quant_matmul act dtype ") + dt_name(at) + " is not supported on device");
  int slots[4] = {-1, -1, -1, -1};
  int64_t offs[4] = {0, 0, 0, 0};
  for (size_t i = 0; i < n.src.size(); ++i) {
    View v = dev_view_of(n.src[i]);
    slots[i] = vals_[n.src[i]].slot;
    if (!v.is_contiguous()) {  // the kernels take dense, 16-byte-aligned operands
      slots[i] = copy_view_to_slot(v, slots[i], g_.dtype(n.src[i]), n.src[i]);
      v = View::contiguous(v.shape);
    }
    offs[i] = v.offset;
  }
  const Shape& as = g_.shape(n.src[0]);
  Q.act_slot = slots[0]; Q.qw_slot = slots[1]; Q.sc_slot = slots[2]; Q.mn_slot = slots[3];
  Q.act_off = offs[0]; Q.qw_off = offs[1]; Q.sc_off = offs[2]; Q.mn_off = offs[3];
  Q.m = as[0]; Q.k = as[1]; Q.n = n.shape[1];
  Q.group = n.op.qgroup; Q.bits = n.op.qbits; Q.sym = n.op.qsym;
  Q.act_dtype = at;
  Q.wdq_dtype = at;  // bf16 / f16 act: the MFMA GEMM on rounded weights; f32: the generic GEMM
  Q.out_slot = new_slot(SlotKind::Temp, at, Q.m * Q.n * dt_width(at), id);
  // M <= 8: the fused dequant GEMV; int4 with 9 <= M <= 64 (bf16 / f16 act): the fused dequant
  // MFMA kernel; otherwise dequantise once into wdq, then the GEMM
  QuantArgs qa;
  qa.m = (int64_t)Q.m; qa.n = (int64_t)Q.n; qa.k = (int64_t)Q.k; qa.group = (int64_t)Q.group;
  qa.bits = Q.bits; qa.sym = Q.sym; qa.act_type = (int)at;
  qa.mins = Q.sym ? nullptr : reinterpret_cast<const uint16_t*>(16);  // shape check only
  Q.path = quant_gemv_ok(qa) ? QuantStep::GEMV : (quant_mm_ok(qa) ? QuantStep::MFMA : QuantStep::DEQUANT_GEMM);
  if (Q.path == QuantStep::DEQUANT_GEMM)
    Q.wdq_slot = new_slot(SlotKind::Temp, Q.wdq_dtype, Q.n * Q.k * dt_width(Q.wdq_dtype), id);
  if (Q.path == QuantStep::MFMA) {
    if (quant_mm_fused_ok(qa)) {
      // a constant weight, whole: the fused kernel reads its lane-ordered copy
      Q.tile_const = P_.slots_[Q.qw_slot].kind == SlotKind::Const && Q.qw_off == 0 &&
                     P_.slots_[Q.qw_slot].bytes == Q.n * Q.k / 2;
    } else {
      Q.mm_slot = new_slot(SlotKind::Temp, DType::U8, quant_mm_scratch_bytes(qa), id);
    }
  }
  P_.quants_.push_back(Q);
  int step = new_step(Step::QUANT, (int)P_.quants_.size() - 1, "quant");
  for (int i = 0; i < 4; ++i)
    if (slots[i] >= 0) depend(step, slots[i]);
  slot_producer_[Q.out_slot] = step;
  if (Q.wdq_slot >= 0) slot_producer_[Q.wdq_slot] = step;
  if (Q.mm_slot >= 0) slot_producer_[Q.mm_slot] = step;
  Val v;
  v.k = Val::Dev;
  v.slot = Q.out_slot;
  v.view = View::contiguous(n.shape);
  vals_[id] = v;
}

void Planner::visit_sdpa(NodeId id) {
  const Node& n = g_.node(id);
  AttnPattern pat;
  auto it = attn_pat_.find(id);
  if (it != attn_pat_.end()) {
    pat = it->second;
  } else {
    pat.q = n.src[0];
    pat.k = n.src[1];
    pat.v = n.src[2];
    pat.causal = n.op.causal;
    pat.scale = 1.0f / std::sqrt((float)g_.shape(pat.q).back());
  }
  const Shape& qs = g_.shape(pat.q);
  size_t r = qs.size();
  AttnStep A;
  A.s = qs[r - 2];
  A.d = qs[r - 1];
  A.bh = numel(qs) / (A.s * A.d);
  A.scale = pat.scale;
  A.causal = pat.causal;
  A.dtype = g_.dtype(pat.q);
  AttnArgs probe;
  probe.bh = (int64_t)A.bh;
  probe.s = (int64_t)A.s;
  probe.d = (int64_t)A.d;
  probe.dtype = (int)A.dtype;
  probe.causal = A.causal;
  if (!attn_supported(probe) || g_.shape(pat.k) != qs || g_.shape(pat.v) != qs)
    throw Error("kurumi_hip: attention shape/dtype not supported by the flash kernel: " + shape_str(qs) + " " +
                dt_name(A.dtype));
  int slots[3];
  NodeId ins[3] = {pat.q, pat.k, pat.v};
  for (int i = 0; i < 3; ++i) {
    View v = dev_view_of(ins[i]);
    slots[i] = vals_[ins[i]].slot;
    if (!v.is_contiguous()) {
      slots[i] = copy_view_to_slot(v, slots[i], g_.dtype(ins[i]), ins[i]);
    }
  }
  A.q_slot = slots[0];
  A.k_slot = slots[1];
  A.v_slot = slots[2];
  A.o_slot = new_slot(SlotKind::Temp, A.dtype, numel(qs) * dt_width(A.dtype), id);
  P_.attns_.push_back(A);
  int step = new_step(Step::ATTN, (int)P_.attns_.size() - 1, "attention");
  for (int s : slots) depend(step, s);
  slot_producer_[A.o_slot] = step;
  Val v;
  v.k = Val::Dev;
  v.slot = A.o_slot;
  v.view = View::contiguous(n.shape);
  vals_[id] = v;
}

// ---------------- pattern pre-pass ----------------

// Decomposed attention (graph/ops/nn/attention.rs:97-113):
//   raw = dot(q,k; lc=[r-1], rc=[r-1], batch) ; sc = raw * scalar(c) ; [sc += cast(expand(reshape(causal)))]
//   p = softmax(sc, r-1) ; out = dot(p, v; lc=[r-1], rc=[r-2], batch)
bool Planner::match_attention(NodeId d2) {
  const Node& n2 = g_.node(d2);
  if (n2.op.kind != OpKind::DotGeneral) return false;
  size_t r = n2.shape.size();
  if (r < 2) return false;
  std::vector<size_t> batch;
  for (size_t i = 0; i + 2 < r; ++i) batch.push_back(i);
  auto single = [&](NodeId x) { return consumers_[x] == 1 && !root_set_.count(x); };
  if (n2.op.lc != std::vector<size_t>{r - 1} || n2.op.rc != std::vector<size_t>{r - 2} || n2.op.lb != batch ||
      n2.op.rb != batch)
    return false;
  NodeId p = n2.src[0], v = n2.src[1];
  const Node& sm = g_.node(p);
  if (sm.op.kind != OpKind::Softmax || sm.op.axis != r - 1 || !single(p)) return false;
  NodeId sc = sm.src[0];
  if (!single(sc)) return false;
  std::vector<NodeId> absorbed = {p, sc};
  bool causal = false;
  const Node* mul = &g_.node(sc);
  if (mul->op.kind == OpKind::Add) {
    // one operand is the causal bias
    NodeId x0 = mul->src[0], b0 = mul->src[1];
    // The causal bias is Expand(Reshape(C[S,S], [1,..,1,S,S]), score shape), optionally cast
    // (attention.rs:139-153). Both targets are checked: a 0/-inf constant reshaped to, say,
    // [1,S,1,S] would mask along (head, key) instead of (query, key) and must stay unmatched.
    const Shape& score_shape = g_.shape(sc);
    auto is_bias = [&](NodeId b, std::vector<NodeId>& chain) {
      NodeId cur = b;
      if (g_.node(cur).op.kind == OpKind::Cast) { if (!single(cur)) return false; chain.push_back(cur); cur = g_.node(cur).src[0]; }
      if (g_.node(cur).op.kind != OpKind::Expand || !single(cur)) return false;
      if (g_.shape(cur) != score_shape) return false;
      chain.push_back(cur);
      cur = g_.node(cur).src[0];
      if (g_.node(cur).op.kind != OpKind::Reshape || !single(cur)) return false;
      const Shape& rs = g_.shape(cur);
      chain.push_back(cur);
      cur = g_.node(cur).src[0];
      const Node& c = g_.node(cur);
      if (c.op.kind != OpKind::Const || c.op.data_dtype != DType::F32 || c.shape.size() != 2 || c.shape[0] != c.shape[1])
        return false;
      size_t S = c.shape[0];
      if (rs.size() != r || rs[r - 2] != S || rs[r - 1] != S) return false;
      for (size_t i = 0; i + 2 < r; ++i)
        if (rs[i] != 1) return false;
      if (score_shape[r - 2] != S || score_shape[r - 1] != S) return false;
      const float* d = reinterpret_cast<const float*>(c.op.data->data());
      for (size_t i = 0; i < S; ++i)
        for (size_t j = 0; j < S; ++j) {
          float want = j > i ? -INFINITY : 0.f;
          if (!(d[i * S + j] == want)) return false;
        }
      return true;
    };
    std::vector<NodeId> chain;
    if (is_bias(b0, chain)) {
    } else {
      chain.clear();
      if (!is_bias(x0, chain)) return false;
      std::swap(x0, b0);
    }
    causal = true;
    absorbed.insert(absorbed.end(), chain.begin(), chain.end());
    if (!single(x0)) return false;
    absorbed.push_back(x0);
    mul = &g_.node(x0);
  }
  if (mul->op.kind != OpKind::Mul) return false;
  NodeId raw = mul->src[0], scn = mul->src[1];
  double c;
  auto scalar_of = [&](NodeId e, double* out) {
    const Node& en = g_.node(e);
    if (en.op.kind != OpKind::Expand) return false;
    return const_uniform_value(g_.node(en.src[0]), out);
  };
  if (!scalar_of(scn, &c)) {
    std::swap(raw, scn);
    if (!scalar_of(scn, &c)) return false;
  }
  absorbed.push_back(scn);
  const Node& d1 = g_.node(raw);
  if (d1.op.kind != OpKind::DotGeneral || !single(raw)) return false;
  if (d1.op.lc != std::vector<size_t>{r - 1} || d1.op.rc != std::vector<size_t>{r - 1} || d1.op.lb != batch ||
      d1.op.rb != batch)
    return false;
  absorbed.push_back(raw);
  NodeId q = d1.src[0], k = d1.src[1];
  if (g_.shape(q) != g_.shape(k) || g_.shape(q) != g_.shape(v)) return false;
  AttnArgs probe;
  const Shape& qs = g_.shape(q);
  probe.s = (int64_t)qs[r - 2];
  probe.d = (int64_t)qs[r - 1];
  probe.bh = (int64_t)(numel(qs) / (qs[r - 2] * qs[r - 1]));
  probe.dtype = (int)g_.dtype(q);
  probe.causal = causal;
  if (!attn_supported(probe)) return false;
  for (NodeId a : absorbed) absorbed_[a] = true;
  attn_pat_[d2] = AttnPattern{q, k, v, (float)c, causal};
  return true;
}

// fp8 quantized linear (the graph the fp8 mixed-precision pass emits):
//   y = cast_out( mul( mul( dot(cast_f32(xq:f8), cast_f32(wq:f8); lc=[1], rc=[1]), bcast(sx) ), bcast_rows(sw) ) )
bool Planner::match_fp8_epilogue(NodeId castn) {
  const Node& cn = g_.node(castn);
  if (cn.op.kind != OpKind::Cast) return false;
  auto single = [&](NodeId x) { return consumers_[x] == 1 && !root_set_.count(x); };
  NodeId m2 = cn.src[0];
  if (g_.node(m2).op.kind != OpKind::Mul || !single(m2)) return false;
  // e = Expand(Reshape(v, rs), es): the broadcast of a scale vector v. The reshape target rs
  // decides which output axis v runs along, so it is returned for the caller to check (a
  // per-row [M] scale reshaped to [M, 1] must never be taken for a per-column one, even when
  // M == N and the source shapes agree).
  struct Bcast { NodeId v; Shape rs, es; };
  auto bcast_src = [&](NodeId e, Bcast* b) -> bool {
    const Node& en = g_.node(e);
    if (en.op.kind != OpKind::Expand || !single(e)) return false;
    const Node& rn = g_.node(en.src[0]);
    if (rn.op.kind != OpKind::Reshape || !single(en.src[0])) return false;
    *b = Bcast{rn.src[0], rn.shape, en.shape};
    return true;
  };
  // mul = other * bcast(v) (either operand order) with `ok` accepting the broadcast
  auto split = [&](NodeId mul, NodeId* other, Bcast* b, const std::function<bool(const Bcast&)>& ok) {
    const Node& mn = g_.node(mul);
    for (int t = 0; t < 2; ++t) {
      Bcast c;
      if (bcast_src(mn.src[1 - t], &c) && ok(c)) { *other = mn.src[t]; *b = c; return true; }
    }
    return false;
  };
  const Shape& ys = g_.shape(m2);
  if (ys.size() != 2) return false;
  const size_t M = ys[0], N = ys[1];
  // per-column weight scale: sw [N] or [1, N] -> [1, N] -> [M, N]
  auto col_scale = [&](const Bcast& b) {
    const Shape& vs = g_.shape(b.v);
    return b.rs == Shape{1, N} && b.es == Shape{M, N} && (vs == Shape{N} || vs == Shape{1, N}) &&
           g_.dtype(b.v) == DType::F32;
  };
  // per-tensor activation scale: one element -> [1, 1] -> [M, N]
  auto tensor_scale = [&](const Bcast& b) {
    return b.rs == Shape{1, 1} && b.es == Shape{M, N} && numel(g_.shape(b.v)) == 1 && g_.dtype(b.v) == DType::F32;
  };
  NodeId m1, dot;
  Bcast swb, sxb;
  if (!split(m2, &m1, &swb, col_scale)) return false;
  if (g_.node(m1).op.kind != OpKind::Mul || !single(m1)) return false;
  if (!split(m1, &dot, &sxb, tensor_scale)) return false;
  const NodeId sw = swb.v, sx = sxb.v;
  const Node& dn = g_.node(dot);
  if (dn.op.kind != OpKind::DotGeneral || !single(dot) || dn.shape != (Shape{M, N})) return false;
  if (dn.op.lc != std::vector<size_t>{1} || dn.op.rc != std::vector<size_t>{1} || !dn.op.lb.empty()) return false;
  if (dn.dtype != DType::F32) return false;
  NodeId ca = dn.src[0], cb = dn.src[1];
  const Node &can = g_.node(ca), &cbn = g_.node(cb);
  if (can.op.kind != OpKind::Cast || cbn.op.kind != OpKind::Cast) return false;
  NodeId xq = can.src[0], wq = cbn.src[0];
  if (g_.dtype(xq) != DType::F8E4M3 || g_.dtype(wq) != DType::F8E4M3) return false;
  DType od = cn.op.to;
  if (od != DType::BF16 && od != DType::F16 && od != DType::F32) return false;
  // absorb the epilogue chain; the dot visit produces the cast's value
  std::vector<NodeId> ab = {m2, m1, g_.node(m2).src[0] == m1 ? g_.node(m2).src[1] : g_.node(m2).src[0]};
  for (NodeId x : ab) absorbed_[x] = true;
  // the broadcast chains of sx/sw
  for (NodeId mul : {m1, m2}) {
    const Node& mn = g_.node(mul);
    for (NodeId s : mn.src) {
      if (g_.node(s).op.kind == OpKind::Expand && s != dot && s != m1) {
        absorbed_[s] = true;
        absorbed_[g_.node(s).src[0]] = true;
      }
    }
  }
  if (single(ca)) absorbed_[ca] = true;
  if (single(cb)) absorbed_[cb] = true;
  absorbed_[castn] = true;
  fp8_pat_[dot] = Fp8Pattern{castn, xq, wq, sx, sw};
  return true;
}

// The activation half of the e4m3 linear (the chain the e4m3 pass emits, ir/pass_fp8.cpp):
//   xa = max(xf, neg(xf)), am = reduce_max(reduce_max(xa, 1), 0), sx = am * (1/448),
//   xq = cast_e4m3(xf2 * expand(reshape(recip(where(cmp_lt(0, sx), sx, 1)), [1, 1]), [M, K]))
// with xf, xf2 = x or cast_f32(x) and x a bf16 / f16 / f32 [M, K] value (the where makes an
// all-zero x divide by 1; a plain recip(sx) is accepted too). It becomes one ACTQ step
// (two kernels) producing xq and sx, in place of three generated kernels. Every absorbed node
// must be used only inside the chain (sx and xq may have other users: they are materialised).
bool Planner::match_actq(NodeId xq, NodeId sx) {
  auto kind = [&](NodeId n) { return g_.node(n).op.kind; };
  const Node& qn = g_.node(xq);
  if (qn.op.kind != OpKind::Cast || qn.dtype != DType::F8E4M3 || absorbed_[xq]) return false;
  const NodeId mul = qn.src[0];
  if (kind(mul) != OpKind::Mul) return false;
  // one operand is the broadcast reciprocal of sx, the other x as f32
  NodeId inv = 0, invr = 0, invb = 0, xf2 = 0;
  std::vector<NodeId> guard;  // the where(cmp_lt(0, sx), sx, 1) nodes, when present
  // s = expand(const v) with every element v (the builders' scalar)
  auto is_scalar = [&](NodeId e, double v) {
    NodeId c = kind(e) == OpKind::Expand ? g_.node(e).src[0] : e;
    double got;
    return const_uniform_value(g_.node(c), &got) && got == v;
  };
  auto guarded = [&](NodeId w) {
    const Node& wn = g_.node(w);
    if (wn.op.kind != OpKind::Where || wn.src[1] != sx || !is_scalar(wn.src[2], 1.0)) return false;
    const Node& cn = g_.node(wn.src[0]);
    if (cn.op.kind != OpKind::CmpLt || cn.src[1] != sx || !is_scalar(cn.src[0], 0.0)) return false;
    guard = {w, wn.src[0]};
    for (NodeId e : {wn.src[2], cn.src[0]}) {
      guard.push_back(e);
      if (kind(e) == OpKind::Expand) guard.push_back(g_.node(e).src[0]);
    }
    return true;
  };
  bool found = false;
  for (int t = 0; t < 2 && !found; ++t) {
    const NodeId e = g_.node(mul).src[t];
    if (kind(e) != OpKind::Expand) continue;
    const NodeId r = g_.node(e).src[0];
    if (kind(r) != OpKind::Reshape || g_.shape(r) != Shape{1, 1}) continue;
    const NodeId i = g_.node(r).src[0];
    if (kind(i) != OpKind::Recip) continue;
    guard.clear();
    if (g_.node(i).src[0] != sx && !guarded(g_.node(i).src[0])) continue;
    inv = i; invr = r; invb = e; xf2 = g_.node(mul).src[1 - t];
    found = true;
  }
  if (!found) return false;
  auto source_of = [&](NodeId f) -> NodeId {  // x for f = x (f32) or f = cast_f32(x)
    if (g_.dtype(f) != DType::F32) return Graph::kNoNode;
    if (kind(f) == OpKind::Cast) {
      NodeId x = g_.node(f).src[0];
      DType d = g_.dtype(x);
      return d == DType::BF16 || d == DType::F16 ? x : Graph::kNoNode;
    }
    return f;
  };
  const NodeId x = source_of(xf2);
  if (x == Graph::kNoNode) return false;
  const Shape& xs = g_.shape(x);
  if (xs.size() != 2 || g_.shape(invb) != xs || numel(xs) == 0) return false;
  // sx = am * (1/448)
  const Node& sn = g_.node(sx);
  if (sn.op.kind != OpKind::Mul || sn.dtype != DType::F32 || numel(sn.shape) != 1) return false;
  NodeId am = 0, sc = 0;
  found = false;
  for (int t = 0; t < 2 && !found; ++t) {
    NodeId c = sn.src[1 - t], cst = c;
    if (kind(c) == OpKind::Expand) cst = g_.node(c).src[0];
    double v;
    if (!const_uniform_value(g_.node(cst), &v) || g_.node(cst).op.data_dtype != DType::F32 ||
        (float)v != 1.0f / 448.0f)
      continue;
    am = sn.src[t];
    sc = c;
    found = true;
  }
  if (!found) return false;
  const Node& amn = g_.node(am);
  if (amn.op.kind != OpKind::ReduceMax || amn.op.axis != 0) return false;
  const NodeId rm = amn.src[0];
  const Node& rmn = g_.node(rm);
  if (rmn.op.kind != OpKind::ReduceMax || rmn.op.axis != 1 || g_.shape(rm) != Shape{xs[0]}) return false;
  const NodeId xa = rmn.src[0];
  const Node& xan = g_.node(xa);
  if (xan.op.kind != OpKind::Max) return false;
  NodeId xf = 0, ng = 0;
  found = false;
  for (int t = 0; t < 2 && !found; ++t) {
    NodeId a = xan.src[t], b = xan.src[1 - t];
    if (kind(b) == OpKind::Neg && g_.node(b).src[0] == a && source_of(a) == x) {
      xf = a; ng = b;
      found = true;
    }
  }
  if (!found) return false;
  // every absorbed node is used only by nodes of the chain
  std::set<NodeId> chain = {xa, ng, rm, am, inv, invr, invb, mul, sc, xq, sx};
  chain.insert(guard.begin(), guard.end());
  if (xf != x) chain.insert(xf);
  if (xf2 != x) chain.insert(xf2);
  if (kind(sc) == OpKind::Expand) chain.insert(g_.node(sc).src[0]);
  for (NodeId n : chain) {
    if (n == xq || n == sx) continue;
    if (root_set_.count(n) || absorbed_[n]) return false;
    for (NodeId u : users_[n])
      if (!chain.count(u)) return false;
  }
  for (NodeId n : chain)
    if (n != sx && n != xq) absorbed_[n] = true;
  absorbed_[xq] = true;  // produced together with sx
  actq_pat_[sx] = ActqPattern{x, xq};
  return true;
}

void Planner::visit_actq(NodeId sx) {
  const ActqPattern& p = actq_pat_.at(sx);
  const NodeId x = p.x;
  View xv = dev_view_of(x);
  int xs = vals_[x].slot;
  if (xv.padded() || !xv.is_contiguous() || xv.offset != 0) {
    xs = copy_view_to_slot(xv, xs, g_.dtype(x), x);
    xv = View::contiguous(xv.shape);
  }
  ActqStep A;
  A.x_slot = xs;
  A.x_dtype = g_.dtype(x);
  A.n = numel(g_.shape(x));
  A.xq_slot = new_slot(SlotKind::Temp, DType::F8E4M3, A.n, p.xq);
  A.sx_slot = new_slot(SlotKind::Temp, DType::F32, 4, sx);
  A.part_slot = new_slot(SlotKind::Temp, DType::F32, actq_partials_bytes((int64_t)A.n), sx);
  P_.actqs_.push_back(A);
  int step = new_step(Step::ACTQ, (int)P_.actqs_.size() - 1, "actq");
  depend(step, xs);
  slot_producer_[A.xq_slot] = step;
  slot_producer_[A.sx_slot] = step;
  slot_producer_[A.part_slot] = step;
  Val v;
  v.k = Val::Dev;
  v.slot = A.sx_slot;
  v.view = View::contiguous(g_.shape(sx));
  vals_[sx] = v;
  v.slot = A.xq_slot;
  v.view = View::contiguous(g_.shape(p.xq));
  vals_[p.xq] = v;
}

// cast(dot(a, b)) with float dtypes: the GEMM epilogue rounds the f32 accumulator to the dot's
// dtype and stores it converted to the cast's (graph/ops/core/convert.rs cast of a contraction
// result, e.g. the matmul-in-f16 policy of graph/pass/amp.rs:16-40 casting back to f32). Taken
// when the cast narrows or keeps the width (fewer bytes written than the dot's own output) or is
// itself a result of the plan; a widening cast feeding more elementwise work stays with that
// region, which reads the narrower dot output instead.
bool Planner::match_cast_epilogue(NodeId castn) {
  const Node& cn = g_.node(castn);
  NodeId dot = cn.src[0];
  const Node& dn = g_.node(dot);
  if (dn.op.kind != OpKind::DotGeneral || absorbed_[dot] || fp8_pat_.count(dot) || cast_pat_.count(dot)) return false;
  if (consumers_[dot] != 1 || root_set_.count(dot)) return false;
  auto f = [](DType d) { return d == DType::BF16 || d == DType::F16 || d == DType::F32; };
  const DType d = dn.dtype, t = cn.op.to;
  if (!f(d) || !f(t) || d == t) return false;
  if (dt_width(t) > dt_width(d) && !root_set_.count(castn)) return false;
  absorbed_[castn] = true;
  cast_pat_[dot] = castn;
  return true;
}

void Planner::find_patterns() {
  auto order = reachable_multi(g_, P_.roots_);
  consumers_.assign(g_.size(), 0);
  users_.assign(g_.size(), {});
  for (NodeId id : order)
    for (NodeId s : g_.node(id).src) {
      consumers_[s]++;
      users_[s].push_back(id);
    }
  absorbed_.assign(g_.size(), false);
  for (NodeId id : order) {
    const OpKind k = g_.node(id).op.kind;
    if (k == OpKind::DotGeneral && !absorbed_[id]) match_attention(id);
    if (k == OpKind::Cast && !absorbed_[id]) match_fp8_epilogue(id);
  }
  for (auto& kv : fp8_pat_) match_actq(kv.second.xq, kv.second.sx);
  for (NodeId id : order)
    if (g_.node(id).op.kind == OpKind::Cast && !absorbed_[id]) match_cast_epilogue(id);
}

void Planner::visit(NodeId id) {
  const Node& n = g_.node(id);
  if (actq_pat_.count(id)) {
    visit_actq(id);
    return;
  }
  switch (n.op.kind) {
    case OpKind::Input: {
      auto it = P_.input_slots_.find(id);
      int slot;
      if (it == P_.input_slots_.end()) {
        slot = new_slot(SlotKind::Input, n.dtype, numel(n.shape) * dt_width(n.dtype), id);
        P_.input_slots_[id] = slot;
      } else {
        slot = it->second;
      }
      Val v;
      v.k = Val::Dev;
      v.slot = slot;
      v.view = View::contiguous(n.shape);
      vals_[id] = v;
      return;
    }
    case OpKind::Const: {
      int slot = new_slot(SlotKind::Const, n.dtype, numel(n.shape) * dt_width(n.dtype), id);
      Val v;
      v.k = Val::Dev;
      v.slot = slot;
      v.view = View::contiguous(n.shape);
      vals_[id] = v;
      return;
    }
    case OpKind::Detach:
      vals_[id] = vals_[n.src[0]];
      return;
    case OpKind::Iota:
    case OpKind::RandUniform: {
      int rid = new_region(n.shape);
      RNode rn;
      rn.kind = (int)n.op.kind;
      rn.dtype = n.dtype;
      rn.axis = n.op.axis;
      rn.space = Space::Full;
      if (n.op.kind == OpKind::RandUniform) {
        NodeId s = n.src[0];
        View sv = dev_view_of(s);
        View u = sv;
        if (!view_reshape(sv, Shape{1}, &u)) throw Error("planner: rand seed must be a single element");
        View lv;
        lv.shape = P_.regions_[rid].S;
        lv.strides.assign(lv.shape.size(), 0);
        lv.offset = u.offset;
        rn.in = {add_leaf(rid, vals_[s].slot, lv, g_.dtype(s))};
      }
      int r = add_node(rid, rn);
      Val v;
      v.k = Val::LFull;
      v.region = rid;
      v.rn = r;
      vals_[id] = v;
      return;
    }
    case OpKind::Sum: case OpKind::Prod: case OpKind::ReduceMax: case OpKind::ArgReduce:
      // interp/reduce.rs:46 reads element 0 of the axis first: argmax / argmin over an empty
      // axis (with a non-empty result) is an error there too; sum / prod / max fold to identities
      if (n.op.kind == OpKind::ArgReduce && numel(g_.shape(n.src[0])) == 0 && numel(n.shape) > 0)
        throw Error("kurumi_hip: arg_reduce over an empty axis");
      visit_reduce(id);
      return;
    case OpKind::Softmax: case OpKind::RmsNorm:
      visit_rowop(id);
      return;
    case OpKind::Reshape: case OpKind::Expand: case OpKind::Permute: case OpKind::Slice: case OpKind::Flip:
    case OpKind::Pad:
      visit_movement(id);
      return;
    case OpKind::DotGeneral:
      if (attn_pat_.count(id)) { visit_sdpa(id); return; }
      visit_dot(id);
      return;
    case OpKind::Sdpa:
      visit_sdpa(id);
      return;
    case OpKind::QuantMatmul:
      visit_quant(id);
      return;
    default:
      if (is_elementwise(n.op.kind)) {
        if (dt_is_complex(n.dtype) || (n.src.size() && dt_is_complex(g_.dtype(n.src[0]))))
          throw Error("kurumi_hip: complex dtypes are not supported on device");
        visit_elementwise(id);
        return;
      }
      throw Error(std::string("kurumi_hip: op ") + op_name(n.op.kind) + " is not supported on device");
  }
}

void Planner::run() {
  const auto& roots = P_.roots_;
  for (NodeId r : roots) {
    if (r >= g_.size()) throw Error("eval: node id " + std::to_string(r) + " out of range");
    root_set_.insert(r);
  }
  find_patterns();
  vals_.assign(g_.size(), Val{});
  auto order = reachable_multi(g_, roots);
  std::sort(order.begin(), order.end());
  for (NodeId id : order) {
    if (absorbed_[id]) continue;
    visit(id);
  }
  // roots: contiguous device buffers
  for (NodeId r : roots) {
    if (vals_[r].k == Val::None) throw Error("planner: root " + std::to_string(r) + " was not produced");
    materialize(r);
    Val& v = vals_[r];
    if (!v.view.is_contiguous() || P_.slots_[v.slot].kind != SlotKind::Temp) {
      int s = copy_view_to_slot(v.view.shape.empty() ? View::contiguous({1}) : v.view, v.slot, g_.dtype(r), r);
      if (v.view.shape.empty()) {
        View c = v.view;
        c.shape = {1};
        c.strides = {0};
        s = copy_view_to_slot(c, v.slot, g_.dtype(r), r);
      }
      v.slot = s;
      v.view = View::contiguous(g_.shape(r));
    }
    P_.root_vals_.push_back({v.slot, v.view});
  }
  // execution order: topological over deps, stable by creation
  int ns = (int)P_.steps_.size();
  std::vector<int> state(ns, 0);
  std::function<void(int)> dfs = [&](int s) {
    if (state[s] == 2) return;
    if (state[s] == 1) throw Error("planner: dependency cycle");
    state[s] = 1;
    for (int d : P_.steps_[s].deps)
      if (step_alive_[d]) dfs(d);
    state[s] = 2;
    P_.order_.push_back(s);
  };
  for (int s = 0; s < ns; ++s)
    if (step_alive_[s] && (P_.steps_[s].type != Step::REGION || !P_.regions_[P_.steps_[s].index].outputs.empty()))
      dfs(s);  // a region nobody reads (its values were all moved into other regions) is not run
}

// ======================= plan =======================

static bool debug_enabled();

Plan::Plan(const Graph& g, const std::vector<NodeId>& roots, Context* ctx, ConstCache* consts)
    : bg_(&g), roots_(roots), ctx_(ctx) {
  if (roots.empty()) throw Error("eval: no output nodes");
  Planner pl(*this, consts);
  pl.run();
  for (auto& kv : input_slots_) input_meta_[kv.first] = {g.dtype(kv.first), g.shape(kv.first)};
  for (NodeId r : roots_) root_meta_.push_back({g.dtype(r), g.shape(r)});
  compile();
  if (ctx_) {
    try {
      bind_device_buffers(g, consts);
    } catch (...) {
      // the destructor does not run for a constructor that throws: give this plan's buffers
      // back to the pool (an allocation that failed on a full device must not leak the others)
      for (auto& sl : slots_)
        if (!sl.borrowed && sl.buf.ptr) ctx_->pool().release(sl.buf);
      throw;
    }
  }
  bg_ = nullptr;
}

void Plan::bind_device_buffers(const Graph& g, ConstCache* consts) {
  {
    allocate();
    std::map<int, ConstEntry*> const_of;  // slot -> its cache entry
    for (size_t i = 0; i < slots_.size(); ++i) {
      Slot& s = slots_[i];
      if (s.kind == SlotKind::Const) {
        const_refs_.push_back(consts->get(g, s.node));
        s.buf = const_refs_.back()->buf;
        s.borrowed = true;
        const_of[(int)i] = const_refs_.back().get();
      }
    }
    for (QuantStep& Q : quants_)
      if (Q.tile_const) {
        ConstEntry* e = const_of.at(Q.qw_slot);
        const auto key = std::make_pair((int64_t)Q.n, (int64_t)Q.k);
        auto it = e->tiled.find(key);
        if (it == e->tiled.end()) {
          DevBuf t = ctx_->pool().alloc(quant_tiled_bytes(key.first, key.second));
          it = e->tiled.emplace(key, t).first;
          e->nbytes += t.bytes;
          launch_quant_tile_weights(static_cast<const uint8_t*>(e->buf.ptr), static_cast<uint8_t*>(t.ptr), key.first,
                                    key.second, ctx_->stream());
          KU_HIP(hipGetLastError());
        }
        Q.qw_tiled = it->second.ptr;
      }
  }
}

Plan::~Plan() {
  if (hexec_) (void)hipGraphExecDestroy(hexec_);
  if (hgraph_) (void)hipGraphDestroy(hgraph_);
  if (ctx_) {
    for (auto& s : slots_)
      if (!s.borrowed && s.buf.ptr) ctx_->pool().release(s.buf);
  }
}

void Plan::compile() {
  for (int si : order_) {
    Step& s = steps_[si];
    if (s.type == Step::REGION) {
      RegionCode rc = gen_region(regions_[s.index], slots_, s.index);
      s.grid = rc.grid;
      s.block = rc.block;
      s.arg_slots = rc.arg_slots;
      s.label = rc.entry;
      sources_.push_back(rc.src);
      if (ctx_) s.fn = ctx_->modules().get(rc.src, rc.entry);
    } else if (s.type == Step::GEMM) {
      const GemmStep& G = gemms_[s.index];
      GemmArgs a;
      a.sab = G.sab; a.sam = G.sam; a.sak = G.sak; a.sbb = G.sbb; a.sbk = G.sbk; a.sbn = G.sbn;
      a.batch = (int64_t)G.batch; a.m = (int64_t)G.m; a.n = (int64_t)G.n; a.k = (int64_t)G.k;
      a.in_type = (int)G.in_dtype; a.out_type = (int)G.out_dtype;
      if (G.alpha_slot >= 0) a.alpha = reinterpret_cast<const float*>(16);
      std::ostringstream o;
      o << gemm_variant(a) << " b" << G.batch << " m" << G.m << " n" << G.n << " k" << G.k;
      if (G.out_dtype != G.in_dtype && G.alpha_slot < 0) o << " +cast " << dt_name(G.out_dtype);
      s.label = o.str();
    } else if (s.type == Step::ACTQ) {
      const ActqStep& A = actqs_[s.index];
      std::ostringstream o;
      o << "actq_e4m3 " << dt_name(A.x_dtype) << " n" << A.n;
      s.label = o.str();
    } else if (s.type == Step::QUANT) {
      const QuantStep& Q = quants_[s.index];
      std::ostringstream o;
      o << (Q.path == QuantStep::GEMV ? "quant_gemv" : Q.path == QuantStep::MFMA ? "quant_mfma" : "quant_dequant+gemm")
        << " int" << Q.bits << (Q.sym ? "s" : "a") << " g"
        << Q.group << " m" << Q.m << " n" << Q.n << " k" << Q.k;
      s.label = o.str();
    } else {
      const AttnStep& A = attns_[s.index];
      AttnArgs a;
      a.bh = (int64_t)A.bh; a.s = (int64_t)A.s; a.d = (int64_t)A.d; a.causal = A.causal; a.dtype = (int)A.dtype;
      std::ostringstream o;
      o << attn_variant(a) << " bh" << A.bh << " s" << A.s << " d" << A.d << (A.causal ? " causal" : "");
      s.label = o.str();
    }
  }
}

void Plan::allocate() {
  for (auto& s : slots_)
    if (s.kind != SlotKind::Const && !s.buf.ptr) s.buf = ctx_->pool().alloc(std::max<size_t>(s.bytes, 1));
}

std::vector<NodeId> Plan::inputs() const {
  std::vector<NodeId> r;
  for (auto& kv : input_slots_) r.push_back(kv.first);
  return r;
}

void Plan::feed(NodeId input, const Tensor& t) {
  auto it = input_slots_.find(input);
  if (it == input_slots_.end()) return;  // not reachable from the roots
  const auto& meta = input_meta_.at(input);
  if (t.dtype != meta.first || t.shape != meta.second)
    throw Error("feed for input %" + std::to_string(input) + ": got " + dt_name(t.dtype) + shape_str(t.shape) +
                ", expected " + dt_name(meta.first) + shape_str(meta.second));
  Slot& s = slots_[it->second];
  if (t.bytes.size() != s.bytes) throw Error("feed: byte size mismatch");
  if (!s.bytes) return;
  if (debug_enabled()) std::fprintf(stderr, "[kurumi_hip] feed %%%u -> %p (%zu bytes)\n", input, s.buf.ptr, s.bytes);
  ctx_->upload(s.buf.ptr, t.bytes.data(), s.bytes);
  ctx_->profile().launches[(int)Kind::Upload]++;
}

static void* slot_ptr(const std::vector<Slot>& slots, int i) { return slots[i].buf.ptr; }

static bool debug_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("KURUMI_HIP_DEBUG");
    return e && *e && *e != '0';
  }();
  return on;
}

void Plan::launch_step(const Step& s) {
  hipStream_t st = ctx_->stream();
  if (s.type == Step::REGION) {
    std::vector<void*> ptrs(s.arg_slots.size());
    std::vector<void*> args(s.arg_slots.size());
    for (size_t i = 0; i < s.arg_slots.size(); ++i) {
      ptrs[i] = slot_ptr(slots_, s.arg_slots[i]);
      args[i] = &ptrs[i];
    }
    if (s.grid == 0) return;
    KU_HIP(hipModuleLaunchKernel(s.fn.fn, s.grid, 1, 1, s.block, 1, 1, 0, st, args.data(), nullptr));
    ctx_->profile().launches[(int)Kind::Fused]++;
  } else if (s.type == Step::GEMM) {
    const GemmStep& G = gemms_[s.index];
    GemmArgs a;
    size_t iw = dt_width(G.in_dtype);
    a.a = static_cast<const char*>(slot_ptr(slots_, G.a_slot)) + G.a_off * (int64_t)iw;
    a.b = static_cast<const char*>(slot_ptr(slots_, G.b_slot)) + G.b_off * (int64_t)iw;
    a.c = slot_ptr(slots_, G.c_slot);
    a.sab = G.sab; a.sam = G.sam; a.sak = G.sak; a.sbb = G.sbb; a.sbk = G.sbk; a.sbn = G.sbn;
    a.batch = (int64_t)G.batch; a.m = (int64_t)G.m; a.n = (int64_t)G.n; a.k = (int64_t)G.k;
    a.in_type = (int)G.in_dtype;
    a.out_type = (int)G.out_dtype;
    a.round_type = G.round_dtype == DType::BF16 || G.round_dtype == DType::F16 ? (int)G.round_dtype : -1;
    if (G.alpha_slot >= 0) a.alpha = static_cast<const float*>(slot_ptr(slots_, G.alpha_slot)) + G.alpha_off;
    if (G.col_scale_slot >= 0) {
      a.col_scale = static_cast<const float*>(slot_ptr(slots_, G.col_scale_slot)) + G.col_scale_off;
      a.col_scale_stride = G.col_scale_stride;
    }
    if (G.batch * G.m * G.n == 0) return;
    if (debug_enabled())
      std::fprintf(stderr, "[kurumi_hip] gemm a=%p b=%p c=%p sa=(%lld,%lld,%lld) sb=(%lld,%lld,%lld) b%lld m%lld n%lld k%lld in%d out%d\n",
                   a.a, a.b, a.c, (long long)a.sab, (long long)a.sam, (long long)a.sak, (long long)a.sbb,
                   (long long)a.sbk, (long long)a.sbn, (long long)a.batch, (long long)a.m, (long long)a.n,
                   (long long)a.k, a.in_type, a.out_type);
    launch_gemm(a, st);
    KU_HIP(hipGetLastError());
    ctx_->profile().launches[(int)Kind::Gemm]++;
  } else if (s.type == Step::ACTQ) {
    const ActqStep& A = actqs_[s.index];
    ActQArgs a;
    a.x = slot_ptr(slots_, A.x_slot);
    a.x_type = (int)A.x_dtype;
    a.n = (int64_t)A.n;
    a.xq = static_cast<uint8_t*>(slot_ptr(slots_, A.xq_slot));
    a.sx = static_cast<float*>(slot_ptr(slots_, A.sx_slot));
    a.partials = static_cast<float*>(slot_ptr(slots_, A.part_slot));
    launch_actq(a, st);
    KU_HIP(hipGetLastError());
    ctx_->profile().launches[(int)Kind::Fused]++;
  } else if (s.type == Step::QUANT) {
    const QuantStep& Q = quants_[s.index];
    QuantArgs a;
    a.act = static_cast<const char*>(slot_ptr(slots_, Q.act_slot)) + Q.act_off * (int64_t)dt_width(Q.act_dtype);
    a.qw = static_cast<const uint8_t*>(slot_ptr(slots_, Q.qw_slot)) + Q.qw_off;
    a.scales = static_cast<const uint16_t*>(slot_ptr(slots_, Q.sc_slot)) + Q.sc_off;
    if (Q.mn_slot >= 0) a.mins = static_cast<const uint16_t*>(slot_ptr(slots_, Q.mn_slot)) + Q.mn_off;
    a.out = slot_ptr(slots_, Q.out_slot);
    a.m = (int64_t)Q.m; a.n = (int64_t)Q.n; a.k = (int64_t)Q.k; a.group = (int64_t)Q.group;
    a.bits = Q.bits; a.sym = Q.sym;
    a.act_type = (int)Q.act_dtype; a.wdq_type = (int)Q.wdq_dtype;
    if (Q.m * Q.n == 0) return;
    if (Q.path == QuantStep::GEMV) {
      launch_quant_gemv(a, st);
    } else if (Q.path == QuantStep::MFMA) {
      if (Q.mm_slot >= 0) a.mm_scratch = slot_ptr(slots_, Q.mm_slot);
      if (Q.qw_tiled) {
        a.qw = static_cast<const uint8_t*>(Q.qw_tiled);
        a.qw_tiled = true;
      }
      launch_quant_mm(a, st);
    } else {
      a.wdq = slot_ptr(slots_, Q.wdq_slot);
      launch_quant_dequant(a, st);
      KU_HIP(hipGetLastError());
      GemmArgs g;
      g.a = a.act; g.b = a.wdq; g.c = a.out;
      g.sam = (int64_t)Q.k; g.sak = 1; g.sab = 0;
      g.sbn = (int64_t)Q.k; g.sbk = 1; g.sbb = 0;  // B[k][n] = wdq[n][k]: the NT layout
      g.batch = 1; g.m = a.m; g.n = a.n; g.k = a.k;
      g.in_type = (int)Q.wdq_dtype; g.out_type = (int)Q.act_dtype;
      launch_gemm(g, st);
    }
    KU_HIP(hipGetLastError());
    ctx_->profile().launches[(int)Kind::Gemm]++;
  } else {
    const AttnStep& A = attns_[s.index];
    AttnArgs a;
    a.q = slot_ptr(slots_, A.q_slot);
    a.k = slot_ptr(slots_, A.k_slot);
    a.v = slot_ptr(slots_, A.v_slot);
    a.o = slot_ptr(slots_, A.o_slot);
    a.bh = (int64_t)A.bh; a.s = (int64_t)A.s; a.d = (int64_t)A.d;
    a.scale = A.scale;
    a.causal = A.causal;
    a.dtype = (int)A.dtype;
    launch_attention(a, st);
    KU_HIP(hipGetLastError());
    ctx_->profile().launches[(int)Kind::Attention]++;
  }
}

void Plan::launch(bool use_graph) {
  if (!ctx_) throw Error("plan has no device context");
  ctx_->make_current();
  if (use_graph) {
    if (!hexec_) {
      hipStream_t st = ctx_->stream();
      KU_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
      try {
        for (int si : order_) launch_step(steps_[si]);
      } catch (...) {
        hipGraph_t tmp;
        (void)hipStreamEndCapture(st, &tmp);
        throw;
      }
      KU_HIP(hipStreamEndCapture(st, &hgraph_));
      KU_HIP(hipGraphInstantiate(&hexec_, hgraph_, nullptr, nullptr, 0));
    }
    KU_HIP(hipGraphLaunch(hexec_, ctx_->stream()));
    return;
  }
  for (int si : order_) launch_step(steps_[si]);
}

void* Plan::output_ptr(size_t i) const { return slots_[root_vals_.at(i).first].buf.ptr; }

Tensor Plan::download(size_t i) {
  const auto& rv = root_vals_.at(i);
  Tensor t;
  t.dtype = root_meta_.at(i).first;
  t.shape = root_meta_.at(i).second;
  t.bytes.resize(numel(t.shape) * dt_width(t.dtype));  // left uninitialised: the copy writes every byte
  advise_huge(t.bytes.data(), t.bytes.size());
  if (!t.bytes.empty()) ctx_->download(t.bytes.data(), slots_[rv.first].buf.ptr, t.bytes.size());
  ctx_->sync();
  ctx_->profile().launches[(int)Kind::Download]++;
  return t;
}

std::string Plan::step_label(size_t i) const { return steps_[order_.at(i)].label; }

std::vector<std::string> Plan::sources() const { return sources_; }

std::vector<double> Plan::time_steps(int iters) {
  if (!ctx_) throw Error("plan has no device context");
  ctx_->make_current();
  hipStream_t st = ctx_->stream();
  const size_t n = order_.size();
  iters = std::max(iters, 1);
  // Two back-to-back runs of `iters` iterations on the plan's stream (events read once at the
  // end, so the stream never idles): one bracketed by a single pair of events gives the time per
  // iteration; one with events between the steps gives each step's share of it. An event between
  // two kernels keeps the next from starting until the previous has drained, so the per-step
  // events alone would charge every step that drain.
  hipEvent_t t0, t1;
  KU_HIP(hipEventCreate(&t0));
  KU_HIP(hipEventCreate(&t1));
  KU_HIP(hipEventRecord(t0, st));
  for (int it = 0; it < iters; ++it)
    for (size_t i = 0; i < n; ++i) launch_step(steps_[order_[i]]);
  KU_HIP(hipEventRecord(t1, st));
  KU_HIP(hipEventSynchronize(t1));
  float whole = 0.f;
  KU_HIP(hipEventElapsedTime(&whole, t0, t1));
  (void)hipEventDestroy(t0);
  (void)hipEventDestroy(t1);
  std::vector<double> acc(n, 0.0);
  if (n == 1) {
    acc[0] = whole / iters;
    return acc;
  }
  std::vector<hipEvent_t> ev((size_t)iters * (n + 1));
  for (auto& e : ev) KU_HIP(hipEventCreate(&e));
  for (int it = 0; it < iters; ++it) {
    hipEvent_t* e = &ev[(size_t)it * (n + 1)];
    KU_HIP(hipEventRecord(e[0], st));
    for (size_t i = 0; i < n; ++i) {
      launch_step(steps_[order_[i]]);
      KU_HIP(hipEventRecord(e[i + 1], st));
    }
  }
  KU_HIP(hipEventSynchronize(ev.back()));
  double sum = 0.0;
  for (int it = 0; it < iters; ++it) {
    hipEvent_t* e = &ev[(size_t)it * (n + 1)];
    for (size_t i = 0; i < n; ++i) {
      float ms = 0.f;
      KU_HIP(hipEventElapsedTime(&ms, e[i], e[i + 1]));
      acc[i] += ms;
      sum += ms;
    }
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  for (auto& a : acc) a = sum > 0 ? a / sum * (whole / iters) : a / iters;
  return acc;
}

}  // namespace ku::hipbk
