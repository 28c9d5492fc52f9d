// C ABI of libkurumi_hip.so (declared in include/kurumi_hip.h).
//
// Conventions follow the reference C ABI (kurumi/src/capi.rs:24-112): opaque heap handles,
// a thread-local last error, every entry null-checked and exception-safe, builders
// returning KU_ERR, pointer calls returning NULL, int calls returning 0 / -1.
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../../include/kurumi_hip.h"
#include "../hip/backend.h"
#include "../hip/kernels/kernels.h"
#include "errors.h"
#include "handles.h"
#include "../ir/graph.h"
#include "../ir/hostcopy.h"
#include "../ir/quant.h"
#include "../ir/tensor.h"

using ku::NodeId;
using ku::Shape;

// Plans keep the backend they were built on alive (shared ownership): a plan's steps use the
// backend's stream, pools and constant cache, so freeing the KuBackend handle first only drops
// the handle's reference and the backend ends with its last plan.
struct KuBackend { std::shared_ptr<ku::hipbk::HipBackend> b; };
struct KuPlan {
  std::shared_ptr<ku::hipbk::HipBackend> owner;  // null for the process-default backend
  std::shared_ptr<ku::hipbk::Plan> p;            // declared after owner: destroyed first
  uint64_t gid;              // the graph it was compiled on
  ku::hipbk::Hash128 fp;     // and that graph's content, for a run on an equal graph
  NodeId node;
};
struct KuHipPlan {
  std::shared_ptr<ku::hipbk::HipBackend> owner;
  std::unique_ptr<ku::hipbk::Plan> p;  // declared after owner: destroyed first
  ku::hipbk::HipBackend* b;
};

namespace {
thread_local std::string g_last_error;
thread_local bool g_has_error = false;
}  // namespace

void ku::capi::set_err(const std::string& m) {
  g_last_error = m;
  g_has_error = true;
}

namespace {

using ku::capi::guard;
using ku::capi::set_err;

Shape mk_shape(const size_t* s, size_t rank) {
  if (!s && rank) throw ku::Error("null shape pointer");
  return Shape(s, s + rank);
}

template <class F>
KuNode build(KuGraph* g, const char* name, F&& f) {
  if (!g) {
    set_err(std::string(name) + ": null graph handle");
    return KU_ERR;
  }
  return guard<KuNode>(KU_ERR, [&] { return static_cast<KuNode>(f(g->g)); });
}

ku::DType to_dt(uint32_t d) {
  if (d >= ku::kNumDTypes) throw ku::Error("unknown dtype tag " + std::to_string(d));
  return static_cast<ku::DType>(d);
}

// Process-default HIP backend (device 0) for ku_plan_compile, whose reference signature has no
// backend. Created on first use and deliberately never destroyed: static destructors run after
// the HIP runtime may have begun tearing down, and plans still held by the caller point into
// it. The driver returns its device memory when the process ends.
std::mutex g_default_mu;
ku::hipbk::HipBackend* g_default = nullptr;
ku::hipbk::HipBackend* default_backend() {
  std::lock_guard<std::mutex> lk(g_default_mu);
  if (!g_default) g_default = new ku::hipbk::HipBackend(0);
  return g_default;
}

KuPlan* compile_plan(ku::hipbk::HipBackend* b, std::shared_ptr<ku::hipbk::HipBackend> owner, const ku::Graph& g,
                     KuNode node) {
  auto* p = new KuPlan();
  p->owner = std::move(owner);
  try {
    p->p = b->plan_for(g, {node});
    p->gid = g.id();
    p->fp = ku::hipbk::graph_fingerprint(g, {node});
    p->node = node;
  } catch (...) {
    delete p;
    throw;
  }
  return p;
}

}  // namespace

extern "C" {

const char* ku_last_error(void) { return g_has_error ? g_last_error.c_str() : nullptr; }

KuGraph* ku_graph_new(void) { return new KuGraph(); }
void ku_graph_free(KuGraph* g) { delete g; }

KuNode ku_input(KuGraph* g, const size_t* shape, size_t rank, uint32_t dtype) {
  return build(g, "ku_input", [&](ku::Graph& gr) { return gr.input(mk_shape(shape, rank), to_dt(dtype)); });
}
KuNode ku_constant_f32(KuGraph* g, const float* data, size_t len, const size_t* shape, size_t rank) {
  return build(g, "ku_constant_f32", [&](ku::Graph& gr) {
    if (!data && len) throw ku::Error("ku_constant_f32: null data");
    return gr.constant_bytes(ku::DType::F32, reinterpret_cast<const uint8_t*>(data), len * 4, mk_shape(shape, rank));
  });
}
KuNode ku_constant(KuGraph* g, uint32_t dtype, const uint8_t* data, size_t nbytes, const size_t* shape, size_t rank) {
  return build(g, "ku_constant", [&](ku::Graph& gr) {
    if (!data && nbytes) throw ku::Error("ku_constant: null data");
    return gr.constant_bytes(to_dt(dtype), data, nbytes, mk_shape(shape, rank));
  });
}
KuNode ku_scalar(KuGraph* g, KuNode like, float v) {
  return build(g, "ku_scalar", [&](ku::Graph& gr) { return gr.scalar(like, v); });
}

#define KU_BIN(NAME, METHOD) \
  KuNode NAME(KuGraph* g, KuNode a, KuNode b) { return build(g, #NAME, [&](ku::Graph& gr) { return gr.METHOD(a, b); }); }
KU_BIN(ku_add, add)
KU_BIN(ku_sub, sub)
KU_BIN(ku_mul, mul)
KU_BIN(ku_div, div)
KU_BIN(ku_max, max)
KU_BIN(ku_idiv, idiv)
KU_BIN(ku_and, bit_and)
KU_BIN(ku_or, bit_or)
KU_BIN(ku_xor, bit_xor)
KU_BIN(ku_shl, shl)
KU_BIN(ku_shr, shr)
KU_BIN(ku_lt, cmp_lt)
KU_BIN(ku_eq, cmp_eq)
KU_BIN(ku_matmul, matmul)
#undef KU_BIN

KuNode ku_where(KuGraph* g, KuNode c, KuNode a, KuNode b) {
  return build(g, "ku_where", [&](ku::Graph& gr) { return gr.where(c, a, b); });
}

#define KU_UN(NAME, EXPR) \
  KuNode NAME(KuGraph* g, KuNode x) { return build(g, #NAME, [&](ku::Graph& gr) { return EXPR; }); }
KU_UN(ku_neg, gr.neg(x))
KU_UN(ku_recip, gr.recip(x))
KU_UN(ku_sqrt, gr.sqrt(x))
KU_UN(ku_square, gr.square(x))
KU_UN(ku_abs, gr.max(x, gr.neg(x)))
KU_UN(ku_floor, gr.floor(x))
KU_UN(ku_ceil, gr.ceil(x))
KU_UN(ku_round, gr.round(x))
KU_UN(ku_sign, gr.sign(x))
KU_UN(ku_exp, gr.exp(x))
KU_UN(ku_exp2, gr.exp2(x))
KU_UN(ku_ln, gr.ln(x))
KU_UN(ku_log2, gr.log2(x))
KU_UN(ku_sin, gr.sin(x))
KU_UN(ku_cos, gr.cos(x))
KU_UN(ku_relu, gr.relu(x))
KU_UN(ku_sigmoid, gr.sigmoid(x))
KU_UN(ku_silu, gr.silu(x))
KU_UN(ku_tanh, gr.tanh(x))
KU_UN(ku_gelu, gr.gelu(x))
KU_UN(ku_rope, gr.rope(x))
KU_UN(ku_detach, gr.detach(x))
KU_UN(ku_flatten, gr.reshape(x, Shape{ku::numel(gr.shape(x))}))
KU_UN(ku_t, gr.transpose(x, gr.shape(x).size() < 2 ? 0 : gr.shape(x).size() - 2, gr.shape(x).size() < 2 ? 0 : gr.shape(x).size() - 1))
KU_UN(ku_sum_all, gr.sum(gr.reshape(x, Shape{ku::numel(gr.shape(x))}), 0))
#undef KU_UN

#define KU_AX(NAME, EXPR) \
  KuNode NAME(KuGraph* g, KuNode x, size_t axis) { return build(g, #NAME, [&](ku::Graph& gr) { return EXPR; }); }
KU_AX(ku_sum, gr.sum(x, axis))
KU_AX(ku_prod, gr.prod(x, axis))
KU_AX(ku_mean, gr.mean(x, axis))
KU_AX(ku_reduce_max, gr.reduce_max(x, axis))
KU_AX(ku_reduce_min, gr.reduce_min(x, axis))
KU_AX(ku_logsumexp, gr.logsumexp(x, axis))
KU_AX(ku_log_softmax, gr.log_softmax(x, axis))
KU_AX(ku_argmax, gr.argreduce(x, axis, ku::ArgKind::Max))
KU_AX(ku_argmin, gr.argreduce(x, axis, ku::ArgKind::Min))
KU_AX(ku_softmax, gr.softmax(x, axis))
#undef KU_AX

KuNode ku_squeeze(KuGraph* g, KuNode x, size_t axis) {
  return build(g, "ku_squeeze", [&](ku::Graph& gr) {
    Shape s = gr.shape(x);
    if (axis >= s.size()) throw ku::Error("squeeze: axis out of range");
    if (s[axis] == 1) s.erase(s.begin() + axis);
    return gr.reshape(x, s);
  });
}
KuNode ku_unsqueeze(KuGraph* g, KuNode x, size_t axis) {
  return build(g, "ku_unsqueeze", [&](ku::Graph& gr) {
    Shape s = gr.shape(x);
    if (axis > s.size()) throw ku::Error("unsqueeze: axis out of range");
    s.insert(s.begin() + axis, 1);
    return gr.reshape(x, s);
  });
}
KuNode ku_clamp_min(KuGraph* g, KuNode x, float v) {
  return build(g, "ku_clamp_min", [&](ku::Graph& gr) { return gr.max(x, gr.scalar(x, v)); });
}
KuNode ku_rmsnorm(KuGraph* g, KuNode x, size_t axis, float eps) {
  return build(g, "ku_rmsnorm", [&](ku::Graph& gr) { return gr.rmsnorm(x, axis, eps); });
}

KuNode ku_dot_general(KuGraph* g, KuNode a, KuNode b, const size_t* lc, size_t nlc, const size_t* rc, size_t nrc,
                      const size_t* lb, size_t nlb, const size_t* rb, size_t nrb) {
  return build(g, "ku_dot_general", [&](ku::Graph& gr) {
    return gr.dot_general(a, b, mk_shape(lc, nlc), mk_shape(rc, nrc), mk_shape(lb, nlb), mk_shape(rb, nrb));
  });
}

// capi/ops/contract.rs:42-54: mins = KU_ERR selects the symmetric form
KuNode ku_quant_matmul(KuGraph* g, KuNode act, KuNode qweight, KuNode scales, KuNode mins, uint8_t bits,
                       size_t group_size) {
  return build(g, "ku_quant_matmul", [&](ku::Graph& gr) {
    return gr.quant_matmul(act, qweight, scales, mins == KU_ERR ? ku::Graph::kNoNode : mins, bits, group_size);
  });
}

// capi/ops/contract.rs:56-84
void ku_quantize(const float* w, size_t rows, size_t cols, uint8_t bits, size_t group_size, uint32_t symmetric,
                 uint8_t* out_packed, uint16_t* out_scales, uint16_t* out_mins) {
  if (!w || !out_packed || !out_scales) {
    set_err("ku_quantize: null w/out_packed/out_scales");
    return;
  }
  guard<int>(0, [&] {
    ku::Quantized q = ku::quantize(w, rows, cols, bits, group_size, symmetric != 0);
    std::memcpy(out_packed, q.packed.data(), q.packed.size());
    std::memcpy(out_scales, q.scales.data(), q.scales.size() * 2);
    if (!q.mins.empty() && out_mins) std::memcpy(out_mins, q.mins.data(), q.mins.size() * 2);
    return 0;
  });
}

KuNode ku_reshape(KuGraph* g, KuNode x, const size_t* shape, size_t rank) {
  return build(g, "ku_reshape", [&](ku::Graph& gr) { return gr.reshape(x, mk_shape(shape, rank)); });
}
KuNode ku_expand(KuGraph* g, KuNode x, const size_t* shape, size_t rank) {
  return build(g, "ku_expand", [&](ku::Graph& gr) { return gr.expand(x, mk_shape(shape, rank)); });
}
KuNode ku_permute(KuGraph* g, KuNode x, const size_t* perm, size_t rank) {
  return build(g, "ku_permute", [&](ku::Graph& gr) { return gr.permute(x, mk_shape(perm, rank)); });
}
KuNode ku_transpose(KuGraph* g, KuNode x, size_t i, size_t j) {
  return build(g, "ku_transpose", [&](ku::Graph& gr) { return gr.transpose(x, i, j); });
}
KuNode ku_flip(KuGraph* g, KuNode x, const size_t* axes, size_t n) {
  return build(g, "ku_flip", [&](ku::Graph& gr) { return gr.flip(x, mk_shape(axes, n)); });
}
KuNode ku_slice(KuGraph* g, KuNode x, const size_t* ranges, size_t rank) {
  return build(g, "ku_slice", [&](ku::Graph& gr) {
    if (!ranges && rank) throw ku::Error("ku_slice: null ranges");
    std::vector<ku::SliceRange> r;
    for (size_t i = 0; i < rank; ++i) r.push_back({ranges[2 * i], ranges[2 * i + 1], 1});
    return gr.slice(x, r);
  });
}
KuNode ku_slice_step(KuGraph* g, KuNode x, const size_t* ranges, size_t rank) {
  return build(g, "ku_slice_step", [&](ku::Graph& gr) {
    if (!ranges && rank) throw ku::Error("ku_slice_step: null ranges");
    std::vector<ku::SliceRange> r;
    for (size_t i = 0; i < rank; ++i) r.push_back({ranges[3 * i], ranges[3 * i + 1], ranges[3 * i + 2]});
    return gr.slice(x, r);
  });
}
KuNode ku_pad(KuGraph* g, KuNode x, const size_t* pads, size_t rank) {
  return build(g, "ku_pad", [&](ku::Graph& gr) {
    if (!pads && rank) throw ku::Error("ku_pad: null pads");
    std::vector<ku::PadRange> p;
    for (size_t i = 0; i < rank; ++i) p.push_back({pads[2 * i], pads[2 * i + 1]});
    return gr.pad(x, p);
  });
}
KuNode ku_broadcast_to(KuGraph* g, KuNode x, const size_t* shape, size_t rank) {
  return build(g, "ku_broadcast_to", [&](ku::Graph& gr) { return gr.broadcast_to(x, mk_shape(shape, rank)); });
}
KuNode ku_iota(KuGraph* g, const size_t* shape, size_t rank, size_t axis, uint32_t dtype) {
  return build(g, "ku_iota", [&](ku::Graph& gr) { return gr.iota(mk_shape(shape, rank), axis, to_dt(dtype)); });
}
KuNode ku_cast(KuGraph* g, KuNode x, uint32_t dtype) {
  return build(g, "ku_cast", [&](ku::Graph& gr) { return gr.cast(x, to_dt(dtype)); });
}
KuNode ku_bitcast(KuGraph* g, KuNode x, uint32_t dtype) {
  return build(g, "ku_bitcast", [&](ku::Graph& gr) { return gr.bitcast(x, to_dt(dtype)); });
}
KuNode ku_sdpa(KuGraph* g, KuNode q, KuNode k, KuNode v, uint32_t causal) {
  return build(g, "ku_sdpa", [&](ku::Graph& gr) { return gr.sdpa(q, k, v, causal != 0); });
}
KuNode ku_sdpa_decomposed(KuGraph* g, KuNode q, KuNode k, KuNode v, uint32_t causal) {
  return build(g, "ku_sdpa_decomposed", [&](ku::Graph& gr) { return gr.sdpa_decomposed(q, k, v, causal != 0); });
}
KuNode ku_sdpa_fused(KuGraph* g, KuNode q, KuNode k, KuNode v, uint32_t causal) {
  return build(g, "ku_sdpa_fused", [&](ku::Graph& gr) { return gr.sdpa_fused(q, k, v, causal != 0); });
}
KuNode ku_rand_uniform(KuGraph* g, const size_t* shape, size_t rank, uint64_t seed) {
  return build(g, "ku_rand_uniform", [&](ku::Graph& gr) { return gr.rand_uniform(mk_shape(shape, rank), seed); });
}
KuNode ku_randn(KuGraph* g, const size_t* shape, size_t rank, uint64_t seed) {
  return build(g, "ku_randn", [&](ku::Graph& gr) { return gr.randn(mk_shape(shape, rank), seed); });
}
KuNode ku_rand_range(KuGraph* g, const size_t* shape, size_t rank, uint64_t seed, float lo, float hi) {
  return build(g, "ku_rand_range", [&](ku::Graph& gr) { return gr.rand_range(mk_shape(shape, rank), seed, lo, hi); });
}
KuNode ku_amp(KuGraph* g, KuNode root) {
  return build(g, "ku_amp", [&](ku::Graph& gr) { return ku::amp(gr, root); });
}
KuNode ku_amp_fp8(KuGraph* g, KuNode root) {
  return build(g, "ku_amp_fp8", [&](ku::Graph& gr) { return ku::amp_fp8(gr, root); });
}

// ---------------- backend + eval ----------------

KuBackend* ku_backend_new(uint32_t kind) {
  if (kind == KU_CPU) {
    set_err("ku_backend_new: the CPU backend is kurumi's own interpreter; libkurumi_hip provides KU_HIP (2)");
    return nullptr;
  }
  if (kind == KU_METAL) {
    set_err("ku_backend_new: Metal backend is macOS-only");
    return nullptr;
  }
  if (kind != KU_HIP) {
    set_err("ku_backend_new: unknown kind " + std::to_string(kind));
    return nullptr;
  }
  return guard<KuBackend*>(nullptr, [&] {
    auto* b = new KuBackend();
    try {
      b->b = std::make_shared<ku::hipbk::HipBackend>(0);
    } catch (...) {
      delete b;
      throw;
    }
    return b;
  });
}
void ku_backend_free(KuBackend* b) { delete b; }

static KuTensor* eval_impl(KuGraph* g, KuNode node, const KuBackend* b, const ku::Feeds& f) {
  auto outs = b->b->eval_many(g->g, {node}, f);
  return new_ku_tensor(std::move(outs[0]));
}

KuTensor* ku_eval(KuGraph* g, KuNode node, const KuBackend* backend) {
  if (!g || !backend) {
    set_err("ku_eval: null graph/backend handle");
    return nullptr;
  }
  return guard<KuTensor*>(nullptr, [&] { return eval_impl(g, node, backend, ku::Feeds{}); });
}
KuTensor* ku_eval_with(KuGraph* g, KuNode node, const KuBackend* backend, const KuFeeds* feeds) {
  if (!g || !backend || !feeds) {
    set_err("ku_eval_with: null graph/backend/feeds handle");
    return nullptr;
  }
  return guard<KuTensor*>(nullptr, [&] { return eval_impl(g, node, backend, feeds->f); });
}
int32_t ku_eval_many(KuGraph* g, const KuNode* ids, size_t n, const KuBackend* backend, const KuFeeds* feeds,
                     KuTensor** out) {
  if (!g || !backend || !feeds || !out || (!ids && n > 0)) {
    set_err("ku_eval_many: null graph/backend/feeds/ids/out handle");
    return -1;
  }
  return guard<int32_t>(-1, [&] {
    std::vector<NodeId> v(ids, ids + n);
    auto outs = backend->b->eval_many(g->g, v, feeds->f);
    for (size_t i = 0; i < outs.size(); ++i) out[i] = new_ku_tensor(std::move(outs[i]));
    return 0;
  });
}

// ---------------- inspection ----------------

size_t ku_node_count(const KuGraph* g, KuNode root) {
  if (!g) {
    set_err("ku_node_count: null graph handle");
    return 0;
  }
  return guard<size_t>(0, [&] { return ku::reachable_multi(g->g, {root}).size(); });
}
size_t ku_dump(const KuGraph* g, KuNode root, uint8_t* out, size_t cap) {
  if (!g) {
    set_err("ku_dump: null graph handle");
    return 0;
  }
  return guard<size_t>(0, [&] {
    std::string s = ku::dump(g->g, root);
    if (out && cap) std::memcpy(out, s.data(), std::min(cap, s.size()));
    return s.size();
  });
}
size_t ku_node_rank(const KuGraph* g, KuNode node) {
  if (!g) {
    set_err("ku_node_rank: null graph handle");
    return SIZE_MAX;
  }
  return guard<size_t>(SIZE_MAX, [&] { return g->g.shape(node).size(); });
}
void ku_node_shape(const KuGraph* g, KuNode node, size_t* out) {
  if (!g || !out) return;
  guard<int>(0, [&] {
    const Shape& s = g->g.shape(node);
    std::memcpy(out, s.data(), s.size() * sizeof(size_t));
    return 0;
  });
}
uint32_t ku_node_dtype(const KuGraph* g, KuNode node) {
  if (!g) {
    set_err("ku_node_dtype: null graph handle");
    return KU_ERR;
  }
  return guard<uint32_t>(KU_ERR, [&] { return static_cast<uint32_t>(g->g.dtype(node)); });
}

// ---------------- plan-replay ----------------

KuPlan* ku_plan_compile(const KuGraph* g, KuNode node) {
  if (!g) {
    set_err("ku_plan_compile: null graph handle");
    return nullptr;
  }
  return guard<KuPlan*>(nullptr, [&] { return compile_plan(default_backend(), nullptr, g->g, node); });
}
KuPlan* ku_hip_plan_compile_on(const KuBackend* b, const KuGraph* g, KuNode node) {
  if (!b || !g) {
    set_err("ku_hip_plan_compile_on: null backend/graph handle");
    return nullptr;
  }
  return guard<KuPlan*>(nullptr, [&] { return compile_plan(b->b.get(), b->b, g->g, node); });
}
KuTensor* ku_plan_run(const KuPlan* p, const KuGraph* g, const KuFeeds* feeds) {
  if (!p || !g || !feeds) {
    set_err("ku_plan_run: null plan/graph/feeds handle");
    return nullptr;
  }
  return guard<KuTensor*>(nullptr, [&] {
    // realize/plan.rs:45: `g` must be the graph the plan was compiled on (or an equal one)
    if (g->g.id() != p->gid &&
        (p->node >= g->g.size() || ku::hipbk::graph_fingerprint(g->g, {p->node}) != p->fp))
      throw ku::Error("ku_plan_run: the plan was compiled on a different graph");
    ku::hipbk::feed_plan(*p->p, feeds->f);
    p->p->launch(true);
    return new_ku_tensor(p->p->download(0));
  });
}
void ku_plan_free(KuPlan* p) { delete p; }

// ---------------- feeds + tensors ----------------

KuFeeds* ku_feeds_new(void) { return new KuFeeds(); }
void ku_feeds_free(KuFeeds* f) { delete f; }
void ku_feeds_set(KuFeeds* f, KuNode node, const KuTensor* t) {
  if (!f || !t) return;
  f->f[node] = t->t;  // shared, not copied
}

KuTensor* ku_tensor_f32(const float* data, size_t len, const size_t* shape, size_t rank) {
  return guard<KuTensor*>(nullptr, [&] {
    if (!data && len) throw ku::Error("ku_tensor_f32: null data");  // capi/tensor.rs:57-60
    Shape s = mk_shape(shape, rank);
    if (ku::numel(s) != len) throw ku::Error("ku_tensor_f32: len does not match shape");
    ku::Tensor x;
    x.dtype = ku::DType::F32;
    x.shape = s;
    x.bytes.resize(len * 4);
    ku::advise_huge(x.bytes.data(), x.bytes.size());
    ku::par_copy(x.bytes.data(), data, len * 4);
    auto* t = new_ku_tensor(std::move(x));
    return t;
  });
}
KuTensor* ku_tensor_new(uint32_t dtype, const uint8_t* data, size_t nbytes, const size_t* shape, size_t rank) {
  return guard<KuTensor*>(nullptr, [&] {
    if (!data && nbytes) throw ku::Error("ku_tensor_new: null data");
    ku::DType dt = to_dt(dtype);
    Shape s = mk_shape(shape, rank);
    if (ku::numel(s) * ku::dt_width(dt) != nbytes) throw ku::Error("ku_tensor_new: nbytes does not match shape");
    ku::Tensor x;
    x.dtype = dt;
    x.shape = s;
    x.bytes.resize(nbytes);
    ku::advise_huge(x.bytes.data(), nbytes);
    ku::par_copy(x.bytes.data(), data, nbytes);
    auto* t = new_ku_tensor(std::move(x));
    return t;
  });
}
void ku_tensor_free(KuTensor* t) { delete t; }
size_t ku_tensor_rank(const KuTensor* t) { return t ? t->t->shape.size() : 0; }
void ku_tensor_shape(const KuTensor* t, size_t* out) {
  if (t && out) std::memcpy(out, t->t->shape.data(), t->t->shape.size() * sizeof(size_t));
}
size_t ku_tensor_len(const KuTensor* t) { return t ? ku::numel(t->t->shape) : 0; }
uint32_t ku_tensor_dtype(const KuTensor* t) { return t ? static_cast<uint32_t>(t->t->dtype) : KU_ERR; }
ptrdiff_t ku_tensor_data_f32(const KuTensor* t, float* out, size_t cap) {
  if (!t || !out) return -1;
  if (t->t->dtype != ku::DType::F32) {
    set_err("ku_tensor_data_f32: tensor is not F32");
    return -1;
  }
  size_t n = ku::numel(t->t->shape);
  if (cap < n) {
    set_err("ku_tensor_data_f32: buffer too small");
    return -1;
  }
  ku::par_copy(out, t->t->bytes.data(), n * 4);
  return static_cast<ptrdiff_t>(n);
}
size_t ku_tensor_nbytes(const KuTensor* t) { return t ? t->t->bytes.size() : 0; }
void ku_tensor_bytes(const KuTensor* t, uint8_t* out) {
  if (t && out && !t->t->bytes.empty()) ku::par_copy(out, t->t->bytes.data(), t->t->bytes.size());
}

// ---------------- device-resident plans ----------------

KuHipPlan* ku_hip_plan_new(KuGraph* g, const KuNode* roots, size_t n, const KuBackend* backend, const KuFeeds* feeds) {
  if (!g || !roots || !n || !backend || !feeds) {
    set_err("ku_hip_plan_new: null graph/roots/backend/feeds handle");
    return nullptr;
  }
  return guard<KuHipPlan*>(nullptr, [&] {
    auto* p = new KuHipPlan();
    p->owner = backend->b;
    p->b = backend->b.get();
    try {
      p->p = p->b->new_plan(g->g, std::vector<NodeId>(roots, roots + n));
      ku::hipbk::feed_plan(*p->p, feeds->f);
      p->b->ctx().sync();
    } catch (...) {
      delete p;
      throw;
    }
    return p;
  });
}
int32_t ku_hip_plan_feed(KuHipPlan* p, KuNode input, const KuTensor* t) {
  if (!p || !t) return -1;
  return guard<int32_t>(-1, [&] {
    p->p->feed(input, *t->t);
    return 0;
  });
}
int32_t ku_hip_plan_launch(KuHipPlan* p, uint32_t use_graph) {
  if (!p) return -1;
  return guard<int32_t>(-1, [&] {
    p->p->launch(use_graph != 0);
    return 0;
  });
}
int32_t ku_hip_plan_sync(KuHipPlan* p) {
  if (!p) return -1;
  return guard<int32_t>(-1, [&] {
    p->b->ctx().sync();
    return 0;
  });
}
KuTensor* ku_hip_plan_output(KuHipPlan* p, size_t i) {
  if (!p) return nullptr;
  return guard<KuTensor*>(nullptr, [&] { return new_ku_tensor(p->p->download(i)); });
}
size_t ku_hip_plan_num_steps(const KuHipPlan* p) { return p ? p->p->num_steps() : 0; }
size_t ku_hip_plan_step_label(const KuHipPlan* p, size_t i, char* out, size_t cap) {
  if (!p) return 0;
  return guard<size_t>(0, [&] {
    std::string s = p->p->step_label(i);
    if (out && cap) {
      size_t n = std::min(cap - 1, s.size());
      std::memcpy(out, s.data(), n);
      out[n] = 0;
    }
    return s.size();
  });
}
int32_t ku_hip_plan_time_steps(KuHipPlan* p, int32_t iters, double* out_ms, size_t cap) {
  if (!p || !out_ms) return -1;
  return guard<int32_t>(-1, [&] {
    auto t = p->p->time_steps(iters);
    for (size_t i = 0; i < t.size() && i < cap; ++i) out_ms[i] = t[i];
    return static_cast<int32_t>(t.size());
  });
}
double ku_hip_plan_time(KuHipPlan* p, int32_t iters, uint32_t use_graph) {
  if (!p) return -1.0;
  return guard<double>(-1.0, [&] {
    auto& ctx = p->b->ctx();
    ctx.make_current();
    hipEvent_t e0, e1;
    KU_HIP(hipEventCreate(&e0));
    KU_HIP(hipEventCreate(&e1));
    KU_HIP(hipEventRecord(e0, ctx.stream()));
    for (int i = 0; i < iters; ++i) p->p->launch(use_graph != 0);
    KU_HIP(hipEventRecord(e1, ctx.stream()));
    KU_HIP(hipEventSynchronize(e1));
    float ms = 0.f;
    KU_HIP(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return static_cast<double>(ms) / std::max(iters, 1);
  });
}
double ku_hip_plans_time(KuHipPlan* const* plans, size_t n, int32_t iters, uint32_t use_graph) {
  if (!plans || !n) {
    set_err("ku_hip_plans_time: no plans");
    return -1.0;
  }
  for (size_t i = 0; i < n; ++i)
    if (!plans[i] || plans[i]->b != plans[0]->b) {
      set_err("ku_hip_plans_time: null plan, or plans on different backends");
      return -1.0;
    }
  return guard<double>(-1.0, [&] {
    auto& ctx = plans[0]->b->ctx();
    ctx.make_current();
    hipEvent_t e0, e1;
    KU_HIP(hipEventCreate(&e0));
    KU_HIP(hipEventCreate(&e1));
    KU_HIP(hipEventRecord(e0, ctx.stream()));
    for (int i = 0; i < iters; ++i)
      for (size_t j = 0; j < n; ++j) plans[j]->p->launch(use_graph != 0);
    KU_HIP(hipEventRecord(e1, ctx.stream()));
    KU_HIP(hipEventSynchronize(e1));
    float ms = 0.f;
    KU_HIP(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return static_cast<double>(ms) / std::max(iters, 1);
  });
}
void ku_hip_plan_free(KuHipPlan* p) { delete p; }

size_t ku_hip_codegen(KuGraph* g, const KuNode* roots, size_t n, uint32_t compile, uint8_t* out, size_t cap) {
  if (!g || !roots || !n) {
    set_err("ku_hip_codegen: null graph/roots");
    return 0;
  }
  return guard<size_t>(0, [&] {
    ku::hipbk::Plan plan(g->g, std::vector<NodeId>(roots, roots + n), nullptr, nullptr);
    std::string all;
    for (auto& s : plan.sources()) {
      if (compile) ku::hipbk::rtc_compile(s, "ku_codegen");
      all += s;
      all += "\n// ----\n";
    }
    for (size_t i = 0; i < plan.num_steps(); ++i) all += "// step " + std::to_string(i) + ": " + plan.step_label(i) + "\n";
    if (out && cap) std::memcpy(out, all.data(), std::min(cap, all.size()));
    return all.size();
  });
}

int32_t ku_hip_linear_e4m3(const KuBackend* b, const void* x, uint32_t x_dtype, const uint8_t* wq, const float* sw,
                           void* y, uint32_t y_dtype, size_t m, size_t n, size_t k, void* stream) {
  if (!b) {
    set_err("ku_hip_linear_e4m3: null backend handle");
    return -1;
  }
  return guard<int32_t>(-1, [&] {
    ku::hipbk::LinearE4m3Args a;
    a.x = x;
    a.x_type = (int)x_dtype;
    a.wq = wq;
    a.sw = sw;
    a.y = y;
    a.y_type = (int)y_dtype;
    a.m = (int64_t)m;
    a.n = (int64_t)n;
    a.k = (int64_t)k;
    auto& ctx = b->b->ctx();
    ctx.make_current();
    const size_t need = ku::hipbk::linear_e4m3_scratch_bytes(a.m, a.k);
    void* ws = b->b->workspace(need);
    try {
      ku::hipbk::linear_e4m3(a, ws, need, stream ? static_cast<hipStream_t>(stream) : ctx.stream());
    } catch (const std::runtime_error& e) {
      throw ku::Error(std::string("ku_hip_linear_e4m3: ") + e.what());
    }
    return 0;
  });
}

int32_t ku_hip_linear_e4m3_noalloc(const void* x, uint32_t x_dtype, const uint8_t* wq, const float* sw, void* y,
                                   uint32_t y_dtype, size_t m, size_t n, size_t k, void* stream) {
  return guard<int32_t>(-1, [&] {
    ku::hipbk::LinearE4m3Args a;
    a.x = x;
    a.x_type = (int)x_dtype;
    a.wq = wq;
    a.sw = sw;
    a.y = y;
    a.y_type = (int)y_dtype;
    a.m = (int64_t)m;
    a.n = (int64_t)n;
    a.k = (int64_t)k;
    try {
      ku::hipbk::linear_e4m3_noalloc(a, static_cast<hipStream_t>(stream));
    } catch (const std::runtime_error& e) {
      throw ku::Error(std::string("ku_hip_linear_e4m3_noalloc: ") + e.what());
    }
    return 0;
  });
}

uint64_t ku_hip_profile(const KuBackend* b, uint64_t* out, size_t cap) {
  if (!b) return 0;
  auto& pr = b->b->ctx().profile();
  const size_t nk = (size_t)ku::hipbk::Kind::NumKinds;
  uint64_t extra[3] = {b->b->plans_built(), b->b->consts().uploads(), b->b->consts().entries()};
  for (size_t i = 0; out && i < cap && i < nk + 3; ++i) out[i] = i < nk ? pr.launches[i] : extra[i - nk];
  return pr.evals;
}

}  // extern "C"
