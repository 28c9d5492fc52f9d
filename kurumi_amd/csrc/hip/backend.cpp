#include "backend.h"

#include "kernels/kernels.h"

namespace ku::hipbk {

namespace {
constexpr size_t kMaxCachedPlans = 8;
}

HipBackend::HipBackend(int device) {
  ctx_ = std::make_unique<Context>(device);
  consts_ = std::make_unique<ConstCache>(ctx_.get());
  ctx_->make_current();
  init_linear_e4m3_noalloc();  // the no-allocation entry point's scratch on this device
}

HipBackend::~HipBackend() {
  if (ws_.ptr) {
    (void)hipDeviceSynchronize();
    ctx_->pool().release(ws_);
  }
  plans_.clear();
  consts_.reset();
  ctx_.reset();
}

std::unique_ptr<Plan> HipBackend::new_plan(const Graph& g, const std::vector<NodeId>& roots) {
  ctx_->make_current();
  return std::make_unique<Plan>(g, roots, ctx_.get(), consts_.get());
}

std::shared_ptr<Plan> HipBackend::plan_for(const Graph& g, const std::vector<NodeId>& roots) {
  for (auto it = plans_.begin(); it != plans_.end(); ++it) {
    if (it->gid == g.id() && it->gsize == g.size() && it->roots == roots) {
      if (it != plans_.begin()) plans_.splice(plans_.begin(), plans_, it);
      return plans_.front().plan;
    }
  }
  // A plan never reads its graph after construction, so one built for an equal graph serves.
  const Hash128 fp = graph_fingerprint(g, roots);
  for (auto it = plans_.begin(); it != plans_.end(); ++it) {
    if (it->fp == fp && it->roots == roots) {
      it->gid = g.id();
      it->gsize = g.size();
      if (it != plans_.begin()) plans_.splice(plans_.begin(), plans_, it);
      return plans_.front().plan;
    }
  }
  std::shared_ptr<Plan> p(new_plan(g, roots).release());
  plans_built_++;
  plans_.push_front(Entry{g.id(), g.size(), roots, fp, p});
  while (plans_.size() > kMaxCachedPlans) plans_.pop_back();
  return p;
}

void* HipBackend::workspace(size_t bytes) {
  if (ws_.ptr && ws_.bytes >= bytes) return ws_.ptr;
  ctx_->make_current();
  if (ws_.ptr) {
    // kernels of earlier calls (on whatever stream the caller gave) may still read the old one
    KU_HIP(hipDeviceSynchronize());
    ctx_->pool().release(ws_);
    ws_ = DevBuf{};
  }
  ws_ = ctx_->pool().alloc(bytes);
  return ws_.ptr;
}

void feed_plan(Plan& p, const Feeds& feeds) {
  for (NodeId in : p.inputs()) {
    auto it = feeds.find(in);
    if (it == feeds.end()) throw Error("eval: missing feed for Input node %" + std::to_string(in));
    p.feed(in, *it->second);
  }
}

// Mirrors MetalBackend::eval_many_with (kurumi_metal/src/backend.rs:95-109): one shared
// pass over all ids, results downloaded as owned host tensors.
std::vector<Tensor> HipBackend::eval_many(const Graph& g, const std::vector<NodeId>& ids, const Feeds& feeds) {
  if (ids.empty()) return {};
  ctx_->make_current();
  std::shared_ptr<Plan> p = plan_for(g, ids);
  feed_plan(*p, feeds);
  p->launch(false);
  std::vector<Tensor> out;
  out.reserve(ids.size());
  for (size_t i = 0; i < ids.size(); ++i) out.push_back(p->download(i));
  ctx_->profile().evals++;
  return out;
}

}  // namespace ku::hipbk
