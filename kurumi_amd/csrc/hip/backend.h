// HipBackend: the MI355X implementation of the backend seam
// (kurumi_core/src/backend.rs:14-31; the Metal analog is kurumi_metal/src/backend.rs:19-109).
// Every op it accepts runs on the device; an op outside its scope is an error, never a
// silent CPU fallback.
#pragma once
#include <list>
#include <memory>

#include "../ir/tensor.h"
#include "fingerprint.h"
#include "plan.h"
#include "runtime.h"

namespace ku::hipbk {

class HipBackend : public ku::Backend {
 public:
  explicit HipBackend(int device);
  ~HipBackend() override;
  const char* name() const override { return "hip"; }
  std::vector<Tensor> eval_many(const Graph& g, const std::vector<NodeId>& ids, const Feeds& feeds) override;

  // A device plan for `roots`, cached by (graph id, graph size, roots) and, on a miss there,
  // by the content fingerprint of the reachable subgraph, so an identical graph rebuilt per
  // call (the KGPH v2 seam) reuses the plan and its uploaded constants.
  std::shared_ptr<Plan> plan_for(const Graph& g, const std::vector<NodeId>& roots);
  size_t plans_built() const { return plans_built_; }
  std::unique_ptr<Plan> new_plan(const Graph& g, const std::vector<NodeId>& roots);
  Context& ctx() { return *ctx_; }
  // Grow-only device workspace of the direct kernel entry points (ku_hip_linear_e4m3): at least
  // `bytes`, reused by every call on this backend (calls must be ordered on one stream).
  void* workspace(size_t bytes);
  ConstCache& consts() { return *consts_; }

 private:
  std::unique_ptr<Context> ctx_;
  std::unique_ptr<ConstCache> consts_;
  struct Entry {
    uint64_t gid;
    size_t gsize;
    std::vector<NodeId> roots;
    Hash128 fp;
    std::shared_ptr<Plan> plan;
  };
  std::list<Entry> plans_;  // most recent first
  DevBuf ws_;
  size_t plans_built_ = 0;
};

void feed_plan(Plan& p, const Feeds& feeds);

}  // namespace ku::hipbk
