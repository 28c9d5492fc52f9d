// Device plan for one set of graph roots: the fusion planner's output and its executor.
//
// The planner walks the reachable nodes in id (= topological) order, like the Metal
// backend's memoised walk (kurumi_metal/src/backend/eval_walk.rs:73-138) and fusion
// accretion (backend/eval/fused.rs:13-145), but instead of one pointwise tree per kernel it
// builds *line regions*: elementwise chains, reductions along one axis and the values
// broadcast back along that axis, all evaluated by one kernel that owns whole lines.
// `Softmax`, `RmsNorm` and the decomposed softmax chain (interp/nn.rs:18-69,
// graph/ops/nn/activation.rs:122-129) therefore become a single pass over the data.
// Contractions and attention become GEMM / flash-attention steps.
#pragma once
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "../ir/graph.h"
#include "../ir/tensor.h"
#include "runtime.h"

namespace ku::hipbk {

// Element-strided view of a contiguous device buffer (movement ops compose into it;
// the reference's `View{base,strides,out_shape}`, kurumi_metal/src/backend/fuse.rs:70-80).
struct View {
  Shape shape;
  std::vector<int64_t> strides;
  int64_t offset = 0;
  // zero padding (Pad): element c reads offset + sum(c[d] * strides[d]) when every coordinate
  // lies in its window wlo[d] <= c[d] < whi[d], else 0. Windows are in this view's own
  // coordinates, so pads compose with slices, flips, permutes, expands and further pads; the
  // offset may point before the buffer (only valid coordinates are ever read). Empty when the
  // view is not padded.
  std::vector<int64_t> wlo, whi;
  bool padded() const { return !wlo.empty(); }
  static View contiguous(const Shape& s);
  bool is_contiguous() const;
};
bool view_reshape(const View& v, const Shape& to, View* out);
View view_expand(const View& v, const Shape& to);
View view_permute(const View& v, const std::vector<size_t>& perm);
View view_slice(const View& v, const std::vector<SliceRange>& r);
View view_flip(const View& v, const std::vector<size_t>& axes);
View view_pad(const View& v, const std::vector<PadRange>& p);

enum class SlotKind { Input, Const, Temp };
struct Slot {
  SlotKind kind = SlotKind::Temp;
  DType dtype = DType::F32;
  size_t bytes = 0;
  NodeId node = 0;
  DevBuf buf;           // owned unless `borrowed`
  bool borrowed = false;  // const cache buffers belong to the backend
};

enum class Space : uint8_t { Full, Line };

// Region expression node kinds: graph elementwise ops keep their OpKind value; the
// reductions are Sum/Prod/ReduceMax/ArgReduce; the rest are internal.
enum RK : int {
  RK_LEAF = 1000,    // read of leaf `leaf`
  RK_DIV,            // a / b (f32/f64 division, Softmax/RmsNorm)
  RK_EXP,            // natural exp (Softmax)
  RK_SQRT_ADD_EPS,   // sqrt(a / len + eps) (RmsNorm)
  RK_PADSEL,         // in[0] where the coordinate lies in the windows of `win`, else 0 (Pad)
};

struct RNode {
  int kind = RK_LEAF;
  DType dtype = DType::F32;   // value dtype (lowp values are carried as f32, rounded per op)
  Space space = Space::Full;
  std::vector<int> in;
  int leaf = -1;
  DType to = DType::F32;      // Cast/Bitcast target
  ArgKind arg = ArgKind::Max;
  size_t axis = 0;            // Iota axis
  float eps = 0.f;
  int level = 0;
  View win;                   // RK_PADSEL: only its wlo/whi windows are used
};

struct Leaf {
  int slot = -1;
  View view;          // over the region's iteration shape S (LINE leaves: stride 0 on the axis)
  DType dtype = DType::F32;
  // a constant read at one element everywhere (all strides 0, unpadded): its stored bits,
  // emitted as an immediate instead of a load
  bool imm = false;
  uint64_t imm_bits[2] = {0, 0};
};

struct Region {
  Shape S;
  int axis = -1;      // reduction axis; -1 = pure elementwise
  std::vector<RNode> nodes;
  std::vector<Leaf> leaves;
  std::vector<std::pair<int, int>> outputs;  // (rnode, slot)
  bool closed = false;
  std::string name;
};

struct GemmStep {
  // C[b, m, n] = sum_k A[b, m, k] * B[b, k, n] (+ fp8 epilogue scales), C contiguous.
  int a_slot = -1, b_slot = -1, c_slot = -1;
  int64_t a_off = 0, b_off = 0;
  int64_t sab = 0, sam = 0, sak = 0;   // A strides (elements)
  int64_t sbb = 0, sbk = 0, sbn = 0;   // B strides
  size_t batch = 1, m = 0, n = 0, k = 0;
  DType in_dtype = DType::BF16, out_dtype = DType::BF16;
  // fp8 epilogue: C = round(acc * (*alpha) * col_scale[n]); alpha/col_scale from slots
  int alpha_slot = -1, col_scale_slot = -1;
  int64_t alpha_off = 0, col_scale_off = 0, col_scale_stride = 1;
  // fused cast epilogue: round to round_dtype (the dot's bf16 / f16) before storing out_dtype;
  // F32 = no extra rounding
  DType round_dtype = DType::F32;
  std::string variant;
};

// Weight-only quantized matmul: a fused dequant GEMV (M <= 8), the fused dequant MFMA kernel
// (int4, 9 <= M <= 64), else a dequantize pass into `wdq_slot` followed by a GEMM of act x wdq^T.
// `tile_const`: the MFMA path's fused kernel reads a constant weight from its lane-ordered copy
// (`qw_tiled`, held by the constant's cache entry).
struct QuantStep {
  enum Path { GEMV, MFMA, DEQUANT_GEMM };
  Path path = GEMV;
  int act_slot = -1, qw_slot = -1, sc_slot = -1, mn_slot = -1, out_slot = -1, wdq_slot = -1, mm_slot = -1;
  int64_t act_off = 0, qw_off = 0, sc_off = 0, mn_off = 0;  // elements
  size_t m = 0, n = 0, k = 0, group = 0;
  int bits = 4;
  bool sym = true;
  DType act_dtype = DType::BF16, wdq_dtype = DType::BF16;
  bool tile_const = false;
  const void* qw_tiled = nullptr;
};

struct AttnStep {
  int q_slot = -1, k_slot = -1, v_slot = -1, o_slot = -1;
  size_t bh = 0, s = 0, d = 0;
  float scale = 1.f;
  bool causal = false;
  DType dtype = DType::BF16;
};

// Per-tensor e4m3 quantisation of a linear layer's activation (the chain the e4m3 pass emits
// before its GEMM): sx = max|x| * (1/448), xq = e4m3(x * (1/sx)); two kernels, partials scratch.
struct ActqStep {
  int x_slot = -1, xq_slot = -1, sx_slot = -1, part_slot = -1;
  size_t n = 0;
  DType x_dtype = DType::BF16;
};

struct Step {
  enum Type { REGION, GEMM, ATTN, QUANT, ACTQ } type;
  int index;             // into regions / gemms / attns
  std::set<int> deps;    // producer step ids
  // compiled launch (regions)
  KernelFn fn;
  unsigned grid = 0, block = 0;
  std::vector<int> arg_slots;
  std::string label;
};

// One uploaded constant. Plans hold it through a shared_ptr, so a buffer is returned to the
// pool only once neither the cache nor any plan uses it. A packed int4 weight that the fused
// QuantMatmul kernel reads also gets a lane-ordered copy per [n, k] it is read as (one packed
// constant may be reshaped to several; each copy is made once, on the stream, when the first
// plan needs it), counted in `nbytes` and freed only with the entry, since plans and captured
// hipGraphs hold its address.
struct ConstEntry {
  Pool* pool = nullptr;
  DevBuf buf;
  std::map<std::pair<int64_t, int64_t>, DevBuf> tiled;  // (n, k) -> lane-ordered copy
  size_t nbytes = 0;
  uint64_t last_use = 0;
  ~ConstEntry() {
    if (pool) {
      pool->release(buf);
      for (auto& kv : tiled) pool->release(kv.second);
    }
  }
};

class Backend;  // HipBackend (backend.h)

class Plan {
 public:
  // Build the plan for `roots` of `g`. Input shapes come from the graph's Input nodes;
  // `ctx` may be null for a codegen-only plan (no device buffers, no launches).
  Plan(const Graph& g, const std::vector<NodeId>& roots, Context* ctx, class ConstCache* consts);
  ~Plan();

  // Upload an Input's host value (must match the declared shape and dtype).
  void feed(NodeId input, const Tensor& t);
  // Enqueue every step on the context stream (async). With `graph` true the steps are
  // recorded once into a hipGraph and replayed on later calls.
  void launch(bool use_graph = false);
  Tensor download(size_t i);
  size_t num_outputs() const { return roots_.size(); }
  void* output_ptr(size_t i) const;

  // Introspection
  size_t num_steps() const { return order_.size(); }
  std::string step_label(size_t i) const;
  std::vector<std::string> sources() const;
  // Average GPU ms of each step over `iters` launches, timed with hipEvents on the stream.
  std::vector<double> time_steps(int iters);
  std::vector<NodeId> inputs() const;

 private:
  friend class Planner;
  void compile();
  void allocate();
  // device buffers of the slots, the constants from the cache and their lane-ordered copies
  void bind_device_buffers(const Graph& g, ConstCache* consts);
  void launch_step(const Step& s);

  const Graph* bg_ = nullptr;  // the graph being planned; valid during construction only
  std::vector<NodeId> roots_;
  // what feed() and download() check against, so a built plan never reads its graph again
  // (a content-equal graph may reuse it after the original is freed)
  std::map<NodeId, std::pair<DType, Shape>> input_meta_;
  std::vector<std::pair<DType, Shape>> root_meta_;
  std::vector<std::shared_ptr<ConstEntry>> const_refs_;
  Context* ctx_;
  std::vector<Slot> slots_;
  std::vector<Region> regions_;
  std::vector<GemmStep> gemms_;
  std::vector<AttnStep> attns_;
  std::vector<QuantStep> quants_;
  std::vector<ActqStep> actqs_;
  std::vector<Step> steps_;
  std::vector<int> order_;                 // execution order of steps
  std::map<NodeId, int> input_slots_;
  std::vector<std::pair<int, View>> root_vals_;  // slot + view of each root
  std::vector<std::string> sources_;
  hipGraph_t hgraph_ = nullptr;
  hipGraphExec_t hexec_ = nullptr;
};

// Backend-owned cache of uploaded constants (kurumi_metal/src/backend.rs:23-26,
// eval_walk.rs:99-114 key theirs by graph id and node). Here the key is the payload's content
// (dtype, shape, byte count and a 128-bit hash of the bytes), with (graph id, node) as a fast
// path, so a graph rebuilt with the same weights reuses their device copies. Entries that no
// live plan holds are kept up to a byte budget (KURUMI_HIP_CONST_CACHE_MB, default 2048),
// least recently used first out, and all of them are dropped when an allocation fails.
class ConstCache {
 public:
  explicit ConstCache(Context* ctx);
  ~ConstCache();
  std::shared_ptr<ConstEntry> get(const Graph& g, NodeId id);
  // Drop every entry no plan holds; returns the bytes released.
  size_t reclaim();
  size_t entries() const { return by_content_.size(); }
  size_t uploads() const { return uploads_; }

 private:
  struct Key {
    uint64_t h0, h1, nbytes;
    uint32_t dtype;
    Shape shape;
    bool operator<(const Key& o) const {
      if (h0 != o.h0) return h0 < o.h0;
      if (h1 != o.h1) return h1 < o.h1;
      if (nbytes != o.nbytes) return nbytes < o.nbytes;
      if (dtype != o.dtype) return dtype < o.dtype;
      return shape < o.shape;
    }
  };
  void enforce_budget();
  Context* ctx_;
  std::map<Key, std::shared_ptr<ConstEntry>> by_content_;
  std::map<std::pair<uint64_t, NodeId>, Key> by_node_;
  uint64_t clock_ = 0;
  size_t uploads_ = 0;
  size_t budget_;
};

// Generated-source entry points (codegen.cpp)
struct RegionCode {
  std::string src, entry;
  unsigned grid = 0, block = 0;
  std::vector<int> arg_slots;  // leaf/output slots in kernel parameter order
};
RegionCode gen_region(const Region& r, const std::vector<Slot>& slots, int index);

}  // namespace ku::hipbk
