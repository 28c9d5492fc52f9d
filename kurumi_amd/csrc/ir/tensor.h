// Host tensor value and feeds: the owned, row-major little-endian result the backend
// seam returns (kurumi_core/src/dtype.rs:178-192 `TensorVal`, backend.rs:12 `Feeds`).
#pragma once
#include <cstdint>
#include <memory>
#include <new>
#include <type_traits>
#include <utility>
#include <unordered_map>
#include <vector>

#include "dtype.h"
#include "graph.h"

namespace ku {

// std::allocator that default-initialises (leaves uninitialised) the elements `resize` adds. A
// tensor's bytes are always written whole by the copy that fills them, so value-initialising a
// GB-sized download buffer first would be a wasted pass over host memory.
template <class T>
struct NoInitAlloc : std::allocator<T> {
  template <class U>
  struct rebind { using other = NoInitAlloc<U>; };
  NoInitAlloc() noexcept = default;
  template <class U>
  NoInitAlloc(const NoInitAlloc<U>&) noexcept {}
  template <class U>
  void construct(U* p) noexcept(std::is_nothrow_default_constructible<U>::value) { ::new (static_cast<void*>(p)) U; }
  template <class U, class... A>
  void construct(U* p, A&&... a) { ::new (static_cast<void*>(p)) U(std::forward<A>(a)...); }
};
using Bytes = std::vector<uint8_t, NoInitAlloc<uint8_t>>;

struct Tensor {
  DType dtype = DType::F32;
  Shape shape;
  Bytes bytes;
  size_t nbytes() const { return bytes.size(); }
};

using Feeds = std::unordered_map<NodeId, std::shared_ptr<const Tensor>>;

// The backend seam (kurumi_core/src/backend.rs:14-31): evaluate one or several nodes of a
// borrowed graph with `Input` nodes bound by `feeds`; results are owned host tensors.
// `eval_many` shares one pass across ids and must equal per-node evaluation.
class Backend {
 public:
  virtual ~Backend() = default;
  virtual const char* name() const = 0;
  virtual std::vector<Tensor> eval_many(const Graph& g, const std::vector<NodeId>& ids, const Feeds& feeds) = 0;
  Tensor eval_with(const Graph& g, NodeId id, const Feeds& feeds) { return eval_many(g, {id}, feeds)[0]; }
};

}  // namespace ku
