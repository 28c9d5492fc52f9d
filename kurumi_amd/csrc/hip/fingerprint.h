// Content fingerprints of graphs and constant payloads.
//
// The backend caches plans and uploaded constants by graph id (kurumi_metal/src/backend.rs:23-26
// keys its caches the same way). A caller that rebuilds an identical graph per call — the
// KGPH v2 seam decodes a fresh graph from the same bytes every time — would miss both caches,
// so each is also keyed by content: a 128-bit fingerprint of the nodes reachable from the
// roots (node ids, op attributes, dtypes, shapes, sources and constant payload bytes). The
// hash is non-cryptographic (two independent 64-bit multiply-rotate lanes); it guards against
// accidental equality, not against adversarial inputs.
#pragma once
#include <cstddef>
#include <cstdint>
#include <memory>
#include <vector>

#include "../ir/graph.h"

namespace ku::hipbk {

struct Hash128 {
  uint64_t lo = 0, hi = 0;
  bool operator==(const Hash128& o) const { return lo == o.lo && hi == o.hi; }
  bool operator!=(const Hash128& o) const { return !(*this == o); }
  bool operator<(const Hash128& o) const { return hi != o.hi ? hi < o.hi : lo < o.lo; }
};

// Incremental hasher over 64-bit words and byte ranges.
class Hasher {
 public:
  void word(uint64_t w);
  void bytes(const void* p, size_t n);
  Hash128 done() const;

 private:
  uint64_t a_ = 0x243f6a8885a308d3ull, b_ = 0x13198a2e03707344ull, n_ = 0;
};

// Hash of a constant payload, memoised per live payload buffer (graphs share payloads
// immutably, so a buffer's bytes never change while it is alive).
Hash128 payload_hash(const std::shared_ptr<const std::vector<uint8_t>>& data);

// Fingerprint of the subgraph reachable from `roots` (roots included, in order).
Hash128 graph_fingerprint(const Graph& g, const std::vector<NodeId>& roots);

}  // namespace ku::hipbk
