#include "fingerprint.h"

#include <cstring>
#include <map>
#include <mutex>

namespace ku::hipbk {

namespace {
constexpr uint64_t kP1 = 0x9e3779b97f4a7c15ull, kP2 = 0xc2b2ae3d27d4eb4full, kP3 = 0x165667b19e3779f9ull;
inline uint64_t rotl(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
inline uint64_t fmix(uint64_t k) {
  k ^= k >> 33;
  k *= 0xff51afd7ed558ccdull;
  k ^= k >> 33;
  k *= 0xc4ceb9fe1a85ec53ull;
  k ^= k >> 33;
  return k;
}
}  // namespace

void Hasher::word(uint64_t w) {
  a_ = rotl(a_ ^ (w * kP1), 31) * kP2;
  b_ = rotl(b_ + (w ^ kP3), 27) * kP1 + a_;
  ++n_;
}

void Hasher::bytes(const void* p, size_t n) {
  const uint8_t* c = static_cast<const uint8_t*>(p);
  word(n);
  // four words per trip in two independent lanes, folded into the running state per block
  uint64_t x0 = a_, x1 = b_, x2 = a_ ^ kP3, x3 = b_ ^ kP2;
  size_t i = 0;
  for (; i + 32 <= n; i += 32) {
    uint64_t w[4];
    std::memcpy(w, c + i, 32);
    x0 = rotl(x0 ^ (w[0] * kP1), 31) * kP2;
    x1 = rotl(x1 ^ (w[1] * kP2), 29) * kP1;
    x2 = rotl(x2 ^ (w[2] * kP3), 33) * kP2;
    x3 = rotl(x3 ^ (w[3] * kP1), 27) * kP3;
  }
  word(fmix(x0) ^ rotl(fmix(x2), 17));
  word(fmix(x1) ^ rotl(fmix(x3), 41));
  uint64_t tail[4] = {0, 0, 0, 0};
  std::memcpy(tail, c + i, n - i);
  for (uint64_t t : tail) word(t);
}

Hash128 Hasher::done() const { return Hash128{fmix(a_ ^ n_), fmix(b_ + rotl(a_, 23))}; }

namespace {
struct Memo {
  std::weak_ptr<const std::vector<uint8_t>> alive;
  Hash128 h;
};
std::mutex g_memo_mu;
std::map<const void*, Memo> g_memo;
}  // namespace

Hash128 payload_hash(const std::shared_ptr<const std::vector<uint8_t>>& data) {
  if (!data) return Hash128{};
  const void* key = data.get();
  {
    std::lock_guard<std::mutex> lk(g_memo_mu);
    auto it = g_memo.find(key);
    if (it != g_memo.end()) {
      auto live = it->second.alive.lock();
      if (live && live.get() == key) return it->second.h;
      g_memo.erase(it);  // the buffer died and its address was reused
    }
  }
  Hasher h;
  h.bytes(data->data(), data->size());
  Hash128 r = h.done();
  std::lock_guard<std::mutex> lk(g_memo_mu);
  if (g_memo.size() > 4096) {  // drop records of dead payloads
    for (auto it = g_memo.begin(); it != g_memo.end();) it = it->second.alive.expired() ? g_memo.erase(it) : ++it;
  }
  g_memo[key] = Memo{data, r};
  return r;
}

Hash128 graph_fingerprint(const Graph& g, const std::vector<NodeId>& roots) {
  Hasher h;
  h.word(roots.size());
  for (NodeId r : roots) h.word(r);
  auto vec = [&](const std::vector<size_t>& v) {
    h.word(v.size());
    for (size_t x : v) h.word(x);
  };
  for (NodeId id : reachable_multi(g, roots)) {
    const Node& n = g.node(id);
    const Op& op = n.op;
    h.word(id);
    h.word((uint64_t)op.kind);
    h.word((uint64_t)n.dtype);
    vec(n.shape);
    h.word(n.src.size());
    for (NodeId s : n.src) h.word(s);
    h.word((uint64_t)op.to);
    vec(op.shape);
    vec(op.perm);
    vec(op.axes);
    h.word(op.axis);
    h.word((uint64_t)op.arg);
    h.word(op.causal);
    uint32_t eb;
    std::memcpy(&eb, &op.eps, 4);
    h.word(eb);
    h.word(op.ranges.size());
    for (const auto& r : op.ranges) {
      h.word(r.start);
      h.word(r.end);
      h.word(r.step);
    }
    h.word(op.pads.size());
    for (const auto& p : op.pads) {
      h.word(p.lo);
      h.word(p.hi);
    }
    vec(op.lc);
    vec(op.rc);
    vec(op.lb);
    vec(op.rb);
    h.word((uint64_t)(int64_t)op.qbits);
    h.word(op.qgroup);
    h.word(op.qsym);
    h.word((uint64_t)op.data_dtype);
    if (op.kind == OpKind::Const) {
      Hash128 ph = payload_hash(op.data);
      h.word(op.data ? op.data->size() : 0);
      h.word(ph.lo);
      h.word(ph.hi);
    }
  }
  return h.done();
}

}  // namespace ku::hipbk
