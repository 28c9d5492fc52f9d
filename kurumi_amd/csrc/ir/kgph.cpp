// KGPH v2 encoder and decoder. The format is kurumi's, so the tags, the field order and the
// error cases follow the reference (kurumi_core/src/graph/serialize/**); the reader, the
// replay through checked builders and the overflow guards are this file's own.
#include "kgph.h"

#include <cstring>
#include <unordered_map>

namespace ku::kgph {
namespace {

constexpr uint8_t kMagic[4] = {'K', 'G', 'P', 'H'};  // serialize.rs:18
constexpr uint8_t kVersion = 2;                      // serialize.rs:19

// Op tags (encode/op.rs, decode/op.rs:10-87). Tags 0..40 are this IR's OpKind values in
// declaration order; 41..54 are reference ops outside this IR.
static_assert(static_cast<uint32_t>(OpKind::Const) == 0 && static_cast<uint32_t>(OpKind::Add) == 7 &&
                  static_cast<uint32_t>(OpKind::Sum) == 26 && static_cast<uint32_t>(OpKind::Sdpa) == 32 &&
                  static_cast<uint32_t>(OpKind::DotGeneral) == 39 &&
                  static_cast<uint32_t>(OpKind::QuantMatmul) == 40 && static_cast<uint32_t>(OpKind::NumKinds) == 41,
              "OpKind order must match the KGPH v2 op tags");
const char* const kForeignOps[] = {"Solve", "Det", "Cholesky", "Eigh", "Qr", "Eigvals", "Complex",
                                   "Real", "Imag", "Gather", "Scatter", "GatherAlong", "ScatterAlong", "Argsort"};
constexpr uint8_t kFirstForeign = 41, kLastTag = 54;

Error fail(const std::string& m) { return Error("deserialize_graph: " + m); }

// ---------------- writer (encode.rs:113-140) ----------------

struct Writer {
  std::vector<uint8_t> o;
  void u8(uint8_t v) { o.push_back(v); }
  void u32(uint32_t v) { for (int i = 0; i < 4; ++i) o.push_back(static_cast<uint8_t>(v >> (8 * i))); }
  void u64(uint64_t v) { for (int i = 0; i < 8; ++i) o.push_back(static_cast<uint8_t>(v >> (8 * i))); }
  void usize(size_t v) { u64(static_cast<uint64_t>(v)); }
  void f32(float v) { uint32_t b; std::memcpy(&b, &v, 4); u32(b); }
  void boolean(bool v) { u8(v ? 1 : 0); }
  void vec(const std::vector<size_t>& v) {
    u32(static_cast<uint32_t>(v.size()));
    for (size_t x : v) usize(x);
  }
  void str(const std::string& s) {
    u32(static_cast<uint32_t>(s.size()));
    o.insert(o.end(), s.begin(), s.end());
  }
  void dtype(DType d) { u8(static_cast<uint8_t>(d)); }
};

void write_op(Writer& w, const Op& op) {
  w.u8(static_cast<uint8_t>(op.kind));
  switch (op.kind) {
    case OpKind::Const: {
      // storage = dtype tag, u64 byte count, little-endian payload; then the shape
      const std::vector<uint8_t>& d = *op.data;
      w.dtype(op.data_dtype);
      w.u64(d.size());
      w.o.insert(w.o.end(), d.begin(), d.end());
      w.vec(op.shape);
      break;
    }
    case OpKind::Input: w.vec(op.shape); w.dtype(op.to); break;
    case OpKind::Iota: w.vec(op.shape); w.usize(op.axis); w.dtype(op.to); break;
    case OpKind::RandUniform: w.vec(op.shape); break;
    case OpKind::Cast: case OpKind::Bitcast: w.dtype(op.to); break;
    case OpKind::Sum: case OpKind::Prod: case OpKind::ReduceMax: case OpKind::Softmax: w.usize(op.axis); break;
    case OpKind::ArgReduce: w.usize(op.axis); w.u8(op.arg == ArgKind::Max ? 0 : 1); break;
    case OpKind::RmsNorm: w.usize(op.axis); w.f32(op.eps); break;
    case OpKind::Sdpa: w.boolean(op.causal); break;
    case OpKind::Reshape: case OpKind::Expand: w.vec(op.shape); break;
    case OpKind::Permute: w.vec(op.perm); break;
    case OpKind::Slice:
      w.u32(static_cast<uint32_t>(op.ranges.size()));
      for (const SliceRange& r : op.ranges) { w.usize(r.start); w.usize(r.end); w.usize(r.step); }
      break;
    case OpKind::Flip: w.vec(op.axes); break;
    case OpKind::Pad:
      w.u32(static_cast<uint32_t>(op.pads.size()));
      for (const PadRange& p : op.pads) { w.usize(p.lo); w.usize(p.hi); }
      break;
    case OpKind::DotGeneral: w.vec(op.lc); w.vec(op.rc); w.vec(op.lb); w.vec(op.rb); break;
    case OpKind::QuantMatmul: w.u8((uint8_t)op.qbits); w.usize(op.qgroup); w.boolean(op.qsym); break;
    default: break;  // no attributes
  }
}

// encode.rs:79-111: magic, version, nodes (op, src ids), then the entry table.
std::vector<uint8_t> write_blob(const Graph& g, const std::vector<NodeId>& order,
                                const std::unordered_map<NodeId, uint32_t>* remap, const std::vector<Entry>& entries) {
  auto id = [&](NodeId n) { return remap ? remap->at(n) : n; };
  Writer w;
  w.o.insert(w.o.end(), kMagic, kMagic + 4);
  w.u8(kVersion);
  w.u32(static_cast<uint32_t>(order.size()));
  for (NodeId n : order) {
    const Node& nd = g.node(n);
    write_op(w, nd.op);
    w.u32(static_cast<uint32_t>(nd.src.size()));
    for (NodeId s : nd.src) w.u32(id(s));
  }
  w.u32(static_cast<uint32_t>(entries.size()));
  for (const Entry& e : entries) {
    w.str(e.name);
    w.u32(static_cast<uint32_t>(e.outputs.size()));
    for (NodeId o : e.outputs) w.u32(o);
    w.u32(static_cast<uint32_t>(e.inputs.size()));
    for (const Binding& b : e.inputs) {
      w.u32(b.node);
      w.u8(static_cast<uint8_t>(b.role));
      w.str(b.name);
    }
  }
  return std::move(w.o);
}

// ---------------- reader (decode.rs:88-208) ----------------

struct Reader {
  const uint8_t* p;
  size_t n, pos = 0;
  const uint8_t* take(size_t k) {
    if (k > n - pos) throw fail("unexpected end of graph blob");
    const uint8_t* s = p + pos;
    pos += k;
    return s;
  }
  uint8_t u8() { return *take(1); }
  uint32_t u32() {
    const uint8_t* s = take(4);
    return uint32_t(s[0]) | uint32_t(s[1]) << 8 | uint32_t(s[2]) << 16 | uint32_t(s[3]) << 24;
  }
  uint64_t u64() {
    const uint8_t* s = take(8);
    uint64_t v = 0;
    for (int i = 7; i >= 0; --i) v = v << 8 | s[i];
    return v;
  }
  size_t usize() { return static_cast<size_t>(u64()); }
  float f32() { uint32_t b = u32(); float f; std::memcpy(&f, &b, 4); return f; }
  bool boolean() { return u8() != 0; }
  // The element count is attacker-controlled: grow by what the bytes actually hold.
  std::vector<size_t> vec() {
    uint32_t k = u32();
    std::vector<size_t> v;
    for (uint32_t i = 0; i < k; ++i) v.push_back(usize());
    return v;
  }
  DType dtype() {
    uint8_t t = u8();
    if (t >= kNumDTypes) throw fail("unknown dtype tag " + std::to_string(t));
    return static_cast<DType>(t);
  }
  ArgKind argkind() {
    uint8_t t = u8();
    if (t > 1) throw fail("unknown argkind " + std::to_string(t));
    return t == 0 ? ArgKind::Max : ArgKind::Min;
  }
  std::string str();
};

// Length of the UTF-8 sequence at s[0..n) if it is well formed (Unicode Table 3-7: no
// overlongs, no surrogates, <= U+10FFFF); otherwise 0 and *bad = the length of its maximal
// invalid prefix (at least 1).
size_t utf8_seq(const uint8_t* s, size_t n, size_t* bad) {
  uint8_t c = s[0];
  if (c < 0x80) return 1;
  size_t len;
  uint8_t lo = 0x80, hi = 0xBF;  // allowed range of the second byte
  if (c >= 0xC2 && c <= 0xDF) len = 2;
  else if (c >= 0xE0 && c <= 0xEF) { len = 3; if (c == 0xE0) lo = 0xA0; if (c == 0xED) hi = 0x9F; }
  else if (c >= 0xF0 && c <= 0xF4) { len = 4; if (c == 0xF0) lo = 0x90; if (c == 0xF4) hi = 0x8F; }
  else { *bad = 1; return 0; }
  size_t k = 1;
  for (; k < len && k < n; ++k) {
    uint8_t b = s[k];
    bool ok = k == 1 ? (b >= lo && b <= hi) : (b >= 0x80 && b <= 0xBF);
    if (!ok) break;
  }
  if (k == len) return len;
  *bad = k;
  return 0;
}

// What Rust's String::from_utf8 accepts.
bool valid_utf8(const uint8_t* s, size_t n) {
  size_t i = 0, bad;
  while (i < n) {
    size_t k = utf8_seq(s + i, n - i, &bad);
    if (!k) return false;
    i += k;
  }
  return true;
}

std::string Reader::str() {
  uint32_t k = u32();
  const uint8_t* s = take(k);
  if (!valid_utf8(s, k)) throw fail("invalid utf8 in name");
  return std::string(reinterpret_cast<const char*>(s), k);
}

// Element count of a decoded shape, rejecting products that do not fit in 63 bits (a blob can
// declare any dims; the builders' own numel would wrap).
size_t checked_numel(const Shape& s, size_t node) {
  uint64_t n = 1;
  for (size_t d : s)
    if (__builtin_mul_overflow(n, static_cast<uint64_t>(d), &n) || n > (uint64_t(1) << 62))
      throw fail("node " + std::to_string(node) + ": shape " + shape_str(s) + " overflows");
  return static_cast<size_t>(n);
}

// decode/op.rs:10-87: the op tag and its attributes.
Op read_op(Reader& r, size_t node) {
  uint8_t tag = r.u8();
  if (tag >= kFirstForeign && tag <= kLastTag)
    throw fail("node " + std::to_string(node) + ": op " + kForeignOps[tag - kFirstForeign] + " (tag " +
               std::to_string(tag) + ") is outside the kurumi_hip IR");
  if (tag > kLastTag) throw fail("unknown op tag " + std::to_string(tag));
  Op op;
  op.kind = static_cast<OpKind>(tag);
  switch (op.kind) {
    case OpKind::Const: {
      // decode/op.rs:13-23: the payload's whole-element count must equal the shape's; a
      // trailing partial element is dropped, as the reference's from_bytes does.
      DType dt = r.dtype();
      uint64_t nb = r.u64();
      const uint8_t* b = r.take(static_cast<size_t>(nb));
      op.shape = r.vec();
      size_t want = checked_numel(op.shape, node), w = dt_width(dt), have = static_cast<size_t>(nb) / w;
      if (have != want)
        throw fail("Const payload has " + std::to_string(have) + " elements, shape " + shape_str(op.shape) +
                   " needs " + std::to_string(want));
      std::vector<uint8_t> bytes(b, b + want * w);
      if (dt == DType::BOOL)  // convert.rs:110: any nonzero byte is true
        for (uint8_t& x : bytes) x = x != 0;
      op.data_dtype = dt;
      op.data = std::make_shared<const std::vector<uint8_t>>(std::move(bytes));
      break;
    }
    case OpKind::Input: op.shape = r.vec(); op.to = r.dtype(); checked_numel(op.shape, node); break;
    case OpKind::Iota: op.shape = r.vec(); op.axis = r.usize(); op.to = r.dtype(); checked_numel(op.shape, node); break;
    case OpKind::RandUniform: op.shape = r.vec(); checked_numel(op.shape, node); break;
    case OpKind::Cast: case OpKind::Bitcast: op.to = r.dtype(); break;
    case OpKind::Sum: case OpKind::Prod: case OpKind::ReduceMax: case OpKind::Softmax: op.axis = r.usize(); break;
    case OpKind::ArgReduce: op.axis = r.usize(); op.arg = r.argkind(); break;
    case OpKind::RmsNorm: op.axis = r.usize(); op.eps = r.f32(); break;
    case OpKind::Sdpa: op.causal = r.boolean(); break;
    case OpKind::Reshape: case OpKind::Expand: op.shape = r.vec(); checked_numel(op.shape, node); break;
    case OpKind::Permute: op.perm = r.vec(); break;
    case OpKind::Slice: {
      uint32_t k = r.u32();
      for (uint32_t i = 0; i < k; ++i) {
        SliceRange s;
        s.start = r.usize(); s.end = r.usize(); s.step = r.usize();
        op.ranges.push_back(s);
      }
      break;
    }
    case OpKind::Flip: op.axes = r.vec(); break;
    case OpKind::Pad: {
      uint32_t k = r.u32();
      for (uint32_t i = 0; i < k; ++i) {
        PadRange p;
        p.lo = r.usize(); p.hi = r.usize();
        op.pads.push_back(p);
      }
      break;
    }
    case OpKind::DotGeneral: op.lc = r.vec(); op.rc = r.vec(); op.lb = r.vec(); op.rb = r.vec(); break;
    case OpKind::QuantMatmul: op.qbits = r.u8(); op.qgroup = r.usize(); op.qsym = r.boolean(); break;
    default: break;
  }
  return op;
}

size_t arity(const Op& op) {
  const OpKind k = op.kind;
  switch (k) {
    case OpKind::QuantMatmul: return op.qsym ? 3 : 4;  // act, qweight, scales (+ mins)
    case OpKind::Const: case OpKind::Input: case OpKind::Iota: return 0;
    case OpKind::Add: case OpKind::Mul: case OpKind::Max: case OpKind::IDiv: case OpKind::And: case OpKind::Or:
    case OpKind::Xor: case OpKind::Shl: case OpKind::Shr: case OpKind::CmpLt: case OpKind::CmpEq:
    case OpKind::DotGeneral:
      return 2;
    case OpKind::Where: case OpKind::Sdpa: return 3;
    default: return 1;
  }
}

// Append node `i` through the builder that records exactly this op, so every record-time
// check of a live graph also guards a decoded one (decode.rs:61 pushes raw and relies on a
// panic guard instead).
void replay(Graph& g, size_t i, const Op& op, const std::vector<NodeId>& s) {
  if (s.size() != arity(op))
    throw fail("node " + std::to_string(i) + ": " + op_name(op.kind) + " takes " + std::to_string(arity(op)) +
               " sources, got " + std::to_string(s.size()));
  NodeId got;
  switch (op.kind) {
    case OpKind::Const: got = g.constant_bytes(op.data_dtype, op.data->data(), op.data->size(), op.shape); break;
    case OpKind::Input: got = g.input(op.shape, op.to); break;
    case OpKind::Iota: got = g.iota(op.shape, op.axis, op.to); break;
    case OpKind::RandUniform: got = g.rand_uniform_seeded(op.shape, s[0]); break;
    case OpKind::Cast: got = g.cast(s[0], op.to); break;
    case OpKind::Bitcast: got = g.bitcast(s[0], op.to); break;
    case OpKind::Detach: got = g.detach(s[0]); break;
    case OpKind::Add: got = g.add(s[0], s[1]); break;
    case OpKind::Mul: got = g.mul(s[0], s[1]); break;
    case OpKind::Max: got = g.max(s[0], s[1]); break;
    case OpKind::Neg: got = g.neg(s[0]); break;
    case OpKind::IDiv: got = g.idiv(s[0], s[1]); break;
    case OpKind::And: got = g.bit_and(s[0], s[1]); break;
    case OpKind::Or: got = g.bit_or(s[0], s[1]); break;
    case OpKind::Xor: got = g.bit_xor(s[0], s[1]); break;
    case OpKind::Shl: got = g.shl(s[0], s[1]); break;
    case OpKind::Shr: got = g.shr(s[0], s[1]); break;
    case OpKind::CmpLt: got = g.cmp_lt(s[0], s[1]); break;
    case OpKind::CmpEq: got = g.cmp_eq(s[0], s[1]); break;
    case OpKind::Where: got = g.where(s[0], s[1], s[2]); break;
    case OpKind::Recip: got = g.recip(s[0]); break;
    case OpKind::Sqrt: got = g.sqrt(s[0]); break;
    case OpKind::Exp2: got = g.exp2(s[0]); break;
    case OpKind::Log2: got = g.log2(s[0]); break;
    case OpKind::Sin: got = g.sin(s[0]); break;
    case OpKind::Floor: got = g.floor(s[0]); break;
    case OpKind::Sum: got = g.sum(s[0], op.axis); break;
    case OpKind::Prod: got = g.prod(s[0], op.axis); break;
    case OpKind::ReduceMax: got = g.reduce_max(s[0], op.axis); break;
    case OpKind::ArgReduce: got = g.argreduce(s[0], op.axis, op.arg); break;
    case OpKind::Softmax: got = g.softmax(s[0], op.axis); break;
    case OpKind::RmsNorm: got = g.rmsnorm(s[0], op.axis, op.eps); break;
    case OpKind::Sdpa: got = g.sdpa_fused(s[0], s[1], s[2], op.causal); break;
    case OpKind::Reshape: got = g.reshape(s[0], op.shape); break;
    case OpKind::Permute: got = g.permute(s[0], op.perm); break;
    case OpKind::Expand: got = g.expand(s[0], op.shape); break;
    case OpKind::Slice: got = g.slice(s[0], op.ranges); break;
    case OpKind::Flip: got = g.flip(s[0], op.axes); break;
    case OpKind::Pad: {
      const Shape& xs = g.shape(s[0]);
      for (size_t a = 0; a < op.pads.size() && a < xs.size(); ++a) {
        uint64_t d;
        if (__builtin_add_overflow(static_cast<uint64_t>(op.pads[a].lo), static_cast<uint64_t>(xs[a]), &d) ||
            __builtin_add_overflow(d, static_cast<uint64_t>(op.pads[a].hi), &d) || d > (uint64_t(1) << 62))
          throw fail("node " + std::to_string(i) + ": pad overflows");
      }
      got = g.pad(s[0], op.pads);
      break;
    }
    case OpKind::DotGeneral: got = g.dot_general(s[0], s[1], op.lc, op.rc, op.lb, op.rb); break;
    case OpKind::QuantMatmul:
      got = g.quant_matmul(s[0], s[1], s[2], op.qsym ? Graph::kNoNode : s[3], op.qbits, op.qgroup);
      break;
    default: throw fail("unknown op tag " + std::to_string(static_cast<uint32_t>(op.kind)));
  }
  if (got != i) throw fail("node " + std::to_string(i) + ": replay recorded extra nodes");
  checked_numel(g.shape(got), i);  // e.g. an outer product of two huge operands
}

}  // namespace

std::string utf8_lossy(const char* cs) {
  if (!cs) return {};
  const uint8_t* s = reinterpret_cast<const uint8_t*>(cs);
  size_t n = std::strlen(cs), i = 0, bad;
  std::string out;
  while (i < n) {
    size_t k = utf8_seq(s + i, n - i, &bad);
    if (k) {
      out.append(cs + i, k);
      i += k;
    } else {
      out += "\xEF\xBF\xBD";
      i += bad;
    }
  }
  return out;
}

std::vector<uint8_t> encode_arena(const Graph& g, const Entry& entry) {
  std::vector<NodeId> order(g.size());
  for (size_t i = 0; i < order.size(); ++i) order[i] = static_cast<NodeId>(i);
  return write_blob(g, order, nullptr, {entry});
}

std::vector<uint8_t> encode_reachable(const Graph& g, const std::vector<Entry>& entries) {
  std::vector<NodeId> roots;
  for (const Entry& e : entries) roots.insert(roots.end(), e.outputs.begin(), e.outputs.end());
  for (NodeId r : roots) g.node(r);  // an unknown output id is an error, not a silent drop
  std::vector<NodeId> order = reachable_multi(g, roots);
  std::unordered_map<NodeId, uint32_t> remap;
  for (size_t i = 0; i < order.size(); ++i) remap.emplace(order[i], static_cast<uint32_t>(i));
  std::vector<Entry> dense;
  for (const Entry& e : entries) {
    Entry d;
    d.name = e.name;
    for (NodeId o : e.outputs) d.outputs.push_back(remap.at(o));
    for (const Binding& b : e.inputs) {
      auto it = remap.find(b.node);
      if (it != remap.end()) d.inputs.push_back({it->second, b.role, b.name});
    }
    dense.push_back(std::move(d));
  }
  return write_blob(g, order, &remap, dense);
}

Program decode(const uint8_t* bytes, size_t len) {
  if (!bytes && len) throw fail("null blob");
  Reader r{bytes, len};
  if (len < 4 || std::memcmp(r.take(4), kMagic, 4) != 0) throw fail("bad magic (not a KGPH graph blob)");
  uint8_t ver = r.u8();
  if (ver != kVersion) throw fail("unsupported graph blob version " + std::to_string(ver));
  Program p;
  uint32_t n = r.u32();
  for (uint32_t i = 0; i < n; ++i) {
    Op op = read_op(r, i);
    uint32_t sl = r.u32();
    std::vector<NodeId> src;
    for (uint32_t k = 0; k < sl; ++k) {
      uint32_t s = r.u32();
      if (s >= i)  // decode.rs:52-58: replay is in id order, sources must already exist
        throw fail("node " + std::to_string(i) + " references source " + std::to_string(s) + " (not yet built)");
      src.push_back(s);
    }
    replay(p.graph, i, op, src);
  }
  uint32_t ne = r.u32();
  for (uint32_t e = 0; e < ne; ++e) {
    Entry en;
    en.name = r.str();
    uint32_t no = r.u32();
    for (uint32_t k = 0; k < no; ++k) en.outputs.push_back(r.u32());
    uint32_t ni = r.u32();
    for (uint32_t k = 0; k < ni; ++k) {
      Binding b;
      b.node = r.u32();
      uint8_t role = r.u8();
      if (role > 1) throw fail("bad input role " + std::to_string(role));
      b.role = static_cast<Role>(role);
      b.name = r.str();
      en.inputs.push_back(std::move(b));
    }
    p.entries.push_back(std::move(en));
  }
  return p;
}

}  // namespace ku::kgph
