// KGPH v2, kurumi's graph wire format: a self-contained little-endian blob holding a node
// arena (each node its op tag, attributes and source ids) and a table of named entry points
// (output ids plus input bindings). Restated from kurumi_core/src/graph/serialize.rs:1-67
// (framing, MAGIC "KGPH", VERSION 2), serialize/encode.rs:20-140 (blob writer, reachable
// prune + dense remap), serialize/encode/op.rs (per-op tags and attributes) and
// serialize/decode.rs:35-212 + decode/op.rs:10-87 (replay reader).
//
// Decoding is a trust boundary: every length is checked against the bytes that remain, a
// source must name an already-built node, and each node is replayed through the checked graph
// builders, so a malformed blob ends in `ku::Error`, never in an out-of-bounds access.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

#include "graph.h"

namespace ku::kgph {

// serialize.rs:28-41: a weight is bound by name from a weight table, a runtime input is fed.
enum class Role : uint8_t { Weight = 0, Runtime = 1 };

struct Binding {
  NodeId node;
  Role role;
  std::string name;
};

struct Entry {
  std::string name;
  std::vector<NodeId> outputs;
  std::vector<Binding> inputs;
};

// A decoded blob: the rebuilt arena (ids preserved) and its entries.
struct Program {
  Graph graph;
  std::vector<Entry> entries;
};

// serialize_graph (encode.rs:26-34): the whole arena in id order, one entry named "".
std::vector<uint8_t> encode_arena(const Graph& g, const Entry& entry);

// serialize_reachable / serialize_multi (encode.rs:42-76): only the union of the entries'
// output cones, remapped to a dense id range in post order; a binding whose node is outside
// the cone is dropped.
std::vector<uint8_t> encode_reachable(const Graph& g, const std::vector<Entry>& entries);

// A NUL-terminated C string as UTF-8, each maximal invalid subsequence replaced by U+FFFD
// (what the reference's CStr::to_string_lossy does to binding and entry names).
std::string utf8_lossy(const char* s);

// deserialize_multi (decode.rs:28-82). Throws ku::Error on any malformed blob.
Program decode(const uint8_t* bytes, size_t len);

}  // namespace ku::kgph
