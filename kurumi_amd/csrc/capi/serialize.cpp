// C ABI of the KGPH v2 graph blob: ku_graph_serialize*, ku_graph_deserialize and the
// ku_runnable_* accessors (kurumi/src/capi/graph/serialize.rs:34-196 and
// serialize/runnable.rs). Same size-then-write convention and the same null / out-of-range
// answers as the reference: a null array reads as empty, an accessor past the end returns
// 0 or KU_ERR.
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../../include/kurumi_hip.h"
#include "../ir/kgph.h"
#include "errors.h"
#include "handles.h"

using ku::NodeId;
using ku::capi::guard;
using ku::capi::set_err;
namespace kg = ku::kgph;

struct KuRunnable {
  std::unique_ptr<KuGraph> graph;
  std::vector<kg::Entry> entries;
};

namespace {

template <class T>
const T* at(const T* p, size_t n, size_t i) {  // raw_slice(p, n).get(i)
  return (p && i < n) ? p + i : nullptr;
}

std::string cstr(const char* p) { return kg::utf8_lossy(p); }

size_t write_bytes(const std::string& s, uint8_t* out, size_t cap) {
  size_t n = s.size() < cap ? s.size() : cap;
  if (n && out) std::memcpy(out, s.data(), n);
  return s.size();
}
size_t write_bytes(const std::vector<uint8_t>& s, uint8_t* out, size_t cap) {
  size_t n = s.size() < cap ? s.size() : cap;
  if (n && out) std::memcpy(out, s.data(), n);
  return s.size();
}

// serialize.rs:34-65: bindings from the C arrays; role 0 is a weight, anything else runtime.
std::vector<kg::Binding> bindings(const KuNode* nodes, const uint8_t* roles, const char* const* names, size_t off,
                                  size_t n, size_t total) {
  std::vector<kg::Binding> v;
  for (size_t k = off; k < off + n; ++k) {
    const uint8_t* r = at(roles, total, k);
    const char* const* nm = at(names, total, k);
    const KuNode* nd = at(nodes, total, k);
    v.push_back({nd ? *nd : KU_ERR, (r && *r == 0) ? kg::Role::Weight : kg::Role::Runtime, nm ? cstr(*nm) : ""});
  }
  return v;
}

size_t serialize_one(bool reachable, const KuGraph* g, const KuNode* outputs, size_t n_out, const KuNode* in_nodes,
                     const uint8_t* in_roles, const char* const* in_names, size_t n_in, uint8_t* out, size_t cap) {
  if (!g) {
    set_err("ku_graph_serialize: null graph");
    return 0;
  }
  return guard<size_t>(0, [&] {
    kg::Entry e;
    if (outputs) e.outputs.assign(outputs, outputs + n_out);
    e.inputs = bindings(in_nodes, in_roles, in_names, 0, n_in, n_in);
    std::vector<uint8_t> blob = reachable ? kg::encode_reachable(g->g, {e}) : kg::encode_arena(g->g, e);
    return write_bytes(blob, out, cap);
  });
}

const kg::Entry* entry(const KuRunnable* h, size_t i) {
  return (h && i < h->entries.size()) ? &h->entries[i] : nullptr;
}
const kg::Binding* binding(const KuRunnable* h, size_t i, size_t j) {
  const kg::Entry* e = entry(h, i);
  return (e && j < e->inputs.size()) ? &e->inputs[j] : nullptr;
}

}  // namespace

extern "C" {

size_t ku_graph_serialize(const KuGraph* g, const KuNode* outputs, size_t n_out, const KuNode* in_nodes,
                          const uint8_t* in_roles, const char* const* in_names, size_t n_in, uint8_t* out,
                          size_t cap) {
  return serialize_one(false, g, outputs, n_out, in_nodes, in_roles, in_names, n_in, out, cap);
}

size_t ku_graph_serialize_reachable(const KuGraph* g, const KuNode* outputs, size_t n_out, const KuNode* in_nodes,
                                    const uint8_t* in_roles, const char* const* in_names, size_t n_in, uint8_t* out,
                                    size_t cap) {
  return serialize_one(true, g, outputs, n_out, in_nodes, in_roles, in_names, n_in, out, cap);
}

// serialize.rs:115-161
size_t ku_graph_serialize_multi(const KuGraph* g, size_t n_entries, const char* const* names,
                                const uint32_t* out_counts, const KuNode* outputs, const uint32_t* in_counts,
                                const KuNode* in_nodes, const uint8_t* in_roles, const char* const* in_names,
                                uint8_t* out, size_t cap) {
  if (!g) {
    set_err("ku_graph_serialize_multi: null graph");
    return 0;
  }
  return guard<size_t>(0, [&] {
    size_t total_out = 0, total_in = 0;
    for (size_t e = 0; e < n_entries; ++e) {
      const uint32_t* oc = at(out_counts, n_entries, e);
      const uint32_t* ic = at(in_counts, n_entries, e);
      total_out += oc ? *oc : 0;
      total_in += ic ? *ic : 0;
    }
    if (total_out && !outputs) throw ku::Error("ku_graph_serialize_multi: null outputs");
    std::vector<kg::Entry> entries;
    size_t o_off = 0, i_off = 0;
    for (size_t e = 0; e < n_entries; ++e) {
      kg::Entry en;
      const char* const* nm = at(names, n_entries, e);
      en.name = nm ? cstr(*nm) : "";
      const uint32_t* oc = at(out_counts, n_entries, e);
      const uint32_t* ic = at(in_counts, n_entries, e);
      size_t no = oc ? *oc : 0, ni = ic ? *ic : 0;
      en.outputs.assign(outputs + o_off, outputs + o_off + no);
      o_off += no;
      en.inputs = bindings(in_nodes, in_roles, in_names, i_off, ni, total_in);
      i_off += ni;
      entries.push_back(std::move(en));
    }
    return write_bytes(kg::encode_reachable(g->g, entries), out, cap);
  });
}

// serialize.rs:169-196: NULL (with the last error) on a malformed or entry-less blob.
KuRunnable* ku_graph_deserialize(const uint8_t* bytes, size_t len) {
  return guard<KuRunnable*>(nullptr, [&]() -> KuRunnable* {
    kg::Program p = kg::decode(bytes, len);
    if (p.entries.empty()) {
      set_err("ku_graph_deserialize: graph blob has no entries");
      return nullptr;
    }
    auto r = std::make_unique<KuRunnable>();
    r->graph = std::make_unique<KuGraph>();
    r->graph->g = std::move(p.graph);
    r->entries = std::move(p.entries);
    return r.release();
  });
}

// runnable.rs:11-20: moves the graph out and leaves an empty one behind.
KuGraph* ku_runnable_take_graph(KuRunnable* h) {
  if (!h) {
    set_err("ku_runnable_take_graph: null handle");
    return nullptr;
  }
  KuGraph* g = h->graph.release();
  h->graph = std::make_unique<KuGraph>();
  return g;
}

size_t ku_runnable_output_count(const KuRunnable* h) { return ku_runnable_entry_output_count(h, 0); }
KuNode ku_runnable_output(const KuRunnable* h, size_t i) { return ku_runnable_entry_output(h, 0, i); }
size_t ku_runnable_input_count(const KuRunnable* h) { return ku_runnable_entry_input_count(h, 0); }
KuNode ku_runnable_input_node(const KuRunnable* h, size_t i) { return ku_runnable_entry_input_node(h, 0, i); }
uint32_t ku_runnable_input_role(const KuRunnable* h, size_t i) { return ku_runnable_entry_input_role(h, 0, i); }
size_t ku_runnable_input_name(const KuRunnable* h, size_t i, uint8_t* out, size_t cap) {
  return ku_runnable_entry_input_name(h, 0, i, out, cap);
}

size_t ku_runnable_entry_count(const KuRunnable* h) { return h ? h->entries.size() : 0; }
size_t ku_runnable_entry_name(const KuRunnable* h, size_t i, uint8_t* out, size_t cap) {
  const kg::Entry* e = entry(h, i);
  return e ? write_bytes(e->name, out, cap) : 0;
}
size_t ku_runnable_entry_output_count(const KuRunnable* h, size_t i) {
  const kg::Entry* e = entry(h, i);
  return e ? e->outputs.size() : 0;
}
KuNode ku_runnable_entry_output(const KuRunnable* h, size_t i, size_t j) {
  const kg::Entry* e = entry(h, i);
  return (e && j < e->outputs.size()) ? e->outputs[j] : KU_ERR;
}
size_t ku_runnable_entry_input_count(const KuRunnable* h, size_t i) {
  const kg::Entry* e = entry(h, i);
  return e ? e->inputs.size() : 0;
}
KuNode ku_runnable_entry_input_node(const KuRunnable* h, size_t i, size_t j) {
  const kg::Binding* b = binding(h, i, j);
  return b ? b->node : KU_ERR;
}
uint32_t ku_runnable_entry_input_role(const KuRunnable* h, size_t i, size_t j) {
  const kg::Binding* b = binding(h, i, j);
  return b ? static_cast<uint32_t>(b->role) : KU_ERR;
}
size_t ku_runnable_entry_input_name(const KuRunnable* h, size_t i, size_t j, uint8_t* out, size_t cap) {
  const kg::Binding* b = binding(h, i, j);
  return b ? write_bytes(b->name, out, cap) : 0;
}

void ku_runnable_free(KuRunnable* h) { delete h; }

}  // extern "C"
