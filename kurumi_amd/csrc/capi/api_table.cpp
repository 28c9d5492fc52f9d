// ku_hip_api: the prefixed, collision-free way into this library (declared in
// include/kurumi_hip.h). The table's pointers are taken here, inside libkurumi_hip.so, which is
// linked with -Bsymbolic-functions, so they name this library's definitions even when another
// object loaded earlier (kurumi's own cdylib) exports the same ku_* names.
#include <string>

#include "../../../include/kurumi_hip.h"
#include "errors.h"

namespace {

KuHipApi make_table() {
  KuHipApi t{};
  t.version = KU_HIP_API_VERSION;
  t.size = sizeof(KuHipApi);
  t.last_error = &ku_last_error;
  t.backend_new = &ku_backend_new;
  t.backend_free = &ku_backend_free;
  t.graph_new = &ku_graph_new;
  t.graph_free = &ku_graph_free;
  t.graph_deserialize = &ku_graph_deserialize;
  t.runnable_take_graph = &ku_runnable_take_graph;
  t.runnable_output_count = &ku_runnable_output_count;
  t.runnable_output = &ku_runnable_output;
  t.runnable_input_count = &ku_runnable_input_count;
  t.runnable_input_node = &ku_runnable_input_node;
  t.runnable_input_name = &ku_runnable_input_name;
  t.runnable_free = &ku_runnable_free;
  t.eval = &ku_eval;
  t.eval_with = &ku_eval_with;
  t.eval_many = &ku_eval_many;
  t.plan_compile_on = &ku_hip_plan_compile_on;
  t.plan_run = &ku_plan_run;
  t.plan_free = &ku_plan_free;
  t.feeds_new = &ku_feeds_new;
  t.feeds_free = &ku_feeds_free;
  t.feeds_set = &ku_feeds_set;
  t.tensor_new = &ku_tensor_new;
  t.tensor_free = &ku_tensor_free;
  t.tensor_rank = &ku_tensor_rank;
  t.tensor_shape = &ku_tensor_shape;
  t.tensor_dtype = &ku_tensor_dtype;
  t.tensor_nbytes = &ku_tensor_nbytes;
  t.tensor_bytes = &ku_tensor_bytes;
  t.node_count = &ku_node_count;
  t.dump = &ku_dump;
  return t;
}

const KuHipApi g_table = make_table();

}  // namespace

extern "C" const KuHipApi* ku_hip_api(uint32_t version) {
  if (version != KU_HIP_API_VERSION) {
    ku::capi::set_err("ku_hip_api: version " + std::to_string(version) + " not provided (this library: " +
                      std::to_string(KU_HIP_API_VERSION) + ")");
    return nullptr;
  }
  return &g_table;
}
