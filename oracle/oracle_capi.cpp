// TEST INFRASTRUCTURE. C entry points of liboracle_kurumi.so for tests/ and bench.py's
// cpu_baseline (ctypes). Handles are the product's KuGraph / KuFeeds / KuTensor.
#include <cstring>
#include <stdexcept>
#include <string>

#include "oracle.h"

namespace {
thread_local std::string g_err;
}

extern "C" {

const char* kuo_last_error(void) { return g_err.c_str(); }

// Interpret `roots` (interp.rs:25-40 / interpret_many); writes one new KuTensor per root.
int32_t kuo_interpret(const KuGraph* g, const uint32_t* roots, size_t n, const KuFeeds* feeds, KuTensor** out) {
  try {
    ku::Feeds empty;
    std::vector<ku::NodeId> r(roots, roots + n);
    auto res = kuo::interpret(g->g, r, feeds ? feeds->f : empty);
    for (size_t i = 0; i < n; ++i) out[i] = new_ku_tensor(std::move(res[i]));
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

// View-fused evaluator (realize::force); returns 1 when the graph took the fused path,
// 0 when it fell back to the interpreter, -1 on error. `passes` = compute passes taken.
int32_t kuo_realize(const KuGraph* g, uint32_t root, const KuFeeds* feeds, KuTensor** out, int32_t* passes) {
  try {
    ku::Feeds empty;
    ku::Tensor t;
    int p = 0;
    if (kuo::realize(g->g, root, feeds ? feeds->f : empty, &t, &p)) {
      *out = new_ku_tensor(std::move(t));
      if (passes) *passes = p;
      return 1;
    }
    auto res = kuo::interpret(g->g, {root}, feeds ? feeds->f : empty);
    *out = new_ku_tensor(std::move(res[0]));
    if (passes) *passes = -1;
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

uint64_t kuo_threefry2x32(uint64_t key, uint64_t ctr) { return kuo::threefry2x32(key, ctr); }

void kuo_rand_uniform(uint64_t seed, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) out[i] = kuo::uniform_f32(kuo::threefry2x32(seed, i));
}

// Element casts with the reference semantics (for conversion pinning tests).
int32_t kuo_cast(uint32_t from, uint32_t to, const uint8_t* src, size_t n, uint8_t* dst) {
  try {
    ku::Tensor t;
    t.dtype = static_cast<ku::DType>(from);
    t.shape = {n};
    t.bytes.assign(src, src + n * ku::dt_width(t.dtype));
    ku::Tensor r = kuo::cast(t, static_cast<ku::DType>(to));
    std::memcpy(dst, r.bytes.data(), r.bytes.size());
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

}  // extern "C"
