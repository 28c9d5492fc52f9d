// Device layer of the HIP backend: one stream per context, a size-bucketed hipMalloc
// pool recycled per eval, a hipRTC module cache keyed by generated source, and
// per-kind dispatch counters with hipEvent GPU timing.
//
// MI355X analog of kurumi_metal/src/context.rs:23-57 (device + shared encoder),
// context/pool.rs:19-71 (byte-size buffer pool with `recycle`),
// context/pipeline.rs:12-29 (pipeline cache keyed by kernel source) and
// context/profile.rs:7-35 (dispatch-kind counters, GPU time).
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../ir/graph.h"

namespace ku::hipbk {

void hip_check(hipError_t e, const char* what, const char* file, int line);
#define KU_HIP(x) ::ku::hipbk::hip_check((x), #x, __FILE__, __LINE__)

struct DevBuf {
  void* ptr = nullptr;
  size_t bytes = 0;  // capacity
};

// Byte-size bucketed pool. Buffers are rounded up to 256 B (small) or to a 1/8-octave
// bucket (large) so that repeated evals of one graph reuse the same allocations.
class Pool {
 public:
  ~Pool();
  DevBuf alloc(size_t bytes);
  void release(DevBuf b);
  void trim();
  size_t bytes_live() const { return live_; }
  size_t bytes_cached() const { return cached_; }
  // Called when hipMalloc fails, before the retry: each returns buffers it held to the pool
  // (e.g. cached constants that no plan uses) so the trim can free them.
  void add_reclaimer(std::function<size_t()> f) { reclaimers_.push_back(std::move(f)); }
  void clear_reclaimers() { reclaimers_.clear(); }

 private:
  static size_t bucket(size_t bytes);
  std::vector<std::function<size_t()>> reclaimers_;
  std::multimap<size_t, void*> free_;
  size_t live_ = 0, cached_ = 0;
};

struct KernelFn {
  hipModule_t mod = nullptr;
  hipFunction_t fn = nullptr;
};

// Compile generated HIP source for gfx950 with hipRTC; cache code objects in memory
// (by source) and on disk (by a hash of source, options and hipRTC version) so a re-run skips
// the compile. fresh = true ignores the disk copy (and rewrites it).
std::vector<char> rtc_compile(const std::string& src, const std::string& name_hint, bool fresh = false);
std::string rtc_cache_dir();

class ModuleCache {
 public:
  ~ModuleCache();
  KernelFn get(const std::string& src, const std::string& entry);
  size_t compiled() const { return compiled_; }
  size_t hits() const { return hits_; }

 private:
  std::unordered_map<std::string, KernelFn> map_;
  size_t compiled_ = 0, hits_ = 0;
};

// dispatch kinds (the profile counters): fused region, gemm, attention, copy/upload/download
enum class Kind : int { Fused = 0, Gemm, Attention, Upload, Download, NumKinds };
const char* kind_name(Kind k);

struct Profile {
  uint64_t launches[static_cast<int>(Kind::NumKinds)] = {};
  double gpu_ms[static_cast<int>(Kind::NumKinds)] = {};
  uint64_t evals = 0;
};

class Context {
 public:
  // Throws ku::Error when no HIP device is usable (the C ABI maps that to NULL).
  explicit Context(int device);
  ~Context();
  int device() const { return device_; }
  hipStream_t stream() const { return stream_; }
  Pool& pool() { return pool_; }
  ModuleCache& modules() { return modules_; }
  Profile& profile() { return profile_; }
  const std::string& arch() const { return arch_; }
  int num_cus() const { return num_cus_; }
  void sync();
  void make_current() const;
  bool timing() const { return timing_; }
  void set_timing(bool on) { timing_ = on; }
  // Host <-> device copies of tensors crossing the C boundary. Large ones go in 32 MiB chunks
  // through two pinned staging buffers (allocated on first use): the DMA runs at pinned rate
  // and overlaps the multi-threaded host copy of the neighbouring chunk. upload() is ordered on
  // the context stream and may return before its last DMA ends (the host buffer is free on
  // return); download() returns with `host` filled.
  void upload(void* dev, const void* host, size_t n);
  void download(void* host, const void* dev, size_t n);

 private:
  bool ensure_stage();
  int device_;
  hipStream_t stream_ = nullptr;
  Pool pool_;
  ModuleCache modules_;
  Profile profile_;
  std::string arch_;
  int num_cus_ = 0;
  bool timing_ = false;
  void* stage_[2] = {nullptr, nullptr};
  hipEvent_t stage_ev_[2] = {nullptr, nullptr};
  bool stage_recorded_[2] = {false, false};
  bool stage_failed_ = false;
};

}  // namespace ku::hipbk
