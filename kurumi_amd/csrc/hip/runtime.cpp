#include "runtime.h"

#include "../ir/hostcopy.h"

#include <hip/hiprtc.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <thread>

namespace ku::hipbk {

void hip_check(hipError_t e, const char* what, const char* file, int line) {
  if (e == hipSuccess) return;
  std::ostringstream o;
  o << "HIP error " << hipGetErrorName(e) << " (" << hipGetErrorString(e) << ") at " << file << ":" << line << ": "
    << what;
  throw Error(o.str());
}

// ---------------- pool ----------------

size_t Pool::bucket(size_t bytes) {
  if (bytes == 0) bytes = 1;
  if (bytes <= (1u << 20)) return (bytes + 255) & ~size_t(255);
  // 1/8-octave buckets above 1 MiB
  size_t p = 1;
  while ((p << 1) <= bytes) p <<= 1;
  size_t step = p / 8;
  return (bytes + step - 1) / step * step;
}

DevBuf Pool::alloc(size_t bytes) {
  size_t b = bucket(bytes);
  auto it = free_.find(b);
  if (it != free_.end()) {
    DevBuf d{it->second, b};
    free_.erase(it);
    cached_ -= b;
    live_ += b;
    return d;
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, b);
  if (e != hipSuccess) {
    // return reclaimable buffers, release everything cached and retry once
    (void)hipGetLastError();
    for (auto& r : reclaimers_) r();
    trim();
    KU_HIP(hipMalloc(&p, b));
  }
  live_ += b;
  return DevBuf{p, b};
}

void Pool::release(DevBuf d) {
  if (!d.ptr) return;
  live_ -= d.bytes;
  cached_ += d.bytes;
  free_.emplace(d.bytes, d.ptr);
}

void Pool::trim() {
  for (auto& kv : free_) (void)hipFree(kv.second);
  free_.clear();
  cached_ = 0;
}

Pool::~Pool() { trim(); }

// ---------------- rtc ----------------

static uint64_t fnv1a(const std::string& s, uint64_t h = 1469598103934665603ull) {
  for (unsigned char c : s) {
    h ^= c;
    h *= 1099511628211ull;
  }
  return h;
}

static const char* kRtcOpts[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
                                 "-Xclang", "-packed-fp32-ops", "-fno-fast-math"};
static constexpr int kNumRtcOpts = sizeof(kRtcOpts) / sizeof(kRtcOpts[0]);

std::string rtc_cache_dir() {
  if (const char* d = std::getenv("KURUMI_HIP_CACHE")) return d;
  if (const char* h = std::getenv("HOME")) return std::string(h) + "/.cache/kurumi_hip";
  return "/tmp/kurumi_hip_cache";
}

static void mkdirs(const std::string& path) {
  std::string cur;
  for (size_t i = 0; i < path.size(); ++i) {
    cur.push_back(path[i]);
    if (path[i] == '/' || i + 1 == path.size()) ::mkdir(cur.c_str(), 0755);
  }
}

std::vector<char> rtc_compile(const std::string& src, const std::string& name_hint, bool fresh) {
  std::string key;
  for (int i = 0; i < kNumRtcOpts; ++i) key += kRtcOpts[i], key += ' ';
  int ver_major = 0, ver_minor = 0;
  hiprtcVersion(&ver_major, &ver_minor);
  key += std::to_string(ver_major) + "." + std::to_string(ver_minor);
  char hex[32];
  std::snprintf(hex, sizeof hex, "%016llx", (unsigned long long)fnv1a(src, fnv1a(key)));
  bool use_disk = !std::getenv("KURUMI_HIP_NO_DISK_CACHE");
  std::string dir = rtc_cache_dir();
  std::string path = dir + "/" + hex + ".co";
  if (use_disk && !fresh) {
    std::ifstream f(path, std::ios::binary);
    if (f) {
      std::vector<char> co((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
      if (!co.empty()) return co;
    }
  }
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), (name_hint + ".hip").c_str(), 0, nullptr, nullptr) != HIPRTC_SUCCESS)
    throw Error("hiprtcCreateProgram failed for " + name_hint);
  hiprtcResult r = hiprtcCompileProgram(prog, kNumRtcOpts, kRtcOpts);
  if (r != HIPRTC_SUCCESS) {
    size_t ls = 0;
    hiprtcGetProgramLogSize(prog, &ls);
    std::string log(ls, '\0');
    if (ls) hiprtcGetProgramLog(prog, log.data());
    hiprtcDestroyProgram(&prog);
    throw Error("hipRTC compile of " + name_hint + " failed: " + log + "\n--- source ---\n" + src);
  }
  size_t cs = 0;
  hiprtcGetCodeSize(prog, &cs);
  std::vector<char> co(cs);
  hiprtcGetCode(prog, co.data());
  hiprtcDestroyProgram(&prog);
  if (use_disk) {
    // Each writer its own temporary (backends in several threads, or processes, may compile the
    // same source at once) and an atomic rename, so a reader sees a whole file or none; a failed
    // or short write is never renamed into place.
    static std::atomic<uint64_t> seq{0};
    mkdirs(dir);
    const std::string tmp = path + ".tmp" + std::to_string(::getpid()) + "." +
                            std::to_string(std::hash<std::thread::id>{}(std::this_thread::get_id())) + "." +
                            std::to_string(seq.fetch_add(1));
    bool ok;
    {
      std::ofstream f(tmp, std::ios::binary);
      f.write(co.data(), static_cast<std::streamsize>(co.size()));
      f.close();
      ok = !f.fail();
    }
    if (!ok || std::rename(tmp.c_str(), path.c_str()) != 0) std::remove(tmp.c_str());
  }
  return co;
}

KernelFn ModuleCache::get(const std::string& src, const std::string& entry) {
  auto it = map_.find(src);
  if (it != map_.end()) {
    ++hits_;
    return it->second;
  }
  std::vector<char> co = rtc_compile(src, entry);
  KernelFn k;
  if (hipModuleLoadData(&k.mod, co.data()) != hipSuccess) {
    // a code object from the disk cache that does not load (damaged on disk): compile afresh,
    // which also replaces the cached file
    (void)hipGetLastError();
    co = rtc_compile(src, entry, /*fresh=*/true);
    KU_HIP(hipModuleLoadData(&k.mod, co.data()));
  }
  KU_HIP(hipModuleGetFunction(&k.fn, k.mod, entry.c_str()));
  ++compiled_;
  map_.emplace(src, k);
  return k;
}

ModuleCache::~ModuleCache() {
  for (auto& kv : map_) (void)hipModuleUnload(kv.second.mod);
}

const char* kind_name(Kind k) {
  static const char* n[] = {"fused", "gemm", "attention", "upload", "download"};
  int i = static_cast<int>(k);
  return (i >= 0 && i < static_cast<int>(Kind::NumKinds)) ? n[i] : "?";
}

// ---------------- context ----------------

Context::Context(int device) : device_(device) {
  if (const char* f = std::getenv("KURUMI_HIP_FORCE_NO_DEVICE"); f && *f && *f != '0')
    throw Error("no HIP device (KURUMI_HIP_FORCE_NO_DEVICE is set)");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) {
    (void)hipGetLastError();
    throw Error("no HIP device available");
  }
  if (device < 0 || device >= n) throw Error("HIP device index out of range");
  KU_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  KU_HIP(hipGetDeviceProperties(&prop, device));
  arch_ = prop.gcnArchName;
  num_cus_ = prop.multiProcessorCount;
  if (arch_.rfind("gfx950", 0) != 0) throw Error("kurumi_hip targets gfx950 (MI355X); found " + arch_);
  KU_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  if (const char* t = std::getenv("KURUMI_GPUTIME"); t && *t && *t != '0') timing_ = true;
}

Context::~Context() {
  if (stream_) {
    (void)hipSetDevice(device_);
    (void)hipStreamSynchronize(stream_);
    for (int i = 0; i < 2; ++i) {
      if (stage_ev_[i]) (void)hipEventDestroy(stage_ev_[i]);
      if (stage_[i]) (void)hipHostFree(stage_[i]);
    }
    (void)hipStreamDestroy(stream_);
  }
}

namespace {
constexpr size_t kStageChunk = size_t(32) << 20;
// Below this a pageable copy's fixed cost is lower than the staging loop's.
constexpr size_t kStageMin = size_t(4) << 20;
}  // namespace

bool Context::ensure_stage() {
  if (stage_[1]) return true;
  if (stage_failed_) return false;
  for (int i = 0; i < 2; ++i) {
    if (hipHostMalloc(&stage_[i], kStageChunk, hipHostMallocDefault) != hipSuccess) {
      (void)hipGetLastError();
      for (int j = 0; j <= i; ++j) {
        if (stage_[j]) (void)hipHostFree(stage_[j]);
        stage_[j] = nullptr;
      }
      stage_failed_ = true;  // pinned memory unavailable: stay on pageable copies
      return false;
    }
    KU_HIP(hipEventCreateWithFlags(&stage_ev_[i], hipEventDisableTiming));
  }
  return true;
}

void Context::upload(void* dev, const void* host, size_t n) {
  if (!n) return;
  if (n < kStageMin || !ensure_stage()) {
    KU_HIP(hipMemcpyAsync(dev, host, n, hipMemcpyHostToDevice, stream_));
    return;
  }
  for (size_t off = 0, c = 0; off < n; off += kStageChunk, ++c) {
    const int b = int(c & 1);
    const size_t len = std::min(kStageChunk, n - off);
    if (stage_recorded_[b]) KU_HIP(hipEventSynchronize(stage_ev_[b]));  // its last DMA has read it
    par_copy(stage_[b], static_cast<const uint8_t*>(host) + off, len);
    KU_HIP(hipMemcpyAsync(static_cast<uint8_t*>(dev) + off, stage_[b], len, hipMemcpyHostToDevice, stream_));
    KU_HIP(hipEventRecord(stage_ev_[b], stream_));
    stage_recorded_[b] = true;
  }
}

void Context::download(void* host, const void* dev, size_t n) {
  if (!n) return;
  if (n < kStageMin || !ensure_stage()) {
    KU_HIP(hipMemcpyAsync(host, dev, n, hipMemcpyDeviceToHost, stream_));
    sync();
    return;
  }
  const size_t nc = (n + kStageChunk - 1) / kStageChunk;
  auto issue = [&](size_t c) {
    const int b = int(c & 1);
    const size_t off = c * kStageChunk;
    KU_HIP(hipMemcpyAsync(stage_[b], static_cast<const uint8_t*>(dev) + off, std::min(kStageChunk, n - off),
                          hipMemcpyDeviceToHost, stream_));
    KU_HIP(hipEventRecord(stage_ev_[b], stream_));
    stage_recorded_[b] = true;
  };
  issue(0);
  if (nc > 1) issue(1);
  for (size_t c = 0; c < nc; ++c) {
    const int b = int(c & 1);
    const size_t off = c * kStageChunk;
    KU_HIP(hipEventSynchronize(stage_ev_[b]));
    par_copy(static_cast<uint8_t*>(host) + off, stage_[b], std::min(kStageChunk, n - off));
    if (c + 2 < nc) issue(c + 2);
  }
}

void Context::make_current() const { KU_HIP(hipSetDevice(device_)); }

void Context::sync() { KU_HIP(hipStreamSynchronize(stream_)); }

}  // namespace ku::hipbk
