#include "hostcopy.h"

#include <sys/mman.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

namespace ku {

namespace {
constexpr size_t kHuge = size_t(2) << 20;
// Below this a single memcpy is faster than starting threads.
constexpr size_t kSplitMin = size_t(16) << 20;
// Pieces handed to threads start on 4 KiB boundaries so that no page is faulted by two threads.
constexpr size_t kPage = 4096;
}  // namespace

void advise_huge(void* p, size_t n) {
  const uintptr_t b = reinterpret_cast<uintptr_t>(p);
  const uintptr_t lo = (b + kHuge - 1) & ~(uintptr_t)(kHuge - 1);
  const uintptr_t hi = (b + n) & ~(uintptr_t)(kHuge - 1);
  if (hi > lo) (void)madvise(reinterpret_cast<void*>(lo), hi - lo, MADV_HUGEPAGE);
}

int host_copy_threads() {
  static const int n = [] {
    if (const char* e = std::getenv("KURUMI_HOST_COPY_THREADS"); e && *e) {
      int v = std::atoi(e);
      return std::max(1, std::min(v, 64));
    }
    unsigned h = std::thread::hardware_concurrency();
    return (int)std::max(1u, std::min(h ? h : 1u, 8u));
  }();
  return n;
}

void par_copy(void* dst, const void* src, size_t n) {
  if (!n) return;
  const int t = host_copy_threads();
  if (n < kSplitMin || t <= 1) {
    std::memcpy(dst, src, n);
    return;
  }
  auto* d = static_cast<uint8_t*>(dst);
  const auto* s = static_cast<const uint8_t*>(src);
  // piece boundaries on destination page boundaries
  const uintptr_t db = reinterpret_cast<uintptr_t>(d);
  size_t piece = (n + t - 1) / t;
  std::vector<size_t> cut(t + 1, n);
  cut[0] = 0;
  for (int i = 1; i < t; ++i) {
    uintptr_t a = (db + i * piece + kPage - 1) & ~(uintptr_t)(kPage - 1);
    cut[i] = std::min(n, std::max(cut[i - 1], (size_t)(a - db)));
  }
  const size_t* c = cut.data();
  std::vector<std::thread> th;
  th.reserve(t - 1);
  int i = 1;
  for (; i < t; ++i) {
    if (c[i + 1] <= c[i]) continue;
    try {
      th.emplace_back([d, s, c, i] { std::memcpy(d + c[i], s + c[i], c[i + 1] - c[i]); });
    } catch (...) {
      break;  // no more threads: the pieces from i on are copied here
    }
  }
  for (int j = i; j < t; ++j)
    if (c[j + 1] > c[j]) std::memcpy(d + c[j], s + c[j], c[j + 1] - c[j]);
  std::memcpy(d, s, c[1]);
  for (auto& x : th) x.join();
}

}  // namespace ku
