// Kernel timing hook: per-launch HIP event pairs, summed per kernel kind.
#include <atomic>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "profile.hpp"

namespace msa {

namespace {

constexpr int kMaxPairs = 1 << 14;

struct Pair {
  hipEvent_t start = nullptr, stop = nullptr;
  int kind = 0;
};

std::atomic<bool> g_armed{false};
std::mutex g_mu;
std::vector<Pair> g_pool;  // events are created once and reused
int g_used = 0;

}  // namespace

bool prof_armed() { return g_armed.load(std::memory_order_relaxed); }

int prof_open(int kind, hipStream_t st) {
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_used >= kMaxPairs) return -1;
  if (g_used == static_cast<int>(g_pool.size())) {
    Pair p;
    if (hipEventCreate(&p.start) != hipSuccess) return -1;
    if (hipEventCreate(&p.stop) != hipSuccess) {
      (void)hipEventDestroy(p.start);
      return -1;
    }
    g_pool.push_back(p);
  }
  Pair& p = g_pool[g_used];
  p.kind = kind;
  if (hipEventRecord(p.start, st) != hipSuccess) return -1;
  return g_used++;
}

void prof_close(int pair, hipStream_t st) {
  std::lock_guard<std::mutex> lock(g_mu);
  (void)hipEventRecord(g_pool[pair].stop, st);
}

}  // namespace msa

using namespace msa;

extern "C" int msa_profile_begin(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  g_used = 0;
  g_armed.store(true, std::memory_order_relaxed);
  return kOk;
}

extern "C" int64_t msa_profile_end(double* ms, int64_t* launches, int64_t kinds) {
  std::lock_guard<std::mutex> lock(g_mu);
  g_armed.store(false, std::memory_order_relaxed);
  for (int64_t k = 0; k < kinds; ++k) {
    if (ms) ms[k] = 0.0;
    if (launches) launches[k] = 0;
  }
  for (int i = 0; i < g_used; ++i) {
    const Pair& p = g_pool[i];
    if (hipEventSynchronize(p.stop) != hipSuccess) return -1;
    float t = 0.f;
    if (hipEventElapsedTime(&t, p.start, p.stop) != hipSuccess) return -1;
    if (p.kind < kinds) {
      if (ms) ms[p.kind] += t;
      if (launches) launches[p.kind] += 1;
    }
  }
  g_used = 0;
  return kProfKinds;
}
