// Drives dip::HostPool (dynamic-input-pruning_amd/csrc/dip_host_pool.h) on the
// CPU for tests/test_host_pool.py: blocking jobs, start/finish jobs with the
// caller polling per-job flags (the miss stream's pattern), then main returns
// at once, so the exit handlers destroy the pool while its workers may still
// be spinning.  Built with ThreadSanitizer or AddressSanitizer by the test.
#include <atomic>
#include <cstdio>
#include <cstring>
#include <functional>
#include <thread>
#include <vector>

#include "dip_host_pool.h"

int main(int argc, char** argv) {
  const int rounds = argc > 1 ? std::atoi(argv[1]) : 20;
  const int nt = argc > 2 ? std::atoi(argv[2]) : 8;
  std::vector<int> src(1 << 16), dst(1 << 16);
  for (size_t i = 0; i < src.size(); ++i) src[i] = (int)(i * 2654435761u);
  long bad = 0;
  for (int r = 0; r < rounds; ++r) {
    std::fill(dst.begin(), dst.end(), 0);
    const size_t per = src.size() / nt;
    auto job = [&](int t) { std::memcpy(&dst[t * per], &src[t * per], per * sizeof(int)); };
    dip::HostPool::get().run(nt, job);
    bad += std::memcmp(src.data(), dst.data(), per * nt * sizeof(int)) != 0;

    std::fill(dst.begin(), dst.end(), 0);
    std::vector<std::atomic<int>> left(nt);
    for (auto& l : left) l.store(1, std::memory_order_relaxed);
    const std::function<void(int)> job2 = [&](int t) {
      std::memcpy(&dst[t * per], &src[t * per], per * sizeof(int));
      left[t].fetch_sub(1, std::memory_order_release);
    };
    dip::HostPool& pool = dip::HostPool::get();
    pool.start(nt, &job2);
    for (int t = 0; t < nt; ++t)
      while (left[t].load(std::memory_order_acquire) != 0) std::this_thread::yield();
    pool.finish();
    bad += std::memcmp(src.data(), dst.data(), per * nt * sizeof(int)) != 0;
  }
  std::printf("rounds %d threads %d bad %ld\n", rounds, nt, bad);
  return bad ? 1 : 0;  // the pool is destroyed by the exit handlers from here
}
