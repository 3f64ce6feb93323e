// dip_host_pool.h — the persistent host thread pool behind the cache-aware
// miss gather (the pinned index_select of dip_ca.py:148-153).  Plain C++17,
// no HIP: the workers only copy host memory, and every HIP call stays on the
// calling thread.
//
// The cache-aware module gathers once per layer and token, and creating
// threads (or waking them through the kernel) per call costs about as much
// as a chunk's copy, so the pool is created on first use and a worker spins
// for a while on the job counter before it sleeps.  Jobs from different
// caller threads run one after another.
//
// Lifetime: the pool is a function-local static, so it is destroyed by the
// exit handlers of the process (or of the library, when it is unloaded).
// Its destructor waits for a job in flight, raises the stop flag, wakes the
// workers and joins them, so no worker thread outlives the pool's state or
// runs while the C++ runtime is being finalised.  A call that still reaches
// a stopped pool runs its jobs on the calling thread.
#pragma once

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace dip {

class HostPool {
 public:
  static HostPool& get() {
    static HostPool pool;
    return pool;
  }

  HostPool() = default;
  HostPool(const HostPool&) = delete;
  HostPool& operator=(const HostPool&) = delete;
  ~HostPool() { shutdown(); }

  // Stop and join every worker (idempotent).  Waits for a job in flight.
  void shutdown() {
    std::lock_guard<std::mutex> one_job(run_mu_);
    std::vector<std::thread> ts;
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_.store(true, std::memory_order_release);
      gen_.fetch_add(1, std::memory_order_release);
      ts.swap(threads_);
    }
    cv_.notify_all();
    for (auto& t : ts) t.join();
  }

  // Run fn(t) for every t in [0, n) on the caller and up to n - 1 workers;
  // returns when all n calls have returned.
  void run(int n, const std::function<void(int)>& fn) {
    std::lock_guard<std::mutex> one_job(run_mu_);
    if (stop_.load(std::memory_order_acquire)) {
      for (int t = 0; t < n; ++t) fn(t);
      return;
    }
    std::unique_lock<std::mutex> lk(mu_);
    spawn_locked(n - 1);
    publish_locked(n, &fn);
    claim(lk);
    done_cv_.wait(lk, [&] { return finished_ == njobs_; });
    fn_ = nullptr;
  }

  // The same with the caller taking no job: start() publishes n jobs to n
  // workers and returns, so the caller can work on their results as they
  // complete; finish() waits for all of them.  Every start() must be
  // followed by finish() on the same thread, and *fn must live until
  // finish() returns (a pointer, so that no temporary std::function can be
  // bound to it).  On a stopped pool start() runs the jobs itself.
  void start(int n, const std::function<void(int)>* fn) {
    run_mu_.lock();
    if (stop_.load(std::memory_order_acquire)) {
      for (int t = 0; t < n; ++t) (*fn)(t);
      inline_job_ = true;
      return;
    }
    std::unique_lock<std::mutex> lk(mu_);
    spawn_locked(n);
    publish_locked(n, fn);
  }
  void finish() {
    if (inline_job_) {
      inline_job_ = false;
    } else {
      std::unique_lock<std::mutex> lk(mu_);
      done_cv_.wait(lk, [&] { return finished_ == njobs_; });
      fn_ = nullptr;
    }
    run_mu_.unlock();
  }
  static constexpr int max_async_jobs() { return (int)kMaxWorkers; }

 private:
  static constexpr unsigned kMaxWorkers = 63;
  static constexpr auto kSpin = std::chrono::microseconds(2000);

  // Workers until there are `want` (at most kMaxWorkers); mu_ held.  A new
  // worker takes part from the job about to be published on.
  void spawn_locked(int want) {
    while ((int)threads_.size() < want && threads_.size() < kMaxWorkers) {
      const uint64_t g = gen_.load(std::memory_order_relaxed);
      threads_.emplace_back([this, g] { worker(g); });
    }
  }

  void publish_locked(int n, const std::function<void(int)>* fn) {
    fn_ = fn;
    njobs_ = n;
    next_ = 0;
    finished_ = 0;
    gen_.fetch_add(1, std::memory_order_release);
    cv_.notify_all();
  }

  // Take job indices until none is left (mu_ held on entry and exit; the
  // job's fields only change under mu_, so an index always belongs to the
  // fn_ read with it).
  void claim(std::unique_lock<std::mutex>& lk) {
    while (next_ < njobs_) {
      const int t = next_++;
      const std::function<void(int)>* f = fn_;
      lk.unlock();
      (*f)(t);
      lk.lock();
      if (++finished_ == njobs_) done_cv_.notify_all();
    }
  }

  void worker(uint64_t seen) {
    for (;;) {
      // spin (yielding) for the next job, then sleep on the condition
      const auto t0 = std::chrono::steady_clock::now();
      while (gen_.load(std::memory_order_acquire) == seen &&
             std::chrono::steady_clock::now() - t0 < kSpin)
        std::this_thread::yield();
      std::unique_lock<std::mutex> lk(mu_);
      cv_.wait(lk, [&] {
        return gen_.load(std::memory_order_relaxed) != seen ||
               stop_.load(std::memory_order_relaxed);
      });
      if (stop_.load(std::memory_order_relaxed)) return;
      seen = gen_.load(std::memory_order_relaxed);
      claim(lk);
    }
  }

  std::mutex run_mu_, mu_;
  std::condition_variable cv_, done_cv_;
  std::atomic<uint64_t> gen_{0};
  std::atomic<bool> stop_{false};
  const std::function<void(int)>* fn_ = nullptr;
  int njobs_ = 0, next_ = 0, finished_ = 0;
  bool inline_job_ = false;  // the current start() ran its jobs itself
  std::vector<std::thread> threads_;
};

}  // namespace dip
