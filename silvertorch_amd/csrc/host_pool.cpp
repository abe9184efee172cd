// Host thread pool of the plan compiler and the query parser (see
// host_pool.hpp).
#include "host_pool.hpp"

#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdlib>
#include <mutex>
#include <thread>

namespace st {
namespace {

thread_local bool t_in_job = false;  // this thread runs a pool job's fn

class HostPool {
 public:
  static HostPool& get() {
    static HostPool* pool = new HostPool();  // never destroyed: workers may still wait
    return *pool;
  }
  // fn(i) for every i in [0, n), chunks of `chunk` taken in turn by the
  // workers and the caller; fn must not throw.
  void run(int64_t n, int64_t chunk, const std::function<void(int64_t)>& fn) {
    // A call from inside a job (worker or caller) runs alone: the caller
    // already holds job_mu_, and try_lock by the owner is undefined.
    if (t_in_job || getpid() != pid_ || workers_ == 0) {
      for (int64_t i = 0; i < n; ++i) fn(i);
      return;
    }
    std::unique_lock<std::mutex> busy(job_mu_, std::try_to_lock);
    if (!busy.owns_lock()) {
      for (int64_t i = 0; i < n; ++i) fn(i);
      return;
    }
    {
      std::lock_guard<std::mutex> lk(mu_);
      fn_ = &fn;
      n_ = n;
      chunk_ = chunk;
      next_.store(0);
      active_ = workers_;
      ++generation_;
    }
    cv_.notify_all();
    work();
    std::unique_lock<std::mutex> lk(mu_);
    done_cv_.wait(lk, [&] { return active_ == 0; });
    fn_ = nullptr;
  }

 private:
  HostPool() : pid_(getpid()) {
    int threads = static_cast<int>(std::min(8u, std::max(1u, std::thread::hardware_concurrency())));
    if (const char* e = std::getenv("ST_PLAN_THREADS")) threads = std::max(1, std::atoi(e));
    workers_ = threads - 1;
    for (int i = 0; i < workers_; ++i) std::thread([this] { loop(); }).detach();
  }
  void work() {
    t_in_job = true;
    for (;;) {
      const int64_t b = next_.fetch_add(chunk_);
      if (b >= n_) break;
      const int64_t e = std::min(n_, b + chunk_);
      for (int64_t i = b; i < e; ++i) (*fn_)(i);
    }
    t_in_job = false;
  }
  void loop() {
    uint64_t seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return generation_ != seen; });
        seen = generation_;
      }
      work();
      std::lock_guard<std::mutex> lk(mu_);
      if (--active_ == 0) done_cv_.notify_one();
    }
  }
  const pid_t pid_;
  int workers_ = 0;
  std::mutex job_mu_;  // one job at a time
  std::mutex mu_;
  std::condition_variable cv_, done_cv_;
  uint64_t generation_ = 0;
  int active_ = 0;
  const std::function<void(int64_t)>* fn_ = nullptr;
  int64_t n_ = 0, chunk_ = 1;
  std::atomic<int64_t> next_{0};
};

}  // namespace

void host_pool_run(int64_t n, int64_t chunk, const std::function<void(int64_t)>& fn) {
  HostPool::get().run(n, chunk, fn);
}

}  // namespace st
