// A few host threads for the plan compiler and the query parser: workers
// started on first use (ST_PLAN_THREADS sets the total, default
// min(8, hardware threads), the caller included) that share one job at a
// time with the calling thread.  A caller that finds the pool busy, calls
// from inside a job's fn, or runs in a child of the process that started
// it, does the work alone.
#pragma once

#include <cstdint>
#include <functional>

namespace st {

// fn(i) for every i in [0, n), chunks of `chunk` indices taken in turn by
// the workers and the caller; fn must not throw.
void host_pool_run(int64_t n, int64_t chunk, const std::function<void(int64_t)>& fn);

}  // namespace st
