// Measurement probe, not part of the search path: the HBM access pattern of
// the batched search kernel with its evaluation taken out, so that the
// bandwidth this read/write mix reaches on the part can be measured on its
// own (bench.py --probe-pattern).  Built into libst_probe.so, a library of
// its own; nothing in the product calls it.
//
// The grid is the search kernel's: one 1024-thread workgroup per CU walks
// groups of RUN adjacent bundles, w, w + grid, ... .  Per bundle it moves the
// bundle's rows (b x 256 bytes, b <= 512) from HBM into an LDS tile through
// registers with 16-byte non-temporal loads, the next bundle's loads issued
// as soon as the current tile is in LDS (the search kernel's form, whose
// registers hold one tile).  After the group's last bundle it writes the
// group's packed output: RUN * 256 contiguous bytes per query row (Q rows of
// 256 * num_bundles bytes), 16 bytes per lane.  RUN 1 is the search kernel's
// store pattern (four query rows per wave instruction); RUN 2 and 4 measure
// whether longer runs per query row raise the write rate.  MODE 1 drops the
// stores (a 16-byte sink per workgroup keeps the loads live), MODE 2 the
// loads; MODE 5 (RUN 1) issues each wave's four tile reads before its four
// stores instead of reading and storing one query row at a time.  Two streaming kernels give the part's contiguous read and write
// rates for comparison.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#define PROBE_GLOBAL __attribute__((address_space(1)))

constexpr int kThreads = 1024;
constexpr int kTileRows = 512;
constexpr int kPer = kTileRows * 16 / kThreads;  // u32x4 per thread per tile

thread_local std::string g_error;

// The tile's rows [start, start + b) from the uniform base; a bundle whose
// rows would pass the end of the index loads nothing.
__device__ __forceinline__ void load_tile(const u32x4* __restrict__ src, int64_t start,
                                          int64_t b, int64_t numel, u32x4 (&pre)[kPer]) {
  const int lim = (start + b) * 32 <= numel ? static_cast<int>(b * 16) : 0;
  const u32x4* base = src + start * 16;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = static_cast<int>(threadIdx.x) + i * kThreads;
    if (c < lim) pre[i] = __builtin_nontemporal_load(base + c);
  }
}

template <int RUN, int MODE>
__global__ __launch_bounds__(kThreads) void pattern_probe_kernel(
    const int64_t* __restrict__ index, int64_t numel, const int64_t* __restrict__ bbo,
    int64_t nb, int64_t Q, char* __restrict__ out, u32x4* __restrict__ sink) {
  __shared__ u32x4 tile[(kTileRows + 2) * 16];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t grid = gridDim.x;
  const u32x4* src = reinterpret_cast<const u32x4*>(index);
  auto extent = [&](int64_t bnd, int64_t& start, int64_t& b) {
    start = bbo[bnd];
    b = bbo[bnd + 1] - start;
    if (b < 0) b = 0;
    if (b > kTileRows) b = kTileRows;
  };
  // bundle of step t of this workgroup's walk (-1: past the end)
  auto bundle_at = [&](int64_t t) -> int64_t {
    const int64_t bnd = (blockIdx.x + (t / RUN) * grid) * RUN + t % RUN;
    return bnd < nb ? bnd : -1;
  };
  u32x4 pre[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) pre[i] = u32x4{1, 2, 3, 4};
  if (MODE != 2 && bundle_at(0) >= 0) {
    int64_t s, b;
    extent(bundle_at(0), s, b);
    load_tile(src, s, b, numel, pre);
  }
  u32x4 acc{0, 0, 0, 0};
  const int64_t row_bytes = nb * 256;
  constexpr int kRowsPerInsn = 4 / RUN;         // query rows one wave instruction covers
  constexpr int kLanesPerRow = 64 / kRowsPerInsn;
  for (int64_t t = 0;; ++t) {
    const int64_t bnd = bundle_at(t);
    if (bnd < 0) break;
    int64_t s, b;
    extent(bnd, s, b);
    __syncthreads();  // the previous bundle's readers are done with the tile
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = tid + i * kThreads;
      if (c < b * 16) tile[c] = pre[i];
    }
    const int64_t ahead = bundle_at(t + 1);
    if (MODE != 2 && ahead >= 0) {
      int64_t s2, b2;
      extent(ahead, s2, b2);
      load_tile(src, s2, b2, numel, pre);
    }
    __syncthreads();
    const int rows = static_cast<int>(b > 0 ? b : 1);
    if (MODE == 1) {
      acc ^= tile[(tid * 7) % (rows * 16)];
      continue;
    }
    // the group's stores follow its last bundle
    if (t % RUN != RUN - 1 && ahead >= 0) continue;
    const int64_t first = bnd - t % RUN;  // the group's first bundle
    const int64_t run_bytes = (bnd - first + 1) * 256;
    if constexpr (MODE == 5) {
      // each wave's tile reads for four query rows first, then their four
      // stores back to back
      for (int64_t q0 = wave * kRowsPerInsn; q0 < Q; q0 += 64 * kRowsPerInsn) {
        u32x4 val[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t q = q0 + 16 * kRowsPerInsn * j + lane / kLanesPerRow;
          val[j] = tile[(static_cast<int>(q % Q) * 16 + (lane & 15)) % (rows * 16)];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t q = q0 + 16 * kRowsPerInsn * j + lane / kLanesPerRow;
          const int64_t off = static_cast<int64_t>(lane % kLanesPerRow) * 16;
          if (q >= Q || off >= run_bytes) continue;
          __builtin_nontemporal_store(val[j], (PROBE_GLOBAL u32x4*)(out + q * row_bytes + first * 256 + off));
        }
      }
      continue;
    }
    for (int64_t q0 = wave * kRowsPerInsn; q0 < Q; q0 += 16 * kRowsPerInsn) {
      const int64_t q = q0 + lane / kLanesPerRow;
      const int64_t off = static_cast<int64_t>(lane % kLanesPerRow) * 16;
      if (q >= Q || off >= run_bytes) continue;
      const u32x4 val = tile[(static_cast<int>(q) * 16 + (lane & 15)) % (rows * 16)];
      PROBE_GLOBAL u32x4* dst = (PROBE_GLOBAL u32x4*)(out + q * row_bytes + first * 256 + off);
      __builtin_nontemporal_store(val, dst);
    }
  }
  if (MODE == 1) sink[blockIdx.x * kThreads + tid] = acc;
}

// The same loads and stores (RUN 1) from a flatter loop: the workgroup walks
// bundles blockIdx.x, + grid, ... directly, reads its four tile values per
// lane, then stores them in one loop (MODE 6 of st_probe_search_pattern).
__global__ __launch_bounds__(kThreads) void pattern_flat_kernel(
    const int64_t* __restrict__ index, int64_t numel, const int64_t* __restrict__ bbo,
    int64_t nb, int64_t Q, char* __restrict__ out) {
  __shared__ u32x4 tile[(kTileRows + 2) * 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const u32x4* src = reinterpret_cast<const u32x4*>(index);
  auto extent = [&](int64_t bnd, int64_t& s, int64_t& b) {
    s = bbo[bnd];
    b = bbo[bnd + 1] - s;
    if (b < 0) b = 0;
    if (b > kTileRows) b = kTileRows;
  };
  u32x4 pre[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) pre[i] = u32x4{1, 2, 3, 4};
  int64_t bnd = blockIdx.x;
  if (bnd < nb) {
    int64_t s, b;
    extent(bnd, s, b);
    load_tile(src, s, b, numel, pre);
  }
  const int64_t row_bytes = nb * 256;
  for (; bnd < nb; bnd += gridDim.x) {
    int64_t s, b;
    extent(bnd, s, b);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = tid + i * kThreads;
      if (c < b * 16) tile[c] = pre[i];
    }
    const int64_t nx = bnd + gridDim.x;
    if (nx < nb) {
      int64_t s2, b2;
      extent(nx, s2, b2);
      load_tile(src, s2, b2, numel, pre);
    }
    __syncthreads();
    const int rows = static_cast<int>(b > 0 ? b : 1);
    u32x4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      v[j] = tile[(static_cast<int>(wave * 4 + 64 * j + lane / 16) * 16 + (lane & 15)) % (rows * 16)];
    int j = 0;
    for (int64_t q0 = wave * 4; q0 < Q; q0 += 64, ++j) {
      const int64_t q = q0 + lane / 16;
      if (q < Q)
        __builtin_nontemporal_store(v[j & 3], (PROBE_GLOBAL u32x4*)(out + q * row_bytes + bnd * 256 + (lane & 15) * 16));
    }
  }
}

// Reference points of the part: the index read as one contiguous stream
// (non-temporal 16-byte loads, 8 per thread in flight, grid-stride) and the
// output written as one contiguous stream (plain 16-byte stores), the two
// forms that measured fastest for each on this part.
__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u32x4* __restrict__ src,
                                                                int64_t n, u32x4* __restrict__ sink) {
  u32x4 acc{0, 0, 0, 0};
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads * 8;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * 8 + threadIdx.x; base < n;
       base += stride) {
    u32x4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t i = base + static_cast<int64_t>(j) * kThreads;
      v[j] = i < n ? __builtin_nontemporal_load(src + i) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= v[j];
  }
  sink[blockIdx.x * kThreads + threadIdx.x] = acc;
}

__global__ __launch_bounds__(kThreads) void stream_write_kernel(u32x4* __restrict__ dst, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride)
    *(PROBE_GLOBAL u32x4*)(dst + i) = u32x4{static_cast<uint32_t>(i), 1u, 2u, 3u};
}

template <int RUN, int MODE>
hipError_t launch(const int64_t* index, int64_t numel, const int64_t* bbo, int64_t nb, int64_t Q,
                  void* out, void* sink, int grid, hipStream_t s) {
  hipLaunchKernelGGL((pattern_probe_kernel<RUN, MODE>), dim3(grid), dim3(kThreads), 0, s, index,
                     numel, bbo, nb, Q, static_cast<char*>(out), static_cast<u32x4*>(sink));
  return hipGetLastError();
}

}  // namespace

// Runs the probe once on `stream`.  run: adjacent bundles per group, 1, 2 or
// 4; mode: 0 loads and stores, 1 loads only, 2 stores only, 3 the index read
// as one stream, 4 the output written as one stream (run ignored for 3 and
// 4).  out: Q x num_bundles x 256 bytes; sink: grid x 1024 x 16 bytes
// (modes 1 and 3).  Returns 0, or -1 with st_probe_last_error() set.
extern "C" int st_probe_search_pattern(const int64_t* index, int64_t numel,
                                       const int64_t* bundle_b_offsets, int64_t num_bundles,
                                       int64_t num_queries, void* out, void* sink, int run,
                                       int mode, int grid, void* stream) {
  if (index == nullptr || bundle_b_offsets == nullptr || out == nullptr || sink == nullptr ||
      num_bundles <= 0 || num_queries <= 0 || grid <= 0 || (run != 1 && run != 2 && run != 4) ||
      mode < 0 || mode > 6 || (mode >= 5 && run != 1) || (mode == 6 && num_queries > 256)) {
    g_error = "st_probe_search_pattern: invalid arguments";
    return -1;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (mode == 3) {
    hipLaunchKernelGGL(stream_read_kernel, dim3(grid), dim3(kThreads), 0, s,
                       reinterpret_cast<const u32x4*>(index), numel / 2, static_cast<u32x4*>(sink));
  } else if (mode == 4) {
    hipLaunchKernelGGL(stream_write_kernel, dim3(grid), dim3(kThreads), 0, s,
                       static_cast<u32x4*>(out), num_queries * num_bundles * 16);
  }
  if (mode == 3 || mode == 4) {
    e = hipGetLastError();
    if (e != hipSuccess) {
      g_error = std::string("st_probe_search_pattern: ") + hipGetErrorString(e);
      return -1;
    }
    return 0;
  }
  if (mode == 5 || mode == 6) {
    if (mode == 5)
      e = launch<1, 5>(index, numel, bundle_b_offsets, num_bundles, num_queries, out, sink, grid, s);
    else {
      hipLaunchKernelGGL(pattern_flat_kernel, dim3(grid), dim3(kThreads), 0, s, index, numel,
                         bundle_b_offsets, num_bundles, num_queries, static_cast<char*>(out));
      e = hipGetLastError();
    }
    if (e != hipSuccess) {
      g_error = std::string("st_probe_search_pattern: ") + hipGetErrorString(e);
      return -1;
    }
    return 0;
  }
  const int sel = run * 3 + mode;
  switch (sel) {
    case 3: e = launch<1, 0>(index, numel, bundle_b_offsets, num_bundles, num_queries, out, sink, grid, s); break;
    case 4: e = launch<1, 1>(index, numel, bundle_b_offsets, num_bundles, num_queries, out, sink, grid, s); break;
    case 5: e = launch<1, 2>(index, numel, bundle_b_offsets, num_bundles, num_queries, out, sink, grid, s); break;
    case 6: e = launch<2, 0>(index, numel, bundle_b_offsets, num_bundles, num_queries, out, sink, grid, s); break;
    case 7: e = launch<2, 1>(index, numel, bundle_b_offsets, num_bundles, num_queries, out, sink, grid, s); break;
    case 8: e = launch<2, 2>(index, numel, bundle_b_offsets, num_bundles, num_queries, out, sink, grid, s); break;
    case 12: e = launch<4, 0>(index, numel, bundle_b_offsets, num_bundles, num_queries, out, sink, grid, s); break;
    case 13: e = launch<4, 1>(index, numel, bundle_b_offsets, num_bundles, num_queries, out, sink, grid, s); break;
    default: e = launch<4, 2>(index, numel, bundle_b_offsets, num_bundles, num_queries, out, sink, grid, s); break;
  }
  if (e != hipSuccess) {
    g_error = std::string("st_probe_search_pattern: ") + hipGetErrorString(e);
    return -1;
  }
  return 0;
}

extern "C" const char* st_probe_last_error() { return g_error.c_str(); }
