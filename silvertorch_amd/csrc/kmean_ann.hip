// Clustered nearest-neighbour scoring: the consumer step after the bloom
// search.  Replaces fused_kmean_ann (fused_kmean_ann.cpp:85-227,
// fused_kmean_ann_cuda.cu) behind the same operator.
//
// Per query row b the candidate docs are the selected clusters' doc ranges
// [cluster_offsets[cluster_ids[b][p]], + cluster_length[b][p]) in probe
// order; docs failing the row's filter mask are skipped, the rest take
// consecutive output slots (as the reference CPU op lays them out) until the
// row is full; the remaining slots hold the padding values.  Filter bit of
// doc d: bit 63 - d % 64 of word d / 64 (the bloom search's packed mask, read
// as the reference CUDA op reads it); docs past the mask's words pass.
//
// Scores are accumulated per doc in float64, dimension by dimension, with no
// fused multiply-add (as fused_kmean_ann.cpp:45-55 does), then converted to
// the score dtype, so every float score equals the reference CPU op's bit
// for bit; int8 dot products are exact int32 sums.
//
// kmean_count_kernel counts the passing docs of every (row, probe).  Calls
// of fewer than 2,048 pairs then run kmean_ann_kernel, one 512-thread
// workgroup per (row, probe): it starts at the row's count of the earlier
// probes, stages the query in LDS as float64, takes its cluster's docs 4,096
// at a time (8 per thread as pass bits: the filter words shifted to the
// docs), lists the passing ones in LDS in doc order (workgroup scan) and
// scores them, one doc per lane, the rows staged through LDS with whole-line
// loads, into the next output slots.  Larger calls take the balanced form
// (ids listed per pair first, then the scoring spread over the chip by
// groups of 64 slots; see kmean_groups_kernel).  Memory-bound on the
// embedding rows read.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <type_traits>

#include "st_common.hpp"
#include "st_errors.hpp"
#include "wave_ops.hpp"

namespace st {
int cu_count();
namespace {

constexpr int kKmThreads = 512;
constexpr int kKmDocsPerThread = 8;  // docs whose pass bits one thread forms per chunk
// Scoring stages the listed docs' rows through LDS, 64 rows per wave and 64
// bytes of each row per step (16 rows x 64 contiguous bytes per load
// instruction); rows padded to 80 bytes so the lanes' 16-byte reads of their
// own rows fall in distinct banks.
constexpr int kKmSliceBytes = 64;
constexpr int kKmStageStride = 80;
constexpr int kKmAhead = 2;  // staging steps whose loads are in flight
constexpr int kKmWaves = kKmThreads / 64;
constexpr int kKmMaxDim = 1280;

// Embedding / score dtype codes of the C ABI (include/silvertorch_hip.h).
enum KmDtype : int { kKmF32 = 0, kKmF16 = 1, kKmBF16 = 2, kKmI8 = 3, kKmI32 = 4 };


__device__ __forceinline__ float half_to_float(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}
// Float32 -> float16, round to nearest even, computed from the float32 bits
// so that a float64 -> float32 -> float16 chain keeps both roundings (a
// single float64 -> float16 rounding differs when the float32 value sits on
// a float16 half-way point).  NaN -> quiet NaN, |f| >= 65520 -> infinity.
__device__ __forceinline__ uint16_t float_to_half(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return static_cast<uint16_t>(sign | 0x7E00u);
  if (a >= 0x477FF000u) return static_cast<uint16_t>(sign | 0x7C00u);
  if (a < 0x38800000u) {
    // below the smallest normal half: the float32 sum with 0.5 rounds to a
    // multiple of 2^-24 (the ulp of 0.5), which is the subnormal half's unit
    const float r = __uint_as_float(a) + 0.5f;
    return static_cast<uint16_t>(sign | (__float_as_uint(r) - 0x3F000000u));
  }
  return static_cast<uint16_t>(sign | ((a + 0xFFFu + ((a >> 13) & 1u) - 0x38000000u) >> 13));
}
__device__ __forceinline__ float bf16_to_float(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// Round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t float_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  return static_cast<uint16_t>((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// Element d of an embedding row as float (exactly representable) or int.
template <int DT>
__device__ __forceinline__ float elem_f(const void* row, int d) {
  if constexpr (DT == kKmF32) return static_cast<const float*>(row)[d];
  if constexpr (DT == kKmF16) return half_to_float(static_cast<const uint16_t*>(row)[d]);
  if constexpr (DT == kKmBF16) return bf16_to_float(static_cast<const uint16_t*>(row)[d]);
  return 0.f;
}

// Float64 dot product of the doc row with the staged query, sequential over
// d, each product and sum rounded on its own (no contraction).
template <int DT>
__device__ double dot_f64(const void* row, const double* q, int dim) {
#pragma clang fp contract(off)
  double acc = 0.0;
  if ((reinterpret_cast<uintptr_t>(row) & 15u) != 0) {  // no 16-byte loads
    for (int d = 0; d < dim; ++d) acc = acc + static_cast<double>(elem_f<DT>(row, d)) * q[d];
    return acc;
  }
  if constexpr (DT == kKmF32) {
    const float4* r4 = static_cast<const float4*>(row);
    int d = 0;
    for (; d + 4 <= dim; d += 4) {
      const float4 v = r4[d / 4];
      acc = acc + static_cast<double>(v.x) * q[d];
      acc = acc + static_cast<double>(v.y) * q[d + 1];
      acc = acc + static_cast<double>(v.z) * q[d + 2];
      acc = acc + static_cast<double>(v.w) * q[d + 3];
    }
    for (; d < dim; ++d) acc = acc + static_cast<double>(elem_f<DT>(row, d)) * q[d];
  } else {
    const uint4* r8 = static_cast<const uint4*>(row);
    int d = 0;
    for (; d + 8 <= dim; d += 8) {
      const uint4 v = r8[d / 8];
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint16_t lo = static_cast<uint16_t>(w[j] & 0xFFFFu);
        const uint16_t hi = static_cast<uint16_t>(w[j] >> 16);
        const float flo = DT == kKmF16 ? half_to_float(lo) : bf16_to_float(lo);
        const float fhi = DT == kKmF16 ? half_to_float(hi) : bf16_to_float(hi);
        acc = acc + static_cast<double>(flo) * q[d + 2 * j];
        acc = acc + static_cast<double>(fhi) * q[d + 2 * j + 1];
      }
    }
    for (; d < dim; ++d) acc = acc + static_cast<double>(elem_f<DT>(row, d)) * q[d];
  }
  return acc;
}

// Adds the 16-byte piece v of a row, whose first element is d0, to the
// running dot product: the same operations in the same order as dot_f64 /
// dot_i8 (so a staged row gives the same bits).
template <int DT>
__device__ __forceinline__ void acc_piece(const uint4& v, const double* q, const int8_t* qi, int d0,
                                          double& acc, int32_t& iacc) {
#pragma clang fp contract(off)
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  if constexpr (DT == kKmF32) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = acc + static_cast<double>(__uint_as_float(w[j])) * q[d0 + j];
  } else if constexpr (DT == kKmI8) {
#pragma unroll
    for (int j = 0; j < 16; ++j)
      iacc += static_cast<int32_t>(static_cast<int8_t>(w[j / 4] >> (8 * (j % 4)))) *
              static_cast<int32_t>(qi[d0 + j]);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint16_t lo = static_cast<uint16_t>(w[j] & 0xFFFFu);
      const uint16_t hi = static_cast<uint16_t>(w[j] >> 16);
      const float flo = DT == kKmF16 ? half_to_float(lo) : bf16_to_float(lo);
      const float fhi = DT == kKmF16 ? half_to_float(hi) : bf16_to_float(hi);
      acc = acc + static_cast<double>(flo) * q[d0 + 2 * j];
      acc = acc + static_cast<double>(fhi) * q[d0 + 2 * j + 1];
    }
  }
}

__device__ int32_t dot_i8(const int8_t* row, const int8_t* q, int dim) {
  int32_t acc = 0;
  int d = 0;
  if ((reinterpret_cast<uintptr_t>(row) & 15u) == 0) {
    for (; d + 16 <= dim; d += 16) {
      const uint4 v = *reinterpret_cast<const uint4*>(row + d);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 16; ++j)
        acc += static_cast<int32_t>(static_cast<int8_t>(w[j / 4] >> (8 * (j % 4)))) *
               static_cast<int32_t>(q[d + j]);
    }
  }
  for (; d < dim; ++d) acc += static_cast<int32_t>(row[d]) * static_cast<int32_t>(q[d]);
  return acc;
}

struct KmArgs {
  const int64_t* cluster_offsets;
  int64_t num_offsets;
  const int64_t* cluster_ids;
  const int64_t* cluster_length;
  int64_t probes;
  const void* embeddings;
  int64_t total_docs;
  int dim;
  const void* queries;
  int64_t max_per_row;
  const int64_t* filter_mask;
  int64_t filter_rows;
  int64_t filter_cols;
  const int64_t* filter_index;
  const uint16_t* scale;  // int8 only: per-doc float16 divisor
  int64_t divisor;        // int8 only: -1 = none
  int64_t invalid_index;
  void* scores;
  int32_t* indices;
};

// Workgroup-wide exclusive scan of per-thread counts; *total receives the sum.
__device__ __forceinline__ uint32_t block_scan(uint32_t v, uint32_t* wave_sums, uint32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  if (lane == 63) wave_sums[wave] = incl;
  __syncthreads();
  uint32_t before = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < kKmWaves; ++w) {
    const uint32_t s = wave_sums[w];
    before += w < wave ? s : 0u;
    sum += s;
  }
  __syncthreads();  // wave_sums is reused by the next call
  *total = sum;
  return before + incl - v;
}

template <int DT, int ST>
__device__ __forceinline__ void put_score(void* scores, int64_t at, double f64, int32_t i32,
                                          float f32_for_half) {
  if constexpr (ST == kKmF32) static_cast<float*>(scores)[at] = static_cast<float>(f64);
  if constexpr (ST == kKmF16) {
    const float f = DT == kKmI8 ? f32_for_half : static_cast<float>(f64);
    static_cast<uint16_t*>(scores)[at] = float_to_half(f);
  }
  if constexpr (ST == kKmBF16)
    static_cast<uint16_t*>(scores)[at] = float_to_bf16(static_cast<float>(f64));
  if constexpr (ST == kKmI32) static_cast<int32_t*>(scores)[at] = i32;
}

// Pass bits of the 64 docs s .. s + 63 (bit 63 = doc s): doc d passes when it
// is one of the first n, lies in [0, total_docs), and its filter bit (bit
// 63 - d % 64 of mask word d / 64) is set or that word is past the mask.
__device__ __forceinline__ uint64_t pass_bits(const int64_t* mask, int64_t cols, int64_t s, int n,
                                              int64_t total_docs) {
  if (n <= 0) return 0;
  uint64_t bits = n >= 64 ? ~0ull : ~(~0ull >> n);
  // docs outside [0, total_docs)
  if (s < 0) bits &= s + 64 <= 0 ? 0ull : (~0ull >> static_cast<int>(-s));
  if (s + 64 > total_docs) {
    const int64_t keep = total_docs - s;
    bits &= keep <= 0 ? 0ull : (keep >= 64 ? ~0ull : ~(~0ull >> keep));
  }
  if (mask == nullptr || bits == 0) return bits;
  const int64_t w = s >> 6;  // arithmetic shift: s may be negative
  const int o = static_cast<int>(s & 63);
  auto word = [&](int64_t i) -> uint64_t {
    return i < 0 ? 0ull : (i < cols ? static_cast<uint64_t>(mask[i]) : ~0ull);
  };
  uint64_t f = word(w) << o;
  if (o != 0) f |= word(w + 1) >> (64 - o);
  return bits & f;
}

// Pass bits of this thread's docs of chunk `base` of cluster (b, p).
struct KmProbe {
  int64_t start, len;
};

__device__ __forceinline__ KmProbe km_probe(const KmArgs& a, int64_t b, int64_t p) {
  const int64_t cid = a.cluster_ids[b * a.probes + p];
  int64_t len = a.cluster_length[b * a.probes + p];
  // a cluster id outside the offsets or a negative length is an empty
  // cluster (the reference reads out of bounds there)
  if (cid < 0 || cid >= a.num_offsets || len < 0) len = 0;
  return KmProbe{len > 0 ? a.cluster_offsets[cid] : 0, len};
}

// The row's filter words, nullptr without a filter; `none` is set when the
// row's filter_index names no row of the mask (then no doc passes).
__device__ __forceinline__ const int64_t* km_mask_row(const KmArgs& a, int64_t b, bool& none) {
  none = false;
  if (a.filter_mask == nullptr) return nullptr;
  const int64_t frow = a.filter_index != nullptr ? a.filter_index[b] : b;
  none = frow < 0 || frow >= a.filter_rows;
  return none ? nullptr : a.filter_mask + frow * a.filter_cols;
}

__device__ __forceinline__ uint64_t chunk_bits(const KmArgs& a, const int64_t* mask, KmProbe pr,
                                               int64_t base, int64_t& i0) {
  i0 = base + static_cast<int64_t>(threadIdx.x) * kKmDocsPerThread;
  const int n = static_cast<int>(min<int64_t>(max<int64_t>(pr.len - i0, 0), kKmDocsPerThread));
  return pass_bits(mask, a.filter_cols, pr.start + i0, n, a.total_docs);
}

constexpr int64_t kKmChunk = kKmThreads * kKmDocsPerThread;

// Passing docs of each (row, probe): counts[b * probes + p], one wave per
// (row, probe), 64 docs per lane per step.
constexpr int kKmCountThreads = 256;
__global__ __launch_bounds__(kKmCountThreads) void kmean_count_kernel(KmArgs a, int64_t* counts,
                                                                      int64_t items) {
  const int64_t item = static_cast<int64_t>(blockIdx.x) * (kKmCountThreads / 64) + (threadIdx.x >> 6);
  if (item >= items) return;
  const int lane = threadIdx.x & 63;
  const int64_t b = item / a.probes, p = item % a.probes;
  KmProbe pr = km_probe(a, b, p);
  bool none;
  const int64_t* mask = km_mask_row(a, b, none);
  if (none) pr.len = 0;
  int64_t sum = 0;
  for (int64_t i0 = static_cast<int64_t>(lane) * 64; i0 < pr.len; i0 += 64 * 64) {
    const int n = static_cast<int>(min<int64_t>(pr.len - i0, 64));
    sum += __popcll(pass_bits(mask, a.filter_cols, pr.start + i0, n, a.total_docs));
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
  if (lane == 0) counts[item] = sum;
}

// Fills n elements of es bytes (2 or 4) at p with the element `word`
// (its low es bytes): the elements before the first 16-byte boundary one by
// one, then 16-byte stores, then the rest; thread t of nt.
__device__ __forceinline__ void km_fill(char* p, int64_t n, int es, uint32_t word, int t, int nt) {
  const int per = 16 / es;
  int64_t head = static_cast<int64_t>(((16u - (reinterpret_cast<uintptr_t>(p) & 15u)) & 15u) / es);
  if (head > n) head = n;
  auto one = [&](char* q) {
    if (es == 2) *reinterpret_cast<uint16_t*>(q) = static_cast<uint16_t>(word);
    else *reinterpret_cast<uint32_t*>(q) = word;
  };
  if (t < head) one(p + t * es);
  char* q = p + head * es;
  const int64_t m = n - head, units = m / per;
  const uint32_t w = es == 2 ? ((word & 0xFFFFu) | (word << 16)) : word;
  for (int64_t u = t; u < units; u += nt) reinterpret_cast<uint4*>(q)[u] = make_uint4(w, w, w, w);
  for (int64_t i = units * per + t; i < m; i += nt) one(q + i * es);
}

// Padding of slots [s0, s1) of the output row starting at out0: the score
// dtype's most negative finite value (-FLT_MAX, -65504 for float16, 0xFF7F
// for bfloat16) or INT32_MIN, and invalid_index.
template <int ST>
__device__ __forceinline__ void km_pad_range(const KmArgs& a, int64_t out0, int64_t s0, int64_t s1,
                                             int t, int nt) {
  if (s1 <= s0) return;
  const int es = ST == kKmF16 || ST == kKmBF16 ? 2 : 4;
  const uint32_t word = ST == kKmF32 ? 0xFF7FFFFFu
                        : ST == kKmF16 ? 0xFBFFu
                        : ST == kKmBF16 ? 0xFF7Fu
                                        : 0x80000000u;
  km_fill(static_cast<char*>(a.scores) + (out0 + s0) * es, s1 - s0, es, word, t, nt);
  km_fill(reinterpret_cast<char*>(a.indices + out0 + s0), s1 - s0, 4,
          static_cast<uint32_t>(static_cast<int32_t>(a.invalid_index)), t, nt);
}

// DT: embedding dtype; ST: score dtype.  One workgroup per (row, probe):
// its first output slot is the row's passing docs of the earlier probes
// (from counts); per chunk of 4,096 docs of the cluster every thread forms
// the pass bits of 8 docs, the passing docs are listed in LDS in doc order
// (workgroup scan of the counts), then the whole workgroup scores them, one
// doc per lane, into the next slots while the row has room.  The row's last probe (or, without probes, the only
// workgroup) writes the padding.
template <int DT, int ST>
__global__ __launch_bounds__(kKmThreads) __attribute__((amdgpu_waves_per_eu(4))) void kmean_ann_kernel(KmArgs a, const int64_t* counts) {
  __shared__ double qd[kKmMaxDim];
  __shared__ int8_t qi[kKmMaxDim];
  __shared__ uint32_t wave_sums[kKmWaves];
  __shared__ int64_t base_sum[kKmWaves];
  __shared__ int32_t list[kKmThreads * kKmDocsPerThread];
  __shared__ __align__(16) char stage[kKmWaves * 64 * kKmStageStride];
  const int64_t nprobes = a.probes > 0 ? a.probes : 1;
  const int64_t b = blockIdx.x / nprobes, p = blockIdx.x % nprobes;
  const int tid = threadIdx.x;
  const int dim = a.dim;
  const int64_t out0 = b * a.max_per_row;

  // first slot: passing docs of the row's probes before p
  int64_t part = 0;
  if (a.probes > 0)
    for (int64_t q = tid; q < p; q += kKmThreads) part += counts[b * a.probes + q];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off, 64);
  if ((tid & 63) == 0) base_sum[tid >> 6] = part;
  if constexpr (DT == kKmI8) {
    const int8_t* q = static_cast<const int8_t*>(a.queries) + b * dim;
    for (int d = tid; d < dim; d += kKmThreads) qi[d] = q[d];
  } else {
    const size_t es = DT == kKmF32 ? 4 : 2;
    const char* q = static_cast<const char*>(a.queries) + static_cast<size_t>(b) * dim * es;
    for (int d = tid; d < dim; d += kKmThreads) qd[d] = static_cast<double>(elem_f<DT>(q, d));
  }
  __syncthreads();
  int64_t written = 0;
#pragma unroll
  for (int w = 0; w < kKmWaves; ++w) written += base_sum[w];

  const size_t row_bytes = static_cast<size_t>(dim) * (DT == kKmF32 ? 4 : (DT == kKmI8 ? 1 : 2));
  const char* emb = static_cast<const char*>(a.embeddings);
  auto finish = [&](int32_t doc, int64_t slot, double f64, int32_t i32) {
    float f32h = 0.f;
    if constexpr (DT == kKmI8) {
      if (a.scale != nullptr)
        f32h = static_cast<float>(i32) / half_to_float(a.scale[doc]);
      else if (a.divisor != -1)
        f32h = static_cast<float>(i32) / static_cast<float>(a.divisor);
    }
    put_score<DT, ST>(a.scores, out0 + slot, f64, i32, f32h);
    a.indices[out0 + slot] = doc;
  };
  // Unstaged: each thread reads its own row (rows not 16-byte aligned).
  auto score = [&](int32_t doc, int64_t slot) {
    const char* row = emb + static_cast<size_t>(doc) * row_bytes;
    if constexpr (DT == kKmI8)
      finish(doc, slot, 0.0, dot_i8(reinterpret_cast<const int8_t*>(row), qi, dim));
    else
      finish(doc, slot, dot_f64<DT>(row, qd, dim), 0);
  };
  const bool staged = (reinterpret_cast<uintptr_t>(emb) & 15u) == 0 && row_bytes % 16 == 0;
  // Staged: wave w scores list entries [64 g, 64 g + 64) for g = w, w + 8, ...
  // lane l the entry 64 g + l.  Step t of the wave = (group t / nslices, 64-byte
  // slice t % nslices); slices t + 1 .. t + 4 are in flight into registers
  // while slice t is summed from LDS.  LDS ops of one wave execute in order, so the lanes'
  // reads see the whole wave's writes and precede the next step's writes.
  auto score_staged = [&](int64_t m, int64_t slot0) {
    const int wave = tid >> 6, lane = tid & 63;
    char* stg = stage + wave * (64 * kKmStageStride);
    const int pieces = static_cast<int>(row_bytes / 16);
    const int per_slice = kKmSliceBytes / 16;
    const int nslices = (pieces + per_slice - 1) / per_slice;
    const int elems = DT == kKmF32 ? 4 : (DT == kKmI8 ? 16 : 8);  // per piece
    const int64_t ngroups = (m + 63) / 64;
    const int64_t mine = ngroups > wave ? (ngroups - wave + kKmWaves - 1) / kKmWaves : 0;
    const int64_t steps = mine * nslices;
    const int lr = lane >> 2, lp = lane & 3;  // load: row lr + 16 i, piece lp of the slice
    auto load = [&](int64_t t, uint4 (&buf)[4]) {
      const int64_t g = wave + (t / nslices) * kKmWaves;
      const int pc = static_cast<int>(t % nslices) * per_slice + lp;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t li = g * 64 + lr + 16 * i;
        buf[i] = li < m && pc < pieces
                     ? *reinterpret_cast<const uint4*>(emb + static_cast<size_t>(list[li]) * row_bytes +
                                                       static_cast<size_t>(pc) * 16)
                     : make_uint4(0u, 0u, 0u, 0u);
      }
    };
    double acc = 0.0;
    int32_t iacc = 0;
    uint4 buf[kKmAhead][4];  // steps t .. t + kKmAhead - 1 in flight
#pragma unroll
    for (int j = 0; j < kKmAhead; ++j)
      if (j < steps) load(j, buf[j]);
    for (int64_t t0 = 0; t0 < steps; t0 += kKmAhead) {
#pragma unroll
      for (int j = 0; j < kKmAhead; ++j) {
        const int64_t t = t0 + j;
        if (t >= steps) break;
        const int sl = static_cast<int>(t % nslices);
        const int64_t li = (wave + (t / nslices) * kKmWaves) * 64 + lane;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<uint4*>(stg + (lr + 16 * i) * kKmStageStride + lp * 16) = buf[j][i];
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (t + kKmAhead < steps) load(t + kKmAhead, buf[j]);
        if (li < m) {
#pragma unroll
          for (int q = 0; q < per_slice; ++q) {
            const int pc = sl * per_slice + q;
            if (pc < pieces) {
              const uint4 v = *reinterpret_cast<const uint4*>(stg + lane * kKmStageStride + q * 16);
              acc_piece<DT>(v, qd, qi, pc * elems, acc, iacc);
            }
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (sl == nslices - 1) {
          if (li < m) finish(list[li], slot0 + li, acc, iacc);
          acc = 0.0;
          iacc = 0;
        }
      }
    }
  };
  if (a.probes > 0) {
    KmProbe pr = km_probe(a, b, p);
    bool none;
    const int64_t* mask = km_mask_row(a, b, none);
    if (none) pr.len = 0;
    for (int64_t base = 0; base < pr.len && written < a.max_per_row; base += kKmChunk) {
      int64_t i0;
      uint64_t bits = chunk_bits(a, mask, pr, base, i0);
      uint32_t total;
      uint32_t at = block_scan(static_cast<uint32_t>(__popcll(bits)), wave_sums, &total);
      while (bits != 0) {  // this thread's passing docs, in order
        const int j = __clzll(bits);
        list[at++] = static_cast<int32_t>(pr.start + i0 + j);
        bits &= ~(0x8000000000000000ull >> j);
      }
      __syncthreads();
      const int64_t m = min<int64_t>(total, a.max_per_row - written);
      if (staged) {
        score_staged(m, written);
      } else {
        for (int64_t i = tid; i < m; i += 2 * kKmThreads) {
          score(list[i], written + i);
          if (i + kKmThreads < m) score(list[i + kKmThreads], written + i + kKmThreads);
        }
      }
      written += total;
      __syncthreads();  // the list is refilled by the next chunk
    }
  }
  if (p != nprobes - 1) return;
  // padding (as the reference CUDA op pads, simple_index_mm.cuh:99-123)
  km_pad_range<ST>(a, out0, min(written, a.max_per_row), a.max_per_row, tid, kKmThreads);
}

// ------------------------------------------------ balanced form (many pairs)
//
// Calls with at least kKmBalancedPairs (row, probe) pairs are split so that
// the scoring work, not the pairs, is spread evenly: the passing docs per
// query vary by orders of magnitude (a search filter passes 0-54% of a
// cluster), and a workgroup or a wave per pair leaves the chip waiting on
// the heaviest pairs.
//   kmean_count_kernel   passing docs per (row, probe), as above;
//   kmean_groups_kernel  one workgroup: per row its total, its filled slots
//                        n_b = min(total, width) and its groups of 64 slots,
//                        with the exclusive prefix of the groups over rows;
//   kmean_list_kernel    one wave per (row, probe): lists the passing docs
//                        (chunks of 4,096 docs, 64 per lane, offsets in LDS)
//                        and writes their ids into the row's slots; the
//                        row's padding is split over its probes' waves;
//   kmean_score_kernel   a fixed grid of waves; wave w takes the groups
//                        [G w / W, G (w + 1) / W) of the G in the call, reads
//                        each group's 64 ids from the output and scores the
//                        docs from 128-byte slices of their rows (64-byte
//                        for the longest rows) staged through LDS as in
//                        kmean_ann_kernel, the loads of the next step (and
//                        the next group's ids) in flight while a slice is
//                        summed.
constexpr int kKmWaveThreads = 256;  // 4 waves per workgroup
constexpr int kKmWaveDocsPerLane = 64;  // list pass: one 4,096-doc chunk per step
constexpr int kKmWaveChunk = 64 * kKmWaveDocsPerLane;
// scoring stages SL bytes of each of a group's 64 rows per step (SL = 128 or
// 64, a template parameter of kmean_score_kernel): SL / 16 lanes per row,
// 64 / (SL / 16) rows per load instruction; rows padded by 16 bytes so the
// lanes' 16-byte reads of their own rows fall in distinct banks.  A 128-byte
// slice is a whole line, loaded non-temporal with one step in flight (2
// measured no faster); with 64-byte slices a line's second half is read a
// step later from L2, which then has to keep it, so those loads are plain
// (non-temporal ones fetch the line twice), two steps in flight.  64-byte
// slices serve the dims whose 128-byte tile leaves no room for the query.
constexpr int kKmScoreThreads = 256;
constexpr int kKmScorePerCu = 4;  // workgroups per CU at most (LDS permitting)
__host__ __device__ constexpr int km_score_stage(int slice) { return 64 * (slice + 16); }
constexpr int kKmRing = 4;  // groups whose ids and place are held per wave
constexpr int kKmRingBytes = kKmRing * (64 * 4 + 32);  // ids, then a KmGroup (24 bytes) each
__host__ __device__ constexpr int km_score_ahead(int slice) { return slice == 128 ? 1 : 2; }
// the loads may run km_score_ahead groups ahead of the sums (one slice per row)
static_assert(kKmRing > km_score_ahead(64) && kKmRing > km_score_ahead(128) &&
                  (kKmRing & (kKmRing - 1)) == 0,
              "ring size");
constexpr int64_t kKmBalancedPairs = 2048;
constexpr int64_t kKmBalancedMaxRows = 16384;  // rows the single-workgroup prefix takes
constexpr int kKmWaveMaxLds = 65536;           // dynamic LDS of a score workgroup
constexpr int kCuLdsBytes = 160 * 1024;        // LDS of a gfx950 CU
constexpr int kKmGroupsThreads = 1024;

__host__ __device__ constexpr int km_query_bytes(int dim, bool i8) {
  return ((i8 ? dim : 8 * dim) + 15) / 16 * 16;
}
__host__ __device__ constexpr int km_score_wave_lds(int dim, bool i8, int slice) {
  return km_query_bytes(dim, i8) + km_score_stage(slice) + kKmRingBytes;
}

// Workspace of the balanced form after the batch x probes counts, int64:
// row totals [batch], group starts [batch + 1].
__host__ __device__ constexpr int64_t km_balanced_extra(int64_t batch) { return 2 * batch + 1; }

__global__ __launch_bounds__(kKmGroupsThreads) void kmean_groups_kernel(
    const int64_t* __restrict__ counts, int64_t batch, int64_t probes, int64_t width,
    int64_t* __restrict__ rowtot, int64_t* __restrict__ gstart) {
  __shared__ int64_t wave_tot[kKmGroupsThreads / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int64_t carry = 0;
  for (int64_t b0 = 0; b0 < batch; b0 += kKmGroupsThreads) {
    const int64_t b = b0 + threadIdx.x;
    int64_t groups = 0;
    if (b < batch) {
      int64_t total = 0;
      for (int64_t p = 0; p < probes; ++p) total += counts[b * probes + p];
      rowtot[b] = total;
      groups = (min(total, width) + 63) / 64;
    }
    int64_t x = groups;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int64_t y = __shfl_up(x, off, 64);
      if (lane >= off) x += y;
    }
    if (lane == 63) wave_tot[wave] = x;
    __syncthreads();
    int64_t before = 0, sum = 0;
#pragma unroll
    for (int j = 0; j < kKmGroupsThreads / 64; ++j) {
      const int64_t t = wave_tot[j];
      before += j < wave ? t : 0;
      sum += t;
    }
    __syncthreads();
    if (b < batch) gstart[b] = carry + before + x - groups;
    carry += sum;
  }
  if (threadIdx.x == 0) gstart[batch] = carry;
}

template <int ST>
__global__ __launch_bounds__(kKmWaveThreads) void kmean_list_kernel(KmArgs a, const int64_t* counts,
                                                                    const int64_t* rowtot,
                                                                    int64_t pairs) {
  __shared__ uint16_t lists[kKmWaveThreads / 64][kKmWaveChunk];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t pair = static_cast<int64_t>(blockIdx.x) * (kKmWaveThreads / 64) + wv;
  if (pair >= pairs) return;
  uint16_t* list = lists[wv];
  const int64_t b = pair / a.probes, p = pair % a.probes;
  const int64_t out0 = b * a.max_per_row;
  int64_t written = 0;  // the row's passing docs before this probe
  for (int64_t q = lane; q < p; q += 64) written += counts[b * a.probes + q];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) written += __shfl_xor(written, off, 64);
  KmProbe pr = km_probe(a, b, p);
  bool none;
  const int64_t* mask = km_mask_row(a, b, none);
  if (none) pr.len = 0;
  for (int64_t base = 0; base < pr.len && written < a.max_per_row; base += kKmWaveChunk) {
    const int64_t i0 = base + static_cast<int64_t>(lane) * kKmWaveDocsPerLane;
    const int n = static_cast<int>(min<int64_t>(max<int64_t>(pr.len - i0, 0), kKmWaveDocsPerLane));
    uint64_t bits = pass_bits(mask, a.filter_cols, pr.start + i0, n, a.total_docs);
    const uint32_t cnt = static_cast<uint32_t>(__popcll(bits));
    uint32_t total;
    uint32_t at = wave_inclusive_sum(cnt, &total) - cnt;
    while (bits != 0) {  // this lane's passing docs, in order
      const int j = __clzll(bits);
      list[at++] = static_cast<uint16_t>(lane * kKmWaveDocsPerLane + j);
      bits &= ~(0x8000000000000000ull >> j);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int64_t m = min<int64_t>(total, a.max_per_row - written);
    for (int64_t i = lane; i < m; i += 64)
      a.indices[out0 + written + i] = static_cast<int32_t>(pr.start + base + list[i]);
    written += total;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();  // the list is refilled by the next chunk
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // padding: slots [min(total, width), width) of the row, split over its probes
  const int64_t lo = min(rowtot[b], a.max_per_row);
  const int64_t share = (a.max_per_row - lo + a.probes - 1) / a.probes;
  const int64_t s0 = lo + p * share, s1 = min(a.max_per_row, s0 + share);
  km_pad_range<ST>(a, out0, s0, s1, lane, 64);
}

// Place of a group of 64 slots: row, first slot, filled slots in it.
typedef uint32_t km_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 km_load_nt16(const char* p) {
  const km_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const km_u32x4*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

struct KmGroup {
  int64_t b, s0;
  int32_t n, pad;
};
static_assert(sizeof(KmGroup) <= 32, "a ring entry holds 32 bytes");

template <int DT, int ST, int SL>
__global__ __launch_bounds__(kKmScoreThreads) __attribute__((amdgpu_waves_per_eu(4))) void kmean_score_kernel(
    KmArgs a, const int64_t* __restrict__ gstart, const int64_t* __restrict__ rowtot, int64_t batch) {
  extern __shared__ __align__(16) char km_lds[];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t nw = static_cast<int64_t>(gridDim.x) * (kKmScoreThreads / 64);
  const int64_t w = static_cast<int64_t>(blockIdx.x) * (kKmScoreThreads / 64) + wv;
  const int64_t G = gstart[batch];
  const int64_t g_lo = G * w / nw, g_hi = G * (w + 1) / nw;
  if (g_lo >= g_hi) return;
  const int dim = a.dim;
  constexpr int kLanes = SL / 16, kStride = SL + 16, kAhead = km_score_ahead(SL);
  char* mine = km_lds + wv * km_score_wave_lds(dim, DT == kKmI8, SL);
  double* qd = reinterpret_cast<double*>(mine);
  int8_t* qi = reinterpret_cast<int8_t*>(mine);
  char* stg = mine + km_query_bytes(dim, DT == kKmI8);
  int32_t* ring_ids = reinterpret_cast<int32_t*>(stg + km_score_stage(SL));  // [kKmRing][64]
  KmGroup* ring = reinterpret_cast<KmGroup*>(ring_ids + kKmRing * 64);

  // row cursor of the next group to be placed: the largest row b with
  // gstart[b] <= g (rows without groups have gstart[b] == gstart[b + 1])
  int64_t cb = 0, hi = batch;
  while (hi - cb > 1) {
    const int64_t mid = (cb + hi) / 2;
    if (gstart[mid] <= g_lo) cb = mid; else hi = mid;
  }
  int64_t c_start = gstart[cb], c_next = gstart[cb + 1];
  int64_t c_fill = min(rowtot[cb], a.max_per_row);
  auto place = [&](int64_t g) -> KmGroup {
    while (g >= c_next) {
      ++cb;
      c_start = c_next;
      c_next = gstart[cb + 1];
      c_fill = -1;
    }
    if (c_fill < 0) c_fill = min(rowtot[cb], a.max_per_row);
    const int64_t s0 = (g - c_start) * 64;
    return KmGroup{cb, s0, static_cast<int32_t>(min<int64_t>(64, c_fill - s0)), 0};
  };
  // the next group's ids travel in a register, loaded one group ahead
  KmGroup nxt = place(g_lo);
  int32_t nid = lane < nxt.n ? a.indices[nxt.b * a.max_per_row + nxt.s0 + lane] : 0;
  // group g enters: its ids and place go to the ring, group g + 1's ids are loaded
  KmGroup lg{};  // the group whose rows are being loaded
  auto enter = [&](int64_t g) {
    lg = nxt;
    ring_ids[(g & (kKmRing - 1)) * 64 + lane] = nid;
    if (lane == 0) ring[g & (kKmRing - 1)] = lg;
    if (g + 1 < g_hi) {
      nxt = place(g + 1);
      nid = lane < nxt.n ? a.indices[nxt.b * a.max_per_row + nxt.s0 + lane] : 0;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  int64_t qrow = -1;  // row whose query is staged
  auto stage_query = [&](int64_t b) {
    if constexpr (DT == kKmI8) {
      const int8_t* q = static_cast<const int8_t*>(a.queries) + b * dim;
      for (int d = lane; d < dim; d += 64) qi[d] = q[d];
    } else {
      const size_t es = DT == kKmF32 ? 4 : 2;
      const char* q = static_cast<const char*>(a.queries) + static_cast<size_t>(b) * dim * es;
      for (int d = lane; d < dim; d += 64) qd[d] = static_cast<double>(elem_f<DT>(q, d));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    qrow = b;
  };
  const size_t row_bytes = static_cast<size_t>(dim) * (DT == kKmF32 ? 4 : (DT == kKmI8 ? 1 : 2));
  const char* emb = static_cast<const char*>(a.embeddings);
  auto finish = [&](const KmGroup& gr, int32_t doc, double f64, int32_t i32) {
    float f32h = 0.f;
    if constexpr (DT == kKmI8) {
      if (a.scale != nullptr)
        f32h = static_cast<float>(i32) / half_to_float(a.scale[doc]);
      else if (a.divisor != -1)
        f32h = static_cast<float>(i32) / static_cast<float>(a.divisor);
    }
    put_score<DT, ST>(a.scores, gr.b * a.max_per_row + gr.s0 + lane, f64, i32, f32h);
  };
  const bool staged = (reinterpret_cast<uintptr_t>(emb) & 15u) == 0 && row_bytes % 16 == 0;
  if (!staged) {
    for (int64_t g = g_lo; g < g_hi; ++g) {
      enter(g);
      if (lg.b != qrow) stage_query(lg.b);
      if (lane < lg.n) {
        const int32_t doc = ring_ids[(g & (kKmRing - 1)) * 64 + lane];
        const char* row = emb + static_cast<size_t>(doc) * row_bytes;
        if constexpr (DT == kKmI8)
          finish(lg, doc, 0.0, dot_i8(reinterpret_cast<const int8_t*>(row), qi, dim));
        else
          finish(lg, doc, dot_f64<DT>(row, qd, dim), 0);
      }
    }
    return;
  }
  // step t = (group g_lo + t / nslices, SL-byte slice t % nslices)
  const int pieces = static_cast<int>(row_bytes / 16);
  constexpr int per_slice = kLanes;
  constexpr int rows_per_load = 64 / kLanes;
  const int nslices = (pieces + per_slice - 1) / per_slice;
  const int elems = DT == kKmF32 ? 4 : (DT == kKmI8 ? 16 : 8);  // per piece
  const int64_t steps = (g_hi - g_lo) * nslices;
  // load: row lr + rows_per_load i, piece lp of the slice
  const int lr = lane / kLanes, lp = lane % kLanes;
  auto load = [&](int64_t t, uint4 (&buf)[kLanes]) {
    const int64_t g = g_lo + t / nslices;
    const int sl = static_cast<int>(t % nslices);
    if (sl == 0) enter(g);
    const int pc = sl * per_slice + lp;
    const int32_t* ids = ring_ids + (g & (kKmRing - 1)) * 64;
#pragma unroll
    for (int i = 0; i < kLanes; ++i) {
      const int li = lr + rows_per_load * i;
      const char* src = emb + static_cast<size_t>(ids[li]) * row_bytes + static_cast<size_t>(pc) * 16;
      if constexpr (SL == 128)
        buf[i] = li < lg.n && pc < pieces ? km_load_nt16(src) : make_uint4(0u, 0u, 0u, 0u);
      else
        buf[i] = li < lg.n && pc < pieces ? *reinterpret_cast<const uint4*>(src)
                                          : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  double acc = 0.0;
  int32_t iacc = 0;
  uint4 buf[kAhead][kLanes];
#pragma unroll
  for (int j = 0; j < kAhead; ++j)
    if (j < steps) load(j, buf[j]);
  for (int64_t t0 = 0; t0 < steps; t0 += kAhead) {
#pragma unroll
    for (int j = 0; j < kAhead; ++j) {
      const int64_t t = t0 + j;
      if (t >= steps) break;
      const int64_t g = g_lo + t / nslices;
      const int sl = static_cast<int>(t % nslices);
      const KmGroup gr = ring[g & (kKmRing - 1)];
      if (sl == 0 && gr.b != qrow) stage_query(gr.b);
#pragma unroll
      for (int i = 0; i < kLanes; ++i)
        *reinterpret_cast<uint4*>(stg + (lr + rows_per_load * i) * kStride + lp * 16) = buf[j][i];
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      if (t + kAhead < steps) load(t + kAhead, buf[j]);
      if (lane < gr.n) {
#pragma unroll
        for (int q = 0; q < per_slice; ++q) {
          const int pc = sl * per_slice + q;
          if (pc < pieces) {
            const uint4 v = *reinterpret_cast<const uint4*>(stg + lane * kStride + q * 16);
            acc_piece<DT>(v, qd, qi, pc * elems, acc, iacc);
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      if (sl == nslices - 1) {
        if (lane < gr.n) finish(gr, ring_ids[(g & (kKmRing - 1)) * 64 + lane], acc, iacc);
        acc = 0.0;
        iacc = 0;
      }
    }
  }
}

}  // namespace
}  // namespace st

extern "C" int st_kmean_ann_score_dtype(int emb_dtype, int64_t divisor_for_int8,
                                        int has_per_embedding_scale) {
  using namespace st;
  if (emb_dtype != kKmI8) return emb_dtype;
  return (divisor_for_int8 != -1 || has_per_embedding_scale) ? kKmF16 : kKmI32;
}

extern "C" int64_t st_fused_kmean_ann_workspace_bytes(int64_t batch, int64_t probes) {
  using namespace st;
  return batch > 0 && probes > 0
             ? (batch * probes + km_balanced_extra(batch)) * static_cast<int64_t>(sizeof(int64_t))
             : 0;
}

namespace st {
namespace {

// Validates the arguments, fills KmArgs and launches both kernels with
// `counts` (batch x probes int64) as the per-(row, probe) count buffer;
// `counts_capacity` (items) bounds it, -1 = unchecked (caller-sized).
void kmean_run(const int64_t* cluster_offsets, int64_t num_offsets, const int64_t* cluster_ids,
               const int64_t* cluster_length, int64_t batch, int64_t probes, const void* embeddings,
               int64_t total_docs, int64_t dim, int emb_dtype, const void* queries, int64_t max_per_row,
               const int64_t* filter_mask, int64_t filter_rows, int64_t filter_cols,
               const int64_t* filter_index, const uint16_t* per_embedding_scale, int64_t divisor_for_int8,
               int64_t invalid_index_value, int64_t* counts, int64_t counts_capacity, void* scores,
               int32_t* indices, void* stream) {
  ST_CHECK(batch >= 0 && probes >= 0 && total_docs >= 0 && max_per_row >= 0 && num_offsets >= 0,
           "negative sizes");
  ST_CHECK(dim >= 1 && dim <= kKmMaxDim, "embedding dim must be in [1, ", kKmMaxDim, "], got ", dim);
  ST_CHECK(emb_dtype >= kKmF32 && emb_dtype <= kKmI8, "unsupported embedding dtype code ", emb_dtype);
  if (batch == 0 || max_per_row == 0) return;
  ST_CHECK(counts_capacity < 0 || probes == 0 || batch <= counts_capacity / probes,
           "batch x probes = ", batch, " x ", probes, " exceeds the ", counts_capacity,
           " (row, probe) pairs of the no-allocation entry point's scratch");
  ST_CHECK(scores != nullptr && indices != nullptr && queries != nullptr, "null device pointer");
  ST_CHECK(probes == 0 || (cluster_ids != nullptr && cluster_length != nullptr &&
                           cluster_offsets != nullptr),
           "null cluster arrays");
  ST_CHECK(filter_mask == nullptr || (filter_cols >= 0 && filter_rows >= 0),
           "negative filter mask shape");
  ST_CHECK(filter_mask == nullptr || filter_index != nullptr || filter_rows >= batch,
           "filter mask has ", filter_rows, " rows for ", batch, " queries");
  KmArgs a;
  a.cluster_offsets = cluster_offsets;
  a.num_offsets = num_offsets;
  a.cluster_ids = cluster_ids;
  a.cluster_length = cluster_length;
  a.probes = probes;
  a.embeddings = embeddings;
  a.total_docs = embeddings != nullptr ? total_docs : 0;
  a.dim = static_cast<int>(dim);
  a.queries = queries;
  a.max_per_row = max_per_row;
  a.filter_mask = filter_mask;
  a.filter_rows = filter_rows;
  a.filter_cols = filter_cols;
  a.filter_index = filter_index;
  a.scale = emb_dtype == kKmI8 ? per_embedding_scale : nullptr;
  a.divisor = divisor_for_int8;
  a.invalid_index = invalid_index_value;
  a.scores = scores;
  a.indices = indices;
  const int st = st_kmean_ann_score_dtype(emb_dtype, divisor_for_int8, a.scale != nullptr);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t groups = batch * std::max<int64_t>(probes, 1);
  ST_CHECK(groups <= INT32_MAX, "batch x probes = ", groups, " workgroups; at most 2^31 - 1");
  if (probes > 0) {
    ST_CHECK(counts != nullptr, "workspace is null");
    const int64_t items = batch * probes, per = kKmCountThreads / 64;
    hipLaunchKernelGGL(kmean_count_kernel, dim3(static_cast<unsigned>((items + per - 1) / per)),
                       dim3(kKmCountThreads), 0, s, a, counts, items);
  }
  const int64_t pairs = batch * probes;
  // 128-byte slices when their tile leaves room for the query, else 64-byte
  const int waves = kKmScoreThreads / 64;
  const bool i8 = emb_dtype == kKmI8;
  const int slice = waves * km_score_wave_lds(static_cast<int>(dim), i8, 128) <= kKmWaveMaxLds ? 128 : 64;
  const int score_lds = waves * km_score_wave_lds(static_cast<int>(dim), i8, slice);
  if (probes > 0 && pairs >= kKmBalancedPairs && batch <= kKmBalancedMaxRows &&
      score_lds <= kKmWaveMaxLds &&
      (counts_capacity < 0 || pairs + km_balanced_extra(batch) <= counts_capacity)) {
    int64_t* rowtot = counts + pairs;
    int64_t* gstart = rowtot + batch;
    hipLaunchKernelGGL(kmean_groups_kernel, dim3(1), dim3(kKmGroupsThreads), 0, s, counts, batch,
                       probes, max_per_row, rowtot, gstart);
    const dim3 lgrid(static_cast<unsigned>((pairs + 3) / 4)), wblock(kKmWaveThreads);
    switch (st) {
      case kKmF32: hipLaunchKernelGGL(kmean_list_kernel<kKmF32>, lgrid, wblock, 0, s, a, counts, rowtot, pairs); break;
      case kKmF16: hipLaunchKernelGGL(kmean_list_kernel<kKmF16>, lgrid, wblock, 0, s, a, counts, rowtot, pairs); break;
      case kKmBF16: hipLaunchKernelGGL(kmean_list_kernel<kKmBF16>, lgrid, wblock, 0, s, a, counts, rowtot, pairs); break;
      default: hipLaunchKernelGGL(kmean_list_kernel<kKmI32>, lgrid, wblock, 0, s, a, counts, rowtot, pairs);
    }
    // a fixed grid: as many workgroups per CU as its LDS holds, at most
    // kKmScorePerCu, every one resident
    const int per_cu = std::max(1, std::min(kKmScorePerCu, kCuLdsBytes / score_lds));
    const dim3 sgrid(static_cast<unsigned>(per_cu * cu_count())), sblock(kKmScoreThreads);
    auto score = [&](auto sl) {
      constexpr int SL = decltype(sl)::value;
      switch (emb_dtype) {
        case kKmF32: hipLaunchKernelGGL((kmean_score_kernel<kKmF32, kKmF32, SL>), sgrid, sblock, score_lds, s, a, gstart, rowtot, batch); break;
        case kKmF16: hipLaunchKernelGGL((kmean_score_kernel<kKmF16, kKmF16, SL>), sgrid, sblock, score_lds, s, a, gstart, rowtot, batch); break;
        case kKmBF16: hipLaunchKernelGGL((kmean_score_kernel<kKmBF16, kKmBF16, SL>), sgrid, sblock, score_lds, s, a, gstart, rowtot, batch); break;
        default:
          if (st == kKmI32)
            hipLaunchKernelGGL((kmean_score_kernel<kKmI8, kKmI32, SL>), sgrid, sblock, score_lds, s, a, gstart, rowtot, batch);
          else
            hipLaunchKernelGGL((kmean_score_kernel<kKmI8, kKmF16, SL>), sgrid, sblock, score_lds, s, a, gstart, rowtot, batch);
      }
    };
    if (slice == 128)
      score(std::integral_constant<int, 128>{});
    else
      score(std::integral_constant<int, 64>{});
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
      throw Error(ST_ERR_HIP, cat("fused_kmean_ann launch failed: ", hipGetErrorString(e)));
    return;
  }
  const dim3 grid(static_cast<unsigned>(groups)), block(kKmThreads);
  switch (emb_dtype) {
    case kKmF32: hipLaunchKernelGGL((kmean_ann_kernel<kKmF32, kKmF32>), grid, block, 0, s, a, counts); break;
    case kKmF16: hipLaunchKernelGGL((kmean_ann_kernel<kKmF16, kKmF16>), grid, block, 0, s, a, counts); break;
    case kKmBF16: hipLaunchKernelGGL((kmean_ann_kernel<kKmBF16, kKmBF16>), grid, block, 0, s, a, counts); break;
    default:
      if (st == kKmI32)
        hipLaunchKernelGGL((kmean_ann_kernel<kKmI8, kKmI32>), grid, block, 0, s, a, counts);
      else
        hipLaunchKernelGGL((kmean_ann_kernel<kKmI8, kKmF16>), grid, block, 0, s, a, counts);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    throw Error(ST_ERR_HIP, cat("fused_kmean_ann launch failed: ", hipGetErrorString(e)));
}

}  // namespace
}  // namespace st

extern "C" int st_fused_kmean_ann(const int64_t* cluster_offsets, int64_t num_offsets,
                                  const int64_t* cluster_ids, const int64_t* cluster_length,
                                  int64_t batch, int64_t probes, const void* embeddings,
                                  int64_t total_docs, int64_t dim, int emb_dtype,
                                  const void* queries, int64_t max_per_row,
                                  const int64_t* filter_mask, int64_t filter_rows,
                                  int64_t filter_cols, const int64_t* filter_index,
                                  const uint16_t* per_embedding_scale, int64_t divisor_for_int8,
                                  int64_t invalid_index_value, void* workspace, void* scores,
                                  int32_t* indices, void* stream) {
  using namespace st;
  return guarded([&] {
    kmean_run(cluster_offsets, num_offsets, cluster_ids, cluster_length, batch, probes, embeddings,
              total_docs, dim, emb_dtype, queries, max_per_row, filter_mask, filter_rows, filter_cols,
              filter_index, per_embedding_scale, divisor_for_int8, invalid_index_value,
              static_cast<int64_t*>(workspace), -1, scores, indices, stream);
  });
}

// ---------------------------------------------------------------------------
// No-allocation variant: the per-(row, probe) counts live in a file-scope
// device array (one copy per GPU, held until the process ends) instead of a
// caller-provided workspace.  Its address is taken once per device with
// hipGetSymbolAddress, on that device's first call; host code uses only that
// address, never the array's name.  Every (row, probe) count is written by
// kmean_count_kernel before it is read, and in the balanced form every row
// total and group start by kmean_groups_kernel (after the counts, when they
// fit the array; otherwise the call takes the workgroup form), so nothing
// needs clearing between calls.  Calls on one GPU share the array, so they
// must not overlap: calls on one stream are ordered by the stream, and a call
// on another stream than the device's previous call waits for that call (an
// event, created with the scratch address on the device's first call and
// recorded after every call; the host side of the calls is serialised by a
// mutex so that no call slips between another's wait and its record).

namespace st {
namespace {

constexpr int64_t kKmScratchItems = ST_KMEAN_NOALLOC_MAX_PAIRS;
static_assert(kKmScratchItems == (int64_t{1} << 20), "the header's limit and the array size differ");
static __device__ __align__(256) int64_t scratch[kKmScratchItems];

constexpr int kKmMaxDevices = 64;
std::mutex g_scratch_mu;  // held for a whole call (see above)

// Per device: the address of its copy of `scratch`, the event recorded after
// its last call and that call's stream.
struct ScratchDevice {
  void* ptr = nullptr;
  hipEvent_t done = nullptr;
  bool used = false;
  hipStream_t last = nullptr;
};
ScratchDevice g_scratch[kKmMaxDevices];

// The calling thread's current device's scratch state, set up on the
// device's first call (g_scratch_mu held).
ScratchDevice& device_scratch() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) throw Error(ST_ERR_HIP, cat("hipGetDevice failed: ", hipGetErrorString(e)));
  ST_CHECK(dev >= 0 && dev < kKmMaxDevices, "device ordinal ", dev, " out of range");
  ScratchDevice& d = g_scratch[dev];
  if (d.ptr == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      throw Error(ST_ERR_HIP, cat("hipGetSymbolAddress(scratch) failed on device ", dev, ": ",
                                  hipGetErrorString(e)));
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess)
      throw Error(ST_ERR_HIP, cat("hipEventCreateWithFlags failed on device ", dev, ": ",
                                  hipGetErrorString(e)));
    d.done = ev;
    d.ptr = ptr;
  }
  return d;
}

}  // namespace
}  // namespace st

extern "C" int st_fused_kmean_ann_noalloc(
    const int64_t* cluster_offsets, int64_t num_offsets, const int64_t* cluster_ids,
    const int64_t* cluster_length, int64_t batch, int64_t probes, const void* embeddings,
    int64_t total_docs, int64_t dim, int emb_dtype, const void* queries, int64_t max_per_row,
    const int64_t* filter_mask, int64_t filter_rows, int64_t filter_cols,
    const int64_t* filter_index, const uint16_t* per_embedding_scale, int64_t divisor_for_int8,
    int64_t invalid_index_value, void* scores, int32_t* indices, void* stream) {
  using namespace st;
  return guarded([&] {
    ST_CHECK(batch < 0 || probes <= 0 || batch <= kKmScratchItems / probes, "batch x probes = ", batch,
             " x ", probes, " exceeds the ", kKmScratchItems,
             " (row, probe) pairs of the no-allocation entry point's scratch");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    int64_t* counts = nullptr;
    ScratchDevice* d = nullptr;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (batch > 0 && probes > 0 && max_per_row > 0) {
      d = &device_scratch();
      counts = static_cast<int64_t*>(d->ptr);
      if (d->used && d->last != s) {  // the previous call, on another stream, first
        const hipError_t e = hipStreamWaitEvent(s, d->done, 0);
        if (e != hipSuccess)
          throw Error(ST_ERR_HIP, cat("hipStreamWaitEvent failed: ", hipGetErrorString(e)));
      }
    }
    kmean_run(cluster_offsets, num_offsets, cluster_ids, cluster_length, batch, probes, embeddings,
              total_docs, dim, emb_dtype, queries, max_per_row, filter_mask, filter_rows, filter_cols,
              filter_index, per_embedding_scale, divisor_for_int8, invalid_index_value, counts,
              kKmScratchItems, scores, indices, stream);
    if (d != nullptr) {
      const hipError_t e = hipEventRecord(d->done, s);
      if (e != hipSuccess) throw Error(ST_ERR_HIP, cat("hipEventRecord failed: ", hipGetErrorString(e)));
      d->used = true;
      d->last = s;
    }
  });
}
