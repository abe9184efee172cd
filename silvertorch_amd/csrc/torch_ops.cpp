// torch.ops.st.* registration for the MI355X build.
//
// Registers the same schemas as the reference (bloom_indexer.cpp:115-125,
// bloom_index_search.cpp:542-585, expression_query_parser.cpp:456-465) and
// binds both dispatch keys to the HIP implementation behind the C ABI in
// include/silvertorch_hip.h:
//   CUDA key (HIP tensors under ROCm torch): runs on the tensors' device.
//   CPU key: the inputs are copied to the current GPU, the same HIP kernels
//            run, and the results are copied back; without a visible GPU the
//            call raises.  No CPU implementation of the path exists here.
// The parser is host code on both keys, as in the reference
// (expression_query_parser_cuda.cu:27-44).
#include <ATen/ATen.h>
#include <ATen/core/CachingHostAllocator.h>
#include <c10/hip/HIPFunctions.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <Python.h>
#include <torch/library.h>

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/silvertorch_hip.h"

namespace {

using at::Tensor;

void check_st(int rc, const char* what) {
  TORCH_CHECK(rc == ST_OK, what, ": ", st_last_error());
}

void* current_stream(const Tensor& t) {
  return static_cast<void*>(
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream());
}

at::Device gpu_for_cpu_call() {
  TORCH_CHECK(c10::hip::device_count() > 0,
              "silvertorch_amd computes the bloom path with HIP kernels on an "
              "MI355X; no GPU is visible to this process");
  return at::Device(at::kCUDA, c10::hip::current_device());
}

// ---------------------------------------------------------------- build

// Argument checks shared by both dispatch keys (the reference's CPU op checks
// dtypes and b_multiplier first, bloom_indexer.cpp:33-36; the shape check is
// the CUDA op's, bloom_indexer_cuda.cu:114-119).
void check_build_args(const Tensor& feature_ids, const Tensor& feature_offsets,
                      const Tensor& feature_values, double b_multiplier,
                      int64_t k) {
  TORCH_CHECK(feature_ids.scalar_type() == at::kInt, "feature_ids must be int32");
  TORCH_CHECK(feature_offsets.scalar_type() == at::kLong,
              "feature_offsets must be int64");
  TORCH_CHECK(feature_values.scalar_type() == at::kLong,
              "feature_values must be int64");
  TORCH_CHECK(b_multiplier > 1.0, "b_multiplier must be greater than 1.0");
  const int64_t F = feature_ids.numel();
  TORCH_CHECK(F > 0, "feature_ids must not be empty");
  TORCH_CHECK(feature_offsets.numel() >= 1,
              "feature_offsets must hold at least one entry");
  TORCH_CHECK((feature_offsets.numel() - 1) % F == 0, "Feature offsets size ",
              feature_offsets.numel(),
              " must be a multiple of the feature ids size ", F, " plus one");
  TORCH_CHECK(k >= 0 && k <= ST_MAX_BUILD_K, "k must be in [0, ",
              ST_MAX_BUILD_K, "], got ", k);
}

std::tuple<Tensor, Tensor> build_gpu(const Tensor& feature_ids_in,
                                     const Tensor& feature_offsets_in,
                                     const Tensor& feature_values_in,
                                     double b_multiplier, int64_t k,
                                     bool /*fast_build*/) {
  check_build_args(feature_ids_in, feature_offsets_in, feature_values_in,
                   b_multiplier, k);
  TORCH_CHECK(feature_ids_in.is_cuda() && feature_offsets_in.is_cuda() &&
                  feature_values_in.is_cuda(),
              "bloom_index_build inputs must all be GPU tensors");
  const auto dev = feature_ids_in.device();
  TORCH_CHECK(feature_offsets_in.device() == dev &&
                  feature_values_in.device() == dev,
              "bloom_index_build inputs must be on one device");
  const int64_t F = feature_ids_in.numel();

  c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(dev);
  const Tensor ids = feature_ids_in.contiguous();
  const Tensor offsets = feature_offsets_in.contiguous();
  const Tensor values = feature_values_in.contiguous();
  const int64_t N = (offsets.numel() - 1) / F;
  const int64_t nb = (N + ST_DOCS_PER_BUNDLE - 1) / ST_DOCS_PER_BUNDLE;
  void* stream = current_stream(ids);

  auto lopts = at::TensorOptions().dtype(at::kLong).device(dev);
  Tensor bundle_b_offsets = at::empty({nb + 1}, lopts);
  Tensor stats = at::empty({6}, lopts);
  check_st(st_bloom_build_bundle_offsets(offsets.data_ptr<int64_t>(), N, F, k,
                                         b_multiplier,
                                         bundle_b_offsets.data_ptr<int64_t>(),
                                         stats.data_ptr<int64_t>(), stream),
           "bloom_index_build");
  const Tensor st = stats.cpu();  // the index size is data dependent
  const int64_t* s = st.data_ptr<int64_t>();
  TORCH_CHECK(s[2] == 0, "feature_offsets must be non-decreasing");
  TORCH_CHECK(s[3] >= 0 && s[4] <= values.numel(), "feature_offsets range [",
              s[3], ", ", s[4], ") lies outside feature_values (",
              values.numel(), " values)");
  TORCH_CHECK(s[1] <= INT32_MAX, "bundle width ", s[1],
              " exceeds the int32 position range");
  Tensor bloom_index = at::empty({s[0] * ST_COLUMNS_PER_BUNDLE}, lopts);
  check_st(st_bloom_index_build(ids.data_ptr<int32_t>(),
                                offsets.data_ptr<int64_t>(),
                                values.numel() ? values.data_ptr<int64_t>() : nullptr,
                                F, N, values.numel(), k,
                                bundle_b_offsets.data_ptr<int64_t>(), s[1],
                                bloom_index.data_ptr<int64_t>(),
                                bloom_index.numel(), stream),
           "bloom_index_build");
  return {bloom_index, bundle_b_offsets};
}

std::tuple<Tensor, Tensor> build_cpu_tensors(const Tensor& feature_ids,
                                             const Tensor& feature_offsets,
                                             const Tensor& feature_values,
                                             double b_multiplier, int64_t k,
                                             bool fast_build) {
  check_build_args(feature_ids, feature_offsets, feature_values, b_multiplier, k);
  const at::Device gpu = gpu_for_cpu_call();
  auto [index, offsets] =
      build_gpu(feature_ids.to(gpu), feature_offsets.to(gpu),
                feature_values.to(gpu), b_multiplier, k, fast_build);
  return {index.cpu(), offsets.cpu()};
}

// ---------------------------------------------------------------- search

struct PlanHolder {
  st_search_plan* p = nullptr;
  ~PlanHolder() { st_search_plan_destroy(p); }
};

// Pinned ring the search ops upload their plans from: kRingSlots slots of
// kRingSlotBytes per device, allocated on first use and kept for the
// process.  The search call's first kernel copies the plan out of its slot,
// and each of its upload workgroups then stores the slot's use number to one
// of the slot's signal words (st_search_plan_upload_signal): a slot is free
// again once its words hold its last use number, with no event on the stream
// (an event record costs the stream a few microseconds per call).  A plan
// larger than a slot, or a call that finds every slot still in use, takes a
// block of torch's pinned host allocator and its event instead.  An op that
// fails before its search call frees its slot itself (PreparedSearch); a slot
// whose search call failed before its copy ran stays in use.
constexpr int kRingSlots = 16;
constexpr int64_t kRingSlotBytes = 256 << 10;
constexpr int64_t kRingGroupBytes = 64 << 10;  // blob bytes per upload workgroup
constexpr int kRingGroups = static_cast<int>(kRingSlotBytes / kRingGroupBytes);

struct PlanRing {
  std::mutex mu;
  bool ready = false, failed = false;
  uint8_t* data = nullptr;   // kRingSlots * kRingSlotBytes
  uint64_t* words = nullptr; // kRingSlots * kRingGroups signal words
  uint64_t last[kRingSlots] = {};  // use number of each slot's last upload
  int groups[kRingSlots] = {};     // its upload workgroups
  uint64_t uses = 0;
};

PlanRing& plan_ring(int device) {
  static std::mutex mu;
  static std::vector<std::unique_ptr<PlanRing>> rings;
  std::lock_guard<std::mutex> lk(mu);
  if (static_cast<int>(rings.size()) <= device) rings.resize(device + 1);
  if (!rings[device]) rings[device] = std::make_unique<PlanRing>();
  return *rings[device];
}

// A free slot (its data pointer, signal words and new use number), or -1.
int ring_acquire(PlanRing& r, int groups, uint8_t** data, uint64_t** words, uint64_t* use) {
  std::lock_guard<std::mutex> lk(r.mu);
  if (!r.ready && !r.failed) {
    void* d = nullptr;
    void* w = nullptr;
    // fine-grained (coherent) host memory: the device reads each slot's new
    // bytes over PCIe, not a cached copy of the slot's previous plan, and the
    // host sees the signal words as the device stores them
    if (hipHostMalloc(&d, kRingSlots * kRingSlotBytes, hipHostMallocCoherent) == hipSuccess &&
        hipHostMalloc(&w, kRingSlots * kRingGroups * sizeof(uint64_t), hipHostMallocCoherent) ==
            hipSuccess) {
      std::memset(w, 0, kRingSlots * kRingGroups * sizeof(uint64_t));
      // every page written once now: a page's first write faults it in on
      // the host (~4 us per 4 KB page), which would otherwise land on the
      // first call that uses each slot
      std::memset(d, 0, kRingSlots * kRingSlotBytes);
      r.data = static_cast<uint8_t*>(d);
      r.words = static_cast<uint64_t*>(w);
      r.ready = true;
    } else {
      if (d != nullptr) (void)hipHostFree(d);
      (void)hipGetLastError();  // the fallback path serves every call
      r.failed = true;
    }
  }
  if (!r.ready) return -1;
  // the lowest free slot: calls reuse the few slots the calls in flight
  // leave free, whose lines stay in the host's caches
  for (int i = 0; i < kRingSlots; ++i) {
    bool free = true;
    for (int g = 0; g < r.groups[i]; ++g)
      free &= __atomic_load_n(r.words + i * kRingGroups + g, __ATOMIC_ACQUIRE) >= r.last[i];
    if (!free) continue;
    r.last[i] = ++r.uses;
    r.groups[i] = groups;
    *data = r.data + i * kRingSlotBytes;
    *words = r.words + i * kRingGroups;
    *use = r.last[i];
    return i;
  }
  return -1;
}

}  // namespace

// Test hook (not an operator): how many slots of `device`'s pinned plan ring
// are free, or -1 when the ring has not been allocated.
extern "C" int st_torch_plan_ring_free_slots(int device) {
  PlanRing& r = plan_ring(device);
  std::lock_guard<std::mutex> lk(r.mu);
  if (!r.ready) return -1;
  int n = 0;
  for (int i = 0; i < kRingSlots; ++i) {
    bool free = true;
    for (int g = 0; g < r.groups[i]; ++g)
      free &= __atomic_load_n(r.words + i * kRingGroups + g, __ATOMIC_ACQUIRE) >= r.last[i];
    n += free ? 1 : 0;
  }
  return n;
}

namespace {

// Checks, plan compilation, width binding and plan upload shared by the
// search ops.
struct PreparedSearch {
  Tensor index, bbo, blob;  // blob: device copy of the plan
  at::DataPtr host_blob;    // pinned copy the search call uploads from
  PlanHolder plan;
  int64_t Q = 0, nb = 0;
  // The pinned ring slot the plan was copied into: the search call's upload
  // workgroups free it; when the op fails before the search call is made
  // (an allocation, a check), nothing will, and it is freed here.
  uint64_t* ring_words = nullptr;
  int ring_groups = 0;
  uint64_t ring_use = 0;
  bool handed_to_search = false;
  // Runs after the op's launches: the pinned block goes back to torch's host
  // allocator, which reuses it only once the stream has passed them.
  ~PreparedSearch() {
    if (ring_words != nullptr && !handed_to_search)
      for (int g = 0; g < ring_groups; ++g)
        __atomic_store_n(ring_words + g, ring_use, __ATOMIC_RELEASE);
    if (!host_blob) return;
    const auto stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(index.device().index());
    at::getHostAllocator(at::kCUDA)->record_event(host_blob.get(), host_blob.get_context(),
                                                  stream.unwrap());
  }
};

void prepare_search(PreparedSearch& ps, const Tensor& bloom_index_in,
                    const Tensor& bundle_b_offsets_in, const Tensor& plans_data,
                    const Tensor& plans_offsets, int64_t k, int64_t hash_k) {
  TORCH_CHECK(bloom_index_in.is_cuda(), "bloom_index must be a GPU tensor");
  TORCH_CHECK(bloom_index_in.dim() == 1, "bloom_index must be 1-D");
  TORCH_CHECK(bloom_index_in.scalar_type() == at::kLong, "bloom_index must be int64");
  TORCH_CHECK(bundle_b_offsets_in.scalar_type() == at::kLong,
              "bloom_bundle_b_offsets must be int64");
  TORCH_CHECK(bundle_b_offsets_in.device() == bloom_index_in.device(),
              "bloom_bundle_b_offsets must be on the device of bloom_index");
  TORCH_CHECK(bundle_b_offsets_in.numel() >= 1,
              "bloom_bundle_b_offsets must hold at least one entry");
  TORCH_CHECK(plans_data.scalar_type() == at::kChar ||
                  plans_data.scalar_type() == at::kByte,
              "bloom_query_plans_data must be int8");
  TORCH_CHECK(plans_offsets.scalar_type() == at::kLong,
              "bloom_query_plans_offsets must be int64");
  ps.index = bloom_index_in.contiguous();
  ps.bbo = bundle_b_offsets_in.contiguous();
  // Plans are compiled on the host, as the reference decodes them there
  // (bloom_index_search_cuda.cu:1043-1098).
  const Tensor pd = plans_data.to(at::kCPU).contiguous();
  const Tensor po = plans_offsets.to(at::kCPU).contiguous();
  check_st(st_search_plan_create(
               reinterpret_cast<const int8_t*>(pd.data_ptr()), pd.numel(),
               po.data_ptr<int64_t>(), po.numel(), k, hash_k, &ps.plan.p),
           "bloom_index_search_batch");
  ps.Q = st_search_plan_num_queries(ps.plan.p);
  ps.nb = ps.bbo.numel() - 1;
  if (ps.Q == 0 || ps.nb == 0) return;
  // The search call binds the programs to the bundle widths on the device
  // (no copy of the bundle offsets to the host, no synchronisation).
  check_st(st_search_plan_prepare_device_binding(ps.plan.p, ps.nb), "bloom_index_search_batch");
  // The plan bytes go to pinned memory of torch's host allocator, and the
  // search call's first kernel copies them to the device on the caller's
  // stream (no copy-engine hand-off between the previous call's kernels and
  // this call's); the allocator reuses the pinned block only after that
  // stream has passed the call.
  const int64_t blob_bytes = st_search_plan_blob_bytes(ps.plan.p);
  if (blob_bytes <= kRingSlotBytes) {
    const int groups = static_cast<int>((blob_bytes + kRingGroupBytes - 1) / kRingGroupBytes);
    uint8_t* slot = nullptr;
    uint64_t* words = nullptr;
    uint64_t use = 0;
    if (ring_acquire(plan_ring(ps.index.device().index()), groups, &slot, &words, &use) >= 0) {
      ps.ring_words = words;
      ps.ring_groups = groups;
      ps.ring_use = use;
      std::memcpy(slot, st_search_plan_blob(ps.plan.p), blob_bytes);
      check_st(st_search_plan_upload_source(ps.plan.p, slot), "bloom_index_search_batch");
      TORCH_CHECK(st_search_plan_upload_groups(ps.plan.p) == groups,
                  "bloom_index_search_batch: plan upload group count mismatch");
      check_st(st_search_plan_upload_signal(ps.plan.p, words, use), "bloom_index_search_batch");
      ps.blob = at::empty({st_search_plan_device_bytes(ps.plan.p)},
                          at::TensorOptions().dtype(at::kByte).device(ps.index.device()));
      return;
    }
  }
  at::HostAllocator* host_alloc = at::getHostAllocator(at::kCUDA);
  at::DataPtr host = host_alloc->allocate(static_cast<size_t>(blob_bytes));
  std::memcpy(host.get(), st_search_plan_blob(ps.plan.p), blob_bytes);
  check_st(st_search_plan_upload_source(ps.plan.p, host.get()), "bloom_index_search_batch");
  ps.blob = at::empty({st_search_plan_device_bytes(ps.plan.p)},
                      at::TensorOptions().dtype(at::kByte).device(ps.index.device()));
  ps.host_blob = std::move(host);
}

Tensor search_gpu(const Tensor& bloom_index_in, const Tensor& bundle_b_offsets_in,
                  const Tensor& plans_data, const Tensor& plans_offsets,
                  int64_t k, int64_t hash_k, bool return_bool_mask) {
  TORCH_CHECK(bloom_index_in.is_cuda(), "bloom_index must be a GPU tensor");
  c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(bloom_index_in.device());
  PreparedSearch ps;
  prepare_search(ps, bloom_index_in, bundle_b_offsets_in, plans_data, plans_offsets, k,
                 hash_k);
  const auto dev = ps.index.device();
  const int64_t C = ps.nb * ST_COLUMNS_PER_BUNDLE;
  Tensor out = return_bool_mask
                   ? at::empty({ps.Q, C * ST_BITS_PER_COLUMN},
                               at::TensorOptions().dtype(at::kBool).device(dev))
                   : at::empty({ps.Q, C}, at::TensorOptions().dtype(at::kLong).device(dev));
  if (ps.Q == 0 || ps.nb == 0) return out;
  ps.handed_to_search = true;
  check_st(st_bloom_index_search_batch(ps.index.data_ptr<int64_t>(), ps.index.numel(),
                                       ps.bbo.data_ptr<int64_t>(), ps.nb, ps.plan.p,
                                       ps.blob.data_ptr(), return_bool_mask ? 1 : 0,
                                       out.data_ptr(), current_stream(ps.index)),
           "bloom_index_search_batch");
  return out;
}

Tensor search_cpu_tensors(const Tensor& bloom_index, const Tensor& bundle_b_offsets,
                          const Tensor& plans_data, const Tensor& plans_offsets,
                          int64_t k, int64_t hash_k, bool return_bool_mask) {
  TORCH_CHECK(bloom_index.dim() == 1, "bloom_index must be 1-D");
  {  // plan errors surface before any device work, as on the reference CPU op
    const Tensor pd = plans_data.contiguous(), po = plans_offsets.contiguous();
    TORCH_CHECK(po.scalar_type() == at::kLong, "bloom_query_plans_offsets must be int64");
    PlanHolder probe;
    check_st(st_search_plan_create(reinterpret_cast<const int8_t*>(pd.data_ptr()),
                                   pd.numel(), po.data_ptr<int64_t>(), po.numel(),
                                   k, hash_k, &probe.p),
             "bloom_index_search_batch");
  }
  const at::Device gpu = gpu_for_cpu_call();
  return search_gpu(bloom_index.to(gpu), bundle_b_offsets.to(gpu), plans_data,
                    plans_offsets, k, hash_k, return_bool_mask)
      .cpu();
}

// ---------------------------------------------------------------- parser

std::tuple<int64_t, std::vector<Tensor>> parse_batch(
    const c10::List<std::string>& expressions, const Tensor& /*silvertorch_ks*/,
    int64_t bloom_hash_k, bool return_query_plan, int64_t max_sub_queries) {
  std::vector<std::string> owned;
  owned.reserve(expressions.size());
  for (size_t i = 0; i < expressions.size(); ++i) owned.push_back(expressions.get(i));
  std::vector<const char*> ptrs;
  for (const auto& s : owned) ptrs.push_back(s.c_str());
  st_parsed_plans* res = nullptr;
  const int rc = st_parse_expression_query_batch(
      ptrs.data(), static_cast<int64_t>(ptrs.size()), bloom_hash_k,
      return_query_plan ? 1 : 0, max_sub_queries, &res);
  check_st(rc, "parse_expression_query_batch");
  const int64_t nbytes = st_parsed_plans_data_bytes(res);
  const int64_t noff = st_parsed_plans_offsets_len(res);
  Tensor data = at::empty({nbytes}, at::kChar);
  Tensor offs = at::empty({noff}, at::kLong);
  if (nbytes) std::memcpy(data.data_ptr(), st_parsed_plans_data(res), nbytes);
  if (noff) std::memcpy(offs.data_ptr(), st_parsed_plans_offsets(res), noff * 8);
  const int64_t max_stack = st_parsed_plans_max_stack(res);
  st_parsed_plans_destroy(res);
  return {max_stack, {data, offs}};
}

// ------------------------------------------ generate_column_info_for_clusters

std::tuple<Tensor, Tensor, Tensor> column_info(const Tensor& offsets_in,
                                               const Tensor& lengths_in) {
  TORCH_CHECK(offsets_in.sizes() == lengths_in.sizes(),
              "selected_cluster_offsets and selected_cluster_lengths must have "
              "the same shape");
  TORCH_CHECK(offsets_in.dim() == 1 || offsets_in.dim() == 2,
              "selected_cluster_offsets must be 1D or 2D, got ", offsets_in.dim(), "D");
  TORCH_CHECK(offsets_in.scalar_type() == at::kLong &&
                  lengths_in.scalar_type() == at::kLong,
              "cluster offsets and lengths must be int64");
  TORCH_CHECK(offsets_in.device() == lengths_in.device(),
              "cluster offsets and lengths must be on one device");
  const auto dev = offsets_in.device();
  const int64_t n = lengths_in.numel();
  auto opts = at::TensorOptions().device(dev);
  Tensor counts = at::empty({n}, opts.dtype(at::kInt));
  Tensor starts = at::empty({n}, opts.dtype(at::kInt));
  Tensor firsts = at::empty({n}, opts.dtype(at::kChar));
  if (n == 0) return {counts, starts, firsts};
  if (dev.is_cuda()) {
    c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(dev);
    const Tensor o = offsets_in.contiguous(), l = lengths_in.contiguous();
    check_st(st_generate_column_info_for_clusters(
                 o.data_ptr<int64_t>(), l.data_ptr<int64_t>(), n,
                 counts.data_ptr<int32_t>(), starts.data_ptr<int32_t>(),
                 firsts.data_ptr<int8_t>(), current_stream(o)),
             "generate_column_info_for_clusters");
  } else {
    const at::Device gpu = gpu_for_cpu_call();
    auto [c, s, f] = column_info(offsets_in.to(gpu), lengths_in.to(gpu));
    return {c.cpu(), s.cpu(), f.cpu()};
  }
  return {counts, starts, firsts};
}

// ------------------------------------------ cluster-restricted search
// bloom_index_search_batch_return_partial_response(_multiple)
// (bloom_index_search.cpp:246-487): the argument checks are the reference's,
// with its messages; column ranges outside the index and plan indices
// outside the plans, which the reference reads past, raise.

struct PartialPlan {
  PlanHolder plan;
  Tensor blob;  // device copy of the (unbound) plan blob; undefined when
                // each chunk's block carries it (the single-chunk op)
};

void check_partial_args(const Tensor& bloom_index, const Tensor& offsets, const Tensor& lengths,
                        const c10::optional<Tensor>& query_plan_index, int64_t plan_count) {
  TORCH_CHECK(bloom_index.scalar_type() == at::kLong, "bloom_index dtype must be Long");
  TORCH_CHECK(offsets.dim() == 2, "selected_cluster_offsets dim must be 2, but got ", offsets.dim());
  TORCH_CHECK(lengths.dim() == 2, "selected_cluster_lengths dim must be 2, but got ", lengths.dim());
  TORCH_CHECK(offsets.scalar_type() == at::kLong, "selected_cluster_offsets dtype must be Long");
  TORCH_CHECK(lengths.scalar_type() == at::kLong, "selected_cluster_lengths dtype must be Long");
  const int64_t rows = offsets.size(0);
  TORCH_CHECK(rows == lengths.size(0) && offsets.size(1) == lengths.size(1),
              "selected_cluster_offsets must have same shape with selected_cluster_lengths, but got ",
              offsets.sizes(), " vs ", lengths.sizes());
  if (query_plan_index.has_value()) {
    TORCH_CHECK(query_plan_index->dim() == 1, "query_plan_index dim must be 1, but got ",
                query_plan_index->dim());
    TORCH_CHECK(query_plan_index->size(0) == rows,
                "query_plan count must be same with selected_cluster size[0], but got ",
                query_plan_index->size(0), " vs ", rows);
    TORCH_CHECK(query_plan_index->scalar_type() == at::kLong, "query_plan_index dtype must be Long");
  } else {
    TORCH_CHECK(plan_count == rows,
                "query_plan_count must be equal to query_count if no query_plan_index, but got ",
                plan_count, " vs ", rows);
  }
  TORCH_CHECK(bloom_index.dim() == 1, "bloom_index dim must be 1 for v2");
}

void prepare_partial_plan(PartialPlan& pp, const Tensor& plans_data, const Tensor& plans_offsets,
                          int64_t k, int64_t hash_k, at::Device dev, bool upload) {
  TORCH_CHECK(plans_data.scalar_type() == at::kChar || plans_data.scalar_type() == at::kByte,
              "bloom_query_plans_data must be int8");
  TORCH_CHECK(plans_offsets.scalar_type() == at::kLong, "bloom_query_plans_offsets must be int64");
  const Tensor pd = plans_data.to(at::kCPU).contiguous();
  const Tensor po = plans_offsets.to(at::kCPU).contiguous();
  check_st(st_search_plan_create(reinterpret_cast<const int8_t*>(pd.data_ptr()), pd.numel(),
                                 po.data_ptr<int64_t>(), po.numel(), k, hash_k, &pp.plan.p),
           "bloom_index_search_batch_return_partial_response");
  if (!upload) return;
  const int64_t n = st_search_plan_blob_bytes(pp.plan.p);
  Tensor host = at::empty({std::max<int64_t>(n, 1)}, at::TensorOptions().dtype(at::kByte).pinned_memory(true));
  if (n) std::memcpy(host.data_ptr(), st_search_plan_blob(pp.plan.p), n);
  pp.blob = host.to(dev, /*non_blocking=*/true);
}

// The cluster arrays of one chunk on the host (the response length sizes the
// output): device tensors are copied into pinned memory without waiting, so
// the copies overlap the host plan compile; the caller synchronises the
// current stream (`pending`) before the layout reads them.
struct PartialHost {
  Tensor co, cl, pi;
};

Tensor host_copy(const Tensor& x, bool& pending) {
  if (!x.is_cuda()) return x.contiguous();
  // only the current device's stream is synchronised before the layout
  if (x.device().index() != c10::hip::current_device()) return x.to(at::kCPU).contiguous();
  Tensor h = at::empty(x.sizes(), x.options().device(at::kCPU).pinned_memory(true));
  h.copy_(x, /*non_blocking=*/true);
  pending = true;
  return h;
}

PartialHost partial_host(const Tensor& offsets, const Tensor& lengths,
                         const c10::optional<Tensor>& query_plan_index, bool& pending) {
  PartialHost h;
  h.co = host_copy(offsets.contiguous(), pending);
  h.cl = host_copy(lengths.contiguous(), pending);
  if (query_plan_index.has_value()) h.pi = host_copy(query_plan_index->contiguous(), pending);
  return h;
}

// One index chunk: host-side layout from the chunk's cluster arrays (on the
// host already), then the kernel.
std::tuple<Tensor, Tensor, Tensor> partial_chunk(const PartialPlan& pp, const Tensor& index_in,
                                                 const Tensor& bbo_in, const PartialHost& host) {
  TORCH_CHECK(index_in.is_cuda(), "bloom_index must be a GPU tensor");
  TORCH_CHECK(bbo_in.scalar_type() == at::kLong, "bloom_bundle_b_offsets must be int64");
  TORCH_CHECK(bbo_in.device() == index_in.device(),
              "bloom_bundle_b_offsets must be on the device of bloom_index");
  TORCH_CHECK(bbo_in.numel() >= 1, "bloom_bundle_b_offsets must hold at least one entry");
  const auto dev = index_in.device();
  const Tensor index = index_in.contiguous(), bbo = bbo_in.contiguous();
  const Tensor& co = host.co;
  const Tensor& cl = host.cl;
  const Tensor& pi = host.pi;
  const int64_t rows = co.size(0), clusters = co.size(1), n = rows * clusters;
  // the work items, the column cumsum and the first bits (and the plan blob
  // when no device copy of it is shared) in one pinned block and one copy
  // to the device; the returned cumsum and first are views of the device
  // block (one copy and allocation per call instead of four)
  const int64_t blob_bytes = pp.blob.defined() ? 0 : (st_search_plan_blob_bytes(pp.plan.p) + 15) / 16 * 16;
  const int64_t off_items = blob_bytes;
  const int64_t items_bytes =
      (std::max<int64_t>(n, 1) * static_cast<int64_t>(sizeof(st_partial_item)) + 15) / 16 * 16;
  const int64_t off_cumsum = off_items + items_bytes, off_first = off_cumsum + (4 * n + 15) / 16 * 16;
  const int64_t block_bytes = off_first + std::max<int64_t>(n, 1);
  Tensor host_block = at::empty({block_bytes}, at::TensorOptions().dtype(at::kByte).pinned_memory(true));
  uint8_t* hb = host_block.data_ptr<uint8_t>();
  if (blob_bytes) std::memcpy(hb, st_search_plan_blob(pp.plan.p), st_search_plan_blob_bytes(pp.plan.p));
  int64_t num_items = 0, total = 0;
  check_st(st_search_plan_partial_items(pp.plan.p, co.data_ptr<int64_t>(), cl.data_ptr<int64_t>(), rows,
                                        clusters, pi.defined() ? pi.data_ptr<int64_t>() : nullptr,
                                        bbo.numel() - 1, reinterpret_cast<int32_t*>(hb + off_cumsum),
                                        reinterpret_cast<int8_t*>(hb + off_first),
                                        reinterpret_cast<st_partial_item*>(hb + off_items), &num_items,
                                        &total),
           "bloom_index_search_batch_return_partial_response");
  const Tensor block = host_block.to(dev, /*non_blocking=*/true);
  Tensor mask = at::empty({total}, at::TensorOptions().dtype(at::kLong).device(dev));
  if (num_items > 0) {
    check_st(st_bloom_index_search_partial(index.data_ptr<int64_t>(), index.numel(),
                                           bbo.data_ptr<int64_t>(), bbo.numel() - 1, pp.plan.p,
                                           pp.blob.defined() ? pp.blob.data_ptr() : block.data_ptr(),
                                           reinterpret_cast<const st_partial_item*>(
                                               block.data_ptr<uint8_t>() + off_items),
                                           num_items, mask.data_ptr<int64_t>(), current_stream(index)),
             "bloom_index_search_batch_return_partial_response");
  }
  return {block.narrow(0, off_cumsum, 4 * n).view(at::kInt), block.narrow(0, off_first, n).view(at::kChar),
          mask};
}

void sync_current_stream(at::Device dev) {
  c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(dev.index()).synchronize();
}

std::tuple<Tensor, Tensor, Tensor> partial_gpu(const Tensor& bloom_index, const Tensor& bbo,
                                               const Tensor& plans_data, const Tensor& plans_offsets,
                                               const Tensor& offsets, const Tensor& lengths, int64_t k,
                                               int64_t hash_k,
                                               const c10::optional<Tensor>& query_plan_index) {
  check_partial_args(bloom_index, offsets, lengths, query_plan_index, plans_offsets.numel() / 8);
  TORCH_CHECK(bloom_index.is_cuda(), "bloom_index must be a GPU tensor");
  c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(bloom_index.device());
  bool pending = false;
  const PartialHost host = partial_host(offsets, lengths, query_plan_index, pending);
  PartialPlan pp;
  prepare_partial_plan(pp, plans_data, plans_offsets, k, hash_k, bloom_index.device(),
                       /*upload=*/false);
  if (pending) sync_current_stream(bloom_index.device());
  return partial_chunk(pp, bloom_index, bbo, host);
}

std::tuple<Tensor, Tensor, Tensor> partial_cpu(const Tensor& bloom_index, const Tensor& bbo,
                                               const Tensor& plans_data, const Tensor& plans_offsets,
                                               const Tensor& offsets, const Tensor& lengths, int64_t k,
                                               int64_t hash_k,
                                               const c10::optional<Tensor>& query_plan_index) {
  check_partial_args(bloom_index, offsets, lengths, query_plan_index, plans_offsets.numel() / 8);
  const at::Device gpu = gpu_for_cpu_call();
  auto [c, f, m] = partial_gpu(bloom_index.to(gpu), bbo.to(gpu), plans_data, plans_offsets, offsets,
                               lengths, k, hash_k, query_plan_index);
  return {c.cpu(), f.cpu(), m.cpu()};
}

// _multiple: the single-chunk op per chunk with one compiled plan; `fuse`
// changes only the reference CUDA path's launch structure, not the outputs.
std::tuple<std::vector<Tensor>, std::vector<Tensor>, std::vector<Tensor>> partial_multiple(
    const std::vector<Tensor>& indices, const std::vector<Tensor>& bbos, const Tensor& plans_data,
    const Tensor& plans_offsets, const std::vector<Tensor>& offsets,
    const std::vector<Tensor>& lengths, int64_t k, int64_t hash_k,
    const c10::optional<Tensor>& query_plan_index, bool /*fuse*/) {
  const size_t n = indices.size();
  TORCH_CHECK(n > 0, "bloom_index_search_batch_return_partial_response_multiple: "
                     "list_bloom_index should not be empty.");
  TORCH_CHECK(bbos.size() == n,
              "list_bloom_index and list_bloom_bundle_b_offsets should have the same size, got ", n,
              " vs ", bbos.size());
  TORCH_CHECK(offsets.size() == n,
              "list_bloom_index and list_selected_cluster_offsets should have the same size, got ", n,
              " vs ", offsets.size());
  TORCH_CHECK(lengths.size() == n,
              "list_bloom_index and list_selected_cluster_lengths should have the same size, got ", n,
              " vs ", lengths.size());
  for (size_t i = 0; i < n; ++i)
    check_partial_args(indices[i], offsets[i], lengths[i], query_plan_index, plans_offsets.numel() / 8);
  const bool on_cpu = !indices[0].is_cuda();
  const at::Device dev = on_cpu ? gpu_for_cpu_call() : indices[0].device();
  c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(dev);
  bool pending = false;
  std::vector<PartialHost> hosts;
  for (size_t i = 0; i < n; ++i) hosts.push_back(partial_host(offsets[i], lengths[i], query_plan_index, pending));
  PartialPlan pp;
  prepare_partial_plan(pp, plans_data, plans_offsets, k, hash_k, dev, /*upload=*/true);
  if (pending) sync_current_stream(dev);
  std::vector<Tensor> cs, fs, ms;
  for (size_t i = 0; i < n; ++i) {
    auto [c, f, m] = partial_chunk(pp, indices[i].to(dev), bbos[i].to(dev), hosts[i]);
    if (on_cpu) {
      c = c.cpu();
      f = f.cpu();
      m = m.cpu();
    }
    cs.push_back(c);
    fs.push_back(f);
    ms.push_back(m);
  }
  return {cs, fs, ms};
}

// ------------------------------------------ compaction of matching ids
// No reference operator: the reference's users call
// mask[:, :num_docs].nonzero() on the search output (README.md:191-193).

std::tuple<Tensor, Tensor> mask_to_ids_gpu(const Tensor& packed_in, int64_t num_docs,
                                           bool int64_ids) {
  TORCH_CHECK(packed_in.is_cuda(), "packed_mask must be a GPU tensor");
  TORCH_CHECK(packed_in.dim() == 2 && packed_in.scalar_type() == at::kLong,
              "packed_mask must be the 2-D int64 packed search output");
  TORCH_CHECK(num_docs >= 0, "num_docs must be non-negative, got ", num_docs);
  const auto dev = packed_in.device();
  c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(dev);
  const Tensor packed = packed_in.contiguous();
  const int64_t Q = packed.size(0), C = packed.size(1);
  TORCH_CHECK(int64_ids || std::min(num_docs, C * ST_BITS_PER_COLUMN) <= INT32_MAX,
              "int32 ids cannot hold doc ids up to ", num_docs, "; pass int64_ids=True");
  auto opts = at::TensorOptions().device(dev);
  Tensor row_offsets = at::empty({Q + 1}, opts.dtype(at::kLong));
  Tensor ws = at::empty({std::max<int64_t>(st_bloom_compact_workspace_bytes(Q, C), 1)},
                        opts.dtype(at::kByte));
  void* stream = current_stream(packed);
  check_st(st_bloom_compact_offsets(packed.numel() ? packed.data_ptr<int64_t>() : nullptr,
                                    Q, C, num_docs, ws.data_ptr(),
                                    row_offsets.data_ptr<int64_t>(), stream),
           "bloom_mask_to_ids");
  const int64_t total = row_offsets[Q].item<int64_t>();  // the id count sizes the output
  Tensor ids = at::empty({total}, opts.dtype(int64_ids ? at::kLong : at::kInt));
  if (total > 0) {
    check_st(st_bloom_compact_ids(packed.data_ptr<int64_t>(), Q, C, num_docs, ws.data_ptr(),
                                  ids.data_ptr(), int64_ids ? 1 : 0, stream),
             "bloom_mask_to_ids");
  }
  return {ids, row_offsets};
}

std::tuple<Tensor, Tensor> mask_to_ids_cpu(const Tensor& packed, int64_t num_docs,
                                           bool int64_ids) {
  TORCH_CHECK(packed.dim() == 2 && packed.scalar_type() == at::kLong,
              "packed_mask must be the 2-D int64 packed search output");
  const at::Device gpu = gpu_for_cpu_call();
  auto [ids, ro] = mask_to_ids_gpu(packed.to(gpu), num_docs, int64_ids);
  return {ids.cpu(), ro.cpu()};
}

// Search and the count step of the compaction in one pass over the index,
// then the scan, one sync for the id total, and the id writes.
std::tuple<Tensor, Tensor> search_ids_gpu(const Tensor& bloom_index,
                                          const Tensor& bundle_b_offsets,
                                          const Tensor& plans_data,
                                          const Tensor& plans_offsets, int64_t k,
                                          int64_t hash_k, int64_t num_docs,
                                          bool int64_ids) {
  TORCH_CHECK(num_docs >= 0, "num_docs must be non-negative, got ", num_docs);
  TORCH_CHECK(bloom_index.is_cuda(), "bloom_index must be a GPU tensor");
  c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(bloom_index.device());
  {  // before the plan takes a pinned ring slot
    const int64_t C = std::max<int64_t>(bundle_b_offsets.numel() - 1, 0) * ST_COLUMNS_PER_BUNDLE;
    TORCH_CHECK(int64_ids || std::min(num_docs, C * ST_BITS_PER_COLUMN) <= INT32_MAX,
                "int32 ids cannot hold doc ids up to ", num_docs, "; pass int64_ids=True");
  }
  PreparedSearch ps;
  prepare_search(ps, bloom_index, bundle_b_offsets, plans_data, plans_offsets, k, hash_k);
  const auto dev = ps.index.device();
  const int64_t C = ps.nb * ST_COLUMNS_PER_BUNDLE;
  auto opts = at::TensorOptions().device(dev);
  Tensor row_offsets = at::empty({ps.Q + 1}, opts.dtype(at::kLong));
  Tensor packed = at::empty({ps.Q, C}, opts.dtype(at::kLong));
  Tensor ws = at::empty({std::max<int64_t>(st_bloom_compact_workspace_bytes(ps.Q, C), 1)},
                        opts.dtype(at::kByte));
  void* stream = current_stream(ps.index);
  ps.handed_to_search = true;
  check_st(st_bloom_index_search_batch_counts(
               ps.index.data_ptr<int64_t>(), ps.index.numel(), ps.bbo.data_ptr<int64_t>(),
               ps.nb, ps.plan.p, ps.blob.defined() ? ps.blob.data_ptr() : nullptr, num_docs,
               packed.numel() ? packed.data_ptr<int64_t>() : nullptr, ws.data_ptr(),
               row_offsets.data_ptr<int64_t>(), stream),
           "bloom_index_search_batch_ids");
  const int64_t total = row_offsets[ps.Q].item<int64_t>();
  Tensor ids = at::empty({total}, opts.dtype(int64_ids ? at::kLong : at::kInt));
  if (total > 0) {
    check_st(st_bloom_compact_ids(packed.data_ptr<int64_t>(), ps.Q, C, num_docs, ws.data_ptr(),
                                  ids.data_ptr(), int64_ids ? 1 : 0, stream),
             "bloom_index_search_batch_ids");
  }
  return {ids, row_offsets};
}

std::tuple<Tensor, Tensor> search_ids_cpu(const Tensor& bloom_index,
                                          const Tensor& bundle_b_offsets,
                                          const Tensor& plans_data,
                                          const Tensor& plans_offsets, int64_t k,
                                          int64_t hash_k, int64_t num_docs,
                                          bool int64_ids) {
  const Tensor packed = search_cpu_tensors(bloom_index, bundle_b_offsets, plans_data,
                                           plans_offsets, k, hash_k, false);
  return mask_to_ids_cpu(packed, num_docs, int64_ids);
}

// ------------------------------------------ fused filter + top-k
// No reference operator (relatives: fused_kmean_ann's bloom-filtered scoring,
// fused_kmean_ann_cuda.cu:1797-1926, and at::topk).

std::tuple<Tensor, Tensor> filtered_topk_gpu(const Tensor& packed_in, const Tensor& emb_in,
                                             const Tensor& qv_in, int64_t num_docs,
                                             int64_t topk) {
  TORCH_CHECK(packed_in.is_cuda() && emb_in.is_cuda() && qv_in.is_cuda(),
              "filtered_topk inputs must be GPU tensors");
  TORCH_CHECK(packed_in.device() == emb_in.device() && emb_in.device() == qv_in.device(),
              "filtered_topk inputs must be on one device");
  TORCH_CHECK(packed_in.dim() == 2 && packed_in.scalar_type() == at::kLong,
              "packed_mask must be the 2-D int64 packed search output");
  TORCH_CHECK(emb_in.dim() == 2 && emb_in.scalar_type() == at::kBFloat16,
              "doc_embeddings must be a 2-D bfloat16 tensor");
  TORCH_CHECK(qv_in.dim() == 2 && qv_in.scalar_type() == at::kBFloat16,
              "query_embeddings must be a 2-D bfloat16 tensor");
  TORCH_CHECK(qv_in.size(0) == packed_in.size(0), "query_embeddings has ", qv_in.size(0),
              " rows, the mask ", packed_in.size(0), " queries");
  TORCH_CHECK(qv_in.size(1) == emb_in.size(1), "embedding dimensions differ: ", emb_in.size(1),
              " vs ", qv_in.size(1));
  TORCH_CHECK(num_docs >= 0 && num_docs <= emb_in.size(0), "num_docs ", num_docs,
              " must be in [0, ", emb_in.size(0), "] (rows of doc_embeddings)");
  c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(packed_in.device());
  const Tensor packed = packed_in.contiguous(), emb = emb_in.contiguous(),
               qv = qv_in.contiguous();
  const int64_t Q = packed.size(0);
  auto opts = at::TensorOptions().device(packed.device());
  Tensor ids = at::empty({Q, topk}, opts.dtype(at::kLong));
  Tensor scores = at::empty({Q, topk}, opts.dtype(at::kFloat));
  if (Q == 0) return {ids, scores};
  Tensor ws = at::empty({st_filtered_topk_workspace_bytes(Q)}, opts.dtype(at::kByte));
  check_st(st_filtered_topk(packed.numel() ? packed.data_ptr<int64_t>() : nullptr, Q,
                            packed.size(1), num_docs, emb.numel() ? emb.data_ptr() : nullptr,
                            qv.data_ptr(), emb.size(1), topk, ws.data_ptr(),
                            ids.data_ptr<int64_t>(), scores.data_ptr<float>(),
                            current_stream(packed)),
           "filtered_topk");
  return {ids, scores};
}

std::tuple<Tensor, Tensor> filtered_topk_cpu(const Tensor& packed, const Tensor& emb,
                                             const Tensor& qv, int64_t num_docs, int64_t topk) {
  const at::Device gpu = gpu_for_cpu_call();
  auto [ids, scores] = filtered_topk_gpu(packed.to(gpu), emb.to(gpu), qv.to(gpu), num_docs, topk);
  return {ids.cpu(), scores.cpu()};
}

std::tuple<Tensor, Tensor> search_topk_gpu(const Tensor& bloom_index, const Tensor& bundle_b_offsets,
                                           const Tensor& plans_data, const Tensor& plans_offsets,
                                           int64_t k, int64_t hash_k, const Tensor& emb,
                                           const Tensor& qv, int64_t num_docs, int64_t topk) {
  const Tensor packed = search_gpu(bloom_index, bundle_b_offsets, plans_data, plans_offsets, k,
                                   hash_k, /*return_bool_mask=*/false);
  return filtered_topk_gpu(packed, emb, qv, num_docs, topk);
}

std::tuple<Tensor, Tensor> search_topk_cpu(const Tensor& bloom_index, const Tensor& bundle_b_offsets,
                                           const Tensor& plans_data, const Tensor& plans_offsets,
                                           int64_t k, int64_t hash_k, const Tensor& emb,
                                           const Tensor& qv, int64_t num_docs, int64_t topk) {
  const Tensor packed = search_cpu_tensors(bloom_index, bundle_b_offsets, plans_data,
                                           plans_offsets, k, hash_k, false);
  return filtered_topk_cpu(packed, emb, qv, num_docs, topk);
}

// ------------------------------------------ clustered ANN scoring (fused_kmean_ann)
// fused_kmean_ann.cpp:85-227 (argument checks :96-102, output dtypes and
// padding :30-41, :134-165, the row width rounded up to 32 :104-107).

int km_dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return 0;
    case at::kHalf: return 1;
    case at::kBFloat16: return 2;
    case at::kChar: return 3;
    default:
      TORCH_CHECK(false, "fused_kmean_ann: embeddings must be float32, float16, bfloat16 or int8, got ",
                  t);
  }
  return -1;
}

at::ScalarType km_score_type(int code) {
  switch (code) {
    case 0: return at::kFloat;
    case 1: return at::kHalf;
    case 2: return at::kBFloat16;
    default: return at::kInt;
  }
}

std::tuple<Tensor, Tensor> kmean_gpu(const Tensor& cluster_offsets_in, const Tensor& cluster_ids_in,
                                     const Tensor& cluster_length_in, const Tensor& embeddings_in,
                                     const Tensor& queries_in, int64_t max_tensor_size_per_row,
                                     const std::optional<Tensor>& filtering_bit_mask,
                                     int64_t invalid_index_value, int64_t divisor_for_int8,
                                     const std::optional<Tensor>& filtering_bit_index,
                                     const std::optional<Tensor>& per_embedding_scale) {
  TORCH_CHECK(cluster_offsets_in.dim() == 1);
  TORCH_CHECK(cluster_ids_in.dim() == 2);
  TORCH_CHECK(cluster_length_in.dim() == 2);
  TORCH_CHECK(embeddings_in.dim() == 2);
  TORCH_CHECK(queries_in.dim() == 2);
  TORCH_CHECK(cluster_ids_in.size(0) == cluster_length_in.size(0));
  TORCH_CHECK(cluster_ids_in.size(0) == queries_in.size(0));
  TORCH_CHECK(cluster_ids_in.sizes() == cluster_length_in.sizes(),
              "cluster_ids and cluster_length must have the same shape");
  TORCH_CHECK(queries_in.size(1) == embeddings_in.size(1), "queries have dimension ",
              queries_in.size(1), ", embeddings ", embeddings_in.size(1));
  TORCH_CHECK(queries_in.scalar_type() == embeddings_in.scalar_type(),
              "queries and embeddings must have the same dtype");
  TORCH_CHECK(max_tensor_size_per_row >= 0, "max_tensor_size_per_row must be non-negative");
  const at::Device dev = embeddings_in.device();
  TORCH_CHECK(dev.is_cuda(), "fused_kmean_ann inputs must be GPU tensors");
  for (const Tensor* t : {&cluster_offsets_in, &cluster_ids_in, &cluster_length_in, &queries_in})
    TORCH_CHECK(t->device() == dev, "fused_kmean_ann inputs must be on one device");
  c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(dev);
  const int code = km_dtype_code(embeddings_in.scalar_type());
  const Tensor offsets = cluster_offsets_in.to(at::kLong).contiguous();
  const Tensor ids = cluster_ids_in.to(at::kLong).contiguous();
  const Tensor lens = cluster_length_in.to(at::kLong).contiguous();
  const Tensor emb = embeddings_in.contiguous(), q = queries_in.contiguous();
  Tensor mask, findex, scale;
  if (filtering_bit_mask) {
    TORCH_CHECK(filtering_bit_mask->dim() == 2 && filtering_bit_mask->scalar_type() == at::kLong,
                "filtering_bit_mask must be a 2-D int64 tensor");
    TORCH_CHECK(filtering_bit_mask->device() == dev, "filtering_bit_mask must be on the embeddings' device");
    mask = filtering_bit_mask->contiguous();
  }
  if (filtering_bit_index) {
    TORCH_CHECK(filtering_bit_index->numel() == ids.size(0),
                "filtering_bit_index must hold one row per query");
    findex = filtering_bit_index->to(dev, at::kLong).contiguous();
  }
  const bool has_scale = per_embedding_scale.has_value() && code == 3;
  if (has_scale) {
    TORCH_CHECK(per_embedding_scale->numel() >= emb.size(0),
                "per_embedding_scale must hold one value per embedding row");
    scale = per_embedding_scale->to(dev, at::kHalf).contiguous();
  }
  // the reference rounds the row width up to a multiple of 32 (its warp)
  const int64_t width = (max_tensor_size_per_row + 31) / 32 * 32;
  const int64_t B = ids.size(0);
  auto opts = at::TensorOptions().device(dev);
  const int score_code = st_kmean_ann_score_dtype(code, divisor_for_int8, has_scale ? 1 : 0);
  Tensor scores = at::empty({B, width}, opts.dtype(km_score_type(score_code)));
  Tensor indices = at::empty({B, width}, opts.dtype(at::kInt));
  if (B == 0 || width == 0) return {scores, indices};
  // a filtering_bit_index entry outside the mask's rows passes no doc (checked
  // on the device: no host wait)
  if (mask.defined() && !findex.defined()) {
    TORCH_CHECK(mask.size(0) >= B, "filtering_bit_mask has ", mask.size(0), " rows for ", B,
                " queries");
  }
  Tensor ws = at::empty({std::max<int64_t>(st_fused_kmean_ann_workspace_bytes(B, ids.size(1)), 1)},
                        opts.dtype(at::kByte));
  check_st(st_fused_kmean_ann(offsets.numel() ? offsets.data_ptr<int64_t>() : nullptr,
                              offsets.numel(), ids.numel() ? ids.data_ptr<int64_t>() : nullptr,
                              lens.numel() ? lens.data_ptr<int64_t>() : nullptr, B, ids.size(1),
                              emb.numel() ? emb.data_ptr() : nullptr, emb.size(0), emb.size(1), code,
                              q.data_ptr(), width,
                              mask.defined() && mask.numel() ? mask.data_ptr<int64_t>() : nullptr,
                              mask.defined() ? mask.size(0) : 0, mask.defined() ? mask.size(1) : 0,
                              findex.defined() ? findex.data_ptr<int64_t>() : nullptr,
                              has_scale ? reinterpret_cast<const uint16_t*>(scale.data_ptr()) : nullptr,
                              divisor_for_int8, invalid_index_value, ws.data_ptr(),
                              scores.data_ptr(), indices.data_ptr<int32_t>(), current_stream(emb)),
           "fused_kmean_ann");
  return {scores, indices};
}

std::optional<Tensor> opt_to(const std::optional<Tensor>& t, const at::Device& d) {
  if (!t) return std::nullopt;
  return t->to(d);
}

std::tuple<Tensor, Tensor> kmean_cpu(const Tensor& cluster_offsets, const Tensor& cluster_ids,
                                     const Tensor& cluster_length, const Tensor& embeddings,
                                     const Tensor& queries, int64_t max_tensor_size_per_row,
                                     const std::optional<Tensor>& filtering_bit_mask,
                                     int64_t invalid_index_value, int64_t divisor_for_int8,
                                     const std::optional<Tensor>& filtering_bit_index,
                                     const std::optional<Tensor>& per_embedding_scale) {
  const at::Device gpu = gpu_for_cpu_call();
  auto [scores, indices] = kmean_gpu(
      cluster_offsets.to(gpu), cluster_ids.to(gpu), cluster_length.to(gpu), embeddings.to(gpu),
      queries.to(gpu), max_tensor_size_per_row, opt_to(filtering_bit_mask, gpu),
      invalid_index_value, divisor_for_int8, opt_to(filtering_bit_index, gpu),
      opt_to(per_embedding_scale, gpu));
  return {scores.cpu(), indices.cpu()};
}

// fused_kmean_ann_with_partial_masks: the reference's CPU op scores every doc
// of the selected clusters and ignores the partial masks and
// filtering_bit_index (fused_kmean_ann.cpp:229-260); so does this build.
std::tuple<Tensor, Tensor> kmean_partial(
    const Tensor& cluster_offsets, const Tensor& cluster_ids, const Tensor& cluster_length,
    const Tensor& embeddings, const Tensor& queries, int64_t max_tensor_size_per_row,
    const Tensor& /*partial_mask_column_counts_cumsum*/,
    const Tensor& /*partial_mask_first_item_offset_in_column*/,
    const Tensor& /*partial_mask_column_results*/, int64_t invalid_index_value,
    int64_t divisor_for_int8, const std::optional<Tensor>& /*filtering_bit_index*/,
    const std::optional<Tensor>& per_embedding_scale, const std::optional<Tensor>&,
    const std::optional<Tensor>&, const std::optional<Tensor>&, const std::optional<Tensor>&,
    int64_t, int64_t) {
  if (embeddings.is_cuda())
    return kmean_gpu(cluster_offsets, cluster_ids, cluster_length, embeddings, queries,
                     max_tensor_size_per_row, std::nullopt, invalid_index_value,
                     divisor_for_int8, std::nullopt, per_embedding_scale);
  return kmean_cpu(cluster_offsets, cluster_ids, cluster_length, embeddings, queries,
                   max_tensor_size_per_row, std::nullopt, invalid_index_value, divisor_for_int8,
                   std::nullopt, per_embedding_scale);
}

// ..._multiple: one call per chunk (fused_kmean_ann.cpp:262-311, which passes
// no per-embedding scale and ignores `fuse`).
std::tuple<std::vector<Tensor>, std::vector<Tensor>> kmean_partial_multiple(
    const Tensor& queries, const std::vector<Tensor>& list_cluster_offsets,
    const std::vector<Tensor>& list_selected_cluster_ids,
    const std::vector<Tensor>& list_selected_cluster_lengths,
    const std::vector<Tensor>& list_embeddings, const std::vector<int64_t>& list_max_tensor_size_per_row,
    const std::vector<Tensor>& list_counts, const std::vector<Tensor>& list_first,
    const std::vector<Tensor>& list_results, int64_t invalid_index_value, int64_t divisor_for_int8,
    const std::optional<Tensor>& filtering_bit_index,
    const std::optional<std::vector<Tensor>>& /*list_per_embedding_scale*/, bool /*fuse*/) {
  const size_t n = list_cluster_offsets.size();
  TORCH_CHECK(list_selected_cluster_ids.size() == n && list_selected_cluster_lengths.size() == n &&
                  list_embeddings.size() == n && list_max_tensor_size_per_row.size() == n &&
                  list_counts.size() == n && list_first.size() == n && list_results.size() == n,
              "fused_kmean_ann_with_partial_masks_multiple: the lists must have one entry per chunk");
  std::vector<Tensor> scores, indices;
  scores.reserve(n);
  indices.reserve(n);
  for (size_t i = 0; i < n; ++i) {
    auto [s, ix] = kmean_partial(list_cluster_offsets[i], list_selected_cluster_ids[i],
                                 list_selected_cluster_lengths[i], list_embeddings[i], queries,
                                 list_max_tensor_size_per_row[i], list_counts[i], list_first[i],
                                 list_results[i], invalid_index_value, divisor_for_int8,
                                 filtering_bit_index, std::nullopt, std::nullopt, std::nullopt,
                                 std::nullopt, std::nullopt, 0, 0);
    scores.push_back(std::move(s));
    indices.push_back(std::move(ix));
  }
  return {scores, indices};
}

// ------------------------------------------ main + fresh candidate merge

int fresh_score_type(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return ST_SCORE_F32;
    case at::kHalf: return ST_SCORE_F16;
    case at::kBFloat16: return ST_SCORE_BF16;
    case at::kDouble: return ST_SCORE_F64;
    case at::kLong: return ST_SCORE_I64;
    case at::kInt: return ST_SCORE_I32;
    case at::kShort: return ST_SCORE_I16;
    case at::kChar: return ST_SCORE_I8;
    case at::kByte: return ST_SCORE_U8;
    default: TORCH_CHECK(false, "\"topk\" not implemented for '", t, "'");
  }
  return -1;
}

// The data types the reference's gather dispatches on
// (AT_DISPATCH_ALL_TYPES_AND2(Half, BFloat16), fresh_index_post_processing.cpp:88-93).
bool fresh_data_type_ok(at::ScalarType t) {
  switch (t) {
    case at::kByte: case at::kChar: case at::kShort: case at::kInt: case at::kLong:
    case at::kFloat: case at::kDouble: case at::kHalf: case at::kBFloat16:
      return true;
    default:
      return false;
  }
}

// take_top_k_and_gather_from_main_and_fresh (fresh_index_post_processing.cpp:231-270):
// argument checks in the reference's order, then the top-k and one gather
// per key on the device.  kernel_version selects nothing (the reference's
// CPU op ignores it too).
std::tuple<Tensor, Tensor, Tensor, c10::Dict<std::string, Tensor>> fresh_merge_gpu(
    const Tensor& main_scores_in, const Tensor& fresh_scores_in, const Tensor& main_indices_in,
    const Tensor& fresh_indices_in, int64_t k, const std::vector<std::string>& keys,
    const std::vector<Tensor>& list_main_data, const std::vector<Tensor>& list_fresh_data,
    int64_t /*kernel_version*/) {
  TORCH_CHECK(main_scores_in.dim() == 2 && fresh_scores_in.dim() == 2,
              "main_scores and fresh_scores must be 2-D [rows, candidates]");
  TORCH_CHECK(main_scores_in.size(0) == fresh_scores_in.size(0),
              "main_scores and fresh_scores must have the same number of rows");
  const at::Device dev = main_scores_in.device();
  TORCH_CHECK(dev.is_cuda(), "take_top_k_and_gather_from_main_and_fresh inputs must be GPU tensors");
  for (const Tensor* t : {&fresh_scores_in, &main_indices_in, &fresh_indices_in})
    TORCH_CHECK(t->device() == dev, "take_top_k_and_gather_from_main_and_fresh inputs must be on one device");
  c10::hip::OptionalHIPGuardMasqueradingAsCUDA guard(dev);
  const int64_t R = main_scores_in.size(0);
  const int64_t Nf = fresh_scores_in.size(1), Nm = main_scores_in.size(1);
  // at::cat promotes the two score tensors to one type
  const at::ScalarType st_type = at::result_type(fresh_scores_in, main_scores_in);
  const int code = fresh_score_type(st_type);
  const Tensor fs = fresh_scores_in.to(st_type).contiguous();
  const Tensor ms = main_scores_in.to(st_type).contiguous();
  TORCH_CHECK(k >= 0, "selected index k out of range");
  const int64_t kc = std::min<int64_t>(k, Nf + Nm);
  auto opts = at::TensorOptions().device(dev);
  Tensor top_scores = at::empty({R, kc}, opts.dtype(st_type));
  Tensor top_index = at::empty({R, kc}, opts.dtype(at::kLong));
  Tensor from_fresh = at::empty({R, kc}, opts.dtype(at::kBool));
  void* stream = current_stream(fs);
  const int64_t ws_bytes = st_fresh_topk_workspace_bytes(R, kc);
  Tensor ws = at::empty({std::max<int64_t>(ws_bytes, 1)}, opts.dtype(at::kByte));
  check_st(st_fresh_topk(Nm ? ms.data_ptr() : nullptr, Nf ? fs.data_ptr() : nullptr, code, R, Nm,
                         Nf, kc, ws.data_ptr(), top_scores.data_ptr(),
                         top_index.data_ptr<int64_t>(),
                         reinterpret_cast<uint8_t*>(from_fresh.data_ptr<bool>()), stream),
           "take_top_k_and_gather_from_main_and_fresh");

  // gather_data_from_main_and_fresh_index_cpu (fresh_index_post_processing.cpp:165-228)
  TORCH_CHECK(keys.size() == list_main_data.size(),
              "keys and list_main_data should have the same size. ", "keys.size()=", keys.size(),
              ", list_main_data.size()=", list_main_data.size());
  TORCH_CHECK(keys.size() == list_fresh_data.size(),
              "keys and list_fresh_data should have the same size. ", "keys.size()=", keys.size(),
              ", list_fresh_data.size()=", list_fresh_data.size());
  for (size_t i = 0; i < keys.size(); ++i) {
    const Tensor& md = list_main_data[i];
    const Tensor& fd = list_fresh_data[i];
    TORCH_CHECK(md.dim() == fd.dim(), "main_data and fresh_data should have the same dim. ", "key=",
                keys[i], ", main_data.dim()=", md.dim(), ", fresh_data.dim()=", fd.dim());
    if (md.dim() > 1) {
      TORCH_CHECK(md.size(-1) == fd.size(-1),
                  "main_data and fresh_data should have the same number of element in the last dim. "
                  "key=", keys[i], ", main_data.size(-1)=", md.size(-1),
                  ", fresh_data.size(-1)=", fd.size(-1));
    }
    TORCH_CHECK(md.scalar_type() == fd.scalar_type(),
                "main_data and fresh_data should have the same scalar_type. ", "key=", keys[i],
                ", main_data.scalar_type()=", md.scalar_type(),
                ", fresh_data.scalar_type()=", fd.scalar_type());
  }
  c10::Dict<std::string, Tensor> gathered;
  if (!keys.empty()) {
    TORCH_CHECK(main_indices_in.dim() == 2 && fresh_indices_in.dim() == 2,
                "main_indices and fresh_indices must be 2-D");
    TORCH_CHECK(main_indices_in.scalar_type() == at::kInt || main_indices_in.scalar_type() == at::kLong,
                "\"gather_data_from_main_and_fresh_index_cpu_impl_index\" not implemented for '",
                main_indices_in.scalar_type(), "'");
    TORCH_CHECK(fresh_indices_in.scalar_type() == main_indices_in.scalar_type(),
                "expected scalar type ", main_indices_in.scalar_type(),
                " but found ", fresh_indices_in.scalar_type());
    TORCH_CHECK(main_indices_in.size(0) >= R && fresh_indices_in.size(0) >= R,
                "main_indices and fresh_indices must hold a row per score row");
  }
  const Tensor mi = main_indices_in.contiguous(), fi = fresh_indices_in.contiguous();
  for (size_t i = 0; i < keys.size(); ++i) {
    const Tensor& md_in = list_main_data[i];
    const Tensor& fd_in = list_fresh_data[i];
    TORCH_CHECK(md_in.dim() > 0 && md_in.dim() <= 2,
                "The main data dim must be in [1, 2], main_data.dim()=", md_in.dim());
    TORCH_CHECK(fd_in.dim() > 0 && fd_in.dim() <= 2,
                "The fresh data dim must be in [1, 2], fresh_data.dim()=", fd_in.dim());
    TORCH_CHECK(fresh_data_type_ok(md_in.scalar_type()),
                "\"gather_data_from_main_and_fresh_index_cpu_impl\" not implemented for '",
                md_in.scalar_type(), "'");
    TORCH_CHECK(md_in.device() == dev && fd_in.device() == dev,
                "data tensors must be on the scores' device");
    const Tensor md = md_in.contiguous(), fd = fd_in.contiguous();
    const int64_t D = md.dim() == 2 ? md.size(1) : 1;
    Tensor out = md.dim() == 2 ? at::empty({R * kc, D}, md.options())
                               : at::empty({R * kc}, md.options());
    check_st(st_fresh_gather(top_index.data_ptr<int64_t>(), R, kc,
                             fi.numel() ? fi.data_ptr() : nullptr,
                             mi.numel() ? mi.data_ptr() : nullptr,
                             static_cast<int>(mi.element_size()), fi.size(1), mi.size(1), Nf, Nm,
                             fd.numel() ? fd.data_ptr() : nullptr, fd.size(0),
                             md.numel() ? md.data_ptr() : nullptr, md.size(0), D,
                             static_cast<int>(md.element_size()), out.data_ptr(), stream),
             "take_top_k_and_gather_from_main_and_fresh");
    gathered.insert(keys[i], out);
  }
  return {top_scores, top_index, from_fresh, gathered};
}

std::tuple<Tensor, Tensor, Tensor, c10::Dict<std::string, Tensor>> fresh_merge_cpu(
    const Tensor& main_scores, const Tensor& fresh_scores, const Tensor& main_indices,
    const Tensor& fresh_indices, int64_t k, const std::vector<std::string>& keys,
    const std::vector<Tensor>& list_main_data, const std::vector<Tensor>& list_fresh_data,
    int64_t kernel_version) {
  const at::Device gpu = gpu_for_cpu_call();
  std::vector<Tensor> md, fd;
  for (const Tensor& t : list_main_data) md.push_back(t.to(gpu));
  for (const Tensor& t : list_fresh_data) fd.push_back(t.to(gpu));
  auto [s, ix, ff, g] = fresh_merge_gpu(main_scores.to(gpu), fresh_scores.to(gpu),
                                        main_indices.to(gpu), fresh_indices.to(gpu), k, keys, md,
                                        fd, kernel_version);
  c10::Dict<std::string, Tensor> out;
  for (const auto& e : g) out.insert(e.key(), e.value().cpu());
  return {s.cpu(), ix.cpu(), ff.cpu(), out};
}

}  // namespace

TORCH_LIBRARY_FRAGMENT(st, m) {
  // fresh_index_post_processing.cpp:275-287, verbatim
  m.def(
      "take_top_k_and_gather_from_main_and_fresh("
      "Tensor main_scores, "
      "Tensor fresh_scores, "
      "Tensor main_indices, "
      "Tensor fresh_indices, "
      "int k, "
      "str[] keys, "
      "Tensor[] list_main_data, "
      "Tensor[] list_fresh_data, "
      "int kernel_version=2 "
      ") -> (Tensor, Tensor, Tensor, Dict(str, Tensor))");
  m.def(
      "bloom_index_build(Tensor feature_ids, Tensor feature_offsets, "
      "Tensor feature_values, float b_multiplier, int k, "
      "bool fast_build=False) -> (Tensor, Tensor)");
  m.def(
      "bloom_index_search_batch(Tensor bloom_index, "
      "Tensor bloom_bundle_b_offsets, Tensor bloom_query_plans_data, "
      "Tensor bloom_query_plans_offsets, int k, int hash_k, "
      "bool return_bool_mask=True)-> Tensor");
  m.def(
      "parse_expression_query_batch(str[] expressions, Tensor silvertorch_ks, "
      "int bloom_hash_k, bool return_query_plan=True, "
      "int max_sub_queries=5)-> (int, Tensor[])");
  m.def(
      "generate_column_info_for_clusters(Tensor selected_cluster_offsets, "
      "Tensor selected_cluster_lengths) -> (Tensor, Tensor, Tensor)");
  m.def(
      "bloom_index_search_batch_return_partial_response(Tensor bloom_index, "
      "Tensor bloom_bundle_b_offsets, Tensor bloom_query_plans_data, "
      "Tensor bloom_query_plans_offsets, Tensor selected_cluster_offsets, "
      "Tensor selected_cluster_lengths, int k, int hash_k, "
      "Tensor? query_plan_index=None)-> (Tensor, Tensor, Tensor)");
  m.def(
      "bloom_index_search_batch_return_partial_response_multiple(Tensor[] list_bloom_index, "
      "Tensor[] list_bloom_bundle_b_offsets, Tensor bloom_query_plans_data, "
      "Tensor bloom_query_plans_offsets, Tensor[] list_selected_cluster_offsets, "
      "Tensor[] list_selected_cluster_lengths, int k, int hash_k, "
      "Tensor? query_plan_index=None, bool fuse=False)-> (Tensor[], Tensor[], Tensor[])");
  // Ops of this build without a reference counterpart: matching ids as CSR
  // (ids, row_offsets) instead of a mask.
  m.def("bloom_mask_to_ids(Tensor packed_mask, int num_docs, bool int64_ids=False) "
        "-> (Tensor, Tensor)");
  m.def(
      "bloom_index_search_batch_ids(Tensor bloom_index, "
      "Tensor bloom_bundle_b_offsets, Tensor bloom_query_plans_data, "
      "Tensor bloom_query_plans_offsets, int k, int hash_k, int num_docs, "
      "bool int64_ids=False) -> (Tensor, Tensor)");
  // Fused filter + top-k (no reference counterpart): ids int64[Q, topk] and
  // scores float32[Q, topk], padded with -1 / -inf.
  m.def("filtered_topk(Tensor packed_mask, Tensor doc_embeddings, Tensor query_embeddings, "
        "int num_docs, int topk) -> (Tensor, Tensor)");
  m.def(
      "bloom_index_search_topk(Tensor bloom_index, Tensor bloom_bundle_b_offsets, "
      "Tensor bloom_query_plans_data, Tensor bloom_query_plans_offsets, int k, int hash_k, "
      "Tensor doc_embeddings, Tensor query_embeddings, int num_docs, int topk) "
      "-> (Tensor, Tensor)");
  // fused_kmean_ann.cpp:400-455, verbatim
  m.def(
      "fused_kmean_ann("
      "Tensor cluster_offsets, "
      "Tensor cluster_ids, "
      "Tensor cluster_length, "
      "Tensor embeddings, "
      "Tensor queries, "
      "int max_tensor_size_per_row, "
      "Tensor? filtering_bit_mask=None, "
      "int invalid_index_value=-1,"
      "int divisor_for_int8=-1,"
      "Tensor? filtering_bit_index=None, "
      "Tensor? per_embedding_scale=None "
      ") -> (Tensor, Tensor)");
  m.def(
      "fused_kmean_ann_with_partial_masks("
      "Tensor cluster_offsets, "
      "Tensor cluster_ids, "
      "Tensor cluster_length, "
      "Tensor embeddings, "
      "Tensor queries, "
      "int max_tensor_size_per_row, "
      "Tensor partial_mask_column_counts_cumsum, "
      "Tensor partial_mask_first_item_offset_in_column, "
      "Tensor partial_mask_column_results, "
      "int invalid_index_value=-1,"
      "int divisor_for_int8=-1,"
      "Tensor? filtering_bit_index=None, "
      "Tensor? per_embedding_scale=None, "
      "Tensor? cluster_warp_size=None, "
      "Tensor? cluster_warp_rounded_length_cumsum=None, "
      "Tensor? cluster_remaining_length_cumsum=None, "
      "Tensor? cluster_warp_size_cumsum=None, "
      "int total_cluster_rounded_warps=0, "
      "int total_cluster_remaining_warps=0 "
      ") -> (Tensor, Tensor)");
  m.def(
      "fused_kmean_ann_with_partial_masks_multiple("
      "Tensor queries, "
      "Tensor[] list_cluster_offsets, "
      "Tensor[] list_selected_cluster_ids, "
      "Tensor[] list_selected_cluster_lengths, "
      "Tensor[] list_embeddings, "
      "int[] list_max_tensor_size_per_row, "
      "Tensor[] list_partial_mask_column_counts_cumsum, "
      "Tensor[] list_partial_mask_first_item_offset_in_column, "
      "Tensor[] list_partial_mask_column_results, "
      "int invalid_index_value=-1, "
      "int divisor_for_int8=-1, "
      "Tensor? filtering_bit_index=None, "
      "Tensor[]? list_per_embedding_scale=None, "
      "bool fuse=False "
      ") -> (Tensor[], Tensor[])");
}

TORCH_LIBRARY_IMPL(st, CUDA, m) {
  m.impl("bloom_index_build", TORCH_FN(build_gpu));
  m.impl("bloom_index_search_batch", TORCH_FN(search_gpu));
  m.impl("parse_expression_query_batch", TORCH_FN(parse_batch));
  m.impl("generate_column_info_for_clusters", TORCH_FN(column_info));
  m.impl("bloom_index_search_batch_return_partial_response", TORCH_FN(partial_gpu));
  m.impl("bloom_index_search_batch_return_partial_response_multiple", TORCH_FN(partial_multiple));
  m.impl("bloom_mask_to_ids", TORCH_FN(mask_to_ids_gpu));
  m.impl("bloom_index_search_batch_ids", TORCH_FN(search_ids_gpu));
  m.impl("filtered_topk", TORCH_FN(filtered_topk_gpu));
  m.impl("bloom_index_search_topk", TORCH_FN(search_topk_gpu));
  m.impl("fused_kmean_ann", TORCH_FN(kmean_gpu));
  m.impl("fused_kmean_ann_with_partial_masks", TORCH_FN(kmean_partial));
  m.impl("fused_kmean_ann_with_partial_masks_multiple", TORCH_FN(kmean_partial_multiple));
  m.impl("take_top_k_and_gather_from_main_and_fresh", TORCH_FN(fresh_merge_gpu));
}

TORCH_LIBRARY_IMPL(st, CPU, m) {
  m.impl("bloom_index_build", TORCH_FN(build_cpu_tensors));
  m.impl("bloom_index_search_batch", TORCH_FN(search_cpu_tensors));
  m.impl("parse_expression_query_batch", TORCH_FN(parse_batch));
  m.impl("generate_column_info_for_clusters", TORCH_FN(column_info));
  m.impl("bloom_index_search_batch_return_partial_response", TORCH_FN(partial_cpu));
  m.impl("bloom_index_search_batch_return_partial_response_multiple", TORCH_FN(partial_multiple));
  m.impl("bloom_mask_to_ids", TORCH_FN(mask_to_ids_cpu));
  m.impl("bloom_index_search_batch_ids", TORCH_FN(search_ids_cpu));
  m.impl("filtered_topk", TORCH_FN(filtered_topk_cpu));
  m.impl("bloom_index_search_topk", TORCH_FN(search_topk_cpu));
  m.impl("fused_kmean_ann", TORCH_FN(kmean_cpu));
  m.impl("fused_kmean_ann_with_partial_masks", TORCH_FN(kmean_partial));
  m.impl("fused_kmean_ann_with_partial_masks_multiple", TORCH_FN(kmean_partial_multiple));
  m.impl("take_top_k_and_gather_from_main_and_fresh", TORCH_FN(fresh_merge_cpu));
}

// Python module entry point: importing silvertorch_amd._C loads this library,
// whose static initialisers above register torch.ops.st.*.
static PyModuleDef st_module = {PyModuleDef_HEAD_INIT, "_C",
                                "torch.ops.st.* on MI355X (HIP)", -1, nullptr};
PyMODINIT_FUNC PyInit__C(void) { return PyModule_Create(&st_module); }
