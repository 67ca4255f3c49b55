// C ABI of the DSA offload chain: argument validation (the reference adapter
// TORCH_CHECKs, returned as status codes) and kernel dispatch.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/nvdsa.h"
#include "nvdsa_common.h"
#include "nvdsa_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* msg) {
  g_last_error = msg;
  return code;
}

// Validation helper: the first failing requirement wins, like a chain of
// TORCH_CHECKs.
class Check {
 public:
  explicit Check(const char* op) : op_(op) {}
  Check& need(bool cond, int code, const char* msg) {
    if (code_ == NVDSA_OK && !cond) {
      code_ = code;
      msg_ = std::string(op_) + ": " + msg;
    }
    return *this;
  }
  bool ok() const { return code_ == NVDSA_OK; }
  int finish() {
    if (code_ != NVDSA_OK) g_last_error = msg_;
    return code_;
  }

 private:
  const char* op_;
  int code_ = NVDSA_OK;
  std::string msg_;
};

bool dims_are(const nvdsa_tensor* t, int nd) { return t && t->ndim == nd; }
int64_t sz(const nvdsa_tensor* t, int i) { return (t && i < t->ndim) ? t->shape[i] : -1; }
bool same_shape(const nvdsa_tensor* a, const nvdsa_tensor* b) {
  if (!a || !b || a->ndim != b->ndim) return false;
  for (int i = 0; i < a->ndim; ++i)
    if (a->shape[i] != b->shape[i]) return false;
  return true;
}
int64_t numel(const nvdsa_tensor* t) {
  int64_t n = 1;
  for (int i = 0; i < t->ndim; ++i) n *= t->shape[i];
  return n;
}
bool is_half(const nvdsa_tensor* t) {
  return t->dtype == NVDSA_FLOAT16 || t->dtype == NVDSA_BFLOAT16;
}
bool aligned16(const nvdsa_tensor* t) {
  return numel(t) == 0 || (reinterpret_cast<uintptr_t>(t->data) & 15u) == 0;
}
bool aligned4(const nvdsa_tensor* t) {
  return numel(t) == 0 || (reinterpret_cast<uintptr_t>(t->data) & 3u) == 0;
}
bool has_data(const nvdsa_tensor* t) { return numel(t) == 0 || t->data != nullptr; }
// A shape as Python prints a tuple: "(24, 32, 128)", "(24,)".
std::string shape_str(const nvdsa_tensor* t) {
  std::string out = "(";
  for (int i = 0; i < t->ndim; ++i) out += (i ? ", " : "") + std::to_string(t->shape[i]);
  return out + (t->ndim == 1 ? ",)" : ")");
}

nvdsa::Elem elem_of(const nvdsa_tensor* t) {
  return t->dtype == NVDSA_BFLOAT16 ? nvdsa::Elem::kBf16 : nvdsa::Elem::kF16;
}

template <size_t N>
bool all_nonnull(const nvdsa_tensor* const (&ts)[N]) {
  for (auto* t : ts)
    if (!t) return false;
  return true;
}

template <size_t N>
void check_common(Check& c, const nvdsa_tensor* const (&ts)[N], int device,
                  const nvdsa_tensor* host_ok_a = nullptr, const nvdsa_tensor* host_ok_b = nullptr) {
  for (auto* t : ts) {
    c.need(t->contiguous == 1, NVDSA_ERR_LAYOUT, "all inputs must be contiguous");
    c.need(has_data(t), NVDSA_ERR_ARG, "null data pointer");
    const bool host_allowed = (t == host_ok_a || t == host_ok_b);
    c.need(t->device == device || (host_allowed && t->device == NVDSA_HOST_MAPPED_DEVICE),
           NVDSA_ERR_DEVICE, "all inputs must be on the same device");
  }
}

// Timing instrumentation state of the calling thread.
struct ProfState {
  std::vector<hipEvent_t> events;  // 2 per launch
  std::vector<int> ids;
  int capacity = 0;
  int count = 0;
  bool on = false;
};
thread_local ProfState g_prof;

int launch_status(hipError_t e, const char* op) {
  if (e != hipSuccess) {
    g_last_error = std::string(op) + ": HIP launch failed: " + hipGetErrorString(e);
    return NVDSA_ERR_RUNTIME;
  }
  g_last_error.clear();
  return NVDSA_OK;
}

constexpr int64_t kMaxGridThreads = (int64_t{1} << 31);

}  // namespace

namespace nvdsa {

ProfEvents prof_events(int kernel_id) {
  ProfState& p = g_prof;
  ProfEvents ev;
  if (!p.on || p.count >= p.capacity) return ev;
  ev.start = p.events[2 * p.count];
  ev.stop = p.events[2 * p.count + 1];
  p.ids[p.count] = kernel_id;
  ++p.count;
  return ev;
}

}  // namespace nvdsa

extern "C" {

int nvdsa_profile_begin(int32_t capacity) {
  if (capacity <= 0) return fail(NVDSA_ERR_ARG, "profile_begin: capacity must be positive");
  ProfState& p = g_prof;
  while (static_cast<int>(p.events.size()) < 2 * capacity) {
    hipEvent_t e;
    hipError_t err = hipEventCreate(&e);
    if (err != hipSuccess) {
      g_last_error = std::string("profile_begin: hipEventCreate failed: ") + hipGetErrorString(err);
      return NVDSA_ERR_RUNTIME;
    }
    p.events.push_back(e);
  }
  p.ids.assign(capacity, -1);
  p.capacity = capacity;
  p.count = 0;
  p.on = true;
  return NVDSA_OK;
}

int nvdsa_profile_end(float* durations_ms, int32_t* kernel_ids, int32_t capacity, int32_t* recorded) {
  ProfState& p = g_prof;
  p.on = false;
  const int n = std::min(p.count, static_cast<int>(capacity));
  for (int i = 0; i < n; ++i) {
    hipError_t err = hipEventSynchronize(p.events[2 * i + 1]);
    float ms = 0.f;
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, p.events[2 * i], p.events[2 * i + 1]);
    if (err != hipSuccess) {
      g_last_error = std::string("profile_end: ") + hipGetErrorString(err);
      return NVDSA_ERR_RUNTIME;
    }
    if (durations_ms) durations_ms[i] = ms;
    if (kernel_ids) kernel_ids[i] = p.ids[i];
  }
  if (recorded) *recorded = n;
  p.count = 0;
  return NVDSA_OK;
}

const char* nvdsa_kernel_name(int32_t kernel_id) {
  static const char* names[] = {"scatter_copy_kernel", "lim_score_kernel",   "lim_hist_kernel",
                                "lim_mtp_pass_a_kernel", "sfa_split_kernel", "sfa_split_kernel_fused",
                                "sfa_combine_kernel",    "lidu_init_kernel", "lidu_shared_kernel",
                                "lim_threshold_kernel",  "lim_mtp_victims_kernel", "lim_mtp_pass_b_kernel",
                                "sfa_mtp_overlap_kernel", "sfa_split_kernel_copied", "indexer_project_kernel",
                                "indexer_rope_kernel", "persist_blocks_kernel", "lim_classify_kernel",
                                "lim_chunks_kernel",   "lim_resolve_kernel"};
  static_assert(sizeof(names) / sizeof(names[0]) == nvdsa::kKernCount, "one name per kernel id");
  if (kernel_id < 0 || kernel_id >= nvdsa::kKernCount) return "unknown";
  return names[kernel_id];
}

void nvdsa_xcd_roles_record(int32_t on) { nvdsa::sfa_xcd_roles_record(on != 0); }

int nvdsa_xcd_roles(uint32_t* masks, int32_t reset) {
  if (masks == nullptr) return fail(NVDSA_ERR_ARG, "xcd_roles: masks must not be null");
  const hipError_t err = nvdsa::sfa_xcd_roles(masks, reset != 0);
  if (err != hipSuccess) {
    g_last_error = std::string("xcd_roles: ") + hipGetErrorString(err);
    return NVDSA_ERR_RUNTIME;
  }
  return NVDSA_OK;
}

const char* nvdsa_last_error(void) { return g_last_error.c_str(); }

const char* nvdsa_version(void) { return "nvdsa 0.1.0 gfx950"; }

// ------------------------------------------------------------------------
size_t nvdsa_fused_li_manage_workspace_size(int64_t batch, int64_t source_capacity,
                                            int64_t index_heads) {
  (void)index_heads;
  if (batch < 0 || source_capacity < 0) return 0;
  return nvdsa::lim_workspace_bytes(batch, source_capacity, 1);
}

size_t nvdsa_fused_li_manage_mtp_workspace_size(int64_t batch, int64_t source_capacity,
                                                int64_t index_heads) {
  (void)index_heads;
  if (batch < 0 || source_capacity < 0) return 0;
  return nvdsa::lim_workspace_bytes(batch, source_capacity, nvdsa::kMtpQueries);
}

}  // extern "C"

namespace {

// Scratch memory of nvdsa_fused_li_manage_noalloc: one copy of this array per
// GPU the library runs on, held until the process ends.  Host code never
// uses the array's name as an address; it uses the per-device pointer that
// hipGetSymbolAddress returns (noalloc_scratch below).
static __device__ __align__(256) unsigned char scratch[NVDSA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on `device` (the current device), looked up
// once per device; nullptr with the error message set on failure.
void* noalloc_scratch(int device, const char* op) {
  if (device < 0 || device >= kMaxDevices) {
    fail(NVDSA_ERR_DEVICE, (std::string(op) + ": device index out of range").c_str());
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device] == nullptr) {
    // A first call made while the caller captures a graph: the lookup enqueues
    // nothing, but the runtime may load the code object; this thread's capture
    // mode is relaxed for the lookup so that the capture stays valid.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const bool exchanged = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (exchanged) (void)hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess || ptr == nullptr) {
      fail(NVDSA_ERR_RUNTIME,
           (std::string(op) + ": hipGetSymbolAddress(scratch) failed: " + hipGetErrorString(e)).c_str());
      return nullptr;
    }
    g_scratch_ptr[device] = ptr;
  }
  return g_scratch_ptr[device];
}

// fused_li_manage with the workspace given by the caller, or (noalloc) with
// the library's static per-device scratch array.
int fused_li_manage_impl(const char* op, const nvdsa_tensor* query, const nvdsa_tensor* index_weights,
                         const nvdsa_tensor* index_key_cache, const nvdsa_tensor* index_block_table,
                         const nvdsa_tensor* num_candidate_tokens, const nvdsa_tensor* num_cache_tokens,
                         const nvdsa_tensor* req_pool_entries, const nvdsa_tensor* cache_slots_pool,
                         const nvdsa_tensor* topk_src_ids, const nvdsa_tensor* topk_dst_slots,
                         const nvdsa_tensor* miss_counts, void* workspace, size_t workspace_bytes, void* stream,
                         bool noalloc) {
  const nvdsa_tensor* const all[] = {query, index_weights, index_key_cache, index_block_table,
                                     num_candidate_tokens, num_cache_tokens, req_pool_entries,
                                     cache_slots_pool, topk_src_ids, topk_dst_slots, miss_counts};
  if (!all_nonnull(all)) return fail(NVDSA_ERR_ARG, (std::string(op) + ": null tensor argument").c_str());
  Check c(op);
  // ops/fused_li_manage/fused_li_manage_torch_adpt.h:18-92
  c.need(dims_are(query, 3), NVDSA_ERR_SHAPE, "query must be [B, N, 128]")
      .need(sz(query, 1) == 32 || sz(query, 1) == 64, NVDSA_ERR_SHAPE, "index head count must be 32 or 64")
      .need(sz(query, 2) == 128, NVDSA_ERR_SHAPE, "head_dim must be 128")
      .need(dims_are(index_key_cache, 4) && sz(index_key_cache, 1) == 128 && sz(index_key_cache, 2) == 1 &&
                sz(index_key_cache, 3) == 128,
            NVDSA_ERR_SHAPE, "key must be [blocks, 128, 1, 128]")
      .need(dims_are(index_weights, 2) && sz(index_weights, 0) == sz(query, 0) &&
                sz(index_weights, 1) == sz(query, 1),
            NVDSA_ERR_SHAPE, "weights must be [B, N]")
      .need(dims_are(req_pool_entries, 1) && dims_are(num_cache_tokens, 1) && dims_are(num_candidate_tokens, 1),
            NVDSA_ERR_SHAPE, "row metadata must be rank one")
      .need(dims_are(cache_slots_pool, 2) && dims_are(index_block_table, 2), NVDSA_ERR_SHAPE,
            "cache_slots and block_table must be rank two")
      .need(dims_are(topk_src_ids, 3) && sz(topk_src_ids, 1) == 1 && sz(topk_src_ids, 2) == 2048,
            NVDSA_ERR_SHAPE, "source_ids must be [B, 1, 2048]")
      .need(same_shape(topk_dst_slots, topk_src_ids), NVDSA_ERR_SHAPE,
            "destination_slots must match source_ids")
      .need(dims_are(miss_counts, 1), NVDSA_ERR_SHAPE, "miss_counts must be rank one");
  if (c.ok()) {
    const int64_t B = sz(query, 0);
    c.need(B == sz(req_pool_entries, 0) && B == sz(num_cache_tokens, 0) && B == sz(num_candidate_tokens, 0) &&
               B == sz(index_block_table, 0) && B == sz(topk_src_ids, 0) && B == sz(miss_counts, 0),
           NVDSA_ERR_SHAPE, "batch dimensions must match")
        .need(sz(cache_slots_pool, 1) == sz(index_block_table, 1) * 128, NVDSA_ERR_SHAPE,
              "request state width must match block-table capacity")
        .need(sz(cache_slots_pool, 0) > 0 && sz(index_block_table, 1) > 0, NVDSA_ERR_SHAPE,
              "request pool and block table must be non-empty")
        .need(sz(index_block_table, 1) <= (1 << 14), NVDSA_ERR_SHAPE,
              "block-table capacity must be <= 16384 blocks")
        .need(query->dtype == index_key_cache->dtype && query->dtype == index_weights->dtype, NVDSA_ERR_DTYPE,
              "query/key/weights dtypes must match");
    const nvdsa_tensor* const meta[] = {cache_slots_pool, req_pool_entries, num_cache_tokens,
                                        num_candidate_tokens, index_block_table, topk_src_ids,
                                        topk_dst_slots, miss_counts};
    for (auto* t : meta) c.need(t->dtype == NVDSA_INT32, NVDSA_ERR_DTYPE, "metadata must be int32");
    c.need(is_half(query), NVDSA_ERR_DTYPE, "query/key/weights must be fp16 or bf16");
    check_common(c, all, query->device);
    c.need(aligned16(query) && aligned16(index_key_cache), NVDSA_ERR_LAYOUT,
           "query and key cache must be 16-byte aligned");
  }
  if (!c.ok()) return c.finish();
  const int64_t B = sz(query, 0);
  const int64_t cols = sz(index_block_table, 1);
  const size_t need = nvdsa::lim_workspace_bytes(B, cols * 128, 1);
  if (noalloc && need > NVDSA_NOALLOC_SCRATCH_BYTES) {
    const std::string msg = std::string(op) + ": batch " + std::to_string(B) + " x source capacity " +
                            std::to_string(cols * 128) + " needs " + std::to_string(need) +
                            " bytes of scratch, more than the static " +
                            std::to_string(static_cast<size_t>(NVDSA_NOALLOC_SCRATCH_BYTES)) +
                            " bytes; call nvdsa_fused_li_manage with a workspace";
    return fail(NVDSA_ERR_WORKSPACE, msg.c_str());
  }
  if (B == 0) return NVDSA_OK;
  if (noalloc) {
    int current = -1;
    if (hipGetDevice(&current) != hipSuccess || current != query->device)
      return fail(NVDSA_ERR_DEVICE, (std::string(op) + ": the tensors' device must be the current device").c_str());
    workspace = noalloc_scratch(current, op);
    if (workspace == nullptr) return NVDSA_ERR_RUNTIME;  // message set by noalloc_scratch
    workspace_bytes = NVDSA_NOALLOC_SCRATCH_BYTES;
  }
  if (workspace_bytes < need || workspace == nullptr)
    return fail(NVDSA_ERR_WORKSPACE, (std::string(op) + ": workspace too small").c_str());
  nvdsa::LimArgs a{};
  a.query = query->data;
  a.weights = index_weights->data;
  a.key_cache = index_key_cache->data;
  a.block_table = static_cast<const int32_t*>(index_block_table->data);
  a.num_candidates = static_cast<const int32_t*>(num_candidate_tokens->data);
  a.num_cache = static_cast<const int32_t*>(num_cache_tokens->data);
  a.pool_entries = static_cast<const int32_t*>(req_pool_entries->data);
  a.pool = static_cast<int32_t*>(cache_slots_pool->data);
  a.topk_src = static_cast<int32_t*>(topk_src_ids->data);
  a.topk_dst = static_cast<int32_t*>(topk_dst_slots->data);
  a.miss_counts = static_cast<int32_t*>(miss_counts->data);
  a.batch = B;
  a.heads = sz(query, 1);
  a.cols = cols;
  a.key_blocks = sz(index_key_cache, 0);
  a.pool_rows = sz(cache_slots_pool, 0);
  a.source_capacity = cols * 128;
  a.elem = elem_of(query);
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  return launch_status(nvdsa::launch_fused_li_manage(a, static_cast<hipStream_t>(stream)), op);
}

}  // namespace

extern "C" {

int nvdsa_fused_li_manage(const nvdsa_tensor* query, const nvdsa_tensor* index_weights,
                          const nvdsa_tensor* index_key_cache, const nvdsa_tensor* index_block_table,
                          const nvdsa_tensor* num_candidate_tokens, const nvdsa_tensor* num_cache_tokens,
                          const nvdsa_tensor* req_pool_entries, const nvdsa_tensor* cache_slots_pool,
                          const nvdsa_tensor* topk_src_ids, const nvdsa_tensor* topk_dst_slots,
                          const nvdsa_tensor* miss_counts, void* workspace, size_t workspace_bytes,
                          void* stream) {
  return fused_li_manage_impl("fused_li_manage", query, index_weights, index_key_cache, index_block_table,
                              num_candidate_tokens, num_cache_tokens, req_pool_entries, cache_slots_pool,
                              topk_src_ids, topk_dst_slots, miss_counts, workspace, workspace_bytes, stream, false);
}

int nvdsa_fused_li_manage_noalloc(const nvdsa_tensor* query, const nvdsa_tensor* index_weights,
                                  const nvdsa_tensor* index_key_cache, const nvdsa_tensor* index_block_table,
                                  const nvdsa_tensor* num_candidate_tokens, const nvdsa_tensor* num_cache_tokens,
                                  const nvdsa_tensor* req_pool_entries, const nvdsa_tensor* cache_slots_pool,
                                  const nvdsa_tensor* topk_src_ids, const nvdsa_tensor* topk_dst_slots,
                                  const nvdsa_tensor* miss_counts, void* stream) {
  return fused_li_manage_impl("fused_li_manage_noalloc", query, index_weights, index_key_cache, index_block_table,
                              num_candidate_tokens, num_cache_tokens, req_pool_entries, cache_slots_pool,
                              topk_src_ids, topk_dst_slots, miss_counts, nullptr, 0, stream, true);
}

int nvdsa_fused_li_manage_mtp(const nvdsa_tensor* query, const nvdsa_tensor* index_weights,
                              const nvdsa_tensor* index_key_cache, const nvdsa_tensor* index_block_table,
                              const nvdsa_tensor* num_candidate_tokens, const nvdsa_tensor* num_cache_tokens,
                              const nvdsa_tensor* req_pool_entries, const nvdsa_tensor* cache_slots_pool,
                              const nvdsa_tensor* topk_src_ids, const nvdsa_tensor* topk_dst_slots,
                              const nvdsa_tensor* miss_src_ids, const nvdsa_tensor* miss_dst_slots,
                              const nvdsa_tensor* miss_counts, void* workspace, size_t workspace_bytes,
                              void* stream) {
  const nvdsa_tensor* const all[] = {query, index_weights, index_key_cache, index_block_table,
                                     num_candidate_tokens, num_cache_tokens, req_pool_entries,
                                     cache_slots_pool, topk_src_ids, topk_dst_slots, miss_src_ids,
                                     miss_dst_slots, miss_counts};
  if (!all_nonnull(all)) return fail(NVDSA_ERR_ARG, "fused_li_manage_mtp: null tensor argument");
  Check c("fused_li_manage_mtp");
  // ops/fused_li_manage_mtp/fused_li_manage_mtp_torch_adpt.h:20-111
  c.need(dims_are(query, 3) && (sz(query, 1) == 32 || sz(query, 1) == 64) && sz(query, 2) == 128,
         NVDSA_ERR_SHAPE, "query must be [4B, H, 128], H=32 or 64")
      .need(dims_are(req_pool_entries, 1), NVDSA_ERR_SHAPE, "req_pool_entries must be [B]");
  const int64_t B = sz(req_pool_entries, 0);
  c.need(B > 0 && sz(query, 0) == B * nvdsa::kMtpQueries, NVDSA_ERR_SHAPE,
         "requires exactly four packed queries per request")
      .need(dims_are(index_key_cache, 4) && sz(index_key_cache, 0) > 0 && sz(index_key_cache, 1) == 128 &&
                sz(index_key_cache, 2) == 1 && sz(index_key_cache, 3) == 128,
            NVDSA_ERR_SHAPE, "key must be [blocks, 128, 1, 128]")
      .need(dims_are(index_weights, 2) && sz(index_weights, 0) == sz(query, 0) &&
                sz(index_weights, 1) == sz(query, 1),
            NVDSA_ERR_SHAPE, "weights must be [4B, H] and match query heads")
      .need(dims_are(cache_slots_pool, 2) && sz(cache_slots_pool, 0) > 0 && dims_are(num_cache_tokens, 1) &&
                dims_are(num_candidate_tokens, 1) && dims_are(index_block_table, 2) &&
                sz(index_block_table, 1) > 0,
            NVDSA_ERR_SHAPE, "cache metadata has invalid rank or empty capacity")
      .need(sz(num_cache_tokens, 0) == B && sz(num_candidate_tokens, 0) == B && sz(index_block_table, 0) == B,
            NVDSA_ERR_SHAPE, "request metadata batch dimensions must match")
      .need(sz(cache_slots_pool, 1) == sz(index_block_table, 1) * 128, NVDSA_ERR_SHAPE,
            "pool width must match block-table capacity")
      .need(sz(index_block_table, 1) <= (1 << 11), NVDSA_ERR_SHAPE, "source capacity must be <= 2^18 tokens")
      .need(dims_are(topk_dst_slots, 3) && sz(topk_dst_slots, 0) == sz(query, 0) && sz(topk_dst_slots, 1) == 1 &&
                sz(topk_dst_slots, 2) == 2048,
            NVDSA_ERR_SHAPE, "topk_slots must be [4B, 1, 2048]")
      .need(same_shape(topk_src_ids, topk_dst_slots), NVDSA_ERR_SHAPE, "topk_source_ids must match topk_slots")
      .need(dims_are(miss_src_ids, 2) && sz(miss_src_ids, 0) == B && sz(miss_src_ids, 1) == nvdsa::kUnionCap &&
                same_shape(miss_dst_slots, miss_src_ids),
            NVDSA_ERR_SHAPE, "miss outputs must be [B, 8192]")
      .need(dims_are(miss_counts, 1) && sz(miss_counts, 0) == B, NVDSA_ERR_SHAPE, "miss_counts must be [B]")
      .need(query->dtype == index_key_cache->dtype && query->dtype == index_weights->dtype && is_half(query),
            NVDSA_ERR_DTYPE, "query/key/weights must share fp16 or bf16 dtype");
  const nvdsa_tensor* const meta[] = {req_pool_entries, cache_slots_pool, num_cache_tokens, num_candidate_tokens,
                                      index_block_table, topk_dst_slots, topk_src_ids, miss_src_ids,
                                      miss_dst_slots, miss_counts};
  for (auto* t : meta) c.need(t->dtype == NVDSA_INT32, NVDSA_ERR_DTYPE, "metadata and outputs must be int32");
  if (c.ok()) {
    check_common(c, all, query->device);
    c.need(aligned16(query) && aligned16(index_key_cache), NVDSA_ERR_LAYOUT,
           "query and key cache must be 16-byte aligned");
  }
  if (!c.ok()) return c.finish();
  const int64_t cols = sz(index_block_table, 1);
  const size_t need = nvdsa::lim_workspace_bytes(B, cols * 128, nvdsa::kMtpQueries);
  if (workspace_bytes < need || workspace == nullptr)
    return fail(NVDSA_ERR_WORKSPACE, "fused_li_manage_mtp: workspace too small");
  nvdsa::LimArgs a{};
  a.query = query->data;
  a.weights = index_weights->data;
  a.key_cache = index_key_cache->data;
  a.block_table = static_cast<const int32_t*>(index_block_table->data);
  a.num_candidates = static_cast<const int32_t*>(num_candidate_tokens->data);
  a.num_cache = static_cast<const int32_t*>(num_cache_tokens->data);
  a.pool_entries = static_cast<const int32_t*>(req_pool_entries->data);
  a.pool = static_cast<int32_t*>(cache_slots_pool->data);
  a.topk_src = static_cast<int32_t*>(topk_src_ids->data);
  a.topk_dst = static_cast<int32_t*>(topk_dst_slots->data);
  a.miss_src = static_cast<int32_t*>(miss_src_ids->data);
  a.miss_dst = static_cast<int32_t*>(miss_dst_slots->data);
  a.miss_counts = static_cast<int32_t*>(miss_counts->data);
  a.batch = B;
  a.heads = sz(query, 1);
  a.cols = cols;
  a.key_blocks = sz(index_key_cache, 0);
  a.pool_rows = sz(cache_slots_pool, 0);
  a.source_capacity = cols * 128;
  a.elem = elem_of(query);
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  return launch_status(nvdsa::launch_fused_li_manage_mtp(a, static_cast<hipStream_t>(stream)),
                       "fused_li_manage_mtp");
}

// ------------------------------------------------------------------------
int nvdsa_scatter_copy(const nvdsa_tensor* src_ids, const nvdsa_tensor* dst_slots,
                       const nvdsa_tensor* copy_counts, const nvdsa_tensor* hbm_block_table,
                       const nvdsa_tensor* dram_block_table, const nvdsa_tensor* hbm_k_rope,
                       const nvdsa_tensor* hbm_kv_cache, const nvdsa_tensor* dram_k_rope,
                       const nvdsa_tensor* dram_kv_cache, void* stream) {
  const nvdsa_tensor* const all[] = {src_ids, dst_slots, copy_counts, hbm_block_table, dram_block_table,
                                     hbm_k_rope, hbm_kv_cache, dram_k_rope, dram_kv_cache};
  if (!all_nonnull(all)) return fail(NVDSA_ERR_ARG, "scatter_copy: null tensor argument");
  Check c("scatter_copy");
  // ops/kvcache_scatter_copy/kvcache_scatter_copy_torch_adpt.h:16-66
  c.need(dims_are(hbm_k_rope, 3) && sz(hbm_k_rope, 1) == 128 && sz(hbm_k_rope, 2) == 64, NVDSA_ERR_SHAPE,
         "HBM KPE must be [blocks, 128, 64]")
      .need(dims_are(hbm_kv_cache, 3) && sz(hbm_kv_cache, 1) == 128 && sz(hbm_kv_cache, 2) == 512,
            NVDSA_ERR_SHAPE, "HBM CKV must be [blocks, 128, 512]")
      .need(dims_are(dram_k_rope, 3) && sz(dram_k_rope, 1) == 128 && sz(dram_k_rope, 2) == 64, NVDSA_ERR_SHAPE,
            "DRAM KPE must be [blocks, 128, 64]")
      .need(dims_are(dram_kv_cache, 3) && sz(dram_kv_cache, 1) == 128 && sz(dram_kv_cache, 2) == 512,
            NVDSA_ERR_SHAPE, "DRAM CKV must be [blocks, 128, 512]")
      .need(dims_are(hbm_block_table, 2) && dims_are(dram_block_table, 2) && dims_are(src_ids, 2) &&
                dims_are(dst_slots, 2) && dims_are(copy_counts, 1),
            NVDSA_ERR_SHAPE, "tables/indices must be [B, C] and counts [B]")
      .need(same_shape(src_ids, dst_slots), NVDSA_ERR_SHAPE, "source and destination shapes must match")
      .need(sz(src_ids, 1) > 0, NVDSA_ERR_SHAPE, "input capacity must be positive")
      .need(sz(src_ids, 1) <= 65536, NVDSA_ERR_SHAPE, "capacity must be <= 65536")
      .need(sz(copy_counts, 0) == sz(src_ids, 0) && sz(hbm_block_table, 0) == sz(src_ids, 0) &&
                sz(dram_block_table, 0) == sz(src_ids, 0),
            NVDSA_ERR_SHAPE, "batch dimensions must match")
      .need(is_half(hbm_k_rope), NVDSA_ERR_DTYPE, "CKV/KPE must be fp16 or bf16")
      .need(hbm_kv_cache->dtype == hbm_k_rope->dtype && dram_k_rope->dtype == hbm_k_rope->dtype &&
                dram_kv_cache->dtype == hbm_k_rope->dtype,
            NVDSA_ERR_DTYPE, "all CKV/KPE tensors must have the same dtype")
      .need(hbm_block_table->dtype == NVDSA_INT32 && dram_block_table->dtype == NVDSA_INT32 &&
                src_ids->dtype == NVDSA_INT32 && dst_slots->dtype == NVDSA_INT32 &&
                copy_counts->dtype == NVDSA_INT32,
            NVDSA_ERR_DTYPE, "tables, indices, slots and counts must be int32");
  if (c.ok()) {
    check_common(c, all, hbm_k_rope->device, dram_k_rope, dram_kv_cache);
    c.need(aligned16(hbm_k_rope) && aligned16(hbm_kv_cache) && aligned16(dram_k_rope) && aligned16(dram_kv_cache),
           NVDSA_ERR_LAYOUT, "KV caches must be 16-byte aligned");
    c.need(sz(src_ids, 0) * nvdsa::ceil_div(sz(src_ids, 1), 16) * 256 < kMaxGridThreads, NVDSA_ERR_SHAPE,
           "batch x capacity too large for one launch");
  }
  if (!c.ok()) return c.finish();
  nvdsa::ScatterArgs a{};
  a.src_ids = static_cast<const int32_t*>(src_ids->data);
  a.dst_slots = static_cast<const int32_t*>(dst_slots->data);
  a.copy_counts = static_cast<const int32_t*>(copy_counts->data);
  a.hbm_table = static_cast<const int32_t*>(hbm_block_table->data);
  a.dram_table = static_cast<const int32_t*>(dram_block_table->data);
  a.hbm_kpe = hbm_k_rope->data;
  a.hbm_ckv = hbm_kv_cache->data;
  a.dram_kpe = dram_k_rope->data;
  a.dram_ckv = dram_kv_cache->data;
  a.batch = sz(src_ids, 0);
  a.cap = sz(src_ids, 1);
  a.hbm_cols = sz(hbm_block_table, 1);
  a.dram_cols = sz(dram_block_table, 1);
  a.hbm_blocks = std::min(sz(hbm_k_rope, 0), sz(hbm_kv_cache, 0));
  a.dram_blocks = std::min(sz(dram_k_rope, 0), sz(dram_kv_cache, 0));
  return launch_status(nvdsa::launch_scatter_copy(a, static_cast<hipStream_t>(stream)), "scatter_copy");
}

// ------------------------------------------------------------------------
// First-decode LIDU initialisation (nanovllm/models/dsa_offload_ops.py:251-411).
namespace {

// Cache and table checks shared by the two initialisation entry points (the
// 3-D cache views scatter_copy takes, 1-D table rows of one request).
void check_lidu_copy(Check& c, const nvdsa_tensor* slots_row, const nvdsa_tensor* hbm_kpe,
                     const nvdsa_tensor* hbm_ckv, const nvdsa_tensor* dram_kpe, const nvdsa_tensor* dram_ckv,
                     const nvdsa_tensor* hbm_table, const nvdsa_tensor* dram_table) {
  c.need(dims_are(slots_row, 1) && slots_row->dtype == NVDSA_INT32, NVDSA_ERR_SHAPE,
         "cache_slots_row must be a 1-D int32 pool row")
      .need(dims_are(hbm_kpe, 3) && sz(hbm_kpe, 1) == 128 && sz(hbm_kpe, 2) == 64, NVDSA_ERR_SHAPE,
            "HBM KPE must be [blocks, 128, 64]")
      .need(dims_are(hbm_ckv, 3) && sz(hbm_ckv, 1) == 128 && sz(hbm_ckv, 2) == 512, NVDSA_ERR_SHAPE,
            "HBM CKV must be [blocks, 128, 512]")
      .need(dims_are(dram_kpe, 3) && sz(dram_kpe, 1) == 128 && sz(dram_kpe, 2) == 64, NVDSA_ERR_SHAPE,
            "DRAM KPE must be [blocks, 128, 64]")
      .need(dims_are(dram_ckv, 3) && sz(dram_ckv, 1) == 128 && sz(dram_ckv, 2) == 512, NVDSA_ERR_SHAPE,
            "DRAM CKV must be [blocks, 128, 512]")
      .need(dims_are(hbm_table, 1) && dims_are(dram_table, 1) && hbm_table->dtype == NVDSA_INT32 &&
                dram_table->dtype == NVDSA_INT32,
            NVDSA_ERR_SHAPE, "block tables must be 1-D int32 rows")
      .need(is_half(hbm_kpe) && hbm_ckv->dtype == hbm_kpe->dtype && dram_kpe->dtype == hbm_kpe->dtype &&
                dram_ckv->dtype == hbm_kpe->dtype,
            NVDSA_ERR_DTYPE, "all CKV/KPE tensors must share one 16-bit dtype");
}

void fill_lidu_copy(nvdsa::LiduInitArgs& a, const nvdsa_tensor* slots_row, const nvdsa_tensor* hbm_kpe,
                    const nvdsa_tensor* hbm_ckv, const nvdsa_tensor* dram_kpe, const nvdsa_tensor* dram_ckv,
                    const nvdsa_tensor* hbm_table, const nvdsa_tensor* dram_table, int64_t c, void* workspace,
                    size_t workspace_bytes) {
  a.c = c;
  a.pool_row = static_cast<int32_t*>(slots_row->data);
  a.row_len = sz(slots_row, 0);
  a.hbm_kpe = hbm_kpe->data;
  a.hbm_ckv = hbm_ckv->data;
  a.dram_kpe = dram_kpe->data;
  a.dram_ckv = dram_ckv->data;
  a.hbm_table = static_cast<const int32_t*>(hbm_table->data);
  a.hbm_cols = sz(hbm_table, 0);
  a.hbm_blocks = std::min(sz(hbm_kpe, 0), sz(hbm_ckv, 0));
  a.dram_table = static_cast<const int32_t*>(dram_table->data);
  a.dram_cols = sz(dram_table, 0);
  a.dram_blocks = std::min(sz(dram_kpe, 0), sz(dram_ckv, 0));
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
}

}  // namespace

size_t nvdsa_initialize_lidu_row_workspace_size(int64_t source_capacity) {
  if (source_capacity < 0) return 0;
  return nvdsa::lidu_init_workspace_bytes(source_capacity);
}

int nvdsa_initialize_lidu_row(const nvdsa_tensor* query, const nvdsa_tensor* weights,
                              const nvdsa_tensor* index_cache, const nvdsa_tensor* index_block_table,
                              int64_t candidate_len, int64_t cache_tokens, const nvdsa_tensor* cache_slots_row,
                              const nvdsa_tensor* hbm_kpe, const nvdsa_tensor* hbm_ckv, const nvdsa_tensor* dram_kpe,
                              const nvdsa_tensor* dram_ckv, const nvdsa_tensor* hbm_block_table,
                              const nvdsa_tensor* dram_block_table, int64_t block_size, void* workspace,
                              size_t workspace_bytes, void* stream) {
  const nvdsa_tensor* const all[] = {query,   weights, index_cache, index_block_table, cache_slots_row,
                                     hbm_kpe, hbm_ckv, dram_kpe,    dram_ckv,          hbm_block_table,
                                     dram_block_table};
  if (!all_nonnull(all)) return fail(NVDSA_ERR_ARG, "initialize_lidu_row: null tensor argument");
  if (cache_tokens <= 0) {  // no cache budget: nothing to initialise
    g_last_error.clear();
    return NVDSA_OK;
  }
  char msg[160];
  // The reference's argument errors (dsa_offload_ops.py:280-294), then this
  // implementation's limits.
  if (cache_tokens < nvdsa::kTopK) {
    std::snprintf(msg, sizeof(msg), "LIDU nonzero cache budget must be >= %d, got %lld.", nvdsa::kTopK,
                  static_cast<long long>(cache_tokens));
    return fail(NVDSA_ERR_ARG, msg);
  }
  if (candidate_len < cache_tokens) {
    std::snprintf(msg, sizeof(msg), "LIDU cache budget %lld exceeds source length %lld.",
                  static_cast<long long>(cache_tokens), static_cast<long long>(candidate_len));
    return fail(NVDSA_ERR_ARG, msg);
  }
  if (block_size <= 0 || candidate_len % block_size) return fail(NVDSA_ERR_ARG, "LIDU source must consist only of complete blocks.");
  Check c("initialize_lidu_row");
  c.need(block_size == nvdsa::kBlock, NVDSA_ERR_ARG, "block_size must be 128")
      .need(cache_tokens <= nvdsa::kMaxCacheTokens, NVDSA_ERR_ARG, "cache budget must be <= 16383 slots")
      .need(candidate_len <= nvdsa::kMaxActualSeqLen, NVDSA_ERR_ARG, "candidate_len must be < 2^21")
      .need((dims_are(query, 2) || (dims_are(query, 3) && sz(query, 0) == 1)) && sz(query, query->ndim - 1) == 128,
            NVDSA_ERR_SHAPE, "query must be [N, 128]")
      .need(sz(query, query->ndim - 2) == 32 || sz(query, query->ndim - 2) == 64, NVDSA_ERR_SHAPE,
            "index head count must be 32 or 64")
      .need(numel(weights) == sz(query, query->ndim - 2), NVDSA_ERR_SHAPE, "weights must hold one value per head")
      .need(dims_are(index_cache, 4) && sz(index_cache, 1) == 128 && sz(index_cache, 2) == 1 &&
                sz(index_cache, 3) == 128,
            NVDSA_ERR_SHAPE, "index cache must be [blocks, 128, 1, 128]")
      .need(dims_are(index_block_table, 1) && index_block_table->dtype == NVDSA_INT32, NVDSA_ERR_SHAPE,
            "index_block_table must be a 1-D int32 row")
      .need(candidate_len <= sz(index_block_table, 0) * 128, NVDSA_ERR_SHAPE,
            "candidate_len exceeds the index block table")
      .need(is_half(query) && weights->dtype == query->dtype && index_cache->dtype == query->dtype, NVDSA_ERR_DTYPE,
            "query, weights and index cache must share one 16-bit dtype");
  if (c.ok()) check_lidu_copy(c, cache_slots_row, hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, hbm_block_table, dram_block_table);
  if (c.ok()) {
    c.need(candidate_len <= sz(cache_slots_row, 0), NVDSA_ERR_SHAPE, "cache_slots_row is shorter than the source");
    check_common(c, all, query->device, dram_kpe, dram_ckv);
    c.need(aligned16(query) && aligned16(index_cache) && aligned16(hbm_kpe) && aligned16(hbm_ckv) &&
               aligned16(dram_kpe) && aligned16(dram_ckv),
           NVDSA_ERR_LAYOUT, "query, index cache and KV caches must be 16-byte aligned");
    c.need(workspace != nullptr && workspace_bytes >= nvdsa::lidu_init_workspace_bytes(sz(cache_slots_row, 0)),
           NVDSA_ERR_WORKSPACE, "workspace too small");
  }
  if (!c.ok()) return c.finish();
  nvdsa::LiduInitArgs a{};
  a.query = query->data;
  a.weights = weights->data;
  a.key_cache = index_cache->data;
  a.index_table = static_cast<const int32_t*>(index_block_table->data);
  a.index_cols = sz(index_block_table, 0);
  a.key_blocks = sz(index_cache, 0);
  a.heads = sz(query, query->ndim - 2);
  a.elem = elem_of(query);
  a.n = candidate_len;
  fill_lidu_copy(a, cache_slots_row, hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, hbm_block_table, dram_block_table,
                 cache_tokens, workspace, workspace_bytes);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = nvdsa::launch_lidu_init(a, st);
  if (e == hipSuccess) e = nvdsa::launch_lidu_copy(a, st);
  return launch_status(e, "initialize_lidu_row");
}

int nvdsa_initialize_lidu_row_shared(const nvdsa_tensor* cache_slots_row, int64_t cache_tokens,
                                     const nvdsa_tensor* hbm_kpe, const nvdsa_tensor* hbm_ckv,
                                     const nvdsa_tensor* dram_kpe, const nvdsa_tensor* dram_ckv,
                                     const nvdsa_tensor* hbm_block_table, const nvdsa_tensor* dram_block_table,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  const nvdsa_tensor* const all[] = {cache_slots_row, hbm_kpe,         hbm_ckv,         dram_kpe,
                                     dram_ckv,        hbm_block_table, dram_block_table};
  if (!all_nonnull(all)) return fail(NVDSA_ERR_ARG, "initialize_lidu_row_shared: null tensor argument");
  if (cache_tokens <= 0) {
    g_last_error.clear();
    return NVDSA_OK;
  }
  Check c("initialize_lidu_row_shared");
  c.need(cache_tokens <= nvdsa::kMaxCacheTokens, NVDSA_ERR_ARG, "cache budget must be <= 16383 slots");
  check_lidu_copy(c, cache_slots_row, hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, hbm_block_table, dram_block_table);
  if (c.ok()) {
    check_common(c, all, hbm_kpe->device, dram_kpe, dram_ckv);
    c.need(aligned16(hbm_kpe) && aligned16(hbm_ckv) && aligned16(dram_kpe) && aligned16(dram_ckv), NVDSA_ERR_LAYOUT,
           "KV caches must be 16-byte aligned")
        .need(workspace != nullptr && workspace_bytes >= nvdsa::lidu_init_workspace_bytes(sz(cache_slots_row, 0)),
              NVDSA_ERR_WORKSPACE, "workspace too small");
  }
  if (!c.ok()) return c.finish();
  nvdsa::LiduInitArgs a{};
  fill_lidu_copy(a, cache_slots_row, hbm_kpe, hbm_ckv, dram_kpe, dram_ckv, hbm_block_table, dram_block_table,
                 cache_tokens, workspace, workspace_bytes);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = nvdsa::launch_lidu_shared_list(a, st);
  // The reference checks the cached count before copying (its nonzero()
  // synchronises too): read the count the list kernel wrote.
  int32_t found = -1;
  if (e == hipSuccess) e = hipMemcpyAsync(&found, nvdsa::lidu_list_count(a), sizeof(found), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) return launch_status(e, "initialize_lidu_row_shared");
  if (found != cache_tokens) {
    char msg[160];
    std::snprintf(msg, sizeof(msg), "Shared layer LIDU initialization found %d cached tokens, expected %lld.", found,
                  static_cast<long long>(cache_tokens));
    return fail(NVDSA_ERR_RUNTIME, msg);
  }
  return launch_status(nvdsa::launch_lidu_copy(a, st), "initialize_lidu_row_shared");
}

// ------------------------------------------------------------------------
size_t nvdsa_sparse_tail_attention_workspace_size(int64_t query_rows, int64_t heads, int64_t max_kv_tokens) {
  if (query_rows < 0 || heads < 0 || max_kv_tokens < 0) return 0;
  return nvdsa::sfa_workspace_bytes(query_rows, heads, max_kv_tokens);
}

namespace {

// Shared checks of the four attention entry points.  `rows_per_request` is
// 1 (MTP0) or 4 (MTP3); `fused` adds the DRAM-side arguments.
struct AttnTensors {
  const nvdsa_tensor* query_rope;
  const nvdsa_tensor* query;
  const nvdsa_tensor* seq_q;
  const nvdsa_tensor* seq_kv;
  const nvdsa_tensor* num_cache;
  const nvdsa_tensor* topk_dst;
  const nvdsa_tensor* hbm_table;
  const nvdsa_tensor* hbm_kpe;
  const nvdsa_tensor* hbm_ckv;
  const nvdsa_tensor* out;
};

void check_attention(Check& c, const AttnTensors& t, int64_t rows_per_request, bool kv_4d_required,
                     bool power_of_two_heads) {
  c.need(dims_are(t.query, 3) && sz(t.query, 2) == 512, NVDSA_ERR_SHAPE, "query must be [B, N, 512]");
  const int64_t heads = sz(t.query, 1);
  if (power_of_two_heads) {
    c.need(heads > 0 && heads <= 128 && (heads & (heads - 1)) == 0, NVDSA_ERR_SHAPE,
           "query local head count must be a power of two in [1, 128]");
  } else {
    c.need(heads >= 1 && heads <= 128, NVDSA_ERR_SHAPE, "query head count must be in [1, 128]");
  }
  c.need(sz(t.query, 0) >= (rows_per_request == 1 ? 0 : 1), NVDSA_ERR_SHAPE, "query batch must be non-empty");
  const int64_t R = sz(t.query, 0);
  const int64_t B = rows_per_request == 1 ? R : sz(t.num_cache, 0);
  if (rows_per_request != 1) {
    c.need(dims_are(t.num_cache, 1) && B > 0, NVDSA_ERR_SHAPE, "cache_tokens must be [B] with B > 0")
        .need(R == B * rows_per_request, NVDSA_ERR_SHAPE, "requires exactly four packed queries per request");
  }
  (void)kv_4d_required;
  c.need(dims_are(t.hbm_ckv, 4) && sz(t.hbm_ckv, 1) == 128 && sz(t.hbm_ckv, 2) == 1 && sz(t.hbm_ckv, 3) == 512,
         NVDSA_ERR_SHAPE, "key must be [blocks, 128, 1, 512]")
      .need(dims_are(t.query_rope, 3) && sz(t.query_rope, 0) == R && sz(t.query_rope, 1) == heads &&
                sz(t.query_rope, 2) == 64,
            NVDSA_ERR_SHAPE, "query_rope must be [B, N, 64]")
      .need(dims_are(t.hbm_kpe, 4) && sz(t.hbm_kpe, 0) == sz(t.hbm_ckv, 0) && sz(t.hbm_kpe, 1) == 128 &&
                sz(t.hbm_kpe, 2) == 1 && sz(t.hbm_kpe, 3) == 64,
            NVDSA_ERR_SHAPE, "key_rope must be [blocks, 128, 1, 64]")
      .need(dims_are(t.topk_dst, 3) && sz(t.topk_dst, 0) == R && sz(t.topk_dst, 1) == 1 &&
                sz(t.topk_dst, 2) == 2048,
            NVDSA_ERR_SHAPE, "sparse_slots must be [B, 1, 2048]")
      .need(dims_are(t.num_cache, 1) && sz(t.num_cache, 0) == B, NVDSA_ERR_SHAPE, "cache_tokens must be [B]")
      .need(dims_are(t.hbm_table, 2) && sz(t.hbm_table, 0) == B && sz(t.hbm_table, 1) > 0, NVDSA_ERR_SHAPE,
            "block_table must be [B, max_blocks] with max_blocks > 0")
      .need(dims_are(t.seq_q, 1) && sz(t.seq_q, 0) == B && dims_are(t.seq_kv, 1) && sz(t.seq_kv, 0) == B,
            NVDSA_ERR_SHAPE, "actual sequence lengths must be [B]")
      .need(same_shape(t.out, t.query), NVDSA_ERR_SHAPE, "attention_out must have the same shape as query");
  if (!c.ok()) return;
  const int dtype = t.query->dtype;
  c.need(dtype == NVDSA_FLOAT16 || dtype == NVDSA_BFLOAT16, NVDSA_ERR_DTYPE, "supports fp16 or bf16")
      .need(t.hbm_ckv->dtype == dtype && t.query_rope->dtype == dtype && t.hbm_kpe->dtype == dtype &&
                t.out->dtype == dtype,
            NVDSA_ERR_DTYPE, "all floating-point inputs must have the same dtype")
      .need(t.topk_dst->dtype == NVDSA_INT32 && t.num_cache->dtype == NVDSA_INT32 &&
                t.hbm_table->dtype == NVDSA_INT32 && t.seq_q->dtype == NVDSA_INT32 &&
                t.seq_kv->dtype == NVDSA_INT32,
            NVDSA_ERR_DTYPE, "sparse slots, cache metadata, tables and lengths must be int32");
}

void fill_attention_args(nvdsa::SfaArgs& a, const AttnTensors& t, int64_t rows_per_request, double scale,
                         void* workspace, size_t workspace_bytes) {
  a.query_rope = t.query_rope->data;
  a.query = t.query->data;
  a.seq_kv = static_cast<const int32_t*>(t.seq_kv->data);
  a.num_cache = static_cast<const int32_t*>(t.num_cache->data);
  a.topk_dst = static_cast<const int32_t*>(t.topk_dst->data);
  a.hbm_table = static_cast<const int32_t*>(t.hbm_table->data);
  a.hbm_kpe = t.hbm_kpe->data;
  a.hbm_ckv = t.hbm_ckv->data;
  a.out = t.out->data;
  a.batch = sz(t.query, 0) / rows_per_request;
  a.rows_per_request = rows_per_request;
  a.heads = sz(t.query, 1);
  a.hbm_cols = sz(t.hbm_table, 1);
  a.hbm_blocks = sz(t.hbm_ckv, 0);
  a.scale = static_cast<float>(scale);
  a.elem = elem_of(t.query);
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
}

int run_attention(const char* op, const AttnTensors& t, int64_t rows_per_request, bool power_of_two_heads,
                  double scale, void* workspace, size_t workspace_bytes, void* stream) {
  const nvdsa_tensor* const all[] = {t.query_rope, t.query,   t.seq_q,   t.seq_kv,  t.num_cache,
                                     t.topk_dst,   t.hbm_table, t.hbm_kpe, t.hbm_ckv, t.out};
  if (!all_nonnull(all)) return fail(NVDSA_ERR_ARG, "sparse_tail_attention: null tensor argument");
  Check c(op);
  check_attention(c, t, rows_per_request, true, power_of_two_heads);
  if (c.ok()) {
    check_common(c, all, t.query->device);
    c.need(aligned16(t.query) && aligned16(t.query_rope) && aligned16(t.hbm_ckv) && aligned16(t.hbm_kpe) &&
               aligned16(t.out),
           NVDSA_ERR_LAYOUT, "query, KV caches and output must be 16-byte aligned");
  }
  if (!c.ok()) return c.finish();
  nvdsa::SfaArgs a{};
  fill_attention_args(a, t, rows_per_request, scale, workspace, workspace_bytes);
  if (a.batch == 0) return NVDSA_OK;
  if (workspace == nullptr || workspace_bytes < nvdsa::sfa_workspace_bytes(sz(t.query, 0), a.heads, 0))
    return fail(NVDSA_ERR_WORKSPACE, "sparse_tail_attention: workspace too small");
  return launch_status(nvdsa::launch_sparse_tail_attention(a, static_cast<hipStream_t>(stream)), op);
}

}  // namespace

int nvdsa_sparse_tail_attention(const nvdsa_tensor* query_rope, const nvdsa_tensor* query,
                                const nvdsa_tensor* actual_seq_lengths_query,
                                const nvdsa_tensor* actual_seq_lengths_kv, const nvdsa_tensor* num_cache_tokens,
                                const nvdsa_tensor* topk_dst_slots, const nvdsa_tensor* hbm_block_table,
                                const nvdsa_tensor* hbm_k_rope, const nvdsa_tensor* hbm_kv_cache,
                                double scale_value, const nvdsa_tensor* attention_out, void* workspace,
                                size_t workspace_bytes, void* stream) {
  // ops/sparse_tail_attention/sparse_tail_attention_torch_adpt.h:17-88
  AttnTensors t{query_rope,     query,          actual_seq_lengths_query, actual_seq_lengths_kv,
                num_cache_tokens, topk_dst_slots, hbm_block_table,        hbm_k_rope,
                hbm_kv_cache,   attention_out};
  return run_attention("sparse_tail_attention", t, 1, true, scale_value, workspace, workspace_bytes, stream);
}

int nvdsa_sparse_tail_attention_mtp(const nvdsa_tensor* query_rope, const nvdsa_tensor* query,
                                    const nvdsa_tensor* actual_seq_lengths_query,
                                    const nvdsa_tensor* actual_seq_lengths_kv,
                                    const nvdsa_tensor* num_cache_tokens, const nvdsa_tensor* topk_dst_slots,
                                    const nvdsa_tensor* hbm_block_table, const nvdsa_tensor* hbm_k_rope,
                                    const nvdsa_tensor* hbm_kv_cache, double scale_value,
                                    const nvdsa_tensor* attention_out, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  // ops/sparse_tail_attention_mtp/sparse_tail_attention_mtp_torch_adpt.h:18-96
  AttnTensors t{query_rope,     query,          actual_seq_lengths_query, actual_seq_lengths_kv,
                num_cache_tokens, topk_dst_slots, hbm_block_table,        hbm_k_rope,
                hbm_kv_cache,   attention_out};
  return run_attention("sparse_tail_attention_mtp", t, nvdsa::kMtpQueries, true, scale_value, workspace,
                       workspace_bytes, stream);
}

namespace {

int run_fused(const char* op, const AttnTensors& t, int64_t rows_per_request, const nvdsa_tensor* topk_src,
              const nvdsa_tensor* miss_src, const nvdsa_tensor* miss_dst, const nvdsa_tensor* miss_counts,
              const nvdsa_tensor* dram_table, const nvdsa_tensor* dram_kpe, const nvdsa_tensor* dram_ckv,
              double scale, void* workspace, size_t workspace_bytes, void* stream) {
  const bool mtp = rows_per_request != 1;
  const nvdsa_tensor* const base[] = {t.query_rope, t.query,   t.seq_q,   t.seq_kv,  t.num_cache, t.topk_dst,
                                      t.hbm_table,  t.hbm_kpe, t.hbm_ckv, t.out,     topk_src,    miss_counts,
                                      dram_table,   dram_kpe,  dram_ckv};
  if (!all_nonnull(base) || (mtp && (!miss_src || !miss_dst)))
    return fail(NVDSA_ERR_ARG, "fused_copy_sfa: null tensor argument");
  Check c(op);
  check_attention(c, t, rows_per_request, true, false);
  const int64_t R = sz(t.query, 0);
  const int64_t B = mtp ? sz(t.num_cache, 0) : R;
  if (c.ok()) {
    c.need(R >= 1, NVDSA_ERR_SHAPE, "query must have B >= 1");
    // ops/fused_copy_sfa/fused_copy_sfa_torch_adpt.h:44-86 and
    // ops/fused_copy_sfa_mtp/fused_copy_sfa_mtp_torch_adpt.h:56-108
    c.need(dims_are(dram_ckv, 3) && sz(dram_ckv, 1) == 128 && sz(dram_ckv, 2) == 512, NVDSA_ERR_SHAPE,
           "DRAM CKV must be [blocks, 128, 512]")
        .need(dims_are(dram_kpe, 3) && sz(dram_kpe, 0) == sz(dram_ckv, 0) && sz(dram_kpe, 1) == 128 &&
                  sz(dram_kpe, 2) == 64,
              NVDSA_ERR_SHAPE, "DRAM KPE must be [blocks, 128, 64]")
        .need(dims_are(dram_table, 2) && sz(dram_table, 0) == B && (mtp ? sz(dram_table, 1) > 0 : true),
              NVDSA_ERR_SHAPE, "DRAM block table must be [B, max_blocks]")
        .need(dims_are(miss_counts, 1) && sz(miss_counts, 0) == B, NVDSA_ERR_SHAPE, "miss_counts must be [B]");
    if (mtp) {
      c.need(same_shape(topk_src, t.topk_dst), NVDSA_ERR_SHAPE, "topk_source_ids must match topk_slots")
          .need(dims_are(miss_src, 2) && sz(miss_src, 0) == B && sz(miss_src, 1) == nvdsa::kUnionCap &&
                    same_shape(miss_dst, miss_src),
                NVDSA_ERR_SHAPE, "compact union misses must be [B, 8192]");
    } else {
      c.need(dims_are(topk_src, 2) && sz(topk_src, 0) == B && sz(topk_src, 1) == 2048, NVDSA_ERR_SHAPE,
             "topk_src_ids must be [B, 2048]");
    }
    c.need(dram_ckv->dtype == t.query->dtype && dram_kpe->dtype == t.query->dtype, NVDSA_ERR_DTYPE,
           "all fused floating-point inputs must share one dtype")
        .need(topk_src->dtype == NVDSA_INT32 && miss_counts->dtype == NVDSA_INT32 &&
                  dram_table->dtype == NVDSA_INT32 &&
                  (!mtp || (miss_src->dtype == NVDSA_INT32 && miss_dst->dtype == NVDSA_INT32)),
              NVDSA_ERR_DTYPE, "all fused metadata inputs must be int32");
  }
  if (c.ok()) {
    check_common(c, base, t.query->device, dram_kpe, dram_ckv);
    if (mtp) {
      const nvdsa_tensor* const extra[] = {miss_src, miss_dst};
      check_common(c, extra, t.query->device);
    }
    c.need(aligned16(t.query) && aligned16(t.query_rope) && aligned16(t.hbm_ckv) && aligned16(t.hbm_kpe) &&
               aligned16(t.out) && aligned16(dram_ckv) && aligned16(dram_kpe),
           NVDSA_ERR_LAYOUT, "query, KV caches and output must be 16-byte aligned");
  }
  if (!c.ok()) return c.finish();
  nvdsa::SfaArgs a{};
  fill_attention_args(a, t, rows_per_request, scale, workspace, workspace_bytes);
  if (workspace == nullptr || workspace_bytes < nvdsa::sfa_workspace_bytes(R, a.heads, 0))
    return fail(NVDSA_ERR_WORKSPACE, "fused_copy_sfa: workspace too small");
  a.copy_src = static_cast<const int32_t*>(mtp ? miss_src->data : topk_src->data);
  a.copy_dst = static_cast<const int32_t*>(mtp ? miss_dst->data : t.topk_dst->data);
  a.copy_counts = static_cast<const int32_t*>(miss_counts->data);
  a.copy_cap = mtp ? nvdsa::kUnionCap : nvdsa::kTopK;
  a.key_src = mtp ? static_cast<const int32_t*>(topk_src->data) : nullptr;
  a.dram_table = static_cast<const int32_t*>(dram_table->data);
  a.dram_kpe = dram_kpe->data;
  a.dram_ckv = dram_ckv->data;
  a.dram_cols = sz(dram_table, 1);
  a.dram_blocks = sz(dram_ckv, 0);
  return launch_status(nvdsa::launch_fused_copy_sfa(a, static_cast<hipStream_t>(stream)), op);
}

}  // namespace

int nvdsa_fused_copy_sfa(const nvdsa_tensor* query_rope, const nvdsa_tensor* query,
                         const nvdsa_tensor* actual_seq_lengths_query, const nvdsa_tensor* actual_seq_lengths_kv,
                         const nvdsa_tensor* num_cache_tokens, const nvdsa_tensor* topk_dst_slots,
                         const nvdsa_tensor* topk_src_ids, const nvdsa_tensor* miss_counts,
                         const nvdsa_tensor* hbm_block_table, const nvdsa_tensor* dram_block_table,
                         const nvdsa_tensor* hbm_k_rope, const nvdsa_tensor* hbm_kv_cache,
                         const nvdsa_tensor* dram_k_rope, const nvdsa_tensor* dram_kv_cache, double scale_value,
                         const nvdsa_tensor* attention_out, void* workspace, size_t workspace_bytes,
                         void* stream) {
  AttnTensors t{query_rope,     query,          actual_seq_lengths_query, actual_seq_lengths_kv,
                num_cache_tokens, topk_dst_slots, hbm_block_table,        hbm_k_rope,
                hbm_kv_cache,   attention_out};
  return run_fused("fused_copy_sfa", t, 1, topk_src_ids, nullptr, nullptr, miss_counts, dram_block_table,
                   dram_k_rope, dram_kv_cache, scale_value, workspace, workspace_bytes, stream);
}

int nvdsa_fused_copy_sfa_mtp(const nvdsa_tensor* query_rope, const nvdsa_tensor* query,
                             const nvdsa_tensor* actual_seq_lengths_query,
                             const nvdsa_tensor* actual_seq_lengths_kv, const nvdsa_tensor* num_cache_tokens,
                             const nvdsa_tensor* topk_dst_slots, const nvdsa_tensor* topk_src_ids,
                             const nvdsa_tensor* miss_src_ids, const nvdsa_tensor* miss_dst_slots,
                             const nvdsa_tensor* miss_counts, const nvdsa_tensor* hbm_block_table,
                             const nvdsa_tensor* dram_block_table, const nvdsa_tensor* hbm_k_rope,
                             const nvdsa_tensor* hbm_kv_cache, const nvdsa_tensor* dram_k_rope,
                             const nvdsa_tensor* dram_kv_cache, double scale_value,
                             const nvdsa_tensor* attention_out, void* workspace, size_t workspace_bytes,
                             void* stream) {
  AttnTensors t{query_rope,     query,          actual_seq_lengths_query, actual_seq_lengths_kv,
                num_cache_tokens, topk_dst_slots, hbm_block_table,        hbm_k_rope,
                hbm_kv_cache,   attention_out};
  return run_fused("fused_copy_sfa_mtp", t, nvdsa::kMtpQueries, topk_src_ids, miss_src_ids, miss_dst_slots,
                   miss_counts, dram_block_table, dram_k_rope, dram_kv_cache, scale_value, workspace,
                   workspace_bytes, stream);
}

// ------------------------------------------------------------------------
int nvdsa_dsa_indexer_query_rope_inplace(const nvdsa_tensor* q_inout, const nvdsa_tensor* cos,
                                         const nvdsa_tensor* sin, int64_t rope_dim, void* stream) {
  const nvdsa_tensor* const all[] = {q_inout, cos, sin};
  if (!all_nonnull(all)) return fail(NVDSA_ERR_ARG, "dsa_indexer_query_rope_inplace: null tensor argument");
  Check c("dsa_indexer_query_rope_inplace");
  // ops/dsa_indexer_project/dsa_indexer_project_torch_adpt.h:31-90, in its order.
  c.need(dims_are(q_inout, 3), NVDSA_ERR_SHAPE, "q_inout rank mismatch.")
      .need(q_inout->contiguous == 1, NVDSA_ERR_LAYOUT, "q_inout must be contiguous.")
      .need(cos->dtype == q_inout->dtype, NVDSA_ERR_DTYPE, "cos dtype mismatch.")
      .need(dims_are(cos, 4), NVDSA_ERR_SHAPE, "cos rank mismatch.")
      .need(cos->contiguous == 1, NVDSA_ERR_LAYOUT, "cos must be contiguous.")
      .need(sin->dtype == q_inout->dtype, NVDSA_ERR_DTYPE, "sin dtype mismatch.")
      .need(dims_are(sin, 4), NVDSA_ERR_SHAPE, "sin rank mismatch.")
      .need(sin->contiguous == 1, NVDSA_ERR_LAYOUT, "sin must be contiguous.")
      .need(is_half(q_inout), NVDSA_ERR_DTYPE, "q_inout must be float16 or bfloat16.")
      .need(q_inout->device == cos->device && q_inout->device == sin->device && q_inout->device >= 0,
            NVDSA_ERR_DEVICE, "q_inout, cos and sin must be on the same GPU.");
  if (c.ok()) {
    const int64_t T = sz(q_inout, 0), H = sz(q_inout, 1), D = sz(q_inout, 2);
    c.need(T > 0 && H > 0 && D > 0, NVDSA_ERR_SHAPE, "q_inout must be non-empty.")
        .need(sz(cos, 0) == T && sz(sin, 0) == T, NVDSA_ERR_SHAPE, "cos/sin token dimension mismatch.")
        .need(numel(cos) >= T * rope_dim && numel(sin) >= T * rope_dim, NVDSA_ERR_SHAPE,
              "cos/sin storage is smaller than num_tokens * rope_dim.")
        .need(rope_dim > 0 && rope_dim <= D && rope_dim % 16 == 0, NVDSA_ERR_ARG,
              "rope_dim must be positive, no larger than head_dim, and aligned to 16.")
        .need(D <= 256 && D % 16 == 0 && H <= 128, NVDSA_ERR_SHAPE,
              "query RoPE requires head_dim <= 256 aligned to 16 and n_head <= 128.")
        .need(has_data(q_inout) && has_data(cos) && has_data(sin), NVDSA_ERR_ARG, "null data pointer")
        .need(aligned4(q_inout) && aligned4(cos) && aligned4(sin), NVDSA_ERR_LAYOUT,
              "q_inout, cos and sin must be 4-byte aligned");
  }
  if (!c.ok()) return c.finish();
  nvdsa::RopeArgs a{};
  a.q = q_inout->data;
  a.cos = cos->data;
  a.sin = sin->data;
  a.heads = sz(q_inout, 1);
  a.rows = sz(q_inout, 0) * a.heads;
  a.head_dim = sz(q_inout, 2);
  a.rope_dim = rope_dim;
  a.elem = elem_of(q_inout);
  return launch_status(nvdsa::launch_indexer_rope(a, static_cast<hipStream_t>(stream)),
                       "dsa_indexer_query_rope_inplace");
}

int nvdsa_dsa_indexer_project_query_only(const nvdsa_tensor* hidden_states, const nvdsa_tensor* q_c,
                                         const nvdsa_tensor* cos, const nvdsa_tensor* sin,
                                         const nvdsa_tensor* wq_b_weight, const nvdsa_tensor* weights_proj_weight,
                                         const nvdsa_tensor* q_index_out, const nvdsa_tensor* index_weights_out,
                                         int64_t n_head, int64_t head_dim, int64_t rope_dim, double score_scale,
                                         void* stream) {
  const nvdsa_tensor* const req[] = {hidden_states, q_c, cos, sin, wq_b_weight, q_index_out};
  if (!all_nonnull(req)) return fail(NVDSA_ERR_ARG, "dsa_indexer_project_query_only: null tensor argument");
  if ((weights_proj_weight == nullptr) != (index_weights_out == nullptr))
    return fail(NVDSA_ERR_ARG,
                "dsa_indexer_project_query_only: weights_proj_weight and index_weights_out go together");
  const bool with_w = weights_proj_weight != nullptr;
  const int64_t T = sz(hidden_states, 0);
  // The reference's output checks (nanovllm/models/dsa_indexer_project.py:316-319).
  if (!(dims_are(q_index_out, 3) && sz(q_index_out, 0) == T && sz(q_index_out, 1) == n_head &&
        sz(q_index_out, 2) == head_dim)) {
    const std::string m = "q_index_out shape must be (" + std::to_string(T) + ", " + std::to_string(n_head) + ", " +
                          std::to_string(head_dim) + "), got " + shape_str(q_index_out);
    return fail(NVDSA_ERR_SHAPE, m.c_str());
  }
  if (with_w && !(dims_are(index_weights_out, 2) && sz(index_weights_out, 0) == T && sz(index_weights_out, 1) == n_head)) {
    const std::string m = "index_weights_out shape must be (" + std::to_string(T) + ", " + std::to_string(n_head) +
                          "), got " + shape_str(index_weights_out);
    return fail(NVDSA_ERR_SHAPE, m.c_str());
  }
  Check c("dsa_indexer_project_query_only");
  // This implementation's layout limits (projection shapes of
  // nanovllm/models/dsa_indexer_project.py:93-104 and the GLM indexer,
  // nanovllm/models/glm_mla.py:205-219).
  const int64_t kc = nvdsa::indexer_k_chunk();
  c.need(dims_are(hidden_states, 2) && dims_are(q_c, 2) && sz(q_c, 0) == T, NVDSA_ERR_SHAPE,
         "hidden_states and q_c must be [tokens, features] with one row per token")
      .need(dims_are(wq_b_weight, 2) && sz(wq_b_weight, 0) == n_head * head_dim && sz(wq_b_weight, 1) == sz(q_c, 1),
            NVDSA_ERR_SHAPE, "wq_b_weight must be [n_head * head_dim, q_lora_rank]")
      .need(!with_w || (dims_are(weights_proj_weight, 2) && sz(weights_proj_weight, 0) == n_head &&
                        sz(weights_proj_weight, 1) == sz(hidden_states, 1)),
            NVDSA_ERR_SHAPE, "weights_proj_weight must be [n_head, hidden_size]")
      .need(n_head > 0 && n_head % 16 == 0 && head_dim > 0 && head_dim % 16 == 0, NVDSA_ERR_ARG,
            "n_head and head_dim must be positive multiples of 16")
      .need(rope_dim > 0 && rope_dim <= head_dim && rope_dim % 2 == 0, NVDSA_ERR_ARG,
            "rope_dim must be positive, even and no larger than head_dim")
      .need(sz(q_c, 1) > 0 && sz(q_c, 1) % kc == 0, NVDSA_ERR_SHAPE, "q_lora_rank must be a positive multiple of 256")
      .need(!with_w || (sz(hidden_states, 1) > 0 && sz(hidden_states, 1) % 512 == 0), NVDSA_ERR_SHAPE,
            "hidden_size must be a positive multiple of 512")
      .need(is_half(hidden_states) && q_c->dtype == hidden_states->dtype && wq_b_weight->dtype == hidden_states->dtype &&
                cos->dtype == hidden_states->dtype && sin->dtype == hidden_states->dtype &&
                q_index_out->dtype == hidden_states->dtype &&
                (!with_w || (weights_proj_weight->dtype == hidden_states->dtype &&
                             index_weights_out->dtype == hidden_states->dtype)),
            NVDSA_ERR_DTYPE, "all tensors must share one 16-bit dtype (fp16 or bf16)")
      .need(T == 0 || (numel(cos) % T == 0 && numel(sin) == numel(cos) && numel(cos) / T >= rope_dim), NVDSA_ERR_SHAPE,
            "cos/sin must hold at least rope_dim values per token");
  if (c.ok()) {
    check_common(c, req, hidden_states->device);
    if (with_w) {
      const nvdsa_tensor* const w2[] = {weights_proj_weight, index_weights_out};
      check_common(c, w2, hidden_states->device);
    }
    c.need(hidden_states->device >= 0, NVDSA_ERR_DEVICE, "tensors must be on a GPU")
        .need(aligned16(hidden_states) && aligned16(q_c) && aligned16(wq_b_weight) &&
                  (!with_w || aligned16(weights_proj_weight)),
              NVDSA_ERR_LAYOUT, "inputs and projection weights must be 16-byte aligned")
        .need(aligned4(q_index_out) && aligned4(cos) && aligned4(sin) && (!with_w || aligned4(index_weights_out)),
              NVDSA_ERR_LAYOUT, "outputs, cos and sin must be 4-byte aligned");
  }
  if (!c.ok()) return c.finish();
  nvdsa::IndexerArgs a{};
  a.hidden = hidden_states->data;
  a.q_c = q_c->data;
  a.cos = cos->data;
  a.sin = sin->data;
  a.wq_b = wq_b_weight->data;
  a.w_proj = with_w ? weights_proj_weight->data : nullptr;
  a.q_out = q_index_out->data;
  a.w_out = with_w ? index_weights_out->data : nullptr;
  a.tokens = T;
  a.hid = sz(hidden_states, 1);
  a.rank = sz(q_c, 1);
  a.heads = n_head;
  a.head_dim = head_dim;
  a.rope_dim = rope_dim;
  a.cos_stride = T > 0 ? numel(cos) / T : 0;
  a.score_scale = static_cast<float>(score_scale);
  a.elem = elem_of(hidden_states);
  return launch_status(nvdsa::launch_indexer_project(a, static_cast<hipStream_t>(stream)),
                       "dsa_indexer_project_query_only");
}

// ------------------------------------------------------------------------
int nvdsa_persist_prefill_blocks(const nvdsa_tensor* hbm_kv_cache, const nvdsa_tensor* hbm_k_rope,
                                 const nvdsa_tensor* dram_kv_cache, const nvdsa_tensor* dram_k_rope,
                                 const nvdsa_tensor* hbm_block_ids, const nvdsa_tensor* dram_block_ids, void* stream) {
  const nvdsa_tensor* const all[] = {hbm_kv_cache, hbm_k_rope, dram_kv_cache, dram_k_rope, hbm_block_ids,
                                     dram_block_ids};
  if (!all_nonnull(all)) return fail(NVDSA_ERR_ARG, "persist_prefill_blocks: null tensor argument");
  Check c("persist_prefill_blocks");
  auto cache_ok = [](const nvdsa_tensor* t, int64_t width) {
    return (dims_are(t, 3) && sz(t, 1) == 128 && sz(t, 2) == width) ||
           (dims_are(t, 4) && sz(t, 1) == 128 && sz(t, 2) == 1 && sz(t, 3) == width);
  };
  c.need(cache_ok(hbm_kv_cache, 512) && cache_ok(dram_kv_cache, 512), NVDSA_ERR_SHAPE,
         "CKV caches must be [blocks, 128, (1,) 512]")
      .need(cache_ok(hbm_k_rope, 64) && cache_ok(dram_k_rope, 64), NVDSA_ERR_SHAPE,
            "KPE caches must be [blocks, 128, (1,) 64]")
      .need(sz(hbm_kv_cache, 0) == sz(hbm_k_rope, 0) && sz(dram_kv_cache, 0) == sz(dram_k_rope, 0), NVDSA_ERR_SHAPE,
            "CKV and KPE caches must hold the same number of blocks")
      .need(dims_are(hbm_block_ids, 1) && same_shape(hbm_block_ids, dram_block_ids), NVDSA_ERR_SHAPE,
            "block id lists must be rank one and of equal length")
      .need(hbm_block_ids->dtype == NVDSA_INT32 && dram_block_ids->dtype == NVDSA_INT32, NVDSA_ERR_DTYPE,
            "block ids must be int32")
      .need(is_half(hbm_kv_cache) && hbm_k_rope->dtype == hbm_kv_cache->dtype &&
                dram_kv_cache->dtype == hbm_kv_cache->dtype && dram_k_rope->dtype == hbm_kv_cache->dtype,
            NVDSA_ERR_DTYPE, "caches must share one 16-bit dtype");
  if (c.ok()) {
    check_common(c, all, hbm_kv_cache->device, dram_kv_cache, dram_k_rope);
    c.need(hbm_kv_cache->device >= 0, NVDSA_ERR_DEVICE, "HBM caches must be on a GPU")
        .need(aligned16(hbm_kv_cache) && aligned16(hbm_k_rope) && aligned16(dram_kv_cache) && aligned16(dram_k_rope),
              NVDSA_ERR_LAYOUT, "caches must be 16-byte aligned");
  }
  if (!c.ok()) return c.finish();
  nvdsa::PersistArgs a{};
  a.hbm_ckv = hbm_kv_cache->data;
  a.hbm_kpe = hbm_k_rope->data;
  a.dram_ckv = dram_kv_cache->data;
  a.dram_kpe = dram_k_rope->data;
  a.hbm_ids = static_cast<const int32_t*>(hbm_block_ids->data);
  a.dram_ids = static_cast<const int32_t*>(dram_block_ids->data);
  a.count = sz(hbm_block_ids, 0);
  a.hbm_blocks = sz(hbm_kv_cache, 0);
  a.dram_blocks = sz(dram_kv_cache, 0);
  if (a.count * 4 >= kMaxGridThreads / 256) return fail(NVDSA_ERR_SHAPE, "persist_prefill_blocks: too many blocks");
  return launch_status(nvdsa::launch_persist_blocks(a, static_cast<hipStream_t>(stream)), "persist_prefill_blocks");
}

// ------------------------------------------------------------------------
int nvdsa_host_mapped_alloc(size_t bytes, void** host_ptr, void** device_ptr) {
  if (!host_ptr || !device_ptr) return fail(NVDSA_ERR_ARG, "host_mapped_alloc: null output pointer");
  *host_ptr = nullptr;
  *device_ptr = nullptr;
  void* h = nullptr;
  hipError_t e = hipHostMalloc(&h, bytes == 0 ? 1 : bytes, hipHostMallocMapped | hipHostMallocPortable);
  if (e != hipSuccess) {
    g_last_error = std::string("host_mapped_alloc: hipHostMalloc failed: ") + hipGetErrorString(e);
    return NVDSA_ERR_RUNTIME;
  }
  void* d = nullptr;
  e = hipHostGetDevicePointer(&d, h, 0);
  if (e != hipSuccess) {
    (void)hipHostFree(h);
    g_last_error = std::string("host_mapped_alloc: hipHostGetDevicePointer failed: ") + hipGetErrorString(e);
    return NVDSA_ERR_RUNTIME;
  }
  *host_ptr = h;
  *device_ptr = d;
  return NVDSA_OK;
}

int nvdsa_host_mapped_free(void* host_ptr) {
  if (!host_ptr) return NVDSA_OK;
  hipError_t e = hipHostFree(host_ptr);
  if (e != hipSuccess) {
    g_last_error = std::string("host_mapped_free: ") + hipGetErrorString(e);
    return NVDSA_ERR_RUNTIME;
  }
  return NVDSA_OK;
}

}  // extern "C"
