// Host-side launch interface between the C ABI layer (nvdsa_abi.hip) and the
// kernel translation units.  Arguments are already validated by the caller.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace nvdsa {

enum class Elem { kBf16, kF16 };

// Kernel ids of the timing instrumentation (nvdsa_profile_*).
enum KernelId : int {
  kKernScatter = 0,
  kKernLimScore = 1,
  kKernLimHist = 2,
  kKernLimMtpPassA = 3,
  kKernSfaSplit = 4,
  kKernSfaSplitFused = 5,
  kKernSfaCombine = 6,
  kKernLiduInit = 7,
  kKernLiduShared = 8,
  kKernLimThreshold = 9,
  kKernLimMtpVictims = 10,
  kKernLimMtpPassB = 11,
  kKernSfaMtpOverlap = 12,
  kKernSfaSplitCopied = 13,
  kKernIdxProject = 14,
  kKernIdxRope = 15,
  kKernPersist = 16,
  kKernLimClassify = 17,
  kKernLimChunks = 18,
  kKernLimResolve = 19,
  kKernCount = 20
};
// Timing events for the next launch of `kernel_id` when instrumentation is
// on for the calling thread (nvdsa_profile_begin); both null otherwise.
struct ProfEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
ProfEvents prof_events(int kernel_id);

// Launch `kernel` on `stream`.  When timed, the events ride on the kernel's
// own dispatch (hipExtLaunchKernelGGL), so the recorded interval is the
// kernel's execution alone, without the gaps of separate event records.
template <typename F, typename... Args>
inline void launch_kernel(int kernel_id, F kernel, dim3 grid, dim3 block, hipStream_t stream, Args... args) {
  const ProfEvents ev = prof_events(kernel_id);
  if (ev.start != nullptr) {
    hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, ev.start, ev.stop, 0, args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, args...);
  }
}

// ---- scatter_copy --------------------------------------------------------
struct ScatterArgs {
  const int32_t* src_ids;      // [B, cap]
  const int32_t* dst_slots;    // [B, cap]
  const int32_t* copy_counts;  // [B]
  const int32_t* hbm_table;    // [B, hbm_cols]
  const int32_t* dram_table;   // [B, dram_cols]
  void* hbm_kpe;               // [hbm_blocks, 128, 64]
  void* hbm_ckv;               // [hbm_blocks, 128, 512]
  const void* dram_kpe;        // [dram_blocks, 128, 64]
  const void* dram_ckv;        // [dram_blocks, 128, 512]
  int64_t batch;
  int64_t cap;
  int64_t hbm_cols;
  int64_t dram_cols;
  int64_t hbm_blocks;
  int64_t dram_blocks;
};
hipError_t launch_scatter_copy(const ScatterArgs& a, hipStream_t stream);

// ---- fused_li_manage (MTP0 and MTP3) ---------------------------------------
struct LimArgs {
  const void* query;            // [B*Q, H, 128]
  const void* weights;          // [B*Q, H]
  const void* key_cache;        // [key_blocks, 128, 1, 128]
  const int32_t* block_table;   // [B, cols]
  const int32_t* num_candidates;  // [B]
  const int32_t* num_cache;     // [B]
  const int32_t* pool_entries;  // [B]
  int32_t* pool;                // [pool_rows, cols*128]
  int32_t* topk_src;            // [B*Q, 1, 2048]
  int32_t* topk_dst;            // [B*Q, 1, 2048]
  int32_t* miss_src;            // [B, 8192]   (MTP only)
  int32_t* miss_dst;            // [B, 8192]   (MTP only)
  int32_t* miss_counts;         // [B]
  int64_t batch;
  int64_t heads;
  int64_t cols;                 // block-table columns
  int64_t key_blocks;
  int64_t pool_rows;
  int64_t source_capacity;      // cols * 128
  Elem elem;
  void* workspace;
  size_t workspace_bytes;
};
size_t lim_workspace_bytes(int64_t batch, int64_t source_capacity, int queries);
hipError_t launch_fused_li_manage(const LimArgs& a, hipStream_t stream);
hipError_t launch_fused_li_manage_mtp(const LimArgs& a, hipStream_t stream);

// ---- first-decode LIDU initialisation -------------------------------------
struct LiduInitArgs {
  const void* query;            // [H, 128] (one request)
  const void* weights;          // [H]
  const void* key_cache;        // [key_blocks, 128, 1, 128]
  const int32_t* index_table;   // [index_cols]
  int64_t index_cols;
  int64_t key_blocks;
  int64_t heads;
  Elem elem;
  int64_t n;                    // candidate tokens (whole blocks)
  int64_t c;                    // cache budget C
  int32_t* pool_row;            // [row_len] token -> slot
  int64_t row_len;
  void* hbm_kpe;                // [hbm_blocks, 128, 64]
  void* hbm_ckv;                // [hbm_blocks, 128, 512]
  const void* dram_kpe;
  const void* dram_ckv;
  const int32_t* hbm_table;     // [hbm_cols]
  int64_t hbm_cols;
  int64_t hbm_blocks;
  const int32_t* dram_table;    // [dram_cols]
  int64_t dram_cols;
  int64_t dram_blocks;
  void* workspace;
  size_t workspace_bytes;
};
size_t lidu_init_workspace_bytes(int64_t source_capacity);
int64_t lidu_list_capacity();
// Scores, top-C selection, pool row and copy list (then launch_lidu_copy).
hipError_t launch_lidu_init(const LiduInitArgs& a, hipStream_t stream);
// Copy list of a shared layer from the owner's pool row; its length is
// written to lidu_list_count(a) on the device.
hipError_t launch_lidu_shared_list(const LiduInitArgs& a, hipStream_t stream);
const int32_t* lidu_list_count(const LiduInitArgs& a);
// DRAM -> HBM copy of the list (scatter_copy kernel).
hipError_t launch_lidu_copy(const LiduInitArgs& a, hipStream_t stream);

// ---- sparse-tail attention (+ fused copy) --------------------------------
struct SfaArgs {
  const void* query_rope;       // [R, N, 64]
  const void* query;            // [R, N, 512]
  const int32_t* seq_kv;        // [B]
  const int32_t* num_cache;     // [B]
  const int32_t* topk_dst;      // [R, 1, 2048]
  const int32_t* hbm_table;     // [B, hbm_cols]
  void* hbm_kpe;                // [hbm_blocks, 128, 1, 64]
  void* hbm_ckv;                // [hbm_blocks, 128, 1, 512]
  void* out;                    // [R, N, 512]
  int64_t batch;
  int64_t rows_per_request;     // 1 or 4
  int64_t heads;
  int64_t hbm_cols;
  int64_t hbm_blocks;
  float scale;
  Elem elem;
  // fused copy (null when not fused)
  const int32_t* copy_src;      // MTP0: topk_src_ids [B, 2048]; MTP3: miss_src_ids [B, 8192]
  const int32_t* copy_dst;      // MTP0: topk_dst_slots; MTP3: miss_dst_slots
  const int32_t* copy_counts;   // [B]
  int64_t copy_cap;             // 2048 or 8192
  const int32_t* dram_table;    // [B, dram_cols]
  const void* dram_kpe;
  const void* dram_ckv;
  int64_t dram_cols;
  int64_t dram_blocks;
  const int32_t* key_src;       // MTP3 fused: topk_src_ids [R, 2048] (>= 0: a key copied by this call)
  void* workspace;
  size_t workspace_bytes;
};
size_t sfa_workspace_bytes(int64_t query_rows, int64_t heads, int64_t max_kv_tokens);
hipError_t launch_sparse_tail_attention(const SfaArgs& a, hipStream_t stream);
hipError_t launch_fused_copy_sfa(const SfaArgs& a, hipStream_t stream);
// Copies the current device's record of the XCDs the MTP3 overlap kernel's
// copy ([0]) and attention ([1]) workgroups ran on; clears it after the read
// when `reset`.  Synchronises the device.
hipError_t sfa_xcd_roles(uint32_t masks[2], bool reset);
// Whether launches made from now on write that record (off by default).
void sfa_xcd_roles_record(bool on);

// ---- indexer projection (decode query rows and head weights) -------------
struct IndexerArgs {
  const void* hidden;   // [tokens, hid]          16-bit
  const void* q_c;      // [tokens, rank]
  const void* cos;      // [tokens, cos_stride]   (first rope_dim used)
  const void* sin;
  const void* wq_b;     // [heads * head_dim, rank]
  const void* w_proj;   // [heads, hid], or null: weights not computed here
  void* q_out;          // [tokens, heads, head_dim]
  void* w_out;          // [tokens, heads]
  int64_t tokens, hid, rank, heads, head_dim, rope_dim, cos_stride;
  float score_scale;
  Elem elem;
};
// K extents (rank, hid) must be multiples of this.
int64_t indexer_k_chunk();
hipError_t launch_indexer_project(const IndexerArgs& a, hipStream_t stream);

struct RopeArgs {
  void* q;              // [rows = tokens * heads, head_dim], rotated in place
  const void* cos;      // [tokens, rope_dim]
  const void* sin;
  int64_t rows, heads, head_dim, rope_dim;
  Elem elem;
};
hipError_t launch_indexer_rope(const RopeArgs& a, hipStream_t stream);

// ---- prefill -> DRAM persistence ------------------------------------------
struct PersistArgs {
  const void* hbm_ckv;      // [hbm_blocks, 128, 512]
  const void* hbm_kpe;      // [hbm_blocks, 128, 64]
  void* dram_ckv;           // [dram_blocks, 128, 512] (host-mapped)
  void* dram_kpe;           // [dram_blocks, 128, 64]
  const int32_t* hbm_ids;   // [count]
  const int32_t* dram_ids;  // [count]
  int64_t count, hbm_blocks, dram_blocks;
};
hipError_t launch_persist_blocks(const PersistArgs& a, hipStream_t stream);

}  // namespace nvdsa
