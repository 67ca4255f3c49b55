/*
 * nvdsa.h — C ABI of the MI355X (gfx950) DSA stable-decode offload chain.
 *
 * Seven entry points replace the seven torch.library operators that the
 * reference registers under the `nanovllm_dsa` namespace
 * (reference: csrc/nanovllm_ascend_ops/bindings/nanovllm_ops.cpp:645-696);
 * further ones cover the first-decode initialisation, the decode indexer
 * projection that produces the LIM inputs and the prefill -> DRAM
 * persistence of full KV blocks.
 * Each takes its arguments in the same order as the reference schema, as
 * plain tensor descriptors (device address + dtype + shape), plus the HIP
 * stream to launch on.  Every entry point:
 *   - validates shapes / dtypes / layout exactly as the reference adapter's
 *     TORCH_CHECKs do and returns a non-zero nvdsa_status with a message
 *     (nvdsa_last_error) instead of throwing;
 *   - never allocates device memory: scratch space is a caller-provided
 *     workspace whose size the matching *_workspace_size call reports
 *     (the counterpart of aclnnXGetWorkspaceSize + the adapter's workspace
 *     allocation in common/torch_adapter/op_api_common.h:565-600);
 *   - never synchronises the host; it enqueues kernels on `stream` only, so
 *     a sequence of calls is capturable into a HIP graph;
 *   - skips invalid rows silently on the device (zero miss count, zero
 *     attention output, skipped copy pair), as the reference kernels do.
 *
 * All entry points are safe to call from several host threads; the error
 * message is thread-local.
 */
#ifndef NVDSA_H
#define NVDSA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes. */
typedef enum nvdsa_status {
  NVDSA_OK = 0,
  NVDSA_ERR_SHAPE = 1,     /* rank / extent mismatch */
  NVDSA_ERR_DTYPE = 2,     /* element type not accepted */
  NVDSA_ERR_LAYOUT = 3,    /* not contiguous or misaligned */
  NVDSA_ERR_DEVICE = 4,    /* tensors on different devices */
  NVDSA_ERR_WORKSPACE = 5, /* workspace missing or too small */
  NVDSA_ERR_RUNTIME = 6,   /* HIP runtime error while launching */
  NVDSA_ERR_ARG = 7        /* null pointer / bad scalar argument */
} nvdsa_status;

/* Element types. */
typedef enum nvdsa_dtype {
  NVDSA_INT32 = 0,
  NVDSA_FLOAT16 = 1,
  NVDSA_BFLOAT16 = 2,
  NVDSA_FLOAT32 = 3
} nvdsa_dtype;

/* Device ordinal value for pinned host memory that is mapped into the GPU
 * address space (the counterpart of torch_npu.empty_with_swapped_memory,
 * reference nanovllm/engine/model_runner.py:651-652).  Only the two DRAM
 * cache arguments of the copy entry points accept it. */
#define NVDSA_HOST_MAPPED_DEVICE (-1)

/* A dense tensor: `data` is an address the GPU can dereference (HBM, or
 * pinned host memory when device == NVDSA_HOST_MAPPED_DEVICE). */
typedef struct nvdsa_tensor {
  void* data;
  int32_t dtype;      /* nvdsa_dtype */
  int32_t ndim;       /* 0..4 */
  int64_t shape[4];
  int32_t contiguous; /* 1 when row-major dense */
  int32_t device;     /* device ordinal, or NVDSA_HOST_MAPPED_DEVICE */
} nvdsa_tensor;

/* Message of the last failing call on this thread ("" when none). */
const char* nvdsa_last_error(void);

/* Library version string. */
const char* nvdsa_version(void);

/* ---------------------------------------------------------------------- */
/* LightningIndexer top-2048 + HBM slot management, one query per request.
 * Replaces torch.ops.nanovllm_dsa.fused_li_manage
 * (reference: csrc/nanovllm_ascend_ops/bindings/nanovllm_ops.cpp:646-651,
 *  checks: ops/fused_li_manage/fused_li_manage_torch_adpt.h:18-92). */
size_t nvdsa_fused_li_manage_workspace_size(int64_t batch,
                                            int64_t source_capacity,
                                            int64_t index_heads);

int nvdsa_fused_li_manage(const nvdsa_tensor* query,
                          const nvdsa_tensor* index_weights,
                          const nvdsa_tensor* index_key_cache,
                          const nvdsa_tensor* index_block_table,
                          const nvdsa_tensor* num_candidate_tokens,
                          const nvdsa_tensor* num_cache_tokens,
                          const nvdsa_tensor* req_pool_entries,
                          const nvdsa_tensor* cache_slots_pool,
                          const nvdsa_tensor* topk_src_ids,
                          const nvdsa_tensor* topk_dst_slots,
                          const nvdsa_tensor* miss_counts,
                          void* workspace, size_t workspace_bytes,
                          void* stream);

/* Scratch bytes of nvdsa_fused_li_manage_noalloc on each GPU (32 MiB: batch
 * 64 at a 65536-token source capacity fits). */
#define NVDSA_NOALLOC_SCRATCH_BYTES (32u << 20)

/* nvdsa_fused_li_manage without a workspace argument and without allocating.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP-graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The scratch memory is a static array of
 * NVDSA_NOALLOC_SCRATCH_BYTES inside the library, one per GPU, held until
 * the process ends; its address is looked up once per device, on the first
 * call (the tensors' device must be the current device).  The call itself
 * reaches no hipMalloc/hipFree.  Arguments, checks, results and errors are
 * those of nvdsa_fused_li_manage; a batch x source capacity whose scratch
 * (nvdsa_fused_li_manage_workspace_size) exceeds the static size returns
 * NVDSA_ERR_WORKSPACE before anything is launched.  Every call on one GPU
 * uses the same scratch memory, and no state carries over between calls
 * (the kernels initialise what they read), but calls that overlap on one GPU
 * (different streams, or graphs replayed concurrently) race: order them. */
int nvdsa_fused_li_manage_noalloc(const nvdsa_tensor* query,
                                  const nvdsa_tensor* index_weights,
                                  const nvdsa_tensor* index_key_cache,
                                  const nvdsa_tensor* index_block_table,
                                  const nvdsa_tensor* num_candidate_tokens,
                                  const nvdsa_tensor* num_cache_tokens,
                                  const nvdsa_tensor* req_pool_entries,
                                  const nvdsa_tensor* cache_slots_pool,
                                  const nvdsa_tensor* topk_src_ids,
                                  const nvdsa_tensor* topk_dst_slots,
                                  const nvdsa_tensor* miss_counts,
                                  void* stream);

/* Four-query (MTP3) variant: union of four top-2048 sets.
 * Replaces torch.ops.nanovllm_dsa.fused_li_manage_mtp
 * (reference: bindings/nanovllm_ops.cpp:652-658,
 *  checks: ops/fused_li_manage_mtp/fused_li_manage_mtp_torch_adpt.h:20-111). */
size_t nvdsa_fused_li_manage_mtp_workspace_size(int64_t batch,
                                                int64_t source_capacity,
                                                int64_t index_heads);

int nvdsa_fused_li_manage_mtp(const nvdsa_tensor* query,
                              const nvdsa_tensor* index_weights,
                              const nvdsa_tensor* index_key_cache,
                              const nvdsa_tensor* index_block_table,
                              const nvdsa_tensor* num_candidate_tokens,
                              const nvdsa_tensor* num_cache_tokens,
                              const nvdsa_tensor* req_pool_entries,
                              const nvdsa_tensor* cache_slots_pool,
                              const nvdsa_tensor* topk_src_ids,
                              const nvdsa_tensor* topk_dst_slots,
                              const nvdsa_tensor* miss_src_ids,
                              const nvdsa_tensor* miss_dst_slots,
                              const nvdsa_tensor* miss_counts,
                              void* workspace, size_t workspace_bytes,
                              void* stream);

/* DRAM -> HBM copy of CKV (512) / KPE (64) rows by (src_id, dst_slot) pairs.
 * Replaces torch.ops.nanovllm_dsa.scatter_copy
 * (reference: bindings/nanovllm_ops.cpp:659-663,
 *  checks: ops/kvcache_scatter_copy/kvcache_scatter_copy_torch_adpt.h:16-66). */
int nvdsa_scatter_copy(const nvdsa_tensor* src_ids,
                       const nvdsa_tensor* dst_slots,
                       const nvdsa_tensor* copy_counts,
                       const nvdsa_tensor* hbm_block_table,
                       const nvdsa_tensor* dram_block_table,
                       const nvdsa_tensor* hbm_k_rope,
                       const nvdsa_tensor* hbm_kv_cache,
                       const nvdsa_tensor* dram_k_rope,
                       const nvdsa_tensor* dram_kv_cache,
                       void* stream);

/* Absorbed-MLA decode attention over top-2048 slots + dense tail.
 * Replaces torch.ops.nanovllm_dsa.sparse_tail_attention
 * (reference: bindings/nanovllm_ops.cpp:664-669,
 *  checks: ops/sparse_tail_attention/sparse_tail_attention_torch_adpt.h:17-88).
 * The workspace (this size) serves the four attention entry points; calls
 * that may run concurrently need separate workspaces. */
size_t nvdsa_sparse_tail_attention_workspace_size(int64_t query_rows,
                                                  int64_t heads,
                                                  int64_t max_kv_tokens);

int nvdsa_sparse_tail_attention(const nvdsa_tensor* query_rope,
                                const nvdsa_tensor* query,
                                const nvdsa_tensor* actual_seq_lengths_query,
                                const nvdsa_tensor* actual_seq_lengths_kv,
                                const nvdsa_tensor* num_cache_tokens,
                                const nvdsa_tensor* topk_dst_slots,
                                const nvdsa_tensor* hbm_block_table,
                                const nvdsa_tensor* hbm_k_rope,
                                const nvdsa_tensor* hbm_kv_cache,
                                double scale_value,
                                const nvdsa_tensor* attention_out,
                                void* workspace, size_t workspace_bytes,
                                void* stream);

/* MTP3 variant: row 4b+q sees kv_len[b] - (3 - q) tokens.
 * Replaces torch.ops.nanovllm_dsa.sparse_tail_attention_mtp
 * (reference: bindings/nanovllm_ops.cpp:670-675,
 *  checks: ops/sparse_tail_attention_mtp/sparse_tail_attention_mtp_torch_adpt.h:18-96). */
int nvdsa_sparse_tail_attention_mtp(const nvdsa_tensor* query_rope,
                                    const nvdsa_tensor* query,
                                    const nvdsa_tensor* actual_seq_lengths_query,
                                    const nvdsa_tensor* actual_seq_lengths_kv,
                                    const nvdsa_tensor* num_cache_tokens,
                                    const nvdsa_tensor* topk_dst_slots,
                                    const nvdsa_tensor* hbm_block_table,
                                    const nvdsa_tensor* hbm_k_rope,
                                    const nvdsa_tensor* hbm_kv_cache,
                                    double scale_value,
                                    const nvdsa_tensor* attention_out,
                                    void* workspace, size_t workspace_bytes,
                                    void* stream);

/* Copy of the LIM misses fused with sparse-tail attention.
 * Replaces torch.ops.nanovllm_dsa.fused_copy_sfa
 * (reference: bindings/nanovllm_ops.cpp:676-684,
 *  checks: ops/fused_copy_sfa/fused_copy_sfa_torch_adpt.h:7-110). */
int nvdsa_fused_copy_sfa(const nvdsa_tensor* query_rope,
                         const nvdsa_tensor* query,
                         const nvdsa_tensor* actual_seq_lengths_query,
                         const nvdsa_tensor* actual_seq_lengths_kv,
                         const nvdsa_tensor* num_cache_tokens,
                         const nvdsa_tensor* topk_dst_slots,
                         const nvdsa_tensor* topk_src_ids,
                         const nvdsa_tensor* miss_counts,
                         const nvdsa_tensor* hbm_block_table,
                         const nvdsa_tensor* dram_block_table,
                         const nvdsa_tensor* hbm_k_rope,
                         const nvdsa_tensor* hbm_kv_cache,
                         const nvdsa_tensor* dram_k_rope,
                         const nvdsa_tensor* dram_kv_cache,
                         double scale_value,
                         const nvdsa_tensor* attention_out,
                         void* workspace, size_t workspace_bytes,
                         void* stream);

/* MTP3 copy of the union misses fused with MTP3 sparse-tail attention.
 * Replaces torch.ops.nanovllm_dsa.fused_copy_sfa_mtp
 * (reference: bindings/nanovllm_ops.cpp:685-694,
 *  checks: ops/fused_copy_sfa_mtp/fused_copy_sfa_mtp_torch_adpt.h:9-150). */
int nvdsa_fused_copy_sfa_mtp(const nvdsa_tensor* query_rope,
                             const nvdsa_tensor* query,
                             const nvdsa_tensor* actual_seq_lengths_query,
                             const nvdsa_tensor* actual_seq_lengths_kv,
                             const nvdsa_tensor* num_cache_tokens,
                             const nvdsa_tensor* topk_dst_slots,
                             const nvdsa_tensor* topk_src_ids,
                             const nvdsa_tensor* miss_src_ids,
                             const nvdsa_tensor* miss_dst_slots,
                             const nvdsa_tensor* miss_counts,
                             const nvdsa_tensor* hbm_block_table,
                             const nvdsa_tensor* dram_block_table,
                             const nvdsa_tensor* hbm_k_rope,
                             const nvdsa_tensor* hbm_kv_cache,
                             const nvdsa_tensor* dram_k_rope,
                             const nvdsa_tensor* dram_kv_cache,
                             double scale_value,
                             const nvdsa_tensor* attention_out,
                             void* workspace, size_t workspace_bytes,
                             void* stream);

/* ---------------------------------------------------------------------- */
/* First-decode LIDU initialisation of one request (replaces the reference's
 * PyTorch slow path initialize_lidu_row, nanovllm/models/dsa_offload_ops.py:251-360,
 * which the model calls eagerly before the first stable decode step,
 * nanovllm/models/glm_mla.py:1260-1286).  Scores without ReLU
 * (s[t] = sum_h w[h] * q[h].k[t]), the cache_tokens largest over tokens
 * [0, candidate_len) (ties to the lower token), slot i to the i-th smallest
 * selected token (the reference's order is that of torch.topk(sorted=False)),
 * every other entry of the pool row set to -1, and the selected rows copied
 * DRAM -> HBM.  query [H, 128] (or [1, H, 128]), weights [H]; caches in the
 * 3-D views scatter_copy takes; table arguments are 1-D rows.  cache_tokens
 * <= 0 is a no-op; the reference's ValueErrors (cache_tokens < 2048,
 * candidate_len < cache_tokens, incomplete blocks) return NVDSA_ERR_ARG with
 * its message.  Enqueues on `stream` without synchronising. */
size_t nvdsa_initialize_lidu_row_workspace_size(int64_t source_capacity);

int nvdsa_initialize_lidu_row(const nvdsa_tensor* query,
                              const nvdsa_tensor* weights,
                              const nvdsa_tensor* index_cache,
                              const nvdsa_tensor* index_block_table,
                              int64_t candidate_len,
                              int64_t cache_tokens,
                              const nvdsa_tensor* cache_slots_row,
                              const nvdsa_tensor* hbm_kpe,
                              const nvdsa_tensor* hbm_ckv,
                              const nvdsa_tensor* dram_kpe,
                              const nvdsa_tensor* dram_ckv,
                              const nvdsa_tensor* hbm_block_table,
                              const nvdsa_tensor* dram_block_table,
                              int64_t block_size,
                              void* workspace, size_t workspace_bytes,
                              void* stream);

/* IndexShare shared layer (replaces initialize_lidu_row_shared,
 * nanovllm/models/dsa_offload_ops.py:363-411): copy this layer's DRAM rows of
 * every token the owner's pool row caches, ascending token, to its slot.  Like
 * the reference (whose nonzero() synchronises), it waits for `stream` once to
 * compare the cached count with cache_tokens before the copy, and returns
 * NVDSA_ERR_RUNTIME with the reference's message when they differ.  Takes the
 * workspace size of nvdsa_initialize_lidu_row. */
int nvdsa_initialize_lidu_row_shared(const nvdsa_tensor* cache_slots_row,
                                     int64_t cache_tokens,
                                     const nvdsa_tensor* hbm_kpe,
                                     const nvdsa_tensor* hbm_ckv,
                                     const nvdsa_tensor* dram_kpe,
                                     const nvdsa_tensor* dram_ckv,
                                     const nvdsa_tensor* hbm_block_table,
                                     const nvdsa_tensor* dram_block_table,
                                     void* workspace, size_t workspace_bytes,
                                     void* stream);

/* ---------------------------------------------------------------------- */
/* In-place interleaved-pair RoPE of the first rope_dim dims of every
 * [token, head] row of q_inout [T, H, D] (16-bit); cos/sin [T, 1, 1, rope_dim]
 * of the same dtype, token t's values at t * rope_dim.  Per pair (even,
 * odd): even' = even*cos - odd*sin, odd' = odd*cos + even*sin, each product
 * and the sum rounded in fp32, then rounded to nearest even.
 * Replaces torch.ops.nanovllm_dsa.dsa_indexer_query_rope_inplace
 * (reference csrc/nanovllm_ascend_ops/bindings/nanovllm_ops.cpp:713-714;
 * checks ops/dsa_indexer_project/dsa_indexer_project_torch_adpt.h:42-90;
 * kernel ops/dsa_indexer_project/op_kernel/dsa_indexer_project_kernel.cpp:60-176). */
int nvdsa_dsa_indexer_query_rope_inplace(const nvdsa_tensor* q_inout,
                                         const nvdsa_tensor* cos,
                                         const nvdsa_tensor* sin,
                                         int64_t rope_dim,
                                         void* stream);

/* Decode indexer projection in one launch:
 *   q_index_out[t]       = RoPE(round16(q_c[t] . wq_b_weight^T)) viewed [n_head, head_dim]
 *   index_weights_out[t] = round16(round16(hidden_states[t] . weights_proj_weight^T) * score_scale)
 * (the second rounding only when score_scale != 1).  Replaces the
 * PyTorch function dsa_indexer_project_query_only
 * (reference nanovllm/models/dsa_indexer_project.py:296-355) for the case
 * where weights_proj_weight shares the activations' 16-bit dtype; pass both
 * weights_proj_weight and index_weights_out as NULL to compute q only.
 * cos/sin hold numel/T >= rope_dim values per token (the reference's
 * reshape(T, -1)[..., :rope_dim], :28-32).  Limits of this implementation:
 * q_lora_rank a multiple of 256, hidden_size of 512, n_head and head_dim
 * multiples of 16.  No workspace. */
int nvdsa_dsa_indexer_project_query_only(const nvdsa_tensor* hidden_states,
                                         const nvdsa_tensor* q_c,
                                         const nvdsa_tensor* cos,
                                         const nvdsa_tensor* sin,
                                         const nvdsa_tensor* wq_b_weight,
                                         const nvdsa_tensor* weights_proj_weight,
                                         const nvdsa_tensor* q_index_out,
                                         const nvdsa_tensor* index_weights_out,
                                         int64_t n_head,
                                         int64_t head_dim,
                                         int64_t rope_dim,
                                         double score_scale,
                                         void* stream);

/* Prefill -> DRAM persistence of full KV blocks in one launch: for every i,
 * dram_kv_cache[dram_block_ids[i]] = hbm_kv_cache[hbm_block_ids[i]] and the
 * same for the rope caches.  Caches [blocks, 128, 512] / [blocks, 128, 64]
 * (or with the reference's singleton third dim); the DRAM caches may be
 * host-mapped (device NVDSA_HOST_MAPPED_DEVICE).  A pair whose ids do not
 * name a block of the caches is skipped on the device.  Replaces the
 * per-block synchronous copies of GlmMLAAttention.finalize_prefill_offload
 * (reference nanovllm/models/glm_mla.py:883-889).  No workspace. */
int nvdsa_persist_prefill_blocks(const nvdsa_tensor* hbm_kv_cache,
                                 const nvdsa_tensor* hbm_k_rope,
                                 const nvdsa_tensor* dram_kv_cache,
                                 const nvdsa_tensor* dram_k_rope,
                                 const nvdsa_tensor* hbm_block_ids,
                                 const nvdsa_tensor* dram_block_ids,
                                 void* stream);

/* ---------------------------------------------------------------------- */
/* Pinned, device-mapped host memory for the DRAM KV caches: the counterpart
 * of torch_npu.empty_with_swapped_memory (reference
 * nanovllm/engine/model_runner.py:651-652, ut_ops/test_scatter_copy.py:64-72).
 * `*host_ptr` is the CPU address; `*device_ptr` the address kernels use. */
int nvdsa_host_mapped_alloc(size_t bytes, void** host_ptr, void** device_ptr);
int nvdsa_host_mapped_free(void* host_ptr);

/* ---------------------------------------------------------------------- */
/* Kernel-level timing (instrumentation; no counterpart in the reference,
 * whose ut_ops scripts time whole operators with NPU events).  Between
 * nvdsa_profile_begin and nvdsa_profile_end on one host thread, every kernel
 * the entry points launch is bracketed by two hipEventRecord calls on its
 * stream (up to `capacity` launches).  nvdsa_profile_end waits for those
 * events and writes each launch's duration in milliseconds and its kernel id
 * (see nvdsa_kernel_name); *recorded receives the number of launches. */
int nvdsa_profile_begin(int32_t capacity);
int nvdsa_profile_end(float* durations_ms, int32_t* kernel_ids, int32_t capacity, int32_t* recorded);
const char* nvdsa_kernel_name(int32_t kernel_id);

/* ---------------------------------------------------------------------- */
/* Dispatch check (diagnostics; no counterpart in the reference).  The first
 * kernel of nvdsa_fused_copy_sfa_mtp gives workgroups the copy role or the
 * attention role by linear id, assuming the dispatcher deals workgroups to
 * the 8 XCDs round-robin (single-partition mode), so that the host reads of
 * the copy never share an XCD with the attention's HBM reads.  Each of its
 * workgroups records the XCD it ran on: bit x of masks[0] is set when a copy
 * workgroup ran on XCD x, of masks[1] when an attention workgroup did,
 * accumulated on the current device since the last reset.  The masks are
 * disjoint when the assumption held.  Results are correct either way; only
 * the speed depends on it.  With reset != 0 the record is cleared after the
 * read.  Synchronises the device; not for use under graph capture. */
int nvdsa_xcd_roles(uint32_t* masks, int32_t reset);
/* Turns that record on (on != 0) or off for the launches made from then on
 * (a captured graph keeps the setting of its capture). */
void nvdsa_xcd_roles_record(int32_t on);

#ifdef __cplusplus
}
#endif

#endif /* NVDSA_H */
