// sparse_tail_attention(_mtp) and fused_copy_sfa(_mtp): absorbed-MLA decode
// attention over the 2048 selected HBM slots plus the dense tail.
//
// Row rules (ops/sparse_tail_attention/op_kernel/nanovllm_sparse_tail_attention_kernel_mla.h:325-353):
//   L  = kv_len[b] - (MTP3 ? 3 - q : 0)       visible length of query row (b, q)
//   C == 0            -> keys = slots [0, L)
//   2048 <= C <= L    -> keys = topk_dst_slots[row, 0:2048] ++ slots [C, L)
//   otherwise         -> output zeros
// A key is used only when 0 <= slot < L and its block-table entry resolves
// (the s2IdLimit bound of nanovllm_sparse_tail_attention_service_vector_mla.h:792-797).
//   o = softmax(scale * (q . ckv + q_rope . kpe)) . ckv     fp32 accumulate, 16-bit store.
//
// Kernel design (split-KV flash decode):
//   grid = rows x splits x ceil(heads/64); a 512-thread workgroup owns one
//   row, one split of its key list and 64 heads (small non-fused launches:
//   256-thread workgroups of 32 heads, two per CU, see AttnShape).  Its 8
//   wavefronts are 4 pairs, one pair per 16 heads; the two waves of a pair
//   (two per SIMD, so one hides the other's LDS and MFMA latency) split the
//   work by dimension: wave half d takes S's dims [288d, 288d + 288) and the
//   output's latent dims [256d, 256d + 256).  Keys are processed in tiles
//   of 32.  Each lane keeps its query operand (one head, 9 x 16 bytes of
//   its 288 dims) in registers for the whole split; each tile is gathered
//   row-contiguous into LDS (conflict-free 16-byte operand reads for S; the
//   V^T operand of the PV product comes from transposing ds_read_b64_tr_b16
//   reads).  The pair adds its two partial S tiles through LDS, so both
//   waves hold the same S and run the same softmax.  S^T = K . Q^T and
//   O^T = V^T . P^T run on v_mfma_f32_16x16x32; the online softmax is in
//   base 2 with a running max that moves only when exceeded by more than
//   kMaxSlack (few numerator rescales), and P enters the PV product as a
//   bf16/f16 hi+lo pair so its rounding stays at fp32 level.  A second
//   kernel merges the per-split (max, sum, numerator) partials.
//   fused_copy_sfa (MTP0): a row's miss keys are the first miss_counts
//   entries of its list.  The first few splits of the row (kMissSplits, more
//   at small batches and for rows with many misses) take the tiles holding
//   them: each such tile is read once from host-mapped DRAM, stored to its
//   HBM slots and consumed from LDS.  A split's host tiles are sequential
//   (one PCIe round trip each).  The other splits take the HBM-only tiles,
//   so the host-link-bound copy and the HBM-bound attention run side by
//   side.  fused_copy_sfa_mtp: the union misses are not tile-aligned to any
//   one query row, so one launch copies the union on some XCDs while the
//   others attend the keys already in HBM, and a second launch attends the
//   copied keys.
#include <algorithm>
#include <atomic>
#include <cfloat>

#include "nvdsa_common.h"
#include "nvdsa_kernels.h"
#include "row_copy.h"

namespace nvdsa {
namespace {

constexpr int kTileKeys = 32;
constexpr int kAttnThreads = 512;  // the fused and overlap kernels (AttnShape<8>)
constexpr int kHeadsPerBlock = 64;
constexpr int kKStride = kQkDim + 16;      // LDS row of the key tile (elements; 1184 B, fewest bank conflicts)
constexpr int kChunksPerKey = kQkDim * 2 / 16;  // 72 x 16 bytes
constexpr int kSChunks = kQkDim / 32 / 2;  // 9 MFMA k-steps of 32 dims: one wave's half of S
constexpr int kVDims = kCkvDim / 2;        // 256 latent dims of the output per wave
constexpr int kMaxSplits = 64;

// Workgroup shapes of the split attention.  W waves form W/2 pairs, one pair
// per 16 heads (the two waves of a pair split S and the output by dims).
// Both keep two tile buffers (the next tile is stored during the current
// one's PV).
// * W = 8: 64 heads, one workgroup per CU.  The fused kernel (each host tile
//   is read once, so all of a row's heads share it) and the MTP3 overlap
//   launch.
// * W = 4: 32 heads, two workgroups per CU (<= 80 KB of LDS each: the pair
//   exchange of partial S uses the buffer of the next tile, which is free
//   until that tile is stored, at the cost of a third barrier per tile).
//   Small sparse_tail_attention launches (plan_split): twice the workgroups
//   of the 8-wave grid, and the two workgroups of a CU are not tied by one
//   barrier.
//   A row's two head halves read the same key tiles; they are launched on
//   one XCD so the second read hits its L2.
template <int W>
struct AttnShape {
  static_assert(W == 4 || W == 8, "split attention: 4 or 8 waves");
  static constexpr int kThreads = 64 * W;
  static constexpr int kPairs = W / 2;
  static constexpr int kHeads = 16 * kPairs;
  static constexpr bool kAliasExchange = W == 4;  // the pair exchange lives in the next tile's buffer
  static constexpr int kWindowTiles = kThreads / kTileKeys;  // tiles resolved per window (one key per thread)
  static constexpr int kWindowKeys = kThreads;
  // HBM tiles: 8 threads per key; a thread loads kCkvChunks 16-byte chunks of
  // the latent row and, where noted, one of the rope part (W = 8: threads
  // t < 256 take chunks 0-3 of each 8 and the rope chunk, the others chunks
  // 4-7; W = 4: every thread all 8 and the rope chunk).
  static constexpr int kCkvChunks = W == 8 ? 4 : 8;
  // Host tiles (fused, W = 8 only): 2304 16-byte chunks over 512 threads.
  static constexpr int kPf = W == 8 ? 5 : kCkvChunks + 1;  // tile chunks held per thread
};
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMaxSlack = 8.f;  // base-2 headroom of the running max (P < 256)
constexpr int kMissSplits = 2;  // fused: least splits of a row that take its host-sourced tiles
constexpr int kMissWorkgroups = 32;  // fused: target number of host-tile workgroups per launch
// Fused, launches of kMissRuleRows rows or more: miss tiles per miss split
// (rows of at least 6 splits / fewer).
constexpr int kMissTilesPerSplit = 6;
constexpr int kMissTilesPerSplitFew = 12;
constexpr int kMissRuleRows = 16;
constexpr int kFusedMaxSplits = 16;  // fused: most splits per row from kFusedCapRows rows on
constexpr int kFusedCapRows = 8;
constexpr int kFusedSmallSplits = 32;  // fused: most splits per row below kFusedCapRows rows
constexpr int kFusedTargetWgs = 128;  // fused: workgroups per launch above kFusedCapRows rows
constexpr int kFusedTargetWgsSmall = 80;  // fused: workgroups per launch at kFusedCapRows rows

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// ds_read_b64_tr_b16 (gfx950): within each 16-lane group, lane i reads four
// 16-bit values M[i][0..3] at its address; lane l receives
// M[4j + (l >> 2)][l & 3] for j = 0..3.
__device__ inline uint2 lds_read_tr16(const uint16_t* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(const_cast<uint16_t*>(p)));
  return __builtin_bit_cast(uint2, v);
}

struct RowPlan {
  int active;      // 1 when the row attends
  int sparse;      // number of sparse list entries (0 or 2048)
  int tail_start;  // first tail slot
  int count;       // total key list length
  int lvis;        // visible length L
};

__device__ inline RowPlan plan_row(const SfaArgs& a, int64_t row) {
  const int64_t b = row / a.rows_per_request;
  const int q = static_cast<int>(row - b * a.rows_per_request);
  int64_t lvis = a.seq_kv[b];
  if (a.rows_per_request > 1) {
    const int hidden = static_cast<int>(a.rows_per_request) - 1 - q;
    lvis = lvis > hidden ? lvis - hidden : 0;
  }
  if (lvis < 0) lvis = 0;
  const int c = a.num_cache[b];
  RowPlan p{0, 0, 0, 0, static_cast<int>(lvis > INT32_MAX ? INT32_MAX : lvis)};
  if (c == 0) {
    p.active = lvis > 0;
    p.tail_start = 0;
    p.count = p.lvis;
  } else if (c >= kTopK && static_cast<int64_t>(c) <= lvis) {
    p.active = 1;
    p.sparse = kTopK;
    p.tail_start = c;
    p.count = kTopK + (p.lvis - c);
  }
  return p;
}

struct Partials {
  float* o;   // [R][S][H][512]
  float* ml;  // [R][S][H][2]
};

Partials carve(void* ws, int64_t rows, int64_t splits, int64_t heads) {
  Partials p;
  p.o = static_cast<float*>(ws);
  p.ml = reinterpret_cast<float*>(static_cast<char*>(ws) + align256(sizeof(float) * rows * splits * heads * kCkvDim));
  return p;
}

// MTP3 overlap launch: the workgroups on kCopyXcds of the 8 XCDs copy (one
// XCD pulls ~13 GB/s from host memory), the others attend; 32 CUs per XCD,
// one resident workgroup per CU.
constexpr int kCopyXcds = 5;
constexpr int kCopyWgs = kCopyXcds * 32;

// The XCDs each role of sfa_mtp_overlap_kernel ran on since the last reset
// (bit x of [0]: a copy workgroup ran on XCD x; of [1]: an attention
// workgroup), one copy per device, read by sfa_xcd_roles.  The roles are
// given by linear workgroup id on the assumption that the dispatcher deals
// workgroups to the XCDs round-robin; the masks show whether it did.  Only
// launches made while recording is on (sfa_xcd_roles_record, a diagnostic)
// write them: the serving path does no diagnostic writes.
__device__ unsigned int g_xcd_roles[2];
std::atomic<int> g_record_xcd_roles{0};

// Id of the XCD the calling wave runs on (hardware register XCC_ID, bits 3:0).
__device__ inline unsigned int hw_xcd_id() {
  unsigned int v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(v));
  return v;
}
// x extent of a split-attention grid of n (row, split) workgroups: 4-wave
// launches round it up to a multiple of 8, so the head halves of a row's
// split (x, 0) and (x, 1) are dealt to the same XCD.
template <int W>
int64_t split_grid_x(int64_t n) {
  return W == 8 ? n : (n + 7) / 8 * 8;
}

int overlap_splits(int64_t rows, int64_t head_groups) {
  // About one workgroup per two attention CUs: the resident keys' attention
  // stays hidden under the copy, and the combine merges fewer partials (cfg3,
  // 64 rows: one split per row instead of three, combine 10.45 -> 8.6 us).
  int64_t s = ceil_div((8 - kCopyXcds) * 16, rows * head_groups);
  if (s < 1) s = 1;
  if (s > kMaxSplits) s = kMaxSplits;
  return static_cast<int>(s);
}

// Splits per row for a launch of W-wave workgroups (head_groups of
// AttnShape<W>::kHeads heads): the resident workgroups of the 256 CUs (one
// per CU at W = 8, two at W = 4, as the register footprint allows) in a
// single round.
template <int W>
int choose_splits(int64_t rows, int64_t head_groups) {
  if (rows <= 0 || head_groups <= 0) return 1;
  const int64_t target = W == 8 ? 256 : 512;
  int64_t s = target / (rows * head_groups);
  if (s < 1) s = 1;
  if (s > kMaxSplits) s = kMaxSplits;
  return static_cast<int>(s);
}

// Shape of a sparse_tail_attention launch: 4-wave workgroups where the
// 8-wave grid leaves CUs idle -- at most three (row, 64-head group) pairs,
// 64 splits each -- or where most of an 8-wave workgroup's pairs would have
// no head (at most 8 heads); 8-wave ones otherwise.  Kernel times, 8 -> 4
// waves: 64 heads, 1 row 11.4 -> 10.7 us, 3 rows 18.1 -> 17.1, 24 rows
// 27.9 -> 29.4 (not taken); 4 heads, 24 rows 17.6 -> 16.0, 48 rows 29.5 ->
// 22.4; 16 heads, 8 rows 11.7 -> 14.9 (not taken).
struct SplitPlan {
  int waves;
  int splits;
  int64_t hgroups;
};
SplitPlan plan_split(int64_t rows, int64_t heads) {
  if (rows * ceil_div(heads, kHeadsPerBlock) <= 3 || heads <= 8) {
    const int64_t hg = ceil_div(heads, AttnShape<4>::kHeads);
    return {4, choose_splits<4>(rows, hg), hg};
  }
  const int64_t hg = ceil_div(heads, AttnShape<8>::kHeads);
  return {8, choose_splits<8>(rows, hg), hg};
}

// Key selection of a split-attention launch over a row's list:
enum KeyMode : int {
  kKeysAll = 0,      // every sparse entry plus the tail
  kKeysResident = 1, // MTP3 overlap, first launch: sparse entries whose key_src < 0 (HBM-resident) plus the tail
  kKeysCopied = 2,   // MTP3 overlap, second launch: only sparse entries whose key_src >= 0 (copied misses)
};

// One split of one row: block index `bid` = row * splits + split; its
// partials go to split slot split_base + split of splits_total per row.
template <typename T, bool FUSED, int MODE, int W>
__device__ __forceinline__ void sfa_split_body(const SfaArgs& a, const Partials& part, int splits, int split_base,
                                               int splits_total, int64_t bid, int hg) {
  using S = AttnShape<W>;
  static_assert(!FUSED || W == 8, "the fused kernel reads each host tile once for all 64 heads");
  constexpr int kTileElems = kTileKeys * kKStride;
  constexpr int kWindowTiles = S::kWindowTiles;
  constexpr int kPf = S::kPf;
  __shared__ __align__(16) uint16_t ks[2 * kTileElems];  // two key tiles, row-major
  __shared__ int16_t cpos[MODE == kKeysCopied ? kTopK : 1];  // kKeysCopied: list positions of the copied keys
  __shared__ int scan_scratch[W + 1];
  // Partial S of each wave (its half of the dims): 8 floats per lane (4-wave
  // shape: in the next tile's buffer).
  __shared__ float4 s_half[S::kAliasExchange ? 1 : W * 64 * 2];
  // Resolved keys of the current window of kWindowTiles tiles (one per thread):
  // source row (HBM or DRAM), HBM row a DRAM-sourced key is stored to (fused
  // only), flags.
  __shared__ int64_t win_src[S::kWindowKeys];
  __shared__ int64_t win_dst[FUSED ? S::kWindowKeys : 1];
  __shared__ __align__(16) int win_flag[S::kWindowKeys];  // bit 0: attend, bit 1: source is DRAM, bit 2: source valid

  const int64_t row = bid / splits;
  const int split = static_cast<int>(bid - row * splits);
  const int64_t b = row / a.rows_per_request;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int half = wave / S::kPairs;  // dimension half of this wave (uniform)
  const int h0 = hg * S::kHeads + (wave % S::kPairs) * 16;
  const bool wave_active = h0 < a.heads;
  const int head = h0 + l16;
  const int64_t H = a.heads;

  // Query operand of this lane, kept in registers for the whole split:
  // head `head`, dims 288 half + 32 kk + 8 g .. +7 (16-byte chunk
  // 4 (9 half + kk) + g of the 576), zeros for heads beyond H.  Its loads
  // depend on nothing else, so they are issued first and land while the
  // row plan and the first window's keys are resolved.  (An inactive row
  // never multiplies them.)
  uint4 qreg[kSChunks];
  {
    const uint4* qn = static_cast<const uint4*>(a.query) + (row * H + head) * 64;
    const uint4* qr = static_cast<const uint4*>(a.query_rope) + (row * H + head) * 8;
    const bool ok = wave_active && head < a.heads;
#pragma unroll
    for (int kk = 0; kk < kSChunks; ++kk) {
      const int c = 4 * (kSChunks * half + kk) + g;
      qreg[kk] = make_uint4(0, 0, 0, 0);
      if (ok) qreg[kk] = c < 64 ? qn[c] : qr[c - 64];
    }
  }

  RowPlan plan = plan_row(a, row);
  if (MODE == kKeysCopied) {
    // Compact the positions j < 2048 with key_src >= 0 (consecutive runs of
    // kPer per thread, in order); the launch attends those entries only, and
    // no tail.
    int n_copied = 0;
    if (plan.active && plan.sparse > 0) {
      const int32_t* ksrc = a.key_src + row * kTopK;
      constexpr int kPer = kTopK / S::kThreads;
      unsigned bits = 0u;
#pragma unroll
      for (int e = 0; e < kPer; ++e)
        if (ksrc[tid * kPer + e] >= 0) bits |= 1u << e;
      int tot;
      int pos = block_exclusive_scan(__popc(bits), scan_scratch, &tot);
#pragma unroll
      for (int e = 0; e < kPer; ++e)
        if ((bits >> e) & 1u) cpos[pos++] = static_cast<int16_t>(tid * kPer + e);
      n_copied = tot;
      __syncthreads();
    }
    plan.sparse = n_copied;
    plan.count = n_copied;
  }
  // Copy work (fused): MTP0 copies pairs j < miss_counts[b] of the row's own list.
  int copy_count = 0;
  if (FUSED) {
    copy_count = a.copy_counts[b];
    copy_count = copy_count < 0 ? 0 : (copy_count > kTopK ? kTopK : copy_count);
  }
  const int list_len = plan.active ? plan.count : (FUSED ? copy_count : 0);
  const int ntiles = static_cast<int>(ceil_div(list_len, kTileKeys));
  const int64_t pidx = (row * splits_total + split_base + split) * H + head;
  // Tiles of this split: t_first, t_first + t_stride, ... < t_end.  Fused:
  // splits [0, miss_splits) take the tiles holding host-sourced misses (the
  // first ceil(copy_count/32) tiles), the others the HBM-only tiles, so the
  // host-link-bound copies and the HBM-bound tiles proceed side by side
  // instead of every workgroup first stalling on its share of the copy.
  int t_first = split, t_stride = splits, t_end = ntiles;
  const int mtiles = FUSED ? static_cast<int>(ceil_div(copy_count, kTileKeys)) : 0;
  if (FUSED && mtiles > 0 && splits >= 2) {  // (one split per row takes every tile)
    // Launches of kMissRuleRows rows or more: one miss split per
    // kMissTilesPerSplit miss tiles of the row (1 or 2 at cfg1's 3-10 miss
    // tiles), per kMissTilesPerSplitFew with fewer than 6 splits per row (1 at
    // 64 rows of 4 splits, cfg2: step 485.8 / 488.1 -> 482.1 / 480.7 us; 6
    // tiles there: 498.8 / 503.1 us).  Every miss workgroup keeps a whole tile of
    // host reads in flight, and 2-3 per row queued ~8x the link's
    // bandwidth-delay product: the link served some workgroups' first tile
    // after ~85 us, and the HBM-only workgroups on the same XCDs, their reads
    // stalled behind the host reads, ended last (115-124 us against ~110 us
    // for the copies).  24 rows: the fused kernel 116-119 -> 109-110 us and
    // the step 185.0 / 185.4 -> 178.1 / 178.7 us (4, 8 or 12 tiles per miss
    // split: 179.8-181.3, 180.0, 180.5 us).  Smaller launches: about
    // kMissWorkgroups workgroups take host-sourced tiles, at least kMissSplits
    // per row, more per row at small batches (4 at 8 rows: 3% off the
    // 78-layer step), never more than the row's miss tiles; with at least 6
    // splits a row with more than 4 miss tiles per miss split gets a third.
    const int64_t launch_rows = a.batch * a.rows_per_request;
    int miss_splits;
    if (launch_rows >= kMissRuleRows) {
      miss_splits = static_cast<int>(ceil_div(mtiles, splits >= 6 ? kMissTilesPerSplit : kMissTilesPerSplitFew));
    } else {
      miss_splits = static_cast<int>(ceil_div(kMissWorkgroups, launch_rows));
      if (miss_splits > mtiles) miss_splits = mtiles;
      if (miss_splits < kMissSplits) miss_splits = kMissSplits;
      if (splits >= 6 && mtiles > 4 * kMissSplits && miss_splits < 3) miss_splits = 3;
    }
    if (miss_splits > splits - 1) miss_splits = splits - 1;
    if (split < miss_splits) {
      t_first = split;
      t_stride = miss_splits;
      t_end = mtiles < ntiles ? mtiles : ntiles;
    } else {
      t_first = mtiles + (split - miss_splits);
      t_stride = splits - miss_splits;
      t_end = ntiles;
    }
  }
  const int my_tiles = t_first < t_end ? static_cast<int>(ceil_div(t_end - t_first, t_stride)) : 0;

  if (my_tiles == 0) {  // nothing for this split (whole workgroup)
    if (wave_active && head < a.heads && g == 0 && half == 0) {
      part.ml[pidx * 2 + 0] = -INFINITY;
      part.ml[pidx * 2 + 1] = 0.f;
    }
    return;
  }


  const int32_t* topk = a.topk_dst + row * kTopK;
  const int32_t* hbm_row_table = a.hbm_table + b * a.hbm_cols;
  const uint4* hbm_ckv = static_cast<const uint4*>(a.hbm_ckv);
  const uint4* hbm_kpe = static_cast<const uint4*>(a.hbm_kpe);
  const uint4* dram_ckv = static_cast<const uint4*>(a.dram_ckv);
  const uint4* dram_kpe = static_cast<const uint4*>(a.dram_kpe);

  // Resolve the keys of tiles first, first+splits, ... (kWindowTiles of
  // them, one key per thread) into the window arrays.
  auto resolve_window = [&](int first) {
    const int w = tid / kTileKeys;
    const int idx = first + w;  // position in this split's tile sequence
    const int tile = t_first + idx * t_stride;
    const int j = tile * kTileKeys + (tid & (kTileKeys - 1));
    int64_t src = -1, dst = -1;
    int flag = 0;
    if (idx < my_tiles && j < list_len) {
      const int lj = MODE == kKeysCopied ? cpos[j] : j;  // position in the row's list
      const int slot = plan.active ? (j < plan.sparse ? topk[lj] : plan.tail_start + (j - plan.sparse))
                                   : a.copy_dst[b * a.copy_cap + j];
      const bool skip = MODE == kKeysResident && j < plan.sparse && a.key_src[row * kTopK + j] >= 0;
      int64_t hrow = -1;
      if (slot >= 0 && (slot >> kBlockShift) < a.hbm_cols) {
        const int32_t blk = hbm_row_table[slot >> kBlockShift];
        if (blk >= 0 && blk < a.hbm_blocks) hrow = static_cast<int64_t>(blk) * kBlock + (slot & (kBlock - 1));
      }
      if (plan.active && hrow >= 0 && slot < plan.lvis && !skip) {
        flag = 1 | 4;
        src = hrow;
      }
      if (FUSED && j < copy_count) {
        const RowAddr ra = resolve_pair(a.copy_src[b * a.copy_cap + j], a.copy_dst[b * a.copy_cap + j],
                                        a.dram_table + b * a.dram_cols, a.dram_cols, a.dram_blocks, hbm_row_table,
                                        a.hbm_cols, a.hbm_blocks);
        if (ra.src_row >= 0) {
          flag |= 2 | 4;
          src = ra.src_row;
          dst = ra.dst_row;
        }
      }
    }
    win_src[tid] = src;
    if (FUSED) win_dst[tid] = dst;
    win_flag[tid] = flag;
  };
  // Two mappings of a tile's 32 x 72 chunks of 16 bytes onto the threads;
  // both fill the same row-major LDS tile.
  // * HBM tiles: thread t owns key lk = (t & 255) >> 3 and, with lg = t & 7,
  //   the chunks lg + 8j of its row (j < 8: CKV bytes [16 lg + 128 j, +16);
  //   j = 8: KPE bytes [16 lg, +16)).  W = 8: threads t < 256 take j = 0..3
  //   and the KPE chunk, threads t >= 256 take j = 4..7 (the split is by
  //   wave, so uniform); W = 4: every thread all 9.  One window lookup per
  //   thread and tile, immediate offsets.
  // * The fused kernel (host-sourced rows): chunk c = j * 512 + t (j < 5,
  //   c < 2304), so a wave instruction reads one whole KiB of consecutive
  //   row bytes, the request shape the host link serves fastest.
  const int lk = (tid & 255) >> 3;
  const int lg = tid & 7;
  const int ld_half = W == 8 ? (tid >> 8) : 0;  // which CKV chunks of its key the thread moves (uniform per wave)
  constexpr int kTileChunks = kTileKeys * kChunksPerKey;  // 2304
  constexpr int kCkv = S::kCkvChunks;
  auto load_tile = [&](int w, bool host_tile, uint4 (&pf)[kPf]) {
    if (FUSED && host_tile) {
      int t = tid;
      asm volatile("" : "+v"(t));  // recompute the chunk map here (not kept live across the loop)
#pragma unroll
      for (int jj = 0; jj < kPf; ++jj) {
        const int cidx = jj * kAttnThreads + t;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (jj < kPf - 1 || cidx < kTileChunks) {  // (the last round: waves 0-3 only)
          const int k = cidx / kChunksPerKey;
          const int pc = cidx - k * kChunksPerKey;
          const int wk = w * kTileKeys + k;
          const int flag = win_flag[wk];
          const int64_t src = win_src[wk];
          if (flag & 4) {
            const uint4* base = (flag & 2) ? (pc < 64 ? dram_ckv + src * 64 : dram_kpe + src * 8)
                                           : (pc < 64 ? hbm_ckv + src * 64 : hbm_kpe + src * 8);
            v = base[pc < 64 ? pc : pc - 64];
          }
        }
        pf[jj] = v;
      }
      return;
    }
    const int wk = w * kTileKeys + lk;
    const int flag = win_flag[wk];
    const int64_t src = win_src[wk];
    const uint4* ckv = hbm_ckv + src * 64 + lg + 8 * kCkv * ld_half;
    if (flag & 4) {
#pragma unroll
      for (int j = 0; j < kCkv; ++j) pf[j] = ckv[8 * j];
      pf[kCkv] = ld_half == 0 ? hbm_kpe[src * 8 + lg] : make_uint4(0, 0, 0, 0);
    } else {
#pragma unroll
      for (int j = 0; j < kPf; ++j) pf[j] = make_uint4(0, 0, 0, 0);
    }
  };
  auto store_tile = [&](int w, bool host_tile, const uint4 (&pf)[kPf], uint16_t* kt_base) {
    if (FUSED && host_tile) {
      int t = tid;
      asm volatile("" : "+v"(t));  // recompute the chunk map here (not kept live across the loop)
#pragma unroll
      for (int jj = 0; jj < kPf; ++jj) {
        const int cidx = jj * kAttnThreads + t;
        if (jj == kPf - 1 && cidx >= kTileChunks) break;
        const int k = cidx / kChunksPerKey;
        const int pc = cidx - k * kChunksPerKey;
        *reinterpret_cast<uint4*>(&kt_base[k * kKStride + pc * 8]) = pf[jj];
        const int wk = w * kTileKeys + k;
        if (win_flag[wk] & 2) {  // a host-sourced miss: persist it to its HBM slot
          const int64_t dst = win_dst[wk];
          if (pc < 64)
            static_cast<uint4*>(a.hbm_ckv)[dst * 64 + pc] = pf[jj];
          else
            static_cast<uint4*>(a.hbm_kpe)[dst * 8 + (pc - 64)] = pf[jj];
        }
      }
      return;
    }
    uint16_t* rowp = &kt_base[lk * kKStride + lg * 8 + 64 * kCkv * ld_half];
#pragma unroll
    for (int j = 0; j < kCkv; ++j) *reinterpret_cast<uint4*>(rowp + 64 * j) = pf[j];
    if (ld_half == 0) *reinterpret_cast<uint4*>(&kt_base[lk * kKStride + kCkvDim + lg * 8]) = pf[kCkv];
  };

  // The fused kernel reads every tile row per wave: with the key-per-8-lanes
  // mapping on its HBM tiles, the host link under them served the miss tiles
  // more slowly (cfg1 fused kernel 129 -> 138 us).
  auto is_host_tile = [&](int, int) { return FUSED; };
  uint4 pf[kPf];

  const float qscale = a.scale * kLog2e;
  const bool compute = wave_active && plan.active;  // uniform per wave, equal within a pair
  float m_run = -INFINITY;  // running max (base-2 logits) of head `head`
  float l_run = 0.f;        // this lane's share of the running sum
  f32x4_t oacc[kVDims / 16];
#pragma unroll
  for (int i = 0; i < kVDims / 16; ++i) oacc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int my_x = (wave * 64 + lane) * 2;
  const int pair_x = ((wave ^ S::kPairs) * 64 + lane) * 2;

  // Per tile two barriers, (S halves written) and (next tile stored, this
  // tile's PV done); tile w sits in buffer w & 1, tile w + 1 is loaded during
  // S(w) and stored into the other buffer after PV(w)'s reads.  With the pair
  // exchange in that other buffer (4 waves), a third barrier after the
  // exchange reads keeps the store off them.
  for (int first = 0; first < my_tiles; first += kWindowTiles) {
    resolve_window(first);
    __syncthreads();
    load_tile(0, is_host_tile(first, 0), pf);
    store_tile(0, is_host_tile(first, 0), pf, ks);
    __syncthreads();
    const int wtiles = min(kWindowTiles, my_tiles - first);
    for (int w = 0; w < wtiles; ++w) {
      uint16_t* kcur = ks + (w & 1) * kTileElems;
      uint16_t* knext = ks + ((w + 1) & 1) * kTileElems;
      float4* sx = S::kAliasExchange ? reinterpret_cast<float4*>(knext) : s_half;
      float4* my_s = sx + my_x;
      const float4* pair_s = sx + pair_x;
      if (w + 1 < wtiles) load_tile(w + 1, is_host_tile(first, w + 1), pf);  // in flight during S and PV below

      // This wave's half of the S^T tile: two 16-key blocks; lane holds
      // the partial S[head][kt*16 + 4g + i] over dims [288 half, +288).
      f32x4_t sacc[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
      if (compute) {
        // Every operand read is issued before the first MFMA (18 reads in
        // flight instead of a read-wait-multiply chain).
        const uint16_t* krow = &kcur[l16 * kKStride + 288 * half + g * 8];
        uint4 kf[2][kSChunks];
#pragma unroll
        for (int kk = 0; kk < kSChunks; ++kk)
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) kf[kt][kk] = *reinterpret_cast<const uint4*>(krow + kt * 16 * kKStride + kk * 32);
#pragma unroll
        for (int kk = 0; kk < kSChunks; ++kk)
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
            sacc[kt] = T::mfma16(__builtin_bit_cast(typename T::vec8, kf[kt][kk]),
                                 __builtin_bit_cast(typename T::vec8, qreg[kk]), sacc[kt]);
        // (The scheduler otherwise interleaves them back to two in flight.)
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * kSChunks, 0);  // LDS reads
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * kSChunks, 0);  // MFMAs
        my_s[0] = make_float4(sacc[0][0], sacc[0][1], sacc[0][2], sacc[0][3]);
        my_s[1] = make_float4(sacc[1][0], sacc[1][1], sacc[1][2], sacc[1][3]);
      }
      __syncthreads();  // both halves of S written

      float4 o0 = make_float4(0.f, 0.f, 0.f, 0.f), o1 = o0;
      if (compute) {
        o0 = pair_s[0];
        o1 = pair_s[1];
      }
      if constexpr (S::kAliasExchange) __syncthreads();  // every pair read before tile w + 1 is stored over them
      if (compute) {
        // The V^T operands of the whole tile are read first, so their LDS
        // latency passes under the softmax.  A operand V^T[dim][key] from the
        // row-major tile: keys 4g..4g+3 and 16+4g..16+4g+3 (the lanes' S^T
        // columns) at dim 256 half + dt*16 + l16, each 4-key group one
        // transposing LDS read (lane i of a 16-lane group reads dims
        // 4(i&3)..+3 of key i>>2; lane l receives the four keys' values at
        // dim l).
        const int4 f0 = *reinterpret_cast<const int4*>(&win_flag[w * kTileKeys + 4 * g]);
        const int4 f1 = *reinterpret_cast<const int4*>(&win_flag[w * kTileKeys + 16 + 4 * g]);
        const int fl[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
        const uint16_t* v0 = &kcur[(4 * g + (l16 >> 2)) * kKStride + kVDims * half + 4 * (l16 & 3)];
        const uint16_t* v1 = v0 + 16 * kKStride;
        uint2 vlo[kVDims / 16], vhi[kVDims / 16];
#pragma unroll
        for (int dt = 0; dt < kVDims / 16; ++dt) {
          vlo[dt] = lds_read_tr16(v0 + dt * 16);
          vhi[dt] = lds_read_tr16(v1 + dt * 16);
        }
        // S = own half + the pair's half (addition commutes: both waves of
        // the pair hold the same S).
        const float st[8] = {sacc[0][0] + o0.x, sacc[0][1] + o0.y, sacc[0][2] + o0.z, sacc[0][3] + o0.w,
                             sacc[1][0] + o1.x, sacc[1][1] + o1.y, sacc[1][2] + o1.z, sacc[1][3] + o1.w};
        float sv[8];
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int k = kt * 16 + 4 * g + i;
            const float x = (fl[kt * 4 + i] & 1) ? st[kt * 4 + i] * qscale : -INFINITY;
            sv[kt * 4 + i] = x;
            mx = fmaxf(mx, x);
          }
        mx = xor32_op(xor16_op(mx, MaxOp{}), MaxOp{});
        // The reference max only moves when the tile max exceeds it by more
        // than kMaxSlack (base-2 units), so P stays below 2^kMaxSlack and the
        // numerator is rescaled on few tiles (softmax does not depend on the
        // subtracted constant).  While no key has been attended (m_run and
        // the tile max -inf) the subtracted constant is 0: P, the sum and
        // alpha are then all 0 and the tile adds nothing.
        const bool grow = mx > m_run + kMaxSlack;  // also m_run == -inf with a finite tile max
        const float m_new = grow ? mx : m_run;
        const float m_sub = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_sub);  // 1 unless grow; 0 from m_run == -inf
        const bool rescale = __any(grow && m_run != -INFINITY);     // (zero numerators need none)
        m_run = m_new;
        float psum = 0.f;
        float p[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          p[i] = __builtin_amdgcn_exp2f(sv[i] - m_sub);  // (results below 2^-126 flush to 0)
          psum += p[i];
        }
        l_run = l_run * alpha + psum;
        if (rescale) {
#pragma unroll
          for (int dt = 0; dt < kVDims / 16; ++dt) {
            oacc[dt][0] *= alpha;
            oacc[dt][1] *= alpha;
            oacc[dt][2] *= alpha;
            oacc[dt][3] *= alpha;
          }
        }
        // P as a hi + lo pair of 16-bit values: two MFMAs give P . V with
        // ~16 mantissa bits of P instead of 8.  (One rounded P is not
        // enough: with near-uniform attention over thousands of keys the
        // output is a small mean of zero-mean rows, and P's rounding error
        // does not shrink with it.)
        typename T::vec8 pb_hi, pb_lo;
        uint16_t* phs = reinterpret_cast<uint16_t*>(&pb_hi);
        uint16_t* pls = reinterpret_cast<uint16_t*>(&pb_lo);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          phs[i] = T::hi_part(p[i]);
          pls[i] = T::from_finite(p[i] - T::to_float(phs[i]));
        }
#pragma unroll
        for (int dt = 0; dt < kVDims / 16; ++dt) {
          const auto af = __builtin_bit_cast(typename T::vec8, make_uint4(vlo[dt].x, vlo[dt].y, vhi[dt].x, vhi[dt].y));
          oacc[dt] = T::mfma16(af, pb_lo, T::mfma16(af, pb_hi, oacc[dt]));
        }
      }
      if (w + 1 < wtiles) store_tile(w + 1, is_host_tile(first, w + 1), pf, knext);
      __syncthreads();  // tile w + 1 resident; every wave done with tile w and s_half
    }
  }

  // Split partials: max, sum and un-normalised numerator per head (each
  // wave its 256 latent dims; the pair's (max, sum) are equal, half 0
  // writes them).
  if (!wave_active || head >= a.heads) return;
  const float lsum = xor32_op(xor16_op(l_run, AddOp{}), AddOp{});
  if (g == 0 && half == 0) {
    part.ml[pidx * 2 + 0] = m_run;
    part.ml[pidx * 2 + 1] = lsum;
  }
  if (lsum > 0.f) {
    float* od = part.o + pidx * kCkvDim + kVDims * half;
#pragma unroll
    for (int dt = 0; dt < kVDims / 16; ++dt)
      *reinterpret_cast<float4*>(od + dt * 16 + 4 * g) =
          make_float4(oacc[dt][0], oacc[dt][1], oacc[dt][2], oacc[dt][3]);
  }
}

// Two waves per SIMD (one 8-wave or two 4-wave workgroups per CU): the
// compiler may use up to 256 registers per lane and schedule for latency, not
// occupancy.  The grid's x extent may be padded past rows * splits (4-wave
// launches: to a multiple of 8, so workgroup (x, y) shares its XCD with
// (x, y') when the dispatcher deals linear ids round-robin over the 8 XCDs).
template <typename T, bool FUSED, int MODE, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2, 2))) void sfa_split_kernel(
    SfaArgs a, Partials part, int splits, int split_base, int splits_total) {
  if (static_cast<int64_t>(blockIdx.x) >= a.batch * a.rows_per_request * splits) return;
  sfa_split_body<T, FUSED, MODE, W>(a, part, splits, split_base, splits_total, blockIdx.x, blockIdx.y);
}

// MTP3 fused_copy_sfa, first launch: attention over the HBM-resident keys
// (kKeysResident) and the DRAM -> HBM copy of the union misses, side by side
// on separate XCDs.  Workgroups are dealt to the 8 XCDs round-robin by
// linear id (from a starting XCD that can differ between dispatches), so
// those with id mod 8 < kCopyXcds share 5 XCDs: they copy (a grid-stride
// loop over 16-row chunks of every request), the rest attend.  Host reads in flight
// stall HBM reads issued on the same XCD, so the two roles do not share one.
// No workgroup waits on another: the copied keys are attended by a second
// launch on the same stream.
template <typename T>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void sfa_mtp_overlap_kernel(SfaArgs a, Partials part, int splits,
                                                                       int splits_total, ScatterArgs sc,
                                                                       int attn_blocks, int hgroups, int copy_wgs,
                                                                       int record_roles) {
  const int p = blockIdx.x;
  const int xcd = p & 7;
  const int slot = p >> 3;
  if (record_roles != 0 && threadIdx.x == 0) atomicOr(&g_xcd_roles[xcd < kCopyXcds ? 0 : 1], 1u << hw_xcd_id());
  if (xcd < kCopyXcds) {
    // The copy moves 16-pair chunks with 4 waves (scatter_copy_wg); the
    // workgroup's other waves have nothing to copy.
    const int wg = slot * kCopyXcds + xcd;
    if (wg < copy_wgs && threadIdx.x < 256) scatter_copy_wg(sc, wg, copy_wgs);
    return;
  }
  const int i = slot * (8 - kCopyXcds) + (xcd - kCopyXcds);
  if (i >= attn_blocks * hgroups) return;
  sfa_split_body<T, false, kKeysResident, 8>(a, part, splits, 0, splits_total, i % attn_blocks, i / attn_blocks);
}

// Merge split partials: one workgroup per (row, head) of G groups of 128
// threads, 4 of the 512 latent dims per thread; group g merges the splits
// [Bg, Bg + B) (B = 16 and G = ceil(splits / 16), at most 8; rows of at most
// 4, 8 or 12 splits: one group, B = 4, 8 or 12), so every thread loads its
// output slices in one round, all in flight together.  Lane s of each
// wave reads split s's (m, l) (and split s + 64's), so the running max, the
// weights exp2(m_s - max) and the softmax denominator come from one load and
// two wave reductions (every wave computes them).  Within a group the slices
// are summed in split order; the groups' sums are then added in group order
// through LDS.  Splits with l == 0 hold no keys and are skipped.  (A chain of
// one dependent load per split, or one group walking 64 splits 16 at a time,
// is latency-bound: a single row launches 64 splits.)
constexpr int kCombineBatch = 16;
constexpr int kCombineMaxSplits = 2 * kWave;
constexpr int kCombineMaxGroups = kCombineMaxSplits / kCombineBatch;  // 8
static_assert(2 * kMaxSplits <= kCombineMaxSplits, "an MTP3 launch pair merges up to 2 x kMaxSplits splits");

template <typename T, int B>
__global__ __launch_bounds__(128 * kCombineMaxGroups) void sfa_combine_kernel(SfaArgs a, Partials part, int splits) {
  static_assert(B == 4 || B == 8 || B == 12 || B == kCombineBatch, "slices per thread");
  __shared__ float4 gsum[kCombineMaxGroups - 1][128];
  const int64_t H = a.heads;
  const int lane = threadIdx.x & (kWave - 1);
  const int grp = threadIdx.x >> 7;  // split group (uniform per wave)
  const int dq = threadIdx.x & 127;  // dims 4 dq .. 4 dq + 3
  const int groups = blockDim.x >> 7;
  // The partial of (row, split s, head) sits at index base + s * H.
  const int64_t base = static_cast<int64_t>(blockIdx.x) * splits * H + blockIdx.y;
  const float2* mlp = reinterpret_cast<const float2*>(part.ml);
  const float4* op = reinterpret_cast<const float4*>(part.o);
  constexpr int kVec = kCkvDim / 4;
  const int s0 = grp * B;
  float4 x[B];
#pragma unroll
  for (int j = 0; j < B; ++j)  // an index past the last split rereads it (ignored below)
    x[j] = op[(base + min(s0 + j, splits - 1) * H) * kVec + dq];
  float2 v0 = make_float2(0.f, 0.f), v1 = v0;
  if (lane < splits) v0 = mlp[base + lane * H];
  if (lane + kWave < splits) v1 = mlp[base + (lane + kWave) * H];
  const bool live0 = v0.y > 0.f, live1 = v1.y > 0.f;
  float m = fmaxf(live0 ? v0.x : -INFINITY, live1 ? v1.x : -INFINITY);
  m = wave_all_op(m, MaxOp{});
  float w0 = 0.f, w1 = 0.f;
  if (m != -INFINITY) {
    w0 = live0 ? exp2f(v0.x - m) : 0.f;
    w1 = live1 ? exp2f(v1.x - m) : 0.f;
  }
  float total = (live0 ? v0.y * w0 : 0.f) + (live1 ? v1.y * w1 : 0.f);
  total = wave_all_op(total, AddOp{});
  // Consumed here, unconditionally: otherwise the compiler sinks each
  // split's load into its conditional use below, one wait each.
#pragma unroll
  for (int j = 0; j < B; ++j) asm volatile("" : "+v"(x[j].x), "+v"(x[j].y), "+v"(x[j].z), "+v"(x[j].w));
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < B; ++j) {
    const int sp = s0 + j;  // uniform
    const float ws = __builtin_bit_cast(
        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sp < kWave ? w0 : w1), sp & (kWave - 1)));
    if (sp < splits && ws != 0.f) {
      acc.x += x[j].x * ws;
      acc.y += x[j].y * ws;
      acc.z += x[j].z * ws;
      acc.w += x[j].w * ws;
    }
  }
  if (groups > 1) {
    if (grp > 0) gsum[grp - 1][dq] = acc;
    __syncthreads();
    if (grp > 0) return;
    for (int g2 = 1; g2 < groups; ++g2) {
      const float4 o = gsum[g2 - 1][dq];
      acc.x += o.x;
      acc.y += o.y;
      acc.z += o.z;
      acc.w += o.w;
    }
  }
  const float inv = total > 0.f ? 1.f / total : 0.f;
  uint16_t* out = static_cast<uint16_t*>(a.out) + (blockIdx.x * H + blockIdx.y) * kCkvDim + dq * 4;
  const uint32_t lo = static_cast<uint32_t>(T::from_float(acc.x * inv)) |
                      (static_cast<uint32_t>(T::from_float(acc.y * inv)) << 16);
  const uint32_t hi = static_cast<uint32_t>(T::from_float(acc.z * inv)) |
                      (static_cast<uint32_t>(T::from_float(acc.w * inv)) << 16);
  *reinterpret_cast<uint2*>(out) = make_uint2(lo, hi);
}

// Rows of at most 4, 8 or 12 splits take a kernel that loads only that many
// slices per thread (a 16-slice batch rereads the last split for the rest).
template <typename T>
void launch_combine(const SfaArgs& a, const Partials& p, int64_t rows, int splits, hipStream_t stream) {
  const dim3 grid(static_cast<uint32_t>(rows), static_cast<uint32_t>(a.heads));
  if (splits <= 4) {
    launch_kernel(kKernSfaCombine, sfa_combine_kernel<T, 4>, grid, dim3(128), stream, a, p, splits);
    return;
  }
  if (splits <= 8) {
    launch_kernel(kKernSfaCombine, sfa_combine_kernel<T, 8>, grid, dim3(128), stream, a, p, splits);
    return;
  }
  if (splits <= 12) {
    launch_kernel(kKernSfaCombine, sfa_combine_kernel<T, 12>, grid, dim3(128), stream, a, p, splits);
    return;
  }
  const int groups = std::min<int>(kCombineMaxGroups, static_cast<int>(ceil_div(splits, kCombineBatch)));
  launch_kernel(kKernSfaCombine, sfa_combine_kernel<T, kCombineBatch>, grid, dim3(128 * groups), stream, a, p,
                splits);
}

// One non-fused split-attention launch of plan `sp` (partials at split
// slots [split_base, split_base + sp.splits) of `total` per row; the
// 4-wave shape is built for the all-keys mode only).
template <typename T, int MODE>
void launch_split(int kernel_id, const SfaArgs& a, const Partials& p, int64_t rows, const SplitPlan& sp,
                  int split_base, int total, hipStream_t stream) {
  if constexpr (MODE == kKeysAll) {
    if (sp.waves == 4) {
      launch_kernel(kernel_id, sfa_split_kernel<T, false, MODE, 4>,
                    dim3(static_cast<uint32_t>(split_grid_x<4>(rows * sp.splits)), static_cast<uint32_t>(sp.hgroups)),
                    dim3(AttnShape<4>::kThreads), stream, a, p, sp.splits, split_base, total);
      return;
    }
  }
  launch_kernel(kernel_id, sfa_split_kernel<T, false, MODE, 8>,
                dim3(static_cast<uint32_t>(rows * sp.splits), static_cast<uint32_t>(sp.hgroups)),
                dim3(AttnShape<8>::kThreads), stream, a, p, sp.splits, split_base, total);
}

template <typename T, bool FUSED>
hipError_t launch_sfa(const SfaArgs& a, hipStream_t stream) {
  const int64_t rows = a.batch * a.rows_per_request;
  if (rows == 0) return hipSuccess;
  if (!FUSED) {
    const SplitPlan sp = plan_split(rows, a.heads);
    const Partials p = carve(a.workspace, rows, sp.splits, a.heads);
    launch_split<T, kKeysAll>(kKernSfaSplit, a, p, rows, sp, 0, sp.splits, stream);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_combine<T>(a, p, rows, sp.splits, stream);
    return hipGetLastError();
  }
  const int64_t hgroups = ceil_div(a.heads, kHeadsPerBlock);
  // From kFusedCapRows rows on, the fused kernel lasts as long as its
  // host-link-bound miss splits, so its HBM splits can take more tiles each:
  // about 128 workgroups in all (96 at kFusedCapRows rows), 4 to
  // kFusedMaxSplits splits per row, keep the partials (128 KB per split and
  // row at 64 heads) and their merge small while the HBM-only splits still
  // end before the copies.  Measured: 24 rows, 6 splits (10 before): combine
  // 7.0 -> 5.7 us and the step 3 us shorter (4 splits: the fused kernel 4 us
  // longer); 8 rows, 10 splits (32, 16, then 12 before): the 78-layer step
  // 5.60 -> 5.48 ms at 12, then 5.30-5.33 -> 5.26-5.28 ms at 10 (combine 4.3
  // -> 4.1 us; 9 splits: 5.38 ms, 8: 5.33-5.35 ms).  With fewer rows the HBM
  // tiles are the longer path: at most kFusedSmallSplits per row (64 before:
  // graph-replayed steps of 20480-token rows, 1 / 2 / 4 / 6 rows, 50.8 / 58.6 /
  // 71.7 / 82.0 -> 49.0 / 55.1 / 68.6 / 79.5 us; 16 or 24 splits at 1 row
  // slower).
  int splits = choose_splits<8>(rows, hgroups);
  if (rows < kFusedCapRows) splits = std::min(splits, kFusedSmallSplits);
  if (rows >= kFusedCapRows) {
    const int target = rows * hgroups <= kFusedCapRows ? kFusedTargetWgsSmall : kFusedTargetWgs;
    splits = std::min<int>(splits, std::max<int>(4, std::min<int>(kFusedMaxSplits, static_cast<int>(ceil_div(
                                                                  target, rows * hgroups)))));
  }
  const Partials p = carve(a.workspace, rows, splits, a.heads);
  launch_kernel(kKernSfaSplitFused, sfa_split_kernel<T, true, kKeysAll, 8>,
                dim3(static_cast<uint32_t>(rows * splits), static_cast<uint32_t>(hgroups)), dim3(kAttnThreads),
                stream, a, p, splits, 0, splits);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  launch_combine<T>(a, p, rows, splits, stream);
  return hipGetLastError();
}

// MTP3 fused_copy_sfa: the overlap launch (HBM-resident keys + the union
// copy), then the copied keys, then the merge of both launches' partials.
template <typename T>
hipError_t launch_fused_mtp(const SfaArgs& a, hipStream_t stream) {
  const int64_t rows = a.batch * a.rows_per_request;
  if (rows == 0) return hipSuccess;
  const int64_t hgroups = ceil_div(a.heads, kHeadsPerBlock);
  // (MTP3 has at least 4 rows: the copied keys always take the 8-wave shape.)
  const SplitPlan copied{8, choose_splits<8>(rows, hgroups), hgroups};
  const int s1 = overlap_splits(rows, hgroups);
  const int s2 = copied.splits;
  const int total = s1 + s2;
  const Partials p = carve(a.workspace, rows, total, a.heads);
  ScatterArgs sc{};
  sc.src_ids = a.copy_src;
  sc.dst_slots = a.copy_dst;
  sc.copy_counts = a.copy_counts;
  sc.hbm_table = a.hbm_table;
  sc.dram_table = a.dram_table;
  sc.hbm_kpe = a.hbm_kpe;
  sc.hbm_ckv = a.hbm_ckv;
  sc.dram_kpe = a.dram_kpe;
  sc.dram_ckv = a.dram_ckv;
  sc.batch = a.batch;
  sc.cap = a.copy_cap;
  sc.hbm_cols = a.hbm_cols;
  sc.dram_cols = a.dram_cols;
  sc.hbm_blocks = a.hbm_blocks;
  sc.dram_blocks = a.dram_blocks;
  const int attn_blocks = static_cast<int>(rows * s1);
  const int64_t slots = std::max(ceil_div(kCopyWgs, kCopyXcds), ceil_div(attn_blocks * hgroups, 8 - kCopyXcds));
  launch_kernel(kKernSfaMtpOverlap, sfa_mtp_overlap_kernel<T>, dim3(static_cast<uint32_t>(8 * slots)),
                dim3(kAttnThreads), stream, a, p, s1, total, sc, attn_blocks, static_cast<int>(hgroups), kCopyWgs,
                g_record_xcd_roles.load(std::memory_order_relaxed));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  launch_split<T, kKeysCopied>(kKernSfaSplitCopied, a, p, rows, copied, s1, total, stream);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  launch_combine<T>(a, p, rows, total, stream);
  return hipGetLastError();
}

}  // namespace

size_t sfa_workspace_bytes(int64_t query_rows, int64_t heads, int64_t max_kv_tokens) {
  (void)max_kv_tokens;
  const int64_t hg = ceil_div(heads, kHeadsPerBlock);
  const int64_t splits = std::max<int64_t>({choose_splits<8>(query_rows, hg), plan_split(query_rows, heads).splits,
                                            overlap_splits(query_rows, hg) + choose_splits<8>(query_rows, hg)});
  return align256(sizeof(float) * query_rows * splits * heads * kCkvDim) +
         align256(sizeof(float) * query_rows * splits * heads * 2);
}

hipError_t launch_sparse_tail_attention(const SfaArgs& a, hipStream_t stream) {
  return a.elem == Elem::kBf16 ? launch_sfa<Bf16, false>(a, stream) : launch_sfa<F16, false>(a, stream);
}

hipError_t launch_fused_copy_sfa(const SfaArgs& a, hipStream_t stream) {
  if (a.rows_per_request > 1)  // MTP3: the union misses are not tile-aligned to any one query row
    return a.elem == Elem::kBf16 ? launch_fused_mtp<Bf16>(a, stream) : launch_fused_mtp<F16>(a, stream);
  return a.elem == Elem::kBf16 ? launch_sfa<Bf16, true>(a, stream) : launch_sfa<F16, true>(a, stream);
}

void sfa_xcd_roles_record(bool on) { g_record_xcd_roles.store(on ? 1 : 0, std::memory_order_relaxed); }

hipError_t sfa_xcd_roles(uint32_t masks[2], bool reset) {
  hipError_t err = hipDeviceSynchronize();
  if (err == hipSuccess) err = hipMemcpyFromSymbol(masks, HIP_SYMBOL(g_xcd_roles), sizeof(g_xcd_roles));
  if (err == hipSuccess && reset) {
    const unsigned int zero[2] = {0u, 0u};
    err = hipMemcpyToSymbol(HIP_SYMBOL(g_xcd_roles), zero, sizeof(zero));
  }
  return err;
}

}  // namespace nvdsa
