// Wave-level copy of one 576-wide latent KV row (512 CKV + 64 KPE 16-bit
// elements = 1152 bytes) between paged caches.
//
// One 64-lane wavefront moves a row with one 16-byte access per lane for the
// 1024-byte CKV part and 16-byte accesses on lanes 0..7 for the 128-byte KPE
// part, so every access is coalesced and a host-mapped source is read with
// full 64-byte PCIe requests.
#pragma once

#include "nvdsa_common.h"

namespace nvdsa {

struct RowAddr {
  int64_t src_row;  // physical row index in the DRAM caches, -1 = skip
  int64_t dst_row;  // physical row index in the HBM caches
};

// Resolve a (source token, destination slot) pair through the two block
// tables.  Any negative id, column beyond a table, or physical block outside
// its cache makes the pair a no-op, matching the skip rules of the
// reference copy (ops/kvcache_scatter_copy/op_kernel/kvcache_scatter_copy_kernel.h:141-177)
// plus an explicit physical-block bound so a bad table can never fault.
__device__ inline RowAddr resolve_pair(int32_t src, int32_t dst, const int32_t* dram_row_table,
                                       int64_t dram_cols, int64_t dram_blocks,
                                       const int32_t* hbm_row_table, int64_t hbm_cols,
                                       int64_t hbm_blocks) {
  RowAddr r{-1, -1};
  if (src < 0 || dst < 0) return r;
  const int64_t scol = src >> kBlockShift;
  const int64_t dcol = dst >> kBlockShift;
  if (scol >= dram_cols || dcol >= hbm_cols) return r;
  const int32_t sblk = dram_row_table[scol];
  const int32_t dblk = hbm_row_table[dcol];
  if (sblk < 0 || dblk < 0 || sblk >= dram_blocks || dblk >= hbm_blocks) return r;
  r.src_row = static_cast<int64_t>(sblk) * kBlock + (src & (kBlock - 1));
  r.dst_row = static_cast<int64_t>(dblk) * kBlock + (dst & (kBlock - 1));
  return r;
}

struct RowData {
  uint4 ckv;  // lane's 16 bytes of the CKV row
  uint4 kpe;  // lane's 16 bytes of the KPE row (lanes 0..7)
};

__device__ inline RowData load_row(const uint4* __restrict__ ckv, const uint4* __restrict__ kpe,
                                   int64_t row, int lane) {
  RowData d;
  d.ckv = ckv[row * (kCkvDim * 2 / 16) + lane];
  d.kpe = lane < (kKpeDim * 2 / 16) ? kpe[row * (kKpeDim * 2 / 16) + lane] : make_uint4(0, 0, 0, 0);
  return d;
}

__device__ inline void store_row(uint4* __restrict__ ckv, uint4* __restrict__ kpe, int64_t row,
                                 int lane, const RowData& d) {
  ckv[row * (kCkvDim * 2 / 16) + lane] = d.ckv;
  if (lane < (kKpeDim * 2 / 16)) kpe[row * (kKpeDim * 2 / 16) + lane] = d.kpe;
}

// A wavefront copies pairs [first, first + 4) of request b (those below
// `count`): every host load issued before any HBM store, so 4 rows of PCIe
// reads are in flight per wave.  `A` is ScatterArgs (nvdsa_kernels.h).
template <typename A>
__device__ inline void copy_pairs4(const A& a, int64_t b, int64_t first, int64_t count, int lane) {
  constexpr int kRows = 4;
  const int32_t* src_ids = a.src_ids + b * a.cap;
  const int32_t* dst_slots = a.dst_slots + b * a.cap;
  const int32_t* dram_row_table = a.dram_table + b * a.dram_cols;
  const int32_t* hbm_row_table = a.hbm_table + b * a.hbm_cols;
  RowAddr addr[kRows];
#pragma unroll
  for (int j = 0; j < kRows; ++j) {
    const int64_t i = first + j;
    addr[j] = i < count ? resolve_pair(src_ids[i], dst_slots[i], dram_row_table, a.dram_cols, a.dram_blocks,
                                       hbm_row_table, a.hbm_cols, a.hbm_blocks)
                        : RowAddr{-1, -1};
  }
  RowData data[kRows];
#pragma unroll
  for (int j = 0; j < kRows; ++j)
    if (addr[j].src_row >= 0)
      data[j] = load_row(static_cast<const uint4*>(a.dram_ckv), static_cast<const uint4*>(a.dram_kpe), addr[j].src_row,
                         lane);
#pragma unroll
  for (int j = 0; j < kRows; ++j)
    if (addr[j].src_row >= 0)
      store_row(static_cast<uint4*>(a.hbm_ckv), static_cast<uint4*>(a.hbm_kpe), addr[j].dst_row, lane, data[j]);
}

// Workgroup `wg` of `nwg` (4 waves) copies the 16-pair chunks g = wg,
// wg + nwg, ... of the concatenation of every request's copy list (a
// grid-stride loop over all chunks, so every workgroup has work until the
// lists run out).
template <typename A>
__device__ inline void scatter_copy_wg(const A& a, int wg, int nwg) {
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  int64_t base = 0;  // chunks of the requests before b
  for (int64_t b = 0; b < a.batch; ++b) {
    int64_t count = a.copy_counts[b];
    count = count < 0 ? 0 : (count > a.cap ? a.cap : count);
    const int64_t chunks = (count + 15) / 16;
    // first global chunk index >= base that is congruent to wg (mod nwg)
    const int64_t first = base + ((wg - base) % nwg + nwg) % nwg;
    for (int64_t g = first; g < base + chunks; g += nwg) copy_pairs4(a, b, (g - base) * 16 + wave * 4, count, lane);
    base += chunks;
  }
}

}  // namespace nvdsa
