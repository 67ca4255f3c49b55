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

}  // namespace nvdsa
