// Prefill -> DRAM persistence of full KV blocks: for i < count,
//   dram_ckv[dram_ids[i]] = hbm_ckv[hbm_ids[i]]   (128 x 512 16-bit values)
//   dram_kpe[dram_ids[i]] = hbm_kpe[hbm_ids[i]]   (128 x 64)
// The reference copies one block at a time with a synchronous .copy_ per
// cache and block (nanovllm/models/glm_mla.py:883-889); here one launch moves
// every listed block.  A pair whose ids do not name a block of the caches is
// skipped.
//
// Design: the copy is bound by the host link (posted PCIe writes).  Each
// block pair (144 KiB) is split over kPieces workgroups; a thread issues all
// of its 16-byte HBM loads before its host stores, so every wave keeps
// several KiB of writes in flight, and consecutive lanes write consecutive
// 16 bytes (whole 1 KiB runs per wave store).
#include "nvdsa_common.h"
#include "nvdsa_kernels.h"

namespace nvdsa {
namespace {

constexpr int kPersistThreads = 256;
constexpr int kCkvChunks = kBlock * kCkvDim * 2 / 16;  // 8192 x 16 B per block
constexpr int kKpeChunks = kBlock * kKpeDim * 2 / 16;  // 1024
constexpr int kPairChunks = kCkvChunks + kKpeChunks;   // 9216
constexpr int kPieces = 4;
constexpr int kPieceChunks = kPairChunks / kPieces;    // 2304
constexpr int kPerThread = kPieceChunks / kPersistThreads;  // 9
static_assert(kPairChunks % kPieces == 0 && kPieceChunks % kPersistThreads == 0, "persist tiling");

__global__ __launch_bounds__(kPersistThreads) void persist_blocks_kernel(PersistArgs a) {
  const int64_t i = blockIdx.x / kPieces;
  const int piece = blockIdx.x - static_cast<int>(i * kPieces);
  const int32_t hb = a.hbm_ids[i];
  const int32_t db = a.dram_ids[i];
  if (hb < 0 || hb >= a.hbm_blocks || db < 0 || db >= a.dram_blocks) return;
  const uint4* hckv = static_cast<const uint4*>(a.hbm_ckv) + static_cast<int64_t>(hb) * kCkvChunks;
  const uint4* hkpe = static_cast<const uint4*>(a.hbm_kpe) + static_cast<int64_t>(hb) * kKpeChunks;
  uint4* dckv = static_cast<uint4*>(a.dram_ckv) + static_cast<int64_t>(db) * kCkvChunks;
  uint4* dkpe = static_cast<uint4*>(a.dram_kpe) + static_cast<int64_t>(db) * kKpeChunks;
  uint4 v[kPerThread];
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int c = piece * kPieceChunks + j * kPersistThreads + threadIdx.x;
    v[j] = c < kCkvChunks ? hckv[c] : hkpe[c - kCkvChunks];
  }
#pragma unroll
  for (int j = 0; j < kPerThread; ++j) {
    const int c = piece * kPieceChunks + j * kPersistThreads + threadIdx.x;
    if (c < kCkvChunks)
      dckv[c] = v[j];
    else
      dkpe[c - kCkvChunks] = v[j];
  }
}

}  // namespace

hipError_t launch_persist_blocks(const PersistArgs& a, hipStream_t stream) {
  if (a.count == 0) return hipSuccess;
  launch_kernel(kKernPersist, persist_blocks_kernel, dim3(static_cast<uint32_t>(a.count * kPieces)),
                dim3(kPersistThreads), stream, a);
  return hipGetLastError();
}

}  // namespace nvdsa
