// scatter_copy: DRAM (pinned, device-mapped host memory) -> HBM copy of
// latent KV rows selected by (src_id, dst_slot) pairs.
//
// Semantics follow the reference copy kernel
// (ops/kvcache_scatter_copy/op_kernel/kvcache_scatter_copy_kernel.h:48-178):
// for b < B and i < clamp(copy_counts[b], 0, cap), copy token src_ids[b,i] of
// request b's DRAM pages to slot dst_slots[b,i] of its HBM pages, CKV and KPE
// alike, skipping unresolvable pairs.
//
// Design: the copy is bound by the host link, so the kernel only has to keep
// enough 64-byte PCIe reads in flight.  Each wavefront owns kRowsPerWave
// consecutive pairs, issues all of their host loads before any HBM store, and
// every row is moved with one coalesced 16-byte access per lane.
#include "nvdsa_kernels.h"
#include "row_copy.h"

namespace nvdsa {
namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kRowsPerWave = 4;
constexpr int kRowsPerBlock = kWavesPerBlock * kRowsPerWave;

__global__ __launch_bounds__(kWavesPerBlock * kWave) void scatter_copy_kernel(ScatterArgs a,
                                                                             int64_t chunks) {
  const int64_t b = blockIdx.x / chunks;
  const int64_t chunk = blockIdx.x - b * chunks;
  int64_t count = a.copy_counts[b];
  count = count < 0 ? 0 : (count > a.cap ? a.cap : count);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t first = chunk * kRowsPerBlock + wave * kRowsPerWave;
  if (first >= count) return;

  copy_pairs4(a, b, first, count, lane);
}

}  // namespace

hipError_t launch_scatter_copy(const ScatterArgs& a, hipStream_t stream) {
  if (a.batch == 0) return hipSuccess;
  const int64_t chunks = ceil_div(a.cap, kRowsPerBlock);
  const int64_t blocks = a.batch * chunks;
  launch_kernel(kKernScatter, scatter_copy_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kWavesPerBlock * kWave),
                stream, a, chunks);
  return hipGetLastError();
}

}  // namespace nvdsa
