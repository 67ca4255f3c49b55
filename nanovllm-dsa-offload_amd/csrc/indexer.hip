// DSA indexer projection of the decode step: the LIM query rows and head
// weights of each token.
//
//   q[t, h, :]  = RoPE(q_c[t, :] . wq_b[h*D .. h*D+D-1, :]^T)   (first rope_dim dims)
//   w[t, h]     = hidden[t, :] . w_proj[h, :]^T  (x score_scale)
//
// Semantics: nanovllm/models/dsa_indexer_project.py:245-360
// (dsa_indexer_project_query_only): q rounded to 16 bits after the
// projection, then the interleaved-pair RoPE of
// ops/dsa_indexer_project/op_kernel/dsa_indexer_project_kernel.cpp:105-176
// (fp32 x*cos, fp32 rotated*sin, fp32 sum, round to nearest even), the
// weights rounded after the projection and again after the scale
// (_query_only_weights_proj_pure, :74-86).
//
// Design: the q projection is a skinny GEMM (tokens <= 64 per workgroup
// column, thousands of weight rows), bound by reading wq_b once from HBM.
// One launch covers both projections: workgroup x owns 16 rows of wq_b, and
// the head weights are spread over the same workgroups' waves, one wave per
// (token, head) dot product over hidden_size with coalesced 1 KiB loads and
// a fixed-order shuffle reduction (rather than 2 MFMA row tiles that would
// each walk all of hidden_size, or workgroups of their own that would not
// fit beside the q workgroups in one round).  In the q part the weight rows
// are the MFMA A
// operand (16 rows x 32 K per 16x16x32 step) and the tokens the B operand,
// so a lane's four accumulator values are four consecutive output rows of
// one token: the RoPE pairs (2i, 2i+1) meet in one thread after the
// cross-wave reduction.  K is walked in 256-wide chunks spread over the 8
// waves (a wave prefetches its next chunk's weight rows while it multiplies
// the current one).
#include "nvdsa_common.h"
#include "nvdsa_kernels.h"

namespace nvdsa {
namespace {

constexpr int kProjWaves = 8;
constexpr int kProjThreads = kProjWaves * kWave;
constexpr int kRowTile = 16;              // weight rows (outputs) per workgroup
constexpr int kTokTiles = 4;              // 16-token MFMA column tiles per workgroup
constexpr int kTokPerGroup = 16 * kTokTiles;
constexpr int kSteps = 8;                 // MFMA steps per chunk, 32 K each
constexpr int kKChunk = 32 * kSteps;      // 256

// The interleaved-pair rotation of one (even, odd) pair, in fp32 with every
// product and the sum rounded separately (no fused multiply-add), as the
// reference kernel's Mul / Mul / Add.
__device__ inline void rope_pair(float x0, float x1, float c0, float c1, float s0, float s1, float& y0, float& y1) {
#pragma clang fp contract(off)
  y0 = x0 * c0 + (-x1) * s0;
  y1 = x1 * c1 + x0 * s1;
}

// Head weights: wave `wid` of the weight workgroups computes
// w[t, h] = round16(hidden[t] . w_proj[h]) (x score_scale, rounded again),
// t = wid / heads, h = wid % heads.  Lane l accumulates the products of K
// indices 512j + 8l .. +7 in fp32 (ascending j, then ascending element),
// then the lanes combine in a fixed butterfly.
template <typename T>
__device__ __forceinline__ void head_weight(const IndexerArgs& a, int64_t t, int64_t h, int lane) {
  const u32x4_t* x = reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(a.hidden) + t * a.hid) + lane;
  const u32x4_t* w = reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(a.w_proj) + h * a.hid) + lane;
  constexpr int kBatch = 12;  // 12 x 2 loads in flight per lane: all of hidden_size 6144 at once
  const int64_t iters = a.hid / 512;
  float acc = 0.f;
  for (int64_t j0 = 0; j0 < iters; j0 += kBatch) {
    u32x4_t xv[kBatch], wv[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t j = j0 + u < iters ? j0 + u : iters - 1;
      xv[u] = x[64 * j];
      wv[u] = w[64 * j];
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (j0 + u < iters) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc = fmaf(T::to_float(static_cast<uint16_t>(xv[u][e])), T::to_float(static_cast<uint16_t>(wv[u][e])), acc);
          acc = fmaf(T::to_float(static_cast<uint16_t>(xv[u][e] >> 16)),
                     T::to_float(static_cast<uint16_t>(wv[u][e] >> 16)), acc);
        }
      }
    }
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) acc += __shfl_xor(acc, d, 64);
  if (lane == 0) {
    uint16_t o = T::from_float(acc);
    if (a.score_scale != 1.f) o = T::from_float(T::to_float(o) * a.score_scale);
    static_cast<uint16_t*>(a.w_out)[t * a.heads + h] = o;
  }
}

template <typename T>
__global__ __launch_bounds__(kProjThreads) void indexer_project_kernel(IndexerArgs a, int q_tiles) {
  __shared__ f32x4_t red[kProjWaves][kTokTiles][kWave];
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kRowTile;
  const uint16_t* W = static_cast<const uint16_t*>(a.wq_b);
  const uint16_t* X = static_cast<const uint16_t*>(a.q_c);
  const int64_t K = a.rank;
  const int64_t tok0 = static_cast<int64_t>(blockIdx.y) * kTokPerGroup;
  const int64_t ntok = a.tokens;
  const int ntt = static_cast<int>(min<int64_t>(kTokTiles, ceil_div(ntok - tok0, 16)));
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;

  f32x4_t acc[kTokTiles];
#pragma unroll
  for (int tt = 0; tt < kTokTiles; ++tt) acc[tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // Step s of a chunk covers K [32s, 32s+32); lane group g takes its 8
  // values at 8g (the MFMA operand layout), so one load instruction reads 64
  // contiguous bytes of each of 16 rows.  The next chunk's weight rows are
  // loaded before the current chunk's MFMAs.
  const int64_t chunks = K / kKChunk;
  const u32x4_t* wrow = reinterpret_cast<const u32x4_t*>(W + (row0 + r) * K + g * 8);
  u32x4_t wa[kSteps];
  if (wave < chunks) {
#pragma unroll
    for (int s = 0; s < kSteps; ++s) wa[s] = wrow[(wave * kKChunk + 32 * s) / 8];
  }
  // The token group's head weights ride along while those loads are in
  // flight: dot product j of the group (token tok0 + j / heads, head
  // j % heads) belongs to wave (j / q_tiles) % 8 of workgroup j % q_tiles.
  if (a.w_proj != nullptr) {
    const int64_t dots = min<int64_t>(kTokPerGroup, ntok - tok0) * a.heads;
    for (int64_t j = static_cast<int64_t>(wave) * q_tiles + blockIdx.x; j < dots;
         j += static_cast<int64_t>(kProjWaves) * q_tiles)
      head_weight<T>(a, tok0 + j / a.heads, j % a.heads, lane);
  }
  for (int64_t c = wave; c < chunks; c += kProjWaves) {
    const int64_t k0 = c * kKChunk + g * 8;
    u32x4_t xb[kTokTiles][kSteps];
#pragma unroll
    for (int tt = 0; tt < kTokTiles; ++tt) {
      if (tt >= ntt) break;  // uniform
      const int64_t t = tok0 + tt * 16 + r;
      const bool valid = t < ntok;
      const u32x4_t* xp = reinterpret_cast<const u32x4_t*>(X + (valid ? t : ntok - 1) * K + k0);
#pragma unroll
      for (int s = 0; s < kSteps; ++s) {
        const u32x4_t v = xp[4 * s];
        xb[tt][s] = valid ? v : u32x4_t{0u, 0u, 0u, 0u};
      }
    }
    u32x4_t wn[kSteps];
    const int64_t cn = c + kProjWaves;
    if (cn < chunks) {
#pragma unroll
      for (int s = 0; s < kSteps; ++s) wn[s] = wrow[(cn * kKChunk + 32 * s) / 8];
    }
#pragma unroll
    for (int tt = 0; tt < kTokTiles; ++tt) {
      if (tt >= ntt) break;
#pragma unroll
      for (int s = 0; s < kSteps; ++s)
        acc[tt] = T::mfma16(__builtin_bit_cast(typename T::vec8, wa[s]), __builtin_bit_cast(typename T::vec8, xb[tt][s]),
                            acc[tt]);
    }
#pragma unroll
    for (int s = 0; s < kSteps; ++s) wa[s] = wn[s];
  }
#pragma unroll
  for (int tt = 0; tt < kTokTiles; ++tt) red[wave][tt][lane] = acc[tt];
  __syncthreads();

  // One (even, odd) output-row pair of one token per thread.  Lane l of a
  // wave held rows 4(l>>4) .. +3 of token l&15 of each 16-token tile.
  const int p = threadIdx.x & 7;      // row pair within the tile
  const int tl = threadIdx.x >> 3;    // token within the group (0..63)
  const int64_t t = tok0 + tl;
  if (t >= ntok) return;
  const int rho = 2 * p;              // even row
  const int tt = tl >> 4;
  const int src_lane = (rho >> 2) * 16 + (tl & 15);
  float v0 = 0.f, v1 = 0.f;
#pragma unroll
  for (int w = 0; w < kProjWaves; ++w) {  // fixed order: deterministic sums
    const f32x4_t x = red[w][tt][src_lane];
    v0 += x[rho & 3];
    v1 += x[(rho & 3) + 1];
  }
  const int64_t n = row0 + rho;  // output column of the even row
  uint16_t o0 = T::from_float(v0), o1 = T::from_float(v1);
  const int64_t d = n % a.head_dim;
  if (d < a.rope_dim) {
    const uint32_t c2 = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.cos) + t * a.cos_stride + d);
    const uint32_t s2 = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.sin) + t * a.cos_stride + d);
    float y0, y1;
    rope_pair(T::to_float(o0), T::to_float(o1), T::to_float(static_cast<uint16_t>(c2)),
              T::to_float(static_cast<uint16_t>(c2 >> 16)), T::to_float(static_cast<uint16_t>(s2)),
              T::to_float(static_cast<uint16_t>(s2 >> 16)), y0, y1);
    o0 = T::from_float(y0);
    o1 = T::from_float(y1);
  }
  *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.q_out) + t * a.heads * a.head_dim + n) =
      static_cast<uint32_t>(o0) | (static_cast<uint32_t>(o1) << 16);
}

// In-place RoPE of the first rope_dim dims of every [token, head] row: one
// (even, odd) pair per thread (the reference op
// dsa_indexer_query_rope_inplace, dsa_indexer_project_kernel.cpp:60-90).
template <typename T>
__global__ __launch_bounds__(256) void indexer_rope_kernel(RopeArgs a) {
  const int64_t half = a.rope_dim / 2;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= a.rows * half) return;
  const int64_t row = i / half;
  const int64_t d = 2 * (i - row * half);
  const int64_t t = row / a.heads;
  uint32_t* qp = reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.q) + row * a.head_dim + d);
  const uint32_t x2 = *qp;
  const uint32_t c2 = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.cos) + t * a.rope_dim + d);
  const uint32_t s2 = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.sin) + t * a.rope_dim + d);
  float y0, y1;
  rope_pair(T::to_float(static_cast<uint16_t>(x2)), T::to_float(static_cast<uint16_t>(x2 >> 16)),
            T::to_float(static_cast<uint16_t>(c2)), T::to_float(static_cast<uint16_t>(c2 >> 16)),
            T::to_float(static_cast<uint16_t>(s2)), T::to_float(static_cast<uint16_t>(s2 >> 16)), y0, y1);
  *qp = static_cast<uint32_t>(T::from_float(y0)) | (static_cast<uint32_t>(T::from_float(y1)) << 16);
}

template <typename T>
hipError_t launch_project(const IndexerArgs& a, hipStream_t stream) {
  const int q_tiles = static_cast<int>(a.heads * a.head_dim / kRowTile);
  const dim3 grid(static_cast<uint32_t>(q_tiles), static_cast<uint32_t>(ceil_div(a.tokens, kTokPerGroup)));
  launch_kernel(kKernIdxProject, indexer_project_kernel<T>, grid, dim3(kProjThreads), stream, a, q_tiles);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_rope(const RopeArgs& a, hipStream_t stream) {
  const int64_t pairs = a.rows * (a.rope_dim / 2);
  launch_kernel(kKernIdxRope, indexer_rope_kernel<T>, dim3(static_cast<uint32_t>(ceil_div(pairs, 256))), dim3(256),
                stream, a);
  return hipGetLastError();
}

}  // namespace

int64_t indexer_k_chunk() { return kKChunk; }

hipError_t launch_indexer_project(const IndexerArgs& a, hipStream_t stream) {
  if (a.tokens == 0) return hipSuccess;
  return a.elem == Elem::kBf16 ? launch_project<Bf16>(a, stream) : launch_project<F16>(a, stream);
}

hipError_t launch_indexer_rope(const RopeArgs& a, hipStream_t stream) {
  if (a.rows == 0) return hipSuccess;
  return a.elem == Elem::kBf16 ? launch_rope<Bf16>(a, stream) : launch_rope<F16>(a, stream);
}

}  // namespace nvdsa
