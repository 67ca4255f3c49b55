// fused_li_manage / fused_li_manage_mtp: LightningIndexer scores, top-2048
// selection and persistent HBM-slot bookkeeping on gfx950.
//
// Per call:
//   1. lim_score_kernel  — one wavefront per 128-token index block.  The
//      block's key rows are the MFMA B operand (32 tokens x 16 dims per
//      v_mfma_f32_32x32x16), the request's index query rows the A operand
//      (staged once per workgroup in LDS), fp32 accumulation, then ReLU,
//      per-head weight and head reduction in registers.  Scores go to an fp32
//      workspace row per query; the key scan is the only large HBM stream.
//   2. management, chunked: one 512-thread workgroup per 4096-token chunk of
//      a request — the top-2048 threshold, the ordered pass over the
//      candidates against the request's pool row, victim selection, pairing
//      and pool update (MTP0: lim_hist / lim_classify; MTP3:
//      lim_threshold / lim_mtp_pass_a / lim_mtp_victims / lim_mtp_pass_b).
//
// Canonical semantics (the reference leaves victim choice and in-row order
// implementation-defined; these rules make every integer output exact):
//   score  s[t] = sum_h w[h] * max(0, q[h] . K[t])            (fp32 accumulate)
//   select S = 2048 largest s, ties at the threshold taken in ascending t.
//   cached: 0 <= pool[r,t] < C.  hits H = S cached, misses M = S not cached.
//   victims: the |M| non-hit slots of [0,C) with the smallest key, where a
//      slot held by a cached unselected token has key s[t] (MTP: max_q s_q[t])
//      and a slot held by no candidate token ranks below every score; ties in
//      ascending slot.  Victim slots are paired in ascending order with the
//      misses (MTP0: ascending t; MTP3: ordered-union order).
//   MTP0 row:  [M ascending t] ++ [H by descending old slot]
//      (reference BuildHitMissKey, ops/fused_li_manage/op_kernel/fused_li_manage_vector.h:408-416;
//       SortTopKBySlot, fused_li_manage_service_vector.h:424-451).
//   MTP3 rows: each query's 2048 tokens in ascending t, source id = t for a
//      pre-update miss else -1, slot = post-update slot
//      (ops/fused_li_manage_mtp/op_kernel/nanovllm_fused_li_manage_mtp.cpp,
//       ut_ops/test_fused_li_manage_mtp.py:789-960).
#include <cfloat>
#include <climits>

#include "nvdsa_common.h"
#include "nvdsa_kernels.h"

namespace nvdsa {
namespace {

constexpr int kScoreWaves = 4;                  // waves per score workgroup
constexpr int kQStride = kIndexDim + 8;         // padded LDS row (bank spread)
constexpr int kStageStride = 17;                // 16-byte chunks per staged key row (16 + 1 pad)
constexpr int kManageThreads = 512;
constexpr int kDigitBits = 13;                    // radix digit width
constexpr int kBins = 1 << kDigitBits;            // radix histogram bins
constexpr int kBinsPerThread = kBins / kManageThreads;
constexpr int kGatherKeys = 64;                   // radix select: bins this small are ranked directly
constexpr int kHistBits = 12;                     // MTP0: first digit of the chunked threshold search
constexpr int kHistBins = 1 << kHistBits;
constexpr int kGatherPart = 128;                  // MTP0: in-bin tokens a chunk can hand over
constexpr int kRankDirect = 512;                  // MTP0: in-bin tokens ranked pairwise by the last chunk
constexpr int kMissPart = 256;                    // MTP0: definite misses a chunk can hand over
constexpr int kInBinScan = 64;                    // MTP0 last chunk: longer in-bin miss lists are sorted
constexpr int kSpecChunks = 16;                   // MTP0 last chunk: requests of up to this many chunks ...
constexpr int kSpecEntries = 64;                  // ... read this many definite misses per chunk up front
constexpr int kSpecGather = 16;                   // ... and this many in-bin tokens
// MTP0: launches of up to this many chunks (two 512-thread workgroups per CU on
// 256 CUs) resolve each request in its last chunk; larger ones (bs=64 at 64K:
// 1024) classify in a light kernel and resolve in a second one.
constexpr int64_t kResidentChunks = 512;
constexpr int kSlotStride = kMaxCacheTokens + 1;  // 16384 entries per request
constexpr int kTableStride = kSlotStride + kManageThreads;  // workspace slot tables: + one junk word per thread
constexpr uint32_t kStateShift = 24;
constexpr uint32_t kStateFree = 0;
constexpr uint32_t kStateHit = 1;
constexpr uint32_t kStateCand = 2;
constexpr uint32_t kTokenMask = (1u << kStateShift) - 1;

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct LimWs {
  float* scores;        // [B*Q, S_cap]
  uint32_t* slot_table; // [B, kTableStride] token | state << 24
  uint32_t* slot_key;   // [B, kTableStride] score key of candidate slots
  int32_t* part_counts; // [B, parts, 8] per 4096-token chunk: MTP0 definite misses, in-bin tokens; MTP3 misses by first-selecting query, selected per query
  uint32_t* select;     // MTP3: [B*Q, 4] top-2048 threshold key, need_eq, cnt_eq, tie cutoff token
  int32_t* vslot;       // MTP3: [B, 8192] victim slots
  int32_t* nvict;       // MTP3: [B] victims found
  uint8_t* masks;       // MTP3: [B, S_cap] per-token query mask
  int32_t* done;        // MTP0: [B] chunks that finished lim_classify_kernel
  uint2* ranges;        // MTP0: [B, S_cap/128] smallest and largest score key of each 128-token block
  uint32_t* hist;       // MTP0: [B, kHistBins] first-digit histogram of the request's keys
  uint32_t* rowsel;     // MTP0: [B, 4] the request's smallest key, first-digit shift; the bin and the count above it (lim_chunks_kernel)
  uint4* gather;        // MTP0: [B, parts, kGatherPart] each chunk's (token, key, pool slot, -) in the threshold's first-digit bin
  int32_t* missl;       // MTP0: [B, parts, kMissPart] each chunk's definite misses (selected, not cached), in token order
};

// Management runs one workgroup per kChunk-token chunk of a request.
__host__ __device__ inline int64_t mtp_parts(int64_t cap) { return (cap + 4095) / 4096; }

// Workspace layout of one call; with base == nullptr only *bytes is meaningful.
LimWs lim_layout(void* base, int64_t batch, int64_t cap, int queries, size_t* bytes) {
  const uintptr_t p0 = reinterpret_cast<uintptr_t>(base);
  uintptr_t p = p0;
  auto take = [&](size_t n) {
    const uintptr_t q = p;
    p += align256(n);
    return q;
  };
  const size_t B = static_cast<size_t>(batch);
  LimWs w{};
  w.scores = reinterpret_cast<float*>(take(sizeof(float) * B * queries * cap));
  w.slot_table = reinterpret_cast<uint32_t*>(take(sizeof(uint32_t) * B * kTableStride));
  w.slot_key = reinterpret_cast<uint32_t*>(take(sizeof(uint32_t) * B * kTableStride));
  w.part_counts = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * B * mtp_parts(cap) * 8));
  if (queries > 1) {
    w.select = reinterpret_cast<uint32_t*>(take(sizeof(uint32_t) * 4 * B * queries));
    w.vslot = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * B * kUnionCap));
    w.nvict = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * B));
    w.masks = reinterpret_cast<uint8_t*>(take(B * cap));
  } else {
    w.done = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * B));
    w.ranges = reinterpret_cast<uint2*>(take(sizeof(uint2) * B * (cap / kBlock)));
    w.hist = reinterpret_cast<uint32_t*>(take(sizeof(uint32_t) * B * kHistBins));
    w.rowsel = reinterpret_cast<uint32_t*>(take(sizeof(uint32_t) * 4 * B));
    w.gather = reinterpret_cast<uint4*>(take(sizeof(uint4) * B * mtp_parts(cap) * kGatherPart));
    w.missl = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * B * mtp_parts(cap) * kMissPart));
  }
  if (bytes != nullptr) *bytes = p - p0;
  return w;
}

LimWs carve(void* base, int64_t batch, int64_t cap, int queries) { return lim_layout(base, batch, cap, queries, nullptr); }

// Row guards.  MTP0: ops/fused_li_manage/op_kernel/fused_li_manage_kernel.h:261-290,
// plus C <= 16383 (the 14-bit slot payload).  MTP3:
// ops/fused_li_manage_mtp/op_kernel/fused_li_manage_mtp_kernel.h:218-233.
__device__ inline bool lim_row_valid(int n, int c, int r, int64_t cap, int64_t pool_rows) {
  return n > 0 && n <= kMaxActualSeqLen && n <= cap && r >= 0 && r < pool_rows && c >= kTopK &&
         c <= kMaxCacheTokens && c <= n;
}
__device__ inline bool lim_mtp_row_valid(int n, int c, int r, int64_t cap, int64_t pool_rows) {
  const int required = n < kUnionCap ? n : kUnionCap;
  return n >= kTopK && n <= cap && r >= 0 && r < pool_rows && c > 0 && c >= required &&
         c <= kMaxCacheTokens && c <= n;
}

// Order-preserving 32-bit key of a score (one zero: -0 and +0 rank equal).
__device__ inline uint32_t score_key(float s) { return float_key(s == 0.f ? 0.f : s); }

// Smallest and largest of lo / hi over the wave's 64 lanes, left in lane 63.
__device__ inline void wave_minmax_to_lane63(uint32_t& lo, uint32_t& hi) {
  lo = wave_reduce_to_lane63(lo, MinU32Op{});
  hi = wave_reduce_to_lane63(hi, MaxU32Op{});
}

// Tokens each score wave takes: MTP3 (Q > 1) half a key block, MTP0 a whole one.
__host__ __device__ constexpr int score_tokens_per_wave(int q) { return q > 1 ? kBlock / 2 : kBlock; }

// ---------------------------------------------------------------------------
// 1. Scores.
// RELU = false is the first-decode initialisation score (no ReLU,
// nanovllm/models/dsa_offload_ops.py:306-311); there `fixed_n` >= 0 gives the
// candidate count of the single request and the row guards do not apply.
// For MTP0 management (Q == 1, RELU, side.ranges set) each wave also writes
// its block's smallest and largest score key, and the workgroups of a request
// zero the request's state of the chunked management kernels.
template <typename T, int HEADS, int Q, bool RELU>
__global__ __launch_bounds__(kScoreWaves * kWave) void lim_score_kernel(LimArgs a, float* scores, int mtp,
                                                                        int fixed_n, LimWs side) {
  // Tokens per wave and rows per transpose stage: MTP3 waves take half a
  // block (64 tokens) through 16-row stages, so a workgroup needs <= 53 KB of
  // LDS and a wave <= 168 registers -- three workgroups (12 waves) per CU
  // instead of two; MTP0 waves take a whole block through 32-row stages.
  constexpr int kTpw = score_tokens_per_wave(Q);
  constexpr int kStageRows = Q > 1 ? 16 : 32;
  constexpr int kTiles = kTpw / 32;
  __shared__ uint16_t qs[Q * HEADS * kQStride];
  __shared__ float ws[Q * HEADS];
  __shared__ uint4 kstage[kScoreWaves * kStageRows * kStageStride];
  // Workgroup -> (column group, request), XCD by XCD: the dispatcher deals
  // linear workgroup ids to the 8 XCDs in turn, and id p takes the
  // (p mod 8)-th eighth of the grid in order, so each XCD streams a
  // contiguous run of key blocks (when the grid divides by 8).
  int bx = blockIdx.x, by = blockIdx.y;
  if (((gridDim.x * gridDim.y) & 7) == 0) {
    const int p = blockIdx.x + gridDim.x * blockIdx.y;
    const int logical = (p & 7) * static_cast<int>((gridDim.x * gridDim.y) >> 3) + (p >> 3);
    bx = logical % static_cast<int>(gridDim.x);
    by = logical / static_cast<int>(gridDim.x);
  }
  const int b = by;
  int n = fixed_n;
  if (fixed_n < 0) {
    n = a.num_candidates[b];
    const int c = a.num_cache[b];
    const int r = a.pool_entries[b];
    const bool valid = mtp ? lim_mtp_row_valid(n, c, r, a.source_capacity, a.pool_rows)
                           : lim_row_valid(n, c, r, a.source_capacity, a.pool_rows);
    if (!valid) return;
  }
  if (static_cast<int64_t>(bx) * kScoreWaves * kTpw >= n) return;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int grp = lane >> 5;   // k-half of the MFMA operand
  const int col_lane = lane & 31;
  const int64_t t0 = (static_cast<int64_t>(bx) * kScoreWaves + wave) * kTpw;  // the wave's first token
  const int64_t col = t0 / kBlock;                                              // its key block
  const bool has_block = t0 < n;
  const int32_t phys = has_block ? a.block_table[static_cast<int64_t>(b) * a.cols + col] : -1;
  const bool key_ok = has_block && phys >= 0 && phys < a.key_blocks;

  // Prologue, every load issued before any is waited on and with no branch
  // between them (a branch makes the load-counter waits after it count the
  // slowest path): the request's Q*HEADS query rows (16 x 16-byte chunks
  // each) and weights into registers, then the wave's key block (128 rows of
  // 256 bytes), each key load instruction reading 4 whole rows (16 lanes per
  // row).  The query rows go to LDS once their (earlier) loads land, while
  // the key loads are still in flight.  The key block is read through a
  // buffer resource whose range is empty for an unmapped block, so those
  // loads return zeros instead of needing a branch.  The key loads are
  // non-temporal: a call reads each key block once, and a model reads the
  // layer's keys again only after every other layer has run, so keeping them
  // in the L2 and the Infinity Cache only evicts the lines the next kernels
  // read.  (Loading the MFMA operand layout directly -- 32 rows x 32 bytes
  // per instruction -- has the L2 fetch ~1.4x the block's bytes from HBM.
  // Native vector types: uint4 struct copies of these arrays stay in scratch
  // memory.)
  constexpr int kThreads = kScoreWaves * kWave;
  constexpr int kQLoads = Q * HEADS * 16 / kThreads;
  static_assert(Q * HEADS * 16 % kThreads == 0 && Q * HEADS <= kThreads, "score staging layout");
  const u32x4_t* qsrc = static_cast<const u32x4_t*>(a.query) + static_cast<int64_t>(b) * Q * HEADS * 16;
  u32x4_t qv[kQLoads];
#pragma unroll
  for (int k = 0; k < kQLoads; ++k) qv[k] = qsrc[k * kThreads + threadIdx.x];
  const uint16_t w16 = static_cast<const uint16_t*>(a.weights)[static_cast<int64_t>(b) * Q * HEADS +
                                                                threadIdx.x % (Q * HEADS)];
  const char* kbase = static_cast<const char*>(a.key_cache) +
                      (key_ok ? static_cast<int64_t>(phys) * kBlock * 256 + (t0 - col * kBlock) * 256 : 0);
  const __amdgpu_buffer_rsrc_t krsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kbase), 0, key_ok ? kTpw * 256 : 0, kBufferFlags);
  u32x4_t raw[kTpw / 4];
#pragma unroll
  for (int i = 0; i < kTpw / 4; ++i)  // row 4i + lane/16, chunk lane%16
    raw[i] = __builtin_amdgcn_raw_buffer_load_b128(krsrc, (i * kWave + lane) * 16, 0, kLoadNonTemporal);
#pragma unroll
  for (int k = 0; k < kQLoads; ++k) {
    const int i = k * kThreads + threadIdx.x;
    *reinterpret_cast<u32x4_t*>(&qs[(i >> 4) * kQStride + (i & 15) * 8]) = qv[k];
  }
  if (threadIdx.x < Q * HEADS) ws[threadIdx.x] = T::to_float(w16);
  // Only LDS needs ordering here; a full __syncthreads() fence would also
  // wait for the key loads.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");

  constexpr bool kRanges = Q == 1 && RELU;
  const int64_t cap = a.source_capacity;
  if constexpr (kRanges) {
    if (side.ranges != nullptr) {
      // The request's first-digit histogram and finished-chunk counter start
      // at zero; the request's ceil(n / 512) workgroups share the clearing.
      const int active = static_cast<int>(ceil_div(n, kScoreWaves * kTpw));
      uint32_t* h = side.hist + static_cast<int64_t>(b) * kHistBins;
      for (int i = bx * kThreads + threadIdx.x; i < kHistBins; i += active * kThreads)
        h[i] = 0u;
      if (bx == 0 && threadIdx.x == 0) side.done[b] = 0;
    }
  }
  if (!has_block) return;
  float* srow = scores + static_cast<int64_t>(b) * Q * cap;
  uint2* brange = nullptr;
  if constexpr (kRanges)
    if (side.ranges != nullptr) brange = side.ranges + static_cast<int64_t>(b) * (cap / kBlock) + col;
  if (!key_ok) {
    for (int q = 0; q < Q; ++q)
      for (int j = lane; j < kTpw; j += kWave)
        if (t0 + j < n) srow[q * cap + t0 + j] = -FLT_MAX;
    if (brange != nullptr && lane == 0) *brange = make_uint2(score_key(-FLT_MAX), score_key(-FLT_MAX));
    return;
  }
  // Per 32-token tile, a transpose through the wave's own LDS rows into the
  // operand layout: kb[tt][ks] = chunk 2ks+grp of row 32tt+col_lane, in
  // stages of kStageRows rows (with 16-row stages the lanes of the rows in
  // a stage read it).  Only this wave touches these rows.  A wave's LDS
  // operations are performed in its execution order, and the stores and
  // loads below may alias, so the compiler keeps their program order; no
  // fence is needed (one here keeps `raw` in scratch memory).
  uint4* st = kstage + wave * kStageRows * kStageStride;
  uint4 kb[kTiles][8];
#pragma unroll
  for (int tt = 0; tt < kTiles; ++tt) {
#pragma unroll
    for (int r2 = 0; r2 < 32 / kStageRows; ++r2) {
#pragma unroll
      for (int j = 0; j < kStageRows / 4; ++j)
        st[(4 * j + (lane >> 4)) * kStageStride + (lane & 15)] =
            __builtin_bit_cast(uint4, raw[tt * 8 + r2 * (kStageRows / 4) + j]);
      if (col_lane / kStageRows == r2) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) kb[tt][ks] = st[(col_lane % kStageRows) * kStageStride + ks * 2 + grp];
      }
    }
  }

#pragma unroll 1
  for (int q = 0; q < Q; ++q) {
    float part[kTiles] = {};
#pragma unroll
    for (int ht = 0; ht < HEADS / 32; ++ht) {
      float wv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) wv[i] = ws[q * HEADS + ht * 32 + 8 * (i >> 2) + grp * 4 + (i & 3)];
      const uint16_t* qrow = &qs[(q * HEADS + ht * 32 + col_lane) * kQStride + grp * 8];
      uint4 qa[8];
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) qa[ks] = *reinterpret_cast<const uint4*>(qrow + ks * 16);
#pragma unroll
      for (int tt = 0; tt < kTiles; ++tt) {
        f32x16_t acc = {};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
          acc = T::mfma32(__builtin_bit_cast(typename T::vec8, qa[ks]),
                          __builtin_bit_cast(typename T::vec8, kb[tt][ks]), acc);
#pragma unroll
        // ReLU as a signed-integer max on the bit pattern: negative floats
        // (and -0) are negative integers.  fmaxf would also quiet NaNs,
        // one extra instruction per element.
        for (int i = 0; i < 16; ++i)
          part[tt] += wv[i] * (RELU ? __int_as_float(max(__float_as_int(acc[i]), 0)) : acc[i]);
      }
    }
    uint32_t klo = 0xffffffffu, khi = 0u;
#pragma unroll
    for (int tt = 0; tt < kTiles; ++tt) {
      float s = xor32_op(part[tt], AddOp{});  // both halves of the head reduction
      if (s == 0.f) s = 0.f;  // one zero: -0 and +0 rank equal
      const int64_t t = t0 + tt * 32 + col_lane;
      if (grp == 0 && t < n) {
        srow[q * cap + t] = s;
        if constexpr (kRanges) {
          klo = min(klo, score_key(s));
          khi = max(khi, score_key(s));
        }
      }
    }
    if constexpr (kRanges) {
      if (brange != nullptr) {
        wave_minmax_to_lane63(klo, khi);
        if (lane == kWave - 1) *brange = make_uint2(klo, khi);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Block-wide helpers for the 512-thread manage kernels.

constexpr int kItems = 8;                          // consecutive tokens per thread in ordered passes
constexpr int kChunk = kManageThreads * kItems;    // tokens per ordered chunk
static_assert(kChunk == 4096, "mtp_parts() assumes 4096-token chunks");
constexpr int kSlotItems = 4;                      // consecutive slots per thread in slot passes
constexpr int kSlotChunk = kManageThreads * kSlotItems;

struct SelectOut {
  uint32_t thresh;  // key of the k-th largest element
  int need_eq;      // elements equal to thresh that belong to the selection
  int cnt_eq;       // elements equal to thresh (INT_MAX when not counted)
};

// Block-wide min / max of 32-bit keys (every thread gets the result; every
// thread reads the wave results itself).  LDS_ONLY: barriers that order LDS
// only.
template <bool LDS_ONLY = false>
__device__ __forceinline__ void block_minmax(uint32_t& lo, uint32_t& hi, uint32_t* red) {
  wave_minmax_to_lane63(lo, hi);
  const int wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == kWave - 1) {
    red[2 * wid] = lo;
    red[2 * wid + 1] = hi;
  }
  scan_barrier<LDS_ONLY>();
  uint32_t l = 0xffffffffu, h = 0u;
#pragma unroll
  for (int w = 0; w < 16; ++w) {
    if (w < nw) {
      l = min(l, red[2 * w]);
      h = max(h, red[2 * w + 1]);
    }
  }
  // Uniform values (readfirstlane): they steer loops that contain barriers.
  lo = __builtin_amdgcn_readfirstlane(l);
  hi = __builtin_amdgcn_readfirstlane(h);
  scan_barrier<LDS_ONLY>();  // red is reused
}

// k-th largest key among included keys, all of which lie in [kmin, kmax].
// The radix passes work on key - kmin and start at the top bit of the range,
// so the first 13-bit histogram already spreads over all 8192 bins (scores
// share sign and exponent bits; a histogram of the raw top bits would pile
// them into a few bins); a range of up to 26 bits takes two passes.
// visit(fn) calls fn(key) for every included key of the calling thread.
// Requires (#included) >= k >= 1.  `hist` must be zero on entry and is zero
// again on return (each owner clears its bins after reading them).
template <typename Visit>
__device__ __forceinline__ SelectOut radix_select_visit(int k, uint32_t kmin, uint32_t kmax, Visit visit,
                                                        uint32_t* hist,
                                        int* scratch, int* bcast) {
  if (kmax == kmin) return SelectOut{kmin, k, INT_MAX};
  const int tid = threadIdx.x;
  const int L = 32 - __clz(static_cast<int>(kmax - kmin));
  uint32_t prefix = 0, pmask = 0;
  int remaining = k, cnt_eq = 0;
#pragma unroll 1
  for (int hi = L; hi > 0; hi -= kDigitBits) {
    const int lo = hi > kDigitBits ? hi - kDigitBits : 0;
    const uint32_t dmask = (1u << (hi - lo)) - 1u;
    visit([&](uint32_t key) {
      const uint32_t d = key - kmin;
      if ((d & pmask) == prefix) atomicAdd(&hist[(d >> lo) & dmask], 1u);
    });
    __syncthreads();
    // Thread tid owns bins [tb*kBinsPerThread, +kBinsPerThread), threads in
    // descending bin order; find the bin holding the remaining-th largest.
    const int tb = kManageThreads - 1 - tid;
    int cnt[kBinsPerThread];
    int sum = 0;
#pragma unroll
    for (int j = 0; j < kBinsPerThread; ++j) {
      cnt[j] = static_cast<int>(hist[tb * kBinsPerThread + j]);
      hist[tb * kBinsPerThread + j] = 0u;  // ready for the next pass / call
      sum += cnt[j];
    }
    int total;
    int acc = block_exclusive_scan(sum, scratch, &total);
    if (acc < remaining && remaining <= acc + sum) {
#pragma unroll
      for (int j = kBinsPerThread - 1; j >= 0; --j) {
        if (acc < remaining && remaining <= acc + cnt[j]) {
          bcast[0] = tb * kBinsPerThread + j;
          bcast[1] = acc;
          bcast[2] = cnt[j];
        }
        acc += cnt[j];
      }
    }
    __syncthreads();
    prefix |= static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(bcast[0])) << lo;
    pmask |= dmask << lo;
    remaining -= __builtin_amdgcn_readfirstlane(bcast[1]);
    cnt_eq = __builtin_amdgcn_readfirstlane(bcast[2]);
    __syncthreads();
    if (lo > 0 && cnt_eq <= kGatherKeys) {
      // Few keys left in the selected bin: gather them and rank them in one
      // wave instead of running the remaining digit passes.
      if (tid == 0) bcast[3] = 0;
      __syncthreads();
      visit([&](uint32_t key) {
        const uint32_t d = key - kmin;
        if ((d & pmask) == prefix) hist[atomicAdd(&bcast[3], 1)] = d;  // cnt_eq <= kGatherKeys entries
      });
      __syncthreads();
      if (tid < kWave) {
        const uint32_t mine = tid < cnt_eq ? hist[tid] : 0u;
        int greater = 0, equal = 0;
        for (int j = 0; j < cnt_eq; ++j) {
          const uint32_t o = hist[j];
          greater += o > mine ? 1 : 0;
          equal += o == mine ? 1 : 0;
        }
        if (tid < cnt_eq && greater < remaining && remaining <= greater + equal) {  // lanes holding the answer
          bcast[0] = static_cast<int>(mine);
          bcast[1] = remaining - greater;
          bcast[2] = equal;
        }
      }
      __syncthreads();
      const uint32_t x = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(bcast[0]));
      remaining = __builtin_amdgcn_readfirstlane(bcast[1]);
      cnt_eq = __builtin_amdgcn_readfirstlane(bcast[2]);
      if (tid < kGatherKeys) hist[tid] = 0u;  // zero again for the next call
      __syncthreads();
      return SelectOut{x + kmin, remaining, cnt_eq};
    }
  }
  return SelectOut{prefix + kmin, remaining, cnt_eq};
}

// Same, with the keys supplied in groups of four: load(i, key[4], inc[4])
// for group i < ngroups, groups strided over the workgroup.
template <typename Load>
__device__ SelectOut radix_select(int ngroups, int k, uint32_t kmin, uint32_t kmax, Load load, uint32_t* hist,
                                  int* scratch, int* bcast) {
  return radix_select_visit(
      k, kmin, kmax,
      [&](auto&& fn) {
        for (int i = threadIdx.x; i < ngroups; i += kManageThreads) {
          uint32_t key[4];
          bool inc[4];
          load(i, key, inc);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (inc[e]) fn(key[e]);
        }
      },
      hist, scratch, bcast);
}

// Bitwise OR of one word per thread over the workgroup, with barriers that
// order LDS only.  `scratch` must hold blockDim/64 ints.
__device__ inline unsigned block_or_lds(unsigned v, int* scratch) {
  v = wave_reduce_to_lane63(v, OrU32Op{});
  if ((threadIdx.x & 63) == kWave - 1) scratch[threadIdx.x >> 6] = static_cast<int>(v);
  lds_barrier();
  unsigned r = 0u;
  for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) r |= static_cast<unsigned>(scratch[w]);
  lds_barrier();
  return __builtin_amdgcn_readfirstlane(r);
}

template <bool LDS_ONLY = false>
__device__ inline int block_sum(int v, int* scratch) {
  int total;
  (void)block_exclusive_scan<LDS_ONLY>(v, scratch, &total);
  return total;
}

// Exclusive block scan of four packed 16-bit counters (each chunk total must
// stay below 65536: at most kChunk per chunk here), or of any packed fields
// whose block totals fit their widths.  LDS_ONLY: barriers that order LDS
// only (global accesses in flight stay in flight).
template <bool LDS_ONLY = false>
__device__ inline uint64_t block_exclusive_scan4(uint64_t v, uint64_t* scratch, uint64_t* total) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const uint64_t x = wave_inclusive_scan(v);
  if (lane == 63) scratch[wid] = x;
  scan_barrier<LDS_ONLY>();
  uint64_t before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < 16; ++w) {
    if (w < nw) {  // every thread reads the wave totals
      const uint64_t t = scratch[w];
      before += w < wid ? t : 0;
      tot += t;
    }
  }
  *total = (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(tot >> 32))) << 32) |
           static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(tot)));
  scan_barrier<LDS_ONLY>();  // scratch is reused by the next scan
  return before + x - v;
}

__device__ inline int lane16(uint64_t v, int q) { return static_cast<int>((v >> (16 * q)) & 0xffffu); }

// Exclusive block scan of eight packed 16-bit counters (two 64-bit words;
// every counter's block total must stay below 65536).  One pass for all
// eight: DPP wave scans of the 64-bit words, the 8 wave totals go through
// LDS.  Totals are wave-uniform.
__device__ inline void block_exclusive_scan8(uint64_t (&v)[2], uint64_t* scratch, uint64_t (&total)[2]) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const uint64_t x[2] = {wave_inclusive_scan(v[0]), wave_inclusive_scan(v[1])};
  if (lane == 63) {
    scratch[2 * wid] = x[0];
    scratch[2 * wid + 1] = x[1];
  }
  __syncthreads();
  uint64_t before[2] = {0, 0}, tot[2] = {0, 0};
  for (int w = 0; w < nw; ++w) {  // every thread reads the nw wave totals
    const uint64_t t0 = scratch[2 * w], t1 = scratch[2 * w + 1];
    if (w < wid) {
      before[0] += t0;
      before[1] += t1;
    }
    tot[0] += t0;
    tot[1] += t1;
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    v[h] = before[h] + x[h] - v[h];
    total[h] = (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(tot[h] >> 32))) << 32) |
               static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(tot[h])));
  }
  __syncthreads();  // scratch is reused by the next scan
}

__device__ inline int lane16x8(const uint64_t (&v)[2], int i) { return lane16(v[i >> 2], i & 3); }

// Score keys of tokens [t, t + 4) of one score row (tokens >= n excluded).
__device__ inline void load_score_keys(const float* s, int n, int t, uint32_t* key, bool* inc) {
  if (t + 3 < n) {
    const float4 v = *reinterpret_cast<const float4*>(s + t);
    key[0] = score_key(v.x);
    key[1] = score_key(v.y);
    key[2] = score_key(v.z);
    key[3] = score_key(v.w);
    inc[0] = inc[1] = inc[2] = inc[3] = true;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      inc[e] = t + e < n;
      key[e] = inc[e] ? score_key(s[t + e]) : 0u;
    }
  }
}

// Eight consecutive tokens [t0, t0 + 8): score keys and pool slots.
__device__ inline void load_tokens8(const float* s, const int32_t* pool, int n, int t0, uint32_t* u, int32_t* slot,
                                    bool* in) {
  if (t0 + kItems <= n) {
    const float4 a = *reinterpret_cast<const float4*>(s + t0);
    const float4 b = *reinterpret_cast<const float4*>(s + t0 + 4);
    const int4 pa = *reinterpret_cast<const int4*>(pool + t0);
    const int4 pb = *reinterpret_cast<const int4*>(pool + t0 + 4);
    u[0] = score_key(a.x); u[1] = score_key(a.y); u[2] = score_key(a.z); u[3] = score_key(a.w);
    u[4] = score_key(b.x); u[5] = score_key(b.y); u[6] = score_key(b.z); u[7] = score_key(b.w);
    slot[0] = pa.x; slot[1] = pa.y; slot[2] = pa.z; slot[3] = pa.w;
    slot[4] = pb.x; slot[5] = pb.y; slot[6] = pb.z; slot[7] = pb.w;
#pragma unroll
    for (int e = 0; e < kItems; ++e) in[e] = true;
  } else {
#pragma unroll
    for (int e = 0; e < kItems; ++e) {
      in[e] = t0 + e < n;
      u[e] = in[e] ? score_key(s[t0 + e]) : 0u;
      slot[e] = in[e] ? pool[t0 + e] : -1;
    }
  }
}

// Victim slots: the m non-hit slots of [0, c) with the smallest key (free
// slots first), ascending slot on ties, written in ascending slot order to
// vslot[0..min(m, #non-hit)); with vevict, vevict[i] = the unselected token
// that held slot vslot[i] (-1 for a free slot).  Returns the number written.
__device__ __forceinline__ int select_victims(int c, int m, const uint32_t* stab, const uint32_t* skey, int* vslot, uint32_t* hist,
                              int* scratch, int* bcast, uint32_t* red, int* vevict = nullptr) {
  const int tid = threadIdx.x;
  if (m <= 0) return 0;
  // inverted keys: the smallest score is the largest inverted key; free slots
  // (key 0 before inversion) rank first.
  auto inv_key = [&](int i, uint32_t& key) -> bool {
    const uint32_t st = stab[i] >> kStateShift;
    if (st == kStateHit) return false;
    key = ~(st == kStateFree ? 0u : skey[i]);
    return true;
  };
  int local = 0;
  uint32_t lo = 0xffffffffu, hi = 0u;
  for (int i = tid; i < c; i += kManageThreads) {
    uint32_t key;
    if (inv_key(i, key)) {
      ++local;
      lo = min(lo, key);
      hi = max(hi, key);
    }
  }
  const int nonhit = block_sum(local, scratch);
  const bool take_all = m >= nonhit;
  SelectOut sel{0, 0, 0};
  if (!take_all) {
    block_minmax(lo, hi, red);
    sel = radix_select(
        static_cast<int>(ceil_div(c, 4)), m, lo, hi,
        [&](int g, uint32_t* key, bool* inc) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = 4 * g + e;
            inc[e] = i < c && inv_key(i, key[e]);
          }
        },
        hist, scratch, bcast);
  }
  const bool need_rank = !take_all && sel.cnt_eq != sel.need_eq;
  int run = 0, eq_run = 0;
  for (int base = 0; base < c; base += kSlotChunk) {
    const int i0 = base + tid * kSlotItems;
    unsigned vmask = 0, eqmask = 0;
#pragma unroll
    for (int e = 0; e < kSlotItems; ++e) {
      uint32_t key = 0;
      const bool nh = i0 + e < c && inv_key(i0 + e, key);
      if (take_all) {
        if (nh) vmask |= 1u << e;
      } else if (nh) {
        if (key > sel.thresh) vmask |= 1u << e;
        if (key == sel.thresh) {
          if (need_rank) eqmask |= 1u << e;
          else vmask |= 1u << e;
        }
      }
    }
    if (need_rank) {
      int tot;
      int r = eq_run + block_exclusive_scan(__popc(eqmask), scratch, &tot);
#pragma unroll
      for (int e = 0; e < kSlotItems; ++e)
        if ((eqmask >> e) & 1u) {
          if (r < sel.need_eq) vmask |= 1u << e;
          ++r;
        }
      eq_run += tot;
    }
    int tot;
    int pos = run + block_exclusive_scan(__popc(vmask), scratch, &tot);
#pragma unroll
    for (int e = 0; e < kSlotItems; ++e)
      if ((vmask >> e) & 1u) {
        if (pos < m) {
          vslot[pos] = i0 + e;
          if (vevict != nullptr) {
            const uint32_t ent = stab[i0 + e];
            vevict[pos] = (ent >> kStateShift) == kStateCand ? static_cast<int>(ent & kTokenMask) : -1;
          }
        }
        ++pos;
      }
    run += tot;
  }
  __syncthreads();
  return run < m ? run : m;
}

// One ordered step of the tie-cutoff search: this thread's tokens
// [t0, t0 + 32) with key == thresh are the set bits of eqm (bit e = token
// t0 + e); `before` ties precede this step.  The thread holding the tie of
// rank `want` (0-based, ascending token) writes its token to bcast[3].
// Returns the ties seen through this step.  Contains block barriers.
__device__ inline int tie_cutoff_step(unsigned eqm, int t0, int want, int before, int* scratch, int* bcast) {
  int tot;
  const int rk = before + block_exclusive_scan(__popc(eqm), scratch, &tot);
  if (rk <= want && want < rk + __popc(eqm)) {
    unsigned m = eqm;
    for (int k = rk; k < want; ++k) m &= m - 1u;
    bcast[3] = t0 + __builtin_ctz(m);
  }
  return before + tot;
}

// Thread t's slot states and score keys of slots [t*ITEMS, (t+1)*ITEMS), one
// vector load each (tables readable up to ITEMS * kManageThreads entries).
template <int ITEMS>
__device__ __forceinline__ void load_slot_regs(const uint32_t* stab, const uint32_t* skey, uint32_t (&st)[ITEMS],
                                               uint32_t (&kv)[ITEMS]) {
  static_assert(ITEMS % 4 == 0, "vector loads of four slots");
  const int i0 = threadIdx.x * ITEMS;
#pragma unroll
  for (int j = 0; j < ITEMS / 4; ++j) {
    const uint4 a = *reinterpret_cast<const uint4*>(stab + i0 + 4 * j);
    const uint4 b = *reinterpret_cast<const uint4*>(skey + i0 + 4 * j);
    st[4 * j] = a.x; st[4 * j + 1] = a.y; st[4 * j + 2] = a.z; st[4 * j + 3] = a.w;
    kv[4 * j] = b.x; kv[4 * j + 1] = b.y; kv[4 * j + 2] = b.z; kv[4 * j + 3] = b.w;
  }
}

template <int ITEMS>
__device__ __forceinline__ void load_slot_states(const uint32_t* stab, uint32_t (&st)[ITEMS]) {
  static_assert(ITEMS % 4 == 0, "vector loads of four slots");
  const int i0 = threadIdx.x * ITEMS;
#pragma unroll
  for (int j = 0; j < ITEMS / 4; ++j) {
    const uint4 a = *reinterpret_cast<const uint4*>(stab + i0 + 4 * j);
    st[4 * j] = a.x; st[4 * j + 1] = a.y; st[4 * j + 2] = a.z; st[4 * j + 3] = a.w;
  }
}

// select_victims with the slot states and keys held in registers (from
// load_slot_regs): thread t owns slots [t*ITEMS, (t+1)*ITEMS) (slot order =
// thread-major order).  Same result as select_victims; requires
// c <= ITEMS * kManageThreads.
template <int ITEMS, bool LDS_ONLY = false>
__device__ __forceinline__ int select_victims_in_regs(int c, int m, const uint32_t (&st)[ITEMS],
                                                      const uint32_t (&kv)[ITEMS], int* vslot, uint32_t* hist,
                                                      int* scratch, int* bcast, uint32_t* red, int* vevict) {
  const int tid = threadIdx.x;
  if (m <= 0) return 0;
  const int i0 = tid * ITEMS;
  uint32_t key[ITEMS];
  unsigned nh = 0u;  // non-hit slots (victim candidates) below c
#pragma unroll
  for (int e = 0; e < ITEMS; ++e) {
    const uint32_t state = st[e] >> kStateShift;
    key[e] = ~(state == kStateFree ? 0u : kv[e]);  // smallest score = largest inverted key; free slots first
    if (i0 + e < c && state != kStateHit) nh |= 1u << e;
  }
  uint32_t lo = 0xffffffffu, hi = 0u;
#pragma unroll
  for (int e = 0; e < ITEMS; ++e)
    if ((nh >> e) & 1u) {
      lo = min(lo, key[e]);
      hi = max(hi, key[e]);
    }
  const int nonhit = block_sum<LDS_ONLY>(__popc(nh), scratch);
  const bool take_all = m >= nonhit;
  SelectOut sel{0, 0, 0};
  if (!take_all) {
    block_minmax(lo, hi, red);
    sel = radix_select_visit(
        m, lo, hi,
        [&](auto&& fn) {
#pragma unroll
          for (int e = 0; e < ITEMS; ++e)
            if ((nh >> e) & 1u) fn(key[e]);
        },
        hist, scratch, bcast);
  }
  unsigned vmask = 0u, eqmask = 0u;
  if (take_all) {
    vmask = nh;
  } else {
#pragma unroll
    for (int e = 0; e < ITEMS; ++e)
      if ((nh >> e) & 1u) {
        if (key[e] > sel.thresh) vmask |= 1u << e;
        if (key[e] == sel.thresh) eqmask |= 1u << e;
      }
    if (sel.cnt_eq != sel.need_eq) {  // ties at the threshold: lowest slots first
      int tot;
      int r = block_exclusive_scan<LDS_ONLY>(__popc(eqmask), scratch, &tot);
#pragma unroll
      for (int e = 0; e < ITEMS; ++e)
        if ((eqmask >> e) & 1u) {
          if (r < sel.need_eq) vmask |= 1u << e;
          ++r;
        }
    } else {
      vmask |= eqmask;
    }
  }
  int tot;
  int pos = block_exclusive_scan<LDS_ONLY>(__popc(vmask), scratch, &tot);
#pragma unroll
  for (int e = 0; e < ITEMS; ++e)
    if ((vmask >> e) & 1u) {
      if (pos < m) {
        vslot[pos] = i0 + e;
        if (vevict != nullptr)
          vevict[pos] = (st[e] >> kStateShift) == kStateCand ? static_cast<int>(st[e] & kTokenMask) : -1;
      }
      ++pos;
    }
  scan_barrier<LDS_ONLY>();
  return tot < m ? tot : m;
}

template <int ITEMS>
__device__ __forceinline__ int select_victims_regs(int c, int m, const uint32_t* stab, const uint32_t* skey, int* vslot,
                                                   uint32_t* hist, int* scratch, int* bcast, uint32_t* red,
                                                   int* vevict = nullptr) {
  if (m <= 0) return 0;
  uint32_t st[ITEMS], kv[ITEMS];
  load_slot_regs<ITEMS>(stab, skey, st, kv);
  return select_victims_in_regs<ITEMS>(c, m, st, kv, vslot, hist, scratch, bcast, red, vevict);
}

// ---------------------------------------------------------------------------
// Top-2048 threshold of the score row s[0, n) (the row buffer holds cap >= n
// entries).  RES > 0 keeps the row's keys in registers (RES chunks of 4096
// tokens, n <= RES * kChunk) for the radix passes; RES == 0 streams them
// from memory on every pass.  `hist` must be zero on entry and is zero again
// on return.
template <int RES>
__device__ __forceinline__ SelectOut row_threshold(const float* s, int n, int64_t cap, uint32_t* hist, int* scratch,
                                                   int* bcast, uint32_t* red) {
  const int tid = threadIdx.x;
  if constexpr (RES > 0) {
    uint32_t u[RES][kItems];
#pragma unroll
    for (int ch = 0; ch < RES; ++ch) {  // all loads first (redirected past cap, ignored: t >= n)
      const int t0 = ch * kChunk + tid * kItems;
      const int64_t tl = t0 < cap ? t0 : cap - kItems;
      const uint4 x = *reinterpret_cast<const uint4*>(s + tl);
      const uint4 y = *reinterpret_cast<const uint4*>(s + tl + 4);
      u[ch][0] = x.x; u[ch][1] = x.y; u[ch][2] = x.z; u[ch][3] = x.w;
      u[ch][4] = y.x; u[ch][5] = y.y; u[ch][6] = y.z; u[ch][7] = y.w;
    }
    uint32_t lo = 0xffffffffu, hi = 0u;
#pragma unroll
    for (int ch = 0; ch < RES; ++ch)
#pragma unroll
      for (int e = 0; e < kItems; ++e) {
        u[ch][e] = score_key(__uint_as_float(u[ch][e]));
        if (ch * kChunk + tid * kItems + e < n) {
          lo = min(lo, u[ch][e]);
          hi = max(hi, u[ch][e]);
        }
      }
    block_minmax(lo, hi, red);
    // The first digit pass and, when the k-th largest key's bin holds at most
    // kGatherKeys keys, its ranking among them.  The counting pass has no
    // branch per key (the general passes below test each key's prefix and
    // bounds under an exec mask): chunks wholly past n are skipped, and a key
    // past n in the last chunk counts into one of kWave bins past kBins (by
    // lane, against same-address contention), which no scan reads.  The same bins, ranks and outputs as radix_select_visit.
    if (hi != lo) {
      const int L = 32 - __clz(static_cast<int>(hi - lo));
      const int sh = L > kDigitBits ? L - kDigitBits : 0;
      // (An opaque copy of lo: the compiler would otherwise keep every key's
      // difference key - lo from this pass for the later ones, 128 registers.)
      uint32_t lo1 = lo;
      asm volatile("" : "+s"(lo1));
#pragma unroll
      for (int ch = 0; ch < RES; ++ch) {
        if (ch * kChunk >= n) break;  // (uniform)
#pragma unroll
        for (int e = 0; e < kItems; ++e) {
          const bool in = ch * kChunk + tid * kItems + e < n;
          atomicAdd(&hist[in ? (u[ch][e] - lo1) >> sh : kBins + (tid & (kWave - 1))], 1u);
        }
      }
      __syncthreads();
      // Thread tid owns bins [tb kBinsPerThread, +kBinsPerThread), tb = 511 - tid:
      // ascending threads scan descending bins.
      const int tb = kManageThreads - 1 - tid;
      int cnt[kBinsPerThread];
      int sum = 0;
#pragma unroll
      for (int j = 0; j < kBinsPerThread; ++j) {
        cnt[j] = static_cast<int>(hist[tb * kBinsPerThread + j]);
        hist[tb * kBinsPerThread + j] = 0u;
        sum += cnt[j];
      }
      if (tid < kWave) hist[kBins + tid] = 0u;
      int total;
      int acc = block_exclusive_scan(sum, scratch, &total);
      if (acc < kTopK && kTopK <= acc + sum) {
#pragma unroll
        for (int j = kBinsPerThread - 1; j >= 0; --j) {
          if (acc < kTopK && kTopK <= acc + cnt[j]) {
            bcast[0] = tb * kBinsPerThread + j;
            bcast[1] = acc;
            bcast[2] = cnt[j];
          }
          acc += cnt[j];
        }
      }
      __syncthreads();
      const uint32_t bin = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(bcast[0]));
      const int remaining = kTopK - __builtin_amdgcn_readfirstlane(bcast[1]);
      const int inbin = __builtin_amdgcn_readfirstlane(bcast[2]);
      __syncthreads();  // bcast is reused
      if (inbin <= kGatherKeys) {
        if (tid == 0) bcast[3] = 0;
        __syncthreads();
#pragma unroll
        for (int ch = 0; ch < RES; ++ch)
#pragma unroll
          for (int e = 0; e < kItems; ++e) {
            const uint32_t d = u[ch][e] - lo;
            if (ch * kChunk + tid * kItems + e < n && (d >> sh) == bin)
              hist[atomicAdd(&bcast[3], 1)] = d;  // at most inbin <= kGatherKeys entries
          }
        __syncthreads();
        if (tid < kWave) {
          const uint32_t mine = tid < inbin ? hist[tid] : 0u;
          int greater = 0, equal = 0;
          for (int j = 0; j < inbin; ++j) {
            const uint32_t o = hist[j];
            greater += o > mine ? 1 : 0;
            equal += o == mine ? 1 : 0;
          }
          if (tid < inbin && greater < remaining && remaining <= greater + equal) {  // lanes holding the answer
            bcast[0] = static_cast<int>(mine);
            bcast[1] = remaining - greater;
            bcast[2] = equal;
          }
        }
        __syncthreads();
        const uint32_t x = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(bcast[0]));
        const int need = __builtin_amdgcn_readfirstlane(bcast[1]);
        const int eq = __builtin_amdgcn_readfirstlane(bcast[2]);
        if (tid < kGatherKeys) hist[tid] = 0u;  // zero again for the next call
        __syncthreads();
        return SelectOut{x + lo, need, eq};
      }
      // More than kGatherKeys keys in the bin (heavy ties): the general passes
      // from the start (the histogram is zero again).
    }
    return radix_select_visit(
        kTopK, lo, hi,
        [&](auto&& fn) {
#pragma unroll
          for (int ch = 0; ch < RES; ++ch)
#pragma unroll
            for (int e = 0; e < kItems; ++e)
              if (ch * kChunk + tid * kItems + e < n) fn(u[ch][e]);
        },
        hist, scratch, bcast);
  } else {
    const int ngroups = static_cast<int>(ceil_div(n, 4));
    uint32_t lo = 0xffffffffu, hi = 0u;
    for (int g = tid; g < ngroups; g += kManageThreads) {
      uint32_t key[4];
      bool inc[4];
      load_score_keys(s, n, 4 * g, key, inc);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (inc[e]) {
          lo = min(lo, key[e]);
          hi = max(hi, key[e]);
        }
    }
    block_minmax(lo, hi, red);
    return radix_select(
        ngroups, kTopK, lo, hi, [&](int g, uint32_t* key, bool* inc) { load_score_keys(s, n, 4 * g, key, inc); },
        hist, scratch, bcast);
  }
}

// Top-2048 threshold of one (request, query) score row, written to the
// workspace for the MTP3 management kernels.  One workgroup per row; RES > 0
// keeps the row's keys in registers (RES chunks of 4096 tokens).
template <int RES>
__global__ __launch_bounds__(kManageThreads) void lim_threshold_kernel(LimArgs a, LimWs w, int queries, int min_n) {
  __shared__ uint32_t hist[kBins + kWave];  // (+ the bins that keys past n count into)
  __shared__ int scratch[kManageThreads / 64 + 1];
  __shared__ uint32_t red[2 * (kManageThreads / 64) + 2];
  __shared__ int bcast[4];
  const int b = blockIdx.x / queries;
  const int q = blockIdx.x - b * queries;
  const int tid = threadIdx.x;
  const int n = a.num_candidates[b];
  const int c = a.num_cache[b];
  const int r = a.pool_entries[b];
  const bool valid = queries > 1 ? lim_mtp_row_valid(n, c, r, a.source_capacity, a.pool_rows)
                                 : lim_row_valid(n, c, r, a.source_capacity, a.pool_rows);
  if (!valid || n < min_n) return;
  const int64_t cap = a.source_capacity;
  const float* s = w.scores + (static_cast<int64_t>(b) * queries + q) * cap;
  for (int i = tid; i < kBins + kWave; i += kManageThreads) hist[i] = 0u;
  const SelectOut sel = row_threshold<RES>(s, n, cap, hist, scratch, bcast, red);
  // Ties at the threshold go to the lowest tokens: a token with key ==
  // thresh is selected iff token <= cutoff (INT_MAX when all ties are taken).
  int cutoff = INT_MAX;
  if (sel.need_eq != sel.cnt_eq) {  // ties at the threshold (rare): one ordered pass finds the last selected
    const int ngroups = static_cast<int>(ceil_div(n, 4));
    int before = 0;
    for (int g0 = 0; g0 < ngroups; g0 += kManageThreads) {
      const int g = g0 + tid;
      unsigned eqm = 0u;
      if (g < ngroups) {
        uint32_t key[4];
        bool inc[4];
        load_score_keys(s, n, 4 * g, key, inc);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (inc[e] && key[e] == sel.thresh) eqm |= 1u << e;
      }
      before = tie_cutoff_step(eqm, 4 * g, sel.need_eq - 1, before, scratch, bcast);
    }
    __syncthreads();
    cutoff = bcast[3];
  }
  if (tid == 0) {
    uint32_t* out = w.select + (static_cast<int64_t>(b) * queries + q) * 4;
    out[0] = sel.thresh;
    out[1] = static_cast<uint32_t>(sel.need_eq);
    out[2] = static_cast<uint32_t>(sel.cnt_eq);
    out[3] = static_cast<uint32_t>(cutoff);
  }
  // The MTP3 passes start from an all-free slot table.
  if (q == 0) {
    uint32_t* stab = w.slot_table + static_cast<int64_t>(b) * kTableStride;
    for (int i = tid; i < c; i += kManageThreads) stab[i] = kStateFree;
  }
}

// ---------------------------------------------------------------------------
// 2a. MTP0 management, two chunked kernels after the scores, one 512-thread
// workgroup per 4096-token chunk of a request.  (One workgroup per request
// keeps every pass over the request's tokens on one CU, where each pass is
// bound by that CU's vector ALUs: 26 us at 32768 candidates.)
//   lim_hist      the first radix digit (kHistBits wide, relative to the
//                 request's key range, which the score kernel's per-block
//                 ranges give) of every key, into the request's histogram
//                 (LDS, then device atomics); also resets the slot table.
//   lim_classify  every chunk finds the bin holding the 2048th largest key
//                 from the histogram and classifies its tokens outside that
//                 bin (above: selected, below: not): cached tokens go to the
//                 slot table; definite misses (selected, not cached) and the
//                 tokens in the bin are handed over, in token order, in the
//                 chunk's slices of two workspace lists.  The last chunk of
//                 the request to finish (a device-scope counter, nobody
//                 waits) resolves the threshold among the in-bin tokens (ties
//                 to the lower token), classifies them, selects the victims,
//                 and writes the whole output row and the pool update.
// The score kernel zeroes each request's histogram and finished-chunk counter.
constexpr int kHistPerThread = kHistBins / kManageThreads;  // lim_classify: first-digit bins per thread
static_assert(kHistBins % kManageThreads == 0 && (kHistPerThread == 2 || kHistPerThread % 4 == 0),
              "lim_classify: whole vector loads of first-digit bins per thread");
static_assert(kChunk == 4096, "the gather list holds one chunk's worth of tokens");

__device__ inline bool mtp0_selected(uint32_t key, int t, uint32_t thr, int cutoff) {
  return key > thr || (key == thr && t <= cutoff);
}

__device__ inline int hist_shift(uint32_t lo, uint32_t hi) {
  const int bits = hi == lo ? 0 : 32 - __clz(static_cast<int>(hi - lo));
  return bits > kHistBits ? bits - kHistBits : 0;
}

// Score keys of tokens [t0, t0 + 8) (tokens >= n: in = false).
__device__ inline void load_keys8(const float* s, int n, int t0, uint32_t* u, bool* in) {
  if (t0 + kItems <= n) {
    const float4 x = *reinterpret_cast<const float4*>(s + t0);
    const float4 y = *reinterpret_cast<const float4*>(s + t0 + 4);
    u[0] = score_key(x.x); u[1] = score_key(x.y); u[2] = score_key(x.z); u[3] = score_key(x.w);
    u[4] = score_key(y.x); u[5] = score_key(y.y); u[6] = score_key(y.z); u[7] = score_key(y.w);
#pragma unroll
    for (int e = 0; e < kItems; ++e) in[e] = true;
  } else {
#pragma unroll
    for (int e = 0; e < kItems; ++e) {
      in[e] = t0 + e < n;
      u[e] = in[e] ? score_key(s[t0 + e]) : 0u;
    }
  }
}

__global__ __launch_bounds__(kManageThreads) void lim_hist_kernel(LimArgs a, LimWs w, int parts) {
  __shared__ uint32_t hist[kHistBins];
  __shared__ uint32_t red[2 * (kManageThreads / 64) + 2];
  const int b = blockIdx.x / parts;
  const int part = blockIdx.x - b * parts;
  const int tid = threadIdx.x;
  const int n = a.num_candidates[b];
  const int c = a.num_cache[b];
  const int r = a.pool_entries[b];
  if (!lim_row_valid(n, c, r, a.source_capacity, a.pool_rows)) {
    if (part == 0 && tid == 0) a.miss_counts[b] = 0;
    return;
  }
  uint32_t* stab = w.slot_table + static_cast<int64_t>(b) * kTableStride;
  for (int i = part * kManageThreads + tid; i < c; i += parts * kManageThreads) stab[i] = kStateFree;
  if (part * kChunk >= n) return;
  const int64_t cap = a.source_capacity;
  uint32_t u[kItems];
  bool in[kItems];
  load_keys8(w.scores + static_cast<int64_t>(b) * cap, n, part * kChunk + tid * kItems, u, in);
  const uint2* rg = w.ranges + static_cast<int64_t>(b) * (cap / kBlock);
  const int nblocks = static_cast<int>(ceil_div(n, kBlock));
  uint32_t lo = 0xffffffffu, hi = 0u;
  for (int i = tid; i < nblocks; i += kManageThreads) {
    const uint2 v = rg[i];
    lo = min(lo, v.x);
    hi = max(hi, v.y);
  }
  for (int i = tid; i < kHistBins; i += kManageThreads) hist[i] = 0u;
  block_minmax<true>(lo, hi, red);  // its barriers also order the clearing before the counts (the key loads stay in flight)
  const int shift = hist_shift(lo, hi);
  if (part == 0 && tid == 0) {
    w.rowsel[4 * b] = lo;
    w.rowsel[4 * b + 1] = static_cast<uint32_t>(shift);
  }
#pragma unroll
  for (int e = 0; e < kItems; ++e)
    if (in[e]) atomicAdd(&hist[(u[e] - lo) >> shift], 1u);
  __syncthreads();
  uint32_t* gh = w.hist + static_cast<int64_t>(b) * kHistBins;
  for (int i = tid; i < kHistBins; i += kManageThreads) {
    const uint32_t v = hist[i];
    if (v != 0u) atomicAdd(&gh[i], v);
  }
}

// The hit half of an MTP0 output row: positions m, m+1, ... get the hits by
// descending old slot (reference BuildHitMissKey order), the positions a
// corrupt pool (duplicate slots) leaves unfilled get -1, and miss_counts[b]
// = m.
__device__ __forceinline__ void write_hit_rows(const LimArgs& a, int b, int c, int m, const uint32_t* stab,
                                               int* scratch) {
  const int tid = threadIdx.x;
  int32_t* out_src = a.topk_src + static_cast<int64_t>(b) * kTopK;
  int32_t* out_dst = a.topk_dst + static_cast<int64_t>(b) * kTopK;
  // Position p of the descending scan is slot c-1-p.
  int hit_run = 0;
  for (int base = 0; base < c; base += kSlotChunk) {
    const int p0 = base + tid * kSlotItems;
    unsigned hmask = 0;
    uint32_t ent[kSlotItems];
#pragma unroll
    for (int e = 0; e < kSlotItems; ++e) {
      const int i = c - 1 - (p0 + e);
      ent[e] = i >= 0 ? stab[i] : 0u;
      if (i >= 0 && (ent[e] >> kStateShift) == kStateHit) hmask |= 1u << e;
    }
    int tot;
    int pos = m + hit_run + block_exclusive_scan(__popc(hmask), scratch, &tot);
#pragma unroll
    for (int e = 0; e < kSlotItems; ++e)
      if ((hmask >> e) & 1u) {
        if (pos < kTopK) {
          out_src[pos] = static_cast<int32_t>(ent[e] & kTokenMask);
          out_dst[pos] = c - 1 - (p0 + e);
        }
        ++pos;
      }
    hit_run += tot;
  }
  // Positions a corrupt pool (duplicate slots) left unfilled.
  for (int pos = m + hit_run + tid; pos < kTopK; pos += kManageThreads) {
    out_src[pos] = -1;
    out_dst[pos] = -1;
  }
  if (tid == 0) a.miss_counts[b] = m;
}

// LDS of lim_classify_kernel's last chunk (mtp0_resolve).  `region` holds, in
// turn, the in-bin ranking lists, the radix histogram of the selects and the
// ordered miss list.
struct ResolveLds {
  uint32_t* region;   // kBins words
  int* scratch;
  uint64_t* scratch64;
  uint32_t* red;
  int* bcast;
  int* cdm;    // [active] definite misses of each chunk
  int* cim;    // [active] in-bin misses of each chunk; from step 4 each thread's hit slots below its own
  int* doff;   // [active] offset of each chunk's definite misses in dmiss
  int* goff;   // [active] offset of each chunk's in-bin tokens, then the misses before each chunk
  int* dmiss;  // [kTopK] definite misses, chunk by chunk (each in token order)
  int* ibm;    // [kTopK] in-bin misses, any order
  int* nibm;
  int* vsl;    // [kTopK] victim slots
  int* vev;    // [kTopK] token each victim evicts, or -1
};

// Last chunk p with off[p] <= f among chunks [0, active) (off ascending).
__device__ inline int chunk_of(const int* off, int active, int f) {
  int lo_p = 0, hi_p = active - 1;
  while (lo_p < hi_p) {
    const int mid = (lo_p + hi_p + 1) >> 1;
    if (off[mid] <= f) lo_p = mid;
    else hi_p = mid - 1;
  }
  return lo_p;
}

// The last chunk of a request in lim_classify_kernel: the threshold among the
// tokens of the first-digit bin `bin` (the k-th largest of them is the
// request's 2048th largest key), their classification, the victims, and the
// whole output row with the pool update.  counts[p * 8] holds chunk p's
// definite-miss count, counts[p * 8 + 1] its in-bin token count; its slices
// of the hand-over lists hold the first kMissPart / kGatherPart of them.
__device__ __forceinline__ void mtp0_resolve(const LimArgs& a, const LimWs& w, int b, int n, int c, int r, int parts,
                                             int active, uint32_t bin, int k, uint32_t lo, int shift,
                                             const ResolveLds& L) {
  const int tid = threadIdx.x;
  const int64_t cap = a.source_capacity;
  const float* s = w.scores + static_cast<int64_t>(b) * cap;
  int32_t* pool = a.pool + static_cast<int64_t>(r) * cap;
  uint32_t* stab = w.slot_table + static_cast<int64_t>(b) * kTableStride;
  uint32_t* skey = w.slot_key + static_cast<int64_t>(b) * kTableStride;
  const int32_t* counts = w.part_counts + static_cast<int64_t>(b) * parts * 8;
  int32_t* out_src = a.topk_src + static_cast<int64_t>(b) * kTopK;
  int32_t* out_dst = a.topk_dst + static_cast<int64_t>(b) * kTopK;

  // 1. One round trip: the chunk counts (active <= kManageThreads: one chunk
  //    per thread), the first entries of every chunk's hand-over slices (when
  //    active <= kSpecChunks: 32 threads per chunk), and the slot states and
  //    keys the victims are chosen from.  Everything lands in LDS at once (the
  //    in-bin tokens then update their slots there), so no register holds it
  //    across the scans.
  constexpr int kSlotRegs = 4;  // budgets up to kSlotRegs * kManageThreads slots keep their states in registers
  const bool slots_in_regs = c <= kSlotRegs * kManageThreads;
  const bool keyed = c > kTopK;  // victims are chosen by key; at c = kTopK every non-hit slot is one
  const bool spec = active <= kSpecChunks;
  const int sp = tid >> 5, si = tid & 31;
  uint32_t* lkey = L.region;
  int* ltok = reinterpret_cast<int*>(L.region + kRankDirect);
  int* lslot = reinterpret_cast<int*>(L.region + 2 * kRankDirect);
  uint32_t* lst = L.region + 4 * kRankDirect;                           // [kSlotRegs * kManageThreads] slot states
  uint32_t* lkv = lst + kSlotRegs * kManageThreads;                      // and keys
  int* smiss = reinterpret_cast<int*>(lkv + kSlotRegs * kManageThreads);  // [kSpecChunks][kSpecEntries]
  uint32_t* sgat = reinterpret_cast<uint32_t*>(smiss + kSpecChunks * kSpecEntries);  // [kSpecChunks][kSpecGather][3]
  static_assert(4 * kRankDirect + 2 * kSlotRegs * kManageThreads + kSpecChunks * (kSpecEntries + 3 * kSpecGather) <=
                    kBins, "resolve LDS region");
  {
    int dm = 0, ni = 0;
    if (tid < active) {
      dm = counts[tid * 8];
      ni = counts[tid * 8 + 1];
    }
    int32_t sm[2] = {-1, -1};
    uint4 sg = make_uint4(0, 0, 0, 0);
    if (spec && sp < active) {
      const int32_t* ml = w.missl + (static_cast<int64_t>(b) * parts + sp) * kMissPart;
      sm[0] = ml[si];
      sm[1] = ml[si + 32];
      if (si < kSpecGather) sg = w.gather[(static_cast<int64_t>(b) * parts + sp) * kGatherPart + si];
    }
    uint32_t st[kSlotRegs], kv[kSlotRegs];
    if (slots_in_regs) {
      if (keyed)
        load_slot_regs<kSlotRegs>(stab, skey, st, kv);
      else
        load_slot_states<kSlotRegs>(stab, st);
    }
    if (tid < active) {
      L.cdm[tid] = dm;
      L.cim[tid] = ni;  // in-bin count for now; the in-bin miss count below
    }
    if (spec && sp < active) {
      smiss[sp * kSpecEntries + si] = sm[0];
      smiss[sp * kSpecEntries + si + 32] = sm[1];
      if (si < kSpecGather) {
        uint32_t* d = sgat + (sp * kSpecGather + si) * 3;
        d[0] = sg.x;
        d[1] = sg.y;
        d[2] = sg.z;
      }
    }
    if (slots_in_regs) {
#pragma unroll
      for (int e = 0; e < kSlotRegs; ++e) {
        lst[tid * kSlotRegs + e] = st[e];
        if (keyed) lkv[tid * kSlotRegs + e] = kv[e];
      }
    }
  }
  if (tid == 0) *L.nibm = 0;
  const int dm = tid < active ? L.cdm[tid] : 0;  // (the thread's own store)
  const int ni = tid < active ? L.cim[tid] : 0;
  uint64_t tot2;
  const uint64_t ex = block_exclusive_scan4<true>(static_cast<uint64_t>(min(dm, kMissPart)) << 32 |
                                                      static_cast<uint64_t>(min(ni, kGatherPart)),
                                                  L.scratch64, &tot2);
  const int nd = static_cast<int>(tot2 >> 32);          // definite misses handed over
  const int g = static_cast<int>(tot2 & 0xffffffffu);   // in-bin tokens handed over
  if (tid < active) {
    L.doff[tid] = static_cast<int>(ex >> 32);
    L.goff[tid] = static_cast<int>(ex & 0xffffffffu);
  }
  // (The reduction's barriers also publish doff / goff.)
  const unsigned over = block_or_lds((ni > kGatherPart ? 1u : 0u) | (dm > kMissPart ? 2u : 0u) |
                                         (dm > kSpecEntries ? 4u : 0u) | (ni > kSpecGather ? 8u : 0u),
                                     L.scratch);
  const bool gather_over = (over & 1u) != 0;
  const bool miss_over = (over & 2u) != 0;
  const bool direct = !gather_over && g <= kRankDirect;
  // Entries past the ones read up front (all of them when active > kSpecChunks).
  const bool rest = !spec || (over & 4u) != 0 || (direct && (over & 8u) != 0);
  if (tid < active) L.cim[tid] = 0;  // (read above by this thread only)

  // 2. The handed-over definite misses, and the in-bin tokens for the ranking.
  if (spec && sp < active) {
    // Entries of chunk sp handed over: the offsets' differences.
    const int dn = (sp + 1 < active ? L.doff[sp + 1] : nd) - L.doff[sp];
    const int gn = (sp + 1 < active ? L.goff[sp + 1] : g) - L.goff[sp];
    if (si < dn) L.dmiss[L.doff[sp] + si] = smiss[sp * kSpecEntries + si];
    if (si + 32 < dn) L.dmiss[L.doff[sp] + si + 32] = smiss[sp * kSpecEntries + si + 32];
    if (direct && si < gn && si < kSpecGather) {
      const int f = L.goff[sp] + si;
      const uint32_t* d = sgat + (sp * kSpecGather + si) * 3;
      ltok[f] = static_cast<int>(d[0]);
      lkey[f] = d[1];
      lslot[f] = static_cast<int>(d[2]);
    }
  }
  if (rest) {
    for (int f = tid; f < nd; f += kManageThreads) {
      const int p = chunk_of(L.doff, active, f);
      if (spec && f - L.doff[p] < kSpecEntries) continue;
      L.dmiss[f] = w.missl[(static_cast<int64_t>(b) * parts + p) * kMissPart + (f - L.doff[p])];
    }
    if (direct) {
      for (int f = tid; f < g; f += kManageThreads) {
        const int p = chunk_of(L.goff, active, f);
        if (spec && f - L.goff[p] < kSpecGather) continue;
        const uint4 e = w.gather[(static_cast<int64_t>(b) * parts + p) * kGatherPart + (f - L.goff[p])];
        ltok[f] = static_cast<int>(e.x);
        lkey[f] = e.y;
        lslot[f] = static_cast<int>(e.z);
      }
    }
  }
  lds_barrier();

  // 3. The threshold among the in-bin tokens (ties go to the lower token) and
  //    their classification: cached ones into the slot table, misses listed.
  uint32_t thr = 0u;
  int cutoff = INT_MAX;
  auto classify = [&](int t, int32_t slot, bool selected, uint32_t key, bool patch) {
    if (slot >= 0 && slot < c) {
      const uint32_t ent = static_cast<uint32_t>(t) | ((selected ? kStateHit : kStateCand) << kStateShift);
      stab[slot] = ent;
      if (!selected && keyed) skey[slot] = key;
      if (patch) {  // the victims' copy of the slot table
        lst[slot] = ent;
        if (keyed) lkv[slot] = key;
      }
    } else if (selected) {
      atomicAdd(&L.cim[t / kChunk], 1);
      L.ibm[atomicAdd(L.nibm, 1)] = t;  // at most k <= kTopK in-bin tokens are selected
    }
  };
  if (direct) {
    // Rank pairwise: key descending, then token ascending.
    if (tid < g) {
      const int my_t = ltok[tid];
      const uint32_t my_k = lkey[tid];
      const int32_t my_slot = lslot[tid];
      int rank = 0;
      // Four entries per LDS read (the lists hold kRankDirect entries; those
      // past g are skipped).
#pragma unroll 2
      for (int j = 0; j < g; j += 4) {
        const uint4 k4 = *reinterpret_cast<const uint4*>(lkey + j);
        const int4 t4 = *reinterpret_cast<const int4*>(ltok + j);
        const uint32_t kk[4] = {k4.x, k4.y, k4.z, k4.w};
        const int tt4[4] = {t4.x, t4.y, t4.z, t4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          rank += (j + e < g && (kk[e] > my_k || (kk[e] == my_k && tt4[e] < my_t))) ? 1 : 0;
      }
      if (rank == k - 1) {  // the last selected token: the threshold and the tie cutoff
        L.bcast[0] = static_cast<int>(my_k);
        L.bcast[1] = my_t;
      }
      classify(my_t, my_slot, rank < k, my_k, slots_in_regs);
    }
    lds_barrier();  // the slot-table stores stay in flight
    thr = static_cast<uint32_t>(L.bcast[0]);
    cutoff = L.bcast[1];
  } else {
    // More in-bin tokens than the lists hold (heavy ties, or a key range
    // stretched by unmapped index blocks): stream the request's scores.
    uint32_t* hist = L.region;
    for (int i = tid; i < kBins; i += kManageThreads) hist[i] = 0u;
    __syncthreads();
    const uint32_t klo = lo + (bin << shift);  // keys in the bin lie in [klo, khi]
    const uint64_t top = static_cast<uint64_t>(klo) + ((uint64_t{1} << shift) - 1u);
    const uint32_t khi = top > 0xffffffffull ? 0xffffffffu : static_cast<uint32_t>(top);
    const int ngroups = static_cast<int>(ceil_div(n, 4));
    auto load_bin = [&](int gi, uint32_t* key, bool* inc) {
      load_score_keys(s, n, 4 * gi, key, inc);
#pragma unroll
      for (int e = 0; e < 4; ++e) inc[e] = inc[e] && ((key[e] - lo) >> shift) == bin;
    };
    const SelectOut sel = radix_select(ngroups, k, klo, khi, load_bin, hist, L.scratch, L.bcast);
    thr = sel.thresh;
    if (sel.need_eq != sel.cnt_eq) {  // ties at the threshold: one ordered pass finds the last selected
      int before = 0;
      for (int g0 = 0; g0 < ngroups; g0 += kManageThreads) {
        const int gi = g0 + tid;
        unsigned eqm = 0u;
        if (gi < ngroups) {
          uint32_t key[4];
          bool inc[4];
          load_bin(gi, key, inc);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (inc[e] && key[e] == thr) eqm |= 1u << e;
        }
        before = tie_cutoff_step(eqm, 4 * gi, sel.need_eq - 1, before, L.scratch, L.bcast);
      }
      __syncthreads();
      cutoff = L.bcast[3];
    }
    for (int gi = tid; gi < ngroups; gi += kManageThreads) {
      uint32_t key[4];
      bool inc[4];
      load_bin(gi, key, inc);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (inc[e]) classify(4 * gi + e, pool[4 * gi + e], mtp0_selected(key[e], 4 * gi + e, thr, cutoff), key[e], false);
    }
  }
  // The slot table, cim and the in-bin miss list are complete.  Only the
  // global slot table's readers (the streamed paths) need the full barrier.
  if (direct && slots_in_regs)
    lds_barrier();
  else
    __syncthreads();
  // The slot states in registers (their keys only where victims are
  // selected, below).
  uint32_t st[kSlotRegs];
  if (slots_in_regs) {
    const uint32_t* src = direct ? lst : stab;  // (the global table after the streamed classification)
#pragma unroll
    for (int j = 0; j < kSlotRegs; j += 4) {
      const uint4 v = *reinterpret_cast<const uint4*>(src + tid * kSlotRegs + j);
      st[j] = v.x;
      st[j + 1] = v.y;
      st[j + 2] = v.z;
      st[j + 3] = v.w;
    }
  }

  // 4. Misses per chunk, their bases, and the victims.  With the slots in
  //    registers one scan counts the misses before each chunk, the non-hit
  //    slots (victim candidates) and the hit slots before each thread's; when
  //    every non-hit slot is a victim (C = 2048 with a full pool) the victims
  //    come straight from it, in ascending slot order.
  const int mine = tid < active ? L.cdm[tid] + L.cim[tid] : 0;
  const int i0 = tid * kSlotRegs;
  unsigned nh = 0u, hm = 0u;  // this thread's non-hit and hit slots below c
  if (slots_in_regs) {
#pragma unroll
    for (int e = 0; e < kSlotRegs; ++e)
      if (i0 + e < c) {
        if ((st[e] >> kStateShift) == kStateHit)
          hm |= 1u << e;
        else
          nh |= 1u << e;
      }
  }
  // Fields: misses [42, 64), non-hit slots [21, 42), hits [0, 21) (block
  // totals stay below 2^21: at most 512 chunks of 4096 tokens, c < 2^14).
  uint64_t tot4;
  const uint64_t ex4 = block_exclusive_scan4<true>(static_cast<uint64_t>(mine) << 42 |
                                                       static_cast<uint64_t>(__popc(nh)) << 21 | __popc(hm),
                                                   L.scratch64, &tot4);
  constexpr uint64_t kField = (uint64_t{1} << 21) - 1;
  const int base = static_cast<int>(ex4 >> 42);
  const int m_all = static_cast<int>(tot4 >> 42);
  const int nonhit = static_cast<int>((tot4 >> 21) & kField);
  const int nhits = static_cast<int>(tot4 & kField);
  if (tid < active) L.goff[tid] = base;  // goff now holds the misses before each chunk
  L.cim[tid] = static_cast<int>(ex4 & kField);  // hits in lower slots, for step 7 (cim is free now)
  const int m = min(m_all, kTopK);       // misses are selected tokens
  const int nib = *L.nibm;
  int nv;
  if (slots_in_regs && m >= nonhit) {
    int pos = static_cast<int>((ex4 >> 21) & kField);
#pragma unroll
    for (int e = 0; e < kSlotRegs; ++e)
      if ((nh >> e) & 1u) {
        L.vsl[pos] = i0 + e;
        L.vev[pos] = (st[e] >> kStateShift) == kStateCand ? static_cast<int>(st[e] & kTokenMask) : -1;
        ++pos;
      }
    nv = nonhit;
  } else {
    uint32_t kv[kSlotRegs];
    if (slots_in_regs) {
      if (keyed) {
        const uint32_t* src = direct ? lkv : skey;
#pragma unroll
        for (int e = 0; e < kSlotRegs; ++e) kv[e] = src[tid * kSlotRegs + e];
      } else {
        // c = kTopK with more non-hit slots than misses (a pool naming one
        // slot twice): no key table was kept, a candidate slot's key is its
        // token's score.
#pragma unroll
        for (int e = 0; e < kSlotRegs; ++e)
          kv[e] = (st[e] >> kStateShift) == kStateCand ? score_key(s[st[e] & kTokenMask]) : 0u;
      }
    }
    lds_barrier();  // lkv is read before the histogram overwrites it
    uint32_t* hist = L.region;
    for (int i = tid; i < kBins; i += kManageThreads) hist[i] = 0u;
    lds_barrier();
    if (slots_in_regs) {
      nv = select_victims_in_regs<kSlotRegs, true>(c, m, st, kv, L.vsl, hist, L.scratch, L.bcast, L.red, L.vev);
    } else {
      nv = select_victims(c, m, stab, skey, L.vsl, hist, L.scratch, L.bcast, L.red, L.vev);
    }
  }
  lds_barrier();  // the victims and goff are published; the histogram is free again

  // 5. The misses in ascending token order -- a chunk's definite misses and
  //    in-bin misses interleave by token, chunks follow one another -- each
  //    written where its position lands, paired with the ascending victim
  //    slots, with the pool update.  (Pool writes here touch only misses'
  //    entries and evicted tokens', which are unselected, so the ordered pass
  //    below still classifies its chunk's tokens correctly.)
  auto emit = [&](int pos, int t) {
    if (pos >= m) return;
    const int d = pos < nv ? L.vsl[pos] : -1;
    const int evicted = pos < nv ? L.vev[pos] : -1;  // an unselected token, or -1 for a free slot
    out_src[pos] = t;
    out_dst[pos] = d;
    if (d >= 0) {
      if (evicted >= 0) pool[evicted] = -1;
      pool[t] = d;
    }
  };
  // In-bin misses of chunk p below token t.  A short list is scanned; a long
  // one (a cold pool row with many ties at the threshold: up to 2048 entries,
  // every miss scanning them would serialise on this workgroup) is sorted once
  // and searched.
  const bool ib_sorted = nib > kInBinScan;
  if (ib_sorted) {
    int np2 = kInBinScan;
    while (np2 < nib) np2 <<= 1;  // <= kTopK: at most k in-bin tokens are selected
    for (int i = nib + tid; i < np2; i += kManageThreads) L.ibm[i] = INT_MAX;
    lds_barrier();
    for (int size = 2; size <= np2; size <<= 1)  // bitonic sort, ascending
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = tid; i < np2 / 2; i += kManageThreads) {
          const int pos = 2 * i - (i & (stride - 1));
          const int x = L.ibm[pos], y = L.ibm[pos + stride];
          if ((x > y) == ((pos & size) == 0)) {
            L.ibm[pos] = y;
            L.ibm[pos + stride] = x;
          }
        }
        lds_barrier();
      }
  }
  auto lower = [&](int t) {  // sorted in-bin misses below t
    int lo_i = 0, hi_i = nib;
    while (lo_i < hi_i) {
      const int mid = (lo_i + hi_i) >> 1;
      if (L.ibm[mid] < t) lo_i = mid + 1;
      else hi_i = mid;
    }
    return lo_i;
  };
  auto ib_before = [&](int t, int p) {
    if (ib_sorted) return lower(t) - lower(p * kChunk);
    int before_ib = 0;
    for (int j = 0; j < nib; ++j) {
      const int x = L.ibm[j];
      before_ib += (x < t && x >= p * kChunk) ? 1 : 0;
    }
    return before_ib;
  };
  for (int f = tid; f < nd; f += kManageThreads) {
    const int p = chunk_of(L.doff, active, f);
    if (L.cdm[p] > kMissPart) continue;  // placed by the ordered pass below
    const int t = L.dmiss[f];
    emit(L.goff[p] + (f - L.doff[p]) + ib_before(t, p), t);
  }
  for (int j = tid; j < nib; j += kManageThreads) {
    const int t = L.ibm[j];
    const int p = t / kChunk;
    if (L.cdm[p] > kMissPart) continue;
    // Definite misses of chunk p below t: binary search of its sorted slice.
    int lo_i = L.doff[p], hi_i = L.doff[p] + L.cdm[p];
    while (lo_i < hi_i) {
      const int mid = (lo_i + hi_i) >> 1;
      if (L.dmiss[mid] < t) lo_i = mid + 1;
      else hi_i = mid;
    }
    emit(L.goff[p] + (lo_i - L.doff[p]) + ib_before(t, p), t);
  }
  if (miss_over) {
    // Chunks with more definite misses than their slice: one ordered pass
    // over the chunk's tokens (every thread reads its tokens' pool entries
    // before the scan's barriers, ahead of any write of this pass).
    for (int p = 0; p < active; ++p) {
      if (L.cdm[p] <= kMissPart) continue;  // uniform
      const int t0 = p * kChunk + tid * kItems;
      uint32_t u[kItems];
      int32_t slot[kItems];
      bool in[kItems];
      load_tokens8(s, pool, n, t0, u, slot, in);
      unsigned missm = 0u;
#pragma unroll
      for (int e = 0; e < kItems; ++e)
        if (in[e] && mtp0_selected(u[e], t0 + e, thr, cutoff) && !(slot[e] >= 0 && slot[e] < c)) missm |= 1u << e;
      int tot;
      int pos = L.goff[p] + block_exclusive_scan<true>(__popc(missm), L.scratch, &tot);
#pragma unroll
      for (int e = 0; e < kItems; ++e)
        if ((missm >> e) & 1u) {
          emit(pos, t0 + e);
          ++pos;
        }
    }
  }

  // 7. Then the hits by descending old slot (reference BuildHitMissKey order).
  if (!slots_in_regs) {
    write_hit_rows(a, b, c, m, stab, L.scratch);
    return;
  }
  unsigned hm7 = 0u;
#pragma unroll
  for (int e = 0; e < kSlotRegs; ++e)
    if (i0 + e < c && (st[e] >> kStateShift) == kStateHit) hm7 |= 1u << e;
  const int below = L.cim[tid];                 // hits in lower slots (this thread's own word)
  int above = nhits - below - __popc(hm7);      // hits in higher slots
#pragma unroll
  for (int e = kSlotRegs - 1; e >= 0; --e)
    if ((hm7 >> e) & 1u) {
      const int pos = m + above;
      if (pos < kTopK) {
        out_src[pos] = static_cast<int32_t>(st[e] & kTokenMask);
        out_dst[pos] = i0 + e;
      }
      ++above;
    }
  // Positions a corrupt pool (duplicate slots) left unfilled.
  for (int pos = m + nhits + tid; pos < kTopK; pos += kManageThreads) {
    out_src[pos] = -1;
    out_dst[pos] = -1;
  }
  if (tid == 0) a.miss_counts[b] = m;
}

// One 4096-token chunk of an MTP0 request (every launch shape): the row's
// first-digit bin holding the 2048th largest key (from the request's
// histogram) and the count above it; the chunk's cached tokens go to the slot
// table, its definite misses and in-bin tokens to its hand-over slices, its
// counts to part_counts.  The stores stay in flight (LDS-only barriers).
struct ChunkSel {
  uint32_t bin;
  int above;
};

__device__ __forceinline__ ChunkSel classify_chunk(const LimArgs& a, const LimWs& w, int parts, int b, int part, int n,
                                                   int c, int r, uint32_t lo, int shift, int* scratch,
                                                   uint64_t* scratch64, int* bcast) {
  const int tid = threadIdx.x;
  const int64_t cap = a.source_capacity;
  // This chunk's tokens: the loads are in flight during the bin search.
  const int t0 = part * kChunk + tid * kItems;
  uint32_t u[kItems];
  int32_t slot[kItems];
  bool in[kItems];
  load_tokens8(w.scores + static_cast<int64_t>(b) * cap, a.pool + static_cast<int64_t>(r) * cap, n, t0, u, slot, in);
  // The first-digit bin holding the 2048th largest key: thread tid owns bins
  // [P tb, P tb + P), P = kHistPerThread, tb = 511 - tid, so ascending threads
  // scan descending bins.
  int bin = 0, above = 0;
  {
    constexpr int P = kHistPerThread;
    const int tb = kManageThreads - 1 - tid;
    const uint32_t* gh = w.hist + static_cast<int64_t>(b) * kHistBins + P * tb;
    int cnt[P];
    if constexpr (P == 2) {
      const uint2 h = *reinterpret_cast<const uint2*>(gh);
      cnt[0] = static_cast<int>(h.x);
      cnt[1] = static_cast<int>(h.y);
    } else {
#pragma unroll
      for (int j = 0; j < P; j += 4) {
        const uint4 h = *reinterpret_cast<const uint4*>(gh + j);
        cnt[j] = static_cast<int>(h.x);
        cnt[j + 1] = static_cast<int>(h.y);
        cnt[j + 2] = static_cast<int>(h.z);
        cnt[j + 3] = static_cast<int>(h.w);
      }
    }
    int sum = 0;
#pragma unroll
    for (int j = 0; j < P; ++j) sum += cnt[j];
    if (tid == 0) bcast[0] = bcast[1] = 0;  // ordered before the writes below by the scan's barriers
    int total;
    int acc = block_exclusive_scan<true>(sum, scratch, &total);  // the token loads stay in flight
    if (acc < kTopK && kTopK <= acc + sum) {
#pragma unroll
      for (int j = P - 1; j >= 0; --j) {
        if (acc < kTopK && kTopK <= acc + cnt[j]) {
          bcast[0] = P * tb + j;
          bcast[1] = acc;
        }
        acc += cnt[j];
      }
    }
    lds_barrier();
    bin = __builtin_amdgcn_readfirstlane(bcast[0]);
    above = __builtin_amdgcn_readfirstlane(bcast[1]);
  }
  uint32_t* stab = w.slot_table + static_cast<int64_t>(b) * kTableStride;
  uint32_t* skey = w.slot_key + static_cast<int64_t>(b) * kTableStride;
  unsigned missm = 0u, inbin = 0u;
#pragma unroll
  for (int e = 0; e < kItems; ++e) {
    if (!in[e]) continue;
    const uint32_t d = (u[e] - lo) >> shift;
    if (d == static_cast<uint32_t>(bin)) {
      inbin |= 1u << e;
      continue;
    }
    const bool selected = d > static_cast<uint32_t>(bin);
    const int t = t0 + e;
    if (slot[e] >= 0 && slot[e] < c) {
      if (selected) {
        stab[slot[e]] = static_cast<uint32_t>(t) | (kStateHit << kStateShift);
      } else {
        stab[slot[e]] = static_cast<uint32_t>(t) | (kStateCand << kStateShift);
        if (c > kTopK) skey[slot[e]] = u[e];  // (at c = kTopK every non-hit slot is a victim)
      }
    } else if (selected) {
      missm |= 1u << e;
    }
  }
  // One scan for both counts (each below 2^16): definite misses high, in-bin
  // tokens low; both hand-over slices keep token order.
  uint64_t tot;
  // (LDS-only barriers: the slot-table stores stay in flight until the arrival fence.)
  const uint64_t pos =
      block_exclusive_scan4<true>(static_cast<uint64_t>(__popc(missm)) << 16 | __popc(inbin), scratch64, &tot);
  int midx = static_cast<int>((pos >> 16) & 0xffffu);
  int iidx = static_cast<int>(pos & 0xffffu);
  int32_t* ml = w.missl + (static_cast<int64_t>(b) * parts + part) * kMissPart;
  uint4* gl = w.gather + (static_cast<int64_t>(b) * parts + part) * kGatherPart;
#pragma unroll
  for (int e = 0; e < kItems; ++e) {
    if ((missm >> e) & 1u) {
      if (midx < kMissPart) ml[midx] = t0 + e;
      ++midx;
    }
    if ((inbin >> e) & 1u) {
      if (iidx < kGatherPart) gl[iidx] = make_uint4(static_cast<uint32_t>(t0 + e), u[e], static_cast<uint32_t>(slot[e]), 0u);
      ++iidx;
    }
  }
  int32_t* counts = w.part_counts + (static_cast<int64_t>(b) * parts + part) * 8;
  if (tid == 0) {
    counts[0] = static_cast<int>((tot >> 16) & 0xffffu);
    counts[1] = static_cast<int>(tot & 0xffffu);
  }
  return ChunkSel{static_cast<uint32_t>(bin), above};
}

// At most 128 VGPRs (four waves per SIMD): two workgroups per CU, as the ~74 KB of
// LDS allows.  Used while every chunk of the launch is resident at once
// (kResidentChunks); larger launches take lim_chunks_kernel + lim_resolve_kernel.
__global__ __launch_bounds__(kManageThreads, 4) void lim_classify_kernel(LimArgs a, LimWs w, int parts) {
  __shared__ uint32_t region[kBins];
  __shared__ int scratch[kManageThreads / 64 + 1];
  __shared__ uint64_t scratch64[kManageThreads / 64 + 1];
  __shared__ uint32_t red[2 * (kManageThreads / 64) + 2];
  __shared__ int bcast[4];
  __shared__ int cdm[kManageThreads], cim[kManageThreads], doff[kManageThreads], goff[kManageThreads];
  __shared__ int dmiss[kTopK], ibm[kTopK], vsl[kTopK], vev[kTopK];
  __shared__ int nibm;
  __shared__ int last;
  const int b = blockIdx.x / parts;
  const int part = blockIdx.x - b * parts;
  const int tid = threadIdx.x;
  const int n = a.num_candidates[b];
  const int c = a.num_cache[b];
  const int r = a.pool_entries[b];
  if (!lim_row_valid(n, c, r, a.source_capacity, a.pool_rows) || part * kChunk >= n) return;
  const int active = static_cast<int>(ceil_div(n, kChunk));  // chunks that arrive below
  const uint32_t lo = w.rowsel[4 * b];
  const int shift = static_cast<int>(w.rowsel[4 * b + 1]);
  const ChunkSel sel = classify_chunk(a, w, parts, b, part, n, c, r, lo, shift, scratch, scratch64, bcast);
  // The barrier waits for every wave's stores; one release fence then makes
  // them visible device-wide before the arrival count, and the last chunk of
  // the request to arrive acquires the others' (one agent-scope fence each
  // way: a full fence per wave writes back and invalidates the XCD's L2
  // under the other chunks' feet).
  __syncthreads();
  if (tid == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    last = atomicAdd(&w.done[b], 1) == active - 1 ? 1 : 0;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
  if (!last) return;
  const ResolveLds L{region, scratch, scratch64, red, bcast, cdm, cim, doff, goff, dmiss, ibm, &nibm, vsl, vev};
  mtp0_resolve(a, w, b, n, c, r, parts, active, sel.bin, kTopK - sel.above, lo, shift, L);
}

// Launches of more chunks than stay resident next to the last chunk's LDS:
// the chunks alone (a small footprint, so all of them are resident), then
// lim_resolve_kernel, one workgroup per request.  Chunk 0 of a request leaves
// the bin and the count above it in rowsel (every chunk finds the same).
__global__ __launch_bounds__(kManageThreads) void lim_chunks_kernel(LimArgs a, LimWs w, int parts) {
  __shared__ int scratch[kManageThreads / 64 + 1];
  __shared__ uint64_t scratch64[kManageThreads / 64 + 1];
  __shared__ int bcast[4];
  const int b = blockIdx.x / parts;
  const int part = blockIdx.x - b * parts;
  const int n = a.num_candidates[b];
  const int c = a.num_cache[b];
  const int r = a.pool_entries[b];
  if (!lim_row_valid(n, c, r, a.source_capacity, a.pool_rows) || part * kChunk >= n) return;
  const ChunkSel sel = classify_chunk(a, w, parts, b, part, n, c, r, w.rowsel[4 * b],
                                      static_cast<int>(w.rowsel[4 * b + 1]), scratch, scratch64, bcast);
  if (part == 0 && threadIdx.x == 0) {
    w.rowsel[4 * b + 2] = sel.bin;
    w.rowsel[4 * b + 3] = static_cast<uint32_t>(sel.above);
  }
}

__global__ __launch_bounds__(kManageThreads, 4) void lim_resolve_kernel(LimArgs a, LimWs w, int parts) {
  __shared__ uint32_t region[kBins];
  __shared__ int scratch[kManageThreads / 64 + 1];
  __shared__ uint64_t scratch64[kManageThreads / 64 + 1];
  __shared__ uint32_t red[2 * (kManageThreads / 64) + 2];
  __shared__ int bcast[4];
  __shared__ int cdm[kManageThreads], cim[kManageThreads], doff[kManageThreads], goff[kManageThreads];
  __shared__ int dmiss[kTopK], ibm[kTopK], vsl[kTopK], vev[kTopK];
  __shared__ int nibm;
  const int b = blockIdx.x;
  const int n = a.num_candidates[b];
  const int c = a.num_cache[b];
  const int r = a.pool_entries[b];
  if (!lim_row_valid(n, c, r, a.source_capacity, a.pool_rows)) return;
  const uint32_t* sel = w.rowsel + 4 * b;
  const ResolveLds L{region, scratch, scratch64, red, bcast, cdm, cim, doff, goff, dmiss, ibm, &nibm, vsl, vev};
  mtp0_resolve(a, w, b, n, c, r, parts, static_cast<int>(ceil_div(n, kChunk)), sel[2], kTopK - static_cast<int>(sel[3]),
               sel[0], static_cast<int>(sel[1]), L);
}

// ---------------------------------------------------------------------------
// 2b. MTP3 management: union of the four top-2048 sets, in three chunked
// kernels (one workgroup per 4096-token chunk of a request for the passes):
//   pass A   query masks, slot states, per-chunk counts;
//   victims  one workgroup per request: victim radix select over the slots;
//   pass B   union-ordered misses, per-query rows, pool update, each chunk
//            placing its entries after the counts of the chunks before it.
// The threshold kernel has run first: per-query threshold keys with tie
// cutoffs (so a token's selection needs no ordered tie count) and the
// request's slot table reset to free.

struct MtpSelect {
  uint32_t thr[kMtpQueries];
  int cutoff[kMtpQueries];
};

__device__ inline MtpSelect read_mtp_select(const LimWs& w, int b) {
  MtpSelect m;
#pragma unroll
  for (int q = 0; q < kMtpQueries; ++q) {
    const uint32_t* sp = w.select + (static_cast<int64_t>(b) * kMtpQueries + q) * 4;
    m.thr[q] = sp[0];
    m.cutoff[q] = static_cast<int>(sp[3]);
  }
  return m;
}

__global__ __launch_bounds__(kManageThreads) void lim_mtp_pass_a_kernel(LimArgs a, LimWs w, int parts) {
  __shared__ uint64_t scratch64[kManageThreads / 64 + 1];
  const int b = blockIdx.x / parts;
  const int part = blockIdx.x - b * parts;
  const int tid = threadIdx.x;
  const int n = a.num_candidates[b];
  const int c = a.num_cache[b];
  const int r = a.pool_entries[b];
  if (!lim_mtp_row_valid(n, c, r, a.source_capacity, a.pool_rows)) return;
  const int64_t cap = a.source_capacity;
  int32_t* counts = w.part_counts + (static_cast<int64_t>(b) * parts + part) * 8;
  const int t0 = part * kChunk + tid * kItems;
  if (part * kChunk >= n) {  // a chunk past the candidates adds nothing
    if (tid < 8) counts[tid] = 0;
    return;
  }
  const MtpSelect ms = read_mtp_select(w, b);
  const float* s = w.scores + static_cast<int64_t>(b) * kMtpQueries * cap;
  const int32_t* pool = a.pool + static_cast<int64_t>(r) * cap;
  uint32_t* stab = w.slot_table + static_cast<int64_t>(b) * kTableStride;
  uint32_t* skey = w.slot_key + static_cast<int64_t>(b) * kTableStride;
  uint8_t* masks = w.masks + static_cast<int64_t>(b) * cap;

  uint32_t u[kMtpQueries][kItems];
  int32_t slot[kItems];
  bool in[kItems];
  load_tokens8(s, pool, n, t0, u[0], slot, in);
#pragma unroll
  for (int q = 1; q < kMtpQueries; ++q) {
    const float* sq = s + q * cap;
    if (t0 + kItems <= n) {
      const float4 x = *reinterpret_cast<const float4*>(sq + t0);
      const float4 y = *reinterpret_cast<const float4*>(sq + t0 + 4);
      u[q][0] = score_key(x.x); u[q][1] = score_key(x.y); u[q][2] = score_key(x.z); u[q][3] = score_key(x.w);
      u[q][4] = score_key(y.x); u[q][5] = score_key(y.y); u[q][6] = score_key(y.z); u[q][7] = score_key(y.w);
    } else {
#pragma unroll
      for (int e = 0; e < kItems; ++e) u[q][e] = in[e] ? score_key(sq[t0 + e]) : 0u;
    }
  }
  unsigned qmask[kItems];
  uint64_t missp = 0, rowp = 0;
#pragma unroll
  for (int e = 0; e < kItems; ++e) {
    qmask[e] = 0;
    if (!in[e]) continue;
    const int t = t0 + e;
#pragma unroll
    for (int q = 0; q < kMtpQueries; ++q)
      if (u[q][e] > ms.thr[q] || (u[q][e] == ms.thr[q] && t <= ms.cutoff[q])) qmask[e] |= 1u << q;
    const bool cached = slot[e] >= 0 && slot[e] < c;
    if (cached) {
      if (qmask[e]) {
        stab[slot[e]] = static_cast<uint32_t>(t) | (kStateHit << kStateShift);
      } else {
        uint32_t umax = u[0][e];
#pragma unroll
        for (int q = 1; q < kMtpQueries; ++q) umax = u[q][e] > umax ? u[q][e] : umax;
        stab[slot[e]] = static_cast<uint32_t>(t) | (kStateCand << kStateShift);
        skey[slot[e]] = umax;
      }
    } else if (qmask[e]) {
      missp += uint64_t{1} << (16 * __builtin_ctz(qmask[e]));
    }
#pragma unroll
    for (int q = 0; q < kMtpQueries; ++q)
      if ((qmask[e] >> q) & 1u) rowp += uint64_t{1} << (16 * q);
  }
  if (t0 + kItems <= n) {
    const uint32_t m0 = qmask[0] | (qmask[1] << 8) | (qmask[2] << 16) | (qmask[3] << 24);
    const uint32_t m1 = qmask[4] | (qmask[5] << 8) | (qmask[6] << 16) | (qmask[7] << 24);
    *reinterpret_cast<uint2*>(masks + t0) = make_uint2(m0, m1);
  } else {
#pragma unroll
    for (int e = 0; e < kItems; ++e)
      if (in[e]) masks[t0 + e] = static_cast<uint8_t>(qmask[e]);
  }
  uint64_t mtot, rtot;
  (void)block_exclusive_scan4(missp, scratch64, &mtot);
  (void)block_exclusive_scan4(rowp, scratch64, &rtot);
  if (tid < 8) counts[tid] = tid < 4 ? lane16(mtot, tid) : lane16(rtot, tid - 4);
}

__global__ __launch_bounds__(kManageThreads) void lim_mtp_victims_kernel(LimArgs a, LimWs w, int parts) {
  __shared__ uint32_t hist[kBins];
  __shared__ int scratch[kManageThreads / 64 + 1];
  __shared__ uint32_t red[2 * (kManageThreads / 64) + 2];
  __shared__ int bcast[4];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int n = a.num_candidates[b];
  const int c = a.num_cache[b];
  const int r = a.pool_entries[b];
  if (!lim_mtp_row_valid(n, c, r, a.source_capacity, a.pool_rows)) {
    if (tid == 0) a.miss_counts[b] = 0;
    return;
  }
  for (int i = tid; i < kBins; i += kManageThreads) hist[i] = 0u;
  const int32_t* counts = w.part_counts + static_cast<int64_t>(b) * parts * 8;
  int local = 0;
  for (int p = tid; p < parts; p += kManageThreads)
    local += counts[p * 8 + 0] + counts[p * 8 + 1] + counts[p * 8 + 2] + counts[p * 8 + 3];
  const int m = block_sum(local, scratch);  // union misses
  const uint32_t* stab = w.slot_table + static_cast<int64_t>(b) * kTableStride;
  const uint32_t* skey = w.slot_key + static_cast<int64_t>(b) * kTableStride;
  int32_t* vslot = w.vslot + static_cast<int64_t>(b) * kUnionCap;
  const int nv = c <= 16 * kManageThreads ? select_victims_regs<16>(c, m, stab, skey, vslot, hist, scratch, bcast, red)
                                          : select_victims(c, m, stab, skey, vslot, hist, scratch, bcast, red);
  if (tid == 0) {
    w.nvict[b] = nv;
    a.miss_counts[b] = m;
  }
}

__global__ __launch_bounds__(kManageThreads) void lim_mtp_pass_b_kernel(LimArgs a, LimWs w, int parts) {
  __shared__ uint64_t scratch64[kManageThreads / 64 + 1];
  __shared__ uint64_t base[2];
  const int b = blockIdx.x / parts;
  const int part = blockIdx.x - b * parts;
  const int tid = threadIdx.x;
  const int n = a.num_candidates[b];
  const int c = a.num_cache[b];
  const int r = a.pool_entries[b];
  if (!lim_mtp_row_valid(n, c, r, a.source_capacity, a.pool_rows)) return;
  if (part * kChunk >= n) return;
  const int64_t cap = a.source_capacity;
  // Counts of the chunks before this one (exclusive scan over parts, parts <= 512).
  const int32_t* counts = w.part_counts + static_cast<int64_t>(b) * parts * 8;
  uint64_t pm = 0, pr = 0;
  if (tid < parts) {
#pragma unroll
    for (int q = 0; q < kMtpQueries; ++q) {
      pm |= static_cast<uint64_t>(counts[tid * 8 + q]) << (16 * q);
      pr |= static_cast<uint64_t>(counts[tid * 8 + 4 + q]) << (16 * q);
    }
  }
  uint64_t mall, rall;
  const uint64_t pm_before = block_exclusive_scan4(pm, scratch64, &mall);
  const uint64_t pr_before = block_exclusive_scan4(pr, scratch64, &rall);
  if (tid == part) {
    base[0] = pm_before;
    base[1] = pr_before;
  }
  __syncthreads();
  const uint64_t mb = base[0], rb = base[1];
  int gbase[kMtpQueries];  // union order: misses first-selected by q0, then q1, ...
  gbase[0] = 0;
#pragma unroll
  for (int q = 1; q < kMtpQueries; ++q) gbase[q] = gbase[q - 1] + lane16(mall, q - 1);
  const int nv = w.nvict[b];
  const int32_t* vslot = w.vslot + static_cast<int64_t>(b) * kUnionCap;
  const uint32_t* stab = w.slot_table + static_cast<int64_t>(b) * kTableStride;
  int32_t* pool = a.pool + static_cast<int64_t>(r) * cap;
  const uint8_t* masks = w.masks + static_cast<int64_t>(b) * cap;
  int32_t* miss_src = a.miss_src + static_cast<int64_t>(b) * kUnionCap;
  int32_t* miss_dst = a.miss_dst + static_cast<int64_t>(b) * kUnionCap;

  const int t0 = part * kChunk + tid * kItems;
  unsigned mbits[kItems];
  int32_t slot[kItems];
  if (t0 + kItems <= n) {
    const uint2 mm = *reinterpret_cast<const uint2*>(masks + t0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      mbits[e] = (mm.x >> (8 * e)) & 0xffu;
      mbits[e + 4] = (mm.y >> (8 * e)) & 0xffu;
    }
    const int4 pa = *reinterpret_cast<const int4*>(pool + t0);
    const int4 pb = *reinterpret_cast<const int4*>(pool + t0 + 4);
    slot[0] = pa.x; slot[1] = pa.y; slot[2] = pa.z; slot[3] = pa.w;
    slot[4] = pb.x; slot[5] = pb.y; slot[6] = pb.z; slot[7] = pb.w;
  } else {
#pragma unroll
    for (int e = 0; e < kItems; ++e) {
      const bool inb = t0 + e < n;
      mbits[e] = inb ? masks[t0 + e] : 0;
      slot[e] = inb ? pool[t0 + e] : -1;
    }
  }
  uint64_t missp = 0, rowp = 0;
#pragma unroll
  for (int e = 0; e < kItems; ++e) {
    const unsigned mk = mbits[e];
    if (!mk) continue;
    const bool cached = slot[e] >= 0 && slot[e] < c;
    if (!cached) missp += uint64_t{1} << (16 * __builtin_ctz(mk));
#pragma unroll
    for (int q = 0; q < kMtpQueries; ++q)
      if ((mk >> q) & 1u) rowp += uint64_t{1} << (16 * q);
  }
  uint64_t mtot, rtot;
  const uint64_t mrk = block_exclusive_scan4(missp, scratch64, &mtot);
  const uint64_t rrk = block_exclusive_scan4(rowp, scratch64, &rtot);
  int mpos[kMtpQueries], rpos[kMtpQueries];
#pragma unroll
  for (int q = 0; q < kMtpQueries; ++q) {
    mpos[q] = gbase[q] + lane16(mb, q) + lane16(mrk, q);
    rpos[q] = lane16(rb, q) + lane16(rrk, q);
  }
#pragma unroll
  for (int e = 0; e < kItems; ++e) {
    const unsigned mk = mbits[e];
    if (!mk) continue;
    const int t = t0 + e;
    const bool cached = slot[e] >= 0 && slot[e] < c;
    int new_slot = slot[e];
    if (!cached) {
      const int g = __builtin_ctz(mk);
      int pos = 0;
#pragma unroll
      for (int q = 0; q < kMtpQueries; ++q)
        if (q == g) pos = mpos[q]++;
      const int d = pos < nv ? vslot[pos] : -1;
      miss_src[pos] = t;
      miss_dst[pos] = d;
      new_slot = d;
      if (d >= 0) {
        const uint32_t ent = stab[d];
        if ((ent >> kStateShift) == kStateCand) pool[ent & kTokenMask] = -1;  // an unselected token: no chunk reads it
        pool[t] = d;
      }
    }
#pragma unroll
    for (int q = 0; q < kMtpQueries; ++q)
      if ((mk >> q) & 1u) {
        const int i = rpos[q]++;
        const int64_t row = static_cast<int64_t>(b) * kMtpQueries + q;
        if (i < kTopK) {
          a.topk_src[row * kTopK + i] = cached ? -1 : t;
          a.topk_dst[row * kTopK + i] = new_slot;
        }
      }
  }
}

// ---------------------------------------------------------------------------
// 3. First-decode LIDU initialisation (nanovllm/models/dsa_offload_ops.py:251-411).

struct InitWs {
  float* scores;  // [S_cap]
  int32_t* src;   // [16384] selected tokens, ascending
  int32_t* dst;   // [16384] their slots
  int32_t* count; // list length
};

InitWs carve_init(void* base, int64_t cap) {
  char* p = static_cast<char*>(base);
  InitWs w;
  w.scores = reinterpret_cast<float*>(p);
  p += align256(sizeof(float) * cap);
  w.src = reinterpret_cast<int32_t*>(p);
  p += align256(sizeof(int32_t) * kSlotStride);
  w.dst = reinterpret_cast<int32_t*>(p);
  p += align256(sizeof(int32_t) * kSlotStride);
  w.count = reinterpret_cast<int32_t*>(p);
  return w;
}

// Tokens per group of the first-decode selection: 8 chunks of kChunk, thread
// tid holding tokens gbase + k * kChunk + tid * kItems + e of group gbase.
constexpr int kInitGroup = 8;

// Byte range of the buffer resource over the score region: align256(4 row_len)
// (a multiple of the 16-byte loads), capped at 1 GiB so it fits the 32-bit
// field; every load offset stays below 4 (n + one group) < 9 MB (n < 2^21).
__device__ inline int init_score_range(int64_t row_len) {
  return static_cast<int>(min<size_t>(align256(sizeof(float) * row_len), size_t(1) << 30));
}

// One group's score keys: 16 loads per thread in flight together, through a
// buffer resource over the workspace's score region (align256(4 row_len)
// bytes, a multiple of the 16-byte loads, so loads past it return zeros
// without a branch; keys of tokens >= n are never used), turned into
// order-preserving keys in place.
__device__ __forceinline__ void load_init_group(__amdgpu_buffer_rsrc_t rsrc, int64_t gbase,
                                                u32x4_t (&key)[kInitGroup][2]) {
#pragma unroll
  for (int k = 0; k < kInitGroup; ++k)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      key[k][h] = __builtin_amdgcn_raw_buffer_load_b128(
          rsrc, static_cast<int>((gbase + k * kChunk + threadIdx.x * kItems + 4 * h) * 4), 0, 0);
#pragma unroll
  for (int k = 0; k < kInitGroup; ++k)
#pragma unroll
    for (int e = 0; e < kItems; ++e) key[k][e >> 2][e & 3] = score_key(__uint_as_float(key[k][e >> 2][e & 3]));
}

// f(key) for every key of tokens < n in a group: chunks below kfull are
// whole, chunk kfull is cut at n (element e exists iff e < lim), the ones
// above lie past n; kfull is uniform, so the element checks stay in the one
// cut chunk.
template <typename F>
__device__ __forceinline__ void visit_init_group(const u32x4_t (&key)[kInitGroup][2], int kfull, int lim, const F& f) {
#pragma unroll
  for (int k = 0; k < kInitGroup; ++k) {
    if (k < kfull) {
#pragma unroll
      for (int e = 0; e < kItems; ++e) f(key[k][e >> 2][e & 3]);
    } else if (k == kfull) {
#pragma unroll
      for (int e = 0; e < kItems; ++e)
        if (e < lim) f(key[k][e >> 2][e & 3]);
    }
  }
}

// Smallest and largest key of the group's tokens < n (kfull, lim as for
// visit_init_group), folded into lo and hi.
__device__ __forceinline__ void group_minmax(const u32x4_t (&key)[kInitGroup][2], int kfull, int lim, uint32_t& lo,
                                             uint32_t& hi) {
#pragma unroll
  for (int k = 0; k < kInitGroup; ++k) {
    if (k < kfull) {
#pragma unroll
      for (int e = 0; e < kItems; ++e) {
        lo = min(lo, key[k][e >> 2][e & 3]);
        hi = max(hi, key[k][e >> 2][e & 3]);
      }
    } else if (k == kfull) {
#pragma unroll
      for (int e = 0; e < kItems; ++e)
        if (e < lim) {
          lo = min(lo, key[k][e >> 2][e & 3]);
          hi = max(hi, key[k][e >> 2][e & 3]);
        }
    }
  }
}

// The ordered pass over one group: slot positions of its selected tokens
// from one 8-counter block scan (two when tied keys must be ranked: only the
// lowest need_eq tokens equal to the threshold are selected; `eq_run` counts
// the ties of earlier groups), the pool entries (-1 elsewhere; 16-byte stores
// when the row allows) and the copy list.  Token order is chunk-major, so the
// tokens before this thread's chunk-k ones are the earlier chunks' totals
// plus the chunk-k counts of the lower threads.  Returns the group's count.
__device__ __forceinline__ int init_group_order(const u32x4_t (&key)[kInitGroup][2], int kfull, int lim,
                                                const SelectOut& sel, int64_t gbase, int run, int& eq_run,
                                                int32_t* pool_row, int64_t row_len, bool vec_ok, const InitWs& w,
                                                uint64_t* scan64) {
  const int tid = threadIdx.x;
  unsigned selm[kInitGroup], eqm[kInitGroup];
#pragma unroll
  for (int k = 0; k < kInitGroup; ++k) {
    selm[k] = 0u;
    eqm[k] = 0u;
    if (k > kfull) continue;  // uniform
#pragma unroll
    for (int e = 0; e < kItems; ++e) {
      if (k == kfull && e >= lim) continue;
      if (key[k][e >> 2][e & 3] > sel.thresh) selm[k] |= 1u << e;
      if (key[k][e >> 2][e & 3] == sel.thresh) eqm[k] |= 1u << e;
    }
  }
  if (sel.cnt_eq != sel.need_eq) {
    uint64_t ec[2] = {0, 0}, etot[2];
#pragma unroll
    for (int k = 0; k < kInitGroup; ++k) ec[k >> 2] |= static_cast<uint64_t>(__popc(eqm[k])) << (16 * (k & 3));
    block_exclusive_scan8(ec, scan64, etot);
#pragma unroll
    for (int k = 0; k < kInitGroup; ++k) {
      int rk = eq_run + lane16x8(ec, k);
#pragma unroll
      for (int e = 0; e < kItems; ++e)
        if ((eqm[k] >> e) & 1u) {
          if (rk < sel.need_eq) selm[k] |= 1u << e;
          ++rk;
        }
      eq_run += lane16x8(etot, k);
    }
  } else {
#pragma unroll
    for (int k = 0; k < kInitGroup; ++k) selm[k] |= eqm[k];
  }
  uint64_t sc[2] = {0, 0}, stot[2];
#pragma unroll
  for (int k = 0; k < kInitGroup; ++k) sc[k >> 2] |= static_cast<uint64_t>(__popc(selm[k])) << (16 * (k & 3));
  block_exclusive_scan8(sc, scan64, stot);
  int count = 0;
#pragma unroll
  for (int k = 0; k < kInitGroup; ++k) {
    const int64_t t0 = gbase + static_cast<int64_t>(k) * kChunk + tid * kItems;
    int pos = run + count + lane16x8(sc, k);
    int pv[kItems];
#pragma unroll
    for (int e = 0; e < kItems; ++e) {
      pv[e] = -1;
      if ((selm[k] >> e) & 1u) {
        pv[e] = pos;
        if (pos < kSlotStride) {
          w.src[pos] = static_cast<int32_t>(t0 + e);
          w.dst[pos] = pos;
        }
        ++pos;
      }
    }
    if (vec_ok && t0 + kItems <= row_len) {
      *reinterpret_cast<int4*>(pool_row + t0) = make_int4(pv[0], pv[1], pv[2], pv[3]);
      *reinterpret_cast<int4*>(pool_row + t0 + 4) = make_int4(pv[4], pv[5], pv[6], pv[7]);
    } else {
#pragma unroll
      for (int e = 0; e < kItems; ++e)
        if (t0 + e < row_len) pool_row[t0 + e] = pv[e];
    }
    count += lane16x8(stot, k);
  }
  return count;
}

// One workgroup: the C largest linear scores of tokens [0, n) (ties at the
// threshold to the lower tokens), slot i to the i-th smallest selected token,
// the pool row rewritten over its whole length (-1 outside the selection),
// and the (token, slot) copy list.  Any n: every pass (range, radix digits,
// ordered pass) walks the scores group by group, one load round trip per
// group of 32768 tokens.
__global__ __launch_bounds__(kManageThreads) void lidu_init_kernel(const float* s, int n, int c, int32_t* pool_row,
                                                                   int64_t row_len, InitWs w) {
  __shared__ uint32_t hist[kBins];
  __shared__ int scratch[kManageThreads / 64 + 1];
  __shared__ uint32_t red[2 * (kManageThreads / 64) + 2];
  __shared__ int bcast[4];
  __shared__ uint64_t scan64[2 * (kManageThreads / 64)];
  const int tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t srsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(s), 0, init_score_range(row_len), kBufferFlags);
  for (int i = tid; i < kBins; i += kManageThreads) hist[i] = 0u;
  constexpr int kGroupTokens = kInitGroup * kChunk;
  auto each_key = [&](auto f) {
    for (int gbase = 0; gbase < n; gbase += kGroupTokens) {
      u32x4_t key[kInitGroup][2];
      load_init_group(srsrc, gbase, key);
      const int kfull = (n - gbase) / kChunk;
      visit_init_group(key, kfull, n - gbase - kfull * kChunk - tid * kItems, f);
    }
  };
  uint32_t lo = 0xffffffffu, hi = 0u;
  for (int gbase = 0; gbase < n; gbase += kGroupTokens) {
    u32x4_t key[kInitGroup][2];
    load_init_group(srsrc, gbase, key);
    const int kfull = (n - gbase) / kChunk;
    group_minmax(key, kfull, n - gbase - kfull * kChunk - tid * kItems, lo, hi);
  }
  block_minmax(lo, hi, red);
  const SelectOut sel = radix_select_visit(c, lo, hi, each_key, hist, scratch, bcast);
  const bool vec_ok = (reinterpret_cast<uintptr_t>(pool_row) & 15) == 0;  // uniform
  int run = 0, eq_run = 0;
  for (int64_t gbase = 0; gbase < row_len; gbase += kGroupTokens) {
    if (gbase >= n) {  // past the source: nothing selected
      for (int64_t t = gbase + tid; t < min<int64_t>(row_len, gbase + kGroupTokens); t += kManageThreads)
        pool_row[t] = -1;
      continue;
    }
    u32x4_t key[kInitGroup][2];
    load_init_group(srsrc, gbase, key);
    const int kfull = static_cast<int>((n - gbase) / kChunk);
    run += init_group_order(key, kfull, static_cast<int>(n - gbase - kfull * kChunk - tid * kItems), sel, gbase, run,
                            eq_run, pool_row, row_len, vec_ok, w, scan64);
  }
  if (tid == 0) *w.count = run;
}

// lidu_init_kernel for sources of at most one group (32768 tokens): the
// group's keys stay in registers across the range, the radix passes and the
// ordered pass instead of being re-read for each.
__global__ __launch_bounds__(kManageThreads) void lidu_init_reg_kernel(const float* s, int n, int c,
                                                                       int32_t* pool_row, int64_t row_len, InitWs w) {
  __shared__ uint32_t hist[kBins];
  __shared__ int scratch[kManageThreads / 64 + 1];
  __shared__ uint32_t red[2 * (kManageThreads / 64) + 2];
  __shared__ int bcast[4];
  __shared__ uint64_t scan64[2 * (kManageThreads / 64)];
  const int tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t srsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(s), 0, init_score_range(row_len), kBufferFlags);
  u32x4_t key[kInitGroup][2];
  load_init_group(srsrc, 0, key);
  for (int i = tid; i < kBins; i += kManageThreads) hist[i] = 0u;
  const int kfull = n / kChunk;
  const int lim = n - kfull * kChunk - tid * kItems;
  auto each_key = [&](auto f) { visit_init_group(key, kfull, lim, f); };
  uint32_t lo = 0xffffffffu, hi = 0u;
  group_minmax(key, kfull, lim, lo, hi);
  block_minmax(lo, hi, red);
  const SelectOut sel = radix_select_visit(c, lo, hi, each_key, hist, scratch, bcast);
  int eq_run = 0;
  const int run = init_group_order(key, kfull, lim, sel, 0, 0, eq_run, pool_row, row_len,
                                   (reinterpret_cast<uintptr_t>(pool_row) & 15) == 0, w, scan64);
  // The rest of the pool row lies past the source: nothing selected there.
  for (int64_t t = static_cast<int64_t>(kInitGroup) * kChunk + tid; t < row_len; t += kManageThreads)
    pool_row[t] = -1;
  if (tid == 0) *w.count = run;
}

// One workgroup: the (token, slot) list of every entry >= 0 of an owner's
// pool row, ascending token (dsa_offload_ops.py:385-388); the count may
// exceed the list capacity (the caller checks it).
__global__ __launch_bounds__(kManageThreads) void lidu_shared_kernel(const int32_t* pool_row, int64_t row_len,
                                                                     InitWs w) {
  // Groups of 8 chunks of 4096 entries: thread tid reads entries
  // k * kChunk + tid * kItems + e of each chunk k of the group (16-byte loads
  // when the row is 16-byte aligned), all in flight together, and one block
  // scan of eight 16-bit counters orders the group's cached tokens.
  __shared__ uint64_t scan64[2 * (kManageThreads / 64)];
  constexpr int kGroup = 8;
  const int tid = threadIdx.x;
  const bool vec_ok = (reinterpret_cast<uintptr_t>(pool_row) & 15) == 0;  // uniform
  int run = 0;
  for (int64_t gbase = 0; gbase < row_len; gbase += kGroup * kChunk) {
    int32_t v[kGroup][kItems];
#pragma unroll
    for (int k = 0; k < kGroup; ++k) {
      const int64_t t0 = gbase + static_cast<int64_t>(k) * kChunk + tid * kItems;
      if (vec_ok && t0 + kItems <= row_len) {
        const int4 x = *reinterpret_cast<const int4*>(pool_row + t0);
        const int4 y = *reinterpret_cast<const int4*>(pool_row + t0 + 4);
        v[k][0] = x.x; v[k][1] = x.y; v[k][2] = x.z; v[k][3] = x.w;
        v[k][4] = y.x; v[k][5] = y.y; v[k][6] = y.z; v[k][7] = y.w;
      } else {
#pragma unroll
        for (int e = 0; e < kItems; ++e) v[k][e] = t0 + e < row_len ? pool_row[t0 + e] : -1;
      }
    }
    uint64_t cnt[2] = {0, 0}, tot[2];
    unsigned mask[kGroup];
#pragma unroll
    for (int k = 0; k < kGroup; ++k) {
      mask[k] = 0u;
#pragma unroll
      for (int e = 0; e < kItems; ++e)
        if (v[k][e] >= 0) mask[k] |= 1u << e;
      cnt[k >> 2] |= static_cast<uint64_t>(__popc(mask[k])) << (16 * (k & 3));
    }
    block_exclusive_scan8(cnt, scan64, tot);
#pragma unroll
    for (int k = 0; k < kGroup; ++k) {
      const int64_t t0 = gbase + static_cast<int64_t>(k) * kChunk + tid * kItems;
      int pos = run + lane16x8(cnt, k);
#pragma unroll
      for (int e = 0; e < kItems; ++e)
        if ((mask[k] >> e) & 1u) {
          if (pos < kSlotStride) {
            w.src[pos] = static_cast<int32_t>(t0 + e);
            w.dst[pos] = v[k][e];
          }
          ++pos;
        }
      run += lane16x8(tot, k);
    }
  }
  if (tid == 0) *w.count = run;
}

template <typename T>
hipError_t launch_lidu_scores(const LiduInitArgs& a, const InitWs& w, hipStream_t stream) {
  LimArgs la{};
  la.query = a.query;
  la.weights = a.weights;
  la.key_cache = a.key_cache;
  la.block_table = a.index_table;
  la.cols = a.index_cols;
  la.key_blocks = a.key_blocks;
  la.source_capacity = a.row_len;
  la.heads = a.heads;
  la.batch = 1;
  const dim3 grid(static_cast<uint32_t>(ceil_div(ceil_div(a.n, kBlock), kScoreWaves)), 1);
  if (a.heads == 32) {
    launch_kernel(kKernLimScore, lim_score_kernel<T, 32, 1, false>, grid, dim3(kScoreWaves * kWave), stream, la,
                  w.scores, 0, static_cast<int>(a.n), LimWs{});
  } else {
    launch_kernel(kKernLimScore, lim_score_kernel<T, 64, 1, false>, grid, dim3(kScoreWaves * kWave), stream, la,
                  w.scores, 0, static_cast<int>(a.n), LimWs{});
  }
  return hipGetLastError();
}

template <typename T, int Q>
hipError_t launch_lim(const LimArgs& a, hipStream_t stream) {
  const LimWs w = carve(a.workspace, a.batch, a.source_capacity, Q);
  const dim3 grid(static_cast<uint32_t>(ceil_div(a.cols * kBlock, kScoreWaves * score_tokens_per_wave(Q))),
                  static_cast<uint32_t>(a.batch));
  const int mtp = Q > 1 ? 1 : 0;
  const int parts = static_cast<int>(mtp_parts(a.source_capacity));
  // The chunk counts are scanned one part per thread (MTP3 pass B, MTP0's last chunk).
  if (parts > kManageThreads) return hipErrorInvalidValue;
  // MTP0: the score kernel also writes the per-block key ranges and zeroes the chunked passes' state.
  const LimWs side = Q == 1 ? w : LimWs{};
  if (a.heads == 32) {
    launch_kernel(kKernLimScore, lim_score_kernel<T, 32, Q, true>, grid, dim3(kScoreWaves * kWave), stream, a,
                  w.scores, mtp, -1, side);
  } else {
    launch_kernel(kKernLimScore, lim_score_kernel<T, 64, Q, true>, grid, dim3(kScoreWaves * kWave), stream, a,
                  w.scores, mtp, -1, side);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 mgrid(static_cast<uint32_t>(a.batch)), mblock(kManageThreads);
  const dim3 tgrid(static_cast<uint32_t>(a.batch * Q));
  const dim3 pgrid(static_cast<uint32_t>(a.batch * parts));
  if (Q == 1) {
    launch_kernel(kKernLimHist, lim_hist_kernel, pgrid, mblock, stream, a, w, parts);
    if (a.batch * parts <= kResidentChunks) {
      launch_kernel(kKernLimClassify, lim_classify_kernel, pgrid, mblock, stream, a, w, parts);
    } else {
      launch_kernel(kKernLimChunks, lim_chunks_kernel, pgrid, mblock, stream, a, w, parts);
      launch_kernel(kKernLimResolve, lim_resolve_kernel, mgrid, mblock, stream, a, w, parts);
    }
    return hipGetLastError();
  }
  // MTP3: thresholds first, one workgroup per (request, query) score row.
  if (a.source_capacity <= 16 * kChunk)
    launch_kernel(kKernLimThreshold, lim_threshold_kernel<16>, tgrid, mblock, stream, a, w, Q, 0);
  else
    launch_kernel(kKernLimThreshold, lim_threshold_kernel<0>, tgrid, mblock, stream, a, w, Q, 0);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  launch_kernel(kKernLimMtpPassA, lim_mtp_pass_a_kernel, pgrid, mblock, stream, a, w, parts);
  launch_kernel(kKernLimMtpVictims, lim_mtp_victims_kernel, mgrid, mblock, stream, a, w, parts);
  launch_kernel(kKernLimMtpPassB, lim_mtp_pass_b_kernel, pgrid, mblock, stream, a, w, parts);
  return hipGetLastError();
}

}  // namespace

size_t lim_workspace_bytes(int64_t batch, int64_t source_capacity, int queries) {
  size_t bytes = 0;
  (void)lim_layout(nullptr, batch, source_capacity, queries, &bytes);
  return bytes;
}

size_t lidu_init_workspace_bytes(int64_t source_capacity) {
  return align256(sizeof(float) * source_capacity) + 2 * align256(sizeof(int32_t) * kSlotStride) + 256;
}

int64_t lidu_list_capacity() { return kSlotStride; }

hipError_t launch_lidu_init(const LiduInitArgs& a, hipStream_t stream) {
  const InitWs w = carve_init(a.workspace, a.row_len);
  hipError_t e = a.elem == Elem::kBf16 ? launch_lidu_scores<Bf16>(a, w, stream) : launch_lidu_scores<F16>(a, w, stream);
  if (e != hipSuccess) return e;
  const float* s = static_cast<const float*>(w.scores);
  const int n = static_cast<int>(a.n), c = static_cast<int>(a.c);
  // Sources of up to one group (32768 tokens) keep their keys in registers
  // (64 per thread; at 128 the compiler moved the array to scratch memory).
  if (a.n <= kInitGroup * kChunk)
    launch_kernel(kKernLiduInit, lidu_init_reg_kernel, dim3(1), dim3(kManageThreads), stream, s, n, c, a.pool_row,
                  a.row_len, w);
  else
    launch_kernel(kKernLiduInit, lidu_init_kernel, dim3(1), dim3(kManageThreads), stream, s, n, c, a.pool_row,
                  a.row_len, w);
  return hipGetLastError();
}

hipError_t launch_lidu_shared_list(const LiduInitArgs& a, hipStream_t stream) {
  const InitWs w = carve_init(a.workspace, a.row_len);
  launch_kernel(kKernLiduShared, lidu_shared_kernel, dim3(1), dim3(kManageThreads), stream,
                static_cast<const int32_t*>(a.pool_row), a.row_len, w);
  return hipGetLastError();
}

const int32_t* lidu_list_count(const LiduInitArgs& a) { return carve_init(a.workspace, a.row_len).count; }

hipError_t launch_lidu_copy(const LiduInitArgs& a, hipStream_t stream) {
  const InitWs w = carve_init(a.workspace, a.row_len);
  ScatterArgs sa{};
  sa.src_ids = w.src;
  sa.dst_slots = w.dst;
  sa.copy_counts = w.count;
  sa.hbm_table = a.hbm_table;
  sa.dram_table = a.dram_table;
  sa.hbm_kpe = a.hbm_kpe;
  sa.hbm_ckv = a.hbm_ckv;
  sa.dram_kpe = a.dram_kpe;
  sa.dram_ckv = a.dram_ckv;
  sa.batch = 1;
  sa.cap = a.c;
  sa.hbm_cols = a.hbm_cols;
  sa.dram_cols = a.dram_cols;
  sa.hbm_blocks = a.hbm_blocks;
  sa.dram_blocks = a.dram_blocks;
  return launch_scatter_copy(sa, stream);
}

hipError_t launch_fused_li_manage(const LimArgs& a, hipStream_t stream) {
  return a.elem == Elem::kBf16 ? launch_lim<Bf16, 1>(a, stream) : launch_lim<F16, 1>(a, stream);
}

hipError_t launch_fused_li_manage_mtp(const LimArgs& a, hipStream_t stream) {
  return a.elem == Elem::kBf16 ? launch_lim<Bf16, kMtpQueries>(a, stream) : launch_lim<F16, kMtpQueries>(a, stream);
}

}  // namespace nvdsa
