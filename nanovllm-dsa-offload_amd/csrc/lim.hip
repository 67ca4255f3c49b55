// fused_li_manage / fused_li_manage_mtp: LightningIndexer scores, top-2048
// selection and persistent HBM-slot bookkeeping on gfx950.
//
// Two launches per call:
//   1. lim_score_kernel  — one wavefront per 128-token index block.  The
//      block's key rows are the MFMA B operand (32 tokens x 16 dims per
//      v_mfma_f32_32x32x16), the request's index query rows the A operand
//      (staged once per workgroup in LDS), fp32 accumulation, then ReLU,
//      per-head weight and head reduction in registers.  Scores go to an fp32
//      workspace row per query; the key scan is the only large HBM stream.
//   2. lim_manage_kernel(_mtp) — one 1024-thread workgroup per request:
//      radix select of the top-2048 threshold on the scores, one ordered
//      pass over the candidates against the request's pool row, victim
//      selection, pairing and pool update.
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

#include "nvdsa_common.h"
#include "nvdsa_kernels.h"

namespace nvdsa {
namespace {

constexpr int kScoreWaves = 4;                  // waves per score workgroup
constexpr int kQStride = kIndexDim + 8;         // padded LDS row (bank spread)
constexpr int kManageThreads = 1024;
constexpr int kSlotStride = kMaxCacheTokens + 1;  // 16384 entries per request
constexpr uint32_t kStateShift = 24;
constexpr uint32_t kStateFree = 0;
constexpr uint32_t kStateHit = 1;
constexpr uint32_t kStateCand = 2;
constexpr uint32_t kTokenMask = (1u << kStateShift) - 1;

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct LimWs {
  float* scores;        // [B*Q, S_cap]
  uint32_t* slot_table; // [B, 16384] token | state << 24
  uint32_t* slot_key;   // [B, 16384] score key of candidate slots
  int32_t* miss_list;   // [B, 8192]
  uint8_t* masks;       // [B, S_cap] per-token query mask (MTP)
};

LimWs carve(void* base, int64_t batch, int64_t cap, int queries) {
  char* p = static_cast<char*>(base);
  LimWs w;
  w.scores = reinterpret_cast<float*>(p);
  p += align256(sizeof(float) * batch * queries * cap);
  w.slot_table = reinterpret_cast<uint32_t*>(p);
  p += align256(sizeof(uint32_t) * batch * kSlotStride);
  w.slot_key = reinterpret_cast<uint32_t*>(p);
  p += align256(sizeof(uint32_t) * batch * kSlotStride);
  w.miss_list = reinterpret_cast<int32_t*>(p);
  p += align256(sizeof(int32_t) * batch * kUnionCap);
  w.masks = queries > 1 ? reinterpret_cast<uint8_t*>(p) : nullptr;
  return w;
}

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

// ---------------------------------------------------------------------------
// 1. Scores.
template <typename T, int HEADS, int Q>
__global__ __launch_bounds__(kScoreWaves * kWave) void lim_score_kernel(LimArgs a, float* scores, int mtp) {
  __shared__ uint16_t qs[Q * HEADS * kQStride];
  __shared__ float ws[Q * HEADS];
  const int b = blockIdx.y;
  const int n = a.num_candidates[b];
  const int c = a.num_cache[b];
  const int r = a.pool_entries[b];
  const bool valid = mtp ? lim_mtp_row_valid(n, c, r, a.source_capacity, a.pool_rows)
                         : lim_row_valid(n, c, r, a.source_capacity, a.pool_rows);
  if (!valid) return;
  const int64_t col0 = static_cast<int64_t>(blockIdx.x) * kScoreWaves;
  if (col0 * kBlock >= n) return;

  // Stage the request's Q*HEADS query rows (16 x 16-byte chunks each) and weights.
  const uint4* qsrc = static_cast<const uint4*>(a.query) + static_cast<int64_t>(b) * Q * HEADS * 16;
  for (int i = threadIdx.x; i < Q * HEADS * 16; i += blockDim.x) {
    const int row = i >> 4, chunk = i & 15;
    *reinterpret_cast<uint4*>(&qs[row * kQStride + chunk * 8]) = qsrc[i];
  }
  const uint16_t* wsrc = static_cast<const uint16_t*>(a.weights) + static_cast<int64_t>(b) * Q * HEADS;
  for (int i = threadIdx.x; i < Q * HEADS; i += blockDim.x) ws[i] = T::to_float(wsrc[i]);
  __syncthreads();

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int grp = lane >> 5;   // k-half of the MFMA operand
  const int col_lane = lane & 31;
  const int64_t col = col0 + wave;
  const int64_t t0 = col * kBlock;
  if (t0 >= n) return;
  const int64_t cap = a.source_capacity;
  float* srow = scores + static_cast<int64_t>(b) * Q * cap;
  const int32_t phys = a.block_table[static_cast<int64_t>(b) * a.cols + col];
  if (phys < 0 || phys >= a.key_blocks) {
    for (int q = 0; q < Q; ++q)
      for (int j = lane; j < kBlock; j += kWave)
        if (t0 + j < n) srow[q * cap + t0 + j] = -FLT_MAX;
    return;
  }
  // Key tile: 4 token tiles x 8 k-steps, 16 bytes each, all loads issued first.
  const uint4* kp = static_cast<const uint4*>(a.key_cache) + static_cast<int64_t>(phys) * kBlock * 16;
  uint4 kb[4][8];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) kb[tt][ks] = kp[(tt * 32 + col_lane) * 16 + ks * 2 + grp];

#pragma unroll 1
  for (int q = 0; q < Q; ++q) {
    float part[4] = {0.f, 0.f, 0.f, 0.f};
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
      for (int tt = 0; tt < 4; ++tt) {
        f32x16_t acc = {};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
          acc = T::mfma32(__builtin_bit_cast(typename T::vec8, qa[ks]),
                          __builtin_bit_cast(typename T::vec8, kb[tt][ks]), acc);
#pragma unroll
        for (int i = 0; i < 16; ++i) part[tt] += wv[i] * fmaxf(acc[i], 0.f);
      }
    }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      float s = part[tt] + __shfl_xor(part[tt], 32, 64);
      if (s == 0.f) s = 0.f;  // one zero: -0 and +0 rank equal
      const int64_t t = t0 + tt * 32 + col_lane;
      if (grp == 0 && t < n) srow[q * cap + t] = s;
    }
  }
}

// ---------------------------------------------------------------------------
// Block-wide helpers for the 1024-thread manage kernels.

struct SelectOut {
  uint32_t thresh;  // key of the k-th largest element
  int need_eq;      // elements equal to thresh that belong to the selection
  int cnt_eq;       // elements equal to thresh
};

// k-th largest 32-bit key among included elements of [0, n) by an
// 11/11/10-bit radix select.  Requires (#included) >= k >= 1.
template <typename KeyFn>
__device__ SelectOut select_top(int n, int k, KeyFn key_of, uint32_t* hist, int* scratch, int* bcast) {
  uint32_t prefix = 0, pmask = 0;
  int remaining = k;
  int cnt_eq = 0;
  const int tid = threadIdx.x;
#pragma unroll 1
  for (int p = 0; p < 3; ++p) {
    const int shift = p == 0 ? 21 : (p == 1 ? 10 : 0);
    const uint32_t dmask = p == 2 ? 0x3ffu : 0x7ffu;
    for (int i = tid; i < 2048; i += kManageThreads) hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < n; i += kManageThreads) {
      uint32_t key;
      if (!key_of(i, key)) continue;
      if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & dmask], 1u);
    }
    __syncthreads();
    const int tb = kManageThreads - 1 - tid;  // descending bin pairs
    const int hi = static_cast<int>(hist[2 * tb + 1]);
    const int lo = static_cast<int>(hist[2 * tb]);
    int total;
    const int above = block_exclusive_scan(hi + lo, scratch, &total);
    if (above < remaining && remaining <= above + hi) {
      bcast[0] = 2 * tb + 1;
      bcast[1] = above;
      bcast[2] = hi;
    } else if (above + hi < remaining && remaining <= above + hi + lo) {
      bcast[0] = 2 * tb;
      bcast[1] = above + hi;
      bcast[2] = lo;
    }
    __syncthreads();
    prefix |= static_cast<uint32_t>(bcast[0]) << shift;
    pmask |= dmask << shift;
    remaining -= bcast[1];
    cnt_eq = bcast[2];
    __syncthreads();
  }
  return SelectOut{prefix, remaining, cnt_eq};
}

__device__ inline int block_sum(int v, int* scratch) {
  int total;
  (void)block_exclusive_scan(v, scratch, &total);
  return total;
}

// Exclusive block scan of four packed 16-bit counters (each chunk total must
// stay below 65536, which holds for 1024 threads).
__device__ inline uint64_t block_exclusive_scan4(uint64_t v, uint64_t* scratch, uint64_t* total) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  uint64_t x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t lo = __shfl_up(static_cast<uint32_t>(x), d, 64);
    const uint32_t hi = __shfl_up(static_cast<uint32_t>(x >> 32), d, 64);
    if (lane >= d) x += (static_cast<uint64_t>(hi) << 32) | lo;
  }
  if (lane == 63) scratch[wid] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t run = 0;
    for (int w = 0; w < nw; ++w) {
      const uint64_t t = scratch[w];
      scratch[w] = run;
      run += t;
    }
    scratch[nw] = run;
  }
  __syncthreads();
  const uint64_t excl = scratch[wid] + x - v;
  *total = scratch[nw];
  __syncthreads();
  return excl;
}

__device__ inline int lane16(uint64_t v, int q) { return static_cast<int>((v >> (16 * q)) & 0xffffu); }

__device__ inline uint32_t score_key(float s) { return float_key(s == 0.f ? 0.f : s); }

// Victim slots: the m non-hit slots of [0, c) with the smallest key (free
// slots first), ascending slot on ties, written in ascending slot order to
// vslot[0..min(m, #non-hit)).  Returns the number written.
__device__ int select_victims(int c, int m, const uint32_t* stab, const uint32_t* skey, int* vslot, uint32_t* hist,
                              int* scratch, int* bcast) {
  const int tid = threadIdx.x;
  if (m <= 0) return 0;
  int local = 0;
  for (int i = tid; i < c; i += kManageThreads) local += (stab[i] >> kStateShift) != kStateHit;
  const int nonhit = block_sum(local, scratch);
  const bool take_all = m >= nonhit;
  auto inv_key = [&](int i, uint32_t& key) -> bool {
    const uint32_t st = stab[i] >> kStateShift;
    if (st == kStateHit) return false;
    key = ~(st == kStateFree ? 0u : skey[i]);
    return true;
  };
  SelectOut sel{0, 0, 0};
  if (!take_all) sel = select_top(c, m, inv_key, hist, scratch, bcast);
  const bool need_rank = !take_all && sel.cnt_eq != sel.need_eq;
  int run = 0, eq_run = 0;
  for (int base = 0; base < c; base += kManageThreads) {
    const int i = base + tid;
    uint32_t key = 0;
    const bool nonhit_i = i < c && inv_key(i, key);
    bool victim;
    if (take_all) {
      victim = nonhit_i;
    } else {
      const bool gt = nonhit_i && key > sel.thresh;
      const bool eq = nonhit_i && key == sel.thresh;
      victim = gt || (eq && !need_rank);
      if (need_rank) {
        int tot;
        const int rk = block_exclusive_scan(eq ? 1 : 0, scratch, &tot);
        victim = gt || (eq && eq_run + rk < sel.need_eq);
        eq_run += tot;
      }
    }
    int tot;
    const int vp = block_exclusive_scan(victim ? 1 : 0, scratch, &tot);
    if (victim && run + vp < m) vslot[run + vp] = i;
    run += tot;
  }
  __syncthreads();
  return run < m ? run : m;
}

// ---------------------------------------------------------------------------
// 2a. MTP0 management.
__global__ __launch_bounds__(kManageThreads) void lim_manage_kernel(LimArgs a, LimWs w) {
  __shared__ uint32_t hist[2048];
  __shared__ int scratch[kManageThreads / 64 + 1];
  __shared__ int bcast[4];
  __shared__ int vslot[kTopK];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int n = a.num_candidates[b];
  const int c = a.num_cache[b];
  const int r = a.pool_entries[b];
  if (!lim_row_valid(n, c, r, a.source_capacity, a.pool_rows)) {
    if (tid == 0) a.miss_counts[b] = 0;
    return;
  }
  const int64_t cap = a.source_capacity;
  const float* s = w.scores + static_cast<int64_t>(b) * cap;
  int32_t* pool = a.pool + static_cast<int64_t>(r) * cap;
  uint32_t* stab = w.slot_table + static_cast<int64_t>(b) * kSlotStride;
  uint32_t* skey = w.slot_key + static_cast<int64_t>(b) * kSlotStride;
  int32_t* misses = w.miss_list + static_cast<int64_t>(b) * kUnionCap;
  int32_t* out_src = a.topk_src + static_cast<int64_t>(b) * kTopK;
  int32_t* out_dst = a.topk_dst + static_cast<int64_t>(b) * kTopK;

  for (int i = tid; i < c; i += kManageThreads) stab[i] = kStateFree;
  const SelectOut sel = select_top(
      n, kTopK, [&](int i, uint32_t& key) { key = score_key(s[i]); return true; }, hist, scratch, bcast);
  const bool need_rank = sel.cnt_eq != sel.need_eq;

  // Ordered pass over the candidates.
  int eq_run = 0, miss_run = 0;
  for (int base = 0; base < n; base += kManageThreads) {
    const int t = base + tid;
    const bool in = t < n;
    const uint32_t u = in ? score_key(s[t]) : 0u;
    const bool gt = in && u > sel.thresh;
    const bool eq = in && u == sel.thresh;
    bool chosen = gt || (eq && !need_rank);
    if (need_rank) {
      int tot;
      const int rk = block_exclusive_scan(eq ? 1 : 0, scratch, &tot);
      chosen = gt || (eq && eq_run + rk < sel.need_eq);
      eq_run += tot;
    }
    const int32_t slot = in ? pool[t] : -1;
    const bool cached = slot >= 0 && slot < c;
    const bool miss = chosen && !cached;
    int tot;
    const int mp = block_exclusive_scan(miss ? 1 : 0, scratch, &tot);
    if (miss) misses[miss_run + mp] = t;
    miss_run += tot;
    if (cached) {
      if (chosen) {
        stab[slot] = static_cast<uint32_t>(t) | (kStateHit << kStateShift);
      } else {
        stab[slot] = static_cast<uint32_t>(t) | (kStateCand << kStateShift);
        skey[slot] = u;
      }
    }
  }
  __syncthreads();
  const int m = miss_run;
  const int nv = select_victims(c, m, stab, skey, vslot, hist, scratch, bcast);

  // Misses first (ascending token), paired with ascending victim slots.
  for (int i = tid; i < m; i += kManageThreads) {
    const int t = misses[i];
    const int d = i < nv ? vslot[i] : -1;
    out_src[i] = t;
    out_dst[i] = d;
    if (d >= 0) {
      const uint32_t e = stab[d];
      if ((e >> kStateShift) == kStateCand) pool[e & kTokenMask] = -1;
      pool[t] = d;
    }
  }
  // Hits by descending old slot.
  int hit_run = 0;
  for (int base = 0; base < c; base += kManageThreads) {
    const int i = c - 1 - (base + tid);
    const uint32_t e = i >= 0 ? stab[i] : 0u;
    const bool hit = i >= 0 && (e >> kStateShift) == kStateHit;
    int tot;
    const int hp = block_exclusive_scan(hit ? 1 : 0, scratch, &tot);
    const int pos = m + hit_run + hp;
    if (hit && pos < kTopK) {
      out_src[pos] = static_cast<int32_t>(e & kTokenMask);
      out_dst[pos] = i;
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

// ---------------------------------------------------------------------------
// 2b. MTP3 management: union of the four top-2048 sets.
__global__ __launch_bounds__(kManageThreads) void lim_manage_mtp_kernel(LimArgs a, LimWs w) {
  __shared__ uint32_t hist[2048];
  __shared__ int scratch[kManageThreads / 64 + 1];
  __shared__ uint64_t scratch64[kManageThreads / 64 + 1];
  __shared__ int bcast[4];
  __shared__ int vslot[kUnionCap];
  __shared__ uint32_t thr[kMtpQueries];
  __shared__ int need[kMtpQueries];
  __shared__ int rank_needed[kMtpQueries];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int n = a.num_candidates[b];
  const int c = a.num_cache[b];
  const int r = a.pool_entries[b];
  if (!lim_mtp_row_valid(n, c, r, a.source_capacity, a.pool_rows)) {
    if (tid == 0) a.miss_counts[b] = 0;
    return;
  }
  const int64_t cap = a.source_capacity;
  const float* s = w.scores + static_cast<int64_t>(b) * kMtpQueries * cap;
  int32_t* pool = a.pool + static_cast<int64_t>(r) * cap;
  uint32_t* stab = w.slot_table + static_cast<int64_t>(b) * kSlotStride;
  uint32_t* skey = w.slot_key + static_cast<int64_t>(b) * kSlotStride;
  uint8_t* masks = w.masks + static_cast<int64_t>(b) * cap;
  int32_t* miss_src = a.miss_src + static_cast<int64_t>(b) * kUnionCap;
  int32_t* miss_dst = a.miss_dst + static_cast<int64_t>(b) * kUnionCap;

  for (int i = tid; i < c; i += kManageThreads) stab[i] = kStateFree;
  for (int q = 0; q < kMtpQueries; ++q) {
    const float* sq = s + q * cap;
    const SelectOut sel = select_top(
        n, kTopK, [&](int i, uint32_t& key) { key = score_key(sq[i]); return true; }, hist, scratch, bcast);
    if (tid == 0) {
      thr[q] = sel.thresh;
      need[q] = sel.need_eq;
      rank_needed[q] = sel.cnt_eq != sel.need_eq;
    }
  }
  __syncthreads();
  const bool any_rank = rank_needed[0] | rank_needed[1] | rank_needed[2] | rank_needed[3];

  // Pass A: query masks, slot states, union misses per first-selecting query.
  int eq_run[kMtpQueries] = {0, 0, 0, 0};
  int gmiss[kMtpQueries] = {0, 0, 0, 0};
  for (int base = 0; base < n; base += kManageThreads) {
    const int t = base + tid;
    const bool in = t < n;
    uint32_t u[kMtpQueries];
    uint32_t umax = 0;
    uint64_t eqp = 0;
    unsigned mask = 0;
#pragma unroll
    for (int q = 0; q < kMtpQueries; ++q) {
      u[q] = in ? score_key(s[q * cap + t]) : 0u;
      umax = u[q] > umax ? u[q] : umax;
      if (in && u[q] > thr[q]) mask |= 1u << q;
      if (in && u[q] == thr[q]) {
        if (rank_needed[q]) eqp |= uint64_t{1} << (16 * q);
        else mask |= 1u << q;
      }
    }
    if (any_rank) {
      uint64_t tot;
      const uint64_t rk = block_exclusive_scan4(eqp, scratch64, &tot);
#pragma unroll
      for (int q = 0; q < kMtpQueries; ++q) {
        if ((eqp >> (16 * q)) & 1u)
          if (eq_run[q] + lane16(rk, q) < need[q]) mask |= 1u << q;
        eq_run[q] += lane16(tot, q);
      }
    }
    const int32_t slot = in ? pool[t] : -1;
    const bool cached = slot >= 0 && slot < c;
    if (in) masks[t] = static_cast<uint8_t>(mask);
    if (cached) {
      if (mask) {
        stab[slot] = static_cast<uint32_t>(t) | (kStateHit << kStateShift);
      } else {
        stab[slot] = static_cast<uint32_t>(t) | (kStateCand << kStateShift);
        skey[slot] = umax;
      }
    }
    const int g = mask ? __builtin_ctz(mask) : 0;
    const uint64_t missp = (mask && !cached) ? (uint64_t{1} << (16 * g)) : 0;
    uint64_t tot;
    (void)block_exclusive_scan4(missp, scratch64, &tot);
#pragma unroll
    for (int q = 0; q < kMtpQueries; ++q) gmiss[q] += lane16(tot, q);
  }
  __syncthreads();
  const int m = gmiss[0] + gmiss[1] + gmiss[2] + gmiss[3];
  const int gbase[kMtpQueries] = {0, gmiss[0], gmiss[0] + gmiss[1], gmiss[0] + gmiss[1] + gmiss[2]};
  const int nv = select_victims(c, m, stab, skey, vslot, hist, scratch, bcast);

  // Pass B: union-ordered misses, per-query rows, pool update.
  int gm_run[kMtpQueries] = {0, 0, 0, 0};
  int row_run[kMtpQueries] = {0, 0, 0, 0};
  for (int base = 0; base < n; base += kManageThreads) {
    const int t = base + tid;
    const bool in = t < n;
    const unsigned mask = in ? masks[t] : 0u;
    const int32_t slot = mask ? pool[t] : -1;
    const bool cached = slot >= 0 && slot < c;
    const bool miss = mask && !cached;
    const int g = mask ? __builtin_ctz(mask) : 0;
    uint64_t tot;
    const uint64_t mrk = block_exclusive_scan4(miss ? (uint64_t{1} << (16 * g)) : 0, scratch64, &tot);
    int new_slot = slot;
    if (miss) {
      const int pos = gbase[g] + gm_run[g] + lane16(mrk, g);
      const int d = pos < nv ? vslot[pos] : -1;
      miss_src[pos] = t;
      miss_dst[pos] = d;
      new_slot = d;
      if (d >= 0) {
        const uint32_t e = stab[d];
        if ((e >> kStateShift) == kStateCand) pool[e & kTokenMask] = -1;
        pool[t] = d;
      }
    }
#pragma unroll
    for (int q = 0; q < kMtpQueries; ++q) gm_run[q] += lane16(tot, q);
    uint64_t rowp = 0;
#pragma unroll
    for (int q = 0; q < kMtpQueries; ++q)
      if ((mask >> q) & 1u) rowp |= uint64_t{1} << (16 * q);
    const uint64_t rrk = block_exclusive_scan4(rowp, scratch64, &tot);
#pragma unroll
    for (int q = 0; q < kMtpQueries; ++q) {
      if ((mask >> q) & 1u) {
        const int i = row_run[q] + lane16(rrk, q);
        const int64_t row = static_cast<int64_t>(b) * kMtpQueries + q;
        if (i < kTopK) {
          a.topk_src[row * kTopK + i] = miss ? t : -1;
          a.topk_dst[row * kTopK + i] = new_slot;
        }
      }
      row_run[q] += lane16(tot, q);
    }
  }
  if (tid == 0) a.miss_counts[b] = m;
}

template <typename T, int Q>
hipError_t launch_lim(const LimArgs& a, hipStream_t stream) {
  const LimWs w = carve(a.workspace, a.batch, a.source_capacity, Q);
  const dim3 grid(static_cast<uint32_t>(ceil_div(a.cols, kScoreWaves)), static_cast<uint32_t>(a.batch));
  const int mtp = Q > 1 ? 1 : 0;
  prof_before(stream, kKernLimScore);
  if (a.heads == 32) {
    hipLaunchKernelGGL((lim_score_kernel<T, 32, Q>), grid, dim3(kScoreWaves * kWave), 0, stream, a, w.scores, mtp);
  } else {
    hipLaunchKernelGGL((lim_score_kernel<T, 64, Q>), grid, dim3(kScoreWaves * kWave), 0, stream, a, w.scores, mtp);
  }
  prof_after(stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (Q == 1) {
    prof_before(stream, kKernLimManage);
    hipLaunchKernelGGL(lim_manage_kernel, dim3(static_cast<uint32_t>(a.batch)), dim3(kManageThreads), 0, stream, a,
                       w);
  } else {
    prof_before(stream, kKernLimManageMtp);
    hipLaunchKernelGGL(lim_manage_mtp_kernel, dim3(static_cast<uint32_t>(a.batch)), dim3(kManageThreads), 0,
                       stream, a, w);
  }
  prof_after(stream);
  return hipGetLastError();
}

}  // namespace

size_t lim_workspace_bytes(int64_t batch, int64_t source_capacity, int queries) {
  size_t total = align256(sizeof(float) * batch * queries * source_capacity);
  total += 2 * align256(sizeof(uint32_t) * batch * kSlotStride);
  total += align256(sizeof(int32_t) * batch * kUnionCap);
  if (queries > 1) total += align256(static_cast<size_t>(batch) * source_capacity);
  return total;
}

hipError_t launch_fused_li_manage(const LimArgs& a, hipStream_t stream) {
  return a.elem == Elem::kBf16 ? launch_lim<Bf16, 1>(a, stream) : launch_lim<F16, 1>(a, stream);
}

hipError_t launch_fused_li_manage_mtp(const LimArgs& a, hipStream_t stream) {
  return a.elem == Elem::kBf16 ? launch_lim<Bf16, kMtpQueries>(a, stream) : launch_lim<F16, kMtpQueries>(a, stream);
}

}  // namespace nvdsa
