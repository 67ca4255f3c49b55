// Shared constants and device helpers of the gfx950 DSA offload kernels.
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nvdsa {

// Shapes fixed by the operator contracts (reference README_ops.md:19-151,
// nanovllm/config.py:449-478).
constexpr int kBlock = 128;          // tokens per KV / index block
constexpr int kBlockShift = 7;
constexpr int kTopK = 2048;          // sparse selection width
constexpr int kCkvDim = 512;         // latent (nope) width
constexpr int kKpeDim = 64;          // rope width
constexpr int kQkDim = kCkvDim + kKpeDim;
constexpr int kIndexDim = 128;       // index head dim
constexpr int kMtpQueries = 4;       // MTP3 query rows per request
constexpr int kUnionCap = kTopK * kMtpQueries;
// Largest usable cache budget C: the reference packs HBM slots into a 14-bit
// payload field whose all-ones value marks "not cached"
// (ops/fused_li_manage/op_kernel/fused_li_manage_vector.h:53).
constexpr int kMaxCacheTokens = (1 << 14) - 1;
// Largest MTP0 source length (ops/fused_li_manage/op_kernel/fused_li_manage_common.h:52-53).
constexpr int kMaxSourceCapacity = 1 << 21;
constexpr int kMaxActualSeqLen = kMaxSourceCapacity - 1;

constexpr int kWave = 64;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Word 3 of a raw (unformatted, stride 0) buffer resource on CDNA: DATA_FORMAT
// = 32 bit, everything else zero.  A buffer load whose byte offset falls
// outside the resource's num_records returns zeros and touches no memory.
constexpr int kBufferFlags = 0x00020000;
// Cache-policy operand of a buffer load: nt (non-temporal; the line is not
// kept for reuse in the L2 or the memory-side Infinity Cache).
constexpr int kLoadNonTemporal = 2;

// Element type tags: storage is 16-bit either way; MFMA flavour differs.
struct Bf16 {
  using vec8 = bf16x8_t;
  __device__ static inline float to_float(uint16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
  }
  // Round-to-nearest-even fp32 -> bf16 (NaN kept quiet).
  __device__ static inline uint16_t from_float(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
  }
  // Round-to-nearest-even for finite values (no NaN check).
  __device__ static inline uint16_t from_finite(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
  }
  // Leading part of a hi + lo split: truncation (the lo part takes the rest).
  __device__ static inline uint16_t hi_part(float f) { return static_cast<uint16_t>(__float_as_uint(f) >> 16); }
  __device__ static inline f32x16_t mfma32(vec8 a, vec8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static inline f32x4_t mfma16(vec8 a, vec8 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

struct F16 {
  using vec8 = f16x8_t;
  __device__ static inline float to_float(uint16_t v) {
    _Float16 h = __builtin_bit_cast(_Float16, v);
    return static_cast<float>(h);
  }
  __device__ static inline uint16_t from_float(float f) {
    _Float16 h = static_cast<_Float16>(f);
    return __builtin_bit_cast(uint16_t, h);
  }
  __device__ static inline uint16_t from_finite(float f) { return from_float(f); }
  __device__ static inline uint16_t hi_part(float f) { return from_float(f); }
  __device__ static inline f32x16_t mfma32(vec8 a, vec8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static inline f32x4_t mfma16(vec8 a, vec8 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Order-preserving map fp32 -> uint32 (larger float => larger key).
__device__ inline uint32_t float_key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Workgroup barrier that orders LDS only: global loads still in flight stay
// in flight across it (a __syncthreads() would wait for them first).
__device__ inline void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <bool LDS_ONLY>
__device__ inline void scan_barrier() {
  if constexpr (LDS_ONLY)
    lds_barrier();
  else
    __syncthreads();
}

// Inclusive prefix sums over the wave's 64 lanes on the VALU: DPP row shifts
// build each 16-lane row's prefix (shifts 1, 2, 3, then 4 into banks 1-3 and 8
// into banks 2-3), and the row broadcasts add the rows before (lane 15 into
// rows 1 and 3, lane 31 into rows 2 and 3).  Lanes a step leaves out add 0.
// (The LDS-routed shuffles they replace wait one LDS round trip per step.)
template <int CTRL, int ROW_MASK, int BANK_MASK, bool BOUND_ZERO>
__device__ inline uint32_t dpp_u32(uint32_t x) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, ROW_MASK, BANK_MASK, BOUND_ZERO));
}
template <int CTRL, int ROW_MASK, int BANK_MASK, bool BOUND_ZERO>
__device__ inline uint64_t dpp_u64(uint64_t x) {
  const uint32_t lo = dpp_u32<CTRL, ROW_MASK, BANK_MASK, BOUND_ZERO>(static_cast<uint32_t>(x));
  const uint32_t hi = dpp_u32<CTRL, ROW_MASK, BANK_MASK, BOUND_ZERO>(static_cast<uint32_t>(x >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}
template <typename U, int CTRL, int ROW_MASK, int BANK_MASK, bool BOUND_ZERO>
__device__ inline U dpp_any(U x) {
  if constexpr (sizeof(U) == 8)
    return dpp_u64<CTRL, ROW_MASK, BANK_MASK, BOUND_ZERO>(x);
  else
    return dpp_u32<CTRL, ROW_MASK, BANK_MASK, BOUND_ZERO>(x);
}
template <typename U>
__device__ inline U wave_inclusive_scan(U x) {
  U s = x + dpp_any<U, 0x111, 0xf, 0xf, true>(x);  // row_shr:1
  s += dpp_any<U, 0x112, 0xf, 0xf, true>(x);       // row_shr:2
  s += dpp_any<U, 0x113, 0xf, 0xf, true>(x);       // row_shr:3
  s += dpp_any<U, 0x114, 0xf, 0xe, true>(s);       // row_shr:4, lanes 4-15 of each row
  s += dpp_any<U, 0x118, 0xf, 0xc, true>(s);       // row_shr:8, lanes 8-15
  s += dpp_any<U, 0x142, 0xa, 0xf, false>(s);      // row_bcast:15 into rows 1 and 3
  s += dpp_any<U, 0x143, 0xc, 0xf, false>(s);      // row_bcast:31 into rows 2 and 3
  return s;
}

// Cross-lane combines on the VALU.  v_permlane16_swap / v_permlane32_swap
// with the value in both operands leave the values of lanes i and i ^ 16
// (i ^ 32) in the two results, in the same order for both lanes of a pair,
// so a commutative op gives both lanes the same result.
template <typename Op>
__device__ inline float xor16_op(float x, Op op) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
template <typename Op>
__device__ inline float xor32_op(float x, Op op) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// op over all 64 lanes, in every lane: butterflies within each row of 16
// lanes (DPP quad permutes and mirrors), then across rows.
template <typename Op>
__device__ inline float wave_all_op(float x, Op op) {
  auto dpp = [](float v, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), decltype(ctrl)::value, 0xf,
                                                      0xf, false));
  };
  x = op(x, dpp(x, std::integral_constant<int, 0xb1>{}));   // quad_perm [1,0,3,2]
  x = op(x, dpp(x, std::integral_constant<int, 0x4e>{}));   // quad_perm [2,3,0,1]
  x = op(x, dpp(x, std::integral_constant<int, 0x141>{}));  // row_half_mirror
  x = op(x, dpp(x, std::integral_constant<int, 0x140>{}));  // row_mirror
  x = xor16_op(x, op);
  return xor32_op(x, op);
}
// An idempotent op (min, max, or) over the wave's 64 lanes, left in lane 63:
// butterflies within each row of 16 lanes (DPP quad permutes and mirrors),
// then the row broadcasts (lane 15 into rows 1 and 3, lane 31 into rows 2
// and 3).  Lanes a broadcast leaves out combine with their own value.
template <typename Op>
__device__ inline uint32_t wave_reduce_to_lane63(uint32_t x, Op op) {
  auto dpp = [](uint32_t v, auto ctrl, auto row_mask) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v),
                                                             decltype(ctrl)::value, decltype(row_mask)::value, 0xf,
                                                             false));
  };
  using std::integral_constant;
  x = op(x, dpp(x, integral_constant<int, 0xb1>{}, integral_constant<int, 0xf>{}));   // quad_perm [1,0,3,2]
  x = op(x, dpp(x, integral_constant<int, 0x4e>{}, integral_constant<int, 0xf>{}));   // quad_perm [2,3,0,1]
  x = op(x, dpp(x, integral_constant<int, 0x141>{}, integral_constant<int, 0xf>{}));  // row_half_mirror
  x = op(x, dpp(x, integral_constant<int, 0x140>{}, integral_constant<int, 0xf>{}));  // row_mirror
  x = op(x, dpp(x, integral_constant<int, 0x142>{}, integral_constant<int, 0xa>{}));  // row_bcast:15
  return op(x, dpp(x, integral_constant<int, 0x143>{}, integral_constant<int, 0xc>{}));  // row_bcast:31
}
struct MinU32Op {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a < b ? a : b; }
};
struct MaxU32Op {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; }
};
struct OrU32Op {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a | b; }
};
struct MaxOp {
  __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct AddOp {
  __device__ float operator()(float a, float b) const { return a + b; }
};

// Block-wide exclusive prefix sum of one int per thread (blockDim <= 1024,
// multiple of 64).  `scratch` must hold blockDim/64 + 1 ints.  Returns the
// exclusive prefix; *total receives the block sum.  Every thread reads the
// wave totals itself (independent LDS reads instead of one thread's chain).
// Contains barriers: full ones, or with LDS_ONLY barriers that order LDS only
// (for callers whose global writes nobody reads before a later full barrier).
template <bool LDS_ONLY = false>
__device__ inline int block_exclusive_scan(int v, int* scratch, int* total) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int x = static_cast<int>(wave_inclusive_scan(static_cast<uint32_t>(v)));
  if (lane == 63) scratch[wid] = x;
  scan_barrier<LDS_ONLY>();
  int before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < 16; ++w) {
    if (w < nw) {
      const int t = scratch[w];
      before += w < wid ? t : 0;
      tot += t;
    }
  }
  *total = __builtin_amdgcn_readfirstlane(tot);  // uniform: may steer barrier-containing code
  scan_barrier<LDS_ONLY>();  // scratch is reused by the next scan
  return before + x - v;
}

// Exclusive prefix of a 0/1 flag within the wave using a ballot.
__device__ inline int wave_flag_prefix(bool flag, uint64_t* ballot_out) {
  const uint64_t b = __ballot(flag);
  const int lane = threadIdx.x & 63;
  const uint64_t below = lane == 0 ? 0ull : (b & ((~0ull) >> (64 - lane)));
  *ballot_out = b;
  return __popcll(below);
}

}  // namespace nvdsa
