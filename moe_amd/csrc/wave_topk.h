// Wave-wide top-k on wave64: the rank rule shared by the routers and the
// routing statistics.  A wave holds one row of up to 64*NV values, value j
// of lane L being entry j*64 + L; entries rank by value, descending, and
// equal values by lower index.  The order is total: a NaN (of either sign)
// ranks above every number, as torch.topk places NaN first, NaNs among
// themselves by index; -0 and +0 are equal values.
#pragma once
#include <type_traits>

#include "common.h"

namespace moe {

// True when candidate (va, ea) ranks before (vb, eb).
__device__ __forceinline__ bool ranks_before(float va, int ea, float vb, int eb) {
  const bool na = va != va, nb = vb != vb;
  if (na | nb) return na && (!nb || ea < eb);
  return va > vb || (va == vb && ea < eb);
}

// Wave-wide arg-max of (v, e) under ranks_before; every lane gets the result.
// Within rows of 16 lanes by DPP (xor 1, xor 2 quad permutes, then the
// half-row and row mirrors), all in VALU with no LDS-routed shuffles; then
// the four row results are read out (v_readlane) and compared as uniform
// values.  ranks_before is a total order, so the result does not depend on
// the pairing.
__device__ __forceinline__ void take_better(float& v, int& e, float ov, int oe) {
  if (ranks_before(ov, oe, v, e)) {
    v = ov;
    e = oe;
  }
}
template <int CTRL>
__device__ __forceinline__ void dpp_argmax_step(float& v, int& e) {
  const float ov = __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
  const int oe = __builtin_amdgcn_update_dpp(0, e, CTRL, 0xF, 0xF, false);
  take_better(v, e, ov, oe);
}
__device__ __forceinline__ void wave_argmax(float& v, int& e) {
  dpp_argmax_step<0xB1>(v, e);   // quad_perm [1,0,3,2]
  dpp_argmax_step<0x4E>(v, e);   // quad_perm [2,3,0,1]
  dpp_argmax_step<0x141>(v, e);  // row_half_mirror: lane i <-> 7-i of each 8
  dpp_argmax_step<0x140>(v, e);  // row_mirror: lane i <-> 15-i of each 16
  const int vi = __builtin_bit_cast(int, v);
  float bv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, 0));
  int be = __builtin_amdgcn_readlane(e, 0);
#pragma unroll
  for (int r = 16; r < 64; r += 16)
    take_better(bv, be, __builtin_bit_cast(float, __builtin_amdgcn_readlane(vi, r)),
                __builtin_amdgcn_readlane(e, r));
  v = bv;
  e = be;
}

// Best not-yet-taken entry held by this lane (e = j*64 + lane).
template <int NV>
__device__ __forceinline__ void lane_best(const float (&val)[NV], uint64_t taken, int lane,
                                          float& bv, int& be) {
  bv = -INFINITY;
  be = 0x7fffffff;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    if (!((taken >> j) & 1ull)) {
      int e = j * 64 + lane;
      if (ranks_before(val[j], e, bv, be)) { bv = val[j]; be = e; }
    }
  }
}


// ---------------------------------------------------------------------------
// Group top-k: G = 8 or 16 consecutive lanes own one row (64/G rows per
// wave), V entries per lane (entries g*V .. g*V+V-1 of lane g of the group).
// Entries are ranked through one ordered 64-bit key each, (value mapped to
// an unsigned order) << 32 | (2^32 - 1 - index): larger key = ranks first,
// so a single unsigned max implements "value descending, lower index on
// equal values".  -0 is folded into +0 first (equal values compare by index
// only); every NaN is mapped to the positive quiet NaN first, which lands
// above every number (as in torch.topk) whatever the NaN's sign bit.
__device__ __forceinline__ uint64_t rank_key(float v, int idx) {
  uint32_t b = v != v ? 0x7fc00000u : __float_as_uint(v + 0.0f);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)b << 32) | (uint32_t)(0xffffffffu - (uint32_t)idx);
}
__device__ __forceinline__ float key_value(uint64_t k) {
  uint32_t b = (uint32_t)(k >> 32);
  b = (b & 0x80000000u) ? (b & 0x7fffffffu) : ~b;
  return __uint_as_float(b);
}
__device__ __forceinline__ int key_index(uint64_t k) {
  return (int)(0xffffffffu - (uint32_t)k);
}

// One butterfly step within rows of 16 lanes (every source lane is valid).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, CTRL, 0xF, 0xF, true);
}
// The steps that combine G consecutive lanes (G = 2, 4, 8, 16): quad xor 1,
// quad xor 2, half-row mirror (lane i <-> 7-i of each 8), row mirror (lane
// i <-> 15-i of each 16).  Both partners of a step compute op(a, b) of the
// same two values, so every lane of the group ends with the same result.
template <int G, typename F>
__device__ __forceinline__ void group_steps(F&& step) {
  if constexpr (G >= 2) step(std::integral_constant<int, 0xB1>{});
  if constexpr (G >= 4) step(std::integral_constant<int, 0x4E>{});
  if constexpr (G >= 8) step(std::integral_constant<int, 0x141>{});
  if constexpr (G >= 16) step(std::integral_constant<int, 0x140>{});
}
// 32-bit form for bf16 values and indices below 2^16: the same order from
// the bf16 bits (value exact), one unsigned max per comparison.
__device__ __forceinline__ uint32_t rank_key16(uint32_t bf_bits, int idx) {
  uint32_t b = bf_bits == 0x8000u ? 0u : bf_bits;  // -0 -> +0
  if ((b & 0x7f80u) == 0x7f80u && (b & 0x7fu)) b = 0x7fc0u;  // any NaN -> +qNaN
  b = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
  return (b << 16) | (0xffffu - (uint32_t)idx);
}
__device__ __forceinline__ float key_value(uint32_t k) {
  uint32_t b = k >> 16;
  b = (b & 0x8000u) ? (b & 0x7fffu) : (~b & 0xffffu);
  return __uint_as_float(b << 16);
}
__device__ __forceinline__ int key_index(uint32_t k) { return (int)(0xffffu - (k & 0xffffu)); }
template <int G>
__device__ __forceinline__ uint32_t group_max_key(uint32_t k) {
  group_steps<G>([&](auto c) {
    const uint32_t o = dpp_u32<decltype(c)::value>(k);
    k = o > k ? o : k;
  });
  return k;
}
template <int G>
__device__ __forceinline__ uint64_t group_max_key(uint64_t k) {
  group_steps<G>([&](auto c) {
    constexpr int CTRL = decltype(c)::value;
    const uint64_t o = ((uint64_t)dpp_u32<CTRL>((uint32_t)(k >> 32)) << 32) |
                       dpp_u32<CTRL>((uint32_t)k);
    k = o > k ? o : k;
  });
  return k;
}
template <int G>
__device__ __forceinline__ float group_max(float v) {
  group_steps<G>([&](auto c) {
    v = fmaxf(v, __uint_as_float(dpp_u32<decltype(c)::value>(__float_as_uint(v))));
  });
  return v;
}
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  group_steps<G>([&](auto c) { v += __uint_as_float(dpp_u32<decltype(c)::value>(__float_as_uint(v))); });
  return v;
}

// Lanes per token and experts per lane of the group kernels, or G = 0 when
// E and K call for the wave-per-token kernels.
static inline void group_shape(int E, int K, int& G, int& V) {
  G = K <= 8 ? 8 : (K <= 16 ? 16 : 0);
  if (G == 8 && E > 8 * 16) G = 16;
  if (G == 0 || E > G * 16) {
    G = 0;
    return;
  }
  const int need = (E + G - 1) / G;
  V = need <= 4 ? 4 : (need <= 8 ? 8 : 16);
}

// Wave-wide maximum of a 64-bit key: DPP within rows of 16 lanes, then the
// four row results compared as uniform values.
__device__ __forceinline__ uint64_t readlane_u64(uint64_t k, int l) {
  return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(k >> 32), l) << 32) |
         (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, l);
}

// Extracts the K best entries in rank order from their rank keys (0 for an
// entry that takes no part); lane k < K receives the k-th selected expert id
// and its key (other lanes get 0).  Keys are unique (the index is part of
// the key), so round k's winner is the largest key below round k-1's
// winner: each lane takes the minimum of thr-1-key over its entries (keys
// at or above thr wrap past thr-1 and lose), the wave the maximum of the
// lanes' results.
template <int NV>
__device__ __forceinline__ int wave_topk_keys(const uint64_t (&key)[NV], int lane, int K,
                                              uint64_t& mine) {
  uint64_t thr = ~0ull;
  mine = 0;
  for (int k = 0; k < K; ++k) {
    const uint64_t lim = thr - 1;
    uint64_t d = lim - key[0];
#pragma unroll
    for (int j = 1; j < NV; ++j) {
      const uint64_t dj = lim - key[j];
      d = dj < d ? dj : d;
    }
    uint64_t b = d <= lim ? lim - d : 0ull;
    b = group_max_key<16>(b);
    uint64_t w = readlane_u64(b, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16) {
      const uint64_t o = readlane_u64(b, r);
      w = o > w ? o : w;
    }
    thr = w;
    mine = lane == k ? w : mine;
  }
  return lane < K ? key_index(mine) : 0;
}

// The same from values (entry j*64 + lane; entries in `taken` take no part).
template <int NV>
__device__ __forceinline__ int wave_topk(const float (&val)[NV], uint64_t taken, int lane, int K) {
  uint64_t key[NV], mine;
#pragma unroll
  for (int j = 0; j < NV; ++j)
    key[j] = ((taken >> j) & 1ull) ? 0ull : rank_key(val[j], j * 64 + lane);
  return wave_topk_keys<NV>(key, lane, K, mine);
}

}  // namespace moe
