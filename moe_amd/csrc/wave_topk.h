// Wave-wide top-k on wave64: the rank rule shared by the routers and the
// routing statistics.  A wave holds one row of up to 64*NV values, value j
// of lane L being entry j*64 + L; entries rank by value, descending, and
// equal values by lower index.
#pragma once
#include "common.h"

namespace moe {

// True when candidate (va, ea) ranks before (vb, eb).
__device__ __forceinline__ bool ranks_before(float va, int ea, float vb, int eb) {
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

// Extracts the K best of val (not in `taken`) in rank order; lane k < K
// receives the k-th selected expert id (other lanes get 0).
template <int NV>
__device__ __forceinline__ int wave_topk(const float (&val)[NV], uint64_t taken, int lane, int K) {
  int mine = 0;
  for (int k = 0; k < K; ++k) {
    float bv;
    int be;
    lane_best<NV>(val, taken, lane, bv, be);
    wave_argmax(bv, be);
    if (lane == k) mine = be;
    if ((be & 63) == lane) taken |= 1ull << (be >> 6);
  }
  return mine;
}

}  // namespace moe
