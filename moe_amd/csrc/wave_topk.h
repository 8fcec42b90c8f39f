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
__device__ __forceinline__ void wave_argmax(float& v, int& e) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(v, o, 64);
    int oe = __shfl_xor(e, o, 64);
    if (ranks_before(ov, oe, v, e)) { v = ov; e = oe; }
  }
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
