// Softmax top-K of one token on a group of G consecutive lanes: the core
// shared by the softmax router kernel (router.hip) and the gating linear
// with the router fused into its epilogue (gemm.hip), so that both produce
// the same bits.  Lane g of the group holds the token's entries
// e0 = g*V .. e0+V-1 as fp32 values v (-inf past E) with their rank keys
// (wave_topk.h: value descending, lower index first on equal values).
// Reference: Qwen3MoeTopKRouter.forward, src/models/modeling_qwen3_moe.py:
// 269-274 (softmax in fp32, top-k, renormalisation by the sum, no epsilon).
#pragma once
#include "wave_topk.h"

namespace moe {

// exp(v - max) per entry (0 past E) and their group sum s; m = the max.
// A NaN logit makes every prob of the row NaN, and the reference ranks the
// probs: the row's entries then all tie and rank by index (the keys are
// replaced by NaN keys).
template <int G, int V, typename Key>
__device__ __forceinline__ void group_softmax(const float (&v)[V], Key (&key)[V], int e0, int E,
                                              float (&p)[V], float& m, float& s) {
  uint32_t nan_row = 0;
#pragma unroll
  for (int j = 0; j < V; ++j) nan_row |= (uint32_t)(v[j] != v[j]);
  if (group_max_key<G>(nan_row)) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int e = e0 + j;
      if constexpr (sizeof(Key) == 4) key[j] = e < E ? rank_key16(0x7fc0u, e) : 0u;
      else key[j] = e < E ? rank_key(__builtin_nanf(""), e) : 0ull;
    }
  }
  m = -INFINITY;
#pragma unroll
  for (int j = 0; j < V; ++j) m = fmaxf(m, v[j]);
  m = group_max<G>(m);
  s = 0.f;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    p[j] = (e0 + j < E) ? expf(v[j] - m) : 0.f;
    s += p[j];
  }
  s = group_sum<G>(s);
}

// K rounds of a group max over the keys; lane g < K receives the g-th
// selection: its prob p = exp(value - m) * rs (the same bits as the probs row
// written with rs = 1/s), renormalised by the group sum of the selected
// probs, and its expert.  Keys are unique (the index is part of the key), so
// round k's winner is the largest key below round k-1's winner: each lane
// takes the minimum of thr-1-key (keys at or above thr wrap past thr-1 and
// lose), and the keys themselves stay untouched.
template <int G, int V, typename Key>
__device__ __forceinline__ void group_topk(const Key (&key)[V], float m, float rs, int g, int K,
                                           int renorm, float& my_w, int& my_e) {
  Key thr = ~(Key)0;  // every key of a valid entry is below it
  Key mine = 0;
  for (int k = 0; k < K; ++k) {
    const Key lim = thr - 1;
    Key d = lim - key[0];
#pragma unroll
    for (int j = 1; j < V; ++j) {
      const Key dj = lim - key[j];
      d = dj < d ? dj : d;
    }
    Key b = d <= lim ? lim - d : (Key)0;  // this lane's largest key below thr
    b = group_max_key<G>(b);
    thr = b;
    mine = g == k ? b : mine;
  }
  const float pe = g < K ? expf(key_value(mine) - m) * rs : 0.f;
  my_w = pe;
  if (renorm) my_w = pe / group_sum<G>(pe);
  my_e = key_index(mine);
}

}  // namespace moe
