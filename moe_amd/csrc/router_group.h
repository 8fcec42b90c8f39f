// Softmax top-K of one token on a group of G consecutive lanes: the core
// shared by the softmax router kernel (router.hip) and the gating linear
// with the router fused into its epilogue (gemm.hip), so that both produce
// the same bits; and the DeepSeek router's sigmoid top-K core of that fused
// epilogue.  Lane g of the group holds the token's entries
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

// The input of the DeepSeek router kernels: logits (scores = sigmoid,
// fp32 arithmetic after it: src/models/router.py:107-138), or, with
// scores_in, the scores themselves -- the reference's torch.sigmoid of bf16
// logits under bf16 autocast, passed as fp32 values -- after which the
// weights follow torch's bf16 arithmetic: their sum rounded to bf16 (+1e-20),
// the quotient and the scaled weight each rounded to bf16.
__device__ __forceinline__ float dsk_score(float x, int scores_in) {
  return scores_in ? x : sigmoidf_(x);
}
__device__ __forceinline__ float dsk_weight(float v, float ssum, int renorm, float scaling,
                                            int scores_in) {
  if (scores_in) {
    if (renorm) v = round_bf(v / round_bf(round_bf(ssum) + 1e-20f));
    if (scaling > 0.f) v = round_bf(v * scaling);
  } else {
    if (renorm) v = v / (ssum + 1e-20f);
    if (scaling > 0.f) v = v * scaling;
  }
  return v;
}

// DeepSeek-V3 selection of one token on a group of G lanes (the router
// kernel, router.hip, and the gating linear's fused epilogue, gemm.hip, so
// that both produce the same bits): lane g holds the token's entries
// e0 = g*V .. e0+V-1 as unbiased sigmoid scores sc and rank keys of the
// biased scores (0 past E).  With ngroups > 0 the experts form ngroups equal
// groups of eg = E/ngroups (ngroups <= G); each group is scored by the sum of
// its (K / gtopk) best biased scores, added best first, the gtopk best groups
// (higher score first, lower group id on equal scores) are kept and the
// other groups' entries drop out (router.py:22-70).  Then K rounds of a group
// max over the keys; the winner's owner lane hands its unbiased score to the
// group (router.py:130) and counts the selection in cnt (when count), the
// scores are summed in rank order for the renormalisation (+1e-20) and
// lane g < K receives the g-th weight and expert (router.py:133-138), in
// torch's bf16 arithmetic when scores_in (dsk_weight).  The order of every
// step is that of the wave-per-token router kernel as well, so the
// selection and the weights are its bit for bit on the same scores.
template <int G, int V>
__device__ __forceinline__ void group_sigmoid_topk(const float (&sc)[V], uint64_t (&key)[V],
                                                   const int (&grp)[V], int g, int K,
                                                   int ngroups, int gtopk, int renorm,
                                                   float scaling, int scores_in, bool count,
                                                   int (&cnt)[V], float& my_w, int& my_e) {
  if (ngroups > 0) {
    const int per = K / gtopk;
    float gv = -INFINITY;  // lane g < ngroups: group g's score
    for (int gi = 0; gi < ngroups; ++gi) {
      uint64_t gk[V];
#pragma unroll
      for (int j = 0; j < V; ++j) gk[j] = grp[j] == gi ? key[j] : 0ull;
      float acc = 0.f;
      for (int q = 0; q < per; ++q) {
        uint64_t b = gk[0];
#pragma unroll
        for (int j = 1; j < V; ++j) b = gk[j] > b ? gk[j] : b;
        b = group_max_key<G>(b);
        acc += key_value(b);
#pragma unroll
        for (int j = 0; j < V; ++j) gk[j] = gk[j] == b ? 0ull : gk[j];
      }
      gv = g == gi ? acc : gv;
    }
    uint64_t gkey = g < ngroups ? rank_key(gv, g) : 0ull;
    uint32_t keep = 0;
    for (int q = 0; q < gtopk; ++q) {
      const uint64_t b = group_max_key<G>(gkey);
      keep |= 1u << key_index(b);
      gkey = gkey == b ? 0ull : gkey;
    }
#pragma unroll
    for (int j = 0; j < V; ++j)
      if (grp[j] < 0 || !((keep >> grp[j]) & 1u)) key[j] = 0ull;
  }
  float ssum = 0.f;
  my_w = 0.f;
  my_e = 0;
  for (int k = 0; k < K; ++k) {
    uint64_t b = key[0];
#pragma unroll
    for (int j = 1; j < V; ++j) b = key[j] > b ? key[j] : b;
    b = group_max_key<G>(b);
    float own = -INFINITY;  // the winner's unbiased score, on its owner lane
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const bool hit = key[j] == b;
      own = hit ? sc[j] : own;
      key[j] = hit ? 0ull : key[j];
      cnt[j] += (hit && count) ? 1 : 0;
    }
    const float sk = group_max<G>(own);
    ssum += sk;
    if (g == k) {
      my_w = sk;
      my_e = key_index(b);
    }
  }
  my_w = dsk_weight(my_w, ssum, renorm, scaling, scores_in);
}

}  // namespace moe
