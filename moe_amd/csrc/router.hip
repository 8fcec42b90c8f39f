// Router kernels: softmax top-k (Qwen3MoeTopKRouter) and sigmoid + expert
// bias top-k (DeepSeekRouter), forward and backward.
//
// One wave64 owns one token at a time.  The token's E scores live in
// registers, NV = ceil(E/64) per lane (expert e = j*64 + lane), and the
// top-K is extracted with K rounds of a wave-wide arg-max over
// (value, -expert id), so equal values resolve to the lower expert id.
// Reference: src/models/modeling_qwen3_moe.py:266-275,
//            src/models/router.py:22-70 and :103-155.
#include "common.h"
#include "router_group.h"
#include "wave_topk.h"

#include <cmath>

namespace moe {
namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kMaxExperts = 4096;  // NV <= 64

__device__ __forceinline__ float load_logit(const void* p, int dtype, int64_t i) {
  return dtype == MOE_DTYPE_BF16 ? bf2f(((const bf16*)p)[i]) : ((const float*)p)[i];
}

template <int NV>
__global__ __launch_bounds__(64 * kWavesPerBlock) void softmax_topk_kernel(
    const void* __restrict__ logits, int logits_dtype, const float* __restrict__ offset,
    int64_t T, int E, int K, int renorm, float* __restrict__ probs, float* __restrict__ topk_w,
    int64_t* __restrict__ topk_idx, float* __restrict__ tpe) {
  // One token per wave (grid_wave), entry j*64 + lane in slot j of a lane.
  // Registers per lane: the values (two passes: max, then exp/sum/store)
  // and then only their rank keys; the winners' probs are recomputed from
  // their keys (key_value returns the value exactly, -0 as +0, which gives
  // the same exp), bit-identical to the stored row.
  extern __shared__ int hist[];  // [E] when tpe != nullptr
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // token index stays scalar
  if (tpe) {
    for (int e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
    __syncthreads();
  }
  const int64_t nwaves = (int64_t)gridDim.x * kWavesPerBlock;
  for (int64_t t = (int64_t)blockIdx.x * kWavesPerBlock + wid; t < T; t += nwaves) {
    float v[NV];
    bool nan_here = false;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int e = j * 64 + lane;
      v[j] = e < E ? load_logit(logits, logits_dtype, t * E + e) + (offset ? offset[e] : 0.0f)
                   : -INFINITY;
      nan_here |= v[j] != v[j];
    }
    // A NaN logit makes every prob of the row NaN, and the reference ranks
    // the probs: the row's entries then all tie and rank by index.
    if (__ballot(nan_here)) {
#pragma unroll
      for (int j = 0; j < NV; ++j)
        if (j * 64 + lane < E) v[j] = __builtin_nanf("");
    }
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NV; ++j) m = fmaxf(m, v[j]);
    m = wave_max(m);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) s += (j * 64 + lane < E) ? expf(v[j] - m) : 0.f;
    s = wave_sum(s);
    uint64_t key[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int e = j * 64 + lane;
      if (e < E) probs[t * E + e] = expf(v[j] - m) / s;
      key[j] = e < E ? rank_key(v[j], e) : 0ull;
    }
    // Softmax is monotone, so ranking the (offset) logits ranks the probs;
    // equal logits give bit-equal probs and resolve to the lower expert id.
    uint64_t kk;
    const int ek = wave_topk_keys<NV>(key, lane, K, kk);
    float wk = lane < K ? expf(key_value(kk) - m) / s : 0.f;
    if (renorm) {
      // Sum in rank order on every lane (K <= 64 values read one by one).
      float ssum = 0.f;
      for (int k = 0; k < K; ++k)
        ssum += __builtin_bit_cast(float,
                                   __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk), k));
      wk = wk / ssum;
    }
    if (lane < K) {
      topk_w[t * K + lane] = wk;
      topk_idx[t * K + lane] = ek;
      if (tpe && ek >= 0 && ek < E) atomicAdd(&hist[ek], 1);
    }
    __builtin_amdgcn_wave_barrier();
  }
  if (tpe) {
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x)
      if (hist[e]) atomicAdd(&tpe[e], (float)hist[e]);
  }
}

// DeepSeek router with G lanes per token, as softmax_topk_group_kernel:
// scores = sigmoid(logits) stored, then the selection core shared with the
// fused gating linear (router_group.h: group scores and kept groups when
// ngroups > 0, each group on one lane; rank keys of the biased scores, the
// winner's unbiased score taken from its owner lane, weights renormalised by
// their sum in rank order (+1e-20), scaled), cast.  VEC: E == G*V, fp32 rows
// moved as 16-byte vectors.
template <int G, int V, bool VEC>
__global__ __launch_bounds__(64 * kWavesPerBlock) void sigmoid_topk_group_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int64_t T, int E, int K,
    int renorm, float scaling, int ngroups, int gtopk, float* __restrict__ scores,
    void* __restrict__ topk_w, int w_dtype, int64_t* __restrict__ topk_idx,
    float* __restrict__ tpe, int scores_in) {
  extern __shared__ int hist[];  // [E] when tpe != nullptr
  constexpr int TPW = 64 / G;
  const int lane = threadIdx.x & 63, g = lane & (G - 1), sub = lane / G;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (tpe) {
    for (int e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
    __syncthreads();
  }
  const int e0 = g * V;
  // each entry's expert group (ngroups > 0), fixed per lane
  int grp[V], cnt[V];
  const int eg = ngroups > 0 ? E / ngroups : 1;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    grp[j] = e0 + j < E ? (e0 + j) / eg : -1;
    cnt[j] = 0;
  }
  const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock * TPW;
  for (int64_t tb = ((int64_t)blockIdx.x * kWavesPerBlock + wid) * TPW; tb < T; tb += stride) {
    const int64_t t = tb + sub;
    const bool tok = t < T;
    const int64_t tt = tok ? t : T - 1;
    float sc[V];
    if constexpr (VEC) {
      const f32x4* src = (const f32x4*)(logits + tt * E + e0);
#pragma unroll
      for (int q = 0; q < V / 4; ++q) {
        const f32x4 a = src[q];
#pragma unroll
        for (int h = 0; h < 4; ++h) sc[4 * q + h] = dsk_score(a[h], scores_in);
      }
      if (tok && scores) {
        f32x4* dst = (f32x4*)(scores + t * E + e0);
#pragma unroll
        for (int q = 0; q < V / 4; ++q)
          dst[q] = f32x4{sc[4 * q], sc[4 * q + 1], sc[4 * q + 2], sc[4 * q + 3]};
      }
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int e = e0 + j;
        sc[j] = e < E ? dsk_score(logits[tt * E + e], scores_in) : 0.f;
        if (tok && e < E && scores) scores[t * E + e] = sc[j];
      }
    }
    uint64_t key[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int e = e0 + j;
      key[j] = e < E ? rank_key(sc[j] + (bias ? bias[e] : 0.0f), e) : 0ull;
    }
    float my_w;
    int my_e;
    group_sigmoid_topk<G, V>(sc, key, grp, g, K, ngroups, gtopk, renorm, scaling, scores_in,
                             false, cnt, my_w, my_e);
    if (tok && g < K) {
      if (w_dtype == MOE_DTYPE_BF16)
        ((bf16*)topk_w)[t * K + g] = f2bf(my_w);
      else
        ((float*)topk_w)[t * K + g] = my_w;
      topk_idx[t * K + g] = my_e;
      if (tpe) atomicAdd(&hist[my_e], 1);
    }
  }
  if (tpe) {
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x)
      if (hist[e]) atomicAdd(&tpe[e], (float)hist[e]);
  }
}

// The same softmax router for E <= 16*G experts and K <= G: G lanes per
// token (64/G tokens per wave), V consecutive experts per lane, ranks through
// rank_key with G-lane DPP butterflies.  Per token this takes about a fifth
// of the VALU instructions of the wave-per-token kernel, which at E = 128 is
// VALU-bound (64-lane reductions repeated K times for 2 values per lane).
// probs = exp(v - max) * (1 / sum) with the sum over the group in a fixed
// butterfly order; the selected weights are those probs (recomputed
// bit-identically from the winning key), renormalised by their group sum.
// The gating linear's fused epilogue (gemm.hip) runs the same core
// (router_group.h) and writes the same bits.
template <int G, int V, bool KEY16, bool VEC>
__global__ __launch_bounds__(64 * kWavesPerBlock) void softmax_topk_group_kernel(
    const void* __restrict__ logits, int logits_dtype, const float* __restrict__ offset,
    int64_t T, int E, int K, int renorm, float* __restrict__ probs, float* __restrict__ topk_w,
    int64_t* __restrict__ topk_idx, float* __restrict__ tpe) {
  // KEY16: bf16 logits without offset, ranked by 32-bit keys from the bf16
  // bits; otherwise 64-bit keys from the fp32 values.  VEC: E == G*V (every
  // lane owns V real experts), so a lane's logits and probs move as 16-byte
  // vectors (a token's row is contiguous across its G lanes).
  using Key = std::conditional_t<KEY16, uint32_t, uint64_t>;
  extern __shared__ int hist[];  // [E] when tpe != nullptr
  constexpr int TPW = 64 / G;    // tokens per wave
  const int lane = threadIdx.x & 63, g = lane & (G - 1), sub = lane / G;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (tpe) {
    for (int e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
    __syncthreads();
  }
  const int e0 = g * V;
  const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock * TPW;
  for (int64_t tb = ((int64_t)blockIdx.x * kWavesPerBlock + wid) * TPW; tb < T; tb += stride) {
    const int64_t t = tb + sub;
    const bool tok = t < T;
    float v[V];
    Key key[V];
    if constexpr (VEC && KEY16) {
      static_assert(V % 8 == 0, "16-byte bf16 vectors");
      const u32x4* src = (const u32x4*)((const uint16_t*)logits + (tok ? t : 0) * E + e0);
#pragma unroll
      for (int q = 0; q < V / 8; ++q) {
        const u32x4 w = tok ? src[q] : u32x4{0xff80ff80u, 0xff80ff80u, 0xff80ff80u, 0xff80ff80u};
#pragma unroll
        for (int h = 0; h < 8; ++h) {
          const uint32_t bits = (w[h >> 1] >> (16 * (h & 1))) & 0xffffu;
          v[q * 8 + h] = __uint_as_float(bits << 16);
          key[q * 8 + h] = rank_key16(bits, e0 + q * 8 + h);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int e = e0 + j;
        const bool in = tok && e < E;
        if constexpr (KEY16) {
          const uint32_t bits = in ? (uint32_t)((const uint16_t*)logits)[t * E + e] : 0xff80u;
          v[j] = __uint_as_float(bits << 16);  // -inf outside the row
          key[j] = e < E ? rank_key16(bits, e) : 0u;
        } else {
          v[j] = in ? load_logit(logits, logits_dtype, t * E + e) + (offset ? offset[e] : 0.f)
                    : -INFINITY;
          key[j] = e < E ? rank_key(v[j], e) : 0ull;
        }
      }
    }
    float m, s, p[V];
    group_softmax<G, V>(v, key, e0, E, p, m, s);
    const float rs = 1.f / s;
    if constexpr (VEC) {
      if (tok) {
        f32x4* dst = (f32x4*)(probs + t * E + e0);
#pragma unroll
        for (int q = 0; q < V / 4; ++q)
          dst[q] = f32x4{p[4 * q] * rs, p[4 * q + 1] * rs, p[4 * q + 2] * rs, p[4 * q + 3] * rs};
      }
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int e = e0 + j;
        if (tok && e < E) probs[t * E + e] = p[j] * rs;
      }
    }
    float my_w;
    int my_e;
    group_topk<G, V>(key, m, rs, g, K, renorm, my_w, my_e);
    if (tok && g < K) {
      topk_w[t * K + g] = my_w;
      topk_idx[t * K + g] = my_e;
      if (tpe) atomicAdd(&hist[my_e], 1);
    }
  }
  if (tpe) {
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x)
      if (hist[e]) atomicAdd(&tpe[e], (float)hist[e]);
  }
}

// The group kernel's variants: 32-bit keys for bf16 logits without offset,
// 16-byte vectors when the experts fill the G lanes exactly.
template <int G, int V>
void launch_softmax_group(bool key16, int grid, size_t shm, hipStream_t st, const void* logits,
                          int dtype, const float* offset, int64_t T, int E, int K, int renorm,
                          float* probs, float* w, int64_t* idx, float* tpe) {
#define MOE_GROUP_LAUNCH(K16, VEC)                                                         \
  softmax_topk_group_kernel<G, V, K16, VEC><<<grid, 64 * kWavesPerBlock, shm, st>>>(        \
      logits, dtype, offset, T, E, K, renorm, probs, w, idx, tpe)
  if constexpr (V % 8 == 0) {
    if (E == G * V && al16(logits) && al16(probs)) {
      if (key16) MOE_GROUP_LAUNCH(true, true);
      else MOE_GROUP_LAUNCH(false, true);
      return;
    }
  }
  if (key16) MOE_GROUP_LAUNCH(true, false);
  else MOE_GROUP_LAUNCH(false, false);
#undef MOE_GROUP_LAUNCH
}

int grid_group(int64_t T, int G) {
  const int64_t per_block = (int64_t)kWavesPerBlock * (64 / G) * 2;  // two token batches per wave
  int64_t blocks = (T + per_block - 1) / per_block;
  if (blocks > 8192) blocks = 8192;
  return (int)(blocks < 1 ? 1 : blocks);
}

template <int NV, bool GROUPS>
__global__ __launch_bounds__(64 * kWavesPerBlock) void sigmoid_topk_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int64_t T, int E, int K,
    int renorm, float scaling, int num_groups, int group_topk, float* __restrict__ scores,
    void* __restrict__ topk_w, int w_dtype, int64_t* __restrict__ topk_idx,
    float* __restrict__ tpe, int scores_in) {
  extern __shared__ int hist[];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // token index stays scalar
  if (tpe) {
    for (int e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
    __syncthreads();
  }
  const int64_t nwaves = (int64_t)gridDim.x * kWavesPerBlock;
  // One token per wave (grid_wave), entry j*64 + lane in slot j of a lane.
  // The flat selection keeps only the entries' rank keys in registers; the
  // winners' unbiased scores are recomputed from their logits (the same
  // function of the same input: bit-identical to the stored scores).
  for (int64_t t = (int64_t)blockIdx.x * kWavesPerBlock + wid; t < T; t += nwaves) {
    int ek;
    if constexpr (!GROUPS) {
      uint64_t key[NV];
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int e = j * 64 + lane;
        if (e < E) {
          const float sc = dsk_score(logits[t * E + e], scores_in);
          if (scores) scores[t * E + e] = sc;
          key[j] = rank_key(sc + (bias ? bias[e] : 0.0f), e);
        } else {
          key[j] = 0ull;
        }
      }
      uint64_t kk;
      ek = wave_topk_keys<NV>(key, lane, K, kk);
    } else {
      float b[NV];
      uint64_t taken = 0;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        int e = j * 64 + lane;
        if (e < E) {
          const float sc = dsk_score(logits[t * E + e], scores_in);
          if (scores) scores[t * E + e] = sc;
          b[j] = sc + (bias ? bias[e] : 0.0f);
        } else {
          b[j] = -INFINITY;
          taken |= 1ull << j;
        }
      }
      // Group-limited selection (router.py:22-70): score each group by the
      // sum of its top (K / group_topk) biased scores, keep group_topk groups.
      const int eg = E / num_groups, per = K / group_topk;
      float gv = -INFINITY;  // lane g holds group g's score
      for (int g = 0; g < num_groups; ++g) {
        uint64_t gtaken = taken;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
          int e = j * 64 + lane;
          if (e / eg != g) gtaken |= 1ull << j;
        }
        float acc = 0.f;
        for (int q = 0; q < per; ++q) {
          float bv;
          int be;
          lane_best<NV>(b, gtaken, lane, bv, be);
          wave_argmax(bv, be);
          acc += bv;
          if ((be & 63) == lane) gtaken |= 1ull << (be >> 6);
        }
        if (lane == g) gv = acc;
      }
      // Pick group_topk groups (higher score first, lower group id on ties).
      int gi = lane < num_groups ? lane : 0x7fffffff;
      uint64_t keep = 0;
      bool gone = lane >= num_groups;
      for (int q = 0; q < group_topk; ++q) {
        float bv = gone ? -INFINITY : gv;
        int be = gone ? 0x7fffffff : gi;
        wave_argmax(bv, be);
        keep |= 1ull << be;
        if (be == lane) gone = true;
      }
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        int e = j * 64 + lane;
        if (e < E && !((keep >> (e / eg)) & 1ull)) taken |= 1ull << j;
      }
      ek = wave_topk<NV>(b, taken, lane, K);
    }
    float wk = lane < K ? dsk_score(logits[t * E + ek], scores_in) : 0.f;
    float ssum = 0.f;
    if (renorm)
      for (int k = 0; k < K; ++k)
        ssum += __builtin_bit_cast(float,
                                   __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk), k));
    wk = dsk_weight(wk, ssum, renorm, scaling, scores_in);
    if (lane < K) {
      if (w_dtype == MOE_DTYPE_BF16)
        ((bf16*)topk_w)[t * K + lane] = f2bf(wk);
      else
        ((float*)topk_w)[t * K + lane] = wk;
      topk_idx[t * K + lane] = ek;
      if (tpe && ek >= 0 && ek < E) atomicAdd(&hist[ek], 1);
    }
    __builtin_amdgcn_wave_barrier();
  }
  if (tpe) {
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x)
      if (hist[e]) atomicAdd(&tpe[e], (float)hist[e]);
  }
}

// DeepSeek router (flat top-k) for large E: one workgroup of four waves per
// token.  Wave w ranks the entries e = j*256 + w*64 + lane (j < SL): their
// sigmoid scores are stored, their rank keys (biased score, index) kept in
// registers, and the wave's K best keys (wave_topk_keys) go to LDS; wave 0
// then ranks the 4K candidates (one per lane) the same way.  The order is
// the rank order of every other router kernel, so the selection is the same
// as the one-wave kernel's; the winners' unbiased scores are recomputed from
// their logits (bit-identical to the stored scores), renormalised by their
// sum in rank order (+1e-20), scaled, cast.  K <= 16.
template <int SL>
__global__ __launch_bounds__(256) void sigmoid_topk_split_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int64_t T, int E, int K,
    int renorm, float scaling, float* __restrict__ scores, void* __restrict__ topk_w,
    int w_dtype, int64_t* __restrict__ topk_idx, float* __restrict__ tpe, int scores_in) {
  __shared__ uint64_t cand[4 * 16];
  extern __shared__ int hist[];  // [E] when tpe != nullptr
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (tpe) {
    for (int e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
  }
  for (int64_t t = blockIdx.x; t < T; t += gridDim.x) {
    const float* lrow = logits + t * E;
    float* srow = scores + t * E;
    uint64_t key[SL];
#pragma unroll
    for (int j = 0; j < SL; ++j) {
      const int e = j * 256 + wid * 64 + lane;
      key[j] = 0ull;
      if (e < E) {
        const float sc = dsk_score(lrow[e], scores_in);
        if (scores) srow[e] = sc;
        key[j] = rank_key(sc + (bias ? bias[e] : 0.0f), e);
      }
    }
    uint64_t mine;
    wave_topk_keys<SL>(key, lane, K, mine);
    __syncthreads();  // the previous token's candidates have been read
    if (lane < K) cand[wid * K + lane] = mine;
    __syncthreads();
    if (wid == 0) {
      uint64_t c[1] = {lane < 4 * K ? cand[lane] : 0ull};
      uint64_t kk;
      const int ek = wave_topk_keys<1>(c, lane, K, kk);
      float wk = lane < K ? dsk_score(lrow[ek], scores_in) : 0.f;
      float ssum = 0.f;
      if (renorm)
        for (int k = 0; k < K; ++k)
          ssum += __builtin_bit_cast(float,
                                     __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk), k));
      wk = dsk_weight(wk, ssum, renorm, scaling, scores_in);
      if (lane < K) {
        if (w_dtype == MOE_DTYPE_BF16)
          ((bf16*)topk_w)[t * K + lane] = f2bf(wk);
        else
          ((float*)topk_w)[t * K + lane] = wk;
        topk_idx[t * K + lane] = ek;
        if (tpe) atomicAdd(&hist[ek], 1);
      }
    }
  }
  if (tpe) {
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x)
      if (hist[e]) atomicAdd(&tpe[e], (float)hist[e]);
  }
}

// d(renormalised weights) -> d(gathered values): w_k = v_k / (S + eps).
// Every lane k < K holds (v_k, g_k); returns dv_k.
__device__ __forceinline__ float renorm_backward(float vk, float gk, int K, float eps) {
  float ssum = 0.f, gv = 0.f;
  const float gvk = gk * vk;
  for (int k = 0; k < K; ++k) {  // k is uniform: lane reads, not shuffles
    ssum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, vk), k));
    gv += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gvk), k));
  }
  float den = ssum + eps;
  return gk / den - gv / (den * den);
}

// The softmax router's backward for E == G*V (V a multiple of 8) and K <= G:
// G lanes per token as in the forward group kernel, rows moved as 16-byte
// vectors, the K routed (expert, gradient) pairs broadcast from the group's
// lanes k < K in rank order (same sums as renorm_backward).
template <int G, int V>
__global__ __launch_bounds__(64 * kWavesPerBlock) void softmax_topk_bwd_group_kernel(
    const float* __restrict__ probs, const int64_t* __restrict__ idx,
    const float* __restrict__ dw, const float* __restrict__ dprobs, int64_t T, int E, int K,
    int renorm, void* __restrict__ dlogits, int dl_dtype) {
  static_assert(V % 8 == 0, "16-byte vectors");
  constexpr int TPW = 64 / G;
  const int lane = threadIdx.x & 63, g = lane & (G - 1), base = lane - g, sub = lane / G;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int e0 = g * V;
  const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock * TPW;
  for (int64_t tb = ((int64_t)blockIdx.x * kWavesPerBlock + wid) * TPW; tb < T; tb += stride) {
    const int64_t t = tb + sub;
    const bool tok = t < T;
    const int64_t tt = tok ? t : T - 1;  // rows past T load a valid row and store nothing
    const int ek = g < K ? (int)idx[tt * K + g] : 0;
    const float gk = g < K ? dw[tt * K + g] : 0.f;
    const float vk = g < K ? probs[tt * E + ek] : 0.f;
    float dv = gk;
    if (renorm) {
      float ssum = 0.f, gv = 0.f;
      for (int k = 0; k < K; ++k) {
        ssum += __shfl(vk, base + k, 64);
        gv += __shfl(gk * vk, base + k, 64);
      }
      dv = gk / ssum - gv / (ssum * ssum);
    }
    float p[V], dp[V];
    const f32x4* prow = (const f32x4*)(probs + tt * E + e0);
#pragma unroll
    for (int q = 0; q < V / 4; ++q) {
      const f32x4 a = prow[q];
      const f32x4 d = dprobs ? ((const f32x4*)(dprobs + tt * E + e0))[q] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        p[4 * q + h] = a[h];
        dp[4 * q + h] = d[h];
      }
    }
    for (int k = 0; k < K; ++k) {
      const int e = __shfl(ek, base + k, 64);
      const float gg = __shfl(dv, base + k, 64);
#pragma unroll
      for (int j = 0; j < V; ++j)
        if (e == e0 + j) dp[j] += gg;
    }
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) dot += p[j] * dp[j];
    dot = group_sum<G>(dot);
    if (!tok) continue;
    if (dl_dtype == MOE_DTYPE_BF16) {
      u32x4* out = (u32x4*)((bf16*)dlogits + t * E + e0);
#pragma unroll
      for (int q = 0; q < V / 8; ++q) {
        u32x4 w;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const int j = 8 * q + 2 * h;
          w[h] = pack_bf2((dp[j] - dot) * p[j], (dp[j + 1] - dot) * p[j + 1]);
        }
        out[q] = w;
      }
    } else {
      f32x4* out = (f32x4*)((float*)dlogits + t * E + e0);
#pragma unroll
      for (int q = 0; q < V / 4; ++q)
        out[q] = f32x4{(dp[4 * q] - dot) * p[4 * q], (dp[4 * q + 1] - dot) * p[4 * q + 1],
                       (dp[4 * q + 2] - dot) * p[4 * q + 2], (dp[4 * q + 3] - dot) * p[4 * q + 3]};
    }
  }
}

template <int NV>
__global__ __launch_bounds__(64 * kWavesPerBlock) void softmax_topk_bwd_kernel(
    const float* __restrict__ probs, const int64_t* __restrict__ idx,
    const float* __restrict__ dw, const float* __restrict__ dprobs, int64_t T, int E, int K,
    int renorm, void* __restrict__ dlogits, int dl_dtype) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t nwaves = (int64_t)gridDim.x * kWavesPerBlock;
  for (int64_t t = (int64_t)blockIdx.x * kWavesPerBlock + wid; t < T; t += nwaves) {
    int ek = lane < K ? (int)idx[t * K + lane] : -1;
    float vk = lane < K ? probs[t * E + ek] : 0.f;
    float gk = lane < K ? dw[t * K + lane] : 0.f;
    float dv = renorm ? renorm_backward(vk, gk, K, 0.f) : gk;
    float p[NV], dp[NV];
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      int e = j * 64 + lane;
      p[j] = e < E ? probs[t * E + e] : 0.f;
      dp[j] = (e < E && dprobs) ? dprobs[t * E + e] : 0.f;
    }
    for (int k = 0; k < K; ++k) {
      int e = __shfl(ek, k, 64);
      float g = __shfl(dv, k, 64);
#pragma unroll
      for (int j = 0; j < NV; ++j)
        if (e == j * 64 + lane) dp[j] += g;
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) dot += p[j] * dp[j];
    dot = wave_sum(dot);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      int e = j * 64 + lane;
      if (e < E) {
        float g = (dp[j] - dot) * p[j];
        if (dl_dtype == MOE_DTYPE_BF16)
          ((bf16*)dlogits)[t * E + e] = f2bf(g);
        else
          ((float*)dlogits)[t * E + e] = g;
      }
    }
  }
}

// The DeepSeek router's backward with G lanes per token (E == G*V, V a
// multiple of 4, K <= G): rows as 16-byte vectors, the routed (expert,
// gradient) pairs broadcast from the group's lanes k < K in rank order.
template <int G, int V>
__global__ __launch_bounds__(64 * kWavesPerBlock) void sigmoid_topk_bwd_group_kernel(
    const float* __restrict__ scores, const int64_t* __restrict__ idx,
    const void* __restrict__ dw, int w_dtype, const float* __restrict__ dscores, int64_t T,
    int E, int K, int renorm, float scaling, float* __restrict__ dlogits) {
  static_assert(V % 4 == 0, "16-byte vectors");
  constexpr int TPW = 64 / G;
  const int lane = threadIdx.x & 63, g = lane & (G - 1), base = lane - g, sub = lane / G;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int e0 = g * V;
  const int64_t stride = (int64_t)gridDim.x * kWavesPerBlock * TPW;
  for (int64_t tb = ((int64_t)blockIdx.x * kWavesPerBlock + wid) * TPW; tb < T; tb += stride) {
    const int64_t t = tb + sub;
    const bool tok = t < T;
    const int64_t tt = tok ? t : T - 1;
    const int ek = g < K ? (int)idx[tt * K + g] : 0;
    const float vk = g < K ? scores[tt * E + ek] : 0.f;
    float gk = 0.f;
    if (g < K)
      gk = w_dtype == MOE_DTYPE_BF16 ? bf2f(((const bf16*)dw)[tt * K + g])
                                     : ((const float*)dw)[tt * K + g];
    if (scaling > 0.f) gk *= scaling;
    float dv = gk;
    if (renorm) {
      float ssum = 0.f, gv = 0.f;
      for (int k = 0; k < K; ++k) {
        ssum += __shfl(vk, base + k, 64);
        gv += __shfl(gk * vk, base + k, 64);
      }
      const float den = ssum + 1e-20f;
      dv = gk / den - gv / (den * den);
    }
    float y[V], ds[V];
    const f32x4* yrow = (const f32x4*)(scores + tt * E + e0);
#pragma unroll
    for (int q = 0; q < V / 4; ++q) {
      const f32x4 a = yrow[q];
      const f32x4 d = dscores ? ((const f32x4*)(dscores + tt * E + e0))[q] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        y[4 * q + h] = a[h];
        ds[4 * q + h] = d[h];
      }
    }
    for (int k = 0; k < K; ++k) {
      const int e = __shfl(ek, base + k, 64);
      const float gg = __shfl(dv, base + k, 64);
#pragma unroll
      for (int j = 0; j < V; ++j)
        if (e == e0 + j) ds[j] += gg;
    }
    if (!tok) continue;
    f32x4* out = (f32x4*)(dlogits + t * E + e0);
#pragma unroll
    for (int q = 0; q < V / 4; ++q)
      out[q] = f32x4{ds[4 * q] * (1.f - y[4 * q]) * y[4 * q],
                     ds[4 * q + 1] * (1.f - y[4 * q + 1]) * y[4 * q + 1],
                     ds[4 * q + 2] * (1.f - y[4 * q + 2]) * y[4 * q + 2],
                     ds[4 * q + 3] * (1.f - y[4 * q + 3]) * y[4 * q + 3]};
  }
}

template <int NV>
__global__ __launch_bounds__(64 * kWavesPerBlock) void sigmoid_topk_bwd_kernel(
    const float* __restrict__ scores, const int64_t* __restrict__ idx,
    const void* __restrict__ dw, int w_dtype, const float* __restrict__ dscores, int64_t T,
    int E, int K, int renorm, float scaling, float* __restrict__ dlogits) {
  // Per wave, an E-float LDS row that stays zero between tokens: the K routed
  // gradients are written at their experts, read back by every entry's owner
  // lane (one LDS read per entry instead of K compares), and cleared again.
  extern __shared__ float routed[];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  float* const row = routed + wid * E;
  for (int e = lane; e < E; e += 64) row[e] = 0.f;
  __builtin_amdgcn_wave_barrier();
  const int64_t nwaves = (int64_t)gridDim.x * kWavesPerBlock;
  for (int64_t t = (int64_t)blockIdx.x * kWavesPerBlock + wid; t < T; t += nwaves) {
    // The row's scores are loaded first, so that their latency overlaps
    // the dependent id -> routed-score loads.
    float y[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int e = j * 64 + lane;
      y[j] = e < E ? scores[t * E + e] : 0.f;
    }
    int ek = lane < K ? (int)idx[t * K + lane] : -1;
    float vk = lane < K ? scores[t * E + ek] : 0.f;
    float gk = 0.f;
    if (lane < K)
      gk = w_dtype == MOE_DTYPE_BF16 ? bf2f(((const bf16*)dw)[t * K + lane])
                                     : ((const float*)dw)[t * K + lane];
    if (scaling > 0.f) gk *= scaling;
    float dv = renorm ? renorm_backward(vk, gk, K, 1e-20f) : gk;
    const bool routed_ok = lane < K && ek >= 0 && ek < E;  // top-k ids are distinct
    if (routed_ok) row[ek] = dv;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      int e = j * 64 + lane;
      if (e < E) {
        const float ds = dscores ? dscores[t * E + e] : 0.f;
        dlogits[t * E + e] = (ds + row[e]) * (1.f - y[j]) * y[j];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (routed_ok) row[ek] = 0.f;
  }
}

int grid_for(int64_t T) {
  int64_t waves = T;
  int64_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  return (int)blocks;
}

// Wave-per-token kernels: one token per wave up to 32768 waves (their
// rounds are latency-bound chains, so occupancy is what hides them).
int grid_wave(int64_t T) {
  int64_t blocks = (T + kWavesPerBlock - 1) / kWavesPerBlock;
  if (blocks > 8192) blocks = 8192;
  if (blocks < 1) blocks = 1;
  return (int)blocks;
}

#define MOE_DISPATCH_NV(E, KERNEL, ...)                          \
  do {                                                           \
    int nv_ = ((E) + 63) / 64;                                   \
    if (nv_ <= 1) KERNEL<1><<<__VA_ARGS__;                       \
    else if (nv_ <= 2) KERNEL<2><<<__VA_ARGS__;                  \
    else if (nv_ <= 4) KERNEL<4><<<__VA_ARGS__;                  \
    else if (nv_ <= 8) KERNEL<8><<<__VA_ARGS__;                  \
    else if (nv_ <= 16) KERNEL<16><<<__VA_ARGS__;                \
    else if (nv_ <= 32) KERNEL<32><<<__VA_ARGS__;                \
    else KERNEL<64><<<__VA_ARGS__;                               \
  } while (0)

#define MOE_DISPATCH_NV_G(E, G, KERNEL, ...)                     \
  do {                                                           \
    int nv_ = ((E) + 63) / 64;                                   \
    if (nv_ <= 1) KERNEL<1, G><<<__VA_ARGS__;                    \
    else if (nv_ <= 2) KERNEL<2, G><<<__VA_ARGS__;               \
    else if (nv_ <= 4) KERNEL<4, G><<<__VA_ARGS__;               \
    else if (nv_ <= 8) KERNEL<8, G><<<__VA_ARGS__;               \
    else if (nv_ <= 16) KERNEL<16, G><<<__VA_ARGS__;             \
    else if (nv_ <= 32) KERNEL<32, G><<<__VA_ARGS__;             \
    else KERNEL<64, G><<<__VA_ARGS__;                            \
  } while (0)

int check_router_shape(int64_t T, int E, int K) {
  MOE_REQUIRE(T >= 0, MOE_ERR_ARG, "router: T=%lld must be >= 0", (long long)T);
  MOE_REQUIRE(E >= 1 && E <= kMaxExperts, MOE_ERR_ARG, "router: E=%d outside [1,%d]", E,
              kMaxExperts);
  MOE_REQUIRE(K >= 1 && K <= E && K <= 64, MOE_ERR_ARG, "router: K=%d outside [1,min(E,64)]",
              K);
  return MOE_OK;
}

}  // namespace
}  // namespace moe

using namespace moe;

extern "C" int moe_amd_router_softmax_topk(const void* logits, int logits_dtype,
                                           const float* logit_offset, int64_t T, int E, int K,
                                           int renormalize, float* probs, float* topk_weights,
                                           int64_t* topk_index, float* tokens_per_expert,
                                           void* stream) {
  int rc = check_router_shape(T, E, K);
  if (rc) return rc;
  MOE_REQUIRE(logits_dtype == MOE_DTYPE_F32 || logits_dtype == MOE_DTYPE_BF16, MOE_ERR_DTYPE,
              "router_softmax_topk: logits dtype %d", logits_dtype);
  MOE_REQUIRE(T == 0 || (logits && probs && topk_weights && topk_index), MOE_ERR_ARG,
              "router_softmax_topk: null pointer");
  if (T == 0) return MOE_OK;
  size_t shm = tokens_per_expert ? (size_t)E * sizeof(int) : 0;
  int G, V;
  group_shape(E, K, G, V);
  hipStream_t st = (hipStream_t)stream;
#define MOE_SOFTMAX_GROUP(G_, V_)                                                     \
  launch_softmax_group<G_, V_>(key16, grid_group(T, G_), shm, st, logits, logits_dtype, \
                               logit_offset, T, E, K, renormalize, probs, topk_weights,  \
                               topk_index, tokens_per_expert)
  const bool key16 = logits_dtype == MOE_DTYPE_BF16 && !logit_offset;
  if (G == 8 && V == 4) MOE_SOFTMAX_GROUP(8, 4);
  else if (G == 8 && V == 8) MOE_SOFTMAX_GROUP(8, 8);
  else if (G == 8) MOE_SOFTMAX_GROUP(8, 16);
  else if (G == 16 && V == 4) MOE_SOFTMAX_GROUP(16, 4);
  else if (G == 16 && V == 8) MOE_SOFTMAX_GROUP(16, 8);
  else if (G == 16) MOE_SOFTMAX_GROUP(16, 16);
  else
    MOE_DISPATCH_NV(E, softmax_topk_kernel, grid_wave(T), 64 * kWavesPerBlock, shm,
                    st >>>(logits, logits_dtype, logit_offset, T, E, K, renormalize, probs,
                           topk_weights, topk_index, tokens_per_expert));
#undef MOE_SOFTMAX_GROUP
  return check_launch("router_softmax_topk");
}

extern "C" int moe_amd_router_softmax_topk_backward(const float* probs, const int64_t* topk_index,
                                                    const float* d_topk_weights,
                                                    const float* d_probs, int64_t T, int E,
                                                    int K, int renormalize, void* d_logits,
                                                    int d_logits_dtype, void* stream) {
  int rc = check_router_shape(T, E, K);
  if (rc) return rc;
  MOE_REQUIRE(d_logits_dtype == MOE_DTYPE_F32 || d_logits_dtype == MOE_DTYPE_BF16,
              MOE_ERR_DTYPE, "router_softmax_topk_backward: dtype %d", d_logits_dtype);
  MOE_REQUIRE(T == 0 || (probs && topk_index && d_topk_weights && d_logits), MOE_ERR_ARG,
              "router_softmax_topk_backward: null pointer");
  if (T == 0) return MOE_OK;
  int G, V;
  group_shape(E, K, G, V);
  if (G && E == G * V && V % 8 == 0 && al16(probs) && al16(d_probs) && al16(d_logits)) {
    hipStream_t st = (hipStream_t)stream;
#define MOE_BWD_GROUP(G_, V_)                                                               \
  softmax_topk_bwd_group_kernel<G_, V_><<<grid_group(T, G_), 64 * kWavesPerBlock, 0, st>>>( \
      probs, topk_index, d_topk_weights, d_probs, T, E, K, renormalize, d_logits, d_logits_dtype)
    if (G == 8 && V == 8) MOE_BWD_GROUP(8, 8);
    else if (G == 8) MOE_BWD_GROUP(8, 16);
    else if (V == 8) MOE_BWD_GROUP(16, 8);
    else MOE_BWD_GROUP(16, 16);
#undef MOE_BWD_GROUP
    return check_launch("router_softmax_topk_backward");
  }
  MOE_DISPATCH_NV(E, softmax_topk_bwd_kernel, grid_for(T), 64 * kWavesPerBlock, 0,
                  (hipStream_t)stream >>>(probs, topk_index, d_topk_weights, d_probs, T, E, K,
                                          renormalize, d_logits, d_logits_dtype));
  return check_launch("router_softmax_topk_backward");
}

namespace {
// Both DeepSeek router entry points: from logits (scores = sigmoid, stored)
// or, with scores_in, from given scores (logits holds them; scores is null).
int sigmoid_topk_run(const float* logits, const float* expert_bias, int64_t T, int E, int K,
                     int renormalize, float scaling_factor, int num_groups, int group_topk,
                     float* scores, void* topk_weights, int weights_dtype, int64_t* topk_index,
                     float* tokens_per_expert, void* stream, int scores_in) {
  int rc = check_router_shape(T, E, K);
  if (rc) return rc;
  MOE_REQUIRE(weights_dtype == MOE_DTYPE_F32 || weights_dtype == MOE_DTYPE_BF16, MOE_ERR_DTYPE,
              "router_sigmoid_topk: weights dtype %d", weights_dtype);
  MOE_REQUIRE(T == 0 || (logits && (scores || scores_in) && topk_weights && topk_index),
              MOE_ERR_ARG, "router_sigmoid_topk: null pointer");
  if (num_groups > 0) {
    MOE_REQUIRE(num_groups <= 64 && E % num_groups == 0 && group_topk >= 1 &&
                    group_topk <= num_groups && K % group_topk == 0 &&
                    (E / num_groups) * group_topk >= K,
                MOE_ERR_ARG,
                "router_sigmoid_topk: bad grouping (E=%d K=%d groups=%d group_topk=%d)", E, K,
                num_groups, group_topk);
  }
  if (T == 0) return MOE_OK;
  if (!(scaling_factor > 0.f)) scaling_factor = 0.f;
  size_t shm = tokens_per_expert ? (size_t)E * sizeof(int) : 0;
  int G, V;
  group_shape(E, K, G, V);
  // G lanes per token: flat top-k, or expert groups that each fit one lane's
  // group score (num_groups <= G)
  if (G && (num_groups <= 0 || num_groups <= G)) {
    hipStream_t st = (hipStream_t)stream;
    const bool vec = E == G * V && al16(logits) && al16(scores);
    const int ng = num_groups > 0 ? num_groups : 0, gk = num_groups > 0 ? group_topk : 0;
#define MOE_SIGMOID_GROUP(G_, V_, VEC_)                                                       \
  sigmoid_topk_group_kernel<G_, V_, VEC_><<<grid_group(T, G_), 64 * kWavesPerBlock, shm, st>>>( \
      logits, expert_bias, T, E, K, renormalize, scaling_factor, ng, gk, scores, topk_weights, \
      weights_dtype, topk_index, tokens_per_expert, scores_in)
#define MOE_SIGMOID_GROUP_V(G_, V_)            \
  do {                                          \
    if (vec) MOE_SIGMOID_GROUP(G_, V_, true);   \
    else MOE_SIGMOID_GROUP(G_, V_, false);      \
  } while (0)
    if (G == 8 && V == 4) MOE_SIGMOID_GROUP_V(8, 4);
    else if (G == 8 && V == 8) MOE_SIGMOID_GROUP_V(8, 8);
    else if (G == 8) MOE_SIGMOID_GROUP_V(8, 16);
    else if (V == 4) MOE_SIGMOID_GROUP_V(16, 4);
    else if (V == 8) MOE_SIGMOID_GROUP_V(16, 8);
    else MOE_SIGMOID_GROUP_V(16, 16);
#undef MOE_SIGMOID_GROUP_V
#undef MOE_SIGMOID_GROUP
    return check_launch("router_sigmoid_topk");
  }
  if (num_groups <= 0 && E > 256 && K <= 16) {
    hipStream_t st = (hipStream_t)stream;
    const int64_t blocks = T < 32768 ? T : 32768;
#define MOE_SIGMOID_SPLIT(SL_)                                                                \
  sigmoid_topk_split_kernel<SL_><<<(int)blocks, 256, shm, st>>>(                              \
      logits, expert_bias, T, E, K, renormalize, scaling_factor, scores, topk_weights,        \
      weights_dtype, topk_index, tokens_per_expert, scores_in)
    const int sl = (E + 255) / 256;
    if (sl <= 2) MOE_SIGMOID_SPLIT(2);
    else if (sl <= 4) MOE_SIGMOID_SPLIT(4);
    else if (sl <= 7) MOE_SIGMOID_SPLIT(7);
    else if (sl <= 8) MOE_SIGMOID_SPLIT(8);
    else MOE_SIGMOID_SPLIT(16);
#undef MOE_SIGMOID_SPLIT
    return check_launch("router_sigmoid_topk");
  }
  if (num_groups > 0) {
    MOE_DISPATCH_NV_G(E, true, sigmoid_topk_kernel, grid_wave(T), 64 * kWavesPerBlock, shm,
                      (hipStream_t)stream >>>(logits, expert_bias, T, E, K, renormalize,
                                              scaling_factor, num_groups, group_topk, scores,
                                              topk_weights, weights_dtype, topk_index,
                                              tokens_per_expert, scores_in));
  } else {
    MOE_DISPATCH_NV_G(E, false, sigmoid_topk_kernel, grid_wave(T), 64 * kWavesPerBlock, shm,
                      (hipStream_t)stream >>>(logits, expert_bias, T, E, K, renormalize,
                                              scaling_factor, num_groups, group_topk, scores,
                                              topk_weights, weights_dtype, topk_index,
                                              tokens_per_expert, scores_in));
  }
  return check_launch("router_sigmoid_topk");
}
}  // namespace

extern "C" int moe_amd_router_sigmoid_topk(const float* logits, const float* expert_bias,
                                           int64_t T, int E, int K, int renormalize,
                                           float scaling_factor, int num_groups, int group_topk,
                                           float* scores, void* topk_weights, int weights_dtype,
                                           int64_t* topk_index, float* tokens_per_expert,
                                           void* stream) {
  return sigmoid_topk_run(logits, expert_bias, T, E, K, renormalize, scaling_factor, num_groups,
                          group_topk, scores, topk_weights, weights_dtype, topk_index,
                          tokens_per_expert, stream, 0);
}

extern "C" int moe_amd_router_sigmoid_topk_scores(const float* scores, const float* expert_bias,
                                                  int64_t T, int E, int K, int renormalize,
                                                  float scaling_factor, int num_groups,
                                                  int group_topk, void* topk_weights,
                                                  int weights_dtype, int64_t* topk_index,
                                                  float* tokens_per_expert, void* stream) {
  return sigmoid_topk_run(scores, expert_bias, T, E, K, renormalize, scaling_factor, num_groups,
                          group_topk, nullptr, topk_weights, weights_dtype, topk_index,
                          tokens_per_expert, stream, 1);
}

extern "C" int moe_amd_router_sigmoid_topk_backward(const float* scores,
                                                    const int64_t* topk_index,
                                                    const void* d_topk_weights,
                                                    int weights_dtype, const float* d_scores,
                                                    int64_t T, int E, int K, int renormalize,
                                                    float scaling_factor, float* d_logits,
                                                    void* stream) {
  int rc = check_router_shape(T, E, K);
  if (rc) return rc;
  MOE_REQUIRE(weights_dtype == MOE_DTYPE_F32 || weights_dtype == MOE_DTYPE_BF16, MOE_ERR_DTYPE,
              "router_sigmoid_topk_backward: weights dtype %d", weights_dtype);
  MOE_REQUIRE(T == 0 || (scores && topk_index && d_topk_weights && d_logits), MOE_ERR_ARG,
              "router_sigmoid_topk_backward: null pointer");
  if (T == 0) return MOE_OK;
  if (!(scaling_factor > 0.f)) scaling_factor = 0.f;
  int G, V;
  group_shape(E, K, G, V);
  if (G && E == G * V && V % 4 == 0 && al16(scores) && al16(d_scores) && al16(d_logits)) {
    hipStream_t st = (hipStream_t)stream;
#define MOE_SIGMOID_BWD_GROUP(G_, V_)                                                           \
  sigmoid_topk_bwd_group_kernel<G_, V_><<<grid_group(T, G_), 64 * kWavesPerBlock, 0, st>>>(     \
      scores, topk_index, d_topk_weights, weights_dtype, d_scores, T, E, K, renormalize,        \
      scaling_factor, d_logits)
    if (G == 8 && V == 4) MOE_SIGMOID_BWD_GROUP(8, 4);
    else if (G == 8 && V == 8) MOE_SIGMOID_BWD_GROUP(8, 8);
    else if (G == 8) MOE_SIGMOID_BWD_GROUP(8, 16);
    else if (V == 4) MOE_SIGMOID_BWD_GROUP(16, 4);
    else if (V == 8) MOE_SIGMOID_BWD_GROUP(16, 8);
    else MOE_SIGMOID_BWD_GROUP(16, 16);
#undef MOE_SIGMOID_BWD_GROUP
    return check_launch("router_sigmoid_topk_backward");
  }
  MOE_DISPATCH_NV(E, sigmoid_topk_bwd_kernel, grid_for(T), 64 * kWavesPerBlock,
                  (size_t)kWavesPerBlock * E * sizeof(float),
                  (hipStream_t)stream >>>(scores, topk_index, d_topk_weights, weights_dtype,
                                          d_scores, T, E, K, renormalize, scaling_factor,
                                          d_logits));
  return check_launch("router_sigmoid_topk_backward");
}
