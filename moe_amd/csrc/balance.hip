// Routing consumers: the quantities the training loop derives from each
// MoE layer's router outputs, computed in one pass over the [T, E] router
// probabilities (or scores) per layer instead of the reference's
// topk + one_hot + mean chains and per-metric host reads.
//
//   topk_stats      weighted top-k selection counts, weighted column sums of
//                   the probabilities, and the k-th / (k+1)-th margin
//                   (src/models/load_balancing.py:45-88,
//                    src/utils/routing_stats.py:53-80, :143-191)
//   seq_stats       per-sequence selection counts and mean normalised scores
//                   of the DeepSeek-V3 sequence-wise loss (load_balancing.py:
//                   134-166), and its backward through the normalisation
//   switch_aux_bwd  the Switch loss gradient, a per-expert coefficient times
//                   a per-token weight
//   update_biases   the aux-loss-free expert-bias update of every router in
//                   one launch (train.py:79-139)
//
// Every sum is deterministic: a lane accumulates the experts it owns in
// registers, the waves of a block are combined in wave order, and the block
// partials are reduced in block order (in fp64).  No float atomics.
#include "common.h"
#include "wave_topk.h"

namespace moe {
namespace {

constexpr int kWaves = 4;
constexpr int kTokensPerWave = 8;  // topk_stats: tokens per wave (grid sizing)
constexpr int kSeqChunk = 64;      // seq_stats: tokens per block

__device__ __forceinline__ float load_val(const void* p, int dtype, int64_t i) {
  return dtype == MOE_DTYPE_BF16 ? bf2f(((const bf16*)p)[i]) : ((const float*)p)[i];
}

int stats_blocks(int64_t T) {
  int64_t b = (T + kWaves * kTokensPerWave - 1) / (kWaves * kTokensPerWave);
  if (b > 1024) b = 1024;
  if (b < 1) b = 1;
  return (int)b;
}

// Combines the four waves' per-lane accumulators of one [E] vector in wave
// order and writes the block's partial.  `buf` holds kWaves * 64 floats.
template <int NV>
__device__ void block_combine(const float (&acc)[NV], int E, float* buf, float* out) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    __syncthreads();
    buf[wid * 64 + lane] = acc[j];
    __syncthreads();
    if (wid == 0) {
      float s = buf[lane];
      for (int w = 1; w < kWaves; ++w) s += buf[w * 64 + lane];
      const int e = j * 64 + lane;
      if (e < E) out[e] = s;
    }
  }
}

// The same statistics with G lanes per token (E <= 16*G, K <= G): lane g of
// a group owns experts g*V .. g*V+V-1, ranks through rank_key with G-lane DPP
// butterflies (as the softmax router's group kernel).  The block partial is
// the sum over the block's kWaves*64/G token groups in group order, through
// LDS ([groups][E] floats, dynamic shared memory).
template <int G, int V>
__global__ __launch_bounds__(64 * kWaves) void topk_stats_group_kernel(
    const void* __restrict__ probs, int dtype, const float* __restrict__ tok_w, int64_t T, int E,
    int K, float* __restrict__ part_cnt, float* __restrict__ part_sum,
    double* __restrict__ part_margin) {
  constexpr int TPW = 64 / G, ROWS = kWaves * TPW;
  extern __shared__ float sbuf[];  // [ROWS][E]
  __shared__ double msh[ROWS], mmn[ROWS];
  const int lane = threadIdx.x & 63, g = lane & (G - 1), sub = lane / G;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = wid * TPW + sub, e0 = g * V;
  const bool vec = E == G * V && (dtype == MOE_DTYPE_F32 ? V % 4 == 0 : V % 8 == 0) &&
                   (((uintptr_t)probs & 15) == 0);
  float cnt[V], psum[V];
#pragma unroll
  for (int j = 0; j < V; ++j) cnt[j] = psum[j] = 0.f;
  double msum = 0.0;
  float mmin = INFINITY;
  const int64_t stride = (int64_t)gridDim.x * kWaves * TPW;
  for (int64_t tb = ((int64_t)blockIdx.x * kWaves + wid) * TPW; tb < T; tb += stride) {
    const int64_t t = tb + sub;
    const bool tok = t < T;
    const int64_t tt = tok ? t : T - 1;
    const float w = tok ? (tok_w ? tok_w[t] : 1.f) : 0.f;
    float v[V];
    if (vec) {
      if (dtype == MOE_DTYPE_F32) {
        const f32x4* src = (const f32x4*)((const float*)probs + tt * E + e0);
#pragma unroll
        for (int q = 0; q < V / 4; ++q) {
          const f32x4 a = src[q];
#pragma unroll
          for (int h = 0; h < 4; ++h) v[4 * q + h] = a[h];
        }
      } else {
        const u32x4* src = (const u32x4*)((const bf16*)probs + tt * E + e0);
#pragma unroll
        for (int q = 0; q < (V + 7) / 8; ++q) {
          const u32x4 a = src[q];
#pragma unroll
          for (int h = 0; h < 8; ++h)
            if (8 * q + h < V) v[8 * q + h] = (h & 1) ? bf_hi(a[h >> 1]) : bf_lo(a[h >> 1]);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j)
        v[j] = e0 + j < E ? load_val(probs, dtype, tt * E + e0 + j) : -INFINITY;
    }
    uint64_t key[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      if (tok && e0 + j < E) psum[j] += w * v[j];
      key[j] = e0 + j < E ? rank_key(v[j], e0 + j) : 0ull;
    }
    float vk = 0.f;  // value of the k-th selection
    for (int k = 0; k < K; ++k) {
      uint64_t b = key[0];
#pragma unroll
      for (int j = 1; j < V; ++j) b = key[j] > b ? key[j] : b;
      b = group_max_key<G>(b);
#pragma unroll
      for (int j = 0; j < V; ++j) key[j] = key[j] == b ? 0ull : key[j];
      vk = key_value(b);
    }
    if (tok) {
#pragma unroll
      for (int j = 0; j < V; ++j)
        if (e0 + j < E && key[j] == 0ull) cnt[j] += w;  // selected (real keys are never 0)
    }
    if (K < E) {  // margin between the k-th and (k+1)-th largest value
      uint64_t b = key[0];
#pragma unroll
      for (int j = 1; j < V; ++j) b = key[j] > b ? key[j] : b;
      b = group_max_key<G>(b);
      const float m = vk - key_value(b);
      if (tok) {
        msum += (double)m;
        mmin = fminf(mmin, m);
      }
    }
  }
  // Block partials: rows in group order, per expert.
  auto combine = [&](const float (&acc)[V], float* out) {
    __syncthreads();
#pragma unroll
    for (int j = 0; j < V; ++j)
      if (e0 + j < E) sbuf[row * E + e0 + j] = acc[j];
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      float s = 0.f;
      for (int r = 0; r < ROWS; ++r) s += sbuf[r * E + e];
      out[e] = s;
    }
  };
  combine(cnt, part_cnt + (size_t)blockIdx.x * E);
  combine(psum, part_sum + (size_t)blockIdx.x * E);
  if (g == 0) {
    msh[row] = msum;
    mmn[row] = (double)mmin;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double sm = 0.0, mn = INFINITY;
    for (int r = 0; r < ROWS; ++r) {
      sm += msh[r];
      mn = fmin(mn, mmn[r]);
    }
    part_margin[blockIdx.x * 2] = sm;
    part_margin[blockIdx.x * 2 + 1] = mn;
  }
}

// One wave per token (grid-stride).  Per block: partial weighted selection
// counts [E], weighted probability sums [E], and the margin sum and minimum.
template <int NV>
__global__ __launch_bounds__(64 * kWaves) void topk_stats_kernel(
    const void* __restrict__ probs, int dtype, const float* __restrict__ tok_w, int64_t T, int E,
    int K, float* __restrict__ part_cnt, float* __restrict__ part_sum,
    double* __restrict__ part_margin) {
  __shared__ float buf[kWaves * 64];
  __shared__ double mbuf[kWaves * 2];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float cnt[NV], psum[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) cnt[j] = psum[j] = 0.f;
  double msum = 0.0;
  float mmin = INFINITY;
  const int64_t nwaves = (int64_t)gridDim.x * kWaves;
  for (int64_t t = (int64_t)blockIdx.x * kWaves + wid; t < T; t += nwaves) {
    const float w = tok_w ? tok_w[t] : 1.f;
    float v[NV];
    uint64_t taken = 0;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int e = j * 64 + lane;
      if (e < E) {
        v[j] = load_val(probs, dtype, t * E + e);
        psum[j] += w * v[j];
      } else {
        v[j] = -INFINITY;
        taken |= 1ull << j;
      }
    }
    const uint64_t pad = taken;
    float vk = 0.f;  // value of the k-th selection
    for (int k = 0; k < K; ++k) {
      float bv;
      int be;
      lane_best<NV>(v, taken, lane, bv, be);
      wave_argmax(bv, be);
      vk = bv;
      if ((be & 63) == lane) taken |= 1ull << (be >> 6);
    }
#pragma unroll
    for (int j = 0; j < NV; ++j)
      if (((taken & ~pad) >> j) & 1ull) cnt[j] += w;
    if (K < E) {  // margin between the k-th and (k+1)-th largest value
      float bv;
      int be;
      lane_best<NV>(v, taken, lane, bv, be);
      wave_argmax(bv, be);
      const float m = vk - bv;
      msum += (double)m;
      mmin = fminf(mmin, m);
    }
  }
  block_combine<NV>(cnt, E, buf, part_cnt + (size_t)blockIdx.x * E);
  block_combine<NV>(psum, E, buf, part_sum + (size_t)blockIdx.x * E);
  if (lane == 0) {
    mbuf[wid * 2] = msum;
    mbuf[wid * 2 + 1] = (double)mmin;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double s = 0.0, m = INFINITY;
    for (int w = 0; w < kWaves; ++w) {
      s += mbuf[w * 2];
      m = fmin(m, mbuf[w * 2 + 1]);
    }
    part_margin[blockIdx.x * 2] = s;
    part_margin[blockIdx.x * 2 + 1] = m;
  }
}

// Fixed-order wave reduction of one fp64 value per lane (butterfly).
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// One wave per expert (blocks 0..E-1): lane l sums the partials of blocks l,
// l+64, ... in order, then the lanes are combined by a fixed butterfly.
// Block E reduces the margin partials the same way.
__global__ __launch_bounds__(64) void topk_stats_finalize_kernel(
    const float* __restrict__ part_cnt, const float* __restrict__ part_sum,
    const double* __restrict__ part_margin, int nblk, int E, double* __restrict__ counts,
    double* __restrict__ sums, double* __restrict__ margin) {
  const int lane = threadIdx.x, e = blockIdx.x;
  if (e < E) {
    double c = 0.0, s = 0.0;
    for (int b = lane; b < nblk; b += 64) {
      c += (double)part_cnt[(size_t)b * E + e];
      s += (double)part_sum[(size_t)b * E + e];
    }
    c = wave_sum_f64(c);
    s = wave_sum_f64(s);
    if (lane == 0) {
      counts[e] = c;
      sums[e] = s;
    }
  } else {
    double s = 0.0, m = INFINITY;
    for (int b = lane; b < nblk; b += 64) {
      s += part_margin[b * 2];
      m = fmin(m, part_margin[b * 2 + 1]);
    }
    s = wave_sum_f64(s);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmin(m, __shfl_xor(m, o, 64));
    if (lane == 0) {
      margin[0] = s;
      margin[1] = m;
    }
  }
}

// Block (c, b): tokens [c*kSeqChunk, ...) of sequence b.  Normalised scores
// s' = s / (sum s + 1e-20) per token; per block the selection counts of the
// sequence's experts (the routed indices if given, else the top-k of s') and
// the sums of s'.
// seq_stats with G lanes per token (as topk_stats_group_kernel): block
// (chunk c, sequence b) covers kSeqChunk tokens; the partial is the sum over
// the block's token groups in group order through LDS.
template <int G, int V>
__global__ __launch_bounds__(64 * kWaves) void seq_stats_group_kernel(
    const void* __restrict__ scores, int dtype, const int64_t* __restrict__ selected, int64_t S,
    int E, int K, float* __restrict__ part_cnt, float* __restrict__ part_sum) {
  constexpr int TPW = 64 / G, ROWS = kWaves * TPW;
  extern __shared__ float sbuf[];  // [ROWS][E]
  const int lane = threadIdx.x & 63, g = lane & (G - 1), sub = lane / G;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = wid * TPW + sub, e0 = g * V;
  const int b = blockIdx.y, c = blockIdx.x;
  const bool vec = E == G * V && (dtype == MOE_DTYPE_F32 ? V % 4 == 0 : V % 8 == 0) &&
                   (((uintptr_t)scores & 15) == 0);
  float cnt[V], psum[V];
#pragma unroll
  for (int j = 0; j < V; ++j) cnt[j] = psum[j] = 0.f;
  const int64_t s0 = (int64_t)c * kSeqChunk;
  const int64_t s1 = s0 + kSeqChunk < S ? s0 + kSeqChunk : S;
  for (int64_t sb = s0 + (int64_t)wid * TPW; sb < s1; sb += kWaves * TPW) {
    const int64_t st = sb + sub;
    const bool tok = st < s1;
    const int64_t t = (int64_t)b * S + (tok ? st : s1 - 1);
    float v[V];
    if (vec) {
      if (dtype == MOE_DTYPE_F32) {
        const f32x4* src = (const f32x4*)((const float*)scores + t * E + e0);
#pragma unroll
        for (int q = 0; q < V / 4; ++q) {
          const f32x4 a = src[q];
#pragma unroll
          for (int h = 0; h < 4; ++h) v[4 * q + h] = a[h];
        }
      } else {
        const u32x4* src = (const u32x4*)((const bf16*)scores + t * E + e0);
#pragma unroll
        for (int q = 0; q < (V + 7) / 8; ++q) {
          const u32x4 a = src[q];
#pragma unroll
          for (int h = 0; h < 8; ++h)
            if (8 * q + h < V) v[8 * q + h] = (h & 1) ? bf_hi(a[h >> 1]) : bf_lo(a[h >> 1]);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) v[j] = e0 + j < E ? load_val(scores, dtype, t * E + e0 + j) : 0.f;
    }
    float rs = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) rs += v[j];
    rs = group_sum<G>(rs) + 1e-20f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      v[j] = v[j] / rs;
      if (tok && e0 + j < E) psum[j] += v[j];
    }
    if (selected) {
      for (int k = 0; k < K; ++k) {
        const int64_t ek = selected[t * K + k];
#pragma unroll
        for (int j = 0; j < V; ++j)
          if (tok && ek == e0 + j) cnt[j] += 1.f;
      }
    } else {
      uint64_t key[V];
#pragma unroll
      for (int j = 0; j < V; ++j) key[j] = e0 + j < E ? rank_key(v[j], e0 + j) : 0ull;
      for (int k = 0; k < K; ++k) {
        uint64_t m = key[0];
#pragma unroll
        for (int j = 1; j < V; ++j) m = key[j] > m ? key[j] : m;
        m = group_max_key<G>(m);
#pragma unroll
        for (int j = 0; j < V; ++j) key[j] = key[j] == m ? 0ull : key[j];
      }
      if (tok) {
#pragma unroll
        for (int j = 0; j < V; ++j)
          if (e0 + j < E && key[j] == 0ull) cnt[j] += 1.f;  // selected (real keys are never 0)
      }
    }
  }
  const size_t slot = ((size_t)b * gridDim.x + c) * E;
  auto combine = [&](const float (&acc)[V], float* out) {
    __syncthreads();
#pragma unroll
    for (int j = 0; j < V; ++j)
      if (e0 + j < E) sbuf[row * E + e0 + j] = acc[j];
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      float sm = 0.f;
      for (int r = 0; r < ROWS; ++r) sm += sbuf[r * E + e];
      out[e] = sm;
    }
  };
  combine(cnt, part_cnt + slot);
  combine(psum, part_sum + slot);
}

template <int NV>
__global__ __launch_bounds__(64 * kWaves) void seq_stats_kernel(
    const void* __restrict__ scores, int dtype, const int64_t* __restrict__ selected, int64_t S,
    int E, int K, float* __restrict__ part_cnt, float* __restrict__ part_sum) {
  __shared__ float buf[kWaves * 64];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.y, c = blockIdx.x;
  float cnt[NV], psum[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) cnt[j] = psum[j] = 0.f;
  const int64_t s0 = (int64_t)c * kSeqChunk;
  const int64_t s1 = s0 + kSeqChunk < S ? s0 + kSeqChunk : S;
  for (int64_t st = s0 + wid; st < s1; st += kWaves) {
    const int64_t t = (int64_t)b * S + st;
    float v[NV];
    uint64_t taken = 0;
    float rs = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int e = j * 64 + lane;
      v[j] = e < E ? load_val(scores, dtype, t * E + e) : 0.f;
      rs += v[j];
      if (e >= E) taken |= 1ull << j;
    }
    rs = wave_sum(rs) + 1e-20f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      v[j] = v[j] / rs;
      psum[j] += v[j];
    }
    if (selected) {
      for (int k = 0; k < K; ++k) {
        const int64_t ek = selected[t * K + k];
        if (ek >= 0 && ek < E && (ek & 63) == lane) {
#pragma unroll
          for (int j = 0; j < NV; ++j)
            if ((ek >> 6) == j) cnt[j] += 1.f;
        }
      }
    } else {
      const uint64_t pad = taken;
#pragma unroll
      for (int j = 0; j < NV; ++j)
        if ((pad >> j) & 1ull) v[j] = -INFINITY;
      for (int k = 0; k < K; ++k) {
        float bv;
        int be;
        lane_best<NV>(v, taken, lane, bv, be);
        wave_argmax(bv, be);
        if ((be & 63) == lane) taken |= 1ull << (be >> 6);
      }
#pragma unroll
      for (int j = 0; j < NV; ++j)
        if (((taken & ~pad) >> j) & 1ull) cnt[j] += 1.f;
    }
  }
  const size_t slot = ((size_t)b * gridDim.x + c) * E;
  block_combine<NV>(cnt, E, buf, part_cnt + slot);
  block_combine<NV>(psum, E, buf, part_sum + slot);
}

// One wave per (b, e): counts[b][e] = sum over chunks, mean[b][e] = sum over
// chunks / S, in the fixed order of wave_sum_f64.
__global__ __launch_bounds__(64) void seq_stats_finalize_kernel(
    const float* __restrict__ part_cnt, const float* __restrict__ part_sum, int nchunk, int B,
    int E, int64_t S, double* __restrict__ counts, double* __restrict__ mean) {
  const int lane = threadIdx.x;
  const int64_t i = blockIdx.x;
  const int b = (int)(i / E), e = (int)(i % E);
  double c = 0.0, s = 0.0;
  for (int k = lane; k < nchunk; k += 64) {
    const size_t o = ((size_t)b * nchunk + k) * E + e;
    c += (double)part_cnt[o];
    s += (double)part_sum[o];
  }
  c = wave_sum_f64(c);
  s = wave_sum_f64(s);
  if (lane == 0) {
    counts[i] = c;
    mean[i] = s / (double)S;
  }
}

// d s from d s' through s' = s / (sum s + eps): (g - <g, s'>) / (sum s + eps),
// with g[t][e] = coef[b(t)][e].
template <int NV>
__global__ __launch_bounds__(64 * kWaves) void seq_aux_bwd_kernel(
    const void* __restrict__ scores, int dtype, const double* __restrict__ coef, int64_t T,
    int64_t S, int E, void* __restrict__ d_scores) {
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * kWaves;
  for (int64_t t = (int64_t)blockIdx.x * kWaves + wid; t < T; t += nwaves) {
    const int64_t b = t / S;
    float v[NV], g[NV];
    float rs = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int e = j * 64 + lane;
      v[j] = e < E ? load_val(scores, dtype, t * E + e) : 0.f;
      g[j] = e < E ? (float)coef[b * E + e] : 0.f;
      rs += v[j];
    }
    rs = wave_sum(rs) + 1e-20f;
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) dot += g[j] * (v[j] / rs);
    dot = wave_sum(dot);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int e = j * 64 + lane;
      if (e < E) {
        const float d = (g[j] - dot) / rs;
        if (dtype == MOE_DTYPE_BF16) ((bf16*)d_scores)[t * E + e] = f2bf(d);
        else ((float*)d_scores)[t * E + e] = d;
      }
    }
  }
}

// grad[t][e] = coef[e] * (w ? w[t] : 1).
__global__ __launch_bounds__(256) void switch_aux_bwd_kernel(const double* __restrict__ coef,
                                                             const float* __restrict__ tok_w,
                                                             int64_t T, int E, int dtype,
                                                             void* __restrict__ grad) {
  const int64_t n = T * (int64_t)E;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / E;
    const int e = (int)(i - t * E);
    const float g = (float)coef[e] * (tok_w ? tok_w[t] : 1.f);
    if (dtype == MOE_DTYPE_BF16) ((bf16*)grad)[i] = f2bf(g);
    else ((float*)grad)[i] = g;
  }
}

// One block: every router's bias moves by sign(mean - count) * rate (per
// layer, pooled over layers, or alpha-blended), in fp32 with the reference's
// operation order; counts are then zeroed.  stats = mean, unbiased std, min,
// max of all new biases (fp64).
__global__ __launch_bounds__(1024) void update_biases_kernel(float* const* __restrict__ counts,
                                                             float* const* __restrict__ biases,
                                                             int L, int E, float rate,
                                                             int is_global, float alpha,
                                                             float one_minus_alpha,
                                                             double* __restrict__ stats) {
  extern __shared__ float sh[];  // lmean[L+1] (per layer, then pooled), pool[E]
  __shared__ double red[1024];
  float* lmean = sh;
  float* pool = sh + L + 1;
  const int tid = threadIdx.x;
  // Counts are integers below 2^24, so every fp32 sum below is exact in any
  // order and each mean is one rounding of sum / E, as in the reference.
  for (int e = tid; e < E; e += blockDim.x) {
    float s = 0.f;
    for (int k = 0; k < L; ++k) s += counts[k][e];
    pool[e] = s;
  }
  for (int l = tid; l < L; l += blockDim.x) {
    float s = 0.f;
    for (int e = 0; e < E; ++e) s += counts[l][e];
    lmean[l] = s / (float)E;
  }
  __syncthreads();
  if (tid == 0) {
    float s = 0.f;
    for (int e = 0; e < E; ++e) s += pool[e];
    lmean[L] = s / (float)E;
  }
  __syncthreads();
  auto sgn = [](float x) { return (float)((x > 0.f) - (x < 0.f)); };
  for (int64_t i = tid; i < (int64_t)L * E; i += blockDim.x) {
    const int l = (int)(i / E), e = (int)(i % E);
    const float c = counts[l][e];
    float d;
    if (is_global) {
      const float gd = sgn(lmean[L] - pool[e]) * rate;
      if (alpha > 0.f) {
        const float ld = sgn(lmean[l] - c) * rate;
        d = __fadd_rn(__fmul_rn(alpha, ld), __fmul_rn(one_minus_alpha, gd));
      } else {
        d = gd;
      }
    } else {
      d = sgn(lmean[l] - c) * rate;
    }
    biases[l][e] = __fadd_rn(biases[l][e], d);
  }
  __syncthreads();
  for (int64_t i = tid; i < (int64_t)L * E; i += blockDim.x) counts[i / E][i % E] = 0.f;
  // Statistics of the new biases (fixed-order tree reductions).
  const int64_t n = (int64_t)L * E;
  double s = 0.0, mn = INFINITY, mx = -INFINITY;
  for (int64_t i = tid; i < n; i += blockDim.x) {
    const double v = (double)biases[i / E][i % E];
    s += v;
    mn = fmin(mn, v);
    mx = fmax(mx, v);
  }
  auto tree = [&](double v, int op) {
    red[tid] = v;
    __syncthreads();
    for (int o = blockDim.x / 2; o > 0; o >>= 1) {
      if (tid < o) {
        const double a = red[tid], b2 = red[tid + o];
        red[tid] = op == 0 ? a + b2 : (op == 1 ? fmin(a, b2) : fmax(a, b2));
      }
      __syncthreads();
    }
    const double r = red[0];
    __syncthreads();
    return r;
  };
  const double mean = tree(s, 0) / (double)n;
  mn = tree(mn, 1);
  mx = tree(mx, 2);
  double q = 0.0;
  for (int64_t i = tid; i < n; i += blockDim.x) {
    const double v = (double)biases[i / E][i % E] - mean;
    q += v * v;
  }
  q = tree(q, 0);
  if (tid == 0) {
    stats[0] = mean;
    stats[1] = n > 1 ? sqrt(q / (double)(n - 1)) : 0.0;
    stats[2] = mn;
    stats[3] = mx;
  }
}

#define MOE_DISPATCH_NV_B(E, KERNEL, ...)                        \
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

int check_stats_shape(int64_t T, int E, int K, int dtype, const char* who) {
  MOE_REQUIRE(T >= 0 && E >= 1 && E <= 4096, MOE_ERR_ARG, "%s: T=%lld E=%d out of range", who,
              (long long)T, E);
  MOE_REQUIRE(K >= 1 && K <= E && K <= 64, MOE_ERR_ARG, "%s: K=%d outside [1,min(E,64)]", who, K);
  MOE_REQUIRE(dtype == MOE_DTYPE_F32 || dtype == MOE_DTYPE_BF16, MOE_ERR_DTYPE,
              "%s: dtype %d (fp32 or bf16)", who, dtype);
  return MOE_OK;
}

size_t seq_chunks(int64_t S) { return (size_t)((S + kSeqChunk - 1) / kSeqChunk); }

}  // namespace
}  // namespace moe

using namespace moe;

extern "C" size_t moe_amd_topk_stats_workspace_size(int64_t T, int E) {
  if (T < 0 || E < 1) return 0;
  const size_t nb = (size_t)stats_blocks(T);
  return align_up(nb * (size_t)E * 2 * sizeof(float), 16) + nb * 2 * sizeof(double);
}

extern "C" int moe_amd_topk_stats(const void* probs, int probs_dtype, const float* token_weights,
                                  int64_t T, int E, int K, void* workspace,
                                  size_t workspace_bytes, double* counts, double* prob_sums,
                                  double* margin, void* stream) {
  const char* who = "topk_stats";
  int rc = check_stats_shape(T, E, K, probs_dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(counts && prob_sums && margin && (T == 0 || probs), MOE_ERR_ARG,
              "%s: null pointer", who);
  const size_t need = moe_amd_topk_stats_workspace_size(T, E);
  MOE_REQUIRE(workspace && workspace_bytes >= need, MOE_ERR_WORKSPACE,
              "%s: workspace of %zu bytes needed", who, need);
  MOE_REQUIRE(((uintptr_t)workspace & 15) == 0, MOE_ERR_ALIGN, "%s: workspace alignment", who);
  hipStream_t st = (hipStream_t)stream;
  const int nb = stats_blocks(T);
  float* pc = (float*)workspace;
  float* ps = pc + (size_t)nb * E;
  double* pm = (double*)((char*)workspace + align_up((size_t)nb * E * 2 * sizeof(float), 16));
  if (T == 0) {
    topk_stats_finalize_kernel<<<E + 1, 64, 0, st>>>(pc, ps, pm, 0, E, counts, prob_sums, margin);
    return check_launch(who);
  }
  int G, V;
  group_shape(E, K, G, V);
  if (G) {
    const size_t shm = (size_t)kWaves * (64 / G) * E * sizeof(float);
#define MOE_STATS_GROUP(G_, V_)                                                        \
  topk_stats_group_kernel<G_, V_><<<nb, 64 * kWaves, shm, st>>>(probs, probs_dtype,     \
                                                                token_weights, T, E, K, \
                                                                pc, ps, pm)
    if (G == 8 && V == 4) MOE_STATS_GROUP(8, 4);
    else if (G == 8 && V == 8) MOE_STATS_GROUP(8, 8);
    else if (G == 8) MOE_STATS_GROUP(8, 16);
    else if (V == 4) MOE_STATS_GROUP(16, 4);
    else if (V == 8) MOE_STATS_GROUP(16, 8);
    else MOE_STATS_GROUP(16, 16);
#undef MOE_STATS_GROUP
  } else {
    MOE_DISPATCH_NV_B(E, topk_stats_kernel, nb, 64 * kWaves, 0, st>>>(
        probs, probs_dtype, token_weights, T, E, K, pc, ps, pm));
  }
  topk_stats_finalize_kernel<<<E + 1, 64, 0, st>>>(pc, ps, pm, nb, E, counts, prob_sums, margin);
  return check_launch(who);
}

extern "C" size_t moe_amd_seq_stats_workspace_size(int64_t T, int E, int B) {
  if (T < 0 || E < 1 || B < 1 || T % B) return 0;
  return (size_t)B * seq_chunks(T / B) * (size_t)E * 2 * sizeof(float);
}

extern "C" int moe_amd_seq_stats(const void* scores, int scores_dtype,
                                 const int64_t* selected, int64_t T, int E, int K, int B,
                                 void* workspace, size_t workspace_bytes, double* counts,
                                 double* mean_scores, void* stream) {
  const char* who = "seq_stats";
  int rc = check_stats_shape(T, E, K, scores_dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(B >= 1 && T % B == 0 && T > 0, MOE_ERR_ARG,
              "%s: T=%lld must be a positive multiple of the batch size %d", who, (long long)T,
              B);
  MOE_REQUIRE(scores && counts && mean_scores, MOE_ERR_ARG, "%s: null pointer", who);
  const size_t need = moe_amd_seq_stats_workspace_size(T, E, B);
  MOE_REQUIRE(workspace && workspace_bytes >= need, MOE_ERR_WORKSPACE,
              "%s: workspace of %zu bytes needed", who, need);
  const int64_t S = T / B;
  const int nc = (int)seq_chunks(S);
  MOE_REQUIRE(nc < 65536 && B < 65536 && (int64_t)B * E < ((int64_t)1 << 31), MOE_ERR_UNSUPPORTED,
              "%s: grid too large", who);
  hipStream_t st = (hipStream_t)stream;
  float* pc = (float*)workspace;
  float* ps = pc + (size_t)B * nc * E;
  int G, V;
  group_shape(E, K, G, V);
  if (G) {
    const size_t shm = (size_t)kWaves * (64 / G) * E * sizeof(float);
#define MOE_SEQ_GROUP(G_, V_)                                                                 \
  seq_stats_group_kernel<G_, V_><<<dim3(nc, B), 64 * kWaves, shm, st>>>(scores, scores_dtype, \
                                                                        selected, S, E, K, pc, ps)
    if (G == 8 && V == 4) MOE_SEQ_GROUP(8, 4);
    else if (G == 8 && V == 8) MOE_SEQ_GROUP(8, 8);
    else if (G == 8) MOE_SEQ_GROUP(8, 16);
    else if (V == 4) MOE_SEQ_GROUP(16, 4);
    else if (V == 8) MOE_SEQ_GROUP(16, 8);
    else MOE_SEQ_GROUP(16, 16);
#undef MOE_SEQ_GROUP
  } else {
    MOE_DISPATCH_NV_B(E, seq_stats_kernel, dim3(nc, B), 64 * kWaves, 0, st>>>(
        scores, scores_dtype, selected, S, E, K, pc, ps));
  }
  seq_stats_finalize_kernel<<<(unsigned)((int64_t)B * E), 64, 0, st>>>(pc, ps, nc, B, E, S,
                                                                        counts, mean_scores);
  return check_launch(who);
}

extern "C" int moe_amd_seq_aux_backward(const void* scores, int scores_dtype,
                                        const double* coef, int64_t T, int E, int B,
                                        void* d_scores, void* stream) {
  const char* who = "seq_aux_backward";
  int rc = check_stats_shape(T, E, 1, scores_dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(B >= 1 && T % B == 0, MOE_ERR_ARG, "%s: T must be a multiple of B", who);
  MOE_REQUIRE(T == 0 || (scores && coef && d_scores), MOE_ERR_ARG, "%s: null pointer", who);
  if (T == 0) return MOE_OK;
  const int64_t S = T / B;
  int64_t nb = (T + kWaves * 8 - 1) / (kWaves * 8);
  if (nb > 4096) nb = 4096;
  MOE_DISPATCH_NV_B(E, seq_aux_bwd_kernel, (unsigned)nb, 64 * kWaves, 0,
                    (hipStream_t)stream>>>(scores, scores_dtype, coef, T, S, E, d_scores));
  return check_launch(who);
}

extern "C" int moe_amd_switch_aux_backward(const double* coef, const float* token_weights,
                                           int64_t T, int E, int grad_dtype, void* grad,
                                           void* stream) {
  const char* who = "switch_aux_backward";
  MOE_REQUIRE(T >= 0 && E >= 1, MOE_ERR_ARG, "%s: bad sizes", who);
  MOE_REQUIRE(grad_dtype == MOE_DTYPE_F32 || grad_dtype == MOE_DTYPE_BF16, MOE_ERR_DTYPE,
              "%s: dtype %d", who, grad_dtype);
  MOE_REQUIRE(T == 0 || (coef && grad), MOE_ERR_ARG, "%s: null pointer", who);
  if (T == 0) return MOE_OK;
  int64_t nb = (T * (int64_t)E + 255) / 256;
  if (nb > 8192) nb = 8192;
  switch_aux_bwd_kernel<<<(unsigned)nb, 256, 0, (hipStream_t)stream>>>(coef, token_weights, T, E,
                                                                      grad_dtype, grad);
  return check_launch(who);
}

extern "C" int moe_amd_update_expert_biases(float* const* counts, float* const* biases, int L,
                                            int E, float update_rate, int is_global,
                                            double alpha, double* stats, void* stream) {
  const char* who = "update_expert_biases";
  MOE_REQUIRE(L >= 1 && E >= 1 && (int64_t)L * E < ((int64_t)1 << 30), MOE_ERR_ARG,
              "%s: L=%d E=%d", who, L, E);
  MOE_REQUIRE(counts && biases && stats, MOE_ERR_ARG, "%s: null pointer", who);
  const size_t shm = (size_t)(L + 1 + E) * sizeof(float);
  MOE_REQUIRE(shm <= 56 * 1024, MOE_ERR_ARG, "%s: L + E too large", who);
  update_biases_kernel<<<1, 1024, shm, (hipStream_t)stream>>>(
      counts, biases, L, E, update_rate, is_global, (float)alpha, (float)(1.0 - alpha), stats);
  return check_launch(who);
}
