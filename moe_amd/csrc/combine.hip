// Weighted combine (unpermute + sum over K) and the two gather-shaped
// backward kernels of the expert layer.  All three are HBM-bound row
// gathers: one wave per token, each lane moving 16 bytes per step, so every
// routed row is read as full contiguous 128-byte lines.
// Reference: transformers/integrations/moe.py:461-478 (forward combine) and
// :393-395 (the hidden_states[perm // K] gather whose backward is dX).
#include "common.h"

namespace moe {
namespace {

constexpr int kWaves = 4;
constexpr int kChunks = 1;  // 64*N-element row chunks whose loads are issued together

template <typename T> struct Vec;
// Loads and stores are non-temporal: every routed row is read once and every
// output row written once, so they bypass the caches' retention (measured:
// a streaming read reaches 7.0 TB/s this way against 6.3 TB/s with plain
// loads).  load_raw keeps the 16 bytes packed (4 VGPRs) until they are
// consumed, so more rows can be in flight per lane.
template <> struct Vec<bf16> {
  static constexpr int N = 8;  // elements per 16-byte lane access
  typedef u32x4 Raw;
  __device__ static Raw load_raw(const bf16* p) { return __builtin_nontemporal_load((const u32x4*)p); }
  __device__ static float get(const Raw& r, int i) { return (i & 1) ? bf_hi(r[i >> 1]) : bf_lo(r[i >> 1]); }
  __device__ static void load(const bf16* p, float (&v)[8]) {
    u32x4 w = __builtin_nontemporal_load((const u32x4*)p);
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[2 * i] = bf_lo(w[i]); v[2 * i + 1] = bf_hi(w[i]); }
  }
  __device__ static void store(bf16* p, const float (&v)[8]) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack_bf2(v[2 * i], v[2 * i + 1]);
    __builtin_nontemporal_store(w, (u32x4*)p);
  }
  __device__ static float round(float v) { return round_bf(v); }
};
template <> struct Vec<float> {
  static constexpr int N = 4;
  typedef f32x4 Raw;
  __device__ static Raw load_raw(const float* p) { return __builtin_nontemporal_load((const f32x4*)p); }
  __device__ static float get(const Raw& r, int i) { return r[i]; }
  __device__ static void load(const float* p, float (&v)[4]) {
    f32x4 w = __builtin_nontemporal_load((const f32x4*)p);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = w[i];
  }
  __device__ static void store(float* p, const float (&v)[4]) {
    f32x4 w = {v[0], v[1], v[2], v[3]};
    __builtin_nontemporal_store(w, (f32x4*)p);
  }
  __device__ static float round(float v) { return v; }
};

__device__ __forceinline__ float load_w(const void* w, int wdt, int64_t i) {
  return wdt == MOE_DTYPE_BF16 ? bf2f(((const bf16*)w)[i]) : ((const float*)w)[i];
}

// The K routed rows of token t (slot and weight), read once by lanes 0..K-1
// and made wave-uniform, so that all K row loads of a step can be issued
// before any of them is consumed.
template <int KM>
__device__ __forceinline__ void token_rows(const int* __restrict__ slot, const void* __restrict__ w,
                                           int wdt, int64_t t, int lane, int (&s)[KM],
                                           float (&wk)[KM]) {
  const int my_s = lane < KM ? slot[t * KM + lane] : 0;
  const float my_w = (w && lane < KM) ? load_w(w, wdt, t * KM + lane) : 0.f;
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    s[k] = __builtin_amdgcn_readlane(my_s, k);
    wk[k] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_w), k));
  }
}

// KM > 0: the top-k is KM (all loads of a row chunk in flight at once);
// KM == 0: any K, rows loaded one after the other.
template <typename T, int KM>
__global__ __launch_bounds__(64 * kWaves) void combine_kernel(
    const T* __restrict__ y, const int* __restrict__ slot, const int* __restrict__ offsets,
    const void* __restrict__ w, int wdt, int64_t ntok, int K, int E, int H, T* __restrict__ out) {
  constexpr int N = Vec<T>::N;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nvalid = offsets[E];
  const int64_t nw = (int64_t)gridDim.x * kWaves;
  for (int64_t t = (int64_t)blockIdx.x * kWaves + wid; t < ntok; t += nw) {
    if constexpr (KM > 0) {
      int sk[KM];
      float wk[KM];
      token_rows<KM>(slot, w, wdt, t, lane, sk, wk);
      const bool rp = wdt == MOE_DTYPE_BF16 && sizeof(T) == 2;
      for (int h0 = lane * N; h0 < H; h0 += 64 * N * kChunks) {
        typename Vec<T>::Raw v[kChunks][KM];
#pragma unroll
        for (int c = 0; c < kChunks; ++c)
#pragma unroll
          for (int k = 0; k < KM; ++k)
            if (sk[k] < nvalid && h0 + c * 64 * N < H)
              v[c][k] = Vec<T>::load_raw(y + (int64_t)sk[k] * H + h0 + c * 64 * N);
#pragma unroll
        for (int c = 0; c < kChunks; ++c) {
          if (h0 + c * 64 * N >= H) break;
          float acc[N];
#pragma unroll
          for (int i = 0; i < N; ++i) acc[i] = 0.f;
#pragma unroll
          for (int k = 0; k < KM; ++k) {
            if (sk[k] >= nvalid) continue;  // sentinel: masked to zero in the reference
#pragma unroll
            for (int i = 0; i < N; ++i) {
              float prod = Vec<T>::get(v[c][k], i) * wk[k];
              if (rp) prod = round_bf(prod);
              acc[i] += prod;
            }
          }
          Vec<T>::store(out + t * H + h0 + c * 64 * N, acc);
        }
      }
    } else {
      for (int h0 = lane * N; h0 < H; h0 += 64 * N) {
        float acc[N];
#pragma unroll
        for (int i = 0; i < N; ++i) acc[i] = 0.f;
        for (int k = 0; k < K; ++k) {
          const int s = slot[t * K + k];
          if (s >= nvalid) continue;  // sentinel: masked to zero in the reference
          const float wk = load_w(w, wdt, t * K + k);
          float v[N];
          Vec<T>::load(y + (int64_t)s * H + h0, v);
#pragma unroll
          for (int i = 0; i < N; ++i) {
            float prod = v[i] * wk;
            if (wdt == MOE_DTYPE_BF16 && sizeof(T) == 2) prod = round_bf(prod);
            acc[i] += prod;
          }
        }
        Vec<T>::store(out + t * H + h0, acc);
      }
    }
  }
}

template <typename T, int KM>
__global__ __launch_bounds__(64 * kWaves) void combine_bwd_kernel(
    const T* __restrict__ dout, const T* __restrict__ y, const int* __restrict__ slot,
    const int* __restrict__ offsets, const void* __restrict__ w, int wdt, int64_t ntok, int K,
    int E, int H, T* __restrict__ dy, void* __restrict__ dw) {
  constexpr int N = Vec<T>::N;
  const bool round_prod = (wdt == MOE_DTYPE_BF16 && sizeof(T) == 2);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nvalid = offsets[E];
  const int64_t nw = (int64_t)gridDim.x * kWaves;
  for (int64_t t = (int64_t)blockIdx.x * kWaves + wid; t < ntok; t += nw) {
    if constexpr (KM > 0) {
      // dout's chunk once, the KM routed rows' chunks in flight together; the
      // dot products accumulate per lane in chunk order, as below.
      int sk[KM];
      float wk[KM], dot[KM];
      token_rows<KM>(slot, w, wdt, t, lane, sk, wk);
#pragma unroll
      for (int k = 0; k < KM; ++k) dot[k] = 0.f;
      for (int h0 = lane * N; h0 < H; h0 += 64 * N) {
        float g[N], v[KM][N];
        Vec<T>::load(dout + t * H + h0, g);
#pragma unroll
        for (int k = 0; k < KM; ++k)
          if (sk[k] < nvalid) Vec<T>::load(y + (int64_t)sk[k] * H + h0, v[k]);
#pragma unroll
        for (int k = 0; k < KM; ++k) {
          if (sk[k] >= nvalid) continue;
          float d[N];
#pragma unroll
          for (int i = 0; i < N; ++i) {
            d[i] = g[i] * wk[k];
            float pr = g[i] * v[k][i];
            dot[k] += round_prod ? round_bf(pr) : pr;
          }
          Vec<T>::store(dy + (int64_t)sk[k] * H + h0, d);
        }
      }
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        const float dk = wave_sum(dot[k]);
        if (lane == 0) {
          if (wdt == MOE_DTYPE_BF16)
            ((bf16*)dw)[t * KM + k] = f2bf(dk);
          else
            ((float*)dw)[t * KM + k] = dk;
        }
      }
      continue;
    }
    for (int k = 0; k < K; ++k) {
      const int s = slot[t * K + k];
      const bool valid = s < nvalid;
      const float wk = load_w(w, wdt, t * K + k);
      float dot = 0.f;
      if (valid) {
        for (int h0 = lane * N; h0 < H; h0 += 64 * N) {
          float g[N], v[N], d[N];
          Vec<T>::load(dout + t * H + h0, g);
          Vec<T>::load(y + (int64_t)s * H + h0, v);
#pragma unroll
          for (int i = 0; i < N; ++i) {
            d[i] = g[i] * wk;
            float pr = g[i] * v[i];
            dot += round_prod ? round_bf(pr) : pr;
          }
          Vec<T>::store(dy + (int64_t)s * H + h0, d);
        }
      }
      dot = wave_sum(dot);
      if (lane == 0) {
        if (wdt == MOE_DTYPE_BF16)
          ((bf16*)dw)[t * K + k] = f2bf(dot);
        else
          ((float*)dw)[t * K + k] = dot;
      }
    }
  }
}

template <typename T, int KM>
__global__ __launch_bounds__(64 * kWaves) void gather_bwd_kernel(
    const T* __restrict__ dxs, const int* __restrict__ slot, const int* __restrict__ offsets,
    const T* __restrict__ addend, int64_t ntok, int K, int E, int H, T* __restrict__ dx) {
  constexpr int N = Vec<T>::N;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nvalid = offsets[E];
  const int64_t nw = (int64_t)gridDim.x * kWaves;
  for (int64_t t = (int64_t)blockIdx.x * kWaves + wid; t < ntok; t += nw) {
    int sk[KM > 0 ? KM : 1];
    float wk[KM > 0 ? KM : 1];
    if constexpr (KM > 0) token_rows<KM>(slot, nullptr, 0, t, lane, sk, wk);
    if constexpr (KM > 0) {
      for (int h0 = lane * N; h0 < H; h0 += 64 * N * kChunks) {
        typename Vec<T>::Raw v[kChunks][KM], a[kChunks];
#pragma unroll
        for (int c = 0; c < kChunks; ++c) {
          if (h0 + c * 64 * N >= H) break;
#pragma unroll
          for (int k = 0; k < KM; ++k)
            if (sk[k] < nvalid) v[c][k] = Vec<T>::load_raw(dxs + (int64_t)sk[k] * H + h0 + c * 64 * N);
          if (addend) a[c] = Vec<T>::load_raw(addend + t * H + h0 + c * 64 * N);
        }
#pragma unroll
        for (int c = 0; c < kChunks; ++c) {
          if (h0 + c * 64 * N >= H) break;
          float acc[N];
#pragma unroll
          for (int i = 0; i < N; ++i) acc[i] = 0.f;
#pragma unroll
          for (int k = 0; k < KM; ++k) {
            if (sk[k] >= nvalid) continue;
#pragma unroll
            for (int i = 0; i < N; ++i) acc[i] += Vec<T>::get(v[c][k], i);
          }
          if (addend) {
            // a second gradient of the same tensor: round the sum to T first,
            // as autograd's accumulation of two T-typed gradients does
#pragma unroll
            for (int i = 0; i < N; ++i) acc[i] = Vec<T>::round(acc[i]) + Vec<T>::get(a[c], i);
          }
          Vec<T>::store(dx + t * H + h0 + c * 64 * N, acc);
        }
      }
      continue;
    }
    for (int h0 = lane * N; h0 < H; h0 += 64 * N) {
      float acc[N];
#pragma unroll
      for (int i = 0; i < N; ++i) acc[i] = 0.f;
      {
        for (int k = 0; k < K; ++k) {
          const int s = slot[t * K + k];
          if (s >= nvalid) continue;
          float v[N];
          Vec<T>::load(dxs + (int64_t)s * H + h0, v);
#pragma unroll
          for (int i = 0; i < N; ++i) acc[i] += v[i];
        }
      }
      if (addend) {
        // a second gradient of the same tensor: round the sum to T first, as
        // autograd's accumulation of two T-typed gradients does
        float a[N];
        Vec<T>::load(addend + t * H + h0, a);
#pragma unroll
        for (int i = 0; i < N; ++i) acc[i] = Vec<T>::round(acc[i]) + a[i];
      }
      Vec<T>::store(dx + t * H + h0, acc);
    }
  }
}

int grid_tokens(int64_t ntok) {
  int64_t b = (ntok + kWaves - 1) / kWaves;
  if (b > 32768) b = 32768;
  return (int)(b < 1 ? 1 : b);
}

int check_rows(int64_t T, int K, int E, int H, int dtype, const char* who) {
  MOE_REQUIRE(dtype == MOE_DTYPE_BF16 || dtype == MOE_DTYPE_F32, MOE_ERR_DTYPE, "%s: dtype %d",
              who, dtype);
  MOE_REQUIRE(T >= 0 && K >= 1 && E >= 1 && H >= 1, MOE_ERR_ARG, "%s: bad sizes", who);
  const int n = dtype == MOE_DTYPE_BF16 ? 8 : 4;
  MOE_REQUIRE(H % n == 0, MOE_ERR_ARG, "%s: H=%d must be a multiple of %d", who, H, n);
  return MOE_OK;
}


// Launches KERNEL<T, KM> with KM = K for the common top-k values, else the
// any-K form (KM = 0).
#define MOE_DISPATCH_K(K, KERNEL, T, ...)                       \
  do {                                                          \
    switch (K) {                                                \
      case 1: KERNEL<T, 1><<<__VA_ARGS__; break;                \
      case 2: KERNEL<T, 2><<<__VA_ARGS__; break;                \
      case 4: KERNEL<T, 4><<<__VA_ARGS__; break;                \
      case 6: KERNEL<T, 6><<<__VA_ARGS__; break;                \
      case 8: KERNEL<T, 8><<<__VA_ARGS__; break;                \
      default: KERNEL<T, 0><<<__VA_ARGS__; break;               \
    }                                                           \
  } while (0)

// d_w[i] = sum over c < n_part of partials[i * n_part + c] (fp32, in c
// order), rounded once to the weights' dtype; 0 for sentinel entries (slot
// past the real experts' rows), which no GEMM tile covers.
__global__ __launch_bounds__(256) void weight_grad_reduce_kernel(
    const float* __restrict__ part, int n_part, const int* __restrict__ slot,
    const int* __restrict__ offsets, int E, int64_t n, void* __restrict__ out, int out_bf16) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float acc = 0.f;
  if (slot[i] < offsets[E]) {
    const float* pp = part + i * n_part;
    for (int c = 0; c < n_part; ++c) acc += pp[c];
  }
  if (out_bf16)
    ((bf16*)out)[i] = f2bf(acc);
  else
    ((float*)out)[i] = acc;
}

}  // namespace
}  // namespace moe

using namespace moe;

extern "C" int moe_amd_combine(const void* y, const int32_t* slot, const int32_t* offsets,
                               const void* topk_weights, int weights_dtype, int64_t T, int K,
                               int E, int H, int dtype, void* out, void* stream) {
  const char* who = "combine";
  int rc = check_rows(T, K, E, H, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(weights_dtype == MOE_DTYPE_BF16 || weights_dtype == MOE_DTYPE_F32, MOE_ERR_DTYPE,
              "%s: weights dtype %d", who, weights_dtype);
  MOE_REQUIRE(offsets && (T == 0 || (out && y && slot && topk_weights)), MOE_ERR_ARG,
              "%s: null pointer", who);
  MOE_REQUIRE(al16(out) && (T == 0 || al16(y)), MOE_ERR_ALIGN, "%s: misaligned pointer", who);
  if (T == 0) return MOE_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MOE_DTYPE_BF16)
    MOE_DISPATCH_K(K, combine_kernel, bf16, grid_tokens(T), 64 * kWaves, 0, st>>>(
        (const bf16*)y, slot, offsets, topk_weights, weights_dtype, T, K, E, H, (bf16*)out));
  else
    MOE_DISPATCH_K(K, combine_kernel, float, grid_tokens(T), 64 * kWaves, 0, st>>>(
        (const float*)y, slot, offsets, topk_weights, weights_dtype, T, K, E, H, (float*)out));
  return check_launch(who);
}

extern "C" int moe_amd_combine_backward(const void* d_out, const void* y, const int32_t* slot,
                                        const int32_t* offsets, const void* topk_weights,
                                        int weights_dtype, int64_t T, int K, int E, int H,
                                        int dtype, void* d_y, void* d_topk_weights,
                                        void* stream) {
  const char* who = "combine_backward";
  int rc = check_rows(T, K, E, H, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(weights_dtype == MOE_DTYPE_BF16 || weights_dtype == MOE_DTYPE_F32, MOE_ERR_DTYPE,
              "%s: weights dtype %d", who, weights_dtype);
  MOE_REQUIRE(offsets && (T == 0 || (d_out && y && slot && topk_weights && d_y && d_topk_weights)),
              MOE_ERR_ARG, "%s: null pointer", who);
  MOE_REQUIRE(T == 0 || (al16(d_out) && al16(y) && al16(d_y)), MOE_ERR_ALIGN,
              "%s: misaligned pointer", who);
  if (T == 0) return MOE_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MOE_DTYPE_BF16)
    MOE_DISPATCH_K(K, combine_bwd_kernel, bf16, grid_tokens(T), 64 * kWaves, 0, st>>>(
        (const bf16*)d_out, (const bf16*)y, slot, offsets, topk_weights, weights_dtype, T, K, E,
        H, (bf16*)d_y, d_topk_weights));
  else
    MOE_DISPATCH_K(K, combine_bwd_kernel, float, grid_tokens(T), 64 * kWaves, 0, st>>>(
        (const float*)d_out, (const float*)y, slot, offsets, topk_weights, weights_dtype, T, K,
        E, H, (float*)d_y, d_topk_weights));
  return check_launch(who);
}

int gather_backward_impl(const void* d_xs, const int32_t* slot, const int32_t* offsets,
                         const void* addend, int64_t T, int K, int E, int H, int dtype, void* d_x,
                         void* stream, const char* who) {
  int rc = check_rows(T, K, E, H, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(offsets && (T == 0 || (d_x && d_xs && slot)), MOE_ERR_ARG, "%s: null pointer",
              who);
  MOE_REQUIRE(al16(d_x) && (T == 0 || al16(d_xs)) && (!addend || al16(addend)), MOE_ERR_ALIGN,
              "%s: misaligned pointer", who);
  if (T == 0) return MOE_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MOE_DTYPE_BF16)
    MOE_DISPATCH_K(K, gather_bwd_kernel, bf16, grid_tokens(T), 64 * kWaves, 0, st>>>(
        (const bf16*)d_xs, slot, offsets, (const bf16*)addend, T, K, E, H, (bf16*)d_x));
  else
    MOE_DISPATCH_K(K, gather_bwd_kernel, float, grid_tokens(T), 64 * kWaves, 0, st>>>(
        (const float*)d_xs, slot, offsets, (const float*)addend, T, K, E, H, (float*)d_x));
  return check_launch(who);
}

extern "C" int moe_amd_gather_backward(const void* d_xs, const int32_t* slot,
                                       const int32_t* offsets, int64_t T, int K, int E, int H,
                                       int dtype, void* d_x, void* stream) {
  return gather_backward_impl(d_xs, slot, offsets, nullptr, T, K, E, H, dtype, d_x, stream,
                              "gather_backward");
}

extern "C" int moe_amd_gather_backward_add(const void* d_xs, const int32_t* slot,
                                           const int32_t* offsets, const void* addend, int64_t T,
                                           int K, int E, int H, int dtype, void* d_x,
                                           void* stream) {
  MOE_REQUIRE(addend || T == 0, MOE_ERR_ARG, "gather_backward_add: null addend");
  return gather_backward_impl(d_xs, slot, offsets, addend, T, K, E, H, dtype, d_x, stream,
                              "gather_backward_add");
}

extern "C" int moe_amd_weight_grad_reduce(const float* partials, int n_part, const int32_t* slot,
                                          const int32_t* offsets, int64_t T, int K, int E,
                                          void* d_topk_weights, int weights_dtype, void* stream) {
  const char* who = "weight_grad_reduce";
  MOE_REQUIRE(T >= 0 && K >= 1 && E >= 1 && n_part >= 1, MOE_ERR_ARG, "%s: bad sizes", who);
  MOE_REQUIRE(weights_dtype == MOE_DTYPE_F32 || weights_dtype == MOE_DTYPE_BF16, MOE_ERR_ARG,
              "%s: weights_dtype must be fp32 or bf16", who);
  MOE_REQUIRE(offsets && (T == 0 || (partials && slot && d_topk_weights)), MOE_ERR_ARG,
              "%s: null pointer", who);
  const int64_t n = T * K;
  if (n == 0) return MOE_OK;
  weight_grad_reduce_kernel<<<(unsigned)((n + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      partials, n_part, slot, offsets, E, n, d_topk_weights, weights_dtype == MOE_DTYPE_BF16);
  return check_launch(who);
}
