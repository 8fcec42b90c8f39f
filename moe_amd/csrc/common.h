// Shared types, status codes and small device helpers for the MoE expert-layer
// kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <atomic>
#include <stdint.h>
#include <stddef.h>

#include "../../include/moe_amd.h"

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace moe {

// Records a human-readable message for moe_amd_last_error() (thread-local).
void set_error(const char* fmt, ...);
// Maps a pending HIP launch error to MOE_ERR_HIP (and records its text).
int check_launch(const char* what);

#define MOE_REQUIRE(cond, code, ...)      \
  do {                                    \
    if (!(cond)) {                        \
      ::moe::set_error(__VA_ARGS__);      \
      return (code);                      \
    }                                     \
  } while (0)

static inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Raises `kernel`'s dynamic-LDS limit to `bytes` on the current device the
// first time it is launched there (`done` is that kernel's own per-device
// record); later launches on the device make no call besides the launch.
static inline hipError_t set_dynamic_lds_once(std::atomic<int> (&done)[64], const void* kernel,
                                              int bytes) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  const bool cached = dev >= 0 && dev < 64;
  if (cached && done[dev].load(std::memory_order_acquire) >= bytes) return hipSuccess;
  err = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (err == hipSuccess && cached) done[dev].store(bytes, std::memory_order_release);
  return err;
}

// ---- GEMM tile plan (written by the permutation, read by the GEMMs) -----
// int32 tile_starts[3][E+1]: exclusive prefix of ceil(count_e / BM) for the
// row-tile heights BM = 64, 128, 256; int32 row_tile: the index of the height
// the token-grouped GEMMs run with (the one of least tiles x (BM + 256), the
// rows and weight columns a 256-column tile streams; the larger on ties);
// then, 16-byte aligned, for each BM an int4 table info[ceil(S/BM) + E] =
// {expert, first row, end row, 0} of every row tile in expert order.
constexpr int kTileSizes[3] = {64, 128, 256};
static inline size_t plan_row_tile_offset(int E) { return (size_t)3 * (E + 1) * sizeof(int); }
static inline int64_t plan_max_tiles(int64_t S, int E, int b) {
  return (S + kTileSizes[b] - 1) / kTileSizes[b] + E;
}
static inline size_t plan_info_offset(int64_t S, int E, int b) {
  size_t off = align_up(plan_row_tile_offset(E) + sizeof(int), 16);
  for (int i = 0; i < b; ++i) off += 16 * (size_t)plan_max_tiles(S, E, i);
  return off;
}
// Then the schedule of the two dW GEMMs (tiles of one expert cost its row
// count): int32 queue[2][16] (per dW GEMM: the tile counters of 8 per-XCD
// queues and a count of finished workgroups; zeroed by the permutation and
// reset by each GEMM's last workgroup), int32 xstart[32] (experts of XCD x
// are xorder[xstart[x] .. xstart[x+1]), 9 used; at kSchedXnz + x the number
// of them that have rows, which come first), int32 xorder[E] (experts
// dealt to the XCDs heaviest first, in serpentine order).
static inline size_t plan_sched_offset(int64_t S, int E) { return plan_info_offset(S, E, 3); }
constexpr int kSchedQueueInts = 32, kSchedStartInts = 32, kSchedXnz = 16;
static inline size_t plan_bytes(int64_t S, int E) {
  return plan_sched_offset(S, E) + align_up((size_t)(kSchedQueueInts + kSchedStartInts + E) * 4, 16);
}

// True for a null or 16-byte aligned pointer (the vector paths' requirement).
static inline bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// ---- bf16 helpers -------------------------------------------------------
// Conversions go through clang's __bf16 type, which rounds to nearest-even
// (the same rounding torch applies when it stores an fp32 result as bf16).
__device__ __forceinline__ float bf2f(bf16 v) { return (float)v; }
__device__ __forceinline__ bf16 f2bf(float v) { return (bf16)v; }
__device__ __forceinline__ float round_bf(float v) { return (float)(bf16)v; }

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
// Two floats -> packed bf16 pair (lo in bits 0..15); one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Logistic function and SiLU in fp32, written as x/(1+exp(-x)) the way
// torch's opmath kernels evaluate them.
__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float siluf_(float x) { return x / (1.0f + expf(-x)); }

// Wave64 reductions via DPP-free shuffles (ds_swizzle/permute under the hood).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

}  // namespace moe
