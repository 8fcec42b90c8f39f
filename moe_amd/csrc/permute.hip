// Token permutation: a stable counting sort of the S = T*K routed entries by
// expert id, the GPU form of transformers' sort + histc + cumsum
// (transformers/integrations/moe.py:389-403).
//
//   P1 histogram : one wave per 256-entry chunk, LDS atomics -> per-chunk
//                  counts, stored expert-major [E+1][nchunks].
//   P2 scan      : per-expert exclusive scan over chunks (one block per
//                  expert) + one block that scans the expert totals into
//                  offsets and the per-tile-height GEMM tile prefixes.
//   P3 scatter   : each wave replays its chunk 64 entries at a time; one
//                  ballot per bit of the expert id groups the lanes by
//                  expert (multi-split), the in-wave rank is the popcount of
//                  lower peers, and a per-wave LDS counter carries the rank
//                  across rounds -> stable order.
// Ids outside [0,E) land in bin E (sentinels), after every real expert.
#include <atomic>

#include "common.h"

namespace moe {
namespace {

constexpr int kChunk = 256;        // entries per wave in P1/P3
constexpr int kWaves = 4;          // waves per block in P1/P3

__device__ __forceinline__ int bin_of(int64_t id, int E) {
  return (id >= 0 && id < E) ? (int)id : E;
}

__global__ __launch_bounds__(64 * kWaves) void hist_kernel(const int64_t* __restrict__ ids,
                                                           int64_t S, int E, int64_t nch,
                                                           int* __restrict__ chunk_hist) {
  extern __shared__ int lds[];  // [kWaves][E+1]
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * kWaves + wid;
  int* h = lds + wid * (E + 1);
  for (int e = lane; e <= E; e += 64) h[e] = 0;
  __builtin_amdgcn_wave_barrier();
  if (c < nch) {
    const int64_t beg = c * kChunk;
#pragma unroll
    for (int i = 0; i < kChunk / 64; ++i) {
      int64_t s = beg + i * 64 + lane;
      if (s < S) atomicAdd(&h[bin_of(ids[s], E)], 1);
    }
  }
  __builtin_amdgcn_wave_barrier();
  __syncthreads();
  if (c < nch)
    for (int e = lane; e <= E; e += 64) chunk_hist[(int64_t)e * nch + c] = h[e];
}

// Inclusive scan across one wave.
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  return v;
}

// Exclusive scan across the block (blockDim.x multiple of 64, <= 1024).
// Returns the exclusive prefix; *total receives the block sum.
__device__ int block_excl_scan(int v, int* tmp /* >= 16 ints */, int* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int inc = wave_incl_scan(v, lane);
  if (lane == 63) tmp[wid] = inc;
  __syncthreads();
  if (wid == 0) {
    int w = lane < nw ? tmp[lane] : 0;
    int wi = wave_incl_scan(w, lane);
    if (lane < nw) tmp[lane] = wi - w;
    if (lane == nw - 1) tmp[16] = wi;
  }
  __syncthreads();
  int res = inc - v + tmp[wid];
  *total = tmp[16];
  __syncthreads();
  return res;
}

// One block per bin e: exclusive scan of chunk_hist[e][0..nch) in place.
__global__ __launch_bounds__(1024) void chunk_scan_kernel(int* __restrict__ chunk_hist,
                                                         int64_t nch, int* __restrict__ totals) {
  __shared__ int tmp[17];
  const int e = blockIdx.x;
  int* col = chunk_hist + (int64_t)e * nch;
  int carry = 0;
  for (int64_t base = 0; base < nch; base += blockDim.x) {
    int64_t i = base + threadIdx.x;
    int v = i < nch ? col[i] : 0;
    int tot;
    int ex = block_excl_scan(v, tmp, &tot);
    if (i < nch) col[i] = carry + ex;
    carry += tot;
  }
  if (threadIdx.x == 0) totals[e] = carry;
}

// Single block: offsets, counts and the GEMM tile prefixes.
__global__ __launch_bounds__(1024) void finalize_kernel(const int* __restrict__ totals,
                                                        int have_totals, int E,
                                                        int* __restrict__ counts,
                                                        int* __restrict__ offsets,
                                                        int* __restrict__ tile_starts) {
  __shared__ int tmp[17];
  int carry[1 + MOE_NUM_TILE_SIZES] = {0, 0, 0, 0};
  for (int base = 0; base <= E; base += blockDim.x) {
    int e = base + threadIdx.x;
    int n = (have_totals && e <= E) ? totals[e] : 0;
    int tot;
    int ex = block_excl_scan(n, tmp, &tot);
    if (e <= E) {
      offsets[e] = carry[0] + ex;
      if (e < E) counts[e] = n;
    }
    carry[0] += tot;
#pragma unroll
    for (int b = 0; b < MOE_NUM_TILE_SIZES; ++b) {
      int bm = kTileSizes[b];
      int nt = (e < E) ? (n + bm - 1) / bm : 0;
      int ext = block_excl_scan(nt, tmp, &tot);
      if (e <= E) tile_starts[b * (E + 1) + e] = carry[1 + b] + ext;
      carry[1 + b] += tot;
    }
  }
  // The row-tile height of the token-grouped GEMMs: the least rows plus
  // weight columns streamed, tiles x (BM + 256) (the larger height on ties).
  if (threadIdx.x == 0) {
    int best = MOE_NUM_TILE_SIZES - 1;
    int64_t best_cost = (int64_t)carry[best + 1] * (kTileSizes[best] + 256);
    for (int b = MOE_NUM_TILE_SIZES - 2; b >= 0; --b) {
      const int64_t c = (int64_t)carry[1 + b] * (kTileSizes[b] + 256);
      if (c < best_cost) {
        best = b;
        best_cost = c;
      }
    }
    tile_starts[MOE_NUM_TILE_SIZES * (E + 1)] = best;
  }
}

// Grid (E, 3): fills the row-tile table of expert blockIdx.x for tile height
// kTileSizes[blockIdx.y].
__global__ __launch_bounds__(64) void tile_info_kernel(const int* __restrict__ offsets,
                                                       const int* __restrict__ tile_starts,
                                                       int E, int4* __restrict__ info0,
                                                       int4* __restrict__ info1,
                                                       int4* __restrict__ info2) {
  const int e = blockIdx.x, b = blockIdx.y;
  const int bm = kTileSizes[b];
  int4* info = b == 0 ? info0 : (b == 1 ? info1 : info2);
  const int* ts = tile_starts + b * (E + 1);
  const int t0 = ts[e], t1 = ts[e + 1];
  const int r0 = offsets[e], r1 = offsets[e + 1];
  for (int t = t0 + (int)threadIdx.x; t < t1; t += 64)
    info[t] = make_int4(e, r0 + (t - t0) * bm, r1, 0);
}

// Single block of 1024 threads: the dW-GEMM schedule.  Experts are sorted
// by an estimate of their dW tile cost (rows + a fixed epilogue cost, in 63
// log-spaced buckets, heaviest first, and the experts without rows in a
// 64th, last; by expert id within a bucket), then dealt to the 8 XCDs in
// serpentine order (0..7, 7..0, ...), which balances the XCDs' sums.  Each
// XCD's list therefore ends with its experts without rows; xnz[x] counts
// the others (the accumulating dW GEMMs claim only those).  Also zeroes the
// GEMMs' queue counters.
__global__ __launch_bounds__(1024) void dw_schedule_kernel(const int* __restrict__ counts, int E,
                                                           int* __restrict__ queue,
                                                           int* __restrict__ xstart,
                                                           int* __restrict__ xorder) {
  __shared__ int hist[64];
  const int tid = threadIdx.x;
  if (tid < kSchedQueueInts) queue[tid] = 0;
  if (tid < 64) hist[tid] = 0;
  // Experts per XCD under serpentine dealing depend on E only.
  if (tid < kSchedXnz) {
    const int rounds = E / 8, rem = E % 8;
    int acc = 0;
    for (int x = 0; x < 8 && x < tid; ++x) {
      const int lane = (rounds & 1) ? 7 - x : x;  // lane of XCD x in the last round
      acc += rounds + (lane < rem ? 1 : 0);
    }
    xstart[tid] = tid <= 8 ? acc : E;
  }
  __syncthreads();
  auto bucket = [](int n) {
    if (n == 0) return 63;             // no rows: last
    const float c = (float)n + 192.f;  // rows, plus about three k-steps of epilogue
    const int b = (int)(8.f * __log2f(c * (1.f / 192.f)));
    return 62 - min(62, max(0, b));  // 0 = heaviest
  };
  for (int e = tid; e < E; e += blockDim.x) atomicAdd(&hist[bucket(counts[e])], 1);
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int b = 0; b < 64; ++b) {
      const int n = hist[b];
      hist[b] = acc;
      acc += n;
    }
  }
  __syncthreads();
  // The nnz experts with rows take ranks 0..nnz-1; under the serpentine
  // dealing XCD x receives nnz/8 of them, plus one if its lane in the last,
  // partial round is below nnz % 8.
  if (tid < 8) {
    const int nnz = hist[63], rz = nnz / 8, mz = nnz % 8;
    const int lane = (rz & 1) ? 7 - tid : tid;
    xstart[kSchedXnz + tid] = rz + (lane < mz ? 1 : 0);
  }
  // Rank of each expert, heaviest bucket first: its bucket's start plus the
  // number of lower-id experts in the same bucket -- a stable counting sort,
  // so every call writes the same schedule.  Experts go 1024 at a time (one
  // per thread); inside a wave the lanes that share a bucket are found by
  // one ballot per bucket bit, and the waves' per-bucket counts are added
  // in wave order.
  __shared__ int wcnt[16][64];  // per-wave per-bucket counts of the current 1024 experts
  const int lane = tid & 63, wid = tid >> 6;
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int rounds = E / 8, rem = E % 8;
  for (int base = 0; base < E; base += 1024) {
    for (int i = tid; i < 16 * 64; i += blockDim.x) wcnt[i >> 6][i & 63] = 0;
    __syncthreads();
    const int e = base + tid;
    const bool valid = e < E;
    const int b = valid ? bucket(counts[e]) : 0;
    uint64_t peers = __ballot(valid);
    for (int bit = 0; bit < 6; ++bit) {
      const uint64_t m = __ballot((b >> bit) & 1);
      peers &= ((b >> bit) & 1) ? m : ~m;
    }
    if (valid && (peers >> lane) == 1ull) wcnt[wid][b] = __popcll(peers);  // highest peer
    __syncthreads();
    int pos = 0;
    if (valid) {
      pos = hist[b] + __popcll(peers & lt_mask);
      for (int w = 0; w < wid; ++w) pos += wcnt[w][b];
    }
    __syncthreads();  // every rank is formed before the bucket starts move on
    if (tid < 64) {
      int tot = 0;
      for (int w = 0; w < 16; ++w) tot += wcnt[w][tid];
      hist[tid] += tot;
    }
    if (valid) {
      const int r = pos / 8, l = pos % 8;
      const int x = (r & 1) ? 7 - l : l;
      int start = 0;
      for (int y = 0; y < x; ++y) {
        const int ly = (rounds & 1) ? 7 - y : y;
        start += rounds + (ly < rem ? 1 : 0);
      }
      xorder[start + r] = e;
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(64 * kWaves) void scatter_kernel(
    const int64_t* __restrict__ ids, int64_t S, int E, int64_t nch,
    const int* __restrict__ chunk_off, const int* __restrict__ offsets,
    int* __restrict__ row_src, int* __restrict__ slot) {
  extern __shared__ int lds[];  // [kWaves][E+1] running per-expert counters
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * kWaves + wid;
  int* cnt = lds + wid * (E + 1);
  for (int e = lane; e <= E; e += 64) cnt[e] = 0;
  __builtin_amdgcn_wave_barrier();
  if (c >= nch) return;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int key_bits = 1;  // bits of the largest key, E (sentinel bin)
  while ((E >> key_bits) != 0) ++key_bits;
  const int64_t beg = c * kChunk;
  for (int i = 0; i < kChunk / 64; ++i) {
    const int64_t s = beg + i * 64 + lane;
    const bool valid = s < S;
    const int key = valid ? bin_of(ids[s], E) : -1;
    // Lanes sharing this lane's key (multi-split by ballots): one ballot per
    // key bit, each lane keeps the lanes that agree with it on that bit.
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < key_bits; ++b) {
      const uint64_t m = __ballot((key >> b) & 1);
      peers &= ((key >> b) & 1) ? m : ~m;
    }
    int before = 0;
    if (valid) before = cnt[key];
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      int rank = __popcll(peers & lt_mask);
      int dest = offsets[key] + chunk_off[(int64_t)key * nch + c] + before + rank;
      row_src[dest] = (int)s;
      slot[s] = dest;
      // Highest peer bumps the counter once for the whole group.
      if ((peers >> lane) == 1ull) cnt[key] = before + __popcll(peers);
    }
    __builtin_amdgcn_wave_barrier();
  }
}

size_t permute_ws_bytes(int64_t S, int E) {
  int64_t nch = (S + kChunk - 1) / kChunk;
  return align_up(((size_t)(E + 1) * (size_t)nch + (size_t)(E + 1)) * sizeof(int), 256);
}

}  // namespace
}  // namespace moe

using namespace moe;

extern "C" size_t moe_amd_permute_workspace_size(int64_t S, int E) {
  if (S < 0 || E < 1) return 0;
  return permute_ws_bytes(S, E);
}

extern "C" size_t moe_amd_tile_plan_size(int64_t S, int E) {
  if (S < 0 || E < 1) return 0;
  return plan_bytes(S, E);
}

namespace moe {
namespace {

// The permutation proper: validation, then the five kernels on `stream`,
// with `workspace` as the histogram / scan scratch.
int permute_run(const int64_t* topk_index, int64_t S, int E, void* workspace,
                size_t workspace_bytes, int32_t* counts, int32_t* offsets, int32_t* row_src,
                int32_t* slot, void* tile_plan, size_t tile_plan_bytes, void* stream,
                const char* who) {
  MOE_REQUIRE(S >= 0 && S < (int64_t)1 << 31, MOE_ERR_ARG, "%s: S=%lld out of range", who,
              (long long)S);
  MOE_REQUIRE(E >= 1 && E <= 16384, MOE_ERR_ARG, "%s: E=%d out of range", who, E);
  MOE_REQUIRE(counts && offsets && tile_plan, MOE_ERR_ARG, "%s: null output", who);
  MOE_REQUIRE(tile_plan_bytes >= plan_bytes(S, E) && ((uintptr_t)tile_plan & 15) == 0,
              MOE_ERR_WORKSPACE, "%s: tile plan needs %zu bytes, 16-byte aligned", who,
              plan_bytes(S, E));
  MOE_REQUIRE(S == 0 || (topk_index && row_src && slot), MOE_ERR_ARG, "%s: null pointer", who);
  const size_t need = permute_ws_bytes(S, E);
  MOE_REQUIRE(workspace && workspace_bytes >= need, MOE_ERR_WORKSPACE,
              "%s: workspace %zu bytes < %zu needed", who, workspace_bytes, need);
  const size_t lds = (size_t)kWaves * (E + 1) * sizeof(int);
  MOE_REQUIRE(lds <= 160 * 1024, MOE_ERR_ARG, "%s: E=%d needs too much LDS", who, E);
  hipStream_t st = (hipStream_t)stream;
  const int64_t nch = (S + kChunk - 1) / kChunk;
  int* chunk_hist = (int*)workspace;
  int* totals = chunk_hist + (size_t)(E + 1) * nch;
  if (nch > 0) {
    const int blocks = (int)((nch + kWaves - 1) / kWaves);
    hist_kernel<<<blocks, 64 * kWaves, lds, st>>>(topk_index, S, E, nch, chunk_hist);
    chunk_scan_kernel<<<E + 1, 1024, 0, st>>>(chunk_hist, nch, totals);
  }
  int* tile_starts = (int*)tile_plan;
  finalize_kernel<<<1, 1024, 0, st>>>(totals, nch > 0 ? 1 : 0, E, counts, offsets, tile_starts);
  char* pb = (char*)tile_plan;
  tile_info_kernel<<<dim3(E, 3), 64, 0, st>>>(offsets, tile_starts, E,
                                              (int4*)(pb + plan_info_offset(S, E, 0)),
                                              (int4*)(pb + plan_info_offset(S, E, 1)),
                                              (int4*)(pb + plan_info_offset(S, E, 2)));
  int* sched = (int*)(pb + plan_sched_offset(S, E));
  dw_schedule_kernel<<<1, 1024, 0, st>>>(counts, E, sched, sched + kSchedQueueInts,
                                         sched + kSchedQueueInts + kSchedStartInts);
  if (nch > 0) {
    const int blocks = (int)((nch + kWaves - 1) / kWaves);
    scatter_kernel<<<blocks, 64 * kWaves, lds, st>>>(topk_index, S, E, nch, chunk_hist,
                                                     offsets, row_src, slot);
  }
  return check_launch(who);
}

}  // namespace
}  // namespace moe

extern "C" int moe_amd_permute(const int64_t* topk_index, int64_t S, int E, void* workspace,
                               size_t workspace_bytes, int32_t* counts, int32_t* offsets,
                               int32_t* row_src, int32_t* slot, void* tile_plan,
                               size_t tile_plan_bytes, void* stream) {
  return permute_run(topk_index, S, E, workspace, workspace_bytes, counts, offsets, row_src,
                     slot, tile_plan, tile_plan_bytes, stream, "permute");
}

// ---------------------------------------------------------------------------
// Allocation-free variant.  Its scratch is this file-scope device array (one
// copy per GPU, in the code object's global segment, held until the process
// ends).  In host code `scratch` names a host-side stand-in, not a device
// address: the device address of each GPU's copy comes from
// hipGetSymbolAddress, taken once per device (with that device current) on
// the entry point's first call there, and only that address is passed to the
// kernels.  The permutation's scratch is fully rewritten by every call (the
// per-chunk histograms by hist_kernel, the totals by chunk_scan_kernel), so
// nothing in it has to start at zero; calls that overlap on one GPU share the
// array and race.
static __device__ __align__(256) char scratch[MOE_PERMUTE_NOALLOC_SCRATCH_BYTES];

namespace {

std::atomic<void*> g_scratch_dev[64];  // device address of `scratch`, per device

int scratch_address(void** out, const char* who) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  MOE_REQUIRE(err == hipSuccess, MOE_ERR_HIP, "%s: hipGetDevice failed: %s", who,
              hipGetErrorString(err));
  MOE_REQUIRE(dev >= 0 && dev < 64, MOE_ERR_UNSUPPORTED, "%s: device %d out of range", who, dev);
  void* p = g_scratch_dev[dev].load(std::memory_order_acquire);
  if (!p) {
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    MOE_REQUIRE(err == hipSuccess && p, MOE_ERR_HIP, "%s: hipGetSymbolAddress failed: %s", who,
                hipGetErrorString(err));
    g_scratch_dev[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return MOE_OK;
}

}  // namespace

extern "C" int moe_amd_permute_noalloc(const int64_t* topk_index, int64_t S, int E,
                                       int32_t* counts, int32_t* offsets, int32_t* row_src,
                                       int32_t* slot, void* tile_plan, size_t tile_plan_bytes,
                                       void* stream) {
  const char* who = "permute_noalloc";
  MOE_REQUIRE(S >= 0 && S < (int64_t)1 << 31 && E >= 1 && E <= 16384, MOE_ERR_ARG,
              "%s: S=%lld or E=%d out of range", who, (long long)S, E);
  const size_t need = permute_ws_bytes(S, E);
  MOE_REQUIRE(need <= (size_t)MOE_PERMUTE_NOALLOC_SCRATCH_BYTES, MOE_ERR_UNSUPPORTED,
              "%s: S=%lld, E=%d need %zu bytes of scratch, more than the %d-byte static array "
              "(use moe_amd_permute with a workspace)", who, (long long)S, E, need,
              MOE_PERMUTE_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  int rc = scratch_address(&ws, who);
  if (rc) return rc;
  return permute_run(topk_index, S, E, ws, MOE_PERMUTE_NOALLOC_SCRATCH_BYTES, counts, offsets,
                     row_src, slot, tile_plan, tile_plan_bytes, stream, who);
}
