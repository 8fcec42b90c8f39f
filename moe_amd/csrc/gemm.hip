// Grouped bf16 GEMMs of the expert layer on gfx950 MFMA (fp32 accumulate).
//
// One kernel template covers the six GEMMs of the forward and backward pass.
// Each workgroup (4 waves, 2x2) owns a BR x 256 tile of the output C; C's
// columns are its contiguous dimension.  MFMA v_mfma_f32_32x32x16_bf16 is fed
// with the column operand as "A" (so each lane's accumulators hold four
// consecutive output columns -> 8-byte stores) and the row operand as "B".
//
//   mode  C                      rows (grouped)      cols            k
//   G1F   gate_up -> SwiGLU act  routed rows of e    I (gate|up)     H
//   G2F   y                      routed rows of e    H               I
//   G2DX  d_act -> dSwiGLU       routed rows of e    I               H
//   G1DX  d_xs                   routed rows of e    H               2I
//   G2DW  d_down_proj[e]         H                   I               rows of e
//   G1DW  d_gate_up_proj[e]      2I                  H               rows of e
//
// Data path: global -> LDS by DMA (gfx950 `buffer_load_dwordx4 ... lds`: lane
// L of a wave instruction writes 16 bytes at M0 + 16*L), so operands cost no
// VGPRs and no ds_write.  A k-stage is BK = 64 deep, so every row of a
// k-contiguous operand is fetched as one full 128-byte line (64-byte row
// pieces halve a CU's achievable load rate).  LDS is a ring of five 32 KB
// slots, each holding one operand's half of a stage (column half: 256
// features x 64 k; row half: BR rows x 64 k); while stage kt is consumed the
// three following half-stages are in flight, each wave counting its own DMA
// with s_waitcnt vmcnt before the stage barrier.  Two LDS layouts:
//   * k-contiguous operands (activation rows, the forward weights) are kept
//     as [feature][64 k] (128-byte rows, 16-byte chunks XOR-swizzled by
//     (feature >> 1) & 7) and read with ds_read_b128;
//   * k-major operands (the weights of the dX GEMMs, every operand of the dW
//     GEMMs) are copied as they lie, [64 k][features] (16-byte chunks
//     swizzled by (k & 3) << 2), and read with ds_read_b64_tr_b16, whose
//     16-lane transpose turns four 8-byte row reads into one lane's four
//     consecutive k values -- no register transposes.
// The swizzles make every DMA block a contiguous 1 KB and every fragment
// read bank-conflict free.  Global reads are raw buffer loads: reads past a
// tensor's extent return zero, which guards tails and zero-fills the ragged
// k range of the dW GEMMs.
//
// Scheduling: the kernel is persistent (one workgroup per CU).  The tile
// space -- (row tile, column tile) for the token-grouped modes, (expert, row
// tile, column tile) for dW -- is cut into 8 contiguous ranges, one per XCD
// (hardware deals workgroups round-robin over the XCDs), and the XCD's
// workgroups stride through their range, so concurrently running tiles share
// weights and rows in that XCD's L2.  A token-grouped tile reads its
// {expert, first row, end row} from the tile plan written by the
// permutation on the device: skewed and empty experts need no host round
// trip.
//
// Epilogue: accumulators are rounded to bf16 into an LDS staging tile, then
// written out row by row with 16-byte lanes (full-line stores), applying the
// mode's elementwise tail (SwiGLU, dSwiGLU) on the way out.  The stores (and
// the dX epilogue's gate_up reads) are non-temporal: each output is written
// once and consumed by a later kernel, so it should not displace the operand
// lines that concurrently running tiles share in L2 (measured: 1.8% less
// time over the six GEMMs at L, G2F 4%).
//
// Reference: transformers/integrations/moe.py:439-459 (forward grouped_mm),
// :226-242 (per-expert dX / dW formulas of the backward).
#include <atomic>
#include <type_traits>

#include "common.h"
#include "gemm_f32.h"
#include "router_group.h"

namespace moe {
namespace {

constexpr int BK = 64;       // k per stage
constexpr int SLOT = 32768;  // bytes per LDS slot (one operand's half of a stage)
constexpr int NSLOT = 5;     // ring of half-stages: two consumed, three in flight
constexpr int BC = 256;    // output columns per workgroup
// Waves per workgroup, as NW/2 row groups x 2 column groups.  Four waves (one
// per SIMD, 128x128 per wave at BR = 256) measured faster on MI355X than
// eight (two per SIMD, 64x128 per wave), which trade latency hiding for 1.5x
// the LDS fragment traffic.
template <int BR>
constexpr int kWaves = 4;
constexpr int SROW = 260;  // bf16 per row of the epilogue staging tile (520 B: conflict-free)

// RL: the router's dense linear, logits[T, E] = x[T, H] . W_r[E, H]^T.
// RDX: its input gradient, d_x[T, H] = d_logits[T, E] . W_r[E, H].
// RLTK: RLT with the softmax router fused into its epilogue (probs, top-K
//      weights and ids written from the bf16 logits of the staging tile).
// RLTS: RLT with the DeepSeek router fused into its epilogue (fp32 logits
//      staged, sigmoid scores, biased and optionally group-limited top-K,
//      renormalised and scaled weights, selection counts).
// RLT: the same logits computed transposed, rows = experts (W_r, at most one
//      or two row tiles) and columns = tokens, with the MFMA operands
//      swapped so that the tile is stored as logits[T, E]: for E <= 128 a
//      256-column tile of RL would be half padding.
// RDW: its weight gradient split over token chunks c (split-K), fp32
//      partial[c][E][H] = sum_{t in chunk c} d_logits[t, :]^T x[t, :].
// G2DXF and G2DWG are the down GEMMs' backward fused with the combine's
// backward: their row operand is d_out gathered through row_src instead of a
// materialised d_y = w * d_out[token].  G2DXF also scales by the routing
// weight, produces the weight gradient and w * act in its epilogue; G2DWG
// computes d_down_proj[e]^T = (w act)^T d_out[tokens] and stores it
// transposed.
enum Mode { G1F = 0, G2F = 1, G2DX = 2, G1DX = 3, G2DW = 4, G1DW = 5, RL = 6, RDX = 7, RDW = 8,
            G2DXF = 9, G2DWG = 10, RLT = 11, RLTK = 12, RLTS = 13 };

struct GemmArgs {
  const bf16* x;         // hidden_states [T,H]
  const bf16* w;         // gate_up_proj [E,2I,H] or down_proj [E,H,I]
  const bf16* a0;        // act [S,I] (G2F) | dy [S,H] (G2DX,G2DW) | d_gate_up [S,2I] (G1DX,G1DW)
  const bf16* a1;        // act [S,I] (G2DW) | gate_up [S,2I] (G2DX, G2DXF)
  const int* row_src;    // [S]
  const int* offsets;    // [E+1]
  const int* tile_count; // token modes: number of row tiles (tile_starts[E] for BR)
  const int* row_tile;   // token modes: the plan's chosen row-tile index; a launch whose
                         // BR is another one returns at once (null: no choice to honour)
  const int4* tile_info; // token modes: {expert, first row, end row, 0} per row tile
  bf16* out;
  bf16* out2;            // gate_up output of G1F (may be null); w * act [S,I] of G2DXF
  const void* rw;        // G2DXF: routing weights [T*K], fp32 or bf16 (rw_bf16)
  int rw_bf16;
  float* dw_part;        // G2DXF: weight-gradient partials [T*K][n_ct] fp32
  float* out_f32;        // RL: fp32 logits (null: bf16 logits in out); RDW: fp32 partials
  int chunk_rows;        // RDW: tokens per split-K chunk
  int64_t T, S;
  int E, H, I, topk;
  uint32_t tok_mul;      // n / topk == (n * tok_mul) >> tok_shift for 0 <= n < 2^31
  int tok_shift;         // 31 + ceil(log2(topk))
  int n_ct, n_rt, n_tiles;  // n_tiles: dW modes (host-known)
  float* probs;          // RLTK: router outputs probs [T,E] fp32, top-K weights [T,K] fp32,
  float* topk_w;         //   top-K ids [T,K] int64; logit offset [E] (may be null).
  int64_t* topk_idx;     //   RLTS: scores [T,E] fp32 in probs, weights [T,K] (bf16 if
  const float* offset;   //   w_bf16) in topk_w, fp32 logits in out_f32 (may be null)
  int renorm;
  const float* bias;     // RLTS: expert_bias [E] (may be null), scaling factor (0: none),
  float scaling;         //   expert groups (0: flat top-K) and groups kept, counts [E]
  int ngroups, gtopk, w_bf16;  // (may be null)
  float* tpe;
  int* queue;            // G2DW/G1DW: this GEMM's 8 XCD tile counters + finished count (null: static walk)
  const int* xstart;     // ... experts of XCD x: xorder[xstart[x] .. xstart[x+1])
  const int* xorder;
  const int* xnz;        // ... of which the first xnz[x] have rows
  int accumulate;        // G1DW/G2DWG: out[e] += dW[e] in place, experts without rows untouched
};

// Eight bf16 pairs added as torch adds two bf16 tensors: in fp32, then
// rounded to nearest even.
__device__ __forceinline__ u32x4 add_bf16x8(const u32x4& a, const u32x4& b) {
  u32x4 r;
#pragma unroll
  for (int w = 0; w < 4; ++w) r[w] = pack_bf2(bf_lo(a[w]) + bf_lo(b[w]), bf_hi(a[w]) + bf_hi(b[w]));
  return r;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

constexpr uint32_t kOOB = 0x80000000u;  // offset that always reads as zero

typedef __attribute__((address_space(3))) void lds_void_t;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4_t;

// 16-byte DMA of one lane into LDS (lane L lands at lds + 16*L).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, void* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds, 16, voff, 0, 0, 0);
}

// s_waitcnt encodings (gfx9 family): vmcnt in [3:0]+[15:14], lgkmcnt [11:8].
constexpr int vmcnt_imm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | (((n >> 4) & 3) << 14); }
#define WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(vmcnt_imm(n))
// vmcnt(n) and lgkmcnt(0) together.
#define WAIT_VMCNT_LGKM0(n) __builtin_amdgcn_s_waitcnt(vmcnt_imm(n) & ~(15 << 8))

// One transpose read.  The restrict-qualified parameter gives the load an
// alias scope once inlined, which tells the compiler's wait-count insertion
// that it does not alias the in-flight LDS DMA; without it a full
// vmcnt(0) drain is placed before every such read.  Ordering against the DMA
// is explicit in the main loop (s_waitcnt vmcnt + s_barrier).
__device__ __forceinline__ s16x4 read_tr(const lds_s16x4_t* __restrict__ p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_s16x4_t*>(p));
}

typedef __attribute__((address_space(3))) char lds_char_t;

// s + v in one VALU add that the optimizer cannot re-associate.
__device__ __forceinline__ uint32_t opaque_add(uint32_t s, uint32_t v) {
  uint32_t r;
  asm("v_add_u32_e32 %0, %1, %2" : "=v"(r) : "s"(s), "v"(v));
  return r;
}

// One MFMA fragment (8 consecutive k of one feature) from a k-major stage
// region: two transpose reads, k 0..3 and k 4..7.  The addresses stay in the
// LDS address space so that constant parts fold into the instruction offset.
__device__ __forceinline__ bf16x8 tr_frag(const lds_char_t* p0, const lds_char_t* p1) {
  const s16x4 lo = read_tr((const lds_s16x4_t*)p0);
  const s16x4 hi = read_tr((const lds_s16x4_t*)p1);
  const s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}

// Token of a routed row: row_src / topk by multiply-shift (Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994):
// with s = ceil(log2 d) and m = ceil(2^(31+s) / d), m < 2^32 and
// floor(n*m / 2^(31+s)) == floor(n / d) for every 0 <= n < 2^31.
__device__ __forceinline__ int div_topk(int n, uint32_t m, int shift) {
  return (int)(((uint64_t)(uint32_t)n * m) >> shift);
}

// Logistic sigmoid from the hardware base-2 exponential and reciprocal
// (v_exp_f32, v_rcp_f32; about 1 ulp each): 1 / (1 + 2^(-x log2 e)).  The
// epilogues evaluate it once per output element, where an IEEE expf and
// divide would make them VALU-bound.  The results feed bf16 roundings, so
// the ulp-level difference to expf/divide shows up only in rare ties.
// Saturates correctly: x -> -inf gives 0, x -> +inf gives 1.
__device__ __forceinline__ float fast_sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
}

template <int MODE, int BR>
__global__ __launch_bounds__(kWaves<BR> * 64, 1) void grouped_gemm_kernel(GemmArgs p) {
  constexpr int NW = kWaves<BR>;                          // waves, as NW/2 rows x 2 columns
  constexpr int NTHR = NW * 64;
  constexpr bool TOKEN = MODE <= G1DX || MODE == G2DXF;   // rows = routed rows of one expert
  constexpr bool TRL = MODE == RLT || MODE == RLTK || MODE == RLTS;  // transposed router linear
  if constexpr (TOKEN) {
    constexpr int my_tile = BR == 64 ? 0 : (BR == 128 ? 1 : 2);
    if (p.row_tile && __builtin_amdgcn_readfirstlane(*p.row_tile) != my_tile) return;
  }
  constexpr bool DENSE = MODE == RL || MODE == RDX || TRL;  // one "expert", dense rows
  constexpr bool COL_KM = !(MODE == G1F || MODE == G2F || MODE == RL || TRL);  // k-major cols
  constexpr bool ROW_KM = !TOKEN && !DENSE;               // row operand k-major (dW)
  constexpr bool DOWN_DX = MODE == G2DX || MODE == G2DXF;  // column operand down_proj[e], k-major
  constexpr bool GROW = MODE == G1F || MODE == G2DXF;      // row operand: token rows via row_src
  constexpr bool GCOL = MODE == G1DW || MODE == G2DWG;     // column operand: token rows via row_src (k-major)
  constexpr bool DW = MODE == G2DW || MODE == G1DW || MODE == G2DWG;
  constexpr bool SWAP = MODE == G2DWG || TRL;  // MFMA operands swapped: lanes hold 4 consecutive rows
  constexpr int WR = BR / (NW / 2);                       // rows per wave
  constexpr int TJ = WR / 32;                             // MFMA row sub-tiles per wave
  constexpr int TI = 4;                                   // MFMA col sub-tiles per wave (128 cols)
  constexpr int CPW = BC * BK * 2 / 1024 / NW;            // 1 KB DMA blocks per wave, column half
  constexpr int RPW = BR * BK * 2 / 1024 / NW;            // ... row half
  constexpr int NTOK = GCOL ? 1 : 0;                      // gathered-row index loads per stage
  // Ring order: each stage's first half (ring position 2s) is issued a stage
  // before its second half (2s+1), so it has about 1.5 stages of lead to the
  // barrier that needs it, the second half about one.  The row half goes
  // first where that measured faster (G1F's gathered token rows: -1.5% at L;
  // G1DX -0.8%; the dense mode), the column half elsewhere (G2F +3% with the
  // rows first).  The dW GEMMs keep the column half first: their row_src
  // pipeline fetches the gathered column operand's entries a stage ahead.
  constexpr bool ROW_FIRST = MODE == G1F || MODE == G1DX || MODE == RL;
  constexpr int FPW = ROW_FIRST ? RPW : CPW, SPW = ROW_FIRST ? CPW : RPW;  // DMA ops per half
  constexpr int NOPS = NTOK + RPW + CPW;                  // memory ops per main-loop step
  constexpr int NGRP = (BK / 16) * TI;                    // MFMA groups per step
  static_assert(CPW * NW == 32 && RPW * NW * 8 == BR && TJ >= 1, "DMA blocks per wave");
  // PF: the next tile's first stages are issued before this tile's epilogue,
  // which is wave-local and issues exactly NST stores per wave.
  constexpr bool PF = MODE == G1F || MODE == G2F || MODE == G1DX || MODE == G1DW || MODE == G2DWG ||
                      MODE == RDX || MODE == G2DXF;
  constexpr int NST = (MODE == G1F ? 12 : 8) * TJ;
  static_assert(!PF || FPW + NST <= 63, "vmcnt range");
  static_assert(TOKEN || DENSE || BR == 256, "dW modes use 256-row tiles");

  extern __shared__ __attribute__((aligned(16))) bf16 smem[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: LDS DMA targets stay scalar
  const int wr = wid >> 1, wc = wid & 1;
  const int l32 = lane & 31, hl = lane >> 5;
  const int H = p.H, I = p.I, I2 = 2 * p.I;

  // ------------------------------------------------------------ tile walk
  // Static: the tile space is cut into 8 contiguous ranges, one per XCD
  // (workgroups are dealt to the XCDs round-robin), walked with stride
  // nslot.  Dynamic (dW GEMMs with a schedule): tile v belongs to expert
  // xorder[v / tiles-per-expert]; each XCD's experts form a contiguous range
  // of v that its workgroups claim one tile at a time from the XCD's
  // counter, heaviest expert first, then from the other XCDs' counters once
  // their own is exhausted.  Every workgroup stops when all 8 are.
  const int n_tiles = TOKEN ? (*p.tile_count) * p.n_ct : p.n_tiles;
  const int xcd = blockIdx.x & 7, nslot = gridDim.x >> 3;
  const bool dyn = DW && p.queue != nullptr;
  const int per_e = p.n_rt * p.n_ct;
  // Lane x (of 8) holds XCD x's first expert slot and the number of its
  // experts to claim (all, or the xnz[x] with rows), read once: a claim then
  // makes one memory round trip, its atomic.
  int xs_lane = 0, xn_lane = 0;
  if (dyn) {
    const int x = lane & 7;
    xs_lane = p.xstart[x];
    xn_lane = p.accumulate ? p.xnz[x] : p.xstart[x + 1] - xs_lane;
  }
  auto claim = [&]() -> int {
    int* box = (int*)smem;  // free: the previous tile's epilogue ended with a barrier
    // (read out of the lanes by the whole wave, outside the one-lane branch)
    int e0s[8], ns[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int x = (xcd + k) & 7;
      e0s[k] = __builtin_amdgcn_readlane(xs_lane, x);
      ns[k] = __builtin_amdgcn_readlane(xn_lane, x) * per_e;
    }
    if (tid == 0) {
      int v = -1;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int x = (xcd + k) & 7;
        const int e0 = e0s[k], n = ns[k];
        if (n == 0) continue;
        const int j = __hip_atomic_fetch_add(p.queue + x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (j < n) {
          v = e0 * per_e + j;
          break;
        }
      }
      box[0] = v;
    }
    __syncthreads();
    const int v = __builtin_amdgcn_readfirstlane(box[0]);
    __syncthreads();  // read by every wave before the next tile's DMA may land here
    return v;
  };
  const int chunk = (n_tiles + 7) >> 3;
  const int t_end = dyn ? 0 : min(n_tiles, (xcd + 1) * chunk);
  int t = dyn ? claim() : xcd * chunk + (int)(blockIdx.x >> 3);
  if (!dyn && t >= t_end) return;

  struct Tile {
    int e, row0, row_end, ct, kbeg, kend, nk;
  };
  // pre (token modes): the tile's {expert, first row, end row} loaded ahead
  auto decode = [&](int tt, const int4* pre = nullptr) {
    Tile d;
    if constexpr (TOKEN) {
      d.ct = tt % p.n_ct;
      const int4 ti = pre ? *pre : p.tile_info[tt / p.n_ct];
      d.e = ti.x;
      d.row0 = ti.y;
      d.row_end = ti.z;
      d.kbeg = d.kend = 0;
    } else if constexpr (DENSE) {
      d.ct = tt % p.n_ct;
      d.e = 0;
      d.row0 = (tt / p.n_ct) * BR;
      d.row_end = (int)min((int64_t)d.row0 + BR, TRL ? (int64_t)p.E : p.T);
      d.kbeg = d.kend = 0;
    } else {
      const int vi = tt / per_e;
      d.e = dyn ? p.xorder[vi] : vi;
      const int rem = tt - vi * per_e;
      const int rt = rem / p.n_ct;
      d.ct = rem - rt * p.n_ct;
      d.row0 = rt * BR;
      d.row_end = 0;
      if constexpr (MODE == RDW) {
        d.kbeg = (int)min((int64_t)d.e * p.chunk_rows, p.T);
        d.kend = (int)min((int64_t)d.kbeg + p.chunk_rows, p.T);
      } else {
        d.kbeg = p.offsets[d.e];
        d.kend = p.offsets[d.e + 1];
      }
    }
    // Tile fields are wave-uniform; say so, so that the buffer descriptors
    // built from them stay in SGPRs.
    d.e = __builtin_amdgcn_readfirstlane(d.e);
    d.row0 = __builtin_amdgcn_readfirstlane(d.row0);
    d.row_end = __builtin_amdgcn_readfirstlane(d.row_end);
    d.ct = __builtin_amdgcn_readfirstlane(d.ct);
    d.kbeg = __builtin_amdgcn_readfirstlane(d.kbeg);
    d.kend = __builtin_amdgcn_readfirstlane(d.kend);
    int K_len;
    if constexpr (MODE == G1F || DOWN_DX || MODE == RL || TRL) K_len = H;
    else if constexpr (MODE == RDX) K_len = p.E;
    else if constexpr (MODE == G2F) K_len = I;
    else if constexpr (MODE == G1DX) K_len = I2;
    else K_len = d.kend - d.kbeg;
    d.nk = (K_len + BK - 1) / BK;
    return d;
  };

  // ------------------------------------------------------- DMA geometry
  // Wave w fills the 1 KB blocks w, w+NW, w+2NW, ... of each half-stage.  In a
  // k-contiguous half, lane L carries feature 8*blk + L/8 and physical chunk
  // L&7, which holds logical chunk (L&7) ^ ((feature>>1)&7).  In a k-major
  // half it carries k row 2*blk + L/32 and physical chunk L&31, which holds
  // logical chunk (L&31) ^ ((k&3)<<2) (8 features per chunk).
  auto kc_feature = [&](int blk) { return blk * 8 + (lane >> 3); };
  auto kc_chunk = [&](int f) { return (lane & 7) ^ ((f >> 1) & 7); };
  auto km_krow = [&](int blk) { return blk * 2 + (lane >> 5); };
  auto km_chunk = [&](int k) { return (lane & 31) ^ ((k & 3) << 2); };

  // Operand extents: a stage's DMA uses a buffer descriptor rebased to the
  // stage (base + s*step, bytes - s*step, in scalar registers), so the
  // per-lane offsets stay fixed and reads past the extent still return 0.
  const char* cptr = nullptr;
  const char* rptr = nullptr;
  uint32_t cbytes = 0, rbytes = 0;
  uint64_t rbytes64 = 0;  // dW modes: the expert's k-major row operand, any size
  __amdgpu_buffer_rsrc_t isrc;
  uint32_t coff[CPW];  // byte offsets of this lane's column blocks at stage 0
  uint32_t roff[RPW];
  uint32_t cstep = 0, rstep = 0;  // byte advance per stage
  int kb_cur = 0, ke_cur = 0, nk_cur = 0;
  // Descriptor of stage s of an operand.  Stages past the tile's last one
  // are still issued (the wait counts count them) but get an empty extent:
  // their loads return zeros without a memory access, so they add no L2 or
  // HBM traffic and land quickly.
  auto stage_rsrc = [&](const char* ptr, uint32_t bytes, uint32_t adv, int s) {
    // readfirstlane: keep the descriptor scalar (a vector descriptor would
    // turn every DMA into a waterfall loop).
    const uint32_t left =
        __builtin_amdgcn_readfirstlane((s < nk_cur && adv < bytes) ? bytes - adv : 0u);
    return make_rsrc(ptr + adv, left);
  };
  // RLT: each tile walks its k-stages starting at stage ct % nk (wrapping),
  // so that the workgroups, all starting together, read different 128-byte
  // column blocks of their token rows instead of the same block of every
  // row at once (which lands on few HBM channels).  Other modes: identity.
  int krot = 0, knk = 1;
  auto kst = [&](int st) -> uint32_t {
    if constexpr (TRL) {
      int v = st + krot;
      v -= v >= knk ? knk : 0;
      v -= v >= knk ? knk : 0;
      v -= v >= knk ? knk : 0;
      return (uint32_t)v;
    } else {
      return (uint32_t)st;
    }
  };
  // The dW modes' row operand (one expert's rows, k-major) is rebased per
  // stage in 64 bits: an expert may own more than 4 GB of rows (a token
  // listing one expert several times is accepted), and a stage reads at
  // most rstep bytes past its base, so the extent is capped, not wrapped.
  auto row_stage_rsrc = [&](int s) {
    if constexpr (ROW_KM) {
      const uint64_t adv = (uint64_t)(uint32_t)s * rstep;
      const uint64_t left = (s < nk_cur && adv < rbytes64) ? rbytes64 - adv : 0ull;
      return make_rsrc(rptr + adv, __builtin_amdgcn_readfirstlane(
                                       (uint32_t)(left < 0xfffff000ull ? left : 0xfffff000ull)));
    } else {
      const uint32_t adv = kst(s) * rstep;
      return make_rsrc(rptr + adv, __builtin_amdgcn_readfirstlane(
                                       (s < nk_cur && adv < rbytes) ? rbytes - adv : 0u));
    }
  };
  // G2DXF: row_src of this lane's tile rows (wr*WR + j*32 + l32, j < TJ) of
  // the tile that setup() prepared (nsrc) and of the tile being computed
  // (csrc), and the latter's routing weights (raw bits: fp32, or bf16
  // zero-extended).  The epilogue of one tile runs after the next tile's
  // setup, so each tile's values pass from the n- to the c-set at the hand-over.
  int nsrc[TOKEN ? TJ : 1], csrc[TOKEN ? TJ : 1];
  uint32_t cwr[TOKEN ? TJ : 1];

  // rs (gathered rows): the row_src entries of the lane's DMA rows, loaded
  // ahead by rows_load
  auto setup = [&](const Tile& d, const int* rs = nullptr) {
    kb_cur = d.kbeg;
    ke_cur = d.kend;
    nk_cur = d.nk;
    if constexpr (TRL) {
      knk = d.nk > 0 ? d.nk : 1;
      krot = __builtin_amdgcn_readfirstlane(d.ct % knk);
    }
    // Column operand.
    if constexpr (MODE == G1F) {
      cptr = (const char*)(p.w + (int64_t)d.e * I2 * H);
      cbytes = (uint32_t)(I2 * H * 2);
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
        const int f = kc_feature(wid + NW * i);  // tile column: [gate 64 | up 64] per wave column
        const int lc = f & 127;
        const int feat = d.ct * 128 + (f >> 7) * 64 + (lc & 63);
        const int wrow = (lc < 64) ? feat : I + feat;
        coff[i] = (uint32_t)wrow * (uint32_t)(H * 2) + kc_chunk(f) * 16;
      }
      cstep = BK * 2;
    } else if constexpr (TRL) {
      // hidden_states rows [T][H]: tokens are the tile's columns
      cptr = (const char*)p.x;
      cbytes = (uint32_t)(p.T * H * 2);
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
        const int f = kc_feature(wid + NW * i);
        const int64_t tok = (int64_t)d.ct * BC + f;
        coff[i] = tok < p.T ? (uint32_t)tok * (uint32_t)(H * 2) + kc_chunk(f) * 16 : kOOB;
      }
      cstep = BK * 2;
    } else if constexpr (MODE == G2F || MODE == RL) {
      // weight rows [ncol][kdim]: down_proj[e] [H][I], or W_r [E][H]
      const int ncol = MODE == RL ? p.E : H, kdim = MODE == RL ? H : I;
      cptr = (const char*)(p.w + (int64_t)d.e * ncol * kdim);
      cbytes = (uint32_t)(ncol * kdim * 2);
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
        const int f = kc_feature(wid + NW * i);
        const int wrow = d.ct * BC + f;
        coff[i] = wrow < ncol ? (uint32_t)wrow * (uint32_t)(kdim * 2) + kc_chunk(f) * 16 : kOOB;
      }
      cstep = BK * 2;
    } else {
      // k-major column operand: rows of k, features contiguous.
      int ld;
      if constexpr (DOWN_DX) {
        cptr = (const char*)(p.w + (int64_t)d.e * H * I);
        cbytes = (uint32_t)(H * I * 2);
        ld = I;
      } else if constexpr (MODE == RDX) {  // W_r [E][H]: k = expert, features = H
        cptr = (const char*)p.w;
        cbytes = (uint32_t)(p.E * H * 2);
        ld = H;
      } else if constexpr (MODE == G1DX) {
        cptr = (const char*)(p.w + (int64_t)d.e * I2 * H);
        cbytes = (uint32_t)(I2 * H * 2);
        ld = H;
      } else if constexpr (MODE == G2DW) {
        cptr = (const char*)(p.a1 + (int64_t)d.kbeg * I);
        cbytes = (uint32_t)((int64_t)(d.kend - d.kbeg) * I * 2);
        ld = I;
      } else if constexpr (MODE == RDW) {  // hidden_states rows of the chunk
        cptr = (const char*)(p.x + (int64_t)d.kbeg * H);
        cbytes = (uint32_t)((int64_t)(d.kend - d.kbeg) * H * 2);
        ld = H;
      } else {  // G1DW, G2DWG: rows of hidden_states / d_out gathered through row_src
        cptr = (const char*)p.x;
        cbytes = (uint32_t)(p.T * H * 2);
        ld = H;
      }
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
        const int k = km_krow(wid + NW * i);
        const uint32_t fb = (uint32_t)(d.ct * BC + km_chunk(k) * 8) * 2;
        coff[i] = GCOL ? fb : (uint32_t)k * (uint32_t)(ld * 2) + fb;
      }
      cstep = GCOL ? 0 : (uint32_t)BK * ld * 2;
    }
    // Row operand.
    if constexpr (GROW) {  // hidden_states (G1F) or d_out (G2DXF) rows of the routed tokens
      rptr = (const char*)p.x;
      rbytes = (uint32_t)(p.T * H * 2);
#pragma unroll
      for (int i = 0; i < RPW; ++i) {
        const int f = kc_feature(wid + NW * i);
        const int r = min(d.row0 + f, d.row_end - 1);
        const int tok = div_topk(rs ? rs[i] : p.row_src[r], p.tok_mul, p.tok_shift);
        roff[i] = (uint32_t)tok * (uint32_t)(H * 2) + kc_chunk(f) * 16;
      }
      rstep = BK * 2;
    } else if constexpr (TOKEN || DENSE) {
      const int ld = (MODE == G2F) ? I : ((MODE == G2DX || MODE == RL || TRL) ? H : (MODE == RDX ? p.E : I2));
      // The tile's own rows only: the extent fits 32 bits whatever S is.
      rptr = (const char*)(p.a0 + (int64_t)d.row0 * ld);
      rbytes = (uint32_t)((int64_t)min(d.row_end - d.row0, BR) * ld * 2);
#pragma unroll
      for (int i = 0; i < RPW; ++i) {
        const int f = kc_feature(wid + NW * i);
        const int r = min(f, d.row_end - d.row0 - 1);
        roff[i] = (uint32_t)r * (uint32_t)(ld * 2) + kc_chunk(f) * 16;
      }
      rstep = BK * 2;
    } else {
      const int ld = (MODE == G2DW) ? H : (MODE == RDW ? p.E : (MODE == G2DWG ? I : I2));
      rptr = (const char*)(p.a0 + (int64_t)d.kbeg * ld);
      rbytes64 = (uint64_t)(d.kend - d.kbeg) * (uint64_t)ld * 2;
#pragma unroll
      for (int i = 0; i < RPW; ++i) {
        const int k = km_krow(wid + NW * i);
        roff[i] = (uint32_t)k * (uint32_t)(ld * 2) + (uint32_t)(d.row0 + km_chunk(k) * 8) * 2;
      }
      rstep = (uint32_t)BK * ld * 2;
    }
    if constexpr (GCOL) isrc = make_rsrc(p.row_src, (uint32_t)(p.S * 4));
    // G2DXF: row_src of tile row tid, consumed by the epilogue (the load
    // completes under the main loop).
    if constexpr (MODE == G2DXF) {
#pragma unroll
      for (int j = 0; j < TJ; ++j)
        nsrc[j] = p.row_src[min(d.row0 + wr * WR + j * 32 + l32, d.row_end - 1)];
    }
  };

  // The row_src entries setup() reads for a gathered-row tile (G1F, G2DXF).
  auto rows_load = [&](const Tile& d, int (&rs)[GROW ? RPW : 1]) {
    if constexpr (GROW) {
#pragma unroll
      for (int i = 0; i < RPW; ++i)
        rs[i] = p.row_src[min(d.row0 + kc_feature(wid + NW * i), d.row_end - 1)];
    }
  };

  // G1DW, G2DWG: raw row_src entries of stage s, one 64-lane load per wave
  // (lane L: k row L of the stage).  Reads past S return zero.
  auto fetch_tok = [&](int s, int (&tk)[NTOK > 0 ? NTOK : 1]) {
    if constexpr (GCOL)
      tk[0] = __builtin_amdgcn_raw_buffer_load_b32(isrc, (uint32_t)(kb_cur + s * BK + lane) * 4, 0, 0);
  };
  // ... turned in place, once the load has landed, into the byte offset of
  // each k row's token row (token * H * 2), or kOOB for rows past the
  // expert's range; a column block's two k rows are then read out of it
  // with v_readlane when its DMA offsets are formed.
  auto tok_offsets = [&](int s, int (&tk)[NTOK > 0 ? NTOK : 1]) {
    if constexpr (GCOL) {
      // Branch-free select (a branch would mask lanes and wait on the load).
      const uint32_t v = (uint32_t)div_topk(tk[0], p.tok_mul, p.tok_shift) * (uint32_t)(H * 2);
      const uint32_t m = 0u - (uint32_t)(s * BK + lane < ke_cur - kb_cur);
      tk[0] = (int)((v & m) | (kOOB & ~m));
    }
  };

  auto slot_ptr = [&](int h) { return (char*)smem + (h % NSLOT) * SLOT; };

  // DMA of the column half of stage s (ring position 2s).
  auto col_off = [&](int s, int i, const int (&tk)[NTOK > 0 ? NTOK : 1]) -> uint32_t {
    if constexpr (GCOL) {
      // tk: stage s's row offsets (tok_offsets).  A kOOB row stays at or
      // above kOOB plus the column offset (< 2^31), beyond the operand's
      // extent (T * H * 2 < 2^31), so it reads zeros.
      (void)s;
      const int blk = wid + NW * i;  // wave-uniform: k rows 2*blk and 2*blk+1
      const uint32_t ta = (uint32_t)__builtin_amdgcn_readlane(tk[0], 2 * blk);
      const uint32_t tb = (uint32_t)__builtin_amdgcn_readlane(tk[0], 2 * blk + 1);
      return ((lane >> 5) ? tb : ta) + coff[i];
    } else {
      return coff[i];
    }
  };
  auto issue_col = [&](int s, const int (&tk)[NTOK > 0 ? NTOK : 1]) {
    char* base = slot_ptr(2 * s + (ROW_FIRST ? 1 : 0));
    const auto rs = stage_rsrc(cptr, cbytes, kst(s) * cstep, s);
#pragma unroll
    for (int i = 0; i < CPW; ++i) dma16(rs, col_off(s, i, tk), base + (wid + NW * i) * 1024);
  };
  // DMA of the row half of stage s (ring position 2s+1, or 2s if ROW_FIRST).
  auto issue_row = [&](int s) {
    char* base = slot_ptr(2 * s + (ROW_FIRST ? 0 : 1));
    const auto rs = row_stage_rsrc(s);
#pragma unroll
    for (int i = 0; i < RPW; ++i) dma16(rs, roff[i], base + (wid + NW * i) * 1024);
  };

  // Fragment reads.  Per-lane byte offsets within a slot are computed once:
  // k-contiguous operands need one base per k sub-step ks (the swizzle
  // mixes ks into the chunk index) and step 4096 bytes per 32-row sub-tile;
  // k-major operands need one base per sub-tile (the swizzle mixes the
  // sub-tile into the chunk index) and step 8192 bytes per ks and 2048 per
  // transpose half.  A read then costs one add of the slot's base.
  const int tg = lane >> 4, tj = lane & 15;
  const int tka = 8 * (tg >> 1) + (tj >> 2);                  // transpose-read k row (ks 0, half 0)
  const int tsub = 2 * (tg & 1) + ((tj & 3) >> 1);            // chunk within a 32-feature group
  const uint32_t thalf = 8 * (tj & 1);                        // byte half within the chunk
  uint32_t a_off[4], b_off[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if constexpr (!COL_KM)
      a_off[q] = (uint32_t)(wc * 128 + l32) * (BK * 2) + (uint32_t)(((2 * q + hl) ^ ((l32 >> 1) & 7)) * 16);
    else
      a_off[q] = (uint32_t)tka * (BC * 2) +
                 ((uint32_t)((wc * 16 + q * 4 + tsub) ^ ((tka & 3) << 2)) << 4) + thalf;
    if constexpr (!ROW_KM)
      b_off[q] = (uint32_t)(wr * WR + l32) * (BK * 2) + (uint32_t)(((2 * q + hl) ^ ((l32 >> 1) & 7)) * 16);
    else
      b_off[q] = (uint32_t)tka * (BR * 2) +
                 ((uint32_t)((wr * (WR / 8) + q * 4 + tsub) ^ ((tka & 3) << 2)) << 4) + thalf;
  }
  // Column sub-tile i / row sub-tile j of k sub-step ks from the slot at
  // byte offset so.
  // Per step, the slot base is added to the four per-lane offsets of each
  // operand once (opaque to the optimizer, which would otherwise fold the
  // sub-step constants into the scalar slot base and re-add per read); the
  // sub-step and sub-tile parts then ride in the instructions' offsets.
  // The addresses are absolute LDS byte addresses: the base of the dynamic
  // LDS array (a link-time constant the compiler would otherwise add to
  // every read) is folded into the scalar slot base once per step.
  const uint32_t lds0 = (uint32_t)(uintptr_t)(const lds_char_t*)smem;
  auto lds_at = [](uint32_t a) { return (const lds_char_t*)(uintptr_t)a; };
  uint32_t a_adr[4], b_adr[4];
  auto slot_bases = [&](uint32_t sC, uint32_t sR) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      a_adr[q] = opaque_add(lds0 + sC, a_off[q]);
      b_adr[q] = opaque_add(lds0 + sR, b_off[q]);
    }
  };
  auto read_a = [&](int ks, int i) -> bf16x8 {
    if constexpr (!COL_KM) {
      return *(const __attribute__((address_space(3))) bf16x8*)lds_at(a_adr[ks] + i * 4096);
    } else {
      const lds_char_t* q = lds_at(a_adr[i] + ks * (16 * BC * 2));
      return tr_frag(q, q + 4 * BC * 2);
    }
  };
  auto read_b = [&](int ks, int j) -> bf16x8 {
    if constexpr (!ROW_KM) {
      return *(const __attribute__((address_space(3))) bf16x8*)lds_at(b_adr[ks] + j * 4096);
    } else {
      const lds_char_t* q = lds_at(b_adr[j] + ks * (16 * BR * 2));
      return tr_frag(q, q + 4 * BR * 2);
    }
  };

  f32x16 acc[TI][TJ];
  // acc[i][j] += column fragment i x row fragment j.  Register 4q+c of a
  // lane then holds (row l32, column 8q+4hl+c) of the 32x32 sub-tile, or,
  // with the operands swapped, (row 8q+4hl+c, column l32).
  auto mma = [](const bf16x8& a, const bf16x8& b, const f32x16& c) {
    if constexpr (SWAP) return __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  };

  // The main loop's row_src entries (G1DW, G2DWG), shared by the prologue
  // and the loop.
  int tk_a[NTOK > 0 ? NTOK : 1], tk_b[NTOK > 0 ? NTOK : 1], tn[NTOK > 0 ? NTOK : 1];
  // Prologue: the DMA of stage 0 and of stage 1's column half (ring
  // positions 0, 1, 2 = slots 0, 1, 2) of the tile that setup() prepared.
  auto prologue = [&]() {
      // The wait counts rely on issue order; sched_barrier keeps the
      // scheduler from interleaving the groups.
      fetch_tok(0, tk_a);
      fetch_tok(1, tk_b);
      tok_offsets(0, tk_a);
      if constexpr (ROW_FIRST) issue_row(0);
      else issue_col(0, tk_a);
      __builtin_amdgcn_sched_barrier(0);
      fetch_tok(2, tk_a);
      if constexpr (ROW_FIRST) issue_col(0, tk_a);
      else issue_row(0);
      __builtin_amdgcn_sched_barrier(0);
      tok_offsets(1, tk_b);
      if constexpr (ROW_FIRST) issue_row(1);
      else issue_col(1, tk_b);
  };
  // Main loop of tile `cur` (its prologue issued).  after_epi: the previous
  // tile's epilogue stores were issued after this tile's prologue (PF modes).
  auto mainloop = [&](const Tile& cur, bool after_epi) {
    (void)after_epi;
      // Byte offsets of ring positions 2kt + c, c = 0..4, at stage kt.  The
      // positions advance by two per stage, so the five offsets rotate by
      // two at the end of each stage (register moves, not a modulo).
      uint32_t rq[5] = {0, SLOT, 2 * SLOT, 3 * SLOT, 4 * SLOT};
      // Op o of window W(w): the second half of stage w+1 (descriptor rsr)
      // lands at ring offset srow, the first half of stage w+2 (descriptor
      // rsc) at scol; `tk` holds the row_src entries of stage w+2.  A window
      // begins in the last sub-step of the stage before, so its second-half
      // descriptor is formed once there and carried into the next iteration.
      static_assert(TI * NOPS / NGRP <= NTOK + SPW, "a window's first TI groups hold no first-half op");
      auto row_rsrc = [&](int s) { return row_stage_rsrc(s); };
      auto col_rsrc = [&](int s) { return stage_rsrc(cptr, cbytes, kst(s) * cstep, s); };
      // descriptors of the second half of stage s and the first half of stage s
      auto second_rsrc = [&](int s) { return ROW_FIRST ? col_rsrc(s) : row_rsrc(s); };
      auto first_rsrc = [&](int s) { return ROW_FIRST ? row_rsrc(s) : col_rsrc(s); };
      auto win_op = [&](int w, int o, const int (&tk)[NTOK > 0 ? NTOK : 1], uint32_t srow,
                        uint32_t scol, __amdgpu_buffer_rsrc_t rsr, __amdgpu_buffer_rsrc_t rsc) {
        if (o < NTOK) {
          if constexpr (GCOL)
            tn[0] = __builtin_amdgcn_raw_buffer_load_b32(
                isrc, (uint32_t)(kb_cur + (w + 3) * BK + lane) * 4, 0, 0);
        } else if (o < NTOK + SPW) {  // second half of stage w+1, at srow with rsr
          const int i = o - NTOK;
          if constexpr (ROW_FIRST) dma16(rsr, col_off(w + 1, i, tk), (char*)smem + srow + (wid + NW * i) * 1024);
          else dma16(rsr, roff[i], (char*)smem + srow + (wid + NW * i) * 1024);
        } else {  // first half of stage w+2, at scol with rsc
          const int i = o - NTOK - SPW;
          if constexpr (ROW_FIRST) dma16(rsc, roff[i], (char*)smem + scol + (wid + NW * i) * 1024);
          else dma16(rsc, col_off(w + 2, i, tk), (char*)smem + scol + (wid + NW * i) * 1024);
        }
      };
      // Issue order inside an MFMA group: two MFMAs, the group's memory
      // ops, one MFMA, its fragment reads, the last MFMA (measured best
      // among the orders tried).
      auto group_order = [&]() {
        if constexpr (MODE == G1F) {
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);  // VMEM read (the group's 0-2 ops)
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // DS read (2-4 fragment reads)
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        } else {
          // the same, with up to five scalar instructions placed after each
          // of the first three MFMAs (dW GEMMs -1 to -2%, G2F -0.7%; G1F
          // measured no better)
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x004, 5, 0);  // SALU
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);  // VMEM read
          __builtin_amdgcn_sched_group_barrier(0x004, 5, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // DS read
          __builtin_amdgcn_sched_group_barrier(0x004, 5, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
      };
      constexpr int GQ = BK / 16 - 1;  // groups before the last sub-step: NGRP - TI
      constexpr int NLR = TI + TJ;     // fragment reads of a sub-step
      bf16x8 fa[2][TI], fb[2][TJ];
      if constexpr (PF) {
        // the previous tile's NST epilogue stores were issued after this
        // tile's first stages: they may still be in flight
        // (G2DXF: its epilogue waited for gate/up loads issued after this
        // tile's first stages, and loads complete in issue order, so those
        // stages have landed; only its trailing stores may be in flight.)
        if (after_epi) WAIT_VMCNT_LGKM0(MODE == G2DXF ? 63 : FPW + NST);
        else WAIT_VMCNT_LGKM0(FPW);
      } else {
        WAIT_VMCNT_LGKM0(FPW);
      }
      __builtin_amdgcn_s_barrier();  // B(0)
      tok_offsets(2, tk_a);  // its load precedes stage 0's row half, which B(0) waited for
      slot_bases(ROW_FIRST ? (uint32_t)SLOT : 0u, ROW_FIRST ? 0u : (uint32_t)SLOT);
#pragma unroll
      for (int i = 0; i < TI; ++i) fa[0][i] = read_a(0, i);
#pragma unroll
      for (int j = 0; j < TJ; ++j) fb[0][j] = read_b(0, j);
      // the part of W(0) that belongs to the (absent) last sub-step of stage -1
      __amdgpu_buffer_rsrc_t rs_second = second_rsrc(1);  // W(0)'s second half: stage 1
#pragma unroll
      for (int o = 0; o < TI * NOPS / NGRP; ++o) {
        win_op(0, o, tk_a, rq[3], rq[4], rs_second, rs_second);  // ring positions 3 and 4 (no first-half op)
        __builtin_amdgcn_sched_barrier(0);
      }
      for (int kt = 0; kt < cur.nk; ++kt) {
        const __amdgpu_buffer_rsrc_t rs_first = first_rsrc(kt + 2);
        // Sub-steps 0..2 of stage kt; groups TI..NGRP-1 of W(kt).
#pragma unroll
        for (int ks = 0; ks < GQ; ++ks) {
#pragma unroll
          for (int i = 0; i < TI; ++i) {
            const int q = TI + ks * TI + i;
#pragma unroll
            for (int o = q * NOPS / NGRP; o < (q + 1) * NOPS / NGRP; ++o)
              win_op(kt, o, tk_a, rq[3], rq[4], rs_second, rs_first);  // positions 2kt+3, 2kt+4
            if (ks + 1 < GQ) {
              fa[(ks + 1) & 1][i] = read_a(ks + 1, i);
              if (i < TJ) fb[(ks + 1) & 1][i] = read_b(ks + 1, i);
            } else {
              // The last sub-step's fragments, read in the groups before the
              // last one: the barrier's lgkmcnt(0) then finds them landed.
#pragma unroll
              for (int r = i * NLR / (TI - 1); r < (i + 1) * NLR / (TI - 1) && r < NLR; ++r) {
                if (r < TI) fa[1][r] = read_a(GQ, r);
                else fb[1][r - TI] = read_b(GQ, r - TI);
              }
            }
#pragma unroll
            for (int j = 0; j < TJ; ++j)
              acc[i][j] = mma(fa[ks & 1][i], fb[ks & 1][j], acc[i][j]);
            group_order();
            // Scalar instructions (slot offsets, descriptors, M0) may cross
            // the group boundaries; memory ops keep the issue order that the
            // wait counts rely on.
            __builtin_amdgcn_sched_barrier(0x4);
          }
        }
        if constexpr (NTOK > 0) {
#pragma unroll
          for (int i = 0; i < NTOK; ++i) tk_a[i] = tn[i];  // row_src entries of stage kt+3
          tok_offsets(kt + 3, tk_a);  // their load opened this stage's window
        }
        constexpr int LB = GQ & 1;  // fragment buffer of the last sub-step
        static_assert(LB == 1, "sub-step 0 of the next stage reads into buffer 0");
        // lgkmcnt(0): this wave's reads of stage kt are complete before the
        // barrier lets other waves overwrite their slots.  (After the last
        // stage this barrier, the reads of the stage past it and the ops of
        // the window after it are junk, kept to make every iteration alike.)
        WAIT_VMCNT_LGKM0(FPW);
        __builtin_amdgcn_s_barrier();  // B(kt+1)
        // stage kt+1: first half at position 2kt+2, second half at 2kt+3
        slot_bases(ROW_FIRST ? rq[3] : rq[2], ROW_FIRST ? rq[2] : rq[3]);
        // Last sub-step of stage kt, groups 0..TI-1 of W(kt+1), and the
        // fragments of sub-step 0 of stage kt+1.
        rs_second = second_rsrc(kt + 2);
#pragma unroll
        for (int i = 0; i < TI; ++i) {
#pragma unroll
          for (int o = i * NOPS / NGRP; o < (i + 1) * NOPS / NGRP; ++o)
            win_op(kt + 1, o, tk_a, rq[0], rq[1], rs_second, rs_second);  // positions 2kt+5, 2kt+6
          fa[0][i] = read_a(0, i);
          if (i < TJ) fb[0][i] = read_b(0, i);
#pragma unroll
          for (int j = 0; j < TJ; ++j)
            acc[i][j] = mma(fa[1][i], fb[1][j], acc[i][j]);
          group_order();
          __builtin_amdgcn_sched_barrier(0x4);
        }
        const uint32_t r0 = rq[0], r1 = rq[1];
        rq[0] = rq[2];
        rq[1] = rq[3];
        rq[2] = rq[4];
        rq[3] = r0;
        rq[4] = r1;
      }
  };

  // Wave-local epilogue of the PF modes.  The next tile's first stages are
  // already in flight into ring slots 0-2; each wave writes its own
  // WR x 128 block of the finished tile through a private 16 KB region of
  // slots 3-4 (64 rows of 256 bytes at a time, 16-byte chunks XOR-swizzled
  // by row so that the accumulator-layout writes spread over the banks),
  // reads it back in row order and stores whole 256-byte row pieces, 16
  // bytes per lane.  No workgroup barrier; every store is issued
  // unconditionally (rows and columns outside the output get an offset past
  // the descriptor's extent), so the next tile's first wait can leave
  // exactly these NST stores in flight.
  // Fused accumulation (G1DW, G2DWG with p.accumulate): the destination of
  // a tile's dW and the byte offsets of a lane's 32 pieces of 16 bytes in
  // the order the epilogue stores them (two groups of 16, one per pair of
  // 32-row sub-tiles); `pre` holds their old values, loaded eight pieces
  // ahead of their use: the first eight before the staging writes, then one
  // per stored piece (as fast as loading each group's 16 at its start, with
  // 36 fewer VGPRs; all 32 at the epilogue's start, or before the next
  // tile's prologue, measured 4% and 2% slower).
  constexpr bool ACCM = MODE == G1DW || MODE == G2DWG;
  static_assert(!ACCM || TJ == 4, "accumulating epilogue: two groups of two sub-tiles");
  auto dw_rsrc = [&](const Tile& c, int wd) {
    const int ewr = wd >> 1, ewc = wd & 1;
    if constexpr (MODE == G2DWG) {
      const int o0 = c.ct * BC + ewc * 128;
      const int no = min(128, H - o0);
      return make_rsrc(p.out + (int64_t)c.e * H * I + (int64_t)o0 * I,
                       no > 0 ? (uint32_t)no * (uint32_t)I * 2 : 0u);
    } else {
      const int r0 = c.row0 + ewr * WR;
      const int nr = min(WR, I2 - r0);
      return make_rsrc(p.out + (int64_t)c.e * I2 * H + (int64_t)r0 * H,
                       nr > 0 ? (uint32_t)nr * (uint32_t)H * 2 : 0u);
    }
  };
  auto dw_off = [&](const Tile& c, int ln, int wd, int j0, int it) -> uint32_t {
    const int ewr = wd >> 1, ewc = wd & 1;
    if constexpr (MODE == G2DWG) {
      const int o = it * 8 + (ln >> 3), P = ln & 7;
      const int col = c.row0 + ewr * WR + j0 * 32 + (P ^ ((o >> 1) & 7)) * 8;
      return col < I ? (uint32_t)o * I * 2 + (uint32_t)col * 2 : kOOB;
    } else {
      const int rr = it * 4 + (ln >> 4), P = ln & 15;
      const int col = c.ct * BC + ewc * 128 + (P ^ (rr & 15)) * 8, gr = j0 * 32 + rr;
      return col < H ? (uint32_t)gr * H * 2 + (uint32_t)col * 2 : kOOB;
    }
  };
  u32x4 pre[ACCM ? 32 : 1];
  auto epilogue_pf = [&](const Tile& c) {
    // lane- and wave-derived addresses formed here (opaque to the
    // optimizer, which would otherwise hoist them out of the tile loop)
    int ln = lane, wd = wid;
    asm volatile("" : "+v"(ln), "+s"(wd));
    const int el32 = ln & 31, ehl = ln >> 5, ewr = wd >> 1, ewc = wd & 1;
    lds_char_t* const reg = (lds_char_t*)smem + 3 * SLOT + wd * 16384;
    auto st16 = [&](__amdgpu_buffer_rsrc_t rs, uint32_t off, const u32x4& v) {
      __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, 0, 2);  // non-temporal
    };
    // write accumulator rows j0..j0+nj-1 of this wave into the region
    auto write_rows = [&](int j0, int nj) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        if (jj >= nj) break;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const u32x2 v = {pack_bf2(acc[i][j0 + jj][4 * q + 0], acc[i][j0 + jj][4 * q + 1]),
                             pack_bf2(acc[i][j0 + jj][4 * q + 2], acc[i][j0 + jj][4 * q + 3])};
            uint32_t a;
            if constexpr (SWAP) {
              // [output row o = tile column][64 output columns = tile rows]
              const int o = i * 32 + el32;
              const int ch = 4 * jj + q;
              a = (uint32_t)o * 128 + ((uint32_t)(ch ^ ((o >> 1) & 7)) << 4) + ehl * 8;
            } else {
              const int r = jj * 32 + el32;
              const int ch = 4 * i + q;
              a = (uint32_t)r * 256 + ((uint32_t)(ch ^ (r & 15)) << 4) + ehl * 8;
            }
            *(__attribute__((address_space(3))) u32x2*)(reg + a) = v;
          }
      }
    };
    if constexpr (MODE == G2DXF) {
      // g = d_out[token] . down_proj[e] (fp32) leaves through this wave's
      // 16 KB region one row sub-tile (32 rows x 128 features) at a time,
      // 512-byte rows with 16-byte chunks XOR-swizzled by row, and is read
      // back in row order: 16 lanes per row, 8 features per lane, so every
      // gate/up load and every store moves 256 contiguous bytes per row.
      // Per element: d_act = w * g; act = bf16(bf16(silu(gate)) * up)
      // recomputed exactly as G1F stored it; d_up = bf16(d_act * silu),
      // d_gate = bf16(bf16(d_act * up) * sigmoid'); w * act for the dW
      // GEMM; and the weight-gradient partial sum of g * act over the
      // wave's 128 features (a lane's 8 in order, then a fixed butterfly
      // over the row's 16 lanes), stored per (row, column tile, wave
      // column).  Rows and features outside the output get offsets past
      // the descriptors' extents: loads return 0, stores are dropped.
      constexpr int NIT = 8;  // iterations of 4 rows per row sub-tile
      const int fw = c.ct * BC + ewc * 128;
      const int nr = c.row_end - c.row0;  // >= 1
      const int c8 = (ln & 15) * 8, rq = ln >> 4;
      const bool fok = fw + c8 < I;
      const auto rgu = make_rsrc(p.a1 + (int64_t)c.row0 * I2, (uint32_t)nr * (uint32_t)I2 * 2);
      const auto rdg = make_rsrc(p.out + (int64_t)c.row0 * I2, (uint32_t)nr * (uint32_t)I2 * 2);
      const auto raw = make_rsrc(p.out2 + (int64_t)c.row0 * I, (uint32_t)nr * (uint32_t)I * 2);
      const int n_part = 2 * p.n_ct;
      // Byte offsets of the lane's first row and features; row j*32 + it*4
      // further adds a wave-uniform step.  lim: the lane's rows are valid
      // while that step's row count stays below it (never, for features
      // past I).
      const int r0l = ewr * WR + rq;
      const int lim = fok ? nr - r0l : INT32_MIN;
      const uint32_t bg = (uint32_t)r0l * (uint32_t)(I2 * 2) + (uint32_t)(fw + c8) * 2;
      const uint32_t ba = (uint32_t)r0l * (uint32_t)(I * 2) + (uint32_t)(fw + c8) * 2;
      auto og = [&](int j, int it) -> uint32_t {  // gate bytes of (row, lane's features)
        const int d = j * 32 + it * 4;
        return d < lim ? bg + (uint32_t)d * (uint32_t)(I2 * 2) : kOOB;
      };
      auto oa = [&](int j, int it) -> uint32_t {
        const int d = j * 32 + it * 4;
        return d < lim ? ba + (uint32_t)d * (uint32_t)(I * 2) : kOOB;
      };
      // gate/up of iteration n = j*NIT + it are loaded PD iterations ahead
      // (HBM latency: one iteration's arithmetic is ~1 k cycles)
      constexpr int PD = 8, NN = TJ * NIT;
      u32x4 gl[PD], ul[PD];
      auto load = [&](int n) {
        const uint32_t o = og(n / NIT, n % NIT);
        gl[n % PD] = __builtin_amdgcn_raw_buffer_load_b128(rgu, o, 0, 2);
        ul[n % PD] = __builtin_amdgcn_raw_buffer_load_b128(rgu, o + (uint32_t)I * 2, 0, 2);  // kOOB stays out
      };
#pragma unroll
      for (int n = 0; n < PD && n < NN; ++n) load(n);
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        // accumulator rows of sub-tile j -> region, fp32
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int ch = 8 * i + 2 * q + ehl;
            *(__attribute__((address_space(3))) f32x4*)(reg + el32 * 512 + ((ch ^ el32) << 4)) =
                f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                      acc[i][j][4 * q + 3]};
          }
        // the routing weights and row_src of the lane's eight rows of this
        // sub-tile, from the lanes that hold them (fetched together)
        uint32_t wq[NIT];
        int sq[NIT];
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
          wq[it] = (uint32_t)__shfl((int)cwr[j], it * 4 + rq, 64);
          sq[it] = __shfl(csrc[j], it * 4 + rq, 64);
        }
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
          const int n = j * NIT + it, b = n % PD;
          const int r = it * 4 + rq;  // row within the sub-tile
          const int lc = c8 >> 2;     // logical chunk of the lane's first 4 features
          const f32x4 g0 = *(const __attribute__((address_space(3))) f32x4*)(
              reg + r * 512 + ((lc ^ r) << 4));
          const f32x4 g1 = *(const __attribute__((address_space(3))) f32x4*)(
              reg + r * 512 + (((lc + 1) ^ r) << 4));
          const float wgt = __uint_as_float(p.rw_bf16 ? wq[it] << 16 : wq[it]);
          float gq[8], g[8], u[8], sg[8], t[8], sl[8], a[8], da[8], ds[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            gq[e] = e < 4 ? g0[e] : g1[e - 4];
            g[e] = (e & 1) ? bf_hi(gl[b][e >> 1]) : bf_lo(gl[b][e >> 1]);
            u[e] = (e & 1) ? bf_hi(ul[b][e >> 1]) : bf_lo(ul[b][e >> 1]);
            sg[e] = fast_sigmoid(g[e]);
            t[e] = g[e] * sg[e];
          }
          // bf16 roundings two at a time (one v_cvt_pk_bf16_f32 per pair)
          u32x4 dgv, duv, awv;
          float dot = 0.f;
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const int e0 = 2 * w, e1 = 2 * w + 1;
            const uint32_t slp = pack_bf2(t[e0], t[e1]);
            sl[e0] = bf_lo(slp);
            sl[e1] = bf_hi(slp);
            const uint32_t ap = pack_bf2(sl[e0] * u[e0], sl[e1] * u[e1]);
            a[e0] = bf_lo(ap);
            a[e1] = bf_hi(ap);
            da[e0] = wgt * gq[e0];
            da[e1] = wgt * gq[e1];
            const uint32_t dsp = pack_bf2(da[e0] * u[e0], da[e1] * u[e1]);
            ds[e0] = bf_lo(dsp);
            ds[e1] = bf_hi(dsp);
            // sigmoid'(g) (1 + g) form: sg (1 + g (1 - sg)) = sg + t (1 - sg)
            dgv[w] = pack_bf2(ds[e0] * fmaf(t[e0], 1.f - sg[e0], sg[e0]),
                              ds[e1] * fmaf(t[e1], 1.f - sg[e1], sg[e1]));
            duv[w] = pack_bf2(da[e0] * sl[e0], da[e1] * sl[e1]);
            awv[w] = pack_bf2(wgt * a[e0], wgt * a[e1]);
            dot = fmaf(gq[e0], a[e0], dot);
            dot = fmaf(gq[e1], a[e1], dot);
          }
          if (n + PD < NN) load(n + PD);
          const uint32_t o = og(j, it), oaw = oa(j, it);
          __builtin_amdgcn_raw_buffer_store_b128(dgv, rdg, o, 0, 2);
          __builtin_amdgcn_raw_buffer_store_b128(duv, rdg, o + (uint32_t)I * 2, 0, 2);
          __builtin_amdgcn_raw_buffer_store_b128(awv, raw, oaw, 0, 2);
          // the row's partial over the wave's 128 features
          const float tot = group_sum<16>(fok ? dot : 0.f);
          if ((ln & 15) == 0 && j * 32 + it * 4 < nr - r0l)
            p.dw_part[(int64_t)sq[it] * n_part + c.ct * 2 + ewc] = tot;
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    } else if constexpr (MODE == G1F) {
      // tile columns of this wave: [gate 64 | up 64] of features fb..fb+63
      const int fb = c.ct * 128 + ewc * 64;
      const int r0 = c.row0 + ewr * WR;
      const int nr = min(WR, c.row_end - r0);
      const uint32_t rows = nr > 0 ? (uint32_t)nr : 0u;
      const auto ra = make_rsrc(p.out + (int64_t)r0 * I, rows * (uint32_t)I * 2);
      const auto rg = make_rsrc(p.out2 ? p.out2 + (int64_t)r0 * I2 : p.out,
                                p.out2 ? rows * (uint32_t)I2 * 2 : 0u);
#pragma unroll
      for (int j0 = 0; j0 < TJ; j0 += 2) {
        const int nj = TJ - j0 >= 2 ? 2 : 1;
        write_rows(j0, nj);
#pragma unroll
        for (int it = 0; it < 4 * nj; ++it) {
          const int rr = it * 8 + (ln >> 3), f8 = ln & 7;
          const u32x4 gv = *(const __attribute__((address_space(3))) u32x4*)(
              reg + rr * 256 + ((f8 ^ (rr & 15)) << 4));
          const u32x4 uv = *(const __attribute__((address_space(3))) u32x4*)(
              reg + rr * 256 + (((8 + f8) ^ (rr & 15)) << 4));
          u32x4 av;
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float g0 = bf_lo(gv[w]), g1 = bf_hi(gv[w]);
            const float u0 = bf_lo(uv[w]), u1 = bf_hi(uv[w]);
            av[w] = pack_bf2(round_bf(g0 * fast_sigmoid(g0)) * u0, round_bf(g1 * fast_sigmoid(g1)) * u1);
          }
          const int feat = fb + f8 * 8, gr = j0 * 32 + rr;
          const bool ok = feat < I;
          st16(ra, ok ? (uint32_t)gr * I * 2 + (uint32_t)feat * 2 : kOOB, av);
          st16(rg, ok ? (uint32_t)gr * I2 * 2 + (uint32_t)feat * 2 : kOOB, gv);
          st16(rg, ok ? (uint32_t)gr * I2 * 2 + (uint32_t)(I + feat) * 2 : kOOB, uv);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else if constexpr (SWAP) {
      // G2DWG: output d_down_proj[e] [H][I]; output row = tile column,
      // output column = tile row
      const int o0 = c.ct * BC + ewc * 128;
      const int no = min(128, H - o0);
      const auto rs = make_rsrc(p.out + (int64_t)c.e * H * I + (int64_t)o0 * I,
                                no > 0 ? (uint32_t)no * (uint32_t)I * 2 : 0u);
      // accumulating: the old values (`pre`) are added in the store loop
      auto body = [&](auto acc_t) {
        constexpr bool ACC = decltype(acc_t)::value;
#pragma unroll
        for (int j0 = 0; j0 < TJ; j0 += 2) {
          const int nj = TJ - j0 >= 2 ? 2 : 1;
          if constexpr (ACC) {
            if (j0 == 0) {
#pragma unroll
              for (int k = 0; k < 8; ++k)
                pre[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, dw_off(c, ln, wd, 0, k), 0, 0);
            }
          }
          write_rows(j0, nj);
#pragma unroll
          for (int it = 0; it < 16; ++it) {
            const int o = it * 8 + (ln >> 3), P = ln & 7;
            if constexpr (ACC) {
              const int kn = (j0 >> 1) * 16 + it + 8;
              if (kn < 32)
                pre[kn] = __builtin_amdgcn_raw_buffer_load_b128(rs, dw_off(c, ln, wd, (kn >> 4) * 2, kn & 15), 0, 0);
            }
            u32x4 v = *(const __attribute__((address_space(3))) u32x4*)(reg + o * 128 + P * 16);
            if constexpr (ACC) v = add_bf16x8(pre[(j0 >> 1) * 16 + it], v);
            st16(rs, dw_off(c, ln, wd, j0, it), v);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      if constexpr (MODE == G2DWG) {
        if (p.accumulate) body(std::true_type{});
        else body(std::false_type{});
      } else {
        body(std::false_type{});
      }
    } else {
      // y (G2F), d_xs (G1DX): routed rows x H; the gating linear's d_x (RDX):
      // tokens x H; d_gate_up_proj[e] (G1DW): 2I x H
      int r0, nrows_all;
      const bf16* ob;
      if constexpr (TOKEN || MODE == RDX) {
        r0 = c.row0 + ewr * WR;
        nrows_all = c.row_end;
        ob = p.out;
      } else {
        r0 = c.row0 + ewr * WR;
        nrows_all = I2;
        ob = p.out + (int64_t)c.e * I2 * H;
      }
      const int nr = min(WR, nrows_all - r0);
      const auto rs = make_rsrc(ob + (int64_t)r0 * H, nr > 0 ? (uint32_t)nr * (uint32_t)H * 2 : 0u);
      const int cb = c.ct * BC + ewc * 128;
      // G1DW accumulating: as G2DWG's above
      auto body = [&](auto acc_t) {
        constexpr bool ACC = decltype(acc_t)::value;
#pragma unroll
        for (int j0 = 0; j0 < TJ; j0 += 2) {
          const int nj = TJ - j0 >= 2 ? 2 : 1;
          if constexpr (ACC) {
            if (j0 == 0) {
#pragma unroll
              for (int k = 0; k < 8; ++k)
                pre[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, dw_off(c, ln, wd, 0, k), 0, 0);
            }
          }
          write_rows(j0, nj);
#pragma unroll
          for (int it = 0; it < 8 * nj; ++it) {
            const int rr = it * 4 + (ln >> 4), P = ln & 15;
            if constexpr (ACC) {
              const int kn = (j0 >> 1) * 16 + it + 8;
              if (kn < 32)
                pre[kn] = __builtin_amdgcn_raw_buffer_load_b128(rs, dw_off(c, ln, wd, (kn >> 4) * 2, kn & 15), 0, 0);
            }
            u32x4 v = *(const __attribute__((address_space(3))) u32x4*)(reg + rr * 256 + P * 16);
            const int col = cb + (P ^ (rr & 15)) * 8, gr = j0 * 32 + rr;
            uint32_t off = col < H ? (uint32_t)gr * H * 2 + (uint32_t)col * 2 : kOOB;
            if constexpr (ACC) {
              v = add_bf16x8(pre[(j0 >> 1) * 16 + it], v);
              off = dw_off(c, ln, wd, j0, it);
            }
            st16(rs, off, v);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      if constexpr (MODE == G1DW) {
        if (p.accumulate) body(std::true_type{});
        else body(std::false_type{});
      } else {
        body(std::false_type{});
      }
    }
  };
  // RLTS: the selection counts of this lane's experts (entries e0 .. e0+SV-1
  // of its lane group of 8), summed over every token it routes and flushed
  // to the counts once, after the last tile.
  constexpr int SV = MODE == RLTS ? BR / 8 : 1;
  int scnt[SV];
#pragma unroll
  for (int j = 0; j < SV; ++j) scnt[j] = 0;
  if constexpr (PF) {
    // G2DXF: the rows prepared by the last setup() become the computed
    // tile's, and their routing weights are fetched (in flight under the
    // main loop; first used by the epilogue).
    auto take_rows = [&]() {
      if constexpr (MODE == G2DXF) {
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          csrc[j] = nsrc[j];
          cwr[j] = p.rw_bf16 ? (uint32_t)((const uint16_t*)p.rw)[nsrc[j]]
                             : ((const uint32_t*)p.rw)[nsrc[j]];
        }
      }
    };
    // Token modes (static walk): the {expert, first row, end row} of the
    // next two tiles (ti1, ti2) and, for gathered rows, the row_src entries
    // of the next tile's DMA rows (rs1) are loaded a hand-over ahead, before
    // that hand-over's prologue DMA (so that no wait of the main loop counts
    // them), and the hand-over itself waits on no memory.
    constexpr bool PRE = TOKEN;
    int4 ti1 = make_int4(0, 0, 0, 0), ti2 = ti1;
    int rs1[GROW ? RPW : 1];
    auto ti_load = [&](int tt) -> int4 {
      return tt < t_end ? p.tile_info[tt / p.n_ct] : make_int4(0, 0, 0, 0);
    };
    auto ahead = [&](int tt) {  // rs1 <- tile tt's rows (its info in ti1), ti2 <- the next info
      if (tt < t_end) rows_load(decode(tt, &ti1), rs1);
      ti2 = ti_load(tt + nslot);
    };
    // (a dynamic walk may find no tile at all; every workgroup still
    // reaches the finished-count update below)
    Tile cur = decode(dyn ? max(t, 0) : t);
    if (dyn ? t >= 0 : t < t_end) setup(cur);
    if constexpr (PRE) {
      ti1 = ti_load(t + nslot);
      ahead(t + nslot);
    }
    if ((dyn ? t >= 0 : t < t_end) && cur.nk > 0) prologue();
    if (dyn ? t >= 0 : t < t_end) take_rows();
    bool first = true;
    while (dyn ? t >= 0 : t < t_end) {
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
      if (cur.nk > 0) mainloop(cur, !first);
      // The ring is idle: the stages past the last one have landed (empty
      // descriptors) and every wave has finished its LDS reads.
      WAIT_VMCNT_LGKM0(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      const int tn_next = dyn ? claim() : t + nslot;
      const bool more = dyn ? tn_next >= 0 : tn_next < t_end;
      Tile nxt = cur;
      if (more) {
        if constexpr (PRE) {
          nxt = decode(tn_next, &ti1);
          setup(nxt, rs1);
          ti1 = ti2;
          ahead(tn_next + nslot);
        } else {
          nxt = decode(tn_next);
          setup(nxt);
        }
      }
      if (more && nxt.nk > 0) prologue();
      epilogue_pf(cur);
      if (!more) break;
      take_rows();
      cur = nxt;
      t = tn_next;
      first = false;
    }
  } else {
  for (; dyn ? t >= 0 : t < t_end; t = dyn ? claim() : t + nslot) {
    const Tile cur = decode(t);
    setup(cur);
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // --------------------------------------------------------- main loop
    // Ring position h holds the first half (h = 2s: the column half, or the
    // row half where ROW_FIRST) or the second half (h = 2s+1) of stage s, in
    // slot h % 5.  Barrier B(s) comes after each wave has waited until only
    // the last-issued first half (stage s+1) may still be in flight: stage
    // s has landed everywhere, and every wave
    // has finished reading stage s-1.  B(s+1) sits before the last k
    // sub-step of stage s (whose fragments are already in registers), so
    // that the first fragments of stage s+1 are read while those MFMAs run.
    // Window W(s), the memory ops issued after B(s), is: the row_src
    // entries of stage s+3 (G1DW), the DMA of the second half of stage s+1
    // and of the first half of stage s+2 (into stage s-1's slots), in this
    // order, spread over 16 MFMA groups (the last sub-step of stage s-1 and
    // the first three of stage s): issued in one burst they back up the
    // texture pipe and stall MFMA issue.  Stages past the last one are
    // still issued, with empty descriptors (zeros, no memory access), to
    // keep the wait counts exact.
    if (cur.nk > 0) {
      prologue();
      mainloop(cur, false);
    }

    // --------------------------------------------------------- epilogue
    WAIT_VMCNT(0);    // no LDS DMA may still be landing in the stages
    if constexpr (MODE == RLTS) {
      // The DeepSeek router fused into the gating linear.  The fp32 logits
      // of BC tokens x BR experts are staged as [token][expert] (rows of
      // BR + 4 floats); 8 lanes per token then take sigmoid scores, rank
      // keys of the biased scores and the selection (router_group.h) --
      // the arithmetic of router_linear with fp32 logits followed by
      // router_sigmoid_topk, bit for bit -- and write the scores, the
      // top-K weights and ids, and (if asked) the logits.
      constexpr int G = 8, V = SV, TPP = NTHR / G, FROW = BR + 4;
      __syncthreads();  // every wave is done reading the k-stages
      float* const stf = (float*)smem;
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int tokl = wc * 128 + i * 32 + l32;
            const int el = wr * WR + j * 32 + 8 * q + 4 * hl;
            *(f32x4*)(stf + tokl * FROW + el) =
                f32x4{acc[i][j][4 * q + 0], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                      acc[i][j][4 * q + 3]};
          }
      __syncthreads();
      const int g = tid & (G - 1), e0 = g * V;
      const int E = p.E, K = p.topk;
      float bv[V];
      int grp[V];
      const int eg = p.ngroups > 0 ? E / p.ngroups : 1;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int e = e0 + j;
        bv[j] = (p.bias && e < E) ? p.bias[e] : 0.f;
        grp[j] = e < E ? e / eg : -1;
      }
      for (int rr = tid / G; rr < BC; rr += TPP) {
        const int64_t t = (int64_t)cur.ct * BC + rr;
        const bool tok = t < p.T;
        float lg[V], sc[V];
        uint64_t key[V];
#pragma unroll
        for (int q = 0; q < V / 4; ++q) {
          const f32x4 a = *(const f32x4*)(stf + rr * FROW + e0 + 4 * q);
#pragma unroll
          for (int h = 0; h < 4; ++h) lg[4 * q + h] = a[h];
        }
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const int e = e0 + j;
          sc[j] = e < E ? dsk_score(lg[j], 0) : 0.f;
          key[j] = e < E ? rank_key(sc[j] + bv[j], e) : 0ull;
        }
        float my_w;
        int my_e;
        group_sigmoid_topk<G, V>(sc, key, grp, g, K, p.ngroups, p.gtopk, p.renorm, p.scaling, 0,
                                 tok && p.tpe != nullptr, scnt, my_w, my_e);
        if (tok) {
#pragma unroll
          for (int q = 0; q < V / 4; ++q)
            if (e0 + 4 * q < E) {
              *(f32x4*)(p.probs + t * E + e0 + 4 * q) =
                  f32x4{sc[4 * q], sc[4 * q + 1], sc[4 * q + 2], sc[4 * q + 3]};
              if (p.out_f32)
                *(f32x4*)(p.out_f32 + t * E + e0 + 4 * q) =
                    f32x4{lg[4 * q], lg[4 * q + 1], lg[4 * q + 2], lg[4 * q + 3]};
            }
          if (g < K) {
            if (p.w_bf16) ((bf16*)p.topk_w)[t * K + g] = f2bf(my_w);
            else p.topk_w[t * K + g] = my_w;
            p.topk_idx[t * K + g] = my_e;
          }
        }
      }
      __syncthreads();  // staging reads done before the next tile's stages land
      continue;
    }
    if constexpr (MODE == RLT) {
      if (p.out_f32) {
        // fp32 logits: with the operands swapped each lane holds 4
        // consecutive experts of one token, stored as 16 bytes.
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
          for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int e = cur.row0 + wr * WR + j * 32 + 8 * q + 4 * hl;
              const int64_t t = (int64_t)cur.ct * BC + wc * 128 + i * 32 + l32;
              if (t < p.T && e < cur.row_end) {
                const f32x4 v = {acc[i][j][4 * q + 0], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                 acc[i][j][4 * q + 3]};
                *(f32x4*)(p.out_f32 + t * p.E + e) = v;
              }
            }
        __syncthreads();  // every wave is done reading the k-stages
        continue;
      }
    }
    if constexpr (MODE == RL || MODE == RDW) {
      if (p.out_f32) {
        // fp32 output (RL's logits, RDW's partials): each lane stores its
        // accumulators' 4 consecutive columns (16 bytes) directly; these
        // outputs are small (T x E, chunks x E x H).
        const int nrows = MODE == RL ? cur.row_end : p.E;
        const int ld = MODE == RL ? p.E : H;
        float* const ob = MODE == RL ? p.out_f32 : p.out_f32 + (int64_t)cur.e * p.E * H;
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
          for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int r = cur.row0 + wr * WR + j * 32 + l32;
              const int col = cur.ct * BC + wc * 128 + i * 32 + 8 * q + 4 * hl;
              if (r < nrows && col < ld) {
                const f32x4 v = {acc[i][j][4 * q + 0], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                 acc[i][j][4 * q + 3]};
                *(f32x4*)(ob + (int64_t)r * ld + col) = v;
              }
            }
        __syncthreads();  // every wave is done reading the k-stages
        continue;
      }
    }
    __syncthreads();  // every wave is done reading the k-stages
    bf16* stg = smem;  // [BR][SROW] bf16 staging tile
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          u32x2 v = {pack_bf2(acc[i][j][4 * q + 0], acc[i][j][4 * q + 1]),
                     pack_bf2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3])};
          if constexpr (SWAP) {
            // four consecutive tile rows of one column: staged transposed,
            // [column][row], so the store below writes C^T row by row
            const int col = wc * 128 + i * 32 + l32;
            const int row = wr * WR + j * 32 + 8 * q + 4 * hl;
            *(u32x2*)(stg + col * SROW + row) = v;
          } else {
            const int row = wr * WR + j * 32 + l32;
            const int col = wc * 128 + i * 32 + 8 * q + 4 * hl;
            *(u32x2*)(stg + row * SROW + col) = v;
          }
        }
    __syncthreads();
    if constexpr (MODE == G1F) {
      // 128 output features per tile; 16 lanes x 8 features per row, in
      // batches of RB rows (LDS reads first, then math and stores).
      const int fl = (tid & 15) * 8;
      const int scol = (fl >> 6) * 128 + (fl & 63);  // gate column in the staging tile
      const int f = cur.ct * 128 + fl;
      const bool fok = f < I;
      constexpr int RPT = BR / (NTHR / 16);  // rows per thread
      constexpr int RB = RPT < 8 ? RPT : 8, NB = RPT / RB;
      static_assert(NB * RB * (NTHR / 16) == BR, "epilogue batches");
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        u32x4 gv[RB], uv[RB];
#pragma unroll
        for (int q = 0; q < RB; ++q) {
          const int row = (tid >> 4) + (b * RB + q) * (NTHR / 16);
          gv[q] = *(const u32x4*)(stg + row * SROW + scol);
          uv[q] = *(const u32x4*)(stg + row * SROW + scol + 64);
        }
#pragma unroll
        for (int q = 0; q < RB; ++q) {
          const int row = (tid >> 4) + (b * RB + q) * (NTHR / 16);
          const int r = cur.row0 + row;
          u32x4 av;
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float g0 = bf_lo(gv[q][w]), g1 = bf_hi(gv[q][w]);
            const float u0 = bf_lo(uv[q][w]), u1 = bf_hi(uv[q][w]);
            av[w] = pack_bf2(round_bf(g0 * fast_sigmoid(g0)) * u0, round_bf(g1 * fast_sigmoid(g1)) * u1);
          }
          if (r < cur.row_end && fok) {
            __builtin_nontemporal_store(av, (u32x4*)(p.out + (int64_t)r * I + f));
            if (p.out2) {
              __builtin_nontemporal_store(gv[q], (u32x4*)(p.out2 + (int64_t)r * I2 + f));
              __builtin_nontemporal_store(uv[q], (u32x4*)(p.out2 + (int64_t)r * I2 + I + f));
            }
          }
        }
      }
    } else if constexpr (DOWN_DX) {
      // G2DX (the unfused form; G2DXF has its own epilogue): d_act tile
      // (bf16) -> d_gate, d_up with gate/up read back from gate_up.
      // Each thread owns NB batches of RB rows; the gate/up loads of batch
      // b+1 are issued before batch b is computed and stored, so loads never
      // queue behind this thread's stores.  Loads are clamped in bounds
      // (rows past the tile's end re-read its last row) and only the stores
      // are predicated.
      constexpr int RB = 8, NB = BR / (RB * (NTHR / 32));
      const int c0 = (tid & 31) * 8;
      const int f = cur.ct * BC + c0;
      const bool fok = f < I;
      const int fl = fok ? f : 0;
      const bf16* gsrc = p.a1 + fl;
      u32x4 gv[2][RB], uv[2][RB];
      auto load_batch = [&](int b, u32x4 (&g)[RB], u32x4 (&u)[RB]) {
#pragma unroll
        for (int q = 0; q < RB; ++q) {
          const int r = min(cur.row0 + (tid >> 5) + (b * RB + q) * (NTHR / 32), cur.row_end - 1);
          g[q] = __builtin_nontemporal_load((const u32x4*)(gsrc + (int64_t)r * I2));
          u[q] = __builtin_nontemporal_load((const u32x4*)(gsrc + (int64_t)r * I2 + I));
        }
      };
      load_batch(0, gv[0], uv[0]);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (b + 1 < NB) load_batch(b + 1, gv[(b + 1) & 1], uv[(b + 1) & 1]);
#pragma unroll
        for (int q = 0; q < RB; ++q) {
          const int row = (tid >> 5) + (b * RB + q) * (NTHR / 32);
          const int r = cur.row0 + row;
          const u32x4 dav = *(const u32x4*)(stg + row * SROW + c0);
          u32x4 dgv, duv;
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            float dg[2], du[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const float da = h ? bf_hi(dav[w]) : bf_lo(dav[w]);
              const float g = h ? bf_hi(gv[b & 1][q][w]) : bf_lo(gv[b & 1][q][w]);
              const float u = h ? bf_hi(uv[b & 1][q][w]) : bf_lo(uv[b & 1][q][w]);
              const float sg = fast_sigmoid(g);
              const float sl = round_bf(g * sg);          // silu(g) as stored in bf16
              const float ds = round_bf(da * u);          // d silu(g)
              du[h] = da * sl;
              dg[h] = ds * (sg * (1.f + g * (1.f - sg)));
            }
            dgv[w] = pack_bf2(dg[0], dg[1]);
            duv[w] = pack_bf2(du[0], du[1]);
          }
          if (r < cur.row_end && fok) {
            __builtin_nontemporal_store(dgv, (u32x4*)(p.out + (int64_t)r * I2 + f));
            __builtin_nontemporal_store(duv, (u32x4*)(p.out + (int64_t)r * I2 + I + f));
          }
        }
      }
    } else if constexpr (MODE == RLTK) {
      // The softmax router fused into the gating linear.  The staging tile
      // holds the bf16 logits of BC tokens x BR experts ([token][expert]);
      // G lanes per token run the softmax router's top-K core
      // (router_group.h) on them -- the arithmetic of router_linear with
      // bf16 logits followed by router_softmax_topk, bit for bit -- and
      // write probs, the top-K weights and ids, and (if asked) the logits.
      constexpr int G = BR == 128 ? 8 : 16, V = 16, TPP = NTHR / G;
      const int g = tid & (G - 1), e0 = g * V;
      const int E = p.E, K = p.topk;
      const bool has_off = p.offset != nullptr;
      float off[V];
#pragma unroll
      for (int j = 0; j < V; ++j) off[j] = (has_off && e0 + j < E) ? p.offset[e0 + j] : 0.f;
      for (int rr = tid / G; rr < BC; rr += TPP) {
        const int64_t t = (int64_t)cur.ct * BC + rr;
        const bool tok = t < p.T;
        u32x2 raw[V / 4];
#pragma unroll
        for (int q = 0; q < V / 4; ++q) raw[q] = *(const u32x2*)(stg + rr * SROW + e0 + 4 * q);
        float v[V], m, s, pr[V], my_w;
        int my_e;
        if (!has_off) {
          // bf16 values: 32-bit keys (value bits and index), as the router
          // kernel uses for bf16 logits without an offset.
          uint32_t key[V];
#pragma unroll
          for (int j = 0; j < V; ++j) {
            const int e = e0 + j;
            const uint32_t bits = (raw[j >> 2][(j >> 1) & 1] >> (16 * (j & 1))) & 0xffffu;
            v[j] = e < E ? __uint_as_float(bits << 16) : -INFINITY;
            key[j] = e < E ? rank_key16(bits, e) : 0u;
          }
          group_softmax<G, V>(v, key, e0, E, pr, m, s);
          group_topk<G, V>(key, m, 1.f / s, g, K, p.renorm, my_w, my_e);
        } else {
          uint64_t key[V];
#pragma unroll
          for (int j = 0; j < V; ++j) {
            const int e = e0 + j;
            const uint32_t bits = (raw[j >> 2][(j >> 1) & 1] >> (16 * (j & 1))) & 0xffffu;
            v[j] = e < E ? __uint_as_float(bits << 16) + off[j] : -INFINITY;
            key[j] = e < E ? rank_key(v[j], e) : 0ull;
          }
          group_softmax<G, V>(v, key, e0, E, pr, m, s);
          group_topk<G, V>(key, m, 1.f / s, g, K, p.renorm, my_w, my_e);
        }
        const float rs = 1.f / s;
        if (tok) {
#pragma unroll
          for (int q = 0; q < V / 4; ++q)
            if (e0 + 4 * q < E)
              *(f32x4*)(p.probs + t * E + e0 + 4 * q) =
                  f32x4{pr[4 * q] * rs, pr[4 * q + 1] * rs, pr[4 * q + 2] * rs, pr[4 * q + 3] * rs};
          if (g < K) {
            p.topk_w[t * K + g] = my_w;
            p.topk_idx[t * K + g] = my_e;
          }
          if (p.out) {
#pragma unroll
            for (int q = 0; q < V / 4; ++q)
              if (e0 + 4 * q < E) *(u32x2*)(p.out + t * E + e0 + 4 * q) = raw[q];
          }
        }
      }
    } else if constexpr (MODE == RLT) {
      // bf16 logits from the transposed staging: BC token rows of BR
      // experts; BR/8 lanes per row, 16 bytes each.
      constexpr int LPR = BR / 8, RPP = NTHR / LPR;
      const int c0 = (tid % LPR) * 8;
      const int e = cur.row0 + c0;
      for (int rr = tid / LPR; rr < BC; rr += RPP) {
        const int64_t t = (int64_t)cur.ct * BC + rr;
        if (t < p.T && e < p.E)
          __builtin_nontemporal_store(*(const u32x4*)(stg + rr * SROW + c0),
                                      (u32x4*)(p.out + t * p.E + e));
      }
    } else {
      // Plain bf16 tile: y (G2F), d_xs (G1DX), d_down_proj (G2DW, G2DWG
      // from its transposed staging), d_gate_up_proj (G1DW).
      const int c0 = (tid & 31) * 8;
      const int f = (SWAP ? cur.row0 : cur.ct * BC) + c0;
      int nrows, ld;
      bf16* obase;
      if constexpr (TOKEN) {
        nrows = cur.row_end;
        ld = H;
        obase = p.out;
      } else if constexpr (DENSE) {
        nrows = TRL ? (int)p.T : cur.row_end;  // RLT: rows of the stored tile are tokens
        ld = (MODE == RL || TRL) ? p.E : H;
        obase = p.out;
      } else {
        constexpr bool DOWN = MODE == G2DW || MODE == G2DWG;
        nrows = DOWN ? H : I2;
        ld = DOWN ? I : H;
        obase = p.out + (int64_t)cur.e * (DOWN ? (int64_t)H * I : (int64_t)I2 * H);
      }
      // Batches of RB rows: all LDS reads of a batch first, then its stores,
      // so the LDS latency is paid once per batch rather than per row.
      constexpr int RPT = BR / (NTHR / 32);  // rows per thread
      constexpr int RB = RPT < 16 ? RPT : 16, NB = RPT / RB;
      static_assert(NB * RB * (NTHR / 32) == BR, "epilogue batches");
      const bool fok = f < ld;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        u32x4 v[RB];
#pragma unroll
        for (int q = 0; q < RB; ++q) {
          const int row = (tid >> 5) + (b * RB + q) * (NTHR / 32);
          v[q] = *(const u32x4*)(stg + row * SROW + c0);
        }
#pragma unroll
        for (int q = 0; q < RB; ++q) {
          const int row = (tid >> 5) + (b * RB + q) * (NTHR / 32);
          const int r = (SWAP ? cur.ct * BC : cur.row0) + row;
          if (r < nrows && fok) __builtin_nontemporal_store(v[q], (u32x4*)(obase + (int64_t)r * ld + f));
        }
      }
    }
    __syncthreads();  // staging reads done before the next tile's stages land
  }
  }
  if constexpr (MODE == RLTS) {
    // Selection counts: the lanes' counts summed per expert in LDS (free:
    // the last tile ended with a barrier), then one atomic add per expert.
    if (p.tpe) {
      int* const hist = (int*)smem;
      for (int e = tid; e < p.E; e += NTHR) hist[e] = 0;
      __syncthreads();
      const int e0 = (tid & 7) * SV;
#pragma unroll
      for (int j = 0; j < SV; ++j)
        if (scnt[j] && e0 + j < p.E) atomicAdd(&hist[e0 + j], scnt[j]);
      __syncthreads();
      for (int e = tid; e < p.E; e += NTHR)
        if (hist[e]) atomicAdd(&p.tpe[e], (float)hist[e]);
    }
  }
  if (dyn && tid == 0) {
    // The last workgroup to finish resets the counters for the next launch.
    const int d = __hip_atomic_fetch_add(p.queue + 8, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (d == (int)gridDim.x - 1)
      for (int k = 0; k < 9; ++k) __hip_atomic_store(p.queue + k, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

void set_topk(GemmArgs& a, int top_k) {
  a.topk = top_k;
  int sh = 0;
  while ((1 << sh) < top_k) ++sh;
  a.tok_shift = 31 + sh;
  a.tok_mul = (uint32_t)((((uint64_t)1 << (31 + sh)) + (uint64_t)top_k - 1) / (uint64_t)top_k);
}

// Per-device CU count, filled on first use; atomics because host threads
// may launch on the same device concurrently (they store the same value).
std::atomic<int> g_num_cu[64];

int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = g_num_cu[dev].load(std::memory_order_relaxed);
  if (!n) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_num_cu[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

template <int MODE, int BR>
int launch(const GemmArgs& a, int max_tiles, hipStream_t st) {
  constexpr size_t stages = (size_t)NSLOT * SLOT;
  // staging tile of the non-PF epilogues ([BC][SROW] when transposed)
  constexpr size_t staging =
      MODE == RLTS ? (size_t)BC * (BR + 4) * sizeof(float)  // fp32 logits [token][expert]
                   : (size_t)((MODE == G2DWG || MODE == RLT || MODE == RLTK) ? BC : BR) * SROW *
                         sizeof(bf16);
  const size_t lds = stages > staging ? stages : staging;
  if (max_tiles <= 0) return MOE_OK;
  static std::atomic<int> lds_done[64];
  hipError_t err =
      set_dynamic_lds_once(lds_done, (const void*)grouped_gemm_kernel<MODE, BR>, (int)lds);
  if (err != hipSuccess) {
    set_error("grouped_gemm: hipFuncSetAttribute failed: %s", hipGetErrorString(err));
    return MOE_ERR_HIP;
  }
  // Persistent grid: one workgroup per CU (a multiple of the 8 XCDs), never
  // more workgroups than tiles.
  int grid = num_cus() / 8 * 8;
  const int need = (max_tiles + 7) / 8 * 8;
  if (grid > need) grid = need;
  if (grid < 8) grid = 8;
  grouped_gemm_kernel<MODE, BR><<<grid, kWaves<BR> * 64, lds, st>>>(a);
  return check_launch("grouped_gemm");
}

// Row-tile height for the token-grouped GEMMs from the mean rows per expert.
int pick_br(int64_t S, int E) {
  const int64_t avg = S / (E > 0 ? E : 1);
  if (avg >= 512) return 256;
  if (avg >= 128) return 128;
  return 64;
}

// Launches a token-grouped GEMM.  With at least 512 routed rows per expert
// on average every expert that has rows has enough for 256-row tiles, so the
// host picks them.  Below that the rows per *routed-to* expert decide, which
// only the device knows: the permutation wrote the height of least streamed
// bytes into the plan, all three heights are launched, and the two others
// return at once (one scalar load per workgroup).  Results do not depend on
// the height: every output element is one k-ordered MFMA chain either way.
template <int MODE>
int launch_token(GemmArgs a, int64_t S, int E, int ncols_per_tile_out, int ncols_total,
                 const void* tile_plan, hipStream_t st) {
  const char* pb = (const char*)tile_plan;
  a.n_ct = (ncols_total + ncols_per_tile_out - 1) / ncols_per_tile_out;
  const bool device_choice = pick_br(S, E) != 256;
  a.row_tile = device_choice ? (const int*)(pb + plan_row_tile_offset(E)) : nullptr;
  for (int b = device_choice ? 0 : 2; b < 3; ++b) {
    a.tile_count = (const int*)pb + (size_t)b * (E + 1) + E;
    a.tile_info = (const int4*)(pb + plan_info_offset(S, E, b));
    const int64_t max_tiles = plan_max_tiles(S, E, b) * a.n_ct;
    if (max_tiles > (int64_t)1 << 30) {
      set_error("grouped_gemm: too many tiles");
      return MOE_ERR_UNSUPPORTED;
    }
    const int rc = b == 2 ? launch<MODE, 256>(a, (int)max_tiles, st)
                 : b == 1 ? launch<MODE, 128>(a, (int)max_tiles, st)
                          : launch<MODE, 64>(a, (int)max_tiles, st);
    if (rc != MOE_OK) return rc;
  }
  return MOE_OK;
}
int check_common(int64_t S, int E, int H, int I, int dtype, const char* who) {
  MOE_REQUIRE(dtype == MOE_DTYPE_BF16 || dtype == MOE_DTYPE_F32, MOE_ERR_DTYPE,
              "%s: dtype %d is neither bf16 nor fp32", who, dtype);
  MOE_REQUIRE(dtype == MOE_DTYPE_BF16, MOE_ERR_UNSUPPORTED,
              "%s: bf16 only; fp32 layers run the unfused backward (combine_backward, "
              "gemm_down_backward_dx_dswiglu, gemm_down_backward_dw)", who);
  MOE_REQUIRE(S >= 0 && E >= 1 && H > 0 && I > 0, MOE_ERR_ARG, "%s: bad sizes", who);
  MOE_REQUIRE(H % 64 == 0 && I % 64 == 0, MOE_ERR_ARG,
              "%s: H=%d and I=%d must be multiples of 64", who, H, I);
  // The token-grouped GEMMs address a tile's own rows, the dW GEMMs one
  // expert's rows (limits at their entry points); row_src is read through a
  // descriptor of S*4 bytes.
  MOE_REQUIRE(S < ((int64_t)1 << 29), MOE_ERR_UNSUPPORTED, "%s: S=%lld routed rows, limit 2^29",
              who, (long long)S);
  MOE_REQUIRE((int64_t)E * H * 2 * I * 2 < ((int64_t)1 << 40), MOE_ERR_ARG, "%s: weights too large",
              who);
  return MOE_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace
}  // namespace moe

using namespace moe;

#define MOE_ALIGNED(ptr, who) \
  MOE_REQUIRE(aligned16(ptr), MOE_ERR_ALIGN, "%s: pointer %s not 16-byte aligned", who, #ptr)

extern "C" int moe_amd_gemm_gate_up_swiglu(const void* hidden_states, const int32_t* row_src,
                                           int top_k, const int32_t* offsets,
                                           const void* tile_plan, const void* gate_up_proj,
                                           int64_t T, int64_t S, int E, int H, int I, int dtype,
                                           void* gate_up_out, void* act_out, void* stream) {
  const char* who = "gemm_gate_up_swiglu";
  if (dtype == MOE_DTYPE_F32)
    return f32_gate_up_swiglu((const float*)hidden_states, row_src, top_k, offsets, tile_plan,
                              (const float*)gate_up_proj, T, S, E, H, I, (float*)gate_up_out,
                              (float*)act_out, (hipStream_t)stream);
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(top_k >= 1 && S == T * top_k, MOE_ERR_ARG, "%s: S != T*top_k", who);
  MOE_REQUIRE(T * (int64_t)H * 2 < ((int64_t)1 << 31), MOE_ERR_UNSUPPORTED, "%s: T*H too large",
              who);
  MOE_REQUIRE(offsets && tile_plan && gate_up_proj && (S == 0 || (hidden_states && row_src && act_out)),
              MOE_ERR_ARG, "%s: null pointer", who);
  MOE_ALIGNED(hidden_states, who);
  MOE_ALIGNED(gate_up_proj, who);
  MOE_ALIGNED(act_out, who);
  if (gate_up_out) MOE_ALIGNED(gate_up_out, who);
  if (S == 0) return MOE_OK;
  GemmArgs a{};
  a.x = (const bf16*)hidden_states;
  a.w = (const bf16*)gate_up_proj;
  a.row_src = row_src;
  a.offsets = offsets;
  a.out = (bf16*)act_out;
  a.out2 = (bf16*)gate_up_out;
  a.T = T; a.S = S; a.E = E; a.H = H; a.I = I; set_topk(a, top_k);
  return launch_token<G1F>(a, S, E, 128, I, tile_plan, (hipStream_t)stream);
}

extern "C" int moe_amd_gemm_down(const void* act, const int32_t* offsets,
                                 const void* tile_plan, const void* down_proj, int64_t S,
                                 int E, int H, int I, int dtype, void* y_out, void* stream) {
  const char* who = "gemm_down";
  if (dtype == MOE_DTYPE_F32)
    return f32_down((const float*)act, offsets, tile_plan, (const float*)down_proj, S, E, H, I,
                    (float*)y_out, (hipStream_t)stream);
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(offsets && tile_plan && down_proj && (S == 0 || (act && y_out)), MOE_ERR_ARG,
              "%s: null pointer", who);
  MOE_ALIGNED(act, who);
  MOE_ALIGNED(down_proj, who);
  MOE_ALIGNED(y_out, who);
  if (S == 0) return MOE_OK;
  GemmArgs a{};
  a.w = (const bf16*)down_proj;
  a.a0 = (const bf16*)act;
  a.offsets = offsets;
  a.out = (bf16*)y_out;
  a.S = S; a.E = E; a.H = H; a.I = I;
  return launch_token<G2F>(a, S, E, BC, H, tile_plan, (hipStream_t)stream);
}

extern "C" int moe_amd_router_linear(const void* hidden_states, const void* weight, int64_t T,
                                     int E, int H, void* logits, int logits_dtype,
                                     void* stream) {
  const char* who = "router_linear";
  MOE_REQUIRE(T >= 0 && E >= 1 && H > 0, MOE_ERR_ARG, "%s: bad sizes", who);
  MOE_REQUIRE(H % 64 == 0 && E % 8 == 0, MOE_ERR_ARG,
              "%s: H=%d must be a multiple of 64 and E=%d of 8", who, H, E);
  MOE_REQUIRE(logits_dtype == MOE_DTYPE_BF16 || logits_dtype == MOE_DTYPE_F32, MOE_ERR_DTYPE,
              "%s: logits dtype must be bf16 or fp32", who);
  MOE_REQUIRE(weight && (T == 0 || (hidden_states && logits)), MOE_ERR_ARG,
              "%s: null pointer", who);
  MOE_ALIGNED(hidden_states, who);
  MOE_ALIGNED(weight, who);
  MOE_ALIGNED(logits, who);
  // 32-bit byte offsets within one row tile and within the weight.
  MOE_REQUIRE((int64_t)E * H * 2 < ((int64_t)1 << 31), MOE_ERR_UNSUPPORTED,
              "%s: router weight too large", who);
  if (T == 0) return MOE_OK;
  GemmArgs a{};
  a.w = (const bf16*)weight;
  a.a0 = (const bf16*)hidden_states;
  if (logits_dtype == MOE_DTYPE_F32) a.out_f32 = (float*)logits;
  else a.out = (bf16*)logits;
  a.T = T; a.E = E; a.H = H; a.I = 64;
  if (E <= 256 && T * (int64_t)H * 2 < ((int64_t)1 << 31)) {
    // Transposed (RLT): experts as rows, no padding columns for E < 256.
    a.x = (const bf16*)hidden_states;
    a.a0 = (const bf16*)weight;
    a.n_ct = (int)((T + BC - 1) / BC);
    a.n_rt = 1;
    MOE_REQUIRE(a.n_ct < (1 << 30), MOE_ERR_UNSUPPORTED, "%s: too many tiles", who);
    a.n_tiles = a.n_ct;
    if (E <= 128) return launch<RLT, 128>(a, a.n_tiles, (hipStream_t)stream);
    return launch<RLT, 256>(a, a.n_tiles, (hipStream_t)stream);
  }
  a.n_ct = (E + BC - 1) / BC;
  a.n_rt = (int)((T + 255) / 256);
  const int64_t n_tiles = (int64_t)a.n_rt * a.n_ct;
  MOE_REQUIRE(n_tiles < ((int64_t)1 << 30), MOE_ERR_UNSUPPORTED, "%s: too many tiles", who);
  a.n_tiles = (int)n_tiles;
  return launch<RL, 256>(a, a.n_tiles, (hipStream_t)stream);
}

extern "C" int moe_amd_router_linear_softmax_topk(const void* hidden_states, const void* weight,
                                                  int64_t T, int E, int H,
                                                  const float* logit_offset, int K,
                                                  int renormalize, float* probs,
                                                  float* topk_weights, int64_t* topk_index,
                                                  void* logits, void* stream) {
  const char* who = "router_linear_softmax_topk";
  MOE_REQUIRE(T >= 0 && E >= 1 && H > 0 && K >= 1 && K <= E, MOE_ERR_ARG, "%s: bad sizes", who);
  MOE_REQUIRE(H % 64 == 0 && E % 8 == 0, MOE_ERR_ARG,
              "%s: H=%d must be a multiple of 64 and E=%d of 8", who, H, E);
  // The fused epilogue runs the router's group top-K with 16 experts per
  // lane: 8 lanes per token for E in (64, 128] and K <= 8, 16 lanes for E
  // in (128, 256] and K <= 16 (the router kernel's own shapes there).
  const bool g8 = E > 64 && E <= 128 && K <= 8, g16 = E > 128 && E <= 256 && K <= 16;
  MOE_REQUIRE(g8 || g16, MOE_ERR_UNSUPPORTED,
              "%s: E=%d, K=%d outside the fused shapes (64 < E <= 128 with K <= 8, 128 < E <= "
              "256 with K <= 16); use moe_amd_router_linear + moe_amd_router_softmax_topk", who,
              E, K);
  MOE_REQUIRE(weight && (T == 0 || (hidden_states && probs && topk_weights && topk_index)),
              MOE_ERR_ARG, "%s: null pointer", who);
  MOE_ALIGNED(hidden_states, who);
  MOE_ALIGNED(weight, who);
  MOE_ALIGNED(probs, who);
  MOE_REQUIRE(((uintptr_t)logits & 7) == 0, MOE_ERR_ALIGN, "%s: logits not 8-byte aligned", who);
  MOE_REQUIRE(T * (int64_t)H * 2 < ((int64_t)1 << 31) && (int64_t)E * H * 2 < ((int64_t)1 << 31),
              MOE_ERR_UNSUPPORTED, "%s: T*H or E*H too large for 32-bit offsets", who);
  if (T == 0) return MOE_OK;
  GemmArgs a{};
  a.x = (const bf16*)hidden_states;
  a.a0 = (const bf16*)weight;
  a.out = (bf16*)logits;
  a.probs = probs;
  a.topk_w = topk_weights;
  a.topk_idx = topk_index;
  a.offset = logit_offset;
  a.renorm = renormalize;
  a.topk = K;
  a.T = T; a.E = E; a.H = H; a.I = 64;
  a.n_ct = (int)((T + BC - 1) / BC);
  a.n_rt = 1;
  MOE_REQUIRE(a.n_ct < (1 << 30), MOE_ERR_UNSUPPORTED, "%s: too many tiles", who);
  a.n_tiles = a.n_ct;
  if (g8) return launch<RLTK, 128>(a, a.n_tiles, (hipStream_t)stream);
  return launch<RLTK, 256>(a, a.n_tiles, (hipStream_t)stream);
}

extern "C" int moe_amd_router_linear_sigmoid_topk(
    const void* hidden_states, const void* weight, int64_t T, int E, int H,
    const float* expert_bias, int K, int renormalize, float scaling_factor, int num_groups,
    int group_topk, float* scores, void* topk_weights, int weights_dtype, int64_t* topk_index,
    float* tokens_per_expert, float* logits, void* stream) {
  const char* who = "router_linear_sigmoid_topk";
  MOE_REQUIRE(T >= 0 && E >= 1 && H > 0 && K >= 1 && K <= E, MOE_ERR_ARG, "%s: bad sizes", who);
  MOE_REQUIRE(H % 64 == 0 && E % 8 == 0, MOE_ERR_ARG,
              "%s: H=%d must be a multiple of 64 and E=%d of 8", who, H, E);
  // The fused epilogue ranks with 8 lanes per token (K <= 8) and 8 or 16
  // experts per lane (E <= 128), expert groups one lane's score each.
  MOE_REQUIRE(E <= 128 && K <= 8, MOE_ERR_UNSUPPORTED,
              "%s: E=%d, K=%d outside the fused shapes (E <= 128, K <= 8); use "
              "moe_amd_router_linear + moe_amd_router_sigmoid_topk", who, E, K);
  if (num_groups > 0) {
    MOE_REQUIRE(num_groups <= 8 && E % num_groups == 0 && group_topk >= 1 &&
                    group_topk <= num_groups && K % group_topk == 0 &&
                    (E / num_groups) * group_topk >= K,
                MOE_ERR_ARG, "%s: bad grouping (E=%d K=%d groups=%d group_topk=%d; the fused "
                "form takes at most 8 groups)", who, E, K, num_groups, group_topk);
  }
  MOE_REQUIRE(weights_dtype == MOE_DTYPE_F32 || weights_dtype == MOE_DTYPE_BF16, MOE_ERR_DTYPE,
              "%s: weights dtype %d", who, weights_dtype);
  MOE_REQUIRE(weight && (T == 0 || (hidden_states && scores && topk_weights && topk_index)),
              MOE_ERR_ARG, "%s: null pointer", who);
  MOE_ALIGNED(hidden_states, who);
  MOE_ALIGNED(weight, who);
  MOE_ALIGNED(scores, who);
  MOE_ALIGNED(logits, who);
  MOE_REQUIRE(T * (int64_t)H * 2 < ((int64_t)1 << 31) && (int64_t)E * H * 2 < ((int64_t)1 << 31),
              MOE_ERR_UNSUPPORTED, "%s: T*H or E*H too large for 32-bit offsets", who);
  if (T == 0) return MOE_OK;
  GemmArgs a{};
  a.x = (const bf16*)hidden_states;
  a.a0 = (const bf16*)weight;
  a.probs = scores;
  a.topk_w = (float*)topk_weights;
  a.w_bf16 = weights_dtype == MOE_DTYPE_BF16;
  a.topk_idx = topk_index;
  a.out_f32 = logits;
  a.bias = expert_bias;
  a.scaling = scaling_factor > 0.f ? scaling_factor : 0.f;
  a.ngroups = num_groups > 0 ? num_groups : 0;
  a.gtopk = num_groups > 0 ? group_topk : 0;
  a.tpe = tokens_per_expert;
  a.renorm = renormalize;
  a.topk = K;
  a.T = T; a.E = E; a.H = H; a.I = 64;
  a.n_ct = (int)((T + BC - 1) / BC);
  a.n_rt = 1;
  MOE_REQUIRE(a.n_ct < (1 << 30), MOE_ERR_UNSUPPORTED, "%s: too many tiles", who);
  a.n_tiles = a.n_ct;
  if (E <= 64) return launch<RLTS, 64>(a, a.n_tiles, (hipStream_t)stream);
  return launch<RLTS, 128>(a, a.n_tiles, (hipStream_t)stream);
}

namespace {

// d_x[T][H] = bf16(a[T][K] . w[K][H]) on RDX (the reduction runs over the K
// rows of w).  Shapes checked by the callers.
int rdx_run(const void* a_rows, const void* w, int64_t T, int K, int H, void* d_x,
            hipStream_t st, const char* who) {
  MOE_REQUIRE((int64_t)K * H * 2 < ((int64_t)1 << 31), MOE_ERR_UNSUPPORTED,
              "%s: router weight too large", who);
  if (T == 0) return MOE_OK;
  GemmArgs a{};
  a.w = (const bf16*)w;
  a.a0 = (const bf16*)a_rows;
  a.out = (bf16*)d_x;
  a.T = T; a.E = K; a.H = H; a.I = 64;
  a.n_ct = H / BC;
  a.n_rt = (int)((T + 255) / 256);
  const int64_t n_tiles = (int64_t)a.n_rt * a.n_ct;
  MOE_REQUIRE(n_tiles < ((int64_t)1 << 30), MOE_ERR_UNSUPPORTED, "%s: too many tiles", who);
  a.n_tiles = (int)n_tiles;
  return launch<RDX, 256>(a, a.n_tiles, st);
}

}  // namespace

extern "C" int moe_amd_router_linear_backward_dx(const void* d_logits, const void* weight,
                                                 int64_t T, int E, int H, void* d_x,
                                                 void* stream) {
  const char* who = "router_linear_backward_dx";
  MOE_REQUIRE(T >= 0 && E >= 1 && H > 0, MOE_ERR_ARG, "%s: bad sizes", who);
  MOE_REQUIRE(H % 256 == 0 && E % 8 == 0, MOE_ERR_ARG,
              "%s: H=%d must be a multiple of 256 and E=%d of 8", who, H, E);
  MOE_REQUIRE(weight && (T == 0 || (d_logits && d_x)), MOE_ERR_ARG, "%s: null pointer", who);
  MOE_ALIGNED(d_logits, who);
  MOE_ALIGNED(weight, who);
  MOE_ALIGNED(d_x, who);
  return rdx_run(d_logits, weight, T, E, H, d_x, (hipStream_t)stream, who);
}

namespace {

// Split-K reduction of RDW: d_w[e][h] = bf16(sum_c partial[c][e][h]), fp32
// sums in chunk order (deterministic); 4 elements per thread (n % 4 == 0).
// With halves = 2 each chunk's partial holds 2n values, [hi rows | lo rows]
// of a two-term split (see moe_amd_router_linear_backward_f32), and both
// halves are added, hi then lo, chunk by chunk.  With no chunks it writes
// zeros.
__global__ void reduce_chunks_kernel(const float* __restrict__ part, int nchunk, int64_t n,
                                     int halves, bf16* __restrict__ out) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= n) return;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  // eight partials loaded together, then added in chunk order (the loads of
  // a chunk-at-a-time loop each waited for the previous add)
  const int np = nchunk * halves;
  int c = 0;
  for (; c + 8 <= np; c += 8) {
    f32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = *(const f32x4*)(part + (int64_t)(c + u) * n + i);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += v[u];
  }
  for (; c < np; ++c) acc += *(const f32x4*)(part + (int64_t)c * n + i);
  u32x2 w = {pack_bf2(acc[0], acc[1]), pack_bf2(acc[2], acc[3])};
  *(u32x2*)(out + i) = w;
}

int rdw_chunks(int64_t T, int H, int E) {
  // about one workgroup per CU: chunks x (E / 256) row tiles x (H / 256) column tiles
  const int per_chunk = (H / BC) * ((E + 255) / 256);
  int c = num_cus() / (per_chunk > 0 ? per_chunk : 1);
  if (c < 1) c = 1;
  const int64_t max_c = (T + 63) / 64;  // at least 64 tokens per chunk
  if (c > max_c) c = (int)max_c;
  return c < 1 ? 1 : c;
}

size_t rdw_workspace(int64_t T, int E, int H) {
  if (T <= 0 || E <= 0 || H < BC) return 0;
  return (size_t)rdw_chunks(T, H, E) * (size_t)E * (size_t)H * sizeof(float);
}

// d_w[E/halves][H] = bf16(g[T][E]^T . x[T][H]) (rows of the two halves
// summed when halves = 2) on RDW, split over token chunks into fp32 partials
// in ws, then reduced.  Shapes and workspace checked by the callers.
int rdw_run(const void* g, const void* x, int64_t T, int E, int H, void* ws, int halves,
            void* d_w, hipStream_t st, const char* who) {
  const int64_t n = (int64_t)(E / halves) * H;
  if (T == 0) {  // no tokens: a zero gradient (a fill kernel, safe under graph capture)
    reduce_chunks_kernel<<<(unsigned)((n / 4 + 255) / 256), 256, 0, st>>>(nullptr, 0, n, 1,
                                                                         (bf16*)d_w);
    return check_launch(who);
  }
  const int nchunk = rdw_chunks(T, H, E);
  const int64_t chunk_rows = (T + nchunk - 1) / nchunk;
  // chunk byte extents and the d_logits/x offsets stay below 2^31
  MOE_REQUIRE(chunk_rows * (int64_t)(H > E ? H : E) * 2 < ((int64_t)1 << 31),
              MOE_ERR_UNSUPPORTED, "%s: token chunk too large", who);
  GemmArgs a{};
  a.a0 = (const bf16*)g;
  a.x = (const bf16*)x;
  a.out_f32 = (float*)ws;
  a.T = T; a.E = E; a.H = H; a.I = 64;
  a.chunk_rows = (int)chunk_rows;
  a.n_rt = (E + 255) / 256;
  a.n_ct = H / BC;
  const int64_t n_tiles = (int64_t)nchunk * a.n_rt * a.n_ct;
  MOE_REQUIRE(n_tiles < ((int64_t)1 << 30), MOE_ERR_UNSUPPORTED, "%s: too many tiles", who);
  a.n_tiles = (int)n_tiles;
  int rc = launch<RDW, 256>(a, a.n_tiles, st);
  if (rc) return rc;
  reduce_chunks_kernel<<<(unsigned)((n / 4 + 255) / 256), 256, 0, st>>>(
      (const float*)ws, nchunk, n, halves, (bf16*)d_w);
  return check_launch(who);
}

// Two-term bf16 split of fp32 gradients: row t of out [T][2E] holds
// hi = bf16(g[t]) in columns 0..E-1 and lo = bf16(g[t] - hi) in E..2E-1
// (g - hi is exact in fp32, so |g - hi - lo| <= 2^-18 |g|).  4 elements per
// thread (E % 4 == 0).
__global__ void split_bf16x2_kernel(const float* __restrict__ g, int64_t T, int E,
                                    bf16* __restrict__ out) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= T * E) return;
  const int64_t t = i / E;
  const int e = (int)(i - t * E);
  const f32x4 v = *(const f32x4*)(g + i);
  float hi[4], lo[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    hi[q] = round_bf(v[q]);
    lo[q] = v[q] - hi[q];
  }
  bf16* row = out + t * 2 * E + e;
  *(u32x2*)row = u32x2{pack_bf2(hi[0], hi[1]), pack_bf2(hi[2], hi[3])};
  *(u32x2*)(row + E) = u32x2{pack_bf2(lo[0], lo[1]), pack_bf2(lo[2], lo[3])};
}

// Workspace layout of moe_amd_router_linear_backward_f32: the split
// [T][2E] bf16, the stacked weight [2E][H] bf16, RDW's partials.
struct F32Ws {
  size_t split, wdup, part, total;
};
F32Ws f32_ws(int64_t T, int E, int H) {
  F32Ws w{};
  if (T <= 0 || E <= 0 || H <= 0) return w;
  w.split = align_up((size_t)T * 2 * E * sizeof(bf16), 256);
  w.wdup = align_up((size_t)2 * E * H * sizeof(bf16), 256);
  w.part = align_up(rdw_workspace(T, 2 * E, H), 256);
  w.total = w.split + w.wdup + w.part;
  return w;
}

}  // namespace

extern "C" size_t moe_amd_router_linear_backward_dw_workspace_size(int64_t T, int E, int H) {
  return rdw_workspace(T, E, H);
}

extern "C" int moe_amd_router_linear_backward_dw(const void* d_logits, const void* hidden_states,
                                                 int64_t T, int E, int H, void* workspace,
                                                 size_t workspace_bytes, void* d_weight,
                                                 void* stream) {
  const char* who = "router_linear_backward_dw";
  MOE_REQUIRE(T >= 0 && E >= 1 && H > 0, MOE_ERR_ARG, "%s: bad sizes", who);
  MOE_REQUIRE(H % 256 == 0 && E % 8 == 0, MOE_ERR_ARG,
              "%s: H=%d must be a multiple of 256 and E=%d of 8", who, H, E);
  MOE_REQUIRE(d_weight && (T == 0 || (d_logits && hidden_states)), MOE_ERR_ARG,
              "%s: null pointer", who);
  MOE_ALIGNED(d_logits, who);
  MOE_ALIGNED(hidden_states, who);
  MOE_ALIGNED(d_weight, who);
  if (T > 0) {
    const size_t need = rdw_workspace(T, E, H);
    MOE_REQUIRE(workspace && workspace_bytes >= need, MOE_ERR_WORKSPACE,
                "%s: workspace of %zu bytes needed", who, need);
    MOE_ALIGNED(workspace, who);
  }
  return rdw_run(d_logits, hidden_states, T, E, H, workspace, 1, d_weight, (hipStream_t)stream,
                 who);
}

extern "C" size_t moe_amd_router_linear_backward_f32_workspace_size(int64_t T, int E, int H) {
  return f32_ws(T, E, H).total;
}

extern "C" int moe_amd_router_linear_backward_f32(const float* d_logits, const void* hidden_states,
                                                  const void* weight, int64_t T, int E, int H,
                                                  void* workspace, size_t workspace_bytes,
                                                  void* d_x, void* d_weight, void* stream) {
  const char* who = "router_linear_backward_f32";
  MOE_REQUIRE(T >= 0 && E >= 1 && H > 0, MOE_ERR_ARG, "%s: bad sizes", who);
  MOE_REQUIRE(H % 256 == 0 && E % 32 == 0, MOE_ERR_ARG,
              "%s: H=%d must be a multiple of 256 and E=%d of 32", who, H, E);
  MOE_REQUIRE((!d_x || weight) && (T == 0 || (d_logits && (!d_weight || hidden_states))),
              MOE_ERR_ARG, "%s: null pointer", who);
  MOE_ALIGNED(d_logits, who);
  MOE_ALIGNED(hidden_states, who);
  MOE_ALIGNED(weight, who);
  MOE_ALIGNED(d_x, who);
  MOE_ALIGNED(d_weight, who);
  MOE_REQUIRE((int64_t)2 * E * H * 2 < ((int64_t)1 << 31), MOE_ERR_UNSUPPORTED,
              "%s: router weight too large", who);
  hipStream_t st = (hipStream_t)stream;
  if (T == 0) {
    if (d_weight) return rdw_run(nullptr, nullptr, 0, E, H, nullptr, 1, d_weight, st, who);
    return MOE_OK;
  }
  const F32Ws L = f32_ws(T, E, H);
  MOE_REQUIRE(workspace && workspace_bytes >= L.total, MOE_ERR_WORKSPACE,
              "%s: workspace of %zu bytes needed", who, L.total);
  MOE_ALIGNED(workspace, who);
  MOE_REQUIRE(T * 2 * E < ((int64_t)1 << 40), MOE_ERR_UNSUPPORTED, "%s: too many tokens", who);
  char* base = (char*)workspace;
  bf16* split = (bf16*)base;
  bf16* wdup = (bf16*)(base + L.split);
  void* part = base + L.split + L.wdup;
  const int64_t n4 = T * E / 4;
  split_bf16x2_kernel<<<(unsigned)((n4 + 255) / 256), 256, 0, st>>>(d_logits, T, E, split);
  int rc = check_launch(who);
  if (rc) return rc;
  if (d_x) {
    const size_t wb = (size_t)E * H * sizeof(bf16);
    if (hipMemcpyAsync(wdup, weight, wb, hipMemcpyDeviceToDevice, st) != hipSuccess ||
        hipMemcpyAsync((char*)wdup + wb, weight, wb, hipMemcpyDeviceToDevice, st) != hipSuccess)
      return check_launch(who);
    rc = rdx_run(split, wdup, T, 2 * E, H, d_x, st, who);
    if (rc) return rc;
  }
  if (d_weight) return rdw_run(split, hidden_states, T, 2 * E, H, part, 2, d_weight, st, who);
  return MOE_OK;
}

extern "C" int moe_amd_gemm_down_backward_dx_dswiglu(const void* dy, const int32_t* offsets,
                                                     const void* tile_plan,
                                                     const void* down_proj, const void* gate_up,
                                                     int64_t S, int E, int H, int I, int dtype,
                                                     void* d_gate_up, void* stream) {
  const char* who = "gemm_down_backward_dx_dswiglu";
  if (dtype == MOE_DTYPE_F32)
    return f32_down_dx_dswiglu((const float*)dy, offsets, tile_plan, (const float*)down_proj,
                               (const float*)gate_up, S, E, H, I, (float*)d_gate_up,
                               (hipStream_t)stream);
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(offsets && tile_plan && down_proj && (S == 0 || (dy && gate_up && d_gate_up)),
              MOE_ERR_ARG, "%s: null pointer", who);
  MOE_ALIGNED(dy, who);
  MOE_ALIGNED(down_proj, who);
  MOE_ALIGNED(gate_up, who);
  MOE_ALIGNED(d_gate_up, who);
  if (S == 0) return MOE_OK;
  GemmArgs a{};
  a.w = (const bf16*)down_proj;
  a.a0 = (const bf16*)dy;
  a.a1 = (const bf16*)gate_up;
  a.offsets = offsets;
  a.out = (bf16*)d_gate_up;
  a.S = S; a.E = E; a.H = H; a.I = I;
  return launch_token<G2DX>(a, S, E, BC, I, tile_plan, (hipStream_t)stream);
}

// Two weight-gradient partials per routed row and 256-feature column tile
// (one per wave column of 128 features).
extern "C" int moe_amd_gemm_down_backward_dx_fused_parts(int I) { return 2 * ((I + BC - 1) / BC); }

extern "C" int moe_amd_gemm_down_backward_dx_fused(
    const void* d_out, const int32_t* row_src, int top_k, const int32_t* offsets,
    const void* tile_plan, const void* down_proj, const void* gate_up, const void* topk_weights,
    int weights_dtype, int64_t T, int64_t S, int E, int H, int I, int dtype, void* d_gate_up,
    void* act_w, float* dw_partials, void* stream) {
  const char* who = "gemm_down_backward_dx_fused";
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(top_k >= 1 && S == T * top_k, MOE_ERR_ARG, "%s: S != T*top_k", who);
  MOE_REQUIRE(T * (int64_t)H * 2 < ((int64_t)1 << 31), MOE_ERR_UNSUPPORTED, "%s: T*H too large",
              who);
  MOE_REQUIRE(weights_dtype == MOE_DTYPE_F32 || weights_dtype == MOE_DTYPE_BF16, MOE_ERR_ARG,
              "%s: weights_dtype must be fp32 or bf16", who);
  MOE_REQUIRE(offsets && tile_plan && down_proj &&
                  (S == 0 || (d_out && row_src && gate_up && topk_weights && d_gate_up && act_w &&
                              dw_partials)),
              MOE_ERR_ARG, "%s: null pointer", who);
  MOE_ALIGNED(d_out, who);
  MOE_ALIGNED(down_proj, who);
  MOE_ALIGNED(gate_up, who);
  MOE_ALIGNED(d_gate_up, who);
  MOE_ALIGNED(act_w, who);
  if (S == 0) return MOE_OK;
  GemmArgs a{};
  a.x = (const bf16*)d_out;
  a.w = (const bf16*)down_proj;
  a.a1 = (const bf16*)gate_up;
  a.row_src = row_src;
  a.offsets = offsets;
  a.out = (bf16*)d_gate_up;
  a.out2 = (bf16*)act_w;
  a.rw = topk_weights;
  a.rw_bf16 = weights_dtype == MOE_DTYPE_BF16;
  a.dw_part = dw_partials;
  a.T = T; a.S = S; a.E = E; a.H = H; a.I = I; set_topk(a, top_k);
  return launch_token<G2DXF>(a, S, E, BC, I, tile_plan, (hipStream_t)stream);
}

extern "C" int moe_amd_gemm_gate_up_backward_dx(const void* d_gate_up, const int32_t* offsets,
                                                const void* tile_plan,
                                                const void* gate_up_proj, int64_t S, int E,
                                                int H, int I, int dtype, void* d_xs,
                                                void* stream) {
  const char* who = "gemm_gate_up_backward_dx";
  if (dtype == MOE_DTYPE_F32)
    return f32_gate_up_dx((const float*)d_gate_up, offsets, tile_plan, (const float*)gate_up_proj,
                          S, E, H, I, (float*)d_xs, (hipStream_t)stream);
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(offsets && tile_plan && gate_up_proj && (S == 0 || (d_gate_up && d_xs)), MOE_ERR_ARG,
              "%s: null pointer", who);
  MOE_ALIGNED(d_gate_up, who);
  MOE_ALIGNED(gate_up_proj, who);
  MOE_ALIGNED(d_xs, who);
  if (S == 0) return MOE_OK;
  GemmArgs a{};
  a.w = (const bf16*)gate_up_proj;
  a.a0 = (const bf16*)d_gate_up;
  a.offsets = offsets;
  a.out = (bf16*)d_xs;
  a.S = S; a.E = E; a.H = H; a.I = I;
  return launch_token<G1DX>(a, S, E, BC, H, tile_plan, (hipStream_t)stream);
}

// The dW GEMMs claim tiles from the schedule in the tile plan when one is
// given (balanced under skewed routing); without one they walk statically.
void set_dw_schedule(GemmArgs& a, const void* tile_plan, int64_t S, int E, int which) {
  if (!tile_plan) return;
  int* sched = (int*)((char*)const_cast<void*>(tile_plan) + plan_sched_offset(S, E));
  a.queue = sched + 16 * which;
  a.xstart = sched + kSchedQueueInts;
  a.xorder = sched + kSchedQueueInts + kSchedStartInts;
  a.xnz = sched + kSchedQueueInts + kSchedXnz;
}

extern "C" int moe_amd_gemm_down_backward_dw(const void* dy, const void* act,
                                             const int32_t* offsets, const void* tile_plan,
                                             int64_t S, int E, int H, int I, int dtype,
                                             void* d_down_proj, void* stream) {
  const char* who = "gemm_down_backward_dw";
  if (dtype == MOE_DTYPE_F32)  // static tile walk (the schedule is for the bf16 kernels)
    return f32_down_dw((const float*)dy, (const float*)act, offsets, S, E, H, I,
                       (float*)d_down_proj, (hipStream_t)stream);
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  // One expert's dy and act rows (at most S) are addressed with 32-bit offsets.
  MOE_REQUIRE(S * (int64_t)(H > I ? H : I) * 2 < ((int64_t)1 << 32), MOE_ERR_UNSUPPORTED,
              "%s: S*max(H,I) too large", who);
  MOE_REQUIRE((S == 0 || (dy && act)) && offsets && d_down_proj, MOE_ERR_ARG,
              "%s: null pointer", who);
  if (S > 0) {
    MOE_ALIGNED(dy, who);
    MOE_ALIGNED(act, who);
  }
  MOE_ALIGNED(d_down_proj, who);
  GemmArgs a{};
  a.a0 = (const bf16*)dy;
  a.a1 = (const bf16*)act;
  a.offsets = offsets;
  a.out = (bf16*)d_down_proj;
  a.S = S; a.E = E; a.H = H; a.I = I;
  a.n_rt = (H + 255) / 256;
  a.n_ct = (I + BC - 1) / BC;
  a.n_tiles = E * a.n_rt * a.n_ct;
  set_dw_schedule(a, tile_plan, S, E, 0);
  return launch<G2DW, 256>(a, a.n_tiles, (hipStream_t)stream);
}

namespace {
int down_dw_gathered(const void* d_out, const void* act_w, const int32_t* row_src, int top_k,
                     const int32_t* offsets, const void* tile_plan, int64_t T, int64_t S, int E,
                     int H, int I, int dtype, void* d_down_proj, bool accumulate, void* stream,
                     const char* who) {
  MOE_REQUIRE(!accumulate || tile_plan, MOE_ERR_ARG, "%s: needs the tile plan", who);
  MOE_REQUIRE(!accumulate || dtype == MOE_DTYPE_BF16, MOE_ERR_UNSUPPORTED,
              "%s: bf16 gradients only", who);
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(top_k >= 1 && S == T * top_k, MOE_ERR_ARG, "%s: S != T*top_k", who);
  MOE_REQUIRE(T * (int64_t)H * 2 < ((int64_t)1 << 31), MOE_ERR_UNSUPPORTED, "%s: T*H too large",
              who);
  MOE_REQUIRE((S == 0 || (d_out && act_w && row_src)) && offsets && d_down_proj, MOE_ERR_ARG,
              "%s: null pointer", who);
  if (S > 0) {
    MOE_ALIGNED(d_out, who);
    MOE_ALIGNED(act_w, who);
  }
  MOE_ALIGNED(d_down_proj, who);
  GemmArgs a{};
  a.x = (const bf16*)d_out;
  a.a0 = (const bf16*)act_w;
  a.row_src = row_src;
  a.offsets = offsets;
  a.out = (bf16*)d_down_proj;
  a.T = T; a.S = S; a.E = E; a.H = H; a.I = I; set_topk(a, top_k);
  // tiles of d_down_proj[e]^T: I rows x H columns
  a.n_rt = (I + 255) / 256;
  a.n_ct = (H + BC - 1) / BC;
  a.n_tiles = E * a.n_rt * a.n_ct;
  set_dw_schedule(a, tile_plan, S, E, 0);
  a.accumulate = accumulate;
  return launch<G2DWG, 256>(a, a.n_tiles, (hipStream_t)stream);
}
}  // namespace

extern "C" int moe_amd_gemm_down_backward_dw_gathered(const void* d_out, const void* act_w,
                                                      const int32_t* row_src, int top_k,
                                                      const int32_t* offsets,
                                                      const void* tile_plan, int64_t T, int64_t S,
                                                      int E, int H, int I, int dtype,
                                                      void* d_down_proj, void* stream) {
  return down_dw_gathered(d_out, act_w, row_src, top_k, offsets, tile_plan, T, S, E, H, I, dtype,
                          d_down_proj, false, stream, "gemm_down_backward_dw_gathered");
}

extern "C" int moe_amd_gemm_down_backward_dw_gathered_accumulate(
    const void* d_out, const void* act_w, const int32_t* row_src, int top_k,
    const int32_t* offsets, const void* tile_plan, int64_t T, int64_t S, int E, int H, int I,
    int dtype, void* d_down_proj, void* stream) {
  return down_dw_gathered(d_out, act_w, row_src, top_k, offsets, tile_plan, T, S, E, H, I, dtype,
                          d_down_proj, true, stream, "gemm_down_backward_dw_gathered_accumulate");
}

namespace {
int gate_up_dw(const void* d_gate_up, const void* hidden_states, const int32_t* row_src,
               int top_k, const int32_t* offsets, const void* tile_plan, int64_t T, int64_t S,
               int E, int H, int I, int dtype, void* d_gate_up_proj, bool accumulate,
               void* stream, const char* who) {
  MOE_REQUIRE(!accumulate || tile_plan, MOE_ERR_ARG, "%s: needs the tile plan", who);
  MOE_REQUIRE(!accumulate || dtype == MOE_DTYPE_BF16, MOE_ERR_UNSUPPORTED,
              "%s: bf16 gradients only", who);
  if (dtype == MOE_DTYPE_F32 && !accumulate)
    return f32_gate_up_dw((const float*)d_gate_up, (const float*)hidden_states, row_src, top_k,
                          offsets, T, S, E, H, I, (float*)d_gate_up_proj, (hipStream_t)stream);
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(top_k >= 1 && S == T * top_k, MOE_ERR_ARG, "%s: S != T*top_k", who);
  MOE_REQUIRE(T * (int64_t)H * 2 < ((int64_t)1 << 31), MOE_ERR_UNSUPPORTED, "%s: T*H too large",
              who);
  MOE_REQUIRE((S == 0 || (d_gate_up && hidden_states && row_src)) && offsets && d_gate_up_proj,
              MOE_ERR_ARG, "%s: null pointer", who);
  if (S > 0) {
    MOE_ALIGNED(d_gate_up, who);
    MOE_ALIGNED(hidden_states, who);
  }
  MOE_ALIGNED(d_gate_up_proj, who);
  GemmArgs a{};
  a.x = (const bf16*)hidden_states;
  a.a0 = (const bf16*)d_gate_up;
  a.row_src = row_src;
  a.offsets = offsets;
  a.out = (bf16*)d_gate_up_proj;
  a.T = T; a.S = S; a.E = E; a.H = H; a.I = I; set_topk(a, top_k);
  a.n_rt = (2 * I + 255) / 256;
  a.n_ct = (H + BC - 1) / BC;
  a.n_tiles = E * a.n_rt * a.n_ct;
  set_dw_schedule(a, tile_plan, S, E, 1);
  a.accumulate = accumulate;
  return launch<G1DW, 256>(a, a.n_tiles, (hipStream_t)stream);
}
}  // namespace

extern "C" int moe_amd_gemm_gate_up_backward_dw(const void* d_gate_up, const void* hidden_states,
                                                const int32_t* row_src, int top_k,
                                                const int32_t* offsets, const void* tile_plan,
                                                int64_t T, int64_t S, int E, int H, int I,
                                                int dtype, void* d_gate_up_proj, void* stream) {
  return gate_up_dw(d_gate_up, hidden_states, row_src, top_k, offsets, tile_plan, T, S, E, H, I,
                    dtype, d_gate_up_proj, false, stream, "gemm_gate_up_backward_dw");
}

extern "C" int moe_amd_gemm_gate_up_backward_dw_accumulate(
    const void* d_gate_up, const void* hidden_states, const int32_t* row_src, int top_k,
    const int32_t* offsets, const void* tile_plan, int64_t T, int64_t S, int E, int H, int I,
    int dtype, void* d_gate_up_proj, void* stream) {
  return gate_up_dw(d_gate_up, hidden_states, row_src, top_k, offsets, tile_plan, T, S, E, H, I,
                    dtype, d_gate_up_proj, true, stream, "gemm_gate_up_backward_dw_accumulate");
}
