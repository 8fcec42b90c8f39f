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
// Operands are staged through LDS in [row][64 k] bf16 tiles, 128-byte rows,
// with 16-byte chunks XOR-swizzled by (row >> 1) & 7 so that fragment reads
// and both kinds of tile writes are bank-conflict free.  Operands whose
// memory layout is k-major ("transposed": weights in the dX GEMMs, every
// operand of the dW GEMMs) are loaded as 8x8 bf16 blocks and transposed in
// registers with v_perm before the LDS write.  Global loads are raw buffer
// loads: reads past a tensor's extent return zero, which both guards the
// tails and zero-fills the ragged k range of the dW GEMMs.
//
// Scheduling: the kernel is persistent (one workgroup per CU).  The tile
// space -- (row tile, column tile) for the token-grouped modes, (expert, row
// tile, column tile) for dW -- is cut into 8 contiguous ranges, one per XCD
// (hardware deals workgroups round-robin over the XCDs), and the XCD's
// workgroups stride through their range, so concurrently running tiles share
// weights and rows in that XCD's L2.  A token-grouped tile reads its
// {expert, first row, end row} from the tile plan written by the
// permutation on the device: skewed and empty experts need no host round
// trip.  The first k-stage of a workgroup's next tile is loaded before the
// current tile's epilogue, hiding its latency behind the output writes.
//
// Epilogue: accumulators are rounded to bf16 into an LDS staging tile, then
// written out row by row with 16-byte lanes (full-line stores), applying the
// mode's elementwise tail (SwiGLU, dSwiGLU) on the way out.
//
// Reference: transformers/integrations/moe.py:439-459 (forward grouped_mm),
// :226-242 (per-expert dX / dW formulas of the backward).
#include "common.h"

namespace moe {
namespace {

constexpr int BK = 64;    // k per LDS stage
constexpr int BC = 256;   // output columns per workgroup
constexpr int NTHR = 256; // 4 waves
constexpr int SROW = 260; // bf16 per row of the epilogue staging tile (520 B: conflict-free)

enum Mode { G1F = 0, G2F = 1, G2DX = 2, G1DX = 3, G2DW = 4, G1DW = 5 };

struct GemmArgs {
  const bf16* x;         // hidden_states [T,H]
  const bf16* w;         // gate_up_proj [E,2I,H] or down_proj [E,H,I]
  const bf16* a0;        // act [S,I] (G2F) | dy [S,H] (G2DX,G2DW) | d_gate_up [S,2I] (G1DX,G1DW)
  const bf16* a1;        // act [S,I] (G2DW) | gate_up [S,2I] (G2DX)
  const int* row_src;    // [S]
  const int* offsets;    // [E+1]
  const int* tile_count; // token modes: number of row tiles (tile_starts[E] for BR)
  const int4* tile_info; // token modes: {expert, first row, end row, 0} per row tile
  bf16* out;
  bf16* out2;            // gate_up output of G1F (may be null)
  int64_t T, S;
  int E, H, I, topk;
  int n_ct, n_rt, n_tiles;  // n_tiles: dW modes (host-known)
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ u32x4 bload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}

constexpr uint32_t kOOB = 0x80000000u;  // offset that always reads as zero


// Writes an 8x8 bf16 block, transposed, into a [row][64] LDS tile.
// v[r] holds 8 consecutive features of k-row kb*8+r; feature c of the block
// goes to tile row fb*8+c as 8 consecutive k values (16 bytes, chunk kb).
// Odd feature blocks emit their rows in pair-swapped order (c ^ 1) so that
// the 16 lanes of one LDS write phase cover both row parities (no bank
// conflicts); the swap is folded into the v_perm byte selector, so there is
// no data-dependent register selection.
__device__ __forceinline__ void store_transposed(bf16* tile, const u32x4 (&v)[8], int fb, int kb) {
  const int odd = fb & 1;
  const uint32_t sel_a = odd ? 0x07060302u : 0x05040100u;  // feature 2q + odd
  const uint32_t sel_b = odd ? 0x05040100u : 0x07060302u;  // feature 2q + 1 - odd
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    u32x4 a, b;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a[j] = __builtin_amdgcn_perm(v[2 * j + 1][q], v[2 * j][q], sel_a);
      b[j] = __builtin_amdgcn_perm(v[2 * j + 1][q], v[2 * j][q], sel_b);
    }
    const int row_a = fb * 8 + 2 * q + odd;
    const int row_b = row_a ^ 1;
    const int chunk = (kb ^ ((odd * 4 + q) & 7)) << 3;  // swizzle (row >> 1) & 7
    *(u32x4*)(tile + row_a * 64 + chunk) = a;
    *(u32x4*)(tile + row_b * 64 + chunk) = b;
  }
}

template <int MODE, int BR>
__global__ __launch_bounds__(NTHR, 1) void grouped_gemm_kernel(GemmArgs p) {
  constexpr bool TOKEN = MODE <= G1DX;          // rows = routed rows of one expert
  constexpr bool COL_T = !(MODE == G1F || MODE == G2F);
  constexpr int WR = BR / 2;                    // rows per wave
  constexpr int TJ = WR / 32;                   // MFMA row sub-tiles per wave
  constexpr int TI = 4;                         // MFMA col sub-tiles per wave (128 cols)
  constexpr int RPASS = BR / 32;                // direct row-loader passes
  constexpr int STAGE = (BC + BR) * BK;         // bf16 elements per LDS stage
  static_assert(TOKEN || BR == 256, "dW modes use 256-row tiles");

  extern __shared__ __attribute__((aligned(16))) bf16 smem[];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wr = wid >> 1, wc = wid & 1;
  const int l32 = lane & 31, hl = lane >> 5;
  const int H = p.H, I = p.I, I2 = 2 * p.I;

  // ------------------------------------------------------------ tile walk
  const int n_tiles = TOKEN ? (*p.tile_count) * p.n_ct : p.n_tiles;
  const int xcd = blockIdx.x & 7, nslot = gridDim.x >> 3;
  const int chunk = (n_tiles + 7) >> 3;
  const int t_end = min(n_tiles, (xcd + 1) * chunk);
  int t = xcd * chunk + (int)(blockIdx.x >> 3);
  if (t >= t_end) return;

  struct Tile {
    int e, row0, row_end, ct, kbeg, kend, nk;
  };
  auto decode = [&](int tt) {
    Tile d;
    if constexpr (TOKEN) {
      d.ct = tt % p.n_ct;
      const int4 ti = p.tile_info[tt / p.n_ct];
      d.e = ti.x;
      d.row0 = ti.y;
      d.row_end = ti.z;
      d.kbeg = d.kend = 0;
    } else {
      const int per_e = p.n_rt * p.n_ct;
      d.e = tt / per_e;
      const int rem = tt - d.e * per_e;
      const int rt = rem / p.n_ct;
      d.ct = rem - rt * p.n_ct;
      d.row0 = rt * BR;
      d.row_end = 0;
      d.kbeg = p.offsets[d.e];
      d.kend = p.offsets[d.e + 1];
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
    if constexpr (MODE == G1F || MODE == G2DX) K_len = H;
    else if constexpr (MODE == G2F) K_len = I;
    else if constexpr (MODE == G1DX) K_len = I2;
    else K_len = d.kend - d.kbeg;
    d.nk = (K_len + BK - 1) / BK;
    return d;
  };

  // ---------------------------------------------------------------- loaders
  // Direct loader geometry: 16-byte chunk (t & 7) of tile row (t >> 3) + 32*pass.
  const int dchunk = tid & 7, drow = tid >> 3;
  const int dswz = (dchunk ^ ((drow >> 1) & 7)) << 3;
  // Transposed loader geometry: k block kb (8 k rows), feature block fb (8 features).
  const int kb = tid & 7, fb = tid >> 3;

  // Per-tile source descriptors (uniform parts live in SGPRs).
  struct Src {
    __amdgpu_buffer_rsrc_t r, c;
    uint32_t roff[TOKEN ? RPASS : 1];
    uint32_t coff[COL_T ? 1 : 8];
    uint32_t rstride, cstride;
    int kbeg, kend, ct;
  };
  auto setup = [&](const Tile& d, Src& s) {
    s.kbeg = d.kbeg;
    s.kend = d.kend;
    s.ct = d.ct;
    s.rstride = s.cstride = 0;
    // Row operand.
    if constexpr (MODE == G1F) {
      s.r = make_rsrc(p.x, (uint32_t)(p.T * H * 2));
#pragma unroll
      for (int q = 0; q < RPASS; ++q) {
        const int r = min(d.row0 + drow + 32 * q, d.row_end - 1);
        const int tok = p.row_src[r] / p.topk;
        s.roff[q] = (uint32_t)tok * (uint32_t)(H * 2) + dchunk * 16;
      }
    } else if constexpr (TOKEN) {
      const int ld = (MODE == G2F) ? I : (MODE == G2DX ? H : I2);
      s.r = make_rsrc(p.a0 + (int64_t)d.row0 * ld,
                      (uint32_t)((int64_t)(d.row_end - d.row0) * ld * 2));
#pragma unroll
      for (int q = 0; q < RPASS; ++q) {
        const int r = min(drow + 32 * q, d.row_end - d.row0 - 1);
        s.roff[q] = (uint32_t)r * (uint32_t)(ld * 2) + dchunk * 16;
      }
    } else {
      // dW: row operand [rows of e][features], features = C rows.
      const int ld = (MODE == G2DW) ? H : I2;
      s.r = make_rsrc(p.a0 + (int64_t)d.kbeg * ld,
                      (uint32_t)((int64_t)(d.kend - d.kbeg) * ld * 2));
      s.rstride = (uint32_t)ld * 2;
      s.roff[0] = (uint32_t)(kb * 8) * s.rstride + (uint32_t)(d.row0 + fb * 8) * 2;
    }
    // Column operand.
    if constexpr (MODE == G1F) {
      s.c = make_rsrc(p.w + (int64_t)d.e * I2 * H, (uint32_t)(I2 * H * 2));
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int c = drow + 32 * q;  // tile column 0..255: [gate 64 | up 64] per wave column
        const int lc = c & 127;
        const int f = d.ct * 128 + (c >> 7) * 64 + (lc & 63);
        const int wrow = (lc < 64) ? f : I + f;
        s.coff[q] = (uint32_t)wrow * (uint32_t)(H * 2) + dchunk * 16;
      }
    } else if constexpr (MODE == G2F) {
      s.c = make_rsrc(p.w + (int64_t)d.e * H * I, (uint32_t)(H * I * 2));
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int wrow = d.ct * BC + drow + 32 * q;
        s.coff[q] = wrow < H ? (uint32_t)wrow * (uint32_t)(I * 2) + dchunk * 16 : kOOB;
      }
    } else if constexpr (MODE == G2DX) {
      s.c = make_rsrc(p.w + (int64_t)d.e * H * I, (uint32_t)(H * I * 2));
      s.cstride = (uint32_t)I * 2;
      s.coff[0] = (uint32_t)(kb * 8) * s.cstride + (uint32_t)(d.ct * BC + fb * 8) * 2;
    } else if constexpr (MODE == G1DX) {
      s.c = make_rsrc(p.w + (int64_t)d.e * I2 * H, (uint32_t)(I2 * H * 2));
      s.cstride = (uint32_t)H * 2;
      s.coff[0] = (uint32_t)(kb * 8) * s.cstride + (uint32_t)(d.ct * BC + fb * 8) * 2;
    } else if constexpr (MODE == G2DW) {
      s.c = make_rsrc(p.a1 + (int64_t)d.kbeg * I, (uint32_t)((int64_t)(d.kend - d.kbeg) * I * 2));
      s.cstride = (uint32_t)I * 2;
      s.coff[0] = (uint32_t)(kb * 8) * s.cstride + (uint32_t)(d.ct * BC + fb * 8) * 2;
    } else {  // G1DW: gathered hidden_states rows
      s.c = make_rsrc(p.x, (uint32_t)(p.T * H * 2));
      s.coff[0] = 0;
    }
  };

  // One register set holds one k-stage in flight: row operand + column operand.
  struct Regs {
    u32x4 r[TOKEN ? RPASS : 8];
    u32x4 c[8];
  };
  // G1DW gathers hidden_states rows through row_src; the byte offsets of the
  // next stage's rows are fetched one load ahead so that no load waits on a
  // dependent index load.
  uint32_t tokoff[8];
  auto fetch_tok = [&](const Src& s, int kt) {
    if constexpr (MODE == G1DW) {
      const int f0 = s.ct * BC + fb * 8;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int kr = kt * BK + kb * 8 + r;
        uint32_t off = kOOB;
        if (kr < s.kend - s.kbeg && f0 < H)
          off = (uint32_t)(p.row_src[s.kbeg + kr] / p.topk) * (uint32_t)(H * 2) + (uint32_t)f0 * 2;
        tokoff[r] = off;
      }
    }
  };
  auto load_tiles = [&](const Src& s, int kt, Regs& R) {
    const uint32_t kbytes = (uint32_t)kt * BK * 2;
    if constexpr (TOKEN) {
#pragma unroll
      for (int q = 0; q < RPASS; ++q) R.r[q] = bload(s.r, s.roff[q] + kbytes);
    } else {
      const uint32_t base = s.roff[0] + (uint32_t)kt * BK * s.rstride;
#pragma unroll
      for (int r = 0; r < 8; ++r) R.r[r] = bload(s.r, base + r * s.rstride);
    }
    if constexpr (!COL_T) {
#pragma unroll
      for (int q = 0; q < 8; ++q) R.c[q] = bload(s.c, s.coff[q] + kbytes);
    } else if constexpr (MODE == G1DW) {
#pragma unroll
      for (int r = 0; r < 8; ++r) R.c[r] = bload(s.c, tokoff[r]);
      fetch_tok(s, kt + 1);
    } else {
      const uint32_t base = s.coff[0] + (uint32_t)kt * BK * s.cstride;
#pragma unroll
      for (int r = 0; r < 8; ++r) R.c[r] = bload(s.c, base + r * s.cstride);
    }
  };
  auto store_tiles = [&](int stage, const Regs& R) {
    bf16* sC = smem + stage * STAGE;
    bf16* sR = sC + BC * BK;
    if constexpr (!COL_T) {
#pragma unroll
      for (int q = 0; q < 8; ++q)
        *(u32x4*)(sC + (drow + 32 * q) * BK + dswz) = R.c[q];
    } else {
      store_transposed(sC, R.c, fb, kb);
    }
    if constexpr (TOKEN) {
#pragma unroll
      for (int q = 0; q < RPASS; ++q)
        *(u32x4*)(sR + (drow + 32 * q) * BK + dswz) = R.r[q];
    } else {
      store_transposed(sR, R.r, fb, kb);
    }
  };

  f32x16 acc[TI][TJ];
  const int fr_sw = (l32 >> 1) & 7;
  auto read_frags = [&](int stage, int ks, bf16x8 (&af)[TI], bf16x8 (&bfr)[TJ]) {
    const bf16* sC = smem + stage * STAGE;
    const bf16* sR = sC + BC * BK;
    const int csw = ((2 * ks + hl) ^ fr_sw) << 3;
#pragma unroll
    for (int i = 0; i < TI; ++i)
      af[i] = *(const bf16x8*)(sC + (wc * 128 + i * 32 + l32) * BK + csw);
#pragma unroll
    for (int j = 0; j < TJ; ++j)
      bfr[j] = *(const bf16x8*)(sR + (wr * WR + j * 32 + l32) * BK + csw);
  };
  auto mfmas = [&](const bf16x8 (&af)[TI], const bf16x8 (&bfr)[TJ]) {
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
  };

  Tile cur = decode(t);
  Src src;
  setup(cur, src);
  Regs R;
  fetch_tok(src, 0);
  load_tiles(src, 0, R);

  while (true) {
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // ------------------------------------------------------- main loop
    // LDS holds two k-stages; the global loads for stage kt+1 are issued at
    // the top of step kt, land in registers while the MFMAs of step kt run
    // and are written to the other stage before the step's single barrier.
    // The last step is peeled so the loop body is one basic block.
    if (cur.nk > 0) {
      auto kstep = [&](int kt, bool has_next) {
        const int stg = kt & 1;
        if (has_next) load_tiles(src, kt + 1, R);
        // Keep the loads at the top of the step: the scheduler would
        // otherwise sink them next to their LDS stores.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
          bf16x8 af[TI], bfr[TJ];
          read_frags(stg, ks, af, bfr);
          mfmas(af, bfr);
        }
        if (has_next) {
          store_tiles(stg ^ 1, R);
          __syncthreads();
        }
      };
      store_tiles(0, R);
      __syncthreads();
      for (int kt = 0; kt < cur.nk - 1; ++kt) kstep(kt, true);
      kstep(cur.nk - 1, false);
    }

    // --------------------------------------- next tile's first stage load
    const int tn = t + nslot;
    const bool more = tn < t_end;
    Tile nxt = cur;
    if (more) {
      nxt = decode(tn);
      setup(nxt, src);
      fetch_tok(src, 0);
      load_tiles(src, 0, R);
    }

    // --------------------------------------------------------- epilogue
    __syncthreads();  // every wave is done reading the k-stages
    bf16* stg = smem;  // [BR][SROW] bf16 staging tile
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int row = wr * WR + j * 32 + l32;
          const int col = wc * 128 + i * 32 + 8 * q + 4 * hl;
          u32x2 v = {pack_bf2(acc[i][j][4 * q + 0], acc[i][j][4 * q + 1]),
                     pack_bf2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3])};
          *(u32x2*)(stg + row * SROW + col) = v;
        }
    __syncthreads();
    if constexpr (MODE == G1F) {
      // 128 output features per tile; 16 lanes x 8 features per row.
      const int fl = (tid & 15) * 8;
      const int scol = (fl >> 6) * 128 + (fl & 63);  // gate column in the staging tile
      const int f = cur.ct * 128 + fl;
#pragma unroll 4
      for (int row = tid >> 4; row < BR; row += NTHR / 16) {
        const int r = cur.row0 + row;
        if (r < cur.row_end && f < I) {
          const u32x4 gv = *(const u32x4*)(stg + row * SROW + scol);
          const u32x4 uv = *(const u32x4*)(stg + row * SROW + scol + 64);
          u32x4 av;
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float g0 = bf_lo(gv[w]), g1 = bf_hi(gv[w]);
            const float u0 = bf_lo(uv[w]), u1 = bf_hi(uv[w]);
            av[w] = pack_bf2(round_bf(siluf_(g0)) * u0, round_bf(siluf_(g1)) * u1);
          }
          *(u32x4*)(p.out + (int64_t)r * I + f) = av;
          if (p.out2) {
            *(u32x4*)(p.out2 + (int64_t)r * I2 + f) = gv;
            *(u32x4*)(p.out2 + (int64_t)r * I2 + I + f) = uv;
          }
        }
      }
    } else if constexpr (MODE == G2DX) {
      // d_act tile (bf16) -> d_gate, d_up with gate/up read back from gate_up.
      const int c0 = (tid & 31) * 8;
      const int f = cur.ct * BC + c0;
#pragma unroll 2
      for (int row = tid >> 5; row < BR; row += NTHR / 32) {
        const int r = cur.row0 + row;
        if (r < cur.row_end && f < I) {
          const u32x4 dav = *(const u32x4*)(stg + row * SROW + c0);
          const u32x4 gv = *(const u32x4*)(p.a1 + (int64_t)r * I2 + f);
          const u32x4 uv = *(const u32x4*)(p.a1 + (int64_t)r * I2 + I + f);
          u32x4 dgv, duv;
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            float dg[2], du[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const float da = h ? bf_hi(dav[w]) : bf_lo(dav[w]);
              const float g = h ? bf_hi(gv[w]) : bf_lo(gv[w]);
              const float u = h ? bf_hi(uv[w]) : bf_lo(uv[w]);
              const float sg = sigmoidf_(g);
              const float s = round_bf(siluf_(g));       // silu(g) as stored in bf16
              const float ds = round_bf(da * u);          // d silu(g)
              du[h] = da * s;
              dg[h] = ds * (sg * (1.f + g * (1.f - sg)));
            }
            dgv[w] = pack_bf2(dg[0], dg[1]);
            duv[w] = pack_bf2(du[0], du[1]);
          }
          *(u32x4*)(p.out + (int64_t)r * I2 + f) = dgv;
          *(u32x4*)(p.out + (int64_t)r * I2 + I + f) = duv;
        }
      }
    } else {
      // Plain bf16 tile: y (G2F), d_xs (G1DX), d_down_proj (G2DW), d_gate_up_proj (G1DW).
      const int c0 = (tid & 31) * 8;
      const int f = cur.ct * BC + c0;
      int nrows, ld;
      bf16* obase;
      if constexpr (TOKEN) {
        nrows = cur.row_end;
        ld = H;
        obase = p.out;
      } else {
        nrows = (MODE == G2DW) ? H : I2;
        ld = (MODE == G2DW) ? I : H;
        obase = p.out + (int64_t)cur.e * (MODE == G2DW ? (int64_t)H * I : (int64_t)I2 * H);
      }
#pragma unroll 4
      for (int row = tid >> 5; row < BR; row += NTHR / 32) {
        const int r = cur.row0 + row;
        if (r < nrows && f < ld)
          *(u32x4*)(obase + (int64_t)r * ld + f) = *(const u32x4*)(stg + row * SROW + c0);
      }
    }
    if (!more) break;
    __syncthreads();  // staging reads done before stage 0 is overwritten
    t = tn;
    cur = nxt;
  }
}

int g_num_cu[64];

int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!g_num_cu[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_num_cu[dev] = n;
  }
  return g_num_cu[dev];
}

template <int MODE, int BR>
int launch(const GemmArgs& a, int max_tiles, hipStream_t st) {
  constexpr size_t stages = (size_t)2 * (BC + BR) * BK * sizeof(bf16);
  constexpr size_t staging = (size_t)BR * SROW * sizeof(bf16);
  const size_t lds = stages > staging ? stages : staging;
  if (max_tiles <= 0) return MOE_OK;
  hipError_t err = hipFuncSetAttribute((const void*)grouped_gemm_kernel<MODE, BR>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
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
  grouped_gemm_kernel<MODE, BR><<<grid, NTHR, lds, st>>>(a);
  return check_launch("grouped_gemm");
}

// Row-tile height for the token-grouped GEMMs from the mean rows per expert.
int pick_br(int64_t S, int E) {
  const int64_t avg = S / (E > 0 ? E : 1);
  if (avg >= 512) return 256;
  if (avg >= 128) return 128;
  return 64;
}
int tile_index(int br) { return br == 64 ? 0 : (br == 128 ? 1 : 2); }

template <int MODE>
int launch_token(GemmArgs a, int64_t S, int E, int ncols_per_tile_out, int ncols_total,
                 const void* tile_plan, hipStream_t st) {
  const int br = pick_br(S, E);
  const int b = tile_index(br);
  const char* pb = (const char*)tile_plan;
  a.tile_count = (const int*)pb + (size_t)b * (E + 1) + E;
  a.tile_info = (const int4*)(pb + plan_info_offset(S, E, b));
  a.n_ct = (ncols_total + ncols_per_tile_out - 1) / ncols_per_tile_out;
  const int64_t max_tiles = plan_max_tiles(S, E, b) * a.n_ct;
  if (max_tiles > (int64_t)1 << 30) {
    set_error("grouped_gemm: too many tiles");
    return MOE_ERR_UNSUPPORTED;
  }
  if (br == 256) return launch<MODE, 256>(a, (int)max_tiles, st);
  if (br == 128) return launch<MODE, 128>(a, (int)max_tiles, st);
  return launch<MODE, 64>(a, (int)max_tiles, st);
}
int check_common(int64_t S, int E, int H, int I, int dtype, const char* who) {
  MOE_REQUIRE(dtype == MOE_DTYPE_BF16, MOE_ERR_UNSUPPORTED,
              "%s: only bf16 (dtype %d) is implemented on the GPU path", who, MOE_DTYPE_BF16);
  MOE_REQUIRE(S >= 0 && E >= 1 && H > 0 && I > 0, MOE_ERR_ARG, "%s: bad sizes", who);
  MOE_REQUIRE(H % 64 == 0 && I % 64 == 0, MOE_ERR_ARG,
              "%s: H=%d and I=%d must be multiples of 64", who, H, I);
  const int64_t widest = H > 2 * I ? H : 2 * (int64_t)I;
  // Buffer descriptors address at most one expert's rows (<= S) with
  // 32-bit byte offsets.
  MOE_REQUIRE(S * widest * 2 < ((int64_t)1 << 32), MOE_ERR_UNSUPPORTED,
              "%s: S*max(H,2I) too large for 32-bit buffer offsets", who);
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
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(top_k >= 1 && S == T * top_k, MOE_ERR_ARG, "%s: S != T*top_k", who);
  MOE_REQUIRE(T * (int64_t)H * 2 < ((int64_t)1 << 31), MOE_ERR_UNSUPPORTED, "%s: T*H too large",
              who);
  MOE_REQUIRE(hidden_states && row_src && offsets && tile_plan && gate_up_proj && act_out,
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
  a.T = T; a.S = S; a.E = E; a.H = H; a.I = I; a.topk = top_k;
  return launch_token<G1F>(a, S, E, 128, I, tile_plan, (hipStream_t)stream);
}

extern "C" int moe_amd_gemm_down(const void* act, const int32_t* offsets,
                                 const void* tile_plan, const void* down_proj, int64_t S,
                                 int E, int H, int I, int dtype, void* y_out, void* stream) {
  const char* who = "gemm_down";
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(act && offsets && tile_plan && down_proj && y_out, MOE_ERR_ARG,
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

extern "C" int moe_amd_gemm_down_backward_dx_dswiglu(const void* dy, const int32_t* offsets,
                                                     const void* tile_plan,
                                                     const void* down_proj, const void* gate_up,
                                                     int64_t S, int E, int H, int I, int dtype,
                                                     void* d_gate_up, void* stream) {
  const char* who = "gemm_down_backward_dx_dswiglu";
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(dy && offsets && tile_plan && down_proj && gate_up && d_gate_up, MOE_ERR_ARG,
              "%s: null pointer", who);
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

extern "C" int moe_amd_gemm_gate_up_backward_dx(const void* d_gate_up, const int32_t* offsets,
                                                const void* tile_plan,
                                                const void* gate_up_proj, int64_t S, int E,
                                                int H, int I, int dtype, void* d_xs,
                                                void* stream) {
  const char* who = "gemm_gate_up_backward_dx";
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(d_gate_up && offsets && tile_plan && gate_up_proj && d_xs, MOE_ERR_ARG,
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

extern "C" int moe_amd_gemm_down_backward_dw(const void* dy, const void* act,
                                             const int32_t* offsets, int64_t S, int E, int H,
                                             int I, int dtype, void* d_down_proj, void* stream) {
  const char* who = "gemm_down_backward_dw";
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
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
  return launch<G2DW, 256>(a, a.n_tiles, (hipStream_t)stream);
}

extern "C" int moe_amd_gemm_gate_up_backward_dw(const void* d_gate_up, const void* hidden_states,
                                                const int32_t* row_src, int top_k,
                                                const int32_t* offsets, int64_t T, int64_t S,
                                                int E, int H, int I, int dtype,
                                                void* d_gate_up_proj, void* stream) {
  const char* who = "gemm_gate_up_backward_dw";
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
  a.T = T; a.S = S; a.E = E; a.H = H; a.I = I; a.topk = top_k;
  a.n_rt = (2 * I + 255) / 256;
  a.n_ct = (H + BC - 1) / BC;
  a.n_tiles = E * a.n_rt * a.n_ct;
  return launch<G1DW, 256>(a, a.n_tiles, (hipStream_t)stream);
}
