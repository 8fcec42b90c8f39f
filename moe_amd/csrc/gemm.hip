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
// Scheduling: for the token-grouped modes the workgroup id is decoded into
// (row tile, column tile); the row tile is mapped to its expert by a binary
// search over tile_starts (written by the permutation on the device), so
// skewed and empty experts need no host round trip.  Workgroup ids are
// remapped so that each XCD walks a contiguous range of tiles (shared
// weights and rows stay in that XCD's L2).
//
// Reference: transformers/integrations/moe.py:439-459 (forward grouped_mm),
// :226-242 (per-expert dX / dW formulas of the backward).
#include "common.h"

namespace moe {
namespace {

constexpr int BK = 64;    // k per LDS stage
constexpr int BC = 256;   // output columns per workgroup
constexpr int NTHR = 256; // 4 waves

enum Mode { G1F = 0, G2F = 1, G2DX = 2, G1DX = 3, G2DW = 4, G1DW = 5 };

struct GemmArgs {
  const bf16* x;         // hidden_states [T,H]
  const bf16* w;         // gate_up_proj [E,2I,H] or down_proj [E,H,I]
  const bf16* a0;        // act [S,I] (G2F) | dy [S,H] (G2DX,G2DW) | d_gate_up [S,2I] (G1DX,G1DW)
  const bf16* a1;        // act [S,I] (G2DW) | gate_up [S,2I] (G2DX)
  const int* row_src;    // [S]
  const int* offsets;    // [E+1]
  const int* tile_starts;// [E+1] for BR
  bf16* out;
  bf16* out2;            // gate_up output of G1F (may be null)
  int64_t T, S;
  int E, H, I, topk;
  int n_ct, n_rt, n_logical;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ u32x4 bload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}

constexpr uint32_t kOOB = 0x80000000u;  // offset that always reads as zero

// 8x8 bf16 transpose: v[r] holds 8 features of k-row r; w[c] receives the 8
// k values of feature c.
__device__ __forceinline__ void transpose8x8(const u32x4 (&v)[8], u32x4 (&w)[8]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t lo = v[2 * j][q], hi = v[2 * j + 1][q];
      w[2 * q][j] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
      w[2 * q + 1][j] = __builtin_amdgcn_perm(hi, lo, 0x07060302u);
    }
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

  // XCD-aware remap: hardware deals workgroups round-robin over 8 XCDs.
  const int per_xcd = gridDim.x >> 3;
  const int logical = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (logical >= p.n_logical) return;

  const int H = p.H, I = p.I, I2 = 2 * p.I;
  int e, row0, row_end = 0, ct, kbeg = 0, kend = 0, rt;
  if constexpr (TOKEN) {
    ct = logical % p.n_ct;
    rt = logical / p.n_ct;
    const int* ts = p.tile_starts;
    if (rt >= ts[p.E]) return;
    int lo = 0, hi = p.E;  // ts[lo] <= rt < ts[hi]
    while (hi - lo > 1) {
      int mid = (lo + hi) >> 1;
      if (ts[mid] <= rt) lo = mid; else hi = mid;
    }
    e = lo;
    row0 = p.offsets[e] + (rt - ts[e]) * BR;
    row_end = p.offsets[e + 1];
  } else {
    const int per_e = p.n_rt * p.n_ct;
    e = logical / per_e;
    const int rem = logical - e * per_e;
    rt = rem / p.n_ct;
    ct = rem - rt * p.n_ct;
    row0 = rt * BR;
    kbeg = p.offsets[e];
    kend = p.offsets[e + 1];
  }

  // ---------------------------------------------------------------- loaders
  // Direct loader geometry: 16-byte chunk (t & 7) of tile row (t >> 3) + 32*pass.
  const int dchunk = tid & 7, drow = tid >> 3;
  const int dswz = (dchunk ^ ((drow >> 1) & 7)) << 3;
  // Transposed loader geometry: k block kb (8 k rows), feature block fb (8 features).
  const int kb = tid & 7, fb = tid >> 3;
  const int todd = fb & 1;

  int K_len;
  if constexpr (MODE == G1F || MODE == G2DX) K_len = H;
  else if constexpr (MODE == G2F) K_len = I;
  else if constexpr (MODE == G1DX) K_len = I2;
  else K_len = kend - kbeg;
  const int nk = (K_len + BK - 1) / BK;

  // Row operand.
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t roff[TOKEN ? RPASS : 1];
  uint32_t rstride = 0;  // bytes per k row (transposed row operand)
  if constexpr (MODE == G1F) {
    rsrc = make_rsrc(p.x, (uint32_t)(p.T * H * 2));
#pragma unroll
    for (int q = 0; q < RPASS; ++q) {
      int r = min(row0 + drow + 32 * q, row_end - 1);
      int tok = p.row_src[r] / p.topk;
      roff[q] = (uint32_t)tok * (uint32_t)(H * 2) + dchunk * 16;
    }
  } else if constexpr (TOKEN) {
    const bf16* base;
    int ld;
    if constexpr (MODE == G2F) { base = p.a0; ld = I; }
    else if constexpr (MODE == G2DX) { base = p.a0; ld = H; }
    else { base = p.a0; ld = I2; }
    rsrc = make_rsrc(base + (int64_t)row0 * ld, (uint32_t)((int64_t)(row_end - row0) * ld * 2));
#pragma unroll
    for (int q = 0; q < RPASS; ++q) {
      int r = min(drow + 32 * q, row_end - row0 - 1);
      roff[q] = (uint32_t)r * (uint32_t)(ld * 2) + dchunk * 16;
    }
  } else {
    // dW: row operand [rows of e][features], features = C rows.
    const int ld = (MODE == G2DW) ? H : I2;
    rsrc = make_rsrc(p.a0 + (int64_t)kbeg * ld, (uint32_t)((int64_t)(kend - kbeg) * ld * 2));
    rstride = (uint32_t)ld * 2;
    roff[0] = (uint32_t)(kb * 8) * rstride + (uint32_t)(row0 + fb * 8) * 2;
  }

  // Column operand.
  __amdgpu_buffer_rsrc_t csrc;
  uint32_t coff[8];
  uint32_t cstride = 0;
  if constexpr (MODE == G1F) {
    csrc = make_rsrc(p.w + (int64_t)e * I2 * H, (uint32_t)(I2 * H * 2));
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      int c = drow + 32 * q;                 // tile column 0..255
      int lc = c & 127;
      int f = ct * 128 + (c >> 7) * 64 + (lc & 63);
      int wrow = (lc < 64) ? f : I + f;
      coff[q] = (uint32_t)wrow * (uint32_t)(H * 2) + dchunk * 16;
    }
  } else if constexpr (MODE == G2F) {
    csrc = make_rsrc(p.w + (int64_t)e * H * I, (uint32_t)(H * I * 2));
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      int wrow = ct * BC + drow + 32 * q;
      coff[q] = wrow < H ? (uint32_t)wrow * (uint32_t)(I * 2) + dchunk * 16 : kOOB;
    }
  } else if constexpr (MODE == G2DX) {
    csrc = make_rsrc(p.w + (int64_t)e * H * I, (uint32_t)(H * I * 2));
    cstride = (uint32_t)I * 2;
    coff[0] = (uint32_t)(kb * 8) * cstride + (uint32_t)(ct * BC + fb * 8) * 2;
  } else if constexpr (MODE == G1DX) {
    csrc = make_rsrc(p.w + (int64_t)e * I2 * H, (uint32_t)(I2 * H * 2));
    cstride = (uint32_t)H * 2;
    coff[0] = (uint32_t)(kb * 8) * cstride + (uint32_t)(ct * BC + fb * 8) * 2;
  } else if constexpr (MODE == G2DW) {
    csrc = make_rsrc(p.a1 + (int64_t)kbeg * I, (uint32_t)((int64_t)(kend - kbeg) * I * 2));
    cstride = (uint32_t)I * 2;
    coff[0] = (uint32_t)(kb * 8) * cstride + (uint32_t)(ct * BC + fb * 8) * 2;
  } else {  // G1DW: gathered hidden_states rows
    csrc = make_rsrc(p.x, (uint32_t)(p.T * H * 2));
  }

  u32x4 rreg[TOKEN ? RPASS : 8];
  u32x4 creg[8];

  auto load_tiles = [&](int kt) {
    const uint32_t kbytes = (uint32_t)kt * BK * 2;
    if constexpr (TOKEN) {
#pragma unroll
      for (int q = 0; q < RPASS; ++q) rreg[q] = bload(rsrc, roff[q] + kbytes);
    } else {
      const uint32_t base = roff[0] + (uint32_t)kt * BK * rstride;
#pragma unroll
      for (int r = 0; r < 8; ++r) rreg[r] = bload(rsrc, base + r * rstride);
    }
    if constexpr (!COL_T) {
#pragma unroll
      for (int q = 0; q < 8; ++q) creg[q] = bload(csrc, coff[q] + kbytes);
    } else if constexpr (MODE == G1DW) {
      const int f0 = ct * BC + fb * 8;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        int kr = kt * BK + kb * 8 + r;
        uint32_t off = kOOB;
        if (kr < kend - kbeg && f0 < H) {
          int tok = p.row_src[kbeg + kr] / p.topk;
          off = (uint32_t)tok * (uint32_t)(H * 2) + (uint32_t)f0 * 2;
        }
        creg[r] = bload(csrc, off);
      }
    } else {
      const uint32_t base = coff[0] + (uint32_t)kt * BK * cstride;
#pragma unroll
      for (int r = 0; r < 8; ++r) creg[r] = bload(csrc, base + r * cstride);
    }
  };

  auto store_tiles = [&](int stage) {
    bf16* sC = smem + stage * STAGE;
    bf16* sR = sC + BC * BK;
    if constexpr (!COL_T) {
#pragma unroll
      for (int q = 0; q < 8; ++q)
        *(u32x4*)(sC + (drow + 32 * q) * BK + dswz) = creg[q];
    } else {
      u32x4 w[8];
      transpose8x8(creg, w);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        u32x4 val = todd ? w[c ^ 1] : w[c];
        int row = fb * 8 + (c ^ todd);
        int sw = (kb ^ ((todd * 4 + (c >> 1)) & 7)) << 3;
        *(u32x4*)(sC + row * BK + sw) = val;
      }
    }
    if constexpr (TOKEN) {
#pragma unroll
      for (int q = 0; q < RPASS; ++q)
        *(u32x4*)(sR + (drow + 32 * q) * BK + dswz) = rreg[q];
    } else {
      u32x4 w[8];
      transpose8x8(rreg, w);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        u32x4 val = todd ? w[c ^ 1] : w[c];
        int row = fb * 8 + (c ^ todd);
        int sw = (kb ^ ((todd * 4 + (c >> 1)) & 7)) << 3;
        *(u32x4*)(sR + row * BK + sw) = val;
      }
    }
  };

  f32x16 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  if (nk > 0) {
    load_tiles(0);
    store_tiles(0);
    __syncthreads();
  }
  const int fr_sw = (l32 >> 1) & 7;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tiles(kt + 1);
    const bf16* sC = smem + cur * STAGE;
    const bf16* sR = sC + BC * BK;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int csw = ((2 * ks + hl) ^ fr_sw) << 3;
      bf16x8 af[TI], bfr[TJ];
#pragma unroll
      for (int i = 0; i < TI; ++i)
        af[i] = *(const bf16x8*)(sC + (wc * 128 + i * 32 + l32) * BK + csw);
#pragma unroll
      for (int j = 0; j < TJ; ++j)
        bfr[j] = *(const bf16x8*)(sR + (wr * WR + j * 32 + l32) * BK + csw);
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_tiles(cur ^ 1);
    __syncthreads();
  }

  // --------------------------------------------------------------- epilogue
  // acc[i][j][4q+v]: tile column wc*128 + i*32 + 8q + 4*hl + v, tile row
  // wr*WR + j*32 + l32.
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int trow = wr * WR + j * 32 + l32;
    if constexpr (MODE == G1F) {
      const int r = row0 + trow;
      if (r < row_end) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int f = ct * 128 + wc * 64 + i * 32 + 8 * q + 4 * hl;
            if (f < I) {
              float g[4], u[4], a[4];
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                g[v] = round_bf(acc[i][j][4 * q + v]);
                u[v] = round_bf(acc[i + 2][j][4 * q + v]);
                float s = round_bf(siluf_(g[v]));
                a[v] = s * u[v];
              }
              u32x2 av = {pack_bf2(a[0], a[1]), pack_bf2(a[2], a[3])};
              *(u32x2*)(p.out + (int64_t)r * I + f) = av;
              if (p.out2) {
                u32x2 gv = {pack_bf2(g[0], g[1]), pack_bf2(g[2], g[3])};
                u32x2 uv = {pack_bf2(u[0], u[1]), pack_bf2(u[2], u[3])};
                *(u32x2*)(p.out2 + (int64_t)r * I2 + f) = gv;
                *(u32x2*)(p.out2 + (int64_t)r * I2 + I + f) = uv;
              }
            }
          }
      }
    } else if constexpr (MODE == G2DX) {
      const int r = row0 + trow;
      if (r < row_end) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int f = ct * BC + wc * 128 + i * 32 + 8 * q + 4 * hl;
            if (f < I) {
              const u32x2 gv = *(const u32x2*)(p.a1 + (int64_t)r * I2 + f);
              const u32x2 uv = *(const u32x2*)(p.a1 + (int64_t)r * I2 + I + f);
              float g[4] = {bf_lo(gv[0]), bf_hi(gv[0]), bf_lo(gv[1]), bf_hi(gv[1])};
              float u[4] = {bf_lo(uv[0]), bf_hi(uv[0]), bf_lo(uv[1]), bf_hi(uv[1])};
              float dg[4], du[4];
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                const float da = round_bf(acc[i][j][4 * q + v]);
                const float sg = sigmoidf_(g[v]);
                const float s = round_bf(siluf_(g[v]));       // silu(g) as stored in bf16
                const float ds = round_bf(da * u[v]);          // d silu(g)
                du[v] = da * s;
                dg[v] = ds * (sg * (1.f + g[v] * (1.f - sg)));
              }
              u32x2 dgv = {pack_bf2(dg[0], dg[1]), pack_bf2(dg[2], dg[3])};
              u32x2 duv = {pack_bf2(du[0], du[1]), pack_bf2(du[2], du[3])};
              *(u32x2*)(p.out + (int64_t)r * I2 + f) = dgv;
              *(u32x2*)(p.out + (int64_t)r * I2 + I + f) = duv;
            }
          }
      }
    } else {
      // Plain bf16 store: y (G2F), d_xs (G1DX), d_down_proj (G2DW), d_gate_up_proj (G1DW).
      int r, ld, nrows;
      bf16* obase;
      if constexpr (TOKEN) {
        r = row0 + trow;
        nrows = row_end;
        ld = (MODE == G2F || MODE == G1DX) ? H : 0;
        obase = p.out;
      } else {
        r = row0 + trow;
        nrows = (MODE == G2DW) ? H : I2;
        ld = (MODE == G2DW) ? I : H;
        obase = p.out + (int64_t)e * (MODE == G2DW ? (int64_t)H * I : (int64_t)I2 * H);
      }
      const int ncols = ld;
      if (r < nrows) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int f = ct * BC + wc * 128 + i * 32 + 8 * q + 4 * hl;
            if (f < ncols) {
              u32x2 v = {pack_bf2(acc[i][j][4 * q + 0], acc[i][j][4 * q + 1]),
                         pack_bf2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3])};
              *(u32x2*)(obase + (int64_t)r * ld + f) = v;
            }
          }
      }
    }
  }
}

template <int MODE, int BR>
int launch(const GemmArgs& a, hipStream_t st) {
  const size_t lds = (size_t)2 * (BC + BR) * BK * sizeof(bf16);
  if (a.n_logical <= 0) return MOE_OK;
  hipError_t err = hipFuncSetAttribute((const void*)grouped_gemm_kernel<MODE, BR>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (err != hipSuccess) {
    set_error("grouped_gemm: hipFuncSetAttribute failed: %s", hipGetErrorString(err));
    return MOE_ERR_HIP;
  }
  const int grid = (a.n_logical + 7) / 8 * 8;
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
                 const int32_t* tile_starts, hipStream_t st) {
  const int br = pick_br(S, E);
  a.tile_starts = tile_starts + (size_t)tile_index(br) * (E + 1);
  a.n_ct = (ncols_total + ncols_per_tile_out - 1) / ncols_per_tile_out;
  const int64_t max_rt = (S + br - 1) / br + E;
  const int64_t nl = max_rt * a.n_ct;
  if (nl > (int64_t)1 << 30) {
    set_error("grouped_gemm: grid too large");
    return MOE_ERR_UNSUPPORTED;
  }
  a.n_logical = (int)nl;
  if (br == 256) return launch<MODE, 256>(a, st);
  if (br == 128) return launch<MODE, 128>(a, st);
  return launch<MODE, 64>(a, st);
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
                                           const int32_t* tile_starts, const void* gate_up_proj,
                                           int64_t T, int64_t S, int E, int H, int I, int dtype,
                                           void* gate_up_out, void* act_out, void* stream) {
  const char* who = "gemm_gate_up_swiglu";
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(top_k >= 1 && S == T * top_k, MOE_ERR_ARG, "%s: S != T*top_k", who);
  MOE_REQUIRE(T * (int64_t)H * 2 < ((int64_t)1 << 31), MOE_ERR_UNSUPPORTED, "%s: T*H too large",
              who);
  MOE_REQUIRE(hidden_states && row_src && offsets && tile_starts && gate_up_proj && act_out,
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
  return launch_token<G1F>(a, S, E, 128, I, tile_starts, (hipStream_t)stream);
}

extern "C" int moe_amd_gemm_down(const void* act, const int32_t* offsets,
                                 const int32_t* tile_starts, const void* down_proj, int64_t S,
                                 int E, int H, int I, int dtype, void* y_out, void* stream) {
  const char* who = "gemm_down";
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(act && offsets && tile_starts && down_proj && y_out, MOE_ERR_ARG,
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
  return launch_token<G2F>(a, S, E, BC, H, tile_starts, (hipStream_t)stream);
}

extern "C" int moe_amd_gemm_down_backward_dx_dswiglu(const void* dy, const int32_t* offsets,
                                                     const int32_t* tile_starts,
                                                     const void* down_proj, const void* gate_up,
                                                     int64_t S, int E, int H, int I, int dtype,
                                                     void* d_gate_up, void* stream) {
  const char* who = "gemm_down_backward_dx_dswiglu";
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(dy && offsets && tile_starts && down_proj && gate_up && d_gate_up, MOE_ERR_ARG,
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
  return launch_token<G2DX>(a, S, E, BC, I, tile_starts, (hipStream_t)stream);
}

extern "C" int moe_amd_gemm_gate_up_backward_dx(const void* d_gate_up, const int32_t* offsets,
                                                const int32_t* tile_starts,
                                                const void* gate_up_proj, int64_t S, int E,
                                                int H, int I, int dtype, void* d_xs,
                                                void* stream) {
  const char* who = "gemm_gate_up_backward_dx";
  int rc = check_common(S, E, H, I, dtype, who);
  if (rc) return rc;
  MOE_REQUIRE(d_gate_up && offsets && tile_starts && gate_up_proj && d_xs, MOE_ERR_ARG,
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
  return launch_token<G1DX>(a, S, E, BC, H, tile_starts, (hipStream_t)stream);
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
  a.n_logical = E * a.n_rt * a.n_ct;
  return launch<G2DW, 256>(a, (hipStream_t)stream);
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
  a.n_logical = E * a.n_rt * a.n_ct;
  return launch<G1DW, 256>(a, (hipStream_t)stream);
}
