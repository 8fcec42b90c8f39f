// fp32 grouped GEMMs of the expert layer on gfx950 MFMA (v_mfma_f32_32x32x2_f32).
//
// The fp32 configurations of the reference (its CPU-runnable XS standard
// layer) run the experts in fp32: F.grouped_mm on fp32 operands with fp32
// accumulation and no intermediate rounding (transformers/integrations/
// moe.py:439-459 forward, :226-242 backward formulas).  This file is that
// path: the same six GEMMs as the bf16 kernels, unfused backward (the
// combine backward and the gather backward run as their own kernels), every
// product and sum in fp32.
//
//   mode  C [rows x cols]          rows (operand)                 cols (operand)              k
//   F1    gate_up -> act           routed rows (x gathered, kc)   [gate 64 | up 64] (W1, kc)  H
//   F2    y                        routed rows (act, kc)          H (W2[e], kc)               I
//   FDX2  d_act -> d_gate_up       routed rows (dy, kc)           I (W2[e], km)               H
//   FDX1  d_xs                     routed rows (d_gate_up, kc)    H (W1[e], km)               2I
//   FDW2  d_down_proj[e]           H (dy rows of e, km)           I (act rows of e, km)       rows of e
//   FDW1  d_gate_up_proj[e]        2I (d_gate_up rows, km)        H (x gathered, km)          rows of e
//
// (kc: the operand's k index is contiguous in memory; km: its feature index
// is, k strides by rows.)
//
// Workgroup: 256 threads = 4 waves as 2 x 2, a 128 x 128 tile of C, each wave
// a 64 x 64 block of 2 x 2 MFMA sub-tiles (64 fp32 accumulators per lane).
// A k-stage is 32 deep: both operands are loaded global -> registers (16
// bytes per load, coalesced along the contiguous index) and written to LDS
// as [feature][k] rows of 36 floats (144 bytes: the 16-byte fragment reads of
// eight consecutive features hit distinct banks); km operands are transposed
// on the way in.  Two stage buffers: the loads of stage s+1 are in flight
// while stage s is multiplied.  MFMA 32x32x2: lane L supplies feature L % 32
// at k' = L / 32 of each operand; a lane reads 4 consecutive k of its
// feature (k = 8kk + 4(L/32) + s, s = 0..3) with one ds_read_b128 and feeds
// them to four MFMAs, so the k pairs (8kk + s, 8kk + 4 + s) of one call are
// a permutation of the stage's k range.  Output: register 4q+c of a lane
// holds (tile row L % 32, tile column 8q + 4(L/32) + c) of the sub-tile (the
// column operand is MFMA's "A").  Epilogue: the tile is staged in LDS
// (reusing the stage buffers) and written out row by row with 16-byte lanes,
// applying the SwiGLU / dSwiGLU tail in fp32.
//
// Token-grouped tiles come from the permutation's row-tile table for 128-row
// tiles ({expert, first row, end row} per tile, device-side); dW tiles are
// (expert, row tile, column tile), their k range the expert's rows.
#include "common.h"
#include "gemm_f32.h"

namespace moe {
namespace {

constexpr int FBM = 128;          // tile rows
constexpr int FBN = 128;          // tile columns
constexpr int FBK = 32;           // k per stage
constexpr int FLD = FBK + 4;      // floats per feature row of a stage in LDS
constexpr int FSTG = FBN + 4;     // floats per row of the epilogue staging tile
constexpr int FNT = 256;          // threads per workgroup
constexpr int FTILE_TABLE = 1;    // the permutation's 128-row tile table
constexpr size_t kStageFloats = (size_t)(FBM + FBN) * FLD;
constexpr size_t kLdsBytes =
    (2 * kStageFloats > (size_t)FBM * FSTG ? 2 * kStageFloats : (size_t)FBM * FSTG) * sizeof(float);

enum FMode { F1 = 0, F2 = 1, FDX2 = 2, FDX1 = 3, FDW2 = 4, FDW1 = 5 };

struct FArgs {
  const float* x;         // hidden_states [T,H]
  const float* w;         // gate_up_proj [E,2I,H] or down_proj [E,H,I]
  const float* a0;        // act [S,I] (F2) | dy [S,H] (FDX2, FDW2) | d_gate_up [S,2I] (FDX1, FDW1)
  const float* a1;        // gate_up [S,2I] (FDX2) | act [S,I] (FDW2)
  const int* row_src;     // [S]
  const int* offsets;     // [E+1]
  const int* tile_count;  // token modes: number of 128-row tiles
  const int4* tile_info;  // token modes: {expert, first row, end row, 0} per row tile
  float* out;
  float* out2;            // F1: gate_up [S,2I] (may be null)
  int64_t T, S;
  int E, H, I, topk;
  int n_ct, n_rt;         // column tiles; dW modes: row tiles per expert
};

__device__ __forceinline__ f32x4 ld4(const float* p) { return *(const f32x4*)p; }

template <int MODE>
__global__ __launch_bounds__(FNT) void f32_gemm_kernel(FArgs p) {
  constexpr bool TOKEN = MODE == F1 || MODE == F2 || MODE == FDX2 || MODE == FDX1;
  constexpr bool COL_KM = MODE != F1 && MODE != F2;
  constexpr bool ROW_KM = MODE == FDW2 || MODE == FDW1;
  extern __shared__ __attribute__((aligned(16))) float fsm[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wid >> 1, wc = wid & 1;
  const int l32 = lane & 31, hl = lane >> 5;
  const int H = p.H, I = p.I, I2 = 2 * p.I;

  // ------------------------------------------------------------ the tile
  int e, row0 = 0, row_end = 0, ct, rt = 0, kbeg = 0, kend = 0;
  if constexpr (TOKEN) {
    const int rtile = (int)(blockIdx.x / (unsigned)p.n_ct);
    ct = (int)(blockIdx.x % (unsigned)p.n_ct);
    if (rtile >= *p.tile_count) return;
    const int4 ti = p.tile_info[rtile];
    e = ti.x;
    row0 = ti.y;
    row_end = ti.z;
  } else {
    const int per_e = p.n_rt * p.n_ct;
    e = (int)(blockIdx.x / (unsigned)per_e);
    const int rem = (int)(blockIdx.x % (unsigned)per_e);
    rt = rem / p.n_ct;
    ct = rem % p.n_ct;
    kbeg = p.offsets[e];
    kend = p.offsets[e + 1];
  }
  int K_len;
  if constexpr (MODE == F1 || MODE == FDX2) K_len = H;
  else if constexpr (MODE == F2) K_len = I;
  else if constexpr (MODE == FDX1) K_len = I2;
  else K_len = kend - kbeg;
  const int nk = (K_len + FBK - 1) / FBK;

  // ------------------------------------------------------ operand loads
  // kc operand: thread t loads features t/8 + 32i (i = 0..3), k 4(t%8)..+3.
  // km operand: thread t loads k rows t/32 + 8i, features 4(t%32)..+3.
  const int kc_f = tid >> 3, kc_k = (tid & 7) * 4;
  const int km_k = tid >> 5, km_f = (tid & 31) * 4;

  // Row operand, per load i: base pointer of the feature row (kc) or of
  // feature column 0 of the k range (km), and a validity mask.
  const float* rbase[4];
  bool rok[4];
  int64_t rld = 0;  // km: floats between k rows
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (MODE == F1) {
      const int r = row0 + kc_f + 32 * i;
      rok[i] = r < row_end;
      const int tok = rok[i] ? p.row_src[r] / p.topk : 0;
      rbase[i] = p.x + (int64_t)tok * H;
    } else if constexpr (TOKEN) {
      const int ld = MODE == F2 ? I : (MODE == FDX2 ? H : I2);
      const int r = row0 + kc_f + 32 * i;
      rok[i] = r < row_end;
      rbase[i] = p.a0 + (int64_t)(rok[i] ? r : row0) * ld;
    } else {
      const int nf = MODE == FDW2 ? H : I2;  // features of the row operand
      const int f = rt * FBM + km_f;
      rok[i] = f < nf;
      rld = nf;
      rbase[i] = p.a0 + (int64_t)kbeg * nf + (rok[i] ? f : 0);
    }
  }
  // Column operand.
  const float* cbase[4];
  bool cok[4];
  int64_t cld = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (MODE == F1) {
      const int c = kc_f + 32 * i;  // tile column: gate features 0..63, up features 64..127
      const int feat = ct * 64 + (c & 63);
      cok[i] = feat < I;
      const int wrow = (c < 64 ? 0 : I) + (cok[i] ? feat : 0);
      cbase[i] = p.w + ((int64_t)e * I2 + wrow) * H;
    } else if constexpr (MODE == F2) {
      const int h = ct * FBN + kc_f + 32 * i;
      cok[i] = h < H;
      cbase[i] = p.w + ((int64_t)e * H + (cok[i] ? h : 0)) * I;
    } else {
      int nf;
      const float* b;
      if constexpr (MODE == FDX2) {  // down_proj[e] [H][I]: k = h, feature = i
        nf = I;
        b = p.w + (int64_t)e * H * I;
        cld = I;
      } else if constexpr (MODE == FDX1) {  // gate_up_proj[e] [2I][H]: k = j, feature = h
        nf = H;
        b = p.w + (int64_t)e * I2 * H;
        cld = H;
      } else if constexpr (MODE == FDW2) {  // act rows of e [rows][I]
        nf = I;
        b = p.a1 + (int64_t)kbeg * I;
        cld = I;
      } else {  // FDW1: hidden_states rows gathered through row_src (per stage)
        nf = H;
        b = p.x;
        cld = H;
      }
      const int f = ct * FBN + km_f;
      cok[i] = f < nf;
      cbase[i] = b + (cok[i] ? f : 0);
    }
  }

  f32x4 rv[4], cv[4];
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  auto load_stage = [&](int s) {
    const int k0 = s * FBK;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (!ROW_KM) {
        rv[i] = rok[i] ? ld4(rbase[i] + k0 + kc_k) : zero4;
      } else {
        const int k = k0 + km_k + 8 * i;
        rv[i] = (rok[i] && k < K_len) ? ld4(rbase[i] + (int64_t)k * rld) : zero4;
      }
      if constexpr (!COL_KM) {
        cv[i] = cok[i] ? ld4(cbase[i] + k0 + kc_k) : zero4;
      } else if constexpr (MODE == FDW1) {
        const int k = k0 + km_k + 8 * i;
        const bool ok = cok[i] && k < K_len;
        const int tok = ok ? p.row_src[kbeg + k] / p.topk : 0;
        cv[i] = ok ? ld4(cbase[i] + (int64_t)tok * H) : zero4;
      } else {
        const int k = k0 + km_k + 8 * i;
        cv[i] = (cok[i] && k < K_len) ? ld4(cbase[i] + (int64_t)k * cld) : zero4;
      }
    }
  };
  // Stage buffer b: row operand [FBM][FLD] then column operand [FBN][FLD].
  auto store_stage = [&](int b) {
    float* R = fsm + (size_t)b * kStageFloats;
    float* C = R + FBM * FLD;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (!ROW_KM) {
        *(f32x4*)(R + (kc_f + 32 * i) * FLD + kc_k) = rv[i];
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) R[(km_f + j) * FLD + km_k + 8 * i] = rv[i][j];
      }
      if constexpr (!COL_KM) {
        *(f32x4*)(C + (kc_f + 32 * i) * FLD + kc_k) = cv[i];
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) C[(km_f + j) * FLD + km_k + 8 * i] = cv[i][j];
      }
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  if (nk > 0) {
    load_stage(0);
    store_stage(0);
    __syncthreads();
    for (int s = 0; s < nk; ++s) {
      if (s + 1 < nk) load_stage(s + 1);
      const float* R = fsm + (size_t)(s & 1) * kStageFloats;
      const float* C = R + FBM * FLD;
#pragma unroll
      for (int kk = 0; kk < FBK / 8; ++kk) {
        f32x4 a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) a[i] = ld4(C + (wc * 64 + i * 32 + l32) * FLD + kk * 8 + 4 * hl);
#pragma unroll
        for (int j = 0; j < 2; ++j) b[j] = ld4(R + (wr * 64 + j * 32 + l32) * FLD + kk * 8 + 4 * hl);
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][q], b[j][q], acc[i][j], 0, 0, 0);
      }
      // Stage s+1 goes to the other buffer, last read in step s-1 (every
      // wave passed the barrier after that step).
      if (s + 1 < nk) store_stage((s + 1) & 1);
      __syncthreads();
    }
  }

  // ------------------------------------------------------------ epilogue
  // The stage buffers are free (the loop ended with a barrier).
  float* stg = fsm;  // [FBM][FSTG]
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = wr * 64 + j * 32 + l32;
        const int col = wc * 64 + i * 32 + 8 * q + 4 * hl;
        const f32x4 v = {acc[i][j][4 * q + 0], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                         acc[i][j][4 * q + 3]};
        *(f32x4*)(stg + row * FSTG + col) = v;
      }
  __syncthreads();

  if constexpr (MODE == F1) {
    // act = silu(gate) * up, silu(g) = g / (1 + exp(-g)) as torch evaluates it
    const int f4 = (tid & 15) * 4;
    const int feat = ct * 64 + f4;
    for (int rr = tid >> 4; rr < FBM; rr += FNT / 16) {
      const int r = row0 + rr;
      if (r >= row_end || feat >= I) continue;
      const f32x4 g = ld4(stg + rr * FSTG + f4);
      const f32x4 u = ld4(stg + rr * FSTG + 64 + f4);
      f32x4 a;
#pragma unroll
      for (int c = 0; c < 4; ++c) a[c] = g[c] / (1.0f + expf(-g[c])) * u[c];
      *(f32x4*)(p.out + (int64_t)r * I + feat) = a;
      if (p.out2) {
        *(f32x4*)(p.out2 + (int64_t)r * I2 + feat) = g;
        *(f32x4*)(p.out2 + (int64_t)r * I2 + I + feat) = u;
      }
    }
  } else if constexpr (MODE == FDX2) {
    // d_act -> d_gate = d_act * up * sigmoid(g) * (1 + g * (1 - sigmoid(g))),
    //          d_up = d_act * silu(g)   (autograd of silu(gate) * up)
    const int c4 = (tid & 31) * 4;
    const int i0 = ct * FBN + c4;
    for (int rr = tid >> 5; rr < FBM; rr += FNT / 32) {
      const int r = row0 + rr;
      if (r >= row_end || i0 >= I) continue;
      const f32x4 da = ld4(stg + rr * FSTG + c4);
      const f32x4 g = ld4(p.a1 + (int64_t)r * I2 + i0);
      const f32x4 u = ld4(p.a1 + (int64_t)r * I2 + I + i0);
      f32x4 dg, du;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float sg = 1.0f / (1.0f + expf(-g[c]));
        const float sl = g[c] / (1.0f + expf(-g[c]));
        du[c] = da[c] * sl;
        dg[c] = da[c] * u[c] * (sg * (1.0f + g[c] * (1.0f - sg)));
      }
      *(f32x4*)(p.out + (int64_t)r * I2 + i0) = dg;
      *(f32x4*)(p.out + (int64_t)r * I2 + I + i0) = du;
    }
  } else {
    // Plain tile: y (F2), d_xs (FDX1), d_down_proj[e] (FDW2), d_gate_up_proj[e] (FDW1).
    const int c4 = (tid & 31) * 4;
    int nrows, ncols, rbeg;
    int64_t ld;
    float* ob;
    if constexpr (TOKEN) {
      nrows = row_end;
      rbeg = row0;
      ncols = H;
      ld = H;
      ob = p.out;
    } else {
      nrows = MODE == FDW2 ? H : I2;
      rbeg = rt * FBM;
      ncols = MODE == FDW2 ? I : H;
      ld = ncols;
      ob = p.out + (int64_t)e * nrows * ncols;
    }
    const int col = ct * FBN + c4;
    for (int rr = tid >> 5; rr < FBM; rr += FNT / 32) {
      const int r = rbeg + rr;
      if (r < nrows && col < ncols) *(f32x4*)(ob + (int64_t)r * ld + col) = ld4(stg + rr * FSTG + c4);
    }
  }
}

template <int MODE>
int launch_f32(const FArgs& a, int64_t blocks, hipStream_t st, const char* who) {
  if (blocks <= 0) return MOE_OK;
  MOE_REQUIRE(blocks < ((int64_t)1 << 31), MOE_ERR_UNSUPPORTED, "%s: too many tiles", who);
  static std::atomic<int> lds_done[64];
  hipError_t err = set_dynamic_lds_once(lds_done, (const void*)f32_gemm_kernel<MODE>, (int)kLdsBytes);
  if (err != hipSuccess) {
    set_error("%s: hipFuncSetAttribute failed: %s", who, hipGetErrorString(err));
    return MOE_ERR_HIP;
  }
  f32_gemm_kernel<MODE><<<(unsigned)blocks, FNT, kLdsBytes, st>>>(a);
  return check_launch(who);
}

int check_f32(int64_t S, int E, int H, int I, const char* who) {
  MOE_REQUIRE(S >= 0 && E >= 1 && H > 0 && I > 0, MOE_ERR_ARG, "%s: bad sizes", who);
  MOE_REQUIRE(H % 64 == 0 && I % 64 == 0, MOE_ERR_ARG,
              "%s: H=%d and I=%d must be multiples of 64", who, H, I);
  MOE_REQUIRE(S < ((int64_t)1 << 31), MOE_ERR_UNSUPPORTED, "%s: S out of range", who);
  return MOE_OK;
}

bool al16f(const void* p) { return ((uintptr_t)p & 15) == 0; }

#define F32_ALIGNED(ptr, who) \
  MOE_REQUIRE(al16f(ptr), MOE_ERR_ALIGN, "%s: pointer %s not 16-byte aligned", who, #ptr)

// Token-grouped launch: one workgroup per (128-row tile, column tile); the
// row-tile count is on the device, so the grid covers the most tiles the
// plan can hold and surplus workgroups return at once.
template <int MODE>
int launch_f32_token(FArgs a, const void* tile_plan, int ncols_per_tile, int ncols,
                     hipStream_t st, const char* who) {
  const char* pb = (const char*)tile_plan;
  a.tile_count = (const int*)pb + (size_t)FTILE_TABLE * (a.E + 1) + a.E;
  a.tile_info = (const int4*)(pb + plan_info_offset(a.S, a.E, FTILE_TABLE));
  a.n_ct = (ncols + ncols_per_tile - 1) / ncols_per_tile;
  return launch_f32<MODE>(a, plan_max_tiles(a.S, a.E, FTILE_TABLE) * a.n_ct, st, who);
}

}  // namespace

int f32_gate_up_swiglu(const float* x, const int32_t* row_src, int top_k, const int32_t* offsets,
                       const void* tile_plan, const float* w1, int64_t T, int64_t S, int E, int H,
                       int I, float* gate_up, float* act, hipStream_t st) {
  const char* who = "gemm_gate_up_swiglu (fp32)";
  int rc = check_f32(S, E, H, I, who);
  if (rc) return rc;
  MOE_REQUIRE(top_k >= 1 && S == T * top_k, MOE_ERR_ARG, "%s: S != T*top_k", who);
  MOE_REQUIRE(offsets && tile_plan && w1 && (S == 0 || (x && row_src && act)), MOE_ERR_ARG,
              "%s: null pointer", who);
  F32_ALIGNED(x, who);
  F32_ALIGNED(w1, who);
  F32_ALIGNED(act, who);
  F32_ALIGNED(gate_up, who);
  if (S == 0) return MOE_OK;
  FArgs a{};
  a.x = x; a.w = w1; a.row_src = row_src; a.offsets = offsets; a.out = act; a.out2 = gate_up;
  a.T = T; a.S = S; a.E = E; a.H = H; a.I = I; a.topk = top_k;
  return launch_f32_token<F1>(a, tile_plan, 64, I, st, who);
}

int f32_down(const float* act, const int32_t* offsets, const void* tile_plan, const float* w2,
             int64_t S, int E, int H, int I, float* y, hipStream_t st) {
  const char* who = "gemm_down (fp32)";
  int rc = check_f32(S, E, H, I, who);
  if (rc) return rc;
  MOE_REQUIRE(offsets && tile_plan && w2 && (S == 0 || (act && y)), MOE_ERR_ARG,
              "%s: null pointer", who);
  F32_ALIGNED(act, who);
  F32_ALIGNED(w2, who);
  F32_ALIGNED(y, who);
  if (S == 0) return MOE_OK;
  FArgs a{};
  a.w = w2; a.a0 = act; a.offsets = offsets; a.out = y;
  a.S = S; a.E = E; a.H = H; a.I = I;
  return launch_f32_token<F2>(a, tile_plan, FBN, H, st, who);
}

int f32_down_dx_dswiglu(const float* dy, const int32_t* offsets, const void* tile_plan,
                        const float* w2, const float* gate_up, int64_t S, int E, int H, int I,
                        float* d_gate_up, hipStream_t st) {
  const char* who = "gemm_down_backward_dx_dswiglu (fp32)";
  int rc = check_f32(S, E, H, I, who);
  if (rc) return rc;
  MOE_REQUIRE(offsets && tile_plan && w2 && (S == 0 || (dy && gate_up && d_gate_up)),
              MOE_ERR_ARG, "%s: null pointer", who);
  F32_ALIGNED(dy, who);
  F32_ALIGNED(w2, who);
  F32_ALIGNED(gate_up, who);
  F32_ALIGNED(d_gate_up, who);
  if (S == 0) return MOE_OK;
  FArgs a{};
  a.w = w2; a.a0 = dy; a.a1 = gate_up; a.offsets = offsets; a.out = d_gate_up;
  a.S = S; a.E = E; a.H = H; a.I = I;
  return launch_f32_token<FDX2>(a, tile_plan, FBN, I, st, who);
}

int f32_gate_up_dx(const float* dgu, const int32_t* offsets, const void* tile_plan,
                   const float* w1, int64_t S, int E, int H, int I, float* d_xs,
                   hipStream_t st) {
  const char* who = "gemm_gate_up_backward_dx (fp32)";
  int rc = check_f32(S, E, H, I, who);
  if (rc) return rc;
  MOE_REQUIRE(offsets && tile_plan && w1 && (S == 0 || (dgu && d_xs)), MOE_ERR_ARG,
              "%s: null pointer", who);
  F32_ALIGNED(dgu, who);
  F32_ALIGNED(w1, who);
  F32_ALIGNED(d_xs, who);
  if (S == 0) return MOE_OK;
  FArgs a{};
  a.w = w1; a.a0 = dgu; a.offsets = offsets; a.out = d_xs;
  a.S = S; a.E = E; a.H = H; a.I = I;
  return launch_f32_token<FDX1>(a, tile_plan, FBN, H, st, who);
}

int f32_down_dw(const float* dy, const float* act, const int32_t* offsets, int64_t S, int E,
                int H, int I, float* d_w2, hipStream_t st) {
  const char* who = "gemm_down_backward_dw (fp32)";
  int rc = check_f32(S, E, H, I, who);
  if (rc) return rc;
  MOE_REQUIRE(offsets && d_w2 && (S == 0 || (dy && act)), MOE_ERR_ARG, "%s: null pointer", who);
  F32_ALIGNED(dy, who);
  F32_ALIGNED(act, who);
  F32_ALIGNED(d_w2, who);
  FArgs a{};
  a.a0 = dy; a.a1 = act; a.offsets = offsets; a.out = d_w2;
  a.S = S; a.E = E; a.H = H; a.I = I;
  a.n_rt = (H + FBM - 1) / FBM;
  a.n_ct = (I + FBN - 1) / FBN;
  // every expert's tiles are written (zeros for an expert without rows)
  return launch_f32<FDW2>(a, (int64_t)E * a.n_rt * a.n_ct, st, who);
}

int f32_gate_up_dw(const float* dgu, const float* x, const int32_t* row_src, int top_k,
                   const int32_t* offsets, int64_t T, int64_t S, int E, int H, int I,
                   float* d_w1, hipStream_t st) {
  const char* who = "gemm_gate_up_backward_dw (fp32)";
  int rc = check_f32(S, E, H, I, who);
  if (rc) return rc;
  MOE_REQUIRE(top_k >= 1 && S == T * top_k, MOE_ERR_ARG, "%s: S != T*top_k", who);
  MOE_REQUIRE(offsets && d_w1 && (S == 0 || (dgu && x && row_src)), MOE_ERR_ARG,
              "%s: null pointer", who);
  F32_ALIGNED(dgu, who);
  F32_ALIGNED(x, who);
  F32_ALIGNED(d_w1, who);
  FArgs a{};
  a.x = x; a.a0 = dgu; a.row_src = row_src; a.offsets = offsets; a.out = d_w1;
  a.T = T; a.S = S; a.E = E; a.H = H; a.I = I; a.topk = top_k;
  a.n_rt = (2 * I + FBM - 1) / FBM;
  a.n_ct = (H + FBN - 1) / FBN;
  return launch_f32<FDW1>(a, (int64_t)E * a.n_rt * a.n_ct, st, who);
}

}  // namespace moe
