// fp32 grouped GEMMs of the expert layer (gemm_f32.hip), called by the
// grouped-GEMM entry points of gemm.hip when their dtype is MOE_DTYPE_F32.
// Arguments as those entry points document; every pointer is fp32 except the
// int32 routing plan.  Shapes and pointers are checked here.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

int f32_gate_up_swiglu(const float* hidden_states, const int32_t* row_src, int top_k,
                       const int32_t* offsets, const void* tile_plan, const float* gate_up_proj,
                       int64_t T, int64_t S, int E, int H, int I, float* gate_up_out,
                       float* act_out, hipStream_t st);
int f32_down(const float* act, const int32_t* offsets, const void* tile_plan,
             const float* down_proj, int64_t S, int E, int H, int I, float* y_out,
             hipStream_t st);
int f32_down_dx_dswiglu(const float* dy, const int32_t* offsets, const void* tile_plan,
                        const float* down_proj, const float* gate_up, int64_t S, int E, int H,
                        int I, float* d_gate_up, hipStream_t st);
int f32_down_dw(const float* dy, const float* act, const int32_t* offsets, int64_t S, int E,
                int H, int I, float* d_down_proj, hipStream_t st);
int f32_gate_up_dx(const float* d_gate_up, const int32_t* offsets, const void* tile_plan,
                   const float* gate_up_proj, int64_t S, int E, int H, int I, float* d_xs,
                   hipStream_t st);
int f32_gate_up_dw(const float* d_gate_up, const float* hidden_states, const int32_t* row_src,
                   int top_k, const int32_t* offsets, int64_t T, int64_t S, int E, int H, int I,
                   float* d_gate_up_proj, hipStream_t st);

}  // namespace moe
