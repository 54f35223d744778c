// Shared declarations of the fused-FFN kernels (ffn.hip, ffn_wide.hip).
#pragma once

#include "mpk_common.h"

namespace mpk {

struct FfnArgs {
  const void* x;
  const _Float16* w_in;   // [F, D]
  const _Float16* b_in;   // [F]
  const _Float16* w_out;  // [D, F]
  const _Float16* b_out;  // [D]
  const float* residual;  // [M, D]
  const float* gamma;
  const float* beta;
  float* residual_out;
  void* normalized_out;
  int64_t m;
  int f;
  float eps;
};

// Largest hidden width the wide kernel takes (its FP32 b_in sits in LDS).
constexpr int kWideFfnMaxF = 8192;

// Whether the wide kernel (ffn_wide.hip) covers (d, f), and its launcher
// (x_dtype / out_dtype: kF32 or kF16; w_dtype is always kF16).
bool ffn_wide_supported(int d, int f);
hipError_t launch_ffn_wide(const FfnArgs& a, int d, int w_dtype, int x_dtype, int out_dtype, hipStream_t s);
// The role-split wide kernel (vector waves + matrix waves; same shapes as ffn_wide_supported).
hipError_t launch_ffn_roles(const FfnArgs& a, int d, int w_dtype, int x_dtype, int out_dtype, hipStream_t s);

}  // namespace mpk
