// Fused FFN + residual + LayerNorm for gfx950.
//
// Replaces the reference's Triton kernel
//   _mixed_ffn_add_layer_norm_kernel  mixed_precision/triton_linear.py:128-185
// which is hard-wired to D = F = 128; this one covers any D in {32, 64, 128,
// 256, 512} and F a multiple of 32.
//
//   H  = GELU_erf(fp16(X) W_in^T + b_in)        FP32 accumulate, FP32 GELU
//   R' = fp16(H) W_out^T + b_out + R            FP32
//   N' = LayerNorm(R') (two-pass FP32 statistics), stored FP32 or FP16
//
// Structure.  Each wave owns 16*TM token rows and keeps their FP16 X fragments
// in registers for the whole F loop.  The hidden activation never leaves the
// register file: H^T = W_in X^T is computed 32 features at a time with the
// paired row mapping (mpk_common.h), so after bias + GELU + FP16 rounding each
// lane already holds the B operand of the second product R^T += W_out H^T.
// W_in / W_out are staged through LDS in chunks of FC hidden features; when the
// whole F fits (one chunk) the workgroup loads them once and then walks a
// persistent loop over row tiles without further barriers.
#include <algorithm>
#include <type_traits>

#include "ffn.h"

namespace mpk {

template <int D, int FC, int TM, typename XT, typename OT>
__global__ __launch_bounds__(kBlock) void ffn_ln_kernel(FfnArgs a) {
  constexpr int KS = D / 32;   // k-steps of the first product
  constexpr int PN = D / 32;   // output feature pairs
  constexpr int LDI = D + 8;   // W_in chunk row stride (halves)
  constexpr int LDO = FC + 8;  // W_out chunk row stride (halves)
  constexpr int BM = 64 * TM;
  static_assert(D % 32 == 0 && FC % 32 == 0, "shape");

  __shared__ _Float16 wi_lds[FC * LDI];
  __shared__ _Float16 wo_lds[D * LDO];

  const XT* __restrict__ X = static_cast<const XT*>(a.x);
  OT* __restrict__ NO = static_cast<OT*>(a.normalized_out);
  const int64_t M = a.m;
  const int F = a.f;
  const int nchunks = (F + FC - 1) / FC;
  const int64_t ntiles = (M + BM - 1) / BM;

  const int l = threadIdx.x & 63, wave = wave_id();
  const int r = l & 15, g = l >> 4;

  auto load_chunk = [&](int fc) {
    // W_in rows [fc, fc+FC) x all D columns
    for (int c = threadIdx.x; c < FC * (D / 8); c += kBlock) {
      const int row = c / (D / 8), col = (c % (D / 8)) * 8;
      const int gf = fc + row;
      h8 v = gf < F ? *reinterpret_cast<const h8*>(a.w_in + (int64_t)gf * D + col) : zero_h8();
      *reinterpret_cast<h8*>(&wi_lds[row * LDI + col]) = v;
    }
    // W_out all D rows x columns [fc, fc+FC)
    for (int c = threadIdx.x; c < D * (FC / 8); c += kBlock) {
      const int row = c / (FC / 8), col = (c % (FC / 8)) * 8;
      const int gf = fc + col;
      h8 v = gf < F ? *reinterpret_cast<const h8*>(a.w_out + (int64_t)row * F + gf) : zero_h8();
      *reinterpret_cast<h8*>(&wo_lds[row * LDO + col]) = v;
    }
  };

  if (nchunks == 1) {
    load_chunk(0);
    __syncthreads();
  }

  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t m0 = tile * BM + wave * 16 * TM;

    h8 xf[TM][KS];
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      const int64_t m = m0 + 16 * t + r;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) xf[t][ks] = m < M ? load8_as_half(X + m * D + ks * 32 + 8 * g) : zero_h8();
    }

    f4 yacc[PN][2][TM];
#pragma unroll
    for (int p = 0; p < PN; ++p)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int t = 0; t < TM; ++t) yacc[p][tt][t] = zero4();

    for (int ch = 0; ch < nchunks; ++ch) {
      const int fc = ch * FC;
      if (nchunks > 1) {
        __syncthreads();
        load_chunk(fc);
        __syncthreads();
      }
#pragma unroll 1
      for (int q = 0; q < FC / 32; ++q) {
        if (fc + 32 * q >= F) break;
        // H^T pair (32 hidden features x 16*TM rows)
        f4 hacc[2][TM];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int t = 0; t < TM; ++t) hacc[tt][t] = zero4();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            const h8 w = *reinterpret_cast<const h8*>(&wi_lds[(32 * q + pair_row(r, tt)) * LDI + ks * 32 + 8 * g]);
#pragma unroll
            for (int t = 0; t < TM; ++t) hacc[tt][t] = mfma32(w, xf[t][ks], hacc[tt][t]);
          }
        }
        float bin[8];
        load8_f16_to_f32(a.b_in + fc + 32 * q + 8 * g, bin);
        h8 hb[TM];
#pragma unroll
        for (int t = 0; t < TM; ++t)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) hb[t][4 * tt + i] = (_Float16)gelu_erf(hacc[tt][t][i] + bin[4 * tt + i]);
        // R^T += W_out[:, pair] H^T
#pragma unroll
        for (int p = 0; p < PN; ++p)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            const h8 w = *reinterpret_cast<const h8*>(&wo_lds[(32 * p + pair_row(r, tt)) * LDO + 32 * q + 8 * g]);
#pragma unroll
            for (int t = 0; t < TM; ++t) yacc[p][tt][t] = mfma32(w, hb[t], yacc[p][tt][t]);
          }
      }
    }

    // ---- epilogue: + b_out + R, LayerNorm over the row ----
    const float inv_d = 1.0f / (float)D;
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      const int64_t m = m0 + 16 * t + r;
      const bool valid = m < M;
      float sum = 0.f;
#pragma unroll
      for (int p = 0; p < PN; ++p) {
        const int n = 32 * p + 8 * g;
        float bv[8], rv[8];
        load8_f16_to_f32(a.b_out + n, bv);
        if (valid) {
          load8_f32(a.residual + m * D + n, rv);
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) rv[j] = 0.f;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          yacc[p][0][t][i] = (yacc[p][0][t][i] + bv[i]) + rv[i];
          yacc[p][1][t][i] = (yacc[p][1][t][i] + bv[4 + i]) + rv[4 + i];
          sum += yacc[p][0][t][i] + yacc[p][1][t][i];
        }
      }
      const float mean = sum_over_groups(sum) * inv_d;
      float sq = 0.f;
#pragma unroll
      for (int p = 0; p < PN; ++p)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float c = yacc[p][tt][t][i] - mean;
            sq += c * c;
          }
      const float rstd = rsqrtf(sum_over_groups(sq) * inv_d + a.eps);
      if (valid) {
#pragma unroll
        for (int p = 0; p < PN; ++p) {
          const int n = 32 * p + 8 * g;
          float v[8], gm[8], bt[8], o[8];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            v[i] = yacc[p][0][t][i];
            v[4 + i] = yacc[p][1][t][i];
          }
          if (a.residual_out) store8(a.residual_out + m * D + n, v);
          load8_f32(a.gamma + n, gm);
          load8_f32(a.beta + n, bt);
#pragma unroll
          for (int j = 0; j < 8; ++j) o[j] = (v[j] - mean) * rstd * gm[j] + bt[j];
          pin_f32x8(o);  // rounded to FP32, then to the output type (no fused FMA + conversion)
          store8(NO + m * D + n, o);
        }
      }
    }
  }
}

static int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <int D, int FC, int TM, typename XT, typename OT>
static hipError_t launch_ffn(const FfnArgs& a, hipStream_t s) {
  constexpr int BM = 64 * TM;
  const int64_t ntiles = (a.m + BM - 1) / BM;
  int64_t grid = ntiles;
  if (a.f <= FC) {
    // weights resident in LDS: persistent grid, a few workgroups per CU
    const int64_t cap = (int64_t)device_cu_count() * 4;
    if (grid > cap) grid = cap;
  }
  if (grid > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((ffn_ln_kernel<D, FC, TM, XT, OT>), dim3((unsigned)grid), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

template <typename XT, typename OT>
static hipError_t ffn_dispatch(int variant, const FfnArgs& a, int d, hipStream_t s) {
  // variant 3: the wide kernel (d_model 256, 32x32x16 MFMAs, 128-token workgroups)
  if (variant == 3) return launch_ffn_wide(a, d, kF16, std::is_same<XT, float>::value ? kF32 : kF16,
                                           std::is_same<OT, float>::value ? kF32 : kF16, s);
  // variant 4: the role-split wide kernel (d_model 256, vector and matrix waves)
  if (variant == 4) return launch_ffn_roles(a, d, kF16, std::is_same<XT, float>::value ? kF32 : kF16,
                                            std::is_same<OT, float>::value ? kF32 : kF16, s);
  // variant 1: TM=1; variant 2: TM=2 (D <= 256)
  const bool two = variant == 2;
  switch (d) {
    case 32: return two ? launch_ffn<32, 128, 2, XT, OT>(a, s) : launch_ffn<32, 128, 1, XT, OT>(a, s);
    case 64: return two ? launch_ffn<64, 128, 2, XT, OT>(a, s) : launch_ffn<64, 128, 1, XT, OT>(a, s);
    case 128: return two ? launch_ffn<128, 128, 2, XT, OT>(a, s) : launch_ffn<128, 128, 1, XT, OT>(a, s);
    case 256: return two ? launch_ffn<256, 64, 2, XT, OT>(a, s) : launch_ffn<256, 64, 1, XT, OT>(a, s);
    case 512: return launch_ffn<512, 32, 1, XT, OT>(a, s);
    default: return (hipError_t)MPK_EUNSUPPORTED;
  }
}

}  // namespace mpk

using namespace mpk;

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

extern "C" int mpk_ffn_residual_layernorm_auto_variant(int64_t m, int32_t d, int32_t f) {
  if (ffn_wide_supported(d, f)) return 4;
  if (d <= 128 && m >= 64 * 1024) return 2;
  return 1;
}

extern "C" int mpk_ffn_residual_layernorm(const void* x, int x_dtype, const void* w_in, const void* b_in,
                                          const void* w_out, const void* b_out, const float* residual,
                                          const float* gamma, const float* beta, float* residual_out,
                                          void* normalized_out, int normalized_dtype, int64_t m, int32_t d,
                                          int32_t f, float eps, int variant, void* stream) {
  if (!x || !w_in || !b_in || !w_out || !b_out || !residual || !gamma || !beta ||
      !normalized_out || m < 0 || d <= 0 || f <= 0)
    return MPK_EINVAL;
  if ((x_dtype != kF32 && x_dtype != kF16) || (normalized_dtype != kF32 && normalized_dtype != kF16))
    return MPK_EINVAL;
  if (d != 32 && d != 64 && d != 128 && d != 256 && d != 512) return MPK_EUNSUPPORTED;
  if (f % 32 != 0) return MPK_EUNSUPPORTED;
  if (!aligned16(x) || !aligned16(w_in) || !aligned16(b_in) || !aligned16(w_out) || !aligned16(b_out) ||
      !aligned16(residual) || !aligned16(gamma) || !aligned16(beta) || (residual_out && !aligned16(residual_out)) ||
      !aligned16(normalized_out))
    return MPK_EALIGN;
  if (m == 0) return MPK_OK;
  if (variant == 0) variant = mpk_ffn_residual_layernorm_auto_variant(m, d, f);
  if (variant < 1 || variant > 4) return MPK_EUNSUPPORTED;
  FfnArgs a{};
  a.x = x; a.w_in = static_cast<const _Float16*>(w_in); a.b_in = static_cast<const _Float16*>(b_in);
  a.w_out = static_cast<const _Float16*>(w_out); a.b_out = static_cast<const _Float16*>(b_out);
  a.residual = residual; a.gamma = gamma; a.beta = beta; a.residual_out = residual_out;
  a.normalized_out = normalized_out; a.m = m; a.f = f; a.eps = eps;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  const bool xf = x_dtype == kF32, of = normalized_dtype == kF32;
  if (xf) e = of ? ffn_dispatch<float, float>(variant, a, d, s) : ffn_dispatch<float, _Float16>(variant, a, d, s);
  else e = of ? ffn_dispatch<_Float16, float>(variant, a, d, s) : ffn_dispatch<_Float16, _Float16>(variant, a, d, s);
  return (int)e;
}
