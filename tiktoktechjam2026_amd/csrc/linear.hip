// FP16 x FP16 -> FP32 MFMA projection kernels with fused epilogues.
//
// Replaces the reference's Triton kernels
//   _mixed_linear_kernel                 mixed_precision/triton_linear.py:16-69
//     Y = act(fp16(X) W^T + b), act in {identity, exact-erf GELU}, Y fp16|fp32
//   _mixed_linear_add_layer_norm_kernel  mixed_precision/triton_linear.py:72-125
//     R' = fp16(X) W^T + b + R (FP32), N' = LayerNorm(R') (FP32 statistics)
//
// Numerics (same rounding points as the reference): X is rounded to FP16 in
// registers (RNE) on its way into LDS, W and b are FP16, accumulation, bias,
// GELU, residual and LayerNorm are FP32; only the final store rounds.
//
// Structure.  A workgroup (4 waves) owns a BM x BN output tile.  X[BM, KC] and
// W[BN, KC] chunks are staged through LDS (rows padded by 8 halves against bank
// conflicts) and consumed with v_mfma_f32_16x16x32_f16 in the transposed,
// paired layout described in mpk_common.h: each lane ends up owning one token
// row and runs of 8 consecutive output features, so bias/GELU/residual/LN are
// lane-local and every store is 16 (FP16) or 32 (FP32) contiguous bytes.  For
// the LayerNorm epilogue a wave owns whole rows (BN == N), so the row
// statistics need only two cross-lane shuffles.
#include "mpk_common.h"

namespace mpk {

enum Epilogue : int { kEpiBias = 0, kEpiBiasGelu = 1, kEpiResidualLN = 2 };

struct LinearArgs {
  const void* x;
  const _Float16* w;
  const _Float16* bias;
  void* y;                // EPI bias/gelu: Y[M,N]; EPI LN: normalized out N'[M,N]
  const float* residual;  // EPI LN only
  const float* gamma;
  const float* beta;
  float* residual_out;
  int64_t m;
  int n;
  int k;
  float eps;
};

template <int BM, int BN, int KC, int WAVES_M, typename XT, int EPI, typename OT>
__global__ __launch_bounds__(kBlock) void linear_kernel(LinearArgs a) {
  constexpr int WAVES_N = 4 / WAVES_M;
  constexpr int WM = BM / WAVES_M;
  constexpr int WN = BN / WAVES_N;
  constexpr int TM = WM / 16;
  constexpr int PN = WN / 32;
  constexpr int LD = KC + 8;
  static_assert(WAVES_M * WAVES_N == 4, "four waves");
  static_assert(TM * 16 == WM && PN * 32 == WN && KC % 32 == 0, "tile shape");
  static_assert(EPI != kEpiResidualLN || WAVES_N == 1, "LayerNorm epilogue needs whole rows per wave");

  __shared__ _Float16 xs[BM * LD];
  __shared__ _Float16 ws[BN * LD];

  const XT* __restrict__ X = static_cast<const XT*>(a.x);
  const _Float16* __restrict__ W = a.w;
  const int64_t M = a.m;
  const int N = a.n, K = a.k;

  const int nbn = (N + BN - 1) / BN;
  const int tile = xcd_local_tile(blockIdx.x, gridDim.x);
  const int64_t m0 = (int64_t)(tile / nbn) * BM;
  const int n0 = (tile % nbn) * BN;

  const int l = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = l & 15, g = l >> 4;
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;

  f4 acc[PN][2][TM];
#pragma unroll
  for (int p = 0; p < PN; ++p)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int t = 0; t < TM; ++t) acc[p][tt][t] = zero4();

  constexpr int CPR = KC / 8;  // 8-element chunks per LDS row
  for (int k0 = 0; k0 < K; k0 += KC) {
    if (k0 > 0) __syncthreads();
    for (int c = threadIdx.x; c < BM * CPR; c += kBlock) {
      const int row = c / CPR, col = (c % CPR) * 8;
      const int64_t gm = m0 + row;
      const int gk = k0 + col;
      h8 v = (gm < M && gk < K) ? load8_as_half(X + gm * K + gk) : zero_h8();
      *reinterpret_cast<h8*>(&xs[row * LD + col]) = v;
    }
    for (int c = threadIdx.x; c < BN * CPR; c += kBlock) {
      const int row = c / CPR, col = (c % CPR) * 8;
      const int gn = n0 + row;
      const int gk = k0 + col;
      h8 v = (gn < N && gk < K) ? load8_as_half(W + (int64_t)gn * K + gk) : zero_h8();
      *reinterpret_cast<h8*>(&ws[row * LD + col]) = v;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < KC / 32; ++ks) {
      h8 bx[TM];
#pragma unroll
      for (int t = 0; t < TM; ++t)
        bx[t] = *reinterpret_cast<const h8*>(&xs[(wm * WM + 16 * t + r) * LD + ks * 32 + 8 * g]);
#pragma unroll
      for (int p = 0; p < PN; ++p) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const h8 aw =
              *reinterpret_cast<const h8*>(&ws[(wn * WN + 32 * p + pair_row(r, tt)) * LD + ks * 32 + 8 * g]);
#pragma unroll
          for (int t = 0; t < TM; ++t) acc[p][tt][t] = mfma32(aw, bx[t], acc[p][tt][t]);
        }
      }
    }
  }

  OT* __restrict__ Y = static_cast<OT*>(a.y);
  if constexpr (EPI == kEpiBias || EPI == kEpiBiasGelu) {
#pragma unroll
    for (int p = 0; p < PN; ++p) {
      const int n = n0 + wn * WN + 32 * p + 8 * g;
      if (n >= N) continue;
      float bv[8];
      load8_f16_to_f32(a.bias + n, bv);
#pragma unroll
      for (int t = 0; t < TM; ++t) {
        const int64_t m = m0 + wm * WM + 16 * t + r;
        if (m >= M) continue;
        float v[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[i] = acc[p][0][t][i] + bv[i];
          v[4 + i] = acc[p][1][t][i] + bv[4 + i];
        }
        if constexpr (EPI == kEpiBiasGelu) {
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = gelu_erf(v[j]);
        }
        store8(Y + m * N + n, v);
      }
    }
  } else {
    // R' = acc + b + R ; N' = LayerNorm(R') over the whole row (BN == N).
    const float inv_n = 1.0f / (float)N;
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      const int64_t m = m0 + wm * WM + 16 * t + r;
      const bool valid = m < M;
      float v[PN][8];
      float sum = 0.f;
#pragma unroll
      for (int p = 0; p < PN; ++p) {
        const int n = 32 * p + 8 * g;
        float bv[8], rv[8];
        load8_f16_to_f32(a.bias + n, bv);
        if (valid) {
          load8_f32(a.residual + m * N + n, rv);
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) rv[j] = 0.f;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[p][i] = (acc[p][0][t][i] + bv[i]) + rv[i];
          v[p][4 + i] = (acc[p][1][t][i] + bv[4 + i]) + rv[4 + i];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) sum += v[p][j];
      }
      const float mean = sum_over_groups(sum) * inv_n;
      float sq = 0.f;
#pragma unroll
      for (int p = 0; p < PN; ++p)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float c = v[p][j] - mean;
          sq += c * c;
        }
      const float rstd = rsqrtf(sum_over_groups(sq) * inv_n + a.eps);
      if (valid) {
#pragma unroll
        for (int p = 0; p < PN; ++p) {
          const int n = 32 * p + 8 * g;
          store8(a.residual_out + m * N + n, v[p]);
          float gm[8], bt[8], o[8];
          load8_f32(a.gamma + n, gm);
          load8_f32(a.beta + n, bt);
#pragma unroll
          for (int j = 0; j < 8; ++j) o[j] = (v[p][j] - mean) * rstd * gm[j] + bt[j];
          store8(Y + m * N + n, o);
        }
      }
    }
  }
}

template <int BM, int BN, int KC, int WAVES_M, typename XT, int EPI, typename OT>
static hipError_t launch_linear(const LinearArgs& a, hipStream_t s) {
  const int64_t mb = (a.m + BM - 1) / BM;
  const int64_t nb = (a.n + BN - 1) / BN;
  const int64_t grid = mb * nb;
  if (grid > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((linear_kernel<BM, BN, KC, WAVES_M, XT, EPI, OT>), dim3((unsigned)grid), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

// Generic projection tiles (variant ids are part of the dispatch table).
//   1: BM128 BN128 (2x2 waves, 64x64 per wave)   wide N
//   2: BM128 BN64  (4x1 waves, 32x64 per wave)   N multiple of 64
//   3: BM128 BN32  (4x1 waves, 32x32 per wave)   narrow / ragged N
//   4: BM64  BN128 (1x4 waves, 64x32 per wave)   short M, wide N
template <typename XT, int EPI, typename OT>
static hipError_t linear_variant(int variant, const LinearArgs& a, hipStream_t s) {
  switch (variant) {
    case 1: return launch_linear<128, 128, 64, 2, XT, EPI, OT>(a, s);
    case 2: return launch_linear<128, 64, 64, 4, XT, EPI, OT>(a, s);
    case 3: return launch_linear<128, 32, 64, 4, XT, EPI, OT>(a, s);
    case 4: return launch_linear<64, 128, 64, 1, XT, EPI, OT>(a, s);
    default: return (hipError_t)MPK_EUNSUPPORTED;
  }
}

// LayerNorm-epilogue tiles: one wave owns 16*TM whole rows of width D.
//   variant 1: TM=1 (BM=64);  variant 2: TM=2 (BM=128)
template <int D, int KC, typename XT, typename OT>
static hipError_t linear_ln_d(int variant, const LinearArgs& a, hipStream_t s) {
  if (variant == 2 && D <= 128) return launch_linear<128, D, KC, 4, XT, kEpiResidualLN, OT>(a, s);
  if (variant == 1 || variant == 2) return launch_linear<64, D, KC, 4, XT, kEpiResidualLN, OT>(a, s);
  return (hipError_t)MPK_EUNSUPPORTED;
}

template <typename XT, typename OT>
static hipError_t linear_ln(int variant, const LinearArgs& a, hipStream_t s) {
  switch (a.n) {
    case 32: return linear_ln_d<32, 32, XT, OT>(variant, a, s);
    case 64: return linear_ln_d<64, 64, XT, OT>(variant, a, s);
    case 128: return linear_ln_d<128, 128, XT, OT>(variant, a, s);
    case 256: return linear_ln_d<256, 64, XT, OT>(variant, a, s);
    case 512: return linear_ln_d<512, 32, XT, OT>(variant, a, s);
    default: return (hipError_t)MPK_EUNSUPPORTED;
  }
}

}  // namespace mpk

using namespace mpk;

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

extern "C" int mpk_linear_auto_variant(int64_t m, int32_t n, int32_t k) {
  (void)k;
  if (n % 128 == 0 && m >= 128 * 256) return 1;
  if (n % 128 == 0) return 4;
  if (n % 64 == 0) return 2;
  return 3;
}

extern "C" int mpk_linear(const void* x, int x_dtype, const void* w, const void* b, void* y, int y_dtype, int gelu,
                          int64_t m, int32_t n, int32_t k, int variant, void* stream) {
  if (!x || !w || !b || !y || m < 0 || n <= 0 || k <= 0) return MPK_EINVAL;
  if ((x_dtype != kF32 && x_dtype != kF16) || (y_dtype != kF32 && y_dtype != kF16)) return MPK_EINVAL;
  if (n % 8 != 0 || k % 8 != 0) return MPK_EUNSUPPORTED;
  if (!aligned16(x) || !aligned16(w) || !aligned16(b) || !aligned16(y)) return MPK_EALIGN;
  if (m == 0) return MPK_OK;
  if (variant == 0) variant = mpk_linear_auto_variant(m, n, k);
  LinearArgs a{};
  a.x = x; a.w = static_cast<const _Float16*>(w); a.bias = static_cast<const _Float16*>(b); a.y = y;
  a.m = m; a.n = n; a.k = k;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  const bool xf = x_dtype == kF32, yf = y_dtype == kF32;
  if (gelu) {
    if (xf) e = yf ? linear_variant<float, kEpiBiasGelu, float>(variant, a, s)
                   : linear_variant<float, kEpiBiasGelu, _Float16>(variant, a, s);
    else e = yf ? linear_variant<_Float16, kEpiBiasGelu, float>(variant, a, s)
                : linear_variant<_Float16, kEpiBiasGelu, _Float16>(variant, a, s);
  } else {
    if (xf) e = yf ? linear_variant<float, kEpiBias, float>(variant, a, s)
                   : linear_variant<float, kEpiBias, _Float16>(variant, a, s);
    else e = yf ? linear_variant<_Float16, kEpiBias, float>(variant, a, s)
                : linear_variant<_Float16, kEpiBias, _Float16>(variant, a, s);
  }
  return (int)e;
}

extern "C" int mpk_linear_residual_layernorm_auto_variant(int64_t m, int32_t d) {
  (void)d;
  return m >= 128 * 512 ? 2 : 1;
}

extern "C" int mpk_linear_residual_layernorm(const void* x, int x_dtype, const void* w, const void* b,
                                             const float* residual, const float* gamma, const float* beta,
                                             float* residual_out, void* normalized_out, int normalized_dtype,
                                             int64_t m, int32_t d, float eps, int variant, void* stream) {
  if (!x || !w || !b || !residual || !gamma || !beta || !residual_out || !normalized_out || m < 0 || d <= 0)
    return MPK_EINVAL;
  if ((x_dtype != kF32 && x_dtype != kF16) || (normalized_dtype != kF32 && normalized_dtype != kF16))
    return MPK_EINVAL;
  if (d != 32 && d != 64 && d != 128 && d != 256 && d != 512) return MPK_EUNSUPPORTED;
  if (!aligned16(x) || !aligned16(w) || !aligned16(b) || !aligned16(residual) || !aligned16(gamma) ||
      !aligned16(beta) || !aligned16(residual_out) || !aligned16(normalized_out))
    return MPK_EALIGN;
  if (m == 0) return MPK_OK;
  if (variant == 0) variant = mpk_linear_residual_layernorm_auto_variant(m, d);
  LinearArgs a{};
  a.x = x; a.w = static_cast<const _Float16*>(w); a.bias = static_cast<const _Float16*>(b); a.y = normalized_out;
  a.residual = residual; a.gamma = gamma; a.beta = beta; a.residual_out = residual_out;
  a.m = m; a.n = d; a.k = d; a.eps = eps;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  const bool xf = x_dtype == kF32, of = normalized_dtype == kF32;
  if (xf) e = of ? linear_ln<float, float>(variant, a, s) : linear_ln<float, _Float16>(variant, a, s);
  else e = of ? linear_ln<_Float16, float>(variant, a, s) : linear_ln<_Float16, _Float16>(variant, a, s);
  return (int)e;
}
