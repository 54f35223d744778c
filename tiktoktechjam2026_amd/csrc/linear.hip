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
#include <algorithm>
#include <type_traits>

#include "mpk_common.h"

namespace mpk {

enum Epilogue : int {
  kEpiBias = 0,
  kEpiBiasGelu = 1,
  kEpiResidualLN = 2,      // whole rows per wave (row-owning kernel)
  kEpiBiasResidual = 3,
  kEpiResidualLNTile = 4,  // large tiles: a row spans several waves, statistics exchanged through LDS
};

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
  // bias epilogue only (mpk_linear_qscaled): columns below q_cols are multiplied by q_scale
  // in FP32 before the output rounding (the attention's scale * log2(e) folded into q)
  int q_cols;
  float q_scale;
};

// The q_cols / q_scale multiply of a bias epilogue on the 8 outputs at column n (a run of 8
// never straddles q_cols, a multiple of 8); a scalar branch when the call scales nothing.
// The products are pinned as FP32 values, so the output conversion rounds them once more
// to FP16 and cannot be fused with the multiply into one rounding (v_fma_mix).
__device__ __forceinline__ void q_scale8(const LinearArgs& a, int n, float* v) {
  if (a.q_cols > 0) {
    const float s = n < a.q_cols ? a.q_scale : 1.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] *= s;
    pin_f32x8(v);
  }
}

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

  const int l = threadIdx.x & 63, wave = wave_id();
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

  OT* Y = static_cast<OT*>(a.y);  // may alias a.residual (in-place residual add)
  if constexpr (EPI == kEpiBias || EPI == kEpiBiasGelu || EPI == kEpiBiasResidual) {
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
        if constexpr (EPI == kEpiBias) q_scale8(a, n, v);
        if constexpr (EPI == kEpiBiasResidual) {
          float rv[8];
          load8_f32(a.residual + m * N + n, rv);
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] += rv[j];
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
          pin_f32x8(o);  // rounded to FP32, then to the output type (no fused FMA + conversion)
          store8(Y + m * N + n, o);
        }
      }
    }
  }
}


// Large-tile projection for wide models: a BM (tokens) x BN (features) output
// tile per workgroup of BM/128 x BN/64 waves, each wave 128 x 64 (8 token tiles x
// 2 feature pairs).  K is staged in BK-wide chunks (64, or 32 where a wide tile
// needs the LDS) through LDS with a one-chunk register prefetch: double-buffered
// with one barrier per chunk (STAGES == 2), or single-buffered with two (STAGES
// == 1, half the LDS).  Each W fragment read from LDS feeds 8 MFMAs and each X
// fragment 4; a 256 x 256 tile reads 128 FLOPs' worth of operands per byte from
// L2, a 256 x 128 tile 85, a 128 x 512 tile 102.
//
// The kernel is persistent: the grid fills the device once and each workgroup
// walks a strided list of tiles inside its XCD's contiguous share of the tile
// range (workgroups are dispatched to the 8 XCDs round-robin), so the tiles an
// XCD runs at one time share token rows of X in that XCD's L2.  The chunk
// pipeline runs across tile boundaries: the next tile's first chunk is in
// flight while the current tile's last chunk and epilogue execute, which hides
// the load latency that short-K projections (K = 256..512) would otherwise
// expose once per tile.
template <int BM, int BN, int BK, int STAGES, typename XT, int EPI, typename OT>
__global__ __launch_bounds__(BM / 2 * BN / 64) void linear_big_kernel(LinearArgs a) {
  constexpr int WM = 128, WN = 64, TM = WM / 16, PN = WN / 32;
  constexpr int WAVES_M = BM / WM;
  constexpr int NT = 64 * WAVES_M * (BN / WN);  // threads
  // 160-byte (BK 64) or 80-byte (BK 32) rows: the 16 rows of a b128 fragment read hit distinct banks
  constexpr int LD = BK + (BK == 64 ? 16 : 8);
  static_assert(BM % WM == 0 && BN % WN == 0 && (BK == 32 || BK == 64), "tile shape");
  constexpr int CPR = BK / 8;                   // 8-element chunks per staged row
  constexpr int XCH = BM * CPR / NT;            // X chunks per thread
  constexpr int WCH = BN * CPR / NT;            // W chunks per thread
  static_assert(XCH * NT == BM * CPR && WCH * NT == BN * CPR, "staging split");
  static_assert(EPI != kEpiResidualLN, "row LayerNorm needs whole rows per wave");
  static_assert(STAGES == 1 || STAGES == 2, "one or two LDS stages");
  // LayerNorm scratch in the idle W stage: [2 passes][BN / WN][BM] partial row sums,
  // then gamma and beta
  static_assert(EPI != kEpiResidualLNTile || STAGES == 2, "the LayerNorm epilogue uses the idle LDS stage");
  static_assert(EPI != kEpiResidualLNTile || (2 * (BN / WN) * BM + 2 * BN) * 4 <= BN * LD * 2,
                "LayerNorm scratch fits the idle W stage");

  __shared__ _Float16 xs[STAGES][BM * LD];
  __shared__ _Float16 ws[STAGES][BN * LD];
  // LDS position (halves) of 8-element chunk c of tile row `row`
  auto cpos = [](int row, int c) { return row * LD + 8 * c; };

  const XT* __restrict__ X = static_cast<const XT*>(a.x);
  const _Float16* __restrict__ W = a.w;
  const int64_t M = a.m;
  const int N = a.n, K = a.k;
  const int nbn = (N + BN - 1) / BN;
  const int tiles = (int)((M + BM - 1) / BM) * nbn;
  const int nchunks = (K + BK - 1) / BK;

  // This workgroup's tiles: tile, tile + stride, ... < last.  With a grid that
  // is a multiple of 8, XCD x (workgroups b with b % 8 == x) owns tiles
  // [tiles x / 8, tiles (x + 1) / 8); otherwise a plain grid stride.
  const int G = gridDim.x;
  int tile, stride, last;
  if ((G & 7) == 0) {
    const int xcd = blockIdx.x & 7;
    stride = G >> 3;
    last = (int)((int64_t)tiles * (xcd + 1) / 8);
    tile = (int)((int64_t)tiles * xcd / 8) + (blockIdx.x >> 3);
  } else {
    stride = G;
    last = tiles;
    tile = blockIdx.x;
  }
  if (tile >= last) return;                     // uniform per workgroup, before any barrier

  const int l = threadIdx.x & 63, wave = wave_id();
  const int r = l & 15, g = l >> 4;
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;

  f4 acc[PN][2][TM];
#pragma unroll
  for (int p = 0; p < PN; ++p)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int t = 0; t < TM; ++t) acc[p][tt][t] = zero4();

  // Tile loads go through buffer resources that cover only the tile's existing
  // rows: rows past M (or N) read as zeros without per-lane predication.  Only a
  // partial last K chunk (K % 64 != 0) masks columns per lane.
  h8 xr[XCH], wr[WCH];
  const uint32_t xrow_bytes = (uint32_t)K * (uint32_t)sizeof(XT);
  const uint32_t wrow_bytes = (uint32_t)K * 2u;
  auto fetch = [&](int ftile, int k0) {
    const int64_t fm0 = (int64_t)(ftile / nbn) * BM;
    const int fn0 = (ftile % nbn) * BN;
    const uint32_t xrows = (uint32_t)min<int64_t>(BM, M - fm0);
    const uint32_t wrows = (uint32_t)min(BN, N - fn0);
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(X + fm0 * K, xrows * xrow_bytes);
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(W + (int64_t)fn0 * K, wrows * wrow_bytes);
    const bool full_k = k0 + BK <= K;
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int c = threadIdx.x + i * NT;
      const int row = c / CPR, col = (c % CPR) * 8;
      const uint32_t off = row * xrow_bytes + (uint32_t)(k0 + col) * (uint32_t)sizeof(XT);
      xr[i] = full_k || k0 + col < K ? buffer_load8_as_half(xrs, off, X) : zero_h8();
    }
#pragma unroll
    for (int i = 0; i < WCH; ++i) {
      const int c = threadIdx.x + i * NT;
      const int row = c / CPR, col = (c % CPR) * 8;
      const uint32_t off = row * wrow_bytes + (uint32_t)(k0 + col) * 2u;
      wr[i] = full_k || k0 + col < K ? buffer_load8_as_half(wrs, off, W) : zero_h8();
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int c = threadIdx.x + i * NT;
      *reinterpret_cast<h8*>(&xs[buf][cpos(c / CPR, c % CPR)]) = xr[i];
    }
#pragma unroll
    for (int i = 0; i < WCH; ++i) {
      const int c = threadIdx.x + i * NT;
      *reinterpret_cast<h8*>(&ws[buf][cpos(w_slot(c / CPR), c % CPR)]) = wr[i];
    }
  };
  auto compute = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      // Issue every fragment read of this k-step before the first MFMA, so the
      // LDS latency overlaps the reads still in flight instead of stalling
      // each group of four MFMAs.
      h8 wa[PN][2], xb[TM];
#pragma unroll
      for (int p = 0; p < PN; ++p)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
          wa[p][tt] = *reinterpret_cast<const h8*>(&ws[buf][cpos(wn * WN + 32 * p + 16 * tt + r, 4 * ks + g)]);
#pragma unroll
      for (int t = 0; t < TM; ++t)
        xb[t] = *reinterpret_cast<const h8*>(&xs[buf][cpos(wm * WM + 16 * t + r, 4 * ks + g)]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int p = 0; p < PN; ++p)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) acc[p][tt][t] = mfma32(wa[p][tt], xb[t], acc[p][tt][t]);
    }
  };
  OT* Y = static_cast<OT*>(a.y);  // may alias a.residual (in-place residual add)
  // LayerNorm epilogue (N == BN: the tile holds whole rows, spread over the
  // BN/64 waves of a row half).  R' = acc + b + R, then two-pass FP32 row
  // statistics: each wave reduces its 64 features per row across its four lane
  // groups, the per-wave partial sums meet in the idle LDS stage, and every
  // wave finishes the same row sums in the same order.
  auto epilogue_ln = [&](int etile, int obuf) {
    constexpr int NWN = BN / WN;  // waves across a row
    float* red = reinterpret_cast<float*>(&ws[obuf][0]);
    float* gam = red + 2 * NWN * BM;
    float* bet = gam + BN;
    const int64_t m0 = (int64_t)(etile / nbn) * BM;
    const float inv_n = 1.0f / (float)N;
    for (int i = threadIdx.x; i < BN; i += NT) {
      gam[i] = a.gamma[i];
      bet[i] = a.beta[i];
    }
    // pass 1: R' in place of the accumulators, row sums
    {
      float bv[PN][8];
#pragma unroll
      for (int p = 0; p < PN; ++p) load8_f16_to_f32(a.bias + wn * WN + 32 * p + 8 * g, bv[p]);
#pragma unroll
      for (int t = 0; t < TM; ++t) {
        const int row = wm * WM + 16 * t + r;
        const int64_t m = m0 + row;
        float sum = 0.f;
#pragma unroll
        for (int p = 0; p < PN; ++p) {
          const int n = wn * WN + 32 * p + 8 * g;
          float rv[8];
          if (m < M) {
            load8_f32(a.residual + m * N + n, rv);
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) rv[j] = 0.f;
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[p][0][t][i] = (acc[p][0][t][i] + bv[p][i]) + rv[i];
            acc[p][1][t][i] = (acc[p][1][t][i] + bv[p][4 + i]) + rv[4 + i];
            sum += acc[p][0][t][i] + acc[p][1][t][i];
          }
        }
        sum = sum_over_groups(sum);
        if (g == 0) red[wn * BM + row] = sum;
      }
    }
    __syncthreads();
    auto row_mean = [&](int row) {
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < NWN; ++w) sum += red[w * BM + row];
      return sum * inv_n;
    };
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      const int row = wm * WM + 16 * t + r;
      const float mean = row_mean(row);
      float sq = 0.f;
#pragma unroll
      for (int p = 0; p < PN; ++p)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float c = acc[p][tt][t][i] - mean;
            sq += c * c;
          }
      sq = sum_over_groups(sq);
      if (g == 0) red[(NWN + wn) * BM + row] = sq;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      const int row = wm * WM + 16 * t + r;
      const int64_t m = m0 + row;
      const float mean = row_mean(row);
      float sq = 0.f;
#pragma unroll
      for (int w = 0; w < NWN; ++w) sq += red[(NWN + w) * BM + row];
      const float rstd = rsqrtf(sq * inv_n + a.eps);
      if (m >= M) continue;
#pragma unroll
      for (int p = 0; p < PN; ++p) {
        const int n = wn * WN + 32 * p + 8 * g;
        float v[8], o[8], gm[8], bt[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[i] = acc[p][0][t][i];
          v[4 + i] = acc[p][1][t][i];
        }
        store8(a.residual_out + m * N + n, v);
        load8_f32(gam + n, gm);
        load8_f32(bet + n, bt);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = (v[j] - mean) * rstd * gm[j] + bt[j];
        pin_f32x8(o);  // rounded to FP32, then to the output type (no fused FMA + conversion)
        store8(static_cast<OT*>(a.y) + m * N + n, o);
      }
    }
    __syncthreads();  // the scratch stage is restaged next
  };
  auto epilogue = [&](int etile) {
    const int64_t m0 = (int64_t)(etile / nbn) * BM;
    const int n0 = (etile % nbn) * BN;
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
        if constexpr (EPI == kEpiBias) q_scale8(a, n, v);
        if constexpr (EPI == kEpiBiasResidual) {
          float rv[8];
          load8_f32(a.residual + m * N + n, rv);
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] += rv[j];
        }
        store8(Y + m * N + n, v);
      }
    }
  };

  fetch(tile, 0);
  stash(0);
  __syncthreads();
  int c = 0, buf = 0;
  for (;;) {
    int ntile = tile, nc = c + 1;
    if (nc == nchunks) {
      nc = 0;
      ntile = tile + stride;
    }
    const bool more = ntile < last;
    if (more) fetch(ntile, nc * BK);
    compute(buf);
    if (c == nchunks - 1) {
      if constexpr (EPI == kEpiResidualLNTile)
        epilogue_ln(tile, buf ^ 1);
      else
        epilogue(tile);
#pragma unroll
      for (int p = 0; p < PN; ++p)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int t = 0; t < TM; ++t) acc[p][tt][t] = zero4();
    }
    if (!more) break;
    if constexpr (STAGES == 2) {
      buf ^= 1;
      stash(buf);
      __syncthreads();
    } else {
      __syncthreads();
      stash(0);
      __syncthreads();
    }
    tile = ntile;
    c = nc;
  }
}

// Workgroups that fill the device once for a persistent kernel, cached per (device,
// kernel): the kernels share one function-pointer type, so the key is the pointer.
template <typename Kernel>
static int resident_grid(Kernel kernel, int threads, size_t lds) {
  struct Entry { const void* fn; int dev, grid; };
  static Entry cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  const void* fn = reinterpret_cast<const void*>(kernel);
  int free_slot = -1;
  for (int i = 0; i < 64; ++i) {
    if (cached[i].fn == fn && cached[i].dev == dev) return cached[i].grid;
    if (!cached[i].fn && free_slot < 0) free_slot = i;
  }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds) != hipSuccess || per_cu <= 0)
    per_cu = 1;
  if (free_slot >= 0) cached[free_slot] = Entry{fn, dev, cus * per_cu};
  return cus * per_cu;
}

template <int BM, int BN, int BK, int STAGES, typename XT, int EPI, typename OT>
static hipError_t launch_linear_big(const LinearArgs& a, hipStream_t s) {
  constexpr int NT = BM / 2 * BN / 64;
  if (a.k > (1 << 20)) return (hipError_t)MPK_EUNSUPPORTED;  // 32-bit tile offsets: BM rows x K x 4 bytes
  const int64_t tiles = ((a.m + BM - 1) / BM) * ((a.n + BN - 1) / BN);
  if (tiles > 0x7fffffff) return hipErrorInvalidConfiguration;
  auto kernel = linear_big_kernel<BM, BN, BK, STAGES, XT, EPI, OT>;
  int64_t grid = std::min<int64_t>(tiles, resident_grid(kernel, NT, 0));
  if (grid >= 8) grid &= ~int64_t{7};
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(NT), 0, s, a);
  return hipGetLastError();
}

// ---- LDS-DMA projection (FP16 X) ----
// The same 256 x 256 output tiles, wave shapes, paired W-row mapping, MFMAs and
// epilogues as linear_big_kernel<256, 256, ...>, with the operands staged
// differently: X and W chunks 32 wide in K travel global -> LDS as LDS-DMA copies
// (global_load_lds_dwordx4, no registers, no LDS store instructions), through a
// ring of four LDS stages: while chunk q is multiplied, chunk q + 1 is read from
// LDS into fragment registers and chunks q + 2 .. q + 4 are in flight.  Per chunk
// each wave issues four 1-KB copies spread between its 32 MFMAs, waits for its own
// copies of the chunk it is about to read, and meets the other waves at one
// barrier, which also tells it that the stage it refills next has been read by
// everyone.
//
// A staged row is 64 bytes (four 16-byte chunks of 8 k values) with no padding;
// chunk c of row R sits in slot c ^ ((R / 2) % 4).  With that swizzle the
// fragment reads (lane r of a 16-lane group reads row R0 + r at one chunk) count no
// LDS bank conflicts on gfx950, where the plain layout, other XOR swizzles of the
// row bits and even 80-byte padded rows count two-way conflicts (measured with
// SQ_LDS_BANK_CONFLICT).
//
// Rows past M (or N) copy the last existing row (their products only reach output
// rows or columns that are not stored), so every copy reads memory inside X and W.
// Completion is tracked by count: after a wave issues a chunk's copies it issues
// the next two chunks' copies and, when a tile ended in between, that tile's
// output stores; s_waitcnt vmcnt(8 [+ stores]) before the chunk is read means
// that its own copies have landed (vector-memory operations of a wave complete in issue
// order).  Output stores therefore always issue the same number of instructions
// per tile: columns past N go to an offset outside the tile's buffer resource
// and rows past M lie outside it, and the hardware drops both.
constexpr int kDmaMaxN = 8192;  // the bias row lives in LDS

__device__ __forceinline__ int dma_swizzle(int r) { return (r >> 1) & 3; }

template <int EPI, typename OT>
__global__ __launch_bounds__(512) void linear_dma_kernel(LinearArgs a) {
  constexpr int BM = 256, BN = 256, BK = 32, NS = 4;
  constexpr int TM = 8, PN = 2;                         // 128 x 64 per wave, as linear_big_kernel
  constexpr int XBYTES = BM * BK * 2;                   // X part of a stage
  constexpr int SBYTES = (BM + BN) * BK * 2;            // one stage: 32 KB
  constexpr int STORES = TM * PN * (sizeof(OT) == 4 ? 2 : 1);  // store instructions per wave and tile
  static_assert(EPI == kEpiBias || EPI == kEpiBiasGelu || EPI == kEpiBiasResidual, "plain epilogues");
  __shared__ __align__(16) unsigned char stages[NS * SBYTES];
  __shared__ __align__(16) _Float16 bias_s[kDmaMaxN];

  const _Float16* __restrict__ X = static_cast<const _Float16*>(a.x);
  const _Float16* __restrict__ W = a.w;
  const int64_t M = a.m;
  const int N = a.n, K = a.k;
  const int nbn = (N + BN - 1) / BN;
  const int tiles = (int)((M + BM - 1) / BM) * nbn;
  const int nk = K / BK;  // >= 4, checked by the launcher

  // tile list as in linear_big_kernel: XCD x owns a contiguous share of the tiles
  const int G = gridDim.x;
  int tile, stride, last;
  if ((G & 7) == 0) {
    const int xcd = blockIdx.x & 7;
    stride = G >> 3;
    last = (int)((int64_t)tiles * (xcd + 1) / 8);
    tile = (int)((int64_t)tiles * xcd / 8) + (blockIdx.x >> 3);
  } else {
    stride = G;
    last = tiles;
    tile = blockIdx.x;
  }
  if (tile >= last) return;  // uniform per workgroup, before any barrier
  const int nq = ((last - tile + stride - 1) / stride) * nk;  // chunks this workgroup computes

  const int l = threadIdx.x & 63, wave = wave_id();
  const int r = l & 15, g = l >> 4;
  const int wm = wave & 1, wn = wave >> 1;

  for (int i = 8 * (int)threadIdx.x; i < N; i += 8 * 512)
    *reinterpret_cast<h8*>(&bias_s[i]) = *reinterpret_cast<const h8*>(a.bias + i);

  // ---- copies: wave w fills X rows and W slots 32 w .. 32 w + 31 of every stage ----
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)stages;
  const int rr = l >> 2;                                // row within a 16-row copy block
  const int cc = (l & 3) ^ dma_swizzle(rr);             // k chunk this lane copies
  int xrow[2], wfeat[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    xrow[i] = 32 * wave + 16 * i + rr;
    wfeat[i] = 32 * wave + 8 * (rr >> 2) + 4 * i + (rr & 3);  // LDS slot 32 w + 16 i + rr holds pair_row(rr, i)
  }
  uint32_t xoff[2], woff[2];
  const _Float16* xsrc = X;
  const _Float16* wsrc = W;
  int ctile = tile, ckc = 0;  // next chunk to copy
  auto copy_tile = [&](int t) {
    const int64_t m0 = (int64_t)(t / nbn) * BM;
    const int n0 = (t % nbn) * BN;
    const int xmax = (int)min<int64_t>(BM, M - m0) - 1, wmax = min(BN, N - n0) - 1;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      xoff[i] = (uint32_t)(min(xrow[i], xmax) * K + 8 * cc) * 2u;
      woff[i] = (uint32_t)(min(wfeat[i], wmax) * K + 8 * cc) * 2u;
    }
    xsrc = X + m0 * K;
    wsrc = W + (int64_t)n0 * K;
  };
  copy_tile(tile);
  // copy j (0..3) of the current chunk into stage `st`
  auto copy = [&](int j, int st) {
    const uint32_t dst = lds0 + (uint32_t)(st * SBYTES + (j >> 1) * XBYTES + (2 * wave + (j & 1)) * 1024);
    const _Float16* src = ((j >> 1) ? wsrc : xsrc) + ckc * BK;
    dma16((j >> 1) ? woff[j & 1] : xoff[j & 1], src, dst);
  };
  // after the chunk's four copies: the next chunk; past the last one the copies
  // repeat the last chunk into a stage nobody reads again
  auto advance = [&]() {
    if (ckc + 1 < nk) {
      ++ckc;
    } else if (ctile + stride < last) {
      ckc = 0;
      ctile += stride;
      copy_tile(ctile);
    }
  };

  f4 acc[PN][2][TM];
#pragma unroll
  for (int p = 0; p < PN; ++p)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int t = 0; t < TM; ++t) acc[p][tt][t] = zero4();

  const uint32_t lane_off = (uint32_t)(r * 64 + ((g ^ dma_swizzle(r)) << 4));
  OT* Y = static_cast<OT*>(a.y);  // may alias a.residual (in-place residual add)
  auto epilogue = [&](int etile) {
    const int64_t m0 = (int64_t)(etile / nbn) * BM;
    const int n0 = (etile % nbn) * BN;
    const uint32_t rows = (uint32_t)min<int64_t>(BM, M - m0);
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(Y + m0 * N, rows * (uint32_t)N * (uint32_t)sizeof(OT));
    const __amdgpu_buffer_rsrc_t rres =
        make_rsrc(EPI == kEpiBiasResidual ? (const void*)(a.residual + m0 * N) : (const void*)a.x,
                  EPI == kEpiBiasResidual ? rows * (uint32_t)N * 4u : 0u);
    // A row's 64 output columns of this wave are two runs of 32 (p = 0, 1), each
    // stored by four lanes.  Plain epilogues store the two runs of a row back to
    // back, so the halves of an output line (128 bytes at FP16) reach the memory
    // system together (measured on a 262144 x 768 x 256 projection: 10 % faster
    // than storing all p = 0 runs first); the residual epilogue, whose loads wait
    // for the stores before them, keeps the p-major order (faster there).
    h8 bhp[PN];
#pragma unroll
    for (int p = 0; p < PN; ++p) {
      const int n = n0 + wn * 64 + 32 * p + 8 * g;
      bhp[p] = *reinterpret_cast<const h8*>(&bias_s[n < N ? n : 0]);
    }
#pragma unroll
    for (int u = 0; u < TM * PN; ++u) {
      const int t = EPI == kEpiBiasResidual ? u % TM : u / PN;
      const int p = EPI == kEpiBiasResidual ? u / TM : u % PN;
      const int n = n0 + wn * 64 + 32 * p + 8 * g;
      const bool ok = n < N;
      const h8 bh = bhp[p];
      const int row = wm * 128 + 16 * t + r;
      const uint32_t e = (uint32_t)(row * N + n);
      float v[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = acc[p][0][t][i] + (float)bh[i];
        v[4 + i] = acc[p][1][t][i] + (float)bh[4 + i];
      }
      if constexpr (EPI == kEpiBiasGelu) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = gelu_erf(v[j]);
      }
      if constexpr (EPI == kEpiBias) q_scale8(a, n, v);
      if constexpr (EPI == kEpiBiasResidual) {
        typedef float v4 __attribute__((ext_vector_type(4)));
        const uint32_t ro = ok ? e * 4u : 0x80000000u;
        const v4 r0 = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(rres, ro, 0, 0));
        const v4 r1 = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(rres, ro + 16u, 0, 0));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[j] += r0[j];
          v[4 + j] += r1[j];
        }
      }
      buffer_store8(yr, ok ? e * (uint32_t)sizeof(OT) : 0x80000000u, v, Y);
    }
  };

  // Fragments: the W fragments of the chunk being multiplied and of the next one
  // (double-buffered), and the X fragments, each replaced by the next chunk's as soon
  // as its four MFMAs have been issued.  So the LDS reads of chunk q + 1 run beside
  // the MFMAs of chunk q.
  h8 wa[2][PN][2], xb[TM];
  auto read_w = [&](int q, h8 (&w)[PN][2]) {
    const unsigned char* sp = stages + (q & 3) * SBYTES + XBYTES;
#pragma unroll
    for (int p = 0; p < PN; ++p)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
        w[p][tt] = *reinterpret_cast<const h8*>(sp + (wn * 64 + 32 * p + 16 * tt) * 64 + lane_off);
  };
  auto read_x = [&](int q, int t) {
    return *reinterpret_cast<const h8*>(stages + (q & 3) * SBYTES + (wm * 128 + 16 * t) * 64 + lane_off);
  };

  // prologue: chunks 0 .. 3 into stages 0 .. 3, chunk 0's fragments
#pragma unroll
  for (int q = 0; q < NS; ++q) {
#pragma unroll
    for (int j = 0; j < 4; ++j) copy(j, q);
    advance();
  }
  wait_copies<12>();
  lds_barrier();
  read_w(0, wa[0]);
#pragma unroll
  for (int t = 0; t < TM; ++t) xb[t] = read_x(0, t);

  int etile = tile, ekc = 0;  // chunk being multiplied
  auto step = [&](int q, h8 (&wc)[PN][2], h8 (&wnx)[PN][2]) {
    // this wave's copies of chunk q + 1 have landed (issued after them: chunks q + 2
    // and q + 3, and within the first three chunks of a tile after the first, the
    // previous tile's stores), and its fragment reads of chunk q are complete; after
    // the barrier the same holds for every wave, so chunk q's stage is free for
    // chunk q + 4
    if (q >= nk && ekc < 3)
      wait_copies<8 + STORES>();
    else
      wait_copies<8>();
    lds_barrier();
    read_w(q + 1, wnx);
    const int nst = q & 3;
#pragma unroll
    for (int t = 0; t < TM; ++t) {
#pragma unroll
      for (int p = 0; p < PN; ++p)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) acc[p][tt][t] = mfma32(wc[p][tt], xb[t], acc[p][tt][t]);
      __builtin_amdgcn_sched_barrier(0);
      xb[t] = read_x(q + 1, t);
      if ((t & 1) == 0) copy(t >> 1, nst);
      __builtin_amdgcn_sched_barrier(0);
    }
    advance();
    if (ekc == nk - 1) {
      epilogue(etile);
#pragma unroll
      for (int p = 0; p < PN; ++p)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int t = 0; t < TM; ++t) acc[p][tt][t] = zero4();
      ekc = 0;
      etile += stride;
    } else {
      ++ekc;
    }
  };
  // the last step reads the fragments of a chunk past the end: a stage that the
  // surplus copies have filled, read and never used
  for (int q = 0; q < nq; q += 2) {
    step(q, wa[0], wa[1]);
    if (q + 1 >= nq) break;
    step(q + 1, wa[1], wa[0]);
  }
  wait_copies<0>();  // no copy may land in LDS after the workgroup has left it
}

// Variant 8: FP16 X with K % 32 == 0, K >= 128 and N <= kDmaMaxN runs linear_dma_kernel;
// other inputs run variant 7's kernel.
template <typename XT, int EPI, typename OT>
static hipError_t launch_linear_dma(const LinearArgs& a, hipStream_t s) {
  constexpr bool kHalfX = std::is_same<XT, _Float16>::value;
  if constexpr (kHalfX) {
    if (a.k % 32 == 0 && a.k >= 128 && a.k <= (1 << 20) && a.n <= kDmaMaxN) {
      const int64_t tiles = ((a.m + 255) / 256) * ((a.n + 255) / 256);
      if (tiles > 0x7fffffff) return hipErrorInvalidConfiguration;
      auto kernel = linear_dma_kernel<EPI, OT>;
      int64_t grid = std::min<int64_t>(tiles, resident_grid(kernel, 512, 0));
      if (grid >= 8) grid &= ~int64_t{7};
      hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(512), 0, s, a);
      return hipGetLastError();
    }
  }
  return launch_linear_big<256, 256, 64, 2, XT, EPI, OT>(a, s);
}

// ---- X-stationary projection (FP16 X, K = 128 or 256, N % 64 == 0) ----
// For projections with a short K (the d_model-256 QKV projection: 262,144 x 768 x 256),
// each wave keeps its 32 tokens' whole X rows as MFMA fragments in registers (K = 256:
// 64 VGPRs, and as many again for the next tile's rows, loaded one k-step pair per step
// during the current tile's first steps) while the workgroup streams W through LDS in
// 64-row blocks, one block per step.  A step multiplies the workgroup's 256 tokens by the
// block and stores the 256 x 64 results at once: outputs leave as a steady stream of whole
// 128-byte lines (a lane's 8 consecutive features x the four lane groups x the two 32-row
// halves of the block) instead of the large tiles' bursts at tile ends.
//
// The products are those of every other variant - 16x16x32 MFMAs, k-steps in increasing
// order from zero, then bias (and GELU or the q scale) in FP32 - so the results are
// bit-identical to them.  W blocks travel global -> LDS by LDS-DMA copies two steps ahead
// through a ring of three stages; a staged row is K + 16 halves (an odd multiple of 32
// bytes: conflict-free fragment reads) and slot S of a block holds W row
// 32 (S / 32) + pair_row(S % 16, (S / 16) % 2), so lane r of a fragment reads slot r and
// a lane's outputs are 8 consecutive features.  One barrier per step.  Completion is
// tracked by count as in linear_dma_kernel: at the end of step s a wave waits until its
// copies of step s - 1 (the block of step s + 1) have landed, allowing the X loads and
// stores of step s - 1 and the copies, X loads and stores of step s to stay in flight.
constexpr int kXsWaves = 8;
constexpr int kXsTile = 32 * kXsWaves;  // tokens per workgroup tile
constexpr int kXsRows = 64;             // W rows (output features) per step

// f(integral_constant<int, I>) for I = B .. E - 1, in order
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

template <int KS>
struct XsShape {
  static constexpr int K = 32 * KS;
  static constexpr int RU = K / 8 + 2;                            // 16-byte units per staged row
  static constexpr int BLOCKS = RU;                               // 1-KB copies per step (64 RU units)
  static constexpr int CPW = (BLOCKS + kXsWaves - 1) / kXsWaves;  // copy slots per wave
  static constexpr int STAGE = BLOCKS * 1024;                     // bytes per ring stage
  static constexpr int NS = 3;
  static_assert(kXsRows * RU == 64 * BLOCKS, "whole copies");
};

template <int KS, int EPI, typename OT>
__global__ __launch_bounds__(64 * kXsWaves) void linear_xs_kernel(LinearArgs a) {
  using SH = XsShape<KS>;
  constexpr int K = SH::K, CPW = SH::CPW;
  constexpr int STORES = 4 * (sizeof(OT) == 4 ? 2 : 1);  // store instructions per wave and step
  static_assert(EPI == kEpiBias || EPI == kEpiBiasGelu, "plain epilogues");
  __shared__ __align__(16) unsigned char stages[SH::NS * SH::STAGE + 1024];  // + slack for surplus copies
  __shared__ __align__(16) _Float16 bias_s[kDmaMaxN];

  const _Float16* __restrict__ X = static_cast<const _Float16*>(a.x);
  const _Float16* __restrict__ W = a.w;
  const int64_t M = a.m;
  const int N = a.n;
  const int NC = N / kXsRows;  // steps per tile (>= KS, checked by the launcher)
  const int64_t ntiles = (M + kXsTile - 1) / kXsTile;
  // Tile order: XCD x (workgroup b runs on XCD b % 8) owns the x-th eighth of the tiles and
  // walks it upwards.  The fused FFN that writes this projection's input walks the same
  // eighths downwards on the same XCDs, and the attention that reads its output walks them
  // downwards again, so each kernel first reads what the one before wrote last, while it is
  // still in the XCD's L2 and the last-level cache.
  int64_t rs = 0, re = ntiles, slot = blockIdx.x, nsl = gridDim.x;
  if ((gridDim.x & 7) == 0) {
    const int x = blockIdx.x & 7;
    rs = ntiles * x / 8; re = ntiles * (x + 1) / 8; slot = blockIdx.x >> 3; nsl = gridDim.x >> 3;
  }
  if (slot >= re - rs) return;  // uniform per workgroup, before any barrier
  const int my_tiles = (int)((re - rs - 1 - slot) / nsl) + 1;
  auto tile_of = [&](int64_t t) { return rs + slot + t * nsl; };

  const int l = threadIdx.x & 63, wave = wave_id();
  const int r = l & 15, g = l >> 4;

  for (int i = 8 * (int)threadIdx.x; i < N; i += 8 * 64 * kXsWaves)
    *reinterpret_cast<h8*>(&bias_s[i]) = *reinterpret_cast<const h8*>(a.bias + i);

  // ---- copies: slot j of this wave copies block wave + 8 j of a step's W rows ----
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)stages;
  uint32_t coff[CPW], cdst[CPW], cstage[CPW];
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const int b = wave + kXsWaves * j;
    if (b < SH::BLOCKS) {
      const int u = 64 * b + l, slot = u / SH::RU, pos = u % SH::RU;
      const int row = 32 * (slot >> 5) + pair_row(slot & 15, (slot >> 4) & 1);
      coff[j] = pos < K / 8 ? (uint32_t)(row * K + 8 * pos) * 2u : 0u;  // pad units copy element 0
      cdst[j] = lds0 + (uint32_t)(b * 1024);
      cstage[j] = (uint32_t)SH::STAGE;
    } else {
      coff[j] = 0u;
      cdst[j] = lds0 + (uint32_t)(SH::NS * SH::STAGE);  // slack: written, never read
      cstage[j] = 0u;
    }
  }
  // copy slot j of the W block of tile-step c into ring stage st
  auto copy = [&](int j, int c, int st) {
    dma16(coff[j], W + (int64_t)(kXsRows * c) * K, cdst[j] + (uint32_t)st * cstage[j]);
  };

  // ---- X fragments: [t][ks] = token 16 t + r of the wave's 32, k = 32 ks + 8 g .. + 7 ----
  const uint32_t xoff = (uint32_t)(r * K + 8 * g) * 2u;
  auto x_rsrc = [&](int tile_i) {
    const int64_t row0 = tile_of(tile_i) * kXsTile + 32 * wave;
    const uint32_t rows = (uint32_t)max<int64_t>(0, min<int64_t>(32, M - row0));
    return make_rsrc(X + row0 * K, rows * (uint32_t)(K * 2));
  };
  h8 xa[2][KS], xb[2][KS];

  // ---- prologue: the first tile's X, the W blocks of steps 0 and 1 ----
  {
    const __amdgpu_buffer_rsrc_t xr = x_rsrc(0);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        xa[t][ks] = buffer_load8_as_half(xr, xoff + (uint32_t)((16 * t * K + 32 * ks) * 2), X);
  }
#pragma unroll
  for (int q = 0; q < 2; ++q)
#pragma unroll
    for (int j = 0; j < CPW; ++j) copy(j, q % NC, q);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  OT* Y = static_cast<OT*>(a.y);
  int st = 0;  // ring stage of the current step
  // One step: tile-step c of a tile, multiplying the X fragments xc; XI >= 0: the step also
  // loads k-step pair XI of the next tile's X into xn (through a zero-size resource, so
  // without memory traffic, when there is no next tile: the loads stay unconditional and
  // land in xn's own registers).  XPREV: X loads of the step before (-1: decided at run
  // time, for a tile's first step).
  auto step = [&](int c, auto xi_tag, auto xprev_tag, bool prev_loaded, const __amdgpu_buffer_rsrc_t& yr,
                  const __amdgpu_buffer_rsrc_t& xr, h8 (&xc)[2][KS], h8 (&xn)[2][KS]) {
    constexpr int XI = decltype(xi_tag)::value;
    constexpr int XPREV = decltype(xprev_tag)::value;
    // the block of step s + 2 (past the end: a block that nobody reads again)
    const int st2 = st == 0 ? 2 : st - 1;
    const int c2 = c + 2 < NC ? c + 2 : c + 2 - NC;
    const unsigned char* sp = stages + st * SH::STAGE + (r * SH::RU + g) * 16;
    f4 acc[2][2][2];  // [p][tt][t]
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[p][tt][t] = zero4();
    h8 wf[2][2][2];  // [k-step parity][p][tt]
    auto read_w = [&](int ks, h8 (&w)[2][2]) {
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
          w[p][tt] = *reinterpret_cast<const h8*>(sp + ((32 * p + 16 * tt) * SH::RU + 4 * ks) * 16);
    };
    read_w(0, wf[0]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) read_w(ks + 1, wf[(ks + 1) & 1]);
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) acc[p][tt][t] = mfma32(wf[ks & 1][p][tt], xc[t][ks], acc[p][tt][t]);
      if (ks < CPW) copy(ks, c2, st2);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = KS; j < CPW; ++j) copy(j, c2, st2);
    constexpr int XL = XI >= 0 ? 2 : 0;
    if constexpr (XI >= 0) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
        xn[t][XI] = buffer_load8_as_half(xr, xoff + (uint32_t)((16 * t * K + 32 * XI) * 2), X);
    }
    // epilogue: + bias (+ GELU | q scale), a row's two 64-byte runs back to back
    const int nb = kXsRows * c + 8 * g;
    h8 bh[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) bh[p] = *reinterpret_cast<const h8*>(&bias_s[nb + 32 * p]);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[i] = acc[p][0][t][i] + (float)bh[p][i];
          v[4 + i] = acc[p][1][t][i] + (float)bh[p][4 + i];
        }
        if constexpr (EPI == kEpiBiasGelu) {
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = gelu_erf(v[j]);
        }
        if constexpr (EPI == kEpiBias) q_scale8(a, nb + 32 * p, v);
        buffer_store8(yr, (uint32_t)((16 * t + r) * N + nb + 32 * p) * (uint32_t)sizeof(OT), v, Y);
      }
    // this wave's copies of the block of step s + 1 (issued in step s - 1) have landed
    constexpr int BASE = 2 * STORES + CPW + XL;
    if constexpr (XPREV >= 0) {
      wait_copies<BASE + XPREV>();
    } else {
      if (prev_loaded) wait_copies<BASE + 2>();
      else wait_copies<BASE>();
    }
    lds_barrier();
    st = st == 2 ? 0 : st + 1;
  };
  using NoX = std::integral_constant<int, -1>;
  // One tile: steps 0 .. KS - 1 unrolled (each loads one k-step pair of the next tile's X),
  // then the rest as a loop.  A tile's first step follows the previous tile's last, which
  // loaded X only when NC == KS.
  auto run_tile = [&](int tile_i, h8 (&xc)[2][KS], h8 (&xn)[2][KS]) {
    const bool has_next = tile_i + 1 < my_tiles;
    const int64_t row0 = tile_of(tile_i) * kXsTile + 32 * wave;
    const uint32_t rows = (uint32_t)max<int64_t>(0, min<int64_t>(32, M - row0));
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(Y + row0 * N, rows * (uint32_t)N * (uint32_t)sizeof(OT));
    const __amdgpu_buffer_rsrc_t xr = has_next ? x_rsrc(tile_i + 1) : make_rsrc(X, 0u);
    const bool first_prev = tile_i > 0 && NC == KS;
    static_for<0, KS>([&](auto i_tag) {
      constexpr int I = decltype(i_tag)::value;
      step(I, i_tag, std::integral_constant<int, I == 0 ? -1 : 2>{}, first_prev, yr, xr, xc, xn);
    });
#pragma unroll 1
    for (int c = KS; c < NC; ++c) step(c, NoX{}, NoX{}, c == KS, yr, xr, xc, xn);
  };
#pragma unroll 1
  for (int tile_i = 0; tile_i < my_tiles; tile_i += 2) {
    run_tile(tile_i, xa, xb);
    if (tile_i + 1 >= my_tiles) break;
    run_tile(tile_i + 1, xb, xa);
  }
  wait_copies<0>();  // no copy may land in LDS after the workgroup has left it
}

// Variant 9: FP16 X, K = 128 or 256, N % 64 == 0 with N / 64 >= K / 32, bias or bias + GELU
// epilogue runs linear_xs_kernel; other inputs run variant 8.
template <typename XT, int EPI, typename OT>
static hipError_t launch_linear_xs(const LinearArgs& a, hipStream_t s) {
  constexpr bool kOk = std::is_same<XT, _Float16>::value && (EPI == kEpiBias || EPI == kEpiBiasGelu);
  if constexpr (kOk) {
    const int ks = a.k / 32;
    if ((a.k == 128 || a.k == 256) && a.n % kXsRows == 0 && a.n / kXsRows >= ks && a.n <= kDmaMaxN &&
        a.m <= ((int64_t)1 << 40)) {
      const int64_t ntiles = (a.m + kXsTile - 1) / kXsTile;
      auto launch = [&](auto kernel) {
        const int64_t grid = std::min<int64_t>(ntiles, resident_grid(kernel, 64 * kXsWaves, 0));
        hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(64 * kXsWaves), 0, s, a);
        return hipGetLastError();
      };
      if (a.k == 256) return launch(linear_xs_kernel<8, EPI, OT>);
      return launch(linear_xs_kernel<4, EPI, OT>);
    }
  }
  return launch_linear_dma<XT, EPI, OT>(a, s);
}

// ---- projection + residual + LayerNorm with the weights resident in LDS (d = K = 256) ----
// linear_kernel's whole-row LayerNorm variant (same fragments, MFMA order and epilogue
// arithmetic, so the results are bit-identical to variants 1 and 2) restructured for
// streaming: a persistent workgroup loads W (256 x 256 FP16) into LDS once, then each of
// its 8 waves walks 16-row tiles on its own - X fragments straight from memory into
// registers, W fragments from LDS, no barrier after the first - and loads the next
// tile's X before the current tile's epilogue, so its loads, the epilogue's residual
// loads and stores of the 8 waves spread over time instead of meeting at barriers.
constexpr int kResD = 256;
constexpr int kResLdw = kResD + 16;  // W row stride (halves): 544 bytes, conflict-free fragment reads
constexpr int kResWaves = 8;

template <typename OT>
__global__ __launch_bounds__(64 * kResWaves) void linear_ln_resident_kernel(LinearArgs a) {
  constexpr int D = kResD, KS = D / 32, PN = D / 32;
  __shared__ __align__(16) _Float16 ws[D * kResLdw];
  __shared__ __align__(16) float prm[3 * D];  // bias, gamma, beta
  const int64_t M = a.m;
  const int l = threadIdx.x & 63, wave = wave_id();
  const int r = l & 15, g = l >> 4;

  // W rows go to slot w_slot(row), so the 16 lanes of a fragment read consecutive rows
  for (int c = threadIdx.x; c < D * (D / 8); c += 64 * kResWaves) {
    const int row = c / (D / 8), col = (c % (D / 8)) * 8;
    *reinterpret_cast<h8*>(&ws[w_slot(row) * kResLdw + col]) = load8_as_half(a.w + (int64_t)row * D + col);
  }
  for (int i = threadIdx.x; i < D; i += 64 * kResWaves) {
    prm[i] = (float)a.bias[i];
    prm[D + i] = a.gamma[i];
    prm[2 * D + i] = a.beta[i];
  }
  __syncthreads();

  const int64_t ntiles = (M + 15) / 16;
  const int64_t stride = (int64_t)gridDim.x * kResWaves;
  int64_t tile = (int64_t)blockIdx.x * kResWaves + wave;
  if (tile >= ntiles) return;  // after the only barrier

  const _Float16* __restrict__ X = static_cast<const _Float16*>(a.x);
  auto x_rsrc = [&](int64_t t) {
    const int64_t row0 = t * 16;
    const uint32_t rows = (uint32_t)max<int64_t>(0, min<int64_t>(16, M - row0));
    return make_rsrc(X + row0 * D, rows * (uint32_t)(D * 2));
  };
  const uint32_t xoff = (uint32_t)(r * D + 8 * g) * 2u;
  h8 bx[KS];
  {
    const __amdgpu_buffer_rsrc_t xr = x_rsrc(tile);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) bx[ks] = buffer_load8_as_half(xr, xoff + (uint32_t)(64 * ks), X);
  }
  const float inv_n = 1.0f / (float)D;
  OT* __restrict__ Y = static_cast<OT*>(a.y);
  for (; tile < ntiles; tile += stride) {
    f4 acc[PN][2];
#pragma unroll
    for (int p = 0; p < PN; ++p) acc[p][0] = acc[p][1] = zero4();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int p = 0; p < PN; ++p)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const h8 aw = *reinterpret_cast<const h8*>(&ws[(32 * p + 16 * tt + r) * kResLdw + ks * 32 + 8 * g]);
          acc[p][tt] = mfma32(aw, bx[ks], acc[p][tt]);
        }
      // one k-step's 16 fragment reads in flight at a time (unbounded hoisting spills)
      __builtin_amdgcn_sched_barrier(0);
    }
    // the next tile's X, under this tile's epilogue
    if (tile + stride < ntiles) {
      const __amdgpu_buffer_rsrc_t xr = x_rsrc(tile + stride);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) bx[ks] = buffer_load8_as_half(xr, xoff + (uint32_t)(64 * ks), X);
    }
    // R' = acc + b + R ; N' = LayerNorm(R') (whole rows: lane r holds row r's features
    // 32 p + 8 g .. +7, the four lane groups g the rest)
    const uint32_t rows = (uint32_t)max<int64_t>(0, min<int64_t>(16, M - tile * 16));
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.residual + tile * 16 * D, rows * (uint32_t)(D * 4));
    // pass 1: R' in place of the accumulators (the residual read through a buffer
    // resource bounded by the rows that exist), row sums
    float sum = 0.f;
#pragma unroll
    for (int p = 0; p < PN; ++p) {
      const uint32_t off = (uint32_t)(r * D + 32 * p + 8 * g) * 4u;
      const f4 r0 = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rr, off, 0, 0));
      const f4 r1 = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rr, off + 16, 0, 0));
      const float* bp = prm + 32 * p + 8 * g;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[p][0][i] = (acc[p][0][i] + bp[i]) + r0[i];
        acc[p][1][i] = (acc[p][1][i] + bp[4 + i]) + r1[i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) sum += acc[p][0][i];
#pragma unroll
      for (int i = 0; i < 4; ++i) sum += acc[p][1][i];
    }
    const float mean = sum_over_groups(sum) * inv_n;
    float sq = 0.f;
#pragma unroll
    for (int p = 0; p < PN; ++p)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float c = acc[p][tt][i] - mean;
          sq += c * c;
        }
    const float rstd = rsqrtf(sum_over_groups(sq) * inv_n + a.eps);
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.residual_out + tile * 16 * D, rows * (uint32_t)(D * 4));
    const __amdgpu_buffer_rsrc_t yo = make_rsrc(Y + tile * 16 * D, rows * (uint32_t)(D * sizeof(OT)));
#pragma unroll
    for (int p = 0; p < PN; ++p) {
      const int n = 32 * p + 8 * g;
      float v[8], o[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = acc[p][0][i];
        v[4 + i] = acc[p][1][i];
      }
      buffer_store8(ro, (uint32_t)(r * D + n) * 4u, v, a.residual_out);
      const float* gm = prm + D + n;
      const float* bt = prm + 2 * D + n;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = (v[j] - mean) * rstd * gm[j] + bt[j];
      pin_f32x8(o);  // rounded to FP32, then to the output type (no fused FMA + conversion)
      buffer_store8(yo, (uint32_t)(r * D + n) * (uint32_t)sizeof(OT), o, Y);
    }
  }
}

template <typename OT>
static hipError_t launch_linear_ln_resident(const LinearArgs& a, hipStream_t s) {
  if (a.n != kResD || a.k != kResD) return (hipError_t)MPK_EUNSUPPORTED;
  if (a.m > ((int64_t)1 << 40)) return (hipError_t)MPK_EUNSUPPORTED;
  const int64_t ntiles = (a.m + 15) / 16;
  auto kernel = linear_ln_resident_kernel<OT>;
  const int64_t grid = std::min<int64_t>((ntiles + kResWaves - 1) / kResWaves, resident_grid(kernel, 64 * kResWaves, 0));
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(64 * kResWaves), 0, s, a);
  return hipGetLastError();
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
//   5: BM256 BN128 (2x2 waves, 128x64 per wave, double-buffered LDS)   large M and N
//   6: as 5 with single-buffered LDS (two workgroups per CU)
//   7: BM256 BN256 (2x4 waves, 128x64 per wave, double-buffered LDS)
//   8: as 7 with LDS-DMA operand staging (FP16 X; other inputs run 7)
//   9: X-stationary 256-token tiles, W streamed in 64-row blocks (FP16 X, K = 128 or 256,
//      N % 64 == 0, bias / GELU epilogues; other inputs run 8)
template <typename XT, int EPI, typename OT>
static hipError_t linear_variant(int variant, const LinearArgs& a, hipStream_t s) {
  switch (variant) {
    case 1: return launch_linear<128, 128, 64, 2, XT, EPI, OT>(a, s);
    case 2: return launch_linear<128, 64, 64, 4, XT, EPI, OT>(a, s);
    case 3: return launch_linear<128, 32, 64, 4, XT, EPI, OT>(a, s);
    case 4: return launch_linear<64, 128, 64, 1, XT, EPI, OT>(a, s);
    case 5: return launch_linear_big<256, 128, 64, 2, XT, EPI, OT>(a, s);
    case 6: return launch_linear_big<256, 128, 64, 1, XT, EPI, OT>(a, s);
    case 7: return launch_linear_big<256, 256, 64, 2, XT, EPI, OT>(a, s);
    case 8: return launch_linear_dma<XT, EPI, OT>(a, s);
    case 9: return launch_linear_xs<XT, EPI, OT>(a, s);
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
  // variant 4: d = K = 256 with FP16 X, W resident in LDS, independent waves (bit-identical
  // to variants 1 and 2)
  if (variant == 4) {
    if constexpr (std::is_same<XT, _Float16>::value) return launch_linear_ln_resident<OT>(a, s);
    return (hipError_t)MPK_EUNSUPPORTED;
  }
  // variant 3: large GEMM tiles holding whole rows, with the cross-wave LayerNorm
  // epilogue (any K): 256 x 256 tiles for N = 256, 128 x 512 tiles (32-wide K chunks, so
  // that two stages fit the LDS) for N = 512
  if (variant == 3) {
    if (a.n == 256) return launch_linear_big<256, 256, 64, 2, XT, kEpiResidualLNTile, OT>(a, s);
    if (a.n == 512) return launch_linear_big<128, 512, 32, 2, XT, kEpiResidualLNTile, OT>(a, s);
    return (hipError_t)MPK_EUNSUPPORTED;
  }
  if (a.k != a.n) return (hipError_t)MPK_EUNSUPPORTED;
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
  // X-stationary tiles from 256 workgroup tiles on (measured on MI355X with the q-scaled
  // bias epilogue: 262,144 x 768 x 256 in 142 vs 170 us for variant 8, 65,536 x 768 x 256
  // 39 vs 42 us, 65,536 x 384 x 128 17.6 vs 21.4 us)
  if ((k == 128 || k == 256) && n % 64 == 0 && n / 64 >= k / 32 && n <= 8192 && m >= (int64_t)256 * 256) return 9;
  if (n % 256 == 0 && k >= 256 && k <= (1 << 20) && ((m + 255) / 256) * (n / 256) >= 256) return 8;
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

extern "C" int mpk_linear_qscaled(const void* x, int x_dtype, const void* w, const void* b, void* y, int y_dtype,
                                  int64_t m, int32_t n, int32_t k, int32_t q_cols, float q_scale, int variant,
                                  void* stream) {
  if (!x || !w || !b || !y || m < 0 || n <= 0 || k <= 0 || q_cols < 0 || q_cols > n) return MPK_EINVAL;
  if ((x_dtype != kF32 && x_dtype != kF16) || (y_dtype != kF32 && y_dtype != kF16)) return MPK_EINVAL;
  if (n % 8 != 0 || k % 8 != 0 || q_cols % 8 != 0) return MPK_EUNSUPPORTED;
  if (!aligned16(x) || !aligned16(w) || !aligned16(b) || !aligned16(y)) return MPK_EALIGN;
  if (m == 0) return MPK_OK;
  if (variant == 0) variant = mpk_linear_auto_variant(m, n, k);
  LinearArgs a{};
  a.x = x; a.w = static_cast<const _Float16*>(w); a.bias = static_cast<const _Float16*>(b); a.y = y;
  a.m = m; a.n = n; a.k = k;
  a.q_cols = q_cols; a.q_scale = q_scale;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  const bool xf = x_dtype == kF32, yf = y_dtype == kF32;
  if (xf) e = yf ? linear_variant<float, kEpiBias, float>(variant, a, s)
                 : linear_variant<float, kEpiBias, _Float16>(variant, a, s);
  else e = yf ? linear_variant<_Float16, kEpiBias, float>(variant, a, s)
              : linear_variant<_Float16, kEpiBias, _Float16>(variant, a, s);
  return (int)e;
}

extern "C" int mpk_linear_residual_layernorm_auto_variant(int64_t m, int32_t d) {
  if (d == 256) return 3;
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
  if (variant < 1 || variant > 4) return MPK_EUNSUPPORTED;
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

extern "C" int mpk_linear_residual(const void* x, int x_dtype, const void* w, const void* b, const float* residual,
                                   float* y, int64_t m, int32_t n, int32_t k, int variant, void* stream) {
  if (!x || !w || !b || !residual || !y || m < 0 || n <= 0 || k <= 0) return MPK_EINVAL;
  if (x_dtype != kF32 && x_dtype != kF16) return MPK_EINVAL;
  if (n % 8 != 0 || k % 8 != 0) return MPK_EUNSUPPORTED;
  if (!aligned16(x) || !aligned16(w) || !aligned16(b) || !aligned16(residual) || !aligned16(y)) return MPK_EALIGN;
  if (m == 0) return MPK_OK;
  if (variant == 0) variant = mpk_linear_auto_variant(m, n, k);
  LinearArgs a{};
  a.x = x; a.w = static_cast<const _Float16*>(w); a.bias = static_cast<const _Float16*>(b); a.y = y;
  a.residual = residual; a.m = m; a.n = n; a.k = k;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const hipError_t e = x_dtype == kF32 ? linear_variant<float, kEpiBiasResidual, float>(variant, a, s)
                                       : linear_variant<_Float16, kEpiBiasResidual, float>(variant, a, s);
  return (int)e;
}

extern "C" int mpk_linear_add_layernorm(const void* x, int x_dtype, const void* w, const void* b,
                                        const float* residual, const float* gamma, const float* beta,
                                        float* residual_out, void* normalized_out, int normalized_dtype, int64_t m,
                                        int32_t n, int32_t k, float eps, void* stream) {
  if (!x || !w || !b || !residual || !gamma || !beta || !residual_out || !normalized_out || m < 0 || n <= 0 ||
      k <= 0)
    return MPK_EINVAL;
  if ((x_dtype != kF32 && x_dtype != kF16) || (normalized_dtype != kF32 && normalized_dtype != kF16))
    return MPK_EINVAL;
  if ((n != 256 && n != 512) || k % 8 != 0) return MPK_EUNSUPPORTED;
  if (!aligned16(x) || !aligned16(w) || !aligned16(b) || !aligned16(residual) || !aligned16(gamma) ||
      !aligned16(beta) || !aligned16(residual_out) || !aligned16(normalized_out))
    return MPK_EALIGN;
  if (m == 0) return MPK_OK;
  LinearArgs a{};
  a.x = x; a.w = static_cast<const _Float16*>(w); a.bias = static_cast<const _Float16*>(b); a.y = normalized_out;
  a.residual = residual; a.gamma = gamma; a.beta = beta; a.residual_out = residual_out;
  a.m = m; a.n = n; a.k = k; a.eps = eps;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  const bool xf = x_dtype == kF32, of = normalized_dtype == kF32;
  // FP16 X with d = K = 256 and fewer 256-row tiles than a device has CUs: the
  // weights-resident whole-row kernel (16-row wave tiles fill the device; measured on MI355X:
  // 22 vs 42 us at 32,771 rows, 18 vs 30 us at 8,192; level at 65,536, the large tiles ahead
  // at 131,072 and level again at cfg5's 262,144)
  const int v = (!xf && n == kResD && k == kResD && m < (int64_t)256 * 256) ? 4 : 3;
  if (xf) e = of ? linear_ln<float, float>(v, a, s) : linear_ln<float, _Float16>(v, a, s);
  else e = of ? linear_ln<_Float16, float>(v, a, s) : linear_ln<_Float16, _Float16>(v, a, s);
  return (int)e;
}
