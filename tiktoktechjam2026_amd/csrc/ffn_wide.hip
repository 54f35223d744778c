// Wide fused FFN + residual + LayerNorm (d_model 256) on v_mfma_f32_32x32x16_f16.
// Two kernels with identical arithmetic: ffn_wide_kernel (variant 3, one wave per
// SIMD, described here) and ffn_roles_kernel (variant 4, the library's choice: a
// vector wave and a matrix wave per SIMD, described at its definition).
//
// Replaces, for the wide models, the reference's FFN with its residual add and
// the LayerNorm that follows it: mixed_ffn_add_layer_norm
// (mixed_precision/triton_linear.py:327-378, kernel :128-185, hard-wired to
// D = F = 128 there), generalised to D = 256 with any F (a multiple of 32).
// Same rounding points:
//   H  = GELU_erf(fp16(X) W_in^T + b_in)         FP32 accumulate, FP32 GELU, then FP16
//   R' = fp16(H) W_out^T + b_out + R             FP32
//   N' = LayerNorm(R') (two-pass FP32 statistics), stored FP32 or FP16
//
// Work split.  A workgroup of 4 waves (one per SIMD) owns 128 tokens, 32 per
// wave, and walks the hidden layer in 32-feature chunks f0 = 0, 32, ...:
//   stage 1  H^T [32 x 32 tokens] = W_in[f0 + kappa32(rho), :] X^T      (D/16 MFMAs)
//   GELU     register 8s + j of lane (i, h) is hidden feature f0 + 16s + 8h + j of
//            token i (mpk_common.h), i.e. fp16(GELU(H + b_in)) there is the B operand
//            of k-step s of stage 2 - the hidden activation never leaves the registers
//   stage 2  Y^T [D x 32 tokens] += W_out[32p + kappa32(rho), f0 + 16s ..] fp16(H)^T
//                                                                         (2 D/32 MFMAs)
// With output feature 32p + kappa32(rho) in MFMA row rho, lane (i, h) holds
// features 32p + 16r + 8h + 0..7 (r = 0, 1) of token i, so the epilogue
// (+ b_out + residual, LayerNorm over the row, whose other half is in lane
// i + 32) works on runs of 8 features and stores 32 (FP32) / 16 (FP16) bytes.
//
// Pipeline.  Per chunk a wave issues 32 MFMAs (~1024 matrix cycles) and the
// GELU of 16 values per lane (~1000 VALU cycles).  A 32x32x16 MFMA holds the
// VALU issue for about a quarter of its 32 cycles (measured on MI355X), so the
// two overlap when they are independent: iteration g runs the GELU of chunk g
// beside the stage 1 product of chunk g + 1 and the stage 2 product of chunk
// g - 1, in one basic block whose instruction order is pinned (one MFMA, eight
// VALU operations, one LDS read, repeated).  A wave keeps 32 x D FP32
// accumulators (in AGPRs) and its tokens' FP16 X fragments, which is why the
// workgroup runs one wave per SIMD with the whole register file.
//
// Weights stream through LDS, copied global -> LDS by the DMA form of global
// loads (no registers), each chunk two steps before its first use: W_in chunks
// in a ring of 3 buffers (g + 1 read, g + 2 landing, g + 3 issued), W_out chunks
// in a ring of 3 (g - 1 read, g landed, g + 1 issued); one barrier per chunk.  Rows are padded by 16 bytes (W_in 528 B,
// W_out 80 B) so the fragment reads of 16 consecutive lanes hit distinct banks;
// the DMA fills the padded layout linearly and its lanes that fall on padding
// load filler that no fragment read touches.
#include <algorithm>
#include <type_traits>

#include "ffn.h"

namespace mpk {

namespace {

constexpr int kNW = 4;           // waves per workgroup, one per SIMD
constexpr int kNT = 64 * kNW;    // threads
constexpr int kTok = 32 * kNW;   // tokens per tile

template <int D>
struct WideShape {
  static constexpr int KS = D / 16;                          // stage-1 k-steps
  static constexpr int PT = D / 32;                          // stage-2 output tiles
  static constexpr int LDI = D + 8;                          // W_in row stride (halves)
  static constexpr int LDO = 40;                             // W_out row stride (halves)
  static constexpr int WIN_UNITS = 32 * (LDI / 8);           // 16-byte units of a padded W_in chunk
  static constexpr int WOUT_UNITS = D * (LDO / 8);
  static constexpr int WIN_BLOCKS = (WIN_UNITS + 63) / 64;   // 1-KB DMA blocks
  static constexpr int WOUT_BLOCKS = (WOUT_UNITS + 63) / 64;
  static constexpr int WIN_H = WIN_BLOCKS * 512;             // halves per W_in buffer
  static constexpr int WOUT_H = WOUT_BLOCKS * 512;
  static constexpr int BLOCKS = WIN_BLOCKS + WOUT_BLOCKS;    // DMA blocks per chunk
  static constexpr int DMA_J = (BLOCKS + kNW - 1) / kNW;     // DMA slots per wave
  static constexpr int SLACK_H = 512;                        // target of surplus slots
  static constexpr int LDS_H = 3 * WIN_H + 3 * WOUT_H + SLACK_H;
};

// Position in the chunk stream: g % 3, and the chunk ids (g + 3) % C and (g + 1) % C
// of the W_in / W_out copies issued at step g.
struct Ring {
  int g3, in_chunk, out_chunk;
  __device__ void advance(int nchunks) {
    g3 = g3 == 2 ? 0 : g3 + 1;
    in_chunk = in_chunk + 1 == nchunks ? 0 : in_chunk + 1;
    out_chunk = out_chunk + 1 == nchunks ? 0 : out_chunk + 1;
  }
};

// What one chunk step hands to the next: the stage-1 result of the chunk whose GELU
// runs next, its b_in values (feature f0 + 16s + 8h + j in bias[8s + j]) and the
// FP16 GELU of the chunk before it (the stage-2 B operands).  Steps alternate
// between two of these, so no registers are copied between steps.
struct ChunkState {
  f16v h;
  float bias[16];
  h8 hb0, hb1;
};

}  // namespace

template <int D, typename XT, typename OT>
__global__ __launch_bounds__(kNT, 1) void ffn_wide_kernel(FfnArgs a) {
  using SH = WideShape<D>;
  static_assert(D % 32 == 0 && D <= 256, "register budget: 32 x D FP32 accumulators + D/2 X registers per lane");

  __shared__ _Float16 lds[SH::LDS_H];
  __shared__ float prm[3 * D];            // b_out, gamma, beta (FP32)
  __shared__ float bin[kWideFfnMaxF];     // b_in (FP32)
  _Float16* const win_buf = lds;                    // 3 x WIN_H
  _Float16* const wout_buf = lds + 3 * SH::WIN_H;   // 3 x WOUT_H
  _Float16* const slack = wout_buf + 3 * SH::WOUT_H;

  const XT* __restrict__ X = static_cast<const XT*>(a.x);
  const int F = a.f;
  const int C = F / 32;
  const int64_t M = a.m;
  const int64_t ntiles = (M + kTok - 1) / kTok;
  int64_t tile = blockIdx.x;
  if (tile >= ntiles) return;  // uniform per workgroup, before any barrier
  const int my_tiles = (int)((ntiles - 1 - tile) / gridDim.x) + 1;

  const int l = threadIdx.x & 63, wave = wave_id();
  const int li = l & 31, hh = l >> 5;
  const int kr = kappa32(li);

  // ---- DMA slots: slot j*kNW + wave of every chunk copy (wave-uniform kind) ----
  // Per-lane byte offsets relative to the chunk's first element are the same for
  // every chunk; filler lanes (row padding, block rounding, surplus slots) load
  // element 0 of the chunk.
  uint32_t dma_off[SH::DMA_J];
#pragma unroll
  for (int j = 0; j < SH::DMA_J; ++j) {
    const int slot = j * kNW + wave;
    uint32_t off = 0;
    if (slot < SH::WIN_BLOCKS) {
      const int u = slot * 64 + l, row = u / (SH::LDI / 8), pos = u % (SH::LDI / 8);
      off = (row < 32 && pos < D / 8) ? (uint32_t)(row * D + 8 * pos) * 2u : 0u;
    } else if (slot < SH::BLOCKS) {
      const int u = (slot - SH::WIN_BLOCKS) * 64 + l, row = u / (SH::LDO / 8), pos = u % (SH::LDO / 8);
      off = (row < D && pos < 4) ? (uint32_t)(row * F + 8 * pos) * 2u : 0u;
    }
    dma_off[j] = off;
  }
  // Per slot (wave-uniform): LDS destination = dst0 + bi * dst_in + bo * dst_out, and
  // whether the source is W_out - plain scalar arithmetic per copy, no branches.
  const uint32_t lds_win = (uint32_t)(uintptr_t)(lds_void*)win_buf;
  const uint32_t lds_wout = (uint32_t)(uintptr_t)(lds_void*)wout_buf;
  const uint32_t lds_slack = (uint32_t)(uintptr_t)(lds_void*)slack;
  uint32_t dst0[SH::DMA_J], dst_in[SH::DMA_J], dst_out[SH::DMA_J], from_out[SH::DMA_J];
#pragma unroll
  for (int j = 0; j < SH::DMA_J; ++j) {
    const int slot = j * kNW + wave;
    const bool is_in = slot < SH::WIN_BLOCKS, is_out = !is_in && slot < SH::BLOCKS;
    dst0[j] = is_in ? lds_win + (uint32_t)(slot * 1024)
                    : is_out ? lds_wout + (uint32_t)((slot - SH::WIN_BLOCKS) * 1024) : lds_slack;
    dst_in[j] = is_in ? (uint32_t)(SH::WIN_H * 2) : 0u;
    dst_out[j] = is_out ? (uint32_t)(SH::WOUT_H * 2) : 0u;
    from_out[j] = is_out ? 1u : 0u;
  }
  // W_in chunk ci -> W_in buffer bi, W_out chunk co -> W_out buffer bo
  auto issue = [&](int ci, int bi, int co, int bo) {
    const uint64_t src_in = (uint64_t)(uintptr_t)(a.w_in + (int64_t)(32 * ci) * D);
    const uint64_t src_out = (uint64_t)(uintptr_t)(a.w_out + 32 * co);
#pragma unroll
    for (int j = 0; j < SH::DMA_J; ++j) {
      const uint64_t src = src_in + (uint64_t)from_out[j] * (src_out - src_in);
      dma16(dma_off[j], (const void*)(uintptr_t)src, dst0[j] + (uint32_t)bi * dst_in[j] + (uint32_t)bo * dst_out[j]);
    }
  };

  // X fragments of the wave's 32 tokens (stage-1 B operand): d = 16 ks + 8 hh .. +7
  h8 xf[SH::KS];
  auto load_x = [&](int64_t t) {
    const int64_t row0 = t * kTok + 32 * wave;
    const uint32_t rows = (uint32_t)max<int64_t>(0, min<int64_t>(32, M - row0));
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(X + row0 * D, rows * (uint32_t)(D * sizeof(XT)));
#pragma unroll
    for (int ks = 0; ks < SH::KS; ++ks)
      xf[ks] = buffer_load8_as_half(xr, (uint32_t)((li * D + 16 * ks + 8 * hh) * sizeof(XT)), X);
  };

  // b_in (FP32, staged once per workgroup) of chunk c
  auto load_bias = [&](ChunkState& st, int c) {
    const float* bias = bin + 32 * c + 8 * hh;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 b = *reinterpret_cast<const float4*>(bias + 16 * (q >> 1) + 4 * (q & 1));
      st.bias[4 * q] = b.x; st.bias[4 * q + 1] = b.y; st.bias[4 * q + 2] = b.z; st.bias[4 * q + 3] = b.w;
    }
  };

  f16v yacc[SH::PT];  // Y^T accumulators of the tile

  // One chunk step from `in` to `out`.  S1: the stage 1 product of the next chunk
  // (W_in g + 1) into out.h; S2: the stage 2 product of the previous chunk (W_out
  // g - 1, operands in.hb0 / in.hb1); always the GELU of chunk c (in.h + in.bias)
  // into out.hb0 / out.hb1.  The MFMAs and the GELU are independent, so they are
  // written - and fenced - as one interleaved stream: segments of four MFMAs (stage
  // 1 and stage 2 alternating, each fragment read PF MFMAs ahead) beside two GELU
  // elements whose dependency chains interleave.
  auto step = [&](auto s1_tag, auto s2_tag, int c, const Ring& rg, const ChunkState& in, ChunkState& out) {
    constexpr bool S1 = decltype(s1_tag)::value, S2 = decltype(s2_tag)::value;
    constexpr int N1 = S1 ? SH::KS : 0, N2 = S2 ? 2 * SH::PT : 0, N = N1 + N2;
    constexpr int PF = 4;  // fragment prefetch distance
    const int g3p1 = rg.g3 == 2 ? 0 : rg.g3 + 1, g3m1 = rg.g3 == 0 ? 2 : rg.g3 - 1;
    load_bias(out, c + 1 == C ? 0 : c + 1);          // the next GELU's b_in
    issue(rg.in_chunk, rg.g3, rg.out_chunk, g3p1);   // W_in g + 3 -> g % 3, W_out g + 1 -> (g + 1) % 3
    const _Float16* wi = win_buf + g3p1 * SH::WIN_H + kr * SH::LDI + 8 * hh;   // W_in g + 1
    const _Float16* wo = wout_buf + g3m1 * SH::WOUT_H + kr * SH::LDO + 8 * hh;  // W_out g - 1
    // MFMA i: stage 1 k-step i / 2 (even i) and stage 2 fragment (p, s) = (i / 4, (i / 2) % 2)
    // (odd i) when both run; otherwise the one stage in order.
    auto is_s1 = [&](int i) { return N2 == 0 || (N1 != 0 && (i & 1) == 0); };
    auto idx = [&](int i) { return (N1 != 0 && N2 != 0) ? i >> 1 : i; };
    auto frag = [&](int i) {
      const int k = idx(i);
      return is_s1(i) ? *reinterpret_cast<const h8*>(wi + 16 * k)
                      : *reinterpret_cast<const h8*>(wo + 32 * (k >> 1) * SH::LDO + 16 * (k & 1));
    };
    h8 fr[PF];
#pragma unroll
    for (int i = 0; i < PF && i < N; ++i) fr[i] = frag(i);
    if constexpr (S1) {
#pragma unroll
      for (int e = 0; e < 16; ++e) out.h[e] = 0.f;
    }
    auto gelu_one = [&](int e) {
      const _Float16 hv = (_Float16)gelu_erf(in.h[e] + in.bias[e]);
      if (e < 8) out.hb0[e] = hv; else out.hb1[e - 8] = hv;
    };
    constexpr int SEG = N / 4 > 0 ? N / 4 : 1;  // segments of four MFMAs
    constexpr int EPS = 16 / SEG;               // GELU elements per segment
    static_assert(N % 4 == 0 && EPS * SEG == 16, "segment split");
#pragma unroll
    for (int k = 0; k < SEG; ++k) {
#pragma unroll
      for (int i = 4 * k; i < 4 * k + 4 && i < N; ++i) {
        const h8 w = fr[i % PF];
        if (i + PF < N) fr[i % PF] = frag(i + PF);
        if (is_s1(i)) {
          out.h = mfma32x32(w, xf[idx(i)], out.h);
        } else {
          const int q = idx(i);
          yacc[q >> 1] = mfma32x32(w, (q & 1) ? in.hb1 : in.hb0, yacc[q >> 1]);
        }
      }
#pragma unroll
      for (int e = EPS * k; e < EPS * (k + 1); ++e) gelu_one(e);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // stage 2 of a tile's last chunk (W_out chunk g - 1, operands st.hb0 / st.hb1)
  auto tail = [&](const Ring& rg, const ChunkState& st) {
    const _Float16* wo = wout_buf + (rg.g3 == 0 ? 2 : rg.g3 - 1) * SH::WOUT_H + kr * SH::LDO + 8 * hh;
#pragma unroll
    for (int i = 0; i < 2 * SH::PT; ++i)
      yacc[i >> 1] = mfma32x32(*reinterpret_cast<const h8*>(wo + 32 * (i >> 1) * SH::LDO + 16 * (i & 1)),
                               (i & 1) ? st.hb1 : st.hb0, yacc[i >> 1]);
  };

  using T = std::integral_constant<bool, true>;
  using Fa = std::integral_constant<bool, false>;

  // ---- prologue: parameters, W_in chunks 0..2, W_out chunk 0, the first X tile ----
  for (int i = threadIdx.x; i < F; i += kNT) bin[i] = (float)a.b_in[i];
  for (int i = threadIdx.x; i < D; i += kNT) {
    prm[i] = (float)a.b_out[i];
    prm[D + i] = a.gamma[i];
    prm[2 * D + i] = a.beta[i];
  }
  issue(0, 0, 0, 0);                     // W_in 0 -> buffer 0, W_out 0 -> buffer 0
  issue(1 % C, 1, 0, 0);                 // W_in 1 -> buffer 1 (W_out 0 again: same data)
  issue(2 % C, 2, 0, 0);                 // W_in 2 -> buffer 2
  load_x(tile);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // Chunk stream index g (continues across tiles): W_in and W_out chunk g sit in
  // buffer g % 3 of their rings.  At step g the copies of W_in g + 3 and W_out g + 1
  // are issued (into the buffers of W_in g and W_out g - 2, both last read before the
  // previous barrier), two steps before their first use, and the step ends waiting
  // only for the previous step's copies.  The ring position is a small wave-uniform
  // counter.
  Ring g{};
  g.in_chunk = 3 % C;
  g.out_chunk = 1 % C;
  ChunkState sa, sb;
  auto finish = [&](auto tag) {  // end of a step: this wave's older copies landed, workgroup meets
    wait_copies<decltype(tag)::value>();
    lds_barrier();
    g.advance(C);
  };
  using Steady = std::integral_constant<int, SH::DMA_J>;
  using Full = std::integral_constant<int, 0>;
  using TileEnd = std::integral_constant<int, SH::DMA_J + SH::KS>;
  for (int it = 0; it < my_tiles; ++it, tile += gridDim.x) {
#pragma unroll
    for (int p = 0; p < SH::PT; ++p)
#pragma unroll
      for (int e = 0; e < 16; ++e) yacc[p][e] = 0.f;
    // stage 1 of the tile's chunk 0 (W_in chunk g) and its b_in
    {
      const _Float16* wi = win_buf + g.g3 * SH::WIN_H + kr * SH::LDI + 8 * hh;
#pragma unroll
      for (int e = 0; e < 16; ++e) sa.h[e] = 0.f;
#pragma unroll
      for (int ks = 0; ks < SH::KS; ++ks) sa.h = mfma32x32(*reinterpret_cast<const h8*>(wi + 16 * ks), xf[ks], sa.h);
      load_bias(sa, 0);
    }
    lds_barrier();  // W_in buffer g % 3 is the next copy's target
    const bool more = it + 1 < my_tiles;
    // chunk steps: the first (no stage 2 yet), steady ones in pairs (sa -> sb -> sa),
    // the last (no stage 1)
    if (C == 1) {
      step(Fa{}, Fa{}, 0, g, sa, sb);
      if (more) load_x(tile + gridDim.x);
      more ? finish(TileEnd{}) : finish(Steady{});
      tail(g, sb);
    } else {
      step(T{}, Fa{}, 0, g, sa, sb);
      // a full wait once per tile: every load the compiler tracks (spill reloads of the
      // tile prologue included) is complete before the steady loop, whose waits would
      // otherwise also drain the chunk copies in flight
      finish(Full{});
      int c = 1;
#pragma unroll 1
      for (; c + 2 < C; c += 2) {
        step(T{}, T{}, c, g, sb, sa);
        finish(Steady{});
        step(T{}, T{}, c + 1, g, sa, sb);
        finish(Steady{});
      }
      if (c + 1 < C) {  // one steady step left, then the last from sa
        step(T{}, T{}, c, g, sb, sa);
        finish(Steady{});
        step(Fa{}, T{}, C - 1, g, sa, sb);
        if (more) load_x(tile + gridDim.x);  // X fragments are dead after the last stage 1
        more ? finish(TileEnd{}) : finish(Steady{});
        tail(g, sb);
      } else {          // the last from sb
        step(Fa{}, T{}, C - 1, g, sb, sa);
        if (more) load_x(tile + gridDim.x);
        more ? finish(TileEnd{}) : finish(Steady{});
        tail(g, sa);
      }
    }

    // ---- epilogue: + b_out + residual, two-pass LayerNorm over the row, stores ----
    const int64_t row0 = tile * kTok + 32 * wave;
    const uint32_t rows = (uint32_t)max<int64_t>(0, min<int64_t>(32, M - row0));
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.residual + row0 * D, rows * (uint32_t)(D * 4));
    // residual_out NULL: a zero-size resource drops the stores, which still issue (the
    // copy waits count them)
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.residual_out ? a.residual_out + row0 * D : nullptr,
                                                a.residual_out ? rows * (uint32_t)(D * 4) : 0u);
    const __amdgpu_buffer_rsrc_t no =
        make_rsrc(static_cast<OT*>(a.normalized_out) + row0 * D, rows * (uint32_t)(D * sizeof(OT)));
    const float* bo = prm;
    const float* gm = prm + D;
    const float* bt = prm + 2 * D;
    typedef float v4 __attribute__((ext_vector_type(4)));
    float sum = 0.f;
#pragma unroll
    for (int p = 0; p < SH::PT; ++p)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int n = 32 * p + 16 * r + 8 * hh;
        const uint32_t off = (uint32_t)((li * D + n) * 4);
        const v4 r0 = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(rr, off, 0, 0));
        const v4 r1 = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(rr, off + 16, 0, 0));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float v = (yacc[p][8 * r + j] + bo[n + j]) + (j < 4 ? r0[j] : r1[j - 4]);
          yacc[p][8 * r + j] = v;
          sum += v;
        }
        // residual_out leaves here, before the LayerNorm statistics: the stores of all
        // workgroups' epilogues meet in one burst, and the earlier it starts the
        // sooner the next tile's copy waits (which cover these stores) are free
        float vv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) vv[j] = yacc[p][8 * r + j];
        buffer_store8(ro, off, vv, a.residual_out);
      }
    const float inv_d = 1.0f / (float)D;
    const float mean = sum_over_halves(sum) * inv_d;
    float sq = 0.f;
#pragma unroll
    for (int p = 0; p < SH::PT; ++p)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float d0 = yacc[p][e] - mean;
        sq += d0 * d0;
      }
    const float rstd = rsqrtf(sum_over_halves(sq) * inv_d + a.eps);
#pragma unroll
    for (int p = 0; p < SH::PT; ++p)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int n = 32 * p + 16 * r + 8 * hh;
        float o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = (yacc[p][8 * r + j] - mean) * rstd * gm[n + j] + bt[n + j];
        pin_f32x8(o);  // rounded to FP32, then to the output type (no fused FMA + conversion)
        buffer_store8(no, (uint32_t)((li * D + n) * sizeof(OT)), o, static_cast<OT*>(a.normalized_out));
      }
  }
  wait_copies<0>();  // surplus chunk copies issued near the end have landed
}

// ---------------------------------------------------------------------------
// Role-split wide FFN (variant 4): vector waves and matrix waves.
//
// Same work split and rounding points as ffn_wide_kernel (32x32x16 MFMAs, the
// kappa32 row order, 128-token tiles of 4 x 32 tokens, 32-feature hidden chunks),
// but each SIMD runs two waves that share the work of one 32-token slice:
//   vector wave 4 + w  holds the slice's X fragments: the stage-1 product of chunk
//                      g (MFMAs, result kept in registers) interleaved with the
//                      GELU of chunk g - 1, whose FP16 result goes to LDS; it also
//                      issues the weight copies and loads the next tile's X
//   matrix wave w      holds the slice's 32 x D FP32 accumulators: the stage-2
//                      product of chunk g - 2 (operands from LDS) and the tile
//                      epilogue (+ b_out + residual, LayerNorm, stores)
// so the GELU's VALU work runs beside the other wave's MFMAs, each wave needs
// about half the registers of the one-wave-per-SIMD kernel (two fit per SIMD),
// and the waves that wait for the weight copies never store (vmcnt also counts
// stores): the epilogue's stores drain while the next tile runs.
//
// The chunk stream g = 0, 1, ... continues across the workgroup's tiles (chunk
// g % C of tile g / C).  Step g: W_in chunk g is read from buffer g % 3 of its ring
// and W_out chunk g - 2 from buffer (g - 2) % 3 of its ring; the vector waves copy
// W_in chunk g + 2 and W_out chunk g, each into the buffer read last at step g - 1,
// and end the step waiting for their copies of step g - 1.  GELU outputs of chunk
// g - 1 are written at step g into exchange parity (g - 1) % 2 and read at step
// g + 1.  One barrier per step for all 8 waves; a tile's epilogue follows the
// barrier of the step that finishes its stage 2.
namespace {

constexpr int kRW = 8;          // waves per workgroup: 4 matrix + 4 vector
constexpr int kRT = 64 * kRW;   // threads

template <int D>
struct RoleShape {
  static constexpr int KS = D / 16;                           // stage-1 k-steps
  static constexpr int PT = D / 32;                           // stage-2 output tiles
  static constexpr int LDI = D + 8;                           // W_in row stride (halves)
  static constexpr int LDO = 40;                              // W_out row stride (halves)
  static constexpr int WIN_BLOCKS = (32 * (LDI / 8) + 63) / 64;
  static constexpr int WOUT_BLOCKS = (D * (LDO / 8) + 63) / 64;
  static constexpr int WIN_H = WIN_BLOCKS * 512;
  static constexpr int WOUT_H = WOUT_BLOCKS * 512;
  static constexpr int BLOCKS = WIN_BLOCKS + WOUT_BLOCKS;
  static constexpr int DMA_J = (BLOCKS + 3) / 4;              // copies per vector wave
  static constexpr int SLACK_H = 512;
  static constexpr int RING_H = 3 * WIN_H + 3 * WOUT_H + SLACK_H;
  static constexpr int HB_H = 2 * 4 * 2 * 64 * 8;             // [parity][slice][k-step][lane][8] FP16
  static constexpr int LDS_BYTES = RING_H * 2 + HB_H * 2 + kWideFfnMaxF * 2 + 3 * D * 4;
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
};

}  // namespace

template <int D, typename XT, typename OT>
__global__ __launch_bounds__(kRT) void ffn_roles_kernel(FfnArgs a) {
  using SH = RoleShape<D>;
  constexpr int KS = SH::KS, PT = SH::PT;
  static_assert(D % 64 == 0 && D <= 256, "shape");

  __shared__ __align__(16) _Float16 ring[SH::RING_H];
  __shared__ __align__(16) _Float16 hbx[SH::HB_H];
  __shared__ __align__(16) _Float16 bin[kWideFfnMaxF];  // b_in (FP16, as given)
  __shared__ float prm[3 * D];                           // b_out, gamma, beta (FP32)
  _Float16* const win_buf = ring;                        // 3 x WIN_H
  _Float16* const wout_buf = ring + 3 * SH::WIN_H;       // 3 x WOUT_H
  _Float16* const slack = wout_buf + 3 * SH::WOUT_H;

  const int F = a.f;
  const int C = F / 32;
  const int64_t M = a.m;
  const int64_t ntiles = (M + kTok - 1) / kTok;
  // Tile order: XCD x (workgroup b runs on XCD b % 8) owns the x-th eighth of the tiles and
  // walks it downwards.  The out-projection before it writes each eighth upwards on that XCD
  // (its persistent tiles), and the projection after it reads each eighth upwards, so each
  // kernel first reads what the one before wrote last, while it is still in the XCD's L2 and
  // the last-level cache.
  int64_t rs = 0, re = ntiles, slot = blockIdx.x, nsl = gridDim.x;
  if ((gridDim.x & 7) == 0) {
    const int x = blockIdx.x & 7;
    rs = ntiles * x / 8; re = ntiles * (x + 1) / 8; slot = blockIdx.x >> 3; nsl = gridDim.x >> 3;
  }
  if (slot >= re - rs) return;  // uniform per workgroup, before any barrier
  const int my_tiles = (int)((re - rs - 1 - slot) / nsl) + 1;
  auto tile_of = [&](int64_t t) -> int64_t { return re - 1 - (slot + t * nsl); };
  const int G = my_tiles * C;   // steps with a stage-1 product; G + 2 steps in all

  const int l = threadIdx.x & 63, wave = wave_id();
  const int li = l & 31, hh = l >> 5;
  const int sl = wave & 3;      // 32-token slice of the tile
  const int kr = kappa32(li);

  for (int i = threadIdx.x; i < F; i += kRT) bin[i] = a.b_in[i];
  for (int i = threadIdx.x; i < D; i += kRT) {
    prm[i] = (float)a.b_out[i];
    prm[D + i] = a.gamma[i];
    prm[2 * D + i] = a.beta[i];
  }
  using T = std::integral_constant<bool, true>;
  using Fa = std::integral_constant<bool, false>;

  if (wave >= 4) {
    // ============================ vector wave ============================
    // Copy slots: block sl + 4j of the chunk's W_in blocks then W_out blocks
    // (ffn_wide_kernel's padded layouts); surplus slots copy filler into the
    // slack buffer, filler lanes load element 0 of the chunk.
    uint32_t dma_off[SH::DMA_J], dst0[SH::DMA_J], dst_in[SH::DMA_J], dst_out[SH::DMA_J], from_out[SH::DMA_J];
    const uint32_t lds_win = (uint32_t)(uintptr_t)(lds_void*)win_buf;
    const uint32_t lds_wout = (uint32_t)(uintptr_t)(lds_void*)wout_buf;
    const uint32_t lds_slack = (uint32_t)(uintptr_t)(lds_void*)slack;
#pragma unroll
    for (int j = 0; j < SH::DMA_J; ++j) {
      const int slot = sl + 4 * j;
      const bool is_in = slot < SH::WIN_BLOCKS, is_out = !is_in && slot < SH::BLOCKS;
      uint32_t off = 0;
      if (is_in) {
        const int u = slot * 64 + l, row = u / (SH::LDI / 8), pos = u % (SH::LDI / 8);
        off = (row < 32 && pos < D / 8) ? (uint32_t)(row * D + 8 * pos) * 2u : 0u;
      } else if (is_out) {
        const int u = (slot - SH::WIN_BLOCKS) * 64 + l, row = u / (SH::LDO / 8), pos = u % (SH::LDO / 8);
        off = (row < D && pos < 4) ? (uint32_t)(row * F + 8 * pos) * 2u : 0u;
      }
      dma_off[j] = off;
      dst0[j] = is_in ? lds_win + (uint32_t)(slot * 1024)
                      : is_out ? lds_wout + (uint32_t)((slot - SH::WIN_BLOCKS) * 1024) : lds_slack;
      dst_in[j] = is_in ? (uint32_t)(SH::WIN_H * 2) : 0u;
      dst_out[j] = is_out ? (uint32_t)(SH::WOUT_H * 2) : 0u;
      from_out[j] = is_out ? 1u : 0u;
    }
    // W_in chunk ci -> W_in buffer bi, W_out chunk co -> W_out buffer bo
    auto issue = [&](int ci, int bi, int co, int bo) {
      const uint64_t src_in = (uint64_t)(uintptr_t)(a.w_in + (int64_t)(32 * ci) * D);
      const uint64_t src_out = (uint64_t)(uintptr_t)(a.w_out + 32 * co);
#pragma unroll
      for (int j = 0; j < SH::DMA_J; ++j) {
        const uint64_t src = src_in + (uint64_t)from_out[j] * (src_out - src_in);
        dma16(dma_off[j], (const void*)(uintptr_t)src, dst0[j] + (uint32_t)bi * dst_in[j] + (uint32_t)bo * dst_out[j]);
      }
    };

    const XT* __restrict__ X = static_cast<const XT*>(a.x);
    h8 xf[KS];  // X fragments of the slice's 32 tokens: d = 16 ks + 8 hh .. +7
    auto load_x = [&](int64_t t) {
      const int64_t row0 = t * kTok + 32 * sl;
      const uint32_t rows = (uint32_t)max<int64_t>(0, min<int64_t>(32, M - row0));
      const __amdgpu_buffer_rsrc_t xr = make_rsrc(X + row0 * D, rows * (uint32_t)(D * sizeof(XT)));
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        xf[ks] = buffer_load8_as_half(xr, (uint32_t)((li * D + 16 * ks + 8 * hh) * sizeof(XT)), X);
    };
    _Float16* const hb_lane = hbx + sl * (2 * 512) + 8 * l;  // + parity * 4096 + k-step * 512

    issue(0, 0, 0, 0);      // W_in chunk 0 -> buffer 0 (W_out chunk 0 is copied again at step 0)
    issue(1 % C, 1, 0, 0);  // W_in chunk 1 -> buffer 1
    load_x(tile_of(0));
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // Stream position: g, g % 3, the chunks of positions g (stage 1, W_out copy),
    // g - 1 (GELU) and g + 2 (W_in copy), and the tile of position g.
    int g = 0, g3 = 0, cg = 0, cm1 = C - 1, cp2 = 2 % C, tg = 0;
    auto advance = [&]() {
      ++g;
      g3 = g3 == 2 ? 0 : g3 + 1;
      cm1 = cg;
      cg = cg + 1 == C ? 0 : cg + 1;
      cp2 = cp2 + 1 == C ? 0 : cp2 + 1;
      if (cg == 0) ++tg;
    };
    // One step.  LAST (the tile's last chunk): all stage-1 MFMAs first, then the
    // next tile's X is requested and the GELU runs while it arrives; the step ends
    // waiting for every load, which also tells the compiler (it cannot see the
    // asm-issued copies) that nothing it tracks is in flight - otherwise its own
    // wait for the X fragments in the following steps would drain those steps'
    // fresh copies too.  S1 / GELU: whether the step has a stage-1 product / a GELU.
    auto step = [&](auto last_tag, auto s1_tag, auto gelu_tag, const f16v& hin, f16v& hout) {
      constexpr bool LAST = decltype(last_tag)::value;
      constexpr bool S1 = decltype(s1_tag)::value, GELU = decltype(gelu_tag)::value;
      const int g3p2 = g3 == 0 ? 2 : g3 - 1;
      issue(cp2, g3p2, cg, g3);
      float bias[16];
      if constexpr (GELU) {
        const _Float16* bp = bin + 32 * cm1 + 8 * hh;
        const h8 b0 = *reinterpret_cast<const h8*>(bp);
        const h8 b1 = *reinterpret_cast<const h8*>(bp + 16);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          bias[j] = (float)b0[j];
          bias[8 + j] = (float)b1[j];
        }
      }
      h8 hv0, hv1;
      auto gelu_one = [&](int e) {
        const _Float16 v = (_Float16)gelu_erf(hin[e] + bias[e]);
        if (e < 8) hv0[e] = v; else hv1[e - 8] = v;
      };
      if constexpr (S1) {
        const _Float16* wi = win_buf + g3 * SH::WIN_H + kr * SH::LDI + 8 * hh;
        constexpr int PF = 4;
        h8 fr[PF];
#pragma unroll
        for (int i = 0; i < PF; ++i) fr[i] = *reinterpret_cast<const h8*>(wi + 16 * i);
#pragma unroll
        for (int e = 0; e < 16; ++e) hout[e] = 0.f;
        if constexpr (LAST || !GELU) {
#pragma unroll
          for (int i = 0; i < KS; ++i) {
            const h8 w = fr[i % PF];
            if (i + PF < KS) fr[i % PF] = *reinterpret_cast<const h8*>(wi + 16 * (i + PF));
            hout = mfma32x32(w, xf[i], hout);
          }
          if constexpr (LAST) {
            if (tg + 1 < my_tiles) load_x(tile_of(tg + 1));
          }
          if constexpr (GELU) {
#pragma unroll
            for (int e = 0; e < 16; ++e) gelu_one(e);
          }
        } else {
          // segments of four MFMAs beside four GELU elements
          constexpr int SEG = KS / 4, EPS = 16 / SEG;
          static_assert(KS % 4 == 0 && EPS * SEG == 16, "segment split");
#pragma unroll
          for (int k = 0; k < SEG; ++k) {
#pragma unroll
            for (int i = 4 * k; i < 4 * k + 4; ++i) {
              const h8 w = fr[i % PF];
              if (i + PF < KS) fr[i % PF] = *reinterpret_cast<const h8*>(wi + 16 * (i + PF));
              hout = mfma32x32(w, xf[i], hout);
            }
#pragma unroll
            for (int e = EPS * k; e < EPS * (k + 1); ++e) gelu_one(e);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      } else if constexpr (GELU) {
#pragma unroll
        for (int e = 0; e < 16; ++e) gelu_one(e);
      }
      if constexpr (GELU) {
        _Float16* op = hb_lane + ((g - 1) & 1) * 4096;
        *reinterpret_cast<h8*>(op) = hv0;
        *reinterpret_cast<h8*>(op + 512) = hv1;
      }
      if constexpr (LAST && S1) wait_copies<0>();
      else wait_copies<SH::DMA_J>();  // this step's copies may stay in flight
      lds_barrier();
      advance();
    };
    // A step of the stream, LAST or not by its chunk.
    auto any_step = [&](auto s1_tag, auto gelu_tag, const f16v& hin, f16v& hout) {
      if (cg == C - 1) step(T{}, s1_tag, gelu_tag, hin, hout);
      else step(Fa{}, s1_tag, gelu_tag, hin, hout);
    };
    f16v ha, hb;  // stage-1 results of even / odd positions
    any_step(T{}, Fa{}, hb, ha);          // g = 0
#pragma unroll 1
    while (g + 1 < G) {                   // g odd, then g + 1 even
      any_step(T{}, T{}, ha, hb);
      any_step(T{}, T{}, hb, ha);
    }
    if (g < G) any_step(T{}, T{}, ha, hb);  // g = G - 1 when it is odd
    // g = G: the last GELU (of position G - 1), g = G + 1: nothing but the barrier
    if (g & 1) step(Fa{}, Fa{}, T{}, ha, hb);
    else step(Fa{}, Fa{}, T{}, hb, ha);
    step(Fa{}, Fa{}, Fa{}, ha, hb);
    wait_copies<0>();  // surplus copies issued near the end have landed
    return;
  }

  // ============================ matrix wave ============================
  f16v yacc[PT];
#pragma unroll
  for (int p = 0; p < PT; ++p)
#pragma unroll
    for (int e = 0; e < 16; ++e) yacc[p][e] = 0.f;
  __syncthreads();
  const _Float16* const hb_lane = hbx + sl * (2 * 512) + 8 * l;

  // stage 2 of position g - 2: W_out buffer (g - 2) % 3, GELU operands of parity
  // g % 2; all operand reads are issued before the first MFMA
  auto s2 = [&](int b3, int par) {
    constexpr int N = 2 * PT;
    const _Float16* wo = wout_buf + b3 * SH::WOUT_H + kr * SH::LDO + 8 * hh;
    const h8 hb0 = *reinterpret_cast<const h8*>(hb_lane + par * 4096);
    const h8 hb1 = *reinterpret_cast<const h8*>(hb_lane + par * 4096 + 512);
    h8 fr[N];
#pragma unroll
    for (int k = 0; k < N; ++k) fr[k] = *reinterpret_cast<const h8*>(wo + 32 * (k >> 1) * SH::LDO + 16 * (k & 1));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < N; ++i) yacc[i >> 1] = mfma32x32(fr[i], (i & 1) ? hb1 : hb0, yacc[i >> 1]);
  };

  // tile epilogue: + b_out + residual, two-pass LayerNorm over the row, stores.
  // vmcnt counts loads and stores in one in-order counter, so a residual load
  // issued after a store waits for that store too: every residual load is issued
  // before the first store (RUNS_IN_FLIGHT runs of 8 features at a time), and the
  // stores then drain while the next tile runs.  Offsets are a per-lane base plus
  // immediates (the base is laundered so that the compiler does not hoist 32
  // precomputed offsets into registers).
  auto epilogue = [&](int64_t t) {
    const int64_t row0 = t * kTok + 32 * sl;
    const uint32_t rows = (uint32_t)max<int64_t>(0, min<int64_t>(32, M - row0));
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.residual + row0 * D, rows * (uint32_t)(D * 4));
    // residual_out NULL: a zero-size resource drops the stores, which still issue (the
    // copy waits count them)
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.residual_out ? a.residual_out + row0 * D : nullptr,
                                                a.residual_out ? rows * (uint32_t)(D * 4) : 0u);
    const __amdgpu_buffer_rsrc_t no =
        make_rsrc(static_cast<OT*>(a.normalized_out) + row0 * D, rows * (uint32_t)(D * sizeof(OT)));
    const float* bo = prm;
    const float* gm = prm + D;
    const float* bt = prm + 2 * D;
    typedef float v4 __attribute__((ext_vector_type(4)));
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    constexpr int RUNS = 2 * PT;            // runs of 8 features: run i = (p, r) = (i / 2, i % 2)
    constexpr int RUNS_IN_FLIGHT = 8;
    uint32_t base4 = (uint32_t)((li * D + 8 * hh) * 4);
    uint32_t base_o = (uint32_t)((li * D + 8 * hh) * sizeof(OT));
    asm volatile("" : "+v"(base4), "+v"(base_o));
    v4 rv[RUNS_IN_FLIGHT][2];
    auto load_run = [&](int i) {
      const uint32_t off = base4 + (uint32_t)((32 * (i >> 1) + 16 * (i & 1)) * 4);
      rv[i % RUNS_IN_FLIGHT][0] = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(rr, off, 0, 0));
      rv[i % RUNS_IN_FLIGHT][1] = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(rr, off + 16, 0, 0));
    };
#pragma unroll
    for (int i = 0; i < RUNS_IN_FLIGHT; ++i) load_run(i);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < RUNS; ++i) {
      const int p = i >> 1, r = i & 1, n = 32 * p + 16 * r + 8 * hh;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float v = (yacc[p][8 * r + j] + bo[n + j]) + rv[i % RUNS_IN_FLIGHT][j >> 2][j & 3];
        yacc[p][8 * r + j] = v;
        sum += v;
      }
      if (i + RUNS_IN_FLIGHT < RUNS) load_run(i + RUNS_IN_FLIGHT);
    }
#pragma unroll
    for (int i = 0; i < RUNS; ++i) {
      const int p = i >> 1, r = i & 1;
      const uint32_t off = base4 + (uint32_t)((32 * p + 16 * r) * 4);
      const v4 v0 = {yacc[p][8 * r + 0], yacc[p][8 * r + 1], yacc[p][8 * r + 2], yacc[p][8 * r + 3]};
      const v4 v1 = {yacc[p][8 * r + 4], yacc[p][8 * r + 5], yacc[p][8 * r + 6], yacc[p][8 * r + 7]};
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v0), ro, off, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v1), ro, off + 16, 0, 0);
    }
    const float inv_d = 1.0f / (float)D;
    const float mean = sum_over_halves(sum) * inv_d;
    float sq = 0.f;
#pragma unroll
    for (int p = 0; p < PT; ++p)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float d0 = yacc[p][e] - mean;
        sq += d0 * d0;
      }
    const float rstd = rsqrtf(sum_over_halves(sq) * inv_d + a.eps);
#pragma unroll
    for (int p = 0; p < PT; ++p)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int n = 32 * p + 16 * r + 8 * hh;
        float o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = (yacc[p][8 * r + j] - mean) * rstd * gm[n + j] + bt[n + j];
        pin_f32x8(o);  // rounded to FP32, then to the output type (no fused FMA + conversion)
        buffer_store8(no, base_o + (uint32_t)((32 * p + 16 * r) * sizeof(OT)), o, static_cast<OT*>(a.normalized_out));
      }
#pragma unroll
    for (int p = 0; p < PT; ++p)
#pragma unroll
      for (int e = 0; e < 16; ++e) yacc[p][e] = 0.f;
  };

  // steps 0 and 1: no stage 2 yet
  lds_barrier();
  lds_barrier();
  int b3 = 0, c2 = 0;   // (g - 2) % 3 and the chunk of position g - 2
  int64_t t2 = 0;       // tile of position g - 2
  // Residual prefetch: over the PF_STEPS steps before a tile's last one, each matrix
  // wave copies its 32 token rows of the residual (1 KB each, one LDS-DMA copy per
  // row) into the slack LDS area, whose contents nobody reads: the rows are then in
  // the L2 when the epilogue loads them, and the HBM reads of every workgroup's
  // epilogue are spread over those steps instead of arriving at once.  The copies
  // are older than every load the compiler counts, so its vmcnt waits stay exact.
  constexpr int PF_STEPS = 8, PF_ROWS = 32 / PF_STEPS;
  const uint32_t pf_lane = ((uint32_t)l * 16u) % (uint32_t)(D * 4);  // inside the row for any D
  const uint32_t pf_sink = (uint32_t)(uintptr_t)(lds_void*)slack;
#pragma unroll 1
  for (int g = 2; g < G + 2; ++g) {
    s2(b3, g & 1);
    if (c2 >= C - 1 - PF_STEPS && c2 < C - 1) {
      const int64_t r0 = tile_of(t2) * kTok + 32 * sl + PF_ROWS * (c2 - (C - 1 - PF_STEPS));
#pragma unroll
      for (int i = 0; i < PF_ROWS; ++i)
        if (r0 + i < M) dma16(pf_lane, a.residual + (r0 + i) * D, pf_sink);
    }
    // the operand reads are done before the barrier: the next step's copies reuse
    // this W_out buffer
    __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));
    lds_barrier();
    if (c2 == C - 1) epilogue(tile_of(t2));
    b3 = b3 == 2 ? 0 : b3 + 1;
    if (++c2 == C) { c2 = 0; ++t2; }
  }
}

static int wide_cu_count() {
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

template <int D, typename XT, typename OT>
static hipError_t launch_wide(const FfnArgs& a, hipStream_t s) {
  const int64_t ntiles = (a.m + kTok - 1) / kTok;
  const int64_t grid = std::min<int64_t>(ntiles, wide_cu_count());
  hipLaunchKernelGGL((ffn_wide_kernel<D, XT, OT>), dim3((unsigned)grid), dim3(kNT), 0, s, a);
  return hipGetLastError();
}

template <int D, typename XT, typename OT>
static hipError_t launch_roles(const FfnArgs& a, hipStream_t s) {
  const int64_t ntiles = (a.m + kTok - 1) / kTok;
  const int64_t grid = std::min<int64_t>(ntiles, wide_cu_count());
  hipLaunchKernelGGL((ffn_roles_kernel<D, XT, OT>), dim3((unsigned)grid), dim3(kRT), 0, s, a);
  return hipGetLastError();
}

bool ffn_wide_supported(int d, int f) { return d == 256 && f >= 32 && f % 32 == 0 && f <= kWideFfnMaxF; }

hipError_t launch_ffn_roles(const FfnArgs& a, int d, int w_dtype, int x_dtype, int out_dtype, hipStream_t s) {
  if (w_dtype != kF16 || !ffn_wide_supported(d, a.f)) return (hipError_t)MPK_EUNSUPPORTED;
  const bool xf = x_dtype == kF32, of = out_dtype == kF32;
  if (xf) return of ? launch_roles<256, float, float>(a, s) : launch_roles<256, float, _Float16>(a, s);
  return of ? launch_roles<256, _Float16, float>(a, s) : launch_roles<256, _Float16, _Float16>(a, s);
}

// The one-wave kernel takes FP16 X only: with FP32 X its tile loads need more registers than
// the 32 x D accumulators leave, and it would spill.  FP32 X runs on variant 4.
hipError_t launch_ffn_wide(const FfnArgs& a, int d, int w_dtype, int x_dtype, int out_dtype, hipStream_t s) {
  if (w_dtype != kF16 || x_dtype != kF16 || !ffn_wide_supported(d, a.f)) return (hipError_t)MPK_EUNSUPPORTED;
  return out_dtype == kF32 ? launch_wide<256, _Float16, float>(a, s) : launch_wide<256, _Float16, _Float16>(a, s);
}

}  // namespace mpk
