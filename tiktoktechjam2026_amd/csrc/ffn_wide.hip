// Wide fused FFN + residual + LayerNorm (d_model 256) on v_mfma_f32_32x32x16_f16.
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

typedef __attribute__((address_space(3))) void lds_void;

// One 16-byte-per-lane LDS-DMA copy: lane l's 16 bytes at base + voff (base
// wave-uniform, voff per lane) land at LDS byte address lds_base + 16 l
// (lds_base wave-uniform, in M0).  Issued as inline assembly: the compiler does
// not track it, so it neither counts it in its own vmcnt waits nor drains every
// LDS read behind it (it cannot tell the copy's target buffer from the ones being
// read).  Its completion is awaited explicitly with wait_copies.
__device__ __forceinline__ void dma16(uint32_t voff, const void* base, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(base), "s"(lds_base));
}

// Wait until at most N of this wave's vector-memory operations are outstanding
// (they complete in issue order), and for all of its LDS operations.  gfx9
// s_waitcnt encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14.
template <int N>
__device__ __forceinline__ void wait_copies() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier after wait_copies (which has also drained this wave's LDS
// reads).  __syncthreads() would add a release fence, which waits for every
// outstanding load and LDS-DMA copy - including the chunk copies meant to stay in
// flight across it; the acquire fence keeps later LDS reads below the barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

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
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.residual_out + row0 * D, rows * (uint32_t)(D * 4));
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
        buffer_store8(no, (uint32_t)((li * D + n) * sizeof(OT)), o, static_cast<OT*>(a.normalized_out));
      }
  }
  wait_copies<0>();  // surplus chunk copies issued near the end have landed
}

// ---------------------------------------------------------------------------
// Paired-wave wide FFN (variant 4): two waves per SIMD.
//
// A workgroup of 8 waves owns 128 tokens; waves w and w + 4 form a pair that owns
// 32 of them (two 16-token MFMA tiles).  Per 32-feature hidden chunk, on
// v_mfma_f32_16x16x32_f16 in the transposed, paired layout (mpk_common.h):
//   stage 1  wave half hh computes the 16 hidden features f0 + pair_row(q, hh) of
//            its 32 tokens (D/32 k-steps x 2 token tiles), adds b_in and applies the
//            GELU: lane (r, g) of token tile t holds features f0 + 8g + 4hh + 0..3
//   exchange each wave writes its four FP16 values per lane to LDS and reads its
//            partner's, which completes the stage-2 B operand (features f0 + 8g ..
//            +7 of token 16t + r)
//   stage 2  wave half hh accumulates output features [D/2 hh, D/2 (hh + 1)) of its
//            32 tokens: Y^T += W_out[., f0 ..] fp16(H)^T (D/64 x 2 tiles x 2 token tiles)
// so a wave holds 32 x D/2 FP32 accumulators and its tokens' X fragments - about
// half the registers of the one-wave-per-SIMD kernel above - and the two waves of
// a SIMD interleave one's MFMAs with the other's GELU.  The epilogue adds b_out and
// the residual; the LayerNorm row sums of the two halves meet in LDS.
//
// Step g of the workgroup's chunk stream (which continues across its tiles) runs
// the stage-1 product and GELU of chunk g and the stage-2 product of chunk g - 1,
// whose other half the partner wrote to LDS during step g - 1.  Weight chunks are
// copied global -> LDS by DMA two steps ahead, in rings of three buffers (W_in
// chunk g read from buffer g % 3, W_out chunk g - 1 from (g - 1) % 3; step g
// copies W_in g + 2 and W_out g + 1), with one barrier per step.  Rows are padded
// by 16 bytes and stored in slot order (slot 16 tt + r of each 32-row block holds
// row pair_row(r, tt)), so the 16 lanes of a fragment read hit distinct banks; the
// DMA applies that order through its per-lane source offsets.
namespace {

constexpr int kPW = 8;              // waves per workgroup, two per SIMD
constexpr int kPT = 64 * kPW;       // threads
constexpr int kPTok = 128;          // tokens per tile: 4 wave pairs x 32

template <int D>
struct PairShape {
  static constexpr int KS = D / 32;                          // stage-1 k-steps
  static constexpr int PH = D / 64;                          // 32-feature output pairs per half
  static constexpr int LDI = D + 8;                          // W_in row stride (halves)
  static constexpr int LDO = 40;                             // W_out row stride (halves)
  static constexpr int WIN_UNITS = 32 * (LDI / 8);
  static constexpr int WOUT_UNITS = D * (LDO / 8);
  static constexpr int WIN_BLOCKS = (WIN_UNITS + 63) / 64;
  static constexpr int WOUT_BLOCKS = (WOUT_UNITS + 63) / 64;
  static constexpr int WIN_H = WIN_BLOCKS * 512;
  static constexpr int WOUT_H = WOUT_BLOCKS * 512;
  static constexpr int BLOCKS = WIN_BLOCKS + WOUT_BLOCKS;
  static constexpr int DMA_J = (BLOCKS + kPW - 1) / kPW;
  static constexpr int SLACK_H = 512;
  // H-half exchange: [step parity][pair][half][token tile][lane] x 4 halves
  static constexpr int XCH_H = 2 * 4 * 2 * 2 * 64 * 4;
  static constexpr int LDS_H = 3 * WIN_H + 3 * WOUT_H + SLACK_H + XCH_H;
};

// tile row held in LDS slot s (slot 16 tt + r of each 32-row block: row pair_row(r, tt))
__device__ __forceinline__ int slot_row(int s) { return (s & ~31) | pair_row(s & 15, (s >> 4) & 1); }

// LDS-DMA copy as dma16, with one wait state between the m0 write and the copy
__device__ __forceinline__ void dma16p(uint32_t voff, const void* base, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(base), "s"(lds_base));
}

// LDS writes done, workgroup barrier, later LDS reads below it (vector-memory
// operations may stay in flight)
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));
  lds_barrier();
}

// 8 X values as FP16 from a buffer at lane offset voff + scalar offset soff
__device__ __forceinline__ h8 load8_half_so(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, const _Float16*) {
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  const u4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return __builtin_bit_cast(h8, v);
}

__device__ __forceinline__ h8 load8_half_so(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, const float*) {
  typedef float v4 __attribute__((ext_vector_type(4)));
  const v4 a = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
  const v4 b = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, soff, 0));
  h8 h;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = (_Float16)a[j];
    h[4 + j] = (_Float16)b[j];
  }
  return h;
}

// 8 FP32 values stored as OT at byte offset voff.  Stores keep the scalar offset at
// zero: with a register there, the compiler leaves out the wait state the hardware
// needs between a 128-bit store and a VALU write of its data registers, and the
// store then picked up the new value in some lanes.
__device__ __forceinline__ void store8_at(__amdgpu_buffer_rsrc_t r, uint32_t voff, const float* v, _Float16*) {
  h8 h;
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = (_Float16)v[j];
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, h), r, voff, 0, 0);
}

__device__ __forceinline__ void store8_at(__amdgpu_buffer_rsrc_t r, uint32_t voff, const float* v, float*) {
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  typedef float v4 __attribute__((ext_vector_type(4)));
  const v4 a = {v[0], v[1], v[2], v[3]};
  const v4 b = {v[4], v[5], v[6], v[7]};
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, a), r, voff, 0, 0);
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, b), r, voff + 16, 0, 0);
}

// Chunk-stream position: g % 3 and the chunk ids of step g's S1 (g), S2 (g - 1) and
// copies (W_in g + 2, W_out g + 1), all mod C
struct PRing {
  int g3, s1, s2, in_c, out_c;
  __device__ void advance(int nchunks) {
    g3 = g3 == 2 ? 0 : g3 + 1;
    s1 = s1 + 1 == nchunks ? 0 : s1 + 1;
    s2 = s2 + 1 == nchunks ? 0 : s2 + 1;
    in_c = in_c + 1 == nchunks ? 0 : in_c + 1;
    out_c = out_c + 1 == nchunks ? 0 : out_c + 1;
  }
};

}  // namespace

template <int D, typename XT, typename OT>
__global__ __launch_bounds__(kPT) void ffn_pair_kernel(FfnArgs a) {
  using SH = PairShape<D>;
  constexpr int KS = SH::KS, PH = SH::PH;
  static_assert(D % 64 == 0 && D <= 256, "shape");

  __shared__ __align__(16) _Float16 lds[SH::LDS_H];
  __shared__ _Float16 bin[kWideFfnMaxF];   // b_in (FP16, as given)
  __shared__ float prm[3 * D];             // b_out, gamma, beta (FP32)
  __shared__ float red[2][4][2][2][16];    // LayerNorm half-row sums: [pass][pair][half][token tile][row]
  _Float16* const win_buf = lds;                    // 3 x WIN_H
  _Float16* const wout_buf = lds + 3 * SH::WIN_H;   // 3 x WOUT_H
  _Float16* const slack = wout_buf + 3 * SH::WOUT_H;
  _Float16* const xbuf = slack + SH::SLACK_H;       // XCH_H

  const XT* __restrict__ X = static_cast<const XT*>(a.x);
  const int F = a.f;
  const int C = F / 32;
  const int64_t M = a.m;
  const int64_t ntiles = (M + kPTok - 1) / kPTok;
  int64_t tile = blockIdx.x;
  if (tile >= ntiles) return;  // uniform per workgroup, before any barrier
  const int my_tiles = (int)((ntiles - 1 - tile) / gridDim.x) + 1;

  const int l = threadIdx.x & 63, wave = wave_id();
  const int r = l & 15, g = l >> 4;
  const int pi = wave & 3, hh = wave >> 2;  // token pair (32 tokens), half (16 chunk features, D/2 outputs)

  // ---- DMA slots (as in ffn_wide_kernel, with the slot order applied to the source rows) ----
  uint32_t dma_off[SH::DMA_J];
#pragma unroll
  for (int j = 0; j < SH::DMA_J; ++j) {
    const int slot = j * kPW + wave;
    uint32_t off = 0;
    if (slot < SH::WIN_BLOCKS) {
      const int u = slot * 64 + l, srow = u / (SH::LDI / 8), pos = u % (SH::LDI / 8);
      off = (srow < 32 && pos < D / 8) ? (uint32_t)(slot_row(srow) * D + 8 * pos) * 2u : 0u;
    } else if (slot < SH::BLOCKS) {
      const int u = (slot - SH::WIN_BLOCKS) * 64 + l, srow = u / (SH::LDO / 8), pos = u % (SH::LDO / 8);
      off = (srow < D && pos < 4) ? (uint32_t)(slot_row(srow) * F + 8 * pos) * 2u : 0u;
    }
    dma_off[j] = off;
  }
  const uint32_t lds_win = (uint32_t)(uintptr_t)(lds_void*)win_buf;
  const uint32_t lds_wout = (uint32_t)(uintptr_t)(lds_void*)wout_buf;
  const uint32_t lds_slack = (uint32_t)(uintptr_t)(lds_void*)slack;
  uint32_t dst0[SH::DMA_J], dst_in[SH::DMA_J], dst_out[SH::DMA_J], from_out[SH::DMA_J];
#pragma unroll
  for (int j = 0; j < SH::DMA_J; ++j) {
    const int slot = j * kPW + wave;
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
      dma16p(dma_off[j], (const void*)(uintptr_t)src, dst0[j] + (uint32_t)bi * dst_in[j] + (uint32_t)bo * dst_out[j]);
    }
  };

  // X fragments of the pair's 32 tokens (stage-1 B operands): token 16 t + r, d = 32 ks + 8 g .. +7;
  // load_x issues kXLoads vector loads (one 16-byte load per FP16 fragment, two per FP32)
  h8 xf[2][KS];
  constexpr int kXLoads = 2 * KS * (int)(sizeof(XT) / 2);
  static_assert(kXLoads < 64, "vmcnt range");
  // Addresses: one lane offset, the token tile in the scalar offset and the k-step in
  // the instruction's immediate, so no per-fragment offset registers stay live.
  const uint32_t x_lane = (uint32_t)((r * D + 8 * g) * sizeof(XT));
  auto load_x = [&](int64_t t_) {
    const int64_t row0 = t_ * kPTok + 32 * pi;
    const uint32_t rows = (uint32_t)max<int64_t>(0, min<int64_t>(32, M - row0));
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(X + row0 * D, rows * (uint32_t)(D * sizeof(XT)));
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        xf[t][ks] = load8_half_so(xr, x_lane + (uint32_t)(32 * ks * sizeof(XT)), (uint32_t)(16 * t * D * sizeof(XT)), X);
  };

  f4 yacc[2][PH][2];  // Y^T of the tile: token tile t, output pair PH hh + p, MFMA tile tt
  h4 own[2];          // this wave's FP16 GELU half of the last chunk, per token tile
  // Lane offsets (halves) into the LDS buffers: W_in and W_out fragment rows, this
  // wave's and the partner's H-half slots (+ parity * (XCH_H / 2) + t * 256), b_in.
  int wi_lane = (16 * hh + r) * SH::LDI + 8 * g;
  int wo_lane = (32 * PH * hh + r) * SH::LDO + 8 * g;
  int xm_lane = (((pi * 2 + hh) * 2) * 64 + l) * 4;
  int xp_lane = (((pi * 2 + (1 - hh)) * 2) * 64 + l) * 4;
  int bi_lane = 8 * g + 4 * hh;

  // One step of the chunk stream.  S2: the stage-2 product of chunk rg.s2 (needs the
  // partner's half, written last step); S1: the stage-1 product and GELU of chunk
  // rg.s1.  Kind bit 0 (last chunk of a tile): the next tile's X is requested right
  // after the stage-1 product, its last use of the current X.  Kind bit 1 (first chunk
  // of a tile): the stage-1 product runs before the step's copies are issued, so the
  // compiler's wait for the X loads (which cannot see the copies, issued by inline
  // asm) covers only those loads.  A last-chunk step ends with the X loads the only
  // vector-memory operations left in flight: everything issued before them - this
  // step's and the previous step's copies - has landed.
  auto step = [&](auto s2_tag, auto kind_tag, const PRing& rg, int gpar, int64_t next_tile) {
    constexpr bool S2 = decltype(s2_tag)::value;
    constexpr int KIND = decltype(kind_tag)::value;
    constexpr bool LAST = (KIND & 1) != 0, FIRST = (KIND & 2) != 0;
    const int g3p1 = rg.g3 == 2 ? 0 : rg.g3 + 1, g3p2 = rg.g3 == 0 ? 2 : rg.g3 - 1;  // (g + 1) % 3, (g + 2) % 3
    if constexpr (!FIRST) issue(rg.in_c, g3p2, rg.out_c, g3p1);
    // stage 1: 16 hidden features x 32 tokens
    f4 hacc[2] = {zero4(), zero4()};
    {
      const _Float16* wi = win_buf + rg.g3 * SH::WIN_H + wi_lane;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const h8 w = *reinterpret_cast<const h8*>(wi + 32 * ks);
        hacc[0] = mfma32(w, xf[0][ks], hacc[0]);
        hacc[1] = mfma32(w, xf[1][ks], hacc[1]);
      }
    }
    if constexpr (LAST) {
      if (next_tile >= 0) load_x(next_tile);
    }
    if constexpr (FIRST) issue(rg.in_c, g3p2, rg.out_c, g3p1);
    float bias[4];
    {
      const _Float16* bp = bin + 32 * rg.s1 + bi_lane;
#pragma unroll
      for (int i = 0; i < 4; ++i) bias[i] = (float)bp[i];
    }
    if constexpr (S2) {
      // stage 2 of the previous chunk: output features [D/2 hh, D/2 (hh + 1)) x 32 tokens
      h8 hb[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const h4 other = *reinterpret_cast<const h4*>(xbuf + xp_lane + (gpar ^ 1) * (SH::XCH_H / 2) + t * 256);
        const h4 lo = hh == 0 ? own[t] : other, hi = hh == 0 ? other : own[t];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          hb[t][i] = lo[i];
          hb[t][4 + i] = hi[i];
        }
      }
      const _Float16* wo = wout_buf + g3p2 * SH::WOUT_H + wo_lane;  // (g - 1) % 3 == (g + 2) % 3
#pragma unroll
      for (int p = 0; p < PH; ++p)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const h8 w = *reinterpret_cast<const h8*>(wo + (32 * p + 16 * tt) * SH::LDO);
          yacc[0][p][tt] = mfma32(w, hb[0], yacc[0][p][tt]);
          yacc[1][p][tt] = mfma32(w, hb[1], yacc[1][p][tt]);
        }
    }
    // GELU of this chunk's half, handed to the partner
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) own[t][i] = (_Float16)gelu_erf(hacc[t][i] + bias[i]);
      *reinterpret_cast<h4*>(xbuf + xm_lane + gpar * (SH::XCH_H / 2) + t * 256) = own[t];
    }
    if constexpr (LAST && !FIRST) {
      if (next_tile >= 0) wait_copies<kXLoads>();
      else wait_copies<SH::DMA_J>();
    } else {
      wait_copies<SH::DMA_J>();
    }
    lds_barrier();
  };

  // ---- epilogue of a tile: + b_out + residual, LayerNorm over the row, stores ----
  auto epilogue = [&](int64_t etile) {
    const int64_t row0 = etile * kPTok + 32 * pi;
    const uint32_t rows = (uint32_t)max<int64_t>(0, min<int64_t>(32, M - row0));
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.residual + row0 * D, rows * (uint32_t)(D * 4));
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.residual_out + row0 * D, rows * (uint32_t)(D * 4));
    const __amdgpu_buffer_rsrc_t no =
        make_rsrc(static_cast<OT*>(a.normalized_out) + row0 * D, rows * (uint32_t)(D * sizeof(OT)));
    typedef float v4 __attribute__((ext_vector_type(4)));
    // FP32 element offset of (token r, feature 32 PH hh + 8 g) in bytes; token tile t and
    // feature pair p go to the scalar and immediate offsets
    const uint32_t e_lane = (uint32_t)((r * D + 32 * PH * hh + 8 * g) * 4);
    // b_out, gamma and beta are read from LDS here, where they are used: an opaque
    // offset keeps the compiler from hoisting the loop-invariant reads out of the
    // tile loop, where their 96 registers per lane would force spills
    int pofs = 0;
    asm volatile("" : "+v"(pofs));
    const float* const pb = prm + pofs;
    float sum[2] = {0.f, 0.f};
    // one token tile at a time: the X fragments of the next tile and the accumulators
    // are live here, and all the residual loads at once would not fit beside them
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int p = 0; p < PH; ++p) {
        const int n = 32 * (PH * hh + p) + 8 * g;
        const uint32_t off = e_lane + (uint32_t)(128 * p), soff = (uint32_t)(16 * t * D * 4);
        const v4 r0 = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(rr, off, soff, 0));
        const v4 r1 = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(rr, off + 16, soff, 0));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v0 = (yacc[t][p][0][i] + pb[n + i]) + r0[i];
          const float v1 = (yacc[t][p][1][i] + pb[n + 4 + i]) + r1[i];
          yacc[t][p][0][i] = v0;
          yacc[t][p][1][i] = v1;
          sum[t] += v0 + v1;
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    const float inv_d = 1.0f / (float)D;
    float mean[2], rstd[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float s = sum_over_groups(sum[t]);
      if (g == 0) red[0][pi][hh][t][r] = s;
    }
    lds_sync();
#pragma unroll
    for (int t = 0; t < 2; ++t) mean[t] = (red[0][pi][0][t][r] + red[0][pi][1][t][r]) * inv_d;
    float sq[2] = {0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int p = 0; p < PH; ++p)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float c0 = yacc[t][p][tt][i] - mean[t];
            sq[t] += c0 * c0;
          }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float s = sum_over_groups(sq[t]);
      if (g == 0) red[1][pi][hh][t][r] = s;
    }
    lds_sync();
#pragma unroll
    for (int t = 0; t < 2; ++t) rstd[t] = rsqrtf((red[1][pi][0][t][r] + red[1][pi][1][t][r]) * inv_d + a.eps);
    const float* gm = pb + D;
    const float* bt = pb + 2 * D;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int p = 0; p < PH; ++p) {
        const int n = 32 * (PH * hh + p) + 8 * g;
        float v[8], o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          v[j] = yacc[t][p][j >> 2][j & 3];
          o[j] = (v[j] - mean[t]) * rstd[t] * gm[n + j] + bt[n + j];
        }
        store8_at(ro, e_lane + (uint32_t)((16 * t * D + 32 * p) * 4), v, a.residual_out);
        store8_at(no, (e_lane / 4 + (uint32_t)(16 * t * D + 32 * p)) * (uint32_t)sizeof(OT), o,
                  static_cast<OT*>(a.normalized_out));
      }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int p = 0; p < PH; ++p) yacc[t][p][0] = yacc[t][p][1] = zero4();
    // Drain the stores (and spill traffic) here, once per tile: left in flight, the
    // compiler's own waits for them inside the steady steps - it cannot see the
    // asm-issued copies - would also wait for each step's fresh copies.
    wait_copies<0>();
  };

  using T = std::integral_constant<bool, true>;
  using Fa = std::integral_constant<bool, false>;

  // ---- prologue: parameters, W_in chunks 0 and 1, W_out chunk 0, the first X tile ----
  for (int i = threadIdx.x; i < F; i += kPT) bin[i] = a.b_in[i];
  for (int i = threadIdx.x; i < D; i += kPT) {
    prm[i] = (float)a.b_out[i];
    prm[D + i] = a.gamma[i];
    prm[2 * D + i] = a.beta[i];
  }
  issue(0, 0, 0, 0);       // W_in 0 -> buffer 0, W_out 0 -> buffer 0
  issue(1 % C, 1, 0, 0);   // W_in 1 -> buffer 1 (W_out 0 again: same data)
  load_x(tile);
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int p = 0; p < PH; ++p) yacc[t][p][0] = yacc[t][p][1] = zero4();
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  PRing rg{0, 0, C - 1, 2 % C, 1 % C};
  int gpar = 0;
  using K0 = std::integral_constant<int, 0>;  // steady
  using K1 = std::integral_constant<int, 1>;  // last chunk of a tile
  using K2 = std::integral_constant<int, 2>;  // first chunk of a tile
  using K3 = std::integral_constant<int, 3>;  // the only chunk
  // the tile after the current one, or -1
  auto next_of = [&](int it_) -> int64_t { return it_ + 1 < my_tiles ? tile + gridDim.x : -1; };
  // chunk 0 of the first tile (no stage 2 before it)
  if (C == 1) step(Fa{}, K3{}, rg, gpar, next_of(0));
  else step(Fa{}, K2{}, rg, gpar, -1);
  rg.advance(C);
  gpar ^= 1;
  for (int it = 0;;) {
    if (C > 1) {
      const int64_t next = next_of(it);
      // The copy and LDS lane offsets may have been spilled around the epilogue; pin them
      // here so a reload (and the compiler's wait for it) lands before the steady loop,
      // not in it.
#pragma unroll
      for (int j = 0; j < SH::DMA_J; ++j) asm volatile("" : "+v"(dma_off[j]));
      asm volatile("" : "+v"(wi_lane), "+v"(wo_lane), "+v"(xm_lane), "+v"(xp_lane), "+v"(bi_lane));
#pragma unroll 1
      for (int c = 1; c < C - 1; ++c) {
        step(T{}, K0{}, rg, gpar, next);
        rg.advance(C);
        gpar ^= 1;
      }
      step(T{}, K1{}, rg, gpar, next);
      rg.advance(C);
      gpar ^= 1;
    }
    if (++it == my_tiles) break;
    tile += gridDim.x;
    // chunk 0 of the next tile: its step finishes the previous tile's stage 2, whose
    // epilogue follows
    if (C == 1) step(T{}, K3{}, rg, gpar, next_of(it));
    else step(T{}, K2{}, rg, gpar, -1);
    rg.advance(C);
    gpar ^= 1;
    epilogue(tile - gridDim.x);
  }
  // the last tile's last stage 2, no stage 1 (step with S1 on a dead chunk would be
  // wasted: run only S2 by hand)
  {
    const int g3p2 = rg.g3 == 0 ? 2 : rg.g3 - 1;
    h8 hb[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const h4 other = *reinterpret_cast<const h4*>(xbuf + xp_lane + (gpar ^ 1) * (SH::XCH_H / 2) + t * 256);
      const h4 lo = hh == 0 ? own[t] : other, hi = hh == 0 ? other : own[t];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        hb[t][i] = lo[i];
        hb[t][4 + i] = hi[i];
      }
    }
    const _Float16* wo = wout_buf + g3p2 * SH::WOUT_H + wo_lane;
#pragma unroll
    for (int p = 0; p < PH; ++p)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const h8 w = *reinterpret_cast<const h8*>(wo + (32 * p + 16 * tt) * SH::LDO);
        yacc[0][p][tt] = mfma32(w, hb[0], yacc[0][p][tt]);
        yacc[1][p][tt] = mfma32(w, hb[1], yacc[1][p][tt]);
      }
  }
  epilogue(tile);
  wait_copies<0>();  // copies issued near the end have landed before the workgroup ends
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
static hipError_t launch_pair(const FfnArgs& a, hipStream_t s) {
  const int64_t ntiles = (a.m + kPTok - 1) / kPTok;
  const int64_t grid = std::min<int64_t>(ntiles, wide_cu_count());
  hipLaunchKernelGGL((ffn_pair_kernel<D, XT, OT>), dim3((unsigned)grid), dim3(kPT), 0, s, a);
  return hipGetLastError();
}

bool ffn_wide_supported(int d, int f) { return d == 256 && f >= 32 && f % 32 == 0 && f <= kWideFfnMaxF; }

hipError_t launch_ffn_pair(const FfnArgs& a, int d, int w_dtype, int x_dtype, int out_dtype, hipStream_t s) {
  if (w_dtype != kF16 || !ffn_wide_supported(d, a.f)) return (hipError_t)MPK_EUNSUPPORTED;
  const bool xf = x_dtype == kF32, of = out_dtype == kF32;
  if (xf) return of ? launch_pair<256, float, float>(a, s) : launch_pair<256, float, _Float16>(a, s);
  return of ? launch_pair<256, _Float16, float>(a, s) : launch_pair<256, _Float16, _Float16>(a, s);
}

hipError_t launch_ffn_wide(const FfnArgs& a, int d, int w_dtype, int x_dtype, int out_dtype, hipStream_t s) {
  if (w_dtype != kF16 || !ffn_wide_supported(d, a.f)) return (hipError_t)MPK_EUNSUPPORTED;
  const bool xf = x_dtype == kF32, of = out_dtype == kF32;
  if (xf) return of ? launch_wide<256, float, float>(a, s) : launch_wide<256, float, _Float16>(a, s);
  return of ? launch_wide<256, _Float16, float>(a, s) : launch_wide<256, _Float16, _Float16>(a, s);
}

}  // namespace mpk
