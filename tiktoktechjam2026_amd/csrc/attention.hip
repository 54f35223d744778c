// Causal flash attention for gfx950: FP16 MFMA for Q K^T and P V, FP32 online
// softmax statistics and FP32 output accumulation, causal tile skipping.
//
// Replaces the reference's Triton kernels
//   _causal_attention_fp16_fwd  custom_kernel/triton_attention.py:126-232  (FP16 I/O)
//   _causal_attention_fwd       custom_kernel/triton_attention.py:16-123   (FP32 I/O)
// Math per query row (same rounding points as the FP16 reference kernel):
//   s_j*c = (q*c) . k_j  (FP16 operands: q*c split into hi + lo; FP32 accumulate)
//   m   = running max of s*c (FP32, raised lazily);  p_j = 2^(s_j*c - m), c = scale*log2(e)
//   acc += fp16(p_j) * v_j  and  l += fp16(p_j)  (both by the PV MFMA, FP32 accumulate)
//   o   = acc / l, rounded to the output type.
// l sums the same FP16-rounded probabilities that weight V (the reference sums the
// unrounded FP32 p_j); the two sums differ by at most 2^-12 relative (half an FP16
// ulp of o), and this way the weights applied to V sum to exactly one.
// For FP32 inputs (the reference's TF32 kernel) q, k and v are scaled by powers of
// two into FP16's range and then rounded to FP16, which keeps TF32's 10-bit operand
// mantissa and, through the scales, FP32's exponent range (see f32_scale_exp).
//
// Structure.  A workgroup of NW waves owns QB = 16*QT*NW queries of one
// (batch, head); each wave owns 16*QT queries.  Key/value tiles of KTILE rows
// are staged through double-buffered LDS (K row-major, V transposed as key
// pairs) with a one-tile register prefetch and ONE barrier per tile.  Each wave
// computes S^T = K Q^T with the paired row mapping (mpk_common.h), so a lane
// holds one query and 8 consecutive keys per 32-key pair: the row max needs two
// cross-lane swaps, and fp16(P) is already laid out as the B operand of
// O^T = V^T P^T.  Key tiles strictly above a wave's queries are skipped; only
// tiles that straddle the diagonal (or the sequence end, or carry a key mask)
// pay for masking.  Query blocks are issued longest first, and each XCD owns a
// contiguous range of (batch, head) rows so they share K/V through its L2.
#include <type_traits>

#include "mpk_common.h"

namespace mpk {

// (kRescaleLog2, the lazy-raise threshold of the running max, is in mpk_common.h)
constexpr float kRescaleWeight = 256.0f;  // 2^kRescaleLog2: a weight 2^(s*c - m) above it calls for a raise

// FP32 inputs.  FP16 holds magnitudes of about 6e-5 .. 65504 only, where TF32 (the
// reference's FP32 kernel) keeps FP32's exponent range.  Attention is exactly
// invariant under power-of-two scalings: with q' = q 2^-a (per query row),
// k' = k 2^-b and v' = v 2^-e (per workgroup, over the keys it reads),
//   s c = (q' . k') (c 2^(a + b))   and   o = (sum_j p_j v'_j / l) 2^e,
// so the kernels round q', k', v' to FP16 (the same 11-bit significand as before,
// and no overflow for any finite input), multiply the raw product by the per-row factor c 2^(a + b) in the
// FP32 FMA that also subtracts the running max, and scale the output by 2^e.
// Each exponent puts the largest magnitude it covers in [2^13, 2^14): values down to
// 2^-27 of it keep FP16's full precision, smaller ones lose bits (subnormal) and
// those below 2^-38 of it become zero - contributions far below the FP32 rounding
// of the largest terms of a dot product over at most 256 dims.
constexpr int kF16TopExp = 13;
__device__ __forceinline__ int f32_scale_exp(float amax) {
  if (!(amax > 0.f) || !(amax < INFINITY)) return 0;  // all zero (or non-finite): unscaled
  int e;
  (void)frexpf(amax, &e);  // amax = f 2^e, f in [0.5, 1)
  return e - 1 - kF16TopExp;
}

// 8 consecutive FP32 values through a buffer resource, times 2^-sexp, rounded to FP16
__device__ __forceinline__ h8 buffer_load8_scaled(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, int sexp) {
  typedef float v4 __attribute__((ext_vector_type(4)));
  const v4 a = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
  const v4 b = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off + 16, 0, 0));
  h8 h;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = (_Float16)ldexpf(a[j], -sexp);
    h[4 + j] = (_Float16)ldexpf(b[j], -sexp);
  }
  return h;
}

// Largest |x| over rows [0, rows) x cols (cols % 8 == 0) of an FP32 matrix, reduced over
// the workgroup (NT threads; red: NT / 64 floats of LDS).  Every thread must call it.
template <int NT>
__device__ float wg_absmax(const float* base, int64_t row_stride, int rows, int cols, float* red) {
  float m = 0.f;
  const int cpr = cols / 8;
  for (int c = threadIdx.x; c < rows * cpr; c += NT) {
    const float* p = base + (int64_t)(c / cpr) * row_stride + (c % cpr) * 8;
    const float4 x0 = *reinterpret_cast<const float4*>(p);
    const float4 x1 = *reinterpret_cast<const float4*>(p + 4);
    m = fmaxf(m, fmaxf(fmaxf(fabsf(x0.x), fabsf(x0.y)), fmaxf(fabsf(x0.z), fabsf(x0.w))));
    m = fmaxf(m, fmaxf(fmaxf(fabsf(x1.x), fabsf(x1.y)), fmaxf(fabsf(x1.z), fabsf(x1.w))));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) r = fmaxf(r, red[w]);
  __syncthreads();  // red is reused by the next call
  return r;
}

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t qs[4], ks[4], vs[4], os[4];  // element strides: batch, head, seq, dim
  const uint8_t* key_valid;           // optional [B, S] (row stride S), nonzero = valid key
  int batch, heads, seq, causal;
  float c;      // scale * log2(e)
  int group;    // > 0: the 32x32 kernel schedules (batch, head) rows in groups of this many per XCD
};

template <int HD, int KTILE, int NT>
struct AttnShape {
  // HP: the head dim the MFMA tiles see.  hd = 8 runs on the hd = 16 tiles with
  // dims 8..15 of K zero (Q's are zero too) and V^T rows 8..15 never stored.
  static constexpr int HP = HD < 16 ? 16 : HD;
  static constexpr int LDK = HP + 8;      // K tile row stride (halves)
  static constexpr int LDV = KTILE + 8;   // V^T tile row stride (halves)
  static constexpr int CPK = HD / 8;      // 8-element chunks per key row
  static constexpr int CHUNKS = KTILE * CPK;                     // K tile: one 16-byte chunk per item
  static constexpr int PER_THREAD = (CHUNKS + NT - 1) / NT;
  static constexpr int VITEMS = (KTILE / 2) * CPK;               // V tile: a key pair x one chunk per item
  static constexpr int V_PER_THREAD = (VITEMS + NT - 1) / NT;
  static constexpr int DT = HP >= 32 ? HP / 32 : 1;  // output d tiles (pairs of 16, or one tile of 16)
  static constexpr int NP = KTILE / 32;              // key pairs per tile
  static constexpr int KBUF = KTILE * LDK;
  static constexpr int VBUF = HP * LDV;
};

template <int HD, int QT, int KTILE, int NW, typename IT, typename OT, bool KEYMASK>
__global__ __launch_bounds__(64 * NW) void attention_kernel(AttnArgs a) {
  constexpr int NT = 64 * NW;
  using SH = AttnShape<HD, KTILE, NT>;
  constexpr int QB = 16 * QT * NW;
  constexpr int NP = SH::NP;
  constexpr int HP = SH::HP;
  static_assert(HD == 8 || HD == 16 || HD == 32 || HD == 64 || HD == 128 || HD == 256, "head dim");
  static_assert(KTILE % 32 == 0 && KTILE <= NT, "key tile");

  __shared__ _Float16 ks_lds[2][SH::KBUF];
  __shared__ _Float16 vt_lds[2][SH::VBUF];
  __shared__ float kbias[2][KTILE];

  const int S = a.seq;
  const int BH = a.batch * a.heads;
  const int nqb = (S + QB - 1) / QB;
  // Workgroups are dispatched round-robin over the 8 XCDs.  Each XCD gets a
  // contiguous range of (batch, head) rows - neighbouring heads share 128-byte
  // lines of the packed QKV rows - and walks its range longest query block
  // first, so the blocks of one row run close together on one L2.
  int bh, qblock;
  if ((BH & 7) == 0) {
    const int per_xcd = BH >> 3;
    const int slot = blockIdx.x >> 3;
    bh = (blockIdx.x & 7) * per_xcd + slot % per_xcd;
    qblock = nqb - 1 - slot / per_xcd;
  } else {
    bh = blockIdx.x % BH;
    qblock = nqb - 1 - (int)(blockIdx.x / BH);
  }
  const int b = bh / a.heads, h = bh % a.heads;
  const int q0 = qblock * QB;

  const IT* __restrict__ Q = static_cast<const IT*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const IT* __restrict__ Kp = static_cast<const IT*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const IT* __restrict__ Vp = static_cast<const IT*>(a.v) + b * a.vs[0] + h * a.vs[1];
  OT* __restrict__ O = static_cast<OT*>(a.o) + b * a.os[0] + h * a.os[1];
  const uint8_t* kv_valid = KEYMASK ? a.key_valid + (int64_t)b * S : nullptr;

  const int l = threadIdx.x & 63, wave = wave_id();
  const int r = l & 15, g = l >> 4;
  const int qw0 = q0 + wave * 16 * QT;       // first query of this wave
  const int qw_last = qw0 + 16 * QT - 1;     // last query of this wave

  const int kv_end = a.causal ? min(q0 + QB, S) : S;  // keys [0, kv_end) can matter
  const int ntiles = (kv_end + KTILE - 1) / KTILE;

  // FP32 inputs: power-of-two exponents for K and V over the keys this workgroup reads
  // (see f32_scale_exp); FP16 inputs are used as they are.
  constexpr bool F32IN = std::is_same<IT, float>::value;
  int kexp = 0, vexp = 0;
  if constexpr (F32IN) {
    __shared__ float red[NW];
    kexp = __builtin_amdgcn_readfirstlane(
        f32_scale_exp(wg_absmax<NT>(reinterpret_cast<const float*>(Kp), a.ks[2], kv_end, HD, red)));
    vexp = __builtin_amdgcn_readfirstlane(
        f32_scale_exp(wg_absmax<NT>(reinterpret_cast<const float*>(Vp), a.vs[2], kv_end, HD, red)));
  }

  // ---- Q fragments (B operand of S^T = K Q^T), kept in registers ----
  // FP16 inputs: q is pre-multiplied by c = scale*log2(e) in FP32 and split into FP16
  // hi + lo (hi + lo = q*c to ~2^-22 relative), so two MFMAs give s*c - m directly in
  // the FP32 accumulator (which starts at -m): no per-score scaling FMA, and the
  // exponent argument is more accurate than rounding s*c separately.
  // FP32 inputs: q' = fp16(q 2^-a) per query row (hi only, exact), and the raw product
  // becomes s*c - m in one FMA with the row's factor ceff = c 2^(a + kexp).
  constexpr int QK_STEPS = HP >= 32 ? HP / 32 : 1;
  h8 qh[QT][QK_STEPS], ql[QT][QK_STEPS];
  h4 qh16[QT], ql16[QT];
  float ceff[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int q = qw0 + 16 * t + r;
    ceff[t] = a.c;
    if constexpr (F32IN) {
      // lane (r, g) holds dims 4g .. 4g+3 (HP 16) or kq*32 + 8g .. +7 of query row q
      float raw[QK_STEPS][8];
      float mx = 0.f;
#pragma unroll
      for (int kq = 0; kq < QK_STEPS; ++kq)
#pragma unroll
        for (int j = 0; j < 8; ++j) raw[kq][j] = 0.f;
      if (q < S) {
        const float* src = reinterpret_cast<const float*>(Q) + (int64_t)q * a.qs[2];
        if constexpr (HP == 16) {
          if (4 * g < HD) {
            const float4 x = *reinterpret_cast<const float4*>(src + 4 * g);
            raw[0][0] = x.x; raw[0][1] = x.y; raw[0][2] = x.z; raw[0][3] = x.w;
          }
        } else {
#pragma unroll
          for (int kq = 0; kq < QK_STEPS; ++kq) {
            const float4 x0 = *reinterpret_cast<const float4*>(src + kq * 32 + 8 * g);
            const float4 x1 = *reinterpret_cast<const float4*>(src + kq * 32 + 8 * g + 4);
            raw[kq][0] = x0.x; raw[kq][1] = x0.y; raw[kq][2] = x0.z; raw[kq][3] = x0.w;
            raw[kq][4] = x1.x; raw[kq][5] = x1.y; raw[kq][6] = x1.z; raw[kq][7] = x1.w;
          }
        }
      }
#pragma unroll
      for (int kq = 0; kq < QK_STEPS; ++kq)
#pragma unroll
        for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(raw[kq][j]));
      const int qexp = f32_scale_exp(max_over_groups(mx));
      ceff[t] = ldexpf(a.c, qexp + kexp);
      if constexpr (HP == 16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) qh16[t][j] = (_Float16)ldexpf(raw[0][j], -qexp);
      } else {
#pragma unroll
        for (int kq = 0; kq < QK_STEPS; ++kq)
#pragma unroll
          for (int j = 0; j < 8; ++j) qh[t][kq][j] = (_Float16)ldexpf(raw[kq][j], -qexp);
      }
    } else if constexpr (HP == 16) {
      float v[4] = {0.f, 0.f, 0.f, 0.f};
      if (q < S && 4 * g < HD) {
        const IT* src = Q + (int64_t)q * a.qs[2] + 4 * g;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (float)(_Float16)src[j] * a.c;
      }
      pin_f32x4(v);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        qh16[t][j] = (_Float16)v[j];
        ql16[t][j] = (_Float16)(v[j] - (float)qh16[t][j]);
      }
    } else {
#pragma unroll
      for (int kq = 0; kq < QK_STEPS; ++kq) {
        const h8 raw = q < S ? load8_as_half(Q + (int64_t)q * a.qs[2] + kq * 32 + 8 * g) : zero_h8();
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (float)raw[j] * a.c;
        pin_f32x8(v);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          qh[t][kq][j] = (_Float16)v[j];
          ql[t][kq][j] = (_Float16)(v[j] - (float)qh[t][kq][j]);
        }
      }
    }
  }

  // ---- running statistics (log2 units) and output accumulators ----
  // mrow: running max of s*c for the query row; fresh: the row has not seen a
  // visible key yet (its tiles are computed without the -mrow offset).
  float mrow[QT];
  bool fresh[QT];
  f4 oacc[QT][SH::DT][2];
  // Row sums of fp16(P) come out of the PV product: an extra A operand whose
  // row 0 is all ones gives sum_k P[q][k] in row 0 of lsum (lanes of group 0).
  f4 lsum_acc[QT];
  h8 ones_row;
#pragma unroll
  for (int j = 0; j < 8; ++j) ones_row[j] = r == 0 ? (_Float16)1.0f : (_Float16)0.0f;
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    mrow[t] = 0.f;
    fresh[t] = true;
    lsum_acc[t] = zero4();
#pragma unroll
    for (int dt = 0; dt < SH::DT; ++dt) oacc[t][dt][0] = oacc[t][dt][1] = zero4();
  }

  // ---- register prefetch of one K/V tile ----
  // K items: one 16-byte chunk of one key row, stored as-is.  V items: the same
  // chunk of two consecutive keys, stored transposed as 8 dwords (d, key pair),
  // so a wave's 64 lanes write consecutive key pairs of two d rows per
  // instruction - no bank conflicts, and a quarter of the 16-bit stores.
  h8 kreg[SH::PER_THREAD], vreg[SH::V_PER_THREAD][2];
  float breg = 0.f;
  // Buffer resources cover only the tile's keys that exist (min(KTILE, S - kb)
  // rows), so the hardware returns zeros for keys past the end of the sequence.
  const uint32_t krow_bytes = (uint32_t)(a.ks[2] * (int64_t)sizeof(IT));
  const uint32_t vrow_bytes = (uint32_t)(a.vs[2] * (int64_t)sizeof(IT));
  auto fetch = [&](int kb) {
    const uint32_t rows = (uint32_t)min(KTILE, S - kb);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(Kp + (int64_t)kb * a.ks[2], rows * krow_bytes);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(Vp + (int64_t)kb * a.vs[2], rows * vrow_bytes);
#pragma unroll
    for (int i = 0; i < SH::PER_THREAD; ++i) {
      const int c = threadIdx.x + i * NT;
      const int key = c / SH::CPK, col = (c % SH::CPK) * 8;
      if (c < SH::CHUNKS) {
        const uint32_t off = key * krow_bytes + col * (uint32_t)sizeof(IT);
        if constexpr (F32IN) kreg[i] = buffer_load8_scaled(kr, off, kexp);
        else kreg[i] = buffer_load8_as_half(kr, off, Kp);
      }
    }
#pragma unroll
    for (int i = 0; i < SH::V_PER_THREAD; ++i) {
      const int c = threadIdx.x + i * NT;
      const int kp = c % (KTILE / 2), col = (c / (KTILE / 2)) * 8;
      if (c < SH::VITEMS) {
        const uint32_t off = 2 * kp * vrow_bytes + col * (uint32_t)sizeof(IT);
        if constexpr (F32IN) {
          vreg[i][0] = buffer_load8_scaled(vr, off, vexp);
          vreg[i][1] = buffer_load8_scaled(vr, off + vrow_bytes, vexp);
        } else {
          vreg[i][0] = buffer_load8_as_half(vr, off, Vp);
          vreg[i][1] = buffer_load8_as_half(vr, off + vrow_bytes, Vp);
        }
      }
    }
    if (threadIdx.x < KTILE) {
      const int gk = kb + threadIdx.x;
      bool valid = gk < S;
      if (KEYMASK && valid) valid = kv_valid[gk] != 0;
      breg = valid ? 0.f : -INFINITY;
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < SH::PER_THREAD; ++i) {
      const int c = threadIdx.x + i * NT;
      if (c < SH::CHUNKS) {
        const int key = c / SH::CPK, col = (c % SH::CPK) * 8;
        *reinterpret_cast<h8*>(&ks_lds[buf][key * SH::LDK + col]) = kreg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < SH::V_PER_THREAD; ++i) {
      const int c = threadIdx.x + i * NT;
      if (c < SH::VITEMS) {
        const int kp = c % (KTILE / 2), col = (c / (KTILE / 2)) * 8;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          typedef _Float16 h2 __attribute__((ext_vector_type(2)));
          h2 pair;
          pair[0] = vreg[i][0][j];
          pair[1] = vreg[i][1][j];
          *reinterpret_cast<h2*>(&vt_lds[buf][(col + j) * SH::LDV + 2 * kp]) = pair;
        }
      }
    }
    if (threadIdx.x < KTILE) kbias[buf][threadIdx.x] = breg;
  };

  // ---- one key tile: S^T, online softmax, O^T += V^T P^T ----
  // FIRST: the tile may hold a row's first visible key, so rows can still be
  // "fresh" (their scores were computed without the -mrow offset).  Without a
  // key mask every row sees key 0, so only tile 0 needs that handling and the
  // steady-state tiles skip it.
  auto process = [&](const int kb, const _Float16* ksb, const _Float16* vtb, const float* kbb, auto first_tag) {
    constexpr bool MAYBE_FRESH = decltype(first_tag)::value || KEYMASK;
    if (a.causal && kb > qw_last) return;  // whole tile is in this wave's future
    // Key pairs [0, npv) hold keys visible to some query of this wave; in a
    // causal tile on the diagonal only the last of them straddles it (queries of
    // a wave are 16-aligned, pairs 32-aligned) and the pairs after it are skipped.
    const int npv = a.causal ? min(NP, (qw_last - kb) / 32 + 1) : NP;
    const bool need_causal = a.causal && kb + 32 * npv - 1 > qw0;  // last visible pair straddles the diagonal
    const bool need_bias = KEYMASK || kb + KTILE > S;               // padded keys or keys past the end

    // S^T = K (Q*c)^T - m for the visible key pairs x 16*QT queries
    f4 sc[NP][2][QT];  // [key pair][tile in pair][q tile]
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      if (p >= npv) break;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int krow = 32 * p + pair_row(r, tt);
#pragma unroll
        for (int t = 0; t < QT; ++t) {
          const float c0 = (F32IN || (MAYBE_FRESH && fresh[t])) ? 0.f : -mrow[t];
          sc[p][tt][t] = f4{c0, c0, c0, c0};
        }
        if constexpr (HP == 16) {
          const h4 ka = *reinterpret_cast<const h4*>(&ksb[krow * SH::LDK + 4 * g]);
#pragma unroll
          for (int t = 0; t < QT; ++t) {
            sc[p][tt][t] = mfma16(ka, qh16[t], sc[p][tt][t]);
            if constexpr (!F32IN) sc[p][tt][t] = mfma16(ka, ql16[t], sc[p][tt][t]);
          }
        } else {
#pragma unroll
          for (int kq = 0; kq < QK_STEPS; ++kq) {
            const h8 ka = *reinterpret_cast<const h8*>(&ksb[krow * SH::LDK + kq * 32 + 8 * g]);
#pragma unroll
            for (int t = 0; t < QT; ++t) {
              sc[p][tt][t] = mfma32(ka, qh[t][kq], sc[p][tt][t]);
              if constexpr (!F32IN) sc[p][tt][t] = mfma32(ka, ql[t][kq], sc[p][tt][t]);
            }
          }
        }
        if constexpr (F32IN) {  // raw q' . k' -> s*c - m
#pragma unroll
          for (int t = 0; t < QT; ++t) {
            const float negm = (MAYBE_FRESH && fresh[t]) ? 0.f : -mrow[t];
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[p][tt][t][i] = fmaf(sc[p][tt][t][i], ceff[t], negm);
          }
        }
      }
    }

    // Masks.  Key kb + 32p + 8g + 4tt + i is visible to query qw0 + 16t + r iff
    // it is not past it; only pair npv-1 can hold keys past some of the wave's queries.
    if (need_causal) {
      const int pl = npv - 1;
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        const int lim = qw0 + 16 * t + r - kb - 32 * pl - 8 * g;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          if (p != pl) continue;
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (4 * tt + i > lim) sc[p][tt][t][i] = -INFINITY;
        }
      }
    }
    if (need_bias) {
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        if (p >= npv) break;
#pragma unroll
        for (int t = 0; t < QT; ++t)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[p][tt][t][i] += kbb[32 * p + 8 * g + 4 * tt + i];
      }
    }

    // Online softmax.  Scores arrive as s*c - mrow.  The running max is only
    // raised when a tile exceeds it by more than kRescaleLog2; otherwise the
    // stale max is kept and p may reach 2^kRescaleLog2.  acc and l share the
    // scale, so o = acc / l is unchanged.  Fresh rows adopt their first finite max.
    // Each lane first takes the max of its own scores of the row; the reduction
    // over the row's four lane groups is only needed when some lane's partial
    // max calls for a shift (a fresh row, or one above the threshold).
    float pm[QT];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      float mx = sc[0][0][t][0];
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        if (p >= npv) break;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[p][tt][t][i]);
      }
      pm[t] = mx;
    }
    bool any_shift = false;
#pragma unroll
    for (int t = 0; t < QT; ++t) any_shift |= (MAYBE_FRESH && fresh[t]) || pm[t] > kRescaleLog2;
    if (__builtin_amdgcn_ballot_w64(any_shift)) {  // the first tile, and rarely after it
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        const float mx = max_over_groups(pm[t]);
        const bool is_fresh = MAYBE_FRESH && fresh[t];
        const bool shift_row = is_fresh ? (mx > -INFINITY) : (mx > kRescaleLog2);
        const float shift = shift_row ? mx : 0.f;
        if (shift_row && !is_fresh) {
          const float alpha = __builtin_amdgcn_exp2f(-shift);
          lsum_acc[t] *= alpha;
#pragma unroll
          for (int dt = 0; dt < SH::DT; ++dt) {
            oacc[t][dt][0] *= alpha;
            oacc[t][dt][1] *= alpha;
          }
        }
        if (shift_row) {
          mrow[t] = is_fresh ? shift : mrow[t] + shift;
          fresh[t] = false;
        }
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          if (p >= npv) break;
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[p][tt][t][i] -= shift;
        }
      }
    }

    // fp16(P) as the B operand of the PV product, then O^T += V^T P^T and the row sums of P
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      if (p >= npv) break;
      h8 pf[QT];
#pragma unroll
      for (int t = 0; t < QT; ++t)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) pf[t][4 * tt + i] = (_Float16)__builtin_amdgcn_exp2f(sc[p][tt][t][i]);
#pragma unroll
      for (int t = 0; t < QT; ++t) lsum_acc[t] = mfma32(ones_row, pf[t], lsum_acc[t]);
      if constexpr (HP == 16) {
        const h8 va = *reinterpret_cast<const h8*>(&vtb[r * SH::LDV + 32 * p + 8 * g]);
#pragma unroll
        for (int t = 0; t < QT; ++t) oacc[t][0][0] = mfma32(va, pf[t], oacc[t][0][0]);
      } else {
#pragma unroll
        for (int dt = 0; dt < SH::DT; ++dt)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            const int drow = 32 * dt + pair_row(r, tt);
            const h8 va = *reinterpret_cast<const h8*>(&vtb[drow * SH::LDV + 32 * p + 8 * g]);
#pragma unroll
            for (int t = 0; t < QT; ++t) oacc[t][dt][tt] = mfma32(va, pf[t], oacc[t][dt][tt]);
          }
      }
    }
  };

  // Double-buffered pipeline, one barrier per tile: tile i+1 is fetched into
  // registers while tile i is processed, then staged into the other buffer
  // (last read in iteration i-1, which every wave left before the barrier).
  if constexpr (HD < HP) {
    // the padding dims are never staged: zero them once (K's feed the QK^T sums)
    for (int i = threadIdx.x; i < 2 * SH::KBUF; i += NT) (&ks_lds[0][0])[i] = (_Float16)0.0f;
    for (int i = threadIdx.x; i < 2 * SH::VBUF; i += NT) (&vt_lds[0][0])[i] = (_Float16)0.0f;
    __syncthreads();
  }
  fetch(0);
  stash(0);
  __syncthreads();
  for (int tile = 0; tile < ntiles; ++tile) {
    const int cur = tile & 1;
    const bool more = tile + 1 < ntiles;
    if (more) fetch((tile + 1) * KTILE);
    if (tile == 0)
      process(0, ks_lds[cur], vt_lds[cur], kbias[cur], std::true_type{});
    else
      process(tile * KTILE, ks_lds[cur], vt_lds[cur], kbias[cur], std::false_type{});
    if (more) stash(cur ^ 1);
    __syncthreads();
  }

  // ---- normalise and store ----
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int q = qw0 + 16 * t + r;
    const float lsum = sum_over_groups(lsum_acc[t][0]);
    float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    if constexpr (F32IN) inv = ldexpf(inv, vexp);  // o = (sum p v') / l * 2^vexp
    if (q >= S) continue;
    OT* dst = O + (int64_t)q * a.os[2];
    if constexpr (HP == 16) {
      // lane group g holds d = 4g .. 4g+3
      if (4 * g < HD) {
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = oacc[t][0][0][i] * inv;
        pin_f32x4(o);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[4 * g + i] = (OT)o[i];
      }
    } else {
#pragma unroll
      for (int dt = 0; dt < SH::DT; ++dt) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[i] = oacc[t][dt][0][i] * inv;
          v[4 + i] = oacc[t][dt][1][i] * inv;
        }
        pin_f32x8(v);
        store8(dst + 32 * dt + 8 * g, v);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 32x32 variant for head_dim 32 / 64: S^T = K Q^T and O^T = V^T P^T on
// v_mfma_f32_32x32x16_f16, whose long issue-to-result time lets the softmax
// VALU work of the same wave run beside it (the 16x16x32 form leaves little
// room for that, and at these head dims the softmax is the larger cost).
//
// 32x32x16 operand layouts and the kappa32 row map are described in mpk_common.h:
// MFMA row rho of a 32-row block is fed from row kappa32(rho) of the tile (keys
// for S^T, head dims for O^T), so the lane (i, h) accumulator register e = 8s + j
// holds tile row 16s + 8h + j.  For S^T that is the B operand of the two 16-key
// steps of the P V product; for O^T it is 2 x 8 consecutive head dims of query i.
// Each lane owns one query (i) and half of its keys, so a row max is a
// lane-local max plus one permlane32 swap.
//
// Scores are computed raw (s = q.k, FP16 operands, FP32 accumulate) and mapped
// to the exponent as fma(s, |c|, -m) with the query negated when the scale is
// negative: one rounding, as in the reference's scaled dot followed by the max
// subtraction.  (Folding c into a hi + lo split of q, as attention_kernel does,
// doubles the S^T MFMAs; measured on MI355X that lengthens each wave's
// MFMA -> softmax -> MFMA chain by more than the FMA it saves.)  Per score the
// VALU runs the FMA, the exponential (half the FMA rate on gfx950, not
// overlapped with other VALU work), the max and the FP16 conversion, which makes
// it the binding unit at these head dims.  Row sums of fp16(P) come from a 16x16x32 product with a 0/1
// A operand (rows 0 and 1 pick the queries i and i + 16 out of the P fragment
// layout), so l sums exactly the FP16 weights that multiply V.
// PS: q arrives pre-multiplied by scale * log2(e) (mpk_causal_attention_prescaled), so the
// scores are already in log2 units: c = 1, and on steady tiles the S^T accumulator starts at
// -m, which leaves p = 2^(acc) with no per-score FMA.
template <int HD, int NW, int KTILE, typename IT, typename OT, bool KEYMASK, bool PS = false>
// (four waves per SIMD, i.e. at most 128 VGPRs, for FP16 input at head dim 32 with 64-key
// tiles; FP32 input carries a per-row score factor, one register more, and runs at three)
__global__ __launch_bounds__(64 * NW) __attribute__((
    amdgpu_waves_per_eu(HD == 32 && KTILE == 64 && std::is_same<IT, _Float16>::value ? 4 : 1)))
void attention32_kernel(AttnArgs a) {
  static_assert(!PS || std::is_same<IT, _Float16>::value, "pre-scaled q is FP16");
  constexpr int NT = 64 * NW;
  using SH = AttnShape<HD, KTILE, NT>;
  constexpr int QB = 32 * NW;     // queries per workgroup, 32 per wave
  constexpr int NB = KTILE / 32;  // 32-key blocks per tile
  constexpr int QS = HD / 16;     // 16-wide head-dim steps of S^T
  constexpr int DT = HD / 32;     // 32-row head-dim tiles of O^T
  static_assert(HD == 32 || HD == 64, "head dim");
  static_assert(KTILE % 32 == 0 && KTILE <= NT, "key tile");

  __shared__ __align__(16) _Float16 ks_lds[2][SH::KBUF];
  // V is staged row-major like K (one 16-byte store per chunk); the P V product
  // reads its V^T fragments with LDS transpose loads (ds_read_b64_tr_b16).  Each
  // 32-lane half of such a read covers 4 consecutive keys x 64 bytes of head dims,
  // which meet no bank conflict on gfx950 only when the row stride is an odd
  // multiple of 64 bytes (measured with SQ_LDS_BANK_CONFLICT; the K tile's
  // 16-byte-padded stride, right for the K fragment reads, conflicts two ways here):
  // unpadded rows at hd 32.  (At hd 64 that takes 192-byte rows, which measured no
  // faster than the K stride; hd 64 keeps it.)
  constexpr int LDVR = HD == 32 ? HD : SH::LDK;
  __shared__ __align__(16) _Float16 vr_lds[2][KTILE * LDVR];
  __shared__ float kbias[2][KTILE];

  const int S = a.seq;
  const int BH = a.batch * a.heads;
  const int nqb = (S + QB - 1) / QB;
  // As in attention_kernel, each XCD owns a contiguous range of (batch, head) rows.  When
  // the launch runs many rounds of workgroups (group > 0, set by the launcher), the XCD walks
  // its range in groups of `group` rows, each group's query blocks longest first: the
  // workgroups in flight on an XCD then share the K/V prefixes of about `group` rows, which
  // fit its L2 (at B 64, H 8, S 4096, hd 32 the fetched bytes drop from 2.41 GB to 0.59 GB
  // per launch).  Otherwise the XCD runs one query block of every row of its range at a
  // time, longest first.  Both orders keep the longest blocks first, so no XCD ends with a
  // long block started late.
  int bh, qblock;
  if ((BH & 7) == 0) {
    const int per_xcd = BH >> 3;
    const int slot = blockIdx.x >> 3;
    if (a.group > 0) {
      // each XCD walks its range's groups from the last down: the QKV projection walks the
      // same eighths of the tokens upwards on the same XCDs, so the rows it wrote last are
      // read first, while they are still in the XCD's L2 and the last-level cache
      const int G = a.group, per_grp = G * nqb;
      const int grp = slot / per_grp, r = slot - grp * per_grp;
      const int ngrp = per_xcd / G;
      bh = (blockIdx.x & 7) * per_xcd + (ngrp - 1 - grp) * G + r % G;
      qblock = nqb - 1 - r / G;
    } else {
      bh = (blockIdx.x & 7) * per_xcd + slot % per_xcd;
      qblock = nqb - 1 - slot / per_xcd;
    }
  } else {
    bh = blockIdx.x % BH;
    qblock = nqb - 1 - (int)(blockIdx.x / BH);
  }
  const int b = bh / a.heads, h = bh % a.heads;
  const int q0 = qblock * QB;

  const IT* __restrict__ Q = static_cast<const IT*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const IT* __restrict__ Kp = static_cast<const IT*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const IT* __restrict__ Vp = static_cast<const IT*>(a.v) + b * a.vs[0] + h * a.vs[1];
  OT* __restrict__ O = static_cast<OT*>(a.o) + b * a.os[0] + h * a.os[1];
  const uint8_t* kv_valid = KEYMASK ? a.key_valid + (int64_t)b * S : nullptr;

  const int l = threadIdx.x & 63, wave = wave_id();
  const int qi = l & 31, hf = l >> 5;
  const int qw0 = q0 + 32 * wave;  // first query of this wave (32-aligned, as are key blocks)
  const int q = qw0 + qi;
  const int trow = kappa32(qi);    // tile row this lane feeds as an A-operand row

  const int kv_end = a.causal ? min(q0 + QB, S) : S;
  const int ntiles = (kv_end + KTILE - 1) / KTILE;

  // FP32 inputs: power-of-two exponents for K and V over the keys this workgroup reads,
  // and per query row for q (see f32_scale_exp); FP16 inputs are used as they are.
  constexpr bool F32IN = std::is_same<IT, float>::value;
  int kexp = 0, vexp = 0;
  if constexpr (F32IN) {
    __shared__ float red[NW];
    kexp = __builtin_amdgcn_readfirstlane(
        f32_scale_exp(wg_absmax<NT>(reinterpret_cast<const float*>(Kp), a.ks[2], kv_end, HD, red)));
    vexp = __builtin_amdgcn_readfirstlane(
        f32_scale_exp(wg_absmax<NT>(reinterpret_cast<const float*>(Vp), a.vs[2], kv_end, HD, red)));
  }

  // Q fragments (B operand of S^T): query q, head dims 16 st + 8 hf .. +7; negated for a
  // negative scale, so scores map to the exponent as fma(s, |c|, -m).  FP32 inputs: q' =
  // fp16(q 2^-a) for the row's exponent a, and c becomes |c| 2^(a + kexp).
  float c = PS ? 1.0f : fabsf(a.c);
  const bool neg = !PS && a.c < 0.f;
  h8 qf[QS];
  if constexpr (F32IN) {
    // two passes over the row (the maximum first, then the scaled conversion), so no
    // FP32 copy of q stays live across the exponent's cross-lane exchange
    const float* src = reinterpret_cast<const float*>(Q) + (int64_t)q * a.qs[2] + 8 * hf;
    auto load8 = [&](int st, float (&x)[8]) {
      float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
      if (q < S) {
        x0 = *reinterpret_cast<const float4*>(src + 16 * st);
        x1 = *reinterpret_cast<const float4*>(src + 16 * st + 4);
      }
      x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w;
      x[4] = x1.x; x[5] = x1.y; x[6] = x1.z; x[7] = x1.w;
    };
    float mx = 0.f;
#pragma unroll
    for (int st = 0; st < QS; ++st) {
      float x[8];
      load8(st, x);
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(x[j]));
    }
    // lanes qi and qi + 32 hold the two halves of query q's head dims
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    const int qexp = f32_scale_exp(fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])));
    c = ldexpf(c, qexp + kexp);
#pragma unroll
    for (int st = 0; st < QS; ++st) {
      float x[8];
      load8(st, x);
      h8 v;
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = (_Float16)ldexpf(x[j], -qexp);
      if (neg) v = -v;
      qf[st] = v;
    }
  } else {
#pragma unroll
    for (int st = 0; st < QS; ++st) {
      h8 v = q < S ? load8_as_half(Q + (int64_t)q * a.qs[2] + 16 * st + 8 * hf) : zero_h8();
      if (neg) v = -v;
      qf[st] = v;
    }
  }

  // 0/1 A operand of the row-sum product (16x16x32 layout: lane l holds row l % 16,
  // k = 8 (l / 16) .. +7): row 0 sums the P columns of query i, row 1 of query i + 16.
  h8 ones;
  {
    const int row = l & 15, grp = l >> 4;
    const bool one = (row == 0 && (grp & 1) == 0) || (row == 1 && (grp & 1) == 1);
#pragma unroll
    for (int j = 0; j < 8; ++j) ones[j] = one ? (_Float16)1.0f : (_Float16)0.0f;
  }

  float mrow = 0.f;     // running max of s*c (log2 units) of this lane's query
  bool fresh = true;    // no visible key seen yet
  // Pre-scaled steady tiles start every S^T block at -m with one 32x32x8 MFMA instead of
  // VALU moves: A selects k = 0 for every key row (msel), B holds fp16(-m) of the lane's
  // query at k = 0 (mneg, lanes 0..31), so D[key][query] = -m.  For that the row max is
  // kept as an FP16 value: rounded to the nearest one when raised (any m works, as long as
  // acc and l share it; within 0.5 of the true max, weights stay <= 2^0.5) while every
  // |m| of the wave is below kExactMaxLimit; once one is not (mwide, sticky), the steady
  // tiles splat the FP32 -m with moves instead.
  typedef _Float16 h4m __attribute__((ext_vector_type(4)));
  h4m msel, mneg;
#pragma unroll
  for (int j = 0; j < 4; ++j) msel[j] = (_Float16)0.0f, mneg[j] = (_Float16)0.0f;
  if (hf == 0) msel[0] = (_Float16)1.0f;
  constexpr float kExactMaxLimit = 2048.f;  // FP16 spacing <= 1 below it
  int mwide = 0;
  auto round_m = [&](float m) { return (PS && fabsf(m) < kExactMaxLimit) ? (float)(_Float16)m : m; };
  // after every update of mrow, in wave-uniform control flow (the ballot needs all lanes)
  auto set_mneg = [&]() {
    if constexpr (PS) {
      if (hf == 0) mneg[0] = (_Float16)(-mrow);
      mwide = __builtin_amdgcn_readfirstlane(
          mwide | (__builtin_amdgcn_ballot_w64(!(fabsf(mrow) < kExactMaxLimit)) != 0));
    }
  };
  f16v oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[dt][e] = 0.f;
  f4 lsum = zero4();    // lanes 0..15: [0] = l of query i, [1] = l of query i + 16

  // ---- register prefetch / LDS staging of one K/V tile (both row-major) ----
  h8 kreg[SH::PER_THREAD], vreg[SH::PER_THREAD];
  float breg = 0.f;
  // Key bias (-inf for masked keys and keys past the sequence end): staged only for
  // tiles that read it, which is every tile with a key mask and otherwise only a tile
  // that runs past the sequence end (wave-uniform).
  bool bias_staged = false;
  const uint32_t krow_bytes = (uint32_t)(a.ks[2] * (int64_t)sizeof(IT));
  const uint32_t vrow_bytes = (uint32_t)(a.vs[2] * (int64_t)sizeof(IT));
  // FP16 inputs at head dim 32: K and V tiles travel global -> LDS as LDS-DMA copies (1 KB
  // each, no registers; K rows padded to LDK halves, the pad units filled from the row's
  // start; keys past the sequence copy its last row, which the key bias masks), issued
  // round-robin by the waves at the start of a step and awaited (vmcnt 0: the loop issues no
  // other vector-memory operation) before its barrier.  Measured on MI355X in one process,
  // outputs bit-identical: cfg5 forward 48.61-48.63 vs 49.03-49.06 ms, cfg2 level; at head
  // dim 64 (cfg4) the register staging below stays, 2.594 vs 2.603 ms.
  constexpr bool DMA_KV = !F32IN && HD == 32;
  constexpr int KUP = SH::LDK / 8, VUP = LDVR / 8, KU = HD / 8;
  constexpr int KCOPIES = KTILE * KUP / 64, VCOPIES = KTILE * VUP / 64;
  static_assert(!DMA_KV || (KTILE * KUP % 64 == 0 && KTILE * VUP % 64 == 0), "whole copies");
  auto fetch_dma = [&](int kb, int buf) {
    const int last = S - 1 - kb;  // last key of the sequence, relative to the tile
    const uint32_t kl = (uint32_t)(uintptr_t)(lds_void*)ks_lds[buf];
    const uint32_t vl = (uint32_t)(uintptr_t)(lds_void*)vr_lds[buf];
    const _Float16* kbase = reinterpret_cast<const _Float16*>(Kp) + (int64_t)kb * a.ks[2];
    const _Float16* vbase = reinterpret_cast<const _Float16*>(Vp) + (int64_t)kb * a.vs[2];
    for (int j = wave; j < KCOPIES + VCOPIES; j += NW) {
      if (j < KCOPIES) {
        const int u = 64 * j + l, key = min(u / KUP, last), pos = u % KUP;
        dma16((uint32_t)key * krow_bytes + (pos < KU ? 16u * pos : 0u), kbase, (uint32_t)__builtin_amdgcn_readfirstlane((int)(kl + 1024u * j)));
      } else {
        const int u = 64 * (j - KCOPIES) + l, key = min(u / VUP, last), pos = u % VUP;
        dma16((uint32_t)key * vrow_bytes + (pos < KU ? 16u * pos : 0u), vbase, (uint32_t)__builtin_amdgcn_readfirstlane((int)(vl + 1024u * (j - KCOPIES))));
      }
    }
    bias_staged = KEYMASK || kb + KTILE > S;
    if (bias_staged && threadIdx.x < KTILE) {
      const int gk = kb + threadIdx.x;
      bool valid = gk < S;
      if (KEYMASK && valid) valid = kv_valid[gk] != 0;
      kbias[buf][threadIdx.x] = valid ? 0.f : -INFINITY;
    }
  };
  auto fetch = [&](int kb) {
    const uint32_t rows = (uint32_t)min(KTILE, S - kb);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(Kp + (int64_t)kb * a.ks[2], rows * krow_bytes);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(Vp + (int64_t)kb * a.vs[2], rows * vrow_bytes);
#pragma unroll
    for (int i = 0; i < SH::PER_THREAD; ++i) {
      const int cc = threadIdx.x + i * NT;
      const int key = cc / SH::CPK, col = (cc % SH::CPK) * 8;
      if (cc < SH::CHUNKS) {
        const uint32_t off = key * krow_bytes + col * (uint32_t)sizeof(IT);
        if constexpr (F32IN) kreg[i] = buffer_load8_scaled(kr, off, kexp);
        else kreg[i] = buffer_load8_as_half(kr, off, Kp);
      }
    }
#pragma unroll
    for (int i = 0; i < SH::PER_THREAD; ++i) {
      const int cc = threadIdx.x + i * NT;
      const int key = cc / SH::CPK, col = (cc % SH::CPK) * 8;
      if (cc < SH::CHUNKS) {
        const uint32_t off = key * vrow_bytes + col * (uint32_t)sizeof(IT);
        if constexpr (F32IN) vreg[i] = buffer_load8_scaled(vr, off, vexp);
        else vreg[i] = buffer_load8_as_half(vr, off, Vp);
      }
    }
    bias_staged = KEYMASK || kb + KTILE > S;
    if (bias_staged && threadIdx.x < KTILE) {
      const int gk = kb + threadIdx.x;
      bool valid = gk < S;
      if (KEYMASK && valid) valid = kv_valid[gk] != 0;
      breg = valid ? 0.f : -INFINITY;
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < SH::PER_THREAD; ++i) {
      const int cc = threadIdx.x + i * NT;
      if (cc < SH::CHUNKS) {
        const int key = cc / SH::CPK, col = (cc % SH::CPK) * 8;
        *reinterpret_cast<h8*>(&ks_lds[buf][key * SH::LDK + col]) = kreg[i];
        *reinterpret_cast<h8*>(&vr_lds[buf][key * LDVR + col]) = vreg[i];
      }
    }
    if (bias_staged && threadIdx.x < KTILE) kbias[buf][threadIdx.x] = breg;
  };
  // V^T fragment (A operand of O^T = V^T P^T) from the row-major V tile: MFMA row i
  // (head dim 32 dt + kappa(i)) and keys k0 .. k0 + 7, as two transpose loads.  Within
  // each 16-lane group a transpose load hands lane j element (j % 4) of the 8 bytes read
  // by lane 4 m + j / 4, for m = 0..3; so lane r of group G reads key k0 + r / 4 (+4) at
  // the 4 dims starting at 32 dt + 16 (G & 1) + 8 (q & 1) + 4 (q >> 1), q = r % 4, and
  // every lane receives 4 consecutive keys of its own row's dim.
  typedef short s4v __attribute__((ext_vector_type(4)));
  const int vtr_r = l & 15, vtr_g = l >> 4, vtr_q = vtr_r & 3;
  const int vtr_dim = 16 * (vtr_g & 1) + 8 * (vtr_q & 1) + 4 * (vtr_q >> 1);
  auto vt_frag = [&](const _Float16* vrb, int dt, int k0) {
    const _Float16* p0 = vrb + (k0 + (vtr_r >> 2)) * LDVR + 32 * dt + vtr_dim;
    const s4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4v*)(p0));
    const s4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4v*)(p0 + 4 * LDVR));
    typedef _Float16 h4v __attribute__((ext_vector_type(4)));
    const h4v a = __builtin_bit_cast(h4v, lo), b = __builtin_bit_cast(h4v, hi);
    h8 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = a[j];
      v[4 + j] = b[j];
    }
    return v;
  };

  // ---- one key tile ----
  // The S^T products of all of the tile's 32-key blocks are issued first; the
  // softmax and P V of block nb then run on the VALU while the MFMAs of the
  // later blocks are still in flight, so one wave keeps both units busy.  The
  // running max is checked once per tile.
  // EDGE: the tile may hold blocks in the wave's future, the diagonal block, keys
  // past the sequence end or masked keys; steady-state tiles skip those checks.
  auto process = [&](const int kb, const _Float16* ksb, const _Float16* vtb, const float* kbb, auto first_tag,
                     auto edge_tag) {
    constexpr bool MAYBE_FRESH = decltype(first_tag)::value || KEYMASK;
    constexpr bool EDGE = decltype(edge_tag)::value;
    // blocks [0, nbv) hold keys visible to some query of the wave (wave-uniform)
    const int nbv = (EDGE && a.causal) ? min(NB, (qw0 - kb) / 32 + 1) : NB;
    if (EDGE && nbv <= 0) return;
    const bool need_bias = KEYMASK || kb + KTILE > S;

    // S^T (32 keys x 32 queries) per block, raw scores (pre-scaled steady tiles: minus m)
    constexpr bool STEADY = !EDGE && !MAYBE_FRESH && HD == 32 && KTILE == 64;
    const float sc0 = (PS && STEADY) ? -mrow : 0.f;
    f16v sc[NB];
    f16v cinit;  // pre-scaled steady tiles: -m in every register, the start of each block's S^T
    if constexpr (PS && STEADY) {
      if (__builtin_amdgcn_readfirstlane(mwide) == 0) {
        cinit = __builtin_amdgcn_mfma_f32_32x32x8f16(msel, mneg, f16v{}, 0, 0, 0);
      } else {
        // -m splat: one pair (-m, -m), then seven 64-bit moves instead of fifteen 32-bit
        // ones (the compiler splats a scalar with 32-bit moves only; the immediate keeps
        // the seven statements distinct so they are not merged into one).  The hazard
        // recognizer counts an asm statement's outputs as VALU writes and puts the wait
        // states an MFMA source needs after them.
        typedef float f2v __attribute__((ext_vector_type(2)));
        typedef double d8v __attribute__((ext_vector_type(8)));
        const f2v pr = {sc0, sc0};
        const double dp = __builtin_bit_cast(double, pr);
        d8v dv;
        dv[0] = dp;
#pragma unroll
        for (int i = 1; i < 8; ++i) {
          double t;
          asm("v_mov_b64 %0, %1 ; %2" : "=v"(t) : "v"(dp), "n"(i));
          dv[i] = t;
        }
        cinit = __builtin_bit_cast(f16v, dv);
      }
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (EDGE && nb >= nbv) break;
      if constexpr (PS && STEADY) {
        sc[nb] = cinit;
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) sc[nb][e] = sc0;
      }
#pragma unroll
      for (int st = 0; st < QS; ++st) {
        const h8 ka = *reinterpret_cast<const h8*>(&ksb[(32 * nb + trow) * SH::LDK + 16 * st + 8 * hf]);
        sc[nb] = mfma32x32(ka, qf[st], sc[nb]);
      }
    }
    if constexpr (EDGE) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if (nb >= nbv) break;
        // register e holds key kb + 32 nb + 16 (e >> 3) + 8 hf + (e & 7)
        if (a.causal && kb + 32 * nb == qw0) {  // the block on the diagonal: keys past the query are masked
          const int lim = qi - 8 * hf;
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (16 * (e >> 3) + (e & 7) > lim) sc[nb][e] = -INFINITY;
        }
        if (need_bias) {
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            const float* kbp = kbb + 32 * nb + 16 * s2 + 8 * hf;
            const float4 b0 = *reinterpret_cast<const float4*>(kbp);
            const float4 b1 = *reinterpret_cast<const float4*>(kbp + 4);
            sc[nb][8 * s2 + 0] += b0.x; sc[nb][8 * s2 + 1] += b0.y;
            sc[nb][8 * s2 + 2] += b0.z; sc[nb][8 * s2 + 3] += b0.w;
            sc[nb][8 * s2 + 4] += b1.x; sc[nb][8 * s2 + 5] += b1.y;
            sc[nb][8 * s2 + 6] += b1.z; sc[nb][8 * s2 + 7] += b1.w;
          }
        }
      }
    }

    // online softmax with a lazily raised max (see attention_kernel): the row max
    // is raised only when a score exceeds it by more than kRescaleLog2.
    // raise_max: the lane-local max over the tile decides whether the row-wide one
    // is needed at all; if so the row max is raised and O and l are rescaled.
    auto raise_max = [&]() {
      float mx = sc[0][0];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if (EDGE && nb >= nbv) break;
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sc[nb][e]);
      }
      const float ms = mx * c;  // this lane's max of s*c
      const bool want = (MAYBE_FRESH && fresh) || ms - mrow > kRescaleLog2;
      if (__builtin_amdgcn_ballot_w64(want)) {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ms), __float_as_uint(ms), false, false);
        const float full = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
        const bool is_fresh = MAYBE_FRESH && fresh;
        const bool shift_row = is_fresh ? (full > -INFINITY) : (full - mrow > kRescaleLog2);
        float alpha = 1.f;
        if (shift_row) {
          const float mnew = round_m(full);
          if (!is_fresh) alpha = __builtin_amdgcn_exp2f(mrow - mnew);
          mrow = mnew;
          fresh = false;
        }
        set_mneg();  // all lanes (the ballot inside needs the whole wave)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
        // the row sums of queries (l % 16) and (l % 16) + 16 live in lanes 0..15
        const float a0 = __shfl(alpha, l & 15), a1 = __shfl(alpha, (l & 15) + 16);
        lsum[0] *= a0;
        lsum[1] *= a1;
      }
    };
    // p = 2^(s c - m) rounded to FP16 for block nb: the two 16-key B fragments
    auto weights = [&](int nb, h8 (&pf)[2]) {
      const float negm = -mrow;
#pragma unroll
      for (int e = 0; e < 16; ++e) pf[e >> 3][e & 7] = (_Float16)__builtin_amdgcn_exp2f(fmaf(sc[nb][e], c, negm));
    };
    // l += the FP16 weights; O^T += V^T P^T
    auto accumulate = [&](int nb, const h8 (&pf)[2]) {
      lsum = mfma32(ones, pf[0], lsum);
      lsum = mfma32(ones, pf[1], lsum);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const h8 va = vt_frag(vtb, dt, 32 * nb + 16 * s2 + 8 * hf);
          oacc[dt] = mfma32x32(va, pf[s2], oacc[dt]);
        }
    };

    // (head dim 32 with 64-key tiles only: the tile's weights held at once cost a
    // wave per SIMD of occupancy at head dim 64 and with 128-key tiles)
    if constexpr (STEADY) {
      // Steady tiles: the weights are computed from the current row max first, and
      // the rescale test runs on them - a weight above 2^kRescaleLog2 means a score
      // above the max by more than kRescaleLog2 (an overflowing weight is +inf,
      // which counts too; FP16 rounding lets scores up to ~7e-4 above the threshold
      // pass, where the score test below would fire - both keep o = acc / l exact) -
      // as 3-input packed FP16 maxima over the weight registers,
      // NB * 4 instructions instead of the 16 NB FP32 ones over the scores.  Only
      // when it fires (rarely once a row has seen its first keys) are the scores
      // computed again (the K tile is still in LDS; keeping them would cost the
      // registers of a wave per SIMD), the score-based test above run and the
      // weights recomputed.
      static_assert(DT == 1, "one 32-row head-dim tile");
      // The first block's V^T fragments are read before the test: its branch would
      // keep them below it, with their LDS latency in front of the first P V MFMA.
      const h8 va0[2] = {vt_frag(vtb, 0, 8 * hf), vt_frag(vtb, 0, 16 + 8 * hf)};
      h8 pf[NB][2];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if constexpr (PS) {
#pragma unroll
          for (int e = 0; e < 16; ++e) pf[nb][e >> 3][e & 7] = (_Float16)__builtin_amdgcn_exp2f(sc[nb][e]);
        } else {
          weights(nb, pf[nb]);
        }
      }
      typedef _Float16 h2v __attribute__((ext_vector_type(2)));
      auto pair = [&](int k) {  // packed weight pair k of the tile (NB * 8 pairs, one register each)
        const h8 v = pf[k >> 3][(k >> 2) & 1];
        const int w = 2 * (k & 3);
        return h2v{v[w], v[w + 1]};
      };
      h2v pm = __builtin_elementwise_maximum(pair(0), pair(1));
#pragma unroll
      for (int k = 2; k < NB * 8; k += 2)
        pm = __builtin_elementwise_maximum(__builtin_elementwise_maximum(pm, pair(k)), pair(k + 1));
      const float pmax = fmaxf((float)pm[0], (float)pm[1]);
      if (__builtin_amdgcn_ballot_w64(!(pmax <= kRescaleWeight))) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          sc[nb] = f16v{};
#pragma unroll
          for (int st = 0; st < QS; ++st) {
            const h8 ka = *reinterpret_cast<const h8*>(&ksb[(32 * nb + trow) * SH::LDK + 16 * st + 8 * hf]);
            sc[nb] = mfma32x32(ka, qf[st], sc[nb]);
          }
        }
        raise_max();
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) weights(nb, pf[nb]);
      }
      lsum = mfma32(ones, pf[0][0], lsum);
      lsum = mfma32(ones, pf[0][1], lsum);
      oacc[0] = mfma32x32(va0[0], pf[0][0], oacc[0]);
      oacc[0] = mfma32x32(va0[1], pf[0][1], oacc[0]);
#pragma unroll
      for (int nb = 1; nb < NB; ++nb) accumulate(nb, pf[nb]);
    } else {
      // the score-based test, then each block's weights, row sums and P V
      float mx = sc[0][0];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if (EDGE && nb >= nbv) break;
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sc[nb][e]);
      }
      const float ms = mx * c;  // this lane's max of s*c
      const bool want = (MAYBE_FRESH && fresh) || ms - mrow > kRescaleLog2;
      if (__builtin_amdgcn_ballot_w64(want)) {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ms), __float_as_uint(ms), false, false);
        const float full = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
        const bool is_fresh = MAYBE_FRESH && fresh;
        const bool shift_row = is_fresh ? (full > -INFINITY) : (full - mrow > kRescaleLog2);
        float alpha = 1.f;
        if (shift_row) {
          const float mnew = round_m(full);
          if (!is_fresh) alpha = __builtin_amdgcn_exp2f(mrow - mnew);
          mrow = mnew;
          fresh = false;
        }
        set_mneg();  // all lanes (the ballot inside needs the whole wave)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
        const float a0 = __shfl(alpha, l & 15), a1 = __shfl(alpha, (l & 15) + 16);
        lsum[0] *= a0;
        lsum[1] *= a1;
      }
      const float negm = -mrow;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if (EDGE && nb >= nbv) break;
        h8 pf[2];
#pragma unroll
        for (int e = 0; e < 16; ++e) pf[e >> 3][e & 7] = (_Float16)__builtin_amdgcn_exp2f(fmaf(sc[nb][e], c, negm));
        lsum = mfma32(ones, pf[0], lsum);
        lsum = mfma32(ones, pf[1], lsum);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            const h8 va = vt_frag(vtb, dt, 32 * nb + 16 * s2 + 8 * hf);
            oacc[dt] = mfma32x32(va, pf[s2], oacc[dt]);
          }
      }
    }
  };

  // One step per key tile: prefetch the next tile into registers (or copy it into the other
  // LDS buffer by LDS-DMA), process this one, stage the next into the other LDS buffer, one
  // barrier.  Tiles below the
  // workgroup's first query (and inside the sequence) are visible to every query
  // of every wave and run the check-free steady-state body in a loop of their
  // own; the split point is workgroup-uniform, so every wave meets the same
  // barriers.
  // At head dim 32 the steady-state loop runs two tiles per iteration with
  // compile-time buffer indices (odd tile: buffer 1, even tile: buffer 0), so its
  // LDS addresses are a per-lane base plus immediates.
  auto step_in = [&](int tile, int cur, auto first_tag, auto edge_tag) {
    const int kb = tile * KTILE;
    const bool more = tile + 1 < ntiles;
    if constexpr (DMA_KV) {
      if (more) fetch_dma(kb + KTILE, cur ^ 1);
    } else {
      if (more) fetch(kb + KTILE);
    }
    process(kb, ks_lds[cur], vr_lds[cur], kbias[cur], first_tag, edge_tag);
    if constexpr (DMA_KV) {
      wait_copies<0>();
    } else {
      if (more) stash(cur ^ 1);
    }
    __syncthreads();
  };
  auto step = [&](int tile, auto first_tag, auto edge_tag) { step_in(tile, tile & 1, first_tag, edge_tag); };
  const int steady_end = KEYMASK ? 1 : max(1, min(ntiles, (a.causal ? min(q0, S) : S) / KTILE));

  if constexpr (DMA_KV) {
    fetch_dma(0, 0);
    wait_copies<0>();
  } else {
    fetch(0);
    stash(0);
  }
  __syncthreads();
  step(0, std::true_type{}, std::true_type{});
  int tile = 1;
  if constexpr (HD == 32 && KTILE == 64) {
    for (; tile + 1 < steady_end; tile += 2) {
      step_in(tile, 1, std::false_type{}, std::false_type{});
      step_in(tile + 1, 0, std::false_type{}, std::false_type{});
    }
    if (tile < steady_end) step_in(tile++, 1, std::false_type{}, std::false_type{});
  } else {
    // (unrolled, head dim 64 needs two registers more than four waves per SIMD allow)
    for (; tile < steady_end; ++tile) step(tile, std::false_type{}, std::false_type{});
  }
  for (; tile < ntiles; ++tile) step(tile, std::false_type{}, std::true_type{});

  // ---- normalise and store: lane (i, hf) holds head dims 32 dt + 16 s + 8 hf + j in register 8 s + j ----
  const float a0 = __shfl(lsum[0], qi & 15), a1 = __shfl(lsum[1], qi & 15);
  const float lrow = qi < 16 ? a0 : a1;
  float inv = lrow > 0.f ? 1.0f / lrow : 0.f;
  if constexpr (F32IN) inv = ldexpf(inv, vexp);  // o = (sum p v') / l * 2^vexp
  if (q < S) {
    OT* dst = O + (int64_t)q * a.os[2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = oacc[dt][8 * s2 + j] * inv;
        pin_f32x8(v);
        store8(dst + 32 * dt + 16 * s2 + 8 * hf, v);
      }
  }
}

template <int HD, int NW, int KTILE, typename IT, typename OT, bool PS = false>
static hipError_t launch_attn32(const AttnArgs& a0, hipStream_t s) {
  constexpr int QB = 32 * NW;
  const int64_t nqb = (a0.seq + QB - 1) / QB;
  const int64_t grid = nqb * a0.batch * a0.heads;
  // Grouped schedule (see the kernel) when every XCD runs at least 1024 workgroups, i.e.
  // many rounds of its resident workgroups: groups of 8 rows measured fastest at B 64, H 8,
  // S 4096 (833 us against 869 us for the ungrouped order; groups of 4 fetch the fewest
  // bytes but ran 890 us).  With fewer rounds all rows of an XCD are in flight anyway.
  AttnArgs a = a0;
  const int64_t rows = (int64_t)a.batch * a.heads;
  a.group = (rows % 64 == 0 && (rows / 8) * nqb >= 1024) ? 8 : 0;
  if (grid > 0x7fffffff) return hipErrorInvalidConfiguration;
  if (a.key_valid)
    hipLaunchKernelGGL((attention32_kernel<HD, NW, KTILE, IT, OT, true, PS>), dim3((unsigned)grid), dim3(64 * NW), 0, s,
                       a);
  else
    hipLaunchKernelGGL((attention32_kernel<HD, NW, KTILE, IT, OT, false, PS>), dim3((unsigned)grid), dim3(64 * NW), 0,
                       s, a);
  return hipGetLastError();
}

template <int HD, int QT, int KTILE, int NW, typename IT, typename OT>
static hipError_t launch_attn(const AttnArgs& a, hipStream_t s) {
  constexpr int QB = 16 * QT * NW;
  const int64_t nqb = (a.seq + QB - 1) / QB;
  const int64_t grid = nqb * a.batch * a.heads;
  if (grid > 0x7fffffff) return hipErrorInvalidConfiguration;
  if (a.key_valid)
    hipLaunchKernelGGL((attention_kernel<HD, QT, KTILE, NW, IT, OT, true>), dim3((unsigned)grid), dim3(64 * NW), 0,
                       s, a);
  else
    hipLaunchKernelGGL((attention_kernel<HD, QT, KTILE, NW, IT, OT, false>), dim3((unsigned)grid), dim3(64 * NW), 0,
                       s, a);
  return hipGetLastError();
}

// Tile variants (queries per wave x keys per tile x waves per workgroup):
//   1: 16 x 64 x 4     2: 32 x 64 x 4     3: 32 x 128 x 4     4: 32 x 64 x 8     5: 16 x 128 x 4
// and, for head_dim 32 / 64 only, the 32x32 kernel (32 queries per wave):
//   6: 32 x 64 x 4     7: 32 x 64 x 8     8: 32 x 128 x 4
template <int HD, typename IT, typename OT>
static hipError_t attn_variant(int variant, const AttnArgs& a, hipStream_t s) {
  switch (variant) {
    case 1: return launch_attn<HD, 1, 64, 4, IT, OT>(a, s);
    case 2: return launch_attn<HD, 2, 64, 4, IT, OT>(a, s);
    case 3: return launch_attn<HD, 2, 128, 4, IT, OT>(a, s);
    case 4: return launch_attn<HD, 2, 64, 8, IT, OT>(a, s);
    case 5: return launch_attn<HD, 1, 128, 4, IT, OT>(a, s);
    default: return (hipError_t)MPK_EUNSUPPORTED;
  }
}

// hd = 256: one tile shape (16 queries/wave, 32-key tiles, 4 waves), whatever the
// variant id - the K and V^T tiles of larger shapes do not leave room in LDS and
// registers for more than one workgroup per CU.
template <typename IT, typename OT>
static hipError_t attn_variant_256(int variant, const AttnArgs& a, hipStream_t s) {
  if (variant < 1 || variant > 5) return (hipError_t)MPK_EUNSUPPORTED;
  return launch_attn<256, 1, 32, 4, IT, OT>(a, s);
}

// 32x32 variants (head_dim 32 and 64): 6: 4 waves x 64-key tiles  7: 8 waves x 64  8: 4 waves x 128
template <int HD, typename IT, typename OT, bool PS = false>
static hipError_t attn32_variant(int variant, const AttnArgs& a, hipStream_t s) {
  switch (variant) {
    case 6: return launch_attn32<HD, 4, 64, IT, OT, PS>(a, s);
    case 7: return launch_attn32<HD, 8, 64, IT, OT, PS>(a, s);
    case 8: return launch_attn32<HD, 4, 128, IT, OT, PS>(a, s);
    default: return (hipError_t)MPK_EUNSUPPORTED;
  }
}

template <typename IT, typename OT>
static hipError_t attn_dispatch(int variant, const AttnArgs& a, int hd, hipStream_t s) {
  if (variant >= 6) {
    if (hd == 32) return attn32_variant<32, IT, OT>(variant, a, s);
    if (hd == 64) return attn32_variant<64, IT, OT>(variant, a, s);
    return (hipError_t)MPK_EUNSUPPORTED;
  }
  switch (hd) {
    case 8: return attn_variant<8, IT, OT>(variant, a, s);
    case 16: return attn_variant<16, IT, OT>(variant, a, s);
    case 32: return attn_variant<32, IT, OT>(variant, a, s);
    case 64: return attn_variant<64, IT, OT>(variant, a, s);
    case 128: return attn_variant<128, IT, OT>(variant, a, s);
    case 256: return attn_variant_256<IT, OT>(variant, a, s);
    default: return (hipError_t)MPK_EUNSUPPORTED;
  }
}

}  // namespace mpk

using namespace mpk;

// Built-in choice, from MI355X sweeps.  Below 256 keys, and for head dims 128 and
// 256, the 16x16 kernel with 16 queries per wave (variant 1: most workgroups).
// From 256 keys on, head dims 32 and 64 run the 32x32 kernel: 4-wave workgroups
// with 64-key tiles (variant 6), except 8-wave workgroups (variant 7) for
// head_dim 32 at S >= 4096 and for head_dim 64 below 1024 keys.  Head dims 8 and
// 16 take 32 queries per wave from 512 keys (variant 2) and 8-wave workgroups
// from 4096 keys (variant 4).
extern "C" int mpk_attention_auto_variant(int32_t batch, int32_t heads, int32_t seq_len, int32_t head_dim) {
  (void)batch; (void)heads;
  if (head_dim >= 128 || seq_len < 256) return 1;
  if (head_dim == 32) return seq_len >= 4096 ? 7 : 6;
  if (head_dim == 64) return seq_len < 1024 ? 7 : 6;
  return seq_len >= 4096 ? 4 : seq_len >= 512 ? 2 : 1;
}

extern "C" int mpk_causal_attention(const void* q, const void* k, const void* v, void* o, int io_dtype,
                                    int out_dtype, const int64_t* q_strides, const int64_t* k_strides,
                                    const int64_t* v_strides, const int64_t* o_strides, int32_t batch,
                                    int32_t heads, int32_t seq_len, int32_t head_dim, float scale, int causal,
                                    const uint8_t* key_valid, int variant, void* stream) {
  if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides) return MPK_EINVAL;
  if (batch < 0 || heads <= 0 || seq_len < 0) return MPK_EINVAL;
  if ((io_dtype != kF32 && io_dtype != kF16) || (out_dtype != kF32 && out_dtype != kF16)) return MPK_EINVAL;
  if (head_dim != 8 && head_dim != 16 && head_dim != 32 && head_dim != 64 && head_dim != 128 && head_dim != 256)
    return MPK_EUNSUPPORTED;
  const int64_t* st[4] = {q_strides, k_strides, v_strides, o_strides};
  const void* base[4] = {q, k, v, o};
  for (int i = 0; i < 4; ++i) {
    if (st[i][3] != 1) return MPK_EUNSUPPORTED;  // head-dim elements must be contiguous
    const int esz = (i == 3 ? out_dtype : io_dtype) == kF32 ? 4 : 2;
    if ((reinterpret_cast<uintptr_t>(base[i]) & 15u) != 0) return MPK_EALIGN;
    for (int j = 0; j < 3; ++j)
      if ((st[i][j] * esz) % 16 != 0) return MPK_EALIGN;
  }
  if (batch == 0 || seq_len == 0) return MPK_OK;
  if (variant == 0) variant = mpk_attention_auto_variant(batch, heads, seq_len, head_dim);
  if (variant < 1 || variant > 8) return MPK_EUNSUPPORTED;
  AttnArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = o;
  for (int j = 0; j < 4; ++j) {
    a.qs[j] = q_strides[j]; a.ks[j] = k_strides[j]; a.vs[j] = v_strides[j]; a.os[j] = o_strides[j];
  }
  a.key_valid = key_valid;
  a.batch = batch; a.heads = heads; a.seq = seq_len; a.causal = causal ? 1 : 0;
  a.c = scale * 1.4426950408889634f;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  if (io_dtype == kF16)
    e = out_dtype == kF16 ? attn_dispatch<_Float16, _Float16>(variant, a, head_dim, s)
                          : attn_dispatch<_Float16, float>(variant, a, head_dim, s);
  else
    e = out_dtype == kF16 ? attn_dispatch<float, _Float16>(variant, a, head_dim, s)
                          : attn_dispatch<float, float>(variant, a, head_dim, s);
  return (int)e;
}

// q pre-multiplied by scale * log2(e) in FP32 and rounded to FP16 by its producer
// (mpk_linear_qscaled): the 32x32 kernel (head dims 32 and 64, FP16 q / k / v) without the
// per-score scale.  variant 0 picks among 6-8 as mpk_attention_auto_variant does from 256 keys.
extern "C" int mpk_causal_attention_prescaled(const void* q, const void* k, const void* v, void* o, int out_dtype,
                                              const int64_t* q_strides, const int64_t* k_strides,
                                              const int64_t* v_strides, const int64_t* o_strides, int32_t batch,
                                              int32_t heads, int32_t seq_len, int32_t head_dim, int causal,
                                              const uint8_t* key_valid, int variant, void* stream) {
  if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides) return MPK_EINVAL;
  if (batch < 0 || heads <= 0 || seq_len < 0) return MPK_EINVAL;
  if (out_dtype != kF32 && out_dtype != kF16) return MPK_EINVAL;
  if (head_dim != 32 && head_dim != 64) return MPK_EUNSUPPORTED;
  // built-in choice at head dim 32: 8-wave workgroups where their launch runs the grouped
  // schedule (many rounds of workgroups: cfg5's B64 H8 S4096 per microbatch), where the whole
  // cfg5 forward measured 47.50-47.58 ms against 48.18-48.28 ms with 4-wave workgroups in one
  // process on MI355X (the kernel alone had been 783 vs 764 us before the layer chain's tile
  // order; cfg2's S1024 is level); 4-wave workgroups otherwise.  Head dim 64 as
  // mpk_attention_auto_variant.
  if (variant == 0) {
    const int64_t rows = (int64_t)batch * heads, nqb8 = ((int64_t)seq_len + 255) / 256;
    const bool grouped8 = rows % 64 == 0 && (rows / 8) * nqb8 >= 1024;
    variant = head_dim == 32 ? (grouped8 ? 7 : 6) : (seq_len < 1024 ? 7 : 6);
  }
  if (variant < 6 || variant > 8) return MPK_EUNSUPPORTED;
  const int64_t* st[4] = {q_strides, k_strides, v_strides, o_strides};
  const void* base[4] = {q, k, v, o};
  for (int i = 0; i < 4; ++i) {
    if (st[i][3] != 1) return MPK_EUNSUPPORTED;
    const int esz = (i == 3 && out_dtype == kF32) ? 4 : 2;
    if ((reinterpret_cast<uintptr_t>(base[i]) & 15u) != 0) return MPK_EALIGN;
    for (int j = 0; j < 3; ++j)
      if ((st[i][j] * esz) % 16 != 0) return MPK_EALIGN;
  }
  if (batch == 0 || seq_len == 0) return MPK_OK;
  AttnArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = o;
  for (int j = 0; j < 4; ++j) {
    a.qs[j] = q_strides[j]; a.ks[j] = k_strides[j]; a.vs[j] = v_strides[j]; a.os[j] = o_strides[j];
  }
  a.key_valid = key_valid;
  a.batch = batch; a.heads = heads; a.seq = seq_len; a.causal = causal ? 1 : 0;
  a.c = 1.0f;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  if (head_dim == 32)
    e = out_dtype == kF16 ? attn32_variant<32, _Float16, _Float16, true>(variant, a, s)
                          : attn32_variant<32, _Float16, float, true>(variant, a, s);
  else
    e = out_dtype == kF16 ? attn32_variant<64, _Float16, _Float16, true>(variant, a, s)
                          : attn32_variant<64, _Float16, float, true>(variant, a, s);
  return (int)e;
}
