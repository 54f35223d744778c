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
// For FP32 inputs (the reference's TF32 kernel) q, k, v are rounded to FP16 on
// load, which keeps the same 10-bit operand mantissa as TF32.
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
#include "mpk_common.h"

namespace mpk {

// The running max (log2 units) is raised only when a tile exceeds it by more than this.
constexpr float kRescaleLog2 = 8.0f;

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t qs[4], ks[4], vs[4], os[4];  // element strides: batch, head, seq, dim
  const uint8_t* key_valid;           // optional [B, S] (row stride S), nonzero = valid key
  int batch, heads, seq, causal;
  float c;  // scale * log2(e)
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

  const int l = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = l & 15, g = l >> 4;
  const int qw0 = q0 + wave * 16 * QT;       // first query of this wave
  const int qw_last = qw0 + 16 * QT - 1;     // last query of this wave

  // ---- Q fragments (B operand of S^T = K Q^T), kept in registers ----
  // q is pre-multiplied by c = scale*log2(e) in FP32 and split into FP16 hi + lo
  // (hi + lo = q*c to ~2^-22 relative), so two MFMAs give s*c - m directly in
  // the FP32 accumulator (which starts at -m): no per-score scaling FMA, and the
  // exponent argument is more accurate than rounding s*c separately.
  constexpr int QK_STEPS = HP >= 32 ? HP / 32 : 1;
  h8 qh[QT][QK_STEPS], ql[QT][QK_STEPS];
  h4 qh16[QT], ql16[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int q = qw0 + 16 * t + r;
    if constexpr (HP == 16) {
      float v[4] = {0.f, 0.f, 0.f, 0.f};
      if (q < S && 4 * g < HD) {
        const IT* src = Q + (int64_t)q * a.qs[2] + 4 * g;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (float)(_Float16)src[j] * a.c;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        qh16[t][j] = (_Float16)v[j];
        ql16[t][j] = (_Float16)(v[j] - (float)qh16[t][j]);
      }
    } else {
#pragma unroll
      for (int kq = 0; kq < QK_STEPS; ++kq) {
        const h8 raw = q < S ? load8_as_half(Q + (int64_t)q * a.qs[2] + kq * 32 + 8 * g) : zero_h8();
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float v = (float)raw[j] * a.c;
          qh[t][kq][j] = (_Float16)v;
          ql[t][kq][j] = (_Float16)(v - (float)qh[t][kq][j]);
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

  const int kv_end = a.causal ? min(q0 + QB, S) : S;  // keys [0, kv_end) can matter
  const int ntiles = (kv_end + KTILE - 1) / KTILE;

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
      if (c < SH::CHUNKS) kreg[i] = buffer_load8_as_half(kr, key * krow_bytes + col * (uint32_t)sizeof(IT), Kp);
    }
#pragma unroll
    for (int i = 0; i < SH::V_PER_THREAD; ++i) {
      const int c = threadIdx.x + i * NT;
      const int kp = c % (KTILE / 2), col = (c / (KTILE / 2)) * 8;
      if (c < SH::VITEMS) {
        const uint32_t off = 2 * kp * vrow_bytes + col * (uint32_t)sizeof(IT);
        vreg[i][0] = buffer_load8_as_half(vr, off, Vp);
        vreg[i][1] = buffer_load8_as_half(vr, off + vrow_bytes, Vp);
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
  auto process = [&](const int kb, const _Float16* ksb, const _Float16* vtb, const float* kbb) {
    if (a.causal && kb > qw_last) return;  // whole tile is in this wave's future
    const bool need_causal = a.causal && kb + KTILE - 1 > qw0;  // tile straddles this wave's diagonal
    const bool need_bias = KEYMASK || kb + KTILE > S;          // padded keys or keys past the end

    // S^T = K (Q*c)^T - m for KTILE keys x 16*QT queries
    f4 sc[NP][2][QT];  // [key pair][tile in pair][q tile]
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int krow = 32 * p + pair_row(r, tt);
#pragma unroll
        for (int t = 0; t < QT; ++t) {
          const float c0 = fresh[t] ? 0.f : -mrow[t];
          sc[p][tt][t] = f4{c0, c0, c0, c0};
        }
        if constexpr (HP == 16) {
          const h4 ka = *reinterpret_cast<const h4*>(&ksb[krow * SH::LDK + 4 * g]);
#pragma unroll
          for (int t = 0; t < QT; ++t) {
            sc[p][tt][t] = mfma16(ka, qh16[t], sc[p][tt][t]);
            sc[p][tt][t] = mfma16(ka, ql16[t], sc[p][tt][t]);
          }
        } else {
#pragma unroll
          for (int kq = 0; kq < QK_STEPS; ++kq) {
            const h8 ka = *reinterpret_cast<const h8*>(&ksb[krow * SH::LDK + kq * 32 + 8 * g]);
#pragma unroll
            for (int t = 0; t < QT; ++t) {
              sc[p][tt][t] = mfma32(ka, qh[t][kq], sc[p][tt][t]);
              sc[p][tt][t] = mfma32(ka, ql[t][kq], sc[p][tt][t]);
            }
          }
        }
      }

    // Online softmax.  Scores arrive as s*c - mrow.  The running max is only
    // raised when a tile exceeds it by more than kRescaleLog2; otherwise the
    // stale max is kept and p may reach 2^kRescaleLog2.  acc and l share the
    // scale, so o = acc / l is unchanged.  Fresh rows adopt their first finite max.
    h8 pf[QT][NP];  // fp16(P) as the B operand of the PV product, per key pair
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      if (need_causal) {
        // key kb + 32p + 8g + 4tt + i is visible iff it is <= query qw0 + 16t + r
        const int lim = qw0 + 16 * t + r - kb - 8 * g;
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (32 * p + 4 * tt + i > lim) sc[p][tt][t][i] = -INFINITY;
      }
      if (need_bias) {
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[p][tt][t][i] += kbb[32 * p + 8 * g + 4 * tt + i];
      }
      float mx = sc[0][0][t][0];
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[p][tt][t][i]);
      mx = max_over_groups(mx);
      const bool shift_row = fresh[t] ? (mx > -INFINITY) : (mx > kRescaleLog2);
      if (__builtin_amdgcn_ballot_w64(shift_row)) {  // rare after the first tile
        const float shift = shift_row ? mx : 0.f;
        if (shift_row && !fresh[t]) {
          const float alpha = __builtin_amdgcn_exp2f(-shift);
          lsum_acc[t] *= alpha;
#pragma unroll
          for (int dt = 0; dt < SH::DT; ++dt) {
            oacc[t][dt][0] *= alpha;
            oacc[t][dt][1] *= alpha;
          }
        }
        if (shift_row) {
          mrow[t] = fresh[t] ? shift : mrow[t] + shift;
          fresh[t] = false;
        }
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[p][tt][t][i] -= shift;
      }
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) pf[t][p][4 * tt + i] = (_Float16)__builtin_amdgcn_exp2f(sc[p][tt][t][i]);
    }

    // O^T += V^T P^T, and the row sums of P
#pragma unroll
    for (int p = 0; p < NP; ++p) {
#pragma unroll
      for (int t = 0; t < QT; ++t) lsum_acc[t] = mfma32(ones_row, pf[t][p], lsum_acc[t]);
      if constexpr (HP == 16) {
        const h8 va = *reinterpret_cast<const h8*>(&vtb[r * SH::LDV + 32 * p + 8 * g]);
#pragma unroll
        for (int t = 0; t < QT; ++t) oacc[t][0][0] = mfma32(va, pf[t][p], oacc[t][0][0]);
      } else {
#pragma unroll
        for (int dt = 0; dt < SH::DT; ++dt)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            const int drow = 32 * dt + pair_row(r, tt);
            const h8 va = *reinterpret_cast<const h8*>(&vtb[drow * SH::LDV + 32 * p + 8 * g]);
#pragma unroll
            for (int t = 0; t < QT; ++t) oacc[t][dt][tt] = mfma32(va, pf[t][p], oacc[t][dt][tt]);
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
    process(tile * KTILE, ks_lds[cur], vt_lds[cur], kbias[cur]);
    if (more) stash(cur ^ 1);
    __syncthreads();
  }

  // ---- normalise and store ----
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int q = qw0 + 16 * t + r;
    const float lsum = sum_over_groups(lsum_acc[t][0]);
    const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    if (q >= S) continue;
    OT* dst = O + (int64_t)q * a.os[2];
    if constexpr (HP == 16) {
      // lane group g holds d = 4g .. 4g+3
      if (4 * g < HD) {
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[4 * g + i] = (OT)(oacc[t][0][0][i] * inv);
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
        store8(dst + 32 * dt + 8 * g, v);
      }
    }
  }
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

template <typename IT, typename OT>
static hipError_t attn_dispatch(int variant, const AttnArgs& a, int hd, hipStream_t s) {
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

// Built-in choice, from MI355X sweeps: short sequences favour 16 queries per wave
// (more workgroups); long ones 32 queries per wave, and 8-wave workgroups at S >= 4096.
extern "C" int mpk_attention_auto_variant(int32_t batch, int32_t heads, int32_t seq_len, int32_t head_dim) {
  (void)batch; (void)heads;
  if (head_dim >= 128 || seq_len < 512) return 1;
  return seq_len >= 4096 ? 4 : 2;
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
  if (variant < 1 || variant > 5) return MPK_EUNSUPPORTED;
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
