// Whole-layer tail fusion for narrow models (gfx950).
//
// Everything in a pre-LN block after attention is token-local, so one kernel
// takes the attention context of a row tile all the way to the next layer's
// packed QKV projection:
//
//   x'  = fp16(ctx) Wo^T + bo + x                      (FP32)
//   n2  = LN2(x')                                      (FP32 stats, FP16 operand)
//   x'' = fp16(GELU_erf(n2 Win^T + bin)) Wout^T + bout + x'    (FP32)
//   n1  = LN1_next(x'')                                (FP32 stats, FP16 operand)
//   qkv = n1 Wqkv_next^T + bqkv_next                   (FP32 accumulate, FP16 store)
//   (last layer: out = LN_final(x'') in FP32 instead of n1 / qkv)
//
// This is the composition of the reference's kernels
//   _mixed_linear_add_layer_norm_kernel (mixed_precision/triton_linear.py:72-125),
//   _mixed_ffn_add_layer_norm_kernel    (:128-185) and
//   _mixed_linear_kernel                (:16-69, the next layer's QKV projection)
// with exactly the same rounding points; only x'' and qkv (or the final
// output) are written to HBM.  A second entry runs just the last stage for the
// first layer (x -> LN1 -> QKV).
//
// Structure.  Row-owner design: each wave owns 16*TM token rows for the whole
// chain.  Every product is computed transposed with the paired row mapping
// (mpk_common.h), so each stage's output, after its epilogue, is already the
// FP16 B operand of the next product - activations never leave the register
// file.  Wo, Win and Wout are loaded into LDS once per (persistent) workgroup;
// the QKV weights live in LDS when they fit, otherwise each wave streams its
// A fragments from L2.  Workgroups have 8 waves (2 per SIMD) sharing one copy
// of the weights.
#include <atomic>

#include "mpk_common.h"

namespace mpk {

struct TailArgs {
  const _Float16* ctx;  // [M, D] attention context (stage 1 only)
  const float* x;       // [M, D] residual stream in
  const _Float16* wo;   // [D, D]
  const _Float16* bo;   // [D]
  const float* g2;      // LN2 gamma / beta
  const float* be2;
  const _Float16* win;   // [F, D]
  const _Float16* bin;   // [F]
  const _Float16* wout;  // [D, F]
  const _Float16* bout;  // [D]
  const float* g1;       // next LayerNorm (LN1 of the next layer, or the final norm)
  const float* be1;
  const _Float16* wqkv;  // [3D, D] next layer's packed QKV (unless LAST)
  const _Float16* bqkv;  // [3D]
  float* x_out;          // [M, D] residual stream out (stage 1 only)
  void* out;             // qkv FP16 [M, 3D], or final normalized FP32 [M, D] when LAST
  int64_t m;
  int f;
  float eps2, eps1;
  // attention stage (mpk_attention_layer_tail only): this layer's packed QKV [m, 3d] FP16
  // (read, never written: the kernel writes the next layer's into `out`), the sequence
  // length, causality and scale * log2(e)
  const _Float16* qkv_in;
  int seq, causal;
  float attn_c;
  // the next QKV's q columns [0, D) multiplied by q_scale in FP32 before the FP16 rounding
  // (q_on != 0: mpk_layer_tail_qscaled / mpk_layernorm_qkv_qscaled, for the pre-scaled attention)
  int q_on;
  float q_scale;
};

constexpr int kLdsBudget = 160 * 1024;

// Where the next layer's QKV weights live.
//   kQkvLds: in LDS; every wave projects its own rows (row-owner).
//   kQkvReg: stationary in registers, wave w holding output columns
//            [w*3D/8, (w+1)*3D/8); the normalized rows of the whole workgroup
//            are exchanged through LDS and every wave projects all of them.
enum QkvMode : int { kQkvLds = 1, kQkvReg = 2 };

// W: waves per workgroup (8, or 4 where 8-wave tiles would leave CUs idle).
// Row strides: 16x16x32 fragment reads (lane r of a 16-lane group reads row R0 + r, the
// four groups four consecutive 16-byte chunks) count no LDS bank conflicts on gfx950 when
// the stride is an odd multiple of 32 bytes, and two-way conflicts when it is an odd
// multiple of 16 bytes (measured with SQ_LDS_BANK_CONFLICT).  D + 16 and F + 16 halves are
// odd multiples of 32 bytes for every supported width (multiples of 32).  Weight rows are
// stored at LDS row w_slot(row), so the 16 rows of a fragment are consecutive.
// ATTN (the fused attention + tail kernel): the parameters follow the weights and the
// attention stage's tiles overlay the QKV row ring, which is idle while attention runs.
template <int D, int F, int TM, bool STAGE1, bool QKV, int QMODE, int W, bool ATTN = false>
struct TailShape {
  static constexpr int LDD = D + 16;  // row stride of [*, D] tiles (halves)
  static constexpr int LDF = F + 16;  // row stride of Wout [D, F] (halves)
  static constexpr int WO = 0;
  static constexpr int WIN = WO + (STAGE1 ? D * LDD : 0);
  static constexpr int WOUT = WIN + (STAGE1 ? F * LDD : 0);
  static constexpr int WQKV = WOUT + (STAGE1 ? D * LDF : 0);
  static constexpr int NBUF = WQKV + (QKV && QMODE == kQkvLds ? 3 * D * LDD : 0);
  static constexpr int TOTAL = NBUF + (QKV && QMODE == kQkvReg ? 16 * TM * W * LDD : 0);
  // Small per-feature parameters, staged once per workgroup as FP32 after the
  // FP16 region (offsets in floats): b_o, LN2 gamma/beta, b_in, b_out (STAGE1),
  // the next LayerNorm's gamma/beta, and b_qkv (QKV).
  static constexpr int P_BO = 0;
  static constexpr int P_G2 = P_BO + (STAGE1 ? D : 0);
  static constexpr int P_BE2 = P_G2 + (STAGE1 ? D : 0);
  static constexpr int P_BIN = P_BE2 + (STAGE1 ? D : 0);
  static constexpr int P_BOUT = P_BIN + (STAGE1 ? F : 0);
  static constexpr int P_G1 = P_BOUT + (STAGE1 ? D : 0);
  static constexpr int P_BE1 = P_G1 + D;
  static constexpr int P_BQKV = P_BE1 + D;
  static constexpr int NPARAM = P_BQKV + (QKV ? 3 * D : 0);
  static constexpr int RING_HALVES = TOTAL - NBUF;                                 // QKV row ring
  static constexpr int PARAM_OFF = ((ATTN ? NBUF : TOTAL) + 7) / 8 * 8;            // halves; 16-byte aligned
  static constexpr int RING = ATTN ? PARAM_OFF + (2 * NPARAM + 7) / 8 * 8 : NBUF;  // halves
  static constexpr int BYTES = ATTN ? (RING + RING_HALVES) * 2 : PARAM_OFF * 2 + NPARAM * 4;
  static constexpr int ATT_OFF_BYTES = RING * 2;  // the attention tiles (ATTN only)
};

// Two-phase staging of a [ROWS, COLS] FP16 matrix into LDS (row stride LD, row j at
// LDS row w_slot(j)): load() issues all of this thread's global reads, store() writes
// them to LDS, so the reads of every staged array can be in flight together.
template <int ROWS, int COLS, int LD, bool ON, int NT>
struct MatStage {
  static_assert(!ON || ROWS % 32 == 0, "w_slot permutes rows within groups of 32");
  static constexpr int CPR = COLS / 8;
  static constexpr int CHUNKS = ON ? ROWS * CPR : 0;
  static constexpr int PER = ON ? (CHUNKS + NT - 1) / NT : 1;
  h8 v[PER];
  __device__ __forceinline__ void load(const _Float16* src) {
    if constexpr (ON) {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int c = threadIdx.x + i * NT;
        if (c < CHUNKS) v[i] = *reinterpret_cast<const h8*>(&src[(int64_t)(c / CPR) * COLS + (c % CPR) * 8]);
      }
    }
  }
  __device__ __forceinline__ void store(_Float16* dst) const {
    if constexpr (ON) {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int c = threadIdx.x + i * NT;
        if (c < CHUNKS) *reinterpret_cast<h8*>(&dst[w_slot(c / CPR) * LD + (c % CPR) * 8]) = v[i];
      }
    }
  }
};

// Two-phase staging of n (1 <= n <= 2 NT) FP16 or FP32 parameters as FP32, up to two
// per thread.  The reads are unconditional (threads past n re-read element n - 1), so
// no branch separates them from the other prologue reads.
template <typename T, int NT>
struct ParamStage {
  T v[2];
  __device__ __forceinline__ void load(const T* src, int n) {
    v[0] = src[min((int)threadIdx.x, n - 1)];
    v[1] = src[min((int)threadIdx.x + NT, n - 1)];
  }
  __device__ __forceinline__ void store(float* dst, int n) const {
    if ((int)threadIdx.x < n) dst[threadIdx.x] = (float)v[0];
    if ((int)threadIdx.x + NT < n) dst[threadIdx.x + NT] = (float)v[1];
  }
};

// 8 consecutive FP32 parameters from LDS.
__device__ __forceinline__ void lds8(const float* p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// Row statistics of v (lane holds one row, features 32p + 8g + j; the row is spread over the 4 lane groups).
template <int PN>
__device__ __forceinline__ void row_stats(const float (&v)[PN][8], float inv_d, float eps, float& mean, float& rstd) {
  float sum = 0.f;
#pragma unroll
  for (int p = 0; p < PN; ++p)
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += v[p][j];
  mean = sum_over_groups(sum) * inv_d;
  float sq = 0.f;
#pragma unroll
  for (int p = 0; p < PN; ++p)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float c = v[p][j] - mean;
      sq += c * c;
    }
  rstd = rsqrtf(sum_over_groups(sq) * inv_d + eps);
}

// Per-tile inputs of one wave, prefetched one tile ahead.
template <int D, int TM, bool STAGE1>
struct TileIn {
  h8 ctx[STAGE1 ? TM : 1][D / 32];
  float x[TM][D / 32][8];
};

template <int D, int TM, bool STAGE1, bool LOAD_CTX = STAGE1>
__device__ __forceinline__ void load_tile(TileIn<D, TM, STAGE1>& in, const TailArgs& a, int64_t m0, int r, int g) {
  constexpr int PN = D / 32;
  typedef float v4 __attribute__((ext_vector_type(4)));
  // buffer resources over the rows that exist: rows past M read as zeros
  const uint32_t rows = (uint32_t)(a.m - m0 <= 0 ? 0 : (a.m - m0 < 16 * TM ? a.m - m0 : 16 * TM));
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x + m0 * D, rows * (uint32_t)(D * 4));
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    const uint32_t row = (uint32_t)(16 * t + r);
    if constexpr (STAGE1 && LOAD_CTX) {
      const __amdgpu_buffer_rsrc_t crs = make_rsrc(a.ctx + m0 * D, rows * (uint32_t)(D * 2));
#pragma unroll
      for (int ks = 0; ks < PN; ++ks)
        in.ctx[t][ks] = buffer_load8_as_half(crs, (row * D + ks * 32 + 8 * g) * 2u, a.ctx);
    }
#pragma unroll
    for (int p = 0; p < PN; ++p) {
      const uint32_t off = (row * D + 32 * p + 8 * g) * 4u;
      const v4 lo = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
      const v4 hi = __builtin_bit_cast(v4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off + 16, 0, 0));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        in.x[t][p][j] = lo[j];
        in.x[t][p][4 + j] = hi[j];
      }
    }
  }
}

// ---- attention stage (head dim HD = 32 or 16) of the fused attention + layer-tail kernel ----
// The context of a wave's 16 TM rows, computed in the kernel instead of read from HBM: per
// head, the arithmetic of attention_kernel<HD, TM, 64, W, FP16 in/out, no key mask>
// (attention.hip) - q c split into FP16 hi + lo, S^T = K (q c)^T - m on 16x16x32 (hd 32)
// or 16x16x16 (hd 16) MFMAs (the accumulator starts at -m), a running max raised lazily
// (by more than kRescaleLog2 only), p = exp2(.) rounded to FP16, l and O^T = V^T P^T by
// MFMAs, o = fp16(O / l) - over the same 64-key tiles, so the context is bit-identical to
// that kernel's output.  It ends as the out-projection's B operand: lane (r, g) holds
// features 32 ks + 8g .. +7 of row 16 t + r in ctx[t][ks].  At hd 32 that is where the
// PV product leaves head ks; at hd 16 (lane group g holds dims 4g .. 4g+3 of a head) the
// wave passes its rows through a private LDS area.  All rows of the workgroup lie in one
// sequence (the launcher checks seq % rows == 0).
// A step is one 64-key tile of every head: the workgroup's rows are few (64), so a step per
// (head, tile) would leave each step bound by a memory latency; a step per tile exposes one
// latency per tile at most, and the heads' softmax chains run interleaved in one wave.  The
// tiles go through NB LDS buffers (2 where they fit beside the weights, else 1 with the
// next tile held in registers across the step).
constexpr int kAttnKT = 64;                     // keys per tile
constexpr int kAttnLDV = kAttnKT + 8;           // V^T tile row stride (halves)
template <int HD>
struct AttnTile {
  static constexpr int LDK = HD + 8;            // K tile row stride (halves; 16-byte padded)
  static constexpr int KBUF = kAttnKT * LDK;    // halves per K tile of one head
  static constexpr int VBUF = HD * kAttnLDV;    // halves per V^T tile of one head
};
// bytes of one buffer: K and V^T tiles of every head, then the key bias [KT] (floats)
template <int D, int HD>
constexpr int attn_buf_bytes() {
  return (D / HD) * (AttnTile<HD>::KBUF + AttnTile<HD>::VBUF) * 2 + kAttnKT * 4;
}
// hd 16: each wave's rows of the context (FP16), after the buffers
template <int D, int HD, int TM, int W>
constexpr int attn_xchg_bytes() { return HD == 16 ? W * 16 * TM * D * 2 : 0; }

// Registers of the attention stage's global reads: one K / V tile of every head with its
// key bias, and the wave's raw queries.  The queries are read (and split) before the first
// tile is requested; issuing the first tile's reads earlier, ahead of the weight prologue,
// measured slower at d_model 128 (registers held across the prologue push the
// register-resident QKV weights into AGPRs).
template <int D, int HD, int TM, int W>
struct AttnRegs {
  static constexpr int H = D / HD;
  static constexpr int NT = 64 * W;
  static constexpr int KT = kAttnKT;
  static constexpr int CPR = D / 8;                    // 16-byte chunks of a key's K (or V) row
  static constexpr int CHUNKS = KT * CPR;              // K tile: one chunk per item
  static constexpr int PER_THREAD = (CHUNKS + NT - 1) / NT;
  static constexpr int VITEMS = (KT / 2) * CPR;        // V tile: a key pair x one chunk per item
  static constexpr int V_PER_THREAD = (VITEMS + NT - 1) / NT;
  static constexpr int U = H * TM;                     // row tiles u = h TM + t
  h8 kreg[PER_THREAD], vreg[V_PER_THREAD][2];
  h8 qraw[HD == 32 ? U : 1];
  h4 qraw16[HD == 16 ? U : 1];
  float breg;

  // K and V rows kb .. kb + KT - 1 of every head of the sequence at seq (S positions)
  __device__ __forceinline__ void fetch(const _Float16* seq, int S, int kb) {
    const uint32_t row_bytes = (uint32_t)(3 * D * 2);
    const _Float16* Kp = seq + (int64_t)kb * (3 * D) + D;
    const _Float16* Vp = Kp + D;
    const uint32_t rows = (uint32_t)min(KT, S - kb);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(Kp, rows * row_bytes);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(Vp, rows * row_bytes);
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int cc = threadIdx.x + i * NT;
      const int key = cc / CPR, col = (cc % CPR) * 8;
      if (cc < CHUNKS) kreg[i] = buffer_load8_as_half(kr, key * row_bytes + col * 2u, Kp);
    }
#pragma unroll
    for (int i = 0; i < V_PER_THREAD; ++i) {
      const int cc = threadIdx.x + i * NT;
      const int kp = cc % (KT / 2), col = (cc / (KT / 2)) * 8;
      if (cc < VITEMS) {
        const uint32_t off = 2 * kp * row_bytes + col * 2u;
        vreg[i][0] = buffer_load8_as_half(vr, off, Vp);
        vreg[i][1] = buffer_load8_as_half(vr, off + row_bytes, Vp);
      }
    }
    breg = kb + (int)threadIdx.x < S ? 0.f : -INFINITY;
  }
  // lane (r, g): query row qw0 + 16 t + r of head h, for u = h TM + t: dims 8g .. 8g + 7
  // (hd 32) or 4g .. 4g + 3 (hd 16)
  __device__ __forceinline__ void load_q(const _Float16* seq, int S, int qw0, int r, int g) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int q = qw0 + 16 * (u % TM) + r;
      const _Float16* src = seq + (int64_t)q * (3 * D) + HD * (u / TM);
      if constexpr (HD == 32) {
        qraw[u] = q < S ? *reinterpret_cast<const h8*>(src + 8 * g) : zero_h8();
      } else {
        h4 z;
#pragma unroll
        for (int j = 0; j < 4; ++j) z[j] = (_Float16)0.0f;
        qraw16[u] = q < S ? *reinterpret_cast<const h4*>(src + 4 * g) : z;
      }
    }
  }
};

template <int D, int HD, int TM, int W, int NB>
__device__ __forceinline__ void tail_attention(const TailArgs& a, unsigned char* att_lds, int64_t wg0,
                                               h8 (&ctx)[TM][D / 32]) {
  static_assert(NB == 1 || NB == 2, "one or two tile buffers");
  static_assert(HD == 16 || HD == 32, "head dim");
  constexpr int H = D / HD;
  constexpr int NT = 64 * W;
  constexpr int ROWS = 16 * TM * W;
  constexpr int KT = kAttnKT;
  constexpr int NP = KT / 32;                          // key pairs per tile
  using R = AttnRegs<D, HD, TM, W>;
  using AT = AttnTile<HD>;
  R st;
  constexpr int CPR = R::CPR, CHUNKS = R::CHUNKS, PER_THREAD = R::PER_THREAD;
  constexpr int VITEMS = R::VITEMS, V_PER_THREAD = R::V_PER_THREAD;
  constexpr int BUF = attn_buf_bytes<D, HD>();
  auto ks_of = [&](int buf, int h) {
    return reinterpret_cast<_Float16*>(att_lds + buf * BUF) + h * AT::KBUF;
  };
  auto vt_of = [&](int buf, int h) {
    return reinterpret_cast<_Float16*>(att_lds + buf * BUF) + H * AT::KBUF + h * AT::VBUF;
  };
  auto kbias_of = [&](int buf) {
    return reinterpret_cast<float*>(reinterpret_cast<_Float16*>(att_lds + buf * BUF) + H * (AT::KBUF + AT::VBUF));
  };

  const int S = a.seq;
  const int64_t bseq = wg0 / S;
  const int pos0 = (int)(wg0 - bseq * S);              // the workgroup's first position
  const int l = threadIdx.x & 63, wave = wave_id();
  const int r = l & 15, g = l >> 4;
  const int qw0 = pos0 + wave * 16 * TM;               // first query of this wave
  const int qw_last = qw0 + 16 * TM - 1;
  const int kv_end = a.causal ? min(pos0 + ROWS, S) : S;
  const int ntiles = (kv_end + KT - 1) / KT;
  const _Float16* seq = a.qkv_in + bseq * (int64_t)S * (3 * D);
  const float c = a.attn_c;

  h8 ones_row;  // row 0 of the row-sum product's A operand: all ones
#pragma unroll
  for (int j = 0; j < 8; ++j) ones_row[j] = r == 0 ? (_Float16)1.0f : (_Float16)0.0f;

  auto stash = [&](int buf) {  // K row-major and V transposed, per head
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int cc = threadIdx.x + i * NT;
      if (cc < CHUNKS) {
        const int key = cc / CPR, col = (cc % CPR) * 8;
        *reinterpret_cast<h8*>(&ks_of(buf, col / HD)[key * AT::LDK + col % HD]) = st.kreg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < V_PER_THREAD; ++i) {
      const int cc = threadIdx.x + i * NT;
      if (cc < VITEMS) {
        const int kp = cc % (KT / 2), col = (cc / (KT / 2)) * 8;
        _Float16* vt = vt_of(buf, col / HD);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          typedef _Float16 h2 __attribute__((ext_vector_type(2)));
          h2 pair;
          pair[0] = st.vreg[i][0][j];
          pair[1] = st.vreg[i][1][j];
          *reinterpret_cast<h2*>(&vt[(col % HD + j) * kAttnLDV + 2 * kp]) = pair;
        }
      }
    }
    if (threadIdx.x < KT) kbias_of(buf)[threadIdx.x] = st.breg;
  };

  // Row tiles u = h TM + t (head h, rows 16 t ..): every step below runs over all of them,
  // so a wave has H TM independent chains (it is alone on its SIMD at these sizes).
  constexpr int U = H * TM;
  constexpr int DT = HD == 32 ? 2 : 1;                 // O^T accumulators per row tile
  // q c in FP32, split into FP16 hi + lo.  Every FP32 value that is then converted to FP16
  // (q c here, o / l at the end) is pinned first (pin_f32), as in attention_kernel, so both
  // round to FP32 and then to FP16.
  st.load_q(seq, S, qw0, r, g);
  h8 qh[HD == 32 ? U : 1], ql[HD == 32 ? U : 1];
  h4 qh16[HD == 16 ? U : 1], ql16[HD == 16 ? U : 1];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if constexpr (HD == 32) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = (float)st.qraw[u][j] * c;
      pin_f32x8(v);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        qh[u][j] = (_Float16)v[j];
        ql[u][j] = (_Float16)(v[j] - (float)qh[u][j]);
      }
    } else {
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = (float)st.qraw16[u][j] * c;
      pin_f32x4(v);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        qh16[u][j] = (_Float16)v[j];
        ql16[u][j] = (_Float16)(v[j] - (float)qh16[u][j]);
      }
    }
  }
  float mrow[U];
  bool fresh[U];
  f4 oacc[U][DT], lsum_acc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    mrow[u] = 0.f;
    fresh[u] = true;
    lsum_acc[u] = zero4();
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[u][dt] = zero4();
  }

  // one key tile of every head: S^T, online softmax, O^T += V^T P^T (attention_kernel's process)
  auto process_all = [&](const int kb, const int buf, auto first_tag) {
    constexpr bool MAYBE_FRESH = decltype(first_tag)::value;
    if (a.causal && kb > qw_last) return;  // whole tile is in this wave's future
    const float* kbb = kbias_of(buf);
    const int npv = a.causal ? min(NP, (qw_last - kb) / 32 + 1) : NP;
    const bool need_causal = a.causal && kb + 32 * npv - 1 > qw0;
    const bool need_bias = kb + KT > S;
    f4 sc[NP][2][U];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      if (p >= npv) break;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int krow = 32 * p + pair_row(r, tt);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float c0 = (MAYBE_FRESH && fresh[u]) ? 0.f : -mrow[u];
          sc[p][tt][u] = f4{c0, c0, c0, c0};
        }
        if constexpr (HD == 32) {
          h8 ka[H];
#pragma unroll
          for (int h = 0; h < H; ++h) ka[h] = *reinterpret_cast<const h8*>(&ks_of(buf, h)[krow * AT::LDK + 8 * g]);
#pragma unroll
          for (int u = 0; u < U; ++u) {
            sc[p][tt][u] = mfma32(ka[u / TM], qh[u], sc[p][tt][u]);
            sc[p][tt][u] = mfma32(ka[u / TM], ql[u], sc[p][tt][u]);
          }
        } else {
          h4 ka[H];
#pragma unroll
          for (int h = 0; h < H; ++h) ka[h] = *reinterpret_cast<const h4*>(&ks_of(buf, h)[krow * AT::LDK + 4 * g]);
#pragma unroll
          for (int u = 0; u < U; ++u) {
            sc[p][tt][u] = mfma16(ka[u / TM], qh16[u], sc[p][tt][u]);
            sc[p][tt][u] = mfma16(ka[u / TM], ql16[u], sc[p][tt][u]);
          }
        }
      }
    }
    if (need_causal) {
      const int pl = npv - 1;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int lim = qw0 + 16 * (u % TM) + r - kb - 32 * pl - 8 * g;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          if (p != pl) continue;
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (4 * tt + i > lim) sc[p][tt][u][i] = -INFINITY;
        }
      }
    }
    if (need_bias) {
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        if (p >= npv) break;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[p][tt][u][i] += kbb[32 * p + 8 * g + 4 * tt + i];
      }
    }
    float pm[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float mx = sc[0][0][u][0];
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        if (p >= npv) break;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[p][tt][u][i]);
      }
      pm[u] = mx;
    }
    // a row tile that needs no shift gets shift 0 below (x - 0 == x), so testing every head
    // at once leaves each head's arithmetic as attention_kernel's
    bool any_shift = false;
#pragma unroll
    for (int u = 0; u < U; ++u) any_shift |= (MAYBE_FRESH && fresh[u]) || pm[u] > kRescaleLog2;
    if (__builtin_amdgcn_ballot_w64(any_shift)) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float mx = max_over_groups(pm[u]);
        const bool is_fresh = MAYBE_FRESH && fresh[u];
        const bool shift_row = is_fresh ? (mx > -INFINITY) : (mx > kRescaleLog2);
        const float shift = shift_row ? mx : 0.f;
        if (shift_row && !is_fresh) {
          const float alpha = __builtin_amdgcn_exp2f(-shift);
          lsum_acc[u] *= alpha;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) oacc[u][dt] *= alpha;
        }
        if (shift_row) {
          mrow[u] = is_fresh ? shift : mrow[u] + shift;
          fresh[u] = false;
        }
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          if (p >= npv) break;
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[p][tt][u][i] -= shift;
        }
      }
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      if (p >= npv) break;
      h8 pf[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) pf[u][4 * tt + i] = (_Float16)__builtin_amdgcn_exp2f(sc[p][tt][u][i]);
#pragma unroll
      for (int u = 0; u < U; ++u) lsum_acc[u] = mfma32(ones_row, pf[u], lsum_acc[u]);
      if constexpr (HD == 32) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int drow = pair_row(r, tt);
          h8 va[H];
#pragma unroll
          for (int h = 0; h < H; ++h) va[h] = *reinterpret_cast<const h8*>(&vt_of(buf, h)[drow * kAttnLDV + 32 * p + 8 * g]);
#pragma unroll
          for (int u = 0; u < U; ++u) oacc[u][tt] = mfma32(va[u / TM], pf[u], oacc[u][tt]);
        }
      } else {
        h8 va[H];
#pragma unroll
        for (int h = 0; h < H; ++h) va[h] = *reinterpret_cast<const h8*>(&vt_of(buf, h)[r * kAttnLDV + 32 * p + 8 * g]);
#pragma unroll
        for (int u = 0; u < U; ++u) oacc[u][0] = mfma32(va[u / TM], pf[u], oacc[u][0]);
      }
    }
  };

  // the first tile is requested after the queries; the caller's previous LDS use of this
  // area (the QKV row ring) must be finished before it is stashed
  st.fetch(seq, S, 0);
  __syncthreads();
  stash(0);
  __syncthreads();
  for (int tile = 0; tile < ntiles; ++tile) {
    const bool more = tile + 1 < ntiles;
    const int buf = NB == 2 ? (tile & 1) : 0;
    if (more) st.fetch(seq, S, (tile + 1) * KT);
    if (tile == 0)
      process_all(0, buf, std::true_type{});
    else
      process_all(tile * KT, buf, std::false_type{});
    if (more) {
      if constexpr (NB == 1) __syncthreads();  // every wave is done with the buffer
      stash(NB == 2 ? buf ^ 1 : 0);
    }
    __syncthreads();  // the stashed tile is visible; the last one also frees the area
  }
  if constexpr (HD == 32) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float lsum = sum_over_groups(lsum_acc[u][0]);
      const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
      float o[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[i] = oacc[u][0][i] * inv;
        o[4 + i] = oacc[u][1][i] * inv;
      }
      pin_f32x8(o);
#pragma unroll
      for (int i = 0; i < 8; ++i) ctx[u % TM][u / TM][i] = (_Float16)o[i];
    }
  } else {
    // lane (r, g) holds dims 4g .. 4g+3 of head h for row 16 t + r: through this wave's LDS rows
    _Float16* xw = reinterpret_cast<_Float16*>(att_lds + NB * BUF) + wave * (16 * TM * D);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float lsum = sum_over_groups(lsum_acc[u][0]);
      const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
      float of[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) of[i] = oacc[u][0][i] * inv;
      pin_f32x4(of);
      h4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = (_Float16)of[i];
      *reinterpret_cast<h4*>(&xw[(16 * (u % TM) + r) * D + HD * (u / TM) + 4 * g]) = o;
    }
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int ks = 0; ks < D / 32; ++ks)
        ctx[t][ks] = *reinterpret_cast<const h8*>(&xw[(16 * t + r) * D + 32 * ks + 8 * g]);
  }
}

// LDS of the fused kernel: two attention buffers where they fit, else one
template <int D, int F, int TM, bool QKV, int QMODE, int W, int AHD>
constexpr int attn_nbuf() {
  using SH = TailShape<D, F, TM, true, QKV, QMODE, W, true>;
  return SH::ATT_OFF_BYTES + 2 * attn_buf_bytes<D, AHD>() + attn_xchg_bytes<D, AHD, TM, W>() <= kLdsBudget ? 2 : 1;
}
template <int D, int F, int TM, bool QKV, int QMODE, int W, int AHD>
constexpr int attn_lds_bytes() {
  using SH = TailShape<D, F, TM, true, QKV, QMODE, W, true>;
  constexpr int att = SH::ATT_OFF_BYTES + attn_nbuf<D, F, TM, QKV, QMODE, W, AHD>() * attn_buf_bytes<D, AHD>() +
                      attn_xchg_bytes<D, AHD, TM, W>();
  return att > SH::BYTES ? att : SH::BYTES;
}

// AHD: 0, or the head dim (16, 32) of the attention stage computed in the kernel.
template <int D, int F, int TM, bool STAGE1, bool LAST, int QMODE, int W, int AHD = 0>
__global__ __launch_bounds__(64 * W) void layer_tail_kernel(TailArgs a) {
  constexpr bool ATTN = AHD != 0;
  static_assert(!ATTN || STAGE1, "the attention stage feeds the out-projection");
  constexpr bool QKV = !LAST;
  constexpr int NT = 64 * W;
  using SH = TailShape<D, F, TM, STAGE1, QKV, QMODE, W, ATTN>;
  constexpr int PN = D / 32;   // feature pairs of a D-wide row
  constexpr int KS = D / 32;   // k-steps over D
  constexpr int FQ = F / 32;   // hidden feature pairs
  constexpr int QP = 3 * D / 32;
  constexpr int ROWS = 16 * TM * W;
  constexpr int QNW = 3 * D / W;           // QKV columns per wave (register mode)
  constexpr int QNT = QNW / 16;            // 16-column tiles per wave (register mode)
  static_assert(D % 32 == 0 && F % 32 == 0, "shape");
  static_assert(QMODE != kQkvReg || QNT * 16 * W == 3 * D, "register mode needs 3D/16 divisible by W");

  extern __shared__ __align__(16) _Float16 lds[];

  const int l = threadIdx.x & 63, wave = wave_id();
  const int r = l & 15, g = l >> 4;

  // Prologue: every global read (weights, parameters, the register-resident QKV
  // weights) is issued before the first LDS write, so it costs one memory latency.
  static_assert(3 * D <= 2 * NT && F <= 2 * NT, "two parameters per thread");
  MatStage<D, D, SH::LDD, STAGE1, NT> s_wo;
  MatStage<F, D, SH::LDD, STAGE1, NT> s_win;
  MatStage<D, F, SH::LDF, STAGE1, NT> s_wout;
  MatStage<3 * D, D, SH::LDD, QKV && QMODE == kQkvLds, NT> s_wqkv;
  // Biases, gammas and betas live in LDS for the whole kernel: read inside the
  // per-tile dependency chain, global loads would put a memory latency between
  // every product and its epilogue.
  ParamStage<_Float16, NT> p_bo, p_bin, p_bout, p_bqkv;
  ParamStage<float, NT> p_g2, p_be2, p_g1, p_be1;
  if constexpr (STAGE1) {
    p_bo.load(a.bo, D);
    p_g2.load(a.g2, D);
    p_be2.load(a.be2, D);
    p_bin.load(a.bin, F);
    p_bout.load(a.bout, D);
  }
  p_g1.load(a.g1, D);
  p_be1.load(a.be1, D);
  if constexpr (QKV) p_bqkv.load(a.bqkv, 3 * D);
  s_wo.load(a.wo);
  s_win.load(a.win);
  s_wout.load(a.wout);
  s_wqkv.load(a.wqkv);
  h8 wq[QKV && QMODE == kQkvReg ? QNT : 1][KS];
  if constexpr (QKV && QMODE == kQkvReg) {
#pragma unroll
    for (int nt = 0; nt < QNT; ++nt)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        wq[nt][ks] = *reinterpret_cast<const h8*>(a.wqkv + (int64_t)(QNW * wave + 16 * nt + r) * D + ks * 32 + 8 * g);
  }
  float* prm = reinterpret_cast<float*>(lds + SH::PARAM_OFF);
  if constexpr (STAGE1) {
    p_bo.store(prm + SH::P_BO, D);
    p_g2.store(prm + SH::P_G2, D);
    p_be2.store(prm + SH::P_BE2, D);
    p_bin.store(prm + SH::P_BIN, F);
    p_bout.store(prm + SH::P_BOUT, D);
  }
  p_g1.store(prm + SH::P_G1, D);
  p_be1.store(prm + SH::P_BE1, D);
  if constexpr (QKV) p_bqkv.store(prm + SH::P_BQKV, 3 * D);
  s_wo.store(lds + SH::WO);
  s_win.store(lds + SH::WIN);
  s_wout.store(lds + SH::WOUT);
  s_wqkv.store(lds + SH::WQKV);
  __syncthreads();

  const float inv_d = 1.0f / (float)D;
  const int64_t M = a.m;
  const int64_t ntiles = (M + ROWS - 1) / ROWS;

  int64_t tile = blockIdx.x;
  TileIn<D, TM, STAGE1> cur;
  load_tile<D, TM, STAGE1, !ATTN>(cur, a, tile * ROWS + wave * 16 * TM, r, g);

  for (; tile < ntiles; tile += gridDim.x) {
    const int64_t wg0 = tile * ROWS;
    const int64_t m0 = wg0 + wave * 16 * TM;
    if constexpr (ATTN) {
      tail_attention<D, AHD, TM, W, attn_nbuf<D, F, TM, QKV, QMODE, W, AHD>()>(
          a, reinterpret_cast<unsigned char*>(lds) + SH::ATT_OFF_BYTES, wg0, cur.ctx);
    }
    // rows of this wave / workgroup that exist (stores to the others are dropped by the buffer resource)
    const uint32_t wrows = (uint32_t)(M - m0 <= 0 ? 0 : (M - m0 < 16 * TM ? M - m0 : 16 * TM));
    const uint32_t grows = (uint32_t)(M - wg0 < ROWS ? M - wg0 : ROWS);

    // xr: the residual stream of this wave's rows (lane holds row m0+16t+r, features 32p+8g+j)
    float xr[TM][PN][8];
    if constexpr (STAGE1) {
      // ---- out-projection + residual + LN2 ----
      h8 n2f[TM][KS];
#pragma unroll
      for (int t = 0; t < TM; ++t) {
        f4 acc[PN][2];
#pragma unroll
        for (int p = 0; p < PN; ++p) acc[p][0] = acc[p][1] = zero4();
        // the bias is requested ahead of the products, so its LDS latency is hidden by them
        float bv[PN][8];
#pragma unroll
        for (int p = 0; p < PN; ++p) lds8(prm + SH::P_BO + 32 * p + 8 * g, bv[p]);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          // the weight fragments of one k-step for every output pair are read before its
          // MFMAs (one LDS latency per group), which then feed 2 PN independent chains
          h8 w[PN][2];
#pragma unroll
          for (int p = 0; p < PN; ++p)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
              w[p][tt] = *reinterpret_cast<const h8*>(
                  &lds[SH::WO + (32 * p + 16 * tt + r) * SH::LDD + ks * 32 + 8 * g]);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int p = 0; p < PN; ++p)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) acc[p][tt] = mfma32(w[p][tt], cur.ctx[t][ks], acc[p][tt]);
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int p = 0; p < PN; ++p) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            xr[t][p][i] = (acc[p][0][i] + bv[p][i]) + cur.x[t][p][i];
            xr[t][p][4 + i] = (acc[p][1][i] + bv[p][4 + i]) + cur.x[t][p][4 + i];
          }
        }
        // LN2's gamma and beta are requested before the row statistics, which hide their latency
        float gm[PN][8], bt[PN][8];
#pragma unroll
        for (int p = 0; p < PN; ++p) {
          lds8(prm + SH::P_G2 + 32 * p + 8 * g, gm[p]);
          lds8(prm + SH::P_BE2 + 32 * p + 8 * g, bt[p]);
        }
        float mean, rstd;
        row_stats<PN>(xr[t], inv_d, a.eps2, mean, rstd);
#pragma unroll
        for (int p = 0; p < PN; ++p) {
          float o[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) o[j] = (xr[t][p][j] - mean) * rstd * gm[p][j] + bt[p][j];
          pin_f32x8(o);  // rounded to FP32, then to the output type (no fused FMA + conversion)
#pragma unroll
          for (int j = 0; j < 8; ++j) n2f[t][p][j] = (_Float16)o[j];
        }
      }

      // ---- FFN: x'' = x' + Wout fp16(GELU(Win n2 + bin)) + bout ----
      f4 yacc[TM][PN][2];
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int p = 0; p < PN; ++p) yacc[t][p][0] = yacc[t][p][1] = zero4();
#pragma unroll 2
      for (int fq = 0; fq < FQ; ++fq) {
        f4 hacc[TM][2];
#pragma unroll
        for (int t = 0; t < TM; ++t) hacc[t][0] = hacc[t][1] = zero4();
        float bi[8];  // requested first: the FFN-in products below hide its latency
        lds8(prm + SH::P_BIN + 32 * fq + 8 * g, bi);
        // Win fragments of this feature pair, read as a group before its MFMAs
        h8 wi[KS][2];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
            wi[ks][tt] = *reinterpret_cast<const h8*>(
                &lds[SH::WIN + (32 * fq + 16 * tt + r) * SH::LDD + ks * 32 + 8 * g]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int t = 0; t < TM; ++t) hacc[t][tt] = mfma32(wi[ks][tt], n2f[t][ks], hacc[t][tt]);
        __builtin_amdgcn_sched_barrier(0);
        h8 hb[TM];
#pragma unroll
        for (int t = 0; t < TM; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            hb[t][i] = (_Float16)gelu_erf(hacc[t][0][i] + bi[i]);
            hb[t][4 + i] = (_Float16)gelu_erf(hacc[t][1][i] + bi[4 + i]);
          }
        // Wout fragments of this hidden pair, read as a group before its MFMAs
        h8 wo[PN][2];
#pragma unroll
        for (int p = 0; p < PN; ++p)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
            wo[p][tt] = *reinterpret_cast<const h8*>(
                &lds[SH::WOUT + (32 * p + 16 * tt + r) * SH::LDF + 32 * fq + 8 * g]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < PN; ++p)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int t = 0; t < TM; ++t) yacc[t][p][tt] = mfma32(wo[p][tt], hb[t], yacc[t][p][tt]);
        __builtin_amdgcn_sched_barrier(0);
      }
      const __amdgpu_buffer_rsrc_t xres = make_rsrc(a.x_out + m0 * D, wrows * (uint32_t)(D * 4));
      float bo2[PN][8];  // all of b_out in one group of LDS reads
#pragma unroll
      for (int p = 0; p < PN; ++p) lds8(prm + SH::P_BOUT + 32 * p + 8 * g, bo2[p]);
#pragma unroll
      for (int t = 0; t < TM; ++t) {
#pragma unroll
        for (int p = 0; p < PN; ++p) {
          const int n = 32 * p + 8 * g;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            xr[t][p][i] = (yacc[t][p][0][i] + bo2[p][i]) + xr[t][p][i];
            xr[t][p][4 + i] = (yacc[t][p][1][i] + bo2[p][4 + i]) + xr[t][p][4 + i];
          }
          buffer_store8(xres, (uint32_t)((16 * t + r) * D + n) * 4u, xr[t][p], a.x_out);
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int p = 0; p < PN; ++p)
#pragma unroll
          for (int j = 0; j < 8; ++j) xr[t][p][j] = cur.x[t][p][j];
    }

    // ---- next LayerNorm, then the next layer's QKV projection (or the final output) ----
    h8 n1f[TM][KS];
    const __amdgpu_buffer_rsrc_t ores = make_rsrc(static_cast<float*>(a.out) + (LAST ? m0 * D : 0),
                                                  LAST ? wrows * (uint32_t)(D * 4) : 0u);
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      // gamma and beta are requested before the row statistics, which hide their latency
      float gm[PN][8], bt[PN][8];
#pragma unroll
      for (int p = 0; p < PN; ++p) {
        lds8(prm + SH::P_G1 + 32 * p + 8 * g, gm[p]);
        lds8(prm + SH::P_BE1 + 32 * p + 8 * g, bt[p]);
      }
      float mean, rstd;
      row_stats<PN>(xr[t], inv_d, a.eps1, mean, rstd);
#pragma unroll
      for (int p = 0; p < PN; ++p) {
        const int n = 32 * p + 8 * g;
        float o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = (xr[t][p][j] - mean) * rstd * gm[p][j] + bt[p][j];
        pin_f32x8(o);  // rounded to FP32, then to the output type (no fused FMA + conversion)
        if constexpr (LAST) {
          buffer_store8(ores, (uint32_t)((16 * t + r) * D + n) * 4u, o, static_cast<float*>(a.out));
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) n1f[t][p][j] = (_Float16)o[j];
        }
      }
    }

    // The next tile's inputs are requested here, once this tile's residual rows
    // are dead, so that their 48+ registers are not held through the
    // out-projection and FFN stages; the QKV stage still covers the load latency.
    TileIn<D, TM, STAGE1> nxt;
    if (tile + gridDim.x < ntiles)
      load_tile<D, TM, STAGE1, !ATTN>(nxt, a, (tile + gridDim.x) * ROWS + wave * 16 * TM, r, g);

    if constexpr (QKV && QMODE == kQkvLds) {
      _Float16* qkv = static_cast<_Float16*>(a.out);
      const __amdgpu_buffer_rsrc_t qres = make_rsrc(qkv + m0 * (3 * D), wrows * (uint32_t)(3 * D * 2));
#pragma unroll 1
      for (int op = 0; op < QP; ++op) {
        f4 qacc[TM][2];
#pragma unroll
        for (int t = 0; t < TM; ++t) qacc[t][0] = qacc[t][1] = zero4();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            const h8 w = *reinterpret_cast<const h8*>(
                &lds[SH::WQKV + (32 * op + 16 * tt + r) * SH::LDD + ks * 32 + 8 * g]);
#pragma unroll
            for (int t = 0; t < TM; ++t) qacc[t][tt] = mfma32(w, n1f[t][ks], qacc[t][tt]);
          }
        const int n = 32 * op + 8 * g;
        float bv[8];
        lds8(prm + SH::P_BQKV + n, bv);
        const bool qcols = a.q_on && 32 * op < D;  // a 32-column block is all q or none (D % 32 == 0)
#pragma unroll
        for (int t = 0; t < TM; ++t) {
          float v[8];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            v[i] = qacc[t][0][i] + bv[i];
            v[4 + i] = qacc[t][1][i] + bv[4 + i];
          }
          if (qcols) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] *= a.q_scale;
            pin_f32x8(v);  // rounded to FP32 first, then to FP16 by the store
          }
          buffer_store8(qres, (uint32_t)((16 * t + r) * (3 * D) + n) * 2u, v, qkv);
        }
      }
    }

    if constexpr (QKV && QMODE == kQkvReg) {
      // publish this wave's normalized rows, then project all workgroup rows onto this wave's columns
      _Float16* nbuf = lds + SH::RING;
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int p = 0; p < PN; ++p)
          *reinterpret_cast<h8*>(&nbuf[(wave * 16 * TM + 16 * t + r) * SH::LDD + 32 * p + 8 * g]) = n1f[t][p];
      __syncthreads();
      _Float16* qkv = static_cast<_Float16*>(a.out);
      const int ncol0 = QNW * wave;
      float bq[QNT][4];
#pragma unroll
      for (int nt = 0; nt < QNT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) bq[nt][i] = prm[SH::P_BQKV + ncol0 + 16 * nt + 4 * g + i];
      const __amdgpu_buffer_rsrc_t qres = make_rsrc(qkv + wg0 * (3 * D), grows * (uint32_t)(3 * D * 2));
#pragma unroll 2
      for (int mt = 0; mt < ROWS / 16; ++mt) {
        h8 bn[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          bn[ks] = *reinterpret_cast<const h8*>(&nbuf[(16 * mt + r) * SH::LDD + ks * 32 + 8 * g]);
        // the QNT column tiles are independent MFMA chains: interleave them
        f4 acc[QNT];
#pragma unroll
        for (int nt = 0; nt < QNT; ++nt) acc[nt] = zero4();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int nt = 0; nt < QNT; ++nt) acc[nt] = mfma32(wq[nt][ks], bn[ks], acc[nt]);
#pragma unroll
        for (int nt = 0; nt < QNT; ++nt) {
          float o[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = acc[nt][i] + bq[nt][i];
          if (a.q_on && ncol0 + 16 * nt < D) {  // wave-uniform: a 16-column tile is all q or none
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] *= a.q_scale;
            pin_f32x4(o);  // rounded to FP32 first, then to FP16 by the store
          }
          buffer_store4(qres, (uint32_t)((16 * mt + r) * (3 * D) + ncol0 + 16 * nt + 4 * g) * 2u, o);
        }
      }
      __syncthreads();  // nbuf is rewritten by the next tile
    }
    cur = nxt;
  }
}

static int tail_cu_count() {
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

template <int D, int F, int TM, bool STAGE1, bool LAST, int QMODE, int W, int AHD>
constexpr int tail_lds_bytes() {
  if constexpr (AHD != 0)
    return attn_lds_bytes<D, F, TM, !LAST, QMODE, W, AHD>();
  else
    return TailShape<D, F, TM, STAGE1, !LAST, QMODE, W>::BYTES;
}

template <int D, int F, int TM, bool STAGE1, bool LAST, int QMODE, int W, int AHD = 0>
static hipError_t launch_tail(const TailArgs& a, hipStream_t s) {
  constexpr int lds_bytes = tail_lds_bytes<D, F, TM, STAGE1, LAST, QMODE, W, AHD>();
  static_assert(lds_bytes <= kLdsBudget, "weights exceed LDS");
  auto kern = layer_tail_kernel<D, F, TM, STAGE1, LAST, QMODE, W, AHD>;
  if (lds_bytes > 64 * 1024) {
    static std::atomic<bool> attribute_set{false};  // once per instantiation
    if (!attribute_set.load(std::memory_order_acquire)) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
      if (e != hipSuccess) return e;
      attribute_set.store(true, std::memory_order_release);
    }
  }
  constexpr int ROWS = 16 * TM * W;
  const int64_t ntiles = (a.m + ROWS - 1) / ROWS;
  const int64_t per_cu = lds_bytes > kLdsBudget / 2 ? 1 : 2;
  int64_t grid = (int64_t)tail_cu_count() * per_cu;
  if (grid > ntiles) grid = ntiles;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * W), lds_bytes, s, a);
  return hipGetLastError();
}

// QKV weights in LDS when the whole set fits, else stationary in registers.
template <int D, int F, bool STAGE1>
constexpr int qkv_mode() {
  return TailShape<D, F, 1, STAGE1, true, kQkvLds, 8>::BYTES <= kLdsBudget ? kQkvLds : kQkvReg;
}

// Variants: 1: 8 waves x 16 rows (128-row tiles); 2: 8 waves x 32 rows, where its LDS
// footprint fits; 3: 4 waves x 16 rows (64-row tiles), for row counts whose 128-row
// tiles would leave CUs idle.
template <int D, int F, bool STAGE1>
static hipError_t tail_variant(int variant, bool last, const TailArgs& a, hipStream_t s) {
  constexpr int QM = qkv_mode<D, F, STAGE1>();
  if constexpr (TailShape<D, F, 2, STAGE1, true, QM, 8>::BYTES <= kLdsBudget) {
    if (variant == 2)
      return last ? launch_tail<D, F, 2, STAGE1, true, QM, 8>(a, s) : launch_tail<D, F, 2, STAGE1, false, QM, 8>(a, s);
  }
  if (variant == 3)
    return last ? launch_tail<D, F, 1, STAGE1, true, QM, 4>(a, s) : launch_tail<D, F, 1, STAGE1, false, QM, 4>(a, s);
  return last ? launch_tail<D, F, 1, STAGE1, true, QM, 8>(a, s) : launch_tail<D, F, 1, STAGE1, false, QM, 8>(a, s);
}

// 64-row tiles when 128-row tiles would not give every CU one
static int tail_auto_variant(int64_t m) { return (m + 127) / 128 < tail_cu_count() ? 3 : 1; }

// Fused attention + tail: 4 waves x 16 rows (64-row tiles; a tile's rows lie in one
// sequence when seq % 64 == 0), where the weights, parameters and the attention area fit.
// Head dims 32 (any of the tail widths) and 16 (d_model 32 and 64).
constexpr int kAttnTailRows = 64;
template <int D, int F, int AHD>
constexpr bool attn_tail_fits() {
  constexpr int QM = qkv_mode<D, F, true>();
  return D % AHD == 0 && (AHD == 32 || D <= 64) && (QM != kQkvReg || (3 * D) % (16 * 4) == 0) &&
         attn_lds_bytes<D, F, 1, true, QM, 4, AHD>() <= kLdsBudget;
}
template <int D, int F, int AHD>
static hipError_t attn_tail_launch_hd(bool last, const TailArgs& a, hipStream_t s) {
  if constexpr (attn_tail_fits<D, F, AHD>()) {
    constexpr int QM = qkv_mode<D, F, true>();
    return last ? launch_tail<D, F, 1, true, true, QM, 4, AHD>(a, s)
                : launch_tail<D, F, 1, true, false, QM, 4, AHD>(a, s);
  } else {
    (void)last; (void)a; (void)s;
    return (hipError_t)MPK_EUNSUPPORTED;
  }
}
template <int D, int F>
static bool attn_tail_fits_hd(int hd) {
  return hd == 32 ? attn_tail_fits<D, F, 32>() : hd == 16 ? attn_tail_fits<D, F, 16>() : false;
}
template <int D, int F>
static hipError_t attn_tail_launch(int hd, bool last, const TailArgs& a, hipStream_t s) {
  return hd == 32 ? attn_tail_launch_hd<D, F, 32>(last, a, s) : attn_tail_launch_hd<D, F, 16>(last, a, s);
}

}  // namespace mpk

using namespace mpk;

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

extern "C" int mpk_layer_tail_supported(int32_t d, int32_t f) {
  return (d == 32 && f == 64) || (d == 64 && (f == 64 || f == 128 || f == 256)) ||
         (d == 128 && f == 128) || (d == 32 && f == 32) || (d == 32 && f == 128);
}

static int layer_tail_entry(const void* ctx, const float* x, const void* w_o, const void* b_o, const float* ln2_w,
                            const float* ln2_b, const void* w_in, const void* b_in, const void* w_out,
                            const void* b_out, const float* next_ln_w, const float* next_ln_b, const void* w_qkv,
                            const void* b_qkv, float* x_out, void* out, int last, int64_t m, int32_t d, int32_t f,
                            float ln2_eps, float next_ln_eps, bool q_on, float q_scale, int variant, void* stream) {
  if (!ctx || !x || !w_o || !b_o || !ln2_w || !ln2_b || !w_in || !b_in || !w_out || !b_out || !next_ln_w ||
      !next_ln_b || !x_out || !out || m < 0)
    return MPK_EINVAL;
  if (!last && (!w_qkv || !b_qkv)) return MPK_EINVAL;
  if (!mpk_layer_tail_supported(d, f)) return MPK_EUNSUPPORTED;
  const void* ptrs[] = {ctx, x, w_o, b_o, ln2_w, ln2_b, w_in, b_in, w_out, b_out, next_ln_w, next_ln_b, x_out, out};
  for (const void* p : ptrs)
    if (!aligned16(p)) return MPK_EALIGN;
  if (!last && (!aligned16(w_qkv) || !aligned16(b_qkv))) return MPK_EALIGN;
  if (m == 0) return MPK_OK;
  if (variant == 0) variant = tail_auto_variant(m);
  if (variant < 1 || variant > 3) return MPK_EUNSUPPORTED;
  TailArgs a{};
  a.ctx = static_cast<const _Float16*>(ctx); a.x = x;
  a.wo = static_cast<const _Float16*>(w_o); a.bo = static_cast<const _Float16*>(b_o); a.g2 = ln2_w; a.be2 = ln2_b;
  a.win = static_cast<const _Float16*>(w_in); a.bin = static_cast<const _Float16*>(b_in);
  a.wout = static_cast<const _Float16*>(w_out); a.bout = static_cast<const _Float16*>(b_out);
  a.g1 = next_ln_w; a.be1 = next_ln_b;
  a.wqkv = static_cast<const _Float16*>(w_qkv); a.bqkv = static_cast<const _Float16*>(b_qkv);
  a.x_out = x_out; a.out = out; a.m = m; a.f = f; a.eps2 = ln2_eps; a.eps1 = next_ln_eps;
  a.q_on = q_on && !last; a.q_scale = q_scale;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool L = last != 0;
  hipError_t e;
  if (d == 32 && f == 32) e = tail_variant<32, 32, true>(variant, L, a, s);
  else if (d == 32 && f == 64) e = tail_variant<32, 64, true>(variant, L, a, s);
  else if (d == 32 && f == 128) e = tail_variant<32, 128, true>(variant, L, a, s);
  else if (d == 64 && f == 64) e = tail_variant<64, 64, true>(variant, L, a, s);
  else if (d == 64 && f == 128) e = tail_variant<64, 128, true>(variant, L, a, s);
  else if (d == 64 && f == 256) e = tail_variant<64, 256, true>(variant, L, a, s);
  else e = tail_variant<128, 128, true>(variant, L, a, s);
  return (int)e;
}

extern "C" int mpk_layer_tail(const void* ctx, const float* x, const void* w_o, const void* b_o, const float* ln2_w,
                              const float* ln2_b, const void* w_in, const void* b_in, const void* w_out,
                              const void* b_out, const float* next_ln_w, const float* next_ln_b, const void* w_qkv,
                              const void* b_qkv, float* x_out, void* out, int last, int64_t m, int32_t d, int32_t f,
                              float ln2_eps, float next_ln_eps, int variant, void* stream) {
  return layer_tail_entry(ctx, x, w_o, b_o, ln2_w, ln2_b, w_in, b_in, w_out, b_out, next_ln_w, next_ln_b, w_qkv,
                          b_qkv, x_out, out, last, m, d, f, ln2_eps, next_ln_eps, false, 1.0f, variant, stream);
}

extern "C" int mpk_layer_tail_qscaled(const void* ctx, const float* x, const void* w_o, const void* b_o,
                                      const float* ln2_w, const float* ln2_b, const void* w_in, const void* b_in,
                                      const void* w_out, const void* b_out, const float* next_ln_w,
                                      const float* next_ln_b, const void* w_qkv, const void* b_qkv, float* x_out,
                                      void* out, int last, int64_t m, int32_t d, int32_t f, float ln2_eps,
                                      float next_ln_eps, float q_scale, int variant, void* stream) {
  return layer_tail_entry(ctx, x, w_o, b_o, ln2_w, ln2_b, w_in, b_in, w_out, b_out, next_ln_w, next_ln_b, w_qkv,
                          b_qkv, x_out, out, last, m, d, f, ln2_eps, next_ln_eps, true, q_scale, variant, stream);
}

extern "C" int mpk_attention_layer_tail_supported(int32_t d, int32_t f, int32_t heads) {
  if (!mpk_layer_tail_supported(d, f) || heads <= 0 || d % heads != 0) return 0;
  const int hd = d / heads;
  if (d == 32 && f == 32) return attn_tail_fits_hd<32, 32>(hd);
  if (d == 32 && f == 64) return attn_tail_fits_hd<32, 64>(hd);
  if (d == 32 && f == 128) return attn_tail_fits_hd<32, 128>(hd);
  if (d == 64 && f == 64) return attn_tail_fits_hd<64, 64>(hd);
  if (d == 64 && f == 128) return attn_tail_fits_hd<64, 128>(hd);
  if (d == 64 && f == 256) return attn_tail_fits_hd<64, 256>(hd);
  return attn_tail_fits_hd<128, 128>(hd);
}

extern "C" int32_t mpk_attention_layer_tail_rows(void) { return kAttnTailRows; }

extern "C" int mpk_attention_layer_tail(const void* qkv_in, const float* x, const void* w_o, const void* b_o,
                                        const float* ln2_w, const float* ln2_b, const void* w_in, const void* b_in,
                                        const void* w_out, const void* b_out, const float* next_ln_w,
                                        const float* next_ln_b, const void* w_qkv, const void* b_qkv, float* x_out,
                                        void* out, int last, int64_t m, int32_t d, int32_t f, int32_t heads,
                                        int32_t seq_len, float scale, int causal, float ln2_eps, float next_ln_eps,
                                        void* stream) {
  if (!qkv_in || !x || !w_o || !b_o || !ln2_w || !ln2_b || !w_in || !b_in || !w_out || !b_out || !next_ln_w ||
      !next_ln_b || !x_out || !out || m < 0 || seq_len <= 0)
    return MPK_EINVAL;
  if (!last && (!w_qkv || !b_qkv)) return MPK_EINVAL;
  if (!mpk_attention_layer_tail_supported(d, f, heads)) return MPK_EUNSUPPORTED;
  if (seq_len % kAttnTailRows != 0 || m % seq_len != 0) return MPK_EUNSUPPORTED;
  const void* ptrs[] = {qkv_in, x, w_o, b_o, ln2_w, ln2_b, w_in, b_in, w_out, b_out, next_ln_w, next_ln_b, x_out, out};
  for (const void* p : ptrs)
    if (!aligned16(p)) return MPK_EALIGN;
  if (!last && (!aligned16(w_qkv) || !aligned16(b_qkv))) return MPK_EALIGN;
  // other workgroups read this layer's K and V while a workgroup writes its rows of the
  // next layer's QKV: the two buffers must not overlap
  {
    const uintptr_t in0 = reinterpret_cast<uintptr_t>(qkv_in), in1 = in0 + (uintptr_t)m * 3 * d * 2;
    const uintptr_t o0 = reinterpret_cast<uintptr_t>(out);
    const uintptr_t o1 = o0 + (uintptr_t)m * (last ? d * 4 : 3 * d * 2);
    if (m > 0 && in0 < o1 && o0 < in1) return MPK_EINVAL;
  }
  if (m == 0) return MPK_OK;
  TailArgs a{};
  a.wo = static_cast<const _Float16*>(w_o); a.bo = static_cast<const _Float16*>(b_o); a.g2 = ln2_w; a.be2 = ln2_b;
  a.x = x;
  a.win = static_cast<const _Float16*>(w_in); a.bin = static_cast<const _Float16*>(b_in);
  a.wout = static_cast<const _Float16*>(w_out); a.bout = static_cast<const _Float16*>(b_out);
  a.g1 = next_ln_w; a.be1 = next_ln_b;
  a.wqkv = static_cast<const _Float16*>(w_qkv); a.bqkv = static_cast<const _Float16*>(b_qkv);
  a.x_out = x_out; a.out = out; a.m = m; a.f = f; a.eps2 = ln2_eps; a.eps1 = next_ln_eps;
  a.qkv_in = static_cast<const _Float16*>(qkv_in);
  a.seq = seq_len; a.causal = causal ? 1 : 0; a.attn_c = scale * 1.4426950408889634f;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool L = last != 0;
  hipError_t e;
  const int hd = d / heads;
  if (d == 32 && f == 32) e = attn_tail_launch<32, 32>(hd, L, a, s);
  else if (d == 32 && f == 64) e = attn_tail_launch<32, 64>(hd, L, a, s);
  else if (d == 32 && f == 128) e = attn_tail_launch<32, 128>(hd, L, a, s);
  else if (d == 64 && f == 64) e = attn_tail_launch<64, 64>(hd, L, a, s);
  else if (d == 64 && f == 128) e = attn_tail_launch<64, 128>(hd, L, a, s);
  else if (d == 64 && f == 256) e = attn_tail_launch<64, 256>(hd, L, a, s);
  else e = attn_tail_launch<128, 128>(hd, L, a, s);
  return (int)e;
}

extern "C" int mpk_layernorm_qkv_supported(int32_t d) { return d == 32 || d == 64 || d == 128; }

static int layernorm_qkv_entry(const float* x, const float* ln_w, const float* ln_b, const void* w_qkv,
                               const void* b_qkv, void* qkv, int64_t m, int32_t d, float eps, bool q_on,
                               float q_scale, int variant, void* stream) {
  if (!x || !ln_w || !ln_b || !w_qkv || !b_qkv || !qkv || m < 0) return MPK_EINVAL;
  if (!mpk_layernorm_qkv_supported(d)) return MPK_EUNSUPPORTED;
  const void* ptrs[] = {x, ln_w, ln_b, w_qkv, b_qkv, qkv};
  for (const void* p : ptrs)
    if (!aligned16(p)) return MPK_EALIGN;
  if (m == 0) return MPK_OK;
  if (variant == 0) variant = tail_auto_variant(m);
  if (variant < 1 || variant > 3) return MPK_EUNSUPPORTED;
  TailArgs a{};
  a.x = x; a.g1 = ln_w; a.be1 = ln_b;
  a.wqkv = static_cast<const _Float16*>(w_qkv); a.bqkv = static_cast<const _Float16*>(b_qkv);
  a.out = qkv; a.m = m; a.eps1 = eps;
  a.q_on = q_on; a.q_scale = q_scale;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  switch (d) {
    case 32: e = tail_variant<32, 32, false>(variant, false, a, s); break;
    case 64: e = tail_variant<64, 32, false>(variant, false, a, s); break;
    default: e = tail_variant<128, 32, false>(variant, false, a, s); break;
  }
  return (int)e;
}

extern "C" int mpk_layernorm_qkv(const float* x, const float* ln_w, const float* ln_b, const void* w_qkv,
                                 const void* b_qkv, void* qkv, int64_t m, int32_t d, float eps, int variant,
                                 void* stream) {
  return layernorm_qkv_entry(x, ln_w, ln_b, w_qkv, b_qkv, qkv, m, d, eps, false, 1.0f, variant, stream);
}

extern "C" int mpk_layernorm_qkv_qscaled(const float* x, const float* ln_w, const float* ln_b, const void* w_qkv,
                                         const void* b_qkv, void* qkv, int64_t m, int32_t d, float eps,
                                         float q_scale, int variant, void* stream) {
  return layernorm_qkv_entry(x, ln_w, ln_b, w_qkv, b_qkv, qkv, m, d, eps, true, q_scale, variant, stream);
}
