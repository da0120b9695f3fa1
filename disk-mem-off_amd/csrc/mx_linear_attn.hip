// Qwen3-Next linear-attention (Gated DeltaNet) block on the device:
//   rmsnorm -> qkvz projection -> ba projection -> causal conv + SiLU + gates -> scan
//   -> gated output norm -> out projection -> residual,
// i.e. Qwen3NextExecutor._linear_attn_block (offload_runtime/executors/qwen3_next.py:207-269)
// with _softplus (:27-28), _causal_conv1d (:35-53) and _gated_delta_rule_recurrence
// (:56-95).  The projections of short inputs (and int8 / fp32 weights) run on the grouped
// kernels of the MoE experts as single-group products (HBM-bound weight streaming); long
// inputs with fp16 weights run on the dense MFMA GEMM, qkvz and ba in one launch.
// Everything runs on the caller's stream out of the caller's workspace.
#include <math.h>

#include "mx_common.h"
#include "mx_internal.h"

namespace {

struct LaDims {
  int H, n, dk, dv, K;
  int qd, vd;  // n dk, n dv
  int C;       // conv channels: 2 qd + vd
  int W1, W2;  // row widths of qkvz (2 qd + 2 vd) and ba (qd + n)
};

LaDims dims_of(const MxLinearAttnDesc* d) {
  LaDims m;
  m.H = d->hidden;
  m.n = d->n_heads;
  m.dk = d->head_dim_k;
  m.dv = d->head_dim_v;
  m.K = d->conv_kernel;
  m.qd = m.n * m.dk;
  m.vd = m.n * m.dv;
  m.C = 2 * m.qd + m.vd;
  m.W1 = 2 * m.qd + 2 * m.vd;
  m.W2 = m.qd + m.n;
  return m;
}

int check_desc(const MxLinearAttnDesc* d) {
  if (!d) return MX_ERR_INVALID;
  if (d->hidden <= 0 || d->n_heads <= 0 || d->head_dim_k <= 0 || d->head_dim_v <= 0 ||
      d->conv_kernel <= 0)
    return MX_ERR_INVALID;
  if (d->param_dtype != MX_DT_F32 && d->param_dtype != MX_DT_F16) return MX_ERR_INVALID;
  if (d->weight_dtype != MX_DT_F32 && d->weight_dtype != MX_DT_F16 && d->weight_dtype != MX_DT_I8)
    return MX_ERR_INVALID;
  if (d->conv_kernel > 16) return MX_ERR_UNSUPPORTED;
  const int dk = d->head_dim_k;
  if ((dk & (dk - 1)) || dk < 4 || dk > 512) return MX_ERR_UNSUPPORTED;
  const long w1 = 2l * d->n_heads * (d->head_dim_k + d->head_dim_v);
  if (w1 * d->hidden >= (1l << 31) || (long)d->hidden * d->n_heads * d->head_dim_v >= (1l << 31))
    return MX_ERR_UNSUPPORTED;
  return MX_OK;
}

struct Carve {
  char* base;
  size_t off = 0;
  void* take(size_t n) {
    off = mx_align_up(off, 256);
    void* p = base ? base + off : nullptr;
    off += n;
    return p;
  }
};

struct LaWork {
  MxLinearAttnViews v;
  MxDenseWork dw;      // projections: entry 0 qkvz, 1 ba, 2 out
  void* chunk_ws = nullptr;  // chunked scan: coefficients and chunk states (NULL: sequential)
};

int layout(const MxLinearAttnDesc* d, int T, void* ws, LaWork* w, size_t* total) {
  MX_TRY(check_desc(d));
  if (T < 0) return MX_ERR_INVALID;
  const size_t Tn = T > 0 ? T : 1;
  const LaDims m = dims_of(d);
  const bool f32 = d->weight_dtype == MX_DT_F32;
  Carve c{(char*)ws};
  LaWork t;
  t.v.h32 = (float*)c.take(Tn * m.H * 4);
  t.v.h16 = f32 ? nullptr : c.take(Tn * m.H * 2);
  t.v.qkvz = (float*)c.take(Tn * m.W1 * 4);
  t.v.ba = (float*)c.take(Tn * m.W2 * 4);
  t.v.q = (float*)c.take(Tn * m.qd * 4);
  t.v.kb = (float*)c.take(Tn * m.qd * 4);
  t.v.v = (float*)c.take(Tn * m.vd * 4);
  t.v.decay = (float*)c.take(Tn * m.n * 4);
  t.v.o = (float*)c.take(Tn * m.vd * 4);
  t.v.act = c.take(Tn * m.vd * (f32 ? 4 : 2));
  t.v.y = (float*)c.take(Tn * m.H * 4);
  char* dwb = (char*)c.take(mx_dense_work_bytes((int)Tn, d->weight_dtype, 3));
  mx_dense_work_carve(dwb, (int)Tn, d->weight_dtype, 3, &t.dw);
  const size_t cb = mx_la_chunk_ws_bytes((int)Tn, m.n, m.dk, m.dv);
  t.chunk_ws = cb ? c.take(cb) : nullptr;
  if (w) *w = t;
  if (total) *total = mx_align_up(c.off, 256);
  return MX_OK;
}

// ------------------------------------------------------------------------------------
// Kernels.
// ------------------------------------------------------------------------------------

// Causal depthwise conv + SiLU on the q/k/v channels, beta * k, and the per-head decay.
// Grid (ceil((C + n) / 256), ceil(T / LA_TT)); a thread walks LA_TT consecutive tokens of
// one channel with the last K - 1 inputs in registers (KC = K known at compile time, 0 =
// any K up to 16, re-read from memory).  Channel c < C: out = sum_{j=0}^{K-1} x[t - j, c]
// w[c, j], summed in j order from 0 (qwen3_next.py:49-52), then silu (:238); k channels
// times sigmoid(b) (:244, :89).  Thread C + h: g = -exp(A_log) softplus(a + dt_bias)
// (:249), decay = exp(g) (:84).  Products are rounded before each sum, as NumPy does.
#define LA_TT 16

template <int KC>
__global__ __launch_bounds__(256) void k_la_prep(const float* __restrict__ qkvz,
                                                 const float* __restrict__ ba,
                                                 const void* __restrict__ conv_w,
                                                 const void* __restrict__ a_log,
                                                 const void* __restrict__ dt_bias, int pdt,
                                                 LaDims m, int T, float* __restrict__ q,
                                                 float* __restrict__ kb, float* __restrict__ v,
                                                 float* __restrict__ decay) {
#pragma clang fp contract(off)
  const int t0 = blockIdx.y * LA_TT;
  const int t1 = min(T, t0 + LA_TT);
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c < m.C) {
    float* dst;
    int ld;
    const float* gate = nullptr;
    if (c < m.qd) {
      dst = q + c;
      ld = m.qd;
    } else if (c < 2 * m.qd) {
      dst = kb + (c - m.qd);
      ld = m.qd;
      gate = ba + (c - m.qd);
    } else {
      dst = v + (c - 2 * m.qd);
      ld = m.vd;
    }
    const float* x = qkvz + c;
    if constexpr (KC > 0) {
      // Before token t's shift win[j] = x[t - 1 - j]; after it win[j] = x[t - j].
      float w[KC], win[KC];
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        w[j] = mx_load_param(conv_w, pdt, c * KC + j);
        win[j] = (t0 - 1 - j >= 0) ? x[(size_t)(t0 - 1 - j) * m.W1] : 0.f;
      }
      // All of the thread's inputs first (independent loads in flight together).
      float xs[LA_TT], gs[LA_TT];
#pragma unroll
      for (int i = 0; i < LA_TT; ++i) {
        const int t = min(t0 + i, T - 1);
        xs[i] = x[(size_t)t * m.W1];
        gs[i] = gate ? gate[(size_t)t * m.W2] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < LA_TT; ++i) {
#pragma unroll
        for (int j = KC - 1; j > 0; --j) win[j] = win[j - 1];
        win[0] = xs[i];
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < KC; ++j) acc += win[j] * w[j];
        float s = mx_silu(acc);
        if (gate) s = mx_sigmoid(gs[i]) * s;
        if (t0 + i < t1) dst[(size_t)(t0 + i) * ld] = s;
      }
    } else {
      for (int t = t0; t < t1; ++t) {
        float acc = 0.f;
        for (int j = 0; j < m.K && j <= t; ++j)
          acc += x[(size_t)(t - j) * m.W1] * mx_load_param(conv_w, pdt, c * m.K + j);
        float s = mx_silu(acc);
        if (gate) s = mx_sigmoid(gate[(size_t)t * m.W2]) * s;
        dst[(size_t)t * ld] = s;
      }
    }
  } else if (c < m.C + m.n) {
    const int h = c - m.C;
    float ea = expf(mx_load_param(a_log, pdt, h));
    if (pdt == MX_DT_F16) ea = (float)(half_t)ea;  // np.exp of an fp16 array stays fp16
    const float bias = mx_load_param(dt_bias, pdt, h);
    for (int t = t0; t < t1; ++t) {
      const float a = ba[(size_t)t * m.W2 + m.qd + h] + bias;
      const float sp = a > 20.f ? a : log1pf(expf(a));
      decay[(size_t)t * m.n + h] = expf(-ea * sp);
    }
  }
}

// ------------------------------------------------------------------------------------
// The recurrence:  S[i, c] = S[i, c] * decay_t + v_t[i] * kb_t[c];  o_t[i] = sum_c S[i, c] q_t[c]
// per head (state rows i = value index, columns c = key index), from S = 0.
//
// A block of 4 waves holds RB state rows of one head.  Per chunk of TC tokens it stages
// that head's q and kb, its rows of v and the decays in LDS (double-buffered: the next
// chunk's global loads are in flight while the current chunk runs), so every state
// element reads q and kb from LDS rather than L1.  Full chunks run unrolled and branch-
// free with the (state-independent) LDS reads of later tokens issued ahead of the update
// chain; each output is kept by one lane of its row and all are stored after the chunk.
//
// Two lane mappings:
//  * k_la_scan_wide (dk >= 64): a wave holds 4 rows; lane l holds columns
//    [l * CPL, (l + 1) * CPL) of all 4 (CPL = dk / 64), so the q and kb values a lane
//    reads serve 4 rows.  The 4 dot products are reduce-scattered across the wave with
//    the gfx950 lane swaps (v_permlane32_swap: halves, v_permlane16_swap: rows of 16)
//    and finished by DPP inside each row of 16: 3 swaps + 3 adds + 4 DPP adds for 4 sums.
//  * k_la_scan (dk <= 32): lane (row group, column group) holds CPL columns of one row,
//    the dot product is finished across the L = dk / CPL lanes of the row with DPP.
// ------------------------------------------------------------------------------------
template <int DK_, int RB_>
struct ScanStage {
  static constexpr int DK = DK_, RB = RB_;
  static constexpr int TC = DK >= 512 ? 4 : (DK >= 256 ? 8 : 16);  // tokens per chunk
  static constexpr int NQ = TC * DK;  // floats of q (and of kb) per chunk
  static constexpr int NQ4 = NQ / 4;  // float4 pieces of q (and of kb) per chunk
  static constexpr int QP = (NQ4 + 255) / 256;  // q (and kb) pieces per thread
  static constexpr int NV = TC * RB;  // v values per chunk
  static constexpr int VP = (NV + 255) / 256;
  static constexpr int BUF = 2 * NQ + NV + TC;  // floats per LDS buffer
  static_assert(DK % 4 == 0, "key head size must be a multiple of 4");

  // Registers of one staged chunk.  Offsets are in elements (T * n * max(dk, dv) < 2^31
  // is checked by the launcher).  q and kb: float4 piece i = (token i / (DK / 4), columns
  // 4 (i % (DK / 4)) ..) of head h; v: value i = (token i / RB, row rb0 + i % RB); decay:
  // one per token.
  float4 qv[QP], kv[QP];
  float vv[VP];
  float dd;

  __device__ __forceinline__ void load(const float* __restrict__ q,
                                       const float* __restrict__ kb,
                                       const float* __restrict__ v,
                                       const float* __restrict__ decay, int t0, int T, int n,
                                       int dv, int h, int rb0) {
    const int tid = threadIdx.x;
    const int qd = n * DK, vd = n * dv;
#pragma unroll
    for (int p = 0; p < QP; ++p) {
      const int i = tid + 256 * p;
      const int t = t0 + i / (DK / 4);
      const bool ok = i < NQ4 && t < T;
      const int off = t * qd + h * DK + 4 * (i % (DK / 4));
      qv[p] = ok ? *(const float4*)(q + off) : make_float4(0.f, 0.f, 0.f, 0.f);
      kv[p] = ok ? *(const float4*)(kb + off) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int p = 0; p < VP; ++p) {
      const int i = tid + 256 * p;
      const int t = t0 + i / RB, r2 = rb0 + i % RB;
      vv[p] = (i < NV && t < T && r2 < dv) ? v[t * vd + h * dv + r2] : 0.f;
    }
    dd = (tid < TC && t0 + tid < T) ? decay[(t0 + tid) * n + h] : 0.f;
  }

  __device__ __forceinline__ void store(float* b) const {
    const int tid = threadIdx.x;
#pragma unroll
    for (int p = 0; p < QP; ++p) {
      const int i = tid + 256 * p;
      if (i < NQ4) {
        ((float4*)b)[i] = qv[p];
        ((float4*)(b + NQ))[i] = kv[p];
      }
    }
#pragma unroll
    for (int p = 0; p < VP; ++p) {
      const int i = tid + 256 * p;
      if (i < NV) b[2 * NQ + i] = vv[p];
    }
    if (tid < TC) b[2 * NQ + NV + tid] = dd;
  }
};

// Walks the chunks of [0, T): chunk c is computed from LDS buffer c % 2 while the global
// loads of chunks c + 1 and c + 2 are in flight in two register stages, so every load has
// at least one chunk of compute to arrive before it is written to LDS.  One barrier per
// chunk: the buffer written after chunk c was last read in chunk c - 1, before every wave
// passed the barrier that ended that chunk.  compute(buf, t0) runs one chunk.
template <class St, class F>
__device__ __forceinline__ void la_chunks(const float* __restrict__ q,
                                          const float* __restrict__ kb,
                                          const float* __restrict__ v,
                                          const float* __restrict__ decay, int T, int n, int dv,
                                          int h, int rb0, float (*lds)[St::BUF], F&& compute) {
  constexpr int TC = St::TC;
  const int nchunk = (T + TC - 1) / TC;
  St sa, sb;
  sa.load(q, kb, v, decay, 0, T, n, dv, h, rb0);
  sa.store(lds[0]);
  if (nchunk > 1) sa.load(q, kb, v, decay, TC, T, n, dv, h, rb0);
  if (nchunk > 2) sb.load(q, kb, v, decay, 2 * TC, T, n, dv, h, rb0);
  __syncthreads();
  for (int ch = 0; ch < nchunk; ch += 2) {
    compute(lds[0], ch * TC);  // sa: chunk ch + 1, sb: chunk ch + 2
    if (ch + 1 >= nchunk) break;
    sa.store(lds[1]);
    __syncthreads();
    if (ch + 3 < nchunk) sa.load(q, kb, v, decay, (ch + 3) * TC, T, n, dv, h, rb0);
    compute(lds[1], (ch + 1) * TC);  // sb: chunk ch + 2, sa: chunk ch + 3
    if (ch + 2 >= nchunk) break;
    sb.store(lds[0]);
    __syncthreads();
    if (ch + 4 < nchunk) sb.load(q, kb, v, decay, (ch + 4) * TC, T, n, dv, h, rb0);
  }
}

// Tokens of LDS reads in flight ahead of the recurrence update (full chunks).
#ifndef LA_SCAN_PD
#define LA_SCAN_PD 2
#endif

template <int L>
__device__ __forceinline__ float la_row_sum(float v) {
  if constexpr (L >= 2) v += mx_dpp<MX_DPP_XOR1>(v);
  if constexpr (L >= 4) v += mx_dpp<MX_DPP_XOR2>(v);
  if constexpr (L >= 8) v += mx_dpp<MX_DPP_HALF_MIRROR>(v);
  if constexpr (L >= 16) v += mx_dpp<MX_DPP_MIRROR>(v);
  if constexpr (L >= 32) v += __shfl_xor(v, 16);
  if constexpr (L >= 64) v += __shfl_xor(v, 32);
  return v;
}

// Sums of p[0..3] over the 64 lanes; row j (lanes 16 j .. 16 j + 15) returns the sum of
// p[j].  permlane32_swap(a, b) gives (lanes < 32: a[l], a[l + 32]; lanes >= 32: b[l - 32],
// b[l]), permlane16_swap(a, b) the same between the rows of 16 of each half.  Both
// elements of a swap's result are copied to integers before conversion: this compiler
// folds __builtin_bit_cast(float, r[1]) of the result vector into r[0].
__device__ __forceinline__ float la_swap_sum32(float a, float b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                  false);
  const unsigned x0 = r[0], x1 = r[1];
  return __uint_as_float(x0) + __uint_as_float(x1);
}

__device__ __forceinline__ float la_swap_sum16(float a, float b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                  false);
  const unsigned x0 = r[0], x1 = r[1];
  return __uint_as_float(x0) + __uint_as_float(x1);
}

__device__ __forceinline__ float la_wave_sum4(const float (&p)[4]) {
  const float u0 = la_swap_sum32(p[0], p[2]);
  const float u1 = la_swap_sum32(p[1], p[3]);
  return la_row_sum<16>(la_swap_sum16(u0, u1));
}

template <int CPL>
__global__ __launch_bounds__(256) void k_la_scan_wide(const float* __restrict__ q,
                                                      const float* __restrict__ kb,
                                                      const float* __restrict__ v,
                                                      const float* __restrict__ decay, int T,
                                                      int n, int dv, int bph,
                                                      float* __restrict__ o) {
  constexpr int DK = 64 * CPL, RB = 16;
  using St = ScanStage<DK, RB>;
  constexpr int TC = St::TC, NQ = St::NQ, NV = St::NV;
  __shared__ __align__(16) float lds[2][St::BUF];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = blockIdx.x / bph;
  const int rb0 = (blockIdx.x - h * bph) * RB;  // first value row of this block in head h
  const int r0 = wave * 4;                      // first row of this wave in the block
  const int c0 = lane * CPL;
  const int j = lane >> 4, tl = lane & 15;      // this lane's row (of 4) and token slot
  const int row = rb0 + r0 + j;
  const bool rvalid = row < dv;
  const int vd = n * dv;

  float S[4][CPL];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int c = 0; c < CPL; ++c) S[m][c] = 0.f;

  la_chunks<St>(q, kb, v, decay, T, n, dv, h, rb0, lds, [&](const float* sq, int t0) {
    const float* sk = sq + NQ;
    const float* sv = sk + NQ;
    const float* sd = sv + NV;
    auto token = [&](int tt, const float (&qv)[CPL], const float (&kv)[CPL],
                     const float4& vr, float dd) {
      const float vv[4] = {vr.x, vr.y, vr.z, vr.w};
      float part[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        part[m] = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          S[m][c] = S[m][c] * dd + vv[m] * kv[c];
          part[m] += S[m][c] * qv[c];
        }
      }
      return la_wave_sum4(part);
    };
    auto fetch = [&](int tt, float (&qv)[CPL], float (&kv)[CPL], float4& vr, float& dd) {
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        qv[c] = sq[tt * DK + c0 + c];
        kv[c] = sk[tt * DK + c0 + c];
      }
      vr = *(const float4*)(sv + tt * RB + r0);
      dd = sd[tt];
    };
    if (t0 + TC <= T) {
      constexpr int PD = LA_SCAN_PD;
      float rq[PD + 1][CPL], rk[PD + 1][CPL], rd[PD + 1];
      float4 rv[PD + 1];
      float keep = 0.f;
#pragma unroll
      for (int tt = 0; tt < PD && tt < TC; ++tt) fetch(tt, rq[tt], rk[tt], rv[tt], rd[tt]);
#pragma unroll
      for (int tt = 0; tt < TC; ++tt) {
        if (tt + PD < TC) {
          const int b = (tt + PD) % (PD + 1);
          fetch(tt + PD, rq[b], rk[b], rv[b], rd[b]);
        }
        const int b = tt % (PD + 1);
        const float ov = token(tt, rq[b], rk[b], rv[b], rd[b]);
        keep = tl == tt ? ov : keep;
      }
      if (tl < TC && rvalid) o[(t0 + tl) * vd + h * dv + row] = keep;
    } else {
      for (int tt = 0; tt < T - t0; ++tt) {
        float qv[CPL], kv[CPL], dd;
        float4 vr;
        fetch(tt, qv, kv, vr, dd);
        const float ov = token(tt, qv, kv, vr, dd);
        if (tl == 0 && rvalid) o[(t0 + tt) * vd + h * dv + row] = ov;
      }
    }
  });
}

template <int CPL, int L>
__global__ __launch_bounds__(256) void k_la_scan(const float* __restrict__ q,
                                                 const float* __restrict__ kb,
                                                 const float* __restrict__ v,
                                                 const float* __restrict__ decay, int T, int n,
                                                 int dv, int bph, float* __restrict__ o) {
  constexpr int DK = CPL * L, RW = 64 / L, RB = 4 * RW;
  using St = ScanStage<DK, RB>;
  constexpr int TC = St::TC, NQ = St::NQ, NV = St::NV;
  __shared__ __align__(16) float lds[2][St::BUF];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = blockIdx.x / bph;
  const int rb0 = (blockIdx.x - h * bph) * RB;  // first value row of this block in head h
  const int rr = lane / L, cg = lane % L;
  const int rloc = wave * RW + rr;  // row within the block
  const int row = rb0 + rloc;
  const bool rvalid = row < dv;
  const int c0 = cg * CPL;
  const int vd = n * dv;

  float S[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) S[c] = 0.f;

  la_chunks<St>(q, kb, v, decay, T, n, dv, h, rb0, lds, [&](const float* sq, int t0) {
    const float* sk = sq + NQ;
    const float* sv = sk + NQ;
    const float* sd = sv + NV;
    auto fetch = [&](int tt, float (&qv)[CPL], float (&kv)[CPL], float& vi, float& dd) {
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        qv[c] = sq[tt * DK + c0 + c];
        kv[c] = sk[tt * DK + c0 + c];
      }
      vi = sv[tt * RB + rloc];
      dd = sd[tt];
    };
    auto token = [&](const float (&qv)[CPL], const float (&kv)[CPL], float vi, float dd) {
      float part = 0.f;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        S[c] = S[c] * dd + vi * kv[c];
        part += S[c] * qv[c];
      }
      return la_row_sum<L>(part);
    };
    if (t0 + TC <= T) {
      // Lane cg of a row keeps the outputs of tokens cg, cg + L, ...
      constexpr int NK = (TC + L - 1) / L;
      constexpr int PD = LA_SCAN_PD;
      float keep[NK];
#pragma unroll
      for (int i = 0; i < NK; ++i) keep[i] = 0.f;
      float rq[PD + 1][CPL], rk[PD + 1][CPL], rv[PD + 1], rd[PD + 1];
#pragma unroll
      for (int tt = 0; tt < PD && tt < TC; ++tt) fetch(tt, rq[tt], rk[tt], rv[tt], rd[tt]);
#pragma unroll
      for (int tt = 0; tt < TC; ++tt) {
        if (tt + PD < TC) {
          const int b = (tt + PD) % (PD + 1);
          fetch(tt + PD, rq[b], rk[b], rv[b], rd[b]);
        }
        const int b = tt % (PD + 1);
        const float ov = token(rq[b], rk[b], rv[b], rd[b]);
        keep[tt / L] = cg == tt % L ? ov : keep[tt / L];
      }
#pragma unroll
      for (int i = 0; i < NK; ++i) {
        const int tt = i * L + cg;
        if (tt < TC && rvalid) o[(t0 + tt) * vd + h * dv + row] = keep[i];
      }
    } else {
      for (int tt = 0; tt < T - t0; ++tt) {
        float qv[CPL], kv[CPL], vi, dd;
        fetch(tt, qv, kv, vi, dd);
        const float ov = token(qv, kv, vi, dd);
        if (cg == 0 && rvalid) o[(t0 + tt) * vd + h * dv + row] = ov;
      }
    }
  });
}

template <int CPL, int L>
int launch_scan(const float* q, const float* kb, const float* v, const float* decay, int T,
                int n, int dv, float* o, hipStream_t s) {
  constexpr bool wide = L == 64;
  constexpr int RB = wide ? 16 : 4 * (64 / L);
  const int bph = mx_ceil_div(dv, RB);
  const long blocks = (long)n * bph;
  const long dmax = CPL * L > dv ? CPL * L : dv;
  if (blocks > (1l << 31) - 1 || (long)T * n * dmax >= (1l << 31)) return MX_ERR_UNSUPPORTED;
  if (!mx_aligned16(q) || !mx_aligned16(kb)) return MX_ERR_ALIGNMENT;
  mx_clear_error();
  if constexpr (wide)
    hipLaunchKernelGGL((k_la_scan_wide<CPL>), dim3((unsigned)blocks), dim3(256), 0, s, q, kb,
                       v, decay, T, n, dv, bph, o);
  else
    hipLaunchKernelGGL((k_la_scan<CPL, L>), dim3((unsigned)blocks), dim3(256), 0, s, q, kb, v,
                       decay, T, n, dv, bph, o);
  return mx_launch_status();
}

// Inputs of at least MX_LA_CHUNK_MIN_T tokens run the chunked form on MFMA (mx_la_chunk.hip)
// where it is built for the head sizes; shorter ones (a chain of a few tokens) and other
// head sizes the token-sequential scan.
#ifndef MX_LA_CHUNK_MIN_T
#define MX_LA_CHUNK_MIN_T 64
#endif
int scan_launch(const float* q, const float* kb, const float* v, const float* decay, int T,
                int n, int dk, int dv, float* o, void* chunk_ws, hipStream_t s) {
  if (T >= MX_LA_CHUNK_MIN_T && chunk_ws) {
    const int rc = mx_la_chunked_scan(q, kb, v, decay, T, n, dk, dv, o, chunk_ws, s);
    if (rc != MX_ERR_UNSUPPORTED) return rc;
  }
  switch (dk) {
    case 4: return launch_scan<4, 1>(q, kb, v, decay, T, n, dv, o, s);
    case 8: return launch_scan<8, 1>(q, kb, v, decay, T, n, dv, o, s);
    case 16: return launch_scan<8, 2>(q, kb, v, decay, T, n, dv, o, s);
    case 32: return launch_scan<8, 4>(q, kb, v, decay, T, n, dv, o, s);
    case 64: return launch_scan<1, 64>(q, kb, v, decay, T, n, dv, o, s);
    case 128: return launch_scan<2, 64>(q, kb, v, decay, T, n, dv, o, s);
    case 256: return launch_scan<4, 64>(q, kb, v, decay, T, n, dv, o, s);
    case 512: return launch_scan<8, 64>(q, kb, v, decay, T, n, dv, o, s);
    default: return MX_ERR_UNSUPPORTED;
  }
}

// Gated output norm: act = (w * (o / rms(o))) * silu(z) per token row (qwen3_next.py:
// 264-266, rms_norm of _common.py:73-75), written as fp16 (fp32 for fp32 weights).
template <int RV>
__global__ __launch_bounds__(256) void k_la_gated_norm(const float* __restrict__ o,
                                                       const float* __restrict__ qkvz,
                                                       const void* __restrict__ norm_w,
                                                       int pdt, float eps, LaDims m,
                                                       float* __restrict__ act32,
                                                       half_t* __restrict__ act16) {
#pragma clang fp contract(off)
  const int t = blockIdx.x;
  const float* orow = o + (size_t)t * m.vd;
  const float* z = qkvz + (size_t)t * m.W1 + 2 * m.qd + m.vd;
  __shared__ float red[4];
  if constexpr (RV > 0) {
    // The row fits the register tile (vd <= 256 RV): every load is issued up front.
    float ov[RV], zv[RV], wv[RV];
#pragma unroll
    for (int i = 0; i < RV; ++i) {
      const int c = min((int)threadIdx.x + 256 * i, m.vd - 1);
      ov[i] = orow[c];
      zv[i] = z[c];
      wv[i] = mx_load_param(norm_w, pdt, c);
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < RV; ++i)
      if ((int)threadIdx.x + 256 * i < m.vd) ss += ov[i] * ov[i];
    ss = mx_wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float rms = sqrtf(tot / (float)m.vd + eps);
#pragma unroll
    for (int i = 0; i < RV; ++i) {
      const int c = threadIdx.x + 256 * i;
      if (c >= m.vd) break;
      const float a = (wv[i] * (ov[i] / rms)) * mx_silu(zv[i]);
      if (act16)
        act16[(size_t)t * m.vd + c] = (half_t)a;
      else
        act32[(size_t)t * m.vd + c] = a;
    }
  } else {
    float ss = 0.f;
    for (int c = threadIdx.x; c < m.vd; c += 256) ss += orow[c] * orow[c];
    ss = mx_wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float rms = sqrtf(tot / (float)m.vd + eps);
    for (int c = threadIdx.x; c < m.vd; c += 256) {
      const float a = (mx_load_param(norm_w, pdt, c) * (orow[c] / rms)) * mx_silu(z[c]);
      if (act16)
        act16[(size_t)t * m.vd + c] = (half_t)a;
      else
        act32[(size_t)t * m.vd + c] = a;
    }
  }
}

__global__ __launch_bounds__(256) void k_la_residual(const float* __restrict__ x,
                                                     const float* __restrict__ y, long n4,
                                                     float* __restrict__ out) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i < n4) {
    const float4 a = ((const float4*)x)[i], b = ((const float4*)y)[i];
    ((float4*)out)[i] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
  }
}

int check_weights(const MxLinearAttnDesc* d, const MxLinearAttnWeights* w) {
  if (!w || !w->norm_w || !w->qkvz_w || !w->ba_w || !w->conv_w || !w->a_log || !w->dt_bias ||
      !w->out_norm_w || !w->out_w)
    return MX_ERR_INVALID;
  if (d->weight_dtype == MX_DT_I8 && (!w->qkvz_scale || !w->ba_scale || !w->out_scale))
    return MX_ERR_INVALID;
  if (!mx_aligned16(w->qkvz_w) || !mx_aligned16(w->ba_w) || !mx_aligned16(w->out_w))
    return MX_ERR_ALIGNMENT;
  return MX_OK;
}

int run_stage(int st, const MxLinearAttnDesc* d, const MxLinearAttnWeights* w, const float* x,
              float* out, int T, const LaWork& k, hipStream_t s) {
  const LaDims m = dims_of(d);
  const int wdt = d->weight_dtype;
  const bool f32 = wdt == MX_DT_F32;
  const void* h = f32 ? (const void*)k.v.h32 : k.v.h16;
  switch (st) {
    case 0: {
      MxDenseEntries e = {};
      e.e[0].down = w->qkvz_w;
      e.e[0].down_scale = w->qkvz_scale;
      e.e[1].down = w->ba_w;
      e.e[1].down_scale = w->ba_scale;
      e.e[2].down = w->out_w;
      e.e[2].down_scale = w->out_scale;
      MX_TRY(mx_dense_setup(k.dw, e, T, s));
      return mx_rmsnorm_launch(x, w->norm_w, d->param_dtype, d->eps, T, m.H, k.v.h32, k.v.h16,
                               s);
    }
    case 1:
      if (mx_dense_on_gemm(wdt, T, m.H)) {  // qkvz and ba share h: one GEMM launch
        const MxGemmSeg g[2] = {{w->qkvz_w, k.v.qkvz, m.W1, m.W1}, {w->ba_w, k.v.ba, m.W2, m.W2}};
        return mx_gemm_f16(h, T, m.H, g, 2, s);
      }
      return mx_project(k.dw, 0, wdt, w->qkvz_w, T, m.W1, m.H, h, k.v.qkvz, s);
    case 2:
      if (mx_dense_on_gemm(wdt, T, m.H)) return MX_OK;  // with qkvz in stage 1
      return mx_project(k.dw, 1, wdt, w->ba_w, T, m.W2, m.H, h, k.v.ba, s);
    case 3: {
      const dim3 grid(mx_ceil_div(m.C + m.n, 256), mx_ceil_div(T, LA_TT));
      mx_clear_error();
      if (m.K == 4)
        hipLaunchKernelGGL(k_la_prep<4>, grid, dim3(256), 0, s, k.v.qkvz, k.v.ba, w->conv_w,
                           w->a_log, w->dt_bias, d->param_dtype, m, T, k.v.q, k.v.kb, k.v.v,
                           k.v.decay);
      else
        hipLaunchKernelGGL(k_la_prep<0>, grid, dim3(256), 0, s, k.v.qkvz, k.v.ba, w->conv_w,
                           w->a_log, w->dt_bias, d->param_dtype, m, T, k.v.q, k.v.kb, k.v.v,
                           k.v.decay);
      return mx_launch_status();
    }
    case 4:
      return scan_launch(k.v.q, k.v.kb, k.v.v, k.v.decay, T, m.n, m.dk, m.dv, k.v.o, k.chunk_ws,
                         s);
    case 5:
      mx_clear_error();
      if (m.vd <= 256 * 4)
        hipLaunchKernelGGL(k_la_gated_norm<4>, dim3(T), dim3(256), 0, s, k.v.o, k.v.qkvz,
                           w->out_norm_w, d->param_dtype, d->eps, m, (float*)k.v.act,
                           f32 ? nullptr : (half_t*)k.v.act);
      else if (m.vd <= 256 * 16)
        hipLaunchKernelGGL(k_la_gated_norm<16>, dim3(T), dim3(256), 0, s, k.v.o, k.v.qkvz,
                           w->out_norm_w, d->param_dtype, d->eps, m, (float*)k.v.act,
                           f32 ? nullptr : (half_t*)k.v.act);
      else
        hipLaunchKernelGGL(k_la_gated_norm<0>, dim3(T), dim3(256), 0, s, k.v.o, k.v.qkvz,
                           w->out_norm_w, d->param_dtype, d->eps, m, (float*)k.v.act,
                           f32 ? nullptr : (half_t*)k.v.act);
      return mx_launch_status();
    case 6:
      if (mx_dense_on_gemm(wdt, T, m.vd)) {  // out = x + act W_out^T in the GEMM epilogue
        if (!x || !out) return MX_ERR_INVALID;
        const MxGemmSeg g{w->out_w, out, m.H, m.H, nullptr, x};
        return mx_gemm_f16(k.v.act, T, m.vd, &g, 1, s);
      }
      return mx_project(k.dw, 2, wdt, w->out_w, T, m.H, m.vd, k.v.act, k.v.y, s);
    case 7: {
      if (mx_dense_on_gemm(wdt, T, m.vd)) return MX_OK;  // added in stage 6
      const long n4 = (long)T * m.H / 4;
      mx_clear_error();
      hipLaunchKernelGGL(k_la_residual, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, x,
                         k.v.y, n4, out);
      return mx_launch_status();
    }
    default:
      return MX_ERR_INVALID;
  }
}

int forward(const MxLinearAttnDesc* d, const MxLinearAttnWeights* w, const float* x, float* out,
            int T, void* ws, size_t ws_bytes, hipStream_t s, void* const* events) {
  MX_TRY(check_desc(d));
  MX_TRY(check_weights(d, w));
  if (!x || !out || !ws || T < 0) return MX_ERR_INVALID;
  if (d->hidden % 4) return MX_ERR_UNSUPPORTED;  // float4 residual
  if (!mx_aligned16(x) || !mx_aligned16(out)) return MX_ERR_ALIGNMENT;
  if (T == 0) return MX_OK;
  LaWork k;
  size_t need = 0;
  MX_TRY(layout(d, T, ws, &k, &need));
  if (ws_bytes < need) return MX_ERR_WORKSPACE;
  for (int st = 0; st < MX_LA_N_STAGES; ++st) {
    if (events) MX_TRY(mx_status(hipEventRecord((hipEvent_t)events[st], s)));
    MX_TRY(run_stage(st, d, w, x, out, T, k, s));
  }
  if (events) MX_TRY(mx_status(hipEventRecord((hipEvent_t)events[MX_LA_N_STAGES], s)));
  return MX_OK;
}

}  // namespace

extern "C" int mx_linear_attn_workspace_size(const MxLinearAttnDesc* desc, int32_t tokens,
                                             size_t* nbytes) {
  if (!nbytes) return MX_ERR_INVALID;
  return layout(desc, tokens, nullptr, nullptr, nbytes);
}

extern "C" int mx_linear_attn_views(const MxLinearAttnDesc* desc, int32_t tokens,
                                    void* workspace, MxLinearAttnViews* views) {
  if (!workspace || !views) return MX_ERR_INVALID;
  LaWork k;
  MX_TRY(layout(desc, tokens, workspace, &k, nullptr));
  *views = k.v;
  return MX_OK;
}

extern "C" int mx_linear_attn_forward(const MxLinearAttnDesc* desc,
                                      const MxLinearAttnWeights* weights, const float* x,
                                      float* out, int32_t tokens, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  return forward(desc, weights, x, out, tokens, workspace, workspace_bytes, (hipStream_t)stream,
                 nullptr);
}

extern "C" int mx_linear_attn_forward_profiled(const MxLinearAttnDesc* desc,
                                               const MxLinearAttnWeights* weights,
                                               const float* x, float* out, int32_t tokens,
                                               void* workspace, size_t workspace_bytes,
                                               void* stream, void* const* events,
                                               int32_t n_events) {
  if (!events || n_events != MX_LA_N_STAGES + 1) return MX_ERR_INVALID;
  for (int i = 0; i < n_events; ++i)
    if (!events[i]) return MX_ERR_INVALID;
  return forward(desc, weights, x, out, tokens, workspace, workspace_bytes, (hipStream_t)stream,
                 events);
}

extern "C" int mx_gated_delta_scan(const float* q, const float* kb, const float* v,
                                   const float* decay, int32_t tokens, int32_t n_heads,
                                   int32_t head_dim_k, int32_t head_dim_v, float* o,
                                   void* stream) {
  if (!q || !kb || !v || !decay || !o || tokens < 0 || n_heads <= 0 || head_dim_k <= 0 ||
      head_dim_v <= 0)
    return MX_ERR_INVALID;
  if (tokens == 0) return MX_OK;
  return scan_launch(q, kb, v, decay, tokens, n_heads, head_dim_k, head_dim_v, o, nullptr,
                     (hipStream_t)stream);
}

extern "C" int mx_gated_delta_scan_workspace_size(int32_t tokens, int32_t n_heads,
                                                  int32_t head_dim_k, int32_t head_dim_v,
                                                  size_t* nbytes) {
  if (!nbytes || tokens < 0 || n_heads <= 0 || head_dim_k <= 0 || head_dim_v <= 0)
    return MX_ERR_INVALID;
  *nbytes = tokens >= MX_LA_CHUNK_MIN_T
                ? mx_la_chunk_ws_bytes(tokens, n_heads, head_dim_k, head_dim_v)
                : 0;
  return MX_OK;
}

extern "C" int mx_gated_delta_scan_ws(const float* q, const float* kb, const float* v,
                                      const float* decay, int32_t tokens, int32_t n_heads,
                                      int32_t head_dim_k, int32_t head_dim_v, float* o,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !kb || !v || !decay || !o || tokens < 0 || n_heads <= 0 || head_dim_k <= 0 ||
      head_dim_v <= 0)
    return MX_ERR_INVALID;
  if (tokens == 0) return MX_OK;
  size_t need = 0;
  MX_TRY(mx_gated_delta_scan_workspace_size(tokens, n_heads, head_dim_k, head_dim_v, &need));
  if (need && (!workspace || workspace_bytes < need)) return MX_ERR_WORKSPACE;
  return scan_launch(q, kb, v, decay, tokens, n_heads, head_dim_k, head_dim_v, o,
                     need ? workspace : nullptr, (hipStream_t)stream);
}
