// Chunked form of the gated recurrence of the Qwen3-Next linear-attention block
// (offload_runtime/executors/qwen3_next.py:56-95, with beta * k formed):
//   S_t = d_t S_{t-1} + v_t kb_t^T,   o_t = S_t q_t,   S_0 = 0     (per head, d_t = exp(g_t))
// on fp32 MFMA (v_mfma_f32_16x16x4_f32, full fp32 products and sums).
//
// Over a chunk of C = 64 tokens starting at t0, with S_p the state before the chunk and
// a(t, s) = d_{s+1} ... d_t the decay between tokens s <= t (a(t, t) = 1):
//   o_t = sum_{t0 <= s <= t} a(t, s) (kb_s . q_t) v_s  +  a(t, t0 - 1) S_p q_t
//   S_end = a(end, t0 - 1) S_p + sum_s a(end, s) v_s kb_s^T
// which is the recurrence unrolled over the chunk (exact in real arithmetic).  The first
// sum (intra-chunk) needs no state: k_la_chunk_intra computes it for every (head, chunk)
// in parallel as (Q Kb^T masked and scaled by a) V, writes it to o, and writes the chunk's
// decay coefficients to a small buffer.  The second part walks the chunks of a head in
// order: k_la_chunk_state holds 16 state rows of one head in MFMA accumulators, adds
// a(t, t0 - 1) S_p q_t to o and updates S, one chunk at a time.
//
// The decay factors are formed in double precision from the fp32 decays the reference
// multiplies by: with G_t = sum over the chunk of log(d_r) up to t, a(t, s) =
// exp(G_t - G_s).  A zero decay (exp(g) underflowed) zeroes the state; such a token starts
// a new segment (G restarts at 0 there and factors across it are 0), so no logarithm of
// zero is taken and no difference of huge sums is formed.
#include <math.h>

#include "mx_common.h"
#include "mx_internal.h"

namespace {

constexpr int kC = 64;  // tokens per chunk

typedef __amdgpu_buffer_rsrc_t mx_rsrc_t;

// Buffer descriptor over `bytes` bytes: loads at offsets past the end return zeros.
__device__ __forceinline__ mx_rsrc_t mx_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ int4_t mx_ld16(mx_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

__device__ __forceinline__ float4_t mfma4(float a, float b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Sum over a 16-column group: lane (j, q) holds 4 consecutive columns 4q .. 4q + 3 of its
// A row and of its B column; MFMA e takes element e, so every column is summed once.
__device__ __forceinline__ float4_t mfma_k16(const float4& a, const float4& b, float4_t c) {
  c = mfma4(a.x, b.x, c);
  c = mfma4(a.y, b.y, c);
  c = mfma4(a.z, b.z, c);
  return mfma4(a.w, b.w, c);
}

__device__ __forceinline__ double shfl_up_d(double v, int d) {
  const int lo = __shfl_up(__double2loint(v), d, 64);
  const int hi = __shfl_up(__double2hiint(v), d, 64);
  return __hiloint2double(hi, lo);
}

__device__ __forceinline__ double shfl_d(double v, int src) {
  const int lo = __shfl(__double2loint(v), src, 64);
  const int hi = __shfl(__double2hiint(v), src, 64);
  return __hiloint2double(hi, lo);
}

// One wave, lane l = token t0 + l of the chunk: G_l (log decay from the segment start up to
// and including l) and the last zero-decay token at or before l (-1: none in the chunk).
// Tokens past T take d = 1.
__device__ __forceinline__ void chunk_log_decay(const float* __restrict__ decay, int t0, int T,
                                                int n, int h, double* sG, int* sLR) {
  const int l = threadIdx.x & 63;
  const int t = t0 + l;
  const float d = t < T ? decay[(size_t)t * n + h] : 1.f;
  const bool reset = t < T && !(d > 0.f);
  double p = (d > 0.f) ? log((double)d) : 0.0;
  int lr = reset ? l : -1;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const double pu = shfl_up_d(p, off);
    const int lu = __shfl_up(lr, off, 64);
    if (l >= off) {
      p += pu;
      lr = max(lr, lu);
    }
  }
  const double pr = shfl_d(p, lr >= 0 ? lr : 0);
  sG[l] = lr >= 0 ? p - pr : p;
  sLR[l] = lr;
}

// Coefficients the state walk reads per (head, chunk): a(t, t0 - 1) for the 64 tokens, then
// a(end, s) for the 64 tokens, then a(end, t0 - 1) (padded to 132 floats).
constexpr int kCoef = 132;

// LDS row strides in floats: (stride / 4) odd, so the 16-byte reads of 16 consecutive rows
// at one column group hit distinct bank groups.
template <int W>
struct Pad {
  static constexpr int S = W + 4;
};

// ---- intra-chunk part: o[t] = sum_{t0 <= s <= t} a(t, s) (kb_s . q_t) v_s ---------------
// Block (chunk, head), 4 waves; wave w takes tokens 16 w .. 16 w + 15 of the chunk.  Its q
// rows go straight into MFMA A registers; kb (B of the scores, all 64 tokens) and v (B of
// the products with v) are shared through LDS (row-major, 16-byte stores), and the kb
// region is then reused for each wave's masked scores (A of the products with v).  Wave 0
// also writes the chunk's coefficients for the state walk.
template <int DK, int DV>
__global__ __launch_bounds__(256, 2) void k_la_chunk_intra(const float* __restrict__ q,
                                                           const float* __restrict__ kb,
                                                           const float* __restrict__ v,
                                                           const float* __restrict__ decay,
                                                           int T, int n, int nchunk,
                                                           float* __restrict__ o,
                                                           float* __restrict__ coef) {
  constexpr int SK = Pad<DK>::S, SC = Pad<kC>::S, SV = Pad<DV>::S;
  constexpr int KP = kC * DK / 4 / 256, VP = kC * DV / 4 / 256;  // float4 pieces per thread
  static_assert(4 * 16 * SC <= kC * SK, "masked scores reuse the kb tile");
  __shared__ __align__(16) float sK[kC * SK];    // kb tile, then the masked scores
  __shared__ __align__(16) float sV[kC * SV];    // v tile [token][value row]
  __shared__ double sG[kC];
  __shared__ int sLR[kC];

  const int chunk = blockIdx.x % nchunk, h = blockIdx.x / nchunk;
  const int t0 = chunk * kC;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int j = lane & 15, qq = lane >> 4;
  const int qd = n * DK, vd = n * DV;

  // every global load of the block first, then the LDS stores
  float4 qa[DK / 16];
  const int tq = t0 + 16 * w + j;
#pragma unroll
  for (int u = 0; u < DK / 16; ++u)
    qa[u] = tq < T ? *(const float4*)(q + (size_t)tq * qd + h * DK + 16 * u + 4 * qq)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
  float4 kr[KP], vr[VP];
#pragma unroll
  for (int p = 0; p < KP; ++p) {
    const int i = tid + 256 * p, r = i / (DK / 4), c = 4 * (i % (DK / 4)), t = t0 + r;
    kr[p] = t < T ? *(const float4*)(kb + (size_t)t * qd + h * DK + c)
                  : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int p = 0; p < VP; ++p) {
    const int i = tid + 256 * p, r = i / (DV / 4), c = 4 * (i % (DV / 4)), t = t0 + r;
    vr[p] = t < T ? *(const float4*)(v + (size_t)t * vd + h * DV + c)
                  : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (w == 0) chunk_log_decay(decay, t0, T, n, h, sG, sLR);
#pragma unroll
  for (int p = 0; p < KP; ++p) {
    const int i = tid + 256 * p, r = i / (DK / 4), c = 4 * (i % (DK / 4));
    *(float4*)(sK + r * SK + c) = kr[p];
  }
#pragma unroll
  for (int p = 0; p < VP; ++p) {
    const int i = tid + 256 * p, r = i / (DV / 4), c = 4 * (i % (DV / 4));
    *(float4*)(sV + r * SV + c) = vr[p];
  }
  __syncthreads();

  // scores of this wave's 16 tokens against the chunk's 64: P = Q Kb^T
  float4_t pacc[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) pacc[nt] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < DK / 16; ++u) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const float4 b = *(const float4*)(sK + (16 * nt + j) * SK + 16 * u + 4 * qq);
      pacc[nt] = mfma_k16(qa[u], b, pacc[nt]);
    }
  }
  __syncthreads();  // every wave is done with the kb tile: its region takes the scores
  // causal mask and decay factors; lane (j, qq) holds P[16 w + 4 qq + r][16 nt + j]
  float* myP = sK + w * 16 * SC;
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tl = 16 * w + 4 * qq + r, sl = 16 * nt + j;
      const float f = (sl <= tl && sLR[tl] <= sl) ? expf((float)(sG[tl] - sG[sl])) : 0.f;
      myP[(4 * qq + r) * SC + sl] = pacc[nt][r] * f;
    }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");

  // o = P V over the chunk's 64 tokens; token s = k0 + 4 qq + e of v row 16 nt + j (four
  // rows per lane, one value each: lane groups qq sit 16 banks apart)
  constexpr int NV = DV / 16;
  float4_t oacc[NV];
#pragma unroll
  for (int nt = 0; nt < NV; ++nt) oacc[nt] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k0 = 0; k0 < kC; k0 += 16) {
    const float4 a = *(const float4*)(myP + j * SC + k0 + 4 * qq);
#pragma unroll
    for (int nt = 0; nt < NV; ++nt) {
      const float* vp = sV + (k0 + 4 * qq) * SV + 16 * nt + j;
      const float4 b = make_float4(vp[0], vp[SV], vp[2 * SV], vp[3 * SV]);
      oacc[nt] = mfma_k16(a, b, oacc[nt]);
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = t0 + 16 * w + 4 * qq + r;
    if (t < T) {
#pragma unroll
      for (int nt = 0; nt < NV; ++nt) o[(size_t)t * vd + h * DV + 16 * nt + j] = oacc[nt][r];
    }
  }
  if (w == 0) {
    // coefficients of the state walk, lane l = token l of the chunk
    const int l = lane;
    const int lastv = min(kC, T - t0) - 1;
    const double ge = sG[lastv], gl = sG[l];
    const int lre = sLR[lastv];
    float* cf = coef + ((size_t)h * nchunk + chunk) * kCoef;
    cf[l] = sLR[l] < 0 ? expf((float)gl) : 0.f;
    cf[kC + l] = (l <= lastv && lre <= l) ? expf((float)(ge - gl)) : 0.f;
    if (l == 0) cf[2 * kC] = lre < 0 ? expf((float)ge) : 0.f;
  }
}

// ---- state part: o[t] += a(t, t0 - 1) S_p q_t, then S <- a(end) S_p + sum a(end, s) v kb^T
// Block (head, 16 value rows), 4 waves, walking the chunks in order.  The block keeps the
// transposed state rows S^T[c][i] (c: key column, i: one of its 16 value rows) in MFMA
// accumulators, wave w holding key columns 16 NT w .. 16 NT (w + 1) - 1; lane (j, qq) of a
// tile holds S^T[4 qq + r][j], which is exactly the B operand of the output product when
// lane group qq sums key columns 4 qq .. 4 qq + 3, so the state never leaves registers.
// Each wave forms the output over its own key columns for all 64 tokens (its q columns go
// straight into A registers); the four partial outputs are summed through LDS and added
// to the intra-chunk part already in o.  kb and v enter the state product with 4 tokens
// per lane, so their rows are staged through LDS (row-major, 16-byte stores), double-
// buffered: the next chunk's rows are loaded while this one computes and written to the
// other buffer after it.  Loads go through buffer descriptors (rows past T read zero).
template <int DK>
__global__ __launch_bounds__(256) void k_la_chunk_state(const float* __restrict__ q,
                                                        const float* __restrict__ kb,
                                                        const float* __restrict__ v,
                                                        const float* __restrict__ coef, int T,
                                                        int n, int dv, int nchunk,
                                                        float* __restrict__ o) {
  constexpr int NT = DK / 64;                  // 16-column state tiles per wave
  constexpr int SK = Pad<DK>::S;               // LDS row stride of the kb rows
  constexpr int SV = 16 + 4;                   // LDS row stride of the v rows
  constexpr int SO = 16 + 1;                   // LDS row stride of a partial output
  constexpr int KP = kC * DK / 4 / 256;        // kb float4 pieces per thread and chunk
  __shared__ __align__(16) float sK[2][kC * SK];  // kb rows [token][key column]
  __shared__ __align__(16) float sV[2][kC * SV];  // this block's v columns [token][row]
  __shared__ __align__(16) float sCf[2][kCoef];
  __shared__ float sO[4][kC * SO];

  // Every block of a head reads the same q and kb rows: the blocks of one head run on one
  // XCD (hardware block b runs on XCD b % 8), so those rows come from that XCD's L2 after
  // the first block's read.
  const int bph = dv / 16;  // blocks per head
  int h, slice;
  if ((n & 7) == 0) {
    const int k = blockIdx.x >> 3;
    h = (blockIdx.x & 7) * (n >> 3) + k / bph;
    slice = k % bph;
  } else {
    h = blockIdx.x / bph;
    slice = blockIdx.x % bph;
  }
  const int i0 = 16 * slice;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int j = lane & 15, qq = lane >> 4;
  const int qd = n * DK, vd = n * dv;
  const int cw = 16 * NT * w;  // this wave's first key column
  const uint32_t qrow = (uint32_t)qd * 4, vrow = (uint32_t)vd * 4;
  const mx_rsrc_t rq = mx_rsrc(q, (uint32_t)T * qrow);
  const mx_rsrc_t rk = mx_rsrc(kb, (uint32_t)T * qrow);
  const mx_rsrc_t rv = mx_rsrc(v, (uint32_t)T * vrow);
  const mx_rsrc_t rc = mx_rsrc(coef, (uint32_t)(n * nchunk * kCoef * 4));

  // per-lane offsets: q fragment (token j of a 16-row group, columns cw + 4 qq ..), kb and v
  // rows staged by this thread, coefficients
  const uint32_t q_lane = (uint32_t)j * qrow + (uint32_t)(h * DK + cw + 4 * qq) * 4;
  uint32_t k_lane[KP];
  int k_lds[KP];
#pragma unroll
  for (int p = 0; p < KP; ++p) {
    const int i = tid + 256 * p, r = i / (DK / 4), c = 4 * (i % (DK / 4));
    k_lane[p] = (uint32_t)r * qrow + (uint32_t)(h * DK + c) * 4;
    k_lds[p] = r * SK + c;
  }
  const int vr = tid >> 2, vc = 4 * (tid & 3);  // v: token vr, rows i0 + vc .. + 3
  const uint32_t v_lane = (uint32_t)vr * vrow + (uint32_t)(h * dv + i0 + vc) * 4;

  struct Staged {
    int4_t k[KP];
    int4_t v;
    int4_t cf;
  };
  auto load_staged = [&](Staged& x, int ch) {
    const uint32_t base = (uint32_t)ch * kC * qrow;
#pragma unroll
    for (int p = 0; p < KP; ++p) x.k[p] = mx_ld16(rk, k_lane[p] + base);
    x.v = mx_ld16(rv, v_lane + (uint32_t)ch * kC * vrow);
    x.cf = tid < kCoef / 4 ? mx_ld16(rc, (uint32_t)(((size_t)h * nchunk + ch) * kCoef * 4 + 16 * tid))
                           : (int4_t){0, 0, 0, 0};
  };
  auto store_staged = [&](const Staged& x, int b) {
#pragma unroll
    for (int p = 0; p < KP; ++p) *(int4_t*)(sK[b] + k_lds[p]) = x.k[p];
    *(int4_t*)(sV[b] + vr * SV + vc) = x.v;
    if (tid < kCoef / 4) *(int4_t*)(sCf[b] + 4 * tid) = x.cf;
  };
  struct Direct {
    int4_t qf[4][NT];  // q[t0 + 16 mt + j][cw + 16 u + 4 qq ..]  (A of the output product)
    float oi[4];       // intra-chunk o of token 16 w + 4 qq + r, row i0 + j
  };
  auto load_direct = [&](Direct& x, int ch) {
    const uint32_t base = (uint32_t)ch * kC * qrow;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int u = 0; u < NT; ++u)
        x.qf[mt][u] = mx_ld16(rq, q_lane + base + (uint32_t)(16 * mt) * qrow + 64u * u);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = ch * kC + 16 * w + 4 * qq + r;
      x.oi[r] = t < T ? o[(size_t)t * vd + h * dv + i0 + j] : 0.f;
    }
  };

  float4_t st[NT];
#pragma unroll
  for (int u = 0; u < NT; ++u) st[u] = (float4_t){0.f, 0.f, 0.f, 0.f};

  // one chunk: operands in LDS buffer b and in x.  The output product reads the old state
  // and the new contribution goes into fresh accumulators, so the two groups of MFMAs (four
  // independent chains each, no VALU between them) do not wait on each other; the state is
  // combined at the end: S^T <- a(end) S^T + U^T.
  auto step = [&](const Direct& x, int ch, int b) {
    const float* cf = sCf[b];
    // contribution U^T = sum_s kb_s (a(end, s) v_s)^T: B operands first (v times a(end, s))
    // token s = 16 kg + 4 qq + e: kb[s][cw + 16 u + j] (A) and v[s][i0 + j] a(end, s) (B),
    // four rows per lane read one value each (lane groups qq sit 16 banks apart)
    float bv[4][4];
#pragma unroll
    for (int kg = 0; kg < 4; ++kg) {
      const float4 ws = *(const float4*)(cf + kC + 16 * kg + 4 * qq);
      const float* vp = sV[b] + (16 * kg + 4 * qq) * SV + j;
      bv[kg][0] = vp[0] * ws.x;
      bv[kg][1] = vp[SV] * ws.y;
      bv[kg][2] = vp[2 * SV] * ws.z;
      bv[kg][3] = vp[3 * SV] * ws.w;
    }
    float4 ka[4][NT];
#pragma unroll
    for (int kg = 0; kg < 4; ++kg)
#pragma unroll
      for (int u = 0; u < NT; ++u) {
        const float* kp = sK[b] + (16 * kg + 4 * qq) * SK + cw + 16 * u + j;
        ka[kg][u] = make_float4(kp[0], kp[SK], kp[2 * SK], kp[3 * SK]);
      }
    // partial output over this wave's key columns, all 64 tokens: (q_t S^T) scaled by a(t)
    float4_t op[4], ua[NT], ub[NT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) op[mt] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NT; ++u) ua[u] = ub[u] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NT; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          const float4 a = __builtin_bit_cast(float4, x.qf[mt][u]);
          const float av = e == 0 ? a.x : (e == 1 ? a.y : (e == 2 ? a.z : a.w));
          op[mt] = mfma4(av, st[u][e], op[mt]);
        }
        // two state chains per tile: token groups 0-1 and 2-3
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const float4 k0 = ka[2 * kh][u], k1 = ka[2 * kh + 1][u];
          const float ka0 = e == 0 ? k0.x : (e == 1 ? k0.y : (e == 2 ? k0.z : k0.w));
          const float ka1 = e == 0 ? k1.x : (e == 1 ? k1.y : (e == 2 ? k1.z : k1.w));
          float4_t& acc = kh == 0 ? ua[u] : ub[u];
          acc = mfma4(ka0, bv[2 * kh][e], acc);
          acc = mfma4(ka1, bv[2 * kh + 1][e], acc);
        }
      }
    const float gam = cf[2 * kC];
#pragma unroll
    for (int u = 0; u < NT; ++u) st[u] = st[u] * gam + ua[u] + ub[u];
    // lane (j, qq) holds op[mt][r] for token 16 mt + 4 qq + r, row j
    float* so = sO[w];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        so[(16 * mt + 4 * qq + r) * SO + j] = op[mt][r] * cf[16 * mt + 4 * qq + r];
    (void)ch;
  };
  auto finish = [&](const Direct& x, int ch) {
    const int t0 = ch * kC;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tl = 16 * w + 4 * qq + r, t = t0 + tl;
      float sum = x.oi[r];
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) sum += sO[w2][tl * SO + j];
      if (t < T) o[(size_t)t * vd + h * dv + i0 + j] = sum;
    }
  };

  Staged sg;
  Direct da, db;
  load_staged(sg, 0);
  load_direct(da, 0);
  store_staged(sg, 0);
  __syncthreads();
  // Iteration ch: loads of chunk ch + 1 in flight while chunk ch computes from LDS buffer
  // ch & 1; the staged rows then go to the other buffer.  Two chunks per pass so the
  // direct operands alternate between two register sets without copies.
  for (int ch = 0; ch < nchunk; ch += 2) {
    const bool more1 = ch + 1 < nchunk;
    if (more1) {
      load_staged(sg, ch + 1);
      load_direct(db, ch + 1);
    }
    step(da, ch, 0);
    __syncthreads();  // partial outputs complete; LDS buffer 0 read
    finish(da, ch);
    if (more1) store_staged(sg, 1);
    __syncthreads();  // buffer 1 written, partial outputs read
    if (!more1) break;
    const bool more2 = ch + 2 < nchunk;
    if (more2) {
      load_staged(sg, ch + 2);
      load_direct(da, ch + 2);
    }
    step(db, ch + 1, 1);
    __syncthreads();
    finish(db, ch + 1);
    if (more2) store_staged(sg, 0);
    __syncthreads();
  }
}

template <int DK, int DV>
int launch_chunked(const float* q, const float* kb, const float* v, const float* decay, int T,
                   int n, float* o, float* coef, hipStream_t s) {
  const int nchunk = (T + kC - 1) / kC;
  mx_clear_error();
  hipLaunchKernelGGL((k_la_chunk_intra<DK, DV>), dim3((unsigned)(nchunk * n)), dim3(256), 0, s,
                     q, kb, v, decay, T, n, nchunk, o, coef);
  MX_TRY(mx_launch_status());
  hipLaunchKernelGGL((k_la_chunk_state<DK>), dim3((unsigned)(n * (DV / 16))), dim3(256), 0, s,
                     q, kb, v, coef, T, n, DV, nchunk, o);
  return mx_launch_status();
}

bool chunk_shape(int dk, int dv) { return (dk == 64 || dk == 128) && (dv == 64 || dv == 128); }

}  // namespace

size_t mx_la_chunk_coef_bytes(int T, int n, int dk, int dv) {
  if (T <= 0 || !chunk_shape(dk, dv)) return 0;
  return (size_t)n * ((T + kC - 1) / kC) * kCoef * sizeof(float);
}

// Chunked scan for the head shapes it is built for (key and value heads of 64 or 128), with
// `coef` of mx_la_chunk_coef_bytes; MX_ERR_UNSUPPORTED for other shapes (the caller then
// runs the token-sequential scan).
int mx_la_chunked_scan(const float* q, const float* kb, const float* v, const float* decay,
                       int T, int n, int dk, int dv, float* o, void* coef, hipStream_t s) {
  if (T <= 0 || n <= 0) return MX_ERR_INVALID;
  if (!chunk_shape(dk, dv) || !coef) return MX_ERR_UNSUPPORTED;
  // buffer descriptors: byte offsets below 2^31
  if ((long)T * n * (dk > dv ? dk : dv) * 4 >= (1l << 31)) return MX_ERR_UNSUPPORTED;
  if (!mx_aligned16(q) || !mx_aligned16(kb) || !mx_aligned16(v) || !mx_aligned16(o) ||
      !mx_aligned16(coef))
    return MX_ERR_UNSUPPORTED;
  float* cf = (float*)coef;
  if (dk == 128 && dv == 128) return launch_chunked<128, 128>(q, kb, v, decay, T, n, o, cf, s);
  if (dk == 64 && dv == 64) return launch_chunked<64, 64>(q, kb, v, decay, T, n, o, cf, s);
  if (dk == 128 && dv == 64) return launch_chunked<128, 64>(q, kb, v, decay, T, n, o, cf, s);
  return launch_chunked<64, 128>(q, kb, v, decay, T, n, o, cf, s);
}
