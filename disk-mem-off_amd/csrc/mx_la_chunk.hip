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
// rows go straight into MFMA A registers; kb (B of the scores, all 64 tokens) and v
// (transposed, B of the products with v) are shared through LDS, and the scores' LDS
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
  constexpr int SK = Pad<DK>::S, SC = Pad<kC>::S;
  constexpr int KP = kC * DK / 4 / 256, VP = kC * DV / 4 / 256;  // float4 pieces per thread
  static_assert(4 * 16 * SC <= kC * SK, "masked scores reuse the kb tile");
  __shared__ __align__(16) float sK[kC * SK];    // kb tile, then the masked scores
  __shared__ __align__(16) float sVt[DV * SC];   // v transposed: [value row][token]
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
    sVt[(c + 0) * SC + r] = vr[p].x;
    sVt[(c + 1) * SC + r] = vr[p].y;
    sVt[(c + 2) * SC + r] = vr[p].z;
    sVt[(c + 3) * SC + r] = vr[p].w;
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

  // o = P V over the chunk's 64 tokens
  constexpr int NV = DV / 16;
  float4_t oacc[NV];
#pragma unroll
  for (int nt = 0; nt < NV; ++nt) oacc[nt] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k0 = 0; k0 < kC; k0 += 16) {
    const float4 a = *(const float4*)(myP + j * SC + k0 + 4 * qq);
#pragma unroll
    for (int nt = 0; nt < NV; ++nt) {
      const float4 b = *(const float4*)(sVt + (16 * nt + j) * SC + k0 + 4 * qq);
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
// Each wave forms the output over its own key columns for all 64 tokens; the four partial
// outputs are summed through LDS (double-buffered, one barrier per chunk) and added to the
// intra-chunk part already in o.  The next chunk's operands are loaded while this one
// computes.
template <int DK>
__global__ __launch_bounds__(256) void k_la_chunk_state(const float* __restrict__ q,
                                                        const float* __restrict__ kb,
                                                        const float* __restrict__ v,
                                                        const float* __restrict__ coef, int T,
                                                        int n, int dv, int nchunk,
                                                        float* __restrict__ o) {
  constexpr int NT = DK / 64;  // 16-column state tiles per wave
  constexpr int SO = 16 + 1;   // LDS row stride of a partial output (tokens x 16 rows)
  __shared__ float sO[2][4][kC * SO];

  const int blocks_per_head = dv / 16;
  const int h = blockIdx.x / blocks_per_head, i0 = 16 * (blockIdx.x % blocks_per_head);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int j = lane & 15, qq = lane >> 4;
  const int qd = n * DK, vd = n * dv;
  const int cw = 16 * NT * w;  // this wave's first key column

  // operands of one chunk, in registers
  struct Ops {
    float4 qf[4][NT];  // q[t0 + 16 mt + j][cw + 16 u + 4 qq ..]          (A, output)
    float kf[4][NT][4];  // kb[t0 + 16 kg + 4 qq + e][cw + 16 u + j]        (A, state)
    float vf[4][4];      // v[t0 + 16 kg + 4 qq + e][i0 + j]                 (B, state)
    float et[4];         // a(t, t0 - 1) of token 16 mt + j
    float4 ws[4];        // a(end, s) of tokens 16 kg + 4 qq ..
    float gam;
    float oi[4];         // intra-chunk o of token 16 w + 4 qq + r, row i0 + j
  };
  auto load = [&](Ops& x, int ch) {
    const int t0 = ch * kC;
    const float* cf = coef + ((size_t)h * nchunk + ch) * kCoef;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int t = t0 + 16 * mt + j;
#pragma unroll
      for (int u = 0; u < NT; ++u)
        x.qf[mt][u] = t < T ? *(const float4*)(q + (size_t)t * qd + h * DK + cw + 16 * u + 4 * qq)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
      x.et[mt] = cf[16 * mt + j];
    }
#pragma unroll
    for (int kg = 0; kg < 4; ++kg) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = t0 + 16 * kg + 4 * qq + e;
        const bool ok = t < T;
#pragma unroll
        for (int u = 0; u < NT; ++u)
          x.kf[kg][u][e] = ok ? kb[(size_t)t * qd + h * DK + cw + 16 * u + j] : 0.f;
        x.vf[kg][e] = ok ? v[(size_t)t * vd + h * dv + i0 + j] : 0.f;
      }
      x.ws[kg] = *(const float4*)(cf + kC + 16 * kg + 4 * qq);
    }
    x.gam = cf[2 * kC];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 16 * w + 4 * qq + r;
      x.oi[r] = t < T ? o[(size_t)t * vd + h * dv + i0 + j] : 0.f;
    }
  };

  float4_t st[NT];
#pragma unroll
  for (int u = 0; u < NT; ++u) st[u] = (float4_t){0.f, 0.f, 0.f, 0.f};
  Ops cur, nxt;
  load(cur, 0);
  for (int ch = 0; ch < nchunk; ++ch) {
    if (ch + 1 < nchunk) load(nxt, ch + 1);
    // partial output over this wave's key columns, all 64 tokens: A = a(t) q_t, B = S^T
    float4_t op[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      op[mt] = (float4_t){0.f, 0.f, 0.f, 0.f};
      const float et = cur.et[mt];
#pragma unroll
      for (int u = 0; u < NT; ++u) {
        const float4 a = cur.qf[mt][u];
        op[mt] = mfma4(a.x * et, st[u][0], op[mt]);
        op[mt] = mfma4(a.y * et, st[u][1], op[mt]);
        op[mt] = mfma4(a.z * et, st[u][2], op[mt]);
        op[mt] = mfma4(a.w * et, st[u][3], op[mt]);
      }
    }
    // state update: S^T <- a(end) S^T + sum_s kb_s (a(end, s) v_s)^T
#pragma unroll
    for (int u = 0; u < NT; ++u) st[u] *= cur.gam;
#pragma unroll
    for (int kg = 0; kg < 4; ++kg) {
      const float b0 = cur.vf[kg][0] * cur.ws[kg].x, b1 = cur.vf[kg][1] * cur.ws[kg].y;
      const float b2 = cur.vf[kg][2] * cur.ws[kg].z, b3 = cur.vf[kg][3] * cur.ws[kg].w;
#pragma unroll
      for (int u = 0; u < NT; ++u) {
        st[u] = mfma4(cur.kf[kg][u][0], b0, st[u]);
        st[u] = mfma4(cur.kf[kg][u][1], b1, st[u]);
        st[u] = mfma4(cur.kf[kg][u][2], b2, st[u]);
        st[u] = mfma4(cur.kf[kg][u][3], b3, st[u]);
      }
    }
    // sum of the four waves' partial outputs; lane (j, qq) holds op[mt][r] for token
    // 16 mt + 4 qq + r, row j
    float* so = sO[ch & 1][w];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) so[(16 * mt + 4 * qq + r) * SO + j] = op[mt][r];
    __syncthreads();
    const int t0 = ch * kC;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tl = 16 * w + 4 * qq + r, t = t0 + tl;
      float sum = cur.oi[r];
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) sum += sO[ch & 1][w2][tl * SO + j];
      if (t < T) o[(size_t)t * vd + h * dv + i0 + j] = sum;
    }
    if (ch + 1 < nchunk) cur = nxt;
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
  if ((long)T * n * (dk > dv ? dk : dv) >= (1l << 31)) return MX_ERR_UNSUPPORTED;
  if (!mx_aligned16(q) || !mx_aligned16(kb) || !mx_aligned16(v) || !mx_aligned16(o) ||
      !mx_aligned16(coef))
    return MX_ERR_UNSUPPORTED;
  float* cf = (float*)coef;
  if (dk == 128 && dv == 128) return launch_chunked<128, 128>(q, kb, v, decay, T, n, o, cf, s);
  if (dk == 64 && dv == 64) return launch_chunked<64, 64>(q, kb, v, decay, T, n, o, cf, s);
  if (dk == 128 && dv == 64) return launch_chunked<128, 64>(q, kb, v, decay, T, n, o, cf, s);
  return launch_chunked<64, 128>(q, kb, v, decay, T, n, o, cf, s);
}
