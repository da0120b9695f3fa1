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
// in parallel as (Q Kb^T masked and scaled by a) V and writes it to o.  The second part
// walks the chunks of a head in order: k_la_chunk_state holds 16 state rows of one head
// in MFMA accumulators, adds a(t, t0 - 1) S_p q_t to o and updates S, one chunk at a time.
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

// LDS row strides in floats: (stride / 4) odd, so the 16-byte reads of 16 consecutive rows
// at one column group hit distinct bank groups.
template <int W>
struct Pad {
  static constexpr int S = W + 4;
};

// ---- intra-chunk part: o[t] = sum_{t0 <= s <= t} a(t, s) (kb_s . q_t) v_s ---------------
// Block (chunk, head), 4 waves; wave w takes tokens 16 w .. 16 w + 15 of the chunk.
template <int DK, int DV>
__global__ __launch_bounds__(256) void k_la_chunk_intra(const float* __restrict__ q,
                                                        const float* __restrict__ kb,
                                                        const float* __restrict__ v,
                                                        const float* __restrict__ decay, int T,
                                                        int n, int nchunk,
                                                        float* __restrict__ o) {
  constexpr int SK = Pad<DK>::S, SC = Pad<kC>::S;
  __shared__ __align__(16) float sQ[kC * SK];
  __shared__ __align__(16) float sK[kC * SK];
  __shared__ __align__(16) float sVt[DV * SC];     // v transposed: [value row][token]
  __shared__ __align__(16) float sP[4 * 16 * SC];  // each wave's masked scores
  __shared__ double sG[kC];
  __shared__ int sLR[kC];

  const int chunk = blockIdx.x % nchunk, h = blockIdx.x / nchunk;
  const int t0 = chunk * kC;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int j = lane & 15, qq = lane >> 4;
  const int qd = n * DK, vd = n * DV;

  for (int i = tid; i < kC * DK / 4; i += 256) {
    const int r = i / (DK / 4), c = 4 * (i % (DK / 4)), t = t0 + r;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
    if (t < T) {
      a = *(const float4*)(q + (size_t)t * qd + h * DK + c);
      b = *(const float4*)(kb + (size_t)t * qd + h * DK + c);
    }
    *(float4*)(sQ + r * SK + c) = a;
    *(float4*)(sK + r * SK + c) = b;
  }
  for (int i = tid; i < kC * DV / 4; i += 256) {
    const int r = i / (DV / 4), c = 4 * (i % (DV / 4)), t = t0 + r;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t < T) a = *(const float4*)(v + (size_t)t * vd + h * DV + c);
    sVt[(c + 0) * SC + r] = a.x;
    sVt[(c + 1) * SC + r] = a.y;
    sVt[(c + 2) * SC + r] = a.z;
    sVt[(c + 3) * SC + r] = a.w;
  }
  if (w == 0) chunk_log_decay(decay, t0, T, n, h, sG, sLR);
  __syncthreads();

  // scores of this wave's 16 tokens against the chunk's 64: P = Q Kb^T
  float4_t pacc[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) pacc[nt] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k0 = 0; k0 < DK; k0 += 16) {
    const float4 a = *(const float4*)(sQ + (16 * w + j) * SK + k0 + 4 * qq);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const float4 b = *(const float4*)(sK + (16 * nt + j) * SK + k0 + 4 * qq);
      pacc[nt] = mfma_k16(a, b, pacc[nt]);
    }
  }
  // causal mask and decay factors; lane (j, qq) holds P[16 w + 4 qq + r][16 nt + j]
  float* myP = sP + w * 16 * SC;
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
}

// ---- state part: o[t] += a(t, t0 - 1) S_p q_t, then S <- a(end) S_p + sum a(end, s) v kb^T
// Block (head, 16 value rows), 4 waves, walking the chunks in order.  The state rows live
// in MFMA accumulators (wave w: key columns 16 DK/64 w ..), with a copy in LDS that the
// next chunk's output products read.  The next chunk's q, kb and v are loaded into
// registers while the current chunk computes.
template <int DK>
__global__ __launch_bounds__(256) void k_la_chunk_state(const float* __restrict__ q,
                                                        const float* __restrict__ kb,
                                                        const float* __restrict__ v,
                                                        const float* __restrict__ decay, int T,
                                                        int n, int dv, int nchunk,
                                                        float* __restrict__ o) {
  constexpr int SK = Pad<DK>::S, SC = Pad<kC>::S;
  constexpr int NT = DK / 64;                 // 16-column state tiles per wave
  constexpr int QP = kC * DK / 4 / 256;        // float4 pieces of q (and of kb) per thread
  __shared__ __align__(16) float sQ[kC * SK];
  __shared__ __align__(16) float sKt[DK * SC];  // kb transposed: [key column][token]
  __shared__ __align__(16) float sVt[16 * SC];  // this block's value rows: [row][token]
  __shared__ __align__(16) float sS[16 * SK];   // state rows before the chunk
  __shared__ double sG[kC];
  __shared__ int sLR[kC];
  __shared__ __align__(16) float sE[kC];  // a(t, t0 - 1): weight of S_p q_t
  __shared__ __align__(16) float sW[kC];  // a(end, s): weight of v_s kb_s^T in the new state
  __shared__ float sGam;     // a(end, t0 - 1): decay of S_p over the chunk

  const int blocks_per_head = dv / 16;
  const int h = blockIdx.x / blocks_per_head, i0 = 16 * (blockIdx.x % blocks_per_head);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int j = lane & 15, qq = lane >> 4;
  const int qd = n * DK, vd = n * dv;

  float4_t sacc[NT];
#pragma unroll
  for (int u = 0; u < NT; ++u) sacc[u] = (float4_t){0.f, 0.f, 0.f, 0.f};
  for (int i = tid; i < 16 * SK; i += 256) sS[i] = 0.f;

  float4 rq[QP], rk[QP];
  // v: 64 tokens x 16 rows = 1024 values, 4 per thread
  float rvv[4];
  auto load_all = [&](int t0) {
#pragma unroll
    for (int p = 0; p < QP; ++p) {
      const int i = tid + 256 * p;
      const int r = i / (DK / 4), c = 4 * (i % (DK / 4)), t = t0 + r;
      rq[p] = rk[p] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (t < T) {
        rq[p] = *(const float4*)(q + (size_t)t * qd + h * DK + c);
        rk[p] = *(const float4*)(kb + (size_t)t * qd + h * DK + c);
      }
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int i = tid + 256 * p, r = i >> 4, c = i & 15, t = t0 + r;
      rvv[p] = t < T ? v[(size_t)t * vd + h * dv + i0 + c] : 0.f;
    }
  };
  auto store_all = [&]() {
#pragma unroll
    for (int p = 0; p < QP; ++p) {
      const int i = tid + 256 * p;
      const int r = i / (DK / 4), c = 4 * (i % (DK / 4));
      *(float4*)(sQ + r * SK + c) = rq[p];
      sKt[(c + 0) * SC + r] = rk[p].x;
      sKt[(c + 1) * SC + r] = rk[p].y;
      sKt[(c + 2) * SC + r] = rk[p].z;
      sKt[(c + 3) * SC + r] = rk[p].w;
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int i = tid + 256 * p, r = i >> 4, c = i & 15;
      sVt[c * SC + r] = rvv[p];
    }
  };
  load_all(0);
  for (int ch = 0; ch < nchunk; ++ch) {
    const int t0 = ch * kC;
    store_all();
    if (w == 0) {
      chunk_log_decay(decay, t0, T, n, h, sG, sLR);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
      const int l = lane;
      const double gl = sG[l];
      const int lastv = min(kC, T - t0) - 1;  // last token of the chunk inside T
      const double ge = sG[lastv];
      const int lre = sLR[lastv];
      sE[l] = sLR[l] < 0 ? expf((float)gl) : 0.f;
      sW[l] = (l <= lastv && lre <= l) ? expf((float)(ge - gl)) : 0.f;
      if (l == 0) sGam = lre < 0 ? expf((float)ge) : 0.f;
    }
    __syncthreads();
    if (ch + 1 < nchunk) load_all(t0 + kC);

    // output: o[t, i0 + j] += sum_c a(t, t0 - 1) q_t[c] S_p[j][c] for t = t0 + 16 w + ..
    float ov[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 16 * w + 4 * qq + r;
      ov[r] = t < T ? o[(size_t)t * vd + h * dv + i0 + j] : 0.f;
    }
    float4_t oacc = (float4_t){0.f, 0.f, 0.f, 0.f};
    const float et = sE[16 * w + j];
#pragma unroll
    for (int k0 = 0; k0 < DK; k0 += 16) {
      float4 a = *(const float4*)(sQ + (16 * w + j) * SK + k0 + 4 * qq);
      a.x *= et;
      a.y *= et;
      a.z *= et;
      a.w *= et;
      const float4 b = *(const float4*)(sS + j * SK + k0 + 4 * qq);
      oacc = mfma_k16(a, b, oacc);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 16 * w + 4 * qq + r;
      if (t < T) o[(size_t)t * vd + h * dv + i0 + j] = ov[r] + oacc[r];
    }

    // state: S <- a(end) S_p + sum_s a(end, s) v_s kb_s^T; lane (j, qq) of wave w holds
    // S[4 qq + r][16 (NT w + u) + j]
    const float gam = sGam;
#pragma unroll
    for (int u = 0; u < NT; ++u) sacc[u] *= gam;
#pragma unroll
    for (int k0 = 0; k0 < kC; k0 += 16) {
      float4 a = *(const float4*)(sVt + j * SC + k0 + 4 * qq);
      const float4 ws = *(const float4*)(sW + k0 + 4 * qq);
      a.x *= ws.x;
      a.y *= ws.y;
      a.z *= ws.z;
      a.w *= ws.w;
#pragma unroll
      for (int u = 0; u < NT; ++u) {
        const float4 b = *(const float4*)(sKt + (16 * (NT * w + u) + j) * SC + k0 + 4 * qq);
        sacc[u] = mfma_k16(a, b, sacc[u]);
      }
    }
    __syncthreads();  // every wave is done with sQ, sKt, sVt and sS of this chunk
#pragma unroll
    for (int u = 0; u < NT; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) sS[(4 * qq + r) * SK + 16 * (NT * w + u) + j] = sacc[u][r];
  }
}

template <int DK, int DV>
int launch_chunked(const float* q, const float* kb, const float* v, const float* decay, int T,
                   int n, float* o, hipStream_t s) {
  const int nchunk = (T + kC - 1) / kC;
  mx_clear_error();
  hipLaunchKernelGGL((k_la_chunk_intra<DK, DV>), dim3((unsigned)(nchunk * n)), dim3(256), 0, s,
                     q, kb, v, decay, T, n, nchunk, o);
  MX_TRY(mx_launch_status());
  hipLaunchKernelGGL((k_la_chunk_state<DK>), dim3((unsigned)(n * (DV / 16))), dim3(256), 0, s,
                     q, kb, v, decay, T, n, DV, nchunk, o);
  return mx_launch_status();
}

}  // namespace

// Chunked scan for the shapes it is built for (key and value heads of 64 or 128); returns
// MX_ERR_UNSUPPORTED otherwise, and the caller runs the token-sequential scan.
int mx_la_chunked_scan(const float* q, const float* kb, const float* v, const float* decay,
                       int T, int n, int dk, int dv, float* o, hipStream_t s) {
  if (T <= 0 || n <= 0) return MX_ERR_INVALID;
  if ((long)T * n * (dk > dv ? dk : dv) >= (1l << 31)) return MX_ERR_UNSUPPORTED;
  if (!mx_aligned16(q) || !mx_aligned16(kb) || !mx_aligned16(v)) return MX_ERR_UNSUPPORTED;
  if (dk == 128 && dv == 128) return launch_chunked<128, 128>(q, kb, v, decay, T, n, o, s);
  if (dk == 64 && dv == 64) return launch_chunked<64, 64>(q, kb, v, decay, T, n, o, s);
  if (dk == 128 && dv == 64) return launch_chunked<128, 64>(q, kb, v, decay, T, n, o, s);
  if (dk == 64 && dv == 128) return launch_chunked<64, 128>(q, kb, v, decay, T, n, o, s);
  return MX_ERR_UNSUPPORTED;
}
