// Chunked form of the gated recurrence of the Qwen3-Next linear-attention block
// (offload_runtime/executors/qwen3_next.py:56-95, with beta * k formed):
//   S_t = d_t S_{t-1} + v_t kb_t^T,   o_t = S_t q_t,   S_0 = 0     (per head, d_t = exp(g_t))
// on fp32 MFMA (v_mfma_f32_16x16x4_f32, full fp32 products and sums).
//
// Over a chunk c of C = 64 tokens starting at t0, with S_{c-1} the state before the chunk
// and a(t, s) = d_{s+1} ... d_t the decay between tokens s <= t (a(t, t) = 1):
//   o_t = sum_{t0 <= s <= t} a(t, s) (kb_s . q_t) v_s  +  a(t, t0 - 1) S_{c-1} q_t
//   S_c = a(end, t0 - 1) S_{c-1} + sum_s a(end, s) v_s kb_s^T
// which is the recurrence unrolled over the chunk (exact in real arithmetic).  Three
// launches:
//   k_la_chunk_coef    one wave per (head, chunk): the chunk's coefficients a(end, s) and
//                      a(end, t0 - 1) for the state walk;
//   k_la_chunk_states  walks the chunks of a head in order, the state in MFMA accumulators
//                      (a block per 32 value rows x 64 key columns of a head), adding only
//                      the increments sum_s a(end, s) v_s kb_s^T, and stores every state a
//                      later chunk starts from (S_0 .. S_{nc-2}, fp32);
//   k_la_chunk_out     a block per (chunk, head), all in parallel: the intra-chunk sum as
//                      (Q Kb^T masked and scaled by a) V plus a(t, t0 - 1) S_{c-1} q_t.
// The walk carries no q, o or output product, so its chain per chunk is the increment alone.
//
// The decay factors are formed in double precision from the fp32 decays the reference
// multiplies by: with G_t = sum over the chunk of log(d_r) up to t, a(t, s) =
// exp(G_t - G_s).  A zero decay (exp(g) underflowed) zeroes the state; such a token starts
// a new segment (G restarts at 0 there and factors across it are 0), so no logarithm of
// zero is taken and no difference of huge sums is formed.
#include <math.h>

#include <utility>

#include "mx_common.h"
#include "mx_internal.h"
#include "mx_lds_copy.h"

namespace {

constexpr int kC = 64;  // tokens per chunk

#ifndef MX_OOB
#define MX_OOB 0x80000000u  // an offset outside every buffer descriptor built here
#endif

typedef __amdgpu_buffer_rsrc_t mx_rsrc_t;

// Buffer descriptor over `bytes` bytes: loads at offsets past the end return zeros.
__device__ __forceinline__ mx_rsrc_t mx_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ int4_t mx_ld16(mx_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// f(integral_constant<int, i>) for i = 0 .. N - 1, unrolled at compile time.
template <typename F, int... Is>
__device__ __forceinline__ void mx_static_for_seq(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void mx_static_for(F&& f) {
  mx_static_for_seq(f, std::make_integer_sequence<int, N>{});
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

// fp32 products through bf16 MFMAs: x splits exactly into three bf16 planes, x = p0 + p1 + p2,
// each plane the high half of the residual left by the planes before it (8 + 8 + 8
// significant bits cover fp32's 24).  A dot product over 32 columns is then the six plane
// products with p_a + p_b <= 2 (the three dropped ones are below 2^-21 of the sum of |a b|),
// each exact in the fp32 accumulator, on v_mfma_f32_16x16x32_bf16: 6 x 16 cycles against
// 8 x 32 for v_mfma_f32_16x16x4_f32.  Lane (j, q) passes 8 values (lo: 4 columns, hi: the 4
// columns 16 further), element e of a plane in bits 16 e ..; any assignment of the 32
// columns to (q, e) serves, as long as both operands use the same one.
#ifndef LA_OUT_BF16X3
#define LA_OUT_BF16X3 1  // the output launch's score and inter-chunk products on bf16 planes
#endif
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ void bf16x3_split(const int4_t& lo, const int4_t& hi, int4_t (&p)[3]) {
  uint32_t b[3][8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    uint32_t u = (uint32_t)(e < 4 ? lo[e] : hi[e - 4]);
#pragma unroll
    for (int l = 0; l < 3; ++l) {
      b[l][e] = u;
      if (l < 2) {
        const float r = __builtin_bit_cast(float, u) - __builtin_bit_cast(float, u & 0xFFFF0000u);
        u = __builtin_bit_cast(uint32_t, r);
      }
    }
  }
#pragma unroll
  for (int l = 0; l < 3; ++l)
#pragma unroll
    for (int d = 0; d < 4; ++d) p[l][d] = (int)__builtin_amdgcn_perm(b[l][2 * d + 1], b[l][2 * d], 0x07060302u);
}

__device__ __forceinline__ float4_t mfma_bf16(const int4_t& a, const int4_t& b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ float4_t mfma_bf16x3(const int4_t (&a)[3], const int4_t (&b)[3], float4_t c) {
  c = mfma_bf16(a[2], b[0], c);
  c = mfma_bf16(a[0], b[2], c);
  c = mfma_bf16(a[1], b[1], c);
  c = mfma_bf16(a[1], b[0], c);
  c = mfma_bf16(a[0], b[1], c);
  return mfma_bf16(a[0], b[0], c);
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
__device__ __forceinline__ float chunk_decay_load(const float* __restrict__ decay, int t0,
                                                  int T, int n, int h) {
  const int t = t0 + (threadIdx.x & 63);
  return t < T ? decay[(size_t)t * n + h] : 1.f;
}

// The prefix from the lane's decay d (chunk_decay_load).
__device__ __forceinline__ void chunk_log_decay_of(float d, int t0, int T, double& G, int& LR) {
  const int l = threadIdx.x & 63;
  const bool reset = t0 + l < T && !(d > 0.f);
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
  G = lr >= 0 ? p - pr : p;
  LR = lr;
}

__device__ __forceinline__ void chunk_log_decay_reg(const float* __restrict__ decay, int t0,
                                                    int T, int n, int h, double& G, int& LR) {
  chunk_log_decay_of(chunk_decay_load(decay, t0, T, n, h), t0, T, G, LR);
}

// The same prefix written to LDS (sG, sLR: 64 entries).
__device__ __forceinline__ void chunk_log_decay_lds(float d, int t0, int T, double* sG,
                                                    int* sLR) {
  double G;
  int LR;
  chunk_log_decay_of(d, t0, T, G, LR);
  sG[threadIdx.x & 63] = G;
  sLR[threadIdx.x & 63] = LR;
}

// Coefficient record of a (head, chunk), 1 KiB so that one 64-lane LDS copy moves it:
// a(end, s) for the 64 tokens, then a(end, t0 - 1); the rest is padding.
constexpr int kCoef = 256;

// LDS row strides in floats: (stride / 4) odd, so the 16-byte reads of 16 consecutive rows
// at one column group hit distinct bank groups.
template <int W>
struct Pad {
  static constexpr int S = W + 4;
};

// ---- coefficients: one wave per (head, chunk) ---------------------------------------
__global__ __launch_bounds__(256) void k_la_chunk_coef(const float* __restrict__ decay, int T,
                                                       int n, int nchunk,
                                                       float* __restrict__ coef) {
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);  // h * nchunk + chunk
  if (item >= n * nchunk) return;                        // whole waves
  const int h = item / nchunk, chunk = item % nchunk, t0 = chunk * kC;
  const int l = threadIdx.x & 63;
  double G;
  int LR;
  chunk_log_decay_reg(decay, t0, T, n, h, G, LR);
  const int lastv = min(kC, T - t0) - 1;
  const double ge = shfl_d(G, lastv);
  const int lre = __shfl(LR, lastv, 64);
  float* cf = coef + (size_t)item * kCoef;
  cf[l] = (l <= lastv && lre <= l) ? expf((float)(ge - G)) : 0.f;
  if (l == 0) cf[kC] = lre < 0 ? expf((float)ge) : 0.f;
}

// ---- state walk: S_c = a(end, t0 - 1) S_{c-1} + sum_s a(end, s) v_s kb_s^T ------------
// Block = 32 value rows (i0 ..) x 64 key columns (c0 ..) of one head's state: eight 16 x 16
// tiles, LA_ST_NW waves (4: two tiles per wave, 8: one).  Wave w holds the transposed tiles
// S^T[c0 + 16 ct + ..][i0 + 16 rt + ..] (ct = w % 4) in MFMA accumulators: lane (j, qq) of
// tile rt holds S[i0 + 16 rt + j][c0 + 16 ct + 4 qq + r], r = 0..3, which it stores as one
// 16-byte piece.  The increment of a chunk is U^T = Kb^T (a(end) V): token
// s = 16 kg + 4 qq + e enters as k-slot qq of MFMA (kg, e), A = kb[s][c0 + 16 ct + j],
// B = v[s][i0 + 16 rt + j] a(end, s).
//
// Operands come through an LDS ring of LA_NB chunk slots filled by the buffer loads' LDS
// mode (no register holds a staged piece): per chunk the kb tile (64 tokens x 64 columns,
// 16 KiB), the v tile (64 tokens x 32 rows, 8 KiB) and the coefficient record (1 KiB),
// issued LA_NB - 1 chunks ahead.  Copy lane l of a kb copy loads a 16-byte piece of token
// row r = l / 16 (of its 4 rows), placed at piece position (p + 4 ((r / 4) % 4)) % 16 of the
// 16 in the row; a v copy holds 8 token rows of 8 pieces, row R of the copy holding token
// R ^ ((R / 8) % 2) at piece position (p + 4 ((s / 4) % 2)) % 8.  With these rotations the 64
// lanes of every operand read hit 64 distinct 4-byte banks.  Wave 0 copies the coefficient
// record; the other waves issue an out-of-range copy into a scratch kilobyte instead, and
// copies past the last chunk, and rows past T, use out-of-range offsets too (they return
// zeros and move no data): every wave issues the same number of vector memory operations per
// chunk, so one constant wait count per iteration finds the chunk's copies complete.
#ifndef LA_NB
#define LA_NB 4  // chunk slots of the state walk's LDS ring
#endif
#ifndef LA_ST_NW
#define LA_ST_NW 8  // waves per state-walk block (4 or 8)
#endif

template <int DK, int DV>
__global__ __launch_bounds__(64 * LA_ST_NW) void k_la_chunk_states(const float* __restrict__ kb,
                                                                   const float* __restrict__ v,
                                                                   const float* __restrict__ coef,
                                                                   int T, int n, int nchunk,
                                                                   float* __restrict__ S) {
  constexpr int NB = LA_NB;
  constexpr int NW = LA_ST_NW;
  static_assert(NB >= 2 && NB <= 5, "ring depth");
  static_assert(NW == 4 || NW == 8, "waves per block");
  constexpr int TPW = 8 / NW;           // state tiles per wave
  constexpr int NCH = 4 / TPW;          // accumulator chains per tile
  constexpr int KPW = 16 / NW;          // kb copies per wave and chunk
  constexpr int VPW = 8 / NW;           // v copies per wave and chunk
  constexpr int RBK = DV / 32;          // 32-row blocks per head
  constexpr int BPH = RBK * (DK / 64);  // blocks per head
  constexpr int KB_BYTES = kC * 64 * 4;
  constexpr int V_BYTES = kC * 32 * 4;
  constexpr int CF_OFF = KB_BYTES + V_BYTES;
  constexpr int SLOT = CF_OFF + 2 * 1024;  // + the coefficient record and a scratch kilobyte
  constexpr int P = KPW + VPW + 1;      // copies per wave and chunk
  constexpr int ST = TPW;               // state stores per wave and chunk
  // One LDS variable per slot, every access naming its slot at compile time: the compiler
  // then tells a slot's reads from the copies in flight into the other slots (with a single
  // array it waits for every copy before any read).
  __shared__ __align__(1024) char lds0[SLOT];
  __shared__ __align__(1024) char lds1[SLOT];
  __shared__ __align__(1024) char lds2[NB > 2 ? SLOT : 16];
  __shared__ __align__(1024) char lds3[NB > 3 ? SLOT : 16];
  __shared__ __align__(1024) char lds4[NB > 4 ? SLOT : 16];
  auto slot_of = [&](auto I) -> char* {
    constexpr int i = decltype(I)::value % NB;
    if constexpr (i == 0) return lds0;
    else if constexpr (i == 1) return lds1;
    else if constexpr (i == 2) return lds2;
    else if constexpr (i == 3) return lds3;
    else return lds4;
  };

  // The blocks of a head share kb columns and v rows: they run on one XCD (hardware block b
  // runs on XCD b % 8), so a chunk's rows come from that XCD's L2 after the first read.
  int h, sub;
  if ((n & 7) == 0) {
    const int k = blockIdx.x >> 3;
    h = (blockIdx.x & 7) * (n >> 3) + k / BPH;
    sub = k % BPH;
  } else {
    h = blockIdx.x / BPH;
    sub = blockIdx.x % BPH;
  }
  const int i0 = 32 * (sub % RBK), c0 = 64 * (sub / RBK);
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ct = w & 3, rt0 = (w >> 2) * TPW;  // the wave's key-column tile, first row tile
  const int j = lane & 15, qq = lane >> 4;
  const uint32_t qrow = (uint32_t)n * DK * 4, vrow = (uint32_t)n * DV * 4;
  const mx_rsrc_t rk = mx_rsrc(kb, (uint32_t)T * qrow);
  const mx_rsrc_t rv = mx_rsrc(v, (uint32_t)T * vrow);
  const mx_rsrc_t rc = mx_rsrc(coef, (uint32_t)n * nchunk * kCoef * 4);
  constexpr uint32_t SB = (uint32_t)DV * DK * 4;  // bytes per stored state
  const mx_rsrc_t rs = mx_rsrc(S + (size_t)h * (nchunk - 1) * DV * DK, (uint32_t)(nchunk - 1) * SB);

  // copy offsets of this lane (chunk 0)
  uint32_t k_off[KPW], v_off[VPW];
#pragma unroll
  for (int m = 0; m < KPW; ++m) {
    const int r = 4 * (KPW * w + m) + (lane >> 4);
    const int p = ((lane & 15) - 4 * ((r >> 2) & 3)) & 15;
    k_off[m] = (uint32_t)r * qrow + (uint32_t)(h * DK + c0 + 4 * p) * 4;
  }
#pragma unroll
  for (int m = 0; m < VPW; ++m) {
    const int R = 8 * (VPW * w + m) + (lane >> 3);
    const int s = R ^ ((R >> 3) & 1);
    const int p = ((lane & 7) - 4 * ((s >> 2) & 1)) & 7;
    v_off[m] = (uint32_t)s * vrow + (uint32_t)(h * DV + i0 + 4 * p) * 4;
  }
  // wave 0: the coefficient record; the others: out of range into the scratch kilobyte
  const uint32_t c_oob = w == 0 ? 0u : MX_OOB;
  const int c_dst = w == 0 ? CF_OFF : CF_OFF + 1024;
  const uint32_t c_off = (uint32_t)h * nchunk * kCoef * 4 + 16 * lane;
  auto copies = [&](char* slot, int ch) {
    const uint32_t oob = ch < nchunk ? 0u : MX_OOB;
    const uint32_t kbase = (uint32_t)ch * kC * qrow, vbase = (uint32_t)ch * kC * vrow;
#pragma unroll
    for (int m = 0; m < KPW; ++m)
      mx_copy_to_lds16(rk, slot + 1024 * (KPW * w + m), (kbase + k_off[m]) | oob);
#pragma unroll
    for (int m = 0; m < VPW; ++m)
      mx_copy_to_lds16(rv, slot + KB_BYTES + 1024 * (VPW * w + m), (vbase + v_off[m]) | oob);
    mx_copy_to_lds16(rc, slot + c_dst, (c_off + (uint32_t)ch * kCoef * 4) | oob | c_oob);
  };

  // operand read offsets (floats) of this lane: kb[s][c0 + 16 ct + j] at kq + (16 kg + e) 64;
  // v[s][i0 + 16 rt + j] at (e odd ? vo : ve)[t] + (16 kg + e) 32
  const int kq = 4 * qq * 64 + 4 * ((4 * ct + (j >> 2) + 4 * qq) & 15) + (j & 3);
  const int x = qq >> 1;
  int ve[TPW], vo[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int rt = rt0 + t;
    const int b = 4 * qq * 32 + 4 * ((4 * rt + (j >> 2) + 4 * (qq & 1)) & 7) + (j & 3);
    ve[t] = b + 32 * x;
    vo[t] = b - 32 * x;
  }
  // this lane's stored piece of tile t (bytes, state 0)
  uint32_t s_off[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
    s_off[t] = (uint32_t)((i0 + 16 * (rt0 + t) + j) * DK + c0 + 16 * ct + 4 * qq) * 4;

  float4_t st[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) st[t] = (float4_t){0.f, 0.f, 0.f, 0.f};

  auto step = [&](const char* slot, int ch) {
    const float* K = (const float*)slot;
    const float* V = (const float*)(slot + KB_BYTES);
    const float* CF = (const float*)(slot + CF_OFF);
    float a[4][4], b[TPW][4][4];
#pragma unroll
    for (int kg = 0; kg < 4; ++kg) {
      const float4 ws = *(const float4*)(CF + 16 * kg + 4 * qq);
      const float wv[4] = {ws.x, ws.y, ws.z, ws.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a[kg][e] = K[kq + (16 * kg + e) * 64];
#pragma unroll
        for (int t = 0; t < TPW; ++t)
          b[t][kg][e] = V[((e & 1) ? vo[t] : ve[t]) + (16 * kg + e) * 32] * wv[e];
      }
    }
    // four independent chains: tiles x token groups
    float4_t acc[TPW][NCH];
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int c = 0; c < NCH; ++c) acc[t][c] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4 / NCH; ++kk)
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
          for (int t = 0; t < TPW; ++t) {
            const int kg = c * (4 / NCH) + kk;
            acc[t][c] = mfma4(a[kg][e], b[t][kg][e], acc[t][c]);
          }
    const float gam = CF[kC];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      float4_t u = acc[t][0];
#pragma unroll
      for (int c = 1; c < NCH; ++c) u += acc[t][c];
      st[t] = st[t] * gam + u;
    }
    // S_ch, the state chunk ch + 1 starts from (the last chunk's store is out of range)
#pragma unroll
    for (int t = 0; t < TPW; ++t)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(int4_t, st[t]), rs,
                                             (uint32_t)ch * SB + s_off[t], 0, 0);
  };

  // LDS starts zeroed: a row a copy does not fill holds finite values (a(end, s) = 0 there)
  for (int i = threadIdx.x; i < SLOT / 16; i += 64 * NW) {
    const int4_t z = {0, 0, 0, 0};
    *(int4_t*)(lds0 + 16 * i) = z;
    *(int4_t*)(lds1 + 16 * i) = z;
    if constexpr (NB > 2) *(int4_t*)(lds2 + 16 * i) = z;
    if constexpr (NB > 3) *(int4_t*)(lds3 + 16 * i) = z;
    if constexpr (NB > 4) *(int4_t*)(lds4 + 16 * i) = z;
  }
  __syncthreads();
  mx_static_for<NB - 1>([&](auto I) { copies(slot_of(I), decltype(I)::value); });
  // Iteration c (slot c % NB): wait for chunk c's copies (after them this wave issued the
  // later prologue copies and, per earlier iteration, P copies and ST stores), meet the
  // other waves, issue the copies of chunk c + NB - 1 into the slot chunk c - 1 used,
  // compute chunk c.  The walk runs whole groups of NB chunks, unrolled and branch-free so
  // that every slot is named statically; chunks past the last one compute on out-of-range
  // copies and store out of range.  The first group is peeled for its wait counts.
  mx_static_for<NB>([&](auto I) {
    constexpr int i = decltype(I)::value;
    mx_wait_copies_and_barrier<(NB - 2) * P + (i < NB - 1 ? i : NB - 1) * ST>();
    copies(slot_of(std::integral_constant<int, i + NB - 1>{}), i + NB - 1);
    step(slot_of(I), i);
  });
  for (int c0 = NB; c0 < nchunk; c0 += NB) {
    mx_static_for<NB>([&](auto I) {
      constexpr int i = decltype(I)::value;
      mx_wait_copies_and_barrier<(NB - 2) * P + (NB - 1) * ST>();
      copies(slot_of(std::integral_constant<int, i + NB - 1>{}), c0 + i + NB - 1);
      step(slot_of(I), c0 + i);
    });
  }
  // no copy into LDS may still be in flight when the block ends
  __builtin_amdgcn_s_waitcnt(0x0F70);
}

// ---- output: o[t] = sum_{t0 <= s <= t} a(t, s) (kb_s . q_t) v_s + a(t, t0 - 1) S_{c-1} q_t
// Block (chunk, head), 4 waves.  Wave w owns key tokens 16 w .. 16 w + 15 of the scores and
// value columns CW w .. CW w + CW - 1 (CW = DV / 4) of the output, for all 64 tokens:
//   scores  P[t][16 w + j]     = Q[t] . kb[16 w + j]        A = q rows (LDS), B = kb (registers)
//   inter   O[t][CW w + ..]    = a(t) Q[t] . S[CW w + ..]   A = the same q fragments, B = its
//                                                           state rows (registers)
//   intra   O[t][CW w + ..]   += sum_s P[t][s] v[s][CW w + ..]  A = P (LDS), B = v (LDS)
// so each q fragment read from LDS feeds the score and the inter-chunk MFMAs, and no wave
// loads what another loads: the block reads q, kb, v and the state once.  q and v enter LDS
// by the buffer loads' LDS mode, issued first with the kb and state loads; a q row's 16-byte
// piece p sits at position (p + t % 16) mod (dk / 4) and a v row's at (p + 4 ((t / 4) % 4))
// mod (dv / 4), so the operand reads hit distinct banks.  The masked scores then replace q in
// LDS (64-float rows, piece p of row t at (p + t % 16) mod 16).  Rows past T read as zeros
// through the descriptors, and chunk 0 (which starts from S = 0) reads its state rows out of
// range, also zeros.
template <int DK, int DV>
__global__ __launch_bounds__(256, 2) void k_la_chunk_out(const float* __restrict__ q,
                                                         const float* __restrict__ kb,
                                                         const float* __restrict__ v,
                                                         const float* __restrict__ decay,
                                                         const float* __restrict__ S, int T,
                                                         int n, int nchunk,
                                                         float* __restrict__ o) {
  constexpr int NU = DK / 16;    // 16-column groups of a q / kb / state row
  constexpr int CW = DV / 4;     // value columns per wave
  constexpr int NCT = CW / 16;   // value tiles per wave
  constexpr int QPR = DK / 4;    // 16-byte pieces per q row
  constexpr int VPR = DV / 4;    // 16-byte pieces per v row
  constexpr int NQC = DK / 16;   // q copies per wave (kC * DK * 4 bytes / 1 KiB / 4 waves)
  constexpr int NVC = DV / 16;   // v copies per wave
  static_assert(kC * 64 <= kC * DK, "the scores fit in the q region");
  __shared__ __align__(1024) float sQ[kC * DK];  // q rows, then the masked scores
  __shared__ __align__(1024) float sV[kC * DV];  // v rows
  __shared__ double sG[kC];
  __shared__ int sLR[kC];

  const int chunk = blockIdx.x % nchunk, h = blockIdx.x / nchunk;
  const int t0 = chunk * kC;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, qq = lane >> 4;
  const uint32_t qrow = (uint32_t)n * DK * 4, vrow = (uint32_t)n * DV * 4;
  const uint32_t tq = (uint32_t)t0 * qrow, tv = (uint32_t)t0 * vrow;
  const mx_rsrc_t rq = mx_rsrc(q, (uint32_t)T * qrow);
  const mx_rsrc_t rk = mx_rsrc(kb, (uint32_t)T * qrow);
  const mx_rsrc_t rv = mx_rsrc(v, (uint32_t)T * vrow);
  // wave 0's decays first: its prefix then waits on them alone
  const float dl = w == 0 ? chunk_decay_load(decay, t0, T, n, h) : 1.f;

  // q and v tiles into LDS: copy i fills floats 256 i .. 256 i + 255 of the tile
#pragma unroll
  for (int m = 0; m < NQC; ++m) {
    const int i = NQC * w + m, f = 256 * i + 4 * lane, t = f / DK;
    const int p = ((f % DK) / 4 - (t & 15)) & (QPR - 1);
    mx_copy_to_lds16(rq, (char*)sQ + 1024 * i, tq + (uint32_t)t * qrow + (uint32_t)(h * DK + 4 * p) * 4);
  }
#pragma unroll
  for (int m = 0; m < NVC; ++m) {
    const int i = NVC * w + m, f = 256 * i + 4 * lane, t = f / DV;
    const int p = ((f % DV) / 4 - 4 * ((t >> 2) & 3)) & (VPR - 1);
    mx_copy_to_lds16(rv, (char*)sV + 1024 * i, tv + (uint32_t)t * vrow + (uint32_t)(h * DV + 4 * p) * 4);
  }
  // kb rows 16 w + j (B of the scores): k-slot qq of MFMA (u, e) is column 16 u + 4 qq + e
  int4_t kbr[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u)
    kbr[u] = mx_ld16(rk, tq + (uint32_t)(16 * w + j) * qrow + (uint32_t)(h * DK + 16 * u + 4 * qq) * 4);
  // state rows CW w + 16 ct + j of S_{chunk-1} (B of the inter-chunk products)
  const mx_rsrc_t rs = mx_rsrc(S + (size_t)h * (nchunk - 1) * DV * DK,
                               (uint32_t)(nchunk - 1) * DV * DK * 4);
  const uint32_t s_base = chunk > 0 ? (uint32_t)(chunk - 1) * DV * DK * 4 : MX_OOB;
  int4_t sr[NCT][NU];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
    for (int u = 0; u < NU; ++u)
      sr[ct][u] = mx_ld16(rs, s_base | (uint32_t)(((CW * w + 16 * ct + j) * DK + 16 * u + 4 * qq) * 4));
  if (w == 0) {
    chunk_log_decay_lds(dl, t0, T, sG, sLR);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the prefix is in LDS
  }
  // this wave's q copies, then everyone's (and the decay prefix) are in LDS
  mx_wait_copies_and_barrier<NVC + NU + NCT * NU>();

  // scores and inter-chunk products, one q fragment read per (mt, u)
  float4_t pacc[4], oacc[4][NCT];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    pacc[mt] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) oacc[mt][ct] = (float4_t){0.f, 0.f, 0.f, 0.f};
  }
  if constexpr (LA_OUT_BF16X3) {
    // bf16 planes of kb and of the state rows, per 32-column block m (u = 2m, 2m + 1)
    int4_t kb3[NU / 2][3], s3[NCT][NU / 2][3];
#pragma unroll
    for (int m = 0; m < NU / 2; ++m) {
      bf16x3_split(kbr[2 * m], kbr[2 * m + 1], kb3[m]);
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) bf16x3_split(sr[ct][2 * m], sr[ct][2 * m + 1], s3[ct][m]);
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int t = 16 * mt + j;
#pragma unroll
      for (int m = 0; m < NU / 2; ++m) {
        const int4_t a0 = *(const int4_t*)(sQ + t * DK + 4 * ((8 * m + qq + j) & (QPR - 1)));
        const int4_t a1 = *(const int4_t*)(sQ + t * DK + 4 * ((8 * m + 4 + qq + j) & (QPR - 1)));
        int4_t q3[3];
        bf16x3_split(a0, a1, q3);
        pacc[mt] = mfma_bf16x3(q3, kb3[m], pacc[mt]);
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) oacc[mt][ct] = mfma_bf16x3(q3, s3[ct][m], oacc[mt][ct]);
      }
    }
  } else {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int t = 16 * mt + j;
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const float4 a = *(const float4*)(sQ + t * DK + 4 * ((4 * u + qq + j) & (QPR - 1)));
        pacc[mt] = mfma_k16(a, __builtin_bit_cast(float4, kbr[u]), pacc[mt]);
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
          oacc[mt][ct] = mfma_k16(a, __builtin_bit_cast(float4, sr[ct][u]), oacc[mt][ct]);
      }
    }
  }
  // lane (j, qq) holds P[16 mt + 4 qq + r][16 w + j] and O[16 mt + 4 qq + r][CW w + 16 ct + j]
  float pm[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tl = 16 * mt + 4 * qq + r, sl = 16 * w + j;
      const float at = sLR[tl] < 0 ? expf((float)sG[tl]) : 0.f;
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) oacc[mt][ct][r] *= at;
      const float f = (sl <= tl && sLR[tl] <= sl) ? expf((float)(sG[tl] - sG[sl])) : 0.f;
      pm[mt][r] = pacc[mt][r] * f;
    }
  __syncthreads();  // every wave is done with the q rows: their region takes the scores
  // P[t][s] at row t, piece (s / 4 + t % 16) mod 16
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tl = 16 * mt + 4 * qq + r;
      sQ[tl * 64 + 4 * ((4 * w + (j >> 2) + tl) & 15) + (j & 3)] = pm[mt][r];
    }
  __syncthreads();  // the scores and every wave's v copies are in LDS

  // O[16 mt + ..] += P[16 mt + ..][s] v[s][CW w + 16 ct + ..] over the keys s <= the tile's
  // last token: token s = 16 kg + 4 qq + e is k-slot qq of MFMA (kg, e)
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int t = 16 * mt + j;
#pragma unroll
    for (int kg = 0; kg <= mt; ++kg) {
      const float4 a = *(const float4*)(sQ + t * 64 + 4 * ((4 * kg + qq + j) & 15));
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const int pc = (CW * w + 16 * ct + j) >> 2;
        const float* vp = sV + (16 * kg + 4 * qq) * DV + 4 * ((pc + 4 * qq) & (VPR - 1)) + (j & 3);
        const float4 b = make_float4(vp[0], vp[DV], vp[2 * DV], vp[3 * DV]);
        oacc[mt][ct] = mfma_k16(a, b, oacc[mt][ct]);
      }
    }
  }
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 16 * mt + 4 * qq + r;
      if (t < T) {
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
          o[(size_t)t * n * DV + h * DV + CW * w + 16 * ct + j] = oacc[mt][ct][r];
      }
    }
}

// Workspace: the coefficient records [n][nchunk] (1 KiB each), then the stored states
// [n][nchunk - 1][DV][DK] (fp32).
size_t chunk_coef_bytes(int T, int n) { return (size_t)n * ((T + kC - 1) / kC) * kCoef * 4; }
size_t chunk_state_bytes(int T, int n, int dk, int dv) {
  return (size_t)n * ((T + kC - 1) / kC - 1) * dk * dv * 4;
}

template <int DK, int DV>
int launch_chunked(const float* q, const float* kb, const float* v, const float* decay, int T,
                   int n, float* o, char* ws, hipStream_t s) {
  const int nchunk = (T + kC - 1) / kC;
  float* coef = (float*)ws;
  float* S = (float*)(ws + mx_align_up(chunk_coef_bytes(T, n), 256));
  mx_clear_error();
  if (nchunk > 1) {
    hipLaunchKernelGGL(k_la_chunk_coef, dim3((unsigned)mx_ceil_div(n * nchunk, 4)), dim3(256),
                       0, s, decay, T, n, nchunk, coef);
    MX_TRY(mx_launch_status());
    constexpr int BPH = (DV / 32) * (DK / 64);
    hipLaunchKernelGGL((k_la_chunk_states<DK, DV>), dim3((unsigned)(n * BPH)), dim3(64 * LA_ST_NW), 0, s,
                       kb, v, coef, T, n, nchunk, S);
    MX_TRY(mx_launch_status());
  }
  hipLaunchKernelGGL((k_la_chunk_out<DK, DV>), dim3((unsigned)(nchunk * n)), dim3(256), 0, s,
                     q, kb, v, decay, S, T, n, nchunk, o);
  return mx_launch_status();
}

bool chunk_shape(int dk, int dv) { return (dk == 64 || dk == 128) && (dv == 64 || dv == 128); }

}  // namespace

size_t mx_la_chunk_ws_bytes(int T, int n, int dk, int dv) {
  if (T <= 0 || !chunk_shape(dk, dv)) return 0;
  return mx_align_up(chunk_coef_bytes(T, n), 256) + chunk_state_bytes(T, n, dk, dv);
}

// Chunked scan for the head shapes it is built for (key and value heads of 64 or 128), with
// `ws` of mx_la_chunk_ws_bytes; MX_ERR_UNSUPPORTED for other shapes (the caller then runs
// the token-sequential scan).
int mx_la_chunked_scan(const float* q, const float* kb, const float* v, const float* decay,
                       int T, int n, int dk, int dv, float* o, void* ws, hipStream_t s) {
  if (T <= 0 || n <= 0) return MX_ERR_INVALID;
  if (!chunk_shape(dk, dv) || !ws) return MX_ERR_UNSUPPORTED;
  // buffer descriptors: byte offsets below 2^31
  if ((long)T * n * (dk > dv ? dk : dv) * 4 >= (1l << 31) ||
      chunk_coef_bytes(T, n) >= (1ul << 31) ||
      (size_t)((T + kC - 1) / kC) * dk * dv * 4 >= (1ul << 31))
    return MX_ERR_UNSUPPORTED;
  if (!mx_aligned16(q) || !mx_aligned16(kb) || !mx_aligned16(v) || !mx_aligned16(o) ||
      !mx_aligned16(ws))
    return MX_ERR_UNSUPPORTED;
  char* w = (char*)ws;
  if (dk == 128 && dv == 128) return launch_chunked<128, 128>(q, kb, v, decay, T, n, o, w, s);
  if (dk == 64 && dv == 64) return launch_chunked<64, 64>(q, kb, v, decay, T, n, o, w, s);
  if (dk == 128 && dv == 64) return launch_chunked<128, 64>(q, kb, v, decay, T, n, o, w, s);
  return launch_chunked<64, 128>(q, kb, v, decay, T, n, o, w, s);
}
