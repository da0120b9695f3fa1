// Qwen3-Next gated full-attention block on the device:
//   rmsnorm -> q (+gate) / k / v projections -> qk-norm + partial RoPE -> causal attention
//   (fp32 MFMA, sigmoid gate fused) -> o projection -> residual,
// i.e. Qwen3NextExecutor._full_attn_block (offload_runtime/executors/qwen3_next.py:161-205)
// with rope / partial_rope / rms_norm_no_weight / repeat_kv of
// offload_runtime/executors/_common.py:105-153.  Everything runs on the caller's stream out
// of the caller's workspace.
#include <math.h>

#include "mx_common.h"
#include "mx_internal.h"
#include "mx_lds_copy.h"

namespace {

struct FaDims {
  int H, nh, nkv, hd, rd;
  int qw;  // q_proj rows: 2 nh hd ([q | gate] halves)
  int kw;  // k / v rows: nkv hd
  int od;  // attention output width: nh hd
};

FaDims dims_of(const MxFullAttnDesc* d) {
  FaDims m;
  m.H = d->hidden;
  m.nh = d->n_heads;
  m.nkv = d->n_kv_heads;
  m.hd = d->head_dim;
  m.rd = d->rotary_dim;
  m.qw = 2 * m.nh * m.hd;
  m.kw = m.nkv * m.hd;
  m.od = m.nh * m.hd;
  return m;
}

int check_desc(const MxFullAttnDesc* d) {
  if (!d) return MX_ERR_INVALID;
  if (d->hidden <= 0 || d->n_heads <= 0 || d->n_kv_heads <= 0 || d->head_dim <= 0 ||
      d->rotary_dim < 0 || d->rotary_dim > d->head_dim || !(d->rope_theta > 0.0))
    return MX_ERR_INVALID;
  if (d->n_heads % d->n_kv_heads) return MX_ERR_INVALID;  // repeat_kv needs whole repeats
  if (d->rotary_dim % 2) return MX_ERR_INVALID;           // rope splits the rotary dims in halves
  if (d->param_dtype != MX_DT_F32 && d->param_dtype != MX_DT_F16) return MX_ERR_INVALID;
  if (d->weight_dtype != MX_DT_F32 && d->weight_dtype != MX_DT_F16 && d->weight_dtype != MX_DT_I8)
    return MX_ERR_INVALID;
  if (d->head_dim % 4 || d->head_dim > 256) return MX_ERR_UNSUPPORTED;
  const long qw = 2l * d->n_heads * d->head_dim;
  if (qw * d->hidden >= (1l << 31)) return MX_ERR_UNSUPPORTED;
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

struct FaWork {
  MxFullAttnViews v;
  MxDenseWork dw;  // projections: entry 0 q, 1 k, 2 v, 3 o
  half_t* k16;     // fp16 path: keys [n_kv][Tp][DP] (Tp = T padded to 32 keys, DP = hd padded to 32)
  half_t* v16t;    // fp16 path: values per 32-key tile, transposed [n_kv][Tp / 32][DP][32]
};

constexpr int FA_KT = 32;  // keys per transposed value block (fp16 path)
#ifndef FA_H_S32
#define FA_H_S32 2  // 32-key blocks per attention tile of the fp16 path
#endif
constexpr int FA_TPAD = FA_KT * FA_H_S32;  // keys are padded to whole tiles

int layout(const MxFullAttnDesc* d, int T, void* ws, FaWork* w, size_t* total) {
  MX_TRY(check_desc(d));
  if (T < 0) return MX_ERR_INVALID;
  const size_t Tn = T > 0 ? T : 1;
  const FaDims m = dims_of(d);
  const bool f32 = d->weight_dtype == MX_DT_F32;
  Carve c{(char*)ws};
  FaWork t;
  t.v.h32 = (float*)c.take(Tn * m.H * 4);
  t.v.h16 = f32 ? nullptr : c.take(Tn * m.H * 2);
  t.v.qg = (float*)c.take(Tn * m.qw * 4);
  t.v.k = (float*)c.take(Tn * m.kw * 4);
  t.v.v = (float*)c.take(Tn * m.kw * 4);
  t.v.act = c.take(Tn * m.od * (f32 ? 4 : 2));
  t.v.y = (float*)c.take(Tn * m.H * 4);
  char* dwb = (char*)c.take(mx_dense_work_bytes((int)Tn, d->weight_dtype, 4));
  mx_dense_work_carve(dwb, (int)Tn, d->weight_dtype, 4, &t.dw);
  if (!f32) {
    const size_t tp = (Tn + FA_TPAD - 1) / FA_TPAD * FA_TPAD, dp = (size_t)(m.hd + 31) / 32 * 32;
    t.k16 = (half_t*)c.take((size_t)m.nkv * tp * dp * 2);
    t.v16t = (half_t*)c.take((size_t)m.nkv * tp * dp * 2);
  } else {
    t.k16 = t.v16t = nullptr;
  }
  if (w) *w = t;
  if (total) *total = mx_align_up(c.off, 256);
  return MX_OK;
}

// ------------------------------------------------------------------------------------
// qk-norm + RoPE, in place on the q half of the q projection and on k.  A block per
// (token, rpb head rows), its 4 waves taking the rows in turn, lane handling dims i = lane +
// 64 j (rpb = all the token's rows for long inputs, 4 for short ones, whose few blocks would
// otherwise run the rows of a token one after another).
// y = (x / rms(x)) * w when the norm weight is given (rms_norm_no_weight then the weight,
// _common.py:137-140), then on the first rotary_dim dims the rotate-half RoPE of
// _common.py:105-127: with half = rotary_dim / 2, freq_j = 1 / theta^(j / half) (fp64),
// angle = fp32(t * freq_j), out_i = y_i cos - y_{i+half} sin (i < half), y_i cos +
// y_{i-half} sin (half <= i < rd).  The token's cos / sin table (the same for every head)
// is computed once per block into LDS, so the fp64 power and the fp32 cos / sin run once
// per (block, frequency), not once per (token, head, dim).  Each lane recomputes its partner's
// normalised value from memory (same rms), so there is no cross-lane exchange; all loads of
// a row precede its reduction, all its stores follow it.
template <int EPT>
__global__ __launch_bounds__(256) void k_fa_rope_tok(float* __restrict__ qg,
                                                     float* __restrict__ kk,
                                                     const void* __restrict__ qn_w,
                                                     const void* __restrict__ kn_w, int pdt,
                                                     FaDims m, double theta, float eps,
                                                     int rpb) {
#pragma clang fp contract(off)
  __shared__ float cs[128], sn[128];  // rotary_dim / 2 <= head_dim / 2 <= 128
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = m.rd / 2;
  if (tid < half) {
    const double f = 1.0 / pow(theta, (double)tid / (double)half);
    const float ang = (float)((double)t * f);
    cs[tid] = cosf(ang);
    sn[tid] = sinf(ang);
  }
  __syncthreads();
  const int slot_end = min(m.nh + m.nkv, (int)(blockIdx.y + 1) * rpb);
  for (int slot = blockIdx.y * rpb + wave; slot < slot_end; slot += 4) {
    const bool isq = slot < m.nh;
    float* row = isq ? qg + (size_t)t * m.qw + (size_t)slot * m.hd
                     : kk + (size_t)t * m.kw + (size_t)(slot - m.nh) * m.hd;
    const void* nw = isq ? qn_w : kn_w;
    float x[EPT], xp[EPT], w[EPT], wp[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int i = lane + 64 * j;
      const bool valid = i < m.hd;
      const int ic = valid ? i : 0;
      const int p = ic < m.rd ? (ic < half ? ic + half : ic - half) : ic;
      x[j] = valid ? row[ic] : 0.f;
      xp[j] = valid ? row[p] : 0.f;
      w[j] = nw ? mx_load_param(nw, pdt, ic) : 1.f;
      wp[j] = nw ? mx_load_param(nw, pdt, p) : 1.f;
    }
    float rms = 1.f;
    if (nw) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < EPT; ++j) ss += x[j] * x[j];
      ss = mx_wave_sum(ss);
      rms = sqrtf(ss / (float)m.hd + eps);
    }
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int i = lane + 64 * j;
      if (i >= m.hd) break;
      const float y = nw ? (x[j] / rms) * w[j] : x[j];
      float out = y;
      if (i < m.rd) {
        const float yp = nw ? (xp[j] / rms) * wp[j] : xp[j];
        const int jj = i < half ? i : i - half;
        const float c = cs[jj], sv = sn[jj];
        out = i < half ? y * c - yp * sv : y * c + yp * sv;
      }
      row[i] = out;
    }
  }
}

// ------------------------------------------------------------------------------------
// Causal attention on fp32 MFMA (v_mfma_f32_16x16x4_f32), flash-style.  Block = 4 waves,
// one query head h, 64 queries (16 per wave); key tiles of 16 keys of the head's key/value
// head (h / (n_heads / n_kv_heads), repeat_kv) staged in LDS: K row-major, V transposed.
// Per tile each wave computes S^T = K Q^T (16 keys x 16 queries: lane l holds
// S^T[4 (l / 16) + r][l % 16], so query l % 16 is lane-local) with Q held in registers, then
// the online softmax per query (running max / sum; scores are (q.k) / sqrt(head_dim) with
// keys after the query masked, qwen3_next.py:191-194), and O^T += V^T P, whose B operand is
// exactly the lane's probabilities (the MFMA k-slot of lane l at step r is key 4 (l/16) + r,
// the same key on both operands).  O^T keeps the query in the lane too, so the softmax
// rescale needs no shuffle.  The epilogue divides by the row sum and multiplies by
// sigmoid(gate) (qwen3_next.py:201-202), writing the o_proj input.  Head dims are padded to
// a multiple of 16 with zeros.
// ------------------------------------------------------------------------------------
#ifndef FA_NS
#define FA_NS 2  // 16-key sub-tiles per staged key tile
#endif

#ifndef FA_WPE
#define FA_WPE 2  // waves per SIMD the register budget is sized for
#endif

template <int NC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, FA_WPE))) void k_fa_attn(const float* __restrict__ qg,
                                                 const float* __restrict__ kk,
                                                 const float* __restrict__ vv, FaDims m, int T,
                                                 float sqrt_hd, float* __restrict__ act32,
                                                 half_t* __restrict__ act16) {
  constexpr int DP = NC * 16;      // padded head dim
  constexpr int NS = FA_NS;        // 16-key sub-tiles per tile
  constexpr int KT = 16 * NS;      // keys per tile
  constexpr int KS = DP + 4;       // LDS row stride of the K tile (floats)
  constexpr int VS = KT + 4;       // LDS row stride of the transposed V tile
  constexpr int NP = KT * DP / 4;  // float4 pieces of K (and of V) per tile
  __shared__ __align__(16) float sk[KT * KS];
  __shared__ __align__(16) float svt[DP * VS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = blockIdx.y;
  const int q0 = (gridDim.x - 1 - blockIdx.x) * 64;  // longest query blocks first
  const int qw0 = q0 + wave * 16;
  const int kvh = h / (m.nh / m.nkv);
  const int ql = lane & 15, g = lane >> 4;
  const int qi = qw0 + ql;
  const int qc = min(qi, T - 1);

  // Q fragment (B operand of S^T): qf[c] = Q[qi][16 c + 4 g .. + 3].
  float4 qf[NC];
  const float* qrow = qg + (size_t)qc * m.qw + (size_t)h * m.hd;
  // Loads at clamped (in-row) offsets first, all in flight together; pad dims zeroed after.
#pragma unroll
  for (int c = 0; c < NC; ++c) qf[c] = *(const float4*)(qrow + min(16 * c + 4 * g, m.hd - 4));
#pragma unroll
  for (int c = 0; c < NC; ++c)
    if (16 * c + 4 * g >= m.hd) qf[c] = make_float4(0.f, 0.f, 0.f, 0.f);
  float4_t oacc[NC];
#pragma unroll
  for (int f = 0; f < NC; ++f) oacc[f] = (float4_t){0.f, 0.f, 0.f, 0.f};
  float mrun = -INFINITY, lrun = 0.f;

  const int kend = min(T, q0 + 64);
  const int ntile = (kend + KT - 1) / KT;
  const int wq_last = min(qw0 + 15, T - 1);  // last real query of this wave
  const float* kbase = kk + (size_t)kvh * m.hd;
  const float* vbase = vv + (size_t)kvh * m.hd;

  // Tile staging: piece p = (key p % KT, dims 4 (p / KT) .. + 3), so consecutive threads
  // write consecutive keys (banks) of the transposed V tile.
  for (int kt = 0; kt < ntile; ++kt) {
    const int k0 = kt * KT;
    __syncthreads();  // the previous tile's LDS reads are done
    for (int p = tid; p < NP; p += 256) {
      const int key = p % KT, d4 = (p / KT) * 4;
      const int s = k0 + key;
      float4 k4 = make_float4(0.f, 0.f, 0.f, 0.f), v4 = k4;
      if (s < T && d4 < m.hd) {
        k4 = *(const float4*)(kbase + (size_t)s * m.kw + d4);
        v4 = *(const float4*)(vbase + (size_t)s * m.kw + d4);
      }
      *(float4*)(sk + key * KS + d4) = k4;
      svt[(d4 + 0) * VS + key] = v4.x;
      svt[(d4 + 1) * VS + key] = v4.y;
      svt[(d4 + 2) * VS + key] = v4.z;
      svt[(d4 + 3) * VS + key] = v4.w;
    }
    __syncthreads();
    if (k0 > wq_last) continue;  // every key of the tile is after every query of the wave

    // S^T per 16-key sub-tile j, four independent accumulation chains each (dims 4 e + 16 c
    // go to chain e), summed in a fixed order.
    float sv[NS][4];
    float mt = -INFINITY;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      float4_t sc[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[e] = (float4_t){0.f, 0.f, 0.f, 0.f};
      const float* krow = sk + (16 * j + ql) * KS + 4 * g;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const float4 a = *(const float4*)(krow + 16 * c);
        sc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, qf[c].x, sc[0], 0, 0, 0);
        sc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, qf[c].y, sc[1], 0, 0, 0);
        sc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, qf[c].z, sc[2], 0, 0, 0);
        sc[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, qf[c].w, sc[3], 0, 0, 0);
      }
      const float4_t st = (sc[0] + sc[1]) + (sc[2] + sc[3]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = k0 + 16 * j + 4 * g + r;
        const bool masked = key > qi || key >= T;
        sv[j][r] = masked ? -INFINITY : st[r] / sqrt_hd;
        mt = fmaxf(mt, sv[j][r]);
      }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float mnew = fmaxf(mrun, mt);
    const float alpha = expf(mrun - mnew);  // 0 on the first tile (mrun = -inf)
    float p[NS][4];
    float ps = 0.f;
#pragma unroll
    for (int j = 0; j < NS; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[j][r] = expf(sv[j][r] - mnew);
        ps += p[j][r];
      }
    lrun = lrun * alpha + ps;
    // The accumulators are rescaled only when some query's running max moved (alpha < 1);
    // once the maxima settle most tiles skip the rescale.
    const bool grow = mnew > mrun;
    mrun = mnew;
    if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
      for (int f = 0; f < NC; ++f) oacc[f] *= alpha;
    }
#pragma unroll
    for (int f = 0; f < NC; ++f) {
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const float4 a = *(const float4*)(svt + (16 * f + ql) * VS + 16 * j + 4 * g);
        oacc[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, p[j][0], oacc[f], 0, 0, 0);
        oacc[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, p[j][1], oacc[f], 0, 0, 0);
        oacc[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, p[j][2], oacc[f], 0, 0, 0);
        oacc[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, p[j][3], oacc[f], 0, 0, 0);
      }
    }
  }
  float l = lrun + __shfl_xor(lrun, 16);
  l = l + __shfl_xor(l, 32);
  if (qi >= T) return;
  const float* gate = qg + (size_t)qi * m.qw + (size_t)m.od + (size_t)h * m.hd;
  const size_t orow = (size_t)qi * m.od + (size_t)h * m.hd;
  float4 gv[NC];  // gate loads first (clamped offsets), then the ordered math and stores
#pragma unroll
  for (int f = 0; f < NC; ++f) gv[f] = *(const float4*)(gate + min(16 * f + 4 * g, m.hd - 4));
#pragma unroll
  for (int f = 0; f < NC; ++f) {
    const int d = 16 * f + 4 * g;
    if (d >= m.hd) continue;
    const float a0 = (oacc[f][0] / l) * mx_sigmoid(gv[f].x);
    const float a1 = (oacc[f][1] / l) * mx_sigmoid(gv[f].y);
    const float a2 = (oacc[f][2] / l) * mx_sigmoid(gv[f].z);
    const float a3 = (oacc[f][3] / l) * mx_sigmoid(gv[f].w);
    if (act16) {
      act16[orow + d] = (half_t)a0;
      act16[orow + d + 1] = (half_t)a1;
      act16[orow + d + 2] = (half_t)a2;
      act16[orow + d + 3] = (half_t)a3;
    } else {
      *(float4*)(act32 + orow + d) = make_float4(a0, a1, a2, a3);
    }
  }
}

// ------------------------------------------------------------------------------------
// The same causal attention for fp16 / int8 projections (the block's fp16 path, whose
// output is rounded to fp16 anyway): q, k, v rounded to fp16 and both products on
// v_mfma_f32_16x16x32_f16 with fp32 accumulation; softmax statistics stay fp32.
//
// k_fa_pack_kv first writes fp16 copies of the keys (after RoPE) and values: keys
// row-major per key/value head, values transposed per 32-key tile with the keys of a
// tile in k-slot order (below), so staging a tile is a straight 16-byte copy.
//
// k_fa_attn_h: block = NW waves, one query head, 16 QS NW queries (QS sets of 16 per
// wave); tiles of 32 S32 keys, the next tile's 16-byte pieces loaded into registers while a
// tile computes.
// Each XCD runs whole heads, consecutive ones, so the heads of a key/value head read its
// packed keys and values through one XCD's L2 (Qwen3-Next, 16 heads over 2 key/value
// heads at 4096 tokens: 393 -> 250 us against blocks dealt round-robin over all heads).
//   S^T = K Q^T per 16-key sub-tile: A = K rows (16 keys x 32 dims from LDS), B = the
//     wave's Q (registers, 8 fp16 dims per lane per 32-dim chunk); lane (j, g) gets
//     S^T[4 g + r][j], so query j = lane % 16 is lane-local.
//   O^T += V^T P per 16-dim slab: the MFMA k-slot (g, e) stands for key 4 g + e of
//     sub-tile 0 (e < 4) and key 4 g + e - 4 of sub-tile 1 (e >= 4), so the B operand is
//     exactly the lane's own 8 probabilities, and A is 16 bytes of a V^T row.
// LDS rows are padded (K: +16 B, V^T: +16 B) so the 16-byte fragment reads of a quarter
// wave hit distinct banks.
// ------------------------------------------------------------------------------------
__device__ __forceinline__ int fa_slot(int key) {  // key of a 32-key tile -> k-slot
  return 8 * ((key & 15) >> 2) + (key & 3) + 4 * (key >> 4);
}

__global__ __launch_bounds__(256) void k_fa_pack_kv(const float* __restrict__ kk,
                                                    const float* __restrict__ vv, FaDims m,
                                                    int T, int Tp, int DP,
                                                    half_t* __restrict__ k16,
                                                    half_t* __restrict__ v16t) {
  const int nc8 = DP / 8;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  const long total = (long)m.nkv * Tp * nc8;
  if (i >= total) return;
  const int c8 = (int)(i % nc8);
  const long r = i / nc8;
  const int s = (int)(r % Tp), kvh = (int)(r / Tp);
  half8_t kh, vh;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int d = 8 * c8 + e;
    const bool ok = s < T && d < m.hd;
    const size_t src = (size_t)s * m.kw + (size_t)kvh * m.hd + d;
    kh[e] = (half_t)(ok ? kk[src] : 0.f);
    vh[e] = (half_t)(ok ? vv[src] : 0.f);
  }
  *(half8_t*)(k16 + ((size_t)kvh * Tp + s) * DP + 8 * c8) = kh;
  half_t* vt = v16t + ((size_t)kvh * (Tp / FA_KT) + s / FA_KT) * DP * FA_KT + fa_slot(s % FA_KT);
#pragma unroll
  for (int e = 0; e < 8; ++e) vt[(size_t)(8 * c8 + e) * FA_KT] = vh[e];
}

#ifndef FA_H_WPE
#define FA_H_WPE 2  // waves per SIMD the fp16 attention is compiled for
#endif
#ifndef FA_H_XCD
#define FA_H_XCD 1  // XCD-aware head runs in k_fa_attn_h
#endif

template <int NC, int NW, int S32, int QS>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(FA_H_WPE, FA_H_WPE))) void k_fa_attn_h(const float* __restrict__ qg,
                                                       const half_t* __restrict__ k16,
                                                       const half_t* __restrict__ v16t,
                                                       FaDims m, int T, int Tp, float sqrt_hd,
                                                       half_t* __restrict__ act16) {
  constexpr int DP = NC * 32;          // padded head dim
  constexpr int KT = 32 * S32;         // keys per tile
  constexpr int KR = DP + 8;           // K tile row stride (halfs)
  constexpr int VR = FA_KT + 8;        // V^T row stride (halfs): one row per (32-key block, dim)
  constexpr int NT = 64 * NW;          // threads
  constexpr int KCH = KT * DP / 8;     // 16-byte pieces of a K tile (= of a V^T tile)
  constexpr int PPT = (KCH + NT - 1) / NT;  // pieces of each per thread
  constexpr int WQ = 16 * QS;          // queries per wave (QS sets of 16)
  __shared__ __align__(16) half_t sk[KT * KR];
  __shared__ __align__(16) half_t svt[S32 * DP * VR];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int QB = WQ * NW;
  const int nqb = gridDim.x;
  int h = blockIdx.y, qx = blockIdx.x;  // qx = 0: the longest query block (the last one)
  if (FA_H_XCD) {
    // Blocks go to the 8 XCDs round-robin by linear id.  When every XCD gets whole heads,
    // deal each XCD a run of consecutive heads (so heads sharing a key/value head share
    // that XCD's L2) and order the run longest query block first across its heads.
    const int nb = nqb * gridDim.y, per = nb >> 3;
    if ((nb & 7) == 0 && per % nqb == 0) {
      const int b = blockIdx.x + nqb * blockIdx.y, hpr = per / nqb, i = b >> 3;
      h = (b & 7) * hpr + i % hpr;
      qx = i / hpr;
    }
  }
  const int q0 = (nqb - 1 - qx) * QB;
  const int qw0 = q0 + wave * WQ;
  const int kvh = h / (m.nh / m.nkv);
  const int ql = lane & 15, g = lane >> 4;
  int qi[QS];
#pragma unroll
  for (int u = 0; u < QS; ++u) qi[u] = qw0 + 16 * u + ql;

  half8_t qf[QS][NC];
#pragma unroll
  for (int u = 0; u < QS; ++u) {
    const float* qrow = qg + (size_t)min(qi[u], T - 1) * m.qw + (size_t)h * m.hd;
    // Loads at clamped (in-row) offsets first, all in flight together; pad dims zeroed after.
    float4 qv[2 * NC];
#pragma unroll
    for (int i = 0; i < 2 * NC; ++i)
      qv[i] = *(const float4*)(qrow + min(32 * (i >> 1) + 8 * g + 4 * (i & 1), m.hd - 4));
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float4 v = qv[2 * c + (e >> 2)];
        const float x = (e & 3) == 0 ? v.x : (e & 3) == 1 ? v.y : (e & 3) == 2 ? v.z : v.w;
        qf[u][c][e] = (half_t)(32 * c + 8 * g + e < m.hd ? x : 0.f);
      }
  }
  float4_t oacc[QS][2 * NC];
#pragma unroll
  for (int u = 0; u < QS; ++u)
#pragma unroll
    for (int f = 0; f < 2 * NC; ++f) oacc[u][f] = (float4_t){0.f, 0.f, 0.f, 0.f};
  float mrun[QS], lrun[QS];
#pragma unroll
  for (int u = 0; u < QS; ++u) mrun[u] = -INFINITY, lrun[u] = 0.f;

  const int kend = min(T, q0 + QB);
  const int ntile = (kend + KT - 1) / KT;
  const int wq_last = min(qw0 + WQ - 1, T - 1);
  const half_t* kb = k16 + (size_t)kvh * Tp * DP;
  const half_t* vb = v16t + (size_t)kvh * Tp * DP;  // Tp / KT tiles of DP x KT
  // Scores in the base-2 domain: s2 = (q.k) log2(e) / sqrt(head_dim), p = 2^(s2 - max).
  const float rs = 1.4426950408889634f / sqrt_hd;

  // Staging pieces of this thread: K piece i -> row i / (DP / 8), V^T piece i -> row i / 4
  // (the rows of the S32 value blocks follow each other).
  int4_t pk[PPT], pv[PPT];
#pragma unroll
  for (int u = 0; u < PPT; ++u) {
    const int i = tid + NT * u;
    if (KCH % NT == 0 || i < KCH) {
      pk[u] = ((const int4_t*)kb)[i];
      pv[u] = ((const int4_t*)vb)[i];
    }
  }
  for (int kt = 0; kt < ntile; ++kt) {
    const int k0 = kt * KT;
    __syncthreads();  // the previous tile's LDS reads are done
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
      const int i = tid + NT * u;
      if (KCH % NT == 0 || i < KCH) {
        *(int4_t*)(sk + (i / (DP / 8)) * KR + (i % (DP / 8)) * 8) = pk[u];
        *(int4_t*)(svt + (i >> 2) * VR + (i & 3) * 8) = pv[u];
      }
    }
    __syncthreads();
    if (kt + 1 < ntile) {
      const int4_t* ks = (const int4_t*)(kb + (size_t)(kt + 1) * KT * DP);
      const int4_t* vs = (const int4_t*)(vb + (size_t)(kt + 1) * KT * DP);
#pragma unroll
      for (int u = 0; u < PPT; ++u) {
        const int i = tid + NT * u;
        if (KCH % NT == 0 || i < KCH) {
          pk[u] = ks[i];
          pv[u] = vs[i];
        }
      }
    }
    if (k0 > wq_last) continue;  // every key of the tile is after every query of the wave
    // Only tiles reaching past the wave's first query or past T need the mask.
    const bool need_mask = k0 + KT - 1 > qw0 || k0 + KT > T;

    // S^T sub-tiles: each K fragment read from LDS feeds the QS query sets.
    float sv[QS][2 * S32][4];
#pragma unroll
    for (int b = 0; b < 2 * S32; ++b) {
      float4_t sc[QS];
#pragma unroll
      for (int u = 0; u < QS; ++u) sc[u] = (float4_t){0.f, 0.f, 0.f, 0.f};
      const half_t* krow = sk + (16 * b + ql) * KR + 8 * g;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const half8_t kf = *(const half8_t*)(krow + 32 * c);
#pragma unroll
        for (int u = 0; u < QS; ++u)
          sc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[u][c], sc[u], 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < QS; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) sv[u][b][r] = sc[u][r] * rs;
      if (need_mask) {
#pragma unroll
        for (int u = 0; u < QS; ++u)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = k0 + 16 * b + 4 * g + r;
            if (key > qi[u] || key >= T) sv[u][b][r] = -INFINITY;
          }
      }
    }
    half8_t pf[QS][S32];
#pragma unroll
    for (int u = 0; u < QS; ++u) {
      float mt = -INFINITY;
#pragma unroll
      for (int b = 0; b < 2 * S32; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) mt = fmaxf(mt, sv[u][b][r]);
      mt = fmaxf(mt, __shfl_xor(mt, 16));
      mt = fmaxf(mt, __shfl_xor(mt, 32));
      // A set whose queries all precede the tile sees only -inf here and keeps its max
      // (finite from tile 0 on), so its probabilities are 0 and alpha is 1.
      const float mnew = fmaxf(mrun[u], mt);
      const float alpha = __builtin_amdgcn_exp2f(mrun[u] - mnew);  // 0 on the first tile
      float ps = 0.f;
#pragma unroll
      for (int b = 0; b < 2 * S32; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pv2 = __builtin_amdgcn_exp2f(sv[u][b][r] - mnew);
          ps += pv2;
          pf[u][b >> 1][4 * (b & 1) + r] = (half_t)pv2;
        }
      lrun[u] = lrun[u] * alpha + ps;
      const bool grow = mnew > mrun[u];
      mrun[u] = mnew;
      if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
        for (int f = 0; f < 2 * NC; ++f) oacc[u][f] *= alpha;
      }
    }
    // O^T += V^T P: each V^T fragment read from LDS feeds the QS query sets.
#pragma unroll
    for (int s32 = 0; s32 < S32; ++s32)
#pragma unroll
      for (int f = 0; f < 2 * NC; ++f) {
        const half8_t vf = *(const half8_t*)(svt + (s32 * DP + 16 * f + ql) * VR + 8 * g);
#pragma unroll
        for (int u = 0; u < QS; ++u)
          oacc[u][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[u][s32], oacc[u][f], 0, 0, 0);
      }
  }
#pragma unroll
  for (int u = 0; u < QS; ++u) {
    float l = lrun[u] + __shfl_xor(lrun[u], 16);
    l = l + __shfl_xor(l, 32);
    if (qi[u] >= T) continue;
    const float* gate = qg + (size_t)qi[u] * m.qw + (size_t)m.od + (size_t)h * m.hd;
    const size_t orow = (size_t)qi[u] * m.od + (size_t)h * m.hd;
    float4 gv[2 * NC];  // gate loads first (clamped offsets), then the math and 8-byte stores
#pragma unroll
    for (int f = 0; f < 2 * NC; ++f)
      gv[f] = *(const float4*)(gate + min(16 * f + 4 * g, m.hd - 4));
    const float il = 1.f / l;
#pragma unroll
    for (int f = 0; f < 2 * NC; ++f) {
      const int d = 16 * f + 4 * g;
      if (d >= m.hd) continue;
      typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
      const half4_t o = {(half_t)(oacc[u][f][0] * il * mx_sigmoid(gv[f].x)),
                         (half_t)(oacc[u][f][1] * il * mx_sigmoid(gv[f].y)),
                         (half_t)(oacc[u][f][2] * il * mx_sigmoid(gv[f].z)),
                         (half_t)(oacc[u][f][3] * il * mx_sigmoid(gv[f].w))};
      *(half4_t*)(act16 + orow + d) = o;
    }
  }
}

// ------------------------------------------------------------------------------------
// k_fa_attn_d: the fp16 attention with the key / value tiles copied straight into LDS by
// the buffer loads' LDS mode and two query sets (32 queries) per wave.
// A tile is 32 keys: 2 NC key fragments (16 keys x 32 dims) and 2 NC value fragments (16
// dims x the 32 keys in k-slot order), 1 KiB each, 32 KiB at NC = 8, double-buffered; a
// wave's copies of tile t + 1 are issued right after the barrier that opens tile t, so
// one tile is in flight while one computes, and no register holds a staged piece.  Every
// fragment read from LDS feeds both query sets' MFMAs, half the LDS reads per product of
// one set per wave.  Copy lane l loads row l / 4 of its fragment, so four consecutive
// lanes read one row's 64 contiguous bytes, in the chunk rotation of mx_lds_copy.h under
// which the MFMA operand reads of a fragment are free of bank conflicts.  Keys and values
// come through buffer descriptors over the key / value head's Tp rows (rows past T are the
// packed zeros, masked anyway).  The products, the softmax and the epilogue are those of
// k_fa_attn_h with one 32-key block per tile.
// ------------------------------------------------------------------------------------
#ifndef FA_D_WPE
#define FA_D_WPE 2  // waves per SIMD the LDS-copy attention is compiled for
#endif
#ifndef FA_D_NB
#define FA_D_NB 2  // key / value tile buffers in LDS (2-4)
#endif
#ifndef FA_D_PD
#define FA_D_PD 2  // LDS fragment reads in flight ahead of the MFMAs
#endif
#ifndef FA_D_TAU
#define FA_D_TAU 8.f  // lazy-rescale threshold of the running max (base-2 units)
#endif
#ifndef FA_D_PAIR
#define FA_D_PAIR 1  // long and short query blocks paired on each CU
#endif

// Max over the lanes l, l ^ 16, l ^ 32 and l ^ 48 (one query's four lane groups) without
// going through LDS: permlane16_swap exchanges 16-lane rows 2k and 2k + 1 between its two
// operands and permlane32_swap the wave's halves, so with both operands v the two results
// hold v of the lane and of its partner row (half).
__device__ __forceinline__ float fa_rowmax4(float v) {
  const unsigned b = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  v = fmaxf(__builtin_bit_cast(float, r[0]), __builtin_bit_cast(float, r[1]));
  const unsigned c = __builtin_bit_cast(unsigned, v);
  const auto h = __builtin_amdgcn_permlane32_swap(c, c, false, false);
  return fmaxf(__builtin_bit_cast(float, h[0]), __builtin_bit_cast(float, h[1]));
}

template <int NC, int NW, int QS>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(FA_D_WPE, FA_D_WPE)))
void k_fa_attn_d(const float* __restrict__ qg, const half_t* __restrict__ k16,
                 const half_t* __restrict__ v16t, FaDims m, int T, int Tp, float sqrt_hd,
                 half_t* __restrict__ act16) {
  constexpr int DP = NC * 32;
  constexpr int KT = FA_KT;             // keys per tile
  constexpr int NFK = 2 * NC;           // key fragments per tile (fragment b NC + c)
  constexpr int NF = NFK + 2 * NC;      // then the value fragments (16-dim slabs)
  constexpr int FPW = NF / NW;          // copies per wave and tile
  constexpr int TILE = NF * 1024;
  constexpr int WQ = 16 * QS;
  static_assert(NF % NW == 0 && NFK % NW == 0, "fragments must divide among the waves");
  constexpr int NB = FA_D_NB;           // tile buffers: NB - 1 tiles in flight
  __shared__ __align__(1024) char lds[NB * TILE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int QB = WQ * NW;
  const int nqb = gridDim.x;
  int h = blockIdx.y, qx = blockIdx.x;  // qx = 0: the longest query block (the last one)
  if (FA_H_XCD) {  // whole heads per XCD (as k_fa_attn_h)
    const int nb = nqb * gridDim.y, per = nb >> 3;
    if ((nb & 7) == 0 && per % nqb == 0) {
      const int b = blockIdx.x + nqb * blockIdx.y, hpr = per / nqb, i = b >> 3;
      h = (b & 7) * hpr + i % hpr;
      qx = i / hpr;
      // The XCD's first half of the blocks (the longest query blocks, longest first) takes
      // one slot of each CU and the second half the other: with the second half shortest
      // first, a CU's two query blocks have about the same sum of key tiles (the causal work
      // of query block qx is proportional to nqb - qx).
      if (FA_D_PAIR && (nqb & 1) == 0 && i >= per / 2) qx = nqb - 1 - (i - per / 2) / hpr;
    }
  }
  const int q0 = (nqb - 1 - qx) * QB;
  const int qw0 = q0 + wave * WQ;
  const int kvh = h / (m.nh / m.nkv);
  const int ql = lane & 15, g = lane >> 4;
  int qi[QS];
#pragma unroll
  for (int u = 0; u < QS; ++u) qi[u] = qw0 + 16 * u + ql;

  const uint32_t head_bytes = (uint32_t)Tp * DP * 2;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(k16 + (size_t)kvh * Tp * DP), (short)0, (int)head_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(v16t + (size_t)kvh * Tp * DP), (short)0, (int)head_bytes, 0x00020000);
  const int cr = lane >> 2, cq = mx_frag_copy_chunk(lane);
  const int rpos = mx_frag_read_pos(ql, g);
  // Byte offsets: a lane part (row cr, chunk cq of a fragment) and a wave-uniform part.
  const uint32_t lane_k = (uint32_t)((cr * DP + 8 * cq) * 2);
  const uint32_t lane_v = (uint32_t)((cr * KT + 8 * cq) * 2);
  auto issue = [&](int kt) {
    char* buf = lds + (kt % NB) * TILE;
    const uint32_t t0 = (uint32_t)kt * KT * DP * 2;  // both tiles are KT x DP halfs
#pragma unroll
    for (int i = 0; i < FPW; ++i) {
      const int f = wave + i * NW;
      if (i * NW < NFK)  // key fragment: keys 16 (f / NC) + row, dims 32 (f % NC) + 8 chunk
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rk, (mx_lds_void*)(buf + f * 1024), 16, lane_k,
            (int)(t0 + (uint32_t)((16 * (f / NC) * DP + 32 * (f % NC)) * 2)), 0, 0);
      else  // value fragment: dims 16 (f - NFK) + row of the tile's V^T block
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rv, (mx_lds_void*)(buf + f * 1024), 16, lane_v,
            (int)(t0 + (uint32_t)(16 * (f - NFK) * KT * 2)), 0, 0);
    }
  };

  const int kend = min(T, q0 + QB);
  const int ntile = (kend + KT - 1) / KT;
#pragma unroll
  for (int t = 0; t < NB - 1; ++t)  // in flight while the queries load
    if (t < ntile) issue(t);

  // Scores in the base-2 domain: the queries are scaled by log2(e) / sqrt(head_dim) before
  // rounding to fp16, so S = K Q^T needs no scaling.
  const float rs = 1.4426950408889634f / sqrt_hd;
  // Queries as fp16 MFMA B fragments, four 32-dim chunks at a time (loads at clamped in-row
  // offsets, pad dims zeroed), so the staging registers stay few.
  half8_t qf[QS][NC];
#pragma unroll
  for (int u = 0; u < QS; ++u) {
    const float* qrow = qg + (size_t)min(qi[u], T - 1) * m.qw + (size_t)h * m.hd;
#pragma unroll
    for (int c0 = 0; c0 < NC; c0 += 4) {
      float4 qv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        qv[i] = *(const float4*)(qrow + min(32 * (c0 + (i >> 1)) + 8 * g + 4 * (i & 1), m.hd - 4));
#pragma unroll
      for (int c = c0; c < c0 + 4 && c < NC; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float4 v = qv[2 * (c - c0) + (e >> 2)];
          const float x = (e & 3) == 0 ? v.x : (e & 3) == 1 ? v.y : (e & 3) == 2 ? v.z : v.w;
          qf[u][c][e] = (half_t)(32 * c + 8 * g + e < m.hd ? x * rs : 0.f);
        }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  float4_t oacc[QS][2 * NC];
#pragma unroll
  for (int u = 0; u < QS; ++u)
#pragma unroll
    for (int f = 0; f < 2 * NC; ++f) oacc[u][f] = (float4_t){0.f, 0.f, 0.f, 0.f};
  float mrun[QS], lrun[QS];
#pragma unroll
  for (int u = 0; u < QS; ++u) mrun[u] = -INFINITY, lrun[u] = 0.f;
  const int wq_last = min(qw0 + WQ - 1, T - 1);

  // The wave computes the tiles up to its last query (nt_w of them); past those it only
  // keeps the block's copy pipeline going (two loops, so the accumulators never merge
  // across a skipped tile).
  const int nt_w = min(ntile, wq_last / KT + 1);
  // Wait for tile kt: the copies of the tiles issued after it (up to NB - 2) may stay out.
  static_assert(NB >= 2 && NB <= 4, "2 to 4 tile buffers");
  auto wait_tile = [&](int kt) {
    const int later = min(NB - 2, ntile - 1 - kt);  // tiles issued after kt
    if (NB == 4 && later == 2) mx_wait_copies_and_barrier<(NB == 4 ? 2 * FPW : 0)>();
    else if (NB >= 3 && later == 1) mx_wait_copies_and_barrier<(NB >= 3 ? FPW : 0)>();
    else mx_wait_copies_and_barrier<0>();
  };
  for (int kt = 0; kt < nt_w; ++kt) {
    // This wave's copies of tile kt have landed (those of the later tiles in flight may
    // not have), then everyone's have, and every wave is done with tile kt - 1, whose
    // buffer the copies of tile kt + NB - 1 overwrite.
    wait_tile(kt);
    if (kt + NB - 1 < ntile) issue(kt + NB - 1);
    const int k0 = kt * KT;
    const bool need_mask = k0 + KT - 1 > qw0 || k0 + KT > T;
    const char* buf = lds + (kt % NB) * TILE;
    // Fragments are read FA_D_PD steps ahead of the MFMAs that use them; the scheduling
    // barriers keep the compiler from hoisting every read of the tile (which would need far
    // more registers than two waves per SIMD leave).
    auto frag = [&](int f) { return *(const half8_t*)(buf + f * 1024 + rpos); };
    // S^T in 4 independent accumulator chains per wave: (query set, key half b) and, with
    // one query set, the parity of the 32-dim chunk as well; the fragments are taken
    // chunk-major (c, b), so consecutive MFMAs never wait on each other's results.
    constexpr int PAR = QS == 1 ? 2 : 1;
    float4_t sc[QS][2][PAR];
#pragma unroll
    for (int u = 0; u < QS; ++u)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int p = 0; p < PAR; ++p) sc[u][b][p] = (float4_t){0.f, 0.f, 0.f, 0.f};
    auto kidx = [](int i) { return (i & 1) * NC + (i >> 1); };  // step i -> key fragment b NC + c
    // Fragment ring: step i (key steps, then the value fragments) uses fr[i % PD] and
    // refills it with step i + PD's fragment.
    constexpr int PD = FA_D_PD;
    auto fidx = [&](int i) { return i < NFK ? kidx(i) : i; };
    half8_t fr[PD];
#pragma unroll
    for (int i = 0; i < PD; ++i) fr[i] = frag(fidx(i));
#pragma unroll
    for (int i = 0; i < NFK; ++i) {
      const int b = i & 1, c = i >> 1;
      const half8_t kf = fr[i % PD];
      fr[i % PD] = frag(fidx(i + PD));  // past the keys: the first value fragments
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < QS; ++u)
        sc[u][b][c % PAR] =
            __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[u][c], sc[u][b][c % PAR], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (PAR == 2) {
#pragma unroll
      for (int u = 0; u < QS; ++u)
#pragma unroll
        for (int b = 0; b < 2; ++b) sc[u][b][0] += sc[u][b][1];
    }
    half8_t pf[QS];
#pragma unroll
    for (int u = 0; u < QS; ++u) {
      if (need_mask) {  // tiles on the diagonal or past T
        const int lim = min(qi[u], T - 1) - (k0 + 4 * g);  // last key of the query, tile-relative
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (16 * b + r > lim) sc[u][b][0][r] = -INFINITY;
      }
      float mt = fmaxf(fmaxf(fmaxf(sc[u][0][0][0], sc[u][0][0][1]),
                             fmaxf(sc[u][0][0][2], sc[u][0][0][3])),
                       fmaxf(fmaxf(sc[u][1][0][0], sc[u][1][0][1]),
                             fmaxf(sc[u][1][0][2], sc[u][1][0][3])));
      mt = fa_rowmax4(mt);
      // Lazy rescale: a query's reference max moves only when the tile's max passes it by
      // more than FA_D_TAU (base-2 units), so the probabilities stay below 2^FA_D_TAU (fp16
      // holds them) and the accumulators are rescaled on few tiles.  Tile 0 holds key 0,
      // which every query sees, so the reference is finite from tile 0 on.
      const bool up = mt > mrun[u] + FA_D_TAU;
      if (__builtin_amdgcn_ballot_w64(up)) {
        const float mnew = up ? mt : mrun[u];
        const float alpha = __builtin_amdgcn_exp2f(mrun[u] - mnew);  // 1 where it stays
        lrun[u] *= alpha;
        mrun[u] = mnew;
#pragma unroll
        for (int f = 0; f < 2 * NC; ++f) oacc[u][f] *= alpha;
      }
      float ps = 0.f;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pv2 = __builtin_amdgcn_exp2f(sc[u][b][0][r] - mrun[u]);
          ps += pv2;
          pf[u][4 * b + r] = (half_t)pv2;
        }
      lrun[u] += ps;
    }
#pragma unroll
    for (int i = NFK; i < NF; ++i) {  // value fragment i: dims 16 (i - NFK) ..
      const half8_t vf = fr[i % PD];
      if (i + PD < NF) fr[i % PD] = frag(i + PD);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < QS; ++u)
        oacc[u][i - NFK] =
            __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[u], oacc[u][i - NFK], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  for (int kt = nt_w; kt < ntile; ++kt) {
    wait_tile(kt);
    if (kt + NB - 1 < ntile) issue(kt + NB - 1);
  }
#pragma unroll
  for (int u = 0; u < QS; ++u) {
    float l = lrun[u] + __shfl_xor(lrun[u], 16);
    l = l + __shfl_xor(l, 32);
    if (qi[u] >= T) continue;
    const float* gate = qg + (size_t)qi[u] * m.qw + (size_t)m.od + (size_t)h * m.hd;
    const size_t orow = (size_t)qi[u] * m.od + (size_t)h * m.hd;
    const float il = 1.f / l;
#pragma unroll
    for (int f0 = 0; f0 < 2 * NC; f0 += 4) {  // four 16-dim slabs at a time
      float4 gv[4];
#pragma unroll
      for (int f = 0; f < 4; ++f)
        gv[f] = *(const float4*)(gate + min(16 * (f0 + f) + 4 * g, m.hd - 4));
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const int d = 16 * (f0 + f) + 4 * g;
        if (f0 + f >= 2 * NC || d >= m.hd) continue;
        typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
        const float4_t a = oacc[u][f0 + f];
        const half4_t o = {(half_t)(a[0] * il * mx_sigmoid(gv[f].x)),
                           (half_t)(a[1] * il * mx_sigmoid(gv[f].y)),
                           (half_t)(a[2] * il * mx_sigmoid(gv[f].z)),
                           (half_t)(a[3] * il * mx_sigmoid(gv[f].w))};
        *(half4_t*)(act16 + orow + d) = o;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

#ifndef FA_DMA
#define FA_DMA 1  // LDS-copy attention (k_fa_attn_d) for head dims of 128 and 256
#endif
#ifndef FA_D_NW
#define FA_D_NW 4
#endif
#ifndef FA_D_QS
#define FA_D_QS 2
#endif

#ifndef FA_H_NW
#define FA_H_NW 8  // waves per block of the fp16 attention
#endif
#ifndef FA_H_QS
// Sets of 16 queries per wave of the fp16 attention.  Two sets read each K / V^T fragment
// from LDS once for two MFMAs, but their registers (256 VGPRs + 206 AGPRs) allow one wave
// per SIMD: with 4-wave blocks the Qwen3-Next 4096-token attention took 330 us against
// 250 us for one set in 8-wave blocks (2 waves per SIMD, 194 VGPRs).
#define FA_H_QS 1
#endif

template <int NC>
int launch_attn_h(const float* qg, const float* kk, const float* vv, const FaDims& m, int T,
                  half_t* k16, half_t* v16t, void* act, hipStream_t s) {
  const int Tp = (T + FA_TPAD - 1) / FA_TPAD * FA_TPAD, DP = NC * 32;
  const long pieces = (long)m.nkv * Tp * (DP / 8);
  mx_clear_error();
  hipLaunchKernelGGL(k_fa_pack_kv, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, s, kk,
                     vv, m, T, Tp, DP, k16, v16t);
  MX_TRY(mx_launch_status());
  const float sqrt_hd = (float)sqrt((double)m.hd);
  if constexpr (FA_DMA && NC >= 4) {
    const dim3 grid(mx_ceil_div(T, 16 * FA_D_QS * FA_D_NW), m.nh);
    hipLaunchKernelGGL((k_fa_attn_d<NC, FA_D_NW, FA_D_QS>), grid, dim3(64 * FA_D_NW), 0, s, qg,
                       k16, v16t, m, T, Tp, sqrt_hd, (half_t*)act);
    return mx_launch_status();
  }
  const dim3 grid(mx_ceil_div(T, 16 * FA_H_QS * FA_H_NW), m.nh);
  hipLaunchKernelGGL((k_fa_attn_h<NC, FA_H_NW, FA_H_S32, FA_H_QS>), grid, dim3(64 * FA_H_NW), 0, s, qg,
                     k16, v16t, m, T, Tp, sqrt_hd, (half_t*)act);
  return mx_launch_status();
}

template <int NC>
int launch_attn(const float* qg, const float* kk, const float* vv, const FaDims& m, int T,
                void* act, bool f16, hipStream_t s) {
  const dim3 grid(mx_ceil_div(T, 64), m.nh);
  const float sqrt_hd = (float)sqrt((double)m.hd);
  mx_clear_error();
  hipLaunchKernelGGL((k_fa_attn<NC>), grid, dim3(256), 0, s, qg, kk, vv, m, T, sqrt_hd,
                     f16 ? nullptr : (float*)act, f16 ? (half_t*)act : nullptr);
  return mx_launch_status();
}

int attn_launch(const float* qg, const float* kk, const float* vv, const FaDims& m, int T,
                void* act, bool f16, half_t* k16, half_t* v16t, hipStream_t s) {
  if (f16) {
    if (m.hd <= 32) return launch_attn_h<1>(qg, kk, vv, m, T, k16, v16t, act, s);
    if (m.hd <= 64) return launch_attn_h<2>(qg, kk, vv, m, T, k16, v16t, act, s);
    if (m.hd <= 128) return launch_attn_h<4>(qg, kk, vv, m, T, k16, v16t, act, s);
    if (m.hd <= 256) return launch_attn_h<8>(qg, kk, vv, m, T, k16, v16t, act, s);
    return MX_ERR_UNSUPPORTED;
  }
  if (m.hd <= 16) return launch_attn<1>(qg, kk, vv, m, T, act, f16, s);
  if (m.hd <= 32) return launch_attn<2>(qg, kk, vv, m, T, act, f16, s);
  if (m.hd <= 64) return launch_attn<4>(qg, kk, vv, m, T, act, f16, s);
  if (m.hd <= 128) return launch_attn<8>(qg, kk, vv, m, T, act, f16, s);
  if (m.hd <= 256) return launch_attn<16>(qg, kk, vv, m, T, act, f16, s);
  return MX_ERR_UNSUPPORTED;
}

__global__ __launch_bounds__(256) void k_fa_residual(const float* __restrict__ x,
                                                     const float* __restrict__ y, long n4,
                                                     float* __restrict__ out) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i < n4) {
    const float4 a = ((const float4*)x)[i], b = ((const float4*)y)[i];
    ((float4*)out)[i] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
  }
}

int check_weights(const MxFullAttnDesc* d, const MxFullAttnWeights* w) {
  if (!w || !w->norm_w || !w->q_w || !w->k_w || !w->v_w || !w->o_w) return MX_ERR_INVALID;
  if (d->weight_dtype == MX_DT_I8 && (!w->q_scale || !w->k_scale || !w->v_scale || !w->o_scale))
    return MX_ERR_INVALID;
  if (!mx_aligned16(w->q_w) || !mx_aligned16(w->k_w) || !mx_aligned16(w->v_w) ||
      !mx_aligned16(w->o_w))
    return MX_ERR_ALIGNMENT;
  return MX_OK;
}

int run_stage(int st, const MxFullAttnDesc* d, const MxFullAttnWeights* w, const float* x,
              float* out, int T, const FaWork& k, hipStream_t s) {
  const FaDims m = dims_of(d);
  const int wdt = d->weight_dtype;
  const bool f32 = wdt == MX_DT_F32;
  const void* h = f32 ? (const void*)k.v.h32 : k.v.h16;
  switch (st) {
    case 0: {
      MxDenseEntries e = {};
      e.e[0].down = w->q_w;
      e.e[0].down_scale = w->q_scale;
      e.e[1].down = w->k_w;
      e.e[1].down_scale = w->k_scale;
      e.e[2].down = w->v_w;
      e.e[2].down_scale = w->v_scale;
      e.e[3].down = w->o_w;
      e.e[3].down_scale = w->o_scale;
      MX_TRY(mx_dense_setup(k.dw, e, T, s));
      return mx_rmsnorm_launch(x, w->norm_w, d->param_dtype, d->eps, T, m.H, k.v.h32, k.v.h16,
                               s);
    }
    case 1:
      if (mx_dense_on_gemm(wdt, T, m.H)) {  // q, k and v share h: one GEMM launch
        const MxGemmSeg g[3] = {{w->q_w, k.v.qg, m.qw, m.qw},
                                {w->k_w, k.v.k, m.kw, m.kw},
                                {w->v_w, k.v.v, m.kw, m.kw}};
        return mx_gemm_f16(h, T, m.H, g, 3, s);
      }
      return mx_project(k.dw, 0, wdt, w->q_w, T, m.qw, m.H, h, k.v.qg, s);
    case 2:
      if (mx_dense_on_gemm(wdt, T, m.H)) return MX_OK;  // with q in stage 1
      return mx_project(k.dw, 1, wdt, w->k_w, T, m.kw, m.H, h, k.v.k, s);
    case 3:
      if (mx_dense_on_gemm(wdt, T, m.H)) return MX_OK;
      return mx_project(k.dw, 2, wdt, w->v_w, T, m.kw, m.H, h, k.v.v, s);
    case 4: {
      // Long inputs: one block per token (4096 tokens: 34 us against 41 us with 4 rows per
      // block); short ones: 4 rows per block (one token: 6.8 us against 11.7 us).
      const int rows = m.nh + m.nkv, rpb = T >= 1024 ? rows : 4;
      const dim3 grid(T, mx_ceil_div(rows, rpb));
      mx_clear_error();
      if (m.hd <= 64)
        hipLaunchKernelGGL(k_fa_rope_tok<1>, grid, dim3(256), 0, s, k.v.qg, k.v.k, w->q_norm_w,
                           w->k_norm_w, d->param_dtype, m, d->rope_theta, d->eps, rpb);
      else if (m.hd <= 128)
        hipLaunchKernelGGL(k_fa_rope_tok<2>, grid, dim3(256), 0, s, k.v.qg, k.v.k, w->q_norm_w,
                           w->k_norm_w, d->param_dtype, m, d->rope_theta, d->eps, rpb);
      else
        hipLaunchKernelGGL(k_fa_rope_tok<4>, grid, dim3(256), 0, s, k.v.qg, k.v.k, w->q_norm_w,
                           w->k_norm_w, d->param_dtype, m, d->rope_theta, d->eps, rpb);
      return mx_launch_status();
    }
    case 5:
      return attn_launch(k.v.qg, k.v.k, k.v.v, m, T, k.v.act, !f32, k.k16, k.v16t, s);
    case 6:
      if (mx_dense_on_gemm(wdt, T, m.od)) {  // out = x + act W_o^T in the GEMM epilogue
        if (!x || !out) return MX_ERR_INVALID;
        const MxGemmSeg g{w->o_w, out, m.H, m.H, nullptr, x};
        return mx_gemm_f16(k.v.act, T, m.od, &g, 1, s);
      }
      return mx_project(k.dw, 3, wdt, w->o_w, T, m.H, m.od, k.v.act, k.v.y, s);
    case 7: {
      if (mx_dense_on_gemm(wdt, T, m.od)) return MX_OK;  // added in stage 6
      const long n4 = (long)T * m.H / 4;
      mx_clear_error();
      hipLaunchKernelGGL(k_fa_residual, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, x,
                         k.v.y, n4, out);
      return mx_launch_status();
    }
    default:
      return MX_ERR_INVALID;
  }
}

int forward(const MxFullAttnDesc* d, const MxFullAttnWeights* w, const float* x, float* out,
            int T, void* ws, size_t ws_bytes, hipStream_t s, void* const* events) {
  MX_TRY(check_desc(d));
  MX_TRY(check_weights(d, w));
  if (!x || !out || !ws || T < 0) return MX_ERR_INVALID;
  if (d->hidden % 4) return MX_ERR_UNSUPPORTED;  // float4 residual
  if (!mx_aligned16(x) || !mx_aligned16(out)) return MX_ERR_ALIGNMENT;
  if (T == 0) return MX_OK;
  FaWork k;
  size_t need = 0;
  MX_TRY(layout(d, T, ws, &k, &need));
  if (ws_bytes < need) return MX_ERR_WORKSPACE;
  for (int st = 0; st < MX_FA_N_STAGES; ++st) {
    if (events) MX_TRY(mx_status(hipEventRecord((hipEvent_t)events[st], s)));
    MX_TRY(run_stage(st, d, w, x, out, T, k, s));
  }
  if (events) MX_TRY(mx_status(hipEventRecord((hipEvent_t)events[MX_FA_N_STAGES], s)));
  return MX_OK;
}

}  // namespace

extern "C" int mx_full_attn_workspace_size(const MxFullAttnDesc* desc, int32_t tokens,
                                           size_t* nbytes) {
  if (!nbytes) return MX_ERR_INVALID;
  return layout(desc, tokens, nullptr, nullptr, nbytes);
}

extern "C" int mx_full_attn_views(const MxFullAttnDesc* desc, int32_t tokens, void* workspace,
                                  MxFullAttnViews* views) {
  if (!workspace || !views) return MX_ERR_INVALID;
  FaWork k;
  MX_TRY(layout(desc, tokens, workspace, &k, nullptr));
  *views = k.v;
  return MX_OK;
}

extern "C" int mx_full_attn_forward(const MxFullAttnDesc* desc, const MxFullAttnWeights* weights,
                                    const float* x, float* out, int32_t tokens, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  return forward(desc, weights, x, out, tokens, workspace, workspace_bytes, (hipStream_t)stream,
                 nullptr);
}

extern "C" int mx_full_attn_forward_profiled(const MxFullAttnDesc* desc,
                                             const MxFullAttnWeights* weights, const float* x,
                                             float* out, int32_t tokens, void* workspace,
                                             size_t workspace_bytes, void* stream,
                                             void* const* events, int32_t n_events) {
  if (!events || n_events != MX_FA_N_STAGES + 1) return MX_ERR_INVALID;
  for (int i = 0; i < n_events; ++i)
    if (!events[i]) return MX_ERR_INVALID;
  return forward(desc, weights, x, out, tokens, workspace, workspace_bytes, (hipStream_t)stream,
                 events);
}
