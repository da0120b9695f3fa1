// Grouped SwiGLU expert products on MFMA (gfx950).
//
// Reference: offload_runtime/executors/glm4_moe.py:215-224 (routed experts),
// :234-237 (shared expert) and qwen3_next.py:305-313, :322-324, with linear_t = x @ W.T
// (_common.py:101-103) and silu = x / (1 + exp(-x)) (_common.py:83-84).
//
// Work decomposition.  The dispatch kernel cuts every group (one expert's rows in the
// expert-sorted order) into m-tiles of m_blk = 16*MT rows.  Block (x, y) takes m-tile x
// and four consecutive 16*NBI-column slabs of the output, one per wave.  Each wave owns
// its output columns outright, so waves never synchronise and no LDS is used: every
// weight row is streamed from HBM exactly once per m-tile with 16-byte buffer loads
// (out-of-range lanes read zero through the buffer descriptor's bounds check) and fed
// straight into MFMA B-operand registers.
//
// Fragment layout (16x16 output tile, lane = 16*q + j):
//   B operand: lane holds EPL consecutive elements of weight row n0+j at column
//              chunk*KC + q*EPL  (16 bytes of the row);
//   A operand: lane holds the same EPL columns of activation row m0+j;
//   C:         lane holds C[4*q + r][j], r = 0..3.
// A and B use the same (q, element) -> column assignment, so each MFMA sums every column
// of its chunk exactly once whatever order the instruction reduces them in.
//   fp16 weights: EPL = 8,  one v_mfma_f32_16x16x32_f16 per chunk (A = fp16 activations)
//   int8 weights: EPL = 16, two v_mfma_f32_16x16x32_f16 per chunk after an exact
//                 int8 -> fp16 conversion; the per-row scale is applied in the epilogue
//   fp32 weights: EPL = 4,  four v_mfma_f32_16x16x4_f32 per chunk (A = fp32 activations)
#include "mx_common.h"
#include "mx_internal.h"

typedef __amdgpu_buffer_rsrc_t mx_rsrc_t;
#define MX_RSRC_DW3 0x00020000
#define MX_OOB 0x80000000u  // any offset >= this is outside every descriptor we build

__device__ __forceinline__ mx_rsrc_t mx_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, MX_RSRC_DW3);
}

__device__ __forceinline__ int4_t mx_ld16(mx_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

template <int WF>
struct WTr;
template <>
struct WTr<MX_DT_F16> {
  static constexpr int EPL = 8, ESZ = 2, AESZ = 2, AV = 1;
};
template <>
struct WTr<MX_DT_I8> {
  static constexpr int EPL = 16, ESZ = 1, AESZ = 2, AV = 2;
};
template <>
struct WTr<MX_DT_F32> {
  static constexpr int EPL = 4, ESZ = 4, AESZ = 4, AV = 1;
};

// 16 int8 -> 16 fp16, exact: byte u = q + 128 placed under exponent 0x64 reads as
// 1024 + u in fp16; subtracting 1152 leaves q.
__device__ __forceinline__ void mx_i8_to_f16(int4_t v, half8_t& lo, half8_t& hi) {
  const half2_t bias = {(half_t)1152.0f, (half_t)1152.0f};
  half2_t h[8];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t u = (uint32_t)v[d] ^ 0x80808080u;
    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    h[2 * d] = __builtin_bit_cast(half2_t, p0) - bias;
    h[2 * d + 1] = __builtin_bit_cast(half2_t, p1) - bias;
  }
  lo = (half8_t){h[0][0], h[0][1], h[1][0], h[1][1], h[2][0], h[2][1], h[3][0], h[3][1]};
  hi = (half8_t){h[4][0], h[4][1], h[5][0], h[5][1], h[6][0], h[6][1], h[7][0], h[7][1]};
}

struct ExpertParams {
  const MxExpertPtrs* experts;
  const int* g_expert;
  const int* g_start;
  const int* g_count;
  const int* mt_group;
  const int* mt_row0;
  const int* n_mtiles;
  const int* sorted_tok;  // gate/up: token of each sorted row (A rows are gathered)
  const void* a;          // activations: h (gate/up) or act (down)
  uint32_t a_bytes;
  int lda;                // elements per activation row
  void* out;              // act (gate/up) or y (down)
  int ldo;                // elements per output row
  const float* sorted_w;  // down: routing weight of each sorted row
  int E;
  int N_r, K_r;           // routed expert: output columns, reduction length
  int N_s, K_s;           // shared expert
};

template <int WF, int MT, int NBI, bool GU, int UK>
__global__ __launch_bounds__(256) void k_expert(const ExpertParams p) {
  using Tr = WTr<WF>;
  constexpr int EPL = Tr::EPL, ESZ = Tr::ESZ, AESZ = Tr::AESZ, AV = Tr::AV;
  constexpr int KC = 4 * EPL;          // reduction columns per chunk (per wave)
  constexpr int NF = GU ? 2 * NBI : NBI;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int mt = blockIdx.x;
  if (mt >= *p.n_mtiles) return;
  const int g = p.mt_group[mt];
  const int row0 = p.mt_row0[mt];
  const int eid = p.g_expert[g];
  const int gstart = p.g_start[g];
  const int gcount = p.g_count[g];
  const bool sh = eid == p.E;
  const int N = sh ? p.N_s : p.N_r;
  const int K = sh ? p.K_s : p.K_r;
  const int n0 = (blockIdx.y * 4 + wave) * 16 * NBI;
  if (n0 >= N) return;
  const int mrows = min(16 * MT, gcount - row0);
  const int j = lane & 15, q = lane >> 4;
  const MxExpertPtrs ep = p.experts[eid];

  const uint32_t rowb = (uint32_t)K * ESZ;
  const uint32_t matb = (uint32_t)N * rowb;
  const mx_rsrc_t rb0 = mx_rsrc(GU ? ep.gate : ep.down, matb);
  const mx_rsrc_t rb1 = mx_rsrc(GU ? ep.up : ep.down, matb);
  uint32_t boff[NBI];
#pragma unroll
  for (int f = 0; f < NBI; ++f) {
    const int n = n0 + 16 * f + j;
    boff[f] = n < N ? (uint32_t)n * rowb + q * EPL * ESZ : MX_OOB;
  }
  const mx_rsrc_t ra = mx_rsrc(p.a, p.a_bytes);
  uint32_t aoff[MT];
#pragma unroll
  for (int mi = 0; mi < MT; ++mi) {
    const int m = 16 * mi + j;
    if (m < mrows) {
      const int r = gstart + row0 + m;
      const int arow = GU ? p.sorted_tok[r] : r;
      aoff[mi] = (uint32_t)arow * (uint32_t)p.lda * AESZ + q * EPL * AESZ;
    } else {
      aoff[mi] = MX_OOB;
    }
  }

  float4_t acc[MT][NF];
#pragma unroll
  for (int mi = 0; mi < MT; ++mi)
#pragma unroll
    for (int f = 0; f < NF; ++f) acc[mi][f] = (float4_t){0.f, 0.f, 0.f, 0.f};

  // One chunk of loads.  kin = false turns the lane's loads into zero reads (K tail).
  auto load_chunk = [&](int c, bool kin, int4_t (&b)[NF], int4_t (&a)[MT][AV]) {
    const uint32_t kb = (uint32_t)c * KC * ESZ;
    const uint32_t ka = (uint32_t)c * KC * AESZ;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int fi = GU ? (f % NBI) : f;
      const uint32_t o = kin ? boff[fi] + kb : MX_OOB;
      b[f] = mx_ld16((GU && f >= NBI) ? rb1 : rb0, o);
    }
#pragma unroll
    for (int mi = 0; mi < MT; ++mi)
#pragma unroll
      for (int v = 0; v < AV; ++v) a[mi][v] = mx_ld16(ra, kin ? aoff[mi] + ka + 16 * v : MX_OOB);
  };
  auto mma_chunk = [&](const int4_t (&b)[NF], const int4_t (&a)[MT][AV]) {
    if constexpr (WF == MX_DT_F16) {
#pragma unroll
      for (int mi = 0; mi < MT; ++mi)
#pragma unroll
        for (int f = 0; f < NF; ++f)
          acc[mi][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              __builtin_bit_cast(half8_t, a[mi][0]), __builtin_bit_cast(half8_t, b[f]),
              acc[mi][f], 0, 0, 0);
    } else if constexpr (WF == MX_DT_I8) {
      half8_t blo[NF], bhi[NF];
#pragma unroll
      for (int f = 0; f < NF; ++f) mx_i8_to_f16(b[f], blo[f], bhi[f]);
#pragma unroll
      for (int mi = 0; mi < MT; ++mi)
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          acc[mi][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              __builtin_bit_cast(half8_t, a[mi][0]), blo[f], acc[mi][f], 0, 0, 0);
          acc[mi][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              __builtin_bit_cast(half8_t, a[mi][1]), bhi[f], acc[mi][f], 0, 0, 0);
        }
    } else {
#pragma unroll
      for (int mi = 0; mi < MT; ++mi) {
        const float4_t av = __builtin_bit_cast(float4_t, a[mi][0]);
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          const float4_t bv = __builtin_bit_cast(float4_t, b[f]);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            acc[mi][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], bv[e], acc[mi][f], 0, 0, 0);
        }
      }
    }
  };

  // Full chunks in batches of UK, ping-ponging two register sets so the loads of batch
  // i+1 are in flight while batch i runs on the MFMA pipe.
  const int nfull = K / KC;
  const int nbatch = nfull / UK;
  int4_t bx[UK][NF], ax[UK][MT][AV], by[UK][NF], ay[UK][MT][AV];
  if (nbatch > 0) {
#pragma unroll
    for (int u = 0; u < UK; ++u) load_chunk(u, true, bx[u], ax[u]);
  }
  for (int bt = 0; bt < nbatch; bt += 2) {
    if (bt + 1 < nbatch) {
#pragma unroll
      for (int u = 0; u < UK; ++u) load_chunk((bt + 1) * UK + u, true, by[u], ay[u]);
    }
#pragma unroll
    for (int u = 0; u < UK; ++u) mma_chunk(bx[u], ax[u]);
    if (bt + 1 < nbatch) {
      if (bt + 2 < nbatch) {
#pragma unroll
        for (int u = 0; u < UK; ++u) load_chunk((bt + 2) * UK + u, true, bx[u], ax[u]);
      }
#pragma unroll
      for (int u = 0; u < UK; ++u) mma_chunk(by[u], ay[u]);
    }
  }
  // Remaining chunks (fewer than UK full ones, then a partial one).
  const int nchunks = (K + KC - 1) / KC;
  for (int c = nbatch * UK; c < nchunks; ++c) {
    const bool kin = c * KC + q * EPL < K;
    load_chunk(c, kin, bx[0], ax[0]);
    mma_chunk(bx[0], ax[0]);
  }

  // Epilogue.
  if constexpr (GU) {
#pragma unroll
    for (int f = 0; f < NBI; ++f) {
      const int n = n0 + 16 * f + j;
      if (n >= N) continue;
      float sg = 1.f, su = 1.f;
      if constexpr (WF == MX_DT_I8) {
        sg = (float)((const half_t*)ep.gate_scale)[n];
        su = (float)((const half_t*)ep.up_scale)[n];
      }
#pragma unroll
      for (int mi = 0; mi < MT; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * mi + 4 * q + r;
          if (m < mrows) {
            const float gv = acc[mi][f][r] * sg;
            const float uv = acc[mi][NBI + f][r] * su;
            const float av = mx_silu(gv) * uv;
            const size_t o = (size_t)(gstart + row0 + m) * p.ldo + n;
            if constexpr (WF == MX_DT_F32)
              ((float*)p.out)[o] = av;
            else
              ((half_t*)p.out)[o] = (half_t)av;
          }
        }
    }
  } else {
#pragma unroll
    for (int f = 0; f < NBI; ++f) {
      const int n = n0 + 16 * f + j;
      if (n >= N) continue;
      float sd = 1.f;
      if constexpr (WF == MX_DT_I8) sd = (float)((const half_t*)ep.down_scale)[n];
#pragma unroll
      for (int mi = 0; mi < MT; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * mi + 4 * q + r;
          if (m < mrows) {
            const int row = gstart + row0 + m;
            ((float*)p.out)[(size_t)row * p.ldo + n] = p.sorted_w[row] * (acc[mi][f][r] * sd);
          }
        }
    }
  }
}

// ------------------------------------------------------------------------------------
// Host side.
// ------------------------------------------------------------------------------------
int mx_m_blk_for(int tokens, int weight_dtype) {
  (void)weight_dtype;
  if (tokens <= 16) return 16;
  if (tokens <= 32) return 32;
  return 64;
}

static int expert_check(const MxMoeDesc* d) {
  if (!d) return MX_ERR_INVALID;
  if (d->hidden <= 0 || d->inter <= 0 || d->shared_inter < 0 || d->n_experts <= 0 ||
      d->top_k <= 0)
    return MX_ERR_INVALID;
  int epl;
  switch (d->weight_dtype) {
    case MX_DT_F32: epl = 4; break;
    case MX_DT_F16: epl = 8; break;
    case MX_DT_I8: epl = 16; break;
    default: return MX_ERR_INVALID;
  }
  // Each lane's 16-byte piece must sit inside one row.
  if (d->hidden % epl || d->inter % epl || d->shared_inter % epl) return MX_ERR_UNSUPPORTED;
  // Buffer descriptors address < 2 GiB per matrix.
  const int esz = d->weight_dtype == MX_DT_F32 ? 4 : (d->weight_dtype == MX_DT_F16 ? 2 : 1);
  const long mx = (long)d->hidden * (d->inter > d->shared_inter ? d->inter : d->shared_inter) * esz;
  if (mx >= (1l << 31)) return MX_ERR_UNSUPPORTED;
  return MX_OK;
}

template <int WF, int MT, bool GU>
static void launch_expert(const ExpertParams& p, dim3 grid, hipStream_t s) {
  constexpr int NBI = GU ? 1 : 2;
  constexpr int UK = (WF == MX_DT_I8) ? (MT >= 4 ? 1 : 2) : (MT >= 4 ? 2 : 4);
  mx_clear_error();
  hipLaunchKernelGGL((k_expert<WF, MT, NBI, GU, UK>), grid, dim3(256), 0, s, p);
}

template <bool GU>
static int dispatch_expert(int wdt, int mt, const ExpertParams& p, dim3 grid, hipStream_t s) {
#define MX_EXP_CASE(W)                                   \
  if (wdt == W) {                                        \
    if (mt == 1) launch_expert<W, 1, GU>(p, grid, s);    \
    else if (mt == 2) launch_expert<W, 2, GU>(p, grid, s); \
    else if (mt == 4) launch_expert<W, 4, GU>(p, grid, s); \
    else return MX_ERR_INVALID;                          \
    return mx_launch_status();                           \
  }
  MX_EXP_CASE(MX_DT_F16)
  MX_EXP_CASE(MX_DT_I8)
  MX_EXP_CASE(MX_DT_F32)
#undef MX_EXP_CASE
  return MX_ERR_INVALID;
}

static int mt_from_mblk(int m_blk) {
  return (m_blk == 16 || m_blk == 32 || m_blk == 64) ? m_blk / 16 : 0;
}

extern "C" int mx_expert_gate_up(const MxMoeDesc* desc, const MxExpertPtrs* experts,
                                 int32_t tokens, const void* a, const int32_t* sorted_tok,
                                 const int32_t* g_expert, const int32_t* g_start,
                                 const int32_t* g_count, const int32_t* mt_group,
                                 const int32_t* mt_row0, const int32_t* n_mtiles, int32_t m_blk,
                                 void* act, void* stream) {
  MX_TRY(expert_check(desc));
  if (!experts || !a || !sorted_tok || !g_expert || !g_start || !g_count || !mt_group ||
      !mt_row0 || !n_mtiles || !act || tokens < 0)
    return MX_ERR_INVALID;
  const int mt = mt_from_mblk(m_blk);
  if (!mt) return MX_ERR_INVALID;
  if (tokens == 0) return MX_OK;
  const int aesz = desc->weight_dtype == MX_DT_F32 ? 4 : 2;
  const long abytes = (long)tokens * desc->hidden * aesz;
  if (abytes >= (1l << 31)) return MX_ERR_UNSUPPORTED;
  if (!mx_aligned16(a) || !mx_aligned16(act)) return MX_ERR_ALIGNMENT;
  const int has_shared = desc->shared_inter > 0;
  ExpertParams p;
  p.experts = experts;
  p.g_expert = g_expert;
  p.g_start = g_start;
  p.g_count = g_count;
  p.mt_group = mt_group;
  p.mt_row0 = mt_row0;
  p.n_mtiles = n_mtiles;
  p.sorted_tok = sorted_tok;
  p.a = a;
  p.a_bytes = (uint32_t)abytes;
  p.lda = desc->hidden;
  p.out = act;
  p.ldo = desc->inter > desc->shared_inter ? desc->inter : desc->shared_inter;
  p.sorted_w = nullptr;
  p.E = desc->n_experts;
  p.N_r = desc->inter;
  p.K_r = desc->hidden;
  p.N_s = desc->shared_inter;
  p.K_s = desc->hidden;
  const int nmax = p.ldo;
  dim3 grid(mx_max_mtiles(tokens, desc->top_k, desc->n_experts, has_shared, m_blk),
            mx_ceil_div(nmax, 4 * 16 * 1));
  return dispatch_expert<true>(desc->weight_dtype, mt, p, grid, (hipStream_t)stream);
}

extern "C" int mx_expert_down(const MxMoeDesc* desc, const MxExpertPtrs* experts, int32_t tokens,
                              const void* act, const float* sorted_w, const int32_t* g_expert,
                              const int32_t* g_start, const int32_t* g_count,
                              const int32_t* mt_group, const int32_t* mt_row0,
                              const int32_t* n_mtiles, int32_t m_blk, float* y, void* stream) {
  MX_TRY(expert_check(desc));
  if (!experts || !act || !sorted_w || !g_expert || !g_start || !g_count || !mt_group ||
      !mt_row0 || !n_mtiles || !y || tokens < 0)
    return MX_ERR_INVALID;
  const int mt = mt_from_mblk(m_blk);
  if (!mt) return MX_ERR_INVALID;
  if (tokens == 0) return MX_OK;
  const int has_shared = desc->shared_inter > 0;
  const int aesz = desc->weight_dtype == MX_DT_F32 ? 4 : 2;
  const int lda = desc->inter > desc->shared_inter ? desc->inter : desc->shared_inter;
  const long rows = (long)tokens * desc->top_k + (has_shared ? tokens : 0);
  const long abytes = rows * lda * aesz;
  if (abytes >= (1l << 31)) return MX_ERR_UNSUPPORTED;
  if (!mx_aligned16(act) || !mx_aligned16(y)) return MX_ERR_ALIGNMENT;
  ExpertParams p;
  p.experts = experts;
  p.g_expert = g_expert;
  p.g_start = g_start;
  p.g_count = g_count;
  p.mt_group = mt_group;
  p.mt_row0 = mt_row0;
  p.n_mtiles = n_mtiles;
  p.sorted_tok = nullptr;
  p.a = act;
  p.a_bytes = (uint32_t)abytes;
  p.lda = lda;
  p.out = y;
  p.ldo = desc->hidden;
  p.sorted_w = sorted_w;
  p.E = desc->n_experts;
  p.N_r = desc->hidden;
  p.K_r = desc->inter;
  p.N_s = desc->hidden;
  p.K_s = desc->shared_inter;
  dim3 grid(mx_max_mtiles(tokens, desc->top_k, desc->n_experts, has_shared, m_blk),
            mx_ceil_div(desc->hidden, 4 * 16 * 2));
  return dispatch_expert<false>(desc->weight_dtype, mt, p, grid, (hipStream_t)stream);
}
