// Grouped SwiGLU expert products on MFMA (gfx950).
//
// Reference: offload_runtime/executors/glm4_moe.py:215-224 (routed experts),
// :234-237 (shared expert) and qwen3_next.py:305-313, :322-324, with linear_t = x @ W.T
// (_common.py:101-103) and silu = x / (1 + exp(-x)) (_common.py:83-84).
//
// Work decomposition.  The dispatch kernel cuts every group (one expert's rows in the
// expert-sorted order) into m-tiles of m_blk = 16*MT rows.  Block (x, y) takes m-tile x
// and 4/KS consecutive 16*NBI-column slabs of the output; the KS waves of a slab split
// the reduction and add their partial tiles through LDS at the end (KS = 1: each wave
// owns its columns outright and no LDS is used).  Every weight row is streamed from HBM
// exactly once per m-tile with 16-byte buffer loads (out-of-range lanes read zero
// through the buffer descriptor's bounds check) and fed straight into MFMA B-operand
// registers.
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
#include "mx_route_dev.h"

typedef __amdgpu_buffer_rsrc_t mx_rsrc_t;
#define MX_RSRC_DW3 0x00020000
#define MX_OOB 0x80000000u  // any offset >= this is outside every descriptor we build

__device__ __forceinline__ mx_rsrc_t mx_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, MX_RSRC_DW3);
}

__device__ __forceinline__ int4_t mx_ld16(mx_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// Decode-kernel weight loads carry the nontemporal hint (cache-policy bit nt): at decode
// sizes every weight byte is read once, and a streaming read with nt sustains ~10 % more
// HBM bandwidth on MI355X than the default policy (6.75 vs 6.15 TB/s in a plain read
// probe; the decode block: 1.07 -> 0.96 ms).  The prefill kernel keeps the default
// policy: the sibling m-tiles of a hot expert re-read its weights and find part of them
// in L2 (with nt the 2048-token prefill slowed from 2.19 to 2.58 ms).
// (An exception for the int8 gate/up launch of single-m-frag tiles without a K split,
// default policy there, measured faster only while the timed steps re-read one layer's
// experts from the Infinity Cache; with distinct layers per step it is equal, and off.)
#ifndef MX_W_NT
#define MX_W_NT 1
#endif
#ifndef MX_W_AUX
#define MX_W_AUX 2  // cache-policy bits of the hinted loads (nt)
#endif
#ifndef MX_I8_GU_PLAIN
#define MX_I8_GU_PLAIN 0  // the int8 exception above (default policy) on or off
#endif
template <bool NT>
__device__ __forceinline__ int4_t mx_ldw16(mx_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, (MX_W_NT && NT) ? MX_W_AUX : 0);
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
  int tiled;              // weights in MX_LAYOUT_FRAG16 (else row-major)
  int y16 = 0;            // down, prefill kernel: y rows stored as fp16 (else fp32)
};

// One-token selection inside the gate/up launch (used in place of the top-k/dispatch
// launch when the batch is one token): every wave of every block selects the token's
// experts from the router logits itself, which costs less than the launch it replaces,
// and the first wave of block (0, 0) writes the selection and the dispatch tables that
// the down and combine launches (and the workspace views) read.
typedef MxOneTokenSelect SelectParams;

// Byte offset of the 16-byte piece lane (j, q) loads from fragment row block n16 (first
// row, a multiple of 16 for tiled weights) at chunk 0, and the byte step per chunk.
// Row-major: row n16 + j, column q * EPL.  MX_LAYOUT_FRAG16: 1 KiB fragment per
// (16 rows, KC columns), lane 16 q + j at byte 16 * (16 q + j).
template <int EPL, int ESZ>
__device__ __forceinline__ uint32_t mx_bfrag_base(bool tiled, int n16, int j, int q, int K) {
  constexpr int KC = 4 * EPL;
  return tiled ? (uint32_t)(n16 / 16) * (uint32_t)(K / KC) * 1024u + (uint32_t)(16 * q + j) * 16u
               : (uint32_t)(n16 + j) * (uint32_t)K * ESZ + (uint32_t)q * EPL * ESZ;
}

template <int WF, int MT, int NBI, bool GU, int UK, int KS, bool NT, int SELV>
__global__ __launch_bounds__(256) void k_expert(const ExpertParams p, const SelectParams sp) {
  constexpr bool SEL = SELV > 0;  // SELV: experts per lane of the in-launch selection
  using Tr = WTr<WF>;
  constexpr int EPL = Tr::EPL, ESZ = Tr::ESZ, AESZ = Tr::AESZ, AV = Tr::AV;
  constexpr int KC = 4 * EPL;          // reduction columns per chunk (per wave)
  constexpr int NF = GU ? 2 * NBI : NBI;
  constexpr int SPB = 4 / KS;          // column slabs per block; KS waves share a slab

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slab = wave / KS, ks = wave % KS;
  const int mt = blockIdx.x;
  int row0, eid, gstart, gcount;
  if constexpr (SEL) {
    // One token: tile 0 is the shared expert (when there is one), tile S0 + r the r-th
    // chosen expert in ascending id; each is a group of the token's single row.
    static_assert(GU && MT == 1, "selection runs in the one-token gate/up launch");
    MxSel sel;
    if constexpr (SELV <= 4) {
      sel = mx_topk_select<SELV>(sp.logits, 1, 1, 0, sp.bias, sp.pdt, p.E, sp.E1, sp.k, sp.mode,
                                 sp.norm, sp.scaling);
    } else {
      // Many experts: the block's 4 waves each keep the k best of 64 * SELV / 4 experts,
      // then every wave selects from the 4k candidates (the top-k kernel's small-batch
      // scheme; Qwen3-Next, 512 experts, one token: 29.9 -> 27.9 us per block against one
      // wave selecting from all 512).  Up to 256 experts one wave is as fast.
      __shared__ MxTopkPar par;
      mx_topk_par_cand<SELV / 4>(par, sp.logits, sp.bias, sp.pdt, p.E, sp.E1, sp.k, sp.mode, 4,
                                 wave);
      __syncthreads();
      sel = mx_topk_par_select<2>(par, 0, sp.k, sp.mode, sp.norm, sp.scaling, 4);
    }
    if (blockIdx.x == 0 && blockIdx.y == 0 && wave == 0) {
      const float gsh = mx_shared_gate(sp.logits, 1, 1, 0, p.E, sp.E1, sp.has_seg);
      if (lane < sp.k) {
        sp.ids[lane] = sel.id;
        sp.tw[lane] = sel.w;
      }
      if (lane == 0 && sp.shared_w) sp.shared_w[0] = gsh;
      mx_dispatch_one_token(sel.id, sel.w, sp.shared_w ? gsh : 1.f, sp.k, p.E, sp.has_shared,
                            sp.counts, sp.offsets, sp.sorted_tok, sp.sorted_w, sp.pair_pos,
                            sp.g_expert, sp.g_start, sp.g_count, sp.n_groups, sp.mt_group,
                            sp.mt_row0, sp.n_mtiles);
    }
    const int S0 = sp.has_shared;
    if (mt >= sp.k + S0) return;
    if (mt < S0) {
      eid = p.E;
      gstart = sp.k;
    } else {
      const int id = lane < sp.k ? sel.id : 0x7fffffff;
      int rank = 0;
      for (int i = 0; i < sp.k; ++i) rank += __builtin_amdgcn_readlane(id, i) < id ? 1 : 0;
      const unsigned long long hit = __ballot(lane < sp.k && rank == mt - S0);
      eid = __builtin_amdgcn_readlane(id, __builtin_ctzll(hit));
      gstart = mt - S0;
    }
    row0 = 0;
    gcount = 1;
  } else {
    if (mt >= *p.n_mtiles) return;
    const int g = p.mt_group[mt];
    row0 = p.mt_row0[mt];
    eid = p.g_expert[g];
    gstart = p.g_start[g];
    gcount = p.g_count[g];
  }
  const bool sh = eid == p.E;
  const int N = sh ? p.N_s : p.N_r;
  const int K = sh ? p.K_s : p.K_r;
  if ((int)blockIdx.y * SPB * 16 * NBI >= N) return;  // whole block past this expert
  const int n0 = (blockIdx.y * SPB + slab) * 16 * NBI;
  const bool wact = n0 < N;  // a wave without columns computes zeros and stores nothing
  const int mrows = min(16 * MT, gcount - row0);
  const int j = lane & 15, q = lane >> 4;
  const MxExpertPtrs ep = p.experts[eid];

  const uint32_t rowb = (uint32_t)K * ESZ;
  const uint32_t matb = (uint32_t)N * rowb;
  const mx_rsrc_t rb0 = mx_rsrc(GU ? ep.gate : ep.down, matb);
  const mx_rsrc_t rb1 = mx_rsrc(GU ? ep.up : ep.down, matb);
  const uint32_t bstep = p.tiled ? 1024u : (uint32_t)KC * ESZ;  // bytes per K chunk
  uint32_t boff[NBI];
#pragma unroll
  for (int f = 0; f < NBI; ++f) {
    const int n = n0 + 16 * f + j;
    boff[f] = n < N ? mx_bfrag_base<EPL, ESZ>(p.tiled, n0 + 16 * f, j, q, K) : MX_OOB;
  }
  const mx_rsrc_t ra = mx_rsrc(p.a, p.a_bytes);
  uint32_t aoff[MT];
#pragma unroll
  for (int mi = 0; mi < MT; ++mi) {
    const int m = 16 * mi + j;
    if (m < mrows) {
      const int r = gstart + row0 + m;
      const int arow = SEL ? 0 : (GU ? p.sorted_tok[r] : r);
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

  // This wave's chunks: [cb, ce) of the ceil(K / KC) chunks (K split KS ways in the block).
  const int nchunks = (K + KC - 1) / KC;
  const int cps = (nchunks + KS - 1) / KS;
  const int cb = min(nchunks, ks * cps), ce = min(nchunks, cb + cps);

  // One chunk of loads.  kin = false turns the lane's loads into zero reads (K tail).
  auto load_chunk = [&](int c, bool kin, int4_t (&b)[NF], int4_t (&a)[MT][AV]) {
    const uint32_t kb = (uint32_t)c * bstep;
    const uint32_t ka = (uint32_t)c * KC * AESZ;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int fi = GU ? (f % NBI) : f;
      const uint32_t o = kin ? boff[fi] + kb : MX_OOB;
      b[f] = mx_ldw16<NT>((GU && f >= NBI) ? rb1 : rb0, o);
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
  const int nfull = max(0, min(ce, K / KC) - cb);
  const int nbatch = nfull / UK;
  int4_t bx[UK][NF], ax[UK][MT][AV], by[UK][NF], ay[UK][MT][AV];
  if (nbatch > 0) {
#pragma unroll
    for (int u = 0; u < UK; ++u) load_chunk(cb + u, true, bx[u], ax[u]);
  }
  for (int bt = 0; bt < nbatch; bt += 2) {
    if (bt + 1 < nbatch) {
#pragma unroll
      for (int u = 0; u < UK; ++u) load_chunk(cb + (bt + 1) * UK + u, true, by[u], ay[u]);
    }
#pragma unroll
    for (int u = 0; u < UK; ++u) mma_chunk(bx[u], ax[u]);
    if (bt + 1 < nbatch) {
      if (bt + 2 < nbatch) {
#pragma unroll
        for (int u = 0; u < UK; ++u) load_chunk(cb + (bt + 2) * UK + u, true, bx[u], ax[u]);
      }
#pragma unroll
      for (int u = 0; u < UK; ++u) mma_chunk(by[u], ay[u]);
    }
  }
  // Remaining chunks of the range (fewer than UK full ones, then a partial one).
  for (int c = cb + nbatch * UK; c < ce; ++c) {
    const bool kin = c * KC + q * EPL < K;
    load_chunk(c, kin, bx[0], ax[0]);
    mma_chunk(bx[0], ax[0]);
  }

  // K split: the waves of a slab add their partial tiles in a fixed order.
  if constexpr (KS > 1) {
    __shared__ float4_t red[4][MT * NF][64];
    if (ks > 0) {
#pragma unroll
      for (int mi = 0; mi < MT; ++mi)
#pragma unroll
        for (int f = 0; f < NF; ++f) red[wave][mi * NF + f][lane] = acc[mi][f];
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int s2 = 1; s2 < KS; ++s2)
#pragma unroll
      for (int mi = 0; mi < MT; ++mi)
#pragma unroll
        for (int f = 0; f < NF; ++f) acc[mi][f] += red[wave + s2][mi * NF + f][lane];
  }
  if (!wact) return;

  // Epilogue.  Scales and routing weights are loaded first, at clamped indices, so the
  // loads are in flight together rather than one per predicated store.
  if constexpr (GU) {
    float sg[NBI], su[NBI];
#pragma unroll
    for (int f = 0; f < NBI; ++f) {
      sg[f] = 1.f;
      su[f] = 1.f;
      if constexpr (WF == MX_DT_I8) {
        const int n = min(n0 + 16 * f + j, N - 1);
        sg[f] = (float)((const half_t*)ep.gate_scale)[n];
        su[f] = (float)((const half_t*)ep.up_scale)[n];
      }
    }
#pragma unroll
    for (int f = 0; f < NBI; ++f) {
      const int n = n0 + 16 * f + j;
      if (n >= N) continue;
#pragma unroll
      for (int mi = 0; mi < MT; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * mi + 4 * q + r;
          if (m < mrows) {
            const float gv = acc[mi][f][r] * sg[f];
            const float uv = acc[mi][NBI + f][r] * su[f];
            const float av = mx_silu(gv) * uv;
            const size_t o = (size_t)(gstart + row0 + m) * p.ldo + n;
            if constexpr (WF == MX_DT_F32)
              ((float*)p.out)[o] = av;
            else
              ((half_t*)p.out)[o] = mx_f16_sat(av);
          }
        }
    }
  } else {
    float sd[NBI], wr[MT][4];
#pragma unroll
    for (int f = 0; f < NBI; ++f) {
      sd[f] = 1.f;
      if constexpr (WF == MX_DT_I8)
        sd[f] = (float)((const half_t*)ep.down_scale)[min(n0 + 16 * f + j, N - 1)];
    }
#pragma unroll
    for (int mi = 0; mi < MT; ++mi)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        wr[mi][r] = p.sorted_w[gstart + row0 + min(16 * mi + 4 * q + r, mrows - 1)];
#pragma unroll
    for (int f = 0; f < NBI; ++f) {
      const int n = n0 + 16 * f + j;
      if (n >= N) continue;
#pragma unroll
      for (int mi = 0; mi < MT; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * mi + 4 * q + r;
          if (m < mrows) {
            const int row = gstart + row0 + m;
            ((float*)p.out)[(size_t)row * p.ldo + n] = wr[mi][r] * (acc[mi][f][r] * sd[f]);
          }
        }
    }
  }
}

// ------------------------------------------------------------------------------------
// Prefill regime (m-tiles of 128 rows, fp16 / int8 weights).
//
// With many rows per expert the activation tile is reused by every column slab, so it is
// staged once per block in LDS (double-buffered, rows padded by 16 bytes so the 16-byte
// fragment reads of 8 consecutive lanes hit distinct banks) and shared by the block's 4
// waves (8 for fp16 reductions of 1024-3072 columns, see lds_eight_waves).
// Weights go straight from HBM into MFMA B registers; each wave holds 4 B fragments per
// k-chunk (gate/up: 2 gate + 2 up column blocks; down: 4 column blocks), so every A
// fragment read from LDS feeds 4 MFMAs, and each wave owns a 128-row x 4-fragment tile.
//
// Block order: hardware block b runs on XCD b % 8; the blocks of the actual m-tiles x column
// slabs are dealt to the 8 XCDs in equal contiguous runs, and inside a run a group's blocks
// come together (slabs outer, its m-tiles inner), so the sibling m-tiles of a hot expert
// read each weight slab at about the same time through their XCD's L2 and a single-tile
// group's activation rows are staged from L2 for every slab after the first (see
// k_expert_lds).  (256-row tiles, through wave pairs exchanging weight fragments in LDS,
// measured slower on MI355X: they stage as many activation bytes as weight bytes and
// cannot share a launch with the 128-row tiles without spilling.)
// ------------------------------------------------------------------------------------
// Tunables (compile-time; the defaults are the measured best on MI355X).
//   MX_LDS_RB:      weight stages in flight per wave (even).
//   MX_LDS_RA:      activation stages in flight (even, divides RB).
//   MX_LDS_KM_F16:  MFMA k-steps per stage for fp16 (each weight fragment row is read
//                   KM * 64 contiguous bytes per stage).
#ifndef MX_LDS_RB
#define MX_LDS_RB 4
#endif
// Nontemporal hint on the prefill kernel's weight loads of multi-tile groups, per
// projection; both off.  The sibling m-tiles of hot experts share weight lines through L2
// (GLM-4.7 Zipf prefill with nt for every block: gate/up 1.117 -> 1.336 ms).
#ifndef MX_LDS_NT_GU
#define MX_LDS_NT_GU 0
#endif
#ifndef MX_LDS_NT_DN
#define MX_LDS_NT_DN 0
#endif
// Nontemporal weight loads for the blocks of single-tile groups (no sibling tile reads
// their weights): a uniform branch per block between two copies of the tile body, no
// spills (250-252 VGPRs).  Same box, interleaved: Qwen3-Next 4096 tokens gate/up 497 ->
// 479 us, down 341 -> 335 us; GLM-4.7 2048-token Zipf prefill gate/up 1117 -> 1085 us,
// down 684 -> 639 us.
// Block order inside an XCD run: 0 slab-major (a column slab's m-tiles in a row), 1 tile-
// major (an m-tile's column slabs in a row), 2 expert-major (a group's blocks in a row,
// slabs outer, its m-tiles inner: single-tile groups reuse their staged activation rows
// across slabs through L2, sibling m-tiles of a hot expert read each weight slab
// together).  Same box, interleaved, order 0 / 1 / 2: Qwen3-Next 4096 tokens 978 / 954 /
// 957 us, GLM-4.7 Zipf prefill 1830 / 1865 / 1807 us.
#ifndef MX_LDS_ORDER
#define MX_LDS_ORDER 2
#endif
#ifndef MX_LDS_XCD_REAL
#define MX_LDS_XCD_REAL 1  // XCD runs over the actual m-tiles (else over the mt_max bound)
#endif
#ifndef MX_LDS_NT_SINGLE
#define MX_LDS_NT_SINGLE 1
#endif
#ifndef MX_LDS_RA
#define MX_LDS_RA 4
#endif
#ifndef MX_LDS_KM_F16
#define MX_LDS_KM_F16 2
#endif
#ifndef MX_LDS_RB_KM2
#define MX_LDS_RB_KM2 2
#endif

#ifndef MX_LDS_OCC_F16
#define MX_LDS_OCC_F16 2  // 4-wave fp16 blocks per CU
#endif
#ifndef MX_LDS_APAD
// Padding of a staged activation row (bytes).  With 32 the MFMA operand reads (lane (j, q):
// row j, 16-byte chunk q) and the staging stores run without bank-conflict cycles on gfx950;
// with 16 the reads take twice the LDS cycles.
#define MX_LDS_APAD 32
#endif
#ifndef MX_LDS_8W
#define MX_LDS_8W 1  // 8-wave fp16 blocks where lds_eight_waves picks them
#endif
template <int WF>
struct LdsShape {
  // fp16 fits two 4-wave blocks per CU; the int8 variant (conversion temporaries, 64-
  // column stages) needs the full register file of one block per CU to avoid spills.
  static constexpr int OCC = WF == MX_DT_F16 ? MX_LDS_OCC_F16 : 1;
  // MFMA k-steps per stage: each weight row is read KM * 64 contiguous bytes per stage.
  static constexpr int KM = WF == MX_DT_F16 ? MX_LDS_KM_F16 : 1;
};

// One block's work: MB = 16 * MTX rows (from `base` of group g) x NW waves of 16 * NBIX
// columns (x 2 for gate and up) starting at column n0b; with CH > 1 (down projection), the
// `items` consecutive column slabs of NW * 16 * NBIX columns from n0b one after the other,
// the next slab's first weights and activations loaded while the last stage of the
// previous one computes, and its epilogue run with those loads in flight (the tile's
// routing weights come from LDS, `wrow`, so the epilogue issues no global load that would
// wait for them).
template <int WF, bool GU, int MTX, int NBIX, int NW, bool NT, int CH = 1, bool Y16 = false>
__device__ __forceinline__ void expert_lds_tile(const ExpertParams& p, char* lds, int g,
                                                int base, int trows, int n0b, int items = 1,
                                                const float* wrow = nullptr) {
  static_assert(CH == 1 || (!GU && WF == MX_DT_F16), "slab chains: fp16 down projection");
  static_assert(!(GU && Y16), "fp16 y rows: down projection");
  using Tr = WTr<WF>;
  constexpr int EPL = Tr::EPL, ESZ = Tr::ESZ;
  constexpr int KM = LdsShape<WF>::KM;
  constexpr int KS = 4 * EPL * KM;           // reduction columns per stage
  constexpr int MB = 16 * MTX;
  constexpr int NF = GU ? 2 * NBIX : NBIX;
  constexpr int AROW = KS * 2 + MX_LDS_APAD;  // LDS bytes per staged activation row
  constexpr int ATILE = MB * AROW;
  constexpr int CPR = KS * 2 / 16;           // 16-byte chunks per row and stage
  constexpr int ACH = MB * CPR / (64 * NW);  // chunks each thread stages
  constexpr int RB = KM == 1 ? MX_LDS_RB : MX_LDS_RB_KM2;  // weight stages in flight
  constexpr int RA = (WF == MX_DT_F16 && GU && KM == 1) ? MX_LDS_RA : 2;  // activation stages
  static_assert(RB % RA == 0 && RA % 2 == 0, "ring sizes must divide the unroll");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int eid = p.g_expert[g];
  const int gstart = p.g_start[g];
  const bool sh = eid == p.E;
  const int N = sh ? p.N_s : p.N_r;
  const int K = sh ? p.K_s : p.K_r;
  const int n0 = n0b + wave * 16 * NBIX;
  const bool wact = n0 < N;
  const int j = lane & 15, q = lane >> 4;
  const MxExpertPtrs ep = p.experts[eid];

  const uint32_t rowb = (uint32_t)K * ESZ;
  const uint32_t matb = (uint32_t)N * rowb;
  const mx_rsrc_t rb0 = mx_rsrc(GU ? ep.gate : ep.down, matb);
  const mx_rsrc_t rb1 = mx_rsrc(GU ? ep.up : ep.down, matb);
  const uint32_t bstep = p.tiled ? 1024u : (uint32_t)4 * EPL * ESZ;  // bytes per K chunk
  uint32_t boff[NBIX];
#pragma unroll
  for (int f = 0; f < NBIX; ++f) {
    const int n = n0 + 16 * f + j;
    boff[f] = (wact && n < N) ? mx_bfrag_base<EPL, ESZ>(p.tiled, n0 + 16 * f, j, q, K)
                              : MX_OOB;
  }
  // Slab chains: weight bytes from one slab to the next (the fragment base is linear in
  // the first column of a 16-row block).
  constexpr int SLABW = NW * 16 * NBIX;
  const uint32_t dslab = p.tiled ? (uint32_t)(SLABW / 16) * (uint32_t)(K / (4 * EPL)) * 1024u
                                 : (uint32_t)SLABW * rowb;

  // Activation chunks this thread stages: fixed rows of the tile, advancing columns.
  const mx_rsrc_t ra = mx_rsrc(p.a, p.a_bytes);
  uint32_t agoff[ACH];
  int alds[ACH], acol[ACH];
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int c = tid + 64 * NW * i;
    const int row = c / CPR, cc = c % CPR;
    acol[i] = cc * 8;
    alds[i] = row * AROW + cc * 16;
    if (row < trows) {
      const int r = gstart + base + row;
      const int arow = GU ? p.sorted_tok[r] : r;
      agoff[i] = (uint32_t)arow * (uint32_t)p.lda * 2 + cc * 16;
    } else {
      agoff[i] = MX_OOB;
    }
  }

  float4_t acc[MTX][NF];
#pragma unroll
  for (int mi = 0; mi < MTX; ++mi)
#pragma unroll
    for (int f = 0; f < NF; ++f) acc[mi][f] = (float4_t){0.f, 0.f, 0.f, 0.f};

  auto load_a = [&](int st, int4_t (&ar)[ACH]) {
    const int k0 = st * KS;
#pragma unroll
    for (int i = 0; i < ACH; ++i)
      ar[i] = mx_ld16(ra, (k0 + acol[i] < K) ? agoff[i] + (uint32_t)k0 * 2 : MX_OOB);
  };
  // sb: byte offset of the slab in a slab chain (0 otherwise).
  auto load_b = [&](int st, int4_t (&br)[KM][NF], uint32_t sb = 0) {
#pragma unroll
    for (int km = 0; km < KM; ++km) {
      const bool kin = st * KS + km * 4 * EPL + q * EPL < K;
      const uint32_t kb = ((uint32_t)st * KM + km) * bstep + sb;
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const int fi = GU ? (f % NBIX) : f;
        // (this exact form: a temporary for the offset makes the compiler spill)
        br[km][f] = mx_ldw16<NT>((GU && f >= NBIX) ? rb1 : rb0,
                                 kin ? boff[fi] + kb : MX_OOB);
      }
    }
  };
  auto store_a = [&](int buf, const int4_t (&ar)[ACH]) {
    char* sbase = lds + buf * ATILE;
#pragma unroll
    for (int i = 0; i < ACH; ++i) *(int4_t*)(sbase + alds[i]) = ar[i];
  };
  auto compute = [&](int buf, const int4_t (&br)[KM][NF]) {
    const char* cbase = lds + buf * ATILE;
    if constexpr (WF == MX_DT_F16) {
#pragma unroll
      for (int km = 0; km < KM; ++km)
#pragma unroll
        for (int mi = 0; mi < MTX; ++mi) {
          const int4_t a = *(const int4_t*)(cbase + (16 * mi + j) * AROW + km * 64 + q * 16);
#pragma unroll
          for (int f = 0; f < NF; ++f)
            acc[mi][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                __builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, br[km][f]),
                acc[mi][f], 0, 0, 0);
        }
    } else {
      half8_t blo[NF], bhi[NF];
#pragma unroll
      for (int f = 0; f < NF; ++f) mx_i8_to_f16(br[0][f], blo[f], bhi[f]);
#pragma unroll
      for (int mi = 0; mi < MTX; ++mi) {
        const char* ap = cbase + (16 * mi + j) * AROW + q * 32;
        const int4_t a0 = *(const int4_t*)ap;
        const int4_t a1 = *(const int4_t*)(ap + 16);
#pragma unroll
        for (int f = 0; f < NF; ++f) {
          acc[mi][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a0),
                                                              blo[f], acc[mi][f], 0, 0, 0);
          acc[mi][f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a1),
                                                              bhi[f], acc[mi][f], 0, 0, 0);
        }
      }
    }
  };

  // Software pipeline: stage s computes from LDS buffer s % 2 and weight set s % RB while
  // the activations of stages s + 1 .. s + RA and the weights of stages s + 1 .. s + RB - 1
  // are in flight; the activations of stage s + 1 go to LDS at the end of stage s.  The
  // global latency is hidden by the ring depths, not by the LDS double buffer.  The loop
  // body is branch-free so the in-order load counter is never drained: stages past the
  // end of K read zeros through the descriptors' bounds check and the stage count is
  // padded to a multiple of RB (a multiple of RA), which also makes every register-set
  // index static.  A wave without columns (edge of a narrower shared expert) has
  // out-of-range weight offsets, computes zeros and skips the epilogue.
  const int nst = (K + KS - 1) / KS;
  const int nst_pad = (nst + RB - 1) / RB * RB;
  int4_t aring[RA][ACH];
  int4_t bring[RB][KM][NF];
  if constexpr (CH > 1) {
    // Slab chain: the same pipeline over `items` slabs in turn.  In the last ring turn of a
    // slab the loads that run ahead (weights RB - 1 stages, activations RA stages) fetch the
    // next slab's first stages: the same activation rows, the weights one slab delta
    // further.  Past the last slab they fetch memory nobody reads (inside the matrix, or
    // out of range and zero), so no load needs a slab check.  Slab widths divide N (the
    // launch checks it), so every lane's columns are inside N.
#pragma unroll
    for (int u = 0; u < RA; ++u) load_a(u, aring[u]);
#pragma unroll
    for (int u = 0; u < RB - 1; ++u) load_b(u, bring[u]);
    store_a(0, aring[0]);
    __syncthreads();
    const int orow = __builtin_amdgcn_readfirstlane(gstart + base);
    const int trs = __builtin_amdgcn_readfirstlane(trows);
    for (int ci = 0; ci < items; ++ci) {
      const uint32_t sb_cur = (uint32_t)ci * dslab, sb_next = sb_cur + dslab;
      for (int s0 = 0; s0 < nst_pad; s0 += RB) {
        const bool last = s0 + RB == nst_pad;
#pragma unroll
        for (int u = 0; u < RB; ++u) {
          const int sbn = s0 + u + RB - 1, san = s0 + u + RA;
          const bool bx = last && sbn >= nst_pad, ax = last && san >= nst_pad;
          load_b(bx ? sbn - nst_pad : sbn, bring[(u + RB - 1) % RB], bx ? sb_next : sb_cur);
          compute(u % 2, bring[u]);
          store_a((u + 1) % 2, aring[(u + 1) % RA]);
          load_a(ax ? san - nst_pad : san, aring[u % RA]);
          __syncthreads();
        }
      }
      // Epilogue of slab ci (the down epilogue below, routing weights from LDS).  The
      // row stride, row count and weight index go through empty asm statements so the
      // compiler recomputes the addresses here instead of hoisting all 32 rows' addresses
      // out of the slab loop (where they spill).
      // Stores through a buffer descriptor of y: 32-bit offsets (the launch checks that y
      // is under 2 GiB).
      // (The lane index is recomputed here, by mbcnt in an asm statement the compiler
      // cannot hoist, so no register holds it across the slab.)
      int ln;
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
      int ldo = p.ldo, tr = trs, orw = orow, q4 = (ln >> 4) * 4, cj = ln & 15;
      asm volatile("" : "+s"(ldo), "+s"(tr), "+s"(orw));
      const int n0c = n0 + ci * SLABW;
      if (n0c < N) {
        constexpr uint32_t YE = Y16 ? 2u : 4u;  // bytes per element of y
        const mx_rsrc_t ry = mx_rsrc(p.out, 0x7fffffffu);
        const uint32_t yb = ((uint32_t)(orw + q4) * (uint32_t)ldo + (uint32_t)(n0c + cj)) * YE;
#pragma unroll
        for (int mi = 0; mi < MTX; ++mi)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = 16 * mi + q4 + r;
            if (m >= tr) continue;
            const uint32_t yo = yb + (uint32_t)(16 * mi + r) * (uint32_t)ldo * YE;
            const float w = wrow[m];
#pragma unroll
            for (int f = 0; f < NBIX; ++f) {
              const float v = w * (acc[mi][f][r] * 1.f);
              if constexpr (Y16)
                __builtin_amdgcn_raw_buffer_store_b16(
                    __builtin_bit_cast(short, mx_f16_sat(v)), ry, yo + 32u * f, 0, 0);
              else
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v), ry,
                                                      yo + 64u * f, 0, 0);
            }
          }
      }
#pragma unroll
      for (int mi = 0; mi < MTX; ++mi)
#pragma unroll
        for (int f = 0; f < NF; ++f) acc[mi][f] = (float4_t){0.f, 0.f, 0.f, 0.f};
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < RA; ++u) load_a(u, aring[u]);
#pragma unroll
  for (int u = 0; u < RB - 1; ++u) load_b(u, bring[u]);
  store_a(0, aring[0]);
  __syncthreads();
  for (int s0 = 0; s0 < nst_pad; s0 += RB) {
#pragma unroll
    for (int u = 0; u < RB; ++u) {
      const int st = s0 + u;
      load_b(st + RB - 1, bring[(u + RB - 1) % RB]);
      compute(u % 2, bring[u]);
      store_a((u + 1) % 2, aring[(u + 1) % RA]);
      load_a(st + RA, aring[u % RA]);
      __syncthreads();
    }
  }
  if (!wact) return;

  const int orow = gstart + base;  // sorted row of the tile's row 0
  if constexpr (GU) {
#pragma unroll
    for (int f = 0; f < NBIX; ++f) {
      const int n = n0 + 16 * f + j;
      if (n >= N) continue;
      float sg = 1.f, su = 1.f;
      if constexpr (WF == MX_DT_I8) {
        sg = (float)((const half_t*)ep.gate_scale)[n];
        su = (float)((const half_t*)ep.up_scale)[n];
      }
#pragma unroll
      for (int mi = 0; mi < MTX; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * mi + 4 * q + r;
          if (m < trows) {
            const float gv = acc[mi][f][r] * sg;
            const float uv = acc[mi][NBIX + f][r] * su;
            ((half_t*)p.out)[(size_t)(orow + m) * p.ldo + n] = mx_f16_sat(mx_silu(gv) * uv);
          }
        }
    }
  } else {
    // Fragments f and f + 1 of a row are the two 64-byte halves of one 128-byte line of y:
    // they are stored by consecutive instructions so that L2 merges them before write-back.
    float sd[NBIX];
#pragma unroll
    for (int f = 0; f < NBIX; ++f) {
      sd[f] = 1.f;
      if constexpr (WF == MX_DT_I8) {
        const int n = n0 + 16 * f + j;
        if (n < N) sd[f] = (float)((const half_t*)ep.down_scale)[n];
      }
    }
#pragma unroll
    for (int mi = 0; mi < MTX; ++mi)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 16 * mi + 4 * q + r;
        if (m >= trows) continue;
        const int row = orow + m;
        const float w = p.sorted_w[row];
#pragma unroll
        for (int f = 0; f < NBIX; ++f) {
          const int n = n0 + 16 * f + j;
          if (n >= N) continue;
          const float v = w * (acc[mi][f][r] * sd[f]);
          if constexpr (Y16)
            ((half_t*)p.out)[(size_t)row * p.ldo + n] = mx_f16_sat(v);
          else
            ((float*)p.out)[(size_t)row * p.ldo + n] = v;
        }
      }
  }
}

// Waves per block of the prefill kernel: 4 (two blocks per CU) or 8 (fp16 only; one block
// per CU, one staged activation tile for twice the columns).  Measured on MI355X with the
// work dealt evenly over the XCDs: 8 waves win for reductions of 1024 columns and more
// (GLM-4.7 gate/up, K = 5120: 1050 -> 983 us; down, K = 1536: 652 -> 621 us; Qwen3-Next
// gate/up, K = 2048: equal) and tie for the Qwen3-Next down, K = 512 (333 -> 334 us).
#ifndef MX_LDS_8W_KMIN
#define MX_LDS_8W_KMIN 1024
#endif
#ifndef MX_LDS_8W_KMAX
#define MX_LDS_8W_KMAX (1 << 30)
#endif
static bool lds_eight_waves(int wdt, int K) {
  return MX_LDS_8W && wdt == MX_DT_F16 && K >= MX_LDS_8W_KMIN && K <= MX_LDS_8W_KMAX;
}

// Slab chains for the fp16 down projection of short reductions (few stages per slab, so a
// block's pipeline fill and epilogue are a large part of its life).
#ifndef MX_LDS_CHAIN
#define MX_LDS_CHAIN 2
#endif
#ifndef MX_LDS_CHAIN_KMAX
#define MX_LDS_CHAIN_KMAX 512
#endif
// The chained epilogue stores whole slabs (64 columns per wave) through 32-bit
// offsets, so every expert's N must be a multiple of 256 and y below 2 GiB.
#ifndef MX_LDS_CHAIN8
#define MX_LDS_CHAIN8 1  // slab chains for 8-wave blocks too
#endif
static int lds_slab_chain(bool gu, int wdt, int nw, const ExpertParams& p, int mt_max) {
  if (gu || wdt != MX_DT_F16 || MX_LDS_CHAIN < 2) return 1;
  if (nw != 4 && !(nw == 8 && MX_LDS_CHAIN8)) return 1;
  if (nw == 4 && (p.K_r > MX_LDS_CHAIN_KMAX || p.K_s > MX_LDS_CHAIN_KMAX)) return 1;
  const int slab = nw * 64;
  if (p.N_r % slab || p.N_s % slab) return 1;
  if ((long)mt_max * 128 * p.ldo * 4 >= (1l << 31) - 1) return 1;
  return MX_LDS_CHAIN;
}

// CH > 1: each block runs up to CH consecutive column slabs of its m-tile in turn
// (expert_lds_tile's slab chain); nblk counts the slabs, the grid the chains.
// Gate/up groups of at most 64 rows on 64-row tiles (the block's tile at half height: half
// the MFMAs and half the activation stage per column stage).  GLM-4.7 2048-token Zipf
// prefill, same box, interleaved: gate/up 1.051 -> 1.041 ms.  (In the down launch's slab
// chains the second tile height pushes the 4-wave variants past 256 VGPRs into spills.)
#ifndef MX_LDS_HALF_TILE
#define MX_LDS_HALF_TILE 1
#endif
template <int WF, bool GU, int NW, int CH = 1, bool Y16 = false>
__global__ __launch_bounds__((64 * NW), (LdsShape<WF>::OCC * 4 / NW)) void k_expert_lds(
    const ExpertParams p, int mt_max, int nslab) {
  constexpr int KS = 4 * WTr<WF>::EPL * LdsShape<WF>::KM;
  constexpr int NBI = GU ? 2 : 4;
  constexpr int MB = 128;
  __shared__ __align__(16) char lds[2 * MB * (KS * 2 + MX_LDS_APAD)];
  __shared__ float wrow[CH > 1 ? MB : 1];
  const int nblk = (nslab + CH - 1) / CH;

  // The grid is sized for mt_max (an upper bound of the m-tile count); the blocks of the
  // actual n_mtiles x nblk tiles are dealt to the 8 XCDs (hardware block b runs on XCD
  // b % 8) in 8 equal contiguous runs, so every XCD gets the same share of the work and the
  // blocks of one run walk the m-tiles of a column slab in order.
  const int b = blockIdx.x;
  const int nmt = min(*p.n_mtiles, mt_max);
  const int real = nmt * nblk;
  const int per = (real + 7) >> 3;
  const int logical = MX_LDS_XCD_REAL ? (b & 7) * per + (b >> 3)
                                      : (b & 7) * (gridDim.x >> 3) + (b >> 3);
  const int span = MX_LDS_XCD_REAL ? nmt : mt_max;
  if (MX_LDS_XCD_REAL && (b >> 3) >= per) return;
  int nb, mt;
  if (MX_LDS_ORDER == 1 && MX_LDS_XCD_REAL) {
    // tile-major: one m-tile's column slabs in a row
    mt = logical / nblk;
    nb = logical - mt * nblk;
    if (mt >= nmt) return;
  } else if (MX_LDS_ORDER == 2 && MX_LDS_XCD_REAL) {
    // expert-major: one group's blocks in a row, column slabs outer and its m-tiles inner
    // (the m-tiles of a group are consecutive in the list; row0 = 128 x tile index).
    const int mtp = logical / nblk;
    if (mtp >= nmt) return;
    const int gg = p.mt_group[mtp];
    const int t0 = mtp - p.mt_row0[mtp] / MB;
    const int ntg = (p.g_count[gg] + MB - 1) / MB;
    const int local = logical - nblk * t0;
    nb = local / ntg;
    mt = t0 + (local - nb * ntg);
  } else {
    nb = logical / span;
    mt = logical - nb * span;
  }
  if (nb >= nblk || mt >= nmt) return;
  const int g = p.mt_group[mt];
  const int row0 = p.mt_row0[mt];
  const int N = p.g_expert[g] == p.E ? p.N_s : p.N_r;
  const int n0b = nb * CH * NW * 16 * NBI;
  if (n0b >= N) return;  // whole block past this expert's columns
  const int trows = min(MB, p.g_count[g] - row0);
  if constexpr (CH > 1) {
    const int items = min(CH, nslab - nb * CH);
    if ((int)threadIdx.x < trows) wrow[threadIdx.x] = p.sorted_w[p.g_start[g] + row0 + threadIdx.x];
    if (MX_LDS_NT_SINGLE && p.g_count[g] <= MB)
      expert_lds_tile<WF, GU, 8, NBI, NW, true, CH, Y16>(p, lds, g, row0, trows, n0b, items,
                                                         wrow);
    else
      expert_lds_tile<WF, GU, 8, NBI, NW, MX_LDS_NT_DN, CH, Y16>(p, lds, g, row0, trows, n0b,
                                                                  items, wrow);
    return;
  }
  if constexpr (GU && MX_LDS_HALF_TILE) {
    if (p.g_count[g] <= MB / 2) {
      expert_lds_tile<WF, GU, 4, NBI, NW, true, 1, Y16>(p, lds, g, row0, trows, n0b);
      return;
    }
  }
  if (MX_LDS_NT_SINGLE && p.g_count[g] <= MB)
    expert_lds_tile<WF, GU, 8, NBI, NW, true, 1, Y16>(p, lds, g, row0, trows, n0b);
  else
    expert_lds_tile<WF, GU, 8, NBI, NW, GU ? MX_LDS_NT_GU : MX_LDS_NT_DN, 1, Y16>(
        p, lds, g, row0, trows, n0b);
}

// ------------------------------------------------------------------------------------
// Host side.
// ------------------------------------------------------------------------------------
#ifndef MX_PREFILL_M_BLK
#define MX_PREFILL_M_BLK 128
#endif
int mx_m_blk_for(int tokens, int weight_dtype) {
  if (tokens <= 16) return 16;
  if (tokens <= 32) return 32;
  if (tokens <= 64 || weight_dtype == MX_DT_F32) return 64;
  return MX_PREFILL_M_BLK;
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
  if (d->weight_layout != MX_LAYOUT_ROWS && d->weight_layout != MX_LAYOUT_FRAG16)
    return MX_ERR_INVALID;
  // Fragment layout: whole fragments only (16 rows, KC = 4 * epl columns).
  if (d->weight_layout == MX_LAYOUT_FRAG16 &&
      (d->hidden % (4 * epl) || d->inter % (4 * epl) || d->shared_inter % (4 * epl)))
    return MX_ERR_UNSUPPORTED;
  // Buffer descriptors address < 2 GiB per matrix.
  const int esz = d->weight_dtype == MX_DT_F32 ? 4 : (d->weight_dtype == MX_DT_F16 ? 2 : 1);
  const long mx = (long)d->hidden * (d->inter > d->shared_inter ? d->inter : d->shared_inter) * esz;
  if (mx >= (1l << 31)) return MX_ERR_UNSUPPORTED;
  return MX_OK;
}

// Decode-kernel shape (compile-time tunables): column blocks of 16 per wave for gate/up
// (x2 for the gate and up halves) and for down, and k-chunks per load batch.
#ifndef MX_DEC_NBI_GU
#define MX_DEC_NBI_GU 1
#endif
#ifndef MX_DEC_NBI_DN
#define MX_DEC_NBI_DN 2
#endif
#ifndef MX_DEC_UK
#define MX_DEC_UK 4
#endif
#ifndef MX_DEC_UK_I8
#define MX_DEC_UK_I8 (MX_DEC_UK / 2)
#endif

// K split inside a block for single-m-frag tiles (m_blk 16).  The split is picked from
// the number of waves the launch would have unsplit (measured on MI355X, fp16 GLM-4.7 and
// Qwen3-Next shapes at 1-8 tokens): a launch far below one wave per SIMD gains from more,
// shorter weight streams; one near a wave per SIMD loses from splitting (gate/up); a
// launch of several waves per SIMD gains tail balance from short waves.  (Down at one
// GLM-4.7 token, 1440 waves unsplit: 23.2 us with a 2-way split, 22.6 us with 4-way.
// Gate/up at one GLM-4.7 token, 864 waves unsplit, distinct layers per step: int8
// 53.5 -> 50.5 us per block with a 2-way split, fp16 equal within noise.)
#ifndef MX_KS_GU_LO
#define MX_KS_GU_LO 1024
#endif
#ifndef MX_KS_GU_HI
#define MX_KS_GU_HI 2048
#endif
#ifndef MX_KS_DN_LO
#define MX_KS_DN_LO 2048
#endif
#ifndef MX_KS_DN_HI
#define MX_KS_DN_HI 4096
#endif
static int decode_ksplit(bool gu, long waves_unsplit) {
  if (gu) return waves_unsplit < MX_KS_GU_LO ? 2 : (waves_unsplit < MX_KS_GU_HI ? 1 : 4);
  return waves_unsplit < MX_KS_DN_LO ? 4 : (waves_unsplit < MX_KS_DN_HI ? 2 : 1);
}

template <int WF, int MT, bool GU, int KS, int SELV = 0>
static void launch_expert_ks(const ExpertParams& p, int mt_max, int nmax, hipStream_t s,
                             const SelectParams& sp = SelectParams{}) {
  constexpr int NBI = GU ? MX_DEC_NBI_GU : MX_DEC_NBI_DN;
  constexpr int UK = (WF == MX_DT_I8) ? (MT >= 4 ? 1 : MX_DEC_UK_I8)
                                      : (MT >= 4 ? 2 : MX_DEC_UK);
  constexpr bool NT = !(MX_I8_GU_PLAIN && WF == MX_DT_I8 && GU && MT == 1 && KS == 1);
  const dim3 grid(mt_max, mx_ceil_div(nmax, (4 / KS) * 16 * NBI));
  mx_clear_error();
  hipLaunchKernelGGL((k_expert<WF, MT, NBI, GU, UK, KS, NT, SELV>), grid, dim3(256), 0, s, p, sp);
}

template <int WF, int SELV>
static void launch_gate_up_select_v(const ExpertParams& p, const SelectParams& sp, int mt_max,
                                    int nmax, hipStream_t s) {
  const long waves = (long)mt_max * mx_ceil_div(nmax, 4 * 16 * MX_DEC_NBI_GU) * 4;
  const int ks = decode_ksplit(true, waves);
  if (ks == 4) return launch_expert_ks<WF, 1, true, 4, SELV>(p, mt_max, nmax, s, sp);
  if (ks == 2) return launch_expert_ks<WF, 1, true, 2, SELV>(p, mt_max, nmax, s, sp);
  launch_expert_ks<WF, 1, true, 1, SELV>(p, mt_max, nmax, s, sp);
}

template <int WF>
static void launch_gate_up_select(const ExpertParams& p, const SelectParams& sp, int mt_max,
                                  int nmax, hipStream_t s) {
  if (p.E <= 256)
    launch_gate_up_select_v<WF, 4>(p, sp, mt_max, nmax, s);
  else
    launch_gate_up_select_v<WF, 8>(p, sp, mt_max, nmax, s);
}

template <int WF, int MT, bool GU>
static void launch_expert(const ExpertParams& p, int mt_max, int nmax, hipStream_t s) {
  if constexpr (MT == 1) {
    constexpr int NBI = GU ? MX_DEC_NBI_GU : MX_DEC_NBI_DN;
    const long waves = (long)mt_max * mx_ceil_div(nmax, 4 * 16 * NBI) * 4;
    const int ks = decode_ksplit(GU, waves);
    if (ks == 4) return launch_expert_ks<WF, 1, GU, 4>(p, mt_max, nmax, s);
    if (ks == 2) return launch_expert_ks<WF, 1, GU, 2>(p, mt_max, nmax, s);
  }
  launch_expert_ks<WF, MT, GU, 1>(p, mt_max, nmax, s);
}

template <bool GU>
static int dispatch_expert(int wdt, int mt, const ExpertParams& p, int mt_max, int nmax,
                           hipStream_t s) {
#define MX_EXP_CASE(W)                                                \
  if (wdt == W) {                                                     \
    if (mt == 1) launch_expert<W, 1, GU>(p, mt_max, nmax, s);         \
    else if (mt == 2) launch_expert<W, 2, GU>(p, mt_max, nmax, s);    \
    else if (mt == 4) launch_expert<W, 4, GU>(p, mt_max, nmax, s);    \
    else return MX_ERR_INVALID;                                       \
    return mx_launch_status();                                        \
  }
  MX_EXP_CASE(MX_DT_F16)
  MX_EXP_CASE(MX_DT_I8)
  MX_EXP_CASE(MX_DT_F32)
#undef MX_EXP_CASE
  return MX_ERR_INVALID;
}

// Direct-load kernel for m_blk 16/32/64; LDS-staged kernel for m_blk 128 (fp16/int8).
// mt_max bounds the m-tile list (the kernels read the actual count from p.n_mtiles).
template <bool GU, bool Y16>
static int launch_lds(int wdt, const ExpertParams& p, int mt_max, int nmax, hipStream_t s) {
  const int nw = lds_eight_waves(wdt, p.K_r) ? 8 : 4;
  const int cols = nw * 16 * (GU ? 2 : 4);
  const int nblk = mx_ceil_div(nmax, cols);
  const int ch = lds_slab_chain(GU, wdt, nw, p, mt_max);
  const long blocks = ((long)mt_max * mx_ceil_div(nblk, ch) + 7) / 8 * 8;
  if (blocks > (1l << 31) - 1) return MX_ERR_UNSUPPORTED;
  mx_clear_error();
  if (!GU && ch == 2 && nw == 8 && MX_LDS_CHAIN8)
    hipLaunchKernelGGL((k_expert_lds<MX_DT_F16, false, 8, 2, Y16>), dim3((unsigned)blocks),
                       dim3(512), 0, s, p, mt_max, nblk);
  else if (!GU && ch == 2)
    hipLaunchKernelGGL((k_expert_lds<MX_DT_F16, false, 4, 2, Y16>), dim3((unsigned)blocks),
                       dim3(256), 0, s, p, mt_max, nblk);
  else if (!GU && ch == 4)
    hipLaunchKernelGGL((k_expert_lds<MX_DT_F16, false, 4, 4, Y16>), dim3((unsigned)blocks),
                       dim3(256), 0, s, p, mt_max, nblk);
  else if (wdt == MX_DT_F16 && nw == 8)
    hipLaunchKernelGGL((k_expert_lds<MX_DT_F16, GU, 8, 1, Y16>), dim3((unsigned)blocks),
                       dim3(512), 0, s, p, mt_max, nblk);
  else if (wdt == MX_DT_F16)
    hipLaunchKernelGGL((k_expert_lds<MX_DT_F16, GU, 4, 1, Y16>), dim3((unsigned)blocks),
                       dim3(256), 0, s, p, mt_max, nblk);
  else
    hipLaunchKernelGGL((k_expert_lds<MX_DT_I8, GU, 4, 1, Y16>), dim3((unsigned)blocks),
                       dim3(256), 0, s, p, mt_max, nblk);
  return mx_launch_status();
}

template <bool GU>
static int launch_grouped_mt(int wdt, const ExpertParams& p, int mt_max, int m_blk, int nmax,
                             hipStream_t s) {
  if (m_blk == 128) {
    if (wdt == MX_DT_F32) return MX_ERR_INVALID;
    if constexpr (!GU)
      if (p.y16) return launch_lds<false, true>(wdt, p, mt_max, nmax, s);
    return launch_lds<GU, false>(wdt, p, mt_max, nmax, s);
  }
  if (p.y16) return MX_ERR_INVALID;  // fp16 y rows come from the prefill kernel only
  if (m_blk != 16 && m_blk != 32 && m_blk != 64) return MX_ERR_INVALID;
  return dispatch_expert<GU>(wdt, m_blk / 16, p, mt_max, nmax, s);
}

template <bool GU>
static int launch_grouped(const MxMoeDesc* d, const ExpertParams& p, int tokens, int m_blk,
                          int nmax, hipStream_t s) {
  const int has_shared = d->shared_inter > 0;
  const int mt_max = mx_max_mtiles(tokens, d->top_k, d->n_experts, has_shared, m_blk);
  return launch_grouped_mt<GU>(d->weight_dtype, p, mt_max, m_blk, nmax, s);
}

// Dense y[T, N] = a[T, K] W[N, K]^T (x the fp16 row scale of int8 weights) on the down-
// projection kernels: one group of T rows, `entry` an expert table entry whose `down`
// (and `down_scale`) is W, `tab` the single-group tables (g_* = {entry 0, row 0, T},
// mt_group = 0, mt_row0 = i * m_blk, n_mtiles = ceil(T / m_blk)) and `ones` [T] of 1.0.
int mx_dense_linear(int wdt, int tiled, const MxExpertPtrs* entry, const MxDenseTables& tab,
                    int T, int N, int K, const void* a, float* y, hipStream_t s) {
  int epl;
  switch (wdt) {
    case MX_DT_F32: epl = 4; break;
    case MX_DT_F16: epl = 8; break;
    case MX_DT_I8: epl = 16; break;
    default: return MX_ERR_INVALID;
  }
  if (T <= 0 || N <= 0 || K <= 0 || !entry || !a || !y) return MX_ERR_INVALID;
  if (K % epl) return MX_ERR_UNSUPPORTED;
  if (tiled && (N % 16 || K % (4 * epl))) return MX_ERR_UNSUPPORTED;
  const int esz = wdt == MX_DT_F32 ? 4 : (wdt == MX_DT_F16 ? 2 : 1);
  const int aesz = wdt == MX_DT_F32 ? 4 : 2;
  if ((long)N * K * esz >= (1l << 31) || (long)T * K * aesz >= (1l << 31))
    return MX_ERR_UNSUPPORTED;
  if (!mx_aligned16(a) || !mx_aligned16(y)) return MX_ERR_ALIGNMENT;
  ExpertParams p;
  p.experts = entry;
  p.g_expert = tab.g_expert;
  p.g_start = tab.g_start;
  p.g_count = tab.g_count;
  p.mt_group = tab.mt_group;
  p.mt_row0 = tab.mt_row0;
  p.n_mtiles = tab.n_mtiles;
  p.sorted_tok = nullptr;
  p.a = a;
  p.a_bytes = (uint32_t)((long)T * K * aesz);
  p.lda = K;
  p.out = y;
  p.ldo = N;
  p.sorted_w = tab.ones;
  p.E = 1;
  p.N_r = N;
  p.K_r = K;
  p.N_s = N;
  p.K_s = K;
  p.tiled = tiled;
  return launch_grouped_mt<false>(wdt, p, mx_ceil_div(T, tab.m_blk), tab.m_blk, N, s);
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
  if (m_blk != 16 && m_blk != 32 && m_blk != 64 && m_blk != 128) return MX_ERR_INVALID;
  if (tokens == 0) return MX_OK;
  const int aesz = desc->weight_dtype == MX_DT_F32 ? 4 : 2;
  const long abytes = (long)tokens * desc->hidden * aesz;
  if (abytes >= (1l << 31)) return MX_ERR_UNSUPPORTED;
  if (!mx_aligned16(a) || !mx_aligned16(act)) return MX_ERR_ALIGNMENT;
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
  p.tiled = desc->weight_layout == MX_LAYOUT_FRAG16;
  return launch_grouped<true>(desc, p, tokens, m_blk, p.ldo, (hipStream_t)stream);
}

int mx_expert_gate_up_select(const MxMoeDesc* desc, const MxExpertPtrs* experts, const void* a,
                             void* act, const MxOneTokenSelect& sp, hipStream_t s) {
  MX_TRY(expert_check(desc));
  if (!experts || !a || !act || !sp.logits || !sp.ids || !sp.tw || !sp.sorted_w) return MX_ERR_INVALID;
  if (!mx_one_token_select_ok(desc)) return MX_ERR_UNSUPPORTED;
  if (!mx_aligned16(a) || !mx_aligned16(act)) return MX_ERR_ALIGNMENT;
  const int aesz = desc->weight_dtype == MX_DT_F32 ? 4 : 2;
  ExpertParams p;
  p.experts = experts;
  p.g_expert = sp.g_expert;
  p.g_start = sp.g_start;
  p.g_count = sp.g_count;
  p.mt_group = sp.mt_group;
  p.mt_row0 = sp.mt_row0;
  p.n_mtiles = sp.n_mtiles;
  p.sorted_tok = sp.sorted_tok;
  p.a = a;
  p.a_bytes = (uint32_t)((long)desc->hidden * aesz);
  p.lda = desc->hidden;
  p.out = act;
  p.ldo = desc->inter > desc->shared_inter ? desc->inter : desc->shared_inter;
  p.sorted_w = nullptr;
  p.E = desc->n_experts;
  p.N_r = desc->inter;
  p.K_r = desc->hidden;
  p.N_s = desc->shared_inter;
  p.K_s = desc->hidden;
  p.tiled = desc->weight_layout == MX_LAYOUT_FRAG16;
  const int mt_max = desc->top_k + (desc->shared_inter > 0 ? 1 : 0);
  switch (desc->weight_dtype) {
    case MX_DT_F16: launch_gate_up_select<MX_DT_F16>(p, sp, mt_max, p.ldo, s); break;
    case MX_DT_I8: launch_gate_up_select<MX_DT_I8>(p, sp, mt_max, p.ldo, s); break;
    case MX_DT_F32: launch_gate_up_select<MX_DT_F32>(p, sp, mt_max, p.ldo, s); break;
    default: return MX_ERR_INVALID;
  }
  return mx_launch_status();
}

extern "C" int mx_expert_down(const MxMoeDesc* desc, const MxExpertPtrs* experts, int32_t tokens,
                              const void* act, const float* sorted_w, const int32_t* g_expert,
                              const int32_t* g_start, const int32_t* g_count,
                              const int32_t* mt_group, const int32_t* mt_row0,
                              const int32_t* n_mtiles, int32_t m_blk, float* y, void* stream) {
  return mx_expert_down_rows(desc, experts, tokens, act, sorted_w, g_expert, g_start, g_count,
                             mt_group, mt_row0, n_mtiles, m_blk, y, false, (hipStream_t)stream);
}

int mx_expert_down_rows(const MxMoeDesc* desc, const MxExpertPtrs* experts, int tokens,
                        const void* act, const float* sorted_w, const int* g_expert,
                        const int* g_start, const int* g_count, const int* mt_group,
                        const int* mt_row0, const int* n_mtiles, int m_blk, void* y, bool y16,
                        hipStream_t stream) {
  MX_TRY(expert_check(desc));
  if (y16 && m_blk != 128) return MX_ERR_INVALID;
  if (!experts || !act || !sorted_w || !g_expert || !g_start || !g_count || !mt_group ||
      !mt_row0 || !n_mtiles || !y || tokens < 0)
    return MX_ERR_INVALID;
  if (m_blk != 16 && m_blk != 32 && m_blk != 64 && m_blk != 128) return MX_ERR_INVALID;
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
  p.tiled = desc->weight_layout == MX_LAYOUT_FRAG16;
  p.y16 = y16;
  return launch_grouped<false>(desc, p, tokens, m_blk, desc->hidden, stream);
}

// ------------------------------------------------------------------------------------
// Row-major -> MX_LAYOUT_FRAG16.  One thread per 16-byte piece: piece l of fragment
// (g, c) comes from row 16 g + (l % 16), bytes 64 c + 16 (l / 16) of that row, and goes
// to byte (g * nch + c) * 1024 + 16 l.  Writes are contiguous per wave; the reads are
// the row-strided pattern the layout exists to avoid, paid once per bound layer.
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_tile_weights(int4_t* __restrict__ dst,
                                                      const char* __restrict__ src,
                                                      long pieces, uint32_t rowb, int nch) {
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  if (t >= pieces) return;
  const long frag = t >> 6;
  const int l = (int)(t & 63);
  const long g = frag / nch;
  const int c = (int)(frag - g * nch);
  const size_t so = (size_t)(g * 16 + (l & 15)) * rowb + (size_t)c * 64 + (size_t)(l >> 4) * 16;
  dst[t] = *(const int4_t*)(src + so);
}

extern "C" int mx_tile_weights(void* dst, const void* src, int32_t rows, int32_t cols,
                               int32_t weight_dtype, void* stream) {
  if (!dst || !src || rows <= 0 || cols <= 0) return MX_ERR_INVALID;
  int esz;
  switch (weight_dtype) {
    case MX_DT_F32: esz = 4; break;
    case MX_DT_F16: esz = 2; break;
    case MX_DT_I8: esz = 1; break;
    default: return MX_ERR_INVALID;
  }
  const long rowb = (long)cols * esz;
  if (rows % 16 || rowb % 64) return MX_ERR_UNSUPPORTED;
  if (!mx_aligned16(dst) || !mx_aligned16(src)) return MX_ERR_ALIGNMENT;
  const long bytes = (long)rows * rowb;
  const char* d0 = (const char*)dst;
  const char* s0 = (const char*)src;
  if (d0 < s0 + bytes && s0 < d0 + bytes) return MX_ERR_INVALID;  // overlap
  if (rowb >= (1l << 32)) return MX_ERR_UNSUPPORTED;
  const long pieces = bytes / 16;
  mx_clear_error();
  hipLaunchKernelGGL(k_tile_weights, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (int4_t*)dst, (const char*)src, pieces,
                     (uint32_t)rowb, (int)(rowb / 64));
  return mx_launch_status();
}
