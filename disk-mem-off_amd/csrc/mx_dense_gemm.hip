// Dense GEMM on MFMA with an LDS-staged operand ring:
//   y_s[M, N_s] (fp32, row stride ldy_s) = a[M, K] . W_s[N_s, K]^T
// for up to MX_GEMM_MAX_SEG weight matrices W_s (nn.Linear row-major) that share the
// activations a.  Two element types:
//  * fp16 operands (v_mfma_f32_16x16x32_f16): the long-input projections of the attention
//    blocks (the q / k / v projections, or qkvz and ba, in one launch).  Reference:
//    linear_t = x @ W.T (offload_runtime/executors/_common.py:101-103) at
//    qwen3_next.py:170-174, :211, :231, :245 and :268.
//  * fp32 operands (v_mfma_f32_16x16x4_f32, full fp32 products), and
//  * fp32 operands carried as two fp16 planes each (SPLIT): x = hi + 2^-11 lo with
//    hi = fp16(x), lo = fp16((x - hi) * 2^11), and a . w = a_hi . w_hi + 2^-11 (a_hi . w_lo
//    + a_lo . w_hi) up to the dropped 2^-22 a_lo . w_lo: three fp16 MFMAs per 32 columns
//    (exact products, fp32 sums) in place of eight fp32 ones, at the same operand bytes;
//  both for the router logits of long inputs, h @ Wr.T at glm4_moe.py:181 and
//  qwen3_next.py:278 (with the shared-expert gate row, qwen3_next.py:328), the reduction
//  split into slices over gridDim.y whose partial sums the top-k adds in slice order.
//
// Block tile BM x BN over one weight segment and one reduction slice; the reduction runs in
// stages of 128 bytes per row (64 fp16 or 32 fp32 columns, two MFMA k-steps of 64 bytes).
// Both operands of a stage are copied from global memory straight into LDS by the buffer
// loads' LDS mode (no register staging), into a ring of NS stage slots: while the waves
// compute stage s, the copies of stages s + 1 .. s + NS - 1 are in flight.  Each copy
// instruction moves one fragment of 8 rows x 128 bytes (1 KiB), so every row piece a copy
// reads is a whole 128-byte line: copies of 64-byte half lines (16 rows x 64 bytes) moved
// half as many bytes per clock from L2 into LDS (26.5 against 51.6 bytes per clock and CU,
// measured on MI355X with a copy-only probe; 4.5 against 5.8 TB/s from HBM).  The LDS mode
// stores lane l's 16 bytes at 16 l, so the lane-to-(row, chunk) map of the copy fixes the
// layout of the fragment in LDS (see below: whole rows, XOR-swizzled chunks, no padding).
// A stage is waited for with an explicit vmcnt (the copies are this loop's only vector
// memory operations) and a barrier without a memory fence: a fence on LDS would also wait
// for every copy still in flight, which would empty the ring at every stage.
// Each wave owns a WM x WN sub-tile (WM / 16 x WN / 16 accumulator tiles), so every A
// fragment read from LDS feeds WN / 16 products and every B fragment WM / 16.  Global
// reads go through buffer descriptors: rows past M or past N_s read zero.  K must be a
// multiple of the stage width (MX_ERR_UNSUPPORTED otherwise).
//
// Operand layout (lane = 16 q + j): at k-step ks an activation lane holds the 16 bytes of
// a[m0 + j] at byte 64 ks + 16 q of the stage, a weight lane those of W[n0 + j]; fp16 feeds
// them to one 16x16x32 MFMA (k = 32 ks + 8 q .. + 7), fp32 to four 16x16x4 MFMAs (the e-th
// takes element e of both, so the four cover the k-step's 16 columns once each).  With the
// weights as the MFMA's A operand the accumulator lane holds y[m0 + j][n0 + 4 q + r],
// r = 0..3.
#include "mx_common.h"
#include "mx_internal.h"
#include "mx_lds_copy.h"

namespace {

typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kRsrcDw3 = 0x00020000;
constexpr uint32_t kOob = 0x80000000u;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, kRsrcDw3);
}

struct GemmSeg {
  const void* w;  // [N, K]
  const void* w_lo;  // SPLIT: the low plane of w
  const float* res;  // residual added by the epilogue (same layout as y) or null
  float* y;       // [M, ldy] for slice 0; slice z at y + z * yslice
  int n;          // N of the segment
  int ldy;
  int nblk;       // column blocks of the segment
};

struct GemmArgs {
  const void* a;  // [M, K]
  const void* a_lo;  // SPLIT: the low plane of a
  int M, K;
  int kslice;     // reduction columns per slice (gridDim.y slices)
  long yslice;    // elements between the outputs of consecutive slices
  int mblk;       // row blocks
  int nseg;
  GemmSeg seg[MX_GEMM_MAX_SEG];
};

constexpr int STAGE_BYTES = MX_GEMM_STAGE_BYTES;  // bytes of each row per stage
constexpr int KSTEPS = STAGE_BYTES / 64;           // MFMA k-steps of 64 bytes per stage
constexpr int FRAG_ROWS = 1024 / STAGE_BYTES;      // rows per 1 KiB copy fragment
constexpr int BLK16 = 16 * STAGE_BYTES;            // bytes of a 16-row operand block per stage
static_assert(STAGE_BYTES == 128, "the copy and read maps below are for 128-byte rows");
#ifndef MX_GEMM_GM
#define MX_GEMM_GM 4  // row blocks per group of the block order (0: one column block at a time)
#endif

// Copy lane l of a fragment loads row l / 8 of it, 16-byte chunk (l % 8) ^ (l / 8), so
// every 8 consecutive lanes read one row's 128 contiguous bytes and the chunk c of row r
// lands in slot c ^ r of the row's 128 bytes in LDS.  The operand read of lane (j, q) at
// k-step ks (row j of a 16-row block, chunk 4 ks + q) is then free of bank conflicts on
// gfx950 (SQ_LDS_BANK_CONFLICT 0 with a read-only probe; without the XOR the 16-byte reads
// of a wave take four times the LDS cycles).
__device__ __forceinline__ int gemm_copy_chunk(int l) { return (l & 7) ^ (l >> 3); }
__device__ __forceinline__ int gemm_read_pos(int j, int q, int ks) {
  return (j >> 3) * 1024 + (j & 7) * 128 + ((((ks << 2) + q) ^ (j & 7)) << 4);
}

template <typename ET, bool SPLIT, int BM, int BN, int WM, int WN, int NS, int OCC>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64, OCC) void k_gemm_nt(
    const GemmArgs p) {
  constexpr int ES = sizeof(ET);
  constexpr int NWN = BN / WN, NW = (BM / WM) * NWN;
  constexpr int MF = WM / 16, NF = WN / 16;
  constexpr int PL = SPLIT ? 2 : 1;               // planes per operand
  constexpr int FA1 = BM / FRAG_ROWS, FB1 = BN / FRAG_ROWS;  // fragments per plane and stage
  constexpr int FA = PL * FA1, FT = FA + PL * FB1;  // fragments per stage slot: A planes, B planes
  constexpr int SLOT = FT * 1024;
  constexpr int PA = BM * STAGE_BYTES, PB = BN * STAGE_BYTES;  // bytes of one plane per slot
  constexpr int DPW = FT / NW;                    // copies per wave and stage
  static_assert(!SPLIT || ES == 2, "split planes are fp16");
  static_assert(FA1 % NW == 0 && FB1 % NW == 0, "fragments must divide among the waves");
  static_assert(NS >= 2, "a stage ring of at least two slots");
  __shared__ __align__(1024) char lds[NS * SLOT];

  // Blocks are numbered so that consecutive logical ids run on one XCD (hardware block b
  // goes to XCD b % 8).  Logical ids walk groups of MX_GEMM_GM row blocks: the row blocks of
  // a group for one column block, then for the next, so the blocks an XCD runs at once
  // share few operand tiles through its L2 (32 blocks: 4 row x 8 column blocks, 12
  // distinct tiles per stage, where one column block's 16 row blocks and the next's
  // need 18).
  const int nb_total = gridDim.x;
  const int b = blockIdx.x;
  const int logical = (nb_total % 8 == 0) ? (b & 7) * (nb_total >> 3) + (b >> 3) : b;
  int rem, mb;
  if (MX_GEMM_GM > 0) {
    const int ncol = nb_total / p.mblk;
    const int grp = logical / (MX_GEMM_GM * ncol);
    const int first = grp * MX_GEMM_GM;
    const int gm = min(p.mblk - first, MX_GEMM_GM);
    const int in = logical - grp * MX_GEMM_GM * ncol;
    rem = in / gm;
    mb = first + (in - rem * gm);
  } else {
    rem = logical / p.mblk;
    mb = logical - rem * p.mblk;
  }
  int si = 0;
#pragma unroll
  for (int i = 0; i < MX_GEMM_MAX_SEG - 1; ++i)
    if (si == i && i + 1 < p.nseg && rem >= p.seg[i].nblk) {
      rem -= p.seg[i].nblk;
      si = i + 1;
    }
  const GemmSeg sg = p.seg[si];
  const int m0 = mb * BM, n0 = rem * BN;
  const int M = p.M, K = p.K, N = sg.n;
  const int k0 = blockIdx.y * p.kslice;            // this block's reduction slice
  const int kn = min(p.kslice, K - k0);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / NWN, wn = wave % NWN;
  const int j = lane & 15, q = lane >> 4;

  const rsrc_t ra = make_rsrc(p.a, (uint32_t)((size_t)M * K * ES));
  const rsrc_t rb = make_rsrc(sg.w, (uint32_t)((size_t)N * K * ES));
  const rsrc_t ral = SPLIT ? make_rsrc(p.a_lo, (uint32_t)((size_t)M * K * ES)) : ra;
  const rsrc_t rbl = SPLIT ? make_rsrc(sg.w_lo, (uint32_t)((size_t)N * K * ES)) : rb;
  // Fragment f of a slot: A planes [0, FA) (plane f / FA1), then B planes (plane
  // (f - FA) / FB1).  The copy i of every wave lies in one plane (each plane's fragment
  // count is a multiple of NW), so its descriptor is uniform.
  auto rsrc_of = [&](int i) {
    const int f0 = i * NW;
    if (f0 < FA1) return ra;
    if (f0 < FA) return ral;
    if (f0 < FA + FB1) return rb;
    return rbl;
  };
  // The fragments this wave copies: f = wave + i * NW (A fragments first, then B); the
  // lane's source row and its byte offset at stage 0.
  const int cr = lane >> 3, cq = gemm_copy_chunk(lane);
  uint32_t goff[DPW];
#pragma unroll
  for (int i = 0; i < DPW; ++i) {
    const int f = wave + i * NW;
    if (i * NW < FA) {
      const int row = m0 + FRAG_ROWS * (f % FA1) + cr;
      goff[i] = row < M ? ((uint32_t)row * (uint32_t)K + k0) * ES + cq * 16 : kOob;
    } else {
      const int row = n0 + FRAG_ROWS * ((f - FA) % FB1) + cr;
      goff[i] = row < N ? ((uint32_t)row * (uint32_t)K + k0) * ES + cq * 16 : kOob;
    }
  }
  // K and the slice length are multiples of the stage width, so every piece of a stage lies
  // inside its row; rows past M / N have offsets at or above kOob, which stay past the end
  // of the descriptor.
  auto issue = [&](int st) {
    char* slot = lds + (st % NS) * SLOT;
#pragma unroll
    for (int i = 0; i < DPW; ++i) {
      const int f = wave + i * NW;
      mx_copy_to_lds16(rsrc_of(i), slot + f * 1024, goff[i] + (uint32_t)st * STAGE_BYTES);
    }
  };

  // acc[mi][ni] holds the transposed product (the weights are the MFMA's A operand):
  // lane (j, q) has y[m0 + 16 mi + j][n0 + 16 ni + 4 q + r], r = 0..3, so the epilogue
  // stores 4 consecutive columns per lane.
  // SPLIT: acc2 sums the two cross terms a_hi . w_lo + a_lo . w_hi.
  float4_t acc[MF][NF], acc2[SPLIT ? MF : 1][SPLIT ? NF : 1];
#pragma unroll
  for (int mi = 0; mi < MF; ++mi)
#pragma unroll
    for (int ni = 0; ni < NF; ++ni) acc[mi][ni] = (float4_t){0.f, 0.f, 0.f, 0.f};
  if constexpr (SPLIT) {
#pragma unroll
    for (int mi = 0; mi < MF; ++mi)
#pragma unroll
      for (int ni = 0; ni < NF; ++ni) acc2[mi][ni] = (float4_t){0.f, 0.f, 0.f, 0.f};
  }
  int rpos[KSTEPS];
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) rpos[ks] = gemm_read_pos(j, q, ks);

  const int nst = kn / (STAGE_BYTES / ES);
#pragma unroll
  for (int s0 = 0; s0 < NS - 1; ++s0)
    if (s0 < nst) issue(s0);
  for (int st = 0; st < nst; ++st) {
    // This wave's copies of stage st are done (the NS - 2 later stages may still be in
    // flight), then every wave's are, and every wave has finished computing stage st - 1,
    // whose slot the next copies overwrite.
    if (st + NS - 1 <= nst)
      mx_wait_copies_and_barrier<(NS - 2) * DPW>();
    else
      mx_wait_copies_and_barrier<0>();
    if (st + NS - 1 < nst) issue(st + NS - 1);
    const char* slot = lds + (st % NS) * SLOT;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      int4_t af[MF], bf[NF];
#pragma unroll
      for (int mi = 0; mi < MF; ++mi)
        af[mi] = *(const int4_t*)(slot + (wm * MF + mi) * BLK16 + rpos[ks]);
#pragma unroll
      for (int ni = 0; ni < NF; ++ni)
        bf[ni] = *(const int4_t*)(slot + PL * PA + (wn * NF + ni) * BLK16 + rpos[ks]);
      if constexpr (SPLIT) {
        int4_t afl[MF], bfl[NF];
#pragma unroll
        for (int mi = 0; mi < MF; ++mi)
          afl[mi] = *(const int4_t*)(slot + PA + (wm * MF + mi) * BLK16 + rpos[ks]);
#pragma unroll
        for (int ni = 0; ni < NF; ++ni)
          bfl[ni] = *(const int4_t*)(slot + 2 * PA + PB + (wn * NF + ni) * BLK16 + rpos[ks]);
#pragma unroll
        for (int mi = 0; mi < MF; ++mi)
#pragma unroll
          for (int ni = 0; ni < NF; ++ni) {
            const half8_t ah = __builtin_bit_cast(half8_t, af[mi]);
            const half8_t bh = __builtin_bit_cast(half8_t, bf[ni]);
            acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bh, ah, acc[mi][ni], 0, 0, 0);
            acc2[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                __builtin_bit_cast(half8_t, bfl[ni]), ah, acc2[mi][ni], 0, 0, 0);
            acc2[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                bh, __builtin_bit_cast(half8_t, afl[mi]), acc2[mi][ni], 0, 0, 0);
          }
      } else {
#pragma unroll
        for (int mi = 0; mi < MF; ++mi)
#pragma unroll
          for (int ni = 0; ni < NF; ++ni) {
            if constexpr (ES == 2) {
              acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                  __builtin_bit_cast(half8_t, bf[ni]), __builtin_bit_cast(half8_t, af[mi]),
                  acc[mi][ni], 0, 0, 0);
            } else {
              const float4_t av = __builtin_bit_cast(float4_t, af[mi]);
              const float4_t bv = __builtin_bit_cast(float4_t, bf[ni]);
#pragma unroll
              for (int e = 0; e < 4; ++e)
                acc[mi][ni] =
                    __builtin_amdgcn_mfma_f32_16x16x4f32(bv[e], av[e], acc[mi][ni], 0, 0, 0);
            }
          }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // no copy into LDS outlives the block (vmcnt 0)
  if constexpr (SPLIT) {
#pragma unroll
    for (int mi = 0; mi < MF; ++mi)
#pragma unroll
      for (int ni = 0; ni < NF; ++ni)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[mi][ni][r] = fmaf(acc2[mi][ni][r], 1.f / 2048.f, acc[mi][ni][r]);
  }

  // Epilogue: fp32 rows of the segment's output, 4 consecutive columns per lane (a
  // 16-byte store when the row stride and the base allow it), plus the residual when the
  // segment has one (read and written by the same lane, so it may alias the output).
  float* const ybase = sg.y + (size_t)blockIdx.y * p.yslice;
  const bool vec = (sg.ldy & 3) == 0 && ((uintptr_t)ybase & 15) == 0 &&
                   ((uintptr_t)sg.res & 15) == 0;
  // Rows whose stride or base rules out 16-byte stores (the router logits, E + 1 columns):
  // the tile goes through LDS, then consecutive lanes store consecutive columns of a row,
  // in place of 4-byte stores spread over 16 rows per instruction.
  constexpr int LDT = BN + 4;  // row stride of the staged tile (floats)
  if constexpr (BM * LDT * 4 <= NS * SLOT) {
    if (!vec) {
      __syncthreads();  // every wave is past its last read of the ring
      float* so = (float*)lds;
#pragma unroll
      for (int mi = 0; mi < MF; ++mi)
#pragma unroll
        for (int ni = 0; ni < NF; ++ni)
          *(float4_t*)(so + (wm * WM + mi * 16 + j) * LDT + wn * WN + ni * 16 + 4 * q) =
              acc[mi][ni];
      __syncthreads();
      for (int idx = threadIdx.x; idx < BM * BN; idx += NW * 64) {
        const int row = idx / BN, col = idx - row * BN;
        const int m = m0 + row, n = n0 + col;
        if (m < M && n < N) {
          const size_t o = (size_t)m * sg.ldy + n;
          ybase[o] = sg.res ? sg.res[o] + so[row * LDT + col] : so[row * LDT + col];
        }
      }
      return;
    }
  }
#pragma unroll
  for (int mi = 0; mi < MF; ++mi) {
    const int m = m0 + wm * WM + mi * 16 + j;
    if (m >= M) continue;
    float* yrow = ybase + (size_t)m * sg.ldy;
    const float* rrow = sg.res ? sg.res + (size_t)m * sg.ldy : nullptr;
#pragma unroll
    for (int ni = 0; ni < NF; ++ni) {
      const int n = n0 + wn * WN + ni * 16 + 4 * q;
      if (vec && n + 3 < N) {
        float4_t v = acc[mi][ni];
        if (rrow) v += *(const float4_t*)(rrow + n);
        *(float4_t*)(yrow + n) = v;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < N) yrow[n + r] = rrow ? rrow[n + r] + acc[mi][ni][r] : acc[mi][ni][r];
      }
    }
  }
}

template <typename ET, bool SPLIT, int BM, int BN, int WM, int WN, int NS, int OCC>
int launch(GemmArgs& args, const MxGemmSeg* segs, int nseg, int splits, hipStream_t s) {
  args.mblk = mx_ceil_div(args.M, BM);
  long blocks = 0;
  for (int i = 0; i < nseg; ++i) {
    args.seg[i].nblk = mx_ceil_div(segs[i].n, BN);
    blocks += (long)args.seg[i].nblk * args.mblk;
  }
  if (blocks <= 0 || blocks > (1l << 31) - 1 || splits < 1 || splits > 65535)
    return MX_ERR_UNSUPPORTED;
  constexpr int threads = (BM / WM) * (BN / WN) * 64;
  mx_clear_error();
  hipLaunchKernelGGL((k_gemm_nt<ET, SPLIT, BM, BN, WM, WN, NS, OCC>), dim3((unsigned)blocks, splits),
                     dim3(threads), 0, s, args);
  return mx_launch_status();
}

// Shared argument checks; fills args (segments, K, slices) for element size es.
int prepare(GemmArgs& args, const void* a, int M, int K, int es, const MxGemmSeg* segs,
            int nseg, int kslice, long yslice) {
  if (!a || !segs || nseg < 1 || nseg > MX_GEMM_MAX_SEG || M <= 0 || K <= 0 || kslice <= 0)
    return MX_ERR_INVALID;
  const int bke = STAGE_BYTES / es;
  if (K % bke || kslice % bke) return MX_ERR_UNSUPPORTED;  // whole stages only
  if (!mx_aligned16(a)) return MX_ERR_ALIGNMENT;
  if ((long)M * K * es >= (1l << 31)) return MX_ERR_UNSUPPORTED;
  args = GemmArgs{};
  args.a = a;
  args.M = M;
  args.K = K;
  args.kslice = kslice;
  args.yslice = yslice;
  args.nseg = nseg;
  for (int i = 0; i < nseg; ++i) {
    const MxGemmSeg& g = segs[i];
    if (!g.w || !g.y || g.n <= 0 || g.ldy < g.n) return MX_ERR_INVALID;
    if (g.res && kslice != K) return MX_ERR_INVALID;  // a residual needs the whole reduction
    if (!mx_aligned16(g.w)) return MX_ERR_ALIGNMENT;
    if ((long)g.n * K * es >= (1l << 31)) return MX_ERR_UNSUPPORTED;
    args.seg[i].w = g.w;
    args.seg[i].w_lo = g.w_lo;
    args.seg[i].res = g.res;
    args.seg[i].y = g.y;
    args.seg[i].n = g.n;
    args.seg[i].ldy = g.ldy;
  }
  return MX_OK;
}

}  // namespace

#ifndef MX_GEMM_MID
#define MX_GEMM_MID 1  // 256 x 128 tiles for products that fill whole rounds with them
#endif
#ifndef MX_GEMM_TAIL
#define MX_GEMM_TAIL 1  // leftover columns of a partial last round on 128 x 128 tiles
#endif

int mx_gemm_f16(const void* a, int M, int K, const MxGemmSeg* segs, int nseg, hipStream_t s) {
  GemmArgs args;
  MX_TRY(prepare(args, a, M, K, 2, segs, nseg, K, 0));
  long cols = 0;
  for (int i = 0; i < nseg; ++i) cols += segs[i].n;
  // 256 x 256 tiles while they give at least two rounds of blocks on 256 CUs; 128 x 128
  // (four waves, one block per CU with four 32 KiB stage slots: 34 -> 30 us for the k and v
  // projections of the Qwen3-Next 4096-token attention block against two blocks per CU
  // with two slots each) otherwise.
  const long big = (long)mx_ceil_div(M, 256) * mx_ceil_div((int)cols, 256);
  if (big < 512) {
    // 256 x 128 tiles (8 waves of 64 x 64, one block per CU) when they fill whole rounds
    long mid = 0;
    for (int i = 0; i < nseg; ++i) mid += (long)mx_ceil_div(M, 256) * mx_ceil_div(segs[i].n, 128);
    if (MX_GEMM_MID && mid >= 256 && mid % 256 == 0)
      return launch<half_t, false, 256, 128, 64, 64, 3, 1>(args, segs, nseg, 1, s);
    return launch<half_t, false, 128, 128, 64, 64, 4, 1>(args, segs, nseg, 1, s);
  }
  if (MX_GEMM_TAIL && big % 256) {
    // One 256 x 256 block per CU: the blocks past the last whole round would run as a
    // partial round as long as a full one.  The whole rounds take whole 256-column tiles
    // of the segments in order; the columns left over (partial tiles, later segments) go
    // to a second launch on 128 x 128 tiles, which spreads them over all CUs.  Each output
    // element is still computed by one block over the whole reduction.
    int budget = (int)(big / 256 * 256 / mx_ceil_div(M, 256));  // 256-column tiles
    MxGemmSeg head[MX_GEMM_MAX_SEG], tail[MX_GEMM_MAX_SEG];
    int nh = 0, nt = 0;
    for (int i = 0; i < nseg; ++i) {
      const MxGemmSeg& g = segs[i];
      const int take = budget < g.n / 256 ? budget : g.n / 256;
      budget -= take;
      const int n0 = take * 256;
      if (n0 > 0) {
        head[nh] = g;
        head[nh++].n = n0;
      }
      if (n0 < g.n) {
        MxGemmSeg t = g;
        t.w = (const char*)g.w + (size_t)n0 * K * 2;
        t.y = g.y + n0;
        if (g.res) t.res = g.res + n0;
        t.n = g.n - n0;
        tail[nt++] = t;
      }
    }
    if (nh > 0 && nt > 0) {
      GemmArgs ah, at;
      MX_TRY(prepare(ah, a, M, K, 2, head, nh, K, 0));
      MX_TRY(prepare(at, a, M, K, 2, tail, nt, K, 0));
      MX_TRY((launch<half_t, false, 256, 256, 128, 64, 2, 1>(ah, head, nh, 1, s)));
      return launch<half_t, false, 128, 128, 64, 64, 4, 1>(at, tail, nt, 1, s);
    }
  }
  return launch<half_t, false, 256, 256, 128, 64, 2, 1>(args, segs, nseg, 1, s);
}

int mx_gemm_f32_slices(const float* a, int M, int K, const MxGemmSeg* segs, int nseg,
                       int kslice, long yslice, hipStream_t s) {
  GemmArgs args;
  MX_TRY(prepare(args, a, M, K, 4, segs, nseg, kslice, yslice));
  const int splits = mx_ceil_div(K, kslice);
  if (splits > 1 && yslice <= 0) return MX_ERR_INVALID;
  return launch<float, false, 128, 128, 64, 64, 2, 2>(args, segs, nseg, splits, s);
}

int mx_gemm_f16x2_slices(const void* a_hi, const void* a_lo, int M, int K, const MxGemmSeg* segs,
                         int nseg, int kslice, long yslice, hipStream_t s) {
  GemmArgs args;
  MX_TRY(prepare(args, a_hi, M, K, 2, segs, nseg, kslice, yslice));
  if (!a_lo || !mx_aligned16(a_lo)) return a_lo ? MX_ERR_ALIGNMENT : MX_ERR_INVALID;
  for (int i = 0; i < nseg; ++i) {
    if (!segs[i].w_lo) return MX_ERR_INVALID;
    if (!mx_aligned16(segs[i].w_lo)) return MX_ERR_ALIGNMENT;
  }
  args.a_lo = a_lo;
  const int splits = mx_ceil_div(K, kslice);
  if (splits > 1 && yslice <= 0) return MX_ERR_INVALID;
  // 128 x 128 tiles of 8 waves (64 x 32 each), one block per CU (two 64 KiB stage slots).
  return launch<half_t, true, MX_GEMM_SPLIT_BM, MX_GEMM_SPLIT_BN, 64, 32, 2, 1>(args, segs, nseg,
                                                                               splits, s);
}
