// Declarations shared between the translation units of libmoe_mi355x.so (not exported).
#pragma once

#include <hip/hip_runtime.h>

#include "moe_mi355x.h"

// Number of H-slices the router logit launch uses for this shape (weight_dtype of the MoE
// block, or -1 for the stand-alone mx_router_logits).
int mx_router_splits_for(int tokens, int hidden, int n_experts, int has_shared_gate,
                         int param_dtype, int weight_dtype);
// Whether the MoE block's router runs on the split-plane GEMM (its RMSNorm then also
// writes the low plane of h16, and its workspace holds the router rows' planes).
bool mx_router_on_split(int tokens, int hidden, int e1, int weight_dtype);
size_t mx_router_split_bytes(int hidden, int e1);
// Router logit partials from the planes h16 / h16lo and the router rows' planes in
// `wsplit` (mx_router_split_bytes), all written by the block's RMSNorm launch.
int mx_router_logits_split(const void* h16, const void* h16lo, const void* router_w,
                           const void* shared_gate_w, int param_dtype, int tokens, int hidden,
                           int n_experts, int splits, void* wsplit, float* logits, hipStream_t s);
// Rows and columns per block of mx_gemm_f16x2_slices.
#define MX_GEMM_SPLIT_BM 128
#define MX_GEMM_SPLIT_BN 128

// Upper bound of the m-tile list for `tokens` tokens at m_blk rows per tile.
int mx_max_mtiles(int tokens, int top_k, int n_experts, int has_shared, int m_blk);

// Rows per m-tile the expert kernels use for `tokens` tokens.
int mx_m_blk_for(int tokens, int weight_dtype);

// RMSNorm launch (vectorised when the row fits the register tile).
// What the RMSNorm launch writes for the split-plane router GEMM: the router rows' fp16
// planes [E, H] (hi, lo) and, with a shared-expert gate row, that row's logit per token
// (an fp32 dot product with h, into column E of logit slice 0; 0 into the other slices).
struct MxRouterSplitW {
  const void* wr;   // router rows [E, H]
  int pdt;
  int E;
  _Float16* whi;
  _Float16* wlo;
  const void* wsg;  // shared-expert gate row [H] or null
  float* gate_out;  // logits + E: row stride gate_ld, slice stride gate_slice
  int gate_ld;
  long gate_slice;
  int S;
};
// The planes' place in a workspace region of mx_router_split_bytes, and the gate logit's
// place in the logit slices [S, T, E + 1].
MxRouterSplitW mx_router_split_planes(const void* router_w, const void* shared_gate_w,
                                      int param_dtype, int n_experts, int hidden, int tokens,
                                      int splits, void* wsplit, float* logits);
int mx_rmsnorm_launch(const float* x, const void* norm_w, int param_dtype, float eps, int tokens,
                      int hidden, float* h32, void* h16, hipStream_t s, void* h16lo = nullptr,
                      const MxRouterSplitW* rsw = nullptr);

// Decode router (T <= 64): RMSNorm + logits kernel, then a single-workgroup
// top-k/dispatch kernel.  mx_router_decode_ok tells whether the shape and the pointer
// alignment fit it; the launch returns MX_ERR_UNSUPPORTED otherwise.
bool mx_router_decode_ok(const MxMoeDesc* d, const MxMoeWeights* w, int T, const float* x);
// With select_later the top-k/dispatch launch is left out (the one-token gate/up launch
// selects instead; mx_one_token_select_ok).
int mx_router_decode_launch(const MxMoeDesc* d, const MxMoeWeights* w, int T, const float* x,
                            float* h32, void* h16, float* logits, int* ids, float* tw,
                            float* shared_w, int m_blk, int* counts, int* offsets,
                            int* sorted_tok, float* sorted_w, int* pair_pos, int* g_expert,
                            int* g_start, int* g_count, int* n_groups, int* mt_group,
                            int* mt_row0, int* n_mtiles, hipStream_t s,
                            bool select_later = false);

// A one-token batch whose experts are selected inside the gate/up launch (replacing the
// decode top-k/dispatch launch; E <= MX_SEL_MAX_E): the router logits and routing
// configuration, and the selection and dispatch tables the launch writes for the later
// stages.
#ifndef MX_SEL_MAX_E
#define MX_SEL_MAX_E 512
#endif
struct MxOneTokenSelect {
  const float* logits;  // [E1] router logits of the token
  const void* bias;
  int pdt, E1, k, mode, norm, has_seg, has_shared;
  float scaling;
  int* ids;
  float* tw;
  float* shared_w;
  int* counts;
  int* offsets;
  int* sorted_tok;
  float* sorted_w;
  int* pair_pos;
  int* g_expert;
  int* g_start;
  int* g_count;
  int* n_groups;
  int* mt_group;
  int* mt_row0;
  int* n_mtiles;
};
// mx_expert_down with the y rows as fp16 when y16 (the prefill kernel, m_blk 128, only; the
// combine then reads them with mx_combine_rows(..., y16 = true)).
int mx_expert_down_rows(const MxMoeDesc* desc, const MxExpertPtrs* experts, int tokens,
                        const void* act, const float* sorted_w, const int* g_expert,
                        const int* g_start, const int* g_count, const int* mt_group,
                        const int* mt_row0, const int* n_mtiles, int m_blk, void* y, bool y16,
                        hipStream_t stream);
int mx_combine_rows(const float* x, const void* y, const int32_t* pair_pos, int tokens,
                    int hidden, int top_k, int has_shared, float* out, bool y16, hipStream_t s);
bool mx_one_token_select_ok(const MxMoeDesc* d);
int mx_expert_gate_up_select(const MxMoeDesc* desc, const MxExpertPtrs* experts, const void* a,
                             void* act, const MxOneTokenSelect& sp, hipStream_t s);

// Single-group tables for dense products on the grouped-GEMM kernels (device pointers).
struct MxDenseTables {
  const int* g_expert;
  const int* g_start;
  const int* g_count;
  const int* mt_group;
  const int* mt_row0;
  const int* n_mtiles;
  const float* ones;
  int m_blk;
};

// y[T, N] = a[T, K] W[N, K]^T through the down-projection kernels; W (and its int8 row
// scales) is entry->down (->down_scale).  a is fp32 for MX_DT_F32 weights, else fp16.
int mx_dense_linear(int wdt, int tiled, const MxExpertPtrs* entry, const MxDenseTables& tab,
                    int T, int N, int K, const void* a, float* y, hipStream_t s);

// Dense GEMM on MFMA (mx_dense_gemm.hip): y_s[M, N_s] (fp32, row stride ldy_s) =
// a[M, K] W_s[N_s, K]^T for up to MX_GEMM_MAX_SEG weight matrices sharing a.  The reduction
// runs in stages of MX_GEMM_STAGE_BYTES per row, so K (and a slice length) must be a
// multiple of MX_GEMM_KMULT_F16 columns for fp16 operands, MX_GEMM_KMULT_F32 for fp32.
#define MX_GEMM_MAX_SEG 3
#define MX_GEMM_STAGE_BYTES 128
#define MX_GEMM_KMULT_F16 (MX_GEMM_STAGE_BYTES / 2)
#define MX_GEMM_KMULT_F32 (MX_GEMM_STAGE_BYTES / 4)
struct MxGemmSeg {
  const void* w;  // [n, K] row-major (16-byte aligned), element type of a
  float* y;       // [M, ldy] fp32
  int n;
  int ldy;
  const void* w_lo = nullptr;  // mx_gemm_f16x2_slices: the low fp16 plane of w
  const float* res = nullptr;  // mx_gemm_f16: y = res + a W^T (res [M, ldy], may alias y)
};
// fp16 a and W.
int mx_gemm_f16(const void* a, int M, int K, const MxGemmSeg* segs, int nseg, hipStream_t s);
// fp32 a and W, full fp32 products; the reduction is cut into slices of kslice columns
// (a multiple of MX_GEMM_KMULT_F32) and slice z writes its partial sums at y_s + z * yslice.
int mx_gemm_f32_slices(const float* a, int M, int K, const MxGemmSeg* segs, int nseg,
                       int kslice, long yslice, hipStream_t s);
// fp32 operands as two fp16 planes each, x = hi + 2^-11 lo (hi = fp16(x), lo = fp16((x -
// hi) 2^11)): y = a_hi w_hi + 2^-11 (a_hi w_lo + a_lo w_hi), fp32 sums; kslice a multiple
// of MX_GEMM_KMULT_F16, slices as mx_gemm_f32_slices.
int mx_gemm_f16x2_slices(const void* a_hi, const void* a_lo, int M, int K, const MxGemmSeg* segs,
                         int nseg, int kslice, long yslice, hipStream_t s);

// Workspace pieces of the dense projections of an attention block (device pointers):
// expert-table entries (one per projection), single-group m-tile tables and ones[T] for
// the grouped-GEMM kernels.  Long inputs with fp16 weights run on mx_gemm_f16 instead.
#define MX_DENSE_GEMM_MIN_TOKENS 65
#define MX_DENSE_MAX_ENT 4
struct MxDenseEntries {
  MxExpertPtrs e[MX_DENSE_MAX_ENT];  // e[i].down / down_scale = projection i's weights
};
struct MxDenseWork {
  MxExpertPtrs* entries;
  int* tabs;  // g_expert, g_start, g_count, n_mtiles
  int* mt_group;
  int* mt_row0;
  float* ones;
  int m_blk, n_mt, n_ent;
};
size_t mx_dense_work_bytes(int T, int weight_dtype, int n_ent);
void mx_dense_work_carve(char* base, int T, int weight_dtype, int n_ent, MxDenseWork* w);
// Writes the table entries and m-tile tables (one small launch per block call).
int mx_dense_setup(const MxDenseWork& w, const MxDenseEntries& ents, int T, hipStream_t s);
// Whether projections of T tokens with these weights and reduction length K run on
// mx_gemm_f16 (fp16 weights, long inputs, K a multiple of its stage width).
static inline bool mx_dense_on_gemm(int wdt, int T, int K) {
  return wdt == MX_DT_F16 && T >= MX_DENSE_GEMM_MIN_TOKENS && K % MX_GEMM_KMULT_F16 == 0;
}
// y[T, N] = a[T, K] W^T with W = projection `ent` (wmat, its weights, for mx_gemm_f16).
int mx_project(const MxDenseWork& w, int ent, int wdt, const void* wmat, int T, int N, int K,
               const void* a, float* y, hipStream_t s);
// Chunked gated recurrence on fp32 MFMA (mx_la_chunk.hip) for key / value heads of 64 or
// 128, with a 16-byte aligned workspace of mx_la_chunk_ws_bytes (0: shape not supported;
// per-chunk decay coefficients and the state every chunk after the first starts from);
// MX_ERR_UNSUPPORTED for other shapes (the caller then runs the token-sequential scan).
size_t mx_la_chunk_ws_bytes(int T, int n, int dk, int dv);
int mx_la_chunked_scan(const float* q, const float* kb, const float* v, const float* decay,
                       int T, int n, int dk, int dv, float* o, void* ws, hipStream_t s);
