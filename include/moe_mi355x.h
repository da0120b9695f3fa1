/*
 * moe_mi355x.h — C ABI of libmoe_mi355x.so, the MI355X (gfx950) MoE-layer hot path.
 *
 * Every entry point returns int: 0 on success, a positive hipError_t code when a HIP
 * runtime call failed, or a negative MX_ERR_* code for argument errors detected on the
 * host.  No entry point throws across the ABI and no hot-path entry point allocates
 * device memory: the caller owns every buffer, including the workspace (or, for
 * mx_moe_forward_noalloc, the library's own per-device scratch array stands in for it).
 *
 * Pointers are plain addresses.  "Device" pointers are hipMalloc'd (or offsets into a
 * hipMalloc'd layer buffer); streams and events are hipStream_t / hipEvent_t passed as
 * void*.  A NULL stream is the legacy default stream.
 *
 * Reference interfaces replaced (haesookimDev/disk-mem-off):
 *   backend shim  -> offload_runtime/backends/rocm_backend.py:33-119 (ROCmBackend over hip-python)
 *   MoE layer     -> offload_runtime/executors/glm4_moe.py:176-240 (GLM4MoeExecutor._moe_mlp_block)
 *                    offload_runtime/executors/qwen3_next.py:273-333 (Qwen3NextExecutor._moe_mlp_block)
 */
#ifndef MOE_MI355X_H
#define MOE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------------------ */
#define MX_OK 0
#define MX_ERR_INVALID (-1)      /* bad argument: null pointer, bad shape, bad enum        */
#define MX_ERR_UNSUPPORTED (-2)  /* valid request this build does not implement           */
#define MX_ERR_WORKSPACE (-3)    /* workspace smaller than mx_moe_workspace_size() says    */
#define MX_ERR_ALIGNMENT (-4)    /* a weight pointer is not 16-byte aligned                */

/* ---- element types ------------------------------------------------------------------ */
#define MX_DT_F32 0
#define MX_DT_F16 1
#define MX_DT_I8 2 /* expert weights only: int8 values + one fp16 scale per output row */

/* ---- router modes -------------------------------------------------------------------
 * MX_ROUTER_REF_SOFTMAX_BIAS : p = softmax(h.Wr^T + b); top-k on p; weights = p at the
 *                              selected ids; optional renorm; x routed_scaling.
 *                              (glm4_moe.py:181-200, what the reference executes)
 * MX_ROUTER_SIGMOID_SELECT_BIAS : s = sigmoid(h.Wr^T); top-k on s + b; weights = s at the
 *                              selected ids (bias for selection only); optional renorm;
 *                              x routed_scaling.  (GLM-4.5/4.7 checkpoint semantics)
 * MX_ROUTER_SOFTMAX          : p = softmax(h.Wr^T); top-k on p; optional renorm; no bias.
 *                              (qwen3_next.py:278-293; pass routed_scaling = 1)
 * Selected ids come out ordered by descending selection key, ties to the lower id.    */
#define MX_ROUTER_REF_SOFTMAX_BIAS 0
#define MX_ROUTER_SIGMOID_SELECT_BIAS 1
#define MX_ROUTER_SOFTMAX 2

/* ---- expert weight layouts ------------------------------------------------------------
 * MX_LAYOUT_ROWS   : nn.Linear row-major [out, in], as the loader packs the layer.
 * MX_LAYOUT_FRAG16 : the same bytes regrouped into 1 KiB fragments, one per (16 output
 *                    rows, KC input columns) block with KC = 64 bytes / element size
 *                    (16 fp32, 32 fp16, 64 int8); fragment (g, c) sits at byte
 *                    (g * in / KC + c) * 1024 and holds, at byte 16 * (16 q + j), the
 *                    KC / 4 elements W[16 g + j][KC c + (KC / 4) q ...].  The expert
 *                    kernels then read every fragment as one contiguous 1 KiB (the
 *                    row-major form costs a DRAM page per 64 bytes in the prefill
 *                    kernel).  Produced on the device by mx_tile_weights; needs
 *                    out % 16 == 0 and in % KC == 0 for every expert matrix.  Scales
 *                    of int8 weights keep their per-row layout.                      */
#define MX_LAYOUT_ROWS 0
#define MX_LAYOUT_FRAG16 1

/* Per-expert weight pointers (device addresses).  gate/up are [inter, hidden] and down is
 * [hidden, inter], nn.Linear row-major ([out, in]) exactly as packed in the layer buffer
 * (loader/huggingface.py:458-591).  For MX_DT_I8 the *_scale pointers give one fp16 scale
 * per output row; dequantised W[o, i] = q[o, i] * scale[o] (quantize.py:44 with zero
 * point 0 and a per-row scale).  For other dtypes the scale pointers are ignored.    */
typedef struct MxExpertPtrs {
  const void* gate;
  const void* up;
  const void* down;
  const void* gate_scale;
  const void* up_scale;
  const void* down_scale;
} MxExpertPtrs;

/* Static description of one MoE block.  Field meanings follow the executor config keys
 * (glm4_moe.py:70-84, qwen3_next.py:105-133).                                         */
typedef struct MxMoeDesc {
  int32_t hidden;          /* H                                                        */
  int32_t inter;           /* I, moe_intermediate_size                                 */
  int32_t shared_inter;    /* I_s of the shared expert; 0 = no shared expert           */
  int32_t n_experts;       /* E, routed experts                                        */
  int32_t top_k;           /* k, num_experts_per_tok (1 <= k <= min(E, 32))             */
  int32_t router_mode;     /* MX_ROUTER_*                                              */
  int32_t norm_topk_prob;  /* 1: w /= (sum(w) + 1e-20)                                 */
  int32_t weight_dtype;    /* expert weights: MX_DT_F32 / MX_DT_F16 / MX_DT_I8         */
  int32_t param_dtype;     /* norm weight, router weight, bias, shared gate: F32 / F16 */
  int32_t has_bias;        /* e_score_correction_bias present                          */
  int32_t has_shared_gate; /* Qwen3-Next shared_expert_gate present                    */
  float routed_scaling;    /* routed_scaling_factor (1.0 for Qwen3-Next)               */
  float eps;               /* rms_norm_eps                                             */
  int32_t weight_layout;   /* MX_LAYOUT_ROWS / MX_LAYOUT_FRAG16 of the expert weights  */
} MxMoeDesc;

/* Device pointers of one layer's MoE tensors. */
typedef struct MxMoeWeights {
  const void* norm_w;           /* post_attention_layernorm.weight [H]                 */
  const void* router_w;         /* mlp.gate.weight [E, H]                              */
  const void* bias;             /* mlp.gate.e_score_correction_bias [E] or NULL        */
  const void* shared_gate_w;    /* mlp.shared_expert_gate.weight [1, H] or NULL        */
  const MxExpertPtrs* experts;  /* device array of E + 1 entries; entry E = shared     */
} MxMoeWeights;

/* Views into a forward workspace (all device pointers), for inspection after a call. */
typedef struct MxMoeViews {
  float* h32;          /* [T, H] rms-normalised activations; not written by a forward   */
                       /* whose router runs on fp16 planes (T >= 65, fp16 / int8        */
                       /* experts, H a multiple of 64): h16 holds them there            */
  void* h16;           /* [T, H] fp16 copy (NULL for MX_DT_F32 weights)                 */
  float* logits;       /* [S, T, E(+1)] router logit partials (S = router_splits)        */
  int32_t router_splits;
  int32_t* topk_ids;   /* [T, k]                                                        */
  float* topk_w;       /* [T, k] routing weights after renorm and scaling              */
  float* shared_w;     /* [T] shared-expert weight (1, or sigmoid gate)                 */
  int32_t* counts;     /* [E] tokens per routed expert                                  */
  int32_t* offsets;    /* [E + 1] exclusive prefix of counts                            */
  int32_t* sorted_tok; /* [T k + T] token of each expert-sorted row (shared rows last)   */
  float* sorted_w;     /* [T k + T] routing weight of each row                          */
  int32_t* pair_pos;   /* [T, k] row of pair (t, j) in the sorted order                 */
  int32_t* g_expert;   /* [E + 1] expert of group g (group 0 = shared when present)     */
  int32_t* g_start;    /* [E + 1] first sorted row of group g                           */
  int32_t* g_count;    /* [E + 1] rows of group g                                       */
  int32_t* n_groups;   /* [1]                                                           */
  int32_t* mt_group;   /* [max m-tiles] group of each m-tile                            */
  int32_t* mt_row0;    /* [max m-tiles] first row of the m-tile within its group        */
  int32_t* n_mtiles;   /* [1]                                                           */
  int32_t m_blk;       /* rows per m-tile                                               */
  void* act;           /* [T k + T, max(I, I_s)] silu(gate) * up                        */
  void* y;             /* [T k + T, H] weighted expert outputs: fp32, or fp16 when      */
                       /* m_blk is 128 (fp16 / int8 experts, T >= 65)                   */
} MxMoeViews;

/* Static description of the device. */
typedef struct MxDeviceInfo {
  char name[256];
  char arch[64];
  int32_t cu_count;
  int32_t clock_khz;
  int32_t mem_clock_khz;
  int32_t mem_bus_width;
  int64_t total_mem;
  int32_t l2_bytes;
  int32_t lds_per_block;
} MxDeviceInfo;

/* =================================================================================== *
 * Backend shim.  Replaces the hip-python calls of ROCmBackend                          *
 * (offload_runtime/backends/rocm_backend.py:46-119).                                   *
 * =================================================================================== */
const char* mx_error_string(int status);                       /* no counterpart: diagnostics */
int mx_get_device_count(int32_t* count);                       /* no counterpart: probe       */
int mx_device_info(int32_t device, MxDeviceInfo* info);        /* no counterpart: bench peaks */
int mx_set_device(int32_t device);                             /* rocm_backend.py:49  hipSetDevice */
int mx_device_sync(void);                                      /* no counterpart: teardown    */
int mx_malloc(void** ptr, size_t nbytes);                      /* rocm_backend.py:81-83 hipMalloc */
int mx_free(void* ptr);                                        /* rocm_backend.py:85-86 hipFree */
int mx_host_malloc(void** ptr, size_t nbytes);                 /* rocm_backend.py:63-66 hipHostMalloc(n, 0) */
int mx_host_free(void* ptr);                                   /* rocm_backend.py:68-70 hipHostFree */
int mx_memcpy_h2d_async(void* dst, const void* src, size_t nbytes, void* stream); /* rocm_backend.py:88-95 */
int mx_memcpy_d2h_async(void* dst, const void* src, size_t nbytes, void* stream); /* rocm_backend.py:97-104 */
int mx_memcpy_d2d_async(void* dst, const void* src, size_t nbytes, void* stream); /* no counterpart: device copies */
int mx_stream_create(void** stream, int32_t nonblocking);      /* rocm_backend.py:72-76 hipStreamCreateWithFlags */
int mx_stream_destroy(void* stream);                           /* rocm_backend.py:78-79 */
int mx_stream_sync(void* stream);                              /* rocm_backend.py:118-119 */
int mx_event_create(void** event, int32_t timing);             /* rocm_backend.py:108 hipEventCreateWithFlags */
int mx_event_record(void* event, void* stream);                /* rocm_backend.py:109 hipEventRecord */
int mx_event_wait(void* stream, void* event);                  /* rocm_backend.py:115-116 hipStreamWaitEvent */
int mx_event_sync(void* event);                                /* no counterpart: host wait   */
int mx_event_query(void* event, int32_t* done);                /* no counterpart: poll        */
int mx_event_destroy(void* event);                             /* rocm_backend.py:112-113 */
int mx_event_elapsed_ms(float* ms, void* start, void* end);    /* no counterpart: timing      */

/* =================================================================================== *
 * MoE layer.  One call = GLM4MoeExecutor._moe_mlp_block (glm4_moe.py:176-240) or       *
 * Qwen3NextExecutor._moe_mlp_block (qwen3_next.py:273-333) on device-resident data:    *
 *   out = x + sum_j w[t,j] * SwiGLU_{id[t,j]}(h[t]) + shared_w[t] * SwiGLU_shared(h[t]) *
 *   with h = rms_norm(x).  x and out are fp32 [T, H] device buffers (may not alias).    *
 * =================================================================================== */
int mx_moe_workspace_size(const MxMoeDesc* desc, int32_t tokens, size_t* nbytes);
int mx_moe_views(const MxMoeDesc* desc, int32_t tokens, void* workspace, MxMoeViews* views);
int mx_moe_forward(const MxMoeDesc* desc, const MxMoeWeights* weights, const float* x,
                   float* out, int32_t tokens, void* workspace, size_t workspace_bytes,
                   void* stream);
/* Same as mx_moe_forward, and records events[i] on the stream before stage i and
 * events[MX_N_STAGES] after the last stage (n_events must be MX_N_STAGES + 1).
 * Stages: 0 rmsnorm, 1 router logits, 2 router top-k, 3 dispatch, 4 expert gate/up,
 * 5 expert down, 6 combine.                                                           */
#define MX_N_STAGES 7
/* Stages [stage_begin, stage_end) of mx_moe_forward on the same workspace: the router part
 * (0..3) and the expert part (4..6) can run as two calls, with the routed experts' weights
 * copied in between.  Splits the reference's _moe_mlp_block (glm4_moe.py:176-240) at the
 * point where the active expert set (glm4_moe.py:206, set(topk_indices)) is known, which
 * the expert-granular transfer of an offloaded layer needs.                            */
#define MX_STAGE_ROUTE_END 4
int mx_moe_forward_stages(const MxMoeDesc* desc, const MxMoeWeights* weights, const float* x,
                          float* out, int32_t tokens, void* workspace, size_t workspace_bytes,
                          int32_t stage_begin, int32_t stage_end, void* stream);
int mx_moe_forward_profiled(const MxMoeDesc* desc, const MxMoeWeights* weights,
                            const float* x, float* out, int32_t tokens, void* workspace,
                            size_t workspace_bytes, void* stream, void* const* events,
                            int32_t n_events);

/* No counterpart in the reference.  mx_moe_forward for callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  The same computation, without the workspace arguments: the stages run out of
 * a scratch array of MX_NOALLOC_MAX_WORKSPACE bytes that the library holds on every device
 * it runs on until the process ends.  Nothing is allocated and no memset is issued.
 * Returns MX_ERR_WORKSPACE when mx_moe_workspace_size(desc, tokens) exceeds that size;
 * size batches from that function, not from the token count alone (from 65 tokens the
 * prefill-path buffers join the workspace).  With 16 MiB: GLM-4.7 shapes up to 64 tokens
 * (62 with fp32 experts), Qwen3-Next shapes up to 83 (108 with fp32 experts).  Every call on
 * one device shares that device's scratch: calls that overlap on one device (other
 * streams, other host threads) race and must be serialised by the caller; calls on one
 * stream are ordered by it.                                                            */
#define MX_NOALLOC_MAX_WORKSPACE (16u << 20)
int mx_moe_forward_noalloc(const MxMoeDesc* desc, const MxMoeWeights* weights, const float* x,
                           float* out, int32_t tokens, void* stream);

/* ---- individual stages (each replaces the reference lines cited) -------------------- */

/* h32 = w * (x / sqrt(mean(x^2) + eps)), optional fp16 copy h16.  _common.py:73-75. */
int mx_rmsnorm(const float* x, const void* norm_w, int32_t param_dtype, float eps,
               int32_t tokens, int32_t hidden, float* h32, void* h16, void* stream);

/* Router logit partials: logits[s, t, e] = sum over the s-th slice of H of
 * h32[t, :] * Wr[e, :], for e < E; e == E (if shared_gate_w) uses the shared gate row.
 * glm4_moe.py:181, qwen3_next.py:278 and :328.                                        */
int mx_router_logits(const float* h32, const void* router_w, const void* shared_gate_w,
                     int32_t param_dtype, int32_t tokens, int32_t hidden, int32_t n_experts,
                     int32_t splits, float* logits, void* stream);

/* Bias, softmax/sigmoid, top-k, renorm, scaling.  glm4_moe.py:182-200,
 * qwen3_next.py:279-293; shared_w[t] = sigmoid(gate logit) (qwen3_next.py:327-329) or 1. */
int mx_router_topk(const float* logits, int32_t splits, const void* bias, int32_t param_dtype,
                   int32_t tokens, int32_t n_experts, int32_t top_k, int32_t router_mode,
                   int32_t norm_topk_prob, float routed_scaling, int32_t has_shared_gate,
                   int32_t* topk_ids, float* topk_w, float* shared_w, void* stream);

/* Histogram / prefix-sum dispatch: per-expert counts and offsets, the expert-sorted row
 * order (ascending token inside each expert, as h[token_mask] gathers at
 * glm4_moe.py:206-215), its inverse pair_pos, the active-group table (shared group first
 * when has_shared) and the m-tile list with m_blk rows per tile.                      */
int mx_dispatch(const int32_t* topk_ids, const float* topk_w, const float* shared_w,
                int32_t tokens, int32_t top_k, int32_t n_experts, int32_t has_shared,
                int32_t m_blk, int32_t* counts, int32_t* offsets, int32_t* sorted_tok,
                float* sorted_w, int32_t* pair_pos, int32_t* g_expert, int32_t* g_start,
                int32_t* g_count, int32_t* n_groups, int32_t* mt_group, int32_t* mt_row0,
                int32_t* n_mtiles, void* stream);

/* The same tables built by three launches (per-chunk counts and ranks over many
 * workgroups, one scan workgroup, a placement pass): the large-batch form of mx_dispatch
 * (glm4_moe.py:206-215).  `scratch` holds mx_dispatch_scratch_size() bytes; n_experts
 * up to 1365 (MX_ERR_UNSUPPORTED above).                                               */
int mx_dispatch_scratch_size(int32_t tokens, int32_t top_k, int32_t n_experts, size_t* nbytes);
int mx_dispatch_chunked(const int32_t* topk_ids, const float* topk_w, const float* shared_w,
                        int32_t tokens, int32_t top_k, int32_t n_experts, int32_t has_shared,
                        int32_t m_blk, void* scratch, int32_t* counts, int32_t* offsets,
                        int32_t* sorted_tok, float* sorted_w, int32_t* pair_pos,
                        int32_t* g_expert, int32_t* g_start, int32_t* g_count,
                        int32_t* n_groups, int32_t* mt_group, int32_t* mt_row0,
                        int32_t* n_mtiles, void* stream);

/* Grouped expert products over the dispatch tables (glm4_moe.py:218-224, :234-237):
 * gate/up: act[row] = silu(A[tok(row)] . Wg^T) * (A[tok(row)] . Wu^T)
 * down:    y[row]   = sorted_w[row] * (act[row] . Wd^T)
 * A is h16 (fp16/int8 weights) or h32 (fp32 weights).                                 */
int mx_expert_gate_up(const MxMoeDesc* desc, const MxExpertPtrs* experts, int32_t tokens,
                      const void* a, const int32_t* sorted_tok, const int32_t* g_expert,
                      const int32_t* g_start, const int32_t* g_count, const int32_t* mt_group,
                      const int32_t* mt_row0, const int32_t* n_mtiles, int32_t m_blk,
                      void* act, void* stream);
int mx_expert_down(const MxMoeDesc* desc, const MxExpertPtrs* experts, int32_t tokens,
                   const void* act, const float* sorted_w, const int32_t* g_expert,
                   const int32_t* g_start, const int32_t* g_count, const int32_t* mt_group,
                   const int32_t* mt_row0, const int32_t* n_mtiles, int32_t m_blk, float* y,
                   void* stream);

/* out[t] = x[t] + sum_j y[pair_pos[t, j]] + (has_shared ? y[T k + t] : 0).
 * glm4_moe.py:227-231, :238, :240.                                                    */
int mx_combine(const float* x, const float* y, const int32_t* pair_pos, int32_t tokens,
               int32_t hidden, int32_t top_k, int32_t has_shared, float* out, void* stream);

/* ---- synthetic data and offline quantisation (bench / loader plumbing) -------------- */

/* dst[i] = std * N_i, i in [0, n), where N_i is normal number (offset + i) of the
 * counter-based stream (seed, stream_id): SplitMix64 of two counters -> Box-Muller.
 * dtype MX_DT_F32 or MX_DT_F16.  Matches moe_mi355x/gen.py element for element (up to
 * one ulp of the libm used for log/cos).                                             */
int mx_fill_normal(void* dst, int32_t dtype, size_t n, uint64_t seed, uint64_t stream_id,
                   uint64_t offset, float std, void* stream);

/* Per-row symmetric int8: scale[r] = fp16(max|W[r,:]| / 127) (1 for an all-zero row),
 * q[r, c] = clamp(rint(W[r, c] / float(scale[r])), -127, 127).  W is fp32 or fp16
 * [rows, cols] on the device; q int8 [rows, cols]; scale fp16 [rows].                */
int mx_quantize_rows_i8(const void* w, int32_t w_dtype, int32_t rows, int32_t cols, int8_t* q,
                        void* scale, void* stream);

/* Re-layout of one expert matrix [rows, cols] of weight_dtype from MX_LAYOUT_ROWS (src)
 * to MX_LAYOUT_FRAG16 (dst); dst and src must not overlap, both 16-byte aligned;
 * rows % 16 == 0 and cols % KC == 0 (MX_ERR_UNSUPPORTED otherwise).  No counterpart in
 * the reference, whose expert products read the loader layout directly
 * (glm4_moe.py:222-224): it prepares a bound layer for the prefill kernel.           */
int mx_tile_weights(void* dst, const void* src, int32_t rows, int32_t cols,
                    int32_t weight_dtype, void* stream);

/* =================================================================================== *
 * Qwen3-Next linear-attention (Gated DeltaNet) block: Qwen3NextExecutor._linear_attn_block
 * (offload_runtime/executors/qwen3_next.py:207-269) with its helpers _softplus (:27-28),
 * _causal_conv1d (:35-53) and _gated_delta_rule_recurrence (:56-95):
 *   h = rms_norm(x);  [q|k|v|z] = h W_qkvz^T;  [q|k|v] = silu(causal_conv1d([q|k|v]))
 *   [b|a] = h W_ba^T;  beta = sigmoid(b);  g = -exp(A_log) softplus(a + dt_bias)
 *   per head: S_t = exp(g_t) S_{t-1} + v_t (beta_t k_t)^T,  o_t = S_t q_t  (S_0 = 0)
 *   out = x + (rms_norm(o) * silu(z)) W_out^T
 * The reference reshapes q and k with the value-head count, so it runs only with as
 * many key heads as value heads; n_heads is that count.  The state starts at zero on
 * every call (the reference keeps no recurrent state between calls).
 * =================================================================================== */
typedef struct MxLinearAttnDesc {
  int32_t hidden;       /* H                                                            */
  int32_t n_heads;      /* linear_num_key_heads == linear_num_value_heads               */
  int32_t head_dim_k;   /* linear_key_head_dim: a power of two, 4..512                  */
  int32_t head_dim_v;   /* linear_value_head_dim                                        */
  int32_t conv_kernel;  /* linear_conv_kernel_dim, 1..16                                */
  int32_t weight_dtype; /* in_proj_qkvz / in_proj_ba / out_proj: F32 / F16 / I8 (+ scales) */
  int32_t param_dtype;  /* norms, conv1d, A_log, dt_bias: F32 / F16                     */
  float eps;            /* rms_norm_eps                                                 */
} MxLinearAttnDesc;

typedef struct MxLinearAttnWeights {
  const void* norm_w;     /* input_layernorm.weight [H]                                 */
  const void* qkvz_w;     /* linear_attn.in_proj_qkvz.weight [2 n dk + 2 n dv, H]       */
  const void* qkvz_scale; /* fp16 per row for MX_DT_I8, else NULL                       */
  const void* ba_w;       /* linear_attn.in_proj_ba.weight [n dk + n, H]                */
  const void* ba_scale;
  const void* conv_w;     /* linear_attn.conv1d.weight [2 n dk + n dv, (1,) K]          */
  const void* a_log;      /* linear_attn.A_log [n]                                      */
  const void* dt_bias;    /* linear_attn.dt_bias [n]                                    */
  const void* out_norm_w; /* linear_attn.norm.weight [n dv]                             */
  const void* out_w;      /* linear_attn.out_proj.weight [H, n dv]                      */
  const void* out_scale;
} MxLinearAttnWeights;

/* Views into a linear-attention workspace (device pointers), for inspection.          */
typedef struct MxLinearAttnViews {
  float* h32;    /* [T, H] rms_norm(x)                                                  */
  void* h16;     /* [T, H] fp16 copy (NULL for F32 weights)                             */
  float* qkvz;   /* [T, 2 n dk + 2 n dv] h W_qkvz^T                                     */
  float* ba;     /* [T, n dk + n] h W_ba^T                                              */
  float* q;      /* [T, n dk] silu(conv(q))                                             */
  float* kb;     /* [T, n dk] sigmoid(b) * silu(conv(k))                                */
  float* v;      /* [T, n dv] silu(conv(v))                                             */
  float* decay;  /* [T, n] exp(g)                                                       */
  float* o;      /* [T, n dv] recurrence output                                         */
  void* act;     /* [T, n dv] rms_norm(o) * silu(z), fp16 (fp32 for F32 weights)        */
  float* y;      /* [T, H] act W_out^T; not written on the fused-GEMM path (below)      */
} MxLinearAttnViews;

/* Stages: rmsnorm, qkvz, ba, conv+gates, scan, gated norm, out, residual.  With fp16
 * weights, T >= 65 and H (for qkvz / ba) or n dv (for out) a multiple of 64 the
 * projections run on the dense MFMA GEMM: ba is computed in the qkvz launch (stage 2 is
 * then empty, and the _profiled events report ba's time under qkvz), and out = x +
 * act W_out^T is formed in the out launch's epilogue (stage 7 is empty and the view y is
 * not written).                                                                        */
#define MX_LA_N_STAGES 8

int mx_linear_attn_workspace_size(const MxLinearAttnDesc* desc, int32_t tokens,
                                  size_t* nbytes);
int mx_linear_attn_views(const MxLinearAttnDesc* desc, int32_t tokens, void* workspace,
                         MxLinearAttnViews* views);
/* out may alias x (the block reads x first, then writes out element by element). */
int mx_linear_attn_forward(const MxLinearAttnDesc* desc, const MxLinearAttnWeights* weights,
                           const float* x, float* out, int32_t tokens, void* workspace,
                           size_t workspace_bytes, void* stream);
/* Same, with an event recorded before each of the MX_LA_N_STAGES stages and at the end. */
int mx_linear_attn_forward_profiled(const MxLinearAttnDesc* desc,
                                    const MxLinearAttnWeights* weights, const float* x,
                                    float* out, int32_t tokens, void* workspace,
                                    size_t workspace_bytes, void* stream, void* const* events,
                                    int32_t n_events);
/* =================================================================================== *
 * Qwen3-Next gated full-attention block: Qwen3NextExecutor._full_attn_block
 * (offload_runtime/executors/qwen3_next.py:161-205) with rope / partial_rope /
 * rms_norm_no_weight / repeat_kv (offload_runtime/executors/_common.py:105-153):
 *   h = rms_norm(x);  [q | gate] = h W_q^T (halves);  k = h W_k^T;  v = h W_v^T
 *   per head: q = rms_norm_no_weight(q) * q_norm (if given), k likewise; rotate-half RoPE
 *   on the first rotary_dim dims at positions 0 .. T-1
 *   attn = softmax((q k^T) / sqrt(head_dim) + causal mask) v   (k, v heads repeated)
 *   out = x + (attn * sigmoid(gate)) W_o^T
 * Attention runs in fp32 (MFMA 16x16x4 f32).  No KV cache: every call attends over its
 * own T tokens, as in the reference.
 * =================================================================================== */
typedef struct MxFullAttnDesc {
  int32_t hidden;       /* H                                                            */
  int32_t n_heads;      /* num_attention_heads                                          */
  int32_t n_kv_heads;   /* num_key_value_heads (divides n_heads)                        */
  int32_t head_dim;     /* head_dim: a multiple of 4, <= 256                            */
  int32_t rotary_dim;   /* int(head_dim * partial_rotary_factor), even, <= head_dim     */
  int32_t weight_dtype; /* q / k / v / o projections: F32 / F16 / I8 (+ row scales)     */
  int32_t param_dtype;  /* input_layernorm, q_norm, k_norm: F32 / F16                   */
  double rope_theta;    /* rope_theta                                                   */
  float eps;            /* rms_norm_eps                                                 */
} MxFullAttnDesc;

typedef struct MxFullAttnWeights {
  const void* norm_w;   /* input_layernorm.weight [H]                                   */
  const void* q_w;      /* self_attn.q_proj.weight [2 n_heads head_dim, H]              */
  const void* q_scale;  /* fp16 per row for MX_DT_I8, else NULL                         */
  const void* k_w;      /* self_attn.k_proj.weight [n_kv_heads head_dim, H]             */
  const void* k_scale;
  const void* v_w;      /* self_attn.v_proj.weight [n_kv_heads head_dim, H]             */
  const void* v_scale;
  const void* o_w;      /* self_attn.o_proj.weight [H, n_heads head_dim]                */
  const void* o_scale;
  const void* q_norm_w; /* self_attn.q_norm.weight [head_dim] or NULL (no qk norm)      */
  const void* k_norm_w; /* self_attn.k_norm.weight [head_dim] or NULL                   */
} MxFullAttnWeights;

typedef struct MxFullAttnViews {
  float* h32;  /* [T, H] rms_norm(x)                                                    */
  void* h16;   /* [T, H] fp16 copy (NULL for F32 weights)                               */
  float* qg;   /* [T, 2 n_heads head_dim] [q | gate]; q normalised and rotated in place */
  float* k;    /* [T, n_kv_heads head_dim] k, normalised and rotated in place           */
  float* v;    /* [T, n_kv_heads head_dim]                                              */
  void* act;   /* [T, n_heads head_dim] attn * sigmoid(gate), fp16 (fp32 for F32 weights) */
  float* y;    /* [T, H] act W_o^T; not written on the fused-GEMM path (below)          */
} MxFullAttnViews;

/* Stages: rmsnorm, q, k, v, qk-norm+rope, attention, o, residual.  With fp16 weights,
 * T >= 65 and H (for q / k / v) or n_heads head_dim (for o) a multiple of 64 the
 * projections run on the dense MFMA GEMM: k and v are computed in the q launch (stages 2
 * and 3 are then empty, and the _profiled events report their time under q), and out =
 * x + act W_o^T is formed in the o launch's epilogue (stage 7 is empty and the view y is
 * not written).                                                                        */
#define MX_FA_N_STAGES 8

int mx_full_attn_workspace_size(const MxFullAttnDesc* desc, int32_t tokens, size_t* nbytes);
int mx_full_attn_views(const MxFullAttnDesc* desc, int32_t tokens, void* workspace,
                       MxFullAttnViews* views);
/* out may alias x. */
int mx_full_attn_forward(const MxFullAttnDesc* desc, const MxFullAttnWeights* weights,
                         const float* x, float* out, int32_t tokens, void* workspace,
                         size_t workspace_bytes, void* stream);
int mx_full_attn_forward_profiled(const MxFullAttnDesc* desc, const MxFullAttnWeights* weights,
                                  const float* x, float* out, int32_t tokens, void* workspace,
                                  size_t workspace_bytes, void* stream, void* const* events,
                                  int32_t n_events);

/* The recurrence alone (qwen3_next.py:56-95 with beta * k formed): q, kb [T, n dk],
 * v, o [T, n dv], decay [T, n] = exp(g), all fp32 on the device.  Token-sequential.     */
int mx_gated_delta_scan(const float* q, const float* kb, const float* v, const float* decay,
                        int32_t tokens, int32_t n_heads, int32_t head_dim_k,
                        int32_t head_dim_v, float* o, void* stream);
/* The same recurrence (qwen3_next.py:56-95) with a caller workspace: from 64 tokens, for
 * key and value heads of 64 or 128, in chunks of 64 tokens on fp32 MFMA (one pass over the
 * chunks per head carrying the state through the chunks' increments, then every chunk's
 * output in parallel from the state it starts from); other shapes and shorter inputs run
 * the token-sequential scan.  The workspace (16-byte aligned) holds per-chunk decay
 * coefficients and the fp32 state each chunk after the first starts from
 * (mx_gated_delta_scan_workspace_size bytes, about T / 64 * n * dk * dv * 4; 0 when the
 * sequential scan runs); a smaller one gives MX_ERR_WORKSPACE.  The linear-attention
 * block uses this form inside its own workspace.                                       */
int mx_gated_delta_scan_workspace_size(int32_t tokens, int32_t n_heads, int32_t head_dim_k,
                                       int32_t head_dim_v, size_t* nbytes);
int mx_gated_delta_scan_ws(const float* q, const float* kb, const float* v,
                           const float* decay, int32_t tokens, int32_t n_heads,
                           int32_t head_dim_k, int32_t head_dim_v, float* o, void* workspace,
                           size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_MI355X_H */
