// One MoE block on the device: workspace layout and the stage sequence
//   rmsnorm -> router logits -> router top-k -> dispatch -> expert gate/up -> expert down
//   -> combine,
// i.e. GLM4MoeExecutor._moe_mlp_block (offload_runtime/executors/glm4_moe.py:176-240) and
// Qwen3NextExecutor._moe_mlp_block (offload_runtime/executors/qwen3_next.py:273-333).
// Everything runs on the caller's stream out of the caller's workspace; nothing is
// allocated here.
#include <atomic>
#include <mutex>

#include "mx_common.h"
#include "mx_internal.h"
#include "mx_dispatch_dev.h"

// Workspace of mx_moe_forward_noalloc: one array per device, part of the library's code
// object, so that entry point needs no allocation.  Host code must never use this name as
// a device address (on the host it is only a stand-in symbol); it uses the per-device
// address hipGetSymbolAddress returns (noalloc_scratch below).  No byte of it needs to
// start at zero: every stage writes all the workspace that a later stage reads.
static __device__ __align__(256) unsigned char scratch[MX_NOALLOC_MAX_WORKSPACE];

namespace {

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

int check_desc(const MxMoeDesc* d) {
  if (!d) return MX_ERR_INVALID;
  if (d->hidden <= 0 || d->inter <= 0 || d->shared_inter < 0 || d->n_experts <= 0)
    return MX_ERR_INVALID;
  if (d->top_k < 1 || d->top_k > d->n_experts || d->top_k > 32) return MX_ERR_INVALID;
  if (d->router_mode < 0 || d->router_mode > 2) return MX_ERR_INVALID;
  if (d->param_dtype != MX_DT_F32 && d->param_dtype != MX_DT_F16) return MX_ERR_INVALID;
  if (d->weight_dtype != MX_DT_F32 && d->weight_dtype != MX_DT_F16 && d->weight_dtype != MX_DT_I8)
    return MX_ERR_INVALID;
  if (d->has_shared_gate && d->shared_inter == 0) return MX_ERR_INVALID;
  if (d->n_experts > 1024) return MX_ERR_UNSUPPORTED;
  if (d->hidden % 4) return MX_ERR_UNSUPPORTED;
  return MX_OK;
}

// Prefill batches (128-row m-tiles, fp16 / int8 experts) keep the y rows between the down
// and combine launches as fp16: half the bytes of that round trip (written once, read once),
// for one more rounding of each weighted expert row (2^-11 relative) before the fp32 sum.
#ifndef MX_Y_ROWS_FP16
#define MX_Y_ROWS_FP16 1
#endif
bool y_rows_fp16(const MxMoeViews& v) { return MX_Y_ROWS_FP16 && v.m_blk == 128; }

// Decode-sized batches run the decode router (RMSNorm + logits, then top-k + dispatch in
// one workgroup) in place of stages 0-3.
bool use_decode_router(const MxMoeDesc* d, const MxMoeWeights* w, int T, const float* x) {
  return mx_router_decode_ok(d, w, T, x);
}

// Workspace pieces outside the views: the dispatch scratch and, for the split-plane router,
// the low fp16 plane of h and the router rows' planes.
struct Internal {
  void* dscratch = nullptr;
  void* h16lo = nullptr;
  void* wsplit = nullptr;
};

int layout(const MxMoeDesc* d, int T, void* ws, MxMoeViews* v, size_t* total,
           Internal* in = nullptr) {
  MX_TRY(check_desc(d));
  if (T < 0) return MX_ERR_INVALID;
  const int Tn = T > 0 ? T : 1;
  const size_t H = d->hidden, E = d->n_experts, k = d->top_k;
  const int e1 = d->n_experts + (d->has_shared_gate ? 1 : 0);
  const int has_sh = d->shared_inter > 0;
  const int S = mx_router_splits_for(Tn, d->hidden, d->n_experts, d->has_shared_gate,
                                     d->param_dtype, d->weight_dtype);
  const bool split = mx_router_on_split(Tn, d->hidden, e1, d->weight_dtype);
  const int m_blk = mx_m_blk_for(Tn, d->weight_dtype);
  const size_t P = (size_t)Tn * k;
  const size_t R = P + (has_sh ? Tn : 0);
  const size_t imax = d->inter > d->shared_inter ? d->inter : d->shared_inter;
  const size_t mtmax = mx_max_mtiles(Tn, d->top_k, d->n_experts, has_sh, m_blk);
  const size_t aesz = d->weight_dtype == MX_DT_F32 ? 4 : 2;
  Carve c{(char*)ws};
  MxMoeViews t;
  t.h32 = (float*)c.take((size_t)Tn * H * 4);
  t.h16 = d->weight_dtype == MX_DT_F32 ? nullptr : c.take((size_t)Tn * H * 2);
  t.logits = (float*)c.take((size_t)S * Tn * e1 * 4);
  t.router_splits = S;
  t.topk_ids = (int32_t*)c.take(P * 4);
  t.topk_w = (float*)c.take(P * 4);
  t.shared_w = (float*)c.take((size_t)Tn * 4);
  t.counts = (int32_t*)c.take(E * 4);
  t.offsets = (int32_t*)c.take((E + 1) * 4);
  t.sorted_tok = (int32_t*)c.take(R * 4);
  t.sorted_w = (float*)c.take(R * 4);
  t.pair_pos = (int32_t*)c.take(P * 4);
  t.g_expert = (int32_t*)c.take((E + 1) * 4);
  t.g_start = (int32_t*)c.take((E + 1) * 4);
  t.g_count = (int32_t*)c.take((E + 1) * 4);
  t.n_groups = (int32_t*)c.take(4);
  t.mt_group = (int32_t*)c.take(mtmax * 4);
  t.mt_row0 = (int32_t*)c.take(mtmax * 4);
  t.n_mtiles = (int32_t*)c.take(4);
  t.m_blk = m_blk;
  t.act = c.take(R * imax * aesz);
  t.y = c.take(R * H * 4);  // fp32 rows (fp16 rows use the first half)
  size_t dscr = 0;
  MX_TRY(mx_dispatch_scratch_size(Tn, d->top_k, d->n_experts, &dscr));
  void* dispatch_scratch = c.take(dscr);
  void* h16lo = split ? c.take((size_t)Tn * H * 2) : nullptr;
  void* wsplit = split ? c.take(mx_router_split_bytes(d->hidden, e1)) : nullptr;
  if (in) {
    in->dscratch = dispatch_scratch;
    in->h16lo = h16lo;
    in->wsplit = wsplit;
  }
  if (v) *v = t;
  if (total) *total = mx_align_up(c.off, 256);
  return MX_OK;
}

// One token, when stages 1-4 run in one call: the gate/up launch selects the experts
// (and writes the dispatch tables), so the top-k/dispatch launch is left out.
#ifndef MX_SELECT_IN_GATE_UP
#define MX_SELECT_IN_GATE_UP 1
#endif
bool select_in_gate_up(const MxMoeDesc* d, const MxMoeWeights* w, int T, const float* x,
                       int st_begin, int st_end) {
  return MX_SELECT_IN_GATE_UP && T == 1 && st_begin <= 1 && st_end >= 5 &&
         use_decode_router(d, w, T, x) && mx_one_token_select_ok(d);
}

int run_stage(int stage, const MxMoeDesc* d, const MxMoeWeights* w, const float* x, float* out,
              int T, const MxMoeViews& v, const Internal& in, hipStream_t s, bool sel1) {
  void* const dscratch = in.dscratch;
  const int has_sh = d->shared_inter > 0;
  const bool decode = use_decode_router(d, w, T, x);
  if (decode && (stage == 0 || stage == 2 || stage == 3)) return MX_OK;  // in stage 1
  switch (stage) {
    case 0:
      if (!x || !w->norm_w) return MX_ERR_INVALID;
      if (in.h16lo) {  // the split-plane router's planes of h and of the router rows
        const MxRouterSplitW rsw = mx_router_split_planes(
            w->router_w, d->has_shared_gate ? w->shared_gate_w : nullptr, d->param_dtype,
            d->n_experts, d->hidden, T, v.router_splits, in.wsplit, v.logits);
        // The router reads the planes and the experts h16 (the split needs fp16 / int8
        // experts): no later stage reads the fp32 rows, so they are not written (GLM-4.7
        // 2048-token prefill: RMSNorm 27.5 -> 23.5 us).
        return mx_rmsnorm_launch(x, w->norm_w, d->param_dtype, d->eps, T, d->hidden, nullptr,
                                 v.h16, s, in.h16lo, &rsw);
      }
      return mx_rmsnorm_launch(x, w->norm_w, d->param_dtype, d->eps, T, d->hidden, v.h32, v.h16,
                               s);
    case 1:
      if (decode)
        return mx_router_decode_launch(d, w, T, x, v.h32, v.h16, v.logits, v.topk_ids, v.topk_w,
                                       v.shared_w, v.m_blk, v.counts, v.offsets, v.sorted_tok,
                                       v.sorted_w, v.pair_pos, v.g_expert, v.g_start, v.g_count,
                                       v.n_groups, v.mt_group, v.mt_row0, v.n_mtiles, s, sel1);
      if (in.h16lo)
        return mx_router_logits_split(v.h16, in.h16lo, w->router_w,
                                      d->has_shared_gate ? w->shared_gate_w : nullptr,
                                      d->param_dtype, T, d->hidden, d->n_experts, v.router_splits,
                                      in.wsplit, v.logits, s);
      return mx_router_logits(v.h32, w->router_w, d->has_shared_gate ? w->shared_gate_w : nullptr,
                              d->param_dtype, T, d->hidden, d->n_experts, v.router_splits,
                              v.logits, s);
    case 2:
      return mx_router_topk(v.logits, v.router_splits, d->has_bias ? w->bias : nullptr,
                            d->param_dtype, T, d->n_experts, d->top_k, d->router_mode,
                            d->norm_topk_prob, d->routed_scaling, d->has_shared_gate, v.topk_ids,
                            v.topk_w, v.shared_w, s);
    case 3:
      // Many-workgroup dispatch once the single workgroup's serial token walk dominates.
      if (dscratch && T >= 512 && d->n_experts * 48 <= 64 * 1024)
        return mx_dispatch_chunked(v.topk_ids, v.topk_w, v.shared_w, T, d->top_k, d->n_experts,
                                   has_sh, v.m_blk, dscratch, v.counts, v.offsets, v.sorted_tok,
                                   v.sorted_w, v.pair_pos, v.g_expert, v.g_start, v.g_count,
                                   v.n_groups, v.mt_group, v.mt_row0, v.n_mtiles, s);
      return mx_dispatch(v.topk_ids, v.topk_w, v.shared_w, T, d->top_k, d->n_experts, has_sh,
                         v.m_blk, v.counts, v.offsets, v.sorted_tok, v.sorted_w, v.pair_pos,
                         v.g_expert, v.g_start, v.g_count, v.n_groups, v.mt_group, v.mt_row0,
                         v.n_mtiles, s);
    case 4:
      if (sel1) {
        MxOneTokenSelect sp;
        sp.logits = v.logits;
        sp.bias = (d->router_mode == MX_ROUTER_SOFTMAX || !d->has_bias) ? nullptr : w->bias;
        sp.pdt = d->param_dtype;
        sp.E1 = d->n_experts + (d->has_shared_gate ? 1 : 0);
        sp.k = d->top_k;
        sp.mode = d->router_mode;
        sp.norm = d->norm_topk_prob;
        sp.has_seg = d->has_shared_gate;
        sp.has_shared = has_sh;
        sp.scaling = d->routed_scaling;
        sp.ids = v.topk_ids;
        sp.tw = v.topk_w;
        sp.shared_w = v.shared_w;
        sp.counts = v.counts;
        sp.offsets = v.offsets;
        sp.sorted_tok = v.sorted_tok;
        sp.sorted_w = v.sorted_w;
        sp.pair_pos = v.pair_pos;
        sp.g_expert = v.g_expert;
        sp.g_start = v.g_start;
        sp.g_count = v.g_count;
        sp.n_groups = v.n_groups;
        sp.mt_group = v.mt_group;
        sp.mt_row0 = v.mt_row0;
        sp.n_mtiles = v.n_mtiles;
        return mx_expert_gate_up_select(
            d, w->experts, d->weight_dtype == MX_DT_F32 ? (const void*)v.h32 : v.h16, v.act, sp, s);
      }
      return mx_expert_gate_up(d, w->experts, T,
                               d->weight_dtype == MX_DT_F32 ? (const void*)v.h32 : v.h16,
                               v.sorted_tok, v.g_expert, v.g_start, v.g_count, v.mt_group,
                               v.mt_row0, v.n_mtiles, v.m_blk, v.act, s);
    case 5:
      return mx_expert_down_rows(d, w->experts, T, v.act, v.sorted_w, v.g_expert, v.g_start,
                                 v.g_count, v.mt_group, v.mt_row0, v.n_mtiles, v.m_blk, v.y,
                                 y_rows_fp16(v), s);
    case 6:
      if (!x || !out) return MX_ERR_INVALID;
      return mx_combine_rows(x, v.y, v.pair_pos, T, d->hidden, d->top_k, has_sh, out,
                             y_rows_fp16(v), s);
    default:
      return MX_ERR_INVALID;
  }
}

int forward(const MxMoeDesc* d, const MxMoeWeights* w, const float* x, float* out, int T, void* ws,
            size_t ws_bytes, hipStream_t s, void* const* events, int st_begin = 0,
            int st_end = MX_N_STAGES) {
  MX_TRY(check_desc(d));
  if (!w || !x || !out || !ws || T < 0) return MX_ERR_INVALID;
  if (!w->norm_w || !w->router_w || !w->experts) return MX_ERR_INVALID;
  if (d->has_bias && !w->bias) return MX_ERR_INVALID;
  if (d->has_shared_gate && !w->shared_gate_w) return MX_ERR_INVALID;
  if (T == 0) return MX_OK;
  MxMoeViews v;
  size_t need = 0;
  Internal in;
  MX_TRY(layout(d, T, ws, &v, &need, &in));
  if (ws_bytes < need) return MX_ERR_WORKSPACE;
  const bool sel1 = select_in_gate_up(d, w, T, x, st_begin, st_end);
  for (int st = st_begin; st < st_end; ++st) {
    if (events) MX_TRY(mx_status(hipEventRecord((hipEvent_t)events[st], s)));
    MX_TRY(run_stage(st, d, w, x, out, T, v, in, s, sel1));
  }
  if (events) MX_TRY(mx_status(hipEventRecord((hipEvent_t)events[MX_N_STAGES], s)));
  return MX_OK;
}

}  // namespace

extern "C" int mx_moe_workspace_size(const MxMoeDesc* desc, int32_t tokens, size_t* nbytes) {
  if (!nbytes) return MX_ERR_INVALID;
  return layout(desc, tokens, nullptr, nullptr, nbytes);
}

extern "C" int mx_moe_views(const MxMoeDesc* desc, int32_t tokens, void* workspace,
                            MxMoeViews* views) {
  if (!workspace || !views) return MX_ERR_INVALID;
  return layout(desc, tokens, workspace, views, nullptr);
}

extern "C" int mx_moe_forward(const MxMoeDesc* desc, const MxMoeWeights* weights, const float* x,
                              float* out, int32_t tokens, void* workspace, size_t workspace_bytes,
                              void* stream) {
  return forward(desc, weights, x, out, tokens, workspace, workspace_bytes, (hipStream_t)stream,
                 nullptr);
}

extern "C" int mx_moe_forward_profiled(const MxMoeDesc* desc, const MxMoeWeights* weights,
                                       const float* x, float* out, int32_t tokens, void* workspace,
                                       size_t workspace_bytes, void* stream, void* const* events,
                                       int32_t n_events) {
  if (!events || n_events != MX_N_STAGES + 1) return MX_ERR_INVALID;
  for (int i = 0; i < n_events; ++i)
    if (!events[i]) return MX_ERR_INVALID;
  return forward(desc, weights, x, out, tokens, workspace, workspace_bytes, (hipStream_t)stream,
                 events);
}

extern "C" int mx_moe_forward_stages(const MxMoeDesc* desc, const MxMoeWeights* weights,
                                     const float* x, float* out, int32_t tokens, void* workspace,
                                     size_t workspace_bytes, int32_t stage_begin,
                                     int32_t stage_end, void* stream) {
  if (stage_begin < 0 || stage_end > MX_N_STAGES || stage_begin > stage_end)
    return MX_ERR_INVALID;
  return forward(desc, weights, x, out, tokens, workspace, workspace_bytes, (hipStream_t)stream,
                 nullptr, stage_begin, stage_end);
}

// ---- no-allocation entry ------------------------------------------------------------------
namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device, looked up once per device (with
// that device current) and kept.
int noalloc_scratch(void** addr) {
  int dev = 0;
  MX_TRY(mx_status(hipGetDevice(&dev)));
  if (dev < 0 || dev >= kMaxDevices) return MX_ERR_UNSUPPORTED;
  void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (!p) {
      MX_TRY(mx_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))));
      if (!p) return MX_ERR_UNSUPPORTED;
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *addr = p;
  return MX_OK;
}

}  // namespace

extern "C" int mx_moe_forward_noalloc(const MxMoeDesc* desc, const MxMoeWeights* weights,
                                      const float* x, float* out, int32_t tokens, void* stream) {
  size_t need = 0;
  MX_TRY(layout(desc, tokens, nullptr, nullptr, &need));
  if (need > (size_t)MX_NOALLOC_MAX_WORKSPACE) return MX_ERR_WORKSPACE;
  void* ws = nullptr;
  MX_TRY(noalloc_scratch(&ws));
  return forward(desc, weights, x, out, tokens, ws, (size_t)MX_NOALLOC_MAX_WORKSPACE,
                 (hipStream_t)stream, nullptr);
}
