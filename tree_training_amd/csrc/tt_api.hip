// extern "C" entry points: host-side validation, then enqueue-only launches.
#include <math.h>

#include <algorithm>
#include <vector>

#include "tt_common.h"
#include "tt_internal.h"

namespace {

constexpr int kAbiVersion = 9;
constexpr int64_t kMaxTokStride = int64_t(1) << 23;   // elements (bf16; half that for fp32)
inline int64_t max_tok_stride(int dtype) { return dtype == TT_DTYPE_BF16 ? kMaxTokStride : kMaxTokStride / 2; }

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Validates a problem and fills the kernels' view of it.
int make_dev(const tt_attn_problem* p, AttnDev* a) {
    if (!p) return TT_E_ARG;
    if (p->dtype != TT_DTYPE_BF16 && p->dtype != TT_DTYPE_F32) return TT_E_UNSUPPORTED;
    if (p->head_dim != 128) return TT_E_UNSUPPORTED;
    if (p->n_q < 1 || p->n_past < 0 || p->n_heads_q < 1 || p->n_heads_kv < 1) return TT_E_ARG;
    if (p->n_heads_q % p->n_heads_kv != 0) return TT_E_UNSUPPORTED;
    if (p->n_heads_q > 65535 || p->n_heads_kv > 65535) return TT_E_ARG;
    if ((int64_t)p->n_q + p->n_past > 0x3fffffff) return TT_E_ARG;
    if (!(p->scale > 0.0f) || !isfinite(p->scale)) return TT_E_ARG;
    if (!p->q.ptr || !p->k.ptr || !p->v.ptr || !p->key_lo || !p->key_hi || !p->plan) return TT_E_ARG;
    if (p->n_past > 0 && (!p->k_past.ptr || !p->v_past.ptr)) return TT_E_ARG;
    const int n_keys = p->n_q + p->n_past;
    if (p->plan_bytes < tt_plan_bytes_impl(p->n_q, n_keys)) return TT_E_WORKSPACE;
    // the kernels read 16-byte vectors: 8 (bf16) or 4 (fp32) element granularity for strides
    const int64_t gran = p->dtype == TT_DTYPE_BF16 ? 8 : 4;
    const size_t ealign = 16;
    const tt_tensor* ts[5] = {&p->q, &p->k, &p->v, &p->k_past, &p->v_past};
    const int nt = p->n_past > 0 ? 5 : 3;
    for (int i = 0; i < nt; ++i) {
        const tt_tensor* t = ts[i];
        if (t->stride_tok < 128 || t->stride_head < 128 || (t->stride_tok % gran) || (t->stride_head % gran))
            return TT_E_ARG;
        // the kernels address a tile of up to 128 rows with 32-bit byte offsets
        if (t->stride_tok >= max_tok_stride(p->dtype)) return TT_E_ARG;
        if (!aligned(t->ptr, ealign)) return TT_E_ARG;
    }
    a->q = p->q.ptr; a->q_st = p->q.stride_tok; a->q_sh = p->q.stride_head;
    a->k = p->k.ptr; a->k_st = p->k.stride_tok; a->k_sh = p->k.stride_head;
    a->v = p->v.ptr; a->v_st = p->v.stride_tok; a->v_sh = p->v.stride_head;
    a->kp = p->n_past > 0 ? p->k_past.ptr : nullptr;
    a->kp_st = p->k_past.stride_tok; a->kp_sh = p->k_past.stride_head;
    a->vp = p->n_past > 0 ? p->v_past.ptr : nullptr;
    a->vp_st = p->v_past.stride_tok; a->vp_sh = p->v_past.stride_head;
    a->key_lo = p->key_lo;
    a->key_hi = p->key_hi;
    a->n_q = p->n_q;
    a->n_past = p->n_past;
    a->n_keys = n_keys;
    a->hq = p->n_heads_q;
    a->hkv = p->n_heads_kv;
    a->rep = p->n_heads_q / p->n_heads_kv;
    a->n_qb = tt_cdiv(p->n_q, TT_BQ);
    a->n_kt = tt_cdiv(n_keys, TT_BK);
    a->scale = p->scale;
    const PlanLayout L(p->n_q, n_keys);
    a->n_kb = L.n_kb;
    const uint8_t* base = reinterpret_cast<const uint8_t*>(p->plan);
    a->row_cnt = reinterpret_cast<const int32_t*>(base + L.row_cnt);
    a->row_order = reinterpret_cast<const int32_t*>(base + L.row_order);
    a->row_list = reinterpret_cast<const int32_t*>(base + L.row_list);
    a->kb_qlo = reinterpret_cast<const int32_t*>(base + L.kb_qlo);
    a->kb_qhi = reinterpret_cast<const int32_t*>(base + L.kb_qhi);
    a->kb_order = reinterpret_cast<const int32_t*>(base + L.kb_order);
    a->kb_base = reinterpret_cast<const int32_t*>(base + L.kb_base);
    a->kb_srank = reinterpret_cast<const int32_t*>(base + L.kb_srank);
    a->kb_item = reinterpret_cast<const int2*>(base + L.kb_item);
    a->n_items = reinterpret_cast<const int32_t*>(base) + 5;
    return TT_OK;
}

}  // namespace

extern "C" {

int tt_abi_version(void) { return kAbiVersion; }

const char* tt_strerror(int code) {
    switch (code) {
        case TT_OK: return "ok";
        case TT_E_ARG: return "invalid argument (size, null pointer, stride or alignment)";
        case TT_E_UNSUPPORTED: return "unsupported configuration (dtype, head_dim != 128, or Hq % Hkv != 0)";
        case TT_E_HIP: return "HIP kernel launch failed";
        case TT_E_WORKSPACE: return "workspace or plan buffer too small";
        default: return "unknown tree-attention error";
    }
}

size_t tt_meta_workspace_bytes(int32_t n_nodes) { return tt_meta_ws_bytes_impl(n_nodes); }

int tt_meta_build(const int32_t* node_len, const int32_t* node_parent, int32_t n_nodes, int32_t n_tokens,
                  int32_t pos_offset, int32_t* node_start, int32_t* node_off, int32_t* node_hend, int32_t* pos,
                  int32_t* node_of, int32_t* horizon, int32_t* status, void* ws, size_t ws_bytes,
                  void* stream) {
    if (n_nodes < 1 || n_tokens < n_nodes || n_tokens > 0x3fffffff || pos_offset < 0) return TT_E_ARG;
    if (!node_len || !node_parent || !node_start || !node_off || !node_hend || !pos || !horizon || !status ||
        !ws)
        return TT_E_ARG;
    if (ws_bytes < tt_meta_ws_bytes_impl(n_nodes)) return TT_E_WORKSPACE;
    return tt_meta_build_impl(node_len, node_parent, n_nodes, n_tokens, pos_offset, node_start, node_off,
                              node_hend, pos, node_of, horizon, status, ws, (hipStream_t)stream);
}

int tt_keys_build(const float* past_bias, int32_t n_past, const int32_t* horizon, int32_t n_q, int32_t* key_lo,
                  int32_t* key_hi, int32_t* status, void* stream) {
    if (n_q < 1 || n_past < 0 || (int64_t)n_q + n_past > 0x3fffffff) return TT_E_ARG;
    if ((n_past > 0 && !past_bias) || !horizon || !key_lo || !key_hi || !status) return TT_E_ARG;
    return tt_keys_build_impl(past_bias, n_past, horizon, n_q, key_lo, key_hi, status, (hipStream_t)stream);
}

int tt_meta_dense_mask(const int32_t* key_lo, const int32_t* key_hi, int32_t n_keys, int32_t n_q, uint8_t* mask,
                       void* stream) {
    if (n_keys < 1 || n_q < 1 || !key_lo || !key_hi || !mask) return TT_E_ARG;
    if (n_q > 65535) return TT_E_UNSUPPORTED;   // one grid row per query
    return tt_dense_mask_impl(key_lo, key_hi, n_keys, n_q, mask, (hipStream_t)stream);
}

size_t tt_plan_bytes(int32_t n_q, int32_t n_keys) {
    if (n_q < 1 || n_keys < 1) return 0;
    return tt_plan_bytes_impl(n_q, n_keys);
}

int tt_plan_build(const int32_t* key_lo, const int32_t* key_hi, int32_t n_keys, int32_t n_q, void* plan,
                  size_t plan_bytes, void* stream) {
    if (n_q < 1 || n_keys < n_q || n_keys > 0x3fffffff || !key_lo || !key_hi || !plan) return TT_E_ARG;
    if (plan_bytes < tt_plan_bytes_impl(n_q, n_keys)) return TT_E_WORKSPACE;
    return tt_plan_build_impl(key_lo, key_hi, n_keys, n_q, plan, (hipStream_t)stream);
}

static_assert(sizeof(tt_tree_job) == 144, "tt_tree_job layout (bindings mirror it)");
static_assert(sizeof(tt_tensor) == 24 && sizeof(tt_attn_problem) == 200 && sizeof(tt_gdn_problem) == 240 &&
                  sizeof(tt_conv_problem) == 72 && sizeof(tt_prologue_problem) == 120,
              "problem struct layouts (the ctypes bindings mirror them)");

int tt_trees_build(const tt_tree_job* jobs, int32_t n_jobs, void* stream) {
    if (!jobs || n_jobs < 1 || n_jobs > TT_TREE_JOBS_MAX) return TT_E_ARG;
    for (int i = 0; i < n_jobs; ++i) {
        const tt_tree_job& t = jobs[i];
        if (t.n_nodes < 1 || t.n_tokens < t.n_nodes || t.n_past < 0 || t.pos_offset < 0) return TT_E_ARG;
        if ((int64_t)t.n_tokens + t.n_past > 0x3fffffff) return TT_E_ARG;
        if (!t.node_len || !t.node_parent || !t.node_start || !t.node_off || !t.node_hend || !t.pos || !t.horizon ||
            !t.key_lo || !t.key_hi || !t.status || !t.plan || !t.ws || (t.n_past > 0 && !t.past_bias))
            return TT_E_ARG;
        if (!tt_trees_job_fits(t.n_tokens, t.n_tokens + t.n_past)) return TT_E_UNSUPPORTED;
        if (t.plan_bytes < tt_plan_bytes_impl(t.n_tokens, t.n_tokens + t.n_past) ||
            t.ws_bytes < tt_meta_ws_bytes_impl(t.n_nodes))
            return TT_E_WORKSPACE;
    }
    return tt_trees_build_impl(jobs, n_jobs, (hipStream_t)stream);
}

// Key-range splits of a problem's forward and dQ passes (bf16 only).
static int key_splits(const tt_attn_problem* p) {
    return p->dtype == TT_DTYPE_BF16 ? tt_key_splits(p->n_q, p->n_heads_q) : 1;
}
static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }
// fp32 partial rows of a split pass: [splits, n_q, Hq, 128]
static size_t split_part_bytes(const tt_attn_problem* p) {
    const int s = key_splits(p);
    return s > 1 ? align256((size_t)s * p->n_q * p->n_heads_q * 128 * sizeof(float)) : 0;
}
// row max and row sum of each split: [splits, Hq, n_q] each
static size_t split_stat_bytes(const tt_attn_problem* p) {
    const int s = key_splits(p);
    return s > 1 ? align256((size_t)s * p->n_heads_q * p->n_q * sizeof(float)) : 0;
}

size_t tt_attn_fwd_workspace_bytes(const tt_attn_problem* p) {
    if (!p || p->n_q < 1 || p->n_heads_q < 1) return 0;
    return split_part_bytes(p) + 2 * split_stat_bytes(p);
}

int tt_attn_fwd(const tt_attn_problem* p, void* o, float* lse, void* ws, size_t ws_bytes, void* stream) {
    AttnDev a;
    int rc = make_dev(p, &a);
    if (rc != TT_OK) return rc;
    if (!o || !lse) return TT_E_ARG;
    if (!aligned(o, 16)) return TT_E_ARG;
    const size_t need = tt_attn_fwd_workspace_bytes(p);
    if (need > 0 && (!ws || !aligned(ws, 16))) return TT_E_ARG;
    if (ws_bytes < need) return TT_E_WORKSPACE;
    if (p->dtype == TT_DTYPE_BF16) {
        FwdSplit sp{nullptr, nullptr, nullptr, key_splits(p)};
        if (sp.n > 1) {
            uint8_t* w = reinterpret_cast<uint8_t*>(ws);
            sp.o = reinterpret_cast<float*>(w);
            sp.m = reinterpret_cast<float*>(w + split_part_bytes(p));
            sp.l = reinterpret_cast<float*>(w + split_part_bytes(p) + split_stat_bytes(p));
        }
        return tt_fwd_bf16_launch(a, o, lse, sp, (hipStream_t)stream);
    }
    return tt_fwd_f32_launch(a, o, lse, (hipStream_t)stream);
}

// Workspace: delta [Hq, n_q] fp32, then the fp32 dK and dV sums of key tiles
// whose query range is split over several work items, [n_keys, Hkv, head_dim]
// each, then (TT_BWD_DETERMINISTIC) the dK and dV slots of those tiles' later
// items, [tt_det_slots, 128, Hkv, head_dim] each, then (bf16 problems with
// tt_key_splits > 1) the dQ pass's fp32 partials [splits, n_q, Hq, head_dim].
static size_t delta_bytes(const tt_attn_problem* p) {
    return ((size_t)p->n_heads_q * (size_t)p->n_q * sizeof(float) + 255) & ~(size_t)255;
}
// Split key tiles the split sums hold: the caller's exact count, else every
// key tile.
static int64_t split_cap(const tt_attn_problem* p) {
    return p->split_tiles > 0 ? p->split_tiles : (int64_t)tt_cdiv(p->n_q + p->n_past, TT_BKB);
}
static size_t split_rows_bytes(const tt_attn_problem* p) {
    return (size_t)split_cap(p) * TT_BKB * (size_t)p->n_heads_kv * 128 * sizeof(float);
}
// Slots of the deterministic mode: the caller's exact count, else the bound.
static int64_t det_slot_count(const tt_attn_problem* p) {
    return p->det_slots > 0 ? p->det_slots : tt_det_slots(p->n_q, p->n_q + p->n_past);
}
static size_t det_slot_bytes(const tt_attn_problem* p) {
    return (size_t)det_slot_count(p) * TT_BKB * (size_t)p->n_heads_kv * 128 * sizeof(float);
}

size_t tt_attn_bwd_workspace_bytes(const tt_attn_problem* p) {
    if (!p || p->n_q < 1 || p->n_heads_q < 1 || p->n_heads_kv < 1 || p->n_past < 0) return 0;
    if ((int64_t)p->n_q + p->n_past > 0x3fffffff || p->det_slots < 0 || p->split_tiles < 0) return 0;
    size_t b = delta_bytes(p) + 2 * split_rows_bytes(p);
    if (p->bwd_parts & TT_BWD_DETERMINISTIC) b += 2 * det_slot_bytes(p);
    return b + split_part_bytes(p);
}

int tt_attn_bwd(const tt_attn_problem* p, const void* o, const float* lse, tt_tensor d_o, void* dq, void* dk,
                void* dv, float* dk_past_acc, float* dv_past_acc, void* ws, size_t ws_bytes, void* stream) {
    AttnDev a;
    int rc = make_dev(p, &a);
    if (rc != TT_OK) return rc;
    if (!o || !lse || !d_o.ptr || !dq || !dk || !dv || !ws) return TT_E_ARG;
    if ((dk_past_acc == nullptr) != (dv_past_acc == nullptr)) return TT_E_ARG;
    if (p->det_slots < 0 || p->split_tiles < 0) return TT_E_ARG;
    if (ws_bytes < tt_attn_bwd_workspace_bytes(p)) return TT_E_WORKSPACE;
    const int64_t gran = p->dtype == TT_DTYPE_BF16 ? 8 : 4;
    const size_t ealign = 16;
    if (d_o.stride_tok < 128 || d_o.stride_head < 128 || (d_o.stride_tok % gran) || (d_o.stride_head % gran))
        return TT_E_ARG;
    if (d_o.stride_tok >= max_tok_stride(p->dtype)) return TT_E_ARG;
    if (!aligned(d_o.ptr, ealign) || !aligned(o, ealign) || !aligned(dq, ealign) || !aligned(dk, ealign) ||
        !aligned(dv, ealign) || !aligned(ws, 16) || !aligned(dk_past_acc, 16) || !aligned(dv_past_acc, 16))
        return TT_E_ARG;
    BwdDev b;
    b.o = o;
    b.lse = lse;
    b.dout = d_o.ptr;
    b.do_st = d_o.stride_tok;
    b.do_sh = d_o.stride_head;
    b.dq = dq;
    b.dk = dk;
    b.dv = dv;
    b.dk_acc = p->n_past > 0 ? dk_past_acc : nullptr;
    b.dv_acc = p->n_past > 0 ? dv_past_acc : nullptr;
    b.delta = reinterpret_cast<float*>(ws);
    if (p->bwd_parts & ~(TT_BWD_DELTA | TT_BWD_DQ | TT_BWD_DKDV | TT_BWD_DETERMINISTIC)) return TT_E_ARG;
    b.det = (p->bwd_parts & TT_BWD_DETERMINISTIC) ? 1 : 0;
    b.dk_ws = b.dv_ws = b.dk_slot = b.dv_slot = b.dq_part = nullptr;
    b.det_cap = b.det ? det_slot_count(p) : 0;
    b.split_cap = split_cap(p);
    b.n_split = key_splits(p);
    {
        uint8_t* w = reinterpret_cast<uint8_t*>(ws) + delta_bytes(p);
        b.dk_ws = reinterpret_cast<float*>(w);
        b.dv_ws = reinterpret_cast<float*>(w + split_rows_bytes(p));
        w += 2 * split_rows_bytes(p);
        if (b.det) {
            b.dk_slot = reinterpret_cast<float*>(w);
            b.dv_slot = reinterpret_cast<float*>(w + det_slot_bytes(p));
            w += 2 * det_slot_bytes(p);
        }
        if (b.n_split > 1) b.dq_part = reinterpret_cast<float*>(w);
    }
    const int parts = p->bwd_parts & (TT_BWD_DELTA | TT_BWD_DQ | TT_BWD_DKDV);
    b.parts = parts ? parts : (TT_BWD_DELTA | TT_BWD_DQ | TT_BWD_DKDV);
    b.zero_in_dq = p->dtype == TT_DTYPE_BF16 && !b.det && (b.parts & TT_BWD_DQ) && (b.parts & TT_BWD_DKDV);
    if (p->dtype == TT_DTYPE_BF16) return tt_bwd_bf16_launch(a, b, (hipStream_t)stream);
    return tt_bwd_f32_launch(a, b, (hipStream_t)stream);
}

}  // extern "C"

// Visible query range [lo, hi) of every 128-key tile of a DFS pre-order
// forest (own key j: queries [j, subtree end of its node); a visible gateway
// key: every query), as the device's metadata, keys and plan passes derive
// it; n_q = the forest's tokens. TT_OK or TT_E_ARG.
static int tree_tile_ranges(const int32_t* node_len, const int32_t* parent, int n_nodes, const float* past_bias,
                            int n_past, int& n_q, std::vector<int>& lo, std::vector<int>& hi) {
    if (!node_len || !parent || n_nodes < 1 || n_past < 0) return TT_E_ARG;
    // subtree end per node: in DFS pre-order a node's subtree is the run of
    // nodes after it, so children (later nodes) fold into their parents
    std::vector<int64_t> start(n_nodes), end(n_nodes);
    int64_t T = 0;
    for (int u = 0; u < n_nodes; ++u) {
        if (node_len[u] < 1 || parent[u] < -1 || parent[u] >= u) return TT_E_ARG;
        start[u] = T;
        T += node_len[u];
        end[u] = T;
        if (T + n_past > 0x3fffffff) return TT_E_ARG;
    }
    for (int u = n_nodes - 1; u > 0; --u)
        if (parent[u] >= 0 && end[u] > end[parent[u]]) end[parent[u]] = end[u];
    n_q = (int)T;
    const int n_kb = tt_cdiv(n_past + n_q, TT_BKB);
    lo.assign(n_kb, n_q);
    hi.assign(n_kb, 0);
    for (int j = 0; j < n_past; ++j)
        if (!past_bias || past_bias[j] == 0.0f) {
            lo[j / TT_BKB] = 0;
            hi[j / TT_BKB] = n_q;
        }
    for (int u = 0; u < n_nodes; ++u)
        for (int64_t t = start[u]; t < start[u] + node_len[u]; ++t) {
            const int kb = (int)((n_past + t) / TT_BKB);
            lo[kb] = std::min(lo[kb], (int)t);
            hi[kb] = std::max(hi[kb], (int)end[u]);
        }
    for (int kb = 0; kb < n_kb; ++kb)
        if (lo[kb] >= hi[kb]) lo[kb] = hi[kb] = 0;   // a tile no query sees
    return TT_OK;
}

extern "C" {

int tt_attn_det_slots(const int32_t* node_len, const int32_t* parent, int n_nodes, const float* past_bias,
                      int n_past, int64_t* slots) {
    if (!slots) return TT_E_ARG;
    int n_q = 0;
    std::vector<int> lo, hi;
    const int rc = tree_tile_ranges(node_len, parent, n_nodes, past_bias, n_past, n_q, lo, hi);
    if (rc != TT_OK) return rc;
    const int qch = tt_qch(n_q);
    int64_t extra = 0;
    for (size_t kb = 0; kb < lo.size(); ++kb) extra += tt_kb_items(lo[kb], hi[kb], qch) - 1;
    *slots = extra;
    return TT_OK;
}

int tt_attn_split_tiles(const int32_t* node_len, const int32_t* parent, int n_nodes, const float* past_bias,
                        int n_past, int64_t* tiles) {
    if (!tiles) return TT_E_ARG;
    int n_q = 0;
    std::vector<int> lo, hi;
    const int rc = tree_tile_ranges(node_len, parent, n_nodes, past_bias, n_past, n_q, lo, hi);
    if (rc != TT_OK) return rc;
    const int qch = tt_qch(n_q);
    int64_t n = 0;
    for (size_t kb = 0; kb < lo.size(); ++kb) n += tt_kb_items(lo[kb], hi[kb], qch) > 1;
    *tiles = n;
    return TT_OK;
}

size_t tt_gdn_workspace_bytes(const tt_gdn_problem* p) {
    if (!p || p->n_chunks < 1 || p->n_heads_v < 1) return 0;
    return tt_gdn_ws_bytes_impl(p->n_chunks, p->n_heads_v, p->reference_truncated != 0);
}

}  // extern "C"

// Checks a tt_gdn_problem and fills the device view; TT_OK or a TT_E_* code.
static int gdn_problem(const tt_gdn_problem* p, GdnDev& d) {
    if (!p) return TT_E_ARG;
    if (p->dtype != TT_DTYPE_BF16 && p->dtype != TT_DTYPE_F32) return TT_E_UNSUPPORTED;
    if (p->head_dim != 128) return TT_E_UNSUPPORTED;
    if (p->n_tokens < 1 || p->n_nodes < 1 || p->n_nodes > p->n_tokens || p->n_heads_k < 1 || p->n_heads_v < 1)
        return TT_E_ARG;
    if (p->n_heads_v % p->n_heads_k != 0) return TT_E_UNSUPPORTED;
    if (p->n_heads_v > 65535 || !(p->scale > 0.0f) || !isfinite(p->scale)) return TT_E_ARG;
    if (!p->q.ptr || !p->k.ptr || !p->v.ptr || !p->g || !p->beta || !p->node_start || !p->node_len ||
        !p->node_parent || !p->level_nodes || !p->level_offsets || p->n_levels < 1 || !p->node_chunk0 ||
        !p->chunk_node)
        return TT_E_ARG;
    if (p->n_chunks < p->n_nodes || p->n_chunks > p->n_tokens) return TT_E_ARG;
    const int64_t gran = p->dtype == TT_DTYPE_BF16 ? 8 : 4;
    const tt_tensor* ts[3] = {&p->q, &p->k, &p->v};
    for (int i = 0; i < 3; ++i) {
        const tt_tensor* t = ts[i];
        if (t->stride_tok < 128 || t->stride_head < 128 || (t->stride_tok % gran) || (t->stride_head % gran) ||
            !aligned(t->ptr, 16))
            return TT_E_ARG;
    }
    if (p->g_stride_tok < p->n_heads_v || p->beta_stride_tok < p->n_heads_v) return TT_E_ARG;
    if (p->level_offsets[0] != 0 || p->level_offsets[p->n_levels] != p->n_nodes) return TT_E_ARG;
    for (int l = 0; l < p->n_levels; ++l)
        if (p->level_offsets[l + 1] < p->level_offsets[l]) return TT_E_ARG;
    d.q = p->q.ptr; d.q_st = p->q.stride_tok; d.q_sh = p->q.stride_head;
    d.k = p->k.ptr; d.k_st = p->k.stride_tok; d.k_sh = p->k.stride_head;
    d.v = p->v.ptr; d.v_st = p->v.stride_tok; d.v_sh = p->v.stride_head;
    d.g = p->g; d.g_st = p->g_stride_tok;
    d.beta = p->beta; d.b_st = p->beta_stride_tok;
    d.node_start = p->node_start;
    d.node_len = p->node_len;
    d.parent = p->node_parent;
    d.level_nodes = p->level_nodes;
    d.node_chunk0 = p->node_chunk0;
    d.chunk_node = p->chunk_node;
    d.child_off = p->node_child_off;
    d.child = p->node_child;
    d.n_chunks = p->n_chunks;
    d.dtype = p->dtype;
    d.n_tokens = p->n_tokens;
    d.n_nodes = p->n_nodes;
    d.hk = p->n_heads_k;
    d.hv = p->n_heads_v;
    d.rep = p->n_heads_v / p->n_heads_k;
    d.l2 = p->l2norm ? 1 : 0;
    if (p->reference_truncated != 0 && p->reference_truncated != 1) return TT_E_ARG;
    d.trunc = p->reference_truncated;
    d.scale = p->scale;
    if (p->initial_state && !aligned(p->initial_state, 16)) return TT_E_ARG;
    d.init = p->initial_state;
    d.d_states = nullptr;
    d.d_states_last = 0;
    d.d_init = nullptr;
    return TT_OK;
}

extern "C" {

int tt_gdn_tree_fwd(const tt_gdn_problem* p, void* o, float* node_states, void* ws, size_t ws_bytes,
                    void* stream) {
    GdnDev d;
    const int rc = gdn_problem(p, d);
    if (rc != TT_OK) return rc;
    if (!o || !node_states || !ws) return TT_E_ARG;
    if (ws_bytes < tt_gdn_ws_bytes_impl(p->n_chunks, p->n_heads_v, p->reference_truncated != 0)) return TT_E_WORKSPACE;
    if (!aligned(o, 16) || !aligned(node_states, 16) || !aligned(ws, 16)) return TT_E_ARG;
    return tt_gdn_fwd_launch(d, p->level_offsets, p->n_levels, o, node_states, (float*)ws, (hipStream_t)stream);
}

size_t tt_gdn_bwd_workspace_bytes(const tt_gdn_problem* p) {
    if (!p || p->n_chunks < 1 || p->n_nodes < 1 || p->n_heads_v < 1) return 0;
    return tt_gdn_bwd_ws_bytes_impl(p->n_chunks, p->n_nodes, p->n_heads_v, true, p->reference_truncated != 0);
}

size_t tt_gdn_saved_bytes(const tt_gdn_problem* p) {
    if (!p || p->n_chunks < 1 || p->n_heads_v < 1) return 0;
    return tt_gdn_saved_bytes_impl(p->n_chunks, p->n_heads_v, p->reference_truncated != 0);
}

int tt_gdn_tree_fwd_save(const tt_gdn_problem* p, void* o, float* node_states, void* saved, size_t saved_bytes,
                         void* stream) {
    GdnDev d;
    const int rc = gdn_problem(p, d);
    if (rc != TT_OK) return rc;
    if (!o || !node_states || !saved) return TT_E_ARG;
    if (saved_bytes < tt_gdn_saved_bytes_impl(p->n_chunks, p->n_heads_v, p->reference_truncated != 0)) return TT_E_WORKSPACE;
    if (!aligned(o, 16) || !aligned(node_states, 16) || !aligned(saved, 16)) return TT_E_ARG;
    return tt_gdn_fwd_save_launch(d, p->level_offsets, p->n_levels, o, node_states, (float*)saved,
                                  (hipStream_t)stream);
}

size_t tt_gdn_bwd_saved_workspace_bytes(const tt_gdn_problem* p) {
    if (!p || p->n_chunks < 1 || p->n_nodes < 1 || p->n_heads_v < 1) return 0;
    return tt_gdn_bwd_ws_bytes_impl(p->n_chunks, p->n_nodes, p->n_heads_v, false, p->reference_truncated != 0);
}

// Shared argument checks of the two backward entry points.
// d_o and the dq/dk/dv outputs: rows of 128 elements at a token and a head
// stride (at least 128, multiples of 16 bytes), 16-byte aligned.
static bool gdn_rows_ok(const tt_tensor& t, int64_t gran) {
    return t.ptr && t.stride_tok >= 128 && t.stride_head >= 128 && !(t.stride_tok % gran) &&
           !(t.stride_head % gran) && aligned(t.ptr, 16);
}

static int gdn_bwd_args(const tt_gdn_problem* p, GdnDev& d, const tt_tensor& d_o, const tt_tensor& dq,
                        const tt_tensor& dk, const tt_tensor& dv, float* dg, float* dbeta,
                        const float* d_node_states, float* d_initial_state, void* ws) {
    if (!p->node_child_off || !p->node_child) return TT_E_ARG;
    if (!dg || !dbeta || !ws) return TT_E_ARG;
    const int64_t gran = p->dtype == TT_DTYPE_BF16 ? 8 : 4;
    if (!gdn_rows_ok(d_o, gran) || !gdn_rows_ok(dq, gran) || !gdn_rows_ok(dk, gran) || !gdn_rows_ok(dv, gran))
        return TT_E_ARG;
    // the outputs' heads are contiguous and their rows at most 2^30 elements apart
    const tt_tensor* outs[3] = {&dq, &dk, &dv};
    for (const tt_tensor* t : outs) {
        if (t->stride_head != 128) return TT_E_UNSUPPORTED;
        if (t->stride_tok > (int64_t(1) << 30)) return TT_E_ARG;
    }
    if (!aligned(ws, 16) || !aligned(dg, 4) || !aligned(dbeta, 4)) return TT_E_ARG;
    if ((d_node_states && !aligned(d_node_states, 16)) || (d_initial_state && !aligned(d_initial_state, 16)))
        return TT_E_ARG;
    d.dq_st = (int)dq.stride_tok;
    d.dk_st = (int)dk.stride_tok;
    d.dv_st = (int)dv.stride_tok;
    if (p->d_states_last_only != 0 && p->d_states_last_only != 1) return TT_E_ARG;
    d.d_states = d_node_states;
    d.d_states_last = p->d_states_last_only;
    d.d_init = d_initial_state;
    return TT_OK;
}

int tt_gdn_tree_bwd(const tt_gdn_problem* p, tt_tensor d_o, tt_tensor dq, tt_tensor dk, tt_tensor dv, float* dg,
                    float* dbeta, const float* d_node_states, float* d_initial_state, void* ws, size_t ws_bytes,
                    void* stream) {
    GdnDev d;
    int rc = gdn_problem(p, d);
    if (rc != TT_OK) return rc;
    if ((rc = gdn_bwd_args(p, d, d_o, dq, dk, dv, dg, dbeta, d_node_states, d_initial_state, ws)) != TT_OK)
        return rc;
    if (ws_bytes < tt_gdn_bwd_ws_bytes_impl(p->n_chunks, p->n_nodes, p->n_heads_v, true, p->reference_truncated != 0)) return TT_E_WORKSPACE;
    return tt_gdn_bwd_launch(d, p->level_offsets, p->n_levels, d_o.ptr, d_o.stride_tok, d_o.stride_head,
                             const_cast<void*>(dq.ptr), const_cast<void*>(dk.ptr), const_cast<void*>(dv.ptr), dg, dbeta, nullptr, (float*)ws, (hipStream_t)stream);
}

int tt_gdn_tree_bwd_saved(const tt_gdn_problem* p, tt_tensor d_o, tt_tensor dq, tt_tensor dk, tt_tensor dv,
                          float* dg, float* dbeta, const float* d_node_states, float* d_initial_state,
                          const void* saved, size_t saved_bytes, void* ws, size_t ws_bytes, void* stream) {
    GdnDev d;
    int rc = gdn_problem(p, d);
    if (rc != TT_OK) return rc;
    if ((rc = gdn_bwd_args(p, d, d_o, dq, dk, dv, dg, dbeta, d_node_states, d_initial_state, ws)) != TT_OK)
        return rc;
    if (!saved || !aligned(saved, 16)) return TT_E_ARG;
    if (saved_bytes < tt_gdn_saved_bytes_impl(p->n_chunks, p->n_heads_v, p->reference_truncated != 0)) return TT_E_WORKSPACE;
    if (ws_bytes < tt_gdn_bwd_ws_bytes_impl(p->n_chunks, p->n_nodes, p->n_heads_v, false, p->reference_truncated != 0)) return TT_E_WORKSPACE;
    return tt_gdn_bwd_launch(d, p->level_offsets, p->n_levels, d_o.ptr, d_o.stride_tok, d_o.stride_head,
                             const_cast<void*>(dq.ptr), const_cast<void*>(dk.ptr), const_cast<void*>(dv.ptr), dg, dbeta, (const float*)saved, (float*)ws, (hipStream_t)stream);
}

}  // extern "C"

static int conv_problem(const tt_conv_problem* p, ConvDev& d) {
    if (!p) return TT_E_ARG;
    if (p->dtype != TT_DTYPE_BF16 && p->dtype != TT_DTYPE_F32) return TT_E_UNSUPPORTED;
    if (p->kernel_size < 1 || p->kernel_size > 4) return TT_E_UNSUPPORTED;
    if (p->n_tokens < 1 || p->n_channels < 4 || (p->n_channels % 4)) return TT_E_ARG;
    if (!p->x || !p->weight || !p->tok_prev) return TT_E_ARG;
    if (p->x_stride_tok < p->n_channels || (p->x_stride_tok % 4)) return TT_E_ARG;
    const size_t ea = p->dtype == TT_DTYPE_BF16 ? 8 : 16;
    if (!aligned(p->x, ea) || !aligned(p->weight, p->dtype == TT_DTYPE_BF16 ? 2 : 4)) return TT_E_ARG;
    if (p->bias && !aligned(p->bias, p->dtype == TT_DTYPE_BF16 ? 2 : 4)) return TT_E_ARG;
    d.x = p->x; d.x_st = p->x_stride_tok;
    d.weight = p->weight;
    d.bias = p->bias;
    d.prev = p->tok_prev;
    d.next_off = p->tok_next_off;
    d.next = p->tok_next;
    d.dtype = p->dtype;
    d.n_tokens = p->n_tokens;
    d.n_ch = p->n_channels;
    d.k = p->kernel_size;
    return TT_OK;
}

extern "C" {

int tt_tree_conv_fwd(const tt_conv_problem* p, void* y, int64_t y_stride_tok, void* stream) {
    ConvDev d;
    const int rc = conv_problem(p, d);
    if (rc != TT_OK) return rc;
    if (!y || y_stride_tok < p->n_channels || (y_stride_tok % 4) ||
        !aligned(y, p->dtype == TT_DTYPE_BF16 ? 8 : 16))
        return TT_E_ARG;
    return tt_conv_fwd_launch(d, y, y_stride_tok, (hipStream_t)stream);
}

size_t tt_tree_conv_bwd_workspace_bytes(const tt_conv_problem* p) {
    if (!p || p->n_tokens < 1 || p->n_channels < 1 || p->kernel_size < 1 || p->kernel_size > 4) return 0;
    return tt_conv_bwd_ws_bytes_impl(p->n_tokens, p->n_channels, p->kernel_size);
}

int tt_tree_conv_bwd(const tt_conv_problem* p, const void* dy, int64_t dy_stride_tok, void* dx, float* dweight,
                     float* dbias, void* ws, size_t ws_bytes, void* stream) {
    ConvDev d;
    const int rc = conv_problem(p, d);
    if (rc != TT_OK) return rc;
    if (!p->tok_next_off || !p->tok_next || !dy || !dx || !dweight || !ws) return TT_E_ARG;
    const size_t ea = p->dtype == TT_DTYPE_BF16 ? 8 : 16;
    if (dy_stride_tok < p->n_channels || (dy_stride_tok % 4) || !aligned(dy, ea) || !aligned(dx, ea) ||
        !aligned(ws, 16) || !aligned(dweight, 4) || (dbias && !aligned(dbias, 4)))
        return TT_E_ARG;
    if (ws_bytes < tt_conv_bwd_ws_bytes_impl(p->n_tokens, p->n_channels, p->kernel_size)) return TT_E_WORKSPACE;
    return tt_conv_bwd_launch(d, dy, dy_stride_tok, dx, dweight, dbias, (float*)ws, (hipStream_t)stream);
}

}  // extern "C"

static bool prologue_tensor_ok(const tt_tensor& t, int64_t gran) {
    return t.ptr && t.stride_tok >= 128 && t.stride_head >= 128 && !(t.stride_tok % gran) &&
           !(t.stride_head % gran) && aligned(t.ptr, 16);
}

static int prologue_problem(const tt_prologue_problem* p, PrologueDev& d) {
    if (!p) return TT_E_ARG;
    if (p->dtype != TT_DTYPE_BF16 && p->dtype != TT_DTYPE_F32) return TT_E_UNSUPPORTED;
    if (p->head_dim != 128) return TT_E_UNSUPPORTED;
    if (p->n_tokens < 1 || p->n_heads_q < 1 || p->n_heads_kv < 1) return TT_E_ARG;
    if ((int64_t)p->n_tokens * (p->n_heads_q + p->n_heads_kv) > INT32_MAX) return TT_E_ARG;
    if (!(p->eps_q >= 0.0f) || !(p->eps_k >= 0.0f)) return TT_E_ARG;
    const int64_t gran = p->dtype == TT_DTYPE_BF16 ? 8 : 4;
    if (!prologue_tensor_ok(p->q, gran) || !prologue_tensor_ok(p->k, gran)) return TT_E_ARG;
    if (!p->q_weight || !p->k_weight || !p->cos || !p->sin) return TT_E_ARG;
    if (!aligned(p->q_weight, 16) || !aligned(p->k_weight, 16) || !aligned(p->cos, 16) || !aligned(p->sin, 16) ||
        p->cs_stride_tok < 128 || (p->cs_stride_tok % gran))
        return TT_E_ARG;
    d.q = p->q.ptr; d.q_st = p->q.stride_tok; d.q_sh = p->q.stride_head;
    d.k = p->k.ptr; d.k_st = p->k.stride_tok; d.k_sh = p->k.stride_head;
    d.qw = p->q_weight; d.kw = p->k_weight;
    d.cos = p->cos; d.sin = p->sin; d.cs_st = p->cs_stride_tok;
    d.eps_q = p->eps_q; d.eps_k = p->eps_k;
    d.dtype = p->dtype;
    d.n_tokens = p->n_tokens;
    d.hq = p->n_heads_q;
    d.hkv = p->n_heads_kv;
    d.n_rows = p->n_tokens * (p->n_heads_q + p->n_heads_kv);
    return TT_OK;
}

extern "C" {

int tt_qk_prologue_fwd(const tt_prologue_problem* p, void* q_out, void* k_out, void* stream) {
    PrologueDev d;
    const int rc = prologue_problem(p, d);
    if (rc != TT_OK) return rc;
    if (!q_out || !k_out || !aligned(q_out, 16) || !aligned(k_out, 16)) return TT_E_ARG;
    return tt_prologue_fwd_launch(d, q_out, k_out, (hipStream_t)stream);
}

size_t tt_qk_prologue_bwd_workspace_bytes(const tt_prologue_problem* p) {
    return p ? tt_prologue_bwd_ws_bytes_impl() : 0;
}

int tt_qk_prologue_bwd(const tt_prologue_problem* p, tt_tensor dq_out, tt_tensor dk_out, void* dq_raw, void* dk_raw,
                       float* dq_weight, float* dk_weight, void* ws, size_t ws_bytes, void* stream) {
    PrologueDev d;
    const int rc = prologue_problem(p, d);
    if (rc != TT_OK) return rc;
    const int64_t gran = p->dtype == TT_DTYPE_BF16 ? 8 : 4;
    if (!prologue_tensor_ok(dq_out, gran) || !prologue_tensor_ok(dk_out, gran)) return TT_E_ARG;
    if (!dq_raw || !dk_raw || !dq_weight || !dk_weight || !ws || !aligned(dq_raw, 16) || !aligned(dk_raw, 16) ||
        !aligned(ws, 16) || !aligned(dq_weight, 4) || !aligned(dk_weight, 4))
        return TT_E_ARG;
    if (ws_bytes < tt_prologue_bwd_ws_bytes_impl()) return TT_E_WORKSPACE;
    return tt_prologue_bwd_launch(d, dq_out.ptr, dq_out.stride_tok, dq_out.stride_head, dk_out.ptr,
                                  dk_out.stride_tok, dk_out.stride_head, dq_raw, dk_raw, dq_weight, dk_weight,
                                  (float*)ws, (hipStream_t)stream);
}

int tt_ce_rows(int32_t dtype, const void* logits, int64_t ld, int32_t n_rows, int32_t vocab, const int32_t* labels,
               const float* row_scale, int32_t ignore_index, float* loss, void* grad, int64_t ldg, void* stream) {
    if (dtype != TT_DTYPE_BF16 && dtype != TT_DTYPE_F32) return TT_E_UNSUPPORTED;
    if (n_rows < 1 || vocab < 1 || !logits || !labels || !row_scale || !loss || !grad) return TT_E_ARG;
    const int64_t gran = dtype == TT_DTYPE_BF16 ? 8 : 4;
    if (ld < vocab || ldg < vocab || (ld % gran) || (ldg % gran) || !aligned(logits, 16) || !aligned(grad, 16) ||
        !aligned(labels, 4) || !aligned(row_scale, 4) || !aligned(loss, 4))
        return TT_E_ARG;
    return tt_ce_rows_launch(dtype, logits, ld, n_rows, vocab, labels, row_scale, ignore_index, loss, grad, ldg,
                             (hipStream_t)stream);
}

int tt_selftest_mfma32(const void* a, const void* b, float* d, void* stream) {
    if (!a || !b || !d || !aligned(a, 2) || !aligned(b, 2) || !aligned(d, 4)) return TT_E_ARG;
    return tt_selftest_mfma_launch(a, b, d, (hipStream_t)stream);
}

}  // extern "C"
