// Internal launchers shared between the translation units of the library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tree_attn.h"

// Device-side view of a tt_attn_problem (passed to kernels by value).
struct AttnDev {
    const void* q; int64_t q_st, q_sh;
    const void* k; int64_t k_st, k_sh;
    const void* v; int64_t v_st, v_sh;
    const void* kp; int64_t kp_st, kp_sh;
    const void* vp; int64_t vp_st, vp_sh;
    const int32_t* key_lo;
    const int32_t* key_hi;
    const int32_t* row_cnt;   // plan: per query block, number of key tiles
    const int32_t* row_order; // plan: query blocks, heaviest first
    const int32_t* row_list;  // plan: per query block, (kt << 1) | full
    const int32_t* kb_qlo;    // plan: visible query range per 128-key tile
    const int32_t* kb_qhi;
    const int32_t* kb_order;  // plan: key tiles, widest range first
    const int32_t* kb_base;   // plan: first dK/dV work item per key tile (kb_order order)
    const int32_t* kb_srank;  // plan: rank of each key tile among the split ones (-1: not split)
    const int2* kb_item;      // plan: (tile rank, chunk) of each dK/dV work item, in the order they are taken
    const int32_t* n_items;   // plan: number of dK/dV work items
    int n_q, n_past, n_keys, hq, hkv, rep, n_qb, n_kt, n_kb;
    float scale;
};

struct BwdDev {
    const void* o;            // [n_q, hq, 128] contiguous
    const float* lse;         // [hq, n_q]
    const void* dout; int64_t do_st, do_sh;
    void* dq;                 // [n_q, hq, 128]
    void* dk;                 // [n_q, hkv, 128]
    void* dv;
    float* dk_acc;            // [n_past, hkv, 128] fp32 (+=), may be null
    float* dv_acc;
    float* delta;             // workspace [hq, n_q]: rowsum(dO * O)
    float* dk_ws;             // workspace [split_cap * 128, hkv, 128] fp32: split key tiles' dK, tile of
    float* dv_ws;             //   split rank r in rows 128 r .. 128 r + 127; the same for dV
    int64_t split_cap;        // split tiles the workspace holds (tiles beyond write nothing; their keys get NaN)
    float* dk_slot;           // deterministic mode: [tt_det_slots, 128, hkv, 128] fp32, chunks >= 1
    float* dv_slot;           //   of split key tiles (null otherwise)
    int64_t det_cap;          // deterministic mode: slots the workspace holds (tiles beyond get NaN)
    int parts;                // OR of TT_BWD_DELTA / _DQ / _DKDV (never 0 here)
    int det;                  // TT_BWD_DETERMINISTIC given (split tiles summed in chunk order)
    float* dq_part;           // bf16 with tt_key_splits > 1: [splits, n_q, hq, 128] fp32 dQ partials
    int n_split;              // tt_key_splits of the problem (bf16), else 1
    int zero_in_dq;           // the dQ pass clears the split sums for the dK/dV pass of the same call
};

// Key-range split of the bf16 forward (tt_key_splits > 1): per split, the
// unnormalised output [n_q, hq, 128] and the row max (log2 units) and row sum
// [hq, n_q] it is taken against, all fp32.
struct FwdSplit {
    float* o;
    float* m;
    float* l;
    int n;
};

// Device-side view of a tt_gdn_problem.
struct GdnDev {
    const void* q; int64_t q_st, q_sh;
    const void* k; int64_t k_st, k_sh;
    const void* v; int64_t v_st, v_sh;
    const float* g; int64_t g_st;          // [T, Hv] (token stride, heads contiguous)
    const float* beta; int64_t b_st;
    const int32_t* node_start;
    const int32_t* node_len;
    const int32_t* parent;
    const int32_t* level_nodes;            // nodes grouped by tree depth
    const int32_t* node_chunk0;            // first chunk of each node
    const int32_t* chunk_node;             // node of each chunk
    const int32_t* child_off;              // children of node i: child[child_off[i] .. child_off[i+1]) (backward)
    const int32_t* child;
    int dtype, n_tokens, n_nodes, n_chunks, hk, hv, rep, l2;
    int trunc;                             // the reference's I + R + R^2 per node (else the exact rule)
    float scale;
    // Backward outputs dq, dk [T, Hk, 128] and dv [T, Hv, 128]: token
    // strides in elements (heads contiguous; the pointers travel as launch
    // arguments). 32-bit, as every scalar register kept live through the
    // backward chunk kernel's loop costs it schedule quality.
    int dq_st, dk_st, dv_st;
    // The state every root starts from ([Hv, 128, 128] float32; null: zero),
    // the incoming gradient of the node states ([n_nodes, Hv, 128, 128];
    // null: none) and where the backward writes the gradient of the initial
    // state ([Hv, 128, 128]; null: not wanted).
    const float* init;
    const float* d_states;
    int d_states_last;                     // d_states is the last node's [Hv, 128, 128] alone
    float* d_init;
};

// Device-side view of a tt_conv_problem.
struct ConvDev {
    const void* x; int64_t x_st;           // [T, C] rows, channels contiguous
    const void* weight;                    // [C, K]
    const void* bias;                      // [C] or null
    const int32_t* prev;                   // [T] path predecessor (-1: none)
    const int32_t* next_off;               // [T + 1] successor lists (backward)
    const int32_t* next;
    int dtype, n_tokens, n_ch, k;
};

size_t tt_conv_bwd_ws_bytes_impl(int n_tokens, int n_ch, int k);
int tt_conv_fwd_launch(const ConvDev& d, void* y, int64_t y_st, hipStream_t s);
int tt_conv_bwd_launch(const ConvDev& d, const void* dy, int64_t dy_st, void* dx, float* dw, float* db, float* ws,
                       hipStream_t s);

// Device-side view of a tt_prologue_problem.
struct PrologueDev {
    const void* q; int64_t q_st, q_sh;     // projected q [T, Hq, 128]
    const void* k; int64_t k_st, k_sh;     // projected k [T, Hkv, 128]
    const void* qw; const void* kw;        // norm weights [128]
    const void* cos; const void* sin; int64_t cs_st;   // [T, 128]
    float eps_q, eps_k;
    int dtype, n_tokens, hq, hkv, n_rows;  // n_rows = T * (Hq + Hkv)
};

size_t tt_prologue_bwd_ws_bytes_impl();
int tt_prologue_fwd_launch(const PrologueDev& p, void* q_out, void* k_out, hipStream_t s);
int tt_prologue_bwd_launch(const PrologueDev& p, const void* dq_out, int64_t dq_st, int64_t dq_sh, const void* dk_out,
                           int64_t dk_st, int64_t dk_sh, void* dq_raw, void* dk_raw, float* dqw, float* dkw,
                           float* ws, hipStream_t s);

int tt_ce_rows_launch(int dtype, const void* logits, int64_t ld, int n_rows, int vocab, const int32_t* labels,
                      const float* row_scale, int ignore_index, float* loss, void* grad, int64_t ldg,
                      hipStream_t s);

size_t tt_gdn_ws_bytes_impl(int n_chunks, int n_heads_v, bool trunc);
int tt_gdn_fwd_launch(const GdnDev& d, const int32_t* level_offsets, int n_levels, void* out, float* states,
                      float* ws, hipStream_t s);
size_t tt_gdn_saved_bytes_impl(int n_chunks, int n_heads_v, bool trunc);
int tt_gdn_fwd_save_launch(const GdnDev& d, const int32_t* level_offsets, int n_levels, void* out, float* states,
                           float* saved, hipStream_t s);
size_t tt_gdn_bwd_ws_bytes_impl(int n_chunks, int n_nodes, int n_heads_v, bool recompute, bool trunc);
int tt_gdn_bwd_launch(const GdnDev& d, const int32_t* level_offsets, int n_levels, const void* d_o, int64_t do_st,
                      int64_t do_sh, void* dq, void* dk, void* dv, float* dg, float* dbeta, const float* saved,
                      float* ws, hipStream_t s);

// The truncated (reference) mode's node-level terms (tt_gdn_trunc.hip). The
// forward part fills the U and W slots of the chunk terms in `prep`; the
// backward part turns dF = [dV' | dW] into dv, dbeta (complete) and the
// correction's dk^ and node-level dG suffix sums, which the chunk backward adds.
struct GdnTruncBwd {
    float* gn;            // [chunk, Hv, 32] node-level decay (from the forward)
    float* y1;            // [chunk, Hv, 32, 256] R Y0 (from the forward)
    float* dvp;           // [chunk, Hv, 32, 128] dV'
    float* dw;            // [chunk, Hv, 32, 128] dW
    float* df1;           // [chunk, Hv, 32, 256] scratch
    float* dy0;           // [chunk, Hv, 32, 256] scratch
    float* dkr;           // [chunk, Hv, 32, 128] out
    float* dgn;           // [chunk, Hv, 32] out
};
int tt_gdn_trunc_fwd_launch(const GdnDev& d, float* prep, float* gn, float* y1, hipStream_t s);
int tt_gdn_trunc_bwd_launch(const GdnDev& d, const GdnTruncBwd& w, void* dv, float* dbeta, hipStream_t s);

size_t tt_meta_ws_bytes_impl(int n);
int tt_meta_build_impl(const int32_t* len, const int32_t* par, int n, int T, int pos_offset, int32_t* start,
                       int32_t* off, int32_t* hend, int32_t* pos, int32_t* node_of, int32_t* horizon,
                       int32_t* status, void* ws, hipStream_t s);
int tt_keys_build_impl(const float* bias, int n_past, const int32_t* horizon, int n_q, int32_t* key_lo,
                       int32_t* key_hi, int32_t* status, hipStream_t s);
int tt_dense_mask_impl(const int32_t* key_lo, const int32_t* key_hi, int n_keys, int n_q, uint8_t* mask,
                       hipStream_t s);
size_t tt_plan_bytes_impl(int n_q, int n_keys);
int tt_trees_build_impl(const tt_tree_job* jobs, int n_jobs, hipStream_t s);
bool tt_trees_job_fits(int n_tokens, int n_keys);
int tt_plan_build_impl(const int32_t* key_lo, const int32_t* key_hi, int n_keys, int n_q, void* plan,
                       hipStream_t s);

int tt_fwd_bf16_launch(const AttnDev& a, void* o, float* lse, const FwdSplit& sp, hipStream_t s);
int tt_bwd_bf16_launch(const AttnDev& a, const BwdDev& b, hipStream_t s);
int tt_fwd_f32_launch(const AttnDev& a, void* o, float* lse, hipStream_t s);
int tt_bwd_f32_launch(const AttnDev& a, const BwdDev& b, hipStream_t s);
int tt_selftest_mfma_launch(const void* a, const void* b, float* d, hipStream_t s);
