/* tree_attn.h — C ABI of the MI355X tree-attention engine (gfx950, HIP).
 *
 * Every pointer argument is a DEVICE pointer allocated and owned by the caller
 * unless stated otherwise; `stream` is a hipStream_t passed as void*. Calls
 * only enqueue work on `stream` (no host synchronisation, no allocation: the
 * caller supplies every workspace). Arguments are validated on the host before
 * any HIP call; a failed check returns a negative TT_E_* code and launches
 * nothing. No C++ exception crosses this boundary. The library keeps no
 * mutable global state, except the per-GPU scratch array of
 * tt_attn_bwd_noalloc (the one entry point that takes no workspace).
 *
 * Visibility model. A problem has n_q query tokens (the DFS-packed tokens of
 * one tree or one partition) and n_keys = n_past + n_q keys: first the
 * gateway ("past") keys, then the query tokens themselves. Key j is visible to
 * query i iff  key_lo[j] <= i < key_hi[j]. For the tree's own tokens this is
 * the closed form of the reference's dense mask, mask[i,j] <=> j <= i < h[j]
 * with h[j] the exclusive end of the subtree of j's node; a gateway key is
 * visible to every query or to none.
 */
#ifndef TREE_ATTN_H
#define TREE_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    TT_OK = 0,
    TT_E_ARG = -1,          /* bad size, null pointer, stride or layout */
    TT_E_UNSUPPORTED = -2,  /* dtype / head_dim / head ratio not built */
    TT_E_HIP = -3,          /* a HIP launch failed */
    TT_E_WORKSPACE = -4     /* workspace or plan buffer too small */
};

enum { TT_DTYPE_F32 = 0, TT_DTYPE_BF16 = 1 };

/* Parts of the backward (tt_attn_problem.bwd_parts); they must run in this
 * order, each after the previous one on the same stream. Requested in one
 * call, TT_BWD_DELTA and TT_BWD_DQ run as one bf16 kernel (the dQ pass
 * computes the row sums it needs and stores them for TT_BWD_DKDV). */
enum {
    TT_BWD_DELTA = 1,   /* rowsum(dO * O) into the workspace */
    TT_BWD_DQ = 2,      /* dQ (reads the workspace) */
    TT_BWD_DKDV = 4,    /* dK, dV and gateway accumulation (reads the workspace) */
    TT_BWD_DETERMINISTIC = 8   /* modifier, OR'ed with the parts (alone: every part): dK/dV and
                                  gateway sums in a fixed order (bf16 and fp32), so repeated calls on
                                  the same inputs are bitwise equal (more workspace; see tt_attn_bwd) */
};

/* Device-side status bits written by tt_meta_build / tt_keys_build. */
enum {
    TT_STATUS_BAD_LEN = 1,      /* a node with length < 1 */
    TT_STATUS_BAD_PARENT = 2,   /* not DFS pre-order: a parent outside [-1, self), or a node that
                                   comes after its parent's subtree has closed (parents [-1, 0, 0, 1]) */
    TT_STATUS_BAD_TOTAL = 4,    /* sum of node lengths != n_tokens */
    TT_STATUS_BAD_BIAS = 8      /* a gateway bias that is neither 0 nor -inf */
};

int tt_abi_version(void);
const char* tt_strerror(int code);

/* ---- (1) DFS metadata -----------------------------------------------------
 * Replaces build_dfs_tree_info (dfs_tree_forward.py:91-184): depth-based
 * positions (:113-139) and, instead of the dense [N,N] mask (:161-172), the
 * per-token subtree horizon h. Also the per-partition position offset of
 * tree_grad_hybrid.py:307-310 (pos_offset).
 * Input: node_len[n_nodes], node_parent[n_nodes] in DFS pre-order
 * (-1 for a root; parent < child, and every node between a parent and its
 * child is a descendant of that parent: the order build_dfs_tree_info
 * produces). Output (int32):
 *   node_start[n], node_off[n] (sum of ancestor lengths), node_hend[n]
 *   (exclusive end token of the node's subtree), pos[T] = pos_offset +
 *   node_off + offset-in-node, node_of[T], horizon[T] = node_hend[node_of].
 * status: one device int32, OR-ed with TT_STATUS_* bits (caller zeroes it).
 */
size_t tt_meta_workspace_bytes(int32_t n_nodes);
int tt_meta_build(const int32_t* node_len, const int32_t* node_parent, int32_t n_nodes,
                  int32_t n_tokens, int32_t pos_offset,
                  int32_t* node_start, int32_t* node_off, int32_t* node_hend,
                  int32_t* pos, int32_t* node_of, int32_t* horizon, int32_t* status,
                  void* ws, size_t ws_bytes, void* stream);

/* Per-key visible query intervals for [gateway | own] keys. Replaces the
 * additive mask assembly of tree_grad_hybrid.py:312-317 and
 * dfs_tree_forward.py:548-550: past_bias[j] (0 or -inf, float32, may be NULL
 * when n_past == 0) -> [0, n_q) or empty; own key j -> [j, horizon[j]). */
int tt_keys_build(const float* past_bias, int32_t n_past, const int32_t* horizon, int32_t n_q,
                  int32_t* key_lo, int32_t* key_hi, int32_t* status, void* stream);

/* Dense expansion mask[i, j] = key_lo[j] <= i < key_hi[j] as uint8 [n_q, n_keys]:
 * the reference's attn_mask_bool (dfs_tree_forward.py:161-172) for
 * compatibility and parity checks; the attention path never builds it. */
int tt_meta_dense_mask(const int32_t* key_lo, const int32_t* key_hi, int32_t n_keys, int32_t n_q,
                       uint8_t* mask, void* stream);

/* ---- tile plan -------------------------------------------------------------
 * Block-sparsity map of the (query block x key tile) grid: empty tiles are
 * skipped, full tiles run unmasked, partial tiles apply the interval test in
 * the tile. Opaque device buffer; its first 8 bytes hold the uint64 count of
 * visible (query, key) pairs per head, P = sum_j |[lo_j,hi_j) & [0,n_q)|. */
size_t tt_plan_bytes(int32_t n_q, int32_t n_keys);
int tt_plan_build(const int32_t* key_lo, const int32_t* key_hi, int32_t n_keys, int32_t n_q,
                  void* plan, size_t plan_bytes, void* stream);

/* ---- several trees in one call --------------------------------------------
 * tt_meta_build + tt_keys_build + tt_plan_build for up to TT_TREE_JOBS_MAX
 * trees in three launches in all: the per-partition DFS info and gateway
 * masks of tree_grad_hybrid (_dfs_info_for_partition and the bias assembly,
 * tree_grad_hybrid.py:102-153, :193-209, :312-317) for every partition of a
 * step at once. Each job has the inputs and outputs of the three calls, with
 * two differences: key_lo/key_hi are filled from the metadata directly, and
 * *status is overwritten (not OR-ed; no zeroing needed). A job must have
 * n_tokens <= 65536 and at most 2048 query blocks of 128 and key tiles of 128
 * (n_past + n_tokens <= 262144); larger trees use the separate calls
 * (TT_E_UNSUPPORTED). */
#define TT_TREE_JOBS_MAX 16
typedef struct tt_tree_job {
    const int32_t* node_len;    /* [n_nodes], DFS pre-order as for tt_meta_build */
    const int32_t* node_parent;
    const float* past_bias;     /* [n_past] 0 or -inf; NULL when n_past == 0 */
    int32_t* node_start;        /* [n_nodes] each */
    int32_t* node_off;
    int32_t* node_hend;
    int32_t* pos;               /* [n_tokens] each; node_of may be NULL */
    int32_t* node_of;
    int32_t* horizon;
    int32_t* key_lo;            /* [n_past + n_tokens] each */
    int32_t* key_hi;
    int32_t* status;            /* one int32, overwritten with the TT_STATUS_* bits */
    void* plan;                 /* tt_plan_bytes(n_tokens, n_past + n_tokens) */
    size_t plan_bytes;
    void* ws;                   /* tt_meta_workspace_bytes(n_nodes) */
    size_t ws_bytes;
    int32_t n_nodes, n_tokens, pos_offset, n_past;
} tt_tree_job;
int tt_trees_build(const tt_tree_job* jobs, int32_t n_jobs, void* stream);

/* ---- (2)+(3) tree-masked GQA attention -------------------------------------
 * Replaces repeat_kv + F.scaled_dot_product_attention(attn_mask=dense) and its
 * autograd backward (transformers integrations/sdpa_attention.py:79-175,
 * models/qwen3/modeling_qwen3.py:173-207) as called from Qwen3Attention
 * (models/qwen3/modeling_qwen3.py:262-276), and GatewayCache.update's cat of
 * gateway KV with new KV (tree_grad_ckpt_opath.py:92-114): the gateway is
 * the `k_past/v_past` segment, read in place. */
typedef struct tt_tensor {
    const void* ptr;        /* element [t][h][d] at ptr + t*stride_tok + h*stride_head + d */
    int64_t stride_tok;     /* in elements; >= 128, a multiple of 8 (bf16) or 4 (fp32), < 2^23 (bf16) or 2^22 (fp32) */
    int64_t stride_head;    /* in elements; >= 128, a multiple of 8 (bf16) or 4 (fp32); ptr 16-byte aligned */
} tt_tensor;

typedef struct tt_attn_problem {
    int32_t dtype;          /* TT_DTYPE_BF16 or TT_DTYPE_F32; every tensor has it */
    int32_t n_q;            /* query tokens (= own keys) */
    int32_t n_past;         /* gateway keys, 0 for none */
    int32_t n_heads_q;      /* Hq */
    int32_t n_heads_kv;     /* Hkv, Hq % Hkv == 0 (GQA: q head h reads kv head h / (Hq/Hkv)) */
    int32_t head_dim;       /* 128 */
    float scale;            /* softmax scale, head_dim ** -0.5 in Qwen3 */
    int32_t bwd_parts;      /* tt_attn_bwd only: OR of TT_BWD_* (0 = all parts) */
    tt_tensor q, k, v;      /* q: n_q x Hq; k, v: n_q x Hkv */
    tt_tensor k_past, v_past; /* n_past x Hkv; ignored when n_past == 0 */
    const int32_t* key_lo;  /* [n_past + n_q] */
    const int32_t* key_hi;
    const void* plan;       /* built by tt_plan_build for (key_lo, key_hi) */
    size_t plan_bytes;
    int64_t det_slots;      /* tt_attn_bwd with TT_BWD_DETERMINISTIC: the partial-sum slots to reserve,
                               from tt_attn_det_slots for the tree; 0: the bound that holds for any tree */
    int64_t split_tiles;    /* tt_attn_bwd: the split key tiles the fp32 split sums hold, from
                               tt_attn_split_tiles for the tree; 0: every key tile */
} tt_attn_problem;

/* o: [n_q, Hq, head_dim] contiguous, problem dtype; lse: [Hq, n_q] float32
 * (natural-log softmax normaliser, saved for the backward).
 * Small bf16 problems, with at most 256 (128-query block, q head) pairs,
 * cut each pair's keys into S = 4 ranges computed in parallel and merged in
 * a fixed order (deterministic; the rounding differs from an unsplit run).
 * Their partials need a workspace of tt_attn_fwd_workspace_bytes: S * n_q *
 * Hq * 520 bytes (each of three parts rounded up to 256), 0 for every other
 * problem, when ws may be NULL. ws is 16-byte aligned; a smaller ws_bytes
 * returns TT_E_WORKSPACE. */
size_t tt_attn_fwd_workspace_bytes(const tt_attn_problem* p);
int tt_attn_fwd(const tt_attn_problem* p, void* o, float* lse, void* ws, size_t ws_bytes, void* stream);

/* Backward for upstream gradient d_o (n_q x Hq, strides given). Writes
 * dq [n_q,Hq,D], dk/dv [n_q,Hkv,D] (contiguous, problem dtype, overwritten).
 * Gateway gradients are ADDED in float32 to dk_past_acc/dv_past_acc
 * [n_past, Hkv, D] contiguous, 16-byte aligned (the fp32 hook accumulation of
 * tree_grad_hybrid.py:220-225, kept on the device); pass NULL to drop them.
 * Within one call every accumulator element has one writer at a time (plain
 * read-add-write, or fp32 atomics where a key's query range is split), so
 * calls may share accumulators only when ordered on one stream: two calls in
 * flight at once on different streams must not add into the same
 * accumulators.
 * ws must be 16-byte aligned. dq has one writer per element (deterministic;
 * the small bf16 problems whose forward splits keys, above, split the dQ
 * pass the same way, with S * n_q * Hq * 512 more workspace bytes, and add
 * the partials in a fixed order);
 * so do dk and dv, except that keys whose visible query range spans more
 * than W queries, W = half the largest power of two <= n_q clamped to
 * [256, 4096] (split into several work items), sum their dK/dV partials
 * with fp32 atomics, so their rounding can vary from run to run (both
 * dtypes). With TT_BWD_DETERMINISTIC in bwd_parts each of those work items
 * stores its partial sums in a slot of its own and one pass adds them in
 * work-item order: no atomics, bitwise-repeatable dk, dv and gateway sums.
 * The workspace (tt_attn_bwd_workspace_bytes of the problem with the bit set)
 * then grows by 2 * S * 128 * Hkv * 512 bytes: S = det_slots, the exact count
 * of such later work items that tt_attn_det_slots computes on the host from
 * the topology (46 on the 16K agent tree), or with det_slots = 0 the bound
 * n_kb * floor((n_q - 1) / W), n_kb = ceil((n_past + n_q) / 128) (about 4x
 * the bf16 workspace at n_q = 16K). A det_slots below what the plan needs
 * never writes past the workspace: the key tiles whose slots do not fit get
 * NaN gradients (dk, dv, or the gateway accumulators).
 * Only the TT_BWD_DKDV part depends on the bit. */
size_t tt_attn_bwd_workspace_bytes(const tt_attn_problem* p);

/* Host only (no device work): the split_tiles a DFS pre-order forest needs:
 * its 128-key tiles whose visible query range spans more than W queries (see
 * above), whose fp32 dK/dV sums take 2 * 128 * Hkv * 512 bytes of the
 * workspace each (14 tiles, 14 MiB, on the 16K agent tree; with split_tiles =
 * 0 every key tile is counted: 128 MiB there). A split_tiles below what the
 * plan needs never writes past the workspace: the tiles beyond it get NaN
 * gradients (dk, dv; the gateway accumulators in deterministic mode).
 * Same arguments, visibility and errors as tt_attn_det_slots below. */
int tt_attn_split_tiles(const int32_t* node_len, const int32_t* parent, int n_nodes, const float* past_bias,
                        int n_past, int64_t* tiles);

/* Host only (no device work): the det_slots a DFS pre-order forest needs,
 * from node_len/parent [n_nodes] and the gateway bias past_bias [n_past]
 * (0 or -inf per gateway key, host memory; NULL: every gateway key visible),
 * the visibility the tt_meta_build/tt_keys_build/tt_plan_build chain derives
 * on the device: own key j is seen by queries [j, subtree end of its node),
 * a visible gateway key by every query. No counterpart in the reference,
 * whose determinism is torch.use_deterministic_algorithms
 * (verify_hybrid.py:20-25); this sizes the workspace of ours by the tree.
 * TT_OK, or TT_E_ARG for a null pointer, n_nodes < 1, n_past < 0, a length
 * < 1, a parent outside [-1, node) or more than 2^30 keys. */
int tt_attn_det_slots(const int32_t* node_len, const int32_t* parent, int n_nodes, const float* past_bias,
                      int n_past, int64_t* slots);
int tt_attn_bwd(const tt_attn_problem* p, const void* o, const float* lse, tt_tensor d_o,
                void* dq, void* dk, void* dv, float* dk_past_acc, float* dv_past_acc,
                void* ws, size_t ws_bytes, void* stream);

/* No counterpart in the reference: tt_attn_bwd for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments, results and validation as
 * tt_attn_bwd, without ws / ws_bytes: the workspace is a scratch array of
 * TT_NOALLOC_SCRATCH_MB MiB on each GPU, taken by the first call on that GPU
 * (the array's code object loads on first use: a process that never calls
 * this entry point never holds it) and held until the process ends (the
 * current device's, hipGetDevice; `stream` must belong to it). A problem whose tt_attn_bwd_workspace_bytes exceeds it
 * returns TT_E_WORKSPACE (either dtype needs 4 * Hq * n_q bytes plus the
 * split sums, 1 MiB per split tile at Hkv = 8, plus the dQ key-split
 * partials of small bf16 problems: with split_tiles from tt_attn_split_tiles,
 * 16 MiB on the 16K agent tree and 70 MiB on the 48K rollout tree). The call
 * allocates and frees nothing (no hipMalloc, no hipMemsetAsync: what must start at zero is
 * cleared by a kernel). Every call on one GPU uses that GPU's one scratch
 * array, which keeps the last call's contents: calls that overlap on one GPU
 * (other streams, other threads) race and must not be issued; a TT_BWD_*
 * sequence split over several calls must not be interleaved with another
 * call on the same GPU. The first call on each GPU resolves the array's
 * device address (hipGetSymbolAddress, once per device, cached): make that
 * first call outside stream capture, e.g. an ordinary warm-up call before a
 * graph is captured; later calls make no such lookup. */
#define TT_NOALLOC_SCRATCH_MB 96
size_t tt_noalloc_scratch_bytes(void);
int tt_attn_bwd_noalloc(const tt_attn_problem* p, const void* o, const float* lse, tt_tensor d_o,
                        void* dq, void* dk, void* dv, float* dk_past_acc, float* dv_past_acc, void* stream);

/* ---- attention prologue: q/k RMSNorm + rotary embedding -------------------
 * Replaces the per-head q_norm / k_norm and apply_rotary_pos_emb that
 * Qwen3Attention runs between the projections and the attention call
 * (HF/models/qwen3/modeling_qwen3.py:252-257; RMSNorm :59-64, rotate_half and
 * apply_rotary_pos_emb :140-170), at the depth positions the reference passes
 * as position_ids (dfs_tree_forward.py:543-560):
 *   y = w * x / sqrt(mean(x^2) + eps),  out = y * cos + [-y[64:], y[:64]] * sin,
 * fused into one pass that writes q and k in the [T, H, 128] layout of
 * tt_attn_problem. cos/sin are the model's rotary table at each token's
 * position (any rotary scaling variant). */
typedef struct tt_prologue_problem {
    int32_t dtype;          /* TT_DTYPE_BF16 or TT_DTYPE_F32 for every tensor here */
    int32_t n_tokens;
    int32_t n_heads_q;
    int32_t n_heads_kv;
    int32_t head_dim;       /* 128 */
    float eps_q, eps_k;     /* the two norms' epsilons */
    tt_tensor q, k;         /* projected q [T, Hq, 128], k [T, Hkv, 128]; 16-byte aligned rows */
    const void* q_weight;   /* [128] */
    const void* k_weight;   /* [128] */
    const void* cos;        /* [T, 128], element [t][d] at cos + t*cs_stride_tok + d */
    const void* sin;
    int64_t cs_stride_tok;
} tt_prologue_problem;

/* q_out [T, Hq, 128] and k_out [T, Hkv, 128], contiguous. */
int tt_qk_prologue_fwd(const tt_prologue_problem* p, void* q_out, void* k_out, void* stream);
/* Gradients for dq_out / dk_out (strided like q / k): dq_raw, dk_raw
 * contiguous [T, H, 128] in the problem dtype, dq_weight / dk_weight [128]
 * float32 (summed in a fixed order: deterministic). Workspace:
 * tt_qk_prologue_bwd_workspace_bytes (fixed, 1 MiB). */
size_t tt_qk_prologue_bwd_workspace_bytes(const tt_prologue_problem* p);
int tt_qk_prologue_bwd(const tt_prologue_problem* p, tt_tensor dq_out, tt_tensor dk_out, void* dq_raw, void* dk_raw,
                       float* dq_weight, float* dk_weight, void* ws, size_t ws_bytes, void* stream);

/* ---- tree gated delta rule (linear-attention layers) ----------------------
 * Replaces torch_chunk_gated_delta_rule_tree_varlen (tree_dfs_ssm.py:38-156;
 * twin dfs_tree_forward.py:253-353) as called from the patched GDN layer
 * (tree_dfs_ssm.py:399-414): q/k/v of the packed tree, per-node parent-state
 * routing (chunk_parent_map, :131-132). Two semantics:
 *  - reference_truncated = 0: the exact gated delta rule along every
 *    root-to-leaf path (the function's stated contract, :49-52), evaluated in
 *    32-token chunks;
 *  - reference_truncated = 1: what the reference function itself returns. It
 *    treats each whole node as one chunk and builds the within-node
 *    correction from the uncorrected rows (:120-126), A = I + R + R^2 with
 *    R = -strictly_lower(beta k k^T * exp(G_i - G_j)) over the node, G the
 *    node's cumulative log decay: U = A (beta v), W = A (beta e^G k),
 *    V' = U - W S_parent, O = e^G q S_parent + lower(q k^T * D) V'. It equals
 *    the exact rule for nodes of at most 3 tokens (R^3 = 0) and differs for
 *    longer ones.
 *
 * Nodes are in DFS pre-order (parent[i] < i, -1 for a root); node i owns
 * tokens [node_start[i], node_start[i] + node_len[i]) and is cut into
 * ceil(node_len[i] / TT_GDN_CHUNK) consecutive chunks, numbered globally in
 * node order: node_chunk0[i] is node i's first chunk and chunk_node[c] the
 * node of chunk c (n_chunks in all). level_nodes lists every node once,
 * grouped by depth (roots first); level_offsets (HOST memory, n_levels + 1
 * entries, level_offsets[n_levels] = n_nodes) delimits the groups. A node
 * whose parent is not in an earlier group reads an undefined state. Within a
 * group the scans start nodes in the order given: longest first finishes a
 * level soonest. */
#define TT_GDN_CHUNK 32
typedef struct tt_gdn_problem {
    int32_t dtype;          /* TT_DTYPE_BF16 or TT_DTYPE_F32 for q, k, v and o */
    int32_t n_tokens;
    int32_t n_nodes;
    int32_t n_heads_k;      /* q/k heads */
    int32_t n_heads_v;      /* v heads, a multiple of n_heads_k; v head h reads q/k head h / (Hv/Hk) */
    int32_t head_dim;       /* 128 (key and value) */
    int32_t l2norm;         /* 1: q and k are l2-normalised (eps 1e-6) before use */
    float scale;            /* q multiplier after normalisation, usually head_dim^-1/2 */
    tt_tensor q, k, v;      /* [T, H, 128], 16-byte aligned rows */
    const float* g;         /* [T, Hv] log decay (<= 0), element [t][h] at g + t*g_stride_tok + h */
    int64_t g_stride_tok;
    const float* beta;      /* [T, Hv] write strength */
    int64_t beta_stride_tok;
    const int32_t* node_start;   /* device, [n_nodes] */
    const int32_t* node_len;     /* device, [n_nodes] */
    const int32_t* node_parent;  /* device, [n_nodes] */
    const int32_t* level_nodes;  /* device, [n_nodes] */
    const int32_t* level_offsets;/* HOST, [n_levels + 1] */
    int32_t n_levels;
    int32_t n_chunks;
    const int32_t* node_chunk0;  /* device, [n_nodes] */
    const int32_t* chunk_node;   /* device, [n_chunks] */
    /* Children of node i (any order): node_child[node_child_off[i] ..
     * node_child_off[i + 1]). Device, [n_nodes + 1] and [n_nodes]; read by
     * tt_gdn_tree_bwd only (may be NULL for the forward). */
    const int32_t* node_child_off;
    const int32_t* node_child;
    int32_t reference_truncated;  /* 0: exact delta rule; 1: the reference's I + R + R^2 per node */
    /* The state every root starts from (the reference's initial_state,
     * tree_dfs_ssm.py:84-90: all_states[0], read by every node whose parent
     * is -1): device, [Hv, 128, 128] float32 contiguous, 16-byte aligned;
     * NULL: zero. */
    const float* initial_state;
    /* tt_gdn_tree_bwd*: 1 when d_node_states holds the gradient of the last
     * node's state alone ([Hv, 128, 128]: the reference's differentiable
     * last_state, tree_dfs_ssm.py:155), 0 when it holds all [n_nodes, ...]. */
    int32_t d_states_last_only;
} tt_gdn_problem;

/* Workspace of tt_gdn_tree_fwd: per (chunk, v head) the state-independent
 * chunk terms (U, W, A, G) in float32; with reference_truncated also the
 * node-level decay and R (beta [v | e^G k]) rows (about 33 KiB more). */
size_t tt_gdn_workspace_bytes(const tt_gdn_problem* p);
/* o: [T, Hv, 128] contiguous, problem dtype. node_states: [n_nodes, Hv, 128,
 * 128] float32, the state after each node (its children's initial state;
 * kept for the backward). One parallel launch over all chunks, then one
 * launch per tree level. */
int tt_gdn_tree_fwd(const tt_gdn_problem* p, void* o, float* node_states, void* ws, size_t ws_bytes,
                    void* stream);

/* Backward of tt_gdn_tree_fwd's o (what autograd computes through the
 * reference's torch function, tree_dfs_ssm.py:38-156, for the exact rule):
 * given d_o [T, Hv, 128] (problem dtype, strided like q), writes dq, dk [T, Hk,
 * 128] and dv [T, Hv, 128] in the problem dtype, each at its own token
 * stride with contiguous heads (tt_tensor descriptors whose memory is
 * written: stride_head 128, else TT_E_UNSUPPORTED; stride_tok by the rules
 * of q and at most 2^30; e.g. the column blocks of one [T, 2 Hk 128 + Hv 128]
 * row buffer, the gradient of a conv output that a q/k/v split reads, so that
 * no concatenation follows), and dg, dbeta [T, Hv] contiguous float32.
 * d_node_states (NULL: none) is the incoming gradient of node_states ([n_nodes,
 * Hv, 128, 128] float32; the reference's differentiable last_state,
 * tree_dfs_ssm.py:155, is node n_nodes - 1), or with p->d_states_last_only
 * that of the last node's state alone ([Hv, 128, 128]); d_initial_state (NULL: not
 * wanted) receives the gradient of p->initial_state ([Hv, 128, 128] float32,
 * written whole; with a NULL initial_state, the gradient at the zero state).
 * Both 16-byte aligned. It
 * recomputes the forward (keeping every chunk's initial state), runs one
 * reverse launch per tree level (deepest first) for the state gradient, then
 * two launches over all chunks. Workspace: tt_gdn_bwd_workspace_bytes (per
 * (chunk, v head) about 240 KiB; per (node, v head) 128 KiB). */
size_t tt_gdn_bwd_workspace_bytes(const tt_gdn_problem* p);
int tt_gdn_tree_bwd(const tt_gdn_problem* p, tt_tensor d_o, tt_tensor dq, tt_tensor dk, tt_tensor dv, float* dg,
                    float* dbeta, const float* d_node_states, float* d_initial_state, void* ws, size_t ws_bytes,
                    void* stream);

/* The same forward and backward without the backward's recompute of the
 * forward (what autograd keeps through the reference's torch function,
 * tree_dfs_ssm.py:38-156, between its forward and backward):
 * tt_gdn_tree_fwd_save computes o and node_states as tt_gdn_tree_fwd and also
 * keeps, in `saved` (tt_gdn_saved_bytes: per (chunk, v head) the prep terms,
 * the chunk's initial state and V', about 123 KiB), what the backward needs.
 * tt_gdn_tree_bwd_saved then gives the gradients tt_gdn_tree_bwd gives, from
 * `saved` (unchanged since, same problem and inputs) and a scratch workspace of
 * tt_gdn_bwd_saved_workspace_bytes. */
size_t tt_gdn_saved_bytes(const tt_gdn_problem* p);
int tt_gdn_tree_fwd_save(const tt_gdn_problem* p, void* o, float* node_states, void* saved, size_t saved_bytes,
                         void* stream);
size_t tt_gdn_bwd_saved_workspace_bytes(const tt_gdn_problem* p);
int tt_gdn_tree_bwd_saved(const tt_gdn_problem* p, tt_tensor d_o, tt_tensor dq, tt_tensor dk, tt_tensor dv,
                          float* dg, float* dbeta, const float* d_node_states, float* d_initial_state,
                          const void* saved, size_t saved_bytes, void* ws, size_t ws_bytes, void* stream);

/* ---- tree-correct short convolution --------------------------------------
 * Replaces _tree_correct_conv_varlen (tree_dfs_ssm.py:284-346; twin
 * dfs_tree_forward.py:191-246): depthwise causal conv of kernel size K + SiLU
 * over the packed tree, where each node's window reaches into its ancestors'
 * last K-1 inputs (zeros before a root) instead of the DFS neighbours:
 *   y[t][c] = silu(bias[c] + sum_i weight[c][i] * x[prev^(K-1-i)(t)][c]),
 * with tok_prev[t] = t - 1 inside a node, the parent's last token for a node's
 * first token, -1 for a root's first token. The reference's conv reads the
 * channel-major [B, C, T] layout; here rows are tokens (channels contiguous),
 * the layout the q/k/v split after it reads. */
typedef struct tt_conv_problem {
    int32_t dtype;          /* TT_DTYPE_BF16 or TT_DTYPE_F32: x, weight, bias, y, dy, dx */
    int32_t n_tokens;
    int32_t n_channels;     /* multiple of 4 */
    int32_t kernel_size;    /* 1..4 */
    const void* x;          /* [T, C], element [t][c] at x + t*x_stride_tok + c */
    int64_t x_stride_tok;   /* multiple of 4, >= n_channels */
    const void* weight;     /* [C, K] contiguous (conv1d.weight [C, 1, K]) */
    const void* bias;       /* [C] or NULL */
    const int32_t* tok_prev;      /* device, [T] */
    const int32_t* tok_next_off;  /* device, [T + 1]: successors of t (tokens u with tok_prev[u] = t) are */
    const int32_t* tok_next;      /* tok_next[tok_next_off[t] .. tok_next_off[t+1]); backward only */
} tt_conv_problem;

/* y: [T, C] rows y + t*y_stride_tok (multiple of 4, >= n_channels). */
int tt_tree_conv_fwd(const tt_conv_problem* p, void* y, int64_t y_stride_tok, void* stream);
/* Gradients for dy [T, C] (rows dy + t*dy_stride_tok): dx [T, C] contiguous
 * (problem dtype), dweight [C, K] and dbias [C] float32 (dbias may be NULL).
 * Deterministic: the weight gradient is summed in a fixed order, dx gathers
 * over the successor lists. Workspace: tt_tree_conv_bwd_workspace_bytes. */
size_t tt_tree_conv_bwd_workspace_bytes(const tt_conv_problem* p);
int tt_tree_conv_bwd(const tt_conv_problem* p, const void* dy, int64_t dy_stride_tok, void* dx, float* dweight,
                     float* dbias, void* ws, size_t ws_bytes, void* stream);

/* ---- leaf loss: row-wise cross-entropy ------------------------------------
 * The step after the tree forward: the reference scores each leaf with
 * F.cross_entropy(logits, labels, ignore_index) / n_leaves
 * (tree_grad_hybrid.py:546-558, tree_grad_ckpt.py:280-297) on logits of every
 * token. Applied to one chunk of lm_head logits at a time (the caller's
 * GEMMs), this gives each row's weighted loss and its logit gradient in one
 * kernel, so the [T, V] logits never exist at once:
 *   loss[r] = c_r (lse_r - x[r][y_r]),  grad[r][j] = c_r (softmax_r[j] - [j == y_r]);
 * rows labelled ignore_index get loss 0 and a zero gradient; a label outside
 * [0, vocab) gives a NaN loss. grad may be the logits buffer itself (ldg ==
 * ld). Rows ld / ldg apart, 16-byte aligned. */
int tt_ce_rows(int32_t dtype, const void* logits, int64_t ld, int32_t n_rows, int32_t vocab, const int32_t* labels,
               const float* row_scale, int32_t ignore_index, float* loss, void* grad, int64_t ldg, void* stream);

/* ---- device self-test ----------------------------------------------------
 * No counterpart in the reference. Runs one v_mfma_f32_32x32x16_bf16 with the
 * operand and accumulator lane layout the bf16 kernels assume:
 * d[32x32] = a[32x16] @ b[16x32], all row-major (a, b bf16; d float32). */
int tt_selftest_mfma32(const void* a, const void* b, float* d, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TREE_ATTN_H */
