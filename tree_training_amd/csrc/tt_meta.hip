// DFS tree metadata, per-key visibility intervals and the block-sparsity plan.
//
// Replaces build_dfs_tree_info (dfs_tree_forward.py:91-184) and the dense
// additive-mask assembly (dfs_tree_forward.py:548-550, tree_grad_hybrid.py:312-317).
// Node-level work (prefix sums over node lengths, ancestor offsets by pointer
// jumping, subtree ends by a sparse-table next-smaller-or-equal-depth search)
// runs in one workgroup; token-level work (positions, node ids, horizons) runs
// one thread per token. All of it is integer work bound by launch latency and
// HBM, never by arithmetic.
#include "tt_common.h"
#include "tt_internal.h"

namespace {

constexpr int kNodeThreads = 1024;
constexpr int kLdsNodes = 512;    // node arrays in LDS up to this many nodes

__host__ __device__ constexpr int sparse_levels(int n) {
    int L = 1;
    while ((1 << L) <= n) ++L;   // levels r = 0..L-1 with 2^r <= n
    return L;
}

constexpr int kLdsLevels = sparse_levels(kLdsNodes) - 1;   // sparse-table levels 1..L-1 of the largest such tree

// Where a workgroup's node arrays can be read after meta_nodes_body: LDS
// copies for trees of at most kLdsNodes nodes, else the global outputs.
struct NodeView {
    const int32_t* len;
    const int32_t* start;
    const int32_t* off;
    const int32_t* hend;
};

// Node-level metadata in one workgroup of kNodeThreads threads. TT_STATUS_*
// bits are OR-ed into s_err (an LDS word the caller zeroes before the call);
// ends with a barrier after which start, off, hend (and the arrays of the
// returned view) and s_err are visible to the whole workgroup.
__device__ __forceinline__ NodeView meta_nodes_body(
    const int32_t* __restrict__ len, const int32_t* __restrict__ par, int n, int T,
    int32_t* __restrict__ start, int32_t* __restrict__ off, int32_t* __restrict__ hend,
    int& s_err, int32_t* __restrict__ ws) {
    __shared__ int s_scan[kNodeThreads];
    __shared__ int s_carry;
    // Trees of at most kLdsNodes nodes keep the node arrays in LDS (every
    // pointer-jumping round, sparse-table level and read-back is then an LDS
    // round trip, not a global one); larger ones use the workspace and the
    // global outputs.
    __shared__ int32_t s_nodes[(9 + kLdsLevels) * kLdsNodes];
    const int tid = threadIdx.x;
    const bool in_lds = n <= kLdsNodes;
    int32_t* const b = in_lds ? s_nodes : ws;
    int32_t* anc0 = b;
    int32_t* anc1 = b + n;
    int32_t* offb1 = b + 2 * n;
    int32_t* dep0 = b + 3 * n;
    int32_t* dep1 = b + 4 * n;
    int32_t* offb0 = in_lds ? b + 5 * n : off;     // first pointer-jumping buffer of off
    int32_t* w_len = in_lds ? b + 6 * n : nullptr;
    int32_t* w_start = in_lds ? b + 7 * n : start;
    int32_t* w_hend = in_lds ? b + 8 * n : hend;
    int32_t* st = b + (in_lds ? 9 : 5) * n;        // sparse-table levels 1..L-1, n ints each
    if (tid == 0) s_carry = 0;
    __syncthreads();

    // 1. exclusive prefix sum of node lengths -> node_start; validate input.
    for (int base = 0; base < n; base += kNodeThreads) {
        const int i = base + tid;
        int v = 0;
        if (i < n) {
            v = len[i];
            if (in_lds) w_len[i] = v;
            int p = par[i];
            if (v < 1) atomicOr(&s_err, TT_STATUS_BAD_LEN);
            if (p < -1 || p >= i) atomicOr(&s_err, TT_STATUS_BAD_PARENT);
        }
        // a scan within each wave (shuffles), then over the waves' totals
        const int lane = tid & 63, wave = tid >> 6;
        int incl = v;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int up = __shfl_up(incl, o, 64);
            if (lane >= o) incl += up;
        }
        if (lane == 63) s_scan[wave] = incl;
        __syncthreads();
        int before = s_carry;
        for (int w = 0; w < wave; ++w) before += s_scan[w];
        if (i < n) {
            start[i] = before + incl - v;
            if (in_lds) w_start[i] = before + incl - v;
        }
        __syncthreads();
        if (tid == kNodeThreads - 1) s_carry = before + incl;
        __syncthreads();
    }
    if (tid == 0 && s_carry != T) atomicOr(&s_err, TT_STATUS_BAD_TOTAL);
    const int32_t* lenv = in_lds ? w_len : len;

    // 2. pointer jumping: off = sum of ancestor lengths, dep = ancestor count.
    for (int i = tid; i < n; i += kNodeThreads) {
        int p = par[i];
        if (p < -1 || p >= i) p = -1;   // flagged above; keep the walk in bounds
        anc0[i] = p;
        offb0[i] = p >= 0 ? lenv[p] : 0;
        dep0[i] = p >= 0 ? 1 : 0;
    }
    __syncthreads();
    int32_t* a_cur = anc0; int32_t* a_nxt = anc1;
    int32_t* o_cur = offb0; int32_t* o_nxt = offb1;
    int32_t* d_cur = dep0; int32_t* d_nxt = dep1;
    for (;;) {
        int any = 0;
        for (int i = tid; i < n; i += kNodeThreads) {
            int a = a_cur[i];
            if (a >= 0) {
                o_nxt[i] = o_cur[i] + o_cur[a];
                d_nxt[i] = d_cur[i] + d_cur[a];
                int aa = a_cur[a];
                a_nxt[i] = aa;
                any |= (aa >= 0);
            } else {
                o_nxt[i] = o_cur[i];
                d_nxt[i] = d_cur[i];
                a_nxt[i] = -1;
            }
        }
        __syncthreads();                // writes of this round visible
        any = __syncthreads_or(any);
        int32_t* t;
        t = a_cur; a_cur = a_nxt; a_nxt = t;
        t = o_cur; o_cur = o_nxt; o_nxt = t;
        t = d_cur; d_cur = d_nxt; d_nxt = t;
        if (!any) break;
    }
    if (o_cur != off) {
        for (int i = tid; i < n; i += kNodeThreads) off[i] = o_cur[i];
    }
    __syncthreads();

    // 3. subtree end = first later node whose depth <= own depth (pre-order).
    const int L = sparse_levels(n);
    for (int r = 1; r < L; ++r) {
        const int32_t* prev = (r == 1) ? d_cur : st + (size_t)(r - 2) * n;
        int32_t* cur = st + (size_t)(r - 1) * n;
        const int w = 1 << r, hw = w >> 1;
        for (int i = tid; i + w <= n; i += kNodeThreads) cur[i] = min(prev[i], prev[i + hw]);
        __syncthreads();
    }
    for (int c = tid; c < n; c += kNodeThreads) {
        const int thr = d_cur[c];
        int i = c + 1;
        for (int r = L - 1; r >= 0; --r) {
            const int w = 1 << r;
            if (i + w <= n) {
                const int32_t* lev = (r == 0) ? d_cur : st + (size_t)(r - 1) * n;
                if (lev[i] > thr) i += w;
            }
        }
        const int he = (i < n) ? w_start[i] : T;
        hend[c] = he;
        if (in_lds) w_hend[c] = he;
    }
    __syncthreads();   // hend of every node visible

    // 4. pre-order: parent < i alone admits orders such as parents [-1, 0, 0, 1],
    // where node 3's parent subtree has closed (node 2, depth 1, comes first).
    // Given parent < i, a node that starts inside its parent's subtree range
    // for every node is exactly DFS pre-order (every node between a parent and
    // its child is then a descendant of that parent).
    for (int i = tid; i < n; i += kNodeThreads) {
        const int p = par[i];
        if (p >= 0 && p < i && w_start[i] >= w_hend[p]) atomicOr(&s_err, TT_STATUS_BAD_PARENT);
    }
    __syncthreads();
    return NodeView{lenv, w_start, o_cur, w_hend};
}

// Tokens of every node: wave w writes the tokens of nodes w, w + 16, ..., its
// lanes 64 consecutive tokens at a time (no per-token search); with
// key_lo/key_hi, also the own keys' visibility intervals after n_past gateway
// keys. A node outside [0, T) (bad lengths, flagged in the status) writes
// nothing.
__device__ __forceinline__ void meta_tokens_body(const int32_t* __restrict__ len, int n, int T, int pos_offset,
                                                 const int32_t* __restrict__ start, const int32_t* __restrict__ off,
                                                 const int32_t* __restrict__ hend, int32_t* __restrict__ pos,
                                                 int32_t* __restrict__ node_of, int32_t* __restrict__ horizon,
                                                 int n_past, int32_t* __restrict__ key_lo,
                                                 int32_t* __restrict__ key_hi) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int c = wave; c < n; c += kNodeThreads / 64) {
        const int s0 = start[c], e0 = min(s0 + max(len[c], 0), T), o = pos_offset + off[c], h = hend[c];
        for (int i = max(s0, 0) + lane; i < e0; i += 64) {
            pos[i] = o + (i - s0);
            if (node_of) node_of[i] = c;
            horizon[i] = h;
            if (key_lo) {
                key_lo[n_past + i] = i;
                key_hi[n_past + i] = h;
            }
        }
    }
}

__global__ __launch_bounds__(kNodeThreads) void meta_nodes_kernel(
    const int32_t* __restrict__ len, const int32_t* __restrict__ par, int n, int T,
    int32_t* __restrict__ start, int32_t* __restrict__ off, int32_t* __restrict__ hend,
    int32_t* __restrict__ status, int32_t* __restrict__ ws) {
    __shared__ int s_err;
    if (threadIdx.x == 0) s_err = 0;
    meta_nodes_body(len, par, n, T, start, off, hend, s_err, ws);
    if (threadIdx.x == 0 && s_err) atomicOr(status, s_err);
}

// Nodes and tokens in one launch (trees of up to kFusedTokens tokens): after
// the node work, each wave writes the tokens of every 16th node, its lanes
// 64 consecutive tokens at a time (no per-token search).
constexpr int kFusedTokens = 1 << 16;
__global__ __launch_bounds__(kNodeThreads) void meta_tree_kernel(
    const int32_t* __restrict__ len, const int32_t* __restrict__ par, int n, int T, int pos_offset,
    int32_t* __restrict__ start, int32_t* __restrict__ off, int32_t* __restrict__ hend,
    int32_t* __restrict__ pos, int32_t* __restrict__ node_of, int32_t* __restrict__ horizon,
    int32_t* __restrict__ status, int32_t* __restrict__ ws) {
    __shared__ int s_err;
    if (threadIdx.x == 0) s_err = 0;
    const NodeView v = meta_nodes_body(len, par, n, T, start, off, hend, s_err, ws);
    if (threadIdx.x == 0 && s_err) atomicOr(status, s_err);
    meta_tokens_body(v.len, n, T, pos_offset, v.start, v.off, v.hend, pos, node_of, horizon, 0, nullptr, nullptr);
}

__global__ void meta_tokens_kernel(const int32_t* __restrict__ start, const int32_t* __restrict__ off,
                                   const int32_t* __restrict__ hend, int n, int T, int pos_offset,
                                   int32_t* __restrict__ pos, int32_t* __restrict__ node_of,
                                   int32_t* __restrict__ horizon) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= T) return;
    int lo = 0, hi = n - 1;          // largest c with start[c] <= i
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (start[mid] <= i) lo = mid; else hi = mid - 1;
    }
    pos[i] = pos_offset + off[lo] + (i - start[lo]);
    if (node_of) node_of[i] = lo;
    horizon[i] = hend[lo];
}

__global__ void keys_kernel(const float* __restrict__ bias, int n_past, const int32_t* __restrict__ horizon,
                            int n_q, int32_t* __restrict__ key_lo, int32_t* __restrict__ key_hi,
                            int32_t* __restrict__ status) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n_past + n_q) return;
    if (j < n_past) {
        const float b = bias[j];
        int vis = 0;
        if (b == 0.0f) vis = 1;
        else if (!(__builtin_isinf(b) && b < 0.0f)) atomicOr(status, TT_STATUS_BAD_BIAS);
        key_lo[j] = 0;
        key_hi[j] = vis ? n_q : 0;
    } else {
        const int jj = j - n_past;
        key_lo[j] = jj;
        key_hi[j] = horizon[jj];
    }
}

__global__ void dense_mask_kernel(const int32_t* __restrict__ key_lo, const int32_t* __restrict__ key_hi,
                                  int n_keys, int n_q, uint8_t* __restrict__ mask) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    const int i = blockIdx.y;
    if (j >= n_keys || i >= n_q) return;
    mask[(size_t)i * n_keys + j] = (key_lo[j] <= i && i < key_hi[j]) ? 1 : 0;
}

// Visible (query, key) pairs of 256 keys per workgroup, one partial per workgroup.
__device__ __forceinline__ void plan_pairs_part(const int32_t* __restrict__ key_lo, const int32_t* __restrict__ key_hi,
                                                int n_keys, int n_q, int blk, unsigned long long* __restrict__ part) {
    __shared__ unsigned long long s_sum;
    if (threadIdx.x == 0) s_sum = 0;
    __syncthreads();
    const int j = blk * 256 + threadIdx.x;
    long long c = 0;
    if (j < n_keys) {
        const int a = max(key_lo[j], 0), b = min(key_hi[j], n_q);
        c = b > a ? (long long)(b - a) : 0;
    }
    atomicAdd(&s_sum, (unsigned long long)c);
    __syncthreads();
    if (threadIdx.x == 0) part[blk] = s_sum;
}

// One wave per (query block, key tile) pair, one lane per key of the tile.
static_assert(TT_BK == 64, "plan_classify maps the keys of a tile to the lanes of a wave");
__device__ __forceinline__ void plan_classify(const int32_t* __restrict__ key_lo, const int32_t* __restrict__ key_hi,
                                              int n_keys, int n_q, int n_qb, int n_kt, int blk,
                                              uint8_t* __restrict__ cls) {
    const int pair = blk * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (pair >= n_qb * n_kt) return;   // wave-uniform
    const int qb = pair / n_kt, kt = pair - qb * n_kt;
    const int i0 = qb * TT_BQ, i1 = min(i0 + TT_BQ, n_q);
    const int j = kt * TT_BK + lane;
    bool some = false, every = false;
    if (j < n_keys) {
        const int lo = key_lo[j], hi = key_hi[j];
        some = max(lo, i0) < min(hi, i1);
        every = lo <= i0 && hi >= i1;
    }
    const bool any = __ballot(some) != 0, all = __ballot(every) == ~0ull;
    if (lane == 0) cls[pair] = any ? (all ? 2 : 1) : 0;
}

// One wave per query block: compacts the non-empty key tiles, ascending.
__global__ void plan_compact_kernel(const uint8_t* __restrict__ cls, int n_qb, int n_kt,
                                    int32_t* __restrict__ row_cnt, int32_t* __restrict__ row_list) {
    const int row = blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    const int lane = threadIdx.x & 63;
    if (row >= n_qb) return;
    int cnt = 0;
    const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int base = 0; base < n_kt; base += 64) {
        const int kt = base + lane;
        const int c = kt < n_kt ? cls[(size_t)row * n_kt + kt] : 0;
        const unsigned long long m = __ballot(c != 0);
        if (c) row_list[(size_t)row * n_kt + cnt + __popcll(m & below)] = (kt << 1) | (c == 2 ? 1 : 0);
        cnt += __popcll(m);
    }
    if (lane == 0) row_cnt[row] = cnt;
}

// Query blocks ranked by decreasing tile count (ties by index): heavy blocks
// are dispatched first.
__device__ __forceinline__ void plan_row_order(const int32_t* __restrict__ row_cnt, int n_qb, int blk,
                                               int32_t* __restrict__ row_order) {
    const int i = blk * 256 + threadIdx.x;
    if (i >= n_qb) return;
    const int c = row_cnt[i];
    int rank = 0;
    for (int j = 0; j < n_qb; ++j) {
        const int cj = row_cnt[j];
        rank += (cj > c) || (cj == c && j < i);
    }
    row_order[rank] = i;
}

// One wave per 128-key tile: the union of its keys' visible query intervals,
// which is a single range (consecutive lower bounds, non-empty intervals).
__device__ __forceinline__ void plan_kv_range(const int32_t* __restrict__ key_lo, const int32_t* __restrict__ key_hi,
                                              int n_keys, int n_q, int n_kb, int blk, int32_t* __restrict__ kb_qlo,
                                              int32_t* __restrict__ kb_qhi) {
    const int kb = blk * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x & 63;
    if (kb >= n_kb) return;
    int lo = n_q, hi = 0;
    for (int t = lane; t < TT_BKB; t += 64) {
        const int j = kb * TT_BKB + t;
        if (j < n_keys) {
            const int a = max(key_lo[j], 0), b = min(key_hi[j], n_q);
            if (a < b) { lo = min(lo, a); hi = max(hi, b); }
        }
    }
    lo = wave_min_i(lo);
    hi = wave_max_i(hi);
    if (lane == 0) {
        kb_qlo[kb] = lo < hi ? lo : 0;
        kb_qhi[kb] = lo < hi ? hi : 0;
    }
}

__device__ __forceinline__ void plan_kb_order(const int32_t* __restrict__ kb_qlo, const int32_t* __restrict__ kb_qhi,
                                              int n_kb, int blk, int32_t* __restrict__ kb_order) {
    const int i = blk * 256 + threadIdx.x;
    if (i >= n_kb) return;
    const int c = kb_qhi[i] - kb_qlo[i];
    int rank = 0;
    for (int j = 0; j < n_kb; ++j) {
        const int cj = kb_qhi[j] - kb_qlo[j];
        rank += (cj > c) || (cj == c && j < i);
    }
    kb_order[rank] = i;
}

// Exclusive prefix sum of work items per key tile, in kb_order order (one workgroup).
// Plan pass 1: tile classes, per-128-key-tile query ranges and partial pair
// counts, three independent reads of the key intervals in one launch
// (workgroup ranges [0, nb_cls), [nb_cls, nb_cls + nb_kv), then the pairs).
__global__ __launch_bounds__(256) void plan_keys_pass_kernel(const int32_t* __restrict__ key_lo,
                                                             const int32_t* __restrict__ key_hi, int n_keys, int n_q,
                                                             int n_qb, int n_kt, int n_kb, int nb_cls, int nb_kv,
                                                             uint8_t* __restrict__ cls, int32_t* __restrict__ kb_qlo,
                                                             int32_t* __restrict__ kb_qhi,
                                                             unsigned long long* __restrict__ pair_part) {
    const int b = blockIdx.x;
    if (b < nb_cls)
        plan_classify(key_lo, key_hi, n_keys, n_q, n_qb, n_kt, b, cls);
    else if (b < nb_cls + nb_kv)
        plan_kv_range(key_lo, key_hi, n_keys, n_q, n_kb, b - nb_cls, kb_qlo, kb_qhi);
    else
        plan_pairs_part(key_lo, key_hi, n_keys, n_q, b - nb_cls - nb_kv, pair_part);
}

// Plan pass 3: the query-block order and the key-tile order (heaviest first).
__global__ __launch_bounds__(256) void plan_orders_kernel(const int32_t* __restrict__ row_cnt, int n_qb, int nb_ro,
                                                          const int32_t* __restrict__ kb_qlo,
                                                          const int32_t* __restrict__ kb_qhi, int n_kb,
                                                          int32_t* __restrict__ row_order,
                                                          int32_t* __restrict__ kb_order) {
    if ((int)blockIdx.x < nb_ro)
        plan_row_order(row_cnt, n_qb, blockIdx.x, row_order);
    else
        plan_kb_order(kb_qlo, kb_qhi, n_kb, blockIdx.x - nb_ro, kb_order);
}

// Rank of every key tile among the split ones (more than one dK/dV work
// item), in key order, -1 for the others, and their count in the plan header;
// run by a whole workgroup of 1024 threads.
__device__ __forceinline__ void plan_split_ranks(const int32_t* __restrict__ kb_qlo,
                                                 const int32_t* __restrict__ kb_qhi, int n_kb, int qch,
                                                 int32_t* __restrict__ kb_srank, uint8_t* __restrict__ plan) {
    __shared__ int s_w[16];
    __shared__ int s_c;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    if (tid == 0) s_c = 0;
    __syncthreads();
    for (int base = 0; base < n_kb; base += 1024) {
        const int kb = base + tid;
        const int f = (kb < n_kb && tt_kb_items(kb_qlo[kb], kb_qhi[kb], qch) > 1) ? 1 : 0;
        const unsigned long long m = __ballot(f);
        if (lane == 0) s_w[wave] = __popcll(m);
        __syncthreads();
        int before = s_c;
        for (int w = 0; w < wave; ++w) before += s_w[w];
        if (kb < n_kb) kb_srank[kb] = f ? before + __popcll(m & ((1ull << lane) - 1)) : -1;
        __syncthreads();
        if (tid == 0) {
            int tot = 0;
            for (int w = 0; w < 16; ++w) tot += s_w[w];
            s_c += tot;
        }
        __syncthreads();
    }
    if (tid == 0) reinterpret_cast<int32_t*>(plan)[6] = s_c;
}

// The dK/dV work items in the order the persistent grid takes them, as (tile
// rank, chunk) pairs. Up to kSortItems items: longest item first (its query
// range), ties by query window from the top, then by tile rank: the longest
// items start first (a longest-processing-time schedule over the resident
// workgroups), and the workgroups of an XCD (one kv head's items) that start
// together walk the same query window and share its Q / dO in L2. Sorted as
// packed 64-bit keys, a bitonic sort in LDS. Above kSortItems (trees of
// hundreds of thousands of tokens) the list is window-major: every key tile's
// item of the top window, then the next window down, each window's items in
// tile order. Run by a whole workgroup of 1024 threads once kb_base is final;
// n_items = kb_base[n_kb]. Header int32 7: 1 sorted by length, 2 window-major.
constexpr int kSortItems = 4096;
__device__ __forceinline__ void plan_item_list(const int32_t* __restrict__ kb_qlo,
                                               const int32_t* __restrict__ kb_qhi,
                                               const int32_t* __restrict__ kb_order,
                                               const int32_t* __restrict__ kb_base, int n_kb, int n_q, int qch,
                                               int2* __restrict__ kb_item, uint8_t* __restrict__ plan) {
    __shared__ unsigned long long s_key[kSortItems];
    __shared__ int s_w[16];
    __shared__ int s_c;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n_items = kb_base[n_kb];
    if (n_items <= kSortItems) {
        // key: (4096 - length) | (4095 - window) | rank | chunk, 13 + 12 + 12 + 12 bits
        // (n_kb <= n_items, and the windows number at most n_q / 256 + 1 <= n_items / 2 + 1)
        int n = 1;
        while (n < n_items) n <<= 1;
        for (int i = tid; i < n; i += 1024) s_key[i] = ~0ull;
        __syncthreads();
        for (int r = tid; r < n_kb; r += 1024) {
            const int kb = kb_order[r], lo = kb_qlo[kb], hi = kb_qhi[kb], b = kb_base[r];
            const int m = tt_kb_items(lo, hi, qch);
            for (int c = 0; c < m; ++c) {
                int q0, q1;
                tt_kb_item_range(lo, hi, qch, c, q0, q1);
                const int len = min(max(q1 - q0, 0), 4096);
                const int w = min(m > 1 ? lo / qch + c : (hi > lo ? (hi - 1) / qch : 0), 4095);
                s_key[b + c] = ((unsigned long long)(4096 - len) << 36) | ((unsigned long long)(4095 - w) << 24) |
                               ((unsigned long long)r << 12) | (unsigned long long)c;
            }
        }
        __syncthreads();
        for (int k = 2; k <= n; k <<= 1)
            for (int j = k >> 1; j > 0; j >>= 1) {
                for (int i = tid; i < n; i += 1024) {
                    const int p = i ^ j;
                    if (p > i) {
                        const unsigned long long x = s_key[i], y = s_key[p];
                        if ((x > y) == ((i & k) == 0)) {
                            s_key[i] = y;
                            s_key[p] = x;
                        }
                    }
                }
                __syncthreads();
            }
        for (int i = tid; i < n_items; i += 1024) {
            const unsigned long long key = s_key[i];
            kb_item[i] = make_int2((int)((key >> 12) & 4095), (int)(key & 4095));
        }
    } else {
        if (tid == 0) s_c = 0;
        __syncthreads();
        for (int w = (n_q - 1) / qch; w >= 0; --w) {
            for (int base = 0; base < n_kb; base += 1024) {
                const int r = base + tid;
                int f = 0, chunk = 0;
                if (r < n_kb) {
                    const int kb = kb_order[r], lo = kb_qlo[kb], hi = kb_qhi[kb];
                    if (tt_kb_items(lo, hi, qch) > 1) {   // one item per window it touches
                        f = lo / qch <= w && w <= (hi - 1) / qch;
                        chunk = w - lo / qch;
                    } else {                              // its one item, in its top window
                        f = (hi > lo ? (hi - 1) / qch : 0) == w;
                    }
                }
                const unsigned long long m = __ballot(f);
                if (lane == 0) s_w[wave] = __popcll(m);
                __syncthreads();
                int before = s_c;
                for (int x = 0; x < wave; ++x) before += s_w[x];
                if (f) kb_item[before + __popcll(m & ((1ull << lane) - 1))] = make_int2(r, chunk);
                __syncthreads();
                if (tid == 0) {
                    int tot = 0;
                    for (int x = 0; x < 16; ++x) tot += s_w[x];
                    s_c += tot;
                }
                __syncthreads();
            }
        }
    }
    if (tid == 0) reinterpret_cast<int32_t*>(plan)[7] = n_items <= kSortItems ? 1 : 2;
}

// Plan pass 4: the dK/dV work-item offsets of the ordered key tiles, then the
// header (pairs P, n_qb, n_kt, n_kb, n_items, n_split), the split ranks and
// the work-item list.
__global__ __launch_bounds__(1024) void plan_kb_base_kernel(const int32_t* __restrict__ kb_qlo,
                                                            const int32_t* __restrict__ kb_qhi,
                                                            const int32_t* __restrict__ kb_order, int n_kb,
                                                            int qch, int32_t* __restrict__ kb_base,
                                                            int32_t* __restrict__ kb_srank, int2* __restrict__ kb_item,
                                                            int n_q,
                                                            const unsigned long long* __restrict__ pair_part,
                                                            int n_pb, int n_qb, int n_kt, uint8_t* __restrict__ plan) {
    __shared__ unsigned long long s_pairs;
    __shared__ int s_scan[1024];
    __shared__ int s_carry;
    const int tid = threadIdx.x;
    if (tid == 0) {
        s_carry = 0;
        s_pairs = 0;
    }
    __syncthreads();
    unsigned long long pairs = 0;
    for (int i = tid; i < n_pb; i += 1024) pairs += pair_part[i];
    atomicAdd(&s_pairs, pairs);
    for (int base = 0; base < n_kb; base += 1024) {
        const int r = base + tid;
        int v = 0;
        if (r < n_kb) {
            const int kb = kb_order[r];
            v = tt_kb_items(kb_qlo[kb], kb_qhi[kb], qch);
        }
        s_scan[tid] = v;
        __syncthreads();
        for (int o = 1; o < 1024; o <<= 1) {
            const int t = tid >= o ? s_scan[tid - o] : 0;
            __syncthreads();
            s_scan[tid] += t;
            __syncthreads();
        }
        if (r < n_kb) kb_base[r] = s_carry + s_scan[tid] - v;
        __syncthreads();
        if (tid == 1023) s_carry += s_scan[tid];
        __syncthreads();
    }
    __syncthreads();
    if (tid == 0) {
        kb_base[n_kb] = s_carry;
        *reinterpret_cast<unsigned long long*>(plan) = s_pairs;
        int32_t* hdr = reinterpret_cast<int32_t*>(plan);
        hdr[2] = n_qb;
        hdr[3] = n_kt;
        hdr[4] = n_kb;
        hdr[5] = s_carry;
    }
    plan_split_ranks(kb_qlo, kb_qhi, n_kb, qch, kb_srank, plan);
    plan_item_list(kb_qlo, kb_qhi, kb_order, kb_base, n_kb, n_q, qch, kb_item, plan);
}

// Plan passes 2-4 in one workgroup (plans of up to kFinishMax query blocks and
// key tiles): compaction of every query block's tile list (a wave per block),
// both heaviest-first orders (a thread per block / tile), then the work-item
// scan and the header, with the counts and the key-tile order kept in LDS.
constexpr int kFinishMax = 2048;
__device__ __forceinline__ void plan_finish_body(const uint8_t* __restrict__ cls, int n_qb, int n_kt,
                                                 const int32_t* __restrict__ kb_qlo,
                                                 const int32_t* __restrict__ kb_qhi, int n_kb, int qch,
                                                 const unsigned long long* __restrict__ pair_part, int n_pb,
                                                 int32_t* __restrict__ row_cnt, int32_t* __restrict__ row_list,
                                                 int32_t* __restrict__ row_order, int32_t* __restrict__ kb_order,
                                                 int32_t* __restrict__ kb_base, int32_t* __restrict__ kb_srank,
                                                 int2* __restrict__ kb_item, int n_q, uint8_t* __restrict__ plan) {
    __shared__ __attribute__((aligned(16))) int s_cnt[kFinishMax];
    __shared__ int s_kbo[kFinishMax];
    __shared__ __attribute__((aligned(16))) int s_kbw[kFinishMax];   // query range width of each key tile
    __shared__ int s_scan[1024];
    __shared__ int s_carry;
    __shared__ unsigned long long s_pairs;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    if (tid == 0) {
        s_carry = 0;
        s_pairs = 0;
    }
    for (int i = tid; i < n_kb; i += 1024) s_kbw[i] = kb_qhi[i] - kb_qlo[i];
    // compaction: a wave per query block, eight of its blocks (rows wave,
    // wave + 16, ...) at a time; the classes of 256 tiles of all eight rows
    // are loaded at once, so a wave waits on memory once per 256 tiles of
    // eight rows
    const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    constexpr int RB = 8;
    for (int row0 = wave; row0 < n_qb; row0 += 16 * RB) {
        int cnt[RB];
#pragma unroll
        for (int r = 0; r < RB; ++r) cnt[r] = 0;
        for (int base = 0; base < n_kt; base += 256) {
            int cv[RB][4];
#pragma unroll
            for (int r = 0; r < RB; ++r)
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int row = row0 + 16 * r, kt = base + 64 * u + lane;
                    cv[r][u] = (row < n_qb && kt < n_kt) ? cls[(size_t)row * n_kt + kt] : 0;
                }
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const int row = row0 + 16 * r;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int kt = base + 64 * u + lane, c = cv[r][u];
                    const unsigned long long m = __ballot(c != 0);
                    if (c) row_list[(size_t)row * n_kt + cnt[r] + __popcll(m & below)] = (kt << 1) | (c == 2 ? 1 : 0);
                    cnt[r] += __popcll(m);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int row = row0 + 16 * r;
            if (lane == 0 && row < n_qb) {
                s_cnt[row] = cnt[r];
                row_cnt[row] = cnt[r];
            }
        }
    }
    __syncthreads();
    // orders: rank = number of heavier entries (ties by index); query blocks on
    // threads 0-511, key tiles on 512-1023, four entries per LDS read
    {
        const bool rows = tid < 512;
        const int* arr = rows ? s_cnt : s_kbw;
        const int n_e = rows ? n_qb : n_kb;
        for (int i = tid & 511; i < n_e; i += 512) {
            const int c = arr[i];
            int rank = 0, j = 0;
#pragma unroll 4
            for (; j + 4 <= n_e; j += 4) {
                const i32x4 c4 = *(const i32x4*)(arr + j);
#pragma unroll
                for (int e = 0; e < 4; ++e) rank += (c4[e] > c) || (c4[e] == c && j + e < i);
            }
            for (; j < n_e; ++j) rank += (arr[j] > c) || (arr[j] == c && j < i);
            if (rows) {
                row_order[rank] = i;
            } else {
                s_kbo[rank] = i;
                kb_order[rank] = i;
            }
        }
    }
    unsigned long long pairs = 0;
    for (int i = tid; i < n_pb; i += 1024) pairs += pair_part[i];
    atomicAdd(&s_pairs, pairs);
    __syncthreads();
    // work-item offsets of the ordered key tiles: a scan within each wave
    // (shuffles), then over the 16 waves' totals
    for (int base = 0; base < n_kb; base += 1024) {
        const int r = base + tid;
        int v = 0;
        if (r < n_kb) {
            const int kb = s_kbo[r];
            v = tt_kb_items(kb_qlo[kb], kb_qhi[kb], qch);
        }
        int incl = v;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int up = __shfl_up(incl, o, 64);
            if (lane >= o) incl += up;
        }
        if (lane == 63) s_scan[wave] = incl;
        __syncthreads();
        int before = s_carry;
        for (int w = 0; w < wave; ++w) before += s_scan[w];
        if (r < n_kb) kb_base[r] = before + incl - v;
        __syncthreads();
        if (tid == 1023) s_carry = before + incl;
        __syncthreads();
    }
    if (tid == 0) {
        kb_base[n_kb] = s_carry;
        *reinterpret_cast<unsigned long long*>(plan) = s_pairs;
        int32_t* hdr = reinterpret_cast<int32_t*>(plan);
        hdr[2] = n_qb;
        hdr[3] = n_kt;
        hdr[4] = n_kb;
        hdr[5] = s_carry;
    }
    plan_split_ranks(kb_qlo, kb_qhi, n_kb, qch, kb_srank, plan);
    plan_item_list(kb_qlo, kb_qhi, kb_order, kb_base, n_kb, n_q, qch, kb_item, plan);
}

__global__ __launch_bounds__(1024) void plan_finish_kernel(const uint8_t* __restrict__ cls, int n_qb, int n_kt,
                                                           const int32_t* __restrict__ kb_qlo,
                                                           const int32_t* __restrict__ kb_qhi, int n_kb, int qch,
                                                           const unsigned long long* __restrict__ pair_part, int n_pb,
                                                           int32_t* __restrict__ row_cnt, int32_t* __restrict__ row_list,
                                                           int32_t* __restrict__ row_order,
                                                           int32_t* __restrict__ kb_order,
                                                           int32_t* __restrict__ kb_base, int32_t* __restrict__ kb_srank,
                                                           int2* __restrict__ kb_item, int n_q,
                                                           uint8_t* __restrict__ plan) {
    plan_finish_body(cls, n_qb, n_kt, kb_qlo, kb_qhi, n_kb, qch, pair_part, n_pb, row_cnt, row_list, row_order,
                     kb_order, kb_base, kb_srank, kb_item, n_q, plan);
}

// ---------------------------------------------------------------------------
// Several trees (the partitions of a hybrid step) in three launches: nodes,
// tokens and keys (a workgroup per tree), the plan's key pass (grid y = tree),
// the plan's finish (a workgroup per tree). The jobs travel as a kernel
// argument.
// ---------------------------------------------------------------------------
struct TreeJobDev {
    const int32_t* len;
    const int32_t* par;
    const float* bias;
    int32_t* start;
    int32_t* off;
    int32_t* hend;
    int32_t* pos;
    int32_t* node_of;
    int32_t* horizon;
    int32_t* key_lo;
    int32_t* key_hi;
    int32_t* status;
    uint8_t* plan;
    int32_t* ws;
    int n, T, pos_offset, n_past;
};
struct TreeJobsDev {
    TreeJobDev j[TT_TREE_JOBS_MAX];
    int n;
};
static_assert(sizeof(TreeJobsDev) <= 3072, "the jobs travel as one kernel argument");

struct PlanPtrs {
    PlanLayout L;
    int32_t *row_cnt, *row_order, *row_list, *kb_qlo, *kb_qhi, *kb_order, *kb_base, *kb_srank;
    int2* kb_item;
    uint8_t* cls;
    unsigned long long* pair_part;
    int nb_cls, nb_kv;
    __host__ __device__ PlanPtrs(uint8_t* base, int n_q, int n_keys) : L(n_q, n_keys) {
        row_cnt = reinterpret_cast<int32_t*>(base + L.row_cnt);
        row_order = reinterpret_cast<int32_t*>(base + L.row_order);
        row_list = reinterpret_cast<int32_t*>(base + L.row_list);
        kb_qlo = reinterpret_cast<int32_t*>(base + L.kb_qlo);
        kb_qhi = reinterpret_cast<int32_t*>(base + L.kb_qhi);
        kb_order = reinterpret_cast<int32_t*>(base + L.kb_order);
        kb_base = reinterpret_cast<int32_t*>(base + L.kb_base);
        kb_srank = reinterpret_cast<int32_t*>(base + L.kb_srank);
        kb_item = reinterpret_cast<int2*>(base + L.kb_item);
        cls = base + L.cls;
        pair_part = reinterpret_cast<unsigned long long*>(base + L.pair_part);
        nb_cls = tt_cdiv(L.n_qb * L.n_kt, 4);
        nb_kv = tt_cdiv(L.n_kb, 4);
    }
    __host__ __device__ int pass_blocks() const { return nb_cls + nb_kv + L.n_pb; }
};

__global__ __launch_bounds__(kNodeThreads) void trees_meta_keys_kernel(TreeJobsDev J) {
    const TreeJobDev& jb = J.j[blockIdx.x];
    __shared__ int s_err;
    if (threadIdx.x == 0) s_err = 0;
    const NodeView v = meta_nodes_body(jb.len, jb.par, jb.n, jb.T, jb.start, jb.off, jb.hend, s_err, jb.ws);
    meta_tokens_body(v.len, jb.n, jb.T, jb.pos_offset, v.start, v.off, v.hend, jb.pos, jb.node_of, jb.horizon,
                     jb.n_past, jb.key_lo, jb.key_hi);
    for (int j = threadIdx.x; j < jb.n_past; j += kNodeThreads) {   // gateway keys: bias 0 or -inf
        const float b = jb.bias[j];
        if (b != 0.0f && !(__builtin_isinf(b) && b < 0.0f)) atomicOr(&s_err, TT_STATUS_BAD_BIAS);
        jb.key_lo[j] = 0;
        jb.key_hi[j] = b == 0.0f ? jb.T : 0;
    }
    __syncthreads();
    if (threadIdx.x == 0) *jb.status = s_err;
}

__global__ __launch_bounds__(256) void trees_plan_pass_kernel(TreeJobsDev J) {
    const TreeJobDev& jb = J.j[blockIdx.y];
    const int n_keys = jb.n_past + jb.T;
    const PlanPtrs P(jb.plan, jb.T, n_keys);
    const int b = blockIdx.x;
    if (b >= P.pass_blocks()) return;   // workgroup-uniform
    if (b < P.nb_cls)
        plan_classify(jb.key_lo, jb.key_hi, n_keys, jb.T, P.L.n_qb, P.L.n_kt, b, P.cls);
    else if (b < P.nb_cls + P.nb_kv)
        plan_kv_range(jb.key_lo, jb.key_hi, n_keys, jb.T, P.L.n_kb, b - P.nb_cls, P.kb_qlo, P.kb_qhi);
    else
        plan_pairs_part(jb.key_lo, jb.key_hi, n_keys, jb.T, b - P.nb_cls - P.nb_kv, P.pair_part);
}

__global__ __launch_bounds__(1024) void trees_plan_finish_kernel(TreeJobsDev J) {
    const TreeJobDev& jb = J.j[blockIdx.x];
    const PlanPtrs P(jb.plan, jb.T, jb.n_past + jb.T);
    plan_finish_body(P.cls, P.L.n_qb, P.L.n_kt, P.kb_qlo, P.kb_qhi, P.L.n_kb, tt_qch(jb.T), P.pair_part, P.L.n_pb,
                     P.row_cnt, P.row_list, P.row_order, P.kb_order, P.kb_base, P.kb_srank, P.kb_item, jb.T, jb.plan);
}

}  // namespace

int tt_trees_build_impl(const tt_tree_job* jobs, int n_jobs, hipStream_t s) {
    TreeJobsDev J{};
    J.n = n_jobs;
    int max_blocks = 1;
    for (int i = 0; i < n_jobs; ++i) {
        const tt_tree_job& t = jobs[i];
        TreeJobDev& d = J.j[i];
        d.len = t.node_len;
        d.par = t.node_parent;
        d.bias = t.past_bias;
        d.start = t.node_start;
        d.off = t.node_off;
        d.hend = t.node_hend;
        d.pos = t.pos;
        d.node_of = t.node_of;
        d.horizon = t.horizon;
        d.key_lo = t.key_lo;
        d.key_hi = t.key_hi;
        d.status = t.status;
        d.plan = reinterpret_cast<uint8_t*>(t.plan);
        d.ws = reinterpret_cast<int32_t*>(t.ws);
        d.n = t.n_nodes;
        d.T = t.n_tokens;
        d.pos_offset = t.pos_offset;
        d.n_past = t.n_past;
        const PlanPtrs P(nullptr, t.n_tokens, t.n_past + t.n_tokens);
        max_blocks = max(max_blocks, P.pass_blocks());
    }
    hipLaunchKernelGGL(trees_meta_keys_kernel, dim3(n_jobs), dim3(kNodeThreads), 0, s, J);
    hipLaunchKernelGGL(trees_plan_pass_kernel, dim3(max_blocks, n_jobs), dim3(256), 0, s, J);
    hipLaunchKernelGGL(trees_plan_finish_kernel, dim3(n_jobs), dim3(1024), 0, s, J);
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}

// Limits of the batched build (each tree's metadata and plan in one workgroup).
bool tt_trees_job_fits(int n_tokens, int n_keys) {
    const PlanLayout L(n_tokens, n_keys);
    return n_tokens <= kFusedTokens && L.n_qb <= kFinishMax && L.n_kb <= kFinishMax;
}

size_t tt_meta_ws_bytes_impl(int n) {
    if (n <= 0) return 0;
    return (size_t)(5 + sparse_levels(n)) * (size_t)n * sizeof(int32_t) + 256;
}

int tt_meta_build_impl(const int32_t* len, const int32_t* par, int n, int T, int pos_offset,
                       int32_t* start, int32_t* off, int32_t* hend, int32_t* pos, int32_t* node_of,
                       int32_t* horizon, int32_t* status, void* ws, hipStream_t s) {
    if (T <= kFusedTokens) {
        hipLaunchKernelGGL(meta_tree_kernel, dim3(1), dim3(kNodeThreads), 0, s, len, par, n, T, pos_offset, start,
                           off, hend, pos, node_of, horizon, status, reinterpret_cast<int32_t*>(ws));
        return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
    }
    hipLaunchKernelGGL(meta_nodes_kernel, dim3(1), dim3(kNodeThreads), 0, s, len, par, n, T, start, off,
                       hend, status, reinterpret_cast<int32_t*>(ws));
    if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    hipLaunchKernelGGL(meta_tokens_kernel, dim3(tt_cdiv(T, 256)), dim3(256), 0, s, start, off, hend, n, T,
                       pos_offset, pos, node_of, horizon);
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}

int tt_keys_build_impl(const float* bias, int n_past, const int32_t* horizon, int n_q, int32_t* key_lo,
                       int32_t* key_hi, int32_t* status, hipStream_t s) {
    const int nk = n_past + n_q;
    hipLaunchKernelGGL(keys_kernel, dim3(tt_cdiv(nk, 256)), dim3(256), 0, s, bias, n_past, horizon, n_q,
                       key_lo, key_hi, status);
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}

int tt_dense_mask_impl(const int32_t* key_lo, const int32_t* key_hi, int n_keys, int n_q, uint8_t* mask,
                       hipStream_t s) {
    hipLaunchKernelGGL(dense_mask_kernel, dim3(tt_cdiv(n_keys, 256), n_q), dim3(256), 0, s, key_lo, key_hi,
                       n_keys, n_q, mask);
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}

size_t tt_plan_bytes_impl(int n_q, int n_keys) { return PlanLayout(n_q, n_keys).total; }

int tt_plan_build_impl(const int32_t* key_lo, const int32_t* key_hi, int n_keys, int n_q, void* plan,
                       hipStream_t s) {
    const PlanLayout L(n_q, n_keys);
    uint8_t* base = reinterpret_cast<uint8_t*>(plan);
    int32_t* row_cnt = reinterpret_cast<int32_t*>(base + L.row_cnt);
    int32_t* row_order = reinterpret_cast<int32_t*>(base + L.row_order);
    int32_t* row_list = reinterpret_cast<int32_t*>(base + L.row_list);
    int32_t* kb_qlo = reinterpret_cast<int32_t*>(base + L.kb_qlo);
    int32_t* kb_qhi = reinterpret_cast<int32_t*>(base + L.kb_qhi);
    int32_t* kb_order = reinterpret_cast<int32_t*>(base + L.kb_order);
    int32_t* kb_base = reinterpret_cast<int32_t*>(base + L.kb_base);
    int32_t* kb_srank = reinterpret_cast<int32_t*>(base + L.kb_srank);
    int2* kb_item = reinterpret_cast<int2*>(base + L.kb_item);
    uint8_t* cls = base + L.cls;
    unsigned long long* pair_part = reinterpret_cast<unsigned long long*>(base + L.pair_part);
    const int nb_cls = tt_cdiv(L.n_qb * L.n_kt, 4), nb_kv = tt_cdiv(L.n_kb, 4);
    hipLaunchKernelGGL(plan_keys_pass_kernel, dim3(nb_cls + nb_kv + L.n_pb), dim3(256), 0, s, key_lo, key_hi, n_keys,
                       n_q, L.n_qb, L.n_kt, L.n_kb, nb_cls, nb_kv, cls, kb_qlo, kb_qhi, pair_part);
    if (L.n_qb <= kFinishMax && L.n_kb <= kFinishMax) {
        hipLaunchKernelGGL(plan_finish_kernel, dim3(1), dim3(1024), 0, s, cls, L.n_qb, L.n_kt, kb_qlo, kb_qhi, L.n_kb,
                           tt_qch(n_q), pair_part, L.n_pb, row_cnt, row_list, row_order, kb_order, kb_base, kb_srank,
                           kb_item, n_q, base);
        return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
    }
    hipLaunchKernelGGL(plan_compact_kernel, dim3(tt_cdiv(L.n_qb, 4)), dim3(256), 0, s, cls, L.n_qb, L.n_kt,
                       row_cnt, row_list);
    const int nb_ro = tt_cdiv(L.n_qb, 256);
    hipLaunchKernelGGL(plan_orders_kernel, dim3(nb_ro + tt_cdiv(L.n_kb, 256)), dim3(256), 0, s, row_cnt, L.n_qb,
                       nb_ro, kb_qlo, kb_qhi, L.n_kb, row_order, kb_order);
    hipLaunchKernelGGL(plan_kb_base_kernel, dim3(1), dim3(1024), 0, s, kb_qlo, kb_qhi, kb_order, L.n_kb, tt_qch(n_q),
                       kb_base, kb_srank, kb_item, n_q, pair_part, L.n_pb, L.n_qb, L.n_kt, base);
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}
