// Device code shared by the bf16 tree-attention kernels (forward in
// tt_attn_fwd_bf16.hip, backward in tt_attn_bwd_bf16.hip): LDS tile layout,
// MFMA operand reads, global -> LDS staging, visibility masks and
// the workgroup -> tile mapping.
//
// Tree-masked GQA flash attention for gfx950, bf16 in / fp32 accumulate.
//
// Forward and dQ pass (query-major): a workgroup owns TT_BQ = 128 queries of
// one q head; each of its four waves keeps 32 queries in registers and walks
// the non-empty key tiles of the plan. Scores are computed transposed,
// S^T = K Q^T with v_mfma_f32_32x32x16_bf16, so a lane owns one query column:
// the online-softmax row max needs a single cross-half exchange and the
// probabilities feed O^T = V^T P^T straight from the accumulators. K and V
// tiles sit in LDS in their natural [key][d] layout; the V^T (and, for dQ,
// K^T) operands come out of them through gfx950's transposing LDS read
// (ds_read_b64_tr_b16). Tiles are software-pipelined: the next tile's direct
// global -> LDS loads are in flight while the current tile computes out of
// the other LDS stage; one barrier per tile.
//
// dK/dV pass (key-major): a workgroup owns TT_BKB = 128 keys of one kv head;
// each wave keeps K of 32 keys in registers (V of the 128 keys sits in LDS)
// and dK, dV of those keys in fp32 accumulators, and walks a range of queries
// that can see them (for a DFS-packed tree the range is contiguous: [first
// key, subtree end)) for the Hq/Hkv q heads of the group, with Q and dO blocks
// moved into LDS by direct global -> LDS loads (double-buffered) and read both
// row-wise and transposed. Ranges longer than
// tt_qch(n_q) queries (half the largest power of two <= n_q, within
// [256, 4096]) are split into several work items; a persistent grid walks the
// items widest-first.
// Unsplit tiles write dK/dV directly; split tiles add fp32 partial sums into a
// workspace that a finalize pass converts.
//
// Visibility: key j is seen by query i iff key_lo[j] <= i < key_hi[j]; the
// plan marks each (query block, key tile) empty (skipped), full (no mask) or
// partial (interval test per element).
#pragma once

#include "tt_common.h"
#include "tt_internal.h"

namespace {

typedef __bf16 bf16;

constexpr int D = 128;

// LDS tiles hold tokens in their natural [token][d] order. Layouts (64 banks
// x 4 bytes; a 16-byte read serves 16 lanes per LDS pass, a transposed 8-byte
// read 32):
//   ROW_R = 272-byte rows (the dK/dV pass's V, read only as rows): 16
//           consecutive rows start on 16 different 16-byte bank groups, so a
//           row operand read (16 lanes = 16 rows, one chunk) runs in one pass;
//   ROWX, the XOR-swizzled 320-byte rows below (the dK/dV pass's Q and dO
//           blocks, read both ways);
//   row groups (GPITCH below: the forward's and the dQ pass's K and V tiles,
//           read both ways and filled by direct loads).
// Every layout is free of bank conflicts for the reads made of it.
constexpr int ROW_R = D + 8;
template <int S>
__device__ __forceinline__ int tile_off(int r, int d) { return r * S + d; }

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// acc + v[i0] + v[i0+1] + v[i0+2] + v[i0+3] (fp32 accumulation, v_dot2c_f32_bf16).
__device__ __forceinline__ float sum4_bf16(const bf16x8& v, int i0, float acc) {
    const bf16x2 one = {(bf16)1.0f, (bf16)1.0f};
    acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{v[i0], v[i0 + 1]}, one, acc, false);
    return __builtin_amdgcn_fdot2_f32_bf16(bf16x2{v[i0 + 2], v[i0 + 3]}, one, acc, false);
}

// Forward online softmax: the running row max is moved only when a tile's max
// exceeds it by more than this many log2 units.
#define TT_RESCALE_LOG2 8.0f

template <int I>
struct IntC {
    static constexpr int value = I;
};

__device__ __forceinline__ bf16x8 zero8() {
    bf16x8 z;
#pragma unroll
    for (int i = 0; i < 8; ++i) z[i] = (bf16)0.0f;
    return z;
}

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void glb_void;

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
// (i & 3) of the 8-byte chunks read by lanes 4k + (i >> 2), k = 0..3.
__device__ __forceinline__ bf16x4 ds_read_tr(const bf16* p) {
    const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p));
    return __builtin_bit_cast(bf16x4, r);
}

// MFMA operand "row = token, k = 16 head dims": X[r][d0 .. d0+7], d0 % 8 == 0.
template <int S>
__device__ __forceinline__ bf16x8 read_row_operand(const bf16* X, int r, int d0) {
    return *(const bf16x8*)(X + tile_off<S>(r, d0));
}

// Swizzled layout for tiles read both row-wise and transposed many times
// (the dK/dV pass's Q and dO blocks): 320-byte rows, 16-byte chunk c of row r
// stored at chunk c ^ ((r >> 2) & 3). Both read patterns then reach every
// bank once per LDS pass (64 banks x 4 bytes; 16-byte reads serve 16 lanes
// per pass, transposed 8-byte reads 32).
constexpr int ROWX = D + 32;
__device__ __forceinline__ int tile_offx(int r, int d) {
    return r * ROWX + ((((d >> 3) ^ ((r >> 2) & 3))) << 3) + (d & 7);
}

// Lane offsets into a swizzled tile (every access is a lane base plus a
// compile-time offset). Row operand for head dims 16t + 8*half .. +7 of row
// r: at (t odd ? o : e) + 32*(t/2).
struct RowOffsX {
    int e, o;
};
__device__ __forceinline__ RowOffsX row_offsx(int r, int half) {
    const int f = (r >> 2) & 3, b = r * ROWX, x = half ^ (f & 1);
    return {b + 8 * (2 * (f >> 1) + x), b + 8 * (2 * (1 ^ (f >> 1)) + x)};
}
template <int T>
__device__ __forceinline__ bf16x8 read_rowx(const bf16* X, const RowOffsX& ro) {
    return *(const bf16x8*)(X + ((T & 1) ? ro.o : ro.e) + 32 * (T >> 1));
}
// Transposed operand "column = head dim, k = 16 tokens" from a swizzled tile:
// lane l gets X[r0 + kappa(e)][dbase + (l & 31)], kappa(e) = 8*(e/4) +
// 4*(l>>5) + (e%4) -- the accumulator row order, so it pairs with
// probabilities taken straight from a score accumulator; r0 % 16 == 0,
// dbase % 32 == 0.
struct TrOffsX {
    int a, b;   // rows +0..7 and +8..15 of the 16-row group
};
__device__ __forceinline__ TrOffsX tr_offsx(int lane) {
    const int j = lane & 15, grp = lane >> 4, h = grp >> 1;
    const int rl = 4 * h + (j >> 2);
    const int c = 2 * (grp & 1) + ((j & 3) >> 1), p = 4 * (j & 1);
    return {rl * ROWX + ((c ^ h) << 3) + p, (rl + 8) * ROWX + ((c ^ (h ^ 2)) << 3) + p};
}
__device__ __forceinline__ bf16x8 read_trx(const bf16* X, const TrOffsX& to, int r0, int dbase) {
    return cat44(ds_read_tr(X + to.a + r0 * ROWX + dbase), ds_read_tr(X + to.b + r0 * ROWX + dbase));
}

// Row-group layout (the forward's and the dQ pass's key tiles): rows in groups
// of four (1 KB, one direct-load instruction each) at a pitch of 1040 bytes;
// 16-byte chunk c of row r sits at chunk c ^ 4 (r & 3) of its row. Row reads (16 lanes = 16 rows, one
// chunk) and transposed reads (32 lanes = 4 rows x 4 chunks) both reach every
// bank once per LDS pass.
constexpr int GPITCH = 520;   // elements per group of four rows
__device__ __forceinline__ int tile_offg(int r, int d) {
    return (r >> 2) * GPITCH + (r & 3) * D + ((((d >> 3) ^ ((r & 3) << 2))) << 3) + (d & 7);
}
// Row operand of the lane's key row (col of a 32-row half) for head dims
// 16 t + 8 half .. +7: at base[t >> 2][(t >> 1) & 1] + 16 (t & 1).
struct RowOffsG {
    int b[4];
};
__device__ __forceinline__ RowOffsG row_offsg(int col, int half) {
    const int f = col & 3, rb = (col >> 2) * GPITCH + f * D + 8 * half;
    RowOffsG o;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int v = 0; v < 2; ++v) o.b[2 * u + v] = rb + 64 * (u ^ (f >> 1)) + 32 * (v ^ (f & 1));
    return o;
}
template <int T>
__device__ __forceinline__ bf16x8 read_rowg(const bf16* X, const RowOffsG& ro) {
    return *(const bf16x8*)(X + ro.b[T >> 1] + 16 * (T & 1));
}
// Transposed operand (as read_trx) of rows r0 .. r0 + 15 (r0 % 16 == 0), head
// dims 32 db .. +31: at base[db] + (r0 / 4) GPITCH (+ 2 GPITCH: rows + 8).
struct TrOffsG {
    int b[4];
};
__device__ __forceinline__ TrOffsG tr_offsg(int lane) {
    const int j = lane & 15, grp = lane >> 4, h = grp >> 1, q = j >> 2;
    const int c = 2 * (grp & 1) + ((j & 3) >> 1), p = 4 * (j & 1);
    TrOffsG o;
#pragma unroll
    for (int db = 0; db < 4; ++db) o.b[db] = h * GPITCH + q * D + 32 * (db ^ q) + 8 * c + p;
    return o;
}
__device__ __forceinline__ bf16x8 read_trg(const bf16* X, const TrOffsG& to, int r0, int db) {
    const bf16* x = X + to.b[db] + (r0 >> 2) * GPITCH;
    return cat44(ds_read_tr(x), ds_read_tr(x + 2 * GPITCH));
}

template <int I>
struct IntT {
    static constexpr int value = I;
};
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(IntT<I>{});
        static_for<N, I + 1>(f);
    }
}


// Direct global -> LDS staging (buffer_load ... lds): no staging registers and
// no LDS store instructions. One wave instruction moves 64 x 16 bytes from
// per-lane buffer offsets to 1 KB of consecutive LDS bytes (lane l: byte 16 l
// from the LDS address in M0). The loads are issued as inline assembly, so
// the compiler's wait insertion neither tracks nor orders them: the issuing
// wave waits for them (wait_vmem) before the barrier that publishes the data.
// An operation the compiler does not count can only make its own vmcnt waits
// stricter, never too weak, since the counter retires operations in issue
// order.
//
// Raw buffer resource over [base, base + bytes); loads past the end read zeros.
__device__ __forceinline__ i32x4 dma_rsrc(const void* base, uint32_t bytes) {
    const uint64_t p = (uint64_t)base;
    return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)p),
                 __builtin_amdgcn_readfirstlane((int)((uint32_t)(p >> 32) & 0xffff)),
                 __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000};
}
// (The compiler sets M0; the s_nop is the wait state between that write and
// the load that reads it.)
__device__ __forceinline__ void lds_dma16(const i32x4& rsrc, uint32_t lds, uint32_t voff) {
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(voff), "s"(rsrc), "{m0}"(lds) : "memory");
}
// Same, with a uniform byte offset (scalar register) added to every lane's.
__device__ __forceinline__ void lds_dma16s(const i32x4& rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 :
                 : "v"(voff), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(soff)), "{m0}"(lds)
                 : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_void*)p; }
// s_waitcnt vmcnt(0): every vector memory operation of the wave, direct loads
// included, has completed.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// Register staging: thread t holds rows (t/16) + 16*i (i < NROWS/16) at head
// dims 8*(t%16) .. +7 of a tile; 16 lanes cover one 256-byte row, and a wave
// instruction moves four whole rows.
template <int NROWS>
struct RowRegs {
    bf16x8 x[NROWS / 16];
};

template <int NROWS, typename RowPtr>
__device__ __forceinline__ void fetch_rows(RowRegs<NROWS>& r, int tid, RowPtr row_ptr) {
    const int dc = (tid & 15) * 8, r0 = tid >> 4;
#pragma unroll
    for (int i = 0; i < NROWS / 16; ++i) r.x[i] = *(const bf16x8*)(row_ptr(r0 + 16 * i) + dc);
}

// Same, for NROWS rows of one tensor that all exist: row 0 at `base` (a
// uniform pointer), rows `stb` bytes apart. The loads go through a buffer
// resource: base and row steps in scalar registers, one 32-bit lane offset.
template <int NROWS>
__device__ __forceinline__ void fetch_rows_buf(RowRegs<NROWS>& r, int tid, const void* base, uint32_t stb) {
    const uint32_t bytes = (NROWS - 1) * stb + 2 * D;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
    const uint32_t vo = (tid >> 4) * stb + 16 * (tid & 15);
#pragma unroll
    for (int i = 0; i < NROWS / 16; ++i)
        r.x[i] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)vo, (int)(16 * i * stb), 0));
}

// Stores staged rows in a tile of row stride S elements.
template <int NROWS, int S>
__device__ __forceinline__ void store_rows(const RowRegs<NROWS>& r, int tid, bf16* X) {
    const int dc = (tid & 15) * 8, r0 = tid >> 4;
#pragma unroll
    for (int i = 0; i < NROWS / 16; ++i) *(bf16x8*)(X + tile_off<S>(r0 + 16 * i, dc)) = r.x[i];
}

__device__ __forceinline__ const bf16* key_row(const AttnDev& a, int kk, int g, bool isv) {
    if (kk < a.n_past) {
        return isv ? (const bf16*)a.vp + kk * a.vp_st + g * a.vp_sh
                   : (const bf16*)a.kp + kk * a.kp_st + g * a.kp_sh;
    }
    const int64_t t = kk - a.n_past;
    return isv ? (const bf16*)a.v + t * a.v_st + g * a.v_sh : (const bf16*)a.k + t * a.k_st + g * a.k_sh;
}

struct Bounds {
    int lo, hi;
};

__device__ __forceinline__ void fetch_bounds(const AttnDev& a, int kt, Bounds& r) {
    const int t = threadIdx.x;
    if (t < TT_BK) {
        const int kk = kt * TT_BK + t;
        r.lo = kk < a.n_keys ? a.key_lo[kk] : 0;
        r.hi = kk < a.n_keys ? a.key_hi[kk] : 0;
    }
}

// Staging of key tile kt into row-group tiles: waves 0-1 move K, waves 2-3
// V, eight 4-row groups each, by direct loads when the tile lies wholly in the gateway or wholly
// in the own keys; a tile that straddles the two or runs past the last key
// is copied in commit() (rows past the last key alias it; their empty bounds
// mask them).
struct KvTileDma {
    int k0;
    bool direct;
    __device__ __forceinline__ void begin(const AttnDev& a, int kt, int g, bf16* K, bf16* V) {
        k0 = kt * TT_BK;
        const bool past = k0 + TT_BK <= a.n_past;
        direct = !(past || (k0 >= a.n_past && k0 + TT_BK <= a.n_keys));
        if (direct) return;   // uniform
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
        const bool isk = wave < 2;
        const int64_t st = past ? (isk ? a.kp_st : a.vp_st) : (isk ? a.k_st : a.v_st);
        const int64_t sh = past ? (isk ? a.kp_sh : a.vp_sh) : (isk ? a.k_sh : a.v_sh);
        const bf16* t = (const bf16*)(past ? (isk ? a.kp : a.vp) : (isk ? a.k : a.v));
        const int r0 = 32 * (wave & 1);                       // first row of this wave's groups
        const int64_t row0 = (past ? k0 : k0 - a.n_past) + r0;
        const uint32_t stb = 2u * (uint32_t)st;
        const i32x4 rs = dma_rsrc(t + row0 * st + g * sh, 31u * stb + 2u * D);
        const uint32_t vo = (uint32_t)(lane >> 4) * stb + 16u * (uint32_t)((lane & 15) ^ ((lane >> 4) << 2));
        const uint32_t l0 = lds_addr(isk ? K : V) + 2u * GPITCH * (uint32_t)(r0 >> 2);
#pragma unroll
        for (int i = 0; i < 8; ++i) lds_dma16s(rs, l0 + 2u * GPITCH * i, vo, 4u * i * stb);
    }
    __device__ __forceinline__ void commit(const AttnDev& a, int g, bf16* K, bf16* V) {
        if (!direct) {
            wait_vmem();
            return;
        }
        const int dc = (threadIdx.x & 15) * 8, r0 = threadIdx.x >> 4;
        for (int i = 0; i < TT_BK / 16; ++i) {
            const int r = r0 + 16 * i, kk = min(k0 + r, a.n_keys - 1);
            *(bf16x8*)(K + tile_offg(r, dc)) = *(const bf16x8*)(key_row(a, kk, g, false) + dc);
            *(bf16x8*)(V + tile_offg(r, dc)) = *(const bf16x8*)(key_row(a, kk, g, true) + dc);
        }
    }
};

__device__ __forceinline__ void store_bounds(const Bounds& r, int* s_lo, int* s_hi) {
    const int t = threadIdx.x;
    if (t < TT_BK) {
        s_lo[t] = r.lo;
        s_hi[t] = r.hi;
    }
}

// Lane's 32 query-column scores -> -inf where the key is invisible.
__device__ __forceinline__ void mask_scores(f32x16 (&s)[2], const int* s_lo, const int* s_hi, int qi, int half) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int grp = 0; grp < 4; ++grp) {
            const int k0 = 32 * b + 8 * grp + 4 * half;
            const i32x4 lo = *(const i32x4*)(s_lo + k0);
            const i32x4 hi = *(const i32x4*)(s_hi + k0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bool vis = lo[e] <= qi && qi < hi[e];
                s[b][4 * grp + e] = vis ? s[b][4 * grp + e] : -INFINITY;
            }
        }
    }
}

// Which 32-key halves of a tile hold a key visible to any of the wave's 32
// queries [q0, q0 + 32): bit b set for half b (lane l tests key l of the
// tile). Wave-uniform. A half with no such key contributes nothing (every
// score -inf, every probability and dS zero), so a wave skips it.
__device__ __forceinline__ int visible_halves(const int* s_lo, const int* s_hi, int q0, int lane) {
    const bool v = max(s_lo[lane], q0) < min(s_hi[lane], q0 + 32);
    const unsigned long long b = __ballot(v);
    return __builtin_amdgcn_readfirstlane(((unsigned)b != 0u ? 1 : 0) | ((unsigned)(b >> 32) != 0u ? 2 : 0));
}

// As mask_scores, for one 32-key half of the tile (lo/hi point at its first key).
__device__ __forceinline__ void mask_half(f32x16& s, const int* s_lo, const int* s_hi, int qi, int half) {
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
        const int k0 = 8 * grp + 4 * half;
        const i32x4 lo = *(const i32x4*)(s_lo + k0);
        const i32x4 hi = *(const i32x4*)(s_hi + k0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bool vis = lo[e] <= qi && qi < hi[e];
            s[4 * grp + e] = vis ? s[4 * grp + e] : -INFINITY;
        }
    }
}

// blockIdx.x -> (query block, q head). Workgroups are dispatched round-robin
// over the 8 XCDs; each XCD gets the q heads of whole kv-head groups so their
// K/V stay in its L2, and the heaviest query blocks go first.
__device__ __forceinline__ void decode_qblock(const AttnDev& a, int& qb, int& h) {
    const int bid = blockIdx.x;
    if ((a.hq & 7) == 0) {
        const int hpx = a.hq >> 3, xcd = bid & 7, slot = bid >> 3;
        h = xcd * hpx + slot % hpx;
        qb = a.row_order[slot / hpx];
    } else {
        h = bid % a.hq;
        qb = a.row_order[bid / a.hq];
    }
    // Workgroup-uniform: keeps the tile bases and buffer descriptors derived
    // from qb in scalar registers (no per-load uniformity loops).
    qb = __builtin_amdgcn_readfirstlane(qb);
    h = __builtin_amdgcn_readfirstlane(h);
}


// Four fp32 values into element idx.. of a bf16 or fp32 output.
template <typename TOut>
__device__ __forceinline__ void store_out4(void* base, size_t idx, const f32x4& x) {
    if constexpr (sizeof(TOut) == 2) {
        bf16x4 w;
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = (bf16)x[i];
        *(bf16x4*)((bf16*)base + idx) = w;
    } else {
        *(f32x4*)((float*)base + idx) = x;
    }
}

// Split key tiles sum their dK/dV in fp32 rows of the workspace, compacted:
// the tile of split rank r (plan kb_srank) owns rows 128 r .. 128 r + 127, so
// key `key` of tile kb sits in row split_row(...) + key. A tile whose rank is
// beyond the rows the workspace holds (split_cap) writes nothing there, and
// its keys' gradients become NaN in the finalize.
struct SplitRows {
    int64_t row0;   // row of key 0 of the tile's run (rows 128 r - 128 kb + key)
    bool ok;        // the tile is split and its rows fit the workspace
};
__device__ __forceinline__ SplitRows split_rows(const AttnDev& a, const BwdDev& bw, int kb) {
    const int r = a.kb_srank[kb];
    return {((int64_t)r - kb) * TT_BKB, r >= 0 && (int64_t)r < bw.split_cap};
}

// Zero the fp32 sums of a split tile's own keys before the dK/dV pass (split
// gateway keys add straight into the caller's fp32 accumulators; 16-byte
// vectors: the workspace and the gateway accumulators are 16-byte aligned and
// rows are 128 floats), by one workgroup per (key tile kb, kv head g).
__device__ __forceinline__ void split_zero_tile(const AttnDev& a, const BwdDev& bw, int kb, int g) {
    if (tt_kb_items(a.kb_qlo[kb], a.kb_qhi[kb], tt_qch(a.n_q)) <= 1) return;
    const SplitRows sr = split_rows(a, bw, kb);
    if (!sr.ok) return;
    const int k_first = max(kb * TT_BKB, a.n_past), k_end = min(kb * TT_BKB + TT_BKB, a.n_keys);
    for (int e = threadIdx.x; e < (k_end - k_first) * (D / 4); e += 256) {
        const int key = k_first + e / (D / 4);
        const size_t idx = ((size_t)(sr.row0 + key) * a.hkv + g) * D + 4 * (e % (D / 4));
        *(f32x4*)(bw.dk_ws + idx) = (f32x4){};
        *(f32x4*)(bw.dv_ws + idx) = (f32x4){};
    }
}

__global__ __launch_bounds__(256) void bwd_split_zero_kernel(AttnDev a, BwdDev bw) {
    split_zero_tile(a, bw, blockIdx.x, blockIdx.y);
}

// ... and convert them to dk/dv after it: the fp32 sums of a quarter (32
// keys) of tile kb's own keys for kv head g, by one workgroup. Each thread
// issues its four loads before its first store, so the loads' latency is
// paid once rather than four times in a row.
template <typename TOut>
__device__ __forceinline__ void split_convert_quarter(const AttnDev& a, const BwdDev& bw, int kb, int g, int qt) {
    const SplitRows sr = split_rows(a, bw, kb);
    const int k_first = max(kb * TT_BKB + 32 * qt, a.n_past), k_end = min(kb * TT_BKB + 32 * qt + 32, a.n_keys);
    const int n = (k_end - k_first) * (D / 4);
    const float qnan = __int_as_float(0x7fc00000);   // by its bits (built without NaN semantics)
    f32x4 gk[4], gv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = threadIdx.x + 256 * i;
        gk[i] = gv[i] = (f32x4){qnan, qnan, qnan, qnan};
        if (e < n && sr.ok) {
            const size_t widx = ((size_t)(sr.row0 + k_first + e / (D / 4)) * a.hkv + g) * D + 4 * (e % (D / 4));
            gk[i] = *(const f32x4*)(bw.dk_ws + widx);
            gv[i] = *(const f32x4*)(bw.dv_ws + widx);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = threadIdx.x + 256 * i;
        if (e < n) {
            const size_t idx = ((size_t)(k_first + e / (D / 4) - a.n_past) * a.hkv + g) * D + 4 * (e % (D / 4));
            store_out4<TOut>(bw.dk, idx, gk[i]);
            store_out4<TOut>(bw.dv, idx, gv[i]);
        }
    }
}

// Grid (n_kb, Hkv, 4): workgroup z converts the z-th quarter of a split tile.
template <typename TOut>
__global__ __launch_bounds__(256) void bwd_split_finalize_kernel(AttnDev a, BwdDev bw) {
    const int kb = blockIdx.x, g = blockIdx.y;
    if (tt_kb_items(a.kb_qlo[kb], a.kb_qhi[kb], tt_qch(a.n_q)) <= 1) return;
    split_convert_quarter<TOut>(a, bw, kb, g, blockIdx.z);
}

// Deterministic mode: one workgroup per (key tile rank, kv head) sums a split
// tile's partials in item order (first item's in the fp32 rows, then the
// slots) and writes dk/dv, or adds gateway keys' sums to the accumulators.
template <typename TOut>
__global__ __launch_bounds__(256) void bwd_split_finalize_det_kernel(AttnDev a, BwdDev bw) {
    const int rank = blockIdx.x, g = blockIdx.y;
    const int kb = a.kb_order[rank];
    const int m = tt_kb_items(a.kb_qlo[kb], a.kb_qhi[kb], tt_qch(a.n_q));
    if (m <= 1) return;
    const int k_first = kb * TT_BKB, k_end = min(kb * TT_BKB + TT_BKB, a.n_keys);
    const int64_t slot0 = (int64_t)(a.kb_base[rank] - rank) * TT_BKB;   // slot rows of the tile's second item
    const SplitRows sr = split_rows(a, bw, kb);
    // rows or slots the workspace lacks (split_tiles or det_slots below the
    // tree's count): the work items wrote none there, and the tile's
    // gradients are NaN
    const bool lacks = !sr.ok || (int64_t)(a.kb_base[rank] - rank) + (m - 1) > bw.det_cap;
    for (int e = threadIdx.x; e < (k_end - k_first) * (D / 4); e += 256) {
        const int key = k_first + e / (D / 4), d = 4 * (e % (D / 4));
        const size_t widx = ((size_t)key * a.hkv + g) * D + d;
        const size_t cidx = ((size_t)(sr.row0 + key) * a.hkv + g) * D + d;
        f32x4 gk = {}, gv = {};
        if (!lacks) {
            gk = *(const f32x4*)(bw.dk_ws + cidx);
            gv = *(const f32x4*)(bw.dv_ws + cidx);
        }
        for (int c = 1; c < (lacks ? 1 : m); ++c) {
            const size_t sidx = ((size_t)(slot0 + (int64_t)(c - 1) * TT_BKB + key - k_first) * a.hkv + g) * D + d;
            gk += *(const f32x4*)(bw.dk_slot + sidx);
            gv += *(const f32x4*)(bw.dv_slot + sidx);
        }
        if (lacks) {   // a quiet NaN by its bits (this header is also built without NaN semantics)
            const float qnan = __int_as_float(0x7fc00000);
            gk = gv = (f32x4){qnan, qnan, qnan, qnan};
        }
        if (key < a.n_past) {
            if (bw.dk_acc) {
                *(f32x4*)(bw.dk_acc + widx) += gk;
                *(f32x4*)(bw.dv_acc + widx) += gv;
            }
            continue;
        }
        const size_t idx = ((size_t)(key - a.n_past) * a.hkv + g) * D + d;
        store_out4<TOut>(bw.dk, idx, gk);
        store_out4<TOut>(bw.dv, idx, gv);
    }
}


}  // namespace
