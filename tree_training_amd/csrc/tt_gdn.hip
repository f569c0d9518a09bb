// Tree gated delta rule (the linear-attention layers of Qwen3.5-style models)
// over a DFS-packed tree: forward for gfx950.
//
// Semantics: the gated delta rule token by token along every root-to-leaf
// path — each node continues from its parent's final state (zero state for a
// root) — evaluated exactly in TT_GDN_CHUNK = 32-token chunks (a node is cut
// into consecutive chunks; its last chunk may be short):
//   G = cumsum(g), D[i][j] = exp(G_i - G_j) (j <= i),
//   N = -strictly_lower(beta k k^T * D),  T = (I - N)^-1,
//   U = T (beta v),  W = T (beta e^G k),  A = lower_incl(q k^T * D),
//   V' = U - W S,  O = e^G (q S) + A V',  S <- e^{G_last} S + (k e^{G_last - G})^T V'.
// q and k are l2-normalised in the kernels and q is scaled; v head h reads q/k
// head h / (Hv / Hk).
//
// Two kernels:
//  * gdn_prep_kernel — one workgroup per (chunk, v head), all chunks at once:
//    everything that does not depend on the state (A, T by a product of
//    (I + N^(2^r)) factors, U, W, G) into the workspace.
//  * gdn_scan_kernel — one workgroup per (node, v head, 32-column slice of
//    the value dimension; the delta rule is independent per value column),
//    one launch per tree level so a node's parent state (in the caller's
//    node_states buffer) is complete when it starts; walks the node's chunks
//    with its 128 x 32 state slice in LDS.
// Every product is fp32 FMA on the vector ALUs (fp32 end to end).
#include "tt_common.h"
#include "tt_internal.h"

namespace {

constexpr int GD = 128;           // head dim (Dk = Dv)
constexpr int GC = TT_GDN_CHUNK;  // chunk length (32)
constexpr int GT = 256;           // threads per workgroup
constexpr int RS = GD + 4;        // row stride of [GC x GD] tiles (floats): rows 4 banks apart
constexpr int MS = GC + 4;        // row stride of [GC x GC] matrices
constexpr int NSL = 4;            // value-column slices in the scan
constexpr int VS = GD / NSL;      // columns per slice
constexpr int VP = VS + 4;        // row stride of [* x VS] tiles

// Workspace per (chunk, v head), floats: W [GC][GD], U [GC][GD], A [GC][GC], G [GC].
constexpr size_t kWsW = 0, kWsU = GC * GD, kWsA = 2 * GC * GD, kWsG = 2 * GC * GD + GC * GC;
constexpr size_t kWsChunk = kWsG + GC;

template <typename T>
__device__ __forceinline__ void load16(const T* p, float (&x)[16]) {
    if constexpr (sizeof(T) == 2) {
        const bf16x8 a = *(const bf16x8*)p, b = *(const bf16x8*)(p + 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            x[e] = (float)a[e];
            x[8 + e] = (float)b[e];
        }
    } else {
#pragma unroll
        for (int e = 0; e < 16; e += 4) {
            const f32x4 a = *(const f32x4*)(p + e);
            x[e] = a[0]; x[e + 1] = a[1]; x[e + 2] = a[2]; x[e + 3] = a[3];
        }
    }
}

template <typename T>
__device__ __forceinline__ void store4(T* p, const f32x4& x) {
    if constexpr (sizeof(T) == 2) {
        bf16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = (__bf16)x[e];
        *(bf16x4*)p = w;
    } else {
        *(f32x4*)p = x;
    }
}

// Sum over the 8 consecutive lanes that hold one row.
__device__ __forceinline__ float row8_sum(float x) {
    x += __shfl_xor(x, 1);
    x += __shfl_xor(x, 2);
    x += __shfl_xor(x, 4);
    return x;
}

// Chunk `c` -> (first token, length); false for a malformed chunk list.
__device__ __forceinline__ bool chunk_span(const GdnDev& p, int c, int& start, int& len) {
    const int node = p.chunk_node[c];
    if (node < 0 || node >= p.n_nodes) return false;
    const int ci = c - p.node_chunk0[node];
    const int ns = p.node_start[node], nl = p.node_len[node];
    if (ns < 0 || nl < 0 || ns > p.n_tokens - nl || ci < 0 || GC * ci >= nl) return false;
    start = ns + GC * ci;
    len = min(GC, nl - GC * ci);
    return true;
}

// Rows of one chunk (zeros past its length): l2-normalised q (times scale),
// k, and, when V is given, v; thread t handles row t/8, 16 dims.
template <typename TIn>
__device__ __forceinline__ void load_chunk_rows(const GdnDev& p, int start, int len, int h, float* Q, float* K,
                                                float* V) {
    const int t = threadIdx.x, i = t >> 3, d0 = 16 * (t & 7), hk = h / p.rep;
    const bool valid = i < len;
    const int64_t tok = start + i;
    float qv[16], kv[16], vv[16];
    if (valid) {
        load16((const TIn*)p.q + tok * p.q_st + hk * p.q_sh + d0, qv);
        load16((const TIn*)p.k + tok * p.k_st + hk * p.k_sh + d0, kv);
        if (V) load16((const TIn*)p.v + tok * p.v_st + h * p.v_sh + d0, vv);
    } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) qv[e] = kv[e] = vv[e] = 0.0f;
    }
    float sq = 0.0f, sk = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        sq = fmaf(qv[e], qv[e], sq);
        sk = fmaf(kv[e], kv[e], sk);
    }
    sq = row8_sum(sq);
    sk = row8_sum(sk);
    const float fq = (p.l2 ? 1.0f / sqrtf(sq + 1e-6f) : 1.0f) * p.scale;
    const float fk = p.l2 ? 1.0f / sqrtf(sk + 1e-6f) : 1.0f;
#pragma unroll
    for (int e = 0; e < 16; e += 4) {
        *(f32x4*)&Q[i * RS + d0 + e] = (f32x4){qv[e] * fq, qv[e + 1] * fq, qv[e + 2] * fq, qv[e + 3] * fq};
        *(f32x4*)&K[i * RS + d0 + e] = (f32x4){kv[e] * fk, kv[e + 1] * fk, kv[e + 2] * fk, kv[e + 3] * fk};
        if (V) *(f32x4*)&V[i * RS + d0 + e] = (f32x4){vv[e], vv[e + 1], vv[e + 2], vv[e + 3]};
    }
}

// ----------------------------------------------------------------------------
// prep: per (chunk, v head) A, T, U, W, G
// ----------------------------------------------------------------------------
struct PrepLds {
    float Q[GC * RS];
    float K[GC * RS];
    float V[GC * RS];
    float A[GC * MS];
    float N[GC * MS];     // N = -strictly_lower(beta k^ k^T * D), then its powers N^(2^r)
    float Tm[GC * MS];    // T = (I - N)^-1, built as (I + N)(I + N^2)(I + N^4)...
    float G[GC];
    float beta[GC];
};

template <typename TIn>
__global__ __launch_bounds__(GT) void gdn_prep_kernel(GdnDev p, float* __restrict__ ws) {
    __shared__ __attribute__((aligned(16))) PrepLds L;
    const int c = blockIdx.x, h = blockIdx.y;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    int start, len;
    if (!chunk_span(p, c, start, len)) return;
    float* out = ws + ((size_t)c * p.hv + h) * kWsChunk;

    load_chunk_rows<TIn>(p, start, len, h, L.Q, L.K, L.V);
    if (wave == 0) {
        // cumulative decay over the chunk (lanes 0..31; padded rows add 0)
        const bool valid = lane < len;
        const int64_t tok = start + lane;
        float gv = valid ? p.g[tok * p.g_st + h] : 0.0f;
        const float bv = valid ? p.beta[tok * p.b_st + h] : 0.0f;
#pragma unroll
        for (int o = 1; o < GC; o <<= 1) {
            const float up = __shfl_up(gv, o, GC);
            if ((lane & (GC - 1)) >= o) gv += up;
        }
        if (lane < GC) {
            L.G[lane] = gv;
            L.beta[lane] = bv;
            out[kWsG + lane] = gv;
        }
    }
    __syncthreads();

    // A = lower_incl(q^ k^T * D), N = -strictly_lower(beta k^ k^T * D).
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int pi = t + GT * u, i = pi >> 5, j = pi & 31;
        float dqk = 0.0f, dkk = 0.0f;
#pragma unroll 2
        for (int d = 0; d < GD; d += 4) {
            const f32x4 qi = *(const f32x4*)&L.Q[i * RS + d];
            const f32x4 ki = *(const f32x4*)&L.K[i * RS + d];
            const f32x4 kj = *(const f32x4*)&L.K[j * RS + d];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                dqk = fmaf(qi[e], kj[e], dqk);
                dkk = fmaf(ki[e], kj[e], dkk);
            }
        }
        const float dec = j <= i ? expf(L.G[i] - L.G[j]) : 0.0f;
        const float nij = j < i ? -L.beta[i] * dkk * dec : 0.0f;
        L.A[i * MS + j] = dqk * dec;
        out[kWsA + i * GC + j] = dqk * dec;
        L.N[i * MS + j] = nij;
        L.Tm[i * MS + j] = nij + (i == j ? 1.0f : 0.0f);
    }
    __syncthreads();

    // T = (I - N)^-1. N is strictly lower triangular (N^32 = 0), so
    // (I - N)^-1 = (I + N)(I + N^2)(I + N^4)(I + N^8)(I + N^16): starting from
    // T = I + N, P = N, four rounds of P <- P P, then T <- T + T P. Thread t
    // owns row t/8, columns 4*(t%8)..+3 of each product.
    {
        const int ti = t >> 3, tc = 4 * (t & 7);
        for (int r = 0; r < 4; ++r) {
            f32x4 pp = {};
#pragma unroll 4
            for (int m = 0; m < GC; ++m) {
                const f32x4 pm = *(const f32x4*)&L.N[m * MS + tc];
                const float pim = L.N[ti * MS + m];
#pragma unroll
                for (int e = 0; e < 4; ++e) pp[e] = fmaf(pim, pm[e], pp[e]);
            }
            __syncthreads();
            *(f32x4*)&L.N[ti * MS + tc] = pp;
            __syncthreads();
            f32x4 tp = {};
#pragma unroll 4
            for (int m = 0; m < GC; ++m) {
                const f32x4 pm = *(const f32x4*)&L.N[m * MS + tc];
                const float tim = L.Tm[ti * MS + m];
#pragma unroll
                for (int e = 0; e < 4; ++e) tp[e] = fmaf(tim, pm[e], tp[e]);
            }
            __syncthreads();
            *(f32x4*)&L.Tm[ti * MS + tc] += tp;
            __syncthreads();
        }
    }

    // U = T (beta v), W = T (beta e^G k^): thread t owns rows oi0..+3, columns oc0..+3.
    const int oi0 = 4 * (t >> 5), oc0 = 4 * (t & 31);
    f32x4 u[4], w[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) u[a] = w[a] = (f32x4){};
#pragma unroll 1
    for (int j0 = 0; j0 < GC; j0 += 4) {
        f32x4 tr[4];
#pragma unroll
        for (int a = 0; a < 4; ++a) tr[a] = *(const f32x4*)&L.Tm[(oi0 + a) * MS + j0];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int j = j0 + jj;
            const float bj = L.beta[j], bgj = bj * expf(L.G[j]);
            const f32x4 vj = *(const f32x4*)&L.V[j * RS + oc0];
            const f32x4 kj = *(const f32x4*)&L.K[j * RS + oc0];
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const float ta = tr[a][jj];
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    u[a][b] = fmaf(ta * bj, vj[b], u[a][b]);
                    w[a][b] = fmaf(ta * bgj, kj[b], w[a][b]);
                }
            }
        }
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        *(f32x4*)(out + kWsW + (oi0 + a) * GD + oc0) = w[a];
        *(f32x4*)(out + kWsU + (oi0 + a) * GD + oc0) = u[a];
    }
}

// ----------------------------------------------------------------------------
// scan: per (node, v head, value slice), the node's chunks in order
// ----------------------------------------------------------------------------
struct ScanLds {
    float S[GD * VP];     // state slice [Dk][VS]
    float Q[GC * RS];     // q^ * scale
    float K[GC * RS];     // k^
    float W[GC * RS];
    float Vp[GC * VP];    // V' slice
    float A[GC * MS];
    float G[GC];
};

template <typename TIn>
__global__ __launch_bounds__(GT) void gdn_scan_kernel(GdnDev p, int lvl_begin, const float* __restrict__ ws,
                                                      TIn* __restrict__ out, float* __restrict__ states) {
    __shared__ __attribute__((aligned(16))) ScanLds L;
    const int node = p.level_nodes[lvl_begin + blockIdx.x];
    if (node < 0 || node >= p.n_nodes) return;
    const int h = blockIdx.y, col0 = VS * blockIdx.z;
    const int t = threadIdx.x;
    const int start = p.node_start[node], len = p.node_len[node], chunk0 = p.node_chunk0[node];
    int par = p.parent[node];
    if (start < 0 || len < 0 || start > p.n_tokens - len) return;        // malformed node: skipped
    if (chunk0 < 0 || chunk0 > p.n_chunks - tt_cdiv(len, GC)) return;
    if (par >= node || par < -1) par = -1;                               // parents precede children

    // State slice: thread t owns rows sr0..sr0+3, columns sc..sc+3 (of the slice).
    const int sr0 = 4 * (t >> 3), sc = 4 * (t & 7);
    {
        const float* src = par >= 0 ? states + ((size_t)par * p.hv + h) * GD * GD : nullptr;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            f32x4 a = {};
            if (src) a = *(const f32x4*)(src + (sr0 + r) * GD + col0 + sc);
            *(f32x4*)&L.S[(sr0 + r) * VP + sc] = a;
        }
    }
    // [GC x VS] outputs: thread t owns row oi, columns oc..oc+3.
    const int oi = t >> 3, oc = 4 * (t & 7);

    for (int c0 = 0; c0 < len; c0 += GC) {
        const int Lc = min(GC, len - c0);
        const float* cw = ws + ((size_t)(chunk0 + c0 / GC) * p.hv + h) * kWsChunk;
        __syncthreads();   // readers of the previous chunk's tiles are done
        load_chunk_rows<TIn>(p, start + c0, Lc, h, L.Q, L.K, nullptr);
        {
            const int i = t >> 3, d0 = 16 * (t & 7);
#pragma unroll
            for (int e = 0; e < 16; e += 4)
                *(f32x4*)&L.W[i * RS + d0 + e] = *(const f32x4*)(cw + kWsW + i * GD + d0 + e);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int pi = t + GT * e;
                L.A[(pi >> 5) * MS + (pi & 31)] = cw[kWsA + pi];
            }
            if (t < GC) L.G[t] = cw[kWsG + t];
        }
        const f32x4 u = *(const f32x4*)(cw + kWsU + oi * GD + col0 + oc);
        __syncthreads();

        // V' = U - W S and q^ S (both contract over the 128 state rows).
        f32x4 vp = u, qs = {};
#pragma unroll 2
        for (int r0 = 0; r0 < GD; r0 += 4) {
            const f32x4 wr = *(const f32x4*)&L.W[oi * RS + r0];
            const f32x4 qr = *(const f32x4*)&L.Q[oi * RS + r0];
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const f32x4 s = *(const f32x4*)&L.S[(r0 + rr) * VP + oc];
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    vp[b] = fmaf(-wr[rr], s[b], vp[b]);
                    qs[b] = fmaf(qr[rr], s[b], qs[b]);
                }
            }
        }
        *(f32x4*)&L.Vp[oi * VP + oc] = vp;
        __syncthreads();   // V' complete; every reader of S for this chunk is done

        // O = e^G (q^ S) + A V'.
        {
            f32x4 o = qs * expf(L.G[oi]);
#pragma unroll 2
            for (int j0 = 0; j0 < GC; j0 += 4) {
                const f32x4 ar = *(const f32x4*)&L.A[oi * MS + j0];
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const f32x4 v = *(const f32x4*)&L.Vp[(j0 + jj) * VP + oc];
#pragma unroll
                    for (int b = 0; b < 4; ++b) o[b] = fmaf(ar[jj], v[b], o[b]);
                }
            }
            if (oi < Lc) store4(out + ((int64_t)(start + c0 + oi) * p.hv + h) * GD + col0 + oc, o);
        }
        // S <- e^{G_last} S + (k^ e^{G_last - G})^T V'.
        {
            const float gl = L.G[GC - 1], el = expf(gl);
            f32x4 s[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) s[r] = *(const f32x4*)&L.S[(sr0 + r) * VP + sc] * el;
#pragma unroll 4
            for (int i = 0; i < GC; ++i) {
                const float kd = expf(gl - L.G[i]);
                const f32x4 kr = *(const f32x4*)&L.K[i * RS + sr0] * kd;
                const f32x4 v = *(const f32x4*)&L.Vp[i * VP + sc];
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int b = 0; b < 4; ++b) s[r][b] = fmaf(kr[r], v[b], s[r][b]);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) *(f32x4*)&L.S[(sr0 + r) * VP + sc] = s[r];
        }
    }
    __syncthreads();

    // Final state of the node (the initial state of its children).
    float* dst = states + ((size_t)node * p.hv + h) * GD * GD;
#pragma unroll
    for (int r = 0; r < 4; ++r)
        *(f32x4*)(dst + (sr0 + r) * GD + col0 + sc) = *(const f32x4*)&L.S[(sr0 + r) * VP + sc];
}

}  // namespace

size_t tt_gdn_ws_bytes_impl(int n_chunks, int n_heads_v) {
    return (size_t)n_chunks * (size_t)n_heads_v * kWsChunk * sizeof(float);
}

int tt_gdn_fwd_launch(const GdnDev& d, const int32_t* level_offsets, int n_levels, void* out, float* states,
                      float* ws, hipStream_t s) {
    if (d.dtype == TT_DTYPE_BF16)
        hipLaunchKernelGGL(gdn_prep_kernel<__bf16>, dim3(d.n_chunks, d.hv), dim3(GT), 0, s, d, ws);
    else
        hipLaunchKernelGGL(gdn_prep_kernel<float>, dim3(d.n_chunks, d.hv), dim3(GT), 0, s, d, ws);
    if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    for (int l = 0; l < n_levels; ++l) {
        const int b = level_offsets[l], n = level_offsets[l + 1] - b;
        if (n <= 0) continue;
        if (d.dtype == TT_DTYPE_BF16)
            hipLaunchKernelGGL(gdn_scan_kernel<__bf16>, dim3(n, d.hv, NSL), dim3(GT), 0, s, d, b, ws,
                               (__bf16*)out, states);
        else
            hipLaunchKernelGGL(gdn_scan_kernel<float>, dim3(n, d.hv, NSL), dim3(GT), 0, s, d, b, ws,
                               (float*)out, states);
        if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    }
    return TT_OK;
}
