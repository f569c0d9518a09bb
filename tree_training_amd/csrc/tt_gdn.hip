// Tree gated delta rule (the linear-attention layers of Qwen3.5-style models)
// over a DFS-packed tree: forward scan for gfx950.
//
// Semantics: the gated delta rule token by token along every root-to-leaf
// path — each node continues from its parent's final state (zero state for a
// root) — evaluated exactly in 32-token chunks:
//   G = cumsum(g), D[i][j] = exp(G_i - G_j) (j <= i),
//   N = -strictly_lower(beta k k^T * D),  T = (I - N)^-1,
//   U = T (beta v),  W = T (beta e^G k),  V' = U - W S,
//   O = e^G (q S) + lower_incl(q k^T * D) V',
//   S <- e^{G_last} S + (k e^{G_last - G})^T V'.
// q and k are l2-normalised in the kernel and q is scaled; v head h reads q/k
// head h / (Hv / Hk).
//
// Parallelism: one workgroup per (node, v head); nodes are processed one tree
// level per launch, so a node's parent state (written to the caller's
// node_states buffer by the previous launch) is complete when it starts.
// Within a workgroup the 128x128 fp32 state lives in LDS; every product is
// fp32 FMA on the vector ALUs (fp32 end to end, like the reference).
#include "tt_common.h"
#include "tt_internal.h"

namespace {

constexpr int GD = 128;           // head dim (Dk = Dv)
constexpr int GC = 32;            // chunk length
constexpr int GT = 256;           // threads per workgroup
constexpr int RS = GD + 4;        // row stride of the chunk tiles (floats): rows 4 banks apart
constexpr int MS = GC + 4;        // row stride of the chunk x chunk matrices

struct GdnLds {
    float S[GD * GD];     // running state [Dk][Dv]
    float Q[GC * RS];     // q^ * scale
    float K[GC * RS];     // k^
    float V[GC * RS];     // v, then V' = U - W S
    float W[GC * RS];     // T (beta e^G k^)
    float A[GC * MS];     // lower_incl(q^ k^T * D)
    float N[GC * MS];     // N = -strictly_lower(beta k^ k^T * D), then its powers N^(2^r)
    float Tm[GC * MS];    // T = (I - N)^-1, built as (I + N)(I + N^2)(I + N^4)...
    float G[GC];          // cumulative log decay within the chunk
    float beta[GC];
};

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
__device__ __forceinline__ void store4(T* p, const float (&x)[4]) {
    if constexpr (sizeof(T) == 2) {
        bf16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = (__bf16)x[e];
        *(bf16x4*)p = w;
    } else {
        *(f32x4*)p = (f32x4){x[0], x[1], x[2], x[3]};
    }
}

// Sum over the 8 consecutive lanes that hold one row.
__device__ __forceinline__ float row8_sum(float x) {
    x += __shfl_xor(x, 1);
    x += __shfl_xor(x, 2);
    x += __shfl_xor(x, 4);
    return x;
}

template <typename TIn>
__global__ __launch_bounds__(GT) void gdn_fwd_level_kernel(GdnDev p, int lvl_begin, TIn* __restrict__ out,
                                                           float* __restrict__ states) {
    __shared__ __attribute__((aligned(16))) GdnLds L;
    const int node = p.level_nodes[lvl_begin + blockIdx.x];
    if (node < 0 || node >= p.n_nodes) return;
    const int h = blockIdx.y, hk = h / p.rep;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int start = p.node_start[node], len = p.node_len[node];
    int par = p.parent[node];
    if (start < 0 || len < 0 || start > p.n_tokens - len) return;   // malformed node: skipped
    if (par >= node || par < -1) par = -1;                          // parents precede children

    // State ownership for load/store and the state update: thread t holds
    // rows sr0..sr0+7, columns sc0..sc0+7.
    const int sr0 = 8 * (t >> 4), sc0 = 8 * (t & 15);
    {
        const float* src = par >= 0 ? states + ((size_t)par * p.hv + h) * GD * GD : nullptr;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            f32x4 a = {}, b = {};
            if (src) {
                a = *(const f32x4*)(src + (sr0 + r) * GD + sc0);
                b = *(const f32x4*)(src + (sr0 + r) * GD + sc0 + 4);
            }
            *(f32x4*)&L.S[(sr0 + r) * GD + sc0] = a;
            *(f32x4*)&L.S[(sr0 + r) * GD + sc0 + 4] = b;
        }
    }
    // Output blocks of the [GC x GD] products: rows oi0..oi0+3, columns oc0..oc0+3.
    const int oi0 = 4 * (t >> 5), oc0 = 4 * (t & 31);

    for (int c0 = 0; c0 < len; c0 += GC) {
        const int Lc = min(GC, len - c0);
        __syncthreads();   // readers of the previous chunk's tiles and state are done

        // 1. Chunk rows (zeros past the node end): l2-normalised q (scaled), k; v; g; beta.
        {
            const int i = t >> 3, d0 = 16 * (t & 7);
            const bool valid = i < Lc;
            const int64_t tok = start + c0 + i;
            float qv[16], kv[16], vv[16];
            if (valid) {
                load16((const TIn*)p.q + tok * p.q_st + hk * p.q_sh + d0, qv);
                load16((const TIn*)p.k + tok * p.k_st + hk * p.k_sh + d0, kv);
                load16((const TIn*)p.v + tok * p.v_st + h * p.v_sh + d0, vv);
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
                *(f32x4*)&L.Q[i * RS + d0 + e] = (f32x4){qv[e] * fq, qv[e + 1] * fq, qv[e + 2] * fq, qv[e + 3] * fq};
                *(f32x4*)&L.K[i * RS + d0 + e] = (f32x4){kv[e] * fk, kv[e + 1] * fk, kv[e + 2] * fk, kv[e + 3] * fk};
                *(f32x4*)&L.V[i * RS + d0 + e] = (f32x4){vv[e], vv[e + 1], vv[e + 2], vv[e + 3]};
            }
        }
        if (wave == 0) {
            // cumulative decay over the chunk (lanes 0..31; padded rows add 0)
            const bool valid = lane < Lc;
            const int64_t tok = start + c0 + lane;
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
            }
        }
        __syncthreads();

        // 2. A = lower_incl(q^ k^T * D), N = -strictly_lower(beta k^ k^T * D).
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
            L.N[i * MS + j] = nij;
            L.Tm[i * MS + j] = nij + (i == j ? 1.0f : 0.0f);
        }
        __syncthreads();

        // 3. T = (I - N)^-1. N is strictly lower triangular (N^32 = 0), so
        // (I - N)^-1 = (I + N)(I + N^2)(I + N^4)(I + N^8)(I + N^16): starting
        // from T = I + N, P = N, four rounds of P <- P P, then T <- T + T P.
        // Thread t owns row t/8, columns 4*(t%8)..+3 of each product.
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

        // 4. U = T (beta v) (kept in registers), W = T (beta e^G k^).
        float u[4][4], w[4][4];
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b) u[a][b] = w[a][b] = 0.0f;
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
        for (int a = 0; a < 4; ++a) *(f32x4*)&L.W[(oi0 + a) * RS + oc0] = (f32x4){w[a][0], w[a][1], w[a][2], w[a][3]};
        __syncthreads();

        // 5. V' = U - W S (into V: its last readers passed the barrier).
#pragma unroll 1
        for (int r0 = 0; r0 < GD; r0 += 4) {
            f32x4 wr[4], s[4];
#pragma unroll
            for (int a = 0; a < 4; ++a) wr[a] = *(const f32x4*)&L.W[(oi0 + a) * RS + r0];
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) s[rr] = *(const f32x4*)&L.S[(r0 + rr) * GD + oc0];
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
#pragma unroll
                    for (int b = 0; b < 4; ++b) u[a][b] = fmaf(-wr[a][rr], s[rr][b], u[a][b]);
        }
#pragma unroll
        for (int a = 0; a < 4; ++a) *(f32x4*)&L.V[(oi0 + a) * RS + oc0] = (f32x4){u[a][0], u[a][1], u[a][2], u[a][3]};
        __syncthreads();

        // 6. O = e^G (q^ S) + A V'.
        {
            float o[4][4];
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b) o[a][b] = 0.0f;
#pragma unroll 1
            for (int r0 = 0; r0 < GD; r0 += 4) {
                f32x4 qr[4], s[4];
#pragma unroll
                for (int a = 0; a < 4; ++a) qr[a] = *(const f32x4*)&L.Q[(oi0 + a) * RS + r0];
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) s[rr] = *(const f32x4*)&L.S[(r0 + rr) * GD + oc0];
#pragma unroll
                for (int a = 0; a < 4; ++a)
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr)
#pragma unroll
                        for (int b = 0; b < 4; ++b) o[a][b] = fmaf(qr[a][rr], s[rr][b], o[a][b]);
            }
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const float eg = expf(L.G[oi0 + a]);
#pragma unroll
                for (int b = 0; b < 4; ++b) o[a][b] *= eg;
            }
#pragma unroll 1
            for (int j0 = 0; j0 < GC; j0 += 4) {
                f32x4 ar[4], vp[4];
#pragma unroll
                for (int a = 0; a < 4; ++a) ar[a] = *(const f32x4*)&L.A[(oi0 + a) * MS + j0];
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) vp[jj] = *(const f32x4*)&L.V[(j0 + jj) * RS + oc0];
#pragma unroll
                for (int a = 0; a < 4; ++a)
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
                        for (int b = 0; b < 4; ++b) o[a][b] = fmaf(ar[a][jj], vp[jj][b], o[a][b]);
            }
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                if (oi0 + a < Lc) {
                    const int64_t tok = start + c0 + oi0 + a;
                    store4(out + (tok * p.hv + h) * GD + oc0, o[a]);
                }
            }
        }
        __syncthreads();   // every reader of S for this chunk is done

        // 7. S <- e^{G_last} S + (k^ e^{G_last - G})^T V'.
        {
            const float gl = L.G[GC - 1], el = expf(gl);
            float s[8][8];
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const f32x4 a = *(const f32x4*)&L.S[(sr0 + r) * GD + sc0];
                const f32x4 b = *(const f32x4*)&L.S[(sr0 + r) * GD + sc0 + 4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    s[r][e] = a[e] * el;
                    s[r][4 + e] = b[e] * el;
                }
            }
#pragma unroll 1
            for (int i = 0; i < GC; ++i) {
                const float kd = expf(gl - L.G[i]);
                const f32x4 k0 = *(const f32x4*)&L.K[i * RS + sr0], k1 = *(const f32x4*)&L.K[i * RS + sr0 + 4];
                const f32x4 v0 = *(const f32x4*)&L.V[i * RS + sc0], v1 = *(const f32x4*)&L.V[i * RS + sc0 + 4];
                const float kr[8] = {k0[0] * kd, k0[1] * kd, k0[2] * kd, k0[3] * kd,
                                     k1[0] * kd, k1[1] * kd, k1[2] * kd, k1[3] * kd};
                const float vc[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
#pragma unroll
                for (int r = 0; r < 8; ++r)
#pragma unroll
                    for (int c = 0; c < 8; ++c) s[r][c] = fmaf(kr[r], vc[c], s[r][c]);
            }
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                *(f32x4*)&L.S[(sr0 + r) * GD + sc0] = (f32x4){s[r][0], s[r][1], s[r][2], s[r][3]};
                *(f32x4*)&L.S[(sr0 + r) * GD + sc0 + 4] = (f32x4){s[r][4], s[r][5], s[r][6], s[r][7]};
            }
        }
    }
    __syncthreads();

    // Final state of the node (the initial state of its children).
    float* dst = states + ((size_t)node * p.hv + h) * GD * GD;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        *(f32x4*)(dst + (sr0 + r) * GD + sc0) = *(const f32x4*)&L.S[(sr0 + r) * GD + sc0];
        *(f32x4*)(dst + (sr0 + r) * GD + sc0 + 4) = *(const f32x4*)&L.S[(sr0 + r) * GD + sc0 + 4];
    }
}

}  // namespace

int tt_gdn_fwd_launch(const GdnDev& d, const int32_t* level_offsets, int n_levels, void* out, float* states,
                      hipStream_t s) {
    for (int l = 0; l < n_levels; ++l) {
        const int b = level_offsets[l], n = level_offsets[l + 1] - b;
        if (n <= 0) continue;
        if (d.dtype == TT_DTYPE_BF16)
            hipLaunchKernelGGL(gdn_fwd_level_kernel<__bf16>, dim3(n, d.hv), dim3(GT), 0, s, d, b, (__bf16*)out,
                               states);
        else
            hipLaunchKernelGGL(gdn_fwd_level_kernel<float>, dim3(n, d.hv), dim3(GT), 0, s, d, b, (float*)out,
                               states);
        if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    }
    return TT_OK;
}
