// Tree-correct depthwise causal conv + SiLU (the short convolution in front
// of the gated-delta-rule layers) over a DFS-packed tree, forward and backward
// for gfx950.
//
// Every token t has a path predecessor prev[t]: t - 1 inside its node, the
// last token of the parent node for a node's first token, -1 before a root.
// The conv window of t is x[prev^(K-1)(t)], ..., x[prev(t)], x[t] (missing
// entries are zero), so each node sees its ancestors' last K-1 inputs exactly
// as a run of its root-to-node path alone would:
//   y[t][c] = silu(bias[c] + sum_i w[c][i] x[prev^(K-1-i)(t)][c]).
// The backward gathers over the token successor lists (the inverse of prev):
//   dx[u][c] = sum_m w[c][K-1-m] sum_{t : prev^m(t) = u} gp[t][c],
//   gp = dy * silu'(pre),  dw[c][i] = sum_t gp[t][c] x[prev^(K-1-i)(t)][c].
// Layout: token-major rows of C channels; each thread owns 4 channels and
// walks a run of tokens (the predecessor chain is uniform over the workgroup).
// Memory-bound; fp32 arithmetic.
#include "tt_common.h"
#include "tt_internal.h"

namespace {

constexpr int CT = 256;              // threads per workgroup
constexpr int CCH = 4 * CT;          // channels per workgroup
constexpr int CTOK = 64;             // tokens per workgroup (forward, dx)
constexpr int CTOK_W = 128;          // tokens per workgroup (gp + weight-gradient partials)

template <typename T>
__device__ __forceinline__ f32x4 ld4(const T* p) {
    if constexpr (sizeof(T) == 2) {
        const bf16x4 a = *(const bf16x4*)p;
        return (f32x4){(float)a[0], (float)a[1], (float)a[2], (float)a[3]};
    } else {
        return *(const f32x4*)p;
    }
}

template <typename T>
__device__ __forceinline__ void st4(T* p, const f32x4& x) {
    if constexpr (sizeof(T) == 2) {
        bf16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = (__bf16)x[e];
        *(bf16x4*)p = w;
    } else {
        *(f32x4*)p = x;
    }
}

// sigmoid(z) = 1 / (1 + 2^(-z log2 e)) on the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32: about 1 ulp each).
__device__ __forceinline__ float sigmoid_fast(float z) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z * TT_LOG2E));
}

__device__ __forceinline__ int prev_of(const ConvDev& p, int t) {
    if (t < 0) return -1;
    const int u = p.prev[t];
    return (u >= 0 && u < p.n_tokens) ? u : -1;
}

// Window of token t: idx[i] = prev^(K-1-i)(t) (or -1).
template <int K>
__device__ __forceinline__ void window(const ConvDev& p, int t, int (&idx)[K]) {
    idx[K - 1] = t;
#pragma unroll
    for (int i = K - 2; i >= 0; --i) idx[i] = prev_of(p, idx[i + 1]);
}

template <int K, typename T>
__device__ __forceinline__ void load_taps(const ConvDev& p, int c, float (&w)[4][K], float (&b)[4]) {
    const T* wt = (const T*)p.weight;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int i = 0; i < K; ++i) w[e][i] = (float)wt[(int64_t)(c + e) * K + i];
        b[e] = p.bias ? (float)((const T*)p.bias)[c + e] : 0.0f;
    }
}

// The window of consecutive tokens: when prev(t) is the previous token of the
// run (inside a node), t's window is the last one shifted by a row, so only
// x[t] is new; otherwise (a node's first token, the run's first) the rows
// before it are gathered along the predecessor chain. The test is uniform over
// the workgroup (every thread walks the same tokens). x[t] itself is passed
// in: the callers load it one token ahead, so that a wave keeps the next
// token's rows in flight while it computes the current one.
template <int K, typename T>
struct SlidingWindow {
    int idx[K];
    f32x4 xv[K];
    int last = -1;
    __device__ __forceinline__ void advance(const ConvDev& p, int c, int t, const f32x4& xt) {
        if (last >= 0 && prev_of(p, t) == last) {
#pragma unroll
            for (int i = 0; i < K - 1; ++i) {
                idx[i] = idx[i + 1];
                xv[i] = xv[i + 1];
            }
            idx[K - 1] = t;
        } else {
            window<K>(p, t, idx);
#pragma unroll
            for (int i = 0; i < K - 1; ++i)
                xv[i] = idx[i] >= 0 ? ld4((const T*)p.x + (int64_t)idx[i] * p.x_st + c) : (f32x4){};
        }
        xv[K - 1] = xt;
        last = t;
    }
    __device__ __forceinline__ f32x4 preact(const float (&w)[4][K], const float (&b)[4]) const {
        f32x4 acc = {b[0], b[1], b[2], b[3]};
#pragma unroll
        for (int i = 0; i < K; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = fmaf(w[e][i], xv[i][e], acc[e]);
        return acc;
    }
};

template <int K, typename T>
__global__ __launch_bounds__(CT) void conv_fwd_kernel(ConvDev p, T* __restrict__ y, int64_t y_st) {
    const int c = 4 * (blockIdx.y * CT + threadIdx.x);
    if (c >= p.n_ch) return;
    float w[4][K], b[4];
    load_taps<K, T>(p, c, w, b);
    const int t0 = blockIdx.x * CTOK, t1 = min(p.n_tokens, t0 + CTOK);
    const T* xc = (const T*)p.x + c;
    SlidingWindow<K, T> win;
    f32x4 xn = ld4(xc + (int64_t)t0 * p.x_st);    // t0 < n_tokens: the grid covers the tokens
    for (int t = t0; t < t1; ++t) {
        const f32x4 xt = xn;
        if (t + 1 < t1) xn = ld4(xc + (int64_t)(t + 1) * p.x_st);
        win.advance(p, c, t, xt);
        const f32x4 z = win.preact(w, b);
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = z[e] * sigmoid_fast(z[e]);
        st4(y + (int64_t)t * y_st + c, o);
    }
}

// gp = dy * silu'(pre) into the workspace (in the problem's dtype, as the
// reference's bf16 autograd keeps this gradient), and per-workgroup partial sums of
// dw (taps 0..K-1) and db (slot K): part[blockIdx.x][slot][c].
template <int K, typename T>
__global__ __launch_bounds__(CT) void conv_bwd_gp_kernel(ConvDev p, const T* __restrict__ dy, int64_t dy_st,
                                                         T* __restrict__ gp, float* __restrict__ part) {
    const int c = 4 * (blockIdx.y * CT + threadIdx.x);
    if (c >= p.n_ch) return;
    float w[4][K], b[4];
    load_taps<K, T>(p, c, w, b);
    f32x4 aw[K], ab = {};
#pragma unroll
    for (int i = 0; i < K; ++i) aw[i] = (f32x4){};
    const int t0 = blockIdx.x * CTOK_W, t1 = min(p.n_tokens, t0 + CTOK_W);
    const T* xc = (const T*)p.x + c;
    SlidingWindow<K, T> win;
    f32x4 xn = ld4(xc + (int64_t)t0 * p.x_st);    // t0 < n_tokens: the grid covers the tokens
    f32x4 dn = ld4(dy + (int64_t)t0 * dy_st + c);
    for (int t = t0; t < t1; ++t) {
        const f32x4 xt = xn, d = dn;
        if (t + 1 < t1) {
            xn = ld4(xc + (int64_t)(t + 1) * p.x_st);
            dn = ld4(dy + (int64_t)(t + 1) * dy_st + c);
        }
        win.advance(p, c, t, xt);
        const f32x4 z = win.preact(w, b);
        const f32x4* xv = win.xv;
        f32x4 g;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float s = sigmoid_fast(z[e]);
            g[e] = d[e] * s * fmaf(z[e], 1.0f - s, 1.0f);
        }
        st4(gp + (int64_t)t * p.n_ch + c, g);
        ab += g;
#pragma unroll
        for (int i = 0; i < K; ++i) aw[i] += g * xv[i];
    }
    float* pb = part + (size_t)blockIdx.x * (K + 1) * p.n_ch + c;
#pragma unroll
    for (int i = 0; i < K; ++i) *(f32x4*)(pb + (size_t)i * p.n_ch) = aw[i];
    *(f32x4*)(pb + (size_t)K * p.n_ch) = ab;
}

// dx[u] = sum over m < K of w[K-1-m] * (sum of gp over the tokens m steps
// after u). With D_m(u) that sum (D_0(u) = gp[u]), D_m(u) = D_{m-1}(u + 1) when
// u's one successor is u + 1 (inside a node), so the workgroup walks its tokens
// from the last down and, for such a token, shifts the sums of the token after
// it: one new gp row per token, loaded one token ahead. Other tokens (a node's
// last, the range's last) walk their successor lists. Either way every sum is
// taken in the order of the successor lists, so the results do not depend on
// the walk.
template <int K, typename T>
__global__ __launch_bounds__(CT) void conv_bwd_dx_kernel(ConvDev p, const T* __restrict__ gp,
                                                         T* __restrict__ dx) {
    const int c = 4 * (blockIdx.y * CT + threadIdx.x);
    if (c >= p.n_ch) return;
    float w[4][K], b[4];
    load_taps<K, T>(p, c, w, b);
    const int u0 = blockIdx.x * CTOK, u1 = min(p.n_tokens, u0 + CTOK);
    auto g_at = [&](int t) { return ld4(gp + (int64_t)t * p.n_ch + c); };
    auto succ = [&](int t, int& lo, int& hi) {
        lo = max(p.next_off[t], 0);
        hi = min(p.next_off[t + 1], p.n_tokens);
    };
    f32x4 s[K];                       // D_m of the token after u (once `have`)
    bool have = false;
    f32x4 gn = g_at(u1 - 1);          // u0 < u1: the grid covers the tokens
    for (int u = u1 - 1; u >= u0; --u) {
        const f32x4 gu = gn;
        if (u > u0) gn = g_at(u - 1);
        int lo1, hi1;
        succ(u, lo1, hi1);
        if (have && hi1 - lo1 == 1 && p.next[lo1] == u + 1) {
#pragma unroll
            for (int m = K - 1; m >= 1; --m) s[m] = s[m - 1];
            s[0] = gu;
        } else {
#pragma unroll
            for (int m = 0; m < K; ++m) s[m] = (f32x4){};
            s[0] = gu;
            if constexpr (K > 1) {
                for (int a = lo1; a < hi1; ++a) {
                    const int ta = p.next[a];
                    if (ta < 0 || ta >= p.n_tokens) continue;
                    s[1] += g_at(ta);
                    if constexpr (K > 2) {
                        int lo2, hi2;
                        succ(ta, lo2, hi2);
                        for (int bb = lo2; bb < hi2; ++bb) {
                            const int tb = p.next[bb];
                            if (tb < 0 || tb >= p.n_tokens) continue;
                            s[2] += g_at(tb);
                            if constexpr (K > 3) {
                                int lo3, hi3;
                                succ(tb, lo3, hi3);
                                for (int cc = lo3; cc < hi3; ++cc) {
                                    const int tc = p.next[cc];
                                    if (tc < 0 || tc >= p.n_tokens) continue;
                                    s[3] += g_at(tc);
                                }
                            }
                        }
                    }
                }
            }
        }
        have = true;
        f32x4 o = {};
#pragma unroll
        for (int m = 0; m < K; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = fmaf(w[e][K - 1 - m], s[m][e], o[e]);
        st4(dx + (int64_t)u * p.n_ch + c, o);
    }
}

// dw[c][i] and db[c] from the per-workgroup partials (fixed order: deterministic).
// Sum of the per-workgroup partials: a workgroup takes RJ consecutive
// (slot, channel) entries, its CT / RJ thread groups every (CT / RJ)-th partial
// (in a fixed order: deterministic), summed through LDS.
constexpr int RJ = 64;
__global__ __launch_bounds__(CT) void conv_bwd_reduce_kernel(const float* __restrict__ part, int n_parts, int n_ch,
                                                             int K, float* __restrict__ dw, float* __restrict__ db) {
    __shared__ float red[CT];
    const int total = (K + 1) * n_ch;
    const int j = blockIdx.x * RJ + (threadIdx.x % RJ), grp = threadIdx.x / RJ;
    float s = 0.0f;
    if (j < total) {
#pragma unroll 8
        for (int b = grp; b < n_parts; b += CT / RJ) s += part[(size_t)b * total + j];
    }
    red[threadIdx.x] = s;
    __syncthreads();
    if (grp != 0 || j >= total) return;
#pragma unroll
    for (int g2 = 1; g2 < CT / RJ; ++g2) s += red[threadIdx.x + g2 * RJ];
    const int slot = j / n_ch, c = j - slot * n_ch;
    if (slot < K) dw[(size_t)c * K + slot] = s;
    else if (db) db[c] = s;
}

template <int K, typename T>
int conv_fwd_run(const ConvDev& d, void* y, int64_t y_st, hipStream_t s) {
    const dim3 grid(tt_cdiv(d.n_tokens, CTOK), tt_cdiv(d.n_ch, CCH));
    hipLaunchKernelGGL((conv_fwd_kernel<K, T>), grid, dim3(CT), 0, s, d, (T*)y, y_st);
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}

template <int K, typename T>
int conv_bwd_run(const ConvDev& d, const void* dy, int64_t dy_st, void* dx, float* dw, float* db, float* ws,
                 hipStream_t s) {
    const int n_parts = tt_cdiv(d.n_tokens, CTOK_W);
    T* gp = reinterpret_cast<T*>(ws);
    float* part = ws + (size_t)d.n_tokens * d.n_ch;
    hipLaunchKernelGGL((conv_bwd_gp_kernel<K, T>), dim3(n_parts, tt_cdiv(d.n_ch, CCH)), dim3(CT), 0, s, d,
                       (const T*)dy, dy_st, gp, part);
    if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    hipLaunchKernelGGL((conv_bwd_dx_kernel<K, T>), dim3(tt_cdiv(d.n_tokens, CTOK), tt_cdiv(d.n_ch, CCH)), dim3(CT),
                       0, s, d, (const T*)gp, (T*)dx);
    if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    hipLaunchKernelGGL(conv_bwd_reduce_kernel, dim3(tt_cdiv((K + 1) * d.n_ch, RJ)), dim3(CT), 0, s,
                       (const float*)part, n_parts, d.n_ch, K, dw, db);
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}

template <typename T>
int conv_fwd_k(const ConvDev& d, void* y, int64_t y_st, hipStream_t s) {
    switch (d.k) {
        case 1: return conv_fwd_run<1, T>(d, y, y_st, s);
        case 2: return conv_fwd_run<2, T>(d, y, y_st, s);
        case 3: return conv_fwd_run<3, T>(d, y, y_st, s);
        case 4: return conv_fwd_run<4, T>(d, y, y_st, s);
    }
    return TT_E_UNSUPPORTED;
}

template <typename T>
int conv_bwd_k(const ConvDev& d, const void* dy, int64_t dy_st, void* dx, float* dw, float* db, float* ws,
               hipStream_t s) {
    switch (d.k) {
        case 1: return conv_bwd_run<1, T>(d, dy, dy_st, dx, dw, db, ws, s);
        case 2: return conv_bwd_run<2, T>(d, dy, dy_st, dx, dw, db, ws, s);
        case 3: return conv_bwd_run<3, T>(d, dy, dy_st, dx, dw, db, ws, s);
        case 4: return conv_bwd_run<4, T>(d, dy, dy_st, dx, dw, db, ws, s);
    }
    return TT_E_UNSUPPORTED;
}

}  // namespace

size_t tt_conv_bwd_ws_bytes_impl(int n_tokens, int n_ch, int k) {
    const size_t parts = (size_t)tt_cdiv(n_tokens, CTOK_W);
    return ((size_t)n_tokens * n_ch + parts * (k + 1) * n_ch) * sizeof(float);
}

int tt_conv_fwd_launch(const ConvDev& d, void* y, int64_t y_st, hipStream_t s) {
    return d.dtype == TT_DTYPE_BF16 ? conv_fwd_k<__bf16>(d, y, y_st, s) : conv_fwd_k<float>(d, y, y_st, s);
}

int tt_conv_bwd_launch(const ConvDev& d, const void* dy, int64_t dy_st, void* dx, float* dw, float* db, float* ws,
                       hipStream_t s) {
    return d.dtype == TT_DTYPE_BF16 ? conv_bwd_k<__bf16>(d, dy, dy_st, dx, dw, db, ws, s)
                                    : conv_bwd_k<float>(d, dy, dy_st, dx, dw, db, ws, s);
}
