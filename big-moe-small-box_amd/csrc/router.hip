// Router and decode-size route + dispatch.
//
// Selection by rank: every candidate counts the candidates that beat it under the strict total order (larger choice,
// then lower index); rank < k selects it into slot `rank`. The group limit ranks the top-2 of each group the same way,
// then the groups by their top-2 sums. All threads read the same LDS word at each step (broadcast), so a token costs
// E LDS reads per thread and no serial reduction chain; the result is the order the oracle's sequential selection
// produces, independent of scheduling.
#include "bmx_common.hpp"
#include "bmx_internal.hpp"

namespace bmx {

constexpr int RT_THREADS = 1024;
constexpr int RT_MAXE = 1024;
constexpr int RT_MAXG = 64;
constexpr int RT_MAXK = 32;
constexpr int SM_MAXN = 256;       // picks of the fused decode kernel

__device__ __forceinline__ float canon(float v) { return v != v ? -__builtin_huge_valf() : __fadd_rn(v, 0.0f); }
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) { return va > vb || (va == vb && ia < ib); }

struct RouterArgs {
    const uint16_t* logits;
    const float* bias;
    int T, E, topk, G, TG, score_fn, renorm;
    float scale;
    int64_t first;
    int64_t* sel;
    uint16_t* w;
};

struct RouteShared {
    float ch[RT_MAXE] __attribute__((aligned(16)));
    float sc[RT_MAXE];
    float gtop[RT_MAXG][2], gsc[RT_MAXG];
    int gok[RT_MAXG];
    int idx[RT_MAXK];
    float wmax[RT_THREADS / 64];
};

// Route token t with threads [tid0, tid0 + E) of the workgroup (one thread per expert). Writes sel / w of the token and
// leaves the local picks in S.idx. Every thread of the workgroup must call it (it synchronises).
__device__ void route_token(const RouterArgs& a, int t, RouteShared& S)
{
    const int e = threadIdx.x, E = a.E;
    const bool mine = e < E;
    const uint16_t* lg = a.logits + (size_t)t * E;
    float l = mine ? canon(h2f(lg[e])) : -__builtin_huge_valf();
    float mx = 0.0f;
    if (a.score_fn == BMX_SCORE_SOFTMAX)
    {
        float v = l;
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) v = fmaxf(v, __shfl_xor(v, m));
        if ((threadIdx.x & 63) == 0) S.wmax[threadIdx.x >> 6] = v;
        __syncthreads();
        mx = S.wmax[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) mx = fmaxf(mx, S.wmax[w]);
    }
    if (e >= E && e < ((E + 31) & ~31)) S.ch[e] = -__builtin_huge_valf();   // padding never beats a real expert
    if (mine)
    {
        if (a.score_fn == BMX_SCORE_SOFTMAX) { S.sc[e] = exp_fixed(__fsub_rn(l, mx)); S.ch[e] = l; }
        else
        {
            const float s = sigmoid_fixed(l);
            S.sc[e] = s;
            S.ch[e] = canon(a.bias ? __fadd_rn(s, a.bias[e]) : s);
        }
    }
    __syncthreads();
    const int G = a.G, gs = E / G;
    if (G > 1)
    {
        if (mine)
        {
            const int g = e / gs;
            const float c = S.ch[e];
            int r = 0;
            for (int q = g * gs; q < (g + 1) * gs; ++q) r += better(S.ch[q], q, c, e) ? 1 : 0;
            if (r < 2) S.gtop[g][r] = c;
        }
        __syncthreads();
        if (e < G) S.gsc[e] = canon(gs >= 2 ? __fadd_rn(S.gtop[e][0], S.gtop[e][1]) : S.gtop[e][0]);
        __syncthreads();
        if (e < G)
        {
            int r = 0;
            for (int q = 0; q < G; ++q) r += better(S.gsc[q], q, S.gsc[e], e) ? 1 : 0;
            S.gok[e] = r < a.TG;
        }
        __syncthreads();
    }
    const bool allowed = mine && (G <= 1 || S.gok[e / gs]);
    if (allowed)
    {
        const float c = S.ch[e];
        int r = 0;
        if (G <= 1)
        {
            // 32 candidates per step: eight independent 16-byte LDS reads in flight, then the compares
            for (int q0 = 0; q0 < E; q0 += 32)
            {
                float4 v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const float4*>(&S.ch[q0 + 4 * i]);
#pragma unroll
                for (int i = 0; i < 8; ++i)
                {
                    const int q = q0 + 4 * i;
                    r += (better(v[i].x, q, c, e) ? 1 : 0) + (better(v[i].y, q + 1, c, e) ? 1 : 0) +
                         (better(v[i].z, q + 2, c, e) ? 1 : 0) + (better(v[i].w, q + 3, c, e) ? 1 : 0);
                }
            }
        }
        else
        {
            for (int g = 0; g < G; ++g)
            {
                if (!S.gok[g]) continue;
#pragma unroll 4
                for (int q = g * gs; q < (g + 1) * gs; ++q) r += better(S.ch[q], q, c, e) ? 1 : 0;
            }
        }
        if (r < a.topk) S.idx[r] = e;
    }
    __syncthreads();
    if (threadIdx.x == 0)
    {
        float vsum = 0.0f;
        for (int k = 0; k < a.topk; ++k) vsum = __fadd_rn(vsum, S.sc[S.idx[k]]);
        float den = 1.0f;
        if (a.score_fn == BMX_SCORE_SOFTMAX && !a.renorm)
        {
            den = 0.0f;
            for (int q = 0; q < E; ++q) den = __fadd_rn(den, S.sc[q]);
        }
        else if (a.renorm) den = vsum;
        for (int k = 0; k < a.topk; ++k)
        {
            const float v = S.sc[S.idx[k]];
            const float qv = (a.score_fn == BMX_SCORE_SIGMOID && !a.renorm) ? v : __fdiv_rn(v, den);
            a.sel[(size_t)t * a.topk + k] = (int64_t)S.idx[k] + a.first;
            a.w[(size_t)t * a.topk + k] = f2h(__fmul_rn(qv, a.scale));
        }
    }
    __syncthreads();
}

// one workgroup per token
__global__ __launch_bounds__(RT_THREADS) void k_router(RouterArgs a)
{
    __shared__ RouteShared S;
    route_token(a, blockIdx.x, S);
}

// ---- fused decode kernel: route every token, then the counting sort of its picks, in one workgroup ------------------
struct SmallDispatch {
    int shared, rpg;
    bmx_routes r;
};

__global__ __launch_bounds__(RT_THREADS) void k_route_dispatch_small(RouterArgs a, SmallDispatch d)
{
    __shared__ RouteShared S;
    __shared__ int pe[SM_MAXN];          // local expert of each pick (-1: dropped)
    __shared__ int cnt[RT_MAXE + 1];
    const int E = a.E, n = a.T * a.topk, tid = threadIdx.x;
    for (int t = 0; t < a.T; ++t)
    {
        route_token(a, t, S);
        if (tid < a.topk) pe[t * a.topk + tid] = S.idx[tid];
        __syncthreads();
    }
    const int NE = E + (d.shared ? 1 : 0);
    __shared__ int4 pe4[SM_MAXN / 4];        // the picks again, padded with -1 to a multiple of 4
    __shared__ int4 gc4[SM_MAXN / 4];        // per pick: groups of its expert if it is the expert's first pick, else 0
    const int n4 = (n + 3) >> 2;
    int* pev = reinterpret_cast<int*>(pe4);
    int* gcv = reinterpret_cast<int*>(gc4);
    for (int p = tid; p < 4 * n4; p += blockDim.x) pev[p] = p < n ? pe[p] : -1;
    __syncthreads();
    // counts and offsets per expert (the shared segment last)
    int nvalid = 0;
    for (int q = 0; q < n4; ++q)
    {
        const int4 v = pe4[q];
        nvalid += (v.x >= 0) + (v.y >= 0) + (v.z >= 0) + (v.w >= 0);
    }
    for (int e = tid; e < NE; e += blockDim.x)
    {
        int c = 0, below = 0;
        if (e < E)
            for (int q = 0; q < n4; ++q)
            {
                const int4 v = pe4[q];
                c += (v.x == e) + (v.y == e) + (v.z == e) + (v.w == e);
                below += (v.x >= 0 && v.x < e) + (v.y >= 0 && v.y < e) + (v.z >= 0 && v.z < e) + (v.w >= 0 && v.w < e);
            }
        else { c = a.T; below = nvalid; }
        cnt[e] = c;
        d.r.counts[e] = c;
        d.r.offsets[e] = below;
        if (e == NE - 1) d.r.offsets[NE] = below + c;
    }
    __syncthreads();
    for (int p = tid; p < 4 * n4; p += blockDim.x)
    {
        const int e = pev[p];
        int first = e >= 0;
        for (int q = 0; q < p && first; ++q) first = pev[q] != e;
        gcv[p] = first ? (cnt[e] + d.rpg - 1) / d.rpg : 0;
    }
    __syncthreads();
    int nu_r = 0, ng_r = 0;
    for (int q = 0; q < n4; ++q)
    {
        const int4 g = gc4[q];
        nu_r += (g.x > 0) + (g.y > 0) + (g.z > 0) + (g.w > 0);
        ng_r += g.x + g.y + g.z + g.w;
    }
    // rows: stable by (expert, pick); the expert's first pick also places its groups and its uexp entry
    for (int p = tid; p < n; p += blockDim.x)
    {
        const int e = pev[p];
        if (e < 0) { d.r.inv[p] = -1; continue; }
        int row = 0, ui = 0, g0 = 0;
        for (int q4 = 0; q4 < n4; ++q4)
        {
            const int4 v = pe4[q4], g = gc4[q4];
            const int q = 4 * q4;
            row += (v.x >= 0 && (v.x < e || (v.x == e && q < p))) + (v.y >= 0 && (v.y < e || (v.y == e && q + 1 < p))) +
                   (v.z >= 0 && (v.z < e || (v.z == e && q + 2 < p))) + (v.w >= 0 && (v.w < e || (v.w == e && q + 3 < p)));
            ui += (g.x > 0 && v.x < e) + (g.y > 0 && v.y < e) + (g.z > 0 && v.z < e) + (g.w > 0 && v.w < e);
            g0 += (v.x < e ? g.x : 0) + (v.y < e ? g.y : 0) + (v.z < e ? g.z : 0) + (v.w < e ? g.w : 0);
        }
        d.r.inv[p] = row;
        d.r.row_token[row] = p / a.topk;
        d.r.row_slot[row] = p % a.topk;
        d.r.row_expert[row] = e;
        const int ng = gcv[p];
        if (ng > 0)
        {
            const int c = cnt[e];
            d.r.uexp[ui] = e;
            for (int q = 0; q < ng; ++q)
            {
                d.r.groups[3 * (g0 + q) + 0] = e;
                d.r.groups[3 * (g0 + q) + 1] = row + q * d.rpg;
                d.r.groups[3 * (g0 + q) + 2] = min(d.rpg, c - q * d.rpg);
            }
        }
    }
    if (d.shared)
    {
        for (int t = tid; t < a.T; t += blockDim.x)
        {
            d.r.row_token[nvalid + t] = t;
            d.r.row_slot[nvalid + t] = -1;
            d.r.row_expert[nvalid + t] = E;
        }
        for (int q = tid; q * d.rpg < a.T; q += blockDim.x)
        {
            d.r.groups[3 * (ng_r + q) + 0] = E;
            d.r.groups[3 * (ng_r + q) + 1] = nvalid + q * d.rpg;
            d.r.groups[3 * (ng_r + q) + 2] = min(d.rpg, a.T - q * d.rpg);
        }
        if (tid == 0) d.r.uexp[nu_r] = E;
    }
    if (tid == 0)
    {
        *d.r.nuniq = nu_r + (d.shared ? 1 : 0);
        *d.r.ngroups = ng_r + (d.shared ? (a.T + d.rpg - 1) / d.rpg : 0);
    }
}

static int check_router(int T, int E, int topk, int n_group, int topk_group, int score_fn, const void* logits,
                        const void* sel, const void* w)
{
    if (T < 0 || E <= 0 || E > RT_MAXE || topk <= 0 || topk > RT_MAXK || topk > E)
        return set_error(BMX_ERR_ARG, "bmx_router_topk: unsupported sizes T=%d E=%d topk=%d", T, E, topk);
    if (n_group < 1 || n_group > RT_MAXG || E % n_group || topk_group < 1 || topk_group > n_group)
        return set_error(BMX_ERR_ARG, "bmx_router_topk: bad groups n_group=%d topk_group=%d (E=%d)", n_group, topk_group, E);
    if (n_group > 1 && topk > topk_group * (E / n_group))
        return set_error(BMX_ERR_ARG, "bmx_router_topk: topk %d exceeds the experts of %d groups", topk, topk_group);
    if (score_fn != BMX_SCORE_SOFTMAX && score_fn != BMX_SCORE_SIGMOID)
        return set_error(BMX_ERR_ARG, "bmx_router_topk: unknown score function %d", score_fn);
    if (T > 0 && (!logits || !sel || !w)) return set_error(BMX_ERR_ARG, "bmx_router_topk: null pointer");
    return BMX_OK;
}

static RouterArgs router_args(const void* logits, const float* bias, int T, int E, int topk, int n_group,
                              int topk_group, int score_fn, int renorm, float scale, int64_t first, int64_t* sel, void* w)
{
    RouterArgs a;
    a.logits = static_cast<const uint16_t*>(logits); a.bias = bias; a.T = T; a.E = E; a.topk = topk; a.G = n_group;
    a.TG = topk_group; a.score_fn = score_fn; a.renorm = renorm; a.scale = scale; a.first = first; a.sel = sel;
    a.w = static_cast<uint16_t*>(w);
    return a;
}

static unsigned router_threads(int E) { return (unsigned)((E + 63) / 64 * 64); }

int launch_router(const void* logits, const float* bias, int T, int E, int topk, int n_group, int topk_group,
                  int score_fn, int renorm, float scale, int64_t first, int64_t* sel, void* w, hipStream_t s)
{
    int rc = check_router(T, E, topk, n_group, topk_group, score_fn, logits, sel, w);
    if (rc || T == 0) return rc;
    const RouterArgs a = router_args(logits, bias, T, E, topk, n_group, topk_group, score_fn, renorm, scale, first, sel, w);
    hipLaunchKernelGGL(k_router, dim3((unsigned)T), dim3(router_threads(E)), 0, s, a);
    return check_launch("bmx_router_topk");
}

bool route_dispatch_small_fits(int T, int E, int topk) { return (long)T * topk <= SM_MAXN && E <= RT_MAXE; }

int launch_route_dispatch_small(const void* logits, const float* bias, int T, int E, int topk, int n_group,
                                int topk_group, int score_fn, int renorm, float scale, int64_t first, int64_t* sel,
                                void* w, int shared, int rpg, const bmx_routes* routes, hipStream_t s)
{
    int rc = check_router(T, E, topk, n_group, topk_group, score_fn, logits, sel, w);
    if (rc || T == 0) return rc;
    if (!route_dispatch_small_fits(T, E, topk)) return set_error(BMX_ERR_ARG, "route+dispatch: too many picks (%d)", T * topk);
    const RouterArgs a = router_args(logits, bias, T, E, topk, n_group, topk_group, score_fn, renorm, scale, first, sel, w);
    SmallDispatch d;
    d.shared = shared ? 1 : 0;
    d.rpg = rpg;
    d.r = *routes;
    const unsigned nt = router_threads(E) > 256 ? router_threads(E) : 256;
    hipLaunchKernelGGL(k_route_dispatch_small, dim3(1), dim3(nt), 0, s, a, d);
    return check_launch("route + dispatch");
}

}  // namespace bmx
