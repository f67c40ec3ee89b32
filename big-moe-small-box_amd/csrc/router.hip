// Router and decode-size route + dispatch.
//
// One wavefront per token. Lane l holds experts l, l + 64, ...; each pick is a wave-wide argmax under the strict total
// order (larger choice, then lower index): a DPP max of the order-preserving key of the value, then a DPP min of the
// index among the lanes holding that value. The group limit picks each group's top-2 the same way, then the groups by
// their top-2 sums. The order is the one the oracle's sequential selection produces, independent of scheduling.
#include "bmx_common.hpp"
#include "bmx_internal.hpp"

namespace bmx {

constexpr int RT_WAVES = 16;
constexpr int RT_THREADS = RT_WAVES * 64;
constexpr int RT_MAXJ = 16;        // experts per lane: E <= 1024
constexpr int RT_MAXE = RT_MAXJ * 64;
constexpr int RT_MAXG = 64;
constexpr int RT_MAXK = 32;
constexpr int SM_MAXN = 256;       // picks of the fused decode kernel

__device__ __forceinline__ float canon(float v) { return v != v ? -__builtin_huge_valf() : __fadd_rn(v, 0.0f); }
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) { return va > vb || (va == vb && ia < ib); }

// unsigned key with the order of the (canonical, non-NaN) float
__device__ __forceinline__ uint32_t okey(float v)
{
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// wave-wide max / min of a uint32, uniform result: xor 1 and xor 2 within quads, mirrors within half-rows and rows
// (each lane then holds its row's result), then the four rows on the scalar unit
__device__ __forceinline__ uint32_t wave_umax(uint32_t k)
{
    k = max(k, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0xB1, 0xf, 0xf, false));
    k = max(k, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0x4E, 0xf, 0xf, false));
    k = max(k, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0x141, 0xf, 0xf, false));
    k = max(k, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0x140, 0xf, 0xf, false));
    const uint32_t a = __builtin_amdgcn_readlane(k, 0), b = __builtin_amdgcn_readlane(k, 16);
    const uint32_t c = __builtin_amdgcn_readlane(k, 32), d = __builtin_amdgcn_readlane(k, 48);
    return max(max(a, b), max(c, d));
}

__device__ __forceinline__ uint32_t wave_umin(uint32_t k)
{
    k = min(k, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)k, 0xB1, 0xf, 0xf, false));
    k = min(k, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)k, 0x4E, 0xf, 0xf, false));
    k = min(k, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)k, 0x141, 0xf, 0xf, false));
    k = min(k, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)k, 0x140, 0xf, 0xf, false));
    const uint32_t a = __builtin_amdgcn_readlane(k, 0), b = __builtin_amdgcn_readlane(k, 16);
    const uint32_t c = __builtin_amdgcn_readlane(k, 32), d = __builtin_amdgcn_readlane(k, 48);
    return min(min(a, b), min(c, d));
}

// index of the best of (lane candidate v at index i; i < 0 = none) over the wave, -1 if none
__device__ __forceinline__ int wave_argbest(float v, int i)
{
    const uint32_t k = i >= 0 ? okey(v) : 0u;
    const uint32_t m = wave_umax(k);
    if (m == 0u) return -1;
    return (int)wave_umin((i >= 0 && k == m) ? (uint32_t)i : 0xffffffffu);
}

struct RouterArgs {
    const uint16_t* logits;
    const float* bias;
    int T, E, topk, G, TG, score_fn, renorm;
    float scale;
    int64_t first;
    int64_t* sel;
    uint16_t* w;
};

// Route token t with the calling wave. Writes sel / w of the token; returns the pick of slot `lane` (lanes < topk)
// as a local expert id (-1 otherwise).
template <int J>
__device__ int route_token_wave(const RouterArgs& a, int t)
{
    const int lane = threadIdx.x & 63, E = a.E;
    const uint16_t* lg = a.logits + (size_t)t * E;
    float ch[J], sc[J];
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int j = 0; j < J; ++j)
    {
        const int e = lane + 64 * j;
        ch[j] = e < E ? canon(h2f(lg[e])) : -__builtin_huge_valf();
        mx = fmaxf(mx, ch[j]);
    }
    if (a.score_fn == BMX_SCORE_SOFTMAX)
    {
        const uint32_t m = wave_umax(okey(mx));
        mx = __builtin_bit_cast(float, (m & 0x80000000u) ? (m & 0x7fffffffu) : ~m);
    }
#pragma unroll
    for (int j = 0; j < J; ++j)
    {
        const int e = lane + 64 * j;
        if (a.score_fn == BMX_SCORE_SOFTMAX) sc[j] = e < E ? exp_fixed(__fsub_rn(ch[j], mx)) : 0.0f;
        else
        {
            sc[j] = e < E ? sigmoid_fixed(ch[j]) : 0.0f;
            if (e < E) ch[j] = canon(a.bias ? __fadd_rn(sc[j], a.bias[e]) : sc[j]);
        }
    }
    // group limit
    uint64_t gok = ~0ull;
    const int G = a.G, gs = E / G;
    if (G > 1)
    {
        float mygsc = 0.0f;                      // lane g holds group g's score
        for (int g = 0; g < G; ++g)
        {
            float v1 = 0.0f, v2 = 0.0f;
            int i1 = -1, i2 = -1;
#pragma unroll
            for (int j = 0; j < J; ++j)
            {
                const int e = lane + 64 * j;
                if (e >= g * gs && e < (g + 1) * gs && (i1 < 0 || better(ch[j], e, v1, i1))) { v1 = ch[j]; i1 = e; }
            }
            const int b1 = wave_argbest(v1, i1);
#pragma unroll
            for (int j = 0; j < J; ++j)
            {
                const int e = lane + 64 * j;
                if (e >= g * gs && e < (g + 1) * gs && e != b1 && (i2 < 0 || better(ch[j], e, v2, i2))) { v2 = ch[j]; i2 = e; }
            }
            const int b2 = wave_argbest(v2, i2);
            float t1 = 0.0f, t2 = 0.0f;
#pragma unroll
            for (int j = 0; j < J; ++j)
            {
                t1 = (lane + 64 * j == b1) ? ch[j] : t1;
                t2 = (lane + 64 * j == b2) ? ch[j] : t2;
            }
            t1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t1), b1 & 63));
            t2 = b2 >= 0 ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t2), b2 & 63)) : 0.0f;
            if (lane == g) mygsc = canon(b2 >= 0 ? __fadd_rn(t1, t2) : t1);
        }
        gok = 0;
        for (int r = 0; r < a.TG && r < G; ++r)
        {
            const int bg = wave_argbest(mygsc, (lane < G && !((gok >> lane) & 1ull)) ? lane : -1);
            gok |= 1ull << bg;
        }
    }
    // top-k: each lane keeps its best remaining candidate; the winner's lane drops it and rescans
    uint32_t taken = 0;
    auto local_best = [&](float& bv, int& bi, float& bs) {
        bi = -1; bv = 0.0f; bs = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j)
        {
            const int e = lane + 64 * j;
            const bool ok = e < E && !((taken >> j) & 1u) && (G <= 1 || ((gok >> (e / gs)) & 1ull));
            if (ok && (bi < 0 || better(ch[j], e, bv, bi))) { bv = ch[j]; bi = e; bs = sc[j]; }
        }
    };
    float bv, bs;
    int bi;
    local_best(bv, bi, bs);
    int mypick = -1;
    float vsum = 0.0f, myscore = 0.0f;
    for (int k = 0; k < a.topk; ++k)
    {
        const int win = wave_argbest(bv, bi);
        const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bs), win & 63));
        vsum = __fadd_rn(vsum, ws);
        if (lane == k) { mypick = win; myscore = ws; }
        if ((win & 63) == lane)
        {
            taken |= 1u << (win >> 6);
            local_best(bv, bi, bs);
        }
    }
    float den = 1.0f;
    if (a.score_fn == BMX_SCORE_SOFTMAX && !a.renorm)
    {
        den = 0.0f;
        for (int e = 0; e < E; ++e)
        {
            float v = 0.0f;
#pragma unroll
            for (int j = 0; j < J; ++j) v = (j == (e >> 6)) ? sc[j] : v;
            den = __fadd_rn(den, __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), e & 63)));
        }
    }
    else if (a.renorm) den = vsum;
    if (lane < a.topk)
    {
        const float qv = (a.score_fn == BMX_SCORE_SIGMOID && !a.renorm) ? myscore : __fdiv_rn(myscore, den);
        a.sel[(size_t)t * a.topk + lane] = (int64_t)mypick + a.first;
        a.w[(size_t)t * a.topk + lane] = f2h_r(__fmul_rn(qv, a.scale));
    }
    return mypick;
}

template <int J>
__global__ __launch_bounds__(RT_THREADS) void k_router(RouterArgs a)
{
    const int t = blockIdx.x * RT_WAVES + (threadIdx.x >> 6);
    if (t < a.T) route_token_wave<J>(a, t);
}

// ---- fused decode kernel: route every token, then the counting sort of its picks, in one workgroup ------------------
struct SmallDispatch {
    int shared, rpg;
    bmx_routes r;
};

template <int J>
__global__ __launch_bounds__(RT_THREADS) void k_route_dispatch_small(RouterArgs a, SmallDispatch d)
{
    __shared__ int pe[SM_MAXN];          // local expert of each pick (-1: dropped)
    __shared__ int cnt[RT_MAXE + 1];
    const int E = a.E, n = a.T * a.topk, tid = threadIdx.x, lane = tid & 63;
    for (int t = tid >> 6; t < a.T; t += RT_WAVES)
    {
        const int pk = route_token_wave<J>(a, t);
        if (lane < a.topk) pe[t * a.topk + lane] = pk;
    }
    __syncthreads();
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


int launch_router(const void* logits, const float* bias, int T, int E, int topk, int n_group, int topk_group,
                  int score_fn, int renorm, float scale, int64_t first, int64_t* sel, void* w, hipStream_t s)
{
    int rc = check_router(T, E, topk, n_group, topk_group, score_fn, logits, sel, w);
    if (rc || T == 0) return rc;
    const RouterArgs a = router_args(logits, bias, T, E, topk, n_group, topk_group, score_fn, renorm, scale, first, sel, w);
    const dim3 grid((unsigned)((T + RT_WAVES - 1) / RT_WAVES)), block(RT_THREADS);
    const int J = (E + 63) / 64;
    if (J <= 1) hipLaunchKernelGGL(k_router<1>, grid, block, 0, s, a);
    else if (J <= 2) hipLaunchKernelGGL(k_router<2>, grid, block, 0, s, a);
    else if (J <= 4) hipLaunchKernelGGL(k_router<4>, grid, block, 0, s, a);
    else if (J <= 8) hipLaunchKernelGGL(k_router<8>, grid, block, 0, s, a);
    else hipLaunchKernelGGL(k_router<16>, grid, block, 0, s, a);
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
    const int J = (E + 63) / 64;
    const dim3 grid(1), block(RT_THREADS);
    if (J <= 1) hipLaunchKernelGGL(k_route_dispatch_small<1>, grid, block, 0, s, a, d);
    else if (J <= 2) hipLaunchKernelGGL(k_route_dispatch_small<2>, grid, block, 0, s, a, d);
    else if (J <= 4) hipLaunchKernelGGL(k_route_dispatch_small<4>, grid, block, 0, s, a, d);
    else if (J <= 8) hipLaunchKernelGGL(k_route_dispatch_small<8>, grid, block, 0, s, a, d);
    else hipLaunchKernelGGL(k_route_dispatch_small<16>, grid, block, 0, s, a, d);
    return check_launch("route + dispatch");
}

}  // namespace bmx
