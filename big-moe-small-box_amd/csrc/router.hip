// Router and decode-size route + dispatch.
//
// One wavefront per token. Lane l holds experts l, l + 64, ...; the strict total order is larger choice, then lower
// index (a 64-bit key: order-preserving value bits over the complement of the index). The group limit takes each
// group's top-2 by wave-wide DPP maxima of the keys, then the groups by their top-2 sums; the top-k itself is a
// bitwise search for the k-th largest value by wave ballots followed by a rank of the k picks. The order is the one
// the oracle's sequential selection produces, independent of scheduling.
#include "bmx_common.hpp"
#include "bmx_internal.hpp"
#include "router_wave.hpp"

namespace bmx {

template <int J>
__global__ __launch_bounds__(RT_THREADS) void k_router(RouterArgs a)
{
    __shared__ TopkLds tl[RT_WAVES];
    const int t = blockIdx.x * RT_WAVES + (threadIdx.x >> 6);
    if (t < a.T) route_token_wave<J>(a, t, tl[threadIdx.x >> 6]);
}

// ---- fused decode kernel: route every token, then the counting sort of its picks, in one workgroup ------------------
template <int J>
__global__ __launch_bounds__(RT_THREADS) void k_route_dispatch_small(RouterArgs a, SmallDispatch d)
{
    __shared__ int pe[SM_MAXN];          // local expert of each pick (-1: dropped)
    __shared__ int cnt[RT_MAXE + 1];
    __shared__ TopkLds tl[RT_WAVES];
    const int E = a.E, n = a.T * a.topk, tid = threadIdx.x, lane = tid & 63;
    for (int t = tid >> 6; t < a.T; t += RT_WAVES)
    {
        const int pk = route_token_wave<J>(a, t, tl[tid >> 6]);
        if (lane < a.topk) pe[t * a.topk + lane] = pk;
    }
    if (a.T <= 64)
    {
        __shared__ int soff[RT_MAXE + 1];
        __shared__ uint64_t smask[RT_MAXE + 1];
        if (a.T > 1) lds_barrier();          // one token: wave 0 routed it and reads its own LDS writes in order
        if (tid < 64) dispatch_wave<J + 1>(pe, n, E, a.T, a.topk, d, cnt, soff, smask);
        return;
    }
    lds_barrier();
    const int NE = E + (d.shared ? 1 : 0);
    __shared__ int4 pe4[SM_MAXN / 4];        // the picks again, padded with -1 to a multiple of 4
    __shared__ int4 gc4[SM_MAXN / 4];        // per pick: groups of its expert if it is the expert's first pick, else 0
    const int n4 = (n + 3) >> 2;
    int* pev = reinterpret_cast<int*>(pe4);
    int* gcv = reinterpret_cast<int*>(gc4);
    for (int p = tid; p < 4 * n4; p += blockDim.x) pev[p] = p < n ? pe[p] : -1;
    lds_barrier();
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
    lds_barrier();
    for (int p = tid; p < 4 * n4; p += blockDim.x)
    {
        const int e = pev[p];
        int first = e >= 0;
        for (int q = 0; q < p && first; ++q) first = pev[q] != e;
        gcv[p] = first ? (cnt[e] + d.rpg - 1) / d.rpg : 0;
    }
    lds_barrier();
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

int check_router(int T, int E, int topk, int n_group, int topk_group, int score_fn, const void* logits,
                        const void* sel, const void* w)
{
    if (T < 0 || E <= 0 || E > RT_MAXE || topk <= 0 || topk > RT_MAXK || topk > E)
        return set_error(BMX_ERR_ARG, "bmx_router_topk: unsupported sizes T=%d E=%d topk=%d", T, E, topk);
    if (n_group < 1 || n_group > RT_MAXG || E % n_group || topk_group < 1 || topk_group > n_group)
        return set_error(BMX_ERR_ARG, "bmx_router_topk: bad groups n_group=%d topk_group=%d (E=%d)", n_group, topk_group, E);
    if (n_group > 1 && topk > topk_group * (E / n_group))
        return set_error(BMX_ERR_ARG, "bmx_router_topk: topk %d exceeds the experts of %d groups", topk, topk_group);
    if (score_fn != BMX_SCORE_SOFTMAX && score_fn != BMX_SCORE_SIGMOID && score_fn != BMX_SCORE_SQRTSP)
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
    switch (J)
    {
        case 1: hipLaunchKernelGGL(k_router<1>, grid, block, 0, s, a); break;
        case 2: hipLaunchKernelGGL(k_router<2>, grid, block, 0, s, a); break;
        case 3: hipLaunchKernelGGL(k_router<3>, grid, block, 0, s, a); break;
        case 4: hipLaunchKernelGGL(k_router<4>, grid, block, 0, s, a); break;
        case 5: hipLaunchKernelGGL(k_router<5>, grid, block, 0, s, a); break;
        case 6: hipLaunchKernelGGL(k_router<6>, grid, block, 0, s, a); break;
        case 7: case 8: hipLaunchKernelGGL(k_router<8>, grid, block, 0, s, a); break;
        default: hipLaunchKernelGGL(k_router<16>, grid, block, 0, s, a); break;
    }
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
    switch (J)
    {
        case 1: hipLaunchKernelGGL(k_route_dispatch_small<1>, grid, block, 0, s, a, d); break;
        case 2: hipLaunchKernelGGL(k_route_dispatch_small<2>, grid, block, 0, s, a, d); break;
        case 3: hipLaunchKernelGGL(k_route_dispatch_small<3>, grid, block, 0, s, a, d); break;
        case 4: hipLaunchKernelGGL(k_route_dispatch_small<4>, grid, block, 0, s, a, d); break;
        case 5: hipLaunchKernelGGL(k_route_dispatch_small<5>, grid, block, 0, s, a, d); break;
        case 6: hipLaunchKernelGGL(k_route_dispatch_small<6>, grid, block, 0, s, a, d); break;
        case 7: case 8: hipLaunchKernelGGL(k_route_dispatch_small<8>, grid, block, 0, s, a, d); break;
        default: hipLaunchKernelGGL(k_route_dispatch_small<16>, grid, block, 0, s, a, d); break;
    }
    return check_launch("route + dispatch");
}

// The arguments of launch_route_dispatch_small for a one-token gate / up GEMV that routes and dispatches the token itself
int route_fuse_args(const void* logits, const float* bias, int T, int E, int topk, int n_group, int topk_group,
                    int score_fn, int renorm, float scale, int64_t first, int64_t* sel, void* w, int shared, int rpg,
                    const bmx_routes* routes, RouteFuse* out)
{
    int rc = check_router(T, E, topk, n_group, topk_group, score_fn, logits, sel, w);
    if (rc) return rc;
    if (T != 1 || !route_dispatch_small_fits(T, E, topk))
        return set_error(BMX_ERR_ARG, "route in GEMV: one token and at most %d experts", RT_MAXE);
    out->ra = router_args(logits, bias, T, E, topk, n_group, topk_group, score_fn, renorm, scale, first, sel, w);
    out->sd.shared = shared ? 1 : 0;
    out->sd.rpg = rpg;
    out->sd.r = *routes;
    out->J = (E + 63) / 64;
    return BMX_OK;
}

// ---- router projection: logits = z W^T on the MFMA units ----------------------------------------------------------------
// logits[t][e] = RN16(sum_h z[t][h] W[e][h]): z fp16 [T][H] (the MoE input rows), W fp16 [E][H] (the router's gate weight
// as checkpoints store it), fp32 accumulation. Both operands are k-contiguous, so each lane's MFMA fragment (8
// consecutive k of one row of z or one row of W) is one 16-byte load. Workgroup = 32 tokens x 32 experts; its 4 waves
// take the four quarters of H (two accumulators each, alternate k-steps), and the quarter sums are added in wave order.
constexpr int RL_WAVES = 4;
__global__ __launch_bounds__(RL_WAVES * 64) void k_router_logits(const uint16_t* __restrict__ z,
                                                                 const uint16_t* __restrict__ W, int T, int H, int E,
                                                                 uint16_t* __restrict__ out)
{
    __shared__ f32x4 red[RL_WAVES - 1][4][64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int neb = (E + 31) / 32;
    const int tb = blockIdx.x / neb, eb = blockIdx.x % neb;
    const int t = tb * 32 + (lane & 31), e = eb * 32 + (lane & 31);
    const int kq = H / RL_WAVES;
    const int k0 = wave * kq + 8 * (lane >> 5);
    const bool tv = t < T, ev = e < E;
    const uint16_t* zp = z + (size_t)(tv ? t : 0) * H + k0;
    const uint16_t* wp = W + (size_t)(ev ? e : 0) * H + k0;
    const u32x4 zero = {0u, 0u, 0u, 0u};
    f32x16 acc0 = {}, acc1 = {};
    int k = 0;
    for (; k + 32 <= kq; k += 32)
    {
        const u32x4 a0 = tv ? ldg4(zp + k) : zero, b0 = ev ? ldg4(wp + k) : zero;
        const u32x4 a1 = tv ? ldg4(zp + k + 16) : zero, b1 = ev ? ldg4(wp + k + 16) : zero;
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a0), __builtin_bit_cast(f16x8, b0), acc0,
                                                      0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a1), __builtin_bit_cast(f16x8, b1), acc1,
                                                      0, 0, 0);
    }
    if (k < kq)
    {
        const u32x4 a0 = tv ? ldg4(zp + k) : zero, b0 = ev ? ldg4(wp + k) : zero;
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a0), __builtin_bit_cast(f16x8, b0), acc0,
                                                      0, 0, 0);
    }
    f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = acc0[v] + acc1[v];
    if (wave > 0)
#pragma unroll
        for (int q = 0; q < 4; ++q) red[wave - 1][q][lane] = f32x4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
    lds_barrier();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < RL_WAVES - 1; ++w)
#pragma unroll
        for (int q = 0; q < 4; ++q)
        {
            const f32x4 r = red[w][q][lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[4 * q + i] = acc[4 * q + i] + r[i];
        }
    // accumulator element v of lane L: row 8 (v / 4) + 4 (L / 32) + v % 4 (token), column L % 32 (expert)
    if (!ev) return;
#pragma unroll
    for (int v = 0; v < 16; ++v)
    {
        const int tt = tb * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (tt < T) out[(size_t)tt * E + e] = f2h_r(acc[v]);
    }
}

int launch_router_logits(const void* z, const void* W, int T, int H, int E, void* logits, hipStream_t s)
{
    if (T < 0 || E <= 0 || H <= 0 || H % 64)
        return set_error(BMX_ERR_ARG, "bmx_router_logits: T (%d) >= 0, E (%d) > 0 and H (%d) a multiple of 64 required",
                         T, E, H);
    if (T == 0) return BMX_OK;
    if (!z || !W || !logits) return set_error(BMX_ERR_ARG, "bmx_router_logits: null pointer");
    if ((reinterpret_cast<uintptr_t>(z) | reinterpret_cast<uintptr_t>(W)) % 16)
        return set_error(BMX_ERR_ARG, "bmx_router_logits: z and the weight must be 16-byte aligned");
    const long nblk = (long)((T + 31) / 32) * ((E + 31) / 32);
    if (nblk > 0x7fffffffL) return set_error(BMX_ERR_ARG, "bmx_router_logits: too many tiles");
    hipLaunchKernelGGL(k_router_logits, dim3((unsigned)nblk), dim3(RL_WAVES * 64), 0, s, static_cast<const uint16_t*>(z),
                       static_cast<const uint16_t*>(W), T, H, E, static_cast<uint16_t*>(logits));
    return check_launch("bmx_router_logits");
}

}  // namespace bmx
