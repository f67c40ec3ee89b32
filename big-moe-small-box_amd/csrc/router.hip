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

// wave-wide max of a uint32 (softmax's max logit): DPP within rows, then row broadcasts; lane 63 holds the result
__device__ __forceinline__ uint32_t wave_umax(uint32_t k)
{
    k = max(k, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0xB1, 0xf, 0xf, false));
    k = max(k, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0x4E, 0xf, 0xf, false));
    k = max(k, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0x141, 0xf, 0xf, false));
    k = max(k, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0x140, 0xf, 0xf, false));
    k = max(k, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0x142, 0xa, 0xf, false));
    k = max(k, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, 0x143, 0xc, 0xf, false));
    return __builtin_amdgcn_readlane(k, 63);
}

// Selection key of a candidate: the order-preserving key of its value above the complement of its index, so the
// largest key is the larger value and, among equal values, the lower index. 0 = no candidate.
__device__ __forceinline__ uint64_t sel_key(float v, int e)
{
    return ((uint64_t)okey(v) << 32) | (uint64_t)(0xffffffffu - (uint32_t)e);
}
__device__ __forceinline__ int key_index(uint64_t k) { return (int)(0xffffffffu - (uint32_t)k); }

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void kmax_dpp(uint32_t& hi, uint32_t& lo)
{
    const uint32_t ph = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, CTRL, ROW_MASK, 0xf, false);
    const uint32_t pl = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, CTRL, ROW_MASK, 0xf, false);
    const bool take = ph > hi || (ph == hi && pl > lo);
    hi = take ? ph : hi;
    lo = take ? pl : lo;
}

// wave-wide max of a 64-bit key, uniform result: xor 1 and xor 2 within quads, mirrors within half-rows and rows, then
// row 0 into row 1 and row 2 into row 3 (row_bcast:15), rows 0-1 into rows 2-3 (row_bcast:31): lane 63 holds the max
__device__ __forceinline__ uint64_t wave_kmax(uint64_t k)
{
    uint32_t hi = (uint32_t)(k >> 32), lo = (uint32_t)k;
    kmax_dpp<0xB1, 0xf>(hi, lo);
    kmax_dpp<0x4E, 0xf>(hi, lo);
    kmax_dpp<0x141, 0xf>(hi, lo);
    kmax_dpp<0x140, 0xf>(hi, lo);
    kmax_dpp<0x142, 0xa>(hi, lo);
    kmax_dpp<0x143, 0xc>(hi, lo);
    return ((uint64_t)__builtin_amdgcn_readlane(hi, 63) << 32) | __builtin_amdgcn_readlane(lo, 63);
}

// four independent wave-wide maxima, interleaved step by step (their latencies overlap)
__device__ __forceinline__ void wave_kmax4(uint64_t (&k)[4])
{
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) { hi[i] = (uint32_t)(k[i] >> 32); lo[i] = (uint32_t)k[i]; }
#pragma unroll
    for (int i = 0; i < 4; ++i) kmax_dpp<0xB1, 0xf>(hi[i], lo[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) kmax_dpp<0x4E, 0xf>(hi[i], lo[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) kmax_dpp<0x141, 0xf>(hi[i], lo[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) kmax_dpp<0x140, 0xf>(hi[i], lo[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) kmax_dpp<0x142, 0xa>(hi[i], lo[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) kmax_dpp<0x143, 0xc>(hi[i], lo[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        k[i] = ((uint64_t)__builtin_amdgcn_readlane(hi[i], 63) << 32) | __builtin_amdgcn_readlane(lo[i], 63);
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
// as a local expert id (-1 otherwise). Every selection is a wave-wide max of 64-bit keys (value, then lower index).
template <int J>
__device__ int route_token_wave(const RouterArgs& a, int t)
{
    const int lane = threadIdx.x & 63, E = a.E;
    const uint16_t* lg = a.logits + (size_t)t * E;
    float ch[J], sc[J], bias[J];
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int j = 0; j < J; ++j)
    {
        const int e = lane + 64 * j;
        ch[j] = e < E ? canon(h2f(lg[e])) : -__builtin_huge_valf();
        bias[j] = (a.bias && e < E) ? a.bias[e] : 0.0f;
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
            if (e < E) ch[j] = canon(a.bias ? __fadd_rn(sc[j], bias[j]) : sc[j]);
        }
    }
    uint64_t key[J];
#pragma unroll
    for (int j = 0; j < J; ++j)
    {
        const int e = lane + 64 * j;
        key[j] = e < E ? sel_key(ch[j], e) : 0ull;
    }
    // group limit: a group's score is the sum of its two best choices; the topk_group best groups stay eligible
    const int G = a.G, gs = E / G;
    if (G > 1)
    {
        float mygsc = 0.0f;                      // lane g holds group g's score
        for (int g0 = 0; g0 < G; g0 += 4)
        {
            // best and second-best key of groups g0 .. g0 + 3 (groups past G are empty)
            uint64_t k1[4], k2[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const int g = g0 + i;
                uint64_t b = 0;
#pragma unroll
                for (int j = 0; j < J; ++j)
                {
                    const int e = lane + 64 * j;
                    const uint64_t k = (g < G && e >= g * gs && e < (g + 1) * gs) ? key[j] : 0ull;
                    b = k > b ? k : b;
                }
                k1[i] = b;
            }
            wave_kmax4(k1);
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const int g = g0 + i, b1 = key_index(k1[i]);
                uint64_t b = 0;
#pragma unroll
                for (int j = 0; j < J; ++j)
                {
                    const int e = lane + 64 * j;
                    const uint64_t k = (g < G && e >= g * gs && e < (g + 1) * gs && e != b1) ? key[j] : 0ull;
                    b = k > b ? k : b;
                }
                k2[i] = b;
            }
            wave_kmax4(k2);
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const int g = g0 + i;
                if (g >= G) break;
                const int b1 = key_index(k1[i]);
                float t1 = 0.0f, t2 = 0.0f;
#pragma unroll
                for (int j = 0; j < J; ++j)
                {
                    t1 = (lane + 64 * j == b1) ? ch[j] : t1;
                    t2 = (k2[i] && lane + 64 * j == key_index(k2[i])) ? ch[j] : t2;
                }
                t1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t1), b1 & 63));
                if (k2[i])
                    t2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t2), key_index(k2[i]) & 63));
                if (lane == g) mygsc = canon(k2[i] ? __fadd_rn(t1, t2) : t1);
            }
        }
        uint64_t gk = lane < G ? sel_key(mygsc, lane) : 0ull, gok = 0;
        for (int r = 0; r < a.TG && r < G; ++r)
        {
            const int bg = key_index(wave_kmax(gk));
            gok |= 1ull << bg;
            if (lane == bg) gk = 0;
        }
#pragma unroll
        for (int j = 0; j < J; ++j)
        {
            const int e = lane + 64 * j;
            if (e < E && !((gok >> (e / gs)) & 1ull)) key[j] = 0;
        }
    }
    // top-k: each lane offers its best remaining key; the winner's lane clears it and offers its next
    auto lane_best = [&](uint64_t& bk, float& bs) {
        bk = 0;
        bs = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j)
        {
            const bool tk = key[j] > bk;
            bk = tk ? key[j] : bk;
            bs = tk ? sc[j] : bs;
        }
    };
    uint64_t bk;
    float bs;
    lane_best(bk, bs);
    int mypick = -1;
    float vsum = 0.0f, myscore = 0.0f;
    for (int k = 0; k < a.topk; ++k)
    {
        const int win = key_index(wave_kmax(bk));
        const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bs), win & 63));
        vsum = __fadd_rn(vsum, ws);
        if (lane == k) { mypick = win; myscore = ws; }
        if ((win & 63) == lane)
        {
#pragma unroll
            for (int j = 0; j < J; ++j) key[j] = (j == (win >> 6)) ? 0ull : key[j];
            lane_best(bk, bs);
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

// Counting sort of at most 64 picks by one wave, without barriers: pick p in lane p; per-expert counts by LDS atomics,
// offsets / group bases / unique ranks by one wave-wide scan over the experts, each pick's rank among its expert's
// picks by readlane broadcasts. Same output as the workgroup version below.
__device__ void dispatch_wave(const int* pe, int n, int E, int T, int topk, const SmallDispatch& d, int* scnt, int* soff,
                              int* sgo, int* sui)
{
    const int lane = threadIdx.x & 63, NE = E + (d.shared ? 1 : 0), rpg = d.rpg;
    // groups of a count: ceil(c / rpg), a shift when rpg is a power of two (every path's group size is)
    const bool pow2 = (rpg & (rpg - 1)) == 0;
    const int sh = __builtin_ctz((unsigned)rpg);
    auto ngr = [&](int c) { return pow2 ? (c + rpg - 1) >> sh : (c + rpg - 1) / rpg; };
    const int e = lane < n ? pe[lane] : -1;
    for (int x = lane; x < NE; x += 64) scnt[x] = 0;
    if (lane < n && e >= 0) atomicAdd(&scnt[e], 1);
    if (d.shared && lane == 0) scnt[E] = T;
    // each lane scans a run of C consecutive experts; run totals are scanned across the wave
    const int C = (NE + 63) / 64, x0 = lane * C;
    int tc = 0, tg = 0, tu = 0;
    for (int i = 0; i < C; ++i)
    {
        const int x = x0 + i;
        const int c = x < NE ? scnt[x] : 0;
        tc += c;
        tg += ngr(c);
        tu += c > 0;
    }
    int ic = tc, ig = tg, iu = tu;                 // inclusive scans
#pragma unroll
    for (int o = 1; o < 64; o <<= 1)
    {
        const int pc = __shfl_up(ic, o), pg = __shfl_up(ig, o), pu = __shfl_up(iu, o);
        if (lane >= o) { ic += pc; ig += pg; iu += pu; }
    }
    int bc = ic - tc, bg = ig - tg, bu = iu - tu;  // exclusive
    for (int i = 0; i < C; ++i)
    {
        const int x = x0 + i;
        if (x >= NE) break;
        const int c = scnt[x];
        soff[x] = bc;
        sgo[x] = bg;
        sui[x] = bu;
        d.r.counts[x] = c;
        d.r.offsets[x] = bc;
        if (c > 0)
        {
            d.r.uexp[bu] = x;
            for (int q = 0; q * rpg < c; ++q)
            {
                d.r.groups[3 * (bg + q) + 0] = x;
                d.r.groups[3 * (bg + q) + 1] = bc + q * rpg;
                d.r.groups[3 * (bg + q) + 2] = min(rpg, c - q * rpg);
            }
        }
        bc += c;
        bg += ngr(c);
        bu += c > 0;
    }
    if (lane == 63)
    {
        d.r.offsets[NE] = ic;
        *d.r.nuniq = iu;
        *d.r.ngroups = ig;
    }
    // rows of the routed picks: stable by (expert, pick)
    int rank = 0;
    for (int q = 0; q < n; ++q) rank += (__builtin_amdgcn_readlane(e, q) == e) && q < lane;
    if (lane < n)
    {
        if (e < 0) d.r.inv[lane] = -1;
        else
        {
            const int row = soff[e] + rank;
            d.r.inv[lane] = row;
            d.r.row_token[row] = lane / topk;
            d.r.row_slot[row] = lane % topk;
            d.r.row_expert[row] = e;
        }
    }
    if (d.shared)
        for (int t = lane; t < T; t += 64)
        {
            const int row = soff[E] + t;
            d.r.row_token[row] = t;
            d.r.row_slot[row] = -1;
            d.r.row_expert[row] = E;
        }
}

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
    if (n <= 64)
    {
        __shared__ int soff[RT_MAXE + 1], sgo[RT_MAXE + 1], sui[RT_MAXE + 1];
        if (a.T > 1) lds_barrier();          // one token: wave 0 routed it and reads its own LDS writes in order
        if (tid < 64) dispatch_wave(pe, n, E, a.T, a.topk, d, cnt, soff, sgo, sui);
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

}  // namespace bmx
