// The router's wave-level pieces: the top-k selection of one token by one wavefront (route_token_wave) and the
// counting sort of a few hundred picks by one wavefront (dispatch_wave). Shared by the router kernels and by the
// one-token gate / up GEMV, which routes its token itself.
#pragma once
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

// wave-wide min of a uint32, the same steps as wave_umax; uniform result
__device__ __forceinline__ uint32_t wave_umin(uint32_t k)
{
    k = min(k, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)k, 0xB1, 0xf, 0xf, false));
    k = min(k, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)k, 0x4E, 0xf, 0xf, false));
    k = min(k, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)k, 0x141, 0xf, 0xf, false));
    k = min(k, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)k, 0x140, 0xf, 0xf, false));
    k = min(k, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)k, 0x142, 0xa, 0xf, false));
    k = min(k, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)k, 0x143, 0xc, 0xf, false));
    return __builtin_amdgcn_readlane(k, 63);
}

// float of an order-preserving key (the inverse of okey)
__device__ __forceinline__ float unkey(uint32_t u)
{
    return __builtin_bit_cast(float, (u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

// the two largest of (a1 >= a2) and the pair of the lane CTRL selects
template <int CTRL>
__device__ __forceinline__ void top2_dpp(uint32_t& a1, uint32_t& a2)
{
    const uint32_t b1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)a1, CTRL, 0xf, 0xf, false);
    const uint32_t b2 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)a2, CTRL, 0xf, 0xf, false);
    const uint32_t n2 = max(min(a1, b1), max(a2, b2));
    a1 = max(a1, b1);
    a2 = n2;
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

// inclusive prefix sum over the wave (lane order): row shifts 1, 2, 4, 8 within rows of 16, then lane 15 into row 1 and
// lane 47 into row 3 (row_bcast:15), lane 31 into rows 2 and 3 (row_bcast:31)
__device__ __forceinline__ uint32_t wave_scan_add(uint32_t v)
{
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);
    return v;
}

__device__ __forceinline__ uint64_t lanes_below() { return (1ull << (threadIdx.x & 63)) - 1ull; }

// Per-wave LDS of the router.
constexpr int TK_CAP = 128;        // candidates ranked directly; more (many equal values) take the bitwise search
struct TopkLds {
    union {
        struct {
            uint32_t lmax[64];
            alignas(16) uint64_t ck[TK_CAP + 16];   // + room for the zero padding
            float cs[TK_CAP];
        };
        uint32_t vb[RT_MAXE];                       // group limit: the value key of every expert
    };
    alignas(16) uint64_t gk[RT_MAXG];
    int pick[RT_MAXK];
    float psc[RT_MAXK];
};

// The wave's LDS writes are seen by its later LDS reads (one wave, in order); the fences keep the compiler from moving
// accesses across the exchange.
__device__ __forceinline__ void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Top k of the candidates key[j] (sel_key; 0 = not a candidate; at least k candidates) in the order of the sequential
// selection (larger value, then lower index). Lane r < k receives pick r and its score; the return value is the scores
// summed in pick order.
//
// Let M be the k-th largest of the 64 lane maxima: k values are >= M, so every pick is >= M. The values >= M (about k
// of them) are packed into LDS and each is ranked against the others; a step issues all its LDS reads before it waits
// (one round trip each). When ties leave more than TK_CAP such values, the k-th largest value V is found by a bitwise
// search over the value half of the keys (wave ballots, 32 steps), every key above V is taken and the lowest indices
// among those equal to V fill the rest; those k are ranked the same way.
template <int J>
__device__ __forceinline__ float select_topk(const uint64_t (&key)[J], const float (&sc)[J], int k, TopkLds& L,
                                             int& mypick, float& myscore)
{
    const int lane = threadIdx.x & 63;
    const uint64_t below = lanes_below();
    uint32_t hv[J], hm = 0;
#pragma unroll
    for (int j = 0; j < J; ++j)
    {
        hv[j] = (uint32_t)(key[j] >> 32);
        hm = max(hm, hv[j]);
    }
    L.lmax[lane] = hm;
    wave_lds_sync();
    int above = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h)
    {
        uint4 lm[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) lm[q] = reinterpret_cast<const uint4*>(L.lmax)[8 * h + q];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < 8; ++q) above += (lm[q].x > hm) + (lm[q].y > hm) + (lm[q].z > hm) + (lm[q].w > hm);
    }
    const uint32_t M = wave_umin(above < k ? hm : 0xffffffffu);
    bool sel[J];
    int nc = 0;
#pragma unroll
    for (int j = 0; j < J; ++j)
    {
        sel[j] = key[j] != 0ull && hv[j] >= M;
        nc += __builtin_popcountll(__ballot(sel[j]));
    }
    if (nc > TK_CAP)
    {
        uint32_t v = 0;
        for (int b = 31; b >= 0; --b)
        {
            const uint32_t cand = v | (1u << b);
            int cnt = 0;
#pragma unroll
            for (int j = 0; j < J; ++j) cnt += __builtin_popcountll(__ballot(hv[j] >= cand));
            if (cnt >= k) v = cand;
        }
        int need = k;
#pragma unroll
        for (int j = 0; j < J; ++j) need -= __builtin_popcountll(__ballot(hv[j] > v));
#pragma unroll
        for (int j = 0; j < J; ++j)
        {
            const uint64_t meq = __ballot(hv[j] == v);
            const int take = min(need, __builtin_popcountll(meq));
            sel[j] = hv[j] > v || (hv[j] == v && __builtin_popcountll(meq & below) < take);
            need -= take;
        }
        nc = k;
    }
    int base = 0;
#pragma unroll
    for (int j = 0; j < J; ++j)
    {
        const uint64_t ms = __ballot(sel[j]);
        if (sel[j])
        {
            const int slot = base + __builtin_popcountll(ms & below);
            L.ck[slot] = key[j];
            L.cs[slot] = sc[j];
        }
        base += __builtin_popcountll(ms);
    }
    // zero keys up to a multiple of 16 (a zero key is below every candidate)
    const int nc16 = (nc + 15) & ~15;
    if (nc + lane < nc16) L.ck[nc + lane] = 0ull;
    wave_lds_sync();
    for (int c0 = 0; c0 < nc; c0 += 64)
    {
        const int c = c0 + lane;
        const uint64_t my = c < nc ? L.ck[c] : ~0ull;
        int r = 0;
        for (int q = 0; q < nc16; q += 16)
        {
            ulonglong2 v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const ulonglong2*>(&L.ck[q + 2 * i]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 8; ++i) r += (v[i].x > my) + (v[i].y > my);
        }
        if (c < nc && r < k)
        {
            L.pick[r] = key_index(my);
            L.psc[r] = L.cs[c];
        }
    }
    wave_lds_sync();
    mypick = lane < k ? L.pick[lane] : -1;
    myscore = lane < k ? L.psc[lane] : 0.0f;
    float vsum = 0.0f;
    for (int q = 0; q < k; ++q)
        vsum = __fadd_rn(vsum, __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, myscore), q)));
    return vsum;
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

// Route token t with the calling wave. Writes sel / w of the token (unless sel is null); returns the pick of slot
// `lane` (lanes < topk) as a local expert id (-1 otherwise). Every selection is a wave-wide max of 64-bit keys (value,
// then lower index).
template <int J>
__device__ int route_token_wave(const RouterArgs& a, int t, TopkLds& L)
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
            sc[j] = e < E ? (a.score_fn == BMX_SCORE_SQRTSP ? sqrtsp_fixed(ch[j]) : sigmoid_fixed(ch[j])) : 0.0f;
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
    if (G >= 4 && (64 % G) == 0 && E == 64 * J)
    {
        // 64 / G lanes per group (lane l: group l / lpg), each reading J of the group's values from LDS; their top-2
        // merged across the group's lanes by DPP (quad xor 1, xor 2, half-row mirror, row mirror); the groups ranked
        // by (score, lower index) against the G scores in LDS
        const int lpg = 64 / G, g = lane / lpg, sub = lane % lpg;
#pragma unroll
        for (int j = 0; j < J; ++j) L.vb[lane + 64 * j] = (uint32_t)(key[j] >> 32);
        wave_lds_sync();
        uint32_t v[J];
#pragma unroll
        for (int m = 0; m < J; ++m) v[m] = L.vb[g * gs + sub + lpg * m];
        __builtin_amdgcn_sched_barrier(0);
        uint32_t a1 = 0, a2 = 0;
#pragma unroll
        for (int m = 0; m < J; ++m)
        {
            a2 = max(a2, min(a1, v[m]));
            a1 = max(a1, v[m]);
        }
        if (lpg >= 2) top2_dpp<0xB1>(a1, a2);
        if (lpg >= 4) top2_dpp<0x4E>(a1, a2);
        if (lpg >= 8) top2_dpp<0x141>(a1, a2);
        if (lpg >= 16) top2_dpp<0x140>(a1, a2);
        const float gsc = canon(gs >= 2 ? __fadd_rn(unkey(a1), unkey(a2)) : unkey(a1));
        const uint64_t mine = sel_key(gsc, g);
        if (sub == 0) L.gk[g] = mine;
        wave_lds_sync();
        int gr = 0;
        for (int q = 0; q < G; ++q) gr += L.gk[q] > mine;
        const uint64_t ok = __ballot(gr < a.TG);         // lane l: its group is eligible
#pragma unroll
        for (int j = 0; j < J; ++j)
            if (!((ok >> ((lane + 64 * j) / gs * lpg)) & 1ull)) key[j] = 0;
    }
    else if (G > 1)
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
    int mypick;
    float myscore;
    const float vsum = select_topk<J>(key, sc, a.topk, L, mypick, myscore);
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
    if (lane < a.topk && a.sel)          // sel / w null: the picks only (a workgroup that routes for itself)
    {
        const float qv = (a.score_fn != BMX_SCORE_SOFTMAX && !a.renorm) ? myscore : __fdiv_rn(myscore, den);
        a.sel[(size_t)t * a.topk + lane] = (int64_t)mypick + a.first;
        a.w[(size_t)t * a.topk + lane] = f2h_r(__fmul_rn(qv, a.scale));
    }
    return mypick;
}

struct SmallDispatch {
    int shared, rpg;
    bmx_routes r;
};

// Counting sort of at most 256 picks of at most 64 tokens by one wave, without barriers: picks p = lane + 64 i; per
// expert an LDS count and a bit mask of the tokens that picked it (a token picks an expert once, so the picks of an
// expert in pick order are its tokens in order, and a pick's rank among them is the popcount of the mask below its
// token); lane l takes the run of C consecutive experts from l * C (C <= JC: E <= 64 * (JC - 1) plus the shared expert),
// its counts kept in registers; offsets / group bases / unique ranks by one DPP scan of the three run totals. Same
// output as the workgroup version below.
template <int JC>
__device__ void dispatch_wave(const int* pe, int n, int E, int T, int topk, const SmallDispatch& d, int* scnt, int* soff,
                              uint64_t* smask)
{
    const int lane = threadIdx.x & 63, NE = E + (d.shared ? 1 : 0), rpg = d.rpg;
    // groups of a count: ceil(c / rpg), a shift when rpg is a power of two (every path's group size is)
    const bool pow2 = (rpg & (rpg - 1)) == 0;
    const int sh = __builtin_ctz((unsigned)rpg);
    auto ngr = [&](int c) { return pow2 ? (c + rpg - 1) >> sh : (c + rpg - 1) / rpg; };
    int ev[SM_MAXN / 64];
#pragma unroll
    for (int i = 0; i < SM_MAXN / 64; ++i) ev[i] = lane + 64 * i < n ? pe[lane + 64 * i] : -1;
#pragma unroll
    for (int i = 0; i < JC; ++i)
        if (lane + 64 * i < NE)
        {
            scnt[lane + 64 * i] = 0;
            smask[lane + 64 * i] = 0ull;
        }
    wave_lds_sync();
#pragma unroll
    for (int i = 0; i < SM_MAXN / 64; ++i)
        if (ev[i] >= 0)
        {
            atomicAdd(&scnt[ev[i]], 1);
            atomicOr(reinterpret_cast<unsigned long long*>(&smask[ev[i]]), 1ull << ((lane + 64 * i) / topk));
        }
    if (d.shared && lane == 0) scnt[E] = T;
    wave_lds_sync();
    const int C = (NE + 63) / 64, x0 = lane * C;
    int cv[JC];
    int tc = 0, tg = 0, tu = 0;
#pragma unroll
    for (int i = 0; i < JC; ++i)
    {
        cv[i] = (i < C && x0 + i < NE) ? scnt[x0 + i] : 0;
        tc += cv[i];
        tg += ngr(cv[i]);
        tu += cv[i] > 0;
    }
    // one inclusive scan of the three totals packed in 10-bit fields (at most 256 picks and 64 shared rows: every
    // running total stays below 1024)
    const uint32_t inc = wave_scan_add((uint32_t)tc | ((uint32_t)tg << 10) | ((uint32_t)tu << 20));
    const int ic = inc & 1023u, ig = (inc >> 10) & 1023u, iu = inc >> 20;
    int bc = ic - tc, bg = ig - tg, bu = iu - tu;  // exclusive
#pragma unroll
    for (int i = 0; i < JC; ++i)
    {
        const int x = x0 + i, c = cv[i];
        if (i < C && x < NE)
        {
            soff[x] = bc;
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
    wave_lds_sync();
    // rows of the routed picks: stable by (expert, pick)
#pragma unroll
    for (int i = 0; i < SM_MAXN / 64; ++i)
    {
        const int p = lane + 64 * i, e = ev[i];
        if (p >= n) continue;
        if (e < 0)
        {
            d.r.inv[p] = -1;
            continue;
        }
        const int t = p / topk;
        const int row = soff[e] + __builtin_popcountll(smask[e] & ((1ull << t) - 1ull));
        d.r.inv[p] = row;
        d.r.row_token[row] = t;
        d.r.row_slot[row] = p % topk;
        d.r.row_expert[row] = e;
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

// A one-token decode layer's routing handed to its gate / up GEMV, which routes the token itself: the router's and the
// dispatch's arguments and J = ceil(E / 64)
struct RouteFuse {
    RouterArgs ra;
    SmallDispatch sd;
    int J;
};

}  // namespace bmx
