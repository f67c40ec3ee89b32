// Router: one wavefront per token. Scores, optional group limit, top-k and weights, all in registers of one wave;
// selections follow a strict total order (larger choice, then lower index), so they are independent of reduction order.
#include "bmx_common.hpp"
#include "bmx_internal.hpp"

namespace bmx {

constexpr int RT_WAVES = 4;
constexpr int RT_MAXJ = 16;          // experts per lane: E <= 1024
constexpr int RT_MAXG = 64;
constexpr int RT_MAXK = 32;

__device__ __forceinline__ float canon(float v) { return v != v ? -__builtin_huge_valf() : __fadd_rn(v, 0.0f); }

__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) { return va > vb || (va == vb && ia < ib); }

// wave-wide argmax of (v, i) under `better`; idx -1 = none. Every lane returns the winner.
__device__ __forceinline__ void wave_best(float& v, int& i, float& s)
{
#pragma unroll
    for (int m = 1; m < 64; m <<= 1)
    {
        const float ov = __shfl_xor(v, m), os = __shfl_xor(s, m);
        const int oi = __shfl_xor(i, m);
        const bool take = oi >= 0 && (i < 0 || better(ov, oi, v, i));
        if (take) { v = ov; i = oi; s = os; }
    }
}

template <int J>
__global__ __launch_bounds__(RT_WAVES * 64) void k_router(const uint16_t* __restrict__ logits, const float* __restrict__ bias,
                                                          int T, int E, int topk, int G, int TG, int score_fn, int renorm,
                                                          float scale, int64_t first, int64_t* __restrict__ sel,
                                                          uint16_t* __restrict__ wout)
{
    __shared__ float sh_sc[RT_WAVES][J * 64];
    __shared__ float sh_g[RT_WAVES][RT_MAXG];
    __shared__ int sh_idx[RT_WAVES][RT_MAXK];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = blockIdx.x * RT_WAVES + wave;
    if (t >= T) return;
    const uint16_t* lg = logits + (size_t)t * E;
    float sc[J], ch[J];
    float mx = -__builtin_huge_valf();
    if (score_fn == BMX_SCORE_SOFTMAX)
    {
#pragma unroll
        for (int j = 0; j < J; ++j)
        {
            const int e = lane + 64 * j;
            if (e < E) mx = fmaxf(mx, canon(h2f(lg[e])));
        }
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
    }
#pragma unroll
    for (int j = 0; j < J; ++j)
    {
        const int e = lane + 64 * j;
        sc[j] = 0.0f;
        ch[j] = -__builtin_huge_valf();
        if (e < E)
        {
            const float l = canon(h2f(lg[e]));
            if (score_fn == BMX_SCORE_SOFTMAX) { sc[j] = exp_fixed(__fsub_rn(l, mx)); ch[j] = l; }
            else
            {
                sc[j] = sigmoid_fixed(l);
                ch[j] = canon(bias ? __fadd_rn(sc[j], bias[e]) : sc[j]);
            }
            sh_sc[wave][e] = sc[j];
        }
    }
    // group limit: group score = top1 + top2 choice of each group; keep the TG best groups
    uint64_t gmask = ~0ull;
    const int gs = E / G;
    if (G > 1)
    {
        for (int g = 0; g < G; ++g)
        {
            float v1 = 0.0f, s1 = 0.0f;
            int i1 = -1;
#pragma unroll
            for (int j = 0; j < J; ++j)
            {
                const int e = lane + 64 * j;
                if (e >= g * gs && e < (g + 1) * gs && (i1 < 0 || better(ch[j], e, v1, i1))) { v1 = ch[j]; i1 = e; }
            }
            wave_best(v1, i1, s1);
            float v2 = 0.0f, s2 = 0.0f;
            int i2 = -1;
#pragma unroll
            for (int j = 0; j < J; ++j)
            {
                const int e = lane + 64 * j;
                if (e >= g * gs && e < (g + 1) * gs && e != i1 && (i2 < 0 || better(ch[j], e, v2, i2))) { v2 = ch[j]; i2 = e; }
            }
            wave_best(v2, i2, s2);
            if (lane == 0) sh_g[wave][g] = canon(i2 >= 0 ? __fadd_rn(v1, v2) : v1);
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        gmask = 0;
        for (int r = 0; r < TG && r < G; ++r)
        {
            int bg = -1;
            for (int g = 0; g < G; ++g)
                if (!((gmask >> g) & 1ull) && (bg < 0 || better(sh_g[wave][g], g, sh_g[wave][bg], bg))) bg = g;
            gmask |= 1ull << bg;
        }
    }
    // top-k
    uint32_t taken = 0;
    float vsum = 0.0f;
    for (int k = 0; k < topk; ++k)
    {
        float bv = 0.0f, bs = 0.0f;
        int bi = -1;
#pragma unroll
        for (int j = 0; j < J; ++j)
        {
            const int e = lane + 64 * j;
            const bool ok = e < E && !((taken >> j) & 1u) && (G <= 1 || ((gmask >> (e / gs)) & 1ull));
            if (ok && (bi < 0 || better(ch[j], e, bv, bi))) { bv = ch[j]; bi = e; bs = sc[j]; }
        }
        wave_best(bv, bi, bs);
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
        if (lane == 0) sh_idx[wave][k] = bi;
        vsum = __fadd_rn(vsum, bs);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if (lane != 0) return;
    float den = 1.0f;
    if (score_fn == BMX_SCORE_SOFTMAX && !renorm)
    {
        den = 0.0f;
        for (int e = 0; e < E; ++e) den = __fadd_rn(den, sh_sc[wave][e]);
    }
    else if (renorm) den = vsum;
    for (int k = 0; k < topk; ++k)
    {
        const int e = sh_idx[wave][k];
        const float v = sh_sc[wave][e];
        const float q = (score_fn == BMX_SCORE_SIGMOID && !renorm) ? v : __fdiv_rn(v, den);
        sel[(size_t)t * topk + k] = (int64_t)e + first;
        wout[(size_t)t * topk + k] = f2h(__fmul_rn(q, scale));
    }
}

int launch_router(const void* logits, const float* bias, int T, int E, int topk, int n_group, int topk_group,
                  int score_fn, int renorm, float scale, int64_t first, int64_t* sel, void* w, hipStream_t s)
{
    if (T < 0 || E <= 0 || E > RT_MAXJ * 64 || topk <= 0 || topk > RT_MAXK || topk > E)
        return set_error(BMX_ERR_ARG, "bmx_router_topk: unsupported sizes T=%d E=%d topk=%d", T, E, topk);
    if (n_group < 1 || n_group > RT_MAXG || E % n_group || topk_group < 1 || topk_group > n_group)
        return set_error(BMX_ERR_ARG, "bmx_router_topk: bad groups n_group=%d topk_group=%d (E=%d)", n_group, topk_group, E);
    if (n_group > 1 && topk > topk_group * (E / n_group))
        return set_error(BMX_ERR_ARG, "bmx_router_topk: topk %d exceeds the experts of %d groups", topk, topk_group);
    if (score_fn != BMX_SCORE_SOFTMAX && score_fn != BMX_SCORE_SIGMOID)
        return set_error(BMX_ERR_ARG, "bmx_router_topk: unknown score function %d", score_fn);
    if (!logits || !sel || !w) return set_error(BMX_ERR_ARG, "bmx_router_topk: null pointer");
    if (T == 0) return BMX_OK;
    const dim3 grid((T + RT_WAVES - 1) / RT_WAVES), block(RT_WAVES * 64);
    const uint16_t* lg = static_cast<const uint16_t*>(logits);
    uint16_t* wo = static_cast<uint16_t*>(w);
    const int J = (E + 63) / 64;
#define BMX_RT(JJ) hipLaunchKernelGGL(k_router<JJ>, grid, block, 0, s, lg, bias, T, E, topk, n_group, topk_group, score_fn, \
                                      renorm, scale, first, sel, wo)
    if (J <= 1) BMX_RT(1);
    else if (J <= 2) BMX_RT(2);
    else if (J <= 4) BMX_RT(4);
    else if (J <= 8) BMX_RT(8);
    else BMX_RT(16);
#undef BMX_RT
    return check_launch("bmx_router_topk");
}

}  // namespace bmx
