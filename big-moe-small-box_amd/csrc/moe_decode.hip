// Decode-size expert products: bandwidth-bound grouped GEMVs over EXL3 trellis weights decoded in registers.
//
// Work unit = (group of <= MR rows of one expert, 128-column block, k-split). Each workgroup (4 waves) streams the
// trellis tiles of its k-range once, coalesced: half a wave reads one tile-row of 8 tiles (8 x 32 K contiguous bytes),
// four lanes per tile, 64 weights per lane. A lane's 64 weights are 4 output columns x 16 rows, so the only reductions
// are the two half-waves, the four waves (LDS) and the k-splits (workspace partials summed in split order by the last
// workgroup to arrive). All sums happen in a fixed order: results do not depend on scheduling.
//
//   k_gu  : x rows -> input rotation (per matrix suh) -> gate / up GEMV -> fp16 -> epilogue (rotation * svh, activation,
//           * down suh, rotation) -> fp16 down input rows              (exllamav3 kernel A, docs/x16.md:38-54)
//   k_dn  : down input rows -> down GEMV -> fp32 -> rotation * svh -> expert output rows; the last workgroup of each
//           128-column block then sums every token's slots in slot order (+ shared expert)   (x16_red_k order)
#include "bmx_common.hpp"
#include "bmx_internal.hpp"

#include <stdlib.h>

namespace bmx {

constexpr int GV_WAVES = 4;
constexpr int GV_THREADS = GV_WAVES * 64;
constexpr int GV_LDS_X = 32768;       // bytes of staged input rows per workgroup

struct GvArgs {
    const bmx_expert* experts;
    const bmx_expert* shared;
    int E, H, I, act, gated;
    float limit;
    const uint16_t* x;
    const int32_t* row_token;
    const int32_t* groups;
    const int32_t* ngroups;
    uint16_t* act_rows;
    float* y_rows;
    float* part_gu;
    float* part_dn;
    int32_t* cnt_gu;
    int32_t* cnt_dn;
    int32_t* cnt_cb;
    int KS_gu, KS_dn, NB, NBH, R_max;
    float* out;
    const uint16_t* w;
    const int32_t* inv;
    const int32_t* offsets;
    int T, topk, has_shared;
};

template <int F> struct RingTab {
    int q[64];
    constexpr RingTab() : q()
    {
        for (int i = 0; i < 64; ++i) q[i] = ring_end<F>(i) + 16;
    }
};

// 16-bit state at bit Q of a lane's window (MSB-first words); bits above 15 of the result are left as they are
template <int NW1>
__device__ __forceinline__ uint32_t win_state(const uint32_t (&W)[NW1], int q)
{
    const int d = q >> 5, o = q & 31;
    if (o <= 16) return W[d] >> (16 - o);
    return __builtin_amdgcn_alignbit(W[d], W[d + 1], 48 - o);
}

// One tile-row strip for this lane: 64 weights (stream positions 64 s .. 64 s + 63 of its tile) decoded and multiplied
// with MR token rows. xr: LDS fp16 pairs of the strip's 16 input rows, 8 dwords per token row, token stride xstride.
template <int F, int MR>
__device__ __forceinline__ void strip(const uint32_t (&W)[Fmt<F>::TB / 16 + 1], const uint32_t* xr, int xstride,
                                      float (&acc)[4][MR], uint32_t ones)
{
    constexpr RingTab<F> tab;
    uint32_t X[MR][8];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int d = 0; d < 8; ++d) X[m][d] = xr[m * xstride + d];
#pragma unroll
    for (int jj = 0; jj < 64; jj += 2)
    {
        const uint32_t i0 = cb_index(win_state(W, tab.q[jj]), ones);
        const uint32_t i1 = cb_index(win_state(W, tab.q[jj + 1]), ones);
        const f16x2 w2 = cb_weights(i0, i1);
        const int gg = jj >> 3, j = jj & 7;
        const int cidx = (gg >> 2) + (j >= 4 ? 2 : 0);
        const int dw = (gg & 3) + ((j & 2) ? 4 : 0);
#pragma unroll
        for (int m = 0; m < MR; ++m)
            acc[cidx][m] = __builtin_amdgcn_fdot2(w2, __builtin_bit_cast(f16x2, X[m][dw]), acc[cidx][m], false);
    }
}

// A wave's GEMV over tile-rows [tr0, tr0 + ntr) (ntr even; the two half-waves take alternate rows) of the 128-column
// block cb of a matrix with tn tiles per row. xs: LDS input rows, dword (tr - xtr0) * 8 of each token row.
template <int F, int MR>
__device__ __forceinline__ void gemv_wave(const uint8_t* __restrict__ mat, int tn, int cb, int tr0, int ntr,
                                          const uint32_t* xs, int xstride, int xtr0, float (&acc)[4][MR])
{
    constexpr int TB = Fmt<F>::TB, NW = TB / 16;
    const int lane = threadIdx.x & 63, h = lane >> 5, t = (lane >> 2) & 7, s = lane & 3;
    const uint32_t ones = 0x01010101u;
    const size_t row_bytes = (size_t)tn * TB;
    const uint8_t* p = mat + (size_t)(tr0 + h) * row_bytes + (size_t)(cb * 8 + t) * TB + s * (TB / 4);
    uint32_t Wn[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) Wn[i] = ldg_nt(p, i);
    for (int it = 0; it < ntr; it += 2)
    {
        uint32_t W[NW + 1];
#pragma unroll
        for (int i = 0; i < NW; ++i) W[i + 1] = Wn[i];
        W[0] = __builtin_amdgcn_mov_dpp(W[NW], 0x93, 0xf, 0xf, false);   // quad_perm [3,0,1,2]: previous lane's last word
        if (it + 2 < ntr)
        {
            p += 2 * row_bytes;
#pragma unroll
            for (int i = 0; i < NW; ++i) Wn[i] = ldg_nt(p, i);
        }
        strip<F, MR>(W, xs + (tr0 + it + h - xtr0) * 8, xstride, acc, ones);
    }
}

template <int MR>
__device__ __forceinline__ void gemv_any(int fmt, const uint8_t* mat, int tn, int cb, int tr0, int ntr,
                                         const uint32_t* xs, int xstride, int xtr0, float (&acc)[4][MR])
{
    switch (fmt)
    {
        case BMX_TF_K2: gemv_wave<BMX_TF_K2, MR>(mat, tn, cb, tr0, ntr, xs, xstride, xtr0, acc); break;
        case BMX_TF_K25: gemv_wave<BMX_TF_K25, MR>(mat, tn, cb, tr0, ntr, xs, xstride, xtr0, acc); break;
        case BMX_TF_K3: gemv_wave<BMX_TF_K3, MR>(mat, tn, cb, tr0, ntr, xs, xstride, xtr0, acc); break;
        default: gemv_wave<BMX_TF_K4, MR>(mat, tn, cb, tr0, ntr, xs, xstride, xtr0, acc); break;
    }
}

// lane's 4 columns inside the 128-column block
__device__ __forceinline__ int lane_col(int lane, int c)
{
    const int t = (lane >> 2) & 7, s = lane & 3;
    return t * 16 + 2 * s + (c & 1) + ((c & 2) ? 8 : 0);
}

__device__ __forceinline__ float ld_agent(const float* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sum the four waves' partials (red [NM][GV_WAVES][MR][128]) into red[m][0], then, with k-splits, publish the partial
// and let the last workgroup to arrive sum all splits in split order into red[..][0]. Returns false for the others.
template <int MR, int NM>
__device__ bool reduce_splits(float* red, int nr, int KS, int ks, float* part, size_t part_row_stride,
                              size_t part_split_stride, int32_t* counter)
{
    __shared__ int sh_last;
    for (int i = threadIdx.x; i < NM * MR * 128; i += GV_THREADS)
    {
        const int mat = i / (MR * 128), rem = i % (MR * 128);
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < GV_WAVES; ++w) s = s + red[(mat * GV_WAVES + w) * MR * 128 + rem];
        red[(mat * GV_WAVES) * MR * 128 + rem] = s;
    }
    __syncthreads();
    if (KS == 1) return true;
    for (int i = threadIdx.x; i < NM * MR * 128; i += GV_THREADS)
    {
        const int mat = i / (MR * 128), m = (i / 128) % MR, c = i % 128;
        if (m < nr) part[ks * part_split_stride + m * part_row_stride + mat * 128 + c] = red[(mat * GV_WAVES) * MR * 128 + m * 128 + c];
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0)
    {
        const int prev = atomicAdd(counter, 1);
        sh_last = prev == KS - 1;
        if (sh_last) *counter = 0;
    }
    __syncthreads();
    if (!sh_last) return false;
    __threadfence();
    for (int i = threadIdx.x; i < NM * MR * 128; i += GV_THREADS)
    {
        const int mat = i / (MR * 128), m = (i / 128) % MR, c = i % 128;
        if (m >= nr) continue;
        float s = 0.0f;
        for (int q = 0; q < KS; ++q) s = s + ld_agent(part + q * part_split_stride + m * part_row_stride + mat * 128 + c);
        red[(mat * GV_WAVES) * MR * 128 + m * 128 + c] = s;
    }
    __syncthreads();
    return true;
}

// ---- gate / up + epilogue ----------------------------------------------------------------------------------------------
template <int MR>
__global__ __launch_bounds__(GV_THREADS) void k_gu(GvArgs a)
{
    extern __shared__ uint32_t smem[];
    int bid = blockIdx.x;
    const int KS = a.KS_gu, NB = a.NB;
    const int ks = bid % KS;
    bid /= KS;
    const int cb = bid % NB, g = bid / NB;
    if (g >= *a.ngroups) return;
    const int e = a.groups[3 * g], r0 = a.groups[3 * g + 1], nr = a.groups[3 * g + 2];
    const bmx_expert& ex = e == a.E ? *a.shared : a.experts[e];
    const int KR = a.H / KS, k0 = ks * KR, XW = KR / 2;
    uint32_t* xs = smem;                                           // [2][MR][KR / 2]
    float* red = reinterpret_cast<float*>(smem + 2 * MR * XW);     // [2][GV_WAVES][MR][128]
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;

    // input rotation of each token row for gate and up: xt = RN16(H128(x * suh) * R)
    const int nblk = KR / 128;
    for (int u = wave; u < 2 * MR * nblk; u += GV_WAVES)
    {
        const int mat = u / (MR * nblk), rem = u % (MR * nblk), m = rem / nblk, b = rem % nblk;
        uint32_t val = 0;
        if (m < nr)
        {
            const int tok = a.row_token[r0 + m];
            const int k = k0 + b * 128 + 2 * lane;
            const uint32_t xv = ldg(a.x + (size_t)tok * a.H + k, 0);
            const uint32_t sv = ldg(reinterpret_cast<const uint16_t*>(ex.suh[mat]) + k, 0);
            float v0 = h2f(xv & 0xffffu) * h2f(sv & 0xffffu), v1 = h2f(xv >> 16) * h2f(sv >> 16);
            had128_wave(v0, v1);
            val = (uint32_t)f2h(v0 * R_SCALE) | ((uint32_t)f2h(v1 * R_SCALE) << 16);
        }
        xs[(mat * MR + m) * XW + b * 64 + lane] = val;
    }
    __syncthreads();

    const int TRW = KR / 16 / GV_WAVES;
    const int tr0 = k0 / 16 + wave * TRW;
#pragma unroll
    for (int mat = 0; mat < 2; ++mat)
    {
        float acc[4][MR];
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int m = 0; m < MR; ++m) acc[c][m] = 0.0f;
        gemv_any<MR>(ex.fmt[mat], reinterpret_cast<const uint8_t*>(ex.tr[mat]), a.I / 16, cb, tr0, TRW,
                     xs + mat * MR * XW, XW, k0 / 16, acc);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int m = 0; m < MR; ++m) acc[c][m] = acc[c][m] + __shfl_xor(acc[c][m], 32);
        if (lane < 32)
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int m = 0; m < MR; ++m) red[((mat * GV_WAVES + wave) * MR + m) * 128 + lane_col(lane, c)] = acc[c][m];
    }
    __syncthreads();
    const size_t prs = (size_t)a.NB * 256, pss = (size_t)a.R_max * prs;
    if (!reduce_splits<MR, 2>(red, nr, KS, ks, a.part_gu + (size_t)r0 * prs + (size_t)cb * 256, prs, pss,
                              a.cnt_gu + g * NB + cb))
        return;

    // epilogue: one wave per token row, lane l holds columns 2l, 2l + 1
    const int col = cb * 128 + 2 * lane;
    const uint32_t svg = ldg(reinterpret_cast<const uint16_t*>(ex.svh[0]) + col, 0);
    const uint32_t svu = ldg(reinterpret_cast<const uint16_t*>(ex.svh[1]) + col, 0);
    const uint32_t sud = ldg(reinterpret_cast<const uint16_t*>(ex.suh[2]) + col, 0);
    for (int m = wave; m < nr; m += GV_WAVES)
    {
        const float* rg = red + (0 * GV_WAVES) * MR * 128 + m * 128;
        const float* ru = red + (1 * GV_WAVES) * MR * 128 + m * 128;
        float g0 = h2f(f2h(rg[2 * lane])), g1 = h2f(f2h(rg[2 * lane + 1]));
        float u0 = h2f(f2h(ru[2 * lane])), u1 = h2f(f2h(ru[2 * lane + 1]));
        had128_wave(g0, g1);
        had128_wave(u0, u1);
        g0 = (g0 * R_SCALE) * h2f(svg & 0xffffu);
        g1 = (g1 * R_SCALE) * h2f(svg >> 16);
        u0 = (u0 * R_SCALE) * h2f(svu & 0xffffu);
        u1 = (u1 * R_SCALE) * h2f(svu >> 16);
        float a0 = act_gate(a.act, a.gated, g0, u0, a.limit) * h2f(sud & 0xffffu);
        float a1 = act_gate(a.act, a.gated, g1, u1, a.limit) * h2f(sud >> 16);
        had128_wave(a0, a1);
        const uint32_t pk = (uint32_t)f2h(a0 * R_SCALE) | ((uint32_t)f2h(a1 * R_SCALE) << 16);
        *reinterpret_cast<uint32_t*>(a.act_rows + (size_t)(r0 + m) * a.I + col) = pk;
    }
}

// ---- down + output rotation + combine -------------------------------------------------------------------------------
template <int MR>
__global__ __launch_bounds__(GV_THREADS) void k_dn(GvArgs a)
{
    extern __shared__ uint32_t smem[];
    __shared__ int sh_last;
    int bid = blockIdx.x;
    const int KS = a.KS_dn, NBH = a.NBH;
    const int ks = bid % KS;
    bid /= KS;
    const int cb = bid % NBH, g = bid / NBH;
    const int ng = *a.ngroups;
    if (g >= ng) return;
    const int e = a.groups[3 * g], r0 = a.groups[3 * g + 1], nr = a.groups[3 * g + 2];
    const bmx_expert& ex = e == a.E ? *a.shared : a.experts[e];
    const int KR = a.I / KS, k0 = ks * KR, XW = KR / 2;
    uint32_t* xs = smem;                                           // [MR][KR / 2]
    float* red = reinterpret_cast<float*>(smem + MR * XW);         // [GV_WAVES][MR][128]
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int i = threadIdx.x; i < MR * XW; i += GV_THREADS)
    {
        const int m = i / XW, d = i % XW;
        xs[i] = m < nr ? *reinterpret_cast<const uint32_t*>(a.act_rows + (size_t)(r0 + m) * a.I + k0 + 2 * d) : 0u;
    }
    __syncthreads();
    const int TRW = KR / 16 / GV_WAVES;
    const int tr0 = k0 / 16 + wave * TRW;
    float acc[4][MR];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[c][m] = 0.0f;
    gemv_any<MR>(ex.fmt[2], reinterpret_cast<const uint8_t*>(ex.tr[2]), a.H / 16, cb, tr0, TRW, xs, XW, k0 / 16, acc);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[c][m] = acc[c][m] + __shfl_xor(acc[c][m], 32);
    if (lane < 32)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int m = 0; m < MR; ++m) red[(wave * MR + m) * 128 + lane_col(lane, c)] = acc[c][m];
    __syncthreads();
    const size_t prs = (size_t)a.NBH * 128, pss = (size_t)a.R_max * prs;
    if (!reduce_splits<MR, 1>(red, nr, KS, ks, a.part_dn + (size_t)r0 * prs + (size_t)cb * 128, prs, pss,
                              a.cnt_dn + g * NBH + cb))
        return;

    const int col = cb * 128 + 2 * lane;
    const uint32_t svd = ldg(reinterpret_cast<const uint16_t*>(ex.svh[2]) + col, 0);
    for (int m = wave; m < nr; m += GV_WAVES)
    {
        float v0 = red[m * 128 + 2 * lane], v1 = red[m * 128 + 2 * lane + 1];
        had128_wave(v0, v1);
        v0 = (v0 * R_SCALE) * h2f(svd & 0xffffu);
        v1 = (v1 * R_SCALE) * h2f(svd >> 16);
        float* yr = a.y_rows + (size_t)(r0 + m) * a.H + col;
        yr[0] = v0;
        yr[1] = v1;
    }
    if (!a.out) return;

    // combine: the last of the column block's workgroups sums every token's slots in slot order, then the shared row
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0)
    {
        const int prev = atomicAdd(a.cnt_cb + cb, 1);
        sh_last = prev == ng - 1;
        if (sh_last) a.cnt_cb[cb] = 0;
    }
    __syncthreads();
    if (!sh_last) return;
    __threadfence();
    for (int i = threadIdx.x; i < a.T * 128; i += GV_THREADS)
    {
        const int t = i / 128, h = cb * 128 + (i % 128);
        float o = 0.0f;
        for (int k = 0; k < a.topk; ++k)
        {
            const int r = a.inv[t * a.topk + k];
            const float wk = h2f(a.w[t * a.topk + k]);
            if (r < 0 || wk == 0.0f) continue;
            const float p = wk * ld_agent(a.y_rows + (size_t)r * a.H + h);
            o = o + p;
        }
        if (a.has_shared) o = o + ld_agent(a.y_rows + (size_t)(a.offsets[a.E] + t) * a.H + h);
        a.out[(size_t)t * a.H + h] = o;
    }
}

// ---- standalone combine ----------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_combine(const float* __restrict__ y, const int32_t* __restrict__ inv,
                                                 const uint16_t* __restrict__ w, const int32_t* __restrict__ offsets,
                                                 int T, int topk, int H, int E, int has_shared, float* __restrict__ out)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)T * H) return;
    const int t = (int)(i / H), h = (int)(i % H);
    float o = 0.0f;
    for (int k = 0; k < topk; ++k)
    {
        const int r = inv[t * topk + k];
        const float wk = h2f(w[t * topk + k]);
        if (r < 0 || wk == 0.0f) continue;
        const float p = wk * y[(size_t)r * H + h];
        o = o + p;
    }
    if (has_shared) o = o + y[(size_t)(offsets[E] + t) * H + h];
    out[i] = o;
}

__global__ void k_zero_i32(int32_t* p, int n)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0;
}

int launch_zero_i32(int32_t* p, int n, hipStream_t s)
{
    if (n <= 0) return BMX_OK;
    hipLaunchKernelGGL(k_zero_i32, dim3((n + 255) / 256), dim3(256), 0, s, p, n);
    return check_launch("zero");
}

int launch_combine(const float* y_rows, const int32_t* inv, const void* w, const int32_t* offsets, int T, int topk,
                   int H, int E, int has_shared, float* out, hipStream_t s)
{
    if (T <= 0) return BMX_OK;
    const size_t n = (size_t)T * H;
    hipLaunchKernelGGL(k_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, y_rows, inv,
                       static_cast<const uint16_t*>(w), offsets, T, topk, H, E, has_shared, out);
    return check_launch("bmx_combine");
}

// ---- plan ------------------------------------------------------------------------------------------------------------
static int rows_per_group_of(int T) { return T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : 8; }

// smallest divisor d of nblk128 (so the k-range stays a whole number of 128-blocks) reaching `target` workgroups
static int pick_split(int nblk128, int units, int target, int maxks, const char* env)
{
    const char* v = getenv(env);
    if (v && *v)
    {
        const int ks = atoi(v);
        if (ks >= 1 && nblk128 % ks == 0) return ks;
    }
    int best = 1;
    for (int d = 1; d <= nblk128 && d <= maxks; ++d)
    {
        if (nblk128 % d) continue;
        best = d;
        if ((long)units * d >= target) break;
    }
    return best;
}

DecodePlan decode_plan(const MoeShape& m)
{
    DecodePlan p;
    const int MR = rows_per_group_of(m.T);
    p.NB = m.I / 128;
    p.NBH = m.H / 128;
    p.G_max = groups_max(m.T, m.topk, m.E, m.shared, MR);
    p.R_max = m.T * m.topk + (m.shared ? m.T : 0);
    const long uniq = (long)m.T * m.topk + (m.shared ? 1 : 0) < (long)m.E + (m.shared ? 1 : 0)
                          ? (long)m.T * m.topk + (m.shared ? 1 : 0)
                          : (long)m.E + (m.shared ? 1 : 0);
    const long est = uniq + (long)(m.T > MR ? (m.T * m.topk) / (MR * 4) : 0);
    // the staged input rows (2 matrices x MR rows x k-range fp16) must fit GV_LDS_X
    const int max_kr_gu = GV_LDS_X / (2 * MR * 2), max_kr_dn = GV_LDS_X / (MR * 2);
    int ks = pick_split(m.H / 128, (int)(est * p.NB), 1024, m.H / 128, "BMX_KS_GU");
    while (m.H / ks > max_kr_gu) { int d = ks + 1; while ((m.H / 128) % d) ++d; ks = d; }
    p.KS_gu = ks;
    ks = pick_split(m.I / 128, (int)(est * p.NBH), 1024, m.I / 128, "BMX_KS_DN");
    while (m.I / ks > max_kr_dn) { int d = ks + 1; while ((m.I / 128) % d) ++d; ks = d; }
    p.KS_dn = ks;
    p.part_gu_bytes = p.KS_gu > 1 ? (size_t)p.KS_gu * p.R_max * p.NB * 256 * 4 : 0;
    p.part_dn_bytes = p.KS_dn > 1 ? (size_t)p.KS_dn * p.R_max * p.NBH * 128 * 4 : 0;
    p.counters = (size_t)p.G_max * (p.NB + p.NBH) + p.NBH;
    return p;
}

size_t decode_ws_bytes(const MoeShape& m)
{
    const DecodePlan p = decode_plan(m);
    return align_up(p.counters * 4, 256) + align_up(p.part_gu_bytes, 256) + align_up(p.part_dn_bytes, 256) +
           align_up((size_t)p.R_max * m.I * 2, 256);
}

template <int MR>
static void launch_mr(const GvArgs& a, const DecodePlan& p, int stages, hipStream_t s)
{
    const size_t lds_gu = (size_t)2 * MR * (a.H / p.KS_gu) / 2 * 4 + (size_t)2 * GV_WAVES * MR * 128 * 4;
    const size_t lds_dn = (size_t)MR * (a.I / p.KS_dn) / 2 * 4 + (size_t)GV_WAVES * MR * 128 * 4;
    if (stages & 1) hipLaunchKernelGGL(k_gu<MR>, dim3((unsigned)(p.G_max * p.NB * p.KS_gu)), dim3(GV_THREADS), lds_gu, s, a);
    if (stages & 2) hipLaunchKernelGGL(k_dn<MR>, dim3((unsigned)(p.G_max * p.NBH * p.KS_dn)), dim3(GV_THREADS), lds_dn, s, a);
}

int launch_decode_experts(const MoeShape& m, const void* x, const bmx_routes* r, float* y_rows, void* act_rows,
                          void* ws, size_t ws_bytes, float* combine_out, const void* combine_w, hipStream_t s,
                          bool counters_zeroed, int stages)
{
    if (m.H % 128 || m.I % 128 || m.H <= 0 || m.I <= 0)
        return set_error(BMX_ERR_ARG, "moe experts: H (%d) and I (%d) must be multiples of 128", m.H, m.I);
    const DecodePlan p = decode_plan(m);
    if (ws_bytes < decode_ws_bytes(m))
        return set_error(BMX_ERR_WORKSPACE, "moe experts: workspace %zu < %zu", ws_bytes, decode_ws_bytes(m));
    char* w = static_cast<char*>(ws);
    GvArgs a;
    a.experts = m.experts; a.shared = m.shared_ex; a.E = m.E; a.H = m.H; a.I = m.I; a.act = m.act; a.gated = m.gated;
    a.limit = m.limit;
    a.x = static_cast<const uint16_t*>(x);
    a.row_token = r->row_token; a.groups = r->groups; a.ngroups = r->ngroups;
    a.cnt_gu = reinterpret_cast<int32_t*>(w);
    a.cnt_dn = a.cnt_gu + (size_t)p.G_max * p.NB;
    a.cnt_cb = a.cnt_dn + (size_t)p.G_max * p.NBH;
    w += align_up(p.counters * 4, 256);
    a.part_gu = reinterpret_cast<float*>(w);
    w += align_up(p.part_gu_bytes, 256);
    a.part_dn = reinterpret_cast<float*>(w);
    w += align_up(p.part_dn_bytes, 256);
    a.act_rows = act_rows ? static_cast<uint16_t*>(act_rows) : reinterpret_cast<uint16_t*>(w);
    a.y_rows = y_rows;
    a.KS_gu = p.KS_gu; a.KS_dn = p.KS_dn; a.NB = p.NB; a.NBH = p.NBH; a.R_max = p.R_max;
    a.out = combine_out; a.w = static_cast<const uint16_t*>(combine_w); a.inv = r->inv; a.offsets = r->offsets;
    a.T = m.T; a.topk = m.topk; a.has_shared = m.shared;
    if (!counters_zeroed && (stages & 1))
    {
        const int rc = launch_zero_i32(a.cnt_gu, (int)p.counters, s);
        if (rc) return rc;
    }
    switch (rows_per_group_of(m.T))
    {
        case 1: launch_mr<1>(a, p, stages, s); break;
        case 2: launch_mr<2>(a, p, stages, s); break;
        case 4: launch_mr<4>(a, p, stages, s); break;
        default: launch_mr<8>(a, p, stages, s); break;
    }
    return check_launch("moe experts (decode path)");
}

int decode_rows_per_group(int T) { return rows_per_group_of(T); }

}  // namespace bmx
