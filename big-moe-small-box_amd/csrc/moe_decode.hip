// Decode-size expert products: bandwidth-bound grouped GEMVs over EXL3 trellis weights decoded in registers.
//
// Work unit = (group of <= MR rows of one expert, 128-column block, k-split). Each workgroup (4 waves) streams the
// trellis tiles of its k-range once, coalesced: half a wave reads one tile-row of 8 tiles (8 x 32 K contiguous bytes),
// four lanes per tile, 64 weights per lane. A lane's 64 weights are 4 output columns x 16 rows, so the only reductions
// are the two half-waves, the four waves (LDS) and the k-splits (workspace partials summed in split order by the next
// kernel). All sums happen in a fixed order: results do not depend on scheduling.
//
//   k_gemv_part<MR, 2> : x rows -> input rotation (per matrix suh) -> gate / up split-K partial sums
//   k_gu_epi           : splits summed in order -> fp16 gate / up -> epilogue (rotation * svh, activation, * down suh,
//                        rotation) -> fp16 down-input rows                 (exllamav3 kernel A, docs/x16.md:38-54)
//   k_gemv_part<MR, 1> : down-input rows -> down split-K partial sums
//   k_dn_combine       : splits summed in order -> rotation * svh -> every token's slots summed in slot order, + the
//                        shared expert                                     (exllamav3 kernel B, x16_red_k order)
// The kernels hand data over only at kernel boundaries (no inter-workgroup flags or fences inside a kernel).
#include "moe_kernels.hpp"
#include "router_wave.hpp"

#include <stdlib.h>

#include <algorithm>
#include <atomic>

namespace bmx {

constexpr int GV_WAVES = 4;
constexpr int GV_THREADS = GV_WAVES * 64;
constexpr int GV_LDS_X = 32768;       // bytes of staged input rows per workgroup

// One tile-row strip for this lane: 64 weights (stream positions 64 s .. 64 s + 63 of its tile) decoded and multiplied
// with MR token rows. xr: LDS fp16 pairs of the strip's 16 input rows, 8 dwords per token row, token stride xstride.
template <int F, int MR>
__device__ __forceinline__ void strip(const uint32_t (&own)[Fmt<F>::TB / 16], const uint32_t* xr, int xstride,
                                      float (&acc)[4][MR])
{
    constexpr int NW = Fmt<F>::TB / 16;
    // previous lane's last word (quad_perm [3,0,1,2]: lane 0 of the tile takes lane 3's, the ring wraps)
    const uint32_t prev = __builtin_amdgcn_mov_dpp(own[NW - 1], 0x93, 0xf, 0xf, false);
    uint32_t X[MR][8];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int d = 0; d < 8; ++d) X[m][d] = xr[m * xstride + d];
#pragma unroll
    for (int j8 = 0; j8 < 64; j8 += 8)
    {
        uint32_t w[4];
        oct_weights<F>(prev, own, j8, w);
#pragma unroll
        for (int q = 0; q < 4; ++q)
        {
            const int cidx = strip_cidx(j8 + 2 * q), dw = strip_dw(j8 + 2 * q);
#pragma unroll
            for (int m = 0; m < MR; ++m)
                acc[cidx][m] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w[q]), __builtin_bit_cast(f16x2, X[m][dw]),
                                                      acc[cidx][m], false);
        }
    }
}

template <int F, int MR>
__device__ __forceinline__ void gemv_wave_from(const uint8_t* p, size_t row_bytes, uint32_t (&wa)[Fmt<F>::TB / 16],
                                               int ntr, const uint32_t* xb, int xstride, float (&acc)[4][MR]);

// A wave's GEMV over tile-rows [tr0, tr0 + ntr) (ntr even; the two half-waves take alternate rows) of the 128-column
// block cb of a matrix with tn tiles per row. xs: LDS input rows, dword (tr - xtr0) * 8 of each token row. Two register
// sets alternate so the next strip's words are in flight while the current one is decoded.
template <int F, int MR>
__device__ __forceinline__ void gemv_wave(const uint8_t* __restrict__ mat, int tn, int cb, int tr0, int ntr,
                                          const uint32_t* xs, int xstride, int xtr0, float (&acc)[4][MR])
{
    constexpr int TB = Fmt<F>::TB, NW = TB / 16;
    const int lane = threadIdx.x & 63, h = lane >> 5, t = (lane >> 2) & 7, s = lane & 3;
    const size_t row_bytes = (size_t)tn * TB;
    const uint8_t* p = mat + (size_t)(tr0 + h) * row_bytes + (size_t)(cb * 8 + t) * TB + s * (TB / 4);
    uint32_t wa[NW];
    load_words(wa, p);
    gemv_wave_from<F, MR>(p, row_bytes, wa, ntr, xs + (tr0 + h - xtr0) * 8, xstride, acc);
}

// The loop of gemv_wave from the lane's first words wa (already requested, at p)
template <int F, int MR>
__device__ __forceinline__ void gemv_wave_from(const uint8_t* p, size_t row_bytes, uint32_t (&wa)[Fmt<F>::TB / 16],
                                               int ntr, const uint32_t* xb, int xstride, float (&acc)[4][MR])
{
    constexpr int NW = Fmt<F>::TB / 16;
    uint32_t wb[NW];
    int it = 0;
    for (; it + 4 <= ntr; it += 4)
    {
        load_words(wb, p + 2 * row_bytes);
        strip<F, MR>(wa, xb + it * 8, xstride, acc);
        p += 4 * row_bytes;
        if (it + 4 < ntr) load_words(wa, p);
        strip<F, MR>(wb, xb + (it + 2) * 8, xstride, acc);
    }
    if (it < ntr) strip<F, MR>(wa, xb + it * 8, xstride, acc);
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

template <int B>
__device__ __forceinline__ void gu_epi_wave(const GvArgs& a, int r, int cb, uint16_t* dst);
// ---- split-K grouped GEMV -> partial sums ------------------------------------------------------------------------------
// NM = 2: gate and up of the same expert on rotated x rows (the rotation is computed here, per matrix suh); waves 0-1
// take gate and waves 2-3 up, each half of the k-range, so a wave runs one format's code. NM = 1: down on the rotated
// fp16 down-input rows, the four waves a quarter of the k-range each. part[ks][row][cb][mat][128] (mat stride 128, cb
// stride NM * 128). MX: the most rows a group can hold (LDS layout); the GEMV itself runs with the group's own row count
// rounded up to 1, 2, 4 or 8, so a one-token group costs one row of dot products whatever the batch.
constexpr int GV_WPM = GV_WAVES / 2;      // waves per matrix of the gate / up GEMV
template <int MR, int MX, int NM>
__device__ __forceinline__ void gemv_rows(const GvArgs& a, const bmx_expert& ex, int cb, int k0, int KR, int N,
                                          const uint32_t* xs, float* red)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, XW = KR / 2;
    const int WPM = NM == 2 ? GV_WPM : GV_WAVES;           // waves sharing a matrix's k-range
    const int mat = NM == 2 ? wave / GV_WPM : 0, sub = NM == 2 ? wave % GV_WPM : wave;
    const int mi = NM == 2 ? mat : 2;
    const int TRW = KR / 16 / WPM;
    const int tr0 = k0 / 16 + sub * TRW;
    float acc[4][MR];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[c][m] = 0.0f;
    gemv_any<MR>(ex.fmt[mi], reinterpret_cast<const uint8_t*>(ex.tr[mi]), N / 16, cb, tr0, TRW, xs + mat * MX * XW, XW,
                 k0 / 16, acc);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[c][m] = acc[c][m] + xor32_f(acc[c][m]);
    if (lane < 32)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int m = 0; m < MR; ++m) red[(wave * MX + m) * 128 + lane_col(lane, c)] = acc[c][m];
}

// The one-row down GEMV's staging and products (k_gemv_part<1, 1>, input rows from act_rows): the loads of the row's
// k-range are issued first, then each lane's first trellis words (they need the expert record only), and only then is
// the row stored to LDS, so the words' latency runs beside the staging's instead of after the barrier (C2 one-token
// layer 53.02 -> 52.91 us, paired runs). Same products, same order as staging then gemv_rows<1, 1, 1>. XW <= 4 *
// GV_THREADS (checked by the caller).
template <int F>
__device__ __forceinline__ void down1_rows(const GvArgs& a, const bmx_expert& ex, int cb, int k0, int KR, int r0,
                                           uint32_t* xs, float* red)
{
    constexpr int TB = Fmt<F>::TB, NW = TB / 16;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, XW = KR / 2;
    uint32_t xv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int d = threadIdx.x + i * GV_THREADS;
        xv[i] = d < XW ? ldg(a.act_rows + (size_t)r0 * a.I + k0 + 2 * d, 0) : 0u;
    }
    const int TRW = KR / 16 / GV_WAVES, tr0 = k0 / 16 + wave * TRW;
    const int h = lane >> 5, t = (lane >> 2) & 7, s = lane & 3;
    const size_t row_bytes = (size_t)(a.H / 16) * TB;
    const uint8_t* p = reinterpret_cast<const uint8_t*>(ex.tr[2]) + (size_t)(tr0 + h) * row_bytes +
                       (size_t)(cb * 8 + t) * TB + s * (TB / 4);
    uint32_t wa[NW];
    load_words(wa, p);
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int d = threadIdx.x + i * GV_THREADS;
        if (d < XW) xs[d] = xv[i];
    }
    lds_barrier();
    float acc[4][1];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c][0] = 0.0f;
    gemv_wave_from<F, 1>(p, row_bytes, wa, TRW, xs + (tr0 + h - k0 / 16) * 8, XW, acc);
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c][0] = acc[c][0] + xor32_f(acc[c][0]);
    if (lane < 32)
#pragma unroll
        for (int c = 0; c < 4; ++c) red[wave * 128 + lane_col(lane, c)] = acc[c][0];
}

// One work unit (k-split ks, column block cb of a group: expert e, rows r0 .. r0 + nr - 1) of the split-K GEMV. tok1 >= 0:
// the rows' token (a one-token call whose dispatch is being written by another workgroup), else from row_token.
template <int MX, int NM>
__device__ __forceinline__ void gemv_unit(const GvArgs& a, int ks, int cb, int e, int r0, int nr, int tok1)
{
    extern __shared__ uint32_t smem[];
    const int NB = NM == 2 ? a.NB : a.NBH;
    const int KS = NM == 2 ? a.KS_gu : a.KS_dn;
    const bmx_expert& ex = e == a.E ? *a.shared : a.experts[e];
    const int K = NM == 2 ? a.H : a.I, N = NM == 2 ? a.I : a.H;
    const int KR = K / KS, k0 = ks * KR, XW = KR / 2;
    uint32_t* xs = smem;                                           // [NM][MX][KR / 2] fp16 pairs
    float* red = reinterpret_cast<float*>(smem + NM * MX * XW);    // [GV_WAVES][MX][128] (gate / up: waves 0-1 gate)
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    bool pre = false;                  // the one-row down GEMV ran its staging and products itself (down1_rows)

    if (NM == 2)
    {
        // input rotation of each token row for gate and up: xt = RN16(H128(x * suh) * R)
        // units (matrix, row, 128-block) in turn over the waves (counted, not divided: the index math stays scalar)
        const int nblk = KR / 128;
        int u = 0;
        for (int mat = 0; mat < 2; ++mat)
            for (int m = 0; m < nr; ++m)
                for (int b = 0; b < nblk; ++b, ++u)
                {
                    if ((u & (GV_WAVES - 1)) != wave) continue;
                    const int tok = tok1 >= 0 ? tok1 : a.row_token[r0 + m];
                    const int k = k0 + b * 128 + 2 * lane;
                    const uint32_t xv = ldg(a.x + (size_t)tok * a.H + k, 0);
                    const uint32_t sv = ldg(reinterpret_cast<const uint16_t*>(ex.suh[mat]) + k, 0);
                    float v0 = h2f(xv & 0xffffu) * h2f(sv & 0xffffu), v1 = h2f(xv >> 16) * h2f(sv >> 16);
                    had128_wave(v0, v1);
                    xs[(mat * MX + m) * XW + b * 64 + lane] =
                        (uint32_t)f2h_r(v0 * R_SCALE) | ((uint32_t)f2h_r(v1 * R_SCALE) << 16);
                }
    }
    else if (a.act_in_down)
    {
        // the gate / up epilogue of the k-range's blocks, straight into LDS (one wave per row and block)
        const int nblk = KR / 128;
        for (int u = wave; u < nr * nblk; u += GV_WAVES)
            gu_epi_wave<2>(a, r0 + u / nblk, k0 / 128 + u % nblk,     // two splits in flight: the GEMV's registers
                        reinterpret_cast<uint16_t*>(xs + (u / nblk) * XW + (u % nblk) * 64));
    }
    else if (MX == 1 && XW <= 4 * GV_THREADS)
    {
        if constexpr (NM == 1 && MX == 1)
        {
            switch (ex.fmt[2])
            {
                case BMX_TF_K2: down1_rows<BMX_TF_K2>(a, ex, cb, k0, KR, r0, xs, red); break;
                case BMX_TF_K25: down1_rows<BMX_TF_K25>(a, ex, cb, k0, KR, r0, xs, red); break;
                case BMX_TF_K3: down1_rows<BMX_TF_K3>(a, ex, cb, k0, KR, r0, xs, red); break;
                default: down1_rows<BMX_TF_K4>(a, ex, cb, k0, KR, r0, xs, red); break;
            }
            pre = true;
        }
    }
    else
    {
        for (int i = threadIdx.x; i < nr * XW; i += GV_THREADS)
        {
            const int m = i / XW, d = i % XW;
            xs[i] = ldg(a.act_rows + (size_t)(r0 + m) * a.I + k0 + 2 * d, 0);
        }
    }
    // rows nr .. (nr rounded up) of the staged input are read by the GEMV: zero them
    const int mr = nr <= 1 ? 1 : nr <= 2 ? 2 : nr <= 4 ? 4 : 8;
    for (int i = threadIdx.x; i < NM * (mr - nr) * XW; i += GV_THREADS)
    {
        const int mat = i / ((mr - nr) * XW), rem = i % ((mr - nr) * XW);
        xs[(mat * MX + nr) * XW + rem] = 0u;
    }
    if (!pre)
    {
        lds_barrier();
        if (mr == 1) gemv_rows<1, MX, NM>(a, ex, cb, k0, KR, N, xs, red);
        else if (mr == 2) { if constexpr (MX >= 2) gemv_rows<2, MX, NM>(a, ex, cb, k0, KR, N, xs, red); }
        else if (mr == 4) { if constexpr (MX >= 4) gemv_rows<4, MX, NM>(a, ex, cb, k0, KR, N, xs, red); }
        else { if constexpr (MX >= 8) gemv_rows<8, MX, NM>(a, ex, cb, k0, KR, N, xs, red); }
    }
    lds_barrier();
    // the waves of a matrix in order, then one partial per (split, row, block)
    float* part = (NM == 2 ? a.part_gu : a.part_dn) + (((size_t)ks * a.R_max + r0) * NB + cb) * (NM * 128);
    constexpr int WPM = NM == 2 ? GV_WPM : GV_WAVES;
    for (int i = threadIdx.x; i < NM * nr * 128; i += GV_THREADS)
    {
        const int c = i & 127, mat = (i >> 7) & (NM - 1), m = i >> (NM + 6);   // i = (m * NM + mat) * 128 + c
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < WPM; ++w) s = s + red[((mat * WPM + w) * MX + m) * 128 + c];
        part[(size_t)m * NB * NM * 128 + mat * 128 + c] = s;
    }
    (void)KS;
}

// the 4- and 8-row kernels (the product loop's staged input and accumulators grow with the rows) capped at 128 and 168
// VGPRs: 4 and 3 waves per SIMD instead of 3 and 2; the one-row down GEMV at 5 waves per SIMD (96 VGPRs instead of 116:
// C2's 1,152 one-token down workgroups start in one round; down 15.2 -> 14.6 us, the layer 54.6 -> 54.2 us)
template <int MX, int NM>
__global__ __launch_bounds__(GV_THREADS, (MX == 4 ? 4 : MX == 8 ? 3 : MX == 1 && NM == 1 ? 5 : 1)) void k_gemv_part(GvArgs a)
{
    if (NM == 2 && a.split_min > a.T && a.filter != 2 && split_callwide(a))
    {
        // split path, every expert on the mid-size kernel: this launch rotates the rows for it instead
        const long units = 2L * a.offsets[a.NE] * ((a.H / 128 + PREP_BPU - 1) / PREP_BPU);
        for (long u = (long)blockIdx.x * 16 + (threadIdx.x >> 4); u < units; u += (long)gridDim.x * 16) prep_unit(a, u);
        return;
    }
    int bid = blockIdx.x;
    const int KS = NM == 2 ? a.KS_gu : a.KS_dn, NB = NM == 2 ? a.NB : a.NBH;
    const int ks = bid % KS;
    bid /= KS;
    const int cb = bid % NB, g = bid / NB;
    if (g >= *a.ngroups) return;
    const int e = a.groups[3 * g], r0 = a.groups[3 * g + 1], nr = a.groups[3 * g + 2];
    if (group_skipped(a, e)) return;
    if (split_heavy(a, e)) return;          // split path: the mid-size kernel takes this expert's rows
    gemv_unit<MX, NM>(a, ks, cb, e, r0, nr, -1);
}

// LDS of the routing phase of k_gemv_gu_route, inside the kernel's dynamic LDS (the GEMV reuses it afterwards): the
// router wave's own, the picks, the group experts, and the one-wave dispatch's counts, offsets and token masks
template <int J>
struct RouteLds {
    TopkLds tl;
    int pe[64];
    int gex[64];
    int cnt[64 * (J + 1) + 1];
    int off[64 * (J + 1) + 1];
    alignas(8) uint64_t mask[64 * (J + 1) + 1];
};

// The gate / up GEMV of a one-token call that routes the token itself: wave 0 of every workgroup runs the router's
// selection (the same picks everywhere; only workgroup 0 writes sel / w and the dispatch arrays that the later stages
// read), and the workgroup takes its group from the picks: a one-token dispatch lists the picked experts in ascending
// order, one row each (row g for the g-th), then the shared expert (row topk). Saves the route + dispatch launch and the
// loads of the group record.
template <int J>
__global__ __launch_bounds__(GV_THREADS) __attribute__((amdgpu_waves_per_eu(5, 8))) void k_gemv_gu_route(GvArgs a,
                                                                                                          RouteFuse f)
{
    extern __shared__ uint32_t smem[];
    RouteLds<J>& L = *reinterpret_cast<RouteLds<J>*>(smem);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, topk = f.ra.topk;
    int bid = blockIdx.x;
    const int ks = bid % a.KS_gu;
    bid /= a.KS_gu;
    const int cb = bid % a.NB, g = bid / a.NB;
    if (g >= topk + (a.has_shared ? 1 : 0)) return;
    if (g == topk && blockIdx.x != 0)
    {
        // the shared expert's row (topk) needs nothing from the router: these workgroups decode while the others route
        gemv_unit<1, 2>(a, ks, cb, a.E, g, 1, 0);
        return;
    }
    if (wave == 0)
    {
        RouterArgs ra = f.ra;
        if (blockIdx.x != 0) ra.sel = nullptr;
        const int pk = route_token_wave<J>(ra, 0, L.tl);
        if (lane < topk) L.pe[lane] = pk;
        wave_lds_sync();
        if (lane < topk)
        {
            int rank = 0;
            for (int j = 0; j < topk; ++j) rank += L.pe[j] < pk;     // the picks of a token are distinct experts
            L.gex[rank] = pk;
        }
        if (blockIdx.x == 0) dispatch_wave<J + 1>(L.pe, topk, f.ra.E, 1, topk, f.sd, L.cnt, L.off, L.mask);
    }
    __syncthreads();
    const int e = g < topk ? L.gex[g] : a.E;
    __syncthreads();                      // every wave has read the routing LDS before the GEMV reuses it
    gemv_unit<1, 2>(a, ks, cb, e, g, 1, 0);
}

// ---- epilogues: 16 lanes per (row or token, 128-column block), 8 consecutive columns per lane -----------------------------
// UPW work units per wave: 4 (every lane busy) for large launches, 1 (lanes 16-63 idle; four times the waves, so a
// decode-size launch spreads over more CUs) for small ones.
// acc[4 v + i] = sum over splits s = 0, 1, ... ks - 1 in that order of p[s * stride + off(v) + i], off = 0, 4, 128, 132
// (NV = 4: gate 8 | up 8) or 0, 4 (NV = 2). The loads of B splits are issued together before their adds, so a long
// split list costs one memory latency per B splits instead of one per split.
template <int NV, int B>
__device__ __forceinline__ void sum_splits(const float* p, size_t stride, int ks, float (&acc)[NV * 4])
{
#pragma unroll
    for (int i = 0; i < NV * 4; ++i) acc[i] = 0.0f;
    int s = 0;
    for (; s + B <= ks; s += B)
    {
        f32x4 q[B][NV];
#pragma unroll
        for (int b = 0; b < B; ++b)
#pragma unroll
            for (int v = 0; v < NV; ++v) q[b][v] = ldg4f(p + (size_t)(s + b) * stride + (v & 1) * 4 + (v >> 1) * 128);
#pragma unroll
        for (int b = 0; b < B; ++b)
#pragma unroll
            for (int v = 0; v < NV; ++v)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[4 * v + i] = acc[4 * v + i] + q[b][v][i];
    }
    for (; s < ks; ++s)
#pragma unroll
        for (int v = 0; v < NV; ++v)
        {
            const f32x4 q = ldg4f(p + (size_t)s * stride + (v & 1) * 4 + (v >> 1) * 128);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[4 * v + i] = acc[4 * v + i] + q[i];
        }
}

// The same sums for the one-token launches, where a few workgroups wait on this chain of loads and their register count
// does not matter: a short last batch also issues all its loads before the first add (not one round trip per split),
// and the first batch sits outside the loop, in straight-line code, so its loads issue beside the caller's earlier ones
// (a loop entry makes the compiler wait for every load in flight). The large launches keep sum_splits: this form needs
// more registers, which costs them occupancy.
template <int NV, int B>
__device__ __forceinline__ void sum_splits_short_batch(const float* p, size_t stride, int s, int ks,
                                                       float (&acc)[NV * 4])
{
    const int n = ks - s < B ? ks - s : B;       // uniform: the branches below split no wave
    f32x4 q[B][NV];
#pragma unroll
    for (int b = 0; b < B; ++b)
        if (b < n)
#pragma unroll
            for (int v = 0; v < NV; ++v) q[b][v] = ldg4f(p + (size_t)(s + b) * stride + (v & 1) * 4 + (v >> 1) * 128);
#pragma unroll
    for (int b = 0; b < B; ++b)
        if (b < n)
#pragma unroll
            for (int v = 0; v < NV; ++v)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[4 * v + i] = acc[4 * v + i] + q[b][v][i];
}

template <int NV, int B>
__device__ __forceinline__ void sum_splits_short(const float* p, size_t stride, int ks, float (&acc)[NV * 4])
{
#pragma unroll
    for (int i = 0; i < NV * 4; ++i) acc[i] = 0.0f;
    if (ks > 0) sum_splits_short_batch<NV, B>(p, stride, 0, ks, acc);
    for (int s = B; s < ks; s += B) sum_splits_short_batch<NV, B>(p, stride, s, ks, acc);
}

template <int UPW>
__device__ __forceinline__ int ep_unit()
{
    return (blockIdx.x * GV_WAVES + (threadIdx.x >> 6)) * UPW + ((threadIdx.x & 63) >> 4);
}
constexpr long EP_SMALL = 16384;              // launches with fewer units use UPW = 1

// gate / up epilogue: sum of the splits in split order -> fp16 gate / up (the stored GEMV / GEMM results) -> H128 * R * svh
// -> activation -> * down suh -> H128 * R -> fp16 down-input row (exllamav3 kernel A epilogue order,
// engine/kernels/x16/x16_dev.cu:245-283)
template <int UPW>
__global__ __launch_bounds__(GV_THREADS) void k_gu_epi(GvArgs a)
{
    if (UPW == 1 && (threadIdx.x & 63) >= 16) return;
    const int u = ep_unit<UPW>(), j = threadIdx.x & 15;
    const int r = u / a.NB, cb = u % a.NB;
    if (r >= a.offsets[a.NE]) return;
    const int e = a.row_expert[r];
    const bmx_expert& ex = e == a.E ? *a.shared : a.experts[e];
    const int col = cb * 128 + 8 * j;
    float g[8], v[8];
    if (a.gu_half)
    {
        const uint16_t* hp = reinterpret_cast<const uint16_t*>(a.part_gu) + ((size_t)r * a.NB + cb) * 256 + 8 * j;
        unpack8(ldg4(hp), g);
        unpack8(ldg4(hp + 128), v);
    }
    else
    {
        float gu[16];
        sum_splits<4, 4>(a.part_gu + ((size_t)r * a.NB + cb) * 256 + 8 * j, (size_t)a.R_max * a.NB * 256,
                         row_splits<false>(a, r), gu);
#pragma unroll
        for (int i = 0; i < 8; ++i) { g[i] = h2f(f2h_r(gu[i])); v[i] = h2f(f2h_r(gu[8 + i])); }
    }
    had128_x8(g);
    had128_x8(v);
    const float rs = R_SCALE * had128_x8_sign();      // the transforms' lane sign folded into the scale
    float svg[8], svu[8], sud[8];
    unpack8(ldg4(reinterpret_cast<const uint16_t*>(ex.svh[0]) + col), svg);
    unpack8(ldg4(reinterpret_cast<const uint16_t*>(ex.svh[1]) + col), svu);
    unpack8(ldg4(reinterpret_cast<const uint16_t*>(ex.suh[2]) + col), sud);
    float act[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
    {
        const float gi = (g[i] * rs) * svg[i], ui = (v[i] * rs) * svu[i];
        act[i] = (a.fast_act ? act_gate_fast(a.act, a.gated, gi, ui, a.limit) : act_gate(a.act, a.gated, gi, ui, a.limit)) *
                 sud[i];
    }
    had128_x8(act);
#pragma unroll
    for (int i = 0; i < 8; ++i) act[i] = act[i] * rs;
    *reinterpret_cast<u32x4*>(a.act_rows + (size_t)r * a.I + col) = pack8_r(act);
}

// Gate / up epilogue of row r, 128-column block cb, by one wave: its 128 fp16 down-input values go to dst (16 bytes per
// lane of group 0, lane j at dst + 8 j: global memory or LDS). Lane group q = lane >> 4 loads splits q, q + 4, ... B at
// a time (the sums are the same for every B) and the four groups' sums are added pairwise ((q0 + q1) + (q2 + q3)), so the k-splits cost one memory latency
// instead of one per batch; the rest runs as in k_gu_epi (every group computes it, group 0 stores).
template <int B>
__device__ __forceinline__ void gu_epi_wave(const GvArgs& a, int r, int cb, uint16_t* dst)
{
    const int lane = threadIdx.x & 63, q = lane >> 4, j = lane & 15;
    const int nrows = a.offsets[a.NE], e = a.row_expert[r];
    const int col = cb * 128 + 8 * j;
    // the row's scale vectors first: their chain of loads (expert record, then vectors) overlaps the split sums' loads
    u32x4 svg4 = {0u, 0u, 0u, 0u}, svu4 = svg4, sud4 = svg4;
    if (r < nrows)
    {
        const bmx_expert& ex = e == a.E ? *a.shared : a.experts[e];
        svg4 = ldg4(reinterpret_cast<const uint16_t*>(ex.svh[0]) + col);
        svu4 = ldg4(reinterpret_cast<const uint16_t*>(ex.svh[1]) + col);
        sud4 = ldg4(reinterpret_cast<const uint16_t*>(ex.suh[2]) + col);
    }
    float g[8], v[8];
    if (a.gu_half)
    {
        // one fp16 split: every lane group loads the same values
        const uint16_t* hp = reinterpret_cast<const uint16_t*>(a.part_gu) + ((size_t)r * a.NB + cb) * 256 + 8 * j;
        unpack8(ldg4(hp), g);
        unpack8(ldg4(hp + 128), v);
        if (r >= nrows) return;
    }
    else
    {
        const size_t stride = (size_t)a.R_max * a.NB * 256;
        const float* p = a.part_gu + ((size_t)r * a.NB + cb) * 256 + 8 * j + (size_t)q * stride;
        float gu[16];
        const int ks = r < nrows ? row_splits<false>(a, r) : a.KS_gu;
        sum_splits_short<4, B>(p, 4 * stride, (ks - q + 3) / 4, gu);
#pragma unroll
        for (int i = 0; i < 16; ++i) gu[i] = gu[i] + xor16_f(gu[i]);
#pragma unroll
        for (int i = 0; i < 16; ++i) gu[i] = gu[i] + xor32_f(gu[i]);
        if (r >= nrows) return;
#pragma unroll
        for (int i = 0; i < 8; ++i) { g[i] = h2f(f2h_r(gu[i])); v[i] = h2f(f2h_r(gu[8 + i])); }
    }
    had128_x8(g);
    had128_x8(v);
    const float rs = R_SCALE * had128_x8_sign();      // the transforms' lane sign folded into the scale
    float svg[8], svu[8], sud[8];
    unpack8(svg4, svg);
    unpack8(svu4, svu);
    unpack8(sud4, sud);
    float act[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
    {
        const float gi = (g[i] * rs) * svg[i], ui = (v[i] * rs) * svu[i];
        act[i] = act_gate(a.act, a.gated, gi, ui, a.limit) * sud[i];
    }
    had128_x8(act);
#pragma unroll
    for (int i = 0; i < 8; ++i) act[i] = act[i] * rs;
    if (q == 0) *reinterpret_cast<u32x4*>(dst + 8 * j) = pack8_r(act);
}

// Small launches: one wave per (row, 128-column block).
__global__ __launch_bounds__(GV_THREADS) void k_gu_epi_w(GvArgs a)
{
    const int u = blockIdx.x * GV_WAVES + (threadIdx.x >> 6);
    const int r = u / a.NB, cb = u % a.NB;
    if (r >= a.R_max) return;
    gu_epi_wave<4>(a, r, cb, a.act_rows + (size_t)r * a.I + cb * 128);
}

// down output of row r, block cb, lane's 8 columns: sum of the splits -> H128 * R * svh. SHORT (one-token launches): the
// scale vector is loaded before the split sums (its chain of loads overlaps theirs) and the sums take sum_splits_short.
template <bool SHORT>
__device__ __forceinline__ void down_out8(const GvArgs& a, int r, int cb, float (&y)[8])
{
    const int j = threadIdx.x & 15;
    const int e = a.row_expert[r];
    const bmx_expert& ex = e == a.E ? *a.shared : a.experts[e];
    const uint16_t* svp = reinterpret_cast<const uint16_t*>(ex.svh[2]) + cb * 128 + 8 * j;
    const float* pp = a.part_dn + ((size_t)r * a.NBH + cb) * 128 + 8 * j;
    const size_t stride = (size_t)a.R_max * a.NBH * 128;
    u32x4 sv4;
    const int ks = row_splits<true>(a, r);
    if (SHORT)
    {
        sv4 = ldg4(svp);
        sum_splits_short<2, 8>(pp, stride, ks, y);
    }
    else
    {
        sum_splits<2, 8>(pp, stride, ks, y);
        sv4 = ldg4(svp);
    }
    had128_x8(y);
    const float rs = R_SCALE * had128_x8_sign();
    float sv[8];
    unpack8(sv4, sv);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = (y[i] * rs) * sv[i];
}

// the same with non-temporal stores: outputs written once and read by the next layer, not by this call's kernels
__device__ __forceinline__ void store8f_nt(float* p, const float (&y)[8])
{
    const f32x4 a = {y[0], y[1], y[2], y[3]}, b = {y[4], y[5], y[6], y[7]};
    __builtin_nontemporal_store(a, reinterpret_cast<f32x4*>(p));
    __builtin_nontemporal_store(b, reinterpret_cast<f32x4*>(p + 4));
}

__device__ __forceinline__ void store8f(float* p, const float (&y)[8])
{
    *reinterpret_cast<float4*>(p) = make_float4(y[0], y[1], y[2], y[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(y[4], y[5], y[6], y[7]);
}

// ---- down epilogue over rows (expert outputs only) -----------------------------------------------------------------------
template <int UPW>
__global__ __launch_bounds__(GV_THREADS) void k_dn_epi(GvArgs a)
{
    if (UPW == 1 && (threadIdx.x & 63) >= 16) return;
    const int u = ep_unit<UPW>(), j = threadIdx.x & 15;
    const int r = u / a.NBH, cb = u % a.NBH;
    if (r >= a.offsets[a.NE]) return;
    float y[8];
    down_out8<UPW == 1>(a, r, cb, y);
    store8f(a.y_rows + (size_t)r * a.H + cb * 128 + 8 * j, y);
}

// ---- down epilogue + combine -----------------------------------------------------------------------------------------
// out[t] = sum over k ascending of w[t, k] * y(inv[t, k]) (picks with inv < 0 or w = 0 skipped), then + y(shared row)
// (engine/kernels/x16/x16_dev.cu:354-384). Large launches: 16 lanes per (token, 128-column block), the slots in turn.
// With one k-split for every row (the prefill path): CB_BATCH slots at a time (2: 217 us at C3, 3: 219, 6: 245; one
// slot at a time: 256), every load of the batch (the slots' partial rows, their experts' scale vectors) issued before
// the first slot's transform, the same operations in the same order afterwards (so the same bits).
constexpr int CB_BATCH = 2;
__device__ __forceinline__ void combine_batched(const GvArgs& a, int t, int cb, float (&o)[8])
{
    const int j = threadIdx.x & 15;
    const float rs = R_SCALE * had128_x8_sign();
    for (int k0 = 0; k0 < a.topk; k0 += CB_BATCH)
    {
        int r[CB_BATCH];
        float wk[CB_BATCH];
        f32x4 q[CB_BATCH][2];
        u32x4 sv4[CB_BATCH];
#pragma unroll
        for (int b = 0; b < CB_BATCH; ++b)
        {
            const int k = k0 + b;
            r[b] = -1;
            wk[b] = 0.0f;
            if (k < a.topk)
            {
                r[b] = a.inv[t * a.topk + k];
                wk[b] = h2f(a.w[t * a.topk + k]);
            }
        }
#pragma unroll
        for (int b = 0; b < CB_BATCH; ++b)
            if (r[b] >= 0 && wk[b] != 0.0f)
            {
                const float* pp = a.part_dn + ((size_t)r[b] * a.NBH + cb) * 128 + 8 * j;
                q[b][0] = ldg4f(pp);
                q[b][1] = ldg4f(pp + 4);
                const int e = a.row_expert[r[b]];
                const bmx_expert& ex = e == a.E ? *a.shared : a.experts[e];
                sv4[b] = ldg4(reinterpret_cast<const uint16_t*>(ex.svh[2]) + cb * 128 + 8 * j);
            }
#pragma unroll
        for (int b = 0; b < CB_BATCH; ++b)
        {
            if (r[b] < 0 || wk[b] == 0.0f) continue;
            float y[8], sv[8];
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                y[i] = 0.0f + q[b][0][i];
                y[4 + i] = 0.0f + q[b][1][i];
            }
            had128_x8(y);
            unpack8(sv4[b], sv);
#pragma unroll
            for (int i = 0; i < 8; ++i) y[i] = (y[i] * rs) * sv[i];
            if (a.y_rows) store8f(a.y_rows + (size_t)r[b] * a.H + cb * 128 + 8 * j, y);
#pragma unroll
            for (int i = 0; i < 8; ++i)
            {
                const float p = wk[b] * y[i];
                o[i] = o[i] + p;
            }
        }
    }
}

__global__ __launch_bounds__(GV_THREADS) void k_dn_combine(GvArgs a)
{
    const int u = ep_unit<4>(), j = threadIdx.x & 15;
    const int t = u / a.NBH, cb = u % a.NBH;
    if (t >= a.T) return;
    float o[8], y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = 0.0f;
    if (a.KS_dn == 1 && !a.split_min) combine_batched(a, t, cb, o);
    else
    for (int k = 0; k < a.topk; ++k)
    {
        const int r = a.inv[t * a.topk + k];
        const float wk = h2f(a.w[t * a.topk + k]);
        if (r < 0 || wk == 0.0f) continue;
        down_out8<false>(a, r, cb, y);
        if (a.y_rows) store8f(a.y_rows + (size_t)r * a.H + cb * 128 + 8 * j, y);
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            const float p = wk * y[i];
            o[i] = o[i] + p;
        }
    }
    if (a.has_shared)
    {
        const int r = a.offsets[a.E] + t;
        down_out8<false>(a, r, cb, y);
        if (a.y_rows) store8f(a.y_rows + (size_t)r * a.H + cb * 128 + 8 * j, y);
        if (a.sh_gate)
        {
            const float g = shared_gate16(a.x + (size_t)t * a.H, a.sh_gate, a.H);
#pragma unroll
            for (int i = 0; i < 8; ++i)
            {
                const float p = g * y[i];
                o[i] = o[i] + p;
            }
        }
        else
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = o[i] + y[i];
    }
    store8f_nt(a.out + (size_t)t * a.H + cb * 128 + 8 * j, o);
}

// The combine of token t's 128-column block cb by one workgroup: 16-lane group k computes slot k (the shared expert's
// row is slot topk) into ys[k], then group 0 sums them in slot order: the same sums in the same order as k_dn_combine.
// ys: [topk + 1][128] floats and live: [topk + 1] ints of LDS.
constexpr int CB_MAXS = 33;
__device__ __forceinline__ void combine_block(const GvArgs& a, int t, int cb, float (*ys)[128], int* live)
{
    const int k0 = threadIdx.x >> 4, j = threadIdx.x & 15;
    const int ns = a.topk + (a.has_shared ? 1 : 0);
    for (int k = k0; k < ns; k += GV_THREADS / 16)
    {
        int r;
        if (k < a.topk)
        {
            r = a.inv[t * a.topk + k];
            const float wk = h2f(a.w[t * a.topk + k]);      // loaded beside r, not after it
            if (r < 0 || wk == 0.0f)
            {
                if (j == 0) live[k] = 0;
                continue;
            }
        }
        else r = a.offsets[a.E] + t;
        float y[8];
        down_out8<true>(a, r, cb, y);
        if (a.y_rows) store8f(a.y_rows + (size_t)r * a.H + cb * 128 + 8 * j, y);
#pragma unroll
        for (int i = 0; i < 8; ++i) ys[k][8 * j + i] = y[i];
        if (j == 0) live[k] = 1;
    }
    lds_barrier();
    if (k0) return;
    const float g = (a.has_shared && a.sh_gate) ? shared_gate16(a.x + (size_t)t * a.H, a.sh_gate, a.H) : 1.0f;
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = 0.0f;
    for (int k = 0; k < a.topk; ++k)
    {
        if (!live[k]) continue;
        const float wk = h2f(a.w[t * a.topk + k]);
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            const float p = wk * ys[k][8 * j + i];
            o[i] = o[i] + p;
        }
    }
    if (a.has_shared && a.sh_gate)
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
            const float p = g * ys[a.topk][8 * j + i];
            o[i] = o[i] + p;
        }
    else if (a.has_shared)
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = o[i] + ys[a.topk][8 * j + i];
    store8f(a.out + (size_t)t * a.H + cb * 128 + 8 * j, o);
}

// Small launches: one workgroup per (token, 128-column block).
__global__ __launch_bounds__(GV_THREADS) void k_dn_combine_par(GvArgs a)
{
    __shared__ float ys[CB_MAXS][128];
    __shared__ int live[CB_MAXS];
    combine_block(a, blockIdx.x / a.NBH, blockIdx.x % a.NBH, ys, live);
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

int launch_epilogue(const GvArgs& a, int stage, hipStream_t s)
{
    // units -> workgroups of GV_WAVES waves with UPW units each
    auto wgs = [](long units, int upw) { return dim3((unsigned)((units + GV_WAVES * upw - 1) / (GV_WAVES * upw))); };
    const long gu = (long)a.R_max * a.NB, dn = (long)a.R_max * a.NBH, cmb = (long)a.T * a.NBH;
    switch (stage)
    {
        case BMX_STAGE_ACT:
            if (gu >= EP_SMALL) hipLaunchKernelGGL(k_gu_epi<4>, wgs(gu, 4), dim3(GV_THREADS), 0, s, a);
            else hipLaunchKernelGGL(k_gu_epi_w, wgs(gu, 1), dim3(GV_THREADS), 0, s, a);
            break;
        case BMX_STAGE_COMBINE:
            if (cmb >= EP_SMALL) hipLaunchKernelGGL(k_dn_combine, wgs(cmb, 4), dim3(GV_THREADS), 0, s, a);
            else hipLaunchKernelGGL(k_dn_combine_par, dim3((unsigned)cmb), dim3(GV_THREADS), 0, s, a);
            break;
        case BMX_STAGE_DOWN_OUT:
            if (dn >= EP_SMALL) hipLaunchKernelGGL(k_dn_epi<4>, wgs(dn, 4), dim3(GV_THREADS), 0, s, a);
            else hipLaunchKernelGGL(k_dn_epi<1>, wgs(dn, 1), dim3(GV_THREADS), 0, s, a);
            break;
        default: return set_error(BMX_ERR_ARG, "unknown epilogue stage %d", stage);
    }
    return BMX_OK;
}

int decode_gu_grouped(const MoeShape& m)
{
    const DecodePlan p = decode_plan(m);
    return (long)p.R_max * p.NB < EP_SMALL ? 1 : 0;     // k_gu_epi_w and the one-token down prologue: gu_epi_wave
}

// ---- plan ------------------------------------------------------------------------------------------------------------
// BMX_ACT_IN_DOWN=0 keeps the separate gate / up epilogue kernel for one-token calls
static bool act_in_down_allowed()
{
    const char* v = getenv("BMX_ACT_IN_DOWN");
    return !(v && *v == '0');
}

static int rows_per_group_of(int T) { return T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : 8; }

// smallest divisor d of nblk128 (so the k-range stays a whole number of 128-blocks) reaching `target` workgroups
static int pick_split(int nblk128, long units, long target, const char* env)
{
    const char* v = getenv(env);
    if (v && *v)
    {
        const int ks = atoi(v);
        if (ks >= 1 && nblk128 % ks == 0) return ks;
    }
    int best = 1;
    for (int d = 1; d <= nblk128; ++d)
    {
        if (nblk128 % d) continue;
        best = d;
        if (units * d >= target) break;
    }
    return best;
}

static long target_wgs()
{
    const char* v = getenv("BMX_WG_TARGET");
    return (v && *v) ? atol(v) : 1024;
}

DecodePlan decode_plan(const MoeShape& m)
{
    DecodePlan p;
    const int MR = rows_per_group_of(m.T);
    p.NB = m.I / 128;
    p.NBH = m.H / 128;
    p.G_max = groups_max(m.T, m.topk, m.E, m.shared, MR);
    p.R_max = m.T * m.topk + (m.shared ? m.T : 0);
    const long n = (long)m.T * m.topk + (m.shared ? 1 : 0), ne = (long)m.E + (m.shared ? 1 : 0);
    const long uniq = n < ne ? n : ne;
    const long est = uniq + (long)(m.T > MR ? (m.T * m.topk) / (MR * 4) : 0);
    // the staged input rows (NM matrices x MR rows x k-range fp16) must fit GV_LDS_X
    const int max_kr_gu = GV_LDS_X / (2 * MR * 2), max_kr_dn = GV_LDS_X / (MR * 2);
    int ks = pick_split(m.H / 128, est * p.NB, target_wgs(), "BMX_KS_GU");
    while (m.H / ks > max_kr_gu) { int d = ks + 1; while ((m.H / 128) % d) ++d; ks = d; }
    p.KS_gu = ks;
    ks = pick_split(m.I / 128, est * p.NBH, target_wgs(), "BMX_KS_DN");
    while (m.I / ks > max_kr_dn) { int d = ks + 1; while ((m.I / 128) % d) ++d; ks = d; }
    p.KS_dn = ks;
    p.part_gu_bytes = (size_t)p.KS_gu * p.R_max * p.NB * 256 * 4;
    p.part_dn_bytes = (size_t)p.KS_dn * p.R_max * p.NBH * 128 * 4;
    p.counters = 0;
    return p;
}

size_t decode_ws_bytes(const MoeShape& m)
{
    const DecodePlan p = decode_plan(m);
    return align_up(p.part_gu_bytes, 256) + align_up(p.part_dn_bytes, 256) + align_up((size_t)p.R_max * m.I * 2, 256);
}

// stages: bit i = BMX_STAGE i (GATE_UP, ACT, DOWN, COMBINE, DOWN_OUT; PREP launches nothing here: the GEMV rotates)
// the routing gate / up GEMV for ceil(E / 64) = J
template <int J>
static void launch_gu_route(const GvArgs& a, const DecodePlan& p, const RouteFuse& f, size_t lds_gu, hipStream_t s)
{
    const size_t lds = lds_gu > sizeof(RouteLds<J>) ? lds_gu : sizeof(RouteLds<J>);
    hipLaunchKernelGGL(k_gemv_gu_route<J>, dim3((unsigned)(p.G_max * p.NB * p.KS_gu)), dim3(GV_THREADS), lds, s, a, f);
}

template <int MR>
static void launch_mr(const GvArgs& a, const DecodePlan& p, int stages, hipStream_t s, const RouteFuse* rf)
{
    const size_t lds_gu = (size_t)2 * MR * (a.H / p.KS_gu) / 2 * 4 + (size_t)GV_WAVES * MR * 128 * 4;
    const size_t lds_dn = (size_t)MR * (a.I / p.KS_dn) / 2 * 4 + (size_t)GV_WAVES * MR * 128 * 4;
    for (int f = 0; f < 3; ++f)
    {
        const int st = f == 0 ? BMX_STAGE_GATE_UP : f == 1 ? BMX_STAGE_GATE_UP_RESIDENT : BMX_STAGE_GATE_UP_STAGED;
        if (!(stages & (1 << st))) continue;
        GvArgs b = a;
        b.filter = f;
        if (MR == 1 && f == 0 && rf)
            switch (rf->J)
            {
                case 1: launch_gu_route<1>(b, p, *rf, lds_gu, s); break;
                case 2: launch_gu_route<2>(b, p, *rf, lds_gu, s); break;
                case 3: launch_gu_route<3>(b, p, *rf, lds_gu, s); break;
                case 4: launch_gu_route<4>(b, p, *rf, lds_gu, s); break;
                case 5: launch_gu_route<5>(b, p, *rf, lds_gu, s); break;
                case 6: launch_gu_route<6>(b, p, *rf, lds_gu, s); break;
                case 7: case 8: launch_gu_route<8>(b, p, *rf, lds_gu, s); break;
                default: launch_gu_route<16>(b, p, *rf, lds_gu, s); break;
            }
        else
            hipLaunchKernelGGL((k_gemv_part<MR, 2>), dim3((unsigned)(p.G_max * p.NB * p.KS_gu)), dim3(GV_THREADS), lds_gu, s,
                               b);
    }
    if ((stages & (1 << BMX_STAGE_ACT)) && !a.act_in_down) launch_epilogue(a, BMX_STAGE_ACT, s);
    for (int f = 0; f < 3; ++f)
    {
        const int st = f == 0 ? BMX_STAGE_DOWN : f == 1 ? BMX_STAGE_DOWN_RESIDENT : BMX_STAGE_DOWN_STAGED;
        if (!(stages & (1 << st))) continue;
        GvArgs b = a;
        b.filter = f;
        hipLaunchKernelGGL((k_gemv_part<MR, 1>), dim3((unsigned)(p.G_max * p.NBH * p.KS_dn)), dim3(GV_THREADS), lds_dn, s, b);
    }
    if (stages & (1 << BMX_STAGE_COMBINE)) launch_epilogue(a, BMX_STAGE_COMBINE, s);
    if (stages & (1 << BMX_STAGE_DOWN_OUT)) launch_epilogue(a, BMX_STAGE_DOWN_OUT, s);
}

// Compute units of the current device (each device asked once; threads that race on the first call store the same
// value). BMX_CU_COUNT overrides it, so a test can take the split count another device would take.
static int cu_count()
{
    static std::atomic<int> n[64];
    const char* ov = getenv("BMX_CU_COUNT");
    if (ov && *ov && atoi(ov) > 0) return atoi(ov);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = n[dev].load(std::memory_order_relaxed);
    if (!v)
    {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        n[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

// The routing gate / up GEMV pays the routing at the start of every workgroup, so it takes the most k-splits (at most
// the plan's) whose workgroups start in one round (5 per compute unit); a k-range that no longer fits the staged input
// rows, a forced split (BMX_KS_GU) or no such count keeps the plan's. Same results within the layer tolerance (another
// summation order of the k-split partials); bmx_decode_splits describes the separate route + GEMV path.
static int one_round_ks(const DecodePlan& p, const MoeShape& m)
{
    const char* v = getenv("BMX_KS_GU");
    if (v && *v) return p.KS_gu;
    const long cap = 5L * cu_count(), units = (long)p.G_max * p.NB;
    const int nblk = m.H / 128, max_kr = GV_LDS_X / (2 * 1 * 2);
    for (int d = p.KS_gu; d >= 1; --d)
    {
        if (nblk % d) continue;
        if (m.H / d > max_kr) break;
        if (units * d <= cap) return d;
    }
    return p.KS_gu;
}

int launch_decode_experts(const MoeShape& m, const void* x, const bmx_routes* r, float* y_rows, void* act_rows,
                          void* ws, size_t ws_bytes, float* combine_out, const void* combine_w, hipStream_t s, int stages,
                          const RouteFuse* rf)
{
    if (rf && (m.T != 1 || rows_per_group_of(m.T) != 1))
        return set_error(BMX_ERR_ARG, "moe experts: routing inside the GEMV is for one-token calls");
    if (m.H % 128 || m.I % 128 || m.H <= 0 || m.I <= 0)
        return set_error(BMX_ERR_ARG, "moe experts: H (%d) and I (%d) must be multiples of 128", m.H, m.I);
    const DecodePlan p = decode_plan(m);
    if (ws_bytes < decode_ws_bytes(m))
        return set_error(BMX_ERR_WORKSPACE, "moe experts: workspace %zu < %zu", ws_bytes, decode_ws_bytes(m));
    if (!r->row_expert) return set_error(BMX_ERR_ARG, "moe experts: routes without row_expert");
    char* w = static_cast<char*>(ws);
    GvArgs a;
    a.experts = m.experts; a.shared = m.shared_ex; a.E = m.E; a.H = m.H; a.I = m.I; a.act = m.act; a.gated = m.gated;
    a.limit = m.limit;
    a.x = static_cast<const uint16_t*>(x);
    a.row_token = r->row_token; a.groups = r->groups; a.ngroups = r->ngroups; a.row_expert = r->row_expert;
    a.part_gu = reinterpret_cast<float*>(w);
    w += align_up(p.part_gu_bytes, 256);
    a.part_dn = reinterpret_cast<float*>(w);
    w += align_up(p.part_dn_bytes, 256);
    a.act_rows = act_rows ? static_cast<uint16_t*>(act_rows) : reinterpret_cast<uint16_t*>(w);
    a.y_rows = y_rows;
    DecodePlan q = p;                      // the launch's plan (the workspace keeps p's layout; q's partials fit in it)
    if (rf) q.KS_gu = one_round_ks(p, m);
    a.KS_gu = q.KS_gu; a.KS_dn = q.KS_dn; a.NB = q.NB; a.NBH = q.NBH; a.R_max = q.R_max;
    a.NE = m.E + (m.shared ? 1 : 0);
    a.out = combine_out; a.w = static_cast<const uint16_t*>(combine_w); a.inv = r->inv; a.offsets = r->offsets;
    a.T = m.T; a.topk = m.topk; a.has_shared = m.shared;
    a.xt = nullptr;
    a.fresh = m.fresh;
    a.sh_gate = m.shared_gate;
    a.filter = 0;
    // One-row groups (one token) with the activation and the down product in the same call and no act rows asked
    // for: the down GEMV computes the activation of its k-range itself, once per output block instead of once, for
    // one launch and one round trip through memory fewer. Worth it up to 16 output blocks (H <= 2048: 31.0 -> 29.6 us
    // for a 64-expert top-8 layer of H 2048, I 768); at 32 blocks the repeated epilogue costs what it saves.
    a.gu_half = 0;
    a.act_in_down = rows_per_group_of(m.T) == 1 && (stages & (1 << BMX_STAGE_ACT)) && (stages & (1 << BMX_STAGE_DOWN)) &&
                    !act_rows && m.H / 128 <= 16 && act_in_down_allowed();
    switch (rows_per_group_of(m.T))
    {
        case 1: launch_mr<1>(a, q, stages, s, rf); break;
        case 2: launch_mr<2>(a, p, stages, s, nullptr); break;
        case 4: launch_mr<4>(a, p, stages, s, nullptr); break;
        default: launch_mr<8>(a, p, stages, s, nullptr); break;
    }
    return check_launch("moe experts (decode path)");
}

int decode_rows_per_group(int T) { return rows_per_group_of(T); }

// ---- split path ---------------------------------------------------------------------------------------------------------
// The mid-size MFMA kernel decodes an expert once per 32 rows and multiplies on MFMA; the GEMV decodes once per group of
// up to 8 rows and pays an fdot2 per row and weight, but has the shorter start. Measured on the 16-token speculative-
// verify batch (the DeepSeek shape, 4-6 rows per expert): GEMV 172.6, mid-size 128.6 us; on the GLM shape at 8 tokens
// (1.5 rows per expert): GEMV 225.7, mid-size 293. Mixing the two per expert in one call runs both kernels back to back
// and measured worse than either alone (151-168 us, 255-278 us), so the choice is per call: all experts on the
// mid-size kernel when the call averages at least BMX_SPLIT_RATIO rows per unique expert (default 2.5), else all on the
// GEMV; BMX_SPLIT_MIN_ROWS = n also sends experts with at least n rows to the mid-size kernel in a GEMV call (off by
// default: on the GEMV-chosen calls measured, 16- and 32-token batches of both shapes, it only added the idle cost of
// walking the units).
int split_min_rows()
{
    const char* v = getenv("BMX_SPLIT_MIN_ROWS");
    const int n = (v && *v) ? atoi(v) : (1 << 30);
    return n < 1 ? 1 : n;
}

static int split_ratio2()
{
    const char* v = getenv("BMX_SPLIT_RATIO");
    const double r = (v && *v) ? atof(v) : 2.5;
    const int q = (int)(2.0 * r + 0.5);
    return q < 0 ? 0 : q;
}

size_t split_ws_bytes(const MoeShape& m)
{
    const DecodePlan p = decode_plan(m);
    int ksg = 1, ksd = 1;
    split_mid_splits(m, &ksg, &ksd);
    const size_t R = (size_t)p.R_max;
    return align_up((size_t)std::max(p.KS_gu, ksg) * R * p.NB * 256 * 4, 256) +
           align_up((size_t)std::max(p.KS_dn, ksd) * R * p.NBH * 128 * 4, 256) + align_up(R * m.I * 2, 256) +
           align_up((size_t)2 * R * m.H * 2, 256);
}

// One call over both kernels: the heavy experts' rows (split_heavy) on k_mid_gemm over (expert, 32-row chunk)
// units, the others' on k_gemv_part over the dispatch's groups (heavy groups skipped); both write the same partial
// layout, each row with its own kernel's k-split count, which the epilogues read per row. Order on the stream: prep of
// the heavy rows, gate / up (GEMV, then mid), epilogue, down (GEMV, then mid), combine.
int launch_split_experts(const MoeShape& m, const void* x, const bmx_routes* r, float* y_rows, void* act_rows,
                         void* ws, size_t ws_bytes, float* combine_out, const void* combine_w, hipStream_t s, int stages)
{
    if (m.H % 128 || m.I % 128 || m.H <= 0 || m.I <= 0)
        return set_error(BMX_ERR_ARG, "moe experts: H (%d) and I (%d) must be multiples of 128", m.H, m.I);
    if (ws_bytes < split_ws_bytes(m))
        return set_error(BMX_ERR_WORKSPACE, "moe experts: workspace %zu < %zu", ws_bytes, split_ws_bytes(m));
    if (!r->row_expert || !r->counts || !r->uexp || !r->nuniq)
        return set_error(BMX_ERR_ARG, "moe experts: split path needs the routes' counts, uexp, nuniq and row_expert");
    const DecodePlan p = decode_plan(m);
    int ksg = 1, ksd = 1;
    split_mid_splits(m, &ksg, &ksd);
    const size_t R = (size_t)p.R_max;
    char* w = static_cast<char*>(ws);
    GvArgs a;
    a.experts = m.experts; a.shared = m.shared_ex; a.E = m.E; a.H = m.H; a.I = m.I; a.act = m.act; a.gated = m.gated;
    a.limit = m.limit;
    a.x = static_cast<const uint16_t*>(x);
    a.row_token = r->row_token; a.groups = r->groups; a.ngroups = r->ngroups; a.row_expert = r->row_expert;
    a.part_gu = reinterpret_cast<float*>(w);
    w += align_up((size_t)std::max(p.KS_gu, ksg) * R * p.NB * 256 * 4, 256);
    a.part_dn = reinterpret_cast<float*>(w);
    w += align_up((size_t)std::max(p.KS_dn, ksd) * R * p.NBH * 128 * 4, 256);
    uint16_t* own_act = reinterpret_cast<uint16_t*>(w);
    a.act_rows = act_rows ? static_cast<uint16_t*>(act_rows) : own_act;
    w += align_up(R * m.I * 2, 256);
    a.xt = reinterpret_cast<uint16_t*>(w);
    a.y_rows = y_rows;
    a.KS_gu = p.KS_gu; a.KS_dn = p.KS_dn; a.NB = p.NB; a.NBH = p.NBH; a.R_max = p.R_max;
    a.NE = m.E + (m.shared ? 1 : 0);
    a.out = combine_out; a.w = static_cast<const uint16_t*>(combine_w); a.inv = r->inv; a.offsets = r->offsets;
    a.T = m.T; a.topk = m.topk; a.has_shared = m.shared;
    a.fresh = m.fresh;
    a.sh_gate = m.shared_gate;
    a.filter = 0;
    a.act_in_down = 0;
    a.gu_half = 0;
    a.split_min = split_min_rows();
    a.split_ratio2 = split_ratio2() > 0 ? split_ratio2() : 1 << 30;
    a.split_chunks = (m.T + 31) / 32;          // an expert has at most one row per token
    a.KS_gu_mid = ksg;
    a.KS_dn_mid = ksd;
    a.counts = r->counts; a.uexp = r->uexp; a.nuniq = r->nuniq;
    GvArgs b = a;                              // the mid-size kernel's view: its own k-splits
    b.KS_gu = ksg;
    b.KS_dn = ksd;
    const int nu_max = (int)std::min<long>((long)m.T * m.topk, m.E) + (m.shared ? 1 : 0);
    const int MR = rows_per_group_of(m.T);
    auto gemv = [&](int st) {
        switch (MR)
        {
            case 1: launch_mr<1>(a, p, st, s, nullptr); break;
            case 2: launch_mr<2>(a, p, st, s, nullptr); break;
            case 4: launch_mr<4>(a, p, st, s, nullptr); break;
            default: launch_mr<8>(a, p, st, s, nullptr); break;
        }
    };
    // the heavy rows' rotation: a kernel of its own when single experts can be heavy; otherwise the gate / up GEMV's
    // launch does it when the call goes to the mid-size kernel (its groups are idle then)
    if ((stages & (1 << BMX_STAGE_PREP)) && a.split_min <= m.T) launch_split_mid(b, BMX_STAGE_PREP, nu_max, s);
    for (int f = 0; f < 3; ++f)
    {
        const int st = f == 0 ? BMX_STAGE_GATE_UP : f == 1 ? BMX_STAGE_GATE_UP_RESIDENT : BMX_STAGE_GATE_UP_STAGED;
        if (!(stages & (1 << st))) continue;
        gemv(1 << st);
        GvArgs bf = b;
        bf.filter = f;
        launch_split_mid(bf, st, nu_max, s);
    }
    if (stages & (1 << BMX_STAGE_ACT)) launch_epilogue(a, BMX_STAGE_ACT, s);
    for (int f = 0; f < 3; ++f)
    {
        const int st = f == 0 ? BMX_STAGE_DOWN : f == 1 ? BMX_STAGE_DOWN_RESIDENT : BMX_STAGE_DOWN_STAGED;
        if (!(stages & (1 << st))) continue;
        gemv(1 << st);
        GvArgs bf = b;
        bf.filter = f;
        launch_split_mid(bf, st, nu_max, s);
    }
    if (stages & (1 << BMX_STAGE_COMBINE)) launch_epilogue(a, BMX_STAGE_COMBINE, s);
    if (stages & (1 << BMX_STAGE_DOWN_OUT)) launch_epilogue(a, BMX_STAGE_DOWN_OUT, s);
    return check_launch("moe experts (split path)");
}

}  // namespace bmx
