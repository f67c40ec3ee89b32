// Prefill-size expert products: grouped GEMMs on the MFMA units over EXL3 trellis weights, each weight decoded once per
// workgroup into LDS in the MFMA operand layout.
//
// Work unit = (group of <= 128 dispatch rows of one expert, output columns). One workgroup of 4 waves walks K in steps
// of 64 (4 tile-rows): every lane decodes one 64-weight strip of a 16 x 16 tile straight from coalesced trellis reads
// (the decode path's strip mapping: half a wave per tile-row of 8 tiles, four lanes per tile) and stores it as B operand
// fragments of v_mfma_f32_32x32x16_f16 into one of two LDS stages; after one barrier the 4 waves, arranged 2 (rows) x 2
// (columns), run the MFMAs of that step with A fragments read from global memory. fp32 accumulation; each output
// element is one fixed sum (k ascending in MFMA blocks), independent of scheduling.
//
//   k_pf_prep     : rotated gate / up inputs of every dispatch row, xt = RN16(H128(x * suh) * R)
//   k_pf_gemm<2>  : gate and up products of one 128-column block -> fp32 [row][block][gate | up][128]
//   (k_gu_epi)    : fp16 gate / up -> epilogue -> fp16 down-input rows (shared with the decode path)
//   k_pf_gemm<1>  : down products of two 128-column blocks -> fp32 [row][block][128]
//   (k_dn_combine): rotation * svh, slots summed in slot order (shared with the decode path)
#include "moe_kernels.hpp"

namespace bmx {

constexpr int PF_THREADS = 256;
constexpr int PF_M = 128;                    // rows per group
constexpr int PF_STAGE_U4 = 2 * 4 * 4 * 64;  // one LDS stage: [matrix 2][tile-row 4][32-column block 4][lane 64] x 16 B

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4* gptr_u32x4;

__device__ __forceinline__ u32x4 ldg4(const void* p)
{
    return *reinterpret_cast<gptr_u32x4>(reinterpret_cast<uintptr_t>(p));
}

// Workgroups are handed to the 8 XCDs round-robin (block b runs on XCD b % 8). Renumber so that consecutive logical
// blocks share an XCD: the column blocks of one row group then read the group's A rows through the same L2.
__device__ __forceinline__ int xcd_block(int bid, int nblk)
{
    const int q = nblk / 8, rem = nblk % 8, xcd = bid % 8, i = bid / 8;
    return (xcd < rem ? xcd * (q + 1) : rem * (q + 1) + (xcd - rem) * q) + i;
}

// ---- rotated inputs: one wave per (row, matrix) ----------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pf_prep(GvArgs a)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int u = blockIdx.x * 4 + wave;
    const int r = u >> 1, mat = u & 1;
    if (r >= a.offsets[a.NE]) return;
    const int e = a.row_expert[r];
    const bmx_expert& ex = e == a.E ? *a.shared : a.experts[e];
    const uint16_t* xr = a.x + (size_t)a.row_token[r] * a.H;
    const uint16_t* su = reinterpret_cast<const uint16_t*>(ex.suh[mat]);
    uint32_t* dst = reinterpret_cast<uint32_t*>(a.xt + ((size_t)mat * a.R_max + r) * a.H);
    for (int b = 0; b < a.H / 128; ++b)
    {
        const int k = b * 128 + 2 * lane;
        const uint32_t xv = ldg(xr + k, 0);
        const uint32_t sv = ldg(su + k, 0);
        float v0 = h2f(xv & 0xffffu) * h2f(sv & 0xffffu), v1 = h2f(xv >> 16) * h2f(sv >> 16);
        had128_wave(v0, v1);
        dst[b * 64 + lane] = (uint32_t)f2h_r(v0 * R_SCALE) | ((uint32_t)f2h_r(v1 * R_SCALE) << 16);
    }
}

// ---- B operand: one strip decoded into fragments ----------------------------------------------------------------------
// Fragment (matrix, tile-row kt, 32-column block nb) holds, for MFMA lane L, the 8 input rows 8 (L / 32) .. + 7 of column
// 32 nb + L % 32 as 4 dwords (rows 2d, 2d + 1 in dword d). A strip's column c supplies two fragments' worth (rows 0-7 and
// 8-15); they are written as soon as the column is complete.
template <int F>
__device__ __forceinline__ void decode_to_lds(const uint32_t (&own)[Fmt<F>::TB / 16], u32x4* stage, int mat, int kt)
{
    constexpr int NW = Fmt<F>::TB / 16;
    constexpr RingTab<F> tab;
    const int lane = threadIdx.x & 63;
    const uint32_t prev = __builtin_amdgcn_mov_dpp(own[NW - 1], 0x93, 0xf, 0xf, false);
#pragma unroll
    for (int half = 0; half < 2; ++half)
    {
        // positions 32 half .. 32 half + 31 complete columns c = half and half + 2
        uint32_t fr[2][8];
#pragma unroll
        for (int jj = 32 * half; jj < 32 * half + 32; jj += 2)
        {
            const f16x2 w2 = cb_pair(cb_hash(win_state(prev, own, tab.q[jj])), cb_hash(win_state(prev, own, tab.q[jj + 1])));
            fr[strip_cidx(jj) >> 1][strip_dw(jj)] = __builtin_bit_cast(uint32_t, w2);
        }
#pragma unroll
        for (int ci = 0; ci < 2; ++ci)
        {
            const int col = lane_col(lane, half + 2 * ci);
            u32x4* f = stage + ((mat * 4 + kt) * 4 + (col >> 5)) * 64 + (col & 31);
            f[0] = u32x4{fr[ci][0], fr[ci][1], fr[ci][2], fr[ci][3]};
            f[32] = u32x4{fr[ci][4], fr[ci][5], fr[ci][6], fr[ci][7]};
        }
    }
}

// ---- grouped GEMM ----------------------------------------------------------------------------------------------------
// NM = 2: gate and up of 128-column block cb (A = the matrix's rotated rows); NM = 1: down, 128-column blocks 2 cb and
// 2 cb + 1 (A = the down-input rows for both). Wave w: MFMA rows 64 (w & 1) .. + 63 and 32-column blocks 2 (w >> 1),
// 2 (w >> 1) + 1 of both matrices; decode of matrix w >> 1, tile-rows 2 (w & 1) + (lane >> 5) of each step.
struct PfWave {
    const uint16_t* arow[2][2];   // [A source][row block] lane's A row (+ its k offset)
    bool mvalid[2];               // row block has rows
    bool bvalid;                  // second matrix exists (down with an odd block count: the last one does not)
};

template <int NM>
__device__ __forceinline__ void mfma_step(const u32x4* stage, const PfWave& wv, int k0, f32x16 (&acc)[2][2][2])
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wn = wave >> 1;
    constexpr int NA = NM == 2 ? 2 : 1;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
    {
        f16x8 af[NA][2];
#pragma unroll
        for (int m = 0; m < NA; ++m)
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) af[m][mb] = __builtin_bit_cast(f16x8, ldg4(wv.arow[m][mb] + k0 + 16 * ks));
#pragma unroll
        for (int mat = 0; mat < 2; ++mat)
        {
            if (mat == 1 && !wv.bvalid) continue;
#pragma unroll
            for (int nb2 = 0; nb2 < 2; ++nb2)
            {
                const f16x8 bf = __builtin_bit_cast(f16x8, stage[((mat * 4 + ks) * 4 + 2 * wn + nb2) * 64 + lane]);
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
                    if (wv.mvalid[mb])
                        acc[mat][mb][nb2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[NM == 2 ? mat : 0][mb], bf,
                                                                                   acc[mat][mb][nb2], 0, 0, 0);
            }
        }
    }
}

template <int F, int NM>
__device__ __forceinline__ void pf_loop(u32x4 (*stages)[PF_STAGE_U4], const uint8_t* mat_base, int tn, int dcb,
                                        bool dvalid, int K, const PfWave& wv, f32x16 (&acc)[2][2][2])
{
    constexpr int TB = Fmt<F>::TB, NW = TB / 16;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h = lane >> 5, t = (lane >> 2) & 7, s = lane & 3;
    const int dmat = wave >> 1, kt = 2 * (wave & 1) + h;
    const size_t row_bytes = (size_t)tn * TB;
    const uint8_t* p = mat_base + (size_t)kt * row_bytes + (size_t)(dcb * 8 + t) * TB + s * (TB / 4);
    const int KT = K / 64;
    uint32_t wa[NW], wb[NW];
    if (dvalid) load_words(wa, p);
    for (int it = 0; it < KT; it += 2)
    {
        if (dvalid && it + 1 < KT) load_words(wb, p + 4 * row_bytes);
        if (dvalid) decode_to_lds<F>(wa, stages[0], dmat, kt);
        __syncthreads();
        mfma_step<NM>(stages[0], wv, it * 64, acc);
        if (it + 1 < KT)
        {
            if (dvalid && it + 2 < KT) load_words(wa, p + 8 * row_bytes);
            if (dvalid) decode_to_lds<F>(wb, stages[1], dmat, kt);
            __syncthreads();
            mfma_step<NM>(stages[1], wv, (it + 1) * 64, acc);
        }
        p += 8 * row_bytes;
    }
}

template <int NM>
__global__ __launch_bounds__(PF_THREADS) __attribute__((amdgpu_waves_per_eu(2))) void k_pf_gemm(GvArgs a)
{
    __shared__ u32x4 stages[2][PF_STAGE_U4];
    const int NBX = NM == 2 ? a.NB : (a.NBH + 1) / 2;
    const int lid = xcd_block(blockIdx.x, gridDim.x);
    const int g = lid / NBX, cb = lid % NBX;
    if (g >= *a.ngroups) return;
    const int e = a.groups[3 * g], r0 = a.groups[3 * g + 1], nr = a.groups[3 * g + 2];
    const bmx_expert& ex = e == a.E ? *a.shared : a.experts[e];
    const int K = NM == 2 ? a.H : a.I, N = NM == 2 ? a.I : a.H;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wm = wave & 1, wn = wave >> 1;

    PfWave wv;
    const int lk = (lane >> 5) * 8;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
    {
        const int row0 = 64 * wm + 32 * mb;
        wv.mvalid[mb] = row0 < nr;
        // rows past the group's end read its last row (their products are not stored)
        const int row = r0 + min(row0 + (lane & 31), nr - 1);
        if (NM == 2)
        {
            wv.arow[0][mb] = a.xt + (size_t)row * a.H + lk;
            wv.arow[1][mb] = a.xt + ((size_t)a.R_max + row) * a.H + lk;
        }
        else
        {
            wv.arow[0][mb] = a.act_rows + (size_t)row * a.I + lk;
            wv.arow[1][mb] = wv.arow[0][mb];
        }
    }
    wv.bvalid = NM == 2 || 2 * cb + 1 < a.NBH;

    // decode role
    const int dmat = wave >> 1;
    const int mi = NM == 2 ? dmat : 2;
    const int dcb = NM == 2 ? cb : 2 * cb + dmat;
    const bool dvalid = dcb < N / 128;
    const uint8_t* base = reinterpret_cast<const uint8_t*>(ex.tr[mi]);

    f32x16 acc[2][2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int k = 0; k < 2; ++k) acc[i][j][k] = f32x16{};
    switch (ex.fmt[mi])
    {
        case BMX_TF_K2: pf_loop<BMX_TF_K2, NM>(stages, base, N / 16, dcb, dvalid, K, wv, acc); break;
        case BMX_TF_K25: pf_loop<BMX_TF_K25, NM>(stages, base, N / 16, dcb, dvalid, K, wv, acc); break;
        case BMX_TF_K3: pf_loop<BMX_TF_K3, NM>(stages, base, N / 16, dcb, dvalid, K, wv, acc); break;
        default: pf_loop<BMX_TF_K4, NM>(stages, base, N / 16, dcb, dvalid, K, wv, acc); break;
    }

    // accumulator element v of lane L: row 8 (v / 4) + 4 (L / 32) + v % 4, column L % 32 of its 32 x 32 block
#pragma unroll
    for (int mat = 0; mat < 2; ++mat)
    {
        if (mat == 1 && !wv.bvalid) continue;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
        {
            if (!wv.mvalid[mb]) continue;
#pragma unroll
            for (int nb2 = 0; nb2 < 2; ++nb2)
            {
                const int col = 32 * (2 * wn + nb2) + (lane & 31);
#pragma unroll
                for (int v = 0; v < 16; ++v)
                {
                    const int row = 64 * wm + 32 * mb + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                    if (row >= nr) continue;
                    const size_t r = (size_t)(r0 + row);
                    if (NM == 2) a.part_gu[(r * a.NB + cb) * 256 + mat * 128 + col] = acc[mat][mb][nb2][v];
                    else a.part_dn[(r * a.NBH + 2 * cb + mat) * 128 + col] = acc[mat][mb][nb2][v];
                }
            }
        }
    }
}

// ---- plan and launch -------------------------------------------------------------------------------------------------
struct PrefillPlan {
    int NB, NBH, NBX_dn, G_max, R_max;
    size_t xt_bytes, part_gu_bytes, act_bytes, part_dn_bytes;
};

static PrefillPlan prefill_plan(const MoeShape& m)
{
    PrefillPlan p;
    p.NB = m.I / 128;
    p.NBH = m.H / 128;
    p.NBX_dn = (p.NBH + 1) / 2;
    p.G_max = groups_max(m.T, m.topk, m.E, m.shared, PF_M);
    p.R_max = m.T * m.topk + (m.shared ? m.T : 0);
    p.xt_bytes = (size_t)2 * p.R_max * m.H * 2;
    p.part_gu_bytes = (size_t)p.R_max * p.NB * 256 * 4;
    p.act_bytes = (size_t)p.R_max * m.I * 2;
    p.part_dn_bytes = (size_t)p.R_max * p.NBH * 128 * 4;
    return p;
}

int prefill_rows_per_group() { return PF_M; }

size_t prefill_ws_bytes(const MoeShape& m)
{
    const PrefillPlan p = prefill_plan(m);
    return align_up(p.xt_bytes, 256) + align_up(p.part_gu_bytes, 256) + align_up(p.act_bytes, 256) +
           align_up(p.part_dn_bytes, 256);
}

int launch_prefill_experts(const MoeShape& m, const void* x, const bmx_routes* r, float* y_rows, void* act_rows,
                           void* ws, size_t ws_bytes, float* combine_out, const void* combine_w, hipStream_t s,
                           int stages)
{
    if (m.H % 128 || m.I % 128 || m.H <= 0 || m.I <= 0)
        return set_error(BMX_ERR_ARG, "moe experts: H (%d) and I (%d) must be multiples of 128", m.H, m.I);
    if (ws_bytes < prefill_ws_bytes(m))
        return set_error(BMX_ERR_WORKSPACE, "moe experts: workspace %zu < %zu", ws_bytes, prefill_ws_bytes(m));
    if (!r->row_expert) return set_error(BMX_ERR_ARG, "moe experts: routes without row_expert");
    const PrefillPlan p = prefill_plan(m);
    char* w = static_cast<char*>(ws);
    GvArgs a;
    a.experts = m.experts; a.shared = m.shared_ex; a.E = m.E; a.H = m.H; a.I = m.I; a.act = m.act; a.gated = m.gated;
    a.limit = m.limit;
    a.x = static_cast<const uint16_t*>(x);
    a.row_token = r->row_token; a.groups = r->groups; a.ngroups = r->ngroups; a.row_expert = r->row_expert;
    a.xt = reinterpret_cast<uint16_t*>(w);
    w += align_up(p.xt_bytes, 256);
    a.part_gu = reinterpret_cast<float*>(w);
    w += align_up(p.part_gu_bytes, 256);
    a.act_rows = act_rows ? static_cast<uint16_t*>(act_rows) : reinterpret_cast<uint16_t*>(w);
    w += align_up(p.act_bytes, 256);
    a.part_dn = reinterpret_cast<float*>(w);
    a.y_rows = y_rows;
    a.KS_gu = 1; a.KS_dn = 1; a.NB = p.NB; a.NBH = p.NBH; a.R_max = p.R_max;
    a.NE = m.E + (m.shared ? 1 : 0);
    a.out = combine_out; a.w = static_cast<const uint16_t*>(combine_w); a.inv = r->inv; a.offsets = r->offsets;
    a.T = m.T; a.topk = m.topk; a.has_shared = m.shared;
    int rc = BMX_OK;
    if (stages & (1 << BMX_STAGE_PREP))
        hipLaunchKernelGGL(k_pf_prep, dim3((unsigned)((2 * p.R_max + 3) / 4)), dim3(256), 0, s, a);
    if (stages & (1 << BMX_STAGE_GATE_UP))
        hipLaunchKernelGGL(k_pf_gemm<2>, dim3((unsigned)(p.G_max * p.NB)), dim3(PF_THREADS), 0, s, a);
    if (stages & (1 << BMX_STAGE_ACT)) rc = launch_epilogue(a, BMX_STAGE_ACT, s);
    if (!rc && (stages & (1 << BMX_STAGE_DOWN)))
        hipLaunchKernelGGL(k_pf_gemm<1>, dim3((unsigned)(p.G_max * p.NBX_dn)), dim3(PF_THREADS), 0, s, a);
    if (!rc && (stages & (1 << BMX_STAGE_COMBINE))) rc = launch_epilogue(a, BMX_STAGE_COMBINE, s);
    if (!rc && (stages & (1 << BMX_STAGE_DOWN_OUT))) rc = launch_epilogue(a, BMX_STAGE_DOWN_OUT, s);
    if (rc) return rc;
    return check_launch("moe experts (prefill path)");
}

}  // namespace bmx
