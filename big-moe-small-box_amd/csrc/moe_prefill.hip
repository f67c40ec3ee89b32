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
//   k_pf_prep_tok : rotated gate / up inputs of every dispatch row, xt = RN16(H128(x * suh) * R), token-major
//   k_pf_gemm<false> : gate or up products of one 256-column block -> fp32 [row][128-block][gate | up][128]
//   (k_gu_epi)    : fp16 gate / up -> epilogue -> fp16 down-input rows (shared with the decode path)
//   k_pf_gemm<true>  : down products of one 256-column block -> fp32 [row][128-block][128]
//   (k_dn_combine): rotation * svh, slots summed in slot order (shared with the decode path)
#include "moe_kernels.hpp"

#include <algorithm>

namespace bmx {

constexpr int PF_M = 128;                    // rows per group

// Workgroups are handed to the 8 XCDs round-robin (block b runs on XCD b % 8). Renumber so that chunks of 16
// consecutive logical blocks (the column blocks of one row group) share an XCD, and the chunks go round-robin over the
// XCDs: a group's units read its A rows through one L2, and the groups that exist (the grid is sized for the most a batch
// can have) spread over all XCDs. Blocks past the last whole 128-block round keep their number.
__device__ __forceinline__ int xcd_block(int bid, int nblk)
{
    constexpr int C = 16;
    if (bid >= nblk / (8 * C) * (8 * C)) return bid;
    const int xcd = bid % 8, i = bid / 8;
    return ((i / C) * 8 + xcd) * C + i % C;
}

// ---- rotated inputs: 16 lanes per (row, matrix, run of PREP_BPU 128-blocks), 8 consecutive inputs per lane -------------
__global__ __launch_bounds__(256) void k_pf_prep(GvArgs a)
{
    prep_unit(a, (long)blockIdx.x * 16 + (threadIdx.x >> 4));
}

static dim3 prep_grid(int R_max, int H)
{
    return dim3((unsigned)(((long)2 * R_max * ((H / 128 + PREP_BPU - 1) / PREP_BPU) + 15) / 16));
}

// ---- rotated inputs, token-major (the prefill path) --------------------------------------------------------------------
// Unit u = (token, run of PREP_BPU 128-blocks) by a 16-lane group: the token's inputs are loaded once and rotated into
// the rows of all its picks and its shared-expert row, gate and up (the same values as prep_unit, which reads the
// token's inputs once per row and matrix, 12 times at top-6: 441 MB of HBM reads for C3's 805 MB of rows, 205 MB
// here). Lane j first fetches slot k0 + j's row and its expert's suh addresses, so the dependent index loads run once
// per 16 slots, side by side; the slot loop takes them by shuffles within the group.
__device__ __forceinline__ void prep_tok_unit(const GvArgs& a, long u)
{
    const int nblk = a.H / 128, nrun = (nblk + PREP_BPU - 1) / PREP_BPU;
    const int j = threadIdx.x & 15, run = (int)(u % nrun);
    const long t = u / nrun;
    if (t >= a.T) return;                 // the whole 16-lane group: the shuffles below stay inside it
    float xv[PREP_BPU][8];
    const uint16_t* xr = a.x + (size_t)t * a.H + 8 * j;
#pragma unroll
    for (int i = 0; i < PREP_BPU; ++i)
        if (run * PREP_BPU + i < nblk) unpack8(ldg4(xr + 128 * (run * PREP_BPU + i)), xv[i]);
    const int ns = a.topk + (a.has_shared ? 1 : 0);
    for (int k0 = 0; k0 < ns; k0 += 16)
    {
        const int kj = k0 + j;
        int rj = -1;
        if (kj < a.topk) rj = a.inv[t * a.topk + kj];
        else if (kj < ns) rj = a.offsets[a.E] + (int)t;
        uint64_t su0 = 0, su1 = 0;
        if (rj >= 0)
        {
            const int e = a.row_expert[rj];
            const bmx_expert& ex = e == a.E ? *a.shared : a.experts[e];
            su0 = reinterpret_cast<uint64_t>(ex.suh[0]);
            su1 = reinterpret_cast<uint64_t>(ex.suh[1]);
        }
        const int kn = ns - k0 < 16 ? ns - k0 : 16;
        for (int k = 0; k < kn; ++k)
        {
            const int r = __shfl(rj, k, 16);
            if (r < 0) continue;              // a dropped pick: no row
#pragma unroll
            for (int mat = 0; mat < 2; ++mat)
            {
                const uint64_t sa = mat ? su1 : su0;
                const uint32_t lo = __shfl((uint32_t)sa, k, 16), hi = __shfl((uint32_t)(sa >> 32), k, 16);
                const uint16_t* su = reinterpret_cast<const uint16_t*>(((uint64_t)hi << 32) | lo) + 8 * j;
                uint16_t* dst = a.xt + ((size_t)mat * a.R_max + r) * a.H + 8 * j;
#pragma unroll
                for (int i = 0; i < PREP_BPU; ++i)
                {
                    const int b = run * PREP_BPU + i;
                    if (b >= nblk) break;
                    float v[8], s[8];
                    unpack8(ldg4(su + 128 * b), s);
#pragma unroll
                    for (int q = 0; q < 8; ++q) v[q] = xv[i][q] * s[q];
                    had128_x8(v);
#pragma unroll
                    for (int q = 0; q < 8; ++q) v[q] = v[q] * (R_SCALE * had128_x8_sign());
                    __builtin_nontemporal_store(pack8_r(v), reinterpret_cast<u32x4*>(dst + 128 * b));
                }
            }
        }
    }
}

__global__ __launch_bounds__(256) void k_pf_prep_tok(GvArgs a)
{
    prep_tok_unit(a, (long)blockIdx.x * 16 + (threadIdx.x >> 4));
}

static dim3 prep_tok_grid(int T, int H)
{
    const long units = (long)T * ((H / 128 + PREP_BPU - 1) / PREP_BPU);
    return dim3((unsigned)std::max(1L, (units + 15) / 16));
}

// ---- LDS stages ------------------------------------------------------------------------------------------------------
// A stage: [row 128 (256 for a pair of groups)][8 chunks of 16 B] = the k-step's 64 inputs of every row; chunk c of row
//          r sits at slot c ^ ((r >> 1) & 7) of the row, so that the 16 lanes an LDS cycle serves (16 rows, one chunk)
//          hit 16 different 16-byte bank groups. Copied by the decode waves (each lane 32 B of a row per 16 rows) from
//          registers loaded two steps ahead.
// B stage: fragment f = tile-row * 8 + 32-column block (of the 256; of the 128 for a pair), 64 lanes x 16 B; lane L's
//          16 B at slot f * 64 + bsw(f, L), bsw(f, L) = L ^ ((L >> 4) & 1) ^ ((f & 1) << 3): a bijection on each 16-lane
//          block (the MFMA reads stay conflict-free) that spreads the 16 lanes of a decode store over 16 bank groups.
constexpr int PF_A_U4 = 2 * PF_M * 8;
constexpr int PF_B_U4 = 4 * 8 * 64;
__shared__ u32x4 pf_a0[PF_A_U4];
__shared__ u32x4 pf_a1[PF_A_U4];
__shared__ u32x4 pf_b0[PF_B_U4];
__shared__ u32x4 pf_b1[PF_B_U4];

__device__ __forceinline__ u32x4* a_stage(int s) { return s == 0 ? pf_a0 : pf_a1; }
__device__ __forceinline__ u32x4* b_stage(int s) { return s == 0 ? pf_b0 : pf_b1; }
__device__ __forceinline__ int bsw(int f, int L) { return L ^ ((L >> 4) & 1) ^ ((f & 1) << 3); }

// Step barrier: the wave's LDS operations are done (its global loads, register prefetches for later steps, may still be in
// flight; the compiler waits for those where their registers are used).
__device__ __forceinline__ void step_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0); vmcnt (63) and expcnt (7) at their maxima: no wait
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// ---- B operand: half a strip decoded into fragments -------------------------------------------------------------------
// Fragment (tile-row kt, 32-column block nb) holds, for MFMA lane L, the 8 input rows 8 (L / 32) .. + 7 of column
// 32 nb + L % 32 as 4 dwords (rows 2d, 2d + 1 in dword d). Stream positions 32 HALF .. 32 HALF + 31 of a lane's strip are
// columns HALF and HALF + 2 of its four, all 16 rows: two columns' worth of fragments. col0: the first column of the
// lane's 128-column half of the block.
// The lane index as a value the compiler cannot hoist: LDS addresses derived from it are recomputed where they are used
// (a few VALU per step) instead of being kept live across the k-loop, which costs the mid-size kernel its occupancy.
__device__ __forceinline__ int fresh_lane()
{
    int l = threadIdx.x & 63;
    asm volatile("" : "+v"(l));
    return l;
}

template <int F, int HALF>
__device__ __forceinline__ void decode_half(const uint32_t (&own)[Fmt<F>::TB / 16], u32x4* __restrict__ stage, int kt,
                                            int col0, int lane)
{
    constexpr int NW = Fmt<F>::TB / 16;
    // every word of the window is consumed here (a half strip reads only some of them): keeps the prefetched registers
    // allocated until now instead of reused while their load is in flight, which would force a wait on it
#pragma unroll
    for (int k = 0; k < NW; ++k) asm volatile("" :: "v"(own[k]));
    const uint32_t prev = __builtin_amdgcn_mov_dpp(own[NW - 1], 0x93, 0xf, 0xf, false);
    uint32_t fr[2][8];
#pragma unroll
    for (int j8 = 32 * HALF; j8 < 32 * HALF + 32; j8 += 8)
    {
        uint32_t w[4];
        oct_weights<F>(prev, own, j8, w);
#pragma unroll
        for (int q = 0; q < 4; ++q) fr[strip_cidx(j8 + 2 * q) >> 1][strip_dw(j8 + 2 * q)] = w[q];
    }
#pragma unroll
    for (int ci = 0; ci < 2; ++ci)
    {
        const int col = col0 + lane_col(lane, HALF + 2 * ci);
        const int f = kt * 8 + (col >> 5);
        u32x4* fp = stage + f * 64;
        fp[bsw(f, col & 31)] = u32x4{fr[ci][0], fr[ci][1], fr[ci][2], fr[ci][3]};
        fp[bsw(f, (col & 31) + 32)] = u32x4{fr[ci][4], fr[ci][5], fr[ci][6], fr[ci][7]};
    }
}

// A quarter strip: stream positions 32 HALF + 16 SUB .. + 15, the same two columns as decode_half<F, HALF> but only
// input rows 4 SUB .. + 3 and 8 + 4 SUB .. + 3 (dwords 2 SUB, 2 SUB + 1 of each of the column's two fragment slots).
template <int F, int HALF, int SUB>
__device__ __forceinline__ void decode_quarter(const uint32_t (&own)[Fmt<F>::TB / 16], u32x4* __restrict__ stage, int kt,
                                               int col0)
{
    constexpr int NW = Fmt<F>::TB / 16;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < NW; ++k) asm volatile("" :: "v"(own[k]));
    const uint32_t prev = __builtin_amdgcn_mov_dpp(own[NW - 1], 0x93, 0xf, 0xf, false);
    uint32_t fr[2][4];      // [column][dword 2 SUB, 2 SUB + 1 of rows 0-7, then of rows 8-15]
#pragma unroll
    for (int j8 = 32 * HALF + 16 * SUB; j8 < 32 * HALF + 16 * SUB + 16; j8 += 8)
    {
        uint32_t w[4];
        oct_weights<F>(prev, own, j8, w);
#pragma unroll
        for (int q = 0; q < 4; ++q)
        {
            const int dw = strip_dw(j8 + 2 * q);
            fr[strip_cidx(j8 + 2 * q) >> 1][((dw >> 2) << 1) + (dw & 1)] = w[q];
        }
    }
#pragma unroll
    for (int ci = 0; ci < 2; ++ci)
    {
        const int col = col0 + lane_col(lane, HALF + 2 * ci);
        const int f = kt * 8 + (col >> 5);
        u32x4* fp = stage + f * 64;
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint32_t*>(fp + bsw(f, col & 31)) + 2 * SUB) = u32x2{fr[ci][0], fr[ci][1]};
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint32_t*>(fp + bsw(f, (col & 31) + 32)) + 2 * SUB) =
            u32x2{fr[ci][2], fr[ci][3]};
    }
}

// ---- grouped GEMM ----------------------------------------------------------------------------------------------------
// Work unit: (group of <= 128 rows, matrix, 256-column block); 12 waves, one barrier per k-step (64 k). While waves 0-3
// run the MFMAs of step i from A / B stage i % 2, waves 4-11 stage step i + 1: they store the A rows loaded two steps
// earlier and the B fragments decoded from trellis words loaded two steps earlier, and issue the loads of step i + 3.
// Each SIMD holds one MFMA wave and two decode waves, so the decode (VALU; two waves hide its latency) overlaps the MFMAs.
//   MFMA wave w: rows 64 (w & 1) .. + 63 (2 row blocks) x columns 128 (w >> 1) .. + 127 (4 column blocks).
//   decode wave 4 + d: tile-rows 2 (d >> 2) + (lane >> 5), 128-column half (d >> 1) & 1, strip half d & 1; A rows
//     16 d .. 16 d + 15, 32 B per lane.
// DOWN = false: gate (matrix 0) or up (1) of the rotated input rows; DOWN = true: down of the down-input rows.
constexpr int PF_WAVES = 12;

// cb: the 256-column block of one group's unit; the 128-column block of a pair's (pair = 1)
struct PfJob {
    int g, mat, cb, e, r0, nr, K, N, nb128, pair;
    const bmx_expert* ex;
};

// An MFMA wave multiplies the 32-row blocks that hold rows of the group (rows past the group's end inside such a block
// hold copies of its last row) and all its columns (a missing second 128-column half holds stale LDS); neither padding
// is stored. A wave's tile: MBW 32-row blocks x NBW 32-column blocks (2 x 4 for one group's 128 x 256 tile, 4 x 2 for a
// pair's 256 x 128), the waves 2 (rows, wave & 1) x 2 (columns, wave >> 1).
template <int MBW, int NBW>
struct PfFrag {
    f16x8 a[MBW];    // [row block]
    f16x8 b[NBW];    // [column block]
};

// NMB: row blocks of 32 this wave computes (MBW; fewer when the group's rows end inside the wave's blocks)
template <int MBW, int NBW, int NMB>
__device__ __forceinline__ void pf_frag_load(PfFrag<MBW, NBW>& f, const u32x4* __restrict__ sa, const u32x4* __restrict__ sb,
                                             int ks)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wm = wave & 1, wn = wave >> 1;
    const int slot = (2 * ks + (lane >> 5)) ^ ((lane >> 1) & 7);
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb)
        f.a[mb] = __builtin_bit_cast(f16x8, sa[(32 * MBW * wm + 32 * mb + (lane & 31)) * 8 + slot]);
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb)
    {
        const int fi = ks * 8 + NBW * wn + nb;
        f.b[nb] = __builtin_bit_cast(f16x8, sb[fi * 64 + bsw(fi, lane)]);
    }
}

template <int MBW, int NBW, int NMB>
__device__ __forceinline__ void pf_frag_mfma(const PfFrag<MBW, NBW>& f, f32x16 (&acc)[MBW][NBW])
{
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb)
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
            acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[mb], f.b[nb], acc[mb][nb], 0, 0, 0);
}

// one k-step of an MFMA wave: 4 sub-steps of 16 k, the fragments of sub-step ks + 1 read while those of ks feed the MFMAs
template <int MBW, int NBW, int NMB>
__device__ __forceinline__ void pf_mfma_step(const u32x4* __restrict__ sa, const u32x4* __restrict__ sb,
                                             f32x16 (&acc)[MBW][NBW])
{
    PfFrag<MBW, NBW> f0, f1;
    pf_frag_load<MBW, NBW, NMB>(f0, sa, sb, 0);
    pf_frag_load<MBW, NBW, NMB>(f1, sa, sb, 1);
    pf_frag_mfma<MBW, NBW, NMB>(f0, acc);
    pf_frag_load<MBW, NBW, NMB>(f0, sa, sb, 2);
    pf_frag_mfma<MBW, NBW, NMB>(f1, acc);
    pf_frag_load<MBW, NBW, NMB>(f1, sa, sb, 3);
    pf_frag_mfma<MBW, NBW, NMB>(f0, acc);
    pf_frag_mfma<MBW, NBW, NMB>(f1, acc);
}

// the MFMA loop over K (one barrier per step, as the decode waves)
template <int MBW, int NBW, int NMB>
__device__ __forceinline__ void pf_mfma_loop(int KT, f32x16 (&acc)[MBW][NBW])
{
    for (int i = 0; i < KT; ++i)
    {
        pf_mfma_step<MBW, NBW, NMB>(a_stage(i & 1), b_stage(i & 1), acc);
        step_barrier();
    }
}

// A rows of one k-step: lane's 32 bytes (chunks 2 (lane & 3), + 1) of row 16 d + (lane >> 2)
struct PfArow {
    u32x4 c[2];
};

__device__ __forceinline__ void a_fetch(PfArow& r, const uint16_t* rowp, int k0)
{
    const int lane = threadIdx.x & 63;
    const uint16_t* p = rowp + k0 + 16 * (lane & 3);
    r.c[0] = ldg4(p);
    r.c[1] = ldg4(p + 8);
}

__device__ __forceinline__ void a_store(const PfArow& r, u32x4* __restrict__ stage, int row)
{
    const int lane = threadIdx.x & 63, x = (row >> 1) & 7;
#pragma unroll
    for (int j = 0; j < 2; ++j) stage[row * 8 + ((2 * (lane & 3) + j) ^ x)] = r.c[j];
}

// The loop is straight-line code (every step issues the same loads, past-the-end steps re-read the last one, a missing
// second 128-column half decodes the first one's tiles again), so the compiler's wait counts for the prefetched
// registers stay exact and the waits land only where the data is two steps old.
// One group (PAIR false): decode wave 4 + d decodes strip half d & 1 of 128-column half (d >> 1) & 1 and copies A rows
// 16 d .. + 15. A pair (PAIR true, one 128-column block): strip quarter 2 HALF + SUB = d & 3, A rows 32 d .. + 31.
template <int F, int HALF, int SUB, bool PAIR, bool ACOPY>
__device__ __forceinline__ void pf_decoder(const PfJob& jb, const uint8_t* mat_base, const uint16_t* asrc, int d)
{
    constexpr int TB = Fmt<F>::TB, NW = TB / 16, NA = PAIR ? 2 : 1;
    const int lane = threadIdx.x & 63;
    const int h = lane >> 5, t = (lane >> 2) & 7, s = lane & 3;
    const int kt = 2 * (d >> 2) + h, th = (d >> 1) & 1;
    const int tcol = PAIR ? jb.cb : min(2 * jb.cb + th, jb.nb128 - 1);
    const size_t row_bytes = (size_t)(jb.N / 16) * TB, step_bytes = 4 * row_bytes;
    const uint8_t* p = mat_base + (size_t)kt * row_bytes + (size_t)(tcol * 8 + t) * TB + s * (TB / 4);
    const int KT = jb.K / 64;
    // this lane's A rows (rows past the group's end read its last row; their products are not stored)
    int arow[NA];
    const uint16_t* rowp[NA];
#pragma unroll
    for (int j = 0; j < NA; ++j)
    {
        arow[j] = 16 * NA * d + 16 * j + (lane >> 2);
        rowp[j] = asrc + (size_t)(jb.r0 + min(arow[j], jb.nr - 1)) * jb.K;
    }
    auto wp = [&](int step) { return p + (size_t)min(step, KT - 1) * step_bytes; };
    auto ak = [&](int step) { return 64 * min(step, KT - 1); };
    auto dec = [&](const uint32_t (&w)[NW], u32x4* stage) {
        if constexpr (PAIR) decode_quarter<F, HALF, SUB>(w, stage, kt, 0);
        else decode_half<F, HALF>(w, stage, kt, 128 * th, threadIdx.x & 63);
    };
    auto fetch = [&](PfArow (&a)[NA], int step) {
#pragma unroll
        for (int j = 0; j < NA; ++j) a_fetch(a[j], rowp[j], ak(step));
    };
    auto store = [&](const PfArow (&a)[NA], u32x4* stage) {
#pragma unroll
        for (int j = 0; j < NA; ++j) a_store(a[j], stage, arow[j]);
    };
    // DEPTH register sets (words and A rows) in rotation: step s is loaded into set s % DEPTH DEPTH - 1 steps before it
    // is staged. The MFMA waves set the kernel's register count; a group's decoder has the room for a fourth set up to
    // K 3 (six words a strip), a pair's (twice the A rows) or a K 4 one's (eight words) keeps three.
    constexpr int DEPTH = (PAIR || NW > 6) ? 3 : 4;
    uint32_t w[DEPTH][NW];
    PfArow ar[DEPTH][NA];
#pragma unroll
    for (int q = 0; q < DEPTH; ++q)
    {
        if (ACOPY) fetch(ar[q], q);
        load_words<false>(w[q], wp(q));
    }
    dec(w[0], pf_b0);
    if (ACOPY) store(ar[0], pf_a0);
    step_barrier();
    // sub-step q of the trip from step i: load step i + q + DEPTH into set q (staged in the sub-step before), stage step
    // i + q + 1 from set (q + 1) % DEPTH into stage (i + q + 1) % 2
    for (int i = 0; i < KT; i += DEPTH)
    {
#pragma unroll
        for (int q = 0; q < DEPTH; ++q)
        {
            if (ACOPY) fetch(ar[q], i + q + DEPTH);
            load_words<false>(w[q], wp(i + q + DEPTH));
            dec(w[(q + 1) % DEPTH], b_stage((i + q + 1) & 1));
            if (ACOPY) store(ar[(q + 1) % DEPTH], a_stage((i + q + 1) & 1));
            step_barrier();
            if (i + q + 1 >= KT) return;
        }
    }
}

// A rows are copied only where an MFMA wave reads them: the 32-row blocks that hold rows of the group
template <int F, bool PAIR>
__device__ __forceinline__ void pf_decoder_role(const PfJob& jb, const uint8_t* mat_base, const uint16_t* asrc, int d)
{
    const bool acopy = (PAIR ? 32 : 16) * d < (jb.nr + 31) / 32 * 32;
    if (PAIR)
    {
        // quarter d & 3 (a switch on a wave-uniform value: one path per wave)
        switch ((d & 3) + (acopy ? 4 : 0))
        {
            case 0: pf_decoder<F, 0, 0, true, false>(jb, mat_base, asrc, d); break;
            case 1: pf_decoder<F, 0, 1, true, false>(jb, mat_base, asrc, d); break;
            case 2: pf_decoder<F, 1, 0, true, false>(jb, mat_base, asrc, d); break;
            case 3: pf_decoder<F, 1, 1, true, false>(jb, mat_base, asrc, d); break;
            case 4: pf_decoder<F, 0, 0, true, true>(jb, mat_base, asrc, d); break;
            case 5: pf_decoder<F, 0, 1, true, true>(jb, mat_base, asrc, d); break;
            case 6: pf_decoder<F, 1, 0, true, true>(jb, mat_base, asrc, d); break;
            default: pf_decoder<F, 1, 1, true, true>(jb, mat_base, asrc, d); break;
        }
    }
    else if (acopy)
    {
        if (d & 1) pf_decoder<F, 1, 0, false, true>(jb, mat_base, asrc, d);
        else pf_decoder<F, 0, 0, false, true>(jb, mat_base, asrc, d);
    }
    else
    {
        if (d & 1) pf_decoder<F, 1, 0, false, false>(jb, mat_base, asrc, d);
        else pf_decoder<F, 0, 0, false, false>(jb, mat_base, asrc, d);
    }
}

template <int F>
__device__ __forceinline__ void pf_decoder_any(const PfJob& jb, const uint8_t* mat_base, const uint16_t* asrc)
{
    const int d = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6) - 4);
    if (jb.pair) pf_decoder_role<F, true>(jb, mat_base, asrc, d);
    else pf_decoder_role<F, false>(jb, mat_base, asrc, d);
}

// Store of an MFMA wave's products: accumulator element v of lane L is row 8 (v / 4) + 4 (L / 32) + v % 4, column L % 32
// of its 32 x 32 block; rows past the group's end are not stored.
template <bool DOWN, int MBW, int NBW>
__device__ __forceinline__ void pf_store(const GvArgs& a, const PfJob& jb, const f32x16 (&acc)[MBW][NBW])
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wm = wave & 1, wn = wave >> 1;
    // the wave's 128-column output block and its first column in it
    const int cbo = jb.pair ? jb.cb : 2 * jb.cb + wn, c0 = jb.pair ? 32 * NBW * wn : 0;
    if (cbo >= jb.nb128) return;
#pragma unroll
    for (int mb = 0; mb < MBW; ++mb)
    {
        if (32 * MBW * wm + 32 * mb >= jb.nr) continue;
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb)
        {
            const int col = c0 + 32 * nb + (lane & 31);
#pragma unroll
            for (int v = 0; v < 16; ++v)
            {
                const int row = 32 * MBW * wm + 32 * mb + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (row >= jb.nr) continue;
                const size_t r = (size_t)(jb.r0 + row);
                if (DOWN) a.part_dn[(r * a.NBH + cbo) * 128 + col] = acc[mb][nb][v];
                else
                    reinterpret_cast<uint16_t*>(a.part_gu)[(r * a.NB + cbo) * 256 + jb.mat * 128 + col] =
                        f2h_r(0.0f + acc[mb][nb][v]);
            }
        }
    }
}

// The MFMA waves of one tile shape: row blocks past the group's end are neither read nor multiplied (a wave with none
// only keeps the barriers).
template <bool DOWN, int MBW, int NBW>
__device__ __forceinline__ void pf_mfma_wave(const GvArgs& a, const PfJob& jb, int KT)
{
    const int wm = (threadIdx.x >> 6) & 1;
    f32x16 acc[MBW][NBW];
#pragma unroll
    for (int i = 0; i < MBW; ++i)
#pragma unroll
        for (int j = 0; j < NBW; ++j) acc[i][j] = f32x16{};
    const int nmb = min(MBW, max(0, (jb.nr - 32 * MBW * wm + 31) / 32));
    step_barrier();
    switch (nmb)
    {
        case 0: for (int i = 0; i < KT; ++i) step_barrier(); break;
        case 1: pf_mfma_loop<MBW, NBW, 1>(KT, acc); break;
        case 2: pf_mfma_loop<MBW, NBW, 2>(KT, acc); break;
        case 3: if constexpr (MBW >= 3) pf_mfma_loop<MBW, NBW, 3>(KT, acc); break;
        default: if constexpr (MBW >= 4) pf_mfma_loop<MBW, NBW, 4>(KT, acc); break;
    }
    pf_store<DOWN, MBW, NBW>(a, jb, acc);
}

template <bool DOWN>
__global__ __launch_bounds__(PF_WAVES * 64) void k_pf_gemm(GvArgs a)
{
    const int nb128 = DOWN ? a.NBH : a.NB;     // 128-column blocks of the output
    const int NB2 = (nb128 + 1) / 2;
    const int lid = xcd_block(blockIdx.x, gridDim.x);
    PfJob jb;
    jb.nb128 = nb128;
    if (DOWN) { jb.g = lid / NB2; jb.mat = 2; jb.cb = lid % NB2; }
    else { jb.g = lid / (2 * NB2); jb.mat = (lid / NB2) & 1; jb.cb = lid % NB2; }
    if (jb.g >= *a.ngroups) return;
    jb.e = a.groups[3 * jb.g];
    if (group_skipped(a, jb.e)) return;
    jb.r0 = a.groups[3 * jb.g + 1];
    jb.nr = a.groups[3 * jb.g + 2];
    jb.pair = 0;
    if (a.pf_pairs)
    {
        // groups 2 j and 2 j + 1 of an expert (consecutive rows) form a pair; its units are both groups' units, unit
        // (group 2 j + q, 256-column block c) taking 128-column block 2 c + q of all the pair's rows
        const int base = a.offsets[jb.e], cnt = a.offsets[jb.e + 1] - base;
        const int q = (jb.r0 - base) / PF_M, ng = (cnt + PF_M - 1) / PF_M;
        if ((q & 1) || q + 1 < ng)
        {
            const int q0 = q & ~1;
            jb.pair = 1;
            jb.r0 = base + q0 * PF_M;
            jb.nr = min(2 * PF_M, cnt - q0 * PF_M);
            jb.cb = 2 * jb.cb + (q & 1);
            if (jb.cb >= nb128) return;        // an odd block count: the last 256-column block has one half
        }
    }
    jb.ex = jb.e == a.E ? a.shared : a.experts + jb.e;
    jb.K = DOWN ? a.I : a.H;
    jb.N = DOWN ? a.H : a.I;
    const int wave = threadIdx.x >> 6;
    const int KT = jb.K / 64;

    const uint16_t* asrc = DOWN ? a.act_rows : a.xt + (size_t)jb.mat * a.R_max * a.H;
    if (wave >= 4)
    {
        const uint8_t* base = reinterpret_cast<const uint8_t*>(jb.ex->tr[jb.mat]);
        switch (jb.ex->fmt[jb.mat])
        {
            case BMX_TF_K2: pf_decoder_any<BMX_TF_K2>(jb, base, asrc); break;
            case BMX_TF_K25: pf_decoder_any<BMX_TF_K25>(jb, base, asrc); break;
            case BMX_TF_K3: pf_decoder_any<BMX_TF_K3>(jb, base, asrc); break;
            default: pf_decoder_any<BMX_TF_K4>(jb, base, asrc); break;
        }
        return;
    }
    if (jb.pair) pf_mfma_wave<DOWN, 4, 2>(a, jb, KT);
    else pf_mfma_wave<DOWN, 2, 4>(a, jb, KT);
}

// ---- mid-size grouped GEMM: groups of <= 32 rows, every wave decodes and multiplies ------------------------------------
// For decode batches of several tokens (a few rows per expert): work unit = (group of <= 32 rows, matrix, 256-column block,
// k-split). 8 waves; per k-step of 64 each wave decodes half a strip per tile-row exactly as a prefill decode wave does
// (same B fragment layout, pf_b0 / pf_b1), copies 8 bytes of the A rows, and, from the previous step's stage, runs the 4
// MFMAs (32 rows x 32 columns, k 16 each) of its 32-column block. One barrier per step; the fp32 products of each k-split
// go to the partial layout the epilogues sum in split order.
constexpr int MID_M = 32;
constexpr int MID_WAVES = 8;
constexpr int MID_A_U4 = MID_M * 8;
__shared__ u32x4 mid_a0[MID_A_U4];
__shared__ u32x4 mid_a1[MID_A_U4];
__device__ __forceinline__ u32x4* mid_a_stage(int s) { return s == 0 ? mid_a0 : mid_a1; }

struct MidArow {
    uint32_t d[2];
};

// lane's 8 bytes of the A rows of a step: row 4 wave + lane / 16, bytes 8 (lane % 16) of the row's 128 (64 inputs)
__device__ __forceinline__ void mid_a_fetch(MidArow& r, const uint16_t* rowp, int k0)
{
    const uint32_t* p = reinterpret_cast<const uint32_t*>(rowp + k0);
    r.d[0] = ldg(p, 0);
    r.d[1] = ldg(p, 1);
}

__device__ __forceinline__ void mid_a_store(const MidArow& r, u32x4* __restrict__ stage, int lane)
{
    const int row = 4 * (threadIdx.x >> 6) + (lane >> 4), piece = lane & 15;
    uint2* p = reinterpret_cast<uint2*>(stage + row * 8 + ((piece >> 1) ^ ((row >> 1) & 7))) + (piece & 1);
    *p = make_uint2(r.d[0], r.d[1]);
}

// the wave's 32-column block of one step: 4 MFMAs, k 16 each, into one accumulator (the MFMA units are lightly used
// here; a second accumulator would cost the 16 VGPRs that keep the kernel at 128)
__device__ __forceinline__ void mid_mfma_step(const u32x4* __restrict__ sa, const u32x4* __restrict__ sb, f32x16& acc,
                                              int lane)
{
    const int wave = threadIdx.x >> 6;
    f16x8 fa[4], fb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
    {
        const int slot = (2 * ks + (lane >> 5)) ^ ((lane >> 1) & 7), fi = ks * 8 + wave;
        fa[ks] = __builtin_bit_cast(f16x8, sa[(lane & 31) * 8 + slot]);
        fb[ks] = __builtin_bit_cast(f16x8, sb[fi * 64 + bsw(fi, lane)]);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[ks], fb[ks], acc, 0, 0, 0);
}

// steps s0 .. s0 + n - 1 of the unit; straight-line like pf_decoder (loads past the last step re-read it)
template <int F, int HALF>
__device__ __forceinline__ void mid_run(const PfJob& jb, const uint8_t* mat_base, const uint16_t* asrc, int s0, int n,
                                        f32x16& acc)
{
    constexpr int TB = Fmt<F>::TB, NW = TB / 16;
    const int lane = threadIdx.x & 63, d = threadIdx.x >> 6;
    const int h = lane >> 5, t = (lane >> 2) & 7, sl = lane & 3;
    const int kt = 2 * (d >> 2) + h, th = (d >> 1) & 1;
    const int tcol = min(2 * jb.cb + th, jb.nb128 - 1);
    const size_t row_bytes = (size_t)(jb.N / 16) * TB, step_bytes = 4 * row_bytes;
    const uint8_t* p = mat_base + (size_t)kt * row_bytes + (size_t)(tcol * 8 + t) * TB + sl * (TB / 4);
    const int arow = 4 * d + (lane >> 4);
    const uint16_t* rowp = asrc + (size_t)(jb.r0 + min(arow, jb.nr - 1)) * jb.K + 4 * (lane & 15);
    auto wp = [&](int i) { return p + (size_t)(s0 + min(i, n - 1)) * step_bytes; };
    auto ak = [&](int i) { return 64 * (s0 + min(i, n - 1)); };
    // the lane index once per call, opaque to the compiler: the LDS addresses derived from it are this copy's own (the
    // compiler cannot merge them above the format switch, where every copy's set would be live at once)
    const int ln = fresh_lane();
    uint32_t w0[NW], w1[NW];
    MidArow a0, a1;
    mid_a_fetch(a0, rowp, ak(0));
    mid_a_fetch(a1, rowp, ak(1));
    load_words(w0, wp(0));
    load_words(w1, wp(1));
    decode_half<F, HALF>(w0, pf_b0, kt, 128 * th, ln);
    mid_a_store(a0, mid_a0, ln);
    step_barrier();
    // step i: the MFMAs of stage i % 2, the decode of step i + 1 into the other stage, the fetch of step i + 2 (two
    // register sets: the kernel fits 128 VGPRs, so two workgroups share a CU)
    for (int i = 0; i < n; i += 2)
    {
        mid_a_fetch(a0, rowp, ak(i + 2));
        load_words(w0, wp(i + 2));
        mid_mfma_step(mid_a0, pf_b0, acc, ln);
        decode_half<F, HALF>(w1, pf_b1, kt, 128 * th, ln);
        mid_a_store(a1, mid_a1, ln);
        step_barrier();
        if (i + 1 >= n) break;
        mid_a_fetch(a1, rowp, ak(i + 3));
        load_words(w1, wp(i + 3));
        mid_mfma_step(mid_a1, pf_b1, acc, ln);
        decode_half<F, HALF>(w0, pf_b0, kt, 128 * th, ln);
        mid_a_store(a0, mid_a0, ln);
        step_barrier();
    }
}

template <int F>
__device__ __forceinline__ void mid_run_any(const PfJob& jb, const uint8_t* mat_base, const uint16_t* asrc, int s0, int n,
                                            f32x16& acc)
{
    if ((threadIdx.x >> 6) & 1) mid_run<F, 1>(jb, mat_base, asrc, s0, n, acc);
    else mid_run<F, 0>(jb, mat_base, asrc, s0, n, acc);
}

// One unit of the mid-size GEMM: (group or heavy-expert chunk, matrix, 256-column block, k-split) from its index lid.
template <bool DOWN>
__device__ __forceinline__ void mid_unit(const GvArgs& a, int lid)
{
    const int nb128 = DOWN ? a.NBH : a.NB;
    const int NB2 = (nb128 + 1) / 2, KS = DOWN ? a.KS_dn : a.KS_gu;
    const int ksp = lid % KS;
    lid /= KS;
    PfJob jb;
    jb.nb128 = nb128;
    if (DOWN) { jb.g = lid / NB2; jb.mat = 2; jb.cb = lid % NB2; }
    else { jb.g = lid / (2 * NB2); jb.mat = (lid / NB2) & 1; jb.cb = lid % NB2; }
    if (a.split_min)
    {
        // split path: units over (unique expert, chunk of 32 rows); only the heavy experts' rows are computed here
        const int u = jb.g / a.split_chunks, q = jb.g % a.split_chunks;
        if (u >= *a.nuniq) return;
        jb.e = a.uexp[u];
        const int c = a.counts[jb.e];
        if (MID_M * q >= c || !split_heavy(a, jb.e)) return;
        if (group_skipped(a, jb.e)) return;
        jb.r0 = a.offsets[jb.e] + MID_M * q;
        jb.nr = min(MID_M, c - MID_M * q);
    }
    else
    {
        if (jb.g >= *a.ngroups) return;
        jb.e = a.groups[3 * jb.g];
        if (group_skipped(a, jb.e)) return;
        jb.r0 = a.groups[3 * jb.g + 1];
        jb.nr = a.groups[3 * jb.g + 2];
    }
    jb.ex = jb.e == a.E ? a.shared : a.experts + jb.e;
    jb.K = DOWN ? a.I : a.H;
    jb.N = DOWN ? a.H : a.I;
    const int n = jb.K / 64 / KS, s0 = ksp * n;
    const uint16_t* asrc = DOWN ? a.act_rows : a.xt + (size_t)jb.mat * a.R_max * a.H;
    const uint8_t* base = reinterpret_cast<const uint8_t*>(jb.ex->tr[jb.mat]);
    f32x16 acc = f32x16{};
    switch (jb.ex->fmt[jb.mat])
    {
        case BMX_TF_K2: mid_run_any<BMX_TF_K2>(jb, base, asrc, s0, n, acc); break;
        case BMX_TF_K25: mid_run_any<BMX_TF_K25>(jb, base, asrc, s0, n, acc); break;
        case BMX_TF_K3: mid_run_any<BMX_TF_K3>(jb, base, asrc, s0, n, acc); break;
        default: mid_run_any<BMX_TF_K4>(jb, base, asrc, s0, n, acc); break;
    }
    // accumulator element v of lane L: row 8 (v / 4) + 4 (L / 32) + v % 4, column L % 32 of the wave's 32-column block
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int cbo = 2 * jb.cb + (wave >> 2);
    if (cbo >= nb128) return;
    const int col = 32 * (wave & 3) + (lane & 31);
    // row stride of the partial layout (floats); the lane's first row 4 (lane / 32)
    const int rs = DOWN ? a.NBH * 128 : a.NB * 256;
    const size_t r0 = (size_t)ksp * a.R_max + jb.r0 + 4 * (lane >> 5);
    float* out = (DOWN ? a.part_dn + cbo * 128 : a.part_gu + cbo * 256 + jb.mat * 128) + r0 * rs + col;
#pragma unroll
    for (int v = 0; v < 16; ++v)
    {
        const int dr = 8 * (v >> 2) + (v & 3);
        if (dr + 4 * (lane >> 5) >= jb.nr) continue;
        out[(size_t)dr * rs] = acc[v];
    }
}

template <bool DOWN>
__global__ __launch_bounds__(MID_WAVES * 64) __attribute__((amdgpu_waves_per_eu(4))) void k_mid_gemm(GvArgs a)
{
    if (!a.split_min)
    {
        mid_unit<DOWN>(a, xcd_block(blockIdx.x, gridDim.x));
        return;
    }
    // split path: a grid of at most MID_SPLIT_WGS workgroups loops over the units of the call's unique experts, so a call
    // that keeps every expert on the GEMV pays for few idle workgroups (none past the first check when no expert can
    // reach split_min rows)
    if (a.split_min > a.T + 1 && 2 * a.offsets[a.NE] < a.split_ratio2 * *a.nuniq) return;
    const int nb128 = DOWN ? a.NBH : a.NB;
    const int per = (DOWN ? 1 : 2) * ((nb128 + 1) / 2) * (DOWN ? a.KS_dn : a.KS_gu);
    const int units = *a.nuniq * a.split_chunks * per;
    for (int lid = blockIdx.x; lid < units; lid += gridDim.x)
    {
        mid_unit<DOWN>(a, lid);
        __syncthreads();          // the unit's LDS stages are read out before the next unit writes them
    }
}

// ---- plan and launch -------------------------------------------------------------------------------------------------
struct PrefillPlan {
    int NB, NBH, G_max, R_max;
    size_t xt_bytes, part_gu_bytes, act_bytes, part_dn_bytes;
};

static PrefillPlan prefill_plan(const MoeShape& m)
{
    PrefillPlan p;
    p.NB = m.I / 128;
    p.NBH = m.H / 128;
    p.G_max = groups_max(m.T, m.topk, m.E, m.shared, PF_M);
    p.R_max = m.T * m.topk + (m.shared ? m.T : 0);
    p.xt_bytes = (size_t)2 * p.R_max * m.H * 2;
    p.part_gu_bytes = (size_t)p.R_max * p.NB * 256 * 4;
    p.act_bytes = (size_t)p.R_max * m.I * 2;
    p.part_dn_bytes = (size_t)p.R_max * p.NBH * 128 * 4;
    return p;
}

int prefill_rows_per_group() { return PF_M; }

// BMX_PF_PAIRS=0: every group its own 128-row tile (the products are the same bits either way)
static bool prefill_pairs_allowed()
{
    const char* v = getenv("BMX_PF_PAIRS");
    return !(v && *v == '0');
}

// BMX_PF_FAST_ACT=0: the prefill path's epilogue keeps the fixed-sequence activation of the decode path
static bool prefill_fast_act()
{
    const char* v = getenv("BMX_PF_FAST_ACT");
    return !(v && *v == '0');
}

// ---- mid-size path ------------------------------------------------------------------------------------------------------
struct MidPlan {
    int NB, NBH, G_max, R_max, KS_gu, KS_dn;
    size_t xt_bytes, part_gu_bytes, act_bytes, part_dn_bytes;
};

// k-split: the most splits that keep at least 16 k-steps each, gate / up (BMX_MID_MIN_STEPS) and down
// (BMX_MID_MIN_STEPS_DN) (the routing, unknown here, may put all rows on a few experts; splits keep the workgroup count
// up then, at the price of partial sums the epilogue adds). Measured (layer us; 8 / 16 / 32 steps for down): 16 tokens
// on ~10 experts of H 4096, I 2048: 103.7 / 104.4 / 106.6; GLM-shaped 8 tokens: 218 / 214 / 214; DeepSeek-shaped 16
// tokens: 298 / 292 / 295. Gate / up at 8 or 32 steps: 5-7 % slower than 16 on the first.
static int mid_split(int ksteps, bool down)
{
    const char* v = getenv(down ? "BMX_MID_MIN_STEPS_DN" : "BMX_MID_MIN_STEPS");
    const int min_steps = (v && *v) ? atoi(v) : 16;
    for (int d = ksteps; d > 1; --d)
        if (ksteps % d == 0 && ksteps / d >= min_steps) return d;
    return 1;
}

static MidPlan mid_plan(const MoeShape& m)
{
    MidPlan p;
    p.NB = m.I / 128;
    p.NBH = m.H / 128;
    p.G_max = groups_max(m.T, m.topk, m.E, m.shared, MID_M);
    p.R_max = m.T * m.topk + (m.shared ? m.T : 0);
    p.KS_gu = mid_split(m.H / 64, false);
    p.KS_dn = mid_split(m.I / 64, true);
    p.xt_bytes = (size_t)2 * p.R_max * m.H * 2;
    p.part_gu_bytes = (size_t)p.KS_gu * p.R_max * p.NB * 256 * 4;
    p.act_bytes = (size_t)p.R_max * m.I * 2;
    p.part_dn_bytes = (size_t)p.KS_dn * p.R_max * p.NBH * 128 * 4;
    return p;
}

int mid_rows_per_group() { return MID_M; }

size_t mid_ws_bytes(const MoeShape& m)
{
    const MidPlan p = mid_plan(m);
    return align_up(p.xt_bytes, 256) + align_up(p.part_gu_bytes, 256) + align_up(p.act_bytes, 256) +
           align_up(p.part_dn_bytes, 256);
}

int launch_mid_experts(const MoeShape& m, const void* x, const bmx_routes* r, float* y_rows, void* act_rows, void* ws,
                       size_t ws_bytes, float* combine_out, const void* combine_w, hipStream_t s, int stages)
{
    if (m.H % 128 || m.I % 128 || m.H <= 0 || m.I <= 0)
        return set_error(BMX_ERR_ARG, "moe experts: H (%d) and I (%d) must be multiples of 128", m.H, m.I);
    if (ws_bytes < mid_ws_bytes(m))
        return set_error(BMX_ERR_WORKSPACE, "moe experts: workspace %zu < %zu", ws_bytes, mid_ws_bytes(m));
    if (!r->row_expert) return set_error(BMX_ERR_ARG, "moe experts: routes without row_expert");
    const MidPlan p = mid_plan(m);
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
    a.KS_gu = p.KS_gu; a.KS_dn = p.KS_dn; a.NB = p.NB; a.NBH = p.NBH; a.R_max = p.R_max;
    a.NE = m.E + (m.shared ? 1 : 0);
    a.out = combine_out; a.w = static_cast<const uint16_t*>(combine_w); a.inv = r->inv; a.offsets = r->offsets;
    a.T = m.T; a.topk = m.topk; a.has_shared = m.shared;
    a.fresh = m.fresh;
    a.sh_gate = m.shared_gate;
    a.filter = 0;
    a.act_in_down = 0;
    a.gu_half = 0;
    int rc = BMX_OK;
    if (stages & (1 << BMX_STAGE_PREP))
        hipLaunchKernelGGL(k_pf_prep, prep_grid(p.R_max, m.H), dim3(256), 0, s, a);
    for (int f = 0; f < 3; ++f)
    {
        const int st = f == 0 ? BMX_STAGE_GATE_UP : f == 1 ? BMX_STAGE_GATE_UP_RESIDENT : BMX_STAGE_GATE_UP_STAGED;
        if (!(stages & (1 << st))) continue;
        GvArgs b = a;
        b.filter = f;
        hipLaunchKernelGGL(k_mid_gemm<false>, dim3((unsigned)(p.G_max * 2 * ((p.NB + 1) / 2) * p.KS_gu)),
                           dim3(MID_WAVES * 64), 0, s, b);
    }
    if (stages & (1 << BMX_STAGE_ACT)) rc = launch_epilogue(a, BMX_STAGE_ACT, s);
    for (int f = 0; f < 3 && !rc; ++f)
    {
        const int st = f == 0 ? BMX_STAGE_DOWN : f == 1 ? BMX_STAGE_DOWN_RESIDENT : BMX_STAGE_DOWN_STAGED;
        if (!(stages & (1 << st))) continue;
        GvArgs b = a;
        b.filter = f;
        hipLaunchKernelGGL(k_mid_gemm<true>, dim3((unsigned)(p.G_max * ((p.NBH + 1) / 2) * p.KS_dn)),
                           dim3(MID_WAVES * 64), 0, s, b);
    }
    if (!rc && (stages & (1 << BMX_STAGE_COMBINE))) rc = launch_epilogue(a, BMX_STAGE_COMBINE, s);
    if (!rc && (stages & (1 << BMX_STAGE_DOWN_OUT))) rc = launch_epilogue(a, BMX_STAGE_DOWN_OUT, s);
    if (rc) return rc;
    return check_launch("moe experts (mid-size path)");
}

// ---- split path: the heavy experts' share ---------------------------------------------------------------------------
void split_mid_splits(const MoeShape& m, int* ks_gu, int* ks_dn)
{
    const MidPlan p = mid_plan(m);
    *ks_gu = p.KS_gu;
    *ks_dn = p.KS_dn;
}

// The prep of the heavy experts' rows and their mid-size GEMMs. a: the split path's arguments with KS_gu / KS_dn set to
// the mid-size splits (KS_gu_mid / KS_dn_mid); nu_max: the most unique experts a call can have.
constexpr long MID_SPLIT_WGS = 1024;

void launch_split_mid(const GvArgs& a, int stage, int nu_max, hipStream_t s)
{
    const long units = (long)nu_max * a.split_chunks;
    if (stage == BMX_STAGE_PREP)
        hipLaunchKernelGGL(k_pf_prep, prep_grid(a.R_max, a.H), dim3(256), 0, s, a);
    else if (stage == BMX_STAGE_DOWN || stage == BMX_STAGE_DOWN_RESIDENT || stage == BMX_STAGE_DOWN_STAGED)
        hipLaunchKernelGGL(k_mid_gemm<true>, dim3((unsigned)std::min(MID_SPLIT_WGS, units * ((a.NBH + 1) / 2) * a.KS_dn)),
                           dim3(MID_WAVES * 64), 0, s, a);
    else
        hipLaunchKernelGGL(k_mid_gemm<false>,
                           dim3((unsigned)std::min(MID_SPLIT_WGS, units * 2 * ((a.NB + 1) / 2) * a.KS_gu)),
                           dim3(MID_WAVES * 64), 0, s, a);
}

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
    a.fresh = m.fresh;
    a.sh_gate = m.shared_gate;
    a.filter = 0;
    a.act_in_down = 0;
    a.gu_half = 1;
    a.pf_pairs = prefill_pairs_allowed() ? 1 : 0;
    a.fast_act = prefill_fast_act() ? 1 : 0;
    int rc = BMX_OK;
    if (stages & (1 << BMX_STAGE_PREP))
        hipLaunchKernelGGL(k_pf_prep_tok, prep_tok_grid(m.T, m.H), dim3(256), 0, s, a);
    for (int f = 0; f < 3; ++f)
    {
        const int st = f == 0 ? BMX_STAGE_GATE_UP : f == 1 ? BMX_STAGE_GATE_UP_RESIDENT : BMX_STAGE_GATE_UP_STAGED;
        if (!(stages & (1 << st))) continue;
        GvArgs b = a;
        b.filter = f;
        hipLaunchKernelGGL(k_pf_gemm<false>, dim3((unsigned)(p.G_max * 2 * ((p.NB + 1) / 2))), dim3(PF_WAVES * 64), 0, s, b);
    }
    if (stages & (1 << BMX_STAGE_ACT)) rc = launch_epilogue(a, BMX_STAGE_ACT, s);
    for (int f = 0; f < 3 && !rc; ++f)
    {
        const int st = f == 0 ? BMX_STAGE_DOWN : f == 1 ? BMX_STAGE_DOWN_RESIDENT : BMX_STAGE_DOWN_STAGED;
        if (!(stages & (1 << st))) continue;
        GvArgs b = a;
        b.filter = f;
        hipLaunchKernelGGL(k_pf_gemm<true>, dim3((unsigned)(p.G_max * ((p.NBH + 1) / 2))), dim3(PF_WAVES * 64), 0, s, b);
    }
    if (!rc && (stages & (1 << BMX_STAGE_COMBINE))) rc = launch_epilogue(a, BMX_STAGE_COMBINE, s);
    if (!rc && (stages & (1 << BMX_STAGE_DOWN_OUT))) rc = launch_epilogue(a, BMX_STAGE_DOWN_OUT, s);
    if (rc) return rc;
    return check_launch("moe experts (prefill path)");
}

}  // namespace bmx
