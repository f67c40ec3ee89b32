// Pieces shared by the decode (GEMV) and prefill (MFMA) expert-product kernels: the kernel argument block, the
// in-register trellis window, and the epilogue kernels both paths hand their fp32 products to.
#pragma once
#include "bmx_common.hpp"
#include "bmx_internal.hpp"

namespace bmx {

// Arguments of the expert-product kernels. Rows are dispatch rows (expert-major); `part_gu` / `part_dn` hold fp32 products
// as [k-split][row][128-column block][matrix][128] (gate / up) and [k-split][row][128-column block][128] (down).
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
    const int32_t* row_expert;
    float* part_gu;
    float* part_dn;
    int KS_gu, KS_dn, NB, NBH, R_max, NE;
    float* out;
    const uint16_t* w;
    const int32_t* inv;
    const int32_t* offsets;
    int T, topk, has_shared;
    uint16_t* xt;              // prefill: rotated gate / up input rows [2][R_max][H]
    const int32_t* fresh;      // [E] admitted-this-step flags of the expert-slot table, or null
    int filter;                // gate / up or down groups: 0 all, 1 experts not fresh, 2 fresh experts only
    int act_in_down;           // the down GEMV computes its input rows from the gate / up partials (one-row groups)
    int gu_half;               // part_gu holds one split as fp16 [row][128-column block][matrix][128], each value the
                               // epilogue's own rounding of that split's sum (RN of 0.0f + product): same bits downstream
    const uint16_t* sh_gate;   // fp16 [H] or null: the shared expert's output is scaled by sigmoid(x[t] . sh_gate)
    int pf_pairs = 0;          // prefill: two consecutive 128-row groups of one expert run as one 256-row tile
    int fast_act = 0;          // prefill: the gate / up epilogue's activation by act_gate_fast (hardware exp2 / rcp)
    // split path (split_min > 0): an expert is heavy when the call averages at least split_ratio2 / 2 rows per expert
    // (every expert then is), or when it has at least split_min rows itself. Heavy experts run on the mid-size MFMA
    // kernel, in units of up to 32 rows (split_chunks per expert, taken over the unique experts uexp[0 .. *nuniq)), the
    // others on the GEMV; a row's partials have KS_gu_mid / KS_dn_mid splits when its expert is heavy, KS_gu / KS_dn
    // otherwise. 0: off
    int split_min = 0;
    int split_ratio2 = 0;
    int split_chunks = 0;
    int KS_gu_mid = 0, KS_dn_mid = 0;
    const int32_t* counts = nullptr;
    const int32_t* uexp = nullptr;
    const int32_t* nuniq = nullptr;
};

// split path: expert e (a local id, E for the shared expert) runs on the mid-size MFMA kernel (the call's rows over
// its unique experts, both from the dispatch, decide it for every expert at once; a very heavy expert goes there anyway)
__device__ __forceinline__ bool split_heavy(const GvArgs& a, int e)
{
    if (a.split_min <= 0) return false;
    if (2 * a.offsets[a.NE] >= a.split_ratio2 * *a.nuniq) return true;
    return a.split_min <= a.T && a.counts[e] >= a.split_min;
}
// k-splits of the gate / up (DN = false) or down (DN = true) partials of dispatch row r (r < the rows of the call)
template <bool DN>
__device__ __forceinline__ int row_splits(const GvArgs& a, int r)
{
    if (split_heavy(a, a.row_expert[r])) return DN ? a.KS_dn_mid : a.KS_gu_mid;
    return DN ? a.KS_dn : a.KS_gu;
}

// The shared expert's gate of token t, sigmoid(x[t] . sh_gate), by the calling 16-lane group (every lane of the group
// gets it): lane j sums x[h] sh_gate[h] over h = 128 b + 8 j + i, b ascending then i = 0 .. 7, one fp32 fma each (fp16
// inputs are exact in fp32); the 16 lane sums are added by a butterfly over lane ^ 8, ^ 4, ^ 2, ^ 1 (each pair's sum is
// the same on both lanes); then the fixed-sequence sigmoid. The oracle evaluates the same sequence.
__device__ __forceinline__ float shared_gate16(const uint16_t* x, const uint16_t* g, int H)
{
    const int j = threadIdx.x & 15;
    float acc = 0.0f;
    for (int b = 0; b < H / 128; ++b)
    {
        float xv[8], gv[8];
        unpack8(ldg4(x + 128 * b + 8 * j), xv);
        unpack8(ldg4(g + 128 * b + 8 * j), gv);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = __builtin_fmaf(xv[i], gv[i], acc);
    }
    acc = acc + dpp_f<0x128>(acc);     // lane ^ 8 (row_ror:8)
    acc = acc + dpp_xor4(acc);
    acc = acc + dpp_f<0x4E>(acc);      // lane ^ 2
    acc = acc + dpp_f<0xB1>(acc);      // lane ^ 1
    return sigmoid_fixed(acc);
}

// split path: the call averages enough rows per unique expert to run every expert on the mid-size kernel
__device__ __forceinline__ bool split_callwide(const GvArgs& a)
{
    return 2 * a.offsets[a.NE] >= a.split_ratio2 * *a.nuniq;
}

// Rotated gate / up input of one dispatch row for the MFMA paths, xt = RN16(H128(x * suh) * R), by a 16-lane group: unit
// u = (row, matrix, run of PREP_BPU 128-blocks), 8 consecutive inputs per lane. Split path: heavy experts' rows only.
constexpr int PREP_BPU = 4;
__device__ __forceinline__ void prep_unit(const GvArgs& a, long u)
{
    const int nblk = a.H / 128, nrun = (nblk + PREP_BPU - 1) / PREP_BPU;
    const int j = threadIdx.x & 15, run = (int)(u % nrun), mat = (int)((u / nrun) & 1), r = (int)(u / nrun / 2);
    if (r >= a.offsets[a.NE]) return;
    const int e = a.row_expert[r];
    if (a.split_min && !split_heavy(a, e)) return;      // split path: the GEMV rotates the other rows itself
    const bmx_expert& ex = e == a.E ? *a.shared : a.experts[e];
    const uint16_t* xr = a.x + (size_t)a.row_token[r] * a.H + 8 * j;
    const uint16_t* su = reinterpret_cast<const uint16_t*>(ex.suh[mat]) + 8 * j;
    uint16_t* dst = a.xt + ((size_t)mat * a.R_max + r) * a.H + 8 * j;
#pragma unroll
    for (int i = 0; i < PREP_BPU; ++i)
    {
        const int b = run * PREP_BPU + i;
        if (b >= nblk) break;
        float v[8], s[8];
        unpack8(ldg4(xr + 128 * b), v);
        unpack8(ldg4(su + 128 * b), s);
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = v[q] * s[q];
        had128_x8(v);
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = v[q] * (R_SCALE * had128_x8_sign());
        __builtin_nontemporal_store(pack8_r(v), reinterpret_cast<u32x4*>(dst + 128 * b));   // streamed (C3: 265 -> 252 us)
    }
}

// group filter of the split gate / up and down stages (the shared expert, index E, is never fresh)
__device__ __forceinline__ bool group_skipped(const GvArgs& a, int e)
{
    if (!a.filter) return false;
    const bool fr = e < a.E && a.fresh && a.fresh[e];
    return fr != (a.filter == 2);
}

// S(i) + 16 for the 64 stream positions of a 64-weight strip (a strip starts on a 64-position boundary, where the ring
// position is a whole number of 32-bit words for every format)
template <int F> struct RingTab {
    int q[64];
    constexpr RingTab() : q()
    {
        for (int i = 0; i < 64; ++i) q[i] = ring_end<F>(i) + 16;
    }
};

// 16-bit state at bit q of a lane's window (MSB-first words: prev, own[0], own[1], ...); bits above 15 of the result
// are left as they are
template <int NW>
__device__ __forceinline__ uint32_t win_state(uint32_t prev, const uint32_t (&own)[NW], int q)
{
    const int d = q >> 5, o = q & 31;
    const uint32_t hi = d == 0 ? prev : own[d - 1];
    if (o <= 16) return hi >> (16 - o);
    return __builtin_amdgcn_alignbit(hi, own[d], 48 - o);
}

// Window bits [q - 16, q + 16) as one 32-bit value: the state at bit q in its low half, the one at q - 16 in its high
// half (q >= 16)
template <int NW>
__device__ __forceinline__ uint32_t win_pair(uint32_t prev, const uint32_t (&own)[NW], int q)
{
    const int p = q - 16, d = p >> 5, o = p & 31;
    const uint32_t w0 = d == 0 ? prev : own[d - 1];
    if (o == 0) return w0;
    return __builtin_amdgcn_alignbit(w0, own[d], 32 - o);
}

// states that start 16 bits apart in the ring: stream positions i and i + 16 / K for every i of a 64-position strip
template <int F> __host__ __device__ constexpr bool ring_pairs16(int step)
{
    for (int i = 0; i + step < 64; ++i)
        if (ring_end<F>(i + step) - ring_end<F>(i) != 16) return false;
    return true;
}

// Codebook weights of stream positions j8 .. j8 + 7 of a lane's strip (j8 a multiple of 8, a constant after unrolling),
// packed as cb_oct's. K 2 and K 4: the state 16 ring bits before another (8 positions back at K 2, 4 at K 4) is the high
// half of the same 32-bit window, so one funnel shift gives two states and the hash reads the high half by op_sel
// (K 2: half a shift per state; the two octs of a 16-position block share their shifts, which the compiler computes
// once). K 2.5 and K 3 have no such partner: a shift per state.
template <int F, int NW>
__device__ __forceinline__ void oct_weights(uint32_t prev, const uint32_t (&own)[NW], int j8, uint32_t (&w)[4])
{
    constexpr RingTab<F> tab;
    if constexpr (F == BMX_TF_K2)
    {
        static_assert(ring_pairs16<F>(8), "K 2: positions 8 apart start 16 bits apart");
        const int j16 = j8 & ~15;
        uint32_t v[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = win_pair(prev, own, tab.q[j16 + 8 + q]);
        if (j8 & 8) cb_oct(v, w);
        else cb_oct_hi(v, w);
    }
    else if constexpr (F == BMX_TF_K4)
    {
        static_assert(ring_pairs16<F>(4), "K 4: positions 4 apart start 16 bits apart");
        uint32_t v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = win_pair(prev, own, tab.q[j8 + 4 + q]);
        cb_oct_k4(v, w);
    }
    else
    {
        uint32_t st[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) st[q] = win_state(prev, own, tab.q[j8 + q]);
        cb_oct(st, w);
    }
}

// NT: non-temporal loads. The prefill GEMM reads with the default policy instead, since a row group decoded again by
// another workgroup then finds its words in the caches (C3's layer 2 % faster); the decode GEMV (5 % slower without)
// and the mid-size GEMM (1 %) keep the non-temporal loads.
template <bool NT = true, int NW>
__device__ __forceinline__ void load_words(uint32_t (&w)[NW], const uint8_t* p)
{
#pragma unroll
    for (int i = 0; i < NW; ++i) w[i] = NT ? ldg_nt(p, i) : ldg(p, i);
}

// The strip of lane s (= lane & 3) of a tile: stream positions 64 s .. 64 s + 63, i.e. output columns
// 2 s, 2 s + 1, 2 s + 8, 2 s + 9 of the tile, all 16 input rows. Pair jj (positions jj, jj + 1) is rows 2 dw, 2 dw + 1 of
// column index cidx (make_tc_perm, engine/kernels/nv2/ft_core.h:49-62):
__device__ __forceinline__ constexpr int strip_cidx(int jj) { return ((jj >> 3) >> 2) + ((jj & 7) >= 4 ? 2 : 0); }
__device__ __forceinline__ constexpr int strip_dw(int jj) { return ((jj >> 3) & 3) + ((jj & 2) ? 4 : 0); }
// the column (0..127) inside a 128-column block of strip column index c for lane `lane` (tile (lane >> 2) & 7)
__device__ __forceinline__ int lane_col(int lane, int c)
{
    const int t = (lane >> 2) & 7, s = lane & 3;
    return t * 16 + 2 * s + (c & 1) + ((c & 2) ? 8 : 0);
}

// epilogue kernels of moe_decode.hip, launched with the partial layout above (any k-split count)
int launch_epilogue(const GvArgs& a, int stage, hipStream_t s);

// split path, moe_prefill.hip: the k-splits of the mid-size kernel for a call, and the launch of the heavy experts' prep
// (BMX_STAGE_PREP), gate / up GEMMs (any gate / up stage, with a.filter) or down GEMMs (BMX_STAGE_DOWN); a carries
// the mid-size splits in KS_gu / KS_dn
void split_mid_splits(const MoeShape& m, int* ks_gu, int* ks_dn);
void launch_split_mid(const GvArgs& a, int stage, int nu_max, hipStream_t s);

}  // namespace bmx
