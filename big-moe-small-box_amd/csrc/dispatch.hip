// Dispatch: stable counting sort of the picks (t, k) by expert into contiguous row segments.
//   rank within a wave: ballot-based match loop (one pass per distinct expert in the wave)
//   rank within a block: per-wave LDS histograms, exclusive prefix over waves per expert
//   rank overall: block histograms, exclusive prefix over blocks per expert, offsets = exclusive scan of counts
// Small calls (decode) run the whole sort in one workgroup; larger calls use three kernels.
#include "bmx_common.hpp"
#include "bmx_internal.hpp"

namespace bmx {

constexpr int DP_THREADS = 1024;
constexpr int DP_WAVES = DP_THREADS / 64;
constexpr int DP_MAXNE = 513;             // E <= 512 plus the shared segment
constexpr int DP_SINGLE_MAX = 4 * DP_THREADS;

// in-wave stable rank of this lane's expert among the active lanes below it; the lowest lane of each distinct expert
// writes the count of that expert to hist[e]
__device__ __forceinline__ int wave_rank(int e, bool valid, int* hist)
{
    const int lane = threadIdx.x & 63;
    uint64_t active = __ballot(valid);
    int rank = 0;
    while (active)
    {
        const int leader = __builtin_ctzll(active);
        const int el = __builtin_amdgcn_readlane(e, leader);
        const uint64_t m = __ballot(valid && e == el);
        if (valid && e == el)
        {
            rank = __builtin_popcountll(m & ((1ull << lane) - 1ull));
            if (lane == leader) hist[el] = __builtin_popcountll(m);
        }
        active &= ~m;
    }
    return rank;
}

// block-level exclusive prefix of the wave histograms (per expert), in place; adds base[e] and returns the block total
// in base[e] when accumulate
__device__ __forceinline__ void prefix_waves(int* whist, int NE, int* base, bool accumulate)
{
    for (int e = threadIdx.x; e < NE; e += blockDim.x)
    {
        int run = accumulate ? base[e] : 0;
        for (int w = 0; w < DP_WAVES; ++w)
        {
            const int v = whist[w * DP_MAXNE + e];
            whist[w * DP_MAXNE + e] = run;
            run += v;
        }
        base[e] = run;
    }
}

// exclusive scan of cnt[0 .. NE) into off[0 .. NE] by one wave; returns the total
__device__ int scan_wave(const int* cnt, int* off, int NE)
{
    const int lane = threadIdx.x & 63;
    int carry = 0;
    for (int c0 = 0; c0 < NE; c0 += 64)
    {
        const int e = c0 + lane;
        const int v = e < NE ? cnt[e] : 0;
        int incl = v;
#pragma unroll
        for (int m = 1; m < 64; m <<= 1)
        {
            const int o = __shfl_up(incl, m);
            if (lane >= m) incl += o;
        }
        if (e < NE) off[e] = carry + incl - v;
        carry += __shfl(incl, 63);
    }
    if (lane == 0) off[NE] = carry;
    return carry;
}

// groups of at most rpg rows per expert (ascending expert, ascending row) and the ascending list of used experts
__device__ void emit_groups(const int* cnt, const int* off, int NE, int rpg, int32_t* uexp, int32_t* nuniq,
                            int32_t* groups, int32_t* ngroups, int* sh_tmp)
{
    // one wave: per expert the number of groups, scanned; then each expert writes its groups
    const int lane = threadIdx.x & 63;
    int gcarry = 0, ucarry = 0;
    for (int c0 = 0; c0 < NE; c0 += 64)
    {
        const int e = c0 + lane;
        const int c = e < NE ? cnt[e] : 0;
        const int ng = (c + rpg - 1) / rpg;
        const int used = c > 0 ? 1 : 0;
        int gi = ng, ui = used;
#pragma unroll
        for (int m = 1; m < 64; m <<= 1)
        {
            const int og = __shfl_up(gi, m), ou = __shfl_up(ui, m);
            if (lane >= m) { gi += og; ui += ou; }
        }
        if (used) uexp[ucarry + ui - 1] = e;
        const int g0 = gcarry + gi - ng;
        for (int q = 0; q < ng; ++q)
        {
            groups[3 * (g0 + q) + 0] = e;
            groups[3 * (g0 + q) + 1] = off[e] + q * rpg;
            groups[3 * (g0 + q) + 2] = min(rpg, c - q * rpg);
        }
        gcarry += __shfl(gi, 63);
        ucarry += __shfl(ui, 63);
    }
    if (lane == 0) { *ngroups = gcarry; *nuniq = ucarry; }
    (void)sh_tmp;
}

struct DpArgs {
    const int64_t* sel;
    int T, topk, E, shared, rpg;
    int64_t first;
    bmx_routes r;
    int32_t* rank;
    int32_t* blk_hist;
    int32_t* zero_ptr;
    int zero_count;
};

// ---- one workgroup -----------------------------------------------------------------------------------------------
__global__ __launch_bounds__(DP_THREADS) void k_dispatch_single(DpArgs a)
{
    __shared__ int whist[DP_WAVES * DP_MAXNE];
    __shared__ int base[DP_MAXNE];
    __shared__ int off[DP_MAXNE + 1];
    const int n = a.T * a.topk, E = a.E, NE = E + (a.shared ? 1 : 0);
    const int tid = threadIdx.x, wave = tid >> 6;
    for (int i = tid; i < a.zero_count; i += DP_THREADS) a.zero_ptr[i] = 0;
    for (int e = tid; e < NE; e += DP_THREADS) base[e] = 0;
    int myrank[DP_SINGLE_MAX / DP_THREADS];
    int mye[DP_SINGLE_MAX / DP_THREADS];
    const int nchunk = (n + DP_THREADS - 1) / DP_THREADS;
    for (int c = 0; c < DP_SINGLE_MAX / DP_THREADS; ++c)
    {
        if (c >= nchunk) break;
        for (int i = tid; i < DP_WAVES * DP_MAXNE; i += DP_THREADS) whist[i] = 0;
        lds_barrier();
        const int p = c * DP_THREADS + tid;
        int e = -1;
        if (p < n)
        {
            const int64_t g = a.sel[p] - a.first;
            e = (g >= 0 && g < E) ? (int)g : -1;
        }
        const int rk = wave_rank(e, e >= 0, whist + wave * DP_MAXNE);
        lds_barrier();
        prefix_waves(whist, E, base, true);
        lds_barrier();
        myrank[c] = e >= 0 ? whist[wave * DP_MAXNE + e] + rk : -1;
        mye[c] = e;
        lds_barrier();
    }
    if (a.shared && tid == 0) base[E] = a.T;
    lds_barrier();
    if (wave == 0) scan_wave(base, off, NE);
    lds_barrier();
    for (int e = tid; e < NE; e += DP_THREADS) { a.r.counts[e] = base[e]; a.r.offsets[e] = off[e]; }
    if (tid == 0) a.r.offsets[NE] = off[NE];
    for (int c = 0; c < nchunk; ++c)
    {
        const int p = c * DP_THREADS + tid;
        if (p >= n) break;
        const int e = mye[c];
        if (e >= 0)
        {
            const int row = off[e] + myrank[c];
            a.r.inv[p] = row;
            a.r.row_token[row] = p / a.topk;
            a.r.row_slot[row] = p % a.topk;
            a.r.row_expert[row] = e;
        }
        else a.r.inv[p] = -1;
    }
    if (a.shared)
        for (int t = tid; t < a.T; t += DP_THREADS)
        {
            a.r.row_token[off[E] + t] = t;
            a.r.row_slot[off[E] + t] = -1;
            a.r.row_expert[off[E] + t] = E;
        }
    if (wave == 0) emit_groups(base, off, NE, a.rpg, a.r.uexp, a.r.nuniq, a.r.groups, a.r.ngroups, nullptr);
}

// ---- three kernels ---------------------------------------------------------------------------------------------------
// (1) per block of 1024 picks: in-block ranks and the block histogram
__global__ __launch_bounds__(DP_THREADS) void k_dispatch_blocks(DpArgs a)
{
    __shared__ int whist[DP_WAVES * DP_MAXNE];
    __shared__ int base[DP_MAXNE];
    const int n = a.T * a.topk, E = a.E;
    const int tid = threadIdx.x, wave = tid >> 6;
    for (int i = tid; i < DP_WAVES * DP_MAXNE; i += DP_THREADS) whist[i] = 0;
    for (int e = tid; e < E; e += DP_THREADS) base[e] = 0;
    if (blockIdx.x == 0)
        for (int i = tid; i < a.zero_count; i += DP_THREADS) a.zero_ptr[i] = 0;
    lds_barrier();
    const int p = blockIdx.x * DP_THREADS + tid;
    int e = -1;
    if (p < n)
    {
        const int64_t g = a.sel[p] - a.first;
        e = (g >= 0 && g < E) ? (int)g : -1;
    }
    const int rk = wave_rank(e, e >= 0, whist + wave * DP_MAXNE);
    lds_barrier();
    prefix_waves(whist, E, base, false);
    lds_barrier();
    if (p < n) a.rank[p] = e >= 0 ? whist[wave * DP_MAXNE + e] + rk : -1;
    for (int x = tid; x < E; x += DP_THREADS) a.blk_hist[(size_t)blockIdx.x * E + x] = base[x];
}

// (2) one workgroup: prefix over blocks per expert, counts, offsets, groups
__global__ __launch_bounds__(DP_THREADS) void k_dispatch_scan(DpArgs a, int nblk)
{
    __shared__ int cnt[DP_MAXNE];
    __shared__ int off[DP_MAXNE + 1];
    const int E = a.E, NE = E + (a.shared ? 1 : 0);
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += DP_THREADS)
    {
        int run = 0;
        for (int b = 0; b < nblk; ++b)
        {
            int* h = a.blk_hist + (size_t)b * E + e;
            const int v = *h;
            *h = run;
            run += v;
        }
        cnt[e] = run;
    }
    if (a.shared && tid == 0) cnt[E] = a.T;
    lds_barrier();
    if (tid < 64) scan_wave(cnt, off, NE);
    lds_barrier();
    for (int e = tid; e < NE; e += DP_THREADS) { a.r.counts[e] = cnt[e]; a.r.offsets[e] = off[e]; }
    if (tid == 0) a.r.offsets[NE] = off[NE];
    if (a.shared)
        for (int t = tid; t < a.T; t += DP_THREADS)
        {
            a.r.row_token[off[E] + t] = t;
            a.r.row_slot[off[E] + t] = -1;
            a.r.row_expert[off[E] + t] = E;
        }
    if (tid < 64) emit_groups(cnt, off, NE, a.rpg, a.r.uexp, a.r.nuniq, a.r.groups, a.r.ngroups, nullptr);
}

// (3) scatter
__global__ __launch_bounds__(256) void k_dispatch_scatter(DpArgs a)
{
    const int n = a.T * a.topk;
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= n) return;
    const int64_t g = a.sel[p] - a.first;
    if (g < 0 || g >= a.E) { a.r.inv[p] = -1; return; }
    const int e = (int)g, b = p / DP_THREADS;
    const int row = a.r.offsets[e] + a.blk_hist[(size_t)b * a.E + e] + a.rank[p];
    a.r.inv[p] = row;
    a.r.row_token[row] = p / a.topk;
    a.r.row_slot[row] = p % a.topk;
    a.r.row_expert[row] = e;
}

// Most work groups a dispatch can produce: an expert with c rows gives ceil(c / rpg) <= 1 + (c - 1) / rpg groups, so u
// experts with rows in total give at most u + (rows - u) / rpg, largest for the most experts a batch can touch.
int groups_max(int T, int topk, int E, int shared, int rpg)
{
    const long n = (long)T * topk;
    const long ne = E + (shared ? 1 : 0);
    const long rows = n + (shared ? T : 0);
    long u = n + (shared ? 1 : 0);
    if (u > ne) u = ne;
    if (u > rows) u = rows;
    return (int)(u + (rows - u) / rpg);
}

size_t dispatch_ws_bytes(int T, int topk, int E)
{
    const size_t n = (size_t)T * topk;
    if (n <= (size_t)DP_SINGLE_MAX) return 256;
    const size_t nblk = (n + DP_THREADS - 1) / DP_THREADS;
    return align_up(n * 4, 256) + align_up(nblk * (size_t)E * 4, 256);
}

int launch_dispatch(const int64_t* sel, int T, int topk, int E, int64_t first, int shared, int rpg,
                    const bmx_routes* out, void* ws, size_t ws_bytes, int32_t* zero_ptr, int zero_count, hipStream_t s)
{
    if (T < 0 || topk <= 0 || E <= 0 || E + 1 > DP_MAXNE || rpg <= 0)
        return set_error(BMX_ERR_ARG, "bmx_dispatch: unsupported sizes T=%d topk=%d E=%d rows_per_group=%d", T, topk, E, rpg);
    if (!out || !out->counts || !out->offsets || !out->row_token || !out->row_slot || !out->inv || !out->uexp ||
        !out->nuniq || !out->groups || !out->ngroups || !out->row_expert || (T > 0 && !sel))
        return set_error(BMX_ERR_ARG, "bmx_dispatch: null pointer");
    if (ws_bytes < dispatch_ws_bytes(T, topk, E))
        return set_error(BMX_ERR_WORKSPACE, "bmx_dispatch: workspace %zu < %zu", ws_bytes, dispatch_ws_bytes(T, topk, E));
    DpArgs a;
    a.sel = sel; a.T = T; a.topk = topk; a.E = E; a.shared = shared ? 1 : 0; a.rpg = rpg; a.first = first; a.r = *out;
    a.zero_ptr = zero_ptr; a.zero_count = zero_ptr ? zero_count : 0;
    const size_t n = (size_t)T * topk;
    if (n <= (size_t)DP_SINGLE_MAX)
    {
        a.rank = nullptr; a.blk_hist = nullptr;
        hipLaunchKernelGGL(k_dispatch_single, dim3(1), dim3(DP_THREADS), 0, s, a);
        return check_launch("bmx_dispatch");
    }
    const int nblk = (int)((n + DP_THREADS - 1) / DP_THREADS);
    a.rank = static_cast<int32_t*>(ws);
    a.blk_hist = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + align_up(n * 4, 256));
    hipLaunchKernelGGL(k_dispatch_blocks, dim3(nblk), dim3(DP_THREADS), 0, s, a);
    hipLaunchKernelGGL(k_dispatch_scan, dim3(1), dim3(DP_THREADS), 0, s, a, nblk);
    hipLaunchKernelGGL(k_dispatch_scatter, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a);
    return check_launch("bmx_dispatch");
}

}  // namespace bmx
