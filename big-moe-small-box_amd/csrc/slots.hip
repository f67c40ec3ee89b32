// Expert-slot table: the CLOCK step of one layer (one workgroup) and the home -> slot copies of its admissions.
//
// Semantics follow the reference's ec_step_k (engine/ec.py:16-76) with one contract fixed: misses are admitted in
// ascending expert order (the reference collects them with atomics, in no fixed order).
#include <cstdlib>

#include "bmx_common.hpp"
#include "bmx_internal.hpp"
#include "router_wave.hpp"

namespace bmx {

constexpr int SL_THREADS = 512;     // one thread per expert (E <= 512)
constexpr int SL_MAXS = 8192;       // slots the step keeps in LDS (pin and reference bits)

struct SlotArgs {
    bmx_slot_table t;
    const int64_t* sel;
    int64_t first;
    int li, n, admit;
    int pf;       // 0: a step; 1: a prefetch into job buffer `buf` with at most `limit` candidates
    int limit, buf;
    AgentShared* sh;  // or null: the admissions are also published to the copy agent's ring under sequence number seq
    int64_t seq;
    int64_t* need;    // steps that publish: need[li] = the last record the layer's products depend on
    int64_t wait_limit;   // wall-clock ticks a publish waits for its ring slot (and a planned step for its reply)
    int plan;             // 1: a planned step (sh set): request, reply, lanes (PlanArgs)
    PlanArgs pl;
};

__device__ __forceinline__ bool agent_failed(AgentShared* sh)
{
    return __hip_atomic_load(&sh->flags[2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) ||
           __hip_atomic_load(&sh->flags[3], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Until the agent has read record seq - AG_RING out of the ring slot seq will reuse (bounded; false: the agent aborted,
// a wait ran out of time, or this one did, which it records in flags[3]). One lane.
__device__ bool ring_slot_free(AgentShared* sh, int64_t seq, int64_t limit)
{
    const int64_t want = seq - AG_RING;
    const int64_t t0 = wall_clock64();
    for (;;)
    {
        if (agent_failed(sh)) return false;
        const int64_t c = __hip_atomic_load(&sh->consumed, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
        if (c >= want) return true;
        if (wall_clock64() - t0 > limit)
        {
            __hip_atomic_store(&sh->flags[3], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            return false;
        }
        __builtin_amdgcn_s_sleep(2);
    }
}

__device__ __forceinline__ int tile_bytes_dev(int fmt)
{
    return fmt == BMX_TF_K2 ? 64 : fmt == BMX_TF_K25 ? 80 : fmt == BMX_TF_K3 ? 96 : 128;
}

// job buffer of a step (pf = 0: the step's jobs, count in ctl[2]) or of prefetch buffer b (count, then the pairs)
__device__ __forceinline__ int32_t* prefetch_jobs(const bmx_slot_table& t, int b) { return t.pjobs + b * (1 + 2 * t.maxj); }

// Ballot compaction of the flagged experts of the workgroup (thread = candidate index) into `out`, in thread order;
// returns the total. The order within a wave is the lane order, across waves the wave order.
__device__ __forceinline__ int compact_flags(bool flag, int value, int32_t* out, int* wave_cnt)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t b = __ballot(flag);
    if (lane == 0) wave_cnt[wave] = __popcll(b);
    __syncthreads();
    int base = 0, total = 0;
    for (int w = 0; w < SL_THREADS / 64; ++w)
    {
        if (w < wave) base += wave_cnt[w];
        total += wave_cnt[w];
    }
    if (flag) out[base + __popcll(b & ((1ull << lane) - 1ull))] = value;
    __syncthreads();
    return total;
}

// A planned step's request and reply, by the whole workgroup: the picked experts (mark) in ascending order into uq
// with their residency and pick counts (ecnt), the picks and input rows when the call is small enough, published under
// a.seq; then the bounded wait for the planner's reply and each expert's lane into elane (a resident expert is always a
// hit; a lane value the step does not know runs the expert from its home). A call with every expert resident publishes
// nothing and writes its own reply (no CPU pick). Returns 0 when the agent had failed or the
// ring slot or the reply did not come in time (then every lane is VRAM or HOME and the step admits nothing).
__device__ int plan_step(const SlotArgs& a, const uint32_t* mark, const int32_t* ecnt, int32_t* elane, int32_t* uq,
                         int* wave_cnt, int* s_ok)
{
    const int tid = threadIdx.x, E = a.t.E;
    const int32_t* slotof = a.t.slotof + (size_t)a.li * E;
    const bool marked = tid < E && ((mark[tid >> 5] >> (tid & 31)) & 1u);
    const int nu = compact_flags(marked, tid, uq, wave_cnt);
    __shared__ int s_miss;
    if (tid == 0)
    {
        *s_ok = ring_slot_free(a.sh, a.seq, a.wait_limit) ? 1 : 0;
        s_miss = 0;
    }
    __syncthreads();
    for (int u = tid; u < nu; u += SL_THREADS)
        if (slotof[uq[u]] < 0) atomicAdd(&s_miss, 1);
    __syncthreads();
    // a call whose experts are all resident has nothing to plan (the planner never moves a resident expert): no request,
    // no wait; the step writes that call's reply itself (no CPU pick), which is what the CPU partial's add reads
    const bool resident = s_miss == 0;
    PlanReq* rq = &a.sh->req[ring_index(a.seq)];
    const PlanArgs& pl = a.pl;
    const bool picks = a.n <= BMX_PLAN_MAXP;
    const bool has_x = picks && pl.x && pl.xring && pl.T <= BMX_PLAN_MAXT;
    if (*s_ok && !resident)
    {
        for (int u = tid; u < nu; u += SL_THREADS)
        {
            const int e = uq[u];
            rq->ex[u] = e;
            rq->res[u] = slotof[e] >= 0 ? 1 : 0;
            rq->cnt[u] = ecnt[e];
        }
        if (picks)
            for (int i = tid; i < a.n; i += SL_THREADS)
            {
                const int64_t e = a.sel[i] - a.first;
                rq->pe[i] = (e >= 0 && e < E) ? (int32_t)e : -1;
                rq->pw[i] = pl.w[i];
            }
        if (has_x)
        {
            const size_t n16 = (size_t)pl.T * pl.H / 8;
            const u32x4* src = reinterpret_cast<const u32x4*>(pl.x);
            u32x4* dst = reinterpret_cast<u32x4*>(pl.xring + (size_t)ring_index(a.seq) * BMX_PLAN_MAXT * pl.H);
            for (size_t i = tid; i < n16; i += SL_THREADS) dst[i] = src[i];
        }
        if (tid == 0)
        {
            rq->li = a.li;
            rq->nu = nu;
            rq->np = a.n;
            rq->ntok = pl.T;
            rq->topk = pl.topk;
            rq->has_x = has_x ? 1 : 0;
        }
        __threadfence_system();          // this thread's writes to host memory, before the barrier and the publish
    }
    __syncthreads();
    if (tid == 0 && *s_ok && resident)
    {
        PlanRep* wr = &a.sh->rep[ring_index(a.seq)];
        __hip_atomic_store(&wr->ncpu, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(&wr->seq, a.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    else if (tid == 0 && *s_ok)
    {
        __hip_atomic_store(&rq->seq, a.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        const PlanRep* rp = &a.sh->rep[ring_index(a.seq)];
        const int64_t t0 = wall_clock64();
        for (;;)
        {
            if (__hip_atomic_load(&rp->seq, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) == a.seq) break;
            if (agent_failed(a.sh))
            {
                *s_ok = 0;
                break;
            }
            if (wall_clock64() - t0 > a.wait_limit)
            {
                __hip_atomic_store(&a.sh->flags[3], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                *s_ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __syncthreads();
    const int ok = *s_ok;
    const PlanRep* rp = &a.sh->rep[ring_index(a.seq)];
    for (int u = tid; u < nu; u += SL_THREADS)
    {
        const int e = uq[u];
        int ln = ok ? __hip_atomic_load(&rp->lane[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) : BMX_LANE_HOME;
        if (slotof[e] >= 0) ln = BMX_LANE_VRAM;
        else if (ln != BMX_LANE_ADMIT && ln != BMX_LANE_CPU) ln = BMX_LANE_HOME;
        elane[e] = ln;
    }
    __syncthreads();
    for (int i = tid; i < a.n; i += SL_THREADS)
    {
        const int64_t e = a.sel[i] - a.first;
        const int ln = (e >= 0 && e < E) ? elane[e] : -1;
        const bool cpu = ln == BMX_LANE_CPU;
        pl.sel_gpu[i] = cpu ? -1 : a.sel[i];
        pl.w_gpu[i] = cpu ? (uint16_t)0 : pl.w[i];
        if (pl.lanes) pl.lanes[i] = ln;
    }
    return ok;
}

// The step of one workgroup of SL_THREADS threads (k_slot_step, and k_route_slot_step after its routing wave).
__device__ __forceinline__ void slot_step_body(const SlotArgs& a)
{
    __shared__ int32_t pin[SL_MAXS];
    __shared__ int32_t refb[SL_MAXS];
    __shared__ uint32_t mark[16];
    __shared__ int32_t miss[512];
    __shared__ int32_t first_at[512];
    __shared__ int wave_cnt[SL_THREADS / 64];
    __shared__ int n_hit, n_pfused, n_missall, s_ok, ring_ok;
    __shared__ int32_t ecnt[512];        // planned step: picks per expert
    __shared__ int32_t elane[512];       // planned step: lane per expert
    __shared__ int32_t uq[512];          // planned step: the picked experts, ascending
    const bmx_slot_table& t = a.t;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int S = t.S, E = t.E;
    const int epoch = t.ctl[1] + (a.pf ? 0 : 1);
    for (int s = tid; s < S; s += SL_THREADS)
    {
        pin[s] = t.pin[s];
        refb[s] = t.refb[s];
    }
    if (tid < 16) mark[tid] = 0;
    if (tid < E)
    {
        first_at[tid] = INT32_MAX;
        ecnt[tid] = 0;
        elane[tid] = BMX_LANE_VRAM;
    }
    if (tid == 0) n_hit = n_pfused = n_missall = 0;
    // the ring slot check of a publishing step (a round trip to the agent's count in host memory, and a bounded wait if
    // the agent is a ring behind) by the last wave, beside the other waves' work; read after the barriers below
    if (a.sh && !a.plan && tid == SL_THREADS - 64) ring_ok = ring_slot_free(a.sh, a.seq, a.wait_limit) ? 1 : 0;
    __syncthreads();
    int32_t* slotof = t.slotof + (size_t)a.li * E;
    int nmiss;
    if (!a.pf)
    {
        for (int i = tid; i < a.n; i += SL_THREADS)
        {
            const int64_t e = a.sel[i] - a.first;
            if (e >= 0 && e < E)
            {
                atomicOr(&mark[e >> 5], 1u << (e & 31));
                if (a.plan) atomicAdd(&ecnt[e], 1);
            }
        }
        __syncthreads();
        // a planned step: the planner's lanes (a miss is admitted only in BMX_LANE_ADMIT)
        if (a.plan) plan_step(a, mark, ecnt, elane, uq, wave_cnt, &s_ok);
        // hits: reference bit, pinned for this step (the first use of a prefetched slot counts and marks the expert
        // fresh: its copy may still be in flight); misses: compacted in ascending expert order
        const int e = tid;
        bool is_miss = false;
        if (e < E)
        {
            int fr = 0;
            if ((mark[e >> 5] >> (e & 31)) & 1u)
            {
                const int s = slotof[e];
                if (s >= 0)
                {
                    refb[s] = 1;
                    pin[s] = epoch;
                    atomicAdd(&n_hit, 1);
                    if (t.pfl[s])
                    {
                        t.pfl[s] = 0;
                        fr = 1;
                        atomicAdd(&n_pfused, 1);
                    }
                }
                else
                {
                    is_miss = !a.plan || elane[e] == BMX_LANE_ADMIT;
                    atomicAdd(&n_missall, 1);
                }
            }
            t.fresh[e] = fr;
        }
        nmiss = compact_flags(is_miss, e, miss, wave_cnt);
    }
    else
    {
        // prefetch candidates: the first occurrence of each in-range expert, if not resident, in the order given
        int64_t e = -1;
        if (tid < a.n)
        {
            e = a.sel[tid] - a.first;
            if (e >= 0 && e < E) atomicMin(&first_at[e], tid);
            else e = -1;
        }
        __syncthreads();
        const bool cand = e >= 0 && first_at[e] == tid && slotof[e] < 0;
        nmiss = min(compact_flags(cand, (int)e, miss, wave_cnt), a.limit);
    }

    // admissions: one wave sweeps the CLOCK hand 64 slots at a time. Within a chunk every slot is probed once, so taking
    // the first candidate and clearing the reference bits of the unpinned slots before it is the sequential sweep. A
    // prefetch sweeps gently: referenced slots keep their bits, and its admissions start without one.
    if (wave == 0)
    {
        int32_t* jobs = a.pf ? prefetch_jobs(t, a.buf) + 1 : t.jobs;
        SlotPub* pub = nullptr;
        int admit = a.admit;
        if (a.sh)
        {
            // a failed agent (aborted, or a wait ran out of time) copies nothing more: admit nothing, so every expert
            // this step sees runs from its home, and publish nothing
            int ok = 0;
            if (a.plan) ok = s_ok;           // the planned step has waited for its ring slot and its reply
            else ok = ring_ok;
            if (__shfl(ok, 0)) pub = &a.sh->ring[ring_index(a.seq)];
            else admit = 0;
        }
        int hand = t.ctl[0], nj = 0, novictim = 0, evicted = 0, wasted = 0;
        const int chunk = S < 64 ? S : 64;
        const int maxp = a.pf ? S : 2 * S;      // a prefetch passes referenced slots without clearing: one revolution
        for (int k = 0; admit && S > 0 && k < nmiss && nj < t.maxj; ++k)
        {
            const int ex = miss[k];
            int found = -1, probes = 0;
            while (probes < maxp)
            {
                const int nv = min(chunk, maxp - probes);
                int idx = hand + lane;
                if (idx >= S) idx -= S;
                const bool valid = lane < nv;
                const int p = valid ? pin[idx] : 0, rb = valid ? refb[idx] : 0;
                const bool skip = p == epoch || p < 0;
                const bool cand = valid && !skip && !rb;
                const uint64_t cb = __ballot(cand);
                const int upto = cb ? (__ffsll((long long)cb) - 1) : nv;
                if (!a.pf && valid && lane < upto && !skip && rb) refb[idx] = 0;
                if (cb)
                {
                    found = hand + upto;
                    if (found >= S) found -= S;
                    hand = found + 1 == S ? 0 : found + 1;
                    break;
                }
                hand += nv;
                if (hand >= S) hand -= S;
                probes += nv;
            }
            if (found < 0)
            {
                novictim = a.pf ? 0 : 1;
                break;
            }
            if (lane == 0)
            {
                const int s = found, old = t.owner[s];
                if (old >= 0)
                {
                    const int ol = old / E, oe = old % E;
                    t.slotof[old] = -1;
                    bmx_expert* tab = reinterpret_cast<bmx_expert*>(t.tables[ol]);
                    const uint64_t* h = t.home + ((size_t)ol * E + oe) * 3;
                    tab[oe].tr[0] = h[0];
                    tab[oe].tr[1] = h[1];
                    tab[oe].tr[2] = h[2];
                    ++evicted;
                    wasted += t.pfl[s];
                }
                t.owner[s] = a.li * E + ex;
                slotof[ex] = s;
                refb[s] = a.pf ? 0 : 1;     // a prefetched expert keeps no hit bit until a step uses it
                pin[s] = epoch;
                t.pfl[s] = a.pf;
                bmx_expert* tab = reinterpret_cast<bmx_expert*>(t.tables[a.li]);
                const uint64_t b = t.slot_base[s];
                tab[ex].tr[0] = b;
                tab[ex].tr[1] = b + (uint64_t)t.off_u;
                tab[ex].tr[2] = b + (uint64_t)t.off_d;
                jobs[2 * nj] = ex;
                jobs[2 * nj + 1] = s;
                if (!a.pf) t.fresh[ex] = 1;
                if (pub)
                {
                    pub->pairs[2 * nj] = ex;
                    pub->pairs[2 * nj + 1] = s;
                }
            }
            ++nj;
        }
        if (lane == 0)
        {
            if (pub)
            {
                pub->li = a.li;
                pub->n = nj;
                pub->kind = a.pf;
                __hip_atomic_store(&pub->seq, a.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
                if (!a.pf && a.need) a.need[a.li] = nj > 0 ? a.seq : a.seq - 1;
            }
            if (admit && S > 0) t.ctl[0] = hand;
            if (a.pf)
            {
                prefetch_jobs(t, a.buf)[0] = nj;
                t.stats[5] += nj;
            }
            else
            {
                t.ctl[1] = epoch;
                t.ctl[2] = nj;
                t.stats[0] += n_hit;
                t.stats[1] += n_missall;
                t.stats[2] += nj;
                t.stats[3] += novictim;
                t.stats[6] += n_pfused;
            }
            t.stats[4] += evicted;
            t.stats[7] += wasted;
        }
    }
    __syncthreads();
    for (int s = tid; s < S; s += SL_THREADS)
    {
        t.pin[s] = pin[s];
        t.refb[s] = refb[s];
    }
}

__global__ __launch_bounds__(SL_THREADS) void k_slot_step(SlotArgs a)
{
    slot_step_body(a);
}

// A one-token layer call's routing and its step in one launch: wave 0 routes the token (writes sel / w, the picks the
// step reads after its first barrier) while the other waves load the slot state into LDS; then the step. The same
// picks, weights and table state as k_router followed by k_slot_step.
template <int J>
__global__ __launch_bounds__(SL_THREADS) void k_route_slot_step(RouterArgs ra, SlotArgs a)
{
    __shared__ TopkLds tl;
    if ((threadIdx.x >> 6) == 0) route_token_wave<J>(ra, 0, tl);
    slot_step_body(a);
}

// copies of the last step's admissions (buf < 0) or of prefetch buffer buf: blockIdx.y = job; the matrices in `mats`
// (bit 0 gate, 1 up, 2 down); 16-byte chunks, grid-stride
__global__ __launch_bounds__(256) void k_slot_copy(bmx_slot_table t, int li, int mats, int buf)
{
    const int j = blockIdx.y;
    const int32_t* jobs = buf < 0 ? t.jobs : prefetch_jobs(t, buf) + 1;
    if (j >= (buf < 0 ? t.ctl[2] : jobs[-1])) return;
    const int e = jobs[2 * j], s = jobs[2 * j + 1];
    const bmx_expert& ex = reinterpret_cast<const bmx_expert*>(t.tables[li])[e];
    const size_t tiles = (size_t)t.H * t.I / 256;
    const uint64_t b = t.slot_base[s];
    const size_t stride = (size_t)gridDim.x * blockDim.x;
#pragma unroll 1
    for (int m = 0; m < 3; ++m)
    {
        if (!((mats >> m) & 1)) continue;
        const size_t n16 = tiles * tile_bytes_dev(ex.fmt[m]) / 16;
        const u32x4* src = reinterpret_cast<const u32x4*>(t.home[((size_t)li * t.E + e) * 3 + m]);
        u32x4* dst = reinterpret_cast<u32x4*>(b + (m == 0 ? 0 : m == 1 ? (uint64_t)t.off_u : (uint64_t)t.off_d));
        size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
        for (; i + 3 * stride < n16; i += 4 * stride)
        {
            const u32x4 v0 = __builtin_nontemporal_load(src + i), v1 = __builtin_nontemporal_load(src + i + stride);
            const u32x4 v2 = __builtin_nontemporal_load(src + i + 2 * stride);
            const u32x4 v3 = __builtin_nontemporal_load(src + i + 3 * stride);
            dst[i] = v0;
            dst[i + stride] = v1;
            dst[i + 2 * stride] = v2;
            dst[i + 3 * stride] = v3;
        }
        for (; i < n16; i += stride) dst[i] = __builtin_nontemporal_load(src + i);
    }
}

// Staged prefill: layer li's table entries of experts ex[j] (local ids, j < n) point at staging record j (base + j rec,
// the slot geometry) when restore = 0; with restore = 1 each points back at where the expert lives now: its slot if
// it is resident, else its home.
__global__ __launch_bounds__(256) void k_stage_rows(bmx_slot_table t, int li, const int32_t* __restrict__ ex, int n,
                                                    uint64_t base, int restore)
{
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    const int e = ex[j];
    if (e < 0 || e >= t.E) return;
    bmx_expert* tab = reinterpret_cast<bmx_expert*>(t.tables[li]);
    uint64_t a0, a1, a2;
    if (!restore)
    {
        a0 = base + (uint64_t)j * (uint64_t)t.rec;
        a1 = a0 + (uint64_t)t.off_u;
        a2 = a0 + (uint64_t)t.off_d;
    }
    else
    {
        const int s = t.slotof[(size_t)li * t.E + e];
        if (s >= 0)
        {
            a0 = t.slot_base[s];
            a1 = a0 + (uint64_t)t.off_u;
            a2 = a0 + (uint64_t)t.off_d;
        }
        else
        {
            const uint64_t* h = t.home + ((size_t)li * t.E + e) * 3;
            a0 = h[0];
            a1 = h[1];
            a2 = h[2];
        }
    }
    tab[e].tr[0] = a0;
    tab[e].tr[1] = a1;
    tab[e].tr[2] = a2;
}

static int check_table(const bmx_slot_table* t, const char* who)
{
    if (!t) return set_error(BMX_ERR_ARG, "%s: null table", who);
    if (t->L <= 0 || t->E <= 0 || t->E > 512 || t->S < 0 || t->S > SL_MAXS || t->maxj < 0 || t->maxj > 64)
        return set_error(BMX_ERR_ARG, "%s: unsupported L=%d E=%d S=%d maxj=%d (E <= 512, S <= %d, maxj <= 64)", who, t->L,
                         t->E, t->S, t->maxj, SL_MAXS);
    if (t->H <= 0 || t->I <= 0 || t->H % 16 || t->I % 16 || t->rec <= 0 || t->rec % 16 || t->off_u % 16 || t->off_d % 16)
        return set_error(BMX_ERR_ARG, "%s: bad geometry", who);
    if (!t->slotof || !t->owner || !t->refb || !t->pin || !t->ctl || !t->jobs || !t->fresh || !t->stats || !t->home ||
        !t->slot_base || !t->tables || !t->pjobs || !t->pfl)
        return set_error(BMX_ERR_ARG, "%s: null table array", who);
    return BMX_OK;
}

int launch_slot_step(const bmx_slot_table* t, int li, const int64_t* sel, int n, int64_t first, int admit, hipStream_t s,
                     AgentShared* sh, int64_t seq, int64_t* need, int64_t wait_limit, const PlanArgs* plan)
{
    int rc = check_table(t, "bmx_slot_step");
    if (rc) return rc;
    if (li < 0 || li >= t->L || n < 0 || (n && !sel)) return set_error(BMX_ERR_ARG, "bmx_slot_step: bad layer or picks");
    SlotArgs a;
    a.t = *t;
    a.sel = sel;
    a.first = first;
    a.li = li;
    a.n = n;
    a.admit = admit ? 1 : 0;
    a.pf = 0;
    a.limit = 0;
    a.buf = 0;
    a.sh = sh;
    a.seq = seq;
    a.need = need;
    a.wait_limit = wait_limit;
    a.plan = 0;
    a.pl = PlanArgs{};
    if (plan)
    {
        if (!sh) return set_error(BMX_ERR_ARG, "planned step without an agent");
        if (!plan->w || !plan->sel_gpu || !plan->w_gpu || plan->T < 0 || plan->topk <= 0)
            return set_error(BMX_ERR_ARG, "bmx_slot_step_planned: null weights or outputs, or bad T / topk");
        a.plan = 1;
        a.pl = *plan;
    }
    hipLaunchKernelGGL(k_slot_step, dim3(1), dim3(SL_THREADS), 0, s, a);
    return check_launch(plan ? "bmx_slot_step_planned" : "bmx_slot_step");
}

int launch_route_slot_step(const bmx_slot_table* t, int li, const void* logits, const float* bias, int E, int topk,
                           int n_group, int topk_group, int score_fn, int renorm, float scale, int64_t first, int64_t* sel,
                           void* w, int admit, hipStream_t s, AgentShared* sh, int64_t seq, int64_t* need,
                           int64_t wait_limit)
{
    int rc = check_table(t, "bmx_route_slot_step");
    if (rc) return rc;
    if (li < 0 || li >= t->L) return set_error(BMX_ERR_ARG, "bmx_route_slot_step: bad layer %d", li);
    if (E != t->E || E > SL_THREADS)
        return set_error(BMX_ERR_ARG, "bmx_route_slot_step: the router's %d experts are not the table's %d", E, t->E);
    rc = check_router(1, E, topk, n_group, topk_group, score_fn, logits, sel, w);
    if (rc) return rc;
    RouterArgs ra;
    ra.logits = static_cast<const uint16_t*>(logits); ra.bias = bias; ra.T = 1; ra.E = E; ra.topk = topk;
    ra.G = n_group; ra.TG = topk_group; ra.score_fn = score_fn; ra.renorm = renorm; ra.scale = scale; ra.first = first;
    ra.sel = sel; ra.w = static_cast<uint16_t*>(w);
    SlotArgs a;
    a.t = *t;
    a.sel = ra.sel;
    a.first = ra.first;
    a.li = li;
    a.n = ra.topk;
    a.admit = admit ? 1 : 0;
    a.pf = 0;
    a.limit = 0;
    a.buf = 0;
    a.sh = sh;
    a.seq = seq;
    a.need = need;
    a.wait_limit = wait_limit;
    a.plan = 0;
    a.pl = PlanArgs{};
    const dim3 g(1), b(SL_THREADS);
    switch ((ra.E + 63) / 64)
    {
        case 1: hipLaunchKernelGGL(k_route_slot_step<1>, g, b, 0, s, ra, a); break;
        case 2: hipLaunchKernelGGL(k_route_slot_step<2>, g, b, 0, s, ra, a); break;
        case 3: hipLaunchKernelGGL(k_route_slot_step<3>, g, b, 0, s, ra, a); break;
        case 4: hipLaunchKernelGGL(k_route_slot_step<4>, g, b, 0, s, ra, a); break;
        case 5: hipLaunchKernelGGL(k_route_slot_step<5>, g, b, 0, s, ra, a); break;
        case 6: hipLaunchKernelGGL(k_route_slot_step<6>, g, b, 0, s, ra, a); break;
        default: hipLaunchKernelGGL(k_route_slot_step<8>, g, b, 0, s, ra, a); break;
    }
    return check_launch("bmx_route_slot_step");
}

int launch_slot_prefetch(const bmx_slot_table* t, int li, const int64_t* sel, int n, int64_t first, int limit, int buf,
                         hipStream_t s, AgentShared* sh, int64_t seq, int64_t wait_limit)
{
    int rc = check_table(t, "bmx_slot_prefetch");
    if (rc) return rc;
    if (li < 0 || li >= t->L || n < 0 || n > SL_THREADS || (n && !sel))
        return set_error(BMX_ERR_ARG, "bmx_slot_prefetch: bad layer or guesses (n <= %d)", SL_THREADS);
    if (buf < 0 || buf > 1 || limit < 0) return set_error(BMX_ERR_ARG, "bmx_slot_prefetch: bad buffer %d or limit %d", buf, limit);
    SlotArgs a;
    a.t = *t;
    a.sel = sel;
    a.first = first;
    a.li = li;
    a.n = n;
    a.admit = 1;
    a.pf = 1;
    a.limit = limit;
    a.buf = buf;
    a.sh = sh;
    a.seq = seq;
    a.need = nullptr;
    a.wait_limit = wait_limit;
    a.plan = 0;
    a.pl = PlanArgs{};
    hipLaunchKernelGGL(k_slot_step, dim3(1), dim3(SL_THREADS), 0, s, a);
    return check_launch("bmx_slot_prefetch");
}

// workgroups per copy job (BMX_SLOT_COPY_WGS, 1..256): reads of pinned host memory wait microseconds on the link, so a
// few workgroups with several loads in flight per thread keep it busy; more only queue behind it and hold back the
// kernels of other streams
static int copy_wgs()
{
    const char* v = getenv("BMX_SLOT_COPY_WGS");
    const int n = v ? atoi(v) : 64;
    return n < 1 ? 1 : n > 256 ? 256 : n;
}

int launch_slot_copy(const bmx_slot_table* t, int li, int mats, int buf, hipStream_t s)
{
    const char* who = buf < 0 ? "bmx_slot_copy" : "bmx_slot_prefetch_copy";
    int rc = check_table(t, who);
    if (rc) return rc;
    if (li < 0 || li >= t->L) return set_error(BMX_ERR_ARG, "%s: bad layer", who);
    if (mats < 0 || mats > 7) return set_error(BMX_ERR_ARG, "%s: bad matrix mask %d", who, mats);
    if (buf > 1) return set_error(BMX_ERR_ARG, "%s: bad buffer %d", who, buf);
    if (t->maxj == 0 || mats == 0) return BMX_OK;
    hipLaunchKernelGGL(k_slot_copy, dim3((unsigned)copy_wgs(), (unsigned)t->maxj), dim3(256), 0, s, *t, li, mats, buf);
    return check_launch(who);
}

}  // namespace bmx

using namespace bmx;

extern "C" {

int bmx_slot_step(const bmx_slot_table* t, int li, const int64_t* sel, int n, int64_t first, int admit,
                  bmx_stream_t stream)
{
    return launch_slot_step(t, li, sel, n, first, admit, static_cast<hipStream_t>(stream));
}

int bmx_slot_copy(const bmx_slot_table* t, int li, bmx_stream_t stream)
{
    return launch_slot_copy(t, li, 7, -1, static_cast<hipStream_t>(stream));
}

int bmx_slot_copy_mats(const bmx_slot_table* t, int li, int mats, bmx_stream_t stream)
{
    return launch_slot_copy(t, li, mats, -1, static_cast<hipStream_t>(stream));
}

int bmx_slot_prefetch(const bmx_slot_table* t, int li, const int64_t* sel, int n, int64_t first, int limit, int buf,
                      bmx_stream_t stream)
{
    return launch_slot_prefetch(t, li, sel, n, first, limit, buf, static_cast<hipStream_t>(stream));
}

int bmx_slot_prefetch_copy(const bmx_slot_table* t, int li, int buf, int mats, bmx_stream_t stream)
{
    if (buf < 0) return set_error(BMX_ERR_ARG, "bmx_slot_prefetch_copy: bad buffer %d", buf);
    return launch_slot_copy(t, li, mats, buf, static_cast<hipStream_t>(stream));
}

int bmx_slot_stage_async(const void* const* src, void* const* dst, const size_t* bytes, int n, bmx_stream_t stream)
{
    if (n < 0 || (n && (!src || !dst || !bytes))) return set_error(BMX_ERR_ARG, "bmx_slot_stage_async: bad arguments");
    for (int i = 0; i < n; ++i)
    {
        const hipError_t e = hipMemcpyAsync(dst[i], src[i], bytes[i], hipMemcpyDefault, static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return set_error(BMX_ERR_HIP, "bmx_slot_stage_async: copy %d: %s", i, hipGetErrorString(e));
    }
    return BMX_OK;
}

int bmx_slot_stage_rows(const bmx_slot_table* t, int li, const int32_t* experts, int n, uint64_t base, int restore,
                        bmx_stream_t stream)
{
    int rc = check_table(t, "bmx_slot_stage_rows");
    if (rc) return rc;
    if (li < 0 || li >= t->L || n < 0 || n > t->E || (n && !experts))
        return set_error(BMX_ERR_ARG, "bmx_slot_stage_rows: bad layer %d or expert count %d (<= E = %d)", li, n, t->E);
    if (!restore && n && (!base || base % 256))
        return set_error(BMX_ERR_ARG, "bmx_slot_stage_rows: staging base must be a 256-byte aligned address");
    if (!n) return BMX_OK;
    hipLaunchKernelGGL(k_stage_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       *t, li, experts, n, base, restore ? 1 : 0);
    return check_launch("bmx_slot_stage_rows");
}

int bmx_host_device_ptr(void* host, uint64_t* device_addr)
{
    if (!host || !device_addr) return set_error(BMX_ERR_ARG, "bmx_host_device_ptr: null pointer");
    void* d = nullptr;
    const hipError_t e = hipHostGetDevicePointer(&d, host, 0);
    if (e != hipSuccess) return set_error(BMX_ERR_HIP, "bmx_host_device_ptr: %s", hipGetErrorString(e));
    *device_addr = reinterpret_cast<uint64_t>(d);
    return BMX_OK;
}

}  // extern "C"
