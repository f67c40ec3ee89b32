// Copy agent: the expert-slot table's home -> slot copies issued by a host thread on the DMA engines.
//
// The reference stages a layer's missing experts from the host (stage_layer, engine/kernels/nv2/nv2_host.cpp:1558-1593)
// after its controller learns the layer's picks from a ring in mapped host memory (engine/kernels/nv2/nv2_dev.cu:23-95).
// Here the slot-table step kernel publishes its admissions to a ring in fine-grained host memory (payload, then the
// sequence number with a system-scope release); one host thread per agent polls the ring in order and hands each
// admission to the SDMA engines (hsa_amd_memory_async_copy): the gate / up part of every admission of a record under one
// completion signal, then the down matrices under a second that waits for the first, each record after the previous
// one (a slot can be evicted and refilled by the next record). When a part's signal reaches zero the thread stores the
// record's sequence number into that part's flag (fine-grained host memory). A one-wave kernel on the compute stream
// waits for a flag to reach a sequence number, bounded by a time limit.
//
// Why not the copy kernel: a kernel reading pinned host memory at the link's ~57 GB/s holds back HBM-bound kernels on the
// other streams two- to three-fold while it runs; the DMA engines move the same bytes at the same rate with a few per
// cent of interference. Why not hipMemcpyAsync on a stream: HIP keeps a stream's order with packets in the stream's
// hardware queue, which a process shares between streams (four queues by default); a copy ordered behind a queue whose
// head is the wait kernel would wait for it. The SDMA engines' own queues and signals are outside that.
#include <hip/hip_runtime.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <mutex>
#include <thread>
#include <vector>

#include "bmx_internal.hpp"

namespace bmx {

constexpr int AG_PENDING = 256;  // parts in flight
constexpr int AG_SIGNALS = 2 * AG_PENDING;   // a signal is reused only after every part issued after it has retired

// A CPU-lane job: the picks of one planned step that its plan put on the CPU, with the call's input rows
struct CpuJob {
    int64_t seq;
    int li, ntok, topk;
    std::vector<int> pick_e, pick_t;    // in pick order
    std::vector<float> pick_w;
    std::vector<uint16_t> x;            // [ntok][H]
};

}  // namespace bmx

struct bmx_copy_agent {
    bmx_slot_table t;
    std::vector<uint64_t> slot_base;     // [S] slot addresses
    std::vector<uint64_t> home;          // [L * E] address of each expert's record (pinned host or device)
    std::vector<uint8_t> home_host;      // [L * E] 1 = the record is in host memory
    std::vector<int64_t> bytes;          // [L * E * 3] trellis bytes of gate, up, down
    hsa_agent_t gpu{}, cpu{};
    int device = 0;
    bool hsa_up = false;
    bmx::AgentShared* sh = nullptr;      // fine-grained host memory (host address)
    bmx::AgentShared* sh_dev = nullptr;  // the same memory's device address
    int64_t* need = nullptr;             // device [L]: the record each layer's products wait for
    int64_t next_seq = 0;                // last sequence number handed out (caller's thread)
    int64_t wait_ticks = 0;              // wait limit in wall-clock ticks
    int64_t ticks_per_us = 0;
    std::thread th;
    std::atomic<bool> stop{false};
    std::atomic<bool> hold{false};       // the thread reads no new record while set (bmx_copy_agent_control)
    std::atomic<int> error{0};
    std::atomic<int64_t> records{0}, copies{0};
    std::atomic<int64_t> copied_bytes{0};
    // residency plan
    mutable std::mutex plan_mu;
    bmx_plan_policy policy{};            // cpu_on 0: every miss admitted
    std::atomic<int64_t> plans{0}, plan_cpu{0};
    // CPU lane
    bool cpu_ready = false;
    bmx_moe_desc cpu_desc{};
    std::vector<bmx_cpu_expert> cpu_experts;   // [L * E]
    int cpu_threads = 1;
    uint16_t* xring = nullptr;           // [AG_RING][BMX_PLAN_MAXT][H] fp16, pinned host
    uint16_t* xring_dev = nullptr;
    float* cpu_part = nullptr;           // [AG_RING][BMX_PLAN_MAXT][H] fp32, pinned host
    float* cpu_part_dev = nullptr;
    std::vector<int64_t> job_of;         // [AG_RING]: the planned step whose request carried rows (its plan may
                                         // put picks on the CPU lane)
    std::thread cpu_th;
    std::mutex cpu_mu;
    std::condition_variable cpu_cv;
    std::deque<bmx::CpuJob> cpu_q;
    std::atomic<int64_t> cpu_jobs{0};
    std::atomic<int64_t> cpu_ns{0};          // host time the CPU worker spent computing jobs
    double cpu_pick_us[2] = {0.0, 0.0};      // running mean of the worker's time per pick, exact / fast mode
                                             // (under plan_mu; the fast one seeded at set-up)
};

namespace bmx {

// waits until flag `part` reaches seq (or, with need, need[0]: what the layer's last step left there); bounded
__global__ __launch_bounds__(64) void k_copy_wait(AgentShared* sh, int part, int64_t seq, const int64_t* need,
                                                  int64_t limit)
{
    if (threadIdx.x != 0) return;
    if (need) seq = need[0];
    if (seq <= 0) return;      // sequence numbers start at 1 and never wrap (64-bit): nothing published yet
    const int64_t t0 = wall_clock64();
    for (;;)
    {
        const int64_t v = __hip_atomic_load(&sh->flags[part], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
        if (v >= seq) return;
        if (__hip_atomic_load(&sh->flags[2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) ||
            __hip_atomic_load(&sh->flags[3], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM))
            return;
        if (wall_clock64() - t0 > limit)
        {
            __hip_atomic_store(&sh->flags[3], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            return;
        }
        __builtin_amdgcn_s_sleep(2);
    }
}

// out[T][H] += the CPU lane's partial of step seq (ring slot seq % AG_RING), once the job is done (bounded wait by
// thread 0 of each workgroup; nothing is added when the job had no picks or the wait ran out; rows past the job's own
// tokens are left alone). Four values a thread.
__global__ __launch_bounds__(256) void k_cpu_add(AgentShared* sh, const float* part, int64_t seq, float* out, int T,
                                                 int H, int64_t limit)
{
    __shared__ int go, rows;
    if (threadIdx.x == 0)
    {
        go = 0;
        rows = 0;
        const int64_t t0 = wall_clock64();
        // the step's own reply (read by the step before this launch; its ring slot is reused 64 steps later): a plan
        // with no CPU pick has nothing to add, so the worker's completion of the empty job is not waited for
        const PlanRep& rp = sh->rep[(uint64_t)seq % AG_RING];
        const bool none = __hip_atomic_load(&rp.seq, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) == seq &&
                          __hip_atomic_load(&rp.ncpu, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == 0;
        for (; !none;)
        {
            if (__hip_atomic_load(&sh->cpu_done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) >= seq)
            {
                const int slot = (int)((uint64_t)seq % AG_RING);
                go = __hip_atomic_load(&sh->cpu_n[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) > 0;
                rows = __hip_atomic_load(&sh->cpu_t[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                break;
            }
            if (__hip_atomic_load(&sh->flags[2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) ||
                __hip_atomic_load(&sh->flags[3], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM))
                break;
            if (wall_clock64() - t0 > limit)
            {
                __hip_atomic_store(&sh->flags[3], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __syncthreads();
    if (!go) return;
    const float* p = part + (size_t)((uint64_t)seq % AG_RING) * BMX_PLAN_MAXT * H;
    const int i = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (i >= min(T, rows) * H) return;
    const float4 v = *reinterpret_cast<const float4*>(p + i);
    float4 o = *reinterpret_cast<const float4*>(out + i);
    o.x = o.x + v.x;
    o.y = o.y + v.y;
    o.z = o.z + v.z;
    o.w = o.w + v.w;
    *reinterpret_cast<float4*>(out + i) = o;
}

static void agent_fail(bmx_copy_agent* a, int code)
{
    int z = 0;
    a->error.compare_exchange_strong(z, code);
    __atomic_store_n(&a->sh->flags[2], 1, __ATOMIC_RELEASE);
}

static float h2f_host(uint16_t h)
{
    const uint32_t sg = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t f;
    if (e == 0 && m == 0) f = sg;
    else if (e == 0)
    {
        int k = 0;                      // subnormal: m 2^-24, normalised
        uint32_t mm = m;
        while (!(mm & 0x400u)) { mm <<= 1; ++k; }
        f = sg | ((uint32_t)(113 - k) << 23) | ((mm & 0x3ffu) << 13);
    }
    else if (e == 31) f = sg | 0x7f800000u | (m << 13);
    else f = sg | ((e + 112) << 23) | (m << 13);
    float r;
    memcpy(&r, &f, 4);
    return r;
}

// The planner (bmx_plan_policy): lanes of request r into p; the CPU picks of the call into job (when it carries rows).
static void plan_reply(bmx_copy_agent* a, const PlanReq& r, PlanRep& p, CpuJob* job)
{
    bmx_plan_policy pol;
    {
        std::lock_guard<std::mutex> lk(a->plan_mu);
        pol = a->policy;
        const double mean = a->cpu_pick_us[pol.cpu_fast ? 1 : 0];
        if (pol.cpu_measured && mean > 0.0) pol.cpu_expert_us = mean;
    }
    const int nu = r.nu;
    const bool cpu_ok = pol.cpu_on && a->cpu_ready && r.has_x && r.np <= BMX_PLAN_MAXP && r.ntok <= BMX_PLAN_MAXT;
    int nres = 0;
    std::vector<int> miss;
    for (int u = 0; u < nu; ++u)
    {
        if (r.res[u]) { p.lane[u] = BMX_LANE_VRAM; ++nres; }
        else miss.push_back(u);
    }
    std::stable_sort(miss.begin(), miss.end(), [&](int x, int y) {
        return r.cnt[x] != r.cnt[y] ? r.cnt[x] > r.cnt[y] : r.ex[x] < r.ex[y];
    });
    // start times: the GPU's at its base plus the hits (0 with nothing resident), the CPU lane's at its base whenever it
    // may take a miss, so the base sits on both sides of the comparison (engine/kernels/nv2/nv2_host.cpp:1017-1018)
    double g = nres ? pol.gpu_base_us + pol.gpu_hit_us * nres : 0.0;
    double c = (cpu_ok && !miss.empty()) ? pol.cpu_base_us : 0.0;
    int ncpu = 0;
    for (int u : miss)
    {
        const bool home = pol.home_single && r.ntok > 1 && r.cnt[u] == 1;
        const double gc = home ? pol.gpu_home_us : pol.gpu_admit_us;
        const double cc = pol.cpu_expert_us + pol.cpu_token_us * (r.cnt[u] - 1);
        if (cpu_ok && ncpu < pol.max_cpu && std::max(c + cc, g) <= std::max(c, g + gc))
        {
            p.lane[u] = BMX_LANE_CPU;
            c += cc;
            ++ncpu;
        }
        else
        {
            p.lane[u] = home ? BMX_LANE_HOME : BMX_LANE_ADMIT;
            g += gc;
        }
    }
    p.ncpu = ncpu;
    a->plans.fetch_add(1, std::memory_order_relaxed);
    a->plan_cpu.fetch_add(ncpu, std::memory_order_relaxed);
    if (!job) return;
    job->li = r.li;
    job->ntok = r.ntok;
    job->topk = r.topk;
    if (!ncpu) return;
    for (int i = 0; i < r.np; ++i)
    {
        const int e = r.pe[i];
        if (e < 0) continue;
        const int32_t* f = std::lower_bound(r.ex, r.ex + nu, e);
        if (f == r.ex + nu || *f != e || p.lane[f - r.ex] != BMX_LANE_CPU) continue;
        job->pick_e.push_back(e);
        job->pick_t.push_back(i / std::max(1, r.topk));
        job->pick_w.push_back(h2f_host(r.pw[i]));
    }
}

// The CPU-lane worker: jobs (steps with CPU picks) in sequence order; each CPU pick's y row (bit for bit the decode path's, or the fast mode's
// when the policy asks for it), summed w * y in pick order into its token's partial, which goes to the ring slot of the
// job's step, then cpu_done = seq.
static void cpu_loop(bmx_copy_agent* a)
{
    const int H = a->cpu_desc.H, I = a->cpu_desc.I, E = a->t.E;
    std::vector<float> part, y;
    for (;;)
    {
        CpuJob job;
        {
            std::unique_lock<std::mutex> lk(a->cpu_mu);
            a->cpu_cv.wait(lk, [&] { return !a->cpu_q.empty() || a->stop.load(std::memory_order_acquire); });
            if (a->cpu_q.empty()) return;
            job = std::move(a->cpu_q.front());
            a->cpu_q.pop_front();
        }
        const int slot = ring_index(job.seq), n = (int)job.pick_e.size();
        const auto t_job = std::chrono::steady_clock::now();
        bool ok = true;
        int fast = 0;
        if (n > 0)
        {
            int ks_gu = 0, ks_dn = 0, grouped = 0;
            {
                std::lock_guard<std::mutex> lk(a->plan_mu);
                fast = a->policy.cpu_fast;
            }
            bmx_moe_desc d = a->cpu_desc;
            ok = bmx_decode_splits(&d, job.ntok, &ks_gu, &ks_dn, &grouped) == BMX_OK;
            part.assign((size_t)job.ntok * H, 0.0f);
            y.resize(H);
            for (int i = 0; ok && i < n; ++i)
            {
                const int e = job.pick_e[i], tt = job.pick_t[i];
                if (job.li < 0 || job.li >= a->t.L || e < 0 || e >= E || tt < 0 || tt >= job.ntok) { ok = false; break; }
                const bmx_cpu_expert* ce = &a->cpu_experts[(size_t)job.li * E + e];
                const uint16_t* xr = job.x.data() + (size_t)tt * H;
                ok = (fast ? bmx_cpu_expert_rows_fast(ce, H, I, xr, 1, d.act, d.gated, d.act_limit, y.data(), a->cpu_threads)
                           : bmx_cpu_expert_rows(ce, H, I, xr, 1, ks_gu, ks_dn, grouped, d.act, d.gated, d.act_limit,
                                                 y.data(), a->cpu_threads)) == BMX_OK;
                for (int h = 0; ok && h < H; ++h)
                {
                    const float pr = job.pick_w[i] * y[h];
                    part[(size_t)tt * H + h] = part[(size_t)tt * H + h] + pr;
                }
            }
            if (ok) memcpy(a->cpu_part + (size_t)slot * BMX_PLAN_MAXT * H, part.data(), part.size() * 4);
        }
        if (!ok) agent_fail(a, BMX_ERR_ARG);
        __atomic_store_n(&a->sh->cpu_t[slot], job.ntok, __ATOMIC_RELAXED);
        __atomic_store_n(&a->sh->cpu_n[slot], ok ? n : 0, __ATOMIC_RELAXED);
        const int64_t ns =
            std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t_job).count();
        a->cpu_jobs.fetch_add(1, std::memory_order_relaxed);
        a->cpu_ns.fetch_add(ns, std::memory_order_relaxed);
        if (ok && n > 0)
        {
            const double per = 1e-3 * (double)ns / n;
            std::lock_guard<std::mutex> lk(a->plan_mu);
            double& mean = a->cpu_pick_us[fast ? 1 : 0];
            mean = mean > 0.0 ? mean + (per - mean) / 8.0 : per;
        }
        __atomic_store_n(&a->sh->cpu_done, job.seq, __ATOMIC_RELEASE);
    }
}

// Serve request seq: plan, queue its CPU job (a request whose plan put picks on the CPU lane has one, in order), reply.
static void serve_plan(bmx_copy_agent* a, int64_t seq)
{
    const PlanReq& r = a->sh->req[ring_index(seq)];
    PlanRep& p = a->sh->rep[ring_index(seq)];
    if (r.nu < 0 || r.nu > PL_MAXU || r.nu > a->t.E || r.np < 0 || r.ntok < 0 || r.topk <= 0 ||
        (r.has_x && (r.ntok > BMX_PLAN_MAXT || r.np > BMX_PLAN_MAXP)))
    {
        agent_fail(a, BMX_ERR_ARG);
        return;
    }
    CpuJob cj;
    cj.seq = seq;
    plan_reply(a, r, p, r.has_x && a->cpu_ready ? &cj : nullptr);
    const bool job = !cj.pick_e.empty();
    if (job)
    {
        const int H = a->cpu_desc.H;
        const uint16_t* src = a->xring + (size_t)ring_index(seq) * BMX_PLAN_MAXT * H;
        cj.x.assign(src, src + (size_t)r.ntok * H);      // the step's rows leave the ring before the reply
        std::lock_guard<std::mutex> lk(a->cpu_mu);
        a->cpu_q.push_back(std::move(cj));
    }
    __atomic_store_n(&p.seq, seq, __ATOMIC_RELEASE);
    if (job) a->cpu_cv.notify_one();                     // the wake-up's system call after the reply, not before it
}

// The agent thread: records in sequence order; per step record the gate / up copies under one signal, the down copies
// under a second that waits for the first (and the first waits for the previous record's last); per prefetch record one
// copy per admission; flags stored in record order once each part's signal has reached zero.
static void agent_loop(bmx_copy_agent* a)
{
    std::vector<hsa_signal_t> sigs(AG_SIGNALS);
    for (auto& g : sigs)
        if (hsa_signal_create(0, 0, nullptr, &g) != HSA_STATUS_SUCCESS)
        {
            agent_fail(a, BMX_ERR_HIP);
            return;
        }
    struct Pending {
        int sig;        // index into sigs, -1: nothing to wait for
        int part;
        int64_t seq;
    };
    std::deque<Pending> pending;
    int sig_next = 0, last = -1;          // last: signal of the most recent part issued
    int64_t next = 1;
    const int E = a->t.E;
    const uint64_t off_u = (uint64_t)a->t.off_u, off_d = (uint64_t)a->t.off_d;
    auto copy = [&](uint64_t dst, uint64_t src, int64_t n, bool from_host, int sig, int dep) {
        const hsa_signal_t* deps = dep >= 0 ? &sigs[dep] : nullptr;
        if (hsa_amd_memory_async_copy(reinterpret_cast<void*>(dst), a->gpu, reinterpret_cast<const void*>(src),
                                      from_host ? a->cpu : a->gpu, (size_t)n, dep >= 0 ? 1 : 0, deps,
                                      sigs[sig]) != HSA_STATUS_SUCCESS)
        {
            agent_fail(a, BMX_ERR_HIP);
            hsa_signal_subtract_screlease(sigs[sig], 1);     // the part still completes
        }
        a->copies.fetch_add(1, std::memory_order_relaxed);
        a->copied_bytes.fetch_add(n, std::memory_order_relaxed);
    };
    auto last_work = std::chrono::steady_clock::now();
    int64_t served = 0;                   // the last planned step's request answered
    for (;;)
    {
        bool idle = true;
        // a planned step publishes its request under the sequence number of its record and waits for the reply before
        // it publishes the record
        if (served < next && !a->hold.load(std::memory_order_acquire) &&
            __atomic_load_n(&a->sh->req[ring_index(next)].seq, __ATOMIC_ACQUIRE) == next)
        {
            serve_plan(a, next);
            served = next;
            idle = false;
        }
        // retire completed parts in order
        while (!pending.empty())
        {
            const Pending& p = pending.front();
            if (p.sig >= 0)
            {
                const hsa_signal_value_t v = hsa_signal_load_scacquire(sigs[p.sig]);
                if (v > 0) break;
                if (v < 0) agent_fail(a, BMX_ERR_HIP);
            }
            __atomic_store_n(&a->sh->flags[p.part], p.seq, __ATOMIC_RELEASE);
            pending.pop_front();
            idle = false;
        }
        // the next record, if published and if two parts fit
        SlotPub* r = &a->sh->ring[ring_index(next)];
        if ((int)pending.size() + 2 <= AG_PENDING && !a->hold.load(std::memory_order_acquire) &&
            __atomic_load_n(&r->seq, __ATOMIC_ACQUIRE) == next)
        {
            const int n = r->n, li = r->li;
            const int64_t seq = next;
            const bool ok = n >= 0 && n <= a->t.maxj && li >= 0 && li < a->t.L;
            if (!ok) agent_fail(a, BMX_ERR_ARG);
            int nj = 0;
            int e_[64], s_[64];
            for (int j = 0; ok && j < n; ++j)
            {
                const int e = r->pairs[2 * j], s = r->pairs[2 * j + 1];
                if (e < 0 || e >= E || s < 0 || s >= a->t.S)
                {
                    agent_fail(a, BMX_ERR_ARG);
                    continue;
                }
                e_[nj] = e;
                s_[nj++] = s;
            }
            // the ring slot may be written again (by record next + AG_RING) from here on
            __atomic_store_n(&a->sh->consumed, next, __ATOMIC_RELEASE);
            if (nj > 0 && r->kind == 1)
            {
                // a prefetch: nothing waits for its gate / up alone, so one copy per admission (fewer DMA commands)
                const int gs = sig_next;
                sig_next = (sig_next + 2) % AG_SIGNALS;
                hsa_signal_store_relaxed(sigs[gs], nj);
                for (int j = 0; j < nj; ++j)
                {
                    const size_t k = (size_t)li * E + e_[j];
                    copy(a->slot_base[s_[j]], a->home[k], (int64_t)off_d + a->bytes[k * 3 + 2], a->home_host[k], gs, last);
                }
                last = gs;
                pending.push_back({gs, 0, seq});
                pending.push_back({-1, 1, seq});      // retires after the part before it
            }
            else if (nj > 0)
            {
                const int gs = sig_next, ds = (sig_next + 1) % AG_SIGNALS;
                sig_next = (sig_next + 2) % AG_SIGNALS;
                hsa_signal_store_relaxed(sigs[gs], nj);
                hsa_signal_store_relaxed(sigs[ds], nj);
                for (int j = 0; j < nj; ++j)
                {
                    const size_t k = (size_t)li * E + e_[j];
                    copy(a->slot_base[s_[j]], a->home[k], (int64_t)off_u + a->bytes[k * 3 + 1], a->home_host[k], gs, last);
                }
                for (int j = 0; j < nj; ++j)
                {
                    const size_t k = (size_t)li * E + e_[j];
                    copy(a->slot_base[s_[j]] + off_d, a->home[k] + off_d, a->bytes[k * 3 + 2], a->home_host[k], ds, gs);
                }
                last = ds;
                pending.push_back({gs, 0, seq});
                pending.push_back({ds, 1, seq});
            }
            else
            {
                pending.push_back({-1, 0, seq});
                pending.push_back({-1, 1, seq});
            }
            a->records.fetch_add(1, std::memory_order_relaxed);
            ++next;
            idle = false;
        }
        if (idle)
        {
            if (a->stop.load(std::memory_order_acquire) && pending.empty()) break;
            // spin while records keep coming (a decode step publishes one per layer); after 2 ms without any, poll
            // every 50 us so an idle table does not hold a core
            const auto now = std::chrono::steady_clock::now();
            if (pending.empty() && now - last_work > std::chrono::milliseconds(2))
                std::this_thread::sleep_for(std::chrono::microseconds(50));
            else __builtin_ia32_pause();
        }
        else last_work = std::chrono::steady_clock::now();
    }
    for (auto& g : sigs) hsa_signal_destroy(g);
}

struct AgentFind {
    uint32_t bdfid;
    int want_gpu_ordinal, gpu_seen;
    hsa_agent_t gpu, cpu, gpu_by_ordinal;
    bool have_gpu, have_cpu, have_ordinal;
};

static hsa_status_t find_agents(hsa_agent_t ag, void* data)
{
    auto* f = static_cast<AgentFind*>(data);
    hsa_device_type_t type;
    if (hsa_agent_get_info(ag, HSA_AGENT_INFO_DEVICE, &type) != HSA_STATUS_SUCCESS) return HSA_STATUS_SUCCESS;
    if (type == HSA_DEVICE_TYPE_CPU && !f->have_cpu)
    {
        f->cpu = ag;
        f->have_cpu = true;
    }
    else if (type == HSA_DEVICE_TYPE_GPU)
    {
        uint32_t bdf = 0;
        if (hsa_agent_get_info(ag, (hsa_agent_info_t)HSA_AMD_AGENT_INFO_BDFID, &bdf) == HSA_STATUS_SUCCESS &&
            bdf == f->bdfid && !f->have_gpu)
        {
            f->gpu = ag;
            f->have_gpu = true;
        }
        if (f->gpu_seen++ == f->want_gpu_ordinal)
        {
            f->gpu_by_ordinal = ag;
            f->have_ordinal = true;
        }
    }
    return HSA_STATUS_SUCCESS;
}

}  // namespace bmx

using namespace bmx;

extern "C" {

int bmx_copy_agent_create(const bmx_slot_table* t, const uint64_t* home, const int64_t* mat_bytes, bmx_copy_agent** out)
{
    if (!t || !home || !mat_bytes || !out) return set_error(BMX_ERR_ARG, "bmx_copy_agent_create: null argument");
    if (t->L <= 0 || t->E <= 0 || t->S < 0 || t->maxj < 0 || t->maxj > 64 || !t->slot_base)
        return set_error(BMX_ERR_ARG, "bmx_copy_agent_create: bad table");
    *out = nullptr;
    auto* a = new bmx_copy_agent();
    auto fail = [&](int code, const char* what) {
        if (a->need) (void)hipFree(a->need);
        if (a->sh) (void)hipHostFree(a->sh);
        if (a->hsa_up) hsa_shut_down();
        delete a;
        return set_error(code, "bmx_copy_agent_create: %s", what);
    };
    a->t = *t;
    const size_t K = (size_t)t->L * t->E;
    a->home.assign(home, home + K);
    a->bytes.assign(mat_bytes, mat_bytes + K * 3);
    a->home_host.assign(K, 0);
    for (size_t k = 0; k < K; ++k)
    {
        if (a->bytes[k * 3] < 0 || a->bytes[k * 3] > t->off_u || a->bytes[k * 3 + 1] < 0 ||
            t->off_u + a->bytes[k * 3 + 1] > t->off_d || a->bytes[k * 3 + 2] < 0 || t->off_d + a->bytes[k * 3 + 2] > t->rec)
            return fail(BMX_ERR_ARG, "an expert does not fit the slot geometry");
        hipPointerAttribute_t pa;
        if (hipPointerGetAttributes(&pa, reinterpret_cast<void*>(home[k])) != hipSuccess)
            return fail(BMX_ERR_ARG, "a home address is not memory HIP knows");
        if (pa.type == hipMemoryTypeHost) a->home_host[k] = 1;
        else if (pa.type != hipMemoryTypeDevice) return fail(BMX_ERR_ARG, "a home is neither pinned host nor device memory");
    }
    a->slot_base.resize(t->S > 0 ? t->S : 0);
    if (t->S > 0 && hipMemcpy(a->slot_base.data(), t->slot_base, (size_t)t->S * 8, hipMemcpyDeviceToHost) != hipSuccess)
        return fail(BMX_ERR_HIP, "reading slot addresses");
    int rate_khz = 0, bus = 0, dev = 0;
    if (hipGetDevice(&a->device) != hipSuccess ||
        hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, a->device) != hipSuccess || rate_khz <= 0 ||
        hipDeviceGetAttribute(&bus, hipDeviceAttributePciBusId, a->device) != hipSuccess ||
        hipDeviceGetAttribute(&dev, hipDeviceAttributePciDeviceId, a->device) != hipSuccess)
        return fail(BMX_ERR_HIP, "device query");
    a->ticks_per_us = (int64_t)rate_khz / 1000 > 0 ? (int64_t)rate_khz / 1000 : 1;
    a->wait_ticks = (int64_t)rate_khz * 1000 * 5;      // 5 s
    if (hsa_init() != HSA_STATUS_SUCCESS) return fail(BMX_ERR_HIP, "hsa_init");
    a->hsa_up = true;
    AgentFind f{};
    f.bdfid = ((uint32_t)bus << 8) | ((uint32_t)dev << 3);
    f.want_gpu_ordinal = a->device;
    if (hsa_iterate_agents(find_agents, &f) != HSA_STATUS_SUCCESS || !f.have_cpu || !(f.have_gpu || f.have_ordinal))
        return fail(BMX_ERR_HIP, "no HSA agents for the device and the host");
    a->gpu = f.have_gpu ? f.gpu : f.gpu_by_ordinal;
    a->cpu = f.cpu;
    void* p = nullptr;
    if (hipHostMalloc(&p, sizeof(AgentShared), hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess)
        return fail(BMX_ERR_HIP, "host ring");
    a->sh = static_cast<AgentShared*>(p);
    memset(a->sh, 0, sizeof(AgentShared));
    for (int i = 0; i < AG_RING; ++i) a->sh->ring[i].seq = -1;
    void* pd = nullptr;
    if (hipHostGetDevicePointer(&pd, p, 0) != hipSuccess) return fail(BMX_ERR_HIP, "host ring device address");
    a->sh_dev = static_cast<AgentShared*>(pd);
    if (hipMalloc(&a->need, (size_t)t->L * sizeof(int64_t)) != hipSuccess ||
        hipMemset(a->need, 0, (size_t)t->L * sizeof(int64_t)) != hipSuccess)
        return fail(BMX_ERR_HIP, "layer wait targets");
    a->th = std::thread(agent_loop, a);
    *out = a;
    return BMX_OK;
}

int bmx_copy_agent_destroy(bmx_copy_agent* a)
{
    if (!a) return BMX_OK;
    a->stop.store(true, std::memory_order_release);
    if (a->th.joinable()) a->th.join();
    {
        std::lock_guard<std::mutex> lk(a->cpu_mu);
        a->cpu_q.clear();
    }
    a->cpu_cv.notify_all();
    if (a->cpu_th.joinable()) a->cpu_th.join();
    const int err = a->error.load();
    if (a->xring) (void)hipHostFree(a->xring);
    if (a->cpu_part) (void)hipHostFree(a->cpu_part);
    if (a->sh) (void)hipHostFree(a->sh);
    if (a->need) (void)hipFree(a->need);
    if (a->hsa_up) hsa_shut_down();
    delete a;
    return err ? set_error(err, "bmx_copy_agent_destroy: the agent had failed") : BMX_OK;
}

// the failure visible to the host, as a status (0: none)
static int agent_failure(const bmx_copy_agent* a, const char* who)
{
    if (a->error.load()) return set_error(a->error.load(), "%s: copy agent failed (a copy failed or a record was malformed)", who);
    if (__atomic_load_n(&a->sh->flags[2], __ATOMIC_ACQUIRE))
        return set_error(BMX_ERR_HIP, "%s: copy agent aborted", who);
    if (__atomic_load_n(&a->sh->flags[3], __ATOMIC_ACQUIRE))
        return set_error(BMX_ERR_HIP, "%s: a copy wait ran out of time (slot contents since then are not trusted)", who);
    return BMX_OK;
}

int bmx_copy_agent_plan_stats(const bmx_copy_agent* a, int64_t* stats)
{
    if (!a || !stats) return set_error(BMX_ERR_ARG, "bmx_copy_agent_plan_stats: null argument");
    stats[0] = a->plans.load();
    stats[1] = a->plan_cpu.load();
    stats[2] = a->cpu_jobs.load();
    stats[3] = a->cpu_ns.load() / 1000;
    {
        std::lock_guard<std::mutex> lk(a->plan_mu);
        stats[4] = (int64_t)(a->cpu_pick_us[a->policy.cpu_fast ? 1 : 0] * 1e3);
    }
    return BMX_OK;
}

int bmx_copy_agent_control(bmx_copy_agent* a, int hold, int64_t wait_limit_us)
{
    if (!a) return set_error(BMX_ERR_ARG, "bmx_copy_agent_control: null agent");
    if (hold >= 0) a->hold.store(hold != 0, std::memory_order_release);
    if (wait_limit_us > 0) a->wait_ticks = wait_limit_us * a->ticks_per_us;
    return BMX_OK;
}

int bmx_copy_agent_status(const bmx_copy_agent* a, int64_t* stats)
{
    if (!a) return set_error(BMX_ERR_ARG, "bmx_copy_agent_status: null agent");
    if (stats)
    {
        stats[0] = a->records.load();
        stats[1] = a->copies.load();
        stats[2] = a->copied_bytes.load();
        stats[3] = __atomic_load_n(&a->sh->flags[0], __ATOMIC_ACQUIRE);
        stats[4] = __atomic_load_n(&a->sh->flags[1], __ATOMIC_ACQUIRE);
        stats[5] = __atomic_load_n(&a->sh->flags[3], __ATOMIC_ACQUIRE);
    }
    return agent_failure(a, "bmx_copy_agent_status");
}

int bmx_slot_step_agent(const bmx_slot_table* t, bmx_copy_agent* a, int li, const int64_t* sel, int n, int64_t first,
                        int admit, int64_t* seq, bmx_stream_t stream)
{
    if (!a || !seq) return set_error(BMX_ERR_ARG, "bmx_slot_step_agent: null agent or seq");
    const int64_t q = a->next_seq + 1;
    if (li < 0 || li >= a->t.L) return set_error(BMX_ERR_ARG, "bmx_slot_step_agent: bad layer %d", li);
    int rc = agent_failure(a, "bmx_slot_step_agent");
    if (rc) return rc;
    rc = launch_slot_step(t, li, sel, n, first, admit, static_cast<hipStream_t>(stream), a->sh_dev, q, a->need,
                          a->wait_ticks);
    if (rc) return rc;
    a->next_seq = q;
    *seq = q;
    return BMX_OK;
}

int bmx_route_slot_step(const bmx_slot_table* t, bmx_copy_agent* a, int li, const void* logits_fp16, const float* bias,
                        int E, int topk, int n_group, int topk_group, int score_fn, int renorm, float scale, int64_t first,
                        int admit, int64_t* sel, void* w_fp16, int64_t* seq, bmx_stream_t stream)
{
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (!a)
        return launch_route_slot_step(t, li, logits_fp16, bias, E, topk, n_group, topk_group, score_fn, renorm, scale,
                                      first, sel, w_fp16, admit, s, nullptr, 0, nullptr, 0);
    if (!seq) return set_error(BMX_ERR_ARG, "bmx_route_slot_step: null seq with an agent");
    if (li < 0 || li >= a->t.L) return set_error(BMX_ERR_ARG, "bmx_route_slot_step: bad layer %d", li);
    const int64_t q = a->next_seq + 1;
    int rc = agent_failure(a, "bmx_route_slot_step");
    if (rc) return rc;
    rc = launch_route_slot_step(t, li, logits_fp16, bias, E, topk, n_group, topk_group, score_fn, renorm, scale, first,
                                sel, w_fp16, admit, s, a->sh_dev, q, a->need, a->wait_ticks);
    if (rc) return rc;
    a->next_seq = q;
    *seq = q;
    return BMX_OK;
}

int bmx_slot_prefetch_agent(const bmx_slot_table* t, bmx_copy_agent* a, int li, const int64_t* sel, int n,
                            int64_t first, int limit, int64_t* seq, bmx_stream_t stream)
{
    if (!a || !seq) return set_error(BMX_ERR_ARG, "bmx_slot_prefetch_agent: null agent or seq");
    const int64_t q = a->next_seq + 1;
    int rc = agent_failure(a, "bmx_slot_prefetch_agent");
    if (rc) return rc;
    rc = launch_slot_prefetch(t, li, sel, n, first, limit, 0, static_cast<hipStream_t>(stream), a->sh_dev, q,
                              a->wait_ticks);
    if (rc) return rc;
    a->next_seq = q;
    *seq = q;
    return BMX_OK;
}

int bmx_copy_agent_plan(bmx_copy_agent* a, const bmx_plan_policy* p)
{
    if (!a) return set_error(BMX_ERR_ARG, "bmx_copy_agent_plan: null agent");
    bmx_plan_policy q{};
    if (p)
    {
        q = *p;
        if (q.max_cpu < 0 || q.gpu_base_us < 0 || q.gpu_hit_us < 0 || q.gpu_home_us < 0 || q.gpu_admit_us < 0 ||
            q.cpu_base_us < 0 || q.cpu_expert_us < 0 || q.cpu_token_us < 0)
            return set_error(BMX_ERR_ARG, "bmx_copy_agent_plan: negative count or cost");
    }
    std::lock_guard<std::mutex> lk(a->plan_mu);
    a->policy = q;
    return BMX_OK;
}

int bmx_copy_agent_cpu_lane(bmx_copy_agent* a, const bmx_moe_desc* desc, const bmx_cpu_expert* experts, int threads)
{
    if (!a || !desc || !experts) return set_error(BMX_ERR_ARG, "bmx_copy_agent_cpu_lane: null argument");
    if (a->cpu_ready) return set_error(BMX_ERR_ARG, "bmx_copy_agent_cpu_lane: already set up");
    if (desc->E != a->t.E || desc->H != a->t.H || desc->I != a->t.I || desc->H % 128 || desc->I % 128)
        return set_error(BMX_ERR_ARG, "bmx_copy_agent_cpu_lane: the descriptor's shape is not the slot table's");
    // fast-mode rows through the first experts of layer 0: the worker pool, tables and buffers are set up here rather
    // than in the first job, and the median time of the rows after the first seeds the fast mode's measured cost
    // (policy cpu_measured), which a single slow first job would otherwise hold high with no job run to correct it
    double seed_us = 0.0;
    {
        std::vector<uint16_t> z((size_t)desc->H, 0);
        std::vector<float> yz((size_t)desc->H);
        std::vector<double> ts;
        const int ne = std::min(desc->E, 5);
        for (int e = 0; e < ne; ++e)
        {
            const auto t0 = std::chrono::steady_clock::now();
            const int rc = bmx_cpu_expert_rows_fast(&experts[e], desc->H, desc->I, z.data(), 1, desc->act, desc->gated,
                                                    desc->act_limit, yz.data(), threads < 1 ? 1 : threads);
            if (rc) return rc;
            if (e > 0) ts.push_back(std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count());
        }
        if (!ts.empty())
        {
            std::sort(ts.begin(), ts.end());
            seed_us = ts[ts.size() / 2];
        }
    }
    const size_t K = (size_t)a->t.L * a->t.E, n = (size_t)AG_RING * BMX_PLAN_MAXT * desc->H;
    void *x = nullptr, *xd = nullptr, *pp = nullptr, *pd = nullptr;
    if (hipHostMalloc(&x, n * 2, hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess ||
        hipHostGetDevicePointer(&xd, x, 0) != hipSuccess ||
        hipHostMalloc(&pp, n * 4, hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess ||
        hipHostGetDevicePointer(&pd, pp, 0) != hipSuccess)
    {
        if (x) (void)hipHostFree(x);
        if (pp) (void)hipHostFree(pp);
        return set_error(BMX_ERR_HIP, "bmx_copy_agent_cpu_lane: pinned rings");
    }
    a->cpu_desc = *desc;
    a->cpu_experts.assign(experts, experts + K);
    a->cpu_threads = threads < 1 ? 1 : threads;
    a->xring = static_cast<uint16_t*>(x);
    a->xring_dev = static_cast<uint16_t*>(xd);
    a->cpu_part = static_cast<float*>(pp);
    a->cpu_part_dev = static_cast<float*>(pd);
    a->job_of.assign(AG_RING, 0);
    {
        std::lock_guard<std::mutex> lk(a->plan_mu);
        a->cpu_pick_us[1] = seed_us;
    }
    a->cpu_ready = true;
    a->cpu_th = std::thread(cpu_loop, a);
    return BMX_OK;
}

int bmx_slot_step_planned(const bmx_slot_table* t, bmx_copy_agent* a, int li, const int64_t* sel, const void* w_fp16,
                          int T, int topk, int64_t first, int admit, const void* x_fp16, int64_t* sel_gpu, void* w_gpu,
                          int32_t* lanes, int64_t* seq, bmx_stream_t stream)
{
    if (!a || !seq) return set_error(BMX_ERR_ARG, "bmx_slot_step_planned: null agent or seq");
    if (li < 0 || li >= a->t.L) return set_error(BMX_ERR_ARG, "bmx_slot_step_planned: bad layer %d", li);
    if (T < 0 || topk <= 0) return set_error(BMX_ERR_ARG, "bmx_slot_step_planned: bad T %d or topk %d", T, topk);
    if (x_fp16 && (reinterpret_cast<uintptr_t>(x_fp16) & 15))
        return set_error(BMX_ERR_ARG, "bmx_slot_step_planned: x must be 16-byte aligned");
    int rc = agent_failure(a, "bmx_slot_step_planned");
    if (rc) return rc;
    const int n = T * topk;
    const int64_t q = a->next_seq + 1;
    PlanArgs pl;
    pl.w = static_cast<const uint16_t*>(w_fp16);
    pl.T = T;
    pl.topk = topk;
    pl.H = a->t.H;
    const bool rows = a->cpu_ready && x_fp16 && T <= BMX_PLAN_MAXT && n <= BMX_PLAN_MAXP;
    pl.x = rows ? static_cast<const uint16_t*>(x_fp16) : nullptr;
    pl.xring = rows ? a->xring_dev : nullptr;
    pl.sel_gpu = sel_gpu;
    pl.w_gpu = static_cast<uint16_t*>(w_gpu);
    pl.lanes = lanes;
    rc = launch_slot_step(t, li, sel, n, first, admit, static_cast<hipStream_t>(stream), a->sh_dev, q, a->need,
                          a->wait_ticks, &pl);
    if (rc) return rc;
    if (a->cpu_ready) a->job_of[ring_index(q)] = rows ? q : 0;
    a->next_seq = q;
    *seq = q;
    return BMX_OK;
}

int bmx_cpu_lane_add(bmx_copy_agent* a, int64_t seq, float* out, int T, bmx_stream_t stream)
{
    if (!a || !out) return set_error(BMX_ERR_ARG, "bmx_cpu_lane_add: null agent or output");
    if (seq <= 0 || seq > a->next_seq || seq <= a->next_seq - AG_RING || T < 0 || T > BMX_PLAN_MAXT)
        return set_error(BMX_ERR_ARG, "bmx_cpu_lane_add: sequence number %lld is not one of the last %d steps, or T %d "
                         "> %d", (long long)seq, AG_RING, T, BMX_PLAN_MAXT);
    if (!a->cpu_ready || a->job_of[ring_index(seq)] != seq || T == 0) return BMX_OK;   // no CPU job for that step
    if (reinterpret_cast<uintptr_t>(out) & 15) return set_error(BMX_ERR_ARG, "bmx_cpu_lane_add: out must be 16-byte aligned");
    const unsigned wgs = (unsigned)(((size_t)T * a->t.H / 4 + 255) / 256);
    hipLaunchKernelGGL(k_cpu_add, dim3(wgs), dim3(256), 0, static_cast<hipStream_t>(stream), a->sh_dev, a->cpu_part_dev,
                       seq, out, T, a->t.H, a->wait_ticks);
    return check_launch("bmx_cpu_lane_add");
}

int bmx_copy_wait(bmx_copy_agent* a, int64_t seq, int part, bmx_stream_t stream)
{
    if (!a) return set_error(BMX_ERR_ARG, "bmx_copy_wait: null agent");
    if (part < 0 || part > 1 || seq <= 0 || seq > a->next_seq)
        return set_error(BMX_ERR_ARG, "bmx_copy_wait: bad part %d or sequence number %lld", part, (long long)seq);
    hipLaunchKernelGGL(k_copy_wait, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), a->sh_dev, part, seq,
                       nullptr, a->wait_ticks);
    return check_launch("bmx_copy_wait");
}

int bmx_copy_wait_layer(bmx_copy_agent* a, int li, int part, bmx_stream_t stream)
{
    if (!a) return set_error(BMX_ERR_ARG, "bmx_copy_wait_layer: null agent");
    if (part < 0 || part > 1 || li < 0 || li >= a->t.L)
        return set_error(BMX_ERR_ARG, "bmx_copy_wait_layer: bad part %d or layer %d", part, li);
    hipLaunchKernelGGL(k_copy_wait, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), a->sh_dev, part, (int64_t)0,
                       a->need + li, a->wait_ticks);
    return check_launch("bmx_copy_wait_layer");
}

}  // extern "C"
