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

#include <atomic>
#include <chrono>
#include <cstring>
#include <deque>
#include <thread>
#include <vector>

#include "bmx_internal.hpp"

namespace bmx {

constexpr int AG_PENDING = 256;  // parts in flight
constexpr int AG_SIGNALS = 2 * AG_PENDING;   // a signal is reused only after every part issued after it has retired

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

static void agent_fail(bmx_copy_agent* a, int code)
{
    int z = 0;
    a->error.compare_exchange_strong(z, code);
    __atomic_store_n(&a->sh->flags[2], 1, __ATOMIC_RELEASE);
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
    for (;;)
    {
        bool idle = true;
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
    const int err = a->error.load();
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
