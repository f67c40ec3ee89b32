// Host-side internals shared by the bmx translation units: error state and kernel-launch entry points.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/bmx.h"

namespace bmx {

int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int check_launch(const char* what);

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// dequant.hip
int launch_dequant(const void* trellis, int fmt, int k, int n, void* out, hipStream_t s);

// router.hip
int launch_router(const void* logits, const float* bias, int T, int E, int topk, int n_group, int topk_group,
                  int score_fn, int renorm, float scale, int64_t first, int64_t* sel, void* w, hipStream_t s);

int launch_router_logits(const void* z, const void* W, int T, int H, int E, void* logits, hipStream_t s);
bool route_dispatch_small_fits(int T, int E, int topk);
struct RouteFuse;
int route_fuse_args(const void* logits, const float* bias, int T, int E, int topk, int n_group, int topk_group,
                    int score_fn, int renorm, float scale, int64_t first, int64_t* sel, void* w, int shared, int rpg,
                    const bmx_routes* routes, RouteFuse* out);
int launch_route_dispatch_small(const void* logits, const float* bias, int T, int E, int topk, int n_group,
                                int topk_group, int score_fn, int renorm, float scale, int64_t first, int64_t* sel,
                                void* w, int shared, int rpg, const bmx_routes* routes, hipStream_t s);

// dispatch.hip
struct DispatchWs {
    int32_t* rank;      // [T * topk]
    int32_t* blk_hist;  // [nblk * (E + 1)]
};
size_t dispatch_ws_bytes(int T, int topk, int E);
int launch_dispatch(const int64_t* sel, int T, int topk, int E, int64_t first, int shared, int rows_per_group,
                    const bmx_routes* out, void* ws, size_t ws_bytes, int32_t* zero_ptr, int zero_count,
                    hipStream_t s);
int groups_max(int T, int topk, int E, int shared, int rows_per_group);

// moe_decode.hip
struct MoeShape {
    int H, I, E, topk, T, shared, act, gated;
    float limit;
    int64_t first;
    const bmx_expert* experts;
    const bmx_expert* shared_ex;
    const int32_t* fresh;
    const uint16_t* shared_gate;   // fp16 [H] or null
};
struct DecodePlan {
    int KS_gu, KS_dn, NB, NBH, G_max, R_max;
    size_t part_gu_bytes, part_dn_bytes, counters;
};
DecodePlan decode_plan(const MoeShape& m);
int decode_gu_grouped(const MoeShape& m);     // 1: the gate / up epilogue sums the k-splits in four interleaved groups
size_t decode_ws_bytes(const MoeShape& m);
// ws layout: [part_gu][part_dn][act rows (used when act_rows == NULL)]; stages: 1 = gate/up, 2 = down (+ combine)
int launch_decode_experts(const MoeShape& m, const void* x, const bmx_routes* r, float* y_rows, void* act_rows,
                          void* ws, size_t ws_bytes, float* combine_out, const void* combine_w, hipStream_t s, int stages,
                          const RouteFuse* rf = nullptr);
int decode_rows_per_group(int T);
// split path (BMX_PATH_SPLIT): the decode GEMVs for experts with few rows, the mid-size MFMA GEMMs for experts with at
// least split_min_rows() rows, in one call; ws layout [part_gu][part_dn][act rows][xt]
int split_min_rows();
size_t split_ws_bytes(const MoeShape& m);
int launch_split_experts(const MoeShape& m, const void* x, const bmx_routes* r, float* y_rows, void* act_rows,
                         void* ws, size_t ws_bytes, float* combine_out, const void* combine_w, hipStream_t s, int stages);
int launch_combine(const float* y_rows, const int32_t* inv, const void* w, const int32_t* offsets, int T, int topk,
                   int H, int E, int has_shared, float* out, hipStream_t s);
int launch_zero_i32(int32_t* p, int n, hipStream_t s);

// slots.hip
// A step's or prefetch's admissions published to the copy agent (fine-grained host memory): the payload, then seq with a
// system-scope release store. Sequence numbers are 64-bit and start at 1: they never wrap.
struct SlotPub {
    int64_t seq;
    int32_t li, n, kind, pad;     // kind: 0 step, 1 prefetch
    int32_t pairs[2 * 64];        // (expert, slot) of each admission
};
constexpr int AG_RING = 64;       // records in the ring: record q lives in ring[q % AG_RING]
__host__ __device__ inline int ring_index(int64_t seq) { return (int)((uint64_t)seq % AG_RING); }
// The memory a copy agent shares with the kernels. flags[0] gate / up done, flags[1] down done (sequence numbers);
// flags[2] abort (the waits end at once); flags[3] set by a wait that ran out of time. consumed: the last record the
// agent has read out of the ring (its slot may be written again by record consumed + AG_RING). Once flags[2] or
// flags[3] is set, steps admit nothing (every expert they see runs from its home) and publish nothing, and the host
// entry points of the agent report the failure.
// A planned step's request (device -> host) and the planner's reply (host -> device), ring slot seq % AG_RING
constexpr int PL_MAXU = 512;
struct PlanReq {
    int64_t seq;                    // written last (system-scope release)
    int32_t li, nu, np, ntok, topk, has_x;
    int32_t ex[PL_MAXU];            // unique local experts, ascending
    int32_t res[PL_MAXU];           // 1: resident in a VRAM slot at publication
    int32_t cnt[PL_MAXU];           // picks of each
    int32_t pe[BMX_PLAN_MAXP];      // np <= BMX_PLAN_MAXP: local expert of each pick, -1 out of range
    uint16_t pw[BMX_PLAN_MAXP];     // its fp16 weight
};
struct PlanRep {
    int64_t seq;                    // written last
    int32_t ncpu, pad;
    int32_t lane[PL_MAXU];          // BMX_LANE_* of each unique expert
};
struct AgentShared {
    int64_t flags[4];
    int64_t consumed;
    int64_t cpu_done;               // the last planned step whose CPU job has finished (jobs finish in sequence order)
    int64_t pad[2];
    SlotPub ring[AG_RING];
    PlanReq req[AG_RING];
    PlanRep rep[AG_RING];
    int32_t cpu_n[AG_RING];         // CPU picks of the job in that slot (0: nothing to add)
    int32_t cpu_t[AG_RING];         // its tokens: the partial rows the job wrote
};
// A planned step (slots.hip): the request's extra inputs and the step's masked outputs. xring: device address of the
// agent's input-row ring [AG_RING][BMX_PLAN_MAXT][H] fp16 in host memory.
struct PlanArgs {
    const uint16_t* w;
    int T, topk, H;
    const uint16_t* x;
    uint16_t* xring;
    int64_t* sel_gpu;
    uint16_t* w_gpu;
    int32_t* lanes;
};
// router argument checks (bmx_router_topk's), for the entries that route inside other kernels
int check_router(int T, int E, int topk, int n_group, int topk_group, int score_fn, const void* logits, const void* sel,
                 const void* w);
// one token's routing and the slot-table step of layer li in one launch (sh: the copy agent's ring, or null)
int launch_route_slot_step(const bmx_slot_table* t, int li, const void* logits, const float* bias, int E, int topk,
                           int n_group, int topk_group, int score_fn, int renorm, float scale, int64_t first, int64_t* sel,
                           void* w, int admit, hipStream_t s, AgentShared* sh, int64_t seq, int64_t* need,
                           int64_t wait_limit);
// Publishing (sh != null): the step writes ring[seq % AG_RING] once the agent has consumed record seq - AG_RING, waiting
// at most wait_limit wall-clock ticks (then it sets flags[3]). need (steps only): need[li] = the last record layer li's
// next products depend on (seq when the step admitted experts, seq - 1 when it did not: its prefetched hits came with
// earlier records)
int launch_slot_step(const bmx_slot_table* t, int li, const int64_t* sel, int n, int64_t first, int admit, hipStream_t s,
                     AgentShared* sh = nullptr, int64_t seq = 0, int64_t* need = nullptr, int64_t wait_limit = 0,
                     const PlanArgs* plan = nullptr);
int launch_slot_prefetch(const bmx_slot_table* t, int li, const int64_t* sel, int n, int64_t first, int limit, int buf,
                         hipStream_t s, AgentShared* sh = nullptr, int64_t seq = 0, int64_t wait_limit = 0);
int launch_slot_copy(const bmx_slot_table* t, int li, int mats, int buf, hipStream_t s);

// moe_prefill.hip (same ws / stage conventions; ws layout [xt][part_gu][act rows][part_dn])
int prefill_rows_per_group();
int mid_rows_per_group();
size_t mid_ws_bytes(const MoeShape& m);
int launch_mid_experts(const MoeShape& m, const void* x, const bmx_routes* r, float* y_rows, void* act_rows, void* ws,
                       size_t ws_bytes, float* combine_out, const void* combine_w, hipStream_t s, int stages);
size_t prefill_ws_bytes(const MoeShape& m);
int launch_prefill_experts(const MoeShape& m, const void* x, const bmx_routes* r, float* y_rows, void* act_rows,
                           void* ws, size_t ws_bytes, float* combine_out, const void* combine_w, hipStream_t s,
                           int stages);

}  // namespace bmx
