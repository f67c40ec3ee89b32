/*
 * bmx: MI355X-native (gfx950) routed-expert MoE layer. C ABI of libbmx.so.
 *
 * Every entry point is stream-ordered on the hipStream_t it is given (NULL = the legacy default stream), performs no
 * host synchronisation and allocates nothing: the caller owns every buffer, including the workspace sized by the
 * matching *_workspace() query. Pointers are device pointers unless stated. Status: BMX_OK or an error code; the text
 * of the last error of the calling thread is bmx_last_error().
 *
 * Reference interfaces (Big-MoE-Small-Box, paths relative to src/bigmoe/) each entry point stands in for are cited
 * beside it. The reference reaches its layer through exllamav3's BlockSparseMLP hooks (engine/tiers.py:703-739) and
 * the pybind modules bigmoe_ec / bigmoe_nv2 (engine/ec.py:184-189, engine/kernels/nv2/nv2_host.cpp:2081-2139); this
 * library is the native half of the same surface, reached from Python through ctypes (bmx/_lib.py).
 */
#ifndef BMX_H
#define BMX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BMX_ABI_VERSION 6

typedef void* bmx_stream_t; /* hipStream_t */

enum bmx_status {
    BMX_OK = 0,
    BMX_ERR_ARG = 1,         /* invalid argument (shape, format, null pointer, unsupported size) */
    BMX_ERR_HIP = 2,         /* a HIP runtime call failed (launch, copy, event) */
    BMX_ERR_WORKSPACE = 3,   /* workspace smaller than the matching *_workspace() query */
    BMX_ERR_UNSUPPORTED = 4  /* valid request the library does not implement */
};

/* EXL3 trellis formats: the reference's TF_K2 / TF_K25 / TF_K3 numbering (engine/kernels/nv2/ft_n135.h:78-81) plus
 * K 4. A tile is 16 x 16 weights in 32 K bytes; a matrix [k][n] is stored as tiles [k/16][n/16][32 K]. */
enum bmx_trellis_fmt { BMX_TF_K2 = 0, BMX_TF_K25 = 1, BMX_TF_K3 = 2, BMX_TF_K4 = 3 };

/* router score functions: softmax, sigmoid, sqrt(softplus) (exllamav3's ROUTING_ACT_SIGMOID / ROUTING_ACT_SQRTSP as the
 * reference selects them per layer, engine/nv2.py:146-148) */
enum bmx_score { BMX_SCORE_SOFTMAX = 0, BMX_SCORE_SIGMOID = 1, BMX_SCORE_SQRTSP = 2 };

/* expert activations, exllamav3's MOE_COOP_ACT_* numbering (engine/kernels/x16/x16_dev.cu:21-24) */
enum bmx_act { BMX_ACT_SILU = 0, BMX_ACT_GELU = 1, BMX_ACT_RELU2 = 2, BMX_ACT_SILU_OAI = 3 };

/* expert-products path: DECODE = bandwidth-bound grouped GEMVs (the reference's bsz-N decode kernel,
 * engine/kernels/x16/x16_dev.cu:205-392), PREFILL = grouped GEMMs on MFMA in groups of 128 rows (the reference's staged
 * prefill call, engine/tiers.py:673-700), MID = grouped GEMMs on MFMA in groups of 32 rows with k-splits (decode batches
 * of several tokens per expert), SPLIT = the DECODE or the MID kernels chosen on the device from the dispatch: every
 * expert on the MID kernels when the call has at least BMX_SPLIT_RATIO rows per unique expert (default 2.5), else on the
 * DECODE GEMVs except experts with at least BMX_SPLIT_MIN_ROWS rows (default off). AUTO picks PREFILL from
 * BMX_PREFILL_MIN_ROWS routed rows (T * topk; default 2048), MID from BMX_MID_MIN_TOKENS tokens (default 8; environment
 * variables), DECODE below; never SPLIT. */
enum bmx_path { BMX_PATH_AUTO = 0, BMX_PATH_DECODE = 1, BMX_PATH_PREFILL = 2, BMX_PATH_MID = 3, BMX_PATH_SPLIT = 4 };

/* One expert: three EXL3 linears (gate [H->I], up [H->I], down [I->H]). Device-resident array, one entry per expert.
 * tr[] is what the expert-slot table rewrites when an expert moves between its home and a VRAM slot (the reference's
 * per-layer pointer tables multi_{gate,up,down}.ptrs_trellis, engine/tiers.py:321-340). suh / svh are fp16 [k] / [n]. */
typedef struct bmx_expert {
    uint64_t tr[3];
    uint64_t suh[3];
    uint64_t svh[3];
    int32_t fmt[3];
    int32_t reserved;
} bmx_expert;

/* One MoE layer's geometry (exllamav3 BlockSparseMLP attributes the engine reads: num_experts_per_tok,
 * routing_first, num_local_experts, hidden_size, intermediate_size, activation_fn, act_limit, gated;
 * engine/tiers.py:270-275, engine/x16.py:37-56). */
typedef struct bmx_moe_desc {
    int32_t H, I, E, topk;
    int64_t first;               /* global id of local expert 0 (routing_first) */
    int32_t act, gated;
    float act_limit;             /* 0 = off */
    const bmx_expert* experts;   /* device [E] */
    const bmx_expert* shared;    /* device [1] or NULL: shared expert, weight 1, added after the routed slots */
    const int32_t* fresh;        /* device [E] or NULL: 1 = expert admitted to a slot by the last slot-table step (its
                                    copy may still be in flight); read by BMX_STAGE_GATE_UP_RESIDENT / _STAGED */
    const void* shared_gate;     /* device fp16 [H] or NULL: the shared expert's output is scaled by
                                    sigmoid(x[t] . shared_gate) before it is added (x16_red_k's sh_gate_w,
                                    engine/kernels/x16/x16_dev.cu:315-334, 375); NULL: weight 1 */
} bmx_moe_desc;

/* Dispatch output: rows grouped per expert, stable by (expert, token, slot). R = T * topk (+ T with a shared expert,
 * whose segment is expert index E). groups: work units of at most rows_per_group rows of one expert, [e, row0, nrows]. */
typedef struct bmx_routes {
    int32_t* counts;     /* [E + 1] rows per expert */
    int32_t* offsets;    /* [E + 2] exclusive prefix of counts */
    int32_t* row_token;  /* [R] token of each row */
    int32_t* row_slot;   /* [R] slot k of each row (-1: shared expert) */
    int32_t* inv;        /* [T * topk] row of pick (t, k); -1 = dropped pick (id outside [first, first + E)) */
    int32_t* uexp;       /* [E + 1] experts with rows, ascending */
    int32_t* nuniq;      /* [1] */
    int32_t* groups;     /* [bmx_groups_max(...) * 3] */
    int32_t* ngroups;    /* [1] */
    int32_t* row_expert; /* [R] expert of each row (E: shared expert) */
} bmx_routes;

const char* bmx_last_error(void);
int bmx_abi_version(void);
int bmx_tile_bytes(int fmt);

/* ---- EXL3 trellis dequantisation ----
 * trellis [k/16][n/16][tile] -> fp16 [k][n] codebook weights, bit-exact with exllamav3's decode (the reference's CPU
 * restatement: engine/kernels/nv2/ft_core.h:1007-1022 dense_weights; LinearEXL3.get_weight_tensor's trellis stage,
 * called at engine/nv2.py:696). k, n multiples of 16. */
int bmx_exl3_dequant(const void* trellis, int fmt, int k, int n, void* out_fp16, bmx_stream_t stream);

/* ---- router ----
 * exllamav3 routing_fn(bsz, cfg, z, params) -> (sel int64 [bsz, k], w fp16 [bsz, k]) as hooked at
 * engine/tiers.py:707-726 and run at engine/nv2.py:473-487 (routing_ds3_nogroup: sigmoid + selection bias).
 * logits fp16 [T, E]; bias fp32 [E] or NULL (selection only); n_group / topk_group = 1 / 1 for no group limit.
 * Selection: softmax -> top-k of the logits; sigmoid -> top-k of sigmoid(l) + bias; groups -> DeepSeek-V3 group-limited
 * (group score = sum of the top-2 choices, keep topk_group groups). Ties -> lower index. Weights: softmax probability or
 * sigmoid score, renormalised over the picks when renorm, times scale, fp16. E <= 1024, topk <= 32. */
int bmx_router_topk(const void* logits_fp16, const float* bias, int T, int E, int topk, int n_group, int topk_group,
                    int score_fn, int renorm, float scale, int64_t first, int64_t* sel, void* w_fp16,
                    bmx_stream_t stream);

/* Router projection: logits fp16 [T, E] = RN16(z W^T), z fp16 [T, H] (the MoE input rows), weight fp16 [E, H] (the
 * router's gate weight as checkpoints store it), fp32 accumulation on the MFMA units. The projection of exllamav3's
 * routing kernel (routing_ds3_nogroup(z, gate_tensor, logits_out, ...), engine/nv2.py:484-485, whose logits_out is fp16).
 * H a multiple of 64; z and weight 16-byte aligned. */
int bmx_router_logits(const void* z_fp16, const void* weight_fp16, int T, int H, int E, void* logits_fp16,
                      bmx_stream_t stream);

/* ---- dispatch ----
 * Token-to-expert counting sort (the histogram + ascending compaction of nv_pub_k, engine/kernels/nv2/
 * nv2_dev.cu:23-95, as contiguous per-expert row segments). */
int bmx_groups_max(int T, int topk, int E, int shared, int rows_per_group);
size_t bmx_dispatch_workspace(int T, int topk, int E);
int bmx_dispatch(const int64_t* sel, int T, int topk, int E, int64_t first, int shared, int rows_per_group,
                 const bmx_routes* out, void* workspace, size_t workspace_bytes, bmx_stream_t stream);

/* Router and dispatch in one launch, for decode-size calls (T * topk <= 256): the same outputs as bmx_router_topk
 * followed by bmx_dispatch (the reference's nv_pub_k publishes a token's routes in one kernel,
 * engine/kernels/nv2/nv2_dev.cu:23-95). */
int bmx_route_dispatch(const void* logits_fp16, const float* bias, int T, int E, int topk, int n_group, int topk_group,
                       int score_fn, int renorm, float scale, int64_t first, int shared, int rows_per_group, int64_t* sel,
                       void* w_fp16, const bmx_routes* out, bmx_stream_t stream);

/* ---- layer ----
 * The routed experts of one layer call plus the combine: exllamav3's BC_BlockSparseMLP run_bszN(z, sel, rw) writing
 * experts_cfg.out_bszn (engine/nv2.py:634-635) followed by cpu_split_combine (engine/tiers.py:730-739) and the
 * reduction order of x16_red_k (engine/kernels/x16/x16_dev.cu:298-392).
 * x fp16 [T, H]; sel int64 [T, topk], w fp16 [T, topk] (a router's output, or anything with dropped picks marked by
 * ids outside [first, first + E) or weight 0); out fp32 [T, H] = sum over k of w * expert(x) + shared(x).
 * Runs dispatch, the expert products (decode GEMV or prefill MFMA path) and the combine. */
size_t bmx_moe_workspace(const bmx_moe_desc* desc, int T, int path);
int bmx_moe_forward(const bmx_moe_desc* desc, const void* x_fp16, int T, const int64_t* sel, const void* w_fp16,
                    float* out, void* workspace, size_t workspace_bytes, int path, bmx_stream_t stream);

/* Router settings of a layer (exllamav3 routing_cfg as the engine reads it: sigmoid / softmax scoring, selection bias
 * e_score_correction_bias, n_group / topk_group, norm_topk_prob, routed_scaling_factor; engine/nv2.py:146-148). */
typedef struct bmx_router_desc {
    int32_t score_fn, renorm, n_group, topk_group;
    float scale;
    int32_t reserved;
    const float* bias;      /* device fp32 [E] or NULL */
    const void* weight;     /* device fp16 [E, H] or NULL: the router's gate weight, projected from x when the layer call
                               is given no logits (bmx_router_logits) */
} bmx_router_desc;

/* The whole layer call from router logits: router + dispatch (one kernel at decode sizes), expert products, combine.
 * The reference's per-layer sequence routing_fn -> Nv2.layer -> run_bszN -> cpu_split_combine (engine/tiers.py:707-739)
 * with the expert arithmetic of exllamav3. sel int64 [T, topk] and w fp16 [T, topk] receive the routing. logits_fp16
 * NULL: the logits are projected from x with router->weight first (bmx_router_logits, into the workspace). One token on
 * the decode path: the gate / up GEMV routes it and writes the dispatch itself (BMX_ROUTE_IN_GEMV=0: separate launch),
 * with as many gate / up k-splits as start in one round, which can be fewer than bmx_decode_splits reports for the
 * separate calls: the same routing, the output within the layer tolerance of theirs. That count follows the device's
 * compute-unit count (5 workgroups per unit), so one-token outputs can differ in their last bits between devices or
 * partition modes with other unit counts (BMX_CU_COUNT overrides the count; BMX_KS_GU forces the plan's splits). */
size_t bmx_moe_layer_workspace(const bmx_moe_desc* desc, int T, int path);
int bmx_moe_layer(const bmx_moe_desc* desc, const bmx_router_desc* router, const void* x_fp16, const void* logits_fp16,
                  int T, int64_t* sel, void* w_fp16, float* out, void* workspace, size_t workspace_bytes, int path,
                  bmx_stream_t stream);
/* bmx_moe_layer one stage set at a time (bit BMX_STAGE_ROUTE, then PREP, GATE_UP, ACT, DOWN, COMBINE, in that order over
 * calls with the same arguments and workspace): each call launches the kernels of its stages only, so a caller can time
 * them or put work between them. The calls together equal one bmx_moe_layer call bit for bit. */
int bmx_moe_layer_stages(const bmx_moe_desc* desc, const bmx_router_desc* router, const void* x_fp16,
                         const void* logits_fp16, int T, int64_t* sel, void* w_fp16, float* out, void* workspace,
                         size_t workspace_bytes, int path, int stages, bmx_stream_t stream);

/* The same layer call with no workspace argument and no allocation: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * The workspace is the library's own file-scope device array of BMX_SCRATCH_BYTES per GPU (held until the process
 * ends); calls whose bmx_moe_layer_workspace exceeds it fail with BMX_ERR_WORKSPACE (decode and mid-size batches fit,
 * large prefill chunks do not). Every call on a GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams, other threads) race and must be ordered by the caller. Nothing in the array needs to start at zero (each
 * call writes every value it reads). Results are bit-identical to bmx_moe_layer's. */
#define BMX_SCRATCH_BYTES (64u << 20)
int bmx_moe_layer_scratch(const bmx_moe_desc* desc, const bmx_router_desc* router, const void* x_fp16,
                          const void* logits_fp16, int T, int64_t* sel, void* w_fp16, float* out, int path,
                          bmx_stream_t stream);

/* Expert products only, on given routes (from bmx_dispatch with rows_per_group = bmx_rows_per_group(T, topk, path)):
 * y_rows fp32 [R, H] (expert output of each dispatch row), act_rows fp16 [R, I] (the rotated down input) or NULL.
 * bmx_resolve_path: the path (DECODE, PREFILL, MID or SPLIT) that `path` selects for T tokens of topk picks, -1 if
 * invalid. */
int bmx_rows_per_group(int T, int topk, int path);
int bmx_resolve_path(int T, int topk, int path);
size_t bmx_experts_workspace(const bmx_moe_desc* desc, int T, int path);
int bmx_moe_experts(const bmx_moe_desc* desc, const void* x_fp16, int T, const bmx_routes* routes, float* y_rows,
                    void* act_rows_fp16, void* workspace, size_t workspace_bytes, int path, bmx_stream_t stream);

/* bmx_moe_experts one kernel at a time, for callers that schedule or time the stages apart (exllamav3's kernel A /
 * kernel B split, docs/x16.md:38-54). Stages, in order, on the same workspace (bmx_experts_workspace):
 *   BMX_STAGE_PREP     rotated gate / up inputs of every row (PREFILL path; nothing on DECODE, whose GEMV rotates)
 *   BMX_STAGE_GATE_UP  gate / up products (DECODE: split-K GEMV partials; PREFILL: MFMA GEMM on the PREP rows)
 *   BMX_STAGE_ACT      gate / up epilogue -> fp16 down-input rows (act_rows, or the workspace's copy when NULL)
 *   BMX_STAGE_DOWN     down products                                               (reads act rows)
 *   BMX_STAGE_COMBINE  down epilogue + slot-ordered combine into out with weights w (y_rows also written if not NULL)
 *   BMX_STAGE_DOWN_OUT down epilogue into y_rows for every row (instead of COMBINE) */
enum bmx_stage {
    BMX_STAGE_GATE_UP = 0, BMX_STAGE_ACT = 1, BMX_STAGE_DOWN = 2, BMX_STAGE_COMBINE = 3, BMX_STAGE_DOWN_OUT = 4,
    BMX_STAGE_PREP = 5,
    /* BMX_STAGE_GATE_UP split by desc->fresh: the groups of experts that were resident before the slot-table step, and
     * the groups of experts it admitted (run after their copies). Together they equal BMX_STAGE_GATE_UP. */
    BMX_STAGE_GATE_UP_RESIDENT = 6, BMX_STAGE_GATE_UP_STAGED = 7,
    /* bmx_moe_layer_stages only: the router projection (when no logits are given), then the router and the dispatch
     * (these two are BMX_STAGE_GATE_UP's work instead where the one-token gate / up GEMV routes the token itself) */
    BMX_STAGE_ROUTE = 8,
    /* BMX_STAGE_DOWN split the same way (desc->fresh): the resident experts' down products can run while the admitted
     * experts' down parts are still being copied. Together they equal BMX_STAGE_DOWN. (ABI 6) */
    BMX_STAGE_DOWN_RESIDENT = 9, BMX_STAGE_DOWN_STAGED = 10
};
int bmx_moe_stage(const bmx_moe_desc* desc, int stage, const void* x_fp16, int T, const bmx_routes* routes,
                  void* act_rows_fp16, float* y_rows, const void* w_fp16, float* out, void* workspace,
                  size_t workspace_bytes, int path, bmx_stream_t stream);

/* ---- expert-slot table ----
 * (layer, expert) -> VRAM slot (the reference's Pool, engine/tiers.py:275-373, and its step kernel ec_step_k,
 * engine/ec.py:16-76). Every expert has a home holding its three trellis matrices (pinned host memory the GPU reads
 * directly, or device memory); S uniform slots of rec bytes (gate at 0, up at off_u, down at off_d) hold copies of
 * recently used experts. The layer tables' bmx_expert.tr point at the slot of a resident expert and at the home of any
 * other, so the expert kernels read either. All state is device memory the caller allocates and initialises (slotof and
 * owner -1, refb 0, pin 0 or < 0 for a disabled slot, ctl and stats 0, every table entry pointing at its home). Calls on
 * one table are stream-ordered by the caller. H and I give the matrix sizes: H * I / 256 tiles of the expert's format. */
typedef struct bmx_slot_table {
    int32_t L, E, S, maxj;      /* layers, experts per layer (<= 512), slots, admissions per step (<= 64) */
    int32_t H, I;
    int64_t rec, off_u, off_d;  /* slot bytes and the up / down offsets inside a slot (16-byte multiples) */
    int32_t* slotof;            /* [L * E] slot of (layer, expert), -1 = not resident */
    int32_t* owner;             /* [S] li * E + e of the slot's expert, -1 = free */
    int32_t* refb;              /* [S] CLOCK reference bits */
    int32_t* pin;               /* [S] step counter value of the slot's last use; < 0 = slot disabled */
    int32_t* ctl;               /* [4] CLOCK hand, step counter, admissions of the last step, reserved */
    int32_t* jobs;              /* [2 * maxj] (expert, slot) of each admission of the last step */
    int32_t* fresh;             /* [E] 1 = admitted by the last step, or a prefetched expert the step used for the first
                                   time (for bmx_moe_desc.fresh of that layer) */
    int64_t* stats;             /* [8] running hits, misses, admissions, steps without a victim, evictions, prefetch
                                   admissions, prefetched experts used by a step, prefetched experts evicted unused */
    const uint64_t* home;       /* [L * E * 3] device-visible address of each expert's gate, up, down trellis */
    const uint64_t* slot_base;  /* [S] address of each slot */
    const uint64_t* tables;     /* [L] address of each layer's bmx_expert table (E entries) */
    int32_t* pjobs;             /* [2 * (1 + 2 * maxj)] two prefetch job buffers: count, then (expert, slot) pairs */
    int32_t* pfl;               /* [S] 1 = admitted by a prefetch and not used by a step since (caller zeroes) */
} bmx_slot_table;

/* One step of layer li over the picks sel[n] (global ids, local = id - first): the layer's picked experts that are
 * resident are hits (reference bit set, pinned for this step); the others are misses, admitted when admit != 0 in
 * ascending expert order, at most maxj, each into the first slot from the CLOCK hand that is enabled, not pinned this
 * step and whose reference bit is clear (bits of slots passed over are cleared; at most 2 S probes per miss, a miss that
 * finds none ends the step's admissions). An admission evicts the slot's previous expert (its table entry back to its
 * home), points the admitted expert's entry at the slot, and writes a job; fresh marks the admitted experts and the hits
 * on slots a prefetch filled that no step has used yet (their copies may still be in flight, so the layer computes
 * them with its admissions, after the copies). One workgroup; no host synchronisation. Misses that are not admitted run
 * from their home. */
int bmx_slot_step(const bmx_slot_table* t, int li, const int64_t* sel, int n, int64_t first, int admit,
                  bmx_stream_t stream);
/* The copies of the last step's jobs of layer li, home -> slot (a kernel reading the home directly: pinned host memory
 * over PCIe). Run it on a side stream ordered after bmx_slot_step; the admitted experts' gate / up
 * (BMX_STAGE_GATE_UP_STAGED) must be ordered after it. */
int bmx_slot_copy(const bmx_slot_table* t, int li, bmx_stream_t stream);
/* The same copies restricted to the matrices in mats (bit 0 gate, 1 up, 2 down), so that the staged gate / up can start
 * when those two have landed while the down matrices are still in flight (the reference copies whole slots,
 * engine/ec.py:78-105). */
int bmx_slot_copy_mats(const bmx_slot_table* t, int li, int mats, bmx_stream_t stream);
/* Layer-ahead prefetch (the reference's next-layer routing guess, engine/nv2.py:450-487, whose picks it hands on as
 * prefetch hints, engine/kernels/nv2/nv2_dev.cu:75-85 and nv2_host.cpp:1046-1056): the first `limit` distinct guesses
 * sel[n] (n <= 512, best first, ids outside [first, first + E) ignored) that are not resident in layer li are admitted
 * in that order, at most maxj, within the current step counter (slots the last step pinned stay pinned and the counter
 * does not advance) by a gentle CLOCK sweep: the first enabled, unpinned slot from the hand whose reference bit is
 * clear, passing referenced slots without clearing their bits (at most S probes; a guess that finds none ends the
 * prefetch); admitted with the bit clear, so a wrong guess is the next victim. Resident guesses and every reference bit
 * are left alone. Jobs go to
 * prefetch buffer buf (0 or 1), never to the step's, so the copies of the last step may still be in flight. Stream
 * order: after the step of the layer being computed; the copies (bmx_slot_prefetch_copy) on the same side stream as
 * the step copies, before the next step's copies; the next prefetch into the same buffer after those copies. A
 * prefetch never changes a result: the layer's next step hands its prefetched hits to the staged part (fresh). */
int bmx_slot_prefetch(const bmx_slot_table* t, int li, const int64_t* sel, int n, int64_t first, int limit, int buf,
                      bmx_stream_t stream);
/* The copies of prefetch buffer buf's jobs of layer li (matrices in mats, as bmx_slot_copy_mats). */
int bmx_slot_prefetch_copy(const bmx_slot_table* t, int li, int buf, int mats, bmx_stream_t stream);
/* ---- copy agent ----
 * The slot table's home -> slot copies on the DMA engines, issued by a host thread (the reference's host-side staging,
 * engine/kernels/nv2/nv2_host.cpp:1558-1593, fed by picks the device publishes to mapped host memory,
 * engine/kernels/nv2/nv2_dev.cu:23-95). bmx_slot_step_agent / bmx_slot_prefetch_agent run the step / prefetch and publish
 * its admissions under the next sequence number (*seq); the agent's thread hands each published record, in order, to
 * the SDMA engines (per admission the gate / up part, then the down matrices) and marks each part done; bmx_copy_wait
 * orders a stream after a record's part (0 gate / up, 1 down) with a one-wave kernel that polls the mark (bounded: after
 * 5 s it gives up and bmx_copy_agent_status reports it). The records go through a ring of 64 in host memory: a step or
 * prefetch writes its slot only once the agent has read the record 64 before it (bounded the same way; publishing
 * nothing and reporting it when the limit passes). A kernel reading pinned host memory at link speed holds back
 * HBM-bound kernels on other streams; the DMA engines do not. Calls on one agent come from one host thread, its steps on
 * one stream. home[L * E]: each expert's record address (pinned host or device memory; gate at 0, up at off_u, down at
 * off_d, as the slots); mat_bytes[L * E * 3]: its trellis bytes. */
typedef struct bmx_copy_agent bmx_copy_agent;
int bmx_copy_agent_create(const bmx_slot_table* t, const uint64_t* home, const int64_t* mat_bytes,
                          bmx_copy_agent** agent);
int bmx_copy_agent_destroy(bmx_copy_agent* agent);
/* stats (or NULL) [6]: records, copies, bytes copied, gate / up mark, down mark, a wait ran out of time; returns an
 * error if a copy failed, the agent aborted or a wait ran out of time. Such a failure is final: from then on the steps
 * admit nothing (the experts they see run from their homes), bmx_slot_step_agent / bmx_slot_prefetch_agent return the
 * error without launching, and the slot contents of admissions whose copies had not completed are not trusted (the
 * layer calls that read them are to be discarded). Sequence numbers are 64-bit and never wrap. */
int bmx_copy_agent_status(const bmx_copy_agent* agent, int64_t* stats);
/* The residency planner's counts: stats[5] = requests answered, experts put on the CPU lane (summed over requests),
 * CPU jobs done (one per request with picks on the CPU lane), microseconds the CPU lane's worker spent on them, and the
 * running mean per CPU pick of the policy's mode in nanoseconds (what policy cpu_measured prices a CPU expert at; 0
 * while there is none). */
int bmx_copy_agent_plan_stats(const bmx_copy_agent* agent, int64_t* stats);
/* Failure-path control (the reference's controller has no counterpart; for tests that force a failure from the host):
 * hold >= 0 sets whether the agent's thread reads new records (1: it stops reading, so the waits run into their limit);
 * wait_limit_us > 0 sets the limit of the device-side waits launched after the call (default 5 s). */
int bmx_copy_agent_control(bmx_copy_agent* agent, int hold, int64_t wait_limit_us);
int bmx_slot_step_agent(const bmx_slot_table* t, bmx_copy_agent* agent, int li, const int64_t* sel, int n,
                        int64_t first, int admit, int64_t* seq, bmx_stream_t stream);
int bmx_slot_prefetch_agent(const bmx_slot_table* t, bmx_copy_agent* agent, int li, const int64_t* sel, int n,
                            int64_t first, int limit, int64_t* seq, bmx_stream_t stream);
/* A one-token layer call's routing (bmx_router_topk with T = 1; E = the table's experts) and its slot-table step
 * (bmx_slot_step_agent with the token's topk picks, or bmx_slot_step when agent is NULL; seq is then not written) in
 * one launch: the reference's routing_fn followed by the step of Nv2.layer (engine/nv2.py:470-487, then
 * engine/kernels/nv2/nv2_dev.cu:221-367 nv_step_k), whose two kernels this replaces for one token. The step's loads of
 * the slot state run beside the routing. Picks, weights and table state are those of the two calls. (ABI 6) */
int bmx_route_slot_step(const bmx_slot_table* t, bmx_copy_agent* agent, int li, const void* logits_fp16,
                        const float* bias, int E, int topk, int n_group, int topk_group, int score_fn, int renorm,
                        float scale, int64_t first, int admit, int64_t* sel, void* w_fp16, int64_t* seq,
                        bmx_stream_t stream);
int bmx_copy_wait(bmx_copy_agent* agent, int64_t seq, int part, bmx_stream_t stream);
/* Orders a stream after what layer li's products need from the copies (part 0 gate / up, 1 down): its last step's
 * record when that step admitted experts, else the records before it (the prefetches its hits came from); the step
 * leaves the target on the device, so a layer whose experts are in place waits for nothing in flight. */
int bmx_copy_wait_layer(bmx_copy_agent* agent, int li, int part, bmx_stream_t stream);

/* ---- CPU expert lane ----
 * One expert's y rows (fp32 [nr][H]: the down projection after svh, what BMX_STAGE_COMBINE sums in slot order) for nr
 * fp16 input rows [nr][H], computed on host cores bit for bit as the GPU decode path (BMX_PATH_DECODE) computes them for
 * the same rows (the reference's CPU lane, engine/kernels/nv2/nv2_host.cpp and docs/x16.md:1-133, is near-exact; this
 * one is exact: the device kernels sum in a fixed order, their activation is a fixed sequence of IEEE operations, and
 * v_dot2_f32_f16's rounding is emulated). ks_gu, ks_dn and grouped_gu are the device's plan for the call being matched
 * (bmx_decode_splits). Host memory only; threads = worker threads over output columns. Slow: a replay, not a kernel. */
typedef struct bmx_cpu_expert {
    const uint8_t* tr[3];      /* host trellis of gate, up, down */
    const uint16_t* suh[3];    /* host fp16 input scales */
    const uint16_t* svh[3];    /* host fp16 output scales */
    int32_t fmt[3];
    int32_t reserved;
} bmx_cpu_expert;
int bmx_cpu_expert_rows(const bmx_cpu_expert* ex, int H, int I, const uint16_t* x_fp16, int nr, int ks_gu, int ks_dn,
                        int grouped_gu, int act, int gated, float act_limit, float* y_rows, int threads);
/* The CPU lane's fast mode: the same y rows within the layer tolerance, not bit for bit (the reference's lane is not
 * bit-exact either; its host decode, engine/kernels/nv2/ft_core.h, is what this replaces for throughput). The trellis
 * decode gives the device's fp16 weights exactly (the codebook's fp32 FMA rounded once to fp16 equals its exact value for
 * every byte sum, checked at start-up); the products accumulate in fp32 FMAs over chunks of up to eight tile rows read in
 * memory order (the result does not depend on threads), without the device's k-splits or dot2 rounding; the rotations,
 * activation and roundings between the GEMVs are the exact lane's. AVX-512
 * (BW, VBMI, VNNI) when the host has it, else scalar. threads: a pool of that many persistent workers (the calling
 * thread is one), kept for later calls with the same count; calls are serialised on it. */
int bmx_cpu_expert_rows_fast(const bmx_cpu_expert* ex, int H, int I, const uint16_t* x_fp16, int nr, int act,
                             int gated, float act_limit, float* y_rows, int threads);
/* The device plan of a decode-path call of T tokens (bmx_moe_forward and the stage entry points; a one-token
 * bmx_moe_layer may take fewer gate / up splits): k-splits of the gate / up and down GEMVs, and whether the gate / up
 * epilogue sums the splits in four interleaved groups (small launches) or in sequence. */
int bmx_decode_splits(const bmx_moe_desc* desc, int T, int* ks_gu, int* ks_dn, int* grouped_gu);
/* out[i] = a[i].lo * b[i].lo + a[i].hi * b[i].hi + c[i] (fp16 pairs, fp32): bmx_cpu_dot2 emulates the device's
 * v_dot2_f32_f16 on the host; bmx_dot2_f32_f16 runs the instruction (device arrays), to check the emulation. */
int bmx_cpu_dot2(const uint32_t* a, const uint32_t* b, const float* c, float* out, int n);
int bmx_dot2_f32_f16(const uint32_t* a, const uint32_t* b, const float* c, float* out, int n, bmx_stream_t stream);

/* ---- residency plan: request, reply, CPU lane ----
 * The reference's controller protocol (engine/kernels/nv2/nv2_shared.h:36-59 Req / Rep, nv2_dev.cu:23-95 publish and
 * :221-367 nv_step_k reading the reply, nv2_host.cpp:947-1133 plan_and_reply / serve, :1306-1445 the CPU job). A planned
 * step publishes its layer call to the copy agent as a request: the unique experts it picks (ascending), whether each is
 * resident in a VRAM slot, how many picks each has, and for calls of at most BMX_PLAN_MAXP picks the picks themselves
 * (expert, fp16 weight) and, given x, the input rows of up to BMX_PLAN_MAXT tokens. The agent's thread answers each
 * request in sequence order with a lane per unique expert (bmx_plan_policy; a call whose experts are all resident
 * publishes no request, its plan being fixed); the step waits for the reply (bounded by
 * the agent's wait limit; running out of it is the agent failure bmx_copy_agent_status reports, after which the step
 * admits nothing) and applies it:
 *   BMX_LANE_VRAM   resident: a hit (the planner never moves a resident expert)
 *   BMX_LANE_ADMIT  admitted to a slot by the CLOCK step and copied by the agent (at most maxj per step, as
 *                   bmx_slot_step; one that finds no slot runs from its home)
 *   BMX_LANE_HOME   computed by the GPU from its home (the expert kernels read pinned host memory), not admitted
 *   BMX_LANE_CPU    masked out of the GPU's selection (sel_gpu -1, w_gpu 0) and computed by the agent's CPU lane
 * sel_gpu / w_gpu [n]: the selection the GPU computes (the others' picks as given); lanes [n] (or NULL): each pick's
 * lane, -1 for ids outside [first, first + E). */
#define BMX_PLAN_MAXP 64
#define BMX_PLAN_MAXT 8
enum { BMX_LANE_VRAM = 0, BMX_LANE_ADMIT = 1, BMX_LANE_HOME = 2, BMX_LANE_CPU = 3 };
/* The planner: list scheduling of a call's non-resident experts onto two lanes by estimated finish time (the
 * reference's rule, engine/kernels/nv2/nv2_host.cpp:1017-1030). The GPU's time starts at gpu_base_us + gpu_hit_us per
 * resident expert, or at 0 when no expert of the call is resident; the CPU lane's starts at cpu_base_us when the lane
 * is eligible (cpu_on, a CPU lane set up, the call's picks and rows travel with the request) and some expert is not
 * resident, else at 0. The experts not resident are taken by picks descending, then expert ascending (the reference
 * breaks equal pick counts by its cache's recency score first, which this table does not keep); each costs the GPU
 * gpu_admit_us (gpu_home_us when home_single is set, the call has several tokens and only one picked the expert: run
 * from the home rather than take a slot for one read) and the CPU lane cpu_expert_us + cpu_token_us per pick beyond the
 * first; it goes to the CPU lane when the lane is eligible, fewer than max_cpu are there already and the later of the
 * two finish times is then no later than with the GPU taking it, max(c + cost_cpu, g) <= max(c, g + cost_gpu); else to
 * the GPU (BMX_LANE_HOME or BMX_LANE_ADMIT). Default (no policy set): cpu_on 0, home_single 0, every miss
 * BMX_LANE_ADMIT. */
typedef struct bmx_plan_policy {
    int32_t cpu_on, max_cpu, home_single;
    int32_t cpu_fast;          /* 1: the agent's CPU jobs use bmx_cpu_expert_rows_fast; 0: the exact lane */
    int32_t cpu_measured;      /* 1: a CPU expert costs the worker's measured mean per pick in the policy's mode (a
                                  running mean over its jobs, 1/8 weight to the newest; the fast mode's seeded by timed
                                  rows at bmx_copy_agent_cpu_lane) in place of cpu_expert_us once there is one */
    double gpu_base_us, gpu_hit_us, gpu_home_us, gpu_admit_us;
    double cpu_base_us, cpu_expert_us, cpu_token_us;
} bmx_plan_policy;
int bmx_copy_agent_plan(bmx_copy_agent* agent, const bmx_plan_policy* policy);
/* The CPU lane of an agent: experts[L * E] host copies of every layer's experts (trellis, scales, formats; the shared
 * expert never goes to the CPU), desc: the layers' shape and activation (experts, shared and fresh ignored), threads:
 * worker threads per job. Without it the planner puts nothing on the CPU lane. A job computes each CPU pick's y row of
 * its token with bmx_cpu_expert_rows (bit for bit the GPU decode path's row for the call's T), or with
 * bmx_cpu_expert_rows_fast when the policy's cpu_fast is set, and sums w * y in pick order into the token's partial
 * (fp32 [T][H]). */
int bmx_copy_agent_cpu_lane(bmx_copy_agent* agent, const bmx_moe_desc* desc, const bmx_cpu_expert* experts, int threads);
int bmx_slot_step_planned(const bmx_slot_table* t, bmx_copy_agent* agent, int li, const int64_t* sel,
                          const void* w_fp16, int T, int topk, int64_t first, int admit, const void* x_fp16,
                          int64_t* sel_gpu, void* w_gpu, int32_t* lanes, int64_t* seq, bmx_stream_t stream);
/* out[T][H] += the CPU lane's partial of planned step seq (after its combine, the reference's nv_combine_k add,
 * nv2_dev.cu:513-551): waits (bounded, as the copy waits) for the agent's CPU job of seq; adds nothing when the plan put
 * no pick on the CPU. Enqueue it before the 64th step after seq. */
int bmx_cpu_lane_add(bmx_copy_agent* agent, int64_t seq, float* out, int T, bmx_stream_t stream);

/* Host-planned staging: n copies src[i] -> dst[i] of bytes[i] (hipMemcpyAsync, e.g. pinned host -> slot), in order on
 * stream (the reference's stage_layer, engine/kernels/nv2/nv2_host.cpp:1558-1593). */
int bmx_slot_stage_async(const void* const* src, void* const* dst, const size_t* bytes, int n, bmx_stream_t stream);
/* Staged prefill (prefill-size calls admit nothing: engine/tiers.py:395-463): restore = 0 points layer li's table entries
 * of experts[j] (device int32, local ids, j < n <= E) at staging record j, base + j * rec with the slot geometry (the
 * reference's index_copy_ of the staging addresses into the layer's pointer rows, engine/tiers.py:441-451); restore = 1
 * points each back at where the expert lives now, its slot if resident, else its home (nv_restore_k,
 * engine/kernels/nv2/nv2_dev.cu:554-566). base: device address, 256-byte aligned. Stream-ordered, one small kernel. */
int bmx_slot_stage_rows(const bmx_slot_table* t, int li, const int32_t* experts, int n, uint64_t base, int restore,
                        bmx_stream_t stream);
/* Device-visible address of pinned host memory (hipHostGetDevicePointer), for bmx_slot_table.home. */
int bmx_host_device_ptr(void* host, uint64_t* device_addr);

/* Combine: out[t] = sum over k ascending of w[t, k] * y_rows[inv[t, k]] (picks with inv < 0 or w = 0 skipped), then
 * + y_rows[offsets[E] + t] when has_shared (x16_red_k order, engine/kernels/x16/x16_dev.cu:354-384). The shared row is
 * added with weight 1: a layer with a gated shared expert (bmx_moe_desc.shared_gate, weight sigmoid(x . g)) is combined
 * by the layer calls (bmx_moe_forward, bmx_moe_layer, BMX_STAGE_COMBINE of bmx_moe_stage), not by this entry. */
int bmx_combine(const float* y_rows, const int32_t* inv, const void* w_fp16, const int32_t* offsets, int T, int topk,
                int H, int E, int has_shared, float* out, bmx_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* BMX_H */
