// C ABI of libbmx.so (include/bmx.h): argument checks, workspace layout, launch order.
#include "bmx_common.hpp"
#include "bmx_internal.hpp"
#include "router_wave.hpp"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

namespace bmx {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what)
{
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(BMX_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return BMX_OK;
}

static int check_desc(const bmx_moe_desc* d, const char* who)
{
    if (!d) return set_error(BMX_ERR_ARG, "%s: null descriptor", who);
    if (d->H <= 0 || d->I <= 0 || d->H % 128 || d->I % 128)
        return set_error(BMX_ERR_ARG, "%s: H (%d) and I (%d) must be positive multiples of 128", who, d->H, d->I);
    if (d->E <= 0 || d->E > 512 || d->topk <= 0 || d->topk > 32)
        return set_error(BMX_ERR_ARG, "%s: unsupported E=%d topk=%d", who, d->E, d->topk);
    if (!d->experts) return set_error(BMX_ERR_ARG, "%s: null expert table", who);
    if (d->act < BMX_ACT_SILU || d->act > BMX_ACT_SILU_OAI) return set_error(BMX_ERR_ARG, "%s: unknown activation %d", who, d->act);
    if (reinterpret_cast<uintptr_t>(d->shared_gate) % 16)
        return set_error(BMX_ERR_ARG, "%s: the shared expert's gate vector must be 16-byte aligned", who);
    return BMX_OK;
}

static MoeShape shape_of(const bmx_moe_desc* d, int T)
{
    MoeShape m;
    m.H = d->H; m.I = d->I; m.E = d->E; m.topk = d->topk; m.T = T; m.shared = d->shared ? 1 : 0;
    m.act = d->act; m.gated = d->gated; m.limit = d->act_limit; m.first = d->first;
    m.experts = d->experts; m.shared_ex = d->shared; m.fresh = d->fresh;
    m.shared_gate = static_cast<const uint16_t*>(d->shared_gate);
    return m;
}

// routes carved from a workspace
struct RoutesLayout {
    size_t counts, offsets, row_token, row_slot, inv, uexp, nuniq, groups, ngroups, row_expert, total;
};

static RoutesLayout routes_layout(int T, int topk, int E, int shared, int rpg)
{
    RoutesLayout L;
    const size_t NE = (size_t)E + 1, R = (size_t)T * topk + (shared ? T : 0), G = (size_t)groups_max(T, topk, E, shared, rpg);
    size_t o = 0;
    auto take = [&](size_t bytes) { const size_t at = o; o += align_up(bytes, 256); return at; };
    L.counts = take(NE * 4);
    L.offsets = take((NE + 1) * 4);
    L.row_token = take(R * 4 + 4);
    L.row_slot = take(R * 4 + 4);
    L.inv = take((size_t)T * topk * 4 + 4);
    L.uexp = take(NE * 4);
    L.nuniq = take(4);
    L.groups = take(G * 12);
    L.ngroups = take(4);
    L.row_expert = take(R * 4 + 4);
    L.total = o;
    return L;
}

static bmx_routes routes_at(char* base, const RoutesLayout& L)
{
    bmx_routes r;
    r.counts = reinterpret_cast<int32_t*>(base + L.counts);
    r.offsets = reinterpret_cast<int32_t*>(base + L.offsets);
    r.row_token = reinterpret_cast<int32_t*>(base + L.row_token);
    r.row_slot = reinterpret_cast<int32_t*>(base + L.row_slot);
    r.inv = reinterpret_cast<int32_t*>(base + L.inv);
    r.uexp = reinterpret_cast<int32_t*>(base + L.uexp);
    r.nuniq = reinterpret_cast<int32_t*>(base + L.nuniq);
    r.groups = reinterpret_cast<int32_t*>(base + L.groups);
    r.ngroups = reinterpret_cast<int32_t*>(base + L.ngroups);
    r.row_expert = reinterpret_cast<int32_t*>(base + L.row_expert);
    return r;
}

constexpr int STAGES_LAYER = (1 << BMX_STAGE_PREP) | (1 << BMX_STAGE_GATE_UP) | (1 << BMX_STAGE_ACT) | (1 << BMX_STAGE_DOWN) | (1 << BMX_STAGE_COMBINE);

// AUTO: the GEMV path below BMX_MID_MIN_TOKENS tokens, the mid-size MFMA path below BMX_PREFILL_MIN_ROWS routed rows
// (T * topk), the prefill MFMA path from there up
static long env_rows(const char* name, long dflt)
{
    const char* v = getenv(name);
    return (v && *v) ? atol(v) : dflt;
}

// BMX_ROUTE_IN_GEMV=0: a one-token layer call launches route + dispatch before its gate / up GEMV (same results)
static bool route_in_gemv_allowed()
{
    const char* v = getenv("BMX_ROUTE_IN_GEMV");
    return !(v && *v == '0');
}

// AUTO below the prefill threshold: the mid-size MFMA path from BMX_MID_MIN_TOKENS tokens (8), the GEMV path below.
// Measured on MI355X (layer us, GEMV / mid-size): GLM-shaped (H 4096, I 1536) T 4 135 / 146, T 6 196 / 190, T 8 234 /
// 219, T 16 354 / 316, T 32 533 / 432; DeepSeek-shaped (H 4096, I 2048, Zipf routing) T 6 165 / 168, T 8 201 / 193,
// T 32 524 / 450; 16 tokens on ~10 experts 180 / 107; the 64-expert H 2048 layer crosses over later (T 8 72 / 83, T 16
// 98 / 94). Mid-size / prefill (128-row groups): DeepSeek-shaped T 86 (516 rows) 819 / 917, T 256 1426 / 1519, T 512
// 1911 / 1883, T 2048 3546 / 2627; GLM-shaped T 64 554 / 661, T 128 680 / 771. The split path (BMX_PATH_SPLIT) is never
// chosen here: the mid-size path alone is faster wherever the split path would send a call to the MFMA kernels.
static int resolve_path(int path, int T, int topk)
{
    if (path == BMX_PATH_DECODE || path == BMX_PATH_PREFILL || path == BMX_PATH_MID || path == BMX_PATH_SPLIT)
        return path;
    if (path != BMX_PATH_AUTO) return -1;
    const long rows = (long)T * topk;
    if (rows >= env_rows("BMX_PREFILL_MIN_ROWS", 2048)) return BMX_PATH_PREFILL;
    if (T >= env_rows("BMX_MID_MIN_TOKENS", 8)) return BMX_PATH_MID;
    return BMX_PATH_DECODE;
}

static int path_rows_per_group(int path, int T)
{
    return path == BMX_PATH_PREFILL ? prefill_rows_per_group() : path == BMX_PATH_MID ? mid_rows_per_group()
                                                                                       : decode_rows_per_group(T);
}

static size_t experts_ws_bytes(int path, const MoeShape& m)
{
    return path == BMX_PATH_PREFILL ? prefill_ws_bytes(m) : path == BMX_PATH_MID ? mid_ws_bytes(m)
           : path == BMX_PATH_SPLIT ? split_ws_bytes(m) : decode_ws_bytes(m);
}

static int launch_experts(int path, const MoeShape& m, const void* x, const bmx_routes* r, float* y_rows, void* act_rows,
                          void* ws, size_t ws_bytes, float* combine_out, const void* combine_w, hipStream_t s, int stages)
{
    if (path == BMX_PATH_PREFILL)
        return launch_prefill_experts(m, x, r, y_rows, act_rows, ws, ws_bytes, combine_out, combine_w, s, stages);
    if (path == BMX_PATH_MID)
        return launch_mid_experts(m, x, r, y_rows, act_rows, ws, ws_bytes, combine_out, combine_w, s, stages);
    if (path == BMX_PATH_SPLIT)
        return launch_split_experts(m, x, r, y_rows, act_rows, ws, ws_bytes, combine_out, combine_w, s, stages);
    return launch_decode_experts(m, x, r, y_rows, act_rows, ws, ws_bytes, combine_out, combine_w, s, stages);
}

// ---- the allocation-free layer call's workspace ----
// A file-scope device array: every GPU the library runs on holds its own copy for the life of the process. Host code
// never passes the array's name to a kernel (on the host it is a stand-in symbol, not a device address): the address
// of the current device's copy comes from hipGetSymbolAddress, once per device, at that device's first call.
static __device__ __align__(256) uint8_t scratch[BMX_SCRATCH_BYTES];
constexpr int SCRATCH_DEVICES = 64;
static void* g_scratch[SCRATCH_DEVICES];
static std::mutex g_scratch_mu;

static int scratch_of_current_device(void** out)
{
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(BMX_ERR_HIP, "bmx_moe_layer_scratch: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= SCRATCH_DEVICES)
        return set_error(BMX_ERR_UNSUPPORTED, "bmx_moe_layer_scratch: device %d (at most %d devices)", dev, SCRATCH_DEVICES);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev])
    {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(BMX_ERR_HIP, "bmx_moe_layer_scratch: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                             hipGetErrorString(e));
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return BMX_OK;
}

}  // namespace bmx

using namespace bmx;

extern "C" {

const char* bmx_last_error(void) { return g_err; }

int bmx_abi_version(void) { return BMX_ABI_VERSION; }

int bmx_tile_bytes(int fmt) { return tile_bytes_of(fmt); }

int bmx_exl3_dequant(const void* trellis, int fmt, int k, int n, void* out_fp16, bmx_stream_t stream)
{
    if (k < 0 || n < 0 || k % 16 || n % 16) return set_error(BMX_ERR_ARG, "bmx_exl3_dequant: k (%d), n (%d) must be multiples of 16", k, n);
    if (tile_bytes_of(fmt) < 0) return set_error(BMX_ERR_ARG, "bmx_exl3_dequant: unknown trellis format %d", fmt);
    if ((k && n) && (!trellis || !out_fp16)) return set_error(BMX_ERR_ARG, "bmx_exl3_dequant: null pointer");
    if (reinterpret_cast<uintptr_t>(trellis) % 16) return set_error(BMX_ERR_ARG, "bmx_exl3_dequant: trellis must be 16-byte aligned");
    return launch_dequant(trellis, fmt, k, n, out_fp16, static_cast<hipStream_t>(stream));
}

int bmx_router_topk(const void* logits_fp16, const float* bias, int T, int E, int topk, int n_group, int topk_group,
                    int score_fn, int renorm, float scale, int64_t first, int64_t* sel, void* w_fp16, bmx_stream_t stream)
{
    return launch_router(logits_fp16, bias, T, E, topk, n_group, topk_group, score_fn, renorm, scale, first, sel,
                         w_fp16, static_cast<hipStream_t>(stream));
}

int bmx_router_logits(const void* z_fp16, const void* weight_fp16, int T, int H, int E, void* logits_fp16,
                      bmx_stream_t stream)
{
    return launch_router_logits(z_fp16, weight_fp16, T, H, E, logits_fp16, static_cast<hipStream_t>(stream));
}

int bmx_groups_max(int T, int topk, int E, int shared, int rows_per_group)
{
    if (T < 0 || topk <= 0 || E <= 0 || rows_per_group <= 0) return -1;
    return groups_max(T, topk, E, shared, rows_per_group);
}

size_t bmx_dispatch_workspace(int T, int topk, int E) { return dispatch_ws_bytes(T, topk, E); }

int bmx_dispatch(const int64_t* sel, int T, int topk, int E, int64_t first, int shared, int rows_per_group,
                 const bmx_routes* out, void* workspace, size_t workspace_bytes, bmx_stream_t stream)
{
    return launch_dispatch(sel, T, topk, E, first, shared, rows_per_group, out, workspace, workspace_bytes, nullptr, 0,
                           static_cast<hipStream_t>(stream));
}

int bmx_route_dispatch(const void* logits_fp16, const float* bias, int T, int E, int topk, int n_group, int topk_group,
                       int score_fn, int renorm, float scale, int64_t first, int shared, int rows_per_group, int64_t* sel,
                       void* w_fp16, const bmx_routes* out, bmx_stream_t stream)
{
    if (!out || rows_per_group <= 0) return set_error(BMX_ERR_ARG, "bmx_route_dispatch: null routes or rows_per_group");
    if (!route_dispatch_small_fits(T, E, topk))
        return set_error(BMX_ERR_ARG, "bmx_route_dispatch: T * topk = %ld picks exceeds 256 (use bmx_router_topk + "
                         "bmx_dispatch)", (long)T * topk);
    return launch_route_dispatch_small(logits_fp16, bias, T, E, topk, n_group, topk_group, score_fn, renorm, scale, first,
                                       sel, w_fp16, shared, rows_per_group, out, static_cast<hipStream_t>(stream));
}

int bmx_rows_per_group(int T, int topk, int path)
{
    const int p = resolve_path(path, T, topk);
    if (p < 0 || T < 0 || topk <= 0) return -1;
    return path_rows_per_group(p, T);
}

int bmx_decode_splits(const bmx_moe_desc* desc, int T, int* ks_gu, int* ks_dn, int* grouped_gu)
{
    int rc = check_desc(desc, "bmx_decode_splits");
    if (rc) return rc;
    if (T <= 0 || !ks_gu || !ks_dn || !grouped_gu) return set_error(BMX_ERR_ARG, "bmx_decode_splits: bad arguments");
    const MoeShape m = shape_of(desc, T);
    const DecodePlan p = decode_plan(m);
    *ks_gu = p.KS_gu;
    *ks_dn = p.KS_dn;
    *grouped_gu = decode_gu_grouped(m);
    return BMX_OK;
}

static __global__ void k_dot2(const uint32_t* a, const uint32_t* b, const float* c, float* out, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a[i]), __builtin_bit_cast(f16x2, b[i]), c[i], false);
}

int bmx_dot2_f32_f16(const uint32_t* a, const uint32_t* b, const float* c, float* out, int n, bmx_stream_t stream)
{
    if (n < 0 || (n && (!a || !b || !c || !out))) return set_error(BMX_ERR_ARG, "bmx_dot2_f32_f16: bad arguments");
    if (n == 0) return BMX_OK;
    hipLaunchKernelGGL(k_dot2, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream), a, b, c,
                       out, n);
    return check_launch("bmx_dot2_f32_f16");
}

int bmx_resolve_path(int T, int topk, int path) { return T < 0 || topk <= 0 ? -1 : resolve_path(path, T, topk); }

size_t bmx_experts_workspace(const bmx_moe_desc* desc, int T, int path)
{
    if (check_desc(desc, "bmx_experts_workspace") || T < 0) return 0;
    const int p = resolve_path(path, T, desc->topk);
    if (p < 0) return 0;
    return experts_ws_bytes(p, shape_of(desc, T));
}

int bmx_moe_experts(const bmx_moe_desc* desc, const void* x_fp16, int T, const bmx_routes* routes, float* y_rows,
                    void* act_rows_fp16, void* workspace, size_t workspace_bytes, int path, bmx_stream_t stream)
{
    int rc = check_desc(desc, "bmx_moe_experts");
    if (rc) return rc;
    const int p = resolve_path(path, T, desc->topk);
    if (p < 0) return set_error(BMX_ERR_ARG, "bmx_moe_experts: unknown path %d", path);
    if (T < 0) return set_error(BMX_ERR_ARG, "bmx_moe_experts: T < 0");
    if (T == 0) return BMX_OK;
    if (!x_fp16 || !routes || !y_rows || !workspace) return set_error(BMX_ERR_ARG, "bmx_moe_experts: null pointer");
    return launch_experts(p, shape_of(desc, T), x_fp16, routes, y_rows, act_rows_fp16, workspace, workspace_bytes,
                                 nullptr, nullptr, static_cast<hipStream_t>(stream),
                                 (1 << BMX_STAGE_PREP) | (1 << BMX_STAGE_GATE_UP) | (1 << BMX_STAGE_ACT) | (1 << BMX_STAGE_DOWN) |
                                 (1 << BMX_STAGE_DOWN_OUT));
}

int bmx_moe_stage(const bmx_moe_desc* desc, int stage, const void* x_fp16, int T, const bmx_routes* routes,
                  void* act_rows_fp16, float* y_rows, const void* w_fp16, float* out, void* workspace,
                  size_t workspace_bytes, int path, bmx_stream_t stream)
{
    int rc = check_desc(desc, "bmx_moe_stage");
    if (rc) return rc;
    const int p = resolve_path(path, T, desc->topk);
    if (p < 0 || T < 0) return set_error(BMX_ERR_ARG, "bmx_moe_stage: bad path or T");
    if (stage < BMX_STAGE_GATE_UP || stage > BMX_STAGE_DOWN_STAGED || stage == BMX_STAGE_ROUTE)
        return set_error(BMX_ERR_ARG, "bmx_moe_stage: unknown stage %d", stage);
    if ((stage == BMX_STAGE_GATE_UP_RESIDENT || stage == BMX_STAGE_GATE_UP_STAGED || stage == BMX_STAGE_DOWN_RESIDENT ||
         stage == BMX_STAGE_DOWN_STAGED) && !desc->fresh)
        return set_error(BMX_ERR_ARG, "bmx_moe_stage: split gate / up and down stages need desc->fresh");
    if (T == 0) return BMX_OK;
    if (!routes || !workspace) return set_error(BMX_ERR_ARG, "bmx_moe_stage: null pointer");
    if ((stage == BMX_STAGE_GATE_UP || stage == BMX_STAGE_PREP || stage == BMX_STAGE_GATE_UP_RESIDENT ||
         stage == BMX_STAGE_GATE_UP_STAGED) && !x_fp16)
        return set_error(BMX_ERR_ARG, "bmx_moe_stage: gate/up needs x");
    if (stage == BMX_STAGE_COMBINE && (!out || !w_fp16)) return set_error(BMX_ERR_ARG, "bmx_moe_stage: combine needs out and w");
    if (stage == BMX_STAGE_DOWN_OUT && !y_rows) return set_error(BMX_ERR_ARG, "bmx_moe_stage: down_out needs y_rows");
    return launch_experts(p, shape_of(desc, T), x_fp16, routes, y_rows, act_rows_fp16, workspace, workspace_bytes,
                          out, w_fp16, static_cast<hipStream_t>(stream), 1 << stage);
}

int bmx_combine(const float* y_rows, const int32_t* inv, const void* w_fp16, const int32_t* offsets, int T, int topk,
                int H, int E, int has_shared, float* out, bmx_stream_t stream)
{
    if (T < 0 || topk <= 0 || H <= 0 || E <= 0) return set_error(BMX_ERR_ARG, "bmx_combine: bad sizes");
    if (T && (!y_rows || !inv || !w_fp16 || !out || (has_shared && !offsets)))
        return set_error(BMX_ERR_ARG, "bmx_combine: null pointer");
    return launch_combine(y_rows, inv, w_fp16, offsets, T, topk, H, E, has_shared, out, static_cast<hipStream_t>(stream));
}

size_t bmx_moe_workspace(const bmx_moe_desc* desc, int T, int path)
{
    if (check_desc(desc, "bmx_moe_workspace") || T < 0) return 0;
    const int p = resolve_path(path, T, desc->topk);
    if (p < 0) return 0;
    const MoeShape m = shape_of(desc, T);
    const RoutesLayout L = routes_layout(T, desc->topk, desc->E, m.shared, path_rows_per_group(p, T));
    return L.total + align_up(dispatch_ws_bytes(T, desc->topk, desc->E), 256) + align_up(experts_ws_bytes(p, m), 256);
}

int bmx_moe_forward(const bmx_moe_desc* desc, const void* x_fp16, int T, const int64_t* sel, const void* w_fp16,
                    float* out, void* workspace, size_t workspace_bytes, int path, bmx_stream_t stream)
{
    int rc = check_desc(desc, "bmx_moe_forward");
    if (rc) return rc;
    const int p = resolve_path(path, T, desc->topk);
    if (p < 0) return set_error(BMX_ERR_ARG, "bmx_moe_forward: unknown path %d", path);
    if (T < 0) return set_error(BMX_ERR_ARG, "bmx_moe_forward: T < 0");
    if (T == 0) return BMX_OK;
    if (!x_fp16 || !sel || !w_fp16 || !out || !workspace) return set_error(BMX_ERR_ARG, "bmx_moe_forward: null pointer");
    const size_t need = bmx_moe_workspace(desc, T, path);
    if (workspace_bytes < need) return set_error(BMX_ERR_WORKSPACE, "bmx_moe_forward: workspace %zu < %zu", workspace_bytes, need);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const MoeShape m = shape_of(desc, T);
    const int rpg = path_rows_per_group(p, T);
    const RoutesLayout L = routes_layout(T, desc->topk, desc->E, m.shared, rpg);
    char* base = static_cast<char*>(workspace);
    const bmx_routes r = routes_at(base, L);
    char* dws = base + L.total;
    const size_t dws_bytes = align_up(dispatch_ws_bytes(T, desc->topk, desc->E), 256);
    char* ews = dws + dws_bytes;
    const size_t ews_bytes = align_up(experts_ws_bytes(p, m), 256);
    rc = launch_dispatch(sel, T, desc->topk, desc->E, desc->first, m.shared, rpg, &r, dws, dws_bytes, nullptr, 0, s);
    if (rc) return rc;
    return launch_experts(p, m, x_fp16, &r, nullptr, nullptr, ews, ews_bytes, out, w_fp16, s, STAGES_LAYER);
}

// the layer call's workspace: bmx_moe_forward's, then the projected logits [T][E] fp16 (used when no logits are given)
size_t bmx_moe_layer_workspace(const bmx_moe_desc* desc, int T, int path)
{
    const size_t base = bmx_moe_workspace(desc, T, path);
    if (!base) return 0;
    return base + align_up((size_t)T * desc->E * 2, 256);
}

// bmx_moe_layer and bmx_moe_layer_stages: the stages in `stages` (BMX_STAGE_ROUTE and the layer's expert stages) of
// one layer call; every call of a staged sequence recomputes the same host-side plan, so the stages agree on the
// workspace layout and the gate / up k-split count
static int layer_call(const char* fn, const bmx_moe_desc* desc, const bmx_router_desc* router, const void* x_fp16,
                      const void* logits_fp16, int T, int64_t* sel, void* w_fp16, float* out, void* workspace,
                      size_t workspace_bytes, int path, int stages, hipStream_t s)
{
    int rc = check_desc(desc, fn);
    if (rc) return rc;
    if (!router) return set_error(BMX_ERR_ARG, "%s: null router descriptor", fn);
    const int p = resolve_path(path, T, desc->topk);
    if (p < 0) return set_error(BMX_ERR_ARG, "%s: unknown path %d", fn, path);
    if (T < 0) return set_error(BMX_ERR_ARG, "%s: T < 0", fn);
    if (!stages || (stages & ~(STAGES_LAYER | (1 << BMX_STAGE_ROUTE))))
        return set_error(BMX_ERR_ARG, "%s: stage mask 0x%x (route, prep, gate / up, act, down and combine only)", fn,
                         stages);
    if (T == 0) return BMX_OK;
    if (!x_fp16 || !sel || !w_fp16 || !out || !workspace) return set_error(BMX_ERR_ARG, "%s: null pointer", fn);
    if (!logits_fp16 && !router->weight)
        return set_error(BMX_ERR_ARG, "%s: no logits and no router weight to project them with", fn);
    const size_t need = bmx_moe_layer_workspace(desc, T, path);
    if (workspace_bytes < need) return set_error(BMX_ERR_WORKSPACE, "%s: workspace %zu < %zu", fn, workspace_bytes, need);
    const bool route = stages & (1 << BMX_STAGE_ROUTE);
    stages &= STAGES_LAYER;
    if (!logits_fp16)
    {
        void* lg = static_cast<char*>(workspace) + bmx_moe_workspace(desc, T, path);
        if (route)
        {
            rc = launch_router_logits(x_fp16, router->weight, T, desc->H, desc->E, lg, s);
            if (rc) return rc;
        }
        logits_fp16 = lg;
    }
    const MoeShape m = shape_of(desc, T);
    const int rpg = path_rows_per_group(p, T);
    const RoutesLayout L = routes_layout(T, desc->topk, desc->E, m.shared, rpg);
    char* base = static_cast<char*>(workspace);
    const bmx_routes r = routes_at(base, L);
    char* dws = base + L.total;
    const size_t dws_bytes = align_up(dispatch_ws_bytes(T, desc->topk, desc->E), 256);
    char* ews = dws + dws_bytes;
    const size_t ews_bytes = align_up(experts_ws_bytes(p, m), 256);
    if (T == 1 && p == BMX_PATH_DECODE && rpg == 1 && route_dispatch_small_fits(T, desc->E, desc->topk) &&
        route_in_gemv_allowed())
    {
        // one token: the gate / up GEMV routes it and writes the dispatch itself (one launch fewer)
        RouteFuse f;
        rc = route_fuse_args(logits_fp16, router->bias, T, desc->E, desc->topk, router->n_group, router->topk_group,
                             router->score_fn, router->renorm, router->scale, desc->first, sel, w_fp16, m.shared, rpg,
                             &r, &f);
        if (rc || !stages) return rc;
        return launch_decode_experts(m, x_fp16, &r, nullptr, nullptr, ews, ews_bytes, out, w_fp16, s, stages, &f);
    }
    if (route)
    {
        if (route_dispatch_small_fits(T, desc->E, desc->topk))
            rc = launch_route_dispatch_small(logits_fp16, router->bias, T, desc->E, desc->topk, router->n_group,
                                             router->topk_group, router->score_fn, router->renorm, router->scale,
                                             desc->first, sel, w_fp16, m.shared, rpg, &r, s);
        else
        {
            rc = launch_router(logits_fp16, router->bias, T, desc->E, desc->topk, router->n_group, router->topk_group,
                               router->score_fn, router->renorm, router->scale, desc->first, sel, w_fp16, s);
            if (!rc)
                rc = launch_dispatch(sel, T, desc->topk, desc->E, desc->first, m.shared, rpg, &r, dws, dws_bytes, nullptr,
                                     0, s);
        }
        if (rc) return rc;
    }
    if (!stages) return BMX_OK;
    return launch_experts(p, m, x_fp16, &r, nullptr, nullptr, ews, ews_bytes, out, w_fp16, s, stages);
}

int bmx_moe_layer(const bmx_moe_desc* desc, const bmx_router_desc* router, const void* x_fp16, const void* logits_fp16,
                  int T, int64_t* sel, void* w_fp16, float* out, void* workspace, size_t workspace_bytes, int path,
                  bmx_stream_t stream)
{
    return layer_call("bmx_moe_layer", desc, router, x_fp16, logits_fp16, T, sel, w_fp16, out, workspace,
                      workspace_bytes, path, STAGES_LAYER | (1 << BMX_STAGE_ROUTE), static_cast<hipStream_t>(stream));
}

int bmx_moe_layer_stages(const bmx_moe_desc* desc, const bmx_router_desc* router, const void* x_fp16,
                         const void* logits_fp16, int T, int64_t* sel, void* w_fp16, float* out, void* workspace,
                         size_t workspace_bytes, int path, int stages, bmx_stream_t stream)
{
    return layer_call("bmx_moe_layer_stages", desc, router, x_fp16, logits_fp16, T, sel, w_fp16, out, workspace,
                      workspace_bytes, path, stages, static_cast<hipStream_t>(stream));
}

int bmx_moe_layer_scratch(const bmx_moe_desc* desc, const bmx_router_desc* router, const void* x_fp16,
                          const void* logits_fp16, int T, int64_t* sel, void* w_fp16, float* out, int path,
                          bmx_stream_t stream)
{
    int rc = check_desc(desc, "bmx_moe_layer_scratch");
    if (rc) return rc;
    if (T < 0 || resolve_path(path, T, desc->topk) < 0)
        return set_error(BMX_ERR_ARG, "bmx_moe_layer_scratch: bad T (%d) or path (%d)", T, path);
    const size_t need = bmx_moe_layer_workspace(desc, T, path);
    if (need > (size_t)BMX_SCRATCH_BYTES)
        return set_error(BMX_ERR_WORKSPACE, "bmx_moe_layer_scratch: this call needs %zu bytes of workspace, more than the "
                         "%zu of the library's scratch array (call bmx_moe_layer with a workspace instead)", need,
                         (size_t)BMX_SCRATCH_BYTES);
    void* ws = nullptr;
    rc = scratch_of_current_device(&ws);
    if (rc) return rc;
    return bmx_moe_layer(desc, router, x_fp16, logits_fp16, T, sel, w_fp16, out, ws, BMX_SCRATCH_BYTES, path, stream);
}

}  // extern "C"
