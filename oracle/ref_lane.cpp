// C-ABI driver around the reference's CPU lane (engine/kernels/nv2/ft_core.h + ft_n135.h of Big-MoE-Small-Box, compiled
// from the reference tree by oracle/Makefile into oracle/_ref/libreflane.so; never shipped in the product).
//
// TEST INFRASTRUCTURE ONLY: the oracle's tests use it to pin the decode (dense_weights, state_scalar, tf_s) and the
// rounding points (prep_block / out_block), and bench.py times its moe_forward4 as the reference CPU baseline, driven
// the way the reference's cpu_forward drives it (engine/kernels/nv2/nv2_host.cpp:1974-2003).
#include "ft_n135.h"

#include <sched.h>

using namespace n135;

namespace {
struct LaneState
{
    Pool pool;
    Layer layer;
    bool started = false;
};
LaneState* g_lane = nullptr;
bool g_init = false;

void init_once()
{
    if (g_init) return;
    init_perm();
    init_tables();
    init_p16();
    g_init = true;
}
}  // namespace

extern "C" {

void ref_init() { init_once(); }

int ref_vbmi() { init_once(); return vbmi_ok ? 1 : 0; }

// ft_core.h dense_weights (K 3 only): trellis [k/16][n/16][96] -> W fp32 [k][n]
void ref_dense_weights_k3(const uint8_t* tr, int k, int n, float* W)
{
    init_once();
    Mat m{ tr, nullptr, nullptr, k, n };
    std::vector<float> v = dense_weights(m);
    std::memcpy(W, v.data(), v.size() * sizeof(float));
}

uint16_t ref_state_scalar_k3(const uint8_t* tile, int t) { return state_scalar(reinterpret_cast<const uint16_t*>(tile), t); }

float ref_w_gpu(uint16_t st) { return w_gpu(st); }

int ref_perm(int i) { init_once(); return PERM[i]; }

int ref_tf_s(int f, int i) { return tf_s(f, i); }

// prep_block / out_block on one 128-block (fp32 values, fp16 scales)
void ref_prep_block(const float* x, const uint16_t* suh, float* xt) { prep_block(x, suh, xt); }
void ref_prep_block_v(const float* x, const uint16_t* suh, float* xt) { prep_block_v(x, suh, xt); }
void ref_out_block(float* y, const uint16_t* svh) { out_block(y, svh); }
void ref_had128(float* v) { had128(v); }

// ---- lane forward (moe_forward4) -------------------------------------------------------------------------------------
// threads pinned to cpus[0 .. threads) (one per physical core, the reference's lane rule); the caller's affinity is
// restored after the pool starts (nv2_host.cpp cpu_init)
int ref_lane_create(int H, int I, int E, int threads, const int* cpus, float act_limit)
{
    init_once();
    if (g_lane) return -1;
    g_lane = new LaneState();
    std::vector<int> c(cpus, cpus + threads);
    cpu_set_t saved;
    sched_getaffinity(0, sizeof(saved), &saved);
    g_lane->pool.start(threads, c);
    sched_setaffinity(0, sizeof(saved), &saved);
    g_lane->started = true;
    g_lane->layer.H = H;
    g_lane->layer.I = I;
    g_lane->layer.ex.resize(E);
    g_act_limit = act_limit;
    return 0;
}

// one expert's three matrices: trellis pointers, fp16 scales, reference format codes (TF_K2 0, TF_K25 1, TF_K3 2)
int ref_lane_set_expert(int e, const uint8_t* g, const uint8_t* u, const uint8_t* d, const uint16_t* suh_g,
                        const uint16_t* svh_g, const uint16_t* suh_u, const uint16_t* svh_u, const uint16_t* suh_d,
                        const uint16_t* svh_d, int fg, int fu, int fd)
{
    if (!g_lane || e < 0 || e >= int(g_lane->layer.ex.size())) return -1;
    for (int f : { fg, fu, fd }) if (f < 0 || f >= TF_N) return -2;
    const int H = g_lane->layer.H, I = g_lane->layer.I;
    Expert& x = g_lane->layer.ex[e];
    x.g = { g, suh_g, svh_g, H, I, 0, TF_TB[fg], fg };
    x.u = { u, suh_u, svh_u, H, I, 0, TF_TB[fu], fu };
    x.d = { d, suh_d, svh_d, I, H, 0, TF_TB[fd], fd };
    return 0;
}

// x fp32 [m][H] (fp16-valued), sel int32 [m][k] (local expert ids), w fp32 [m][k] -> out fp32 [m][H]; mode -1 = auto
// (I16 when every expert has <= 2 tokens, else AFFINE), as cpu_forward picks it
int ref_lane_forward(const float* x, int m, const int32_t* sel, const float* w, int k, float* out, int mode)
{
    if (!g_lane) return -1;
    std::vector<std::vector<std::pair<int, float>>> route(m);
    std::vector<int> cnt(g_lane->layer.ex.size(), 0);
    int maxm = 0;
    for (int t = 0; t < m; ++t)
        for (int j = 0; j < k; ++j)
        {
            const int e = sel[t * k + j];
            if (e < 0 || e >= int(g_lane->layer.ex.size())) continue;
            route[t].push_back({ e, w[t * k + j] });
            maxm = std::max(maxm, ++cnt[e]);
        }
    const int md = mode >= 0 ? mode : (maxm <= 2 ? 2 : 0);
    moe_forward4(g_lane->pool, g_lane->layer, x, m, route, out, md);
    return md;
}

void ref_lane_destroy()
{
    if (!g_lane) return;
    g_lane->pool.stop();
    delete g_lane;
    g_lane = nullptr;
}

}  // extern "C"
