/*
 * CPU oracle for the routed-expert MoE layer: TEST INFRASTRUCTURE ONLY (see bmx_oracle.h).
 *
 * Reference paths are relative to src/bigmoe/ of Big-MoE-Small-Box. Build: oracle/Makefile (-ffp-contract=off, so
 * every fp32 operation below is rounded exactly where it is written).
 */
#include "bmx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------------------------------------------- */
/* fp16                                                                                                             */
/* ---------------------------------------------------------------------------------------------------------------- */

uint16_t bmxo_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t e = (x >> 23) & 0xffu;
    uint32_t m = x & 0x7fffffu;
    if (e == 0xffu) return (uint16_t)(sign | 0x7c00u | (m ? (0x200u | (m >> 13)) : 0u));
    const int ee = (int)e - 127 + 15;
    if (ee <= 0)
    {
        if (ee < -10) return (uint16_t)sign;
        m |= 0x800000u;
        const int shift = 14 - ee;
        uint32_t hm = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) ++hm;
        return (uint16_t)(sign | hm);
    }
    if (ee >= 31) return (uint16_t)(sign | 0x7c00u);
    const uint32_t hm = m >> 13, rem = m & 0x1fffu;
    uint32_t r = sign | ((uint32_t)ee << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) ++r;   /* a carry moves into the exponent (up to inf) */
    return (uint16_t)r;
}

float bmxo_f16_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu, x;
    if (e == 0)
    {
        if (m == 0) x = sign;
        else
        {
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; ++sh; }
            x = sign | ((uint32_t)(113 - sh) << 23) | ((m & 0x3ffu) << 13);
        }
    }
    else if (e == 31) x = sign | 0x7f800000u | (m << 13);
    else x = sign | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ---------------------------------------------------------------------------------------------------------------- */
/* EXL3 trellis                                                                                                     */
/* ---------------------------------------------------------------------------------------------------------------- */

/* formats: engine/kernels/nv2/ft_n135.h:78-81 (TF_KA / TF_MASK / TF_TB), K 4 added by the same rule (tile = 32 K B) */
static const int KA[BMXO_TF_N] = { 2, 2, 3, 4 };
static const uint32_t KMASK[BMXO_TF_N] = { 0u, 0xAAAAu, 0u, 0u };
static const int TBYTES[BMXO_TF_N] = { 64, 80, 96, 128 };

/* codebook constants: engine/kernels/nv2/ft_core.h:29, 38-39 (MUL1, KINV = h2f(0x1eee), KBIAS = h2f(0xc931)) */
#define MUL1 0x83DCD12Du
#define R_SCALE 0.088388347648f   /* 1/sqrt(128) in fp32: engine/kernels/x16/x16_dev.cu:20, ft_core.h:30 */

int bmxo_tile_bytes(int fmt) { return (fmt >= 0 && fmt < BMXO_TF_N) ? TBYTES[fmt] : -1; }

static int popc16(uint32_t v) { int c = 0; for (int j = 0; j < 16; ++j) c += (v >> j) & 1u; return c; }

/* S(i): ft_n135.h:84-89 (tf_s) and tests/gpu_dsv41_vbmi_tables.py:17-21 */
int bmxo_ring_end(int f, int i)
{
    int s = (i >> 4) * (16 * KA[f] + popc16(KMASK[f]));
    for (int j = 0; j <= (i & 15); ++j) s += KA[f] + (int)((KMASK[f] >> j) & 1u);
    return s;
}

static uint32_t le32(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }

/* state i = ring bits [S(i) - 16, S(i)) of the MSB-first little-endian-u32 ring: tests/gpu_dsv41_vbmi_tables.py:67-81
 * (ring_states), ft_core.h:66-74 (state_scalar, K 3) */
void bmxo_tile_states(const uint8_t* tile, int f, uint16_t* st)
{
    const int nbits = 8 * TBYTES[f], nw = TBYTES[f] / 4;
    for (int i = 0; i < 256; ++i)
    {
        int p = bmxo_ring_end(f, i) - 16;
        p = ((p % nbits) + nbits) % nbits;
        const uint32_t w0 = le32(tile + 4 * ((p >> 5) % nw)), w1 = le32(tile + 4 * (((p >> 5) + 1) % nw));
        const uint64_t cat = ((uint64_t)w0 << 32) | w1;
        st[i] = (uint16_t)(cat >> (48 - (p & 31)));
    }
}

/* stream index -> r * 16 + c: ft_core.h:49-62 (init_perm, exllamav3 make_tc_perm) */
void bmxo_perm(int* perm)
{
    for (int t = 0; t < 32; ++t)
    {
        const int r0 = (t % 4) * 2, c0 = t / 4;
        const int rows[4] = { r0, r0 + 1, r0 + 8, r0 + 9 };
        for (int j = 0; j < 8; ++j) perm[t * 8 + j] = rows[j & 3] * 16 + c0 + (j >= 4 ? 8 : 0);
    }
}

/* ft_core.h:76-80 */
uint32_t bmxo_bytesum(uint16_t st)
{
    const uint32_t x = (uint32_t)st * MUL1;
    return (x & 0xffu) + ((x >> 8) & 0xffu) + ((x >> 16) & 0xffu) + (x >> 24);
}

/* ft_core.h:82-84 (w_gpu): RN16(fma(1024 + s, KINV, KBIAS)); the fma is exact (multiples of 2^-18 below 16) */
uint16_t bmxo_decode_state(uint16_t st)
{
    const double kinv = (double)bmxo_f16_to_f32(0x1eee), kbias = (double)bmxo_f16_to_f32(0xc931);
    const double v = (double)(1024u + bmxo_bytesum(st)) * kinv + kbias;
    return bmxo_f32_to_f16((float)v);
}

/* ft_core.h:1007-1022 (dense_weights): tile (tk, tn) at (tk * n/16 + tn) * tile bytes */
void bmxo_dequant(const uint8_t* trellis, int fmt, int k, int n, uint16_t* out)
{
    int perm[256];
    uint16_t st[256];
    bmxo_perm(perm);
    const int tn = n / 16, tb = TBYTES[fmt];
    for (int tk = 0; tk < k / 16; ++tk)
        for (int t = 0; t < tn; ++t)
        {
            bmxo_tile_states(trellis + ((size_t)tk * tn + t) * tb, fmt, st);
            for (int i = 0; i < 256; ++i)
            {
                const int rc = perm[i];
                out[(size_t)(tk * 16 + rc / 16) * n + t * 16 + rc % 16] = bmxo_decode_state(st[i]);
            }
        }
}

/* ---------------------------------------------------------------------------------------------------------------- */
/* rotations                                                                                                        */
/* ---------------------------------------------------------------------------------------------------------------- */

/* Sylvester order, stages w = 1, 2, 4, ..., 64: ft_core.h:90-95; the GPU butterfly of x16_dev.cu:114-129 adds the same
 * pairs in the same stage order */
void bmxo_had128(float* v)
{
    for (int w = 1; w < 128; w *= 2)
        for (int b = 0; b < 128; b += 2 * w)
            for (int i = 0; i < w; ++i)
            {
                const float a = v[b + i], c = v[b + w + i];
                v[b + i] = a + c;
                v[b + w + i] = a - c;
            }
}

/* ft_core.h:97-103 (prep_block) */
void bmxo_prep(const uint16_t* x, const uint16_t* suh, int k, uint16_t* xt)
{
    float v[128];
    for (int b = 0; b < k / 128; ++b)
    {
        for (int i = 0; i < 128; ++i) v[i] = bmxo_f16_to_f32(x[b * 128 + i]) * bmxo_f16_to_f32(suh[b * 128 + i]);
        bmxo_had128(v);
        for (int i = 0; i < 128; ++i)
        {
            const float t = v[i] * R_SCALE;
            xt[b * 128 + i] = bmxo_f32_to_f16(t);
        }
    }
}

/* ---------------------------------------------------------------------------------------------------------------- */
/* expert                                                                                                           */
/* ---------------------------------------------------------------------------------------------------------------- */

/* act_gate: engine/kernels/x16/x16_dev.cu:68-112 (exact math here; the GPU evaluates the same formulas in fp32) */
static float act_gate(int act, int gated, float g, float u, float limit)
{
    double x;
    if (act == BMXO_ACT_SILU_OAI)
    {
        double gg = g, uu = u;
        if (limit != 0.0f)
        {
            gg = fmin(gg, limit);
            uu = fmin(fmax(uu, -limit), limit);
        }
        const double glu = gg / (1.0 + exp(-1.702 * gg));
        return (float)((uu + 1.0) * glu);
    }
    if (!gated) x = fmax(0.0, (double)u);
    else if (act == BMXO_ACT_SILU) x = (double)g / (1.0 + exp(-(double)g));
    else if (act == BMXO_ACT_GELU)
    {
        const double t = 0.797884560803 * ((double)g + 0.044715 * (double)g * g * g);
        x = 0.5 * g * (1.0 + tanh(t));
    }
    else { x = fmax(0.0, (double)g); x = x * x; }
    double uu = u;
    if (limit != 0.0f)
    {
        uu = fmin(fmax(uu, -limit), limit);
        x = fmin(x, limit);
    }
    return (float)(x * uu);
}

float bmxo_act(int act, int gated, float g, float u, float limit) { return act_gate(act, gated, g, u, limit); }

typedef struct { float* w[3]; } dense3;   /* dequantized gate [H][I], up [H][I], down [I][H] as fp32 */

static void dense_expert(const bmxo_expert* e, int H, int I, dense3* d)
{
    const int kk[3] = { H, H, I }, nn[3] = { I, I, H };
    for (int m = 0; m < 3; ++m)
    {
        const size_t cnt = (size_t)kk[m] * nn[m];
        uint16_t* tmp = (uint16_t*)malloc(cnt * 2);
        d->w[m] = (float*)malloc(cnt * 4);
        bmxo_dequant(e->tr[m], e->fmt[m], kk[m], nn[m], tmp);
        for (size_t i = 0; i < cnt; ++i) d->w[m][i] = bmxo_f16_to_f32(tmp[i]);
        free(tmp);
    }
}

static void dense_free(dense3* d) { for (int m = 0; m < 3; ++m) free(d->w[m]); }

/* y[n] = sum_k x[k] W[k][n], exact-enough fp64 accumulation (ft_core.h:1024-1032 ref_linear) */
static void gemv64(const uint16_t* x, const float* W, int k, int n, double* y)
{
    for (int j = 0; j < n; ++j) y[j] = 0.0;
    for (int i = 0; i < k; ++i)
    {
        const double xv = bmxo_f16_to_f32(x[i]);
        if (xv == 0.0) continue;
        const float* wr = W + (size_t)i * n;
        for (int j = 0; j < n; ++j) y[j] += xv * wr[j];
    }
}

/* One token through one expert at exllamav3's rounding points (docs/x16.md:38-54; epilogue x16_dev.cu:245-283;
 * reduction-side output rotation x16_dev.cu:363-366):
 *   xt = prep(x, suh)                         fp16
 *   gate / up = RN16(RN32(xt . W))            fp16 (stored GEMV results)
 *   g = RN32(RN32(H128(gate) * R) * svh)      fp32, same for u
 *   a = act(g, u) * suh_d ; act = RN16(H128(a) * R)
 *   d = RN32(act . Wd) ; y = RN32(RN32(H128(d) * R) * svh_d)                                                        */
static void expert_dense_forward(const bmxo_expert* e, const dense3* d, int H, int I, int act, int gated, float limit,
                                 const uint16_t* x, float* y, uint16_t* gate_o, uint16_t* up_o, uint16_t* act_o)
{
    uint16_t* xg = (uint16_t*)malloc((size_t)H * 2);
    uint16_t* xu = (uint16_t*)malloc((size_t)H * 2);
    uint16_t* g16 = (uint16_t*)malloc((size_t)I * 2);
    uint16_t* u16 = (uint16_t*)malloc((size_t)I * 2);
    uint16_t* a16 = (uint16_t*)malloc((size_t)I * 2);
    double* acc = (double*)malloc((size_t)(H > I ? H : I) * 8);
    bmxo_prep(x, e->suh[0], H, xg);
    bmxo_prep(x, e->suh[1], H, xu);
    gemv64(xg, d->w[0], H, I, acc);
    for (int j = 0; j < I; ++j) g16[j] = bmxo_f32_to_f16((float)acc[j]);
    gemv64(xu, d->w[1], H, I, acc);
    for (int j = 0; j < I; ++j) u16[j] = bmxo_f32_to_f16((float)acc[j]);
    for (int b = 0; b < I / 128; ++b)
    {
        float g[128], u[128], a[128];
        for (int i = 0; i < 128; ++i) { g[i] = bmxo_f16_to_f32(g16[b * 128 + i]); u[i] = bmxo_f16_to_f32(u16[b * 128 + i]); }
        bmxo_had128(g);
        bmxo_had128(u);
        for (int i = 0; i < 128; ++i)
        {
            float t = g[i] * R_SCALE;
            g[i] = t * bmxo_f16_to_f32(e->svh[0][b * 128 + i]);
            t = u[i] * R_SCALE;
            u[i] = t * bmxo_f16_to_f32(e->svh[1][b * 128 + i]);
            a[i] = act_gate(act, gated, g[i], u[i], limit);
            a[i] = a[i] * bmxo_f16_to_f32(e->suh[2][b * 128 + i]);
        }
        bmxo_had128(a);
        for (int i = 0; i < 128; ++i)
        {
            const float t = a[i] * R_SCALE;
            a16[b * 128 + i] = bmxo_f32_to_f16(t);
        }
    }
    gemv64(a16, d->w[2], I, H, acc);
    for (int b = 0; b < H / 128; ++b)
    {
        float v[128];
        for (int i = 0; i < 128; ++i) v[i] = (float)acc[b * 128 + i];
        bmxo_had128(v);
        for (int i = 0; i < 128; ++i)
        {
            const float t = v[i] * R_SCALE;
            y[b * 128 + i] = t * bmxo_f16_to_f32(e->svh[2][b * 128 + i]);
        }
    }
    if (gate_o) memcpy(gate_o, g16, (size_t)I * 2);
    if (up_o) memcpy(up_o, u16, (size_t)I * 2);
    if (act_o) memcpy(act_o, a16, (size_t)I * 2);
    free(xg); free(xu); free(g16); free(u16); free(a16); free(acc);
}

void bmxo_expert_forward(const bmxo_expert* e, int H, int I, int act, int gated, float limit, const uint16_t* x,
                         float* y, uint16_t* gate, uint16_t* up, uint16_t* act_out)
{
    dense3 d;
    dense_expert(e, H, I, &d);
    expert_dense_forward(e, &d, H, I, act, gated, limit, x, y, gate, up, act_out);
    dense_free(&d);
}

/* Layer: each routed expert decoded once, run on every selected token that picks it; then per token the weighted sum
 * over slots k = 0 .. topk-1 in order (picks with weight 0 or outside [first, first + E) skipped), then + the shared
 * expert (engine/kernels/x16/x16_dev.cu:354-384; engine/kernels/nv2/ft_n135.h:869-896 sums in job order instead). */
/* The shared expert's gate sigmoid(x . g) (x16_red_k's sh_gate_w, engine/kernels/x16/x16_dev.cu:315-334) in the GPU
 * combine's order: sixteen partial sums, partial j over h = 128 b + 8 j + i (b ascending, then i), one fmaf each; the
 * sixteen added by a butterfly (pairs j, j ^ s for s = 8, 4, 2, 1); then the fixed-sequence sigmoid. */
float bmxo_shared_gate(const uint16_t* x, const uint16_t* g, int H)
{
    float acc[16], nxt[16];
    for (int j = 0; j < 16; ++j)
    {
        acc[j] = 0.0f;
        for (int b = 0; b < H / 128; ++b)
            for (int i = 0; i < 8; ++i)
            {
                const int h = 128 * b + 8 * j + i;
                acc[j] = fmaf(bmxo_f16_to_f32(x[h]), bmxo_f16_to_f32(g[h]), acc[j]);
            }
    }
    for (int s = 8; s >= 1; s >>= 1)
    {
        for (int j = 0; j < 16; ++j) nxt[j] = acc[j] + acc[j ^ s];
        memcpy(acc, nxt, sizeof(acc));
    }
    return bmxo_sigmoid(acc[0]);
}

void bmxo_moe_forward(const bmxo_expert* experts, int E, int64_t first, const bmxo_expert* shared,
                      const uint16_t* sh_gate, int H, int I, int act, int gated, float limit, const uint16_t* x, int T,
                      int topk, const int64_t* sel, const uint16_t* w, const int* rows, int nrows, float* out)
{
    const int nr = rows ? nrows : T;
    float* ys = (float*)calloc((size_t)nr * topk * H, 4);
    float* ysh = shared ? (float*)calloc((size_t)nr * H, 4) : NULL;
    unsigned char* used = (unsigned char*)calloc((size_t)E, 1);
    for (int ri = 0; ri < nr; ++ri)
    {
        const int t = rows ? rows[ri] : ri;
        for (int k = 0; k < topk; ++k)
        {
            const int64_t e = sel[(size_t)t * topk + k] - first;
            if (e >= 0 && e < E && bmxo_f16_to_f32(w[(size_t)t * topk + k]) != 0.0f) used[e] = 1;
        }
    }
    for (int e = 0; e < E; ++e)
    {
        if (!used[e]) continue;
        dense3 d;
        dense_expert(&experts[e], H, I, &d);
        for (int ri = 0; ri < nr; ++ri)
        {
            const int t = rows ? rows[ri] : ri;
            for (int k = 0; k < topk; ++k)
                if (sel[(size_t)t * topk + k] - first == e && bmxo_f16_to_f32(w[(size_t)t * topk + k]) != 0.0f)
                    expert_dense_forward(&experts[e], &d, H, I, act, gated, limit, x + (size_t)t * H,
                                         ys + ((size_t)ri * topk + k) * H, NULL, NULL, NULL);
        }
        dense_free(&d);
    }
    if (shared)
    {
        dense3 d;
        dense_expert(shared, H, I, &d);
        for (int ri = 0; ri < nr; ++ri)
        {
            const int t = rows ? rows[ri] : ri;
            expert_dense_forward(shared, &d, H, I, act, gated, limit, x + (size_t)t * H, ysh + (size_t)ri * H, NULL,
                                 NULL, NULL);
        }
        dense_free(&d);
    }
    for (int ri = 0; ri < nr; ++ri)
    {
        const int t = rows ? rows[ri] : ri;
        for (int h = 0; h < H; ++h)
        {
            float o = 0.0f;
            for (int k = 0; k < topk; ++k)
            {
                const int64_t e = sel[(size_t)t * topk + k] - first;
                const float wk = bmxo_f16_to_f32(w[(size_t)t * topk + k]);
                if (e < 0 || e >= E || wk == 0.0f) continue;
                const float p = wk * ys[((size_t)ri * topk + k) * H + h];
                o = o + p;
            }
            if (shared && sh_gate)
            {
                const float p = bmxo_shared_gate(x + (size_t)t * H, sh_gate, H) * ysh[(size_t)ri * H + h];
                o = o + p;
            }
            else if (shared) o = o + ysh[(size_t)ri * H + h];
            out[(size_t)ri * H + h] = o;
        }
    }
    free(ys); free(ysh); free(used);
}

/* ---------------------------------------------------------------------------------------------------------------- */
/* router                                                                                                           */
/* ---------------------------------------------------------------------------------------------------------------- */

/* exp(x) in fp32 by a fixed operation sequence: Cody-Waite range reduction (W. J. Cody and W. Waite, Software Manual
 * for the Elementary Functions, 1980) with n = rint(x / ln 2) and ln 2 split in two (the high / low pair SLEEF's expf
 * uses, 0.693145751953125 + 1.428606765330187e-06), the degree-7 Taylor polynomial of exp in Horner form on
 * |r| <= ln2/2, exact scaling by powers of two. The HIP router evaluates the same sequence, so both produce the same
 * bits. Max relative error ~2 ulp, checked against libm in the tests. */
float bmxo_exp(float x)
{
    if (x != x) return x;
    if (x > 88.72f) return INFINITY;
    if (x < -104.0f) return 0.0f;
    const float n = rintf(x * 1.44269504f);
    float r = fmaf(n, -0.693145751953125f, x);
    r = fmaf(n, -1.428606765330187e-06f, r);
    float p = 1.98412698e-4f;
    p = fmaf(p, r, 1.38888889e-3f);
    p = fmaf(p, r, 8.33333333e-3f);
    p = fmaf(p, r, 4.16666667e-2f);
    p = fmaf(p, r, 1.66666667e-1f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int ni = (int)n;
    /* 2^ni as two normal factors so subnormal results round once, at the last multiply */
    const int n1 = ni / 2, n2 = ni - n1;
    uint32_t b1 = (uint32_t)(n1 + 127) << 23, b2 = (uint32_t)(n2 + 127) << 23;
    float s1, s2;
    memcpy(&s1, &b1, 4);
    memcpy(&s2, &b2, 4);
    const float q = p * s1;
    return q * s2;
}

float bmxo_sigmoid(float x)
{
    const float e = bmxo_exp(-x);
    const float d = 1.0f + e;
    return 1.0f / d;
}

/* sqrt(softplus(x)) = sqrt(max(x, 0) + log1p(exp(-|x|))) by a fixed sequence: log1p(e) = 2 atanh(e / (2 + e)) as the
 * odd series 2 (s + s^3/3 + ... + s^17/17) in Horner form over s^2 (Abramowitz and Stegun 4.1.27; s <= 1/3); correctly
 * rounded division and square root. The HIP router evaluates the same sequence. */
float bmxo_sqrtsp(float x)
{
    if (x != x) return x;
    const float e = bmxo_exp(-fabsf(x));
    const float s = e / (2.0f + e);
    const float s2 = s * s;
    float p = 1.0f / 17.0f;
    p = fmaf(p, s2, 1.0f / 15.0f);
    p = fmaf(p, s2, 1.0f / 13.0f);
    p = fmaf(p, s2, 1.0f / 11.0f);
    p = fmaf(p, s2, 1.0f / 9.0f);
    p = fmaf(p, s2, 1.0f / 7.0f);
    p = fmaf(p, s2, 1.0f / 5.0f);
    p = fmaf(p, s2, 1.0f / 3.0f);
    p = fmaf(p, s2, 1.0f);
    const float l = (2.0f * s) * p;
    return sqrtf(fmaxf(x, 0.0f) + l);
}

/* a ranks before b: larger value, then lower index (ties -> lower index: engine/kernels/nv2/nv2_host.cpp:917) */
static int better(float va, int ia, float vb, int ib) { return va > vb || (va == vb && ia < ib); }

static float canon(float v) { if (v != v) return -INFINITY; return v + 0.0f; }   /* NaN -> -inf, -0 -> +0 */

/* Score / select / weight (exllamav3 routing_fn semantics as the reference calls it: engine/nv2.py:470-487 sigmoid +
 * selection bias "esb"; group-limited top-k of the DeepSeek-V3 router; softmax top-k of Mixtral-style routers).
 *   softmax: choice = logit (softmax is monotone in the logit); weight = exp(l - max) / sum
 *   sigmoid: score = sigmoid(l); choice = score + bias; weight = score
 *   groups : group score = top-2 choice sum in each of n_group equal groups; keep topk_group groups; pick within
 *   weights renormalised over the picks when renorm (sum in slot order), times scale, RN16 */
void bmxo_router(const uint16_t* logits, const float* bias, int T, int E, int topk, int n_group, int topk_group,
                 int score_fn, int renorm, float scale, int64_t first, int64_t* sel, uint16_t* w)
{
    float* sc = (float*)malloc((size_t)E * 4);
    float* ch = (float*)malloc((size_t)E * 4);
    unsigned char* ok = (unsigned char*)malloc((size_t)E);
    unsigned char* taken = (unsigned char*)malloc((size_t)E);
    const int G = n_group > 0 ? n_group : 1, gs = E / G;
    float* gsc = (float*)malloc((size_t)G * 4);
    unsigned char* gsel = (unsigned char*)malloc((size_t)G);
    for (int t = 0; t < T; ++t)
    {
        const uint16_t* lg = logits + (size_t)t * E;
        float mx = -INFINITY;
        for (int e = 0; e < E; ++e) { const float l = canon(bmxo_f16_to_f32(lg[e])); if (l > mx) mx = l; }
        for (int e = 0; e < E; ++e)
        {
            const float l = canon(bmxo_f16_to_f32(lg[e]));
            if (score_fn == BMXO_SCORE_SOFTMAX) { sc[e] = bmxo_exp(l - mx); ch[e] = l; }
            else
            {
                sc[e] = score_fn == BMXO_SCORE_SQRTSP ? bmxo_sqrtsp(l) : bmxo_sigmoid(l);
                ch[e] = canon(bias ? sc[e] + bias[e] : sc[e]);
            }
            ok[e] = 1;
            taken[e] = 0;
        }
        if (G > 1)
        {
            for (int g = 0; g < G; ++g)
            {
                float t1 = -INFINITY, t2 = -INFINITY;
                int i1 = -1;
                for (int e = g * gs; e < (g + 1) * gs; ++e) if (i1 < 0 || better(ch[e], e, t1, i1)) { t1 = ch[e]; i1 = e; }
                int i2 = -1;
                for (int e = g * gs; e < (g + 1) * gs; ++e)
                    if (e != i1 && (i2 < 0 || better(ch[e], e, t2, i2))) { t2 = ch[e]; i2 = e; }
                gsc[g] = canon(i2 >= 0 ? t1 + t2 : t1);
                gsel[g] = 0;
            }
            for (int r = 0; r < topk_group && r < G; ++r)
            {
                int bg = -1;
                for (int g = 0; g < G; ++g) if (!gsel[g] && (bg < 0 || better(gsc[g], g, gsc[bg], bg))) bg = g;
                gsel[bg] = 1;
            }
            for (int e = 0; e < E; ++e) ok[e] = gsel[e / gs];
        }
        float vsum = 0.0f;
        float vals[64];
        int idx[64];
        for (int k = 0; k < topk; ++k)
        {
            int be = -1;
            for (int e = 0; e < E; ++e)
                if (ok[e] && !taken[e] && (be < 0 || better(ch[e], e, ch[be], be))) be = e;
            taken[be] = 1;
            idx[k] = be;
            vals[k] = sc[be];
            vsum = vsum + sc[be];
        }
        float den = 1.0f;
        if (score_fn == BMXO_SCORE_SOFTMAX && !renorm)
        {
            den = 0.0f;
            for (int e = 0; e < E; ++e) den = den + sc[e];
        }
        else if (renorm) den = vsum;
        for (int k = 0; k < topk; ++k)
        {
            const float q = (score_fn != BMXO_SCORE_SOFTMAX && !renorm) ? vals[k] : vals[k] / den;
            const float v = q * scale;
            sel[(size_t)t * topk + k] = (int64_t)idx[k] + first;
            w[(size_t)t * topk + k] = bmxo_f32_to_f16(v);
        }
    }
    free(sc); free(ch); free(ok); free(taken); free(gsc); free(gsel);
}

/* ---------------------------------------------------------------------------------------------------------------- */
/* dispatch                                                                                                         */
/* ---------------------------------------------------------------------------------------------------------------- */

/* Histogram + exclusive prefix + stable scatter (the counting and ascending compaction of engine/kernels/nv2/
 * nv2_dev.cu:34-46 (nv_pub_k), rows grouped per expert as ft_n135.h:912-923 groups jobs, stable by token then slot) */
int bmxo_dispatch(const int64_t* sel, int T, int topk, int E, int64_t first, int shared, int32_t* counts,
                  int32_t* offsets, int32_t* row_token, int32_t* row_slot, int32_t* inv, int32_t* uexp)
{
    const int NE = E + (shared ? 1 : 0);
    int32_t* fill = (int32_t*)calloc((size_t)NE, 4);
    for (int e = 0; e < NE; ++e) counts[e] = 0;
    for (int p = 0; p < T * topk; ++p)
    {
        const int64_t e = sel[p] - first;
        if (e >= 0 && e < E) ++counts[e];
    }
    if (shared) counts[E] = T;
    offsets[0] = 0;
    for (int e = 0; e < NE; ++e) offsets[e + 1] = offsets[e] + counts[e];
    for (int p = 0; p < T * topk; ++p)
    {
        const int64_t e = sel[p] - first;
        if (e >= 0 && e < E)
        {
            const int r = offsets[e] + fill[e]++;
            row_token[r] = p / topk;
            row_slot[r] = p % topk;
            inv[p] = r;
        }
        else inv[p] = -1;
    }
    if (shared)
        for (int t = 0; t < T; ++t) { row_token[offsets[E] + t] = t; row_slot[offsets[E] + t] = -1; }
    int nu = 0;
    for (int e = 0; e < NE; ++e) if (counts[e]) uexp[nu++] = e;
    free(fill);
    return nu;
}

/* ---------------------------------------------------------------------------------------------------------------- */
/* expert-slot table                                                                                                */
/* ---------------------------------------------------------------------------------------------------------------- */

/* CLOCK step: engine/ec.py:16-76 (ec_step_k) with the misses taken in ascending expert order (the reference collects
 * them with a shared-memory atomicAdd, so its order is unspecified): hit -> refb = 1, pin = epoch; per miss the hand
 * skips slots pinned this epoch or disabled (pin < 0), clears set reference bits, and takes the first clear slot within
 * 2 S steps; the victim's owner goes back home (slotof = -1). */
/* the CLOCK admission of the misses miss[nmiss] of layer li (ec_step_k, engine/ec.py:40-76, with misses taken in the
 * order given): each takes the first slot from the hand that is enabled, not pinned in `epoch` and whose reference bit is
 * clear, clearing the bits it passes; a miss that finds none in 2 S probes ends the admissions. A prefetch (pf) sweeps
 * gently: it passes referenced slots without clearing their bits (so at most S probes) and admits with the bit clear. */
static int clock_admit(bmxo_slots* t, int li, const int* miss, int nmiss, int maxj, int epoch, int pf, int32_t* jobs,
                       int32_t* evicted, int32_t* fresh, int64_t* stats)
{
    const int E = t->E, S = t->S;
    int nj = 0, hand = t->hand;
    for (int k = 0; k < nmiss && nj < maxj; ++k)
    {
        const int e = miss[k];
        int found = -1;
        for (int step = 0; step < (pf ? S : 2 * S); ++step)
        {
            const int s = hand;
            hand = (hand + 1 == S) ? 0 : hand + 1;
            if (t->pin[s] == epoch || t->pin[s] < 0) continue;
            if (t->refb[s])
            {
                if (!pf) t->refb[s] = 0;
                continue;
            }
            found = s;
            break;
        }
        if (found < 0) { if (!pf) stats[3] += 1; break; }
        const int s = found, old = t->owner[s];
        if (old >= 0)
        {
            t->slotof[old] = -1;
            stats[4] += 1;
            if (t->pfl[s]) stats[7] += 1;
        }
        evicted[nj] = old;
        t->owner[s] = li * E + e;
        t->slotof[(size_t)li * E + e] = s;
        t->refb[s] = !pf;
        t->pin[s] = epoch;
        t->pfl[s] = pf;
        if (fresh) fresh[e] = 1;
        jobs[2 * nj] = e;
        jobs[2 * nj + 1] = s;
        ++nj;
        stats[pf ? 5 : 2] += 1;
    }
    t->hand = hand;
    return nj;
}

int bmxo_slot_step(bmxo_slots* t, int li, const int64_t* sel, int n, int64_t first, int admit, int maxj, int32_t* jobs,
                   int32_t* evicted, int32_t* fresh, int64_t* stats)
{
    return bmxo_slot_step_lanes(t, li, sel, n, first, admit, maxj, NULL, jobs, evicted, fresh, stats);
}

/* A planned step (include/bmx.h bmx_slot_step_planned): elane[E] (or NULL: every miss admitted) is each expert's lane;
 * a miss joins the admissions only in lane 1 (admit); every miss counts in stats[1]. */
int bmxo_slot_step_lanes(bmxo_slots* t, int li, const int64_t* sel, int n, int64_t first, int admit, int maxj,
                         const int32_t* elane, int32_t* jobs, int32_t* evicted, int32_t* fresh, int64_t* stats)
{
    const int E = t->E, S = t->S;
    unsigned char* mark = (unsigned char*)calloc((size_t)E, 1);
    int* miss = (int*)malloc((size_t)E * sizeof(int));
    const int epoch = ++t->epoch;
    if (fresh) memset(fresh, 0, (size_t)E * sizeof(int32_t));
    for (int i = 0; i < n; ++i)
    {
        const int64_t e = sel[i] - first;
        if (e >= 0 && e < E) mark[e] = 1;
    }
    int nhit = 0, nmiss = 0, nmiss_all = 0, nj = 0;
    int32_t* slotof = t->slotof + (size_t)li * E;
    for (int e = 0; e < E; ++e)
    {
        if (!mark[e]) continue;
        const int s = slotof[e];
        if (s >= 0)
        {
            t->refb[s] = 1;
            t->pin[s] = epoch;
            ++nhit;
            if (t->pfl[s])             /* first use of a prefetched expert: its copy may still be in flight */
            {
                t->pfl[s] = 0;
                stats[6] += 1;
                if (fresh) fresh[e] = 1;
            }
        }
        else
        {
            ++nmiss_all;
            if (!elane || elane[e] == 1) miss[nmiss++] = e;
        }
    }
    stats[0] += nhit;
    stats[1] += nmiss_all;
    if (admit && S > 0) nj = clock_admit(t, li, miss, nmiss, maxj, epoch, 0, jobs, evicted, fresh, stats);
    free(mark);
    free(miss);
    return nj;
}

int bmxo_slot_prefetch(bmxo_slots* t, int li, const int64_t* sel, int n, int64_t first, int limit, int maxj,
                       int32_t* jobs, int32_t* evicted, int64_t* stats)
{
    const int E = t->E;
    unsigned char* seen = (unsigned char*)calloc((size_t)E, 1);
    int* cand = (int*)malloc((size_t)E * sizeof(int));
    int nc = 0;
    for (int i = 0; i < n && nc < limit; ++i)
    {
        const int64_t e = sel[i] - first;
        if (e < 0 || e >= E || seen[e]) continue;
        seen[e] = 1;
        if (t->slotof[(size_t)li * E + e] < 0) cand[nc++] = (int)e;
    }
    int nj = 0;
    if (t->S > 0) nj = clock_admit(t, li, cand, nc, maxj, t->epoch, 1, jobs, evicted, NULL, stats);
    free(seen);
    free(cand);
    return nj;
}
