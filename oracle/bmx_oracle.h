/*
 * CPU oracle for the routed-expert MoE layer: TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only as a reference
 * to check against. The product path (libbmx.so) never links, calls or falls back to it.
 *
 * Plain C99 restatement of the arithmetic of the reference's hot path (Big-MoE-Small-Box + exllamav3 1.6.6 semantics):
 * EXL3 trellis state extraction (integer and fractional K), the tensor-core tile permutation, the mul1 codebook, the
 * 128-point input / output rotations with their fp16 rounding points, the fused gate/up -> activation -> down expert, the
 * weighted combine, the router closed forms, the stable counting-sort dispatch and the CLOCK expert-slot step.
 * Every function names the reference file:line it follows (paths relative to src/bigmoe/ of the reference).
 */
#ifndef BMX_ORACLE_H
#define BMX_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* trellis formats: same numbering as the reference's TF_K2 / TF_K25 / TF_K3 (engine/kernels/nv2/ft_n135.h:78-81),
 * extended with K = 4 (ring of 4 bits per weight, 128-byte tiles) */
enum { BMXO_TF_K2 = 0, BMXO_TF_K25 = 1, BMXO_TF_K3 = 2, BMXO_TF_K4 = 3, BMXO_TF_N = 4 };

/* fp16 <-> fp32, round to nearest even, subnormals kept */
uint16_t bmxo_f32_to_f16(float f);
float bmxo_f16_to_f32(uint16_t h);

int bmxo_tile_bytes(int fmt);
int bmxo_ring_end(int fmt, int i);                        /* S(i): prefix sum of bits per weight, i in [0, 256) */
void bmxo_tile_states(const uint8_t* tile, int fmt, uint16_t* st);  /* st[i] = 16-bit state of stream index i */
void bmxo_perm(int* perm);                                /* perm[i] = r * 16 + c of stream index i */
uint32_t bmxo_bytesum(uint16_t st);                       /* sum of the bytes of st * MUL1 mod 2^32 */
uint16_t bmxo_decode_state(uint16_t st);                  /* fp16 bits of the codebook weight */
/* trellis [k/16][n/16][tile] -> fp16 [k][n] (row = input channel, column = output channel) */
void bmxo_dequant(const uint8_t* trellis, int fmt, int k, int n, uint16_t* out);

/* rotations */
void bmxo_had128(float* v);
/* xt = RN16(H128(x * suh) * 1/sqrt(128)) per 128-block; x, suh, xt fp16 bits, length k */
void bmxo_prep(const uint16_t* x, const uint16_t* suh, int k, uint16_t* xt);

/* activations (exllamav3 MOE_COOP_ACT_* numbering) */
enum { BMXO_ACT_SILU = 0, BMXO_ACT_GELU = 1, BMXO_ACT_RELU2 = 2, BMXO_ACT_SILU_OAI = 3 };

/* a = act_gate(g, u): the epilogue's activation of one gate / up pair (limit 0 = no clamp) */
float bmxo_act(int act, int gated, float g, float u, float limit);

typedef struct {
    const uint8_t* tr[3];     /* gate, up, down trellis */
    const uint16_t* suh[3];   /* fp16 input scales: [H], [H], [I] */
    const uint16_t* svh[3];   /* fp16 output scales: [I], [I], [H] */
    int fmt[3];
} bmxo_expert;

/* One expert on one token: x fp16 [H] -> y fp32 [H]. Optional intermediate outputs (NULL to skip):
 * gate / up fp16 [I] (stored GEMV results before the epilogue), act fp16 [I] (rotated down input). */
void bmxo_expert_forward(const bmxo_expert* e, int H, int I, int act, int gated, float limit, const uint16_t* x,
                         float* y, uint16_t* gate, uint16_t* up, uint16_t* act_out);

/* Full layer on a subset of tokens: out[ti][H] for tokens rows[ti] (rows == NULL: all T tokens).
 * sel int64 [T, topk] global ids (first .. first + E - 1; anything else is a dropped pick), w fp16 bits [T, topk].
 * shared: optional shared expert, added after the routed slots with weight bmxo_shared_gate(x, sh_gate) when sh_gate
 * (fp16 bits [H]) is given, else 1. */
void bmxo_moe_forward(const bmxo_expert* experts, int E, int64_t first, const bmxo_expert* shared,
                      const uint16_t* sh_gate, int H, int I, int act, int gated, float limit, const uint16_t* x, int T,
                      int topk, const int64_t* sel, const uint16_t* w, const int* rows, int nrows, float* out);
/* sigmoid(x . g) in the GPU combine's fixed order (x, g fp16 bits [H], H a multiple of 128) */
float bmxo_shared_gate(const uint16_t* x, const uint16_t* g, int H);

/* router */
enum { BMXO_SCORE_SOFTMAX = 0, BMXO_SCORE_SIGMOID = 1, BMXO_SCORE_SQRTSP = 2 };
float bmxo_exp(float x);        /* the fixed-sequence fp32 exp the HIP router also evaluates */
float bmxo_sigmoid(float x);
float bmxo_sqrtsp(float x);     /* the fixed-sequence sqrt(softplus(x)) the HIP router also evaluates */
/* logits fp16 bits [T, E]; bias fp32 [E] or NULL; n_group / topk_group (1 / 1 = no group limit);
 * out: sel int64 [T, topk] (global ids = local + first), w fp16 bits [T, topk] */
void bmxo_router(const uint16_t* logits, const float* bias, int T, int E, int topk, int n_group, int topk_group,
                 int score_fn, int renorm, float scale, int64_t first, int64_t* sel, uint16_t* w);

/* dispatch: stable counting sort of picks by (expert, token, slot). Picks outside [first, first + E) are dropped
 * (inv = -1). shared != 0 appends a segment for expert index E holding every token once (row_slot = -1).
 * counts [E + 1], offsets [E + 2], row_token / row_slot [T * topk + T], inv [T * topk], uexp [E + 1]; returns nuniq. */
int bmxo_dispatch(const int64_t* sel, int T, int topk, int E, int64_t first, int shared, int32_t* counts,
                  int32_t* offsets, int32_t* row_token, int32_t* row_slot, int32_t* inv, int32_t* uexp);

/* expert-slot table (CLOCK): one step of layer li over the picks sel[n] */
typedef struct {
    int L, E, S;
    int32_t* slotof;   /* [L * E], -1 = not resident */
    int32_t* owner;    /* [S], li * E + e or -1 */
    int32_t* refb;     /* [S] */
    int32_t* pin;      /* [S], epoch of the last use; < 0 = slot disabled */
    int32_t* pfl;      /* [S], 1 = admitted by a prefetch and not used by a step since */
    int32_t hand, epoch;
} bmxo_slots;
/* returns the number of admission jobs written to jobs[2 * j] = e, jobs[2 * j + 1] = slot, evicted[j] = old owner or -1.
 * fresh [E] (or NULL) = 1 for the experts admitted by this step and for the hits on prefetched slots.
 * stats[0..7] += hits, misses, admitted, no_victim, evictions, (prefetch:) admitted, used, evicted unused */
int bmxo_slot_step(bmxo_slots* t, int li, const int64_t* sel, int n, int64_t first, int admit, int maxj, int32_t* jobs,
                   int32_t* evicted, int32_t* fresh, int64_t* stats);
int bmxo_slot_step_lanes(bmxo_slots* t, int li, const int64_t* sel, int n, int64_t first, int admit, int maxj,
                         const int32_t* elane, int32_t* jobs, int32_t* evicted, int32_t* fresh, int64_t* stats);
/* layer-ahead prefetch into layer li's slots: the first `limit` distinct in-range picks of sel[n] (rank order) that are
 * not resident are admitted in that order, at most maxj, within the current epoch (slots pinned by the last step stay
 * pinned; the epoch does not advance) by a gentle CLOCK sweep: the first enabled, unpinned slot from the hand whose
 * reference bit is clear, passing referenced slots without clearing their bits (at most S probes; a guess that finds
 * none ends the prefetch); admitted with the bit clear, so a wrong guess is the next victim. Resident guesses and every
 * reference bit are left alone. */
int bmxo_slot_prefetch(bmxo_slots* t, int li, const int64_t* sel, int n, int64_t first, int limit, int maxj,
                       int32_t* jobs, int32_t* evicted, int64_t* stats);

#ifdef __cplusplus
}
#endif
#endif
