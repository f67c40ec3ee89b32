// Device-side building blocks shared by the bmx kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/bmx.h"

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace bmx {

constexpr int WAVE = 64;
constexpr float R_SCALE = 0.088388347648f;   // 1 / sqrt(128) in fp32 (engine/kernels/x16/x16_dev.cu:20)

// ---- EXL3 trellis formats ------------------------------------------------------------------------------------------
// Ring layout (engine/kernels/nv2/ft_n135.h:74-89; tests/gpu_dsv41_vbmi_tables.py:67-81): weight i of a 256-weight tile
// adds d(i) = KA + bit (i & 15) of MASK bits to a ring of 256 K bits stored MSB-first in little-endian 32-bit words;
// its 16-bit state is ring bits [S(i) - 16, S(i)), S = prefix sum of d. Weight -> position: the tensor-core fragment
// order make_tc_perm (engine/kernels/nv2/ft_core.h:49-62).
template <int F> struct Fmt;
template <> struct Fmt<BMX_TF_K2>  { static constexpr int KA = 2, TB = 64;  static constexpr uint32_t MASK = 0x0000u; };
template <> struct Fmt<BMX_TF_K25> { static constexpr int KA = 2, TB = 80;  static constexpr uint32_t MASK = 0xAAAAu; };
template <> struct Fmt<BMX_TF_K3>  { static constexpr int KA = 3, TB = 96;  static constexpr uint32_t MASK = 0x0000u; };
template <> struct Fmt<BMX_TF_K4>  { static constexpr int KA = 4, TB = 128; static constexpr uint32_t MASK = 0x0000u; };

__host__ __device__ constexpr int popc16(uint32_t m)
{
    int c = 0;
    for (int j = 0; j < 16; ++j) c += (m >> j) & 1u;
    return c;
}

// S(i)
template <int F> __host__ __device__ constexpr int ring_end(int i)
{
    int s = (i >> 4) * (16 * Fmt<F>::KA + popc16(Fmt<F>::MASK));
    for (int j = 0; j <= (i & 15); ++j) s += Fmt<F>::KA + int((Fmt<F>::MASK >> j) & 1u);
    return s;
}

__host__ __device__ inline int tile_bytes_of(int fmt)
{
    switch (fmt)
    {
        case BMX_TF_K2: return 64;
        case BMX_TF_K25: return 80;
        case BMX_TF_K3: return 96;
        case BMX_TF_K4: return 128;
        default: return -1;
    }
}

// codebook constants: MUL1 (engine/kernels/nv2/ft_core.h:29); KINV = fp16 0x1eee, KBIAS = fp16 0xc931 (ft_core.h:38-39)
constexpr uint32_t MUL1 = 0x83DCD12Du;
constexpr uint32_t MUL1_LO = MUL1 & 0xffffu;           // 0xD12D
constexpr uint32_t MUL1_HI_SHL16 = MUL1 & 0xffff0000u; // 0x83DC << 16
constexpr uint32_t KINV_BITS = 0x1eeeu;
constexpr uint32_t KBIAS_BITS = 0xc931u;
constexpr uint32_t F16_1024 = 0x6400u;                 // fp16 bits of 1024.0: 1024 + s (s < 1024) is 0x6400 | s

// global-memory views of generic pointers (addresses read from the expert table are generic; loading through a
// global pointer gives global_load instead of flat_load, which would also count against the LDS wait counter)
typedef const __attribute__((address_space(1))) uint32_t* gptr_u32;
__device__ __forceinline__ uint32_t ldg_nt(const void* p, int i)
{
    return __builtin_nontemporal_load(reinterpret_cast<gptr_u32>(reinterpret_cast<uintptr_t>(p)) + i);
}
__device__ __forceinline__ uint32_t ldg(const void* p, int i)
{
    return reinterpret_cast<gptr_u32>(reinterpret_cast<uintptr_t>(p))[i];
}

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(f16, b); }
__device__ __forceinline__ uint16_t f2h(float v) { return __builtin_bit_cast(uint16_t, (f16)v); }
// RN16 of an fp32 value that is first materialised as fp32: the empty asm keeps the compiler from fusing the producing
// multiply or add with the conversion into one mixed-precision instruction (one rounding instead of the two the
// reference performs: fp32 result, then fp16)
__device__ __forceinline__ uint16_t f2h_r(float v)
{
    asm("" : "+v"(v));
    return f2h(v);
}

// Codebook weights of eight 16-bit states (only the low 16 bits of each state are read; the bits above may hold
// anything), packed in pairs: w[q] = (weight of st[2q + 1]) << 16 | weight of st[2q]. Per state:
//   x = st * MUL1 mod 2^32 = st * 0xD12D + ((st * 0x83DC mod 2^16) << 16)
//     v_pk_mul_lo_u16 (op_sel_hi [0, 1]: the high product of the low half lands in the high half, the low one is 0),
//     then v_mad_u32_u16 (reads the low halves);
//   1024 + bytesum(x) as fp16 bits: v_sad_u8 adds the bytes of x_a to 0x64006400, v_sad_hi_u8 adds those of x_b into
//     the high half (a sum < 1024 never carries out of its half);
//   w = RN16(fma(1024 + s, KINV, KBIAS)) for both halves with one v_pk_fma_f16.
// One asm block: no instruction in it reads a register that a packed instruction with a high-half op_sel wrote, and the
// one wait state the compiler adds after an inline-asm block is paid once per eight weights.
__device__ __forceinline__ void cb_oct(const uint32_t (&st)[8], uint32_t (&w)[4])
{
    uint32_t t[8];
    asm("v_pk_mul_lo_u16 %4, %12, %20 op_sel_hi:[0,1]\n\t"
        "v_pk_mul_lo_u16 %5, %13, %20 op_sel_hi:[0,1]\n\t"
        "v_pk_mul_lo_u16 %6, %14, %20 op_sel_hi:[0,1]\n\t"
        "v_pk_mul_lo_u16 %7, %15, %20 op_sel_hi:[0,1]\n\t"
        "v_pk_mul_lo_u16 %8, %16, %20 op_sel_hi:[0,1]\n\t"
        "v_pk_mul_lo_u16 %9, %17, %20 op_sel_hi:[0,1]\n\t"
        "v_pk_mul_lo_u16 %10, %18, %20 op_sel_hi:[0,1]\n\t"
        "v_pk_mul_lo_u16 %11, %19, %20 op_sel_hi:[0,1]\n\t"
        "v_mad_u32_u16 %4, %12, %21, %4\n\t"
        "v_mad_u32_u16 %5, %13, %21, %5\n\t"
        "v_mad_u32_u16 %6, %14, %21, %6\n\t"
        "v_mad_u32_u16 %7, %15, %21, %7\n\t"
        "v_mad_u32_u16 %8, %16, %21, %8\n\t"
        "v_mad_u32_u16 %9, %17, %21, %9\n\t"
        "v_mad_u32_u16 %10, %18, %21, %10\n\t"
        "v_mad_u32_u16 %11, %19, %21, %11\n\t"
        "v_sad_u8 %0, %4, 0, %22\n\t"
        "v_sad_u8 %1, %6, 0, %22\n\t"
        "v_sad_u8 %2, %8, 0, %22\n\t"
        "v_sad_u8 %3, %10, 0, %22\n\t"
        "v_sad_hi_u8 %0, %5, 0, %0\n\t"
        "v_sad_hi_u8 %1, %7, 0, %1\n\t"
        "v_sad_hi_u8 %2, %9, 0, %2\n\t"
        "v_sad_hi_u8 %3, %11, 0, %3\n\t"
        "v_pk_fma_f16 %0, %0, %23, %24\n\t"
        "v_pk_fma_f16 %1, %1, %23, %24\n\t"
        "v_pk_fma_f16 %2, %2, %23, %24\n\t"
        "v_pk_fma_f16 %3, %3, %23, %24"
        : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3]),
          "=&v"(t[4]), "=&v"(t[5]), "=&v"(t[6]), "=&v"(t[7])
        : "v"(st[0]), "v"(st[1]), "v"(st[2]), "v"(st[3]), "v"(st[4]), "v"(st[5]), "v"(st[6]), "v"(st[7]),
          "s"(MUL1_HI_SHL16), "s"(MUL1_LO), "s"((F16_1024 << 16) | F16_1024), "s"((KINV_BITS << 16) | KINV_BITS),
          "v"((KBIAS_BITS << 16) | KBIAS_BITS));
}

// cb_oct on states held in the high halves of st[0 .. 7] (op_sel on the two multiplies; the rest is cb_oct's).
__device__ __forceinline__ void cb_oct_hi(const uint32_t (&st)[8], uint32_t (&w)[4])
{
    uint32_t t[8];
    asm("v_pk_mul_lo_u16 %4, %12, %20 op_sel:[1,0] op_sel_hi:[1,1]\n\t"
        "v_pk_mul_lo_u16 %5, %13, %20 op_sel:[1,0] op_sel_hi:[1,1]\n\t"
        "v_pk_mul_lo_u16 %6, %14, %20 op_sel:[1,0] op_sel_hi:[1,1]\n\t"
        "v_pk_mul_lo_u16 %7, %15, %20 op_sel:[1,0] op_sel_hi:[1,1]\n\t"
        "v_pk_mul_lo_u16 %8, %16, %20 op_sel:[1,0] op_sel_hi:[1,1]\n\t"
        "v_pk_mul_lo_u16 %9, %17, %20 op_sel:[1,0] op_sel_hi:[1,1]\n\t"
        "v_pk_mul_lo_u16 %10, %18, %20 op_sel:[1,0] op_sel_hi:[1,1]\n\t"
        "v_pk_mul_lo_u16 %11, %19, %20 op_sel:[1,0] op_sel_hi:[1,1]\n\t"
        "v_mad_u32_u16 %4, %12, %21, %4 op_sel:[1,0,0,0]\n\t"
        "v_mad_u32_u16 %5, %13, %21, %5 op_sel:[1,0,0,0]\n\t"
        "v_mad_u32_u16 %6, %14, %21, %6 op_sel:[1,0,0,0]\n\t"
        "v_mad_u32_u16 %7, %15, %21, %7 op_sel:[1,0,0,0]\n\t"
        "v_mad_u32_u16 %8, %16, %21, %8 op_sel:[1,0,0,0]\n\t"
        "v_mad_u32_u16 %9, %17, %21, %9 op_sel:[1,0,0,0]\n\t"
        "v_mad_u32_u16 %10, %18, %21, %10 op_sel:[1,0,0,0]\n\t"
        "v_mad_u32_u16 %11, %19, %21, %11 op_sel:[1,0,0,0]\n\t"
        "v_sad_u8 %0, %4, 0, %22\n\t"
        "v_sad_u8 %1, %6, 0, %22\n\t"
        "v_sad_u8 %2, %8, 0, %22\n\t"
        "v_sad_u8 %3, %10, 0, %22\n\t"
        "v_sad_hi_u8 %0, %5, 0, %0\n\t"
        "v_sad_hi_u8 %1, %7, 0, %1\n\t"
        "v_sad_hi_u8 %2, %9, 0, %2\n\t"
        "v_sad_hi_u8 %3, %11, 0, %3\n\t"
        "v_pk_fma_f16 %0, %0, %23, %24\n\t"
        "v_pk_fma_f16 %1, %1, %23, %24\n\t"
        "v_pk_fma_f16 %2, %2, %23, %24\n\t"
        "v_pk_fma_f16 %3, %3, %23, %24"
        : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3]),
          "=&v"(t[4]), "=&v"(t[5]), "=&v"(t[6]), "=&v"(t[7])
        : "v"(st[0]), "v"(st[1]), "v"(st[2]), "v"(st[3]), "v"(st[4]), "v"(st[5]), "v"(st[6]), "v"(st[7]),
          "s"(MUL1_HI_SHL16), "s"(MUL1_LO), "s"((F16_1024 << 16) | F16_1024), "s"((KINV_BITS << 16) | KINV_BITS),
          "v"((KBIAS_BITS << 16) | KBIAS_BITS));
}

// cb_oct on eight states held in four registers: state q < 4 in the high half of v[q], state q + 4 in its low half.
__device__ __forceinline__ void cb_oct_k4(const uint32_t (&v)[4], uint32_t (&w)[4])
{
    uint32_t t[8];
    asm("v_pk_mul_lo_u16 %4, %12, %16 op_sel:[1,0] op_sel_hi:[1,1]\n\t"
        "v_pk_mul_lo_u16 %5, %13, %16 op_sel:[1,0] op_sel_hi:[1,1]\n\t"
        "v_pk_mul_lo_u16 %6, %14, %16 op_sel:[1,0] op_sel_hi:[1,1]\n\t"
        "v_pk_mul_lo_u16 %7, %15, %16 op_sel:[1,0] op_sel_hi:[1,1]\n\t"
        "v_pk_mul_lo_u16 %8, %12, %16 op_sel_hi:[0,1]\n\t"
        "v_pk_mul_lo_u16 %9, %13, %16 op_sel_hi:[0,1]\n\t"
        "v_pk_mul_lo_u16 %10, %14, %16 op_sel_hi:[0,1]\n\t"
        "v_pk_mul_lo_u16 %11, %15, %16 op_sel_hi:[0,1]\n\t"
        "v_mad_u32_u16 %4, %12, %17, %4 op_sel:[1,0,0,0]\n\t"
        "v_mad_u32_u16 %5, %13, %17, %5 op_sel:[1,0,0,0]\n\t"
        "v_mad_u32_u16 %6, %14, %17, %6 op_sel:[1,0,0,0]\n\t"
        "v_mad_u32_u16 %7, %15, %17, %7 op_sel:[1,0,0,0]\n\t"
        "v_mad_u32_u16 %8, %12, %17, %8\n\t"
        "v_mad_u32_u16 %9, %13, %17, %9\n\t"
        "v_mad_u32_u16 %10, %14, %17, %10\n\t"
        "v_mad_u32_u16 %11, %15, %17, %11\n\t"
        "v_sad_u8 %0, %4, 0, %18\n\t"
        "v_sad_u8 %1, %6, 0, %18\n\t"
        "v_sad_u8 %2, %8, 0, %18\n\t"
        "v_sad_u8 %3, %10, 0, %18\n\t"
        "v_sad_hi_u8 %0, %5, 0, %0\n\t"
        "v_sad_hi_u8 %1, %7, 0, %1\n\t"
        "v_sad_hi_u8 %2, %9, 0, %2\n\t"
        "v_sad_hi_u8 %3, %11, 0, %3\n\t"
        "v_pk_fma_f16 %0, %0, %19, %20\n\t"
        "v_pk_fma_f16 %1, %1, %19, %20\n\t"
        "v_pk_fma_f16 %2, %2, %19, %20\n\t"
        "v_pk_fma_f16 %3, %3, %19, %20"
        : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3]),
          "=&v"(t[4]), "=&v"(t[5]), "=&v"(t[6]), "=&v"(t[7])
        : "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]),
          "s"(MUL1_HI_SHL16), "s"(MUL1_LO), "s"((F16_1024 << 16) | F16_1024), "s"((KINV_BITS << 16) | KINV_BITS),
          "v"((KBIAS_BITS << 16) | KBIAS_BITS));
}

// Workgroup barrier that orders LDS only: waits for the wave's LDS operations, not for its global loads and stores
// (__syncthreads waits for those too). For barriers whose data is exchanged through LDS alone.
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---- 128-point Hadamard over 16 lanes, 8 elements per lane -------------------------------------------------------------
// Lane j of a 16-lane row holds elements 8 j .. 8 j + 7. Same transform and rounding as had128_wave: spans 1, 2, 4 inside
// the lane, spans 8, 16, 32, 64 between lanes j ^ 1, ^ 2, ^ 4, ^ 8 of the row (DPP, no LDS traffic). A cross-lane stage is
// fma(sgn, v, partner), sgn = -1 on the upper lane: sgn * v is exact, so the single rounding equals the reference's
// a + b (lower) and a - b (upper).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float dpp_xor4(float v)
{
    // banks 0, 2 (lane bit 2 clear) read lane + 4 (row_shl:4), banks 1, 3 read lane - 4 (row_shr:4)
    const int b = __builtin_bit_cast(int, v);
    int p = __builtin_amdgcn_update_dpp(b, b, 0x104, 0xf, 0x5, false);
    p = __builtin_amdgcn_update_dpp(p, b, 0x114, 0xf, 0xa, false);
    return __builtin_bit_cast(float, p);
}

// the value of lane ^ 16 / lane ^ 32, register to register (gfx950 v_permlane16_swap / v_permlane32_swap: with both
// operands the same value, the instruction's two results hold the partner values of the two halves)
__device__ __forceinline__ float xor16_f(float v)
{
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    return __builtin_bit_cast(float, (uint32_t)(((threadIdx.x >> 4) & 1) ? r[0] : r[1]));
}
__device__ __forceinline__ float xor32_f(float v)
{
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
    return __builtin_bit_cast(float, (uint32_t)(((threadIdx.x >> 5) & 1) ? r[0] : r[1]));
}

// ---- 128-point Hadamard over a wave: lane l holds elements 2l, 2l + 1 --------------------------------------------------
// Sylvester order, stages of span 1, 2, 4, ..., 64; at each stage the lower element of a pair becomes a + b and the upper
// one a - b (engine/kernels/nv2/ft_core.h:90-95; the cross-lane butterfly of x16_dev.cu:31-129 adds the same pairs in
// the same order). Results are bit-identical to the sequential form. Cross-lane partners by DPP (lane xor 1, 2, 4, 8)
// and the permlane swaps (xor 16, 32); fma(+-1, v, partner) rounds a + b and a - b exactly as the add and the subtract.
__device__ __forceinline__ void had128_wave(float& v0, float& v1)
{
    const int lane = threadIdx.x & 63;
    {
        const float a = v0, b = v1;
        v0 = a + b;
        v1 = a - b;
    }
    const float s1 = (lane & 1) ? -1.0f : 1.0f, s2 = (lane & 2) ? -1.0f : 1.0f, s4 = (lane & 4) ? -1.0f : 1.0f;
    const float s8 = (lane & 8) ? -1.0f : 1.0f, s16 = (lane & 16) ? -1.0f : 1.0f, s32 = (lane & 32) ? -1.0f : 1.0f;
    v0 = __builtin_fmaf(s1, v0, dpp_f<0xB1>(v0));
    v1 = __builtin_fmaf(s1, v1, dpp_f<0xB1>(v1));
    v0 = __builtin_fmaf(s2, v0, dpp_f<0x4E>(v0));
    v1 = __builtin_fmaf(s2, v1, dpp_f<0x4E>(v1));
    v0 = __builtin_fmaf(s4, v0, dpp_xor4(v0));
    v1 = __builtin_fmaf(s4, v1, dpp_xor4(v1));
    v0 = __builtin_fmaf(s8, v0, dpp_f<0x128>(v0));
    v1 = __builtin_fmaf(s8, v1, dpp_f<0x128>(v1));
    v0 = __builtin_fmaf(s16, v0, xor16_f(v0));
    v1 = __builtin_fmaf(s16, v1, xor16_f(v1));
    v0 = __builtin_fmaf(s32, v0, xor32_f(v0));
    v1 = __builtin_fmaf(s32, v1, xor32_f(v1));
}

// had128_x8: the 16-lane form. Spans 1, 2, 4 inside the lane as above; at spans 8, 16, 32, 64 both lanes of a pair
// compute fma(partner, s, own), s = +1 on the lower lane and -1 on the upper one, with the partner read through DPP in
// the same instruction (v_fmac_f32_dpp): a + b on the lower lane, b - a on the upper, where the reference has a - b.
// RN(b - a) = -RN(a - b) exactly, and a sign carried into a later stage is common to both lanes of its pair (they differ
// only in that stage's bit), so it factors out: every output is the reference's value times had128_x8_sign(), which
// is (-1)^popcount(j & 15) for lane j. Callers fold that sign into their next multiply (sign flips are exact, so the
// products carry the reference's bits).
__device__ __forceinline__ float had128_x8_sign()
{
    return (__builtin_popcount(threadIdx.x & 15) & 1) ? -1.0f : 1.0f;
}

// v[e] = fma(v[e] of the DPP partner, s, v[e]) for the 8 values, one v_fmac_f32_dpp each (the compiler keeps the DPP
// move apart from a multiply-accumulate). The leading s_nop gives the two wait states a DPP read needs after a VALU write
// of its source; inside the block each instruction reads a register no earlier one in it wrote.
template <int K>   // 0: quad_perm [1,0,3,2], 1: quad_perm [2,3,0,1], 2: row_ror:8
__device__ __forceinline__ void fmac_dpp_x8(float (&v)[8], float s)
{
#define BMX_FMAC8(D)                                                                                                    \
    asm("s_nop 1\n\t"                                                                                                  \
        "v_fmac_f32_dpp %0, %0, %8 " D "\n\t"                                                                          \
        "v_fmac_f32_dpp %1, %1, %8 " D "\n\t"                                                                          \
        "v_fmac_f32_dpp %2, %2, %8 " D "\n\t"                                                                          \
        "v_fmac_f32_dpp %3, %3, %8 " D "\n\t"                                                                          \
        "v_fmac_f32_dpp %4, %4, %8 " D "\n\t"                                                                          \
        "v_fmac_f32_dpp %5, %5, %8 " D "\n\t"                                                                          \
        "v_fmac_f32_dpp %6, %6, %8 " D "\n\t"                                                                          \
        "v_fmac_f32_dpp %7, %7, %8 " D                                                                                 \
        : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7])                \
        : "v"(s))
    if (K == 0) BMX_FMAC8("quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf");
    else if (K == 1) BMX_FMAC8("quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf");
    else BMX_FMAC8("row_ror:8 row_mask:0xf bank_mask:0xf");
#undef BMX_FMAC8
}

__device__ __forceinline__ void had128_x8(float (&v)[8])
{
#pragma unroll
    for (int s = 1; s < 8; s <<= 1)
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (!(e & s))
            {
                const float a = v[e], b = v[e + s];
                v[e] = a + b;
                v[e + s] = a - b;
            }
    const int lane = threadIdx.x & 63;
    const float s1 = (lane & 1) ? -1.0f : 1.0f, s2 = (lane & 2) ? -1.0f : 1.0f;
    const float s4 = (lane & 4) ? -1.0f : 1.0f, s8 = (lane & 8) ? -1.0f : 1.0f;
    fmac_dpp_x8<0>(v, s1);                                                              // quad_perm [1,0,3,2]
    fmac_dpp_x8<1>(v, s2);                                                              // quad_perm [2,3,0,1]
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = __builtin_fmaf(dpp_xor4(v[e]), s4, v[e]);
    fmac_dpp_x8<2>(v, s8);                                                              // row_ror:8
}

// 16-byte global loads / stores and 8 fp16 <-> 16 bytes
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef const __attribute__((address_space(1))) u32x4* gptr_u32x4;
__device__ __forceinline__ u32x4 ldg4(const void* p)
{
    return *reinterpret_cast<gptr_u32x4>(reinterpret_cast<uintptr_t>(p));
}
// 4 floats (read as a float vector: __builtin_bit_cast of a single element of an integer vector is miscompiled by this
// compiler, every element reads element 0)
typedef const __attribute__((address_space(1))) f32x4* gptr_f32x4;
__device__ __forceinline__ f32x4 ldg4f(const float* p)
{
    return *reinterpret_cast<gptr_f32x4>(reinterpret_cast<uintptr_t>(p));
}
__device__ __forceinline__ void unpack8(const u32x4 w, float (&v)[8])
{
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        v[2 * i] = h2f(w[i] & 0xffffu);
        v[2 * i + 1] = h2f(w[i] >> 16);
    }
}
__device__ __forceinline__ u32x4 pack8_r(const float (&v)[8])
{
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = (uint32_t)f2h_r(v[2 * i]) | ((uint32_t)f2h_r(v[2 * i + 1]) << 16);
    return w;
}

// ---- fixed-sequence fp32 exp (the router's; the oracle evaluates the same sequence) ----------------------------------
// Cody-Waite argument reduction (W. J. Cody and W. Waite, Software Manual for the Elementary Functions, 1980):
// n = rint(x / ln 2), r = x - n ln 2 with ln 2 split into a high part of 17 significant bits and a low part (the split
// SLEEF's expf uses: 0.693145751953125 + 1.428606765330187e-06); exp(r) by the Taylor polynomial of degree 7 in Horner
// form (|r| <= ln 2 / 2); 2^n applied as two exact power-of-two factors, so a subnormal result rounds once.
__device__ __forceinline__ float exp_fixed(float x)
{
    if (x != x) return x;
    if (x > 88.72f) return __builtin_huge_valf();
    if (x < -104.0f) return 0.0f;
    const float n = __builtin_rintf(__fmul_rn(x, 1.44269504f));
    float r = __builtin_fmaf(n, -0.693145751953125f, x);
    r = __builtin_fmaf(n, -1.428606765330187e-06f, r);
    float p = 1.98412698e-4f;
    p = __builtin_fmaf(p, r, 1.38888889e-3f);
    p = __builtin_fmaf(p, r, 8.33333333e-3f);
    p = __builtin_fmaf(p, r, 4.16666667e-2f);
    p = __builtin_fmaf(p, r, 1.66666667e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int ni = (int)n;
    const int n1 = ni / 2, n2 = ni - n1;
    const float s1 = __builtin_bit_cast(float, (uint32_t)(n1 + 127) << 23);
    const float s2 = __builtin_bit_cast(float, (uint32_t)(n2 + 127) << 23);
    return __fmul_rn(__fmul_rn(p, s1), s2);
}

__device__ __forceinline__ float sigmoid_fixed(float x)
{
    const float e = exp_fixed(-x);
    return __fdiv_rn(1.0f, __fadd_rn(1.0f, e));
}

// Correctly rounded fp32 square root. The hardware square root (v_sqrt_f32) is within 1 ulp but not correctly rounded;
// the estimate is moved by one ulp while the Tuckerman test fails (Markstein, IA-64 and Elementary Functions, 2000):
// y = RN(sqrt(a)) iff (y - u_lo / 2)^2 < a < (y + u / 2)^2, u / u_lo the spacing above / below y. The midpoints have
// 25 significant bits, so they and their squares (50 bits) are exact in double; no a has its root exactly on a midpoint.
__device__ __forceinline__ float sqrt_rn(float a)
{
    float y = __builtin_sqrtf(a);
    if (!(a > 0.0f) || !(a < __builtin_huge_valf())) return y;       // 0, negative, inf, NaN: the hardware's result
    const double d = (double)a;
#pragma unroll
    for (int it = 0; it < 2; ++it)
    {
        const uint32_t yb = __builtin_bit_cast(uint32_t, y);          // y > 0 and finite: neighbours by the bits
        const float up = __builtin_bit_cast(float, yb + 1u), dn = __builtin_bit_cast(float, yb - 1u);
        const double mh = 0.5 * ((double)y + (double)up), ml = 0.5 * ((double)y + (double)dn);
        if (mh * mh < d) y = up;
        else if (ml * ml > d) y = dn;
    }
    return y;
}

// sqrt(softplus(x)) = sqrt(max(x, 0) + log1p(exp(-|x|))), the DeepSeek-V4 router's score ("sqrtsoftplus"). log1p(e)
// for e = exp(-|x|) in [0, 1] by the series log(1 + e) = 2 atanh(s) = 2 (s + s^3 / 3 + s^5 / 5 + ...), s = e / (2 + e)
// <= 1/3 (Abramowitz and Stegun 4.1.27), nine terms (relative error below 1e-9 before rounding): no cancellation for
// small e. Correctly rounded division and square root; the oracle evaluates the same sequence.
__device__ __forceinline__ float sqrtsp_fixed(float x)
{
    if (x != x) return x;
    const float e = exp_fixed(-fabsf(x));
    const float s = __fdiv_rn(e, __fadd_rn(2.0f, e));
    const float s2 = __fmul_rn(s, s);
    float p = 1.0f / 17.0f;
    p = __builtin_fmaf(p, s2, 1.0f / 15.0f);
    p = __builtin_fmaf(p, s2, 1.0f / 13.0f);
    p = __builtin_fmaf(p, s2, 1.0f / 11.0f);
    p = __builtin_fmaf(p, s2, 1.0f / 9.0f);
    p = __builtin_fmaf(p, s2, 1.0f / 7.0f);
    p = __builtin_fmaf(p, s2, 1.0f / 5.0f);
    p = __builtin_fmaf(p, s2, 1.0f / 3.0f);
    p = __builtin_fmaf(p, s2, 1.0f);
    const float l = __fmul_rn(__fmul_rn(2.0f, s), p);
    return sqrt_rn(__fadd_rn(fmaxf(x, 0.0f), l));
}

// tanh t = 1 - 2 / (exp(2 t) + 1) on the fixed-sequence exp
__device__ __forceinline__ float tanh_fixed(float t)
{
    const float e = exp_fixed(__fmul_rn(2.0f, t));
    return __fsub_rn(1.0f, __fdiv_rn(2.0f, __fadd_rn(e, 1.0f)));
}

// ---- activations (exllamav3 act_gate semantics, engine/kernels/x16/x16_dev.cu:68-112) ----------------------------------
// Evaluated with the fixed-sequence exp and correctly rounded operations in a stated order (no hardware approximations),
// so that a host CPU reproduces every bit (the CPU expert lane).
__device__ __forceinline__ float act_gate(int act, int gated, float g, float u, float limit)
{
    if (act == BMX_ACT_SILU_OAI)
    {
        if (limit != 0.0f)
        {
            g = fminf(g, limit);
            u = fminf(fmaxf(u, -limit), limit);
        }
        const float glu = __fdiv_rn(g, __fadd_rn(1.0f, exp_fixed(__fmul_rn(-1.702f, g))));
        return __fmul_rn(__fadd_rn(u, 1.0f), glu);
    }
    float x;
    if (!gated) x = fmaxf(0.0f, u);
    else if (act == BMX_ACT_SILU) x = __fdiv_rn(g, __fadd_rn(1.0f, exp_fixed(-g)));
    else if (act == BMX_ACT_GELU)
    {
        const float g3 = __fmul_rn(__fmul_rn(__fmul_rn(0.044715f, g), g), g);
        const float t = __fmul_rn(0.797884560803f, __fadd_rn(g, g3));
        x = __fmul_rn(__fmul_rn(0.5f, g), __fadd_rn(1.0f, tanh_fixed(t)));
    }
    else
    {
        x = fmaxf(0.0f, g);
        x = __fmul_rn(x, x);
    }
    if (limit != 0.0f)
    {
        u = fminf(fmaxf(u, -limit), limit);
        x = fminf(x, limit);
    }
    return __fmul_rn(x, u);
}

// The same activations evaluated with the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32: about 1 ulp each; exp(x)
// as exp2(x log2 e)) instead of the fixed sequence and correctly rounded divisions: for the prefill path, whose rows
// no host lane replays. The results differ from act_gate's in the last bits of fp32, before the epilogue's rotation and
// its single fp16 rounding.
__device__ __forceinline__ float exp_hw(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float rcp_hw(float x) { return __builtin_amdgcn_rcpf(x); }

__device__ __forceinline__ float act_gate_fast(int act, int gated, float g, float u, float limit)
{
    if (act == BMX_ACT_SILU_OAI)
    {
        if (limit != 0.0f)
        {
            g = fminf(g, limit);
            u = fminf(fmaxf(u, -limit), limit);
        }
        const float glu = g * rcp_hw(1.0f + exp_hw(-1.702f * g));
        return (u + 1.0f) * glu;
    }
    float x;
    if (!gated) x = fmaxf(0.0f, u);
    else if (act == BMX_ACT_SILU) x = g * rcp_hw(1.0f + exp_hw(-g));
    else if (act == BMX_ACT_GELU)
    {
        const float t = 0.797884560803f * (g + 0.044715f * g * g * g);
        x = (0.5f * g) * (1.0f - 2.0f * rcp_hw(exp_hw(2.0f * t) + 1.0f));
    }
    else
    {
        x = fmaxf(0.0f, g);
        x = x * x;
    }
    if (limit != 0.0f)
    {
        u = fminf(fmaxf(u, -limit), limit);
        x = fminf(x, limit);
    }
    return x * u;
}

}  // namespace bmx
