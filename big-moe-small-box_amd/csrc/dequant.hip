// EXL3 trellis -> fp16 codebook weights (bit-exact decode), one workgroup per 16 x 16 tile.
#include "bmx_common.hpp"
#include "bmx_internal.hpp"

namespace bmx {

// Eight tiles per workgroup, 32 threads per tile; thread j decodes stream positions 8 j .. 8 j + 7 of its tile:
// state = ring bits [S(i) - 16, S(i)) (two 32-bit words, the second wrapping to the ring's start), codebook weight
// (the decoder the expert kernels use), written to (row, col) = make_tc_perm(i)
// (engine/kernels/nv2/ft_core.h:49-84, 1007-1022 in the reference restate the same steps on the CPU).
template <int F>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ tr, int n, int tiles, uint16_t* __restrict__ out)
{
    constexpr int TB = Fmt<F>::TB, NBITS = 8 * TB, NW = TB / 4;
    __shared__ uint32_t words[8][NW];
    const int sub = threadIdx.x >> 5, lt = threadIdx.x & 31;
    const int tile = blockIdx.x * 8 + sub;
    if (tile < tiles && lt < NW) words[sub][lt] = reinterpret_cast<const uint32_t*>(tr + (size_t)tile * TB)[lt];
    __syncthreads();
    if (tile >= tiles) return;
    const int tiles_n = n / 16;
    const int tk = tile / tiles_n, tn = tile % tiles_n;
    uint32_t st[8], w[4];
#pragma unroll
    for (int q = 0; q < 8; ++q)
    {
        int p = ring_end<F>(8 * lt + q) - 16;
        p = ((p % NBITS) + NBITS) % NBITS;
        const uint32_t w0 = words[sub][(p >> 5) % NW], w1 = words[sub][((p >> 5) + 1) % NW];
        st[q] = (uint32_t)((((uint64_t)w0 << 32) | w1) >> (48 - (p & 31)));   // bits above 15 are not read
    }
    cb_oct(st, w);
#pragma unroll
    for (int q = 0; q < 8; ++q)
    {
        const int i = 8 * lt + q, g = i >> 3, j = i & 7;
        const int r = 2 * (g & 3) + ((j & 3) == 0 ? 0 : (j & 3) == 1 ? 1 : (j & 3) == 2 ? 8 : 9);
        const int c = (g >> 2) + (j >= 4 ? 8 : 0);
        out[(size_t)(tk * 16 + r) * n + tn * 16 + c] = (uint16_t)(w[q >> 1] >> (16 * (q & 1)));
    }
}

int launch_dequant(const void* trellis, int fmt, int k, int n, void* out, hipStream_t s)
{
    const int tiles = (k / 16) * (n / 16);
    if (tiles == 0) return BMX_OK;
    const dim3 grid((unsigned)((tiles + 7) / 8));
    const uint8_t* t = static_cast<const uint8_t*>(trellis);
    uint16_t* o = static_cast<uint16_t*>(out);
    switch (fmt)
    {
        case BMX_TF_K2: hipLaunchKernelGGL(k_dequant<BMX_TF_K2>, grid, dim3(256), 0, s, t, n, tiles, o); break;
        case BMX_TF_K25: hipLaunchKernelGGL(k_dequant<BMX_TF_K25>, grid, dim3(256), 0, s, t, n, tiles, o); break;
        case BMX_TF_K3: hipLaunchKernelGGL(k_dequant<BMX_TF_K3>, grid, dim3(256), 0, s, t, n, tiles, o); break;
        case BMX_TF_K4: hipLaunchKernelGGL(k_dequant<BMX_TF_K4>, grid, dim3(256), 0, s, t, n, tiles, o); break;
        default: return set_error(BMX_ERR_ARG, "bmx_exl3_dequant: unknown trellis format %d", fmt);
    }
    return check_launch("bmx_exl3_dequant");
}

}  // namespace bmx
