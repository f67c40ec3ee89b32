// EXL3 trellis -> fp16 codebook weights (bit-exact decode), one workgroup per 16 x 16 tile.
#include "bmx_common.hpp"
#include "bmx_internal.hpp"

namespace bmx {

// Thread i decodes stream position i of its tile: state = ring bits [S(i) - 16, S(i)) (two 32-bit words, the second
// wrapping to the ring's start), codebook weight, written to (row, col) = make_tc_perm(i)
// (engine/kernels/nv2/ft_core.h:49-84, 1007-1022 in the reference restate the same steps on the CPU).
template <int F>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ tr, int n, uint16_t* __restrict__ out)
{
    constexpr int TB = Fmt<F>::TB, NBITS = 8 * TB, NW = TB / 4;
    __shared__ uint32_t words[NW];
    const int tiles_n = n / 16;
    const int tk = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(tr + (size_t)blockIdx.x * TB);
    const int i = threadIdx.x;
    if (i < NW) words[i] = src[i];
    __syncthreads();
    int p = ring_end<F>(i) - 16;
    p = ((p % NBITS) + NBITS) % NBITS;
    const uint32_t w0 = words[(p >> 5) % NW], w1 = words[((p >> 5) + 1) % NW];
    const uint32_t st = (uint32_t)((((uint64_t)w0 << 32) | w1) >> (48 - (p & 31))) & 0xffffu;
    const uint32_t x = cb_hash(st);
    const f16x2 w = cb_pair(x, x);
    const int g = i >> 3, j = i & 7;
    const int r = 2 * (g & 3) + ((j & 3) == 0 ? 0 : (j & 3) == 1 ? 1 : (j & 3) == 2 ? 8 : 9);
    const int c = (g >> 2) + (j >= 4 ? 8 : 0);
    out[(size_t)(tk * 16 + r) * n + tn * 16 + c] = __builtin_bit_cast(uint16_t, w.x);
}

int launch_dequant(const void* trellis, int fmt, int k, int n, void* out, hipStream_t s)
{
    const unsigned tiles = (unsigned)((k / 16) * (n / 16));
    if (tiles == 0) return BMX_OK;
    const uint8_t* t = static_cast<const uint8_t*>(trellis);
    uint16_t* o = static_cast<uint16_t*>(out);
    switch (fmt)
    {
        case BMX_TF_K2: hipLaunchKernelGGL(k_dequant<BMX_TF_K2>, dim3(tiles), dim3(256), 0, s, t, n, o); break;
        case BMX_TF_K25: hipLaunchKernelGGL(k_dequant<BMX_TF_K25>, dim3(tiles), dim3(256), 0, s, t, n, o); break;
        case BMX_TF_K3: hipLaunchKernelGGL(k_dequant<BMX_TF_K3>, dim3(tiles), dim3(256), 0, s, t, n, o); break;
        case BMX_TF_K4: hipLaunchKernelGGL(k_dequant<BMX_TF_K4>, dim3(tiles), dim3(256), 0, s, t, n, o); break;
        default: return set_error(BMX_ERR_ARG, "bmx_exl3_dequant: unknown trellis format %d", fmt);
    }
    return check_launch("bmx_exl3_dequant");
}

}  // namespace bmx
