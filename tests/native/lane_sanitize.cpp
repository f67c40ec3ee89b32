// Host driver for the CPU lane under the sanitizers (built by tests/test_cpu_lane_sanitize.py with g++ only): random
// experts of every trellis format and several shapes through the fast mode at several worker counts (the rows must not
// depend on the count) and through the exact lane. Exit status: the number of mismatches.
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

#include "bmx.h"

namespace bmx {
// the library's error setter lives in the HIP part; this driver links the CPU lane alone
int set_error(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vfprintf(stderr, fmt, ap);
    va_end(ap);
    fprintf(stderr, "\n");
    return code;
}
}  // namespace bmx

static int tile_bytes(int fmt) { return fmt == BMX_TF_K2 ? 64 : fmt == BMX_TF_K25 ? 80 : fmt == BMX_TF_K3 ? 96 : 128; }

struct Expert {
    std::vector<uint8_t> tr[3];
    std::vector<uint16_t> suh[3], svh[3];
    bmx_cpu_expert ex{};
    Expert(int H, int I, int fmt, std::mt19937& rng)
    {
        const int K[3] = {H, H, I}, N[3] = {I, I, H};
        for (int m = 0; m < 3; ++m)
        {
            tr[m].resize((size_t)K[m] * N[m] / 256 * tile_bytes(fmt));
            for (auto& b : tr[m]) b = (uint8_t)rng();
            suh[m].assign(K[m], 0x3c00);     // 1.0
            svh[m].assign(N[m], 0x3000);     // 0.125
            ex.tr[m] = tr[m].data();
            ex.suh[m] = suh[m].data();
            ex.svh[m] = svh[m].data();
            ex.fmt[m] = fmt;
        }
    }
};

int main(int argc, char** argv)
{
    const bool small = argc > 1;            // fewer cases (the thread sanitizer's run)
    std::mt19937 rng(3);
    std::vector<std::pair<int, int>> shapes = {{256, 128}, {2048, 1536}};
    if (!small) shapes.push_back({1024, 512});
    int bad = 0;
    for (auto [H, I] : shapes)
        for (int fmt = BMX_TF_K2; fmt <= BMX_TF_K4; ++fmt)
            for (int nr : {1, 9})
            {
                Expert e(H, I, fmt, rng);
                std::vector<uint16_t> x((size_t)nr * H);
                for (auto& v : x) v = (uint16_t)(0x3800 + (rng() & 0x3ff));
                std::vector<float> y1((size_t)nr * H), y2((size_t)nr * H);
                if (bmx_cpu_expert_rows_fast(&e.ex, H, I, x.data(), nr, 0, 1, 0.f, y1.data(), small ? 2 : 1) ||
                    bmx_cpu_expert_rows_fast(&e.ex, H, I, x.data(), nr, 0, 1, 0.f, y2.data(), small ? 3 : 7))
                {
                    ++bad;
                    continue;
                }
                for (size_t i = 0; i < y1.size(); ++i)
                    if (!(y1[i] == y2[i]) && !(std::isnan(y1[i]) && std::isnan(y2[i])))
                    {
                        ++bad;
                        break;
                    }
            }
    {
        const int H = 512, I = 256;
        Expert e(H, I, BMX_TF_K3, rng);
        std::vector<uint16_t> x((size_t)3 * H, 0x3c00);
        std::vector<float> y((size_t)3 * H);
        if (bmx_cpu_expert_rows(&e.ex, H, I, x.data(), 3, 2, 1, 1, 0, 1, 0.f, y.data(), small ? 2 : 4)) ++bad;
    }
    printf("lane sanitize: %d mismatches\n", bad);
    return bad;
}
