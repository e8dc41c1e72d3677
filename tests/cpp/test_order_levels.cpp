// Checks unsorted_levels (bevy_synth_amd/csrc/sc_common.hpp), the row-order
// test shared by the neighbour map's rank bitmap and the conv plan, against
// the octree keys built explicitly: for every pair of coords and every level
// count L < kRankLevels, bit L must be clear exactly when a precedes c
// strictly in (b, x >> L, y >> L, z >> L, octree digits of the low L bits),
// the digits read from the coarsest level down, each x | y << 1 | z << 2.
// Host only; run by tests/test_order_levels.py.
#include <cstdio>
#include <random>
#include <tuple>

#include "../../bevy_synth_amd/csrc/sc_common.hpp"

using sc::kRankLevels;
using sc::unsorted_levels;

static long long digits(int4 v, int L)
{
    long long d = 0;
    for (int i = L - 1; i >= 0; --i)
        d = d * 8 + (((v.y >> i) & 1) | ((v.z >> i) & 1) << 1 | ((v.w >> i) & 1) << 2);
    return d;
}

static bool key_less(int4 a, int4 c, int L)
{
    const auto ka = std::make_tuple(a.x, a.y >> L, a.z >> L, a.w >> L, digits(a, L));
    const auto kc = std::make_tuple(c.x, c.y >> L, c.z >> L, c.w >> L, digits(c, L));
    return ka < kc;
}

int main()
{
    std::mt19937_64 rng(20261202);
    long long checked = 0, bad = 0;
    // ranges: tiny (equal roots and equal coords are common), decoder-sized,
    // and full int range with negative values
    const int spans[3] = {8, 1024, 0};
    for (int s = 0; s < 3; ++s) {
        for (int t = 0; t < 400000; ++t) {
            auto draw = [&]() {
                if (spans[s] == 0) return (int)(uint32_t)rng();
                return (int)(rng() % (uint64_t)spans[s]);
            };
            int4 a = make_int4((int)(rng() % 2), draw(), draw(), draw());
            int4 c = a;
            // c: a perturbed in a few coordinates (or not at all)
            const int m = (int)(rng() % 16);
            if (m & 1) c.x = (int)(rng() % 2);
            if (m & 2) c.y = draw();
            if (m & 4) c.z = draw();
            if (m & 8) c.w = draw();
            const uint32_t got = unsorted_levels(a, c);
            for (int L = 0; L < kRankLevels; ++L) {
                const bool want_bad = !key_less(a, c, L);
                if (((got >> L) & 1u) != (uint32_t)want_bad) {
                    if (bad < 10)
                        std::printf("mismatch L=%d a=(%d,%d,%d,%d) c=(%d,%d,%d,%d) got=%u\n", L, a.x, a.y, a.z,
                                    a.w, c.x, c.y, c.z, c.w, got);
                    ++bad;
                }
                ++checked;
            }
        }
    }
    if (bad) {
        std::printf("%lld of %lld checks failed\n", bad, checked);
        return 1;
    }
    std::printf("order levels ok: %lld checks\n", checked);
    return 0;
}
