// Exercises the C++ host mirror (include/burn_flex_gmm_hip.hpp) on the GPU:
// the reference's known-answer tests through the same-named functions, error
// results, and a device-tensor conv checked against a double-precision loop.
#include <cmath>
#include <cstdio>
#include <random>

#include "burn_flex_gmm_hip.hpp"

using namespace burn_flex_gmm_hip;

static int failures = 0;
#define CHECK(cond, ...)                                      \
    do {                                                      \
        if (!(cond)) {                                        \
            std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            std::fprintf(stderr, __VA_ARGS__);                \
            std::fprintf(stderr, "\n");                       \
            ++failures;                                       \
        }                                                     \
    } while (0)

static SparseSubmConvConfig cfg(size_t cin, size_t cout, size_t kd, size_t kh, size_t kw, size_t groups)
{
    SparseSubmConvConfig c;
    c.in_channels = cin;
    c.out_channels = cout;
    c.kernel_d = kd;
    c.kernel_h = kh;
    c.kernel_w = kw;
    c.groups = groups;
    c.in_channels_per_group = cin / groups;
    c.out_channels_per_group = cout / groups;
    return c;
}

static uint16_t to_bf16(float f)
{
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

static float from_bf16(uint16_t h)
{
    uint32_t b = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

int main()
{
    // sparse_decoder_tests.rs:190-236 -> [201, 12]
    {
        auto c = cfg(1, 1, 3, 1, 1, 1);
        std::vector<std::array<uint32_t, 4>> coords{{0, 0, 0, 0}, {0, 1, 0, 0}};
        auto nbr = build_neighbor_rows(c, coords);
        CHECK(nbr.is_ok(), "build_neighbor_rows: %s", nbr.error().c_str());
        std::vector<float> w{10.f, 1.f, 100.f}, b{0.f};
        auto out = sparse_subm_conv_forward_flex_precomputed(c, {w.data(), 3, b.data(), 1}, {1.f, 2.f},
                                                             nbr.value());
        CHECK(out.is_ok(), "conv: %s", out.error().c_str());
        if (out.is_ok()) {
            CHECK(std::fabs(out.value()[0] - 201.f) < 1e-5f, "out[0]=%f", out.value()[0]);
            CHECK(std::fabs(out.value()[1] - 12.f) < 1e-5f, "out[1]=%f", out.value()[1]);
        }
    }
    // sparse_decoder_tests.rs:239-292 -> [-1,0,1] and chunk [-1,0,-1]
    {
        auto c = cfg(1, 1, 3, 1, 1, 1);
        auto full = build_neighbor_rows(c, {{0, 0, 0, 0}, {0, 1, 0, 0}});
        auto chunk = build_neighbor_rows(c, {{0, 0, 0, 0}});
        CHECK(full.is_ok() && chunk.is_ok(), "maps");
        if (full.is_ok() && chunk.is_ok()) {
            CHECK((full.value() == std::vector<int32_t>{-1, 0, 1, 0, 1, -1}), "full map");
            CHECK((chunk.value() == std::vector<int32_t>{-1, 0, -1}), "chunk map");
        }
    }
    // errors come back as Result values with the reference's messages
    {
        auto bad = cfg(4, 8, 3, 3, 3, 2);
        bad.in_channels_per_group = 3;
        auto k = kernel_rows(bad);
        CHECK(k.is_err() && k.error().find("in_channels/group mismatch") != std::string::npos, "%s",
              k.error().c_str());
        auto c = cfg(1, 1, 3, 1, 1, 1);
        std::vector<float> w{1.f, 1.f, 1.f}, b{0.f};
        auto oob = sparse_subm_conv_forward_flex_precomputed(c, {w.data(), 3, b.data(), 1}, {1.f},
                                                             {-1, 0, 5});
        CHECK(oob.is_err() && oob.error().find("out of bounds") != std::string::npos, "%s",
              oob.error().c_str());
        auto big = build_neighbor_rows(c, {{0, 0x80000000u, 0, 0}});
        CHECK(big.is_err() && big.error().find("exceeds i32::MAX") != std::string::npos, "%s",
              big.error().c_str());
    }
    // device tensors: bf16 3x3x3 conv on a small dense block vs a double loop
    {
        const size_t C = 64, nx = 6, ny = 5, nz = 7, N = nx * ny * nz;
        auto c = cfg(C, C, 3, 3, 3, 1);
        std::vector<int32_t> coords;
        for (size_t x = 0; x < nx; ++x)
            for (size_t y = 0; y < ny; ++y)
                for (size_t z = 0; z < nz; ++z) coords.insert(coords.end(), {0, (int)x, (int)y, (int)z});
        std::mt19937 rng(7);
        std::normal_distribution<float> nd(0.f, 1.f);
        std::vector<uint16_t> xb(N * C), wb(C * 27 * C);
        for (auto &v : xb) v = to_bf16(nd(rng));
        for (auto &v : wb) v = to_bf16(nd(rng) * 0.03f);
        std::vector<float> bias(C, 0.25f);
        auto dc = DeviceTensor::from_host(coords.data(), {N, 4}, DType::I32);
        auto dx = DeviceTensor::from_host(xb.data(), {N, C}, DType::BF16);
        auto dw = DeviceTensor::from_host(wb.data(), {C, 3, 3, 3, C}, DType::BF16);
        auto dbias = DeviceTensor::from_host(bias.data(), {C}, DType::F32);
        auto map = neighbor_rows_tensor_from_coords_tensor(c, dc.value());
        CHECK(map.is_ok(), "%s", map.error().c_str());
        ConvOptions opt;
        opt.out_dtype = DType::F32;
        auto out = sparse_subm_conv_forward_hip(c, dx.value(), map.value(), dw.value(), dbias.value(), opt);
        CHECK(out.is_ok(), "%s", out.error().c_str());
        if (map.is_ok() && out.is_ok()) {
            auto m = map.value().to_vec<int32_t>().take();
            auto o = out.value().to_vec<float>().take();
            double max_err = 0, rms = 0;
            std::vector<double> ref(N * C);
            for (size_t r = 0; r < N; ++r)
                for (size_t oc = 0; oc < C; ++oc) {
                    double acc = bias[oc];
                    for (int k = 0; k < 27; ++k) {
                        const int nb = m[r * 27 + k];
                        if (nb < 0) continue;
                        for (size_t i = 0; i < C; ++i)
                            acc += (double)from_bf16(xb[nb * C + i]) * from_bf16(wb[(oc * 27 + k) * C + i]);
                    }
                    ref[r * C + oc] = acc;
                    rms += acc * acc;
                }
            rms = std::sqrt(rms / ref.size());
            for (size_t i = 0; i < ref.size(); ++i)
                max_err = std::max(max_err, std::fabs(o[i] - ref[i]) / std::max(std::fabs(ref[i]), rms));
            CHECK(max_err <= 1e-4, "bf16 conv rel err %g", max_err);
            std::printf("device conv rel err %.3g\n", max_err);

            // the planned conv (plan + packed weights) against the same loop,
            // then with the LayerNorm + SiLU epilogue against the unplanned one
            auto plan = build_conv_plan(c, dc.value(), map.value());
            CHECK(plan.is_ok(), "%s", plan.error().c_str());
            auto wp = pack_conv_weight(c, dw.value());
            CHECK(wp.is_ok(), "%s", wp.error().c_str());
            if (plan.is_ok() && wp.is_ok()) {
                ConvOptions po = opt;
                po.plan = &plan.value();
                po.packed_weight = &wp.value();
                auto pout = sparse_subm_conv_forward_hip(c, dx.value(), map.value(), dw.value(), dbias.value(), po);
                CHECK(pout.is_ok(), "%s", pout.error().c_str());
                if (pout.is_ok()) {
                    auto p = pout.value().to_vec<float>().take();
                    double perr = 0;
                    for (size_t i = 0; i < ref.size(); ++i)
                        perr = std::max(perr, std::fabs(p[i] - ref[i]) / std::max(std::fabs(ref[i]), rms));
                    CHECK(perr <= 1e-4, "planned conv rel err %g", perr);
                    std::printf("planned conv rel err %.3g\n", perr);
                }
                ConvOptions lo = opt, plo = po;
                lo.layer_norm = plo.layer_norm = true;
                lo.silu = plo.silu = true;
                auto a = sparse_subm_conv_forward_hip(c, dx.value(), map.value(), dw.value(), dbias.value(), lo);
                auto b2 = sparse_subm_conv_forward_hip(c, dx.value(), map.value(), dw.value(), dbias.value(), plo);
                CHECK(a.is_ok() && b2.is_ok(), "fused convs");
                if (a.is_ok() && b2.is_ok()) {
                    auto av = a.value().to_vec<float>().take(), bv = b2.value().to_vec<float>().take();
                    double d = 0;
                    for (size_t i = 0; i < av.size(); ++i) d = std::max(d, (double)std::fabs(av[i] - bv[i]));
                    CHECK(d <= 1e-4, "planned LN+SiLU vs unplanned: max abs diff %g", d);
                    std::printf("planned LN+SiLU max diff %.3g\n", d);
                }
                ConvOptions bad = po;
                bad.packed_weight = nullptr;
                auto e = sparse_subm_conv_forward_hip(c, dx.value(), map.value(), dw.value(), dbias.value(), bad);
                CHECK(e.is_err() && e.error().find("go together") != std::string::npos, "plan without packed weights");
            }
        }
    }
    if (failures) {
        std::fprintf(stderr, "%d failure(s)\n", failures);
        return 1;
    }
    std::printf("host api ok\n");
    return 0;
}
