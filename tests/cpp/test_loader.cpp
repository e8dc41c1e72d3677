// Drives include/sparse_decoder_loading.hpp on a safetensors file written by
// tests/test_loader.py and dumps what it loaded, for the Python side to check
// against numpy:
//   test_loader host   FILE OUTDIR   decode only (no GPU): every tensor as f32
//   test_loader device FILE OUTDIR   load the layers onto the device and
//                                    download the weights (compute dtype
//                                    bits) and the packed copies
// Output files: <name>.f32 / <name>.bin raw little-endian, errors.txt with
// one "key: message" line per refused layer, config.txt one line per layer.
#include <cstdio>
#include <string>
#include <vector>

#include "sparse_decoder_loading.hpp"

using namespace burn_flex_gmm_hip;
using namespace burn_flex_gmm_hip::loading;

static bool write_raw(const std::string &path, const void *p, size_t n)
{
    std::FILE *f = std::fopen(path.c_str(), "wb");
    if (!f) return false;
    const bool ok = n == 0 || std::fwrite(p, 1, n, f) == n;
    std::fclose(f);
    return ok;
}

int main(int argc, char **argv)
{
    if (argc != 4) {
        std::fprintf(stderr, "usage: %s host|device FILE OUTDIR\n", argv[0]);
        return 2;
    }
    const std::string mode = argv[1], path = argv[2], out = argv[3];
    auto st = SafeTensors::open(path);
    if (st.is_err()) {
        std::fprintf(stderr, "open: %s\n", st.error().c_str());
        return 1;
    }
    std::FILE *errs = std::fopen((out + "/errors.txt").c_str(), "w");
    std::FILE *cfgs = std::fopen((out + "/config.txt").c_str(), "w");
    if (!errs || !cfgs) return 1;
    int failures = 0;
    if (mode == "host") {
        for (const char *k : {"conv_f32.weight", "conv_f16.weight", "conv_bf16.weight", "conv_f32.bias", "lin.weight",
                              "edge_f16"}) {
            auto t = st.value().load_tensor_f32(k);
            if (t.is_err()) {
                std::fprintf(stderr, "%s: %s\n", k, t.error().c_str());
                ++failures;
                continue;
            }
            write_raw(out + "/" + k + ".f32", t.value().second.data(), t.value().second.size() * 4);
        }
        auto r = round_vec_to_f16(st.value().load_tensor_f32("conv_f32.weight").value().second);
        write_raw(out + "/round_f16.f32", r.data(), r.size() * 4);
        for (const char *k : {"bad_dtype.weight", "missing.weight"}) {
            auto t = st.value().load_tensor_f32(k);
            std::fprintf(errs, "%s: %s\n", k, t.is_err() ? t.error().c_str() : "OK");
        }
        auto v = st.value().load_vector("conv_f32.bias", 63);
        std::fprintf(errs, "vector_len: %s\n", v.is_err() ? v.error().c_str() : "OK");
    } else {
        struct Case {
            const char *name;
            size_t expected_in, expected_out;
            DType dt;
        };
        const Case cases[] = {{"conv_f32", 0, 64, DType::BF16},  {"conv_f16", 32, 64, DType::F16},
                              {"conv_bf16", 32, 0, DType::BF16}, {"conv_f32", 0, 0, DType::F32},
                              {"grouped", 64, 64, DType::BF16},  {"bad_rank", 0, 0, DType::BF16},
                              {"conv_f32", 48, 0, DType::BF16},  {"conv_f32", 0, 65, DType::BF16},
                              {"bias_len", 0, 0, DType::BF16}};
        int idx = 0;
        for (const Case &c : cases) {
            auto L = load_sparse_conv(st.value(), std::string(c.name) + ".weight", std::string(c.name) + ".bias",
                                      c.expected_in, c.expected_out, c.dt);
            const std::string tag = std::to_string(idx++) + "_" + c.name;
            if (L.is_err()) {
                std::fprintf(errs, "%s: %s\n", tag.c_str(), L.error().c_str());
                continue;
            }
            const SparseSubmConvConfig &k = L.value().config;
            std::fprintf(cfgs, "%s %zu %zu %zu %zu %zu %zu %zu %zu %d\n", tag.c_str(), k.in_channels, k.out_channels,
                         k.kernel_d, k.kernel_h, k.kernel_w, k.in_channels_per_group, k.out_channels_per_group,
                         k.groups, L.value().packed ? 1 : 0);
            const DeviceTensor &w = L.value().weight;
            std::vector<uint8_t> wb(w.bytes());
            if (hipMemcpy(wb.data(), w.data(), wb.size(), hipMemcpyDeviceToHost) != hipSuccess) ++failures;
            write_raw(out + "/" + tag + ".weight.bin", wb.data(), wb.size());
            auto bh = L.value().bias.to_vec<float>();
            if (bh.is_err()) ++failures;
            else write_raw(out + "/" + tag + ".bias.f32", bh.value().data(), bh.value().size() * 4);
            if (L.value().packed) {
                std::vector<uint8_t> pb(L.value().packed->bytes());
                if (hipMemcpy(pb.data(), L.value().packed->data(), pb.size(), hipMemcpyDeviceToHost) != hipSuccess)
                    ++failures;
                write_raw(out + "/" + tag + ".packed.bin", pb.data(), pb.size());
            }
        }
        auto lin = load_linear(st.value(), "lin.weight", "lin.bias", 32, 16, DType::F16);
        if (lin.is_err()) {
            std::fprintf(errs, "lin: %s\n", lin.error().c_str());
        } else {
            std::vector<uint8_t> wb(lin.value().weight.bytes());
            if (hipMemcpy(wb.data(), lin.value().weight.data(), wb.size(), hipMemcpyDeviceToHost) != hipSuccess)
                ++failures;
            write_raw(out + "/lin.weight.bin", wb.data(), wb.size());
        }
        auto lin_bad = load_linear(st.value(), "lin.weight", "lin.bias", 31, 0, DType::F16);
        std::fprintf(errs, "lin_bad: %s\n", lin_bad.is_err() ? lin_bad.error().c_str() : "OK");
    }
    std::fclose(errs);
    std::fclose(cfgs);
    if (failures) {
        std::fprintf(stderr, "%d failure(s)\n", failures);
        return 1;
    }
    std::printf("loader %s ok\n", mode.c_str());
    return 0;
}
