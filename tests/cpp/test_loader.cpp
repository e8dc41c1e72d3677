// Drives include/sparse_decoder_loading.hpp on a safetensors file written by
// tests/test_loader.py and dumps what it loaded, for the Python side to check
// against numpy:
//   test_loader host   FILE OUTDIR   decode only (no GPU): every tensor as f32
//   test_loader device FILE OUTDIR   load the layers onto the device and
//                                    download the weights (compute dtype
//                                    bits) and the packed copies
//   test_loader stage FILE OUTDIR S N C C2 DTYPE
//                                    load_decoder_stage(S, N blocks, C -> C2;
//                                    DTYPE bf16 | f16 | f32) and download
//                                    every tensor of the stage as stored on
//                                    the device (stage.<key>.bin), or record
//                                    the refusal in errors.txt
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

static bool dump(const std::string &path, const DeviceTensor &t)
{
    std::vector<uint8_t> b(t.bytes());
    if (!b.empty() && hipMemcpy(b.data(), t.data(), b.size(), hipMemcpyDeviceToHost) != hipSuccess) return false;
    return write_raw(path, b.data(), b.size());
}

// The stage mode: every tensor of the loaded stage under its checkpoint key.
static int run_stage(const SafeTensors &st, const std::string &out, char **argv)
{
    const size_t s = std::stoul(argv[4]), n = std::stoul(argv[5]), c = std::stoul(argv[6]),
                 c2 = std::stoul(argv[7]);
    const std::string dt = argv[8];
    const DType d = dt == "f16" ? DType::F16 : (dt == "f32" ? DType::F32 : DType::BF16);
    auto r = load_decoder_stage(st, s, n, c, c2, true, d);
    std::FILE *errs = std::fopen((out + "/errors.txt").c_str(), "w");
    if (!errs) return 1;
    if (r.is_err()) {
        std::fprintf(errs, "stage: %s\n", r.error().c_str());
        std::fclose(errs);
        std::printf("loader stage refused\n");
        return 0;
    }
    std::fclose(errs);
    const DecoderStageHip &g = r.value();
    bool ok = true;
    auto conv = [&](const std::string &key, const SparseConvLayerHip &L) {
        ok &= dump(out + "/stage." + key + ".weight.bin", L.weight);
        ok &= dump(out + "/stage." + key + ".bias.bin", L.bias);
        if (L.packed) ok &= dump(out + "/stage." + key + ".packed.bin", *L.packed);
    };
    auto lin = [&](const std::string &key, const LinearLayerHip &L) {
        ok &= dump(out + "/stage." + key + ".weight.bin", L.weight);
        ok &= dump(out + "/stage." + key + ".bias.bin", L.bias);
    };
    for (size_t b = 0; b < g.convnext_blocks.size(); ++b) {
        const std::string pre = "blocks." + std::to_string(s) + "." + std::to_string(b);
        const ConvNeXtBlockHip &k = g.convnext_blocks[b];
        conv(pre + ".conv", k.conv);
        ok &= dump(out + "/stage." + pre + ".norm.weight.bin", k.norm_weight);
        ok &= dump(out + "/stage." + pre + ".norm.bias.bin", k.norm_bias);
        lin(pre + ".mlp.0", k.mlp_0);
        lin(pre + ".mlp.2", k.mlp_2);
    }
    if (g.upsample_block) {
        const std::string pre = "blocks." + std::to_string(s) + "." + std::to_string(n);
        const C2SUpsampleBlockHip &u = *g.upsample_block;
        ok &= dump(out + "/stage." + pre + ".norm1.weight.bin", u.norm1_weight);
        ok &= dump(out + "/stage." + pre + ".norm1.bias.bin", u.norm1_bias);
        if (u.to_subdiv) lin(pre + ".to_subdiv", *u.to_subdiv);
        conv(pre + ".conv1", u.conv1);
        conv(pre + ".conv2", u.conv2);
    }
    if (!ok) return 1;
    std::printf("loader stage ok: %zu blocks, upsample %d\n", g.convnext_blocks.size(), g.upsample_block ? 1 : 0);
    return 0;
}

int main(int argc, char **argv)
{
    if (argc != 4 && !(argc == 9 && std::string(argv[1]) == "stage")) {
        std::fprintf(stderr, "usage: %s host|device FILE OUTDIR | stage FILE OUTDIR S N C C2 DTYPE\n", argv[0]);
        return 2;
    }
    const std::string mode = argv[1], path = argv[2], out = argv[3];
    auto st = SafeTensors::open(path);
    if (st.is_err()) {
        std::fprintf(stderr, "open: %s\n", st.error().c_str());
        return 1;
    }
    if (mode == "stage") return run_stage(st.value(), out, argv);
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
