// burn_flex_gmm_hip.hpp -- C++ host mirror of burn_flex_gmm's operator API over
// the C ABI of sparseconv.h (header-only; link libsparseconv.so).
//
// Names, argument meaning and error behaviour follow the Rust crate
// (crates/burn_flex_gmm/src/lib.rs and src/wgpu.rs:405-427):
//   SparseSubmConvConfig                      lib.rs:5-17
//   kernel_rows                               lib.rs:59-67
//   build_neighbor_rows                       lib.rs:69-109 (host slices in/out)
//   sparse_subm_conv_forward_flex_precomputed lib.rs:242-375 (host slices in/out)
//   neighbor_rows_tensor_from_coords_tensor   wgpu/neighbor.rs:977-1006 (device tensors)
//   sparse_subm_conv_forward_hip              wgpu/sparse_conv.rs:310-367 (device tensors)
// Errors are Result<T> values carrying the library's message, as the Rust
// functions return Result<T, String>.  Device tensors own their memory
// (hipMalloc / hipFree), as burn tensors do.
#ifndef BURN_FLEX_GMM_HIP_HPP
#define BURN_FLEX_GMM_HIP_HPP

#include <hip/hip_runtime.h>

#include <array>
#include <cstdint>
#include <cstring>
#include <functional>
#include <memory>
#include <numeric>
#include <optional>
#include <string>
#include <utility>
#include <vector>

#include "sparseconv.h"

namespace burn_flex_gmm_hip {

constexpr int32_t INVALID_NEIGHBOR_ROW = SC_INVALID_NEIGHBOR_ROW;

// Result<T, String>.
template <class T>
class Result {
  public:
    static Result ok(T v) { return Result(std::move(v), std::string()); }
    static Result err(std::string e) { return Result(std::nullopt, std::move(e)); }
    bool is_ok() const { return value_.has_value(); }
    bool is_err() const { return !value_.has_value(); }
    const T &value() const { return *value_; }
    T &value() { return *value_; }
    T take() { return std::move(*value_); }
    const std::string &error() const { return error_; }

  private:
    Result(std::optional<T> v, std::string e) : value_(std::move(v)), error_(std::move(e)) {}
    std::optional<T> value_;
    std::string error_;
};

namespace detail {
inline std::string status_message(int rc)
{
    std::string msg = sc_last_error();
    if (msg.empty()) msg = sc_status_string(rc);
    return msg;
}
}  // namespace detail

// SparseSubmConvConfig, lib.rs:5-17.
struct SparseSubmConvConfig {
    size_t in_channels = 0;
    size_t out_channels = 0;
    size_t kernel_d = 3;
    size_t kernel_h = 3;
    size_t kernel_w = 3;
    size_t in_channels_per_group = 0;
    size_t out_channels_per_group = 0;
    size_t groups = 1;
    std::array<size_t, 3> axis_order{0, 1, 2};
    std::array<int32_t, 3> axis_sign{1, 1, 1};

    sc_conv_config to_c() const
    {
        sc_conv_config c{};
        c.in_channels = (int64_t)in_channels;
        c.out_channels = (int64_t)out_channels;
        c.kernel_d = (int64_t)kernel_d;
        c.kernel_h = (int64_t)kernel_h;
        c.kernel_w = (int64_t)kernel_w;
        c.in_channels_per_group = (int64_t)in_channels_per_group;
        c.out_channels_per_group = (int64_t)out_channels_per_group;
        c.groups = (int64_t)groups;
        for (int j = 0; j < 3; ++j) {
            c.axis_order[j] = (int32_t)axis_order[j];
            c.axis_sign[j] = axis_sign[j];
        }
        return c;
    }
};

struct SparseSubmConvWeights {
    const float *weight;  // [Cout, KD, KH, KW, Cin_g]
    size_t weight_len;
    const float *bias;    // [Cout]
    size_t bias_len;
};

// kernel_rows, lib.rs:59-67.
inline Result<size_t> kernel_rows(const SparseSubmConvConfig &config)
{
    const sc_conv_config c = config.to_c();
    int64_t k = 0;
    const int rc = sc_kernel_rows(&c, &k);
    if (rc != SC_OK) return Result<size_t>::err(detail::status_message(rc));
    return Result<size_t>::ok((size_t)k);
}

enum class DType { F32, BF16, I8, I32, U8, F16 };

inline size_t dtype_bytes(DType d)
{
    switch (d) {
    case DType::F32: return 4;
    case DType::BF16: return 2;
    case DType::I8: return 1;
    case DType::I32: return 4;
    case DType::U8: return 1;
    case DType::F16: return 2;
    }
    return 0;
}

inline int to_sc_dtype(DType d)
{
    switch (d) {
    case DType::F32: return SC_DTYPE_F32;
    case DType::BF16: return SC_DTYPE_BF16;
    case DType::I8: return SC_DTYPE_I8;
    case DType::F16: return SC_DTYPE_F16;
    default: return -1;
    }
}

// A contiguous row-major device tensor owning its memory (the primitive of a
// burn device tensor).
class DeviceTensor {
  public:
    DeviceTensor() = default;

    static Result<DeviceTensor> empty(std::vector<size_t> shape, DType dtype)
    {
        DeviceTensor t;
        t.shape_ = std::move(shape);
        t.dtype_ = dtype;
        const size_t bytes = t.bytes();
        void *p = nullptr;
        if (bytes) {
            const hipError_t e = hipMalloc(&p, bytes);
            if (e != hipSuccess)
                return Result<DeviceTensor>::err(std::string("hipMalloc failed: ") + hipGetErrorString(e));
        }
        t.buf_ = std::shared_ptr<void>(p, [](void *q) {
            if (q) (void)hipFree(q);
        });
        return Result<DeviceTensor>::ok(std::move(t));
    }

    static Result<DeviceTensor> from_host(const void *data, std::vector<size_t> shape, DType dtype,
                                          hipStream_t stream = nullptr)
    {
        auto r = empty(std::move(shape), dtype);
        if (r.is_err() || r.value().bytes() == 0) return r;
        const hipError_t e = hipMemcpyAsync(r.value().data(), data, r.value().bytes(),
                                            hipMemcpyHostToDevice, stream);
        if (e == hipSuccess) {
            const hipError_t e2 = hipStreamSynchronize(stream);
            if (e2 != hipSuccess)
                return Result<DeviceTensor>::err(std::string("upload sync failed: ") + hipGetErrorString(e2));
            return r;
        }
        return Result<DeviceTensor>::err(std::string("upload failed: ") + hipGetErrorString(e));
    }

    template <class T>
    Result<std::vector<T>> to_vec(hipStream_t stream = nullptr) const
    {
        if (sizeof(T) != dtype_bytes(dtype_))
            return Result<std::vector<T>>::err("to_vec: element size does not match the dtype");
        std::vector<T> out(numel());
        if (!out.empty()) {
            hipError_t e = hipMemcpyAsync(out.data(), data(), bytes(), hipMemcpyDeviceToHost, stream);
            if (e == hipSuccess) e = hipStreamSynchronize(stream);
            if (e != hipSuccess)
                return Result<std::vector<T>>::err(std::string("download failed: ") + hipGetErrorString(e));
        }
        return Result<std::vector<T>>::ok(std::move(out));
    }

    const std::vector<size_t> &dims() const { return shape_; }
    DType dtype() const { return dtype_; }
    void *data() const { return buf_.get(); }
    size_t numel() const
    {
        return std::accumulate(shape_.begin(), shape_.end(), (size_t)1, std::multiplies<size_t>());
    }
    size_t bytes() const { return numel() * dtype_bytes(dtype_); }

  private:
    std::vector<size_t> shape_;
    DType dtype_ = DType::F32;
    std::shared_ptr<void> buf_;
};

// neighbor_rows_tensor_from_coords_tensor, wgpu/neighbor.rs:977-1006:
// coords [N, 4] i32 -> neighbour rows [N, K] i32 (lowest row on duplicates).
// Reads the device status back once, as the reference reads its bucket
// overflow counter (wgpu/neighbor.rs:859-879).
inline Result<DeviceTensor> neighbor_rows_tensor_from_coords_tensor(const SparseSubmConvConfig &config,
                                                                    const DeviceTensor &coords,
                                                                    hipStream_t stream = nullptr)
{
    using R = Result<DeviceTensor>;
    if (coords.dtype() != DType::I32 || coords.dims().size() != 2 || coords.dims()[1] != 4)
        return R::err("neighbor map coords must be an i32 [N, 4] tensor");
    auto k = kernel_rows(config);
    if (k.is_err()) return R::err(k.error());
    const size_t n = coords.dims()[0];
    auto out = DeviceTensor::empty({n, k.value()}, DType::I32);
    if (out.is_err()) return out;
    size_t ws_bytes = 0;
    int rc = sc_neighbor_map_workspace_size((int64_t)n, &ws_bytes);
    if (rc != SC_OK) return R::err(detail::status_message(rc));
    auto ws = DeviceTensor::empty({ws_bytes}, DType::U8);
    if (ws.is_err()) return R::err(ws.error());
    const sc_conv_config c = config.to_c();
    rc = sc_neighbor_map_build(&c, (const int32_t *)coords.data(), (int64_t)n, (int64_t)n,
                               (int32_t *)out.value().data(), ws.value().data(), ws_bytes, stream);
    if (rc == SC_OK) rc = sc_neighbor_map_check(ws.value().data(), stream);
    if (rc != SC_OK) return R::err(detail::status_message(rc));
    return out;
}

// Conv plan: row order and per-tile halo tables of one neighbour map.  No
// counterpart in the reference's API; it plays the role of its neighbour
// cache (wgpu.rs:349-382): build it once per map and pass it to every conv on
// that map (ConvOptions::plan).
struct ConvPlan {
    DeviceTensor buf;
    size_t n_in = 0, n_q = 0, kernel_rows = 0;
};

inline Result<ConvPlan> build_conv_plan(const SparseSubmConvConfig &config, const DeviceTensor &coords,
                                        const DeviceTensor &neighbor_rows, hipStream_t stream = nullptr)
{
    using R = Result<ConvPlan>;
    if (coords.dtype() != DType::I32 || coords.dims().size() != 2 || coords.dims()[1] != 4)
        return R::err("conv plan coords must be an i32 [N, 4] tensor");
    auto k = kernel_rows(config);
    if (k.is_err()) return R::err(k.error());
    if (neighbor_rows.dtype() != DType::I32 || neighbor_rows.dims().size() != 2 ||
        neighbor_rows.dims()[1] != k.value())
        return R::err("conv plan neighbor_rows must be an i32 [N_q, K] tensor");
    ConvPlan plan;
    plan.n_in = coords.dims()[0];
    plan.n_q = neighbor_rows.dims()[0];
    plan.kernel_rows = k.value();
    size_t bytes = 0;
    int rc = sc_conv_plan_size((int64_t)plan.n_q, (int64_t)plan.kernel_rows, &bytes);
    if (rc != SC_OK) return R::err(detail::status_message(rc));
    auto buf = DeviceTensor::empty({bytes}, DType::U8);
    if (buf.is_err()) return R::err(buf.error());
    plan.buf = buf.take();
    const sc_conv_config c = config.to_c();
    rc = sc_conv_plan_build(&c, (const int32_t *)coords.data(), (int64_t)plan.n_in,
                            (const int32_t *)neighbor_rows.data(), (int64_t)plan.n_q, plan.buf.data(), bytes,
                            stream);
    if (rc != SC_OK) return R::err(detail::status_message(rc));
    return R::ok(std::move(plan));
}

// Weights packed for the planned conv.  No device counterpart in the
// reference; the role of pack_flex_weight (lib.rs:377-426): once per layer.
// weight [Cout, KD, KH, KW, Cin_g] bf16 | i8 -> packed bytes.
inline Result<DeviceTensor> pack_conv_weight(const SparseSubmConvConfig &config, const DeviceTensor &weight,
                                             hipStream_t stream = nullptr)
{
    using R = Result<DeviceTensor>;
    size_t bytes = 0;
    const sc_conv_config c = config.to_c();
    int rc = sc_conv_weight_pack_size(&c, to_sc_dtype(weight.dtype()), &bytes);
    if (rc != SC_OK) return R::err(detail::status_message(rc));
    auto out = DeviceTensor::empty({bytes}, DType::U8);
    if (out.is_err()) return out;
    rc = sc_conv_weight_pack(&c, to_sc_dtype(weight.dtype()), weight.data(), out.value().data(), stream);
    if (rc != SC_OK) return R::err(detail::status_message(rc));
    return out;
}

struct ConvOptions {
    std::optional<DType> out_dtype;         // default: the input dtype
    const DeviceTensor *w_scale = nullptr;  // [Cout] f32, int8 weights only
    const DeviceTensor *residual = nullptr; // [N_q, Cout] in the output dtype
    // Block epilogue (the decoder's conv -> LayerNorm -> SiLU, + residual):
    bool layer_norm = false;
    const DeviceTensor *ln_weight = nullptr;  // [Cout] f32 or none
    const DeviceTensor *ln_bias = nullptr;    // [Cout] f32 or none
    float ln_eps = 1e-6f;
    bool silu = false;
    // Fast path: a plan of this map and the packed weights (both or neither).
    const ConvPlan *plan = nullptr;
    const DeviceTensor *packed_weight = nullptr;
};

// sparse_subm_conv_forward_wgpu, wgpu/sparse_conv.rs:310-367 (same shape rules,
// validate_tensor_shapes :369-473): input [N_in, Cin] f32|bf16, neighbor_rows
// [N_q, K] i32, weight [Cout, KD, KH, KW, Cin_g] (f32 | bf16 | i8), bias [Cout] f32.
inline Result<DeviceTensor> sparse_subm_conv_forward_hip(const SparseSubmConvConfig &config,
                                                         const DeviceTensor &input,
                                                         const DeviceTensor &neighbor_rows,
                                                         const DeviceTensor &weight,
                                                         const DeviceTensor &bias,
                                                         const ConvOptions &opt = {},
                                                         hipStream_t stream = nullptr)
{
    using R = Result<DeviceTensor>;
    auto k = kernel_rows(config);
    if (k.is_err()) return R::err(k.error());
    if (input.dims().size() != 2)
        return R::err("sparse conv input rank mismatch: got " + std::to_string(input.dims().size()) +
                      " expected 2");
    if (neighbor_rows.dims().size() != 2 || neighbor_rows.dtype() != DType::I32)
        return R::err("sparse conv neighbor_rows must be an i32 rank-2 tensor");
    if (input.dims()[1] != config.in_channels)
        return R::err("sparse conv input channel mismatch: got " + std::to_string(input.dims()[1]) +
                      " expected " + std::to_string(config.in_channels));
    if (neighbor_rows.dims()[1] != k.value())
        return R::err("sparse conv neighbor kernel rows mismatch: got " +
                      std::to_string(neighbor_rows.dims()[1]) + " expected " + std::to_string(k.value()));
    const size_t w_expected = config.out_channels * k.value() * config.in_channels_per_group;
    if (weight.numel() != w_expected)
        return R::err("sparse conv weight len mismatch: got " + std::to_string(weight.numel()) +
                      " expected " + std::to_string(w_expected));
    if (bias.dtype() != DType::F32 || bias.numel() != config.out_channels)
        return R::err("sparse conv bias len mismatch: got " + std::to_string(bias.numel()) +
                      " expected " + std::to_string(config.out_channels));
    const DType od = opt.out_dtype ? *opt.out_dtype : input.dtype();
    const size_t n_q = neighbor_rows.dims()[0];
    auto out = DeviceTensor::empty({n_q, config.out_channels}, od);
    if (out.is_err()) return out;
    if ((opt.plan == nullptr) != (opt.packed_weight == nullptr))
        return R::err("sparse conv: a plan and packed weights go together");
    if (opt.plan && (opt.plan->n_q != n_q || opt.plan->n_in != input.dims()[0] ||
                     opt.plan->kernel_rows != k.value()))
        return R::err("sparse conv: the plan was built for another neighbour map");
    const sc_conv_config c = config.to_c();
    sc_conv_epilogue epi{};
    epi.residual = opt.residual ? opt.residual->data() : nullptr;
    epi.layer_norm = opt.layer_norm ? 1 : 0;
    epi.ln_weight = opt.ln_weight ? (const float *)opt.ln_weight->data() : nullptr;
    epi.ln_bias = opt.ln_bias ? (const float *)opt.ln_bias->data() : nullptr;
    epi.ln_eps = opt.ln_eps;
    epi.silu = opt.silu ? 1 : 0;
    // f32 staging for a LayerNorm the conv tile cannot hold (bf16 output, Cout > 128 or groups > 1)
    size_t ws_bytes = 0;
    int wrc = sc_conv_epilogue_workspace_size(&c, to_sc_dtype(input.dtype()), (int64_t)n_q, to_sc_dtype(od), &epi,
                                              &ws_bytes);
    if (wrc != SC_OK) return R::err(detail::status_message(wrc));
    Result<DeviceTensor> ws = DeviceTensor::empty({ws_bytes}, DType::U8);
    if (ws_bytes) {
        if (ws.is_err()) return R::err(ws.error());
        epi.workspace = ws.value().data();
        epi.workspace_bytes = ws_bytes;
    }
    const float *scale = opt.w_scale ? (const float *)opt.w_scale->data() : nullptr;
    const int rc =
        opt.plan ? sc_subm_conv_forward_planned(
                       &c, to_sc_dtype(input.dtype()), input.data(), (int64_t)input.dims()[0],
                       (const int32_t *)neighbor_rows.data(), (int64_t)n_q, to_sc_dtype(weight.dtype()),
                       weight.data(), opt.packed_weight->data(), scale, (const float *)bias.data(), &epi,
                       to_sc_dtype(od), out.value().data(), opt.plan->buf.data(), stream)
                 : sc_subm_conv_forward_fused(&c, to_sc_dtype(input.dtype()), input.data(),
                                              (int64_t)input.dims()[0], (const int32_t *)neighbor_rows.data(),
                                              (int64_t)n_q, to_sc_dtype(weight.dtype()), weight.data(), scale,
                                              (const float *)bias.data(), &epi, to_sc_dtype(od),
                                              out.value().data(), stream);
    if (rc != SC_OK) return R::err(detail::status_message(rc));
    if (ws_bytes) {  // the staging buffer is freed on return: let the conv finish with it first
        const hipError_t e = hipStreamSynchronize(stream);
        if (e != hipSuccess) return R::err(std::string("hipStreamSynchronize failed: ") + hipGetErrorString(e));
    }
    return out;
}

// build_neighbor_rows, lib.rs:69-109: host coords in, host map out (computed on
// the device; duplicates resolve to the lowest row).
inline Result<std::vector<int32_t>> build_neighbor_rows(const SparseSubmConvConfig &config,
                                                        const std::vector<std::array<uint32_t, 4>> &coords)
{
    using R = Result<std::vector<int32_t>>;
    if (coords.size() > (size_t)INT32_MAX) return R::err("sparse conv coord row count exceeds i32::MAX");
    auto k = kernel_rows(config);
    if (k.is_err()) return R::err(k.error());
    if (coords.empty()) return R::ok({});
    std::vector<int32_t> flat(coords.size() * 4);
    for (size_t i = 0; i < coords.size(); ++i)
        for (int j = 0; j < 4; ++j) {
            if (coords[i][j] > (uint32_t)INT32_MAX)
                return R::err("coord value " + std::to_string(coords[i][j]) +
                              " exceeds i32::MAX for device neighbor kernel");
            flat[4 * i + j] = (int32_t)coords[i][j];
        }
    auto dc = DeviceTensor::from_host(flat.data(), {coords.size(), 4}, DType::I32);
    if (dc.is_err()) return R::err(dc.error());
    auto map = neighbor_rows_tensor_from_coords_tensor(config, dc.value());
    if (map.is_err()) return R::err(map.error());
    return map.value().to_vec<int32_t>();
}

// sparse_subm_conv_forward_flex_precomputed, lib.rs:242-375: host slices in,
// host f32 output out (computed on the device in f32).
inline Result<std::vector<float>> sparse_subm_conv_forward_flex_precomputed(
    const SparseSubmConvConfig &config, SparseSubmConvWeights weights, const std::vector<float> &input,
    const std::vector<int32_t> &neighbor_rows)
{
    using R = Result<std::vector<float>>;
    auto k = kernel_rows(config);
    if (k.is_err()) return R::err(k.error());
    if (weights.bias_len != config.out_channels)
        return R::err("sparse conv bias len mismatch: got " + std::to_string(weights.bias_len) +
                      " expected " + std::to_string(config.out_channels));
    if (neighbor_rows.size() % k.value() != 0)
        return R::err("sparse conv neighbor row len mismatch: got " + std::to_string(neighbor_rows.size()) +
                      " expected a multiple of " + std::to_string(k.value()));
    if (input.size() % config.in_channels != 0)
        return R::err("sparse conv input len mismatch: got " + std::to_string(input.size()) +
                      " expected a multiple of " + std::to_string(config.in_channels));
    const size_t rows = neighbor_rows.size() / k.value();
    const size_t input_rows = input.size() / config.in_channels;
    if (input_rows < rows)
        return R::err("sparse conv input row mismatch: got " + std::to_string(input_rows) +
                      " expected at least " + std::to_string(rows));
    if (rows == 0) return R::ok({});
    for (int32_t v : neighbor_rows) {
        if (v == INVALID_NEIGHBOR_ROW) continue;
        if (v < 0) return R::err("sparse conv neighbor row index is negative: " + std::to_string(v));
        if ((size_t)v >= input_rows)
            return R::err("sparse conv neighbor row index out of bounds: " + std::to_string(v) +
                          " >= " + std::to_string(input_rows));
    }
    auto din = DeviceTensor::from_host(input.data(), {input_rows, config.in_channels}, DType::F32);
    auto dmap = DeviceTensor::from_host(neighbor_rows.data(), {rows, k.value()}, DType::I32);
    auto dw = DeviceTensor::from_host(weights.weight, {weights.weight_len}, DType::F32);
    auto db = DeviceTensor::from_host(weights.bias, {weights.bias_len}, DType::F32);
    for (const auto *r : {&din, &dmap, &dw, &db})
        if (r->is_err()) return R::err(r->error());
    auto out = sparse_subm_conv_forward_hip(config, din.value(), dmap.value(), dw.value(), db.value());
    if (out.is_err()) return R::err(out.error());
    return out.value().to_vec<float>();
}

}  // namespace burn_flex_gmm_hip

#endif  // BURN_FLEX_GMM_HIP_HPP
