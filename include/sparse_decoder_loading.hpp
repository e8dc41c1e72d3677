// sparse_decoder_loading.hpp -- safetensors loading of the TRELLIS2 sparse
// decoder's conv and linear layers onto the device (header-only C++ over the
// C ABI of sparseconv.h, next to burn_flex_gmm_hip.hpp).
//
// Mirrors crates/burn_trellis/src/runtime_model/sparse_decoder_loading.rs:
//   load_tensor_f32    :231-266  f32 / f16 / bf16 payloads decoded to f32
//                                (other dtypes refused), element count checked
//   load_sparse_conv   :93-200   weight [Cout, KD, KH, KW, Cin_g] + bias [Cout]:
//                                groups from the expected input channels,
//                                the same shape checks and messages
//   load_linear        :1-48     weight [Cout, Cin] + bias [Cout]
//   load_linear_dynamic:50-91    the same, output width taken from the file
//   load_vector        :210-229
//   round_vec_to_f16   :202-208  (the compute_fp16 copies: weights and
//                                biases alike, sparse_decoder.rs:780-793)
// and the per-stage part of SparseStructuredLatentDecoder::from_safetensors
// (sparse_decoder_runtime_impl.rs:94-190): load_decoder_stage reads stage s's
// ConvNeXt blocks blocks.{s}.{b}.{conv, norm, mlp.0, mlp.2} and, unless s is
// the last stage, its C2S upsample blocks.{s}.{N}.{norm1, to_subdiv, conv1,
// conv2}, with the reference's expected shapes.
// The layers land on the device in the compute dtype (f32, bf16 with the
// reference's round-to-nearest-even, or f16), and a conv's weights are packed
// once for the planned conv (sc_conv_weight_pack), the role pack_flex_weight
// plays at load time in the reference (:169-183).
//
// The file format (safetensors): an 8-byte little-endian header length N, a
// JSON header of N bytes {name: {"dtype", "shape", "data_offsets": [begin,
// end]}, "__metadata__": {...}}, then the byte buffer the offsets index.
#ifndef SPARSE_DECODER_LOADING_HPP
#define SPARSE_DECODER_LOADING_HPP

#include <cctype>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <utility>
#include <vector>

#include "burn_flex_gmm_hip.hpp"

namespace burn_flex_gmm_hip {
namespace loading {

struct TensorInfo {
    std::string dtype;  // "F32", "F16", "BF16", ...
    std::vector<size_t> shape;
    size_t begin = 0, end = 0;  // byte range in the data buffer
};

namespace detail {

// A JSON reader for the safetensors header: objects, arrays, strings,
// non-negative integers, true / false / null.  Enough for the header's
// grammar; anything else is an error.
class HeaderParser {
  public:
    explicit HeaderParser(const std::string &s) : s_(s) {}

    bool parse(std::map<std::string, TensorInfo> &out, std::string &err)
    {
        skip();
        if (!eat('{')) return fail(err, "header is not a JSON object");
        skip();
        if (eat('}')) return true;
        for (;;) {
            std::string key;
            if (!string(key)) return fail(err, "expected a tensor name");
            skip();
            if (!eat(':')) return fail(err, "expected ':' after '" + key + "'");
            skip();
            if (key == "__metadata__") {
                if (!skip_value()) return fail(err, "malformed __metadata__");
            } else {
                TensorInfo t;
                if (!tensor(t, err)) return false;
                out[key] = std::move(t);
            }
            skip();
            if (eat(',')) {
                skip();
                continue;
            }
            if (eat('}')) return true;
            return fail(err, "expected ',' or '}' in the header");
        }
    }

  private:
    bool fail(std::string &err, const std::string &m)
    {
        err = "safetensors header: " + m + " (at byte " + std::to_string(i_) + ")";
        return false;
    }
    void skip()
    {
        while (i_ < s_.size() && std::isspace((unsigned char)s_[i_])) ++i_;
    }
    bool eat(char c)
    {
        if (i_ < s_.size() && s_[i_] == c) {
            ++i_;
            return true;
        }
        return false;
    }
    bool string(std::string &out)
    {
        if (!eat('"')) return false;
        out.clear();
        while (i_ < s_.size()) {
            const char c = s_[i_++];
            if (c == '"') return true;
            if (c == '\\') {
                if (i_ >= s_.size()) return false;
                const char e = s_[i_++];
                switch (e) {
                case '"': case '\\': case '/': out += e; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u':  // names are ASCII in practice; keep the escape verbatim
                    if (i_ + 4 > s_.size()) return false;
                    out += "\\u" + s_.substr(i_, 4);
                    i_ += 4;
                    break;
                default: return false;
                }
            } else {
                out += c;
            }
        }
        return false;
    }
    bool integer(size_t &v)
    {
        if (i_ >= s_.size() || !std::isdigit((unsigned char)s_[i_])) return false;
        v = 0;
        while (i_ < s_.size() && std::isdigit((unsigned char)s_[i_])) {
            const size_t d = (size_t)(s_[i_++] - '0');
            if (v > (SIZE_MAX - d) / 10) return false;
            v = v * 10 + d;
        }
        return true;
    }
    bool int_array(std::vector<size_t> &out)
    {
        if (!eat('[')) return false;
        out.clear();
        skip();
        if (eat(']')) return true;
        for (;;) {
            size_t v;
            skip();
            if (!integer(v)) return false;
            out.push_back(v);
            skip();
            if (eat(',')) continue;
            return eat(']');
        }
    }
    bool skip_value()
    {
        skip();
        if (i_ >= s_.size()) return false;
        const char c = s_[i_];
        if (c == '"') {
            std::string tmp;
            return string(tmp);
        }
        if (c == '{' || c == '[') {
            const char close = c == '{' ? '}' : ']';
            ++i_;
            skip();
            if (eat(close)) return true;
            for (;;) {
                if (c == '{') {
                    std::string k;
                    if (!string(k)) return false;
                    skip();
                    if (!eat(':')) return false;
                }
                if (!skip_value()) return false;
                skip();
                if (eat(',')) {
                    skip();
                    continue;
                }
                return eat(close);
            }
        }
        for (const char *w : {"true", "false", "null"})
            if (s_.compare(i_, std::strlen(w), w) == 0) {
                i_ += std::strlen(w);
                return true;
            }
        size_t v;
        return integer(v);
    }
    bool tensor(TensorInfo &t, std::string &err)
    {
        if (!eat('{')) return fail(err, "tensor entry is not an object");
        bool has_dtype = false, has_shape = false, has_offsets = false;
        skip();
        if (!eat('}'))
            for (;;) {
                std::string k;
                skip();
                if (!string(k)) return fail(err, "expected a field name");
                skip();
                if (!eat(':')) return fail(err, "expected ':'");
                skip();
                if (k == "dtype") {
                    if (!string(t.dtype)) return fail(err, "dtype is not a string");
                    has_dtype = true;
                } else if (k == "shape") {
                    if (!int_array(t.shape)) return fail(err, "shape is not an integer array");
                    has_shape = true;
                } else if (k == "data_offsets") {
                    std::vector<size_t> o;
                    if (!int_array(o) || o.size() != 2 || o[1] < o[0]) return fail(err, "bad data_offsets");
                    t.begin = o[0];
                    t.end = o[1];
                    has_offsets = true;
                } else if (!skip_value()) {
                    return fail(err, "malformed field '" + k + "'");
                }
                skip();
                if (eat(',')) continue;
                if (eat('}')) break;
                return fail(err, "expected ',' or '}' in a tensor entry");
            }
        if (!has_dtype || !has_shape || !has_offsets) return fail(err, "tensor entry lacks dtype, shape or data_offsets");
        return true;
    }

    const std::string &s_;
    size_t i_ = 0;
};

inline float f16_bits_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t x;
    if (e == 0x1fu) {
        x = sign | 0x7f800000u | (m << 13);
    } else if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f;  // m * 2^-24, exact
        std::memcpy(&x, &v, 4);
        x |= sign;
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

// f32 -> binary16 bits, round to nearest even, subnormals kept, overflow to
// inf (half::f16::from_f32).
inline uint16_t f32_to_f16_bits(float f)
{
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t e = (x >> 23) & 0xffu, m = x & 0x7fffffu;
    if (e == 0xffu) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u | (m >> 13) : 0u));
    const int32_t E = (int32_t)e - 112;
    if (E >= 31) return (uint16_t)(sign | 0x7c00u);
    if (E <= 0) {
        if (E < -10) return (uint16_t)sign;
        const uint32_t M = m | 0x800000u;
        const int shift = 14 - E;
        uint32_t h = M >> shift;
        const uint32_t rem = M & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) ++h;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)E << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

// bf16_round_to_f32's rule (crates/burn_flex_gmm/src/wgpu.rs:63-66).
inline uint16_t f32_to_bf16_bits(float f)
{
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

}  // namespace detail

// An opened safetensors file (read whole into host memory).
class SafeTensors {
  public:
    static Result<SafeTensors> open(const std::string &path)
    {
        using R = Result<SafeTensors>;
        std::FILE *f = std::fopen(path.c_str(), "rb");
        if (!f) return R::err("cannot open safetensors file '" + path + "'");
        SafeTensors st;
        uint8_t len8[8];
        if (std::fread(len8, 1, 8, f) != 8) {
            std::fclose(f);
            return R::err("safetensors file '" + path + "' is shorter than its 8-byte header length");
        }
        uint64_t n = 0;
        for (int i = 7; i >= 0; --i) n = (n << 8) | len8[i];
        std::fseek(f, 0, SEEK_END);
        const long total = std::ftell(f);
        if (total < 8 || n > (uint64_t)(total - 8)) {
            std::fclose(f);
            return R::err("safetensors header length " + std::to_string(n) + " exceeds the file");
        }
        std::string header((size_t)n, '\0');
        std::fseek(f, 8, SEEK_SET);
        const size_t data_len = (size_t)(total - 8) - (size_t)n;
        st.data_.resize(data_len);
        const bool ok = std::fread(&header[0], 1, (size_t)n, f) == (size_t)n &&
                        (data_len == 0 || std::fread(st.data_.data(), 1, data_len, f) == data_len);
        std::fclose(f);
        if (!ok) return R::err("short read of safetensors file '" + path + "'");
        std::string err;
        detail::HeaderParser p(header);
        if (!p.parse(st.tensors_, err)) return R::err(err);
        for (const auto &kv : st.tensors_)
            if (kv.second.end > data_len)
                return R::err("tensor '" + kv.first + "' data_offsets exceed the buffer");
        return R::ok(std::move(st));
    }

    bool contains(const std::string &key) const { return tensors_.count(key) != 0; }

    Result<TensorInfo> info(const std::string &key) const
    {
        auto it = tensors_.find(key);
        if (it == tensors_.end()) return Result<TensorInfo>::err("missing tensor '" + key + "' in safetensors");
        return Result<TensorInfo>::ok(it->second);
    }

    // load_tensor_f32, sparse_decoder_loading.rs:231-266 (+ bytes_to_f32 /
    // f16 / bf16, :268-310): (shape, values decoded to f32).
    Result<std::pair<std::vector<size_t>, std::vector<float>>> load_tensor_f32(const std::string &key) const
    {
        using R = Result<std::pair<std::vector<size_t>, std::vector<float>>>;
        auto it = tensors_.find(key);
        if (it == tensors_.end()) return R::err("missing tensor '" + key + "' in safetensors");
        const TensorInfo &t = it->second;
        const uint8_t *b = data_.data() + t.begin;
        const size_t nbytes = t.end - t.begin;
        std::vector<float> out;
        if (t.dtype == "F32") {
            if (nbytes % 4) return R::err("invalid f32 tensor payload byte length " + std::to_string(nbytes) +
                                          "; must be divisible by 4");
            out.resize(nbytes / 4);
            for (size_t i = 0; i < out.size(); ++i) {
                uint32_t u = (uint32_t)b[4 * i] | ((uint32_t)b[4 * i + 1] << 8) | ((uint32_t)b[4 * i + 2] << 16) |
                             ((uint32_t)b[4 * i + 3] << 24);
                std::memcpy(&out[i], &u, 4);
            }
        } else if (t.dtype == "F16" || t.dtype == "BF16") {
            if (nbytes % 2)
                return R::err(std::string("invalid ") + (t.dtype == "F16" ? "f16" : "bf16") +
                              " tensor payload byte length " + std::to_string(nbytes) + "; must be divisible by 2");
            out.resize(nbytes / 2);
            for (size_t i = 0; i < out.size(); ++i) {
                const uint16_t h = (uint16_t)(b[2 * i] | (b[2 * i + 1] << 8));
                if (t.dtype == "F16") {
                    out[i] = detail::f16_bits_to_f32(h);
                } else {
                    const uint32_t u = (uint32_t)h << 16;
                    std::memcpy(&out[i], &u, 4);
                }
            }
        } else {
            return R::err("tensor '" + key + "' has unsupported dtype " + t.dtype + "; expected f32/f16/bf16");
        }
        size_t expected = 1;
        for (size_t d : t.shape) {
            if (d != 0 && expected > SIZE_MAX / d) return R::err("tensor '" + key + "' shape product overflow");
            expected *= d;
        }
        if (out.size() != expected)
            return R::err("tensor '" + key + "' element count mismatch: expected " + std::to_string(expected) +
                          ", got " + std::to_string(out.size()));
        return R::ok({t.shape, std::move(out)});
    }

    // load_vector, sparse_decoder_loading.rs:210-229.
    Result<std::vector<float>> load_vector(const std::string &key, size_t expected_len) const
    {
        using R = Result<std::vector<float>>;
        auto r = load_tensor_f32(key);
        if (r.is_err()) return R::err(r.error());
        if (r.value().first.size() != 1)
            return R::err("tensor '" + key + "' expected rank=1, got rank=" + std::to_string(r.value().first.size()));
        if (expected_len > 0 && r.value().first[0] != expected_len)
            return R::err("tensor '" + key + "' expected len=" + std::to_string(expected_len) +
                          ", got len=" + std::to_string(r.value().first[0]));
        return R::ok(std::move(r.value().second));
    }

  private:
    std::vector<uint8_t> data_;
    std::map<std::string, TensorInfo> tensors_;
};

// round_vec_to_f16, sparse_decoder_loading.rs:202-208.
inline std::vector<float> round_vec_to_f16(const std::vector<float> &v)
{
    std::vector<float> out(v.size());
    for (size_t i = 0; i < v.size(); ++i) out[i] = detail::f16_bits_to_f32(detail::f32_to_f16_bits(v[i]));
    return out;
}

// Host values -> a device tensor of the compute dtype (f32 as is; bf16 and
// f16 rounded to nearest even).
inline Result<DeviceTensor> upload_as(const std::vector<float> &v, std::vector<size_t> shape, DType dt,
                                      hipStream_t stream = nullptr)
{
    if (dt == DType::F32) return DeviceTensor::from_host(v.data(), std::move(shape), DType::F32, stream);
    std::vector<uint16_t> h(v.size());
    for (size_t i = 0; i < v.size(); ++i)
        h[i] = dt == DType::F16 ? detail::f32_to_f16_bits(v[i]) : detail::f32_to_bf16_bits(v[i]);
    if (dt != DType::F16 && dt != DType::BF16) return Result<DeviceTensor>::err("upload_as: compute dtype f32/bf16/f16");
    return DeviceTensor::from_host(h.data(), std::move(shape), dt, stream);
}

// A bias on the device, f32: rounded to f16 first for the f16 compute dtype
// (the reference's bias_fp16, sparse_decoder_loading.rs:195 and :38, used
// whenever compute_fp16 is on, sparse_decoder.rs:780-793).
inline Result<DeviceTensor> upload_bias(const std::vector<float> &b, DType compute, hipStream_t stream = nullptr)
{
    if (compute == DType::F16) {
        const std::vector<float> r = round_vec_to_f16(b);
        return DeviceTensor::from_host(r.data(), {b.size()}, DType::F32, stream);
    }
    return DeviceTensor::from_host(b.data(), {b.size()}, DType::F32, stream);
}

// A decoder conv layer on the device: the config, the weight in the
// reference layout [Cout, KD, KH, KW, Cin_g] and its packed copy (16-bit
// compute dtypes with Cin_g a multiple of 32) in the compute dtype, bias f32
// (f16-rounded values for the f16 compute dtype).
struct SparseConvLayerHip {
    SparseSubmConvConfig config;
    DeviceTensor weight;
    std::optional<DeviceTensor> packed;
    DeviceTensor bias;
    std::vector<float> weight_host;  // as loaded (f32), for parity checks
    std::vector<float> bias_host;
};

// load_sparse_conv, sparse_decoder_loading.rs:93-200: the same checks and
// messages; groups = expected_in / Cin_g (Cin_g when expected_in is 0).
inline Result<SparseConvLayerHip> load_sparse_conv(const SafeTensors &st, const std::string &weight_key,
                                                   const std::string &bias_key, size_t expected_in,
                                                   size_t expected_out, DType compute, hipStream_t stream = nullptr)
{
    using R = Result<SparseConvLayerHip>;
    auto w = st.load_tensor_f32(weight_key);
    if (w.is_err()) return R::err(w.error());
    const std::vector<size_t> &ws = w.value().first;
    if (ws.size() != 5)
        return R::err("tensor '" + weight_key + "' expected rank=5, got rank=" + std::to_string(ws.size()));
    const size_t out_channels = ws[0], kd = ws[1], kh = ws[2], kw = ws[3], in_pg = ws[4];
    if (kd == 0 || kh == 0 || kw == 0)
        return R::err("tensor '" + weight_key + "' has invalid kernel dims (" + std::to_string(kd) + "," +
                      std::to_string(kh) + "," + std::to_string(kw) + ")");
    if (in_pg == 0) return R::err("tensor '" + weight_key + "' has invalid in_channels_per_group=0");
    if (expected_out > 0 && out_channels != expected_out)
        return R::err("tensor '" + weight_key + "' expected out_channels=" + std::to_string(expected_out) + ", got " +
                      std::to_string(out_channels));
    const size_t in_channels = expected_in > 0 ? expected_in : in_pg;
    if (in_channels < in_pg || in_channels % in_pg != 0)
        return R::err("tensor '" + weight_key + "' expected_in=" + std::to_string(in_channels) +
                      " is incompatible with in_per_group=" + std::to_string(in_pg));
    const size_t groups = in_channels / in_pg;
    if (groups == 0 || out_channels % groups != 0)
        return R::err("tensor '" + weight_key + "' has incompatible grouped channels (groups=" +
                      std::to_string(groups) + ", out_channels=" + std::to_string(out_channels) + ")");
    auto b = st.load_tensor_f32(bias_key);
    if (b.is_err()) return R::err(b.error());
    if (b.value().first.size() != 1 || b.value().first[0] != out_channels)
        return R::err("tensor '" + bias_key + "' expected shape=[" + std::to_string(out_channels) + "]");

    SparseConvLayerHip layer;
    SparseSubmConvConfig &c = layer.config;
    c.in_channels = in_channels;
    c.out_channels = out_channels;
    c.kernel_d = kd;
    c.kernel_h = kh;
    c.kernel_w = kw;
    c.in_channels_per_group = in_pg;
    c.out_channels_per_group = out_channels / groups;
    c.groups = groups;
    layer.weight_host = std::move(w.value().second);
    layer.bias_host = std::move(b.value().second);
    auto wd = upload_as(layer.weight_host, {out_channels, kd, kh, kw, in_pg}, compute, stream);
    if (wd.is_err()) return R::err(wd.error());
    layer.weight = wd.take();
    auto bd = upload_bias(layer.bias_host, compute, stream);
    if (bd.is_err()) return R::err(bd.error());
    layer.bias = bd.take();
    if ((compute == DType::BF16 || compute == DType::F16) && in_pg % 32 == 0) {
        auto p = pack_conv_weight(c, layer.weight, stream);
        if (p.is_err()) return R::err(p.error());
        const hipError_t e = hipStreamSynchronize(stream);
        if (e != hipSuccess) return R::err(std::string("weight packing sync failed: ") + hipGetErrorString(e));
        layer.packed = p.take();
    }
    return R::ok(std::move(layer));
}

// A decoder linear layer on the device: weight [Cout, Cin] in the compute
// dtype, bias f32.
struct LinearLayerHip {
    size_t in_channels = 0, out_channels = 0;
    DeviceTensor weight;
    DeviceTensor bias;
    std::vector<float> weight_host, bias_host;
};

namespace detail {
// The body of load_linear and load_linear_dynamic (expected_out 0: any).
// f32_weight: the weight stays an f32 operand like the bias (f16-rounded for
// the f16 compute dtype) -- the to_subdiv head, whose skinny linear takes f32.
inline Result<LinearLayerHip> load_linear_impl(const SafeTensors &st, const std::string &weight_key,
                                               const std::string &bias_key, size_t expected_in, size_t expected_out,
                                               DType compute, hipStream_t stream, bool f32_weight = false)
{
    using R = Result<LinearLayerHip>;
    auto w = st.load_tensor_f32(weight_key);
    if (w.is_err()) return R::err(w.error());
    const std::vector<size_t> &ws = w.value().first;
    if (ws.size() != 2)
        return R::err("tensor '" + weight_key + "' expected rank=2, got rank=" + std::to_string(ws.size()));
    const size_t out_channels = ws[0], in_channels = ws[1];
    if (expected_in > 0 && in_channels != expected_in)
        return R::err("tensor '" + weight_key + "' expected in_channels=" + std::to_string(expected_in) + ", got " +
                      std::to_string(in_channels));
    if (expected_out > 0 && out_channels != expected_out)
        return R::err("tensor '" + weight_key + "' expected out_channels=" + std::to_string(expected_out) + ", got " +
                      std::to_string(out_channels));
    auto b = st.load_tensor_f32(bias_key);
    if (b.is_err()) return R::err(b.error());
    if (b.value().first.size() != 1 || b.value().first[0] != out_channels)
        return R::err("tensor '" + bias_key + "' expected shape=[" + std::to_string(out_channels) + "]");
    LinearLayerHip layer;
    layer.in_channels = in_channels;
    layer.out_channels = out_channels;
    layer.weight_host = std::move(w.value().second);
    layer.bias_host = std::move(b.value().second);
    auto wd = f32_weight ? upload_as(compute == DType::F16 ? round_vec_to_f16(layer.weight_host) : layer.weight_host,
                                     {out_channels, in_channels}, DType::F32, stream)
                         : upload_as(layer.weight_host, {out_channels, in_channels}, compute, stream);
    if (wd.is_err()) return R::err(wd.error());
    layer.weight = wd.take();
    auto bd = upload_bias(layer.bias_host, compute, stream);
    if (bd.is_err()) return R::err(bd.error());
    layer.bias = bd.take();
    return R::ok(std::move(layer));
}
}  // namespace detail

// load_linear, sparse_decoder_loading.rs:1-48.
inline Result<LinearLayerHip> load_linear(const SafeTensors &st, const std::string &weight_key,
                                          const std::string &bias_key, size_t expected_in, size_t expected_out,
                                          DType compute, hipStream_t stream = nullptr)
{
    return detail::load_linear_impl(st, weight_key, bias_key, expected_in, expected_out, compute, stream);
}

// load_linear_dynamic, sparse_decoder_loading.rs:50-91: the output width is
// the file's (the ConvNeXt MLP's hidden width).
inline Result<LinearLayerHip> load_linear_dynamic(const SafeTensors &st, const std::string &weight_key,
                                                  const std::string &bias_key, size_t expected_in, DType compute,
                                                  hipStream_t stream = nullptr)
{
    return detail::load_linear_impl(st, weight_key, bias_key, expected_in, 0, compute, stream);
}

// A vector (SafeTensors::load_vector: rank 1, length checked when
// expected_len > 0) uploaded as f32: the LayerNorm affine vectors.
inline Result<DeviceTensor> load_vector_device(const SafeTensors &st, const std::string &key, size_t expected_len,
                                               hipStream_t stream = nullptr)
{
    auto v = st.load_vector(key, expected_len);
    if (v.is_err()) return Result<DeviceTensor>::err(v.error());
    return DeviceTensor::from_host(v.value().data(), {v.value().size()}, DType::F32, stream);
}

// TRELLIS2's sparse ConvNeXt block (sparse_decoder.rs, ConvNeXtBlock):
// conv3x3x3 -> LayerNorm(norm) -> mlp.0 -> SiLU -> mlp.2 -> + x.
struct ConvNeXtBlockHip {
    SparseConvLayerHip conv;
    DeviceTensor norm_weight, norm_bias;
    LinearLayerHip mlp_0, mlp_2;
};

// The C2S upsample block (sparse_decoder.rs, C2SUpsampleBlock): norm1 affine,
// the to_subdiv head (Linear Cin -> 8, weight and bias f32 for
// sc_linear_skinny; absent when pred_subdiv is off),
// conv1 Cin -> 8 Cout on the parents, conv2 Cout -> Cout on the children.
struct C2SUpsampleBlockHip {
    size_t in_channels = 0, out_channels = 0;
    DeviceTensor norm1_weight, norm1_bias;
    std::optional<LinearLayerHip> to_subdiv;
    SparseConvLayerHip conv1, conv2;
};

// One decoder stage: its ConvNeXt blocks, then (all but the last stage) the
// upsample to the next resolution.
struct DecoderStageHip {
    std::vector<ConvNeXtBlockHip> convnext_blocks;
    std::optional<C2SUpsampleBlockHip> upsample_block;
};

// Stage stage_idx of the decoder, sparse_decoder_runtime_impl.rs:94-190:
// num_blocks ConvNeXt blocks at stage_channels (model_channels[s]), then,
// when next_channels > 0 (model_channels[s + 1]; 0 for the last stage),
// the upsample blocks.{s}.{num_blocks}.* to next_channels, its to_subdiv
// head read when pred_subdiv is set (the reference's default).  The same
// keys, expected shapes and messages as the reference; the first failure
// is returned.
inline Result<DecoderStageHip> load_decoder_stage(const SafeTensors &st, size_t stage_idx, size_t num_blocks,
                                                  size_t stage_channels, size_t next_channels, bool pred_subdiv,
                                                  DType compute, hipStream_t stream = nullptr)
{
    using R = Result<DecoderStageHip>;
    DecoderStageHip stage;
    for (size_t b = 0; b < num_blocks; ++b) {
        const std::string pre = "blocks." + std::to_string(stage_idx) + "." + std::to_string(b);
        auto conv = load_sparse_conv(st, pre + ".conv.weight", pre + ".conv.bias", stage_channels, stage_channels,
                                     compute, stream);
        if (conv.is_err()) return R::err(conv.error());
        auto nw = load_vector_device(st, pre + ".norm.weight", stage_channels, stream);
        if (nw.is_err()) return R::err(nw.error());
        auto nb = load_vector_device(st, pre + ".norm.bias", stage_channels, stream);
        if (nb.is_err()) return R::err(nb.error());
        auto m0 = load_linear_dynamic(st, pre + ".mlp.0.weight", pre + ".mlp.0.bias", stage_channels, compute, stream);
        if (m0.is_err()) return R::err(m0.error());
        auto m2 = load_linear_dynamic(st, pre + ".mlp.2.weight", pre + ".mlp.2.bias", 0, compute, stream);
        if (m2.is_err()) return R::err(m2.error());
        stage.convnext_blocks.push_back(
            ConvNeXtBlockHip{conv.take(), nw.take(), nb.take(), m0.take(), m2.take()});
    }
    if (next_channels > 0) {
        const std::string pre = "blocks." + std::to_string(stage_idx) + "." + std::to_string(num_blocks);
        if (next_channels > SIZE_MAX / 8) return R::err("conv1_out channels overflow");
        C2SUpsampleBlockHip up;
        up.in_channels = stage_channels;
        up.out_channels = next_channels;
        if (pred_subdiv) {
            auto ts = detail::load_linear_impl(st, pre + ".to_subdiv.weight", pre + ".to_subdiv.bias",
                                               stage_channels, 8, compute, stream, true);
            if (ts.is_err()) return R::err(ts.error());
            up.to_subdiv = ts.take();
        }
        auto n1w = load_vector_device(st, pre + ".norm1.weight", stage_channels, stream);
        if (n1w.is_err()) return R::err(n1w.error());
        up.norm1_weight = n1w.take();
        auto n1b = load_vector_device(st, pre + ".norm1.bias", stage_channels, stream);
        if (n1b.is_err()) return R::err(n1b.error());
        up.norm1_bias = n1b.take();
        auto c1 = load_sparse_conv(st, pre + ".conv1.weight", pre + ".conv1.bias", stage_channels, 8 * next_channels,
                                   compute, stream);
        if (c1.is_err()) return R::err(c1.error());
        up.conv1 = c1.take();
        auto c2 = load_sparse_conv(st, pre + ".conv2.weight", pre + ".conv2.bias", next_channels, next_channels,
                                   compute, stream);
        if (c2.is_err()) return R::err(c2.error());
        up.conv2 = c2.take();
        stage.upsample_block = std::move(up);
    }
    return R::ok(std::move(stage));
}

}  // namespace loading
}  // namespace burn_flex_gmm_hip

#endif  // SPARSE_DECODER_LOADING_HPP
