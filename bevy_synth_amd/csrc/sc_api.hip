// Status plumbing, config helpers and the row-wise block ops (LayerNorm[+SiLU],
// residual add, row gather, C2S skip add, dtype conversion) for gfx950.
#include <cmath>
#include <cstring>
#include <string>

#include "sc_common.hpp"

namespace sc {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int fail(int status, const std::string &msg)
{
    set_error(msg);
    return status;
}

int hip_fail(hipError_t err, const char *what)
{
    return fail(SC_ERR_HIP, std::string(what) + ": " + hipGetErrorString(err));
}

// validate_config, crates/burn_flex_gmm/src/lib.rs:698-725 (same messages).
int validate_config(const sc_conv_config *c)
{
    if (!c) return fail(SC_ERR_NULL, "sparse conv config is NULL");
    if (c->in_channels <= 0 || c->out_channels <= 0)
        return fail(SC_ERR_CONFIG, "sparse conv channel dimensions must be non-zero");
    if (c->kernel_d <= 0 || c->kernel_h <= 0 || c->kernel_w <= 0)
        return fail(SC_ERR_CONFIG, "sparse conv kernel dimensions must be non-zero");
    if (c->groups <= 0) return fail(SC_ERR_CONFIG, "sparse conv groups must be non-zero");
    int64_t t;
    if (!mul_ok(c->in_channels_per_group, c->groups, &t) || t != c->in_channels)
        return fail(SC_ERR_CONFIG, "sparse conv in_channels/group mismatch");
    if (!mul_ok(c->out_channels_per_group, c->groups, &t) || t != c->out_channels)
        return fail(SC_ERR_CONFIG, "sparse conv out_channels/group mismatch");
    bool used[3] = {false, false, false};
    for (int j = 0; j < 3; ++j) {
        int a = c->axis_order[j];
        if (a < 0 || a > 2 || used[a])
            return fail(SC_ERR_CONFIG, "sparse conv axis_order must be a permutation of [0,1,2]");
        used[a] = true;
    }
    int64_t k;
    if (!mul_ok(c->kernel_d, c->kernel_h, &k) || !mul_ok(k, c->kernel_w, &k) || k > INT32_MAX)
        return fail(SC_ERR_OVERFLOW, "sparse conv kernel rows overflow");
    return SC_OK;
}

// ------------------------------------------------------------- kernels

template <typename Tin, typename Tout>
__global__ void convert_kernel(const Tin *__restrict__ in, Tout *__restrict__ out, int64_t n)
{
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        store_from_f32<Tout>(out, i, load_as_f32<Tin>(in, i));
}

template <typename T>
__global__ void silu_kernel(T *x, int64_t n)
{
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float t = load_as_f32<T>(x, i);
        store_from_f32<T>(x, i, silu_f32(t));
    }
}

int silu_inplace(int dtype, void *d, int64_t n, hipStream_t s)
{
    if (n <= 0) return SC_OK;
    const unsigned g = grid_for(n, 256, 8192);
    if (dtype == SC_DTYPE_F32)
        silu_kernel<float><<<g, 256, 0, s>>>((float *)d, n);
    else if (dtype == SC_DTYPE_BF16)
        silu_kernel<uint16_t><<<g, 256, 0, s>>>((uint16_t *)d, n);
    else if (dtype == SC_DTYPE_F16)
        silu_kernel<_Float16><<<g, 256, 0, s>>>((_Float16 *)d, n);
    else
        return fail(SC_ERR_DTYPE, "silu: dtype must be f32, bf16 or f16");
    SC_LAUNCH_CHECK("silu_kernel launch");
    return SC_OK;
}

template <typename T>
__global__ void add_kernel(const T *__restrict__ a, const T *__restrict__ b, T *out, int64_t n)
{
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        store_from_f32<T>(out, i, load_as_f32<T>(a, i) + load_as_f32<T>(b, i));
}

// One wave64 per row, VPL values per lane held in registers (channels <=
// 64*VPL).  Two-pass mean / biased variance in f32, as
// layer_norm_row_stats_kernel (crates/burn_flex_gmm/src/wgpu/ops.rs:162-187)
// and layer_norm_affine_silu_kernel (:418-446); the wave reduction sums in a
// fixed tree order.
// A non-NULL `res` ([rows][channels] in the output dtype) is added after
// SiLU, before the single rounding to the output dtype (the conv block's
// + residual, when the conv could not fuse the row's LayerNorm).
template <typename Tin, typename Tout, int VPL>
__global__ __launch_bounds__(256) void layer_norm_kernel(const Tin *in, int64_t rows, int channels,
                                                         const float *__restrict__ w,
                                                         const float *__restrict__ b, float eps,
                                                         int apply_silu, const Tout *res, Tout *out,
                                                         const uint32_t *gate, const int64_t *row_limit)
{
    if (gate && *gate) return;  // see launch_layer_norm
    if (row_limit && *row_limit < rows) rows = *row_limit > 0 ? *row_limit : 0;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const Tin *x = in + row * channels;
    float v[VPL];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        int j = lane + 64 * i;
        v[i] = j < channels ? load_as_f32<Tin>(x, j) : 0.f;
        s += v[i];
    }
    const float inv_c = 1.0f / (float)channels;
    const float mean = wave_sum(s) * inv_c;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        int j = lane + 64 * i;
        float d = v[i] - mean;
        q += j < channels ? d * d : 0.f;
    }
    const float var = wave_sum(q) * inv_c;
    const float inv_std = rsqrt_f32(var + eps);
    Tout *y = out + row * channels;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        int j = lane + 64 * i;
        if (j < channels) {
            float t = (v[i] - mean) * inv_std;
            if (w) t *= w[j];
            if (b) t += b[j];
            if (apply_silu) t = silu_f32(t);
            if (res) t += load_as_f32<Tout>(res + row * channels, j);
            store_from_f32<Tout>(y, j, t);
        }
    }
}

// Vectorised form for rows of V = channels/VEC 16-byte vectors, V a multiple
// of 8: LPR lanes per row (64/LPR rows per wave), NV vectors per lane, the
// row reductions over the LPR-lane segment (same two-pass f32 statistics).
template <typename Tin>
struct Vec16 {
    static constexpr int N = 16 / (int)sizeof(Tin);
};

template <typename Tin>
__device__ inline void unpack16(const uint4 &u, float *f)
{
    if constexpr (sizeof(Tin) == 4) {
        f[0] = __builtin_bit_cast(float, u.x);
        f[1] = __builtin_bit_cast(float, u.y);
        f[2] = __builtin_bit_cast(float, u.z);
        f[3] = __builtin_bit_cast(float, u.w);
    } else {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = half_lo<Tin>(w[i]);
            f[2 * i + 1] = half_hi<Tin>(w[i]);
        }
    }
}

template <int LPR>
__device__ inline float seg_sum(float v)
{
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// VEC consecutive Tout values (16-byte aligned group) as f32.
template <typename Tout, int VEC>
__device__ inline void load_vec_f32(const Tout *p, float *f)
{
    constexpr int kBytes = VEC * (int)sizeof(Tout);
    if constexpr (kBytes == 16) {
        unpack16<Tout>(*reinterpret_cast<const uint4 *>(p), f);
    } else if constexpr (kBytes == 32) {
        unpack16<Tout>(reinterpret_cast<const uint4 *>(p)[0], f);
        unpack16<Tout>(reinterpret_cast<const uint4 *>(p)[1], f + 4);
    } else {
        static_assert(kBytes == 8 && sizeof(Tout) == 2, "4 16-bit values");
        const uint2 u = *reinterpret_cast<const uint2 *>(p);
        f[0] = half_lo<Tout>(u.x);
        f[1] = half_hi<Tout>(u.x);
        f[2] = half_lo<Tout>(u.y);
        f[3] = half_hi<Tout>(u.y);
    }
}

// NR rows per lane segment, all their loads issued before any statistic, so
// that a wave keeps NR x 1 KB in flight (one row per segment left a 128- or
// 256-channel row kernel at a quarter of HBM bandwidth: latency-bound).
template <typename Tin, typename Tout, int LPR, int NV, int NR>
__global__ __launch_bounds__(256) void layer_norm_vec_kernel(const Tin *in, int64_t rows, int channels,
                                                             const float *__restrict__ w,
                                                             const float *__restrict__ b, float eps,
                                                             int apply_silu, const Tout *res, Tout *out,
                                                             const uint32_t *gate, const int64_t *row_limit)
{
    if (gate && *gate) return;  // see launch_layer_norm
    if (row_limit && *row_limit < rows) rows = *row_limit > 0 ? *row_limit : 0;
    constexpr int VEC = Vec16<Tin>::N;
    constexpr int RPW = 64 / LPR;  // rows per wave and load
    const int lane = threadIdx.x & 63;
    const int seg = lane / LPR, sl = lane % LPR;
    // the wave's NR * RPW consecutive rows; load r covers rows row0 + r RPW + [0, RPW)
    const int64_t row0 = ((int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * (RPW * NR) + seg;
    float v[NR][NV][VEC];
    // the lane's channels are the same in every row: its affine weights once,
    // as 16-byte loads
    float wv[NV][VEC], bv[NV][VEC];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c0 = (sl + i * LPR) * VEC;
#pragma unroll
        for (int e = 0; e < VEC; e += 4) {
            const float4 w4 = w ? *reinterpret_cast<const float4 *>(w + c0 + e) : make_float4(1.f, 1.f, 1.f, 1.f);
            const float4 b4 = b ? *reinterpret_cast<const float4 *>(b + c0 + e) : make_float4(0.f, 0.f, 0.f, 0.f);
            wv[i][e] = w4.x, wv[i][e + 1] = w4.y, wv[i][e + 2] = w4.z, wv[i][e + 3] = w4.w;
            bv[i][e] = b4.x, bv[i][e + 1] = b4.y, bv[i][e + 2] = b4.z, bv[i][e + 3] = b4.w;
        }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int64_t row = row0 + r * RPW;
        const int64_t rr = row < rows ? row : 0;
        const uint4 *x = reinterpret_cast<const uint4 *>(in + rr * channels);
#pragma unroll
        for (int i = 0; i < NV; ++i) unpack16<Tin>(x[sl + i * LPR], v[r][i]);
    }
    const float inv_c = 1.0f / (float)channels;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int64_t row = row0 + r * RPW;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int e = 0; e < VEC; ++e) s += v[r][i][e];
        const float mean = seg_sum<LPR>(s) * inv_c;
        float q = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const float d = v[r][i][e] - mean;
                q += d * d;
            }
        const float inv_std = rsqrt_f32(seg_sum<LPR>(q) * inv_c + eps);
        if (row >= rows) continue;
        Tout *y = out + row * channels;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c0 = (sl + i * LPR) * VEC;
            float t[VEC], rv[VEC];
            if (res) load_vec_f32<Tout, VEC>(res + row * channels + c0, rv);
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                float z = (v[r][i][e] - mean) * inv_std * wv[i][e] + bv[i][e];
                if (apply_silu) z = silu_f32(z);
                if (res) z += rv[e];
                t[e] = z;
            }
            if constexpr (sizeof(Tout) == 2) {
                if constexpr (VEC == 8) {
                    uint4 o;
                    o.x = pack_half2<Tout>(t[0], t[1]);
                    o.y = pack_half2<Tout>(t[2], t[3]);
                    o.z = pack_half2<Tout>(t[4], t[5]);
                    o.w = pack_half2<Tout>(t[6], t[7]);
                    *reinterpret_cast<uint4 *>(y + c0) = o;
                } else {
                    uint2 o;
                    o.x = pack_half2<Tout>(t[0], t[1]);
                    o.y = pack_half2<Tout>(t[2], t[3]);
                    *reinterpret_cast<uint2 *>(y + c0) = o;
                }
            } else {
#pragma unroll
                for (int e = 0; e < VEC; e += 4)
                    *reinterpret_cast<float4 *>(y + c0 + e) = make_float4(t[e], t[e + 1], t[e + 2], t[e + 3]);
            }
        }
    }
}

// Same computation for rows wider than 1024 channels: three passes over the
// row (it stays in L1/L2 between passes).
template <typename Tin, typename Tout>
__global__ __launch_bounds__(256) void layer_norm_wide_kernel(const Tin *in, int64_t rows,
                                                              int channels,
                                                              const float *__restrict__ w,
                                                              const float *__restrict__ b,
                                                              float eps, int apply_silu, const Tout *res,
                                                              Tout *out, const uint32_t *gate,
                                                              const int64_t *row_limit)
{
    if (gate && *gate) return;  // see launch_layer_norm
    if (row_limit && *row_limit < rows) rows = *row_limit > 0 ? *row_limit : 0;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const Tin *x = in + row * channels;
    float s = 0.f;
    for (int j = lane; j < channels; j += 64) s += load_as_f32<Tin>(x, j);
    const float inv_c = 1.0f / (float)channels;
    const float mean = wave_sum(s) * inv_c;
    float q = 0.f;
    for (int j = lane; j < channels; j += 64) {
        float d = load_as_f32<Tin>(x, j) - mean;
        q += d * d;
    }
    const float inv_std = rsqrt_f32(wave_sum(q) * inv_c + eps);
    Tout *y = out + row * channels;
    for (int j = lane; j < channels; j += 64) {
        float t = (load_as_f32<Tin>(x, j) - mean) * inv_std;
        if (w) t *= w[j];
        if (b) t += b[j];
        if (apply_silu) t = silu_f32(t);
        if (res) t += load_as_f32<Tout>(res + row * channels, j);
        store_from_f32<Tout>(y, j, t);
    }
}

// out[a, :] = view[idx[a], :], moving V-sized words; an index outside the
// view yields a zero row (never an out-of-bounds read).
template <typename V>
__global__ void gather_rows_kernel(const V *__restrict__ src, int64_t view_rows, int64_t row_words,
                                   const int32_t *__restrict__ idx, int64_t n_out, V *__restrict__ out)
{
    int64_t total = n_out * row_words;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        int64_t a = e / row_words, w = e - a * row_words;
        int64_t r = idx[a];
        V v{};
        if (r >= 0 && r < view_rows) v = src[r * row_words + w];
        out[e] = v;
    }
}

template <typename T, typename Tp>
__global__ void c2s_skip_add_kernel(T *h, int64_t n, int64_t out_ch, const Tp *__restrict__ parent,
                                    int64_t parent_rows, int64_t parent_ch,
                                    const int32_t *__restrict__ idx, int64_t rep)
{
    const int64_t S = parent_ch / 8;
    int64_t total = n * out_ch;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        int64_t a = e / out_ch, j = e - a * out_ch;
        int64_t li = idx[a];
        if (li < 0 || li >= parent_rows * 8) continue;  // out-of-range index: no skip term
        int64_t p = li >> 3, c = li & 7;
        float s = load_as_f32<Tp>(parent, p * parent_ch + c * S + j / rep);
        store_from_f32<T>(h, e, load_as_f32<T>(h, e) + s);
    }
}

// bf16 output rows, out_ch a multiple of 8, 16-byte aligned: one thread per
// 8-channel vector of h (one 16-byte load and store), 32-bit index math; the
// parent values of the vector's channels are read individually (consecutive
// channels share a parent channel `rep` at a time, so they hit one line).
template <typename Tp>
__global__ void c2s_skip_add_vec_kernel(uint16_t *h, int n, int vpr, const Tp *__restrict__ parent,
                                        int64_t parent_rows, int64_t parent_ch, const int32_t *__restrict__ idx,
                                        int rep)
{
    const int S = (int)(parent_ch / 8);
    const int64_t total = (int64_t)n * vpr;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        const int a = (int)(e / vpr), v = (int)(e - (int64_t)a * vpr);
        const int64_t li = idx[a];
        if (li < 0 || li >= parent_rows * 8) continue;  // out-of-range index: no skip term
        const Tp *pr = parent + (li >> 3) * parent_ch + (li & 7) * S;
        uint4 *hp = reinterpret_cast<uint4 *>(h + (int64_t)e * 8);
        uint4 x = *hp;
        uint32_t w[4] = {x.x, x.y, x.z, x.w};
        const int j0 = 8 * v;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float s0 = load_as_f32<Tp>(pr, (j0 + 2 * u) / rep);
            const float s1 = load_as_f32<Tp>(pr, (j0 + 2 * u + 1) / rep);
            const float lo = bf16_to_f32((uint16_t)(w[u] & 0xFFFFu)) + s0;
            const float hi = bf16_to_f32((uint16_t)(w[u] >> 16)) + s1;
            w[u] = (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
        }
        *hp = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// gate: NULL, or a device word read by every workgroup before anything
// else -- nonzero, the kernel writes nothing (the planned conv's plan status,
// when this kernel normalises what that conv stored).
template <typename Tin, typename Tout>
int launch_layer_norm(const void *in, int64_t rows, int64_t ch, const float *w,
                             const float *b, float eps, int silu, const void *res_, void *out, hipStream_t s,
                             const uint32_t *gate, const int64_t *row_limit)
{
    const unsigned g = grid_for(rows, 4, INT32_MAX);
    const Tin *x = (const Tin *)in;
    Tout *y = (Tout *)out;
    const Tout *res = (const Tout *)res_;
    const int C = (int)ch;
    constexpr int VEC = Vec16<Tin>::N;
    const bool aligned = ((uintptr_t)in % 16 == 0) && ((uintptr_t)out % 16 == 0) && ((uintptr_t)res % 16 == 0) &&
                         ((uintptr_t)w % 16 == 0) && ((uintptr_t)b % 16 == 0);
    if (aligned && C % (VEC * 8) == 0) {
        const int V = C / VEC;  // 16-byte vectors per row, a multiple of 8
        int lpr = 8;
        while (lpr < 64 && V % (lpr * 2) == 0) lpr *= 2;
        const int nv = V / lpr;
        // rows per lane segment: ~4 vectors per lane (8 for f32 rows of one vector per lane)
        const int nr = nv == 1 ? (sizeof(Tin) == 4 ? 8 : 4) : (nv == 2 ? 2 : 1);
        const int64_t rows_per_block = 4 * (64 / lpr) * nr;
        const unsigned gv = grid_for(rows, (int)rows_per_block, INT32_MAX);
#define LN_VEC(L, N, R) \
    layer_norm_vec_kernel<Tin, Tout, L, N, R><<<gv, 256, 0, s>>>(x, rows, C, w, b, eps, silu, res, y, gate, row_limit)
        bool launched = true;
        if (lpr == 8 && nv == 1 && nr == 4) LN_VEC(8, 1, 4);
        else if (lpr == 16 && nv == 1 && nr == 4) LN_VEC(16, 1, 4);
        else if (lpr == 32 && nv == 1 && nr == 4) LN_VEC(32, 1, 4);
        else if (lpr == 64 && nv == 1 && nr == 4) LN_VEC(64, 1, 4);
        else if (lpr == 8 && nv == 1) LN_VEC(8, 1, 8);
        else if (lpr == 16 && nv == 1) LN_VEC(16, 1, 8);
        else if (lpr == 32 && nv == 1) LN_VEC(32, 1, 8);
        else if (lpr == 64 && nv == 1) LN_VEC(64, 1, 8);
        else if (lpr == 64 && nv == 2) LN_VEC(64, 2, 2);
        else if (lpr == 64 && nv == 3) LN_VEC(64, 3, 1);
        else if (lpr == 64 && nv == 4) LN_VEC(64, 4, 1);
        else launched = false;
#undef LN_VEC
        if (launched) {
            SC_LAUNCH_CHECK("layer_norm_vec_kernel launch");
            return SC_OK;
        }
    }
    const int vpl = (C + 63) / 64;
    if (vpl <= 1)
        layer_norm_kernel<Tin, Tout, 1><<<g, 256, 0, s>>>(x, rows, C, w, b, eps, silu, res, y, gate, row_limit);
    else if (vpl <= 2)
        layer_norm_kernel<Tin, Tout, 2><<<g, 256, 0, s>>>(x, rows, C, w, b, eps, silu, res, y, gate, row_limit);
    else if (vpl <= 4)
        layer_norm_kernel<Tin, Tout, 4><<<g, 256, 0, s>>>(x, rows, C, w, b, eps, silu, res, y, gate, row_limit);
    else if (vpl <= 8)
        layer_norm_kernel<Tin, Tout, 8><<<g, 256, 0, s>>>(x, rows, C, w, b, eps, silu, res, y, gate, row_limit);
    else if (vpl <= 16)
        layer_norm_kernel<Tin, Tout, 16><<<g, 256, 0, s>>>(x, rows, C, w, b, eps, silu, res, y, gate, row_limit);
    else
        layer_norm_wide_kernel<Tin, Tout><<<g, 256, 0, s>>>(x, rows, C, w, b, eps, silu, res, y, gate, row_limit);
    SC_LAUNCH_CHECK("layer_norm_kernel launch");
    return SC_OK;
}

// Skinny linear out[r, o] = b[o] + sum_i x[r, i] w[o, i] for Cout <= 8 (the
// C2S to_subdiv head; linear_skinny_kernel, crates/burn_flex_gmm/src/wgpu/
// ops.rs:135-160, which the decoder uses for out_channels <= 8,
// sparse_decoder_wgpu_ops.rs:109-127).  Lane (group g, output o) of a wave
// holds w[o, c0 .. c0+64) in registers per 64-channel chunk and accumulates
// kRows rows of group g (8 groups x kRows = 64 rows per wave pass); the 8
// lanes of a group read the same row slice.  f32 accumulation, chunks and
// channels in increasing order, bias added last.
constexpr int kSkinnyRows = 8;

template <typename Tin>
__global__ __launch_bounds__(256) void linear_skinny_kernel(const Tin *__restrict__ x, int64_t rows, int cin,
                                                            const float *__restrict__ w,
                                                            const float *__restrict__ b, int cout,
                                                            float *__restrict__ out)
{
    const int lane = threadIdx.x & 63;
    const int o = lane & 7, g = lane >> 3;
    const bool live_o = o < cout;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
    const bool vec = cin % 64 == 0;
    for (int64_t base = wave * 64; base < rows; base += nwaves * 64) {
        float acc[kSkinnyRows];
#pragma unroll
        for (int r = 0; r < kSkinnyRows; ++r) acc[r] = 0.f;
        for (int c0 = 0; c0 < cin; c0 += 64) {
            float wr[64];
            const float *wo = w + (int64_t)(live_o ? o : 0) * cin + c0;
#pragma unroll
            for (int i = 0; i < 64; ++i) wr[i] = (live_o && c0 + i < cin) ? wo[i] : 0.f;
#pragma unroll
            for (int r = 0; r < kSkinnyRows; ++r) {
                const int64_t row = base + g * kSkinnyRows + r;
                if (row >= rows) continue;
                const Tin *xr = x + row * cin + c0;
                float a = acc[r];
                if (vec) {
                    constexpr int VEC = 16 / (int)sizeof(Tin);
#pragma unroll
                    for (int v = 0; v < 64 / VEC; ++v) {
                        const uint4 u = reinterpret_cast<const uint4 *>(xr)[v];
                        float f[VEC];
                        if constexpr (sizeof(Tin) == 4) {
                            f[0] = __builtin_bit_cast(float, u.x);
                            f[1] = __builtin_bit_cast(float, u.y);
                            f[2] = __builtin_bit_cast(float, u.z);
                            f[3] = __builtin_bit_cast(float, u.w);
                        } else {
                            const uint32_t q[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                            for (int k = 0; k < 4; ++k) {
                                f[2 * k] = half_lo<Tin>(q[k]);
                                f[2 * k + 1] = half_hi<Tin>(q[k]);
                            }
                        }
#pragma unroll
                        for (int e = 0; e < VEC; ++e) a += f[e] * wr[v * VEC + e];
                    }
                } else {
                    // static indices keep wr in registers (a runtime bound put it in scratch)
#pragma unroll
                    for (int i = 0; i < 64; ++i)
                        if (c0 + i < cin) a += load_as_f32<Tin>(xr, i) * wr[i];
                }
                acc[r] = a;
            }
        }
        if (!live_o) continue;
        const float bo = b ? b[o] : 0.f;
#pragma unroll
        for (int r = 0; r < kSkinnyRows; ++r) {
            const int64_t row = base + g * kSkinnyRows + r;
            if (row < rows) out[row * cout + o] = acc[r] + bo;
        }
    }
}

int layer_norm_rows(int in_dtype, const void *d_in, int64_t rows, int64_t channels, const float *d_w,
                    const float *d_b, float eps, int apply_silu, int out_dtype, const void *d_res, void *d_out,
                    hipStream_t s, const uint32_t *d_gate, const int64_t *d_row_limit)
{
    if (rows < 0 || channels <= 0 || channels > INT32_MAX)
        return fail(SC_ERR_SHAPE, "layer_norm: invalid rows/channels");
    if (rows == 0) return SC_OK;
    if (!d_in || !d_out) return fail(SC_ERR_NULL, "layer_norm: NULL pointer");
#define LN_CASE(DI, TI, DO, TO)                                                                          \
    if (in_dtype == DI && out_dtype == DO)                                                              \
        return launch_layer_norm<TI, TO>(d_in, rows, channels, d_w, d_b, eps, apply_silu, d_res, d_out, s, d_gate, \
                                         d_row_limit);
    LN_CASE(SC_DTYPE_F32, float, SC_DTYPE_F32, float)
    LN_CASE(SC_DTYPE_F32, float, SC_DTYPE_BF16, uint16_t)
    LN_CASE(SC_DTYPE_F32, float, SC_DTYPE_F16, _Float16)
    LN_CASE(SC_DTYPE_BF16, uint16_t, SC_DTYPE_F32, float)
    LN_CASE(SC_DTYPE_BF16, uint16_t, SC_DTYPE_BF16, uint16_t)
    LN_CASE(SC_DTYPE_F16, _Float16, SC_DTYPE_F32, float)
    LN_CASE(SC_DTYPE_F16, _Float16, SC_DTYPE_F16, _Float16)
#undef LN_CASE
    return fail(SC_ERR_DTYPE, "layer_norm: unsupported dtype pair (f32 / bf16 / f16)");
}

// The decoder's post-processing of the to_subdiv logits [rows][8] in place,
// one thread per row: round each logit to f16 and back (quantize_f16 under
// compute_fp16, sparse_decoder_runtime_impl.rs:871-873, host :1205-1207),
// then subtract the row's mean (center_subdivision_logits; row_center_logits,
// sparse_decoder_wgpu_ops.rs:1728-1745: the f32 sum in child order / 8).
__global__ __launch_bounds__(256) void logits_finish_kernel(float *__restrict__ logits, int64_t rows, int round_f16,
                                                           int center)
{
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    float4 *q = reinterpret_cast<float4 *>(logits + r * 8);
    const float4 a = q[0], b = q[1];
    float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    if (round_f16) {
#pragma unroll
        for (int c = 0; c < 8; ++c) v[c] = f16_bits_to_f32(f32_to_f16_bits(v[c]));
    }
    if (center) {
        float sum = 0.f;
#pragma unroll
        for (int c = 0; c < 8; ++c) sum += v[c];
        const float mean = sum / 8.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) v[c] -= mean;
    }
    q[0] = make_float4(v[0], v[1], v[2], v[3]);
    q[1] = make_float4(v[4], v[5], v[6], v[7]);
}

}  // namespace sc

using namespace sc;

extern "C" {

int sc_abi_version(void) { return SC_ABI_VERSION; }

const char *sc_status_string(int s)
{
    switch (s) {
    case SC_OK: return "ok";
    case SC_ERR_CONFIG: return "invalid sparse conv config";
    case SC_ERR_SHAPE: return "shape mismatch";
    case SC_ERR_DTYPE: return "unsupported dtype";
    case SC_ERR_OVERFLOW: return "size overflow";
    case SC_ERR_WORKSPACE: return "workspace too small";
    case SC_ERR_COORD: return "invalid coordinates";
    case SC_ERR_HIP: return "HIP runtime error";
    case SC_ERR_NULL: return "null pointer";
    case SC_ERR_UNSUPPORTED: return "unsupported";
    default: return "unknown status";
    }
}

const char *sc_last_error(void) { return g_last_error.c_str(); }

int sc_validate_config(const sc_conv_config *cfg)
{
    clear_error();
    return validate_config(cfg);
}

int sc_kernel_rows(const sc_conv_config *cfg, int64_t *rows)
{
    clear_error();
    int rc = validate_config(cfg);
    if (rc) return rc;
    if (!rows) return fail(SC_ERR_NULL, "rows out-pointer is NULL");
    *rows = cfg->kernel_d * cfg->kernel_h * cfg->kernel_w;
    return SC_OK;
}

// kernel_layout, crates/burn_flex_gmm/src/lib.rs:727-752.
int sc_kernel_offsets(const sc_conv_config *c, int32_t *offsets, int64_t capacity_rows)
{
    clear_error();
    int rc = validate_config(c);
    if (rc) return rc;
    if (!offsets) return fail(SC_ERR_NULL, "offsets pointer is NULL");
    int64_t K = c->kernel_d * c->kernel_h * c->kernel_w;
    if (capacity_rows < K) return fail(SC_ERR_SHAPE, "offsets capacity below kernel rows");
    const int32_t cd = (int32_t)(c->kernel_d / 2), ch = (int32_t)(c->kernel_h / 2),
                  cw = (int32_t)(c->kernel_w / 2);
    int64_t k = 0;
    for (int64_t kd = 0; kd < c->kernel_d; ++kd)
        for (int64_t kh = 0; kh < c->kernel_h; ++kh)
            for (int64_t kw = 0; kw < c->kernel_w; ++kw, ++k) {
                const int32_t d[3] = {c->axis_sign[0] * ((int32_t)kd - cd),
                                      c->axis_sign[1] * ((int32_t)kh - ch),
                                      c->axis_sign[2] * ((int32_t)kw - cw)};
                int32_t o[3] = {0, 0, 0};
                for (int j = 0; j < 3; ++j) o[c->axis_order[j]] = d[j];
                offsets[3 * k + 0] = o[0];
                offsets[3 * k + 1] = o[1];
                offsets[3 * k + 2] = o[2];
            }
    return SC_OK;
}

int sc_convert(int in_dtype, const void *d_in, int out_dtype, void *d_out, int64_t n,
               sc_stream stream)
{
    clear_error();
    if (n < 0) return fail(SC_ERR_SHAPE, "negative element count");
    if (n == 0) return SC_OK;
    if (!d_in || !d_out) return fail(SC_ERR_NULL, "convert: NULL pointer");
    hipStream_t s = as_stream(stream);
    const unsigned g = grid_for(n, 256, 8192);
    if (in_dtype == SC_DTYPE_F32 && out_dtype == SC_DTYPE_BF16)
        convert_kernel<float, uint16_t><<<g, 256, 0, s>>>((const float *)d_in, (uint16_t *)d_out, n);
    else if (in_dtype == SC_DTYPE_BF16 && out_dtype == SC_DTYPE_F32)
        convert_kernel<uint16_t, float><<<g, 256, 0, s>>>((const uint16_t *)d_in, (float *)d_out, n);
    else if (in_dtype == SC_DTYPE_F32 && out_dtype == SC_DTYPE_F16)
        convert_kernel<float, _Float16><<<g, 256, 0, s>>>((const float *)d_in, (_Float16 *)d_out, n);
    else if (in_dtype == SC_DTYPE_F16 && out_dtype == SC_DTYPE_F32)
        convert_kernel<_Float16, float><<<g, 256, 0, s>>>((const _Float16 *)d_in, (float *)d_out, n);
    else if (in_dtype == out_dtype &&
             (in_dtype == SC_DTYPE_F32 || in_dtype == SC_DTYPE_BF16 || in_dtype == SC_DTYPE_F16)) {
        SC_HIP_CHECK(hipMemcpyAsync(d_out, d_in, (size_t)n * dtype_size(in_dtype),
                                    hipMemcpyDeviceToDevice, s),
                     "convert copy");
        return SC_OK;
    } else
        return fail(SC_ERR_DTYPE, "convert: unsupported dtype pair");
    SC_LAUNCH_CHECK("convert_kernel launch");
    return SC_OK;
}

int sc_add(int dtype, const void *d_a, const void *d_b, int64_t n, void *d_out, sc_stream stream)
{
    clear_error();
    if (n < 0) return fail(SC_ERR_SHAPE, "negative element count");
    if (n == 0) return SC_OK;
    if (!d_a || !d_b || !d_out) return fail(SC_ERR_NULL, "add: NULL pointer");
    hipStream_t s = as_stream(stream);
    const unsigned g = grid_for(n, 256, 8192);
    if (dtype == SC_DTYPE_F32)
        add_kernel<float><<<g, 256, 0, s>>>((const float *)d_a, (const float *)d_b, (float *)d_out, n);
    else if (dtype == SC_DTYPE_BF16)
        add_kernel<uint16_t><<<g, 256, 0, s>>>((const uint16_t *)d_a, (const uint16_t *)d_b,
                                               (uint16_t *)d_out, n);
    else if (dtype == SC_DTYPE_F16)
        add_kernel<_Float16><<<g, 256, 0, s>>>((const _Float16 *)d_a, (const _Float16 *)d_b, (_Float16 *)d_out, n);
    else
        return fail(SC_ERR_DTYPE, "add: dtype must be f32, bf16 or f16");
    SC_LAUNCH_CHECK("add_kernel launch");
    return SC_OK;
}

int sc_layer_norm(int in_dtype, const void *d_in, int64_t rows, int64_t channels, const float *d_w,
                  const float *d_b, float eps, int apply_silu, int out_dtype, void *d_out,
                  sc_stream stream)
{
    clear_error();
    return layer_norm_rows(in_dtype, d_in, rows, channels, d_w, d_b, eps, apply_silu, out_dtype, nullptr, d_out,
                           as_stream(stream));
}

int sc_linear_skinny(int in_dtype, const void *d_x, int64_t rows, int64_t in_channels, const float *d_w,
                     const float *d_b, int64_t out_channels, float *d_out, sc_stream stream)
{
    clear_error();
    if (rows < 0 || in_channels <= 0 || in_channels > INT32_MAX)
        return fail(SC_ERR_SHAPE, "skinny linear: invalid rows/in_channels");
    if (out_channels < 1 || out_channels > 8)
        return fail(SC_ERR_UNSUPPORTED, "skinny linear takes 1..8 output channels");
    if (rows == 0) return SC_OK;
    if (!d_x || !d_w || !d_out) return fail(SC_ERR_NULL, "skinny linear: NULL pointer");
    if ((uintptr_t)d_x % 16 != 0) return fail(SC_ERR_SHAPE, "skinny linear input must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    const unsigned g = grid_for(rows, 4 * 64, 8192);  // 4 waves x 64 rows per block and pass
    if (in_dtype == SC_DTYPE_F32)
        linear_skinny_kernel<float><<<g, 256, 0, s>>>((const float *)d_x, rows, (int)in_channels, d_w, d_b,
                                                     (int)out_channels, d_out);
    else if (in_dtype == SC_DTYPE_BF16)
        linear_skinny_kernel<uint16_t><<<g, 256, 0, s>>>((const uint16_t *)d_x, rows, (int)in_channels, d_w, d_b,
                                                        (int)out_channels, d_out);
    else if (in_dtype == SC_DTYPE_F16)
        linear_skinny_kernel<_Float16><<<g, 256, 0, s>>>((const _Float16 *)d_x, rows, (int)in_channels, d_w, d_b,
                                                        (int)out_channels, d_out);
    else
        return fail(SC_ERR_DTYPE, "skinny linear input must be f32, bf16 or f16");
    SC_LAUNCH_CHECK("linear_skinny_kernel launch");
    return SC_OK;
}

int sc_subdivision_logits_finish(float *d_logits, int64_t rows, int round_f16, int center, sc_stream stream)
{
    clear_error();
    if (rows < 0) return fail(SC_ERR_SHAPE, "subdivision logits: invalid rows");
    if (rows == 0 || (!round_f16 && !center)) return SC_OK;
    if (!d_logits) return fail(SC_ERR_NULL, "subdivision logits: NULL pointer");
    if ((uintptr_t)d_logits % 16 != 0) return fail(SC_ERR_SHAPE, "subdivision logits must be 16-byte aligned");
    logits_finish_kernel<<<grid_for(rows, 256, INT32_MAX), 256, 0, as_stream(stream)>>>(d_logits, rows, round_f16 != 0,
                                                                                     center != 0);
    SC_LAUNCH_CHECK("logits_finish_kernel launch");
    return SC_OK;
}

int sc_gather_rows(int dtype, const void *d_src, int64_t src_rows, int64_t split, int64_t width,
                   const int32_t *d_idx, int64_t n_out, void *d_out, sc_stream stream)
{
    clear_error();
    const size_t ds = dtype_size(dtype);
    if (!ds) return fail(SC_ERR_DTYPE, "gather_rows: unknown dtype");
    if (src_rows < 0 || split <= 0 || width <= 0 || n_out < 0)
        return fail(SC_ERR_SHAPE, "gather_rows: invalid shape");
    if (n_out == 0) return SC_OK;
    if (!d_src || !d_idx || !d_out) return fail(SC_ERR_NULL, "gather_rows: NULL pointer");
    int64_t view_rows;
    if (!mul_ok(src_rows, split, &view_rows)) return fail(SC_ERR_OVERFLOW, "gather_rows overflow");
    hipStream_t s = as_stream(stream);
    const int64_t row_bytes = width * (int64_t)ds;
    const uintptr_t al = (uintptr_t)d_src | (uintptr_t)d_out;
    if (row_bytes % 16 == 0 && al % 16 == 0) {
        int64_t rw = row_bytes / 16;
        gather_rows_kernel<uint4><<<grid_for(n_out * rw, 256, 65536), 256, 0, s>>>(
            (const uint4 *)d_src, view_rows, rw, d_idx, n_out, (uint4 *)d_out);
    } else if (row_bytes % 4 == 0 && al % 4 == 0) {
        int64_t rw = row_bytes / 4;
        gather_rows_kernel<uint32_t><<<grid_for(n_out * rw, 256, 65536), 256, 0, s>>>(
            (const uint32_t *)d_src, view_rows, rw, d_idx, n_out, (uint32_t *)d_out);
    } else {
        gather_rows_kernel<uint8_t><<<grid_for(n_out * row_bytes, 256, 65536), 256, 0, s>>>(
            (const uint8_t *)d_src, view_rows, row_bytes, d_idx, n_out, (uint8_t *)d_out);
    }
    SC_LAUNCH_CHECK("gather_rows_kernel launch");
    return SC_OK;
}

int sc_c2s_skip_add(int dtype, void *d_h, int64_t n, int64_t out_channels, int parent_dtype,
                    const void *d_parent, int64_t parent_rows, int64_t parent_channels,
                    const int32_t *d_idx, sc_stream stream)
{
    clear_error();
    if (n < 0 || out_channels <= 0 || parent_rows < 0 || parent_channels <= 0)
        return fail(SC_ERR_SHAPE, "c2s_skip_add: invalid shape");
    const int64_t S = parent_channels / 8;
    if (parent_channels % 8 != 0 || S == 0 || out_channels % S != 0)
        return fail(SC_ERR_SHAPE, "c2s_skip_add: invalid skip channel ratio (in=" +
                                      std::to_string(parent_channels) +
                                      ", out=" + std::to_string(out_channels) + ")");
    if (n == 0) return SC_OK;
    if (!d_h || !d_parent || !d_idx) return fail(SC_ERR_NULL, "c2s_skip_add: NULL pointer");
    const int64_t rep = out_channels / S;
    hipStream_t s = as_stream(stream);
    if (dtype == SC_DTYPE_BF16 && out_channels % 8 == 0 && (uintptr_t)d_h % 16 == 0 && n <= INT32_MAX &&
        out_channels / 8 <= INT32_MAX && (parent_dtype == SC_DTYPE_BF16 || parent_dtype == SC_DTYPE_F32)) {
        const int vpr = (int)(out_channels / 8);
        const unsigned gv = grid_for(n * vpr, 256, 65536);
        if (parent_dtype == SC_DTYPE_BF16)
            c2s_skip_add_vec_kernel<uint16_t><<<gv, 256, 0, s>>>((uint16_t *)d_h, (int)n, vpr,
                                                                 (const uint16_t *)d_parent, parent_rows,
                                                                 parent_channels, d_idx, (int)rep);
        else
            c2s_skip_add_vec_kernel<float><<<gv, 256, 0, s>>>((uint16_t *)d_h, (int)n, vpr, (const float *)d_parent,
                                                              parent_rows, parent_channels, d_idx, (int)rep);
        SC_LAUNCH_CHECK("c2s_skip_add_vec_kernel launch");
        return SC_OK;
    }
    const unsigned g = grid_for(n * out_channels, 256, 65536);
#define SKIP_LAUNCH(T, TP)                                                                    \
    c2s_skip_add_kernel<T, TP><<<g, 256, 0, s>>>((T *)d_h, n, out_channels, (const TP *)d_parent, \
                                                 parent_rows, parent_channels, d_idx, rep)
    if (dtype == SC_DTYPE_F32 && parent_dtype == SC_DTYPE_F32)
        SKIP_LAUNCH(float, float);
    else if (dtype == SC_DTYPE_F32 && parent_dtype == SC_DTYPE_BF16)
        SKIP_LAUNCH(float, uint16_t);
    else if (dtype == SC_DTYPE_BF16 && parent_dtype == SC_DTYPE_F32)
        SKIP_LAUNCH(uint16_t, float);
    else if (dtype == SC_DTYPE_BF16 && parent_dtype == SC_DTYPE_BF16)
        SKIP_LAUNCH(uint16_t, uint16_t);
    else if (dtype == SC_DTYPE_F16 && parent_dtype == SC_DTYPE_F16)
        SKIP_LAUNCH(_Float16, _Float16);
    else
        return fail(SC_ERR_DTYPE, "c2s_skip_add: dtypes must be f32 or bf16 (or f16 with f16)");
#undef SKIP_LAUNCH
    SC_LAUNCH_CHECK("c2s_skip_add_kernel launch");
    return SC_OK;
}

}  // extern "C"
