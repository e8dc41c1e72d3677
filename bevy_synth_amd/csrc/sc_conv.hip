// Submanifold sparse convolution for gfx950: output-stationary implicit
// gather-GEMM on MFMA.
//
// Replaces the scalar gather-dot kernels of the reference
// (crates/burn_flex_gmm/src/wgpu/sparse_conv_kernels.rs K9-K17: one lane per
// output value re-reading K*Cin inputs and weights from global memory).
//
// Tile = 128 query rows x 128 output channels of one group, 256 threads
// (4 waves in 2x2, each 64x64 = 2x2 MFMA 32x32 blocks).  The reduction runs
// over (kernel offset k, input-channel chunk of 64 bytes):
//   A stage: the 128 neighbour rows map[r, k] of the tile, 64-byte slices,
//            gathered into LDS (zero rows where map = -1);
//   B stage: w[o, k, chunk] for the tile's 128 output channels, read in the
//            reference layout [Cout][K][Cin_g] (Cin-contiguous = the MFMA B
//            operand's K-contiguous column), int8 widened to bf16 exactly.
// Offsets that no row of the tile uses are skipped (a per-tile bitmask built
// from the map block before the main loop).  Double-buffered LDS, one
// barrier per stage; neighbour indices are prefetched one offset ahead.
// bf16 uses v_mfma_f32_32x32x16_bf16, f32 uses v_mfma_f32_32x32x2_f32; both
// accumulate in f32.  Epilogue: * scale[o] (int8) + bias[o] (+ residual).
//
// A scalar kernel (one lane per output value) covers shapes the tile cannot
// take (channel counts that are not multiples of the 64-byte chunk, K > 1024,
// unaligned pointers).
#include "sc_common.hpp"

namespace sc {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kThreads = 256;
constexpr int kChunkBytes = 64;   // bytes of one row's reduction slice per stage
constexpr int kLdsStride = 80;    // padded row pitch in LDS (conflict-free b128 reads)
constexpr int kMaxMaskK = 1024;   // offsets tracked by the per-tile bitmask

struct ConvArgs {
    const void *input;
    const int32_t *map;
    const void *weight;
    const float *w_scale;
    const float *bias;
    const void *residual;
    void *out;
    int64_t n_q;
    int64_t n_in;     // input rows; map entries outside [0, n_in) count as absent
    int64_t cin;      // input row pitch (elements) = in_channels
    int64_t cout;     // output row pitch = out_channels
    int cin_g;
    int cout_g;
    int K;
};

// ------------------------------------------------------------ loaders

template <typename TA>
__device__ inline uint4 load_a_chunk(const TA *input, int64_t cin, int32_t nbr, int64_t col_elem)
{
    if (nbr < 0) return make_uint4(0, 0, 0, 0);  // absent neighbour (or out of range)
    return *reinterpret_cast<const uint4 *>(input + (int64_t)nbr * cin + col_elem);
}

// bf16 / f32 weights: 16 bytes of w[o, k, c0 .. ].
template <typename TW>
__device__ inline uint4 load_w_chunk(const TW *w, int64_t row_elem, bool valid)
{
    if (!valid) return make_uint4(0, 0, 0, 0);
    return *reinterpret_cast<const uint4 *>(w + row_elem);
}

// int8 -> two bf16 words.  |q| <= 128 is exact in bf16.
__device__ inline uint32_t i8pair_to_bf16x2(uint32_t word, int shift)
{
    const float lo = (float)(int8_t)((word >> shift) & 0xff);
    const float hi = (float)(int8_t)((word >> (shift + 8)) & 0xff);
    return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

// Converts 16 int8 into 16 bf16 (two uint4).
__device__ inline void widen_i8x16(uint4 q, uint4 &o0, uint4 &o1)
{
    o0.x = i8pair_to_bf16x2(q.x, 0);
    o0.y = i8pair_to_bf16x2(q.x, 16);
    o0.z = i8pair_to_bf16x2(q.y, 0);
    o0.w = i8pair_to_bf16x2(q.y, 16);
    o1.x = i8pair_to_bf16x2(q.z, 0);
    o1.y = i8pair_to_bf16x2(q.z, 16);
    o1.z = i8pair_to_bf16x2(q.w, 0);
    o1.w = i8pair_to_bf16x2(q.w, 16);
}

__device__ inline int tile_for_block(int b, int G)
{
    // Dispatch assigns workgroup b to XCD b % 8; give each XCD a contiguous
    // range of row tiles so that neighbouring tiles share its L2.
    const int x = b & 7, pos = b >> 3;
    const int q = G >> 3, r = G & 7;
    return x * q + min(x, r) + pos;
}

// ------------------------------------------------------------- MFMA tile

template <typename TA, typename TW, typename TO>
__global__ __launch_bounds__(kThreads, 2) void conv_mfma_kernel(ConvArgs args)
{
    constexpr bool kF32 = sizeof(TA) == 4;
    constexpr int kBK = kChunkBytes / (int)sizeof(TA);  // elements per stage
    constexpr bool kI8 = sizeof(TW) == 1;

    __shared__ __attribute__((aligned(16))) unsigned char s_a[2][kBM * kLdsStride];
    __shared__ __attribute__((aligned(16))) unsigned char s_b[2][kBN * kLdsStride];
    __shared__ uint32_t s_kmask[kMaxMaskK / 32];
    __shared__ int16_t s_klist[kMaxMaskK];
    __shared__ int s_nk;

    const TA *input = static_cast<const TA *>(args.input);
    const TW *weight = static_cast<const TW *>(args.weight);
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int K = args.K;

    const int tile = tile_for_block(blockIdx.x, gridDim.x);
    const int64_t row0 = (int64_t)tile * kBM;
    const int o0 = blockIdx.y * kBN;            // within the group
    const int g = blockIdx.z;
    const int64_t in_col0 = (int64_t)g * args.cin_g;
    const int64_t out_col0 = (int64_t)g * args.cout_g;
    const int nrows = (int)min<int64_t>(kBM, args.n_q - row0);

    // ---- which offsets does this tile use?
    for (int i = tid; i < (K + 31) / 32; i += kThreads) s_kmask[i] = 0;
    __syncthreads();
    const int32_t *map_tile = args.map + row0 * K;
    for (int e = tid; e < nrows * K; e += kThreads) {
        const int32_t v = map_tile[e];
        if (v >= 0 && v < args.n_in) {
            const int k = e % K;
            atomicOr(&s_kmask[k >> 5], 1u << (k & 31));
        }
    }
    __syncthreads();
    if (tid == 0) {
        int nk = 0;
        for (int k = 0; k < K; ++k)
            if (s_kmask[k >> 5] & (1u << (k & 31))) s_klist[nk++] = (int16_t)k;
        s_nk = nk;
    }
    __syncthreads();
    const int nk = s_nk;
    const int nkc = args.cin_g / kBK;  // chunks per offset
    const int S = nk * nkc;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    if (S > 0) {
        // A: thread owns rows ra and ra+64, 16-byte part pa of the 64-byte slice.
        const int ra = tid >> 2, pa = tid & 3;
        const bool va0 = ra < nrows, va1 = ra + 64 < nrows;
        const int64_t a_col = in_col0 + pa * (16 / (int)sizeof(TA));
        // B (bf16/f32): output channels ra and ra+64, part pa.
        // B (int8): output channel tid>>1, 16-int8 half (tid&1).
        const int ob = kI8 ? (tid >> 1) : ra;
        const bool vb0 = o0 + ob < args.cout_g;
        const bool vb1 = !kI8 && (o0 + ob + 64 < args.cout_g);
        const int64_t w_row0 = ((out_col0 + o0 + ob) * (int64_t)K) * args.cin_g;
        const int64_t w_row1 = ((out_col0 + o0 + ob + 64) * (int64_t)K) * args.cin_g;
        const int b_part_elems = kI8 ? (tid & 1) * 16 : pa * (16 / (int)sizeof(TW));

        const int64_t n_in = args.n_in;
        auto load_nbr = [&](int k, int32_t &n0, int32_t &n1) {
            n0 = va0 ? map_tile[(int64_t)ra * K + k] : -1;
            n1 = va1 ? map_tile[(int64_t)(ra + 64) * K + k] : -1;
            if (n0 >= n_in) n0 = -1;
            if (n1 >= n_in) n1 = -1;
        };

        int32_t nb0, nb1, nn0 = -1, nn1 = -1;
        load_nbr(s_klist[0], nb0, nb1);
        if (nk > 1) load_nbr(s_klist[1], nn0, nn1);

        uint4 ra0, ra1, rb0, rb1;
        auto issue_loads = [&](int k, int kc) {
            const int64_t c = a_col + (int64_t)kc * kBK;
            ra0 = load_a_chunk<TA>(input, args.cin, nb0, c);
            ra1 = load_a_chunk<TA>(input, args.cin, nb1, c);
            const int64_t wc = (int64_t)k * args.cin_g + (int64_t)kc * kBK + b_part_elems;
            rb0 = load_w_chunk<TW>(weight, w_row0 + wc, vb0);
            if (!kI8) rb1 = load_w_chunk<TW>(weight, w_row1 + wc, vb1);
        };
        auto store_lds = [&](int buf) {
            unsigned char *a = s_a[buf];
            *reinterpret_cast<uint4 *>(a + ra * kLdsStride + pa * 16) = ra0;
            *reinterpret_cast<uint4 *>(a + (ra + 64) * kLdsStride + pa * 16) = ra1;
            unsigned char *b = s_b[buf];
            if (kI8) {
                uint4 w0, w1;
                widen_i8x16(rb0, w0, w1);
                *reinterpret_cast<uint4 *>(b + ob * kLdsStride + (tid & 1) * 32) = w0;
                *reinterpret_cast<uint4 *>(b + ob * kLdsStride + (tid & 1) * 32 + 16) = w1;
            } else {
                *reinterpret_cast<uint4 *>(b + ra * kLdsStride + pa * 16) = rb0;
                *reinterpret_cast<uint4 *>(b + (ra + 64) * kLdsStride + pa * 16) = rb1;
            }
        };

        issue_loads(s_klist[0], 0);
        store_lds(0);
        __syncthreads();

        int ki_next = 0, kc_next = 0;  // decoded (offset index, chunk) of stage s+1
        const int arow = wm * 64 + (lane & 31);
        const int brow = wn * 64 + (lane & 31);
        const int half = lane >> 5;
        for (int s = 0; s < S; ++s) {
            const bool more = s + 1 < S;
            if (more) {
                if (++kc_next == nkc) {
                    kc_next = 0;
                    ++ki_next;
                    nb0 = nn0;
                    nb1 = nn1;
                    if (ki_next + 1 < nk) load_nbr(s_klist[ki_next + 1], nn0, nn1);
                }
                issue_loads(s_klist[ki_next], kc_next);
            }
            const unsigned char *a = s_a[s & 1];
            const unsigned char *b = s_b[s & 1];
            if constexpr (!kF32) {
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const int off = kk * 32 + half * 16;
                    bf16x8 af[2], bfr[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i)
                        af[i] = __builtin_bit_cast(
                            bf16x8, *reinterpret_cast<const uint4 *>(a + (arow + i * 32) * kLdsStride + off));
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        bfr[j] = __builtin_bit_cast(
                            bf16x8, *reinterpret_cast<const uint4 *>(b + (brow + j * 32) * kLdsStride + off));
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
                }
            } else {
                // Lane half h holds k-elements h*8 .. h*8+7 of the 16-float slice;
                // step kk multiplies element kk of each half.
                float af[2][8], bfr[2][8];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const float4 *p = reinterpret_cast<const float4 *>(a + (arow + i * 32) * kLdsStride + half * 32);
                    const float4 x0 = p[0], x1 = p[1];
                    af[i][0] = x0.x; af[i][1] = x0.y; af[i][2] = x0.z; af[i][3] = x0.w;
                    af[i][4] = x1.x; af[i][5] = x1.y; af[i][6] = x1.z; af[i][7] = x1.w;
                }
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float4 *p = reinterpret_cast<const float4 *>(b + (brow + j * 32) * kLdsStride + half * 32);
                    const float4 x0 = p[0], x1 = p[1];
                    bfr[j][0] = x0.x; bfr[j][1] = x0.y; bfr[j][2] = x0.z; bfr[j][3] = x0.w;
                    bfr[j][4] = x1.x; bfr[j][5] = x1.y; bfr[j][6] = x1.z; bfr[j][7] = x1.w;
                }
#pragma unroll
                for (int kk = 0; kk < 8; ++kk)
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][kk], bfr[j][kk], acc[i][j], 0, 0, 0);
            }
            if (more) store_lds((s + 1) & 1);
            __syncthreads();
        }
    }

    // ---- epilogue.  32x32 MFMA result layout: lane l, element e ->
    //      row 8*(e/4) + 4*(l/32) + e%4, column l%32.
    TO *out = static_cast<TO *>(args.out);
    const TO *res = static_cast<const TO *>(args.residual);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int oc = o0 + wn * 64 + j * 32 + (lane & 31);
        if (oc >= args.cout_g) continue;
        const int64_t o = out_col0 + oc;
        const float bias = args.bias ? args.bias[o] : 0.f;
        const float scale = (kI8 && args.w_scale) ? args.w_scale[o] : 1.f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int r = wm * 64 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (r < nrows) {
                    const int64_t idx = (row0 + r) * args.cout + o;
                    float v = kI8 ? acc[i][j][e] * scale + bias : acc[i][j][e] + bias;
                    if (res) v += load_as_f32<TO>(res, idx);
                    store_from_f32<TO>(out, idx, v);
                }
            }
    }
}

// ------------------------------------------------------------ scalar path

template <typename TA, typename TW, typename TO>
__global__ __launch_bounds__(256) void conv_scalar_kernel(ConvArgs args)
{
    const TA *input = static_cast<const TA *>(args.input);
    const TW *weight = static_cast<const TW *>(args.weight);
    TO *out = static_cast<TO *>(args.out);
    const TO *res = static_cast<const TO *>(args.residual);
    const int64_t total = args.n_q * args.cout;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        const int64_t r = e / args.cout, o = e - r * args.cout;
        const int64_t g = o / args.cout_g;
        float acc = 0.f;
        for (int k = 0; k < args.K; ++k) {
            const int32_t nb = args.map[r * args.K + k];
            if (nb < 0 || nb >= args.n_in) continue;
            const TA *a = input + (int64_t)nb * args.cin + g * args.cin_g;
            const TW *w = weight + (o * args.K + k) * args.cin_g;
            float part = 0.f;
            for (int i = 0; i < args.cin_g; ++i) {
                float wv;
                if constexpr (sizeof(TW) == 1)
                    wv = (float)w[i];
                else
                    wv = load_as_f32<TW>(w, i);
                part += load_as_f32<TA>(a, i) * wv;
            }
            acc += part;
        }
        if constexpr (sizeof(TW) == 1) acc *= args.w_scale ? args.w_scale[o] : 1.f;
        float v = acc + (args.bias ? args.bias[o] : 0.f);
        if (res) v += load_as_f32<TO>(res, e);
        store_from_f32<TO>(out, e, v);
    }
}

template <typename TA, typename TW, typename TO>
int launch_conv(const ConvArgs &a, int groups, bool mfma, hipStream_t s)
{
    if (mfma) {
        const int64_t tiles = (a.n_q + kBM - 1) / kBM;
        const int64_t ntile = (a.cout_g + kBN - 1) / kBN;
        if (tiles > INT32_MAX || ntile > 65535 || groups > 65535)
            return fail(SC_ERR_OVERFLOW, "sparse conv grid overflow");
        dim3 grid((unsigned)tiles, (unsigned)ntile, (unsigned)groups);
        conv_mfma_kernel<TA, TW, TO><<<grid, kThreads, 0, s>>>(a);
        SC_LAUNCH_CHECK("conv_mfma_kernel launch");
    } else {
        conv_scalar_kernel<TA, TW, TO><<<grid_for(a.n_q * a.cout, 256, 65536), 256, 0, s>>>(a);
        SC_LAUNCH_CHECK("conv_scalar_kernel launch");
    }
    return SC_OK;
}

}  // namespace
}  // namespace sc

using namespace sc;

extern "C" int sc_subm_conv_forward(const sc_conv_config *cfg, int act_dtype, const void *d_input,
                                    int64_t n_in, const int32_t *d_map, int64_t n_q, int w_dtype,
                                    const void *d_weight, const float *d_w_scale,
                                    const float *d_bias, const void *d_residual, int out_dtype,
                                    void *d_out, sc_stream stream)
{
    clear_error();
    int rc = validate_config(cfg);
    if (rc) return rc;
    if (n_in < 0 || n_q < 0) return fail(SC_ERR_SHAPE, "negative row count");
    if (n_q > n_in)
        return fail(SC_ERR_SHAPE, "sparse conv neighbor row count exceeds input rows: got " +
                                      std::to_string(n_q) + " input rows " + std::to_string(n_in));
    const bool act_bf16 = act_dtype == SC_DTYPE_BF16, act_f32 = act_dtype == SC_DTYPE_F32;
    if (!(act_bf16 || act_f32)) return fail(SC_ERR_DTYPE, "sparse conv input dtype must be f32 or bf16");
    if (act_f32 && w_dtype != SC_DTYPE_F32)
        return fail(SC_ERR_DTYPE, "sparse conv f32 input needs f32 weights");
    if (act_bf16 && w_dtype != SC_DTYPE_BF16 && w_dtype != SC_DTYPE_I8)
        return fail(SC_ERR_DTYPE, "sparse conv bf16 input needs bf16 or int8 weights");
    if (out_dtype != SC_DTYPE_F32 && out_dtype != SC_DTYPE_BF16)
        return fail(SC_ERR_DTYPE, "sparse conv output dtype must be f32 or bf16");
    if (w_dtype == SC_DTYPE_I8 && !d_w_scale)
        return fail(SC_ERR_NULL, "int8 weights need per-output-channel scales");
    const int64_t K = cfg->kernel_d * cfg->kernel_h * cfg->kernel_w;
    int64_t t;
    if (!mul_ok(n_q, K, &t) || !mul_ok(n_q, cfg->out_channels, &t) ||
        !mul_ok(n_in, cfg->in_channels, &t) || !mul_ok(cfg->out_channels, K, &t) ||
        !mul_ok(t, cfg->in_channels_per_group, &t))
        return fail(SC_ERR_OVERFLOW, "sparse conv size overflow");
    if (cfg->in_channels_per_group > INT32_MAX || cfg->out_channels_per_group > INT32_MAX)
        return fail(SC_ERR_OVERFLOW, "sparse conv channel count overflow");
    if (n_q == 0) return SC_OK;
    if (!d_input || !d_map || !d_weight || !d_out) return fail(SC_ERR_NULL, "sparse conv: NULL pointer");

    ConvArgs a;
    a.input = d_input;
    a.map = d_map;
    a.weight = d_weight;
    a.w_scale = d_w_scale;
    a.bias = d_bias;
    a.residual = d_residual;
    a.out = d_out;
    a.n_q = n_q;
    a.n_in = n_in;
    a.cin = cfg->in_channels;
    a.cout = cfg->out_channels;
    a.cin_g = (int)cfg->in_channels_per_group;
    a.cout_g = (int)cfg->out_channels_per_group;
    a.K = (int)K;

    const size_t asz = dtype_size(act_dtype);
    const int bk = kChunkBytes / (int)asz;
    const uintptr_t align = (uintptr_t)d_input | (uintptr_t)d_weight;
    const bool mfma = (a.cin_g % bk == 0) && K <= kMaxMaskK && (align % 16 == 0);
    const int groups = (int)cfg->groups;
    hipStream_t s = as_stream(stream);
    if (act_f32) {
        if (out_dtype == SC_DTYPE_F32) return launch_conv<float, float, float>(a, groups, mfma, s);
        return launch_conv<float, float, uint16_t>(a, groups, mfma, s);
    }
    if (w_dtype == SC_DTYPE_BF16) {
        if (out_dtype == SC_DTYPE_F32) return launch_conv<uint16_t, uint16_t, float>(a, groups, mfma, s);
        return launch_conv<uint16_t, uint16_t, uint16_t>(a, groups, mfma, s);
    }
    if (out_dtype == SC_DTYPE_F32) return launch_conv<uint16_t, int8_t, float>(a, groups, mfma, s);
    return launch_conv<uint16_t, int8_t, uint16_t>(a, groups, mfma, s);
}
