// Shared helpers for the gfx950 sparse-conv library: status/error plumbing,
// bf16 conversion, wave reductions and launch checks.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/sparseconv.h"

namespace sc {

// ---------------------------------------------------------------- errors
void set_error(const std::string &msg);
void clear_error();
int fail(int status, const std::string &msg);
int hip_fail(hipError_t err, const char *what);

#define SC_HIP_CHECK(expr, what)                                  \
    do {                                                          \
        hipError_t _e = (expr);                                   \
        if (_e != hipSuccess) return ::sc::hip_fail(_e, (what));  \
    } while (0)

// Launch check: catches launch-configuration errors without synchronising.
#define SC_LAUNCH_CHECK(what)                                      \
    do {                                                           \
        hipError_t _e = hipGetLastError();                         \
        if (_e != hipSuccess) return ::sc::hip_fail(_e, (what));   \
    } while (0)

int validate_config(const sc_conv_config *cfg);
// In-place x / (1 + exp(-x)) over n values (f32 or bf16); stream-ordered.
int silu_inplace(int dtype, void *d, int64_t n, hipStream_t s);
// Row LayerNorm (+ SiLU) (+ a residual in the output dtype, added before the
// one rounding to the output dtype); d_res may be NULL.  Stream-ordered.
// d_gate: NULL, or a device word that, when nonzero as the kernel starts,
// makes it write nothing (a planned conv's plan status).
int layer_norm_rows(int in_dtype, const void *d_in, int64_t rows, int64_t channels, const float *d_w,
                    const float *d_b, float eps, int apply_silu, int out_dtype, const void *d_res, void *d_out,
                    hipStream_t s, const uint32_t *d_gate = nullptr, const int64_t *d_row_limit = nullptr);

inline bool mul_ok(int64_t a, int64_t b, int64_t *out)
{
    if (a < 0 || b < 0) return false;
    if (a != 0 && b > INT64_MAX / a) return false;
    *out = a * b;
    return true;
}

inline size_t dtype_size(int dt)
{
    switch (dt) {
    case SC_DTYPE_F32: return 4;
    case SC_DTYPE_BF16: return 2;
    case SC_DTYPE_I8: return 1;
    case SC_DTYPE_F16: return 2;
    default: return 0;
    }
}

inline hipStream_t as_stream(sc_stream s) { return reinterpret_cast<hipStream_t>(s); }

inline unsigned grid_for(int64_t n, int block, int64_t max_blocks = 1 << 20)
{
    int64_t g = (n + block - 1) / block;
    if (g < 1) g = 1;
    if (g > max_blocks) g = max_blocks;
    return static_cast<unsigned>(g);
}

// ------------------------------------------------------------ bf16 bits
// Round-to-nearest-even f32 -> bf16, no NaN special case: the rule of
// bf16_round_to_f32 (crates/burn_flex_gmm/src/wgpu.rs:63-66).
__host__ __device__ inline uint16_t f32_to_bf16(float f)
{
    uint32_t b = __builtin_bit_cast(uint32_t, f);
    uint32_t lsb = (b >> 16) & 1u;
    return static_cast<uint16_t>((b + 0x7fffu + lsb) >> 16);
}

__host__ __device__ inline float bf16_to_f32(uint16_t h)
{
    return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
}

// ------------------------------------------------------------ f16 bits
// IEEE binary16 storage is _Float16 (bf16 storage is uint16_t).  f32 -> f16
// is v_cvt_f16_f32 in the default round-to-nearest-even mode, subnormals
// kept: the rounding of half::f16::from_f32 / burn's F16 cast that the
// reference's f16 fences apply (sparse_decoder_wgpu_ops.rs:1082-1088,
// 1722-1726).
typedef _Float16 f16_t;

__device__ inline uint16_t f32_to_f16_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ inline float f16_bits_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

template <typename T> __device__ inline float load_as_f32(const T *p, int64_t i);
template <> __device__ inline float load_as_f32<float>(const float *p, int64_t i) { return p[i]; }
template <> __device__ inline float load_as_f32<uint16_t>(const uint16_t *p, int64_t i)
{
    return bf16_to_f32(p[i]);
}
template <> __device__ inline float load_as_f32<_Float16>(const _Float16 *p, int64_t i) { return (float)p[i]; }

template <typename T> __device__ inline void store_from_f32(T *p, int64_t i, float v);
template <> __device__ inline void store_from_f32<float>(float *p, int64_t i, float v) { p[i] = v; }
template <> __device__ inline void store_from_f32<uint16_t>(uint16_t *p, int64_t i, float v)
{
    p[i] = f32_to_bf16(v);
}
template <> __device__ inline void store_from_f32<_Float16>(_Float16 *p, int64_t i, float v) { p[i] = (_Float16)v; }

// Two 16-bit values (bf16 or f16 by T) of a 32-bit word -> f32, and back.
template <typename T> __device__ inline float half_lo(uint32_t w)
{
    if constexpr (sizeof(T) == 2 && !__is_same(T, uint16_t)) return f16_bits_to_f32((uint16_t)(w & 0xffffu));
    else return bf16_to_f32((uint16_t)(w & 0xffffu));
}
template <typename T> __device__ inline float half_hi(uint32_t w)
{
    if constexpr (sizeof(T) == 2 && !__is_same(T, uint16_t)) return f16_bits_to_f32((uint16_t)(w >> 16));
    else return bf16_to_f32((uint16_t)(w >> 16));
}
template <typename T> __device__ inline uint32_t pack_half2(float lo, float hi)
{
    if constexpr (__is_same(T, uint16_t))
        return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
    else
        return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
}

// ---------------------------------------------------- kernel offsets
// Offset k of a KD x KH x KW kernel: k = (kd*KH + kh)*KW + kw, deltas
// sign_j * (idx_j - dim_j/2) written to axis order[j]
// (crates/burn_flex_gmm/src/lib.rs:727-752).
struct KernelShape {
    int K, KD, KH, KW;
    int order[3];
    int sign[3];
};

inline KernelShape kernel_shape(const sc_conv_config *cfg)
{
    KernelShape ks;
    ks.KD = (int)cfg->kernel_d;
    ks.KH = (int)cfg->kernel_h;
    ks.KW = (int)cfg->kernel_w;
    ks.K = ks.KD * ks.KH * ks.KW;
    for (int j = 0; j < 3; ++j) {
        ks.order[j] = cfg->axis_order[j];
        ks.sign[j] = cfg->axis_sign[j];
    }
    return ks;
}

__device__ inline void offset_of(const KernelShape &ks, int k, int o[3])
{
    const int hw = ks.KH * ks.KW;
    const int kd = k / hw, rem = k - kd * hw;
    const int kh = rem / ks.KW, kw = rem - kh * ks.KW;
    const int d[3] = {ks.sign[0] * (kd - ks.KD / 2), ks.sign[1] * (kh - ks.KH / 2),
                      ks.sign[2] * (kw - ks.KW / 2)};
    // o[order[j]] = d[j], written as selections (no computed local address)
    for (int a = 0; a < 3; ++a)
        o[a] = ks.order[0] == a ? d[0] : (ks.order[1] == a ? d[1] : (ks.order[2] == a ? d[2] : 0));
}

// ---------------------------------------------------- buffer loads
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Buffer loads: an offset at or beyond the descriptor's byte count reads as
// zero, which is how absent neighbours, rows outside the input and channels
// beyond Cout contribute nothing without a branch.
constexpr uint32_t kOobOffset = 0xC0000000u;

__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// The same buffer resource as make_rsrc as four raw words (base address low
// 32 bits, high 16 bits with stride 0, size in bytes, the same format word),
// for the inline-asm DMA below.
typedef int32_t i32x4_rsrc __attribute__((ext_vector_type(4)));
__device__ inline i32x4_rsrc rsrc_words(const void *base, uint32_t bytes)
{
    const uint64_t a = (uint64_t)(uintptr_t)base;
    return i32x4_rsrc{(int32_t)(uint32_t)a, (int32_t)((a >> 32) & 0xFFFF), (int32_t)bytes, 0x00020000};
}

// One LDS DMA: lane L loads 16 bytes at byte offset voff of the buffer
// (zero when out of range) into LDS bytes [lds + 16 L, +16); lds is uniform
// (it goes to m0; the s_nop covers the m0-write-to-DMA hazard).  Written as
// inline asm because the compiler, which cannot separate the DMA's LDS
// writes from reads of other buffers, otherwise waits for every pending DMA
// before each LDS read.  The compiler does not count these loads: the caller
// waits for them (s_waitcnt vmcnt) before reading what they wrote, and
// before the wave's end.
__device__ inline void lds_dma16(i32x4_rsrc rsrc, uint32_t voff, uint32_t lds)
{
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(lds)
                 : "memory");
}

__device__ inline uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ inline uint2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    return make_uint2(v.x, v.y);
}

__device__ inline uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

// ---------------------------------------------------- activations
// SiLU x * sigmoid(x) = x / (1 + e^-x) on the hardware exponential and
// reciprocal (v_exp_f32 computes 2^y, so e^-x = 2^(-x log2 e); each is
// accurate to about 1 ulp, far below the bf16 / f32 tolerances of the path).
// Large negative x: 2^y overflows to +inf, the reciprocal gives 0 and the
// result -0; large positive x: 2^y underflows to 0 and the result is x.
__device__ inline float silu_f32(float x)
{
    constexpr float kLog2e = 1.4426950408889634f;
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

// 1 / sqrt(x) on the hardware reciprocal square root (about 1 ulp).
__device__ inline float rsqrt_f32(float x) { return __builtin_amdgcn_rsqf(x); }

// ---------------------------------------------------- wave64 reductions
__device__ inline float wave_sum(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ inline int wave_min_i32(int v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = min(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ inline int wave_max_i32(int v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
    return v;
}

// Octree levels of the row-order test below: C2S subdivision emits children
// parent-major, child index ascending, so after L subdivisions below a set
// sorted in (b, x, y, z) the rows are strictly increasing in the key
// (lexicographic index of coords >> L) * 8^L + octree digits of the low L
// bits (coarsest level most significant, a digit x | y << 1 | z << 2).  The
// neighbour map's rank bitmap and the conv plan's row order use it.
constexpr int kRankLevels = 8;

// Bit L set unless a precedes c strictly in the L-level key, for every L <
// kRankLevels, without building the keys.  With h_a the highest bit in which
// the two coords differ along axis a (-1: equal), the root cells (coords >>
// L) differ along x exactly for L <= h_x, and the key order is then the
// order of x; failing that along y for L <= h_y, then z; with equal roots the
// most significant differing octree digit is the one at bit max(h_x, h_y,
// h_z), and within a digit z weighs most, then y, then x.  So the levels
// split into four ranges, each taking one comparison.  (Host and device:
// tests/cpp/test_order_levels.cpp checks it against the keys themselves.)
__host__ __device__ inline int high_bit(uint32_t v) { return v ? 31 - __builtin_clz(v) : -1; }

// Levels 0 .. h as a mask (empty for h < 0, all for h >= kRankLevels - 1).
__host__ __device__ inline uint32_t levels_upto(int h)
{
    constexpr uint32_t kAll = (1u << kRankLevels) - 1u;
    return h < 0 ? 0u : (h >= kRankLevels - 1 ? kAll : (2u << h) - 1u);
}

__host__ __device__ inline uint32_t unsorted_levels(const int4 a, const int4 c)
{
    constexpr uint32_t kAll = (1u << kRankLevels) - 1u;
    if (a.x != c.x) return a.x < c.x ? 0u : kAll;  // batch
    const int hx = high_bit((uint32_t)(a.y ^ c.y)), hy = high_bit((uint32_t)(a.z ^ c.z)),
              hz = high_bit((uint32_t)(a.w ^ c.w));
    const uint32_t rx = levels_upto(hx);            // x roots differ
    const uint32_t ry = levels_upto(hy) & ~rx;      // else y roots differ
    const uint32_t rz = levels_upto(hz) & ~rx & ~ry;
    const uint32_t rd = kAll & ~rx & ~ry & ~rz;     // equal roots: the digits decide
    const int p = hx > hy ? (hx > hz ? hx : hz) : (hy > hz ? hy : hz);
    const bool digit_less = p >= 0 && (hz == p ? a.w < c.w : (hy == p ? a.z < c.z : a.y < c.y));
    const uint32_t less = (a.y < c.y ? rx : 0u) | (a.z < c.z ? ry : 0u) | (a.w < c.w ? rz : 0u) |
                          (digit_less ? rd : 0u);
    return kAll & ~less;
}

__device__ inline int tile_for_block(int b, int G)
{
    // Dispatch assigns workgroup b to XCD b % 8; give each XCD a contiguous
    // range of row tiles so that neighbouring tiles share its L2.
    const int x = b & 7, pos = b >> 3;
    const int q = G >> 3, r = G & 7;
    return x * q + min(x, r) + pos;
}

}  // namespace sc
