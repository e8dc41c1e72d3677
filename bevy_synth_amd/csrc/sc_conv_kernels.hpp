// Kernels of the submanifold sparse conv, included by sc_conv.hip (the f32
// and bf16 forms), sc_conv_i8.hip (int8 weights) and sc_conv_f16.hip (f16);
// each translation unit keeps its instantiations to itself.
// The argument block, tile constants and packed-weight header are shared.
#pragma once

#include "sc_common.hpp"
#include "sc_plan.hpp"

namespace sc {


typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kTileRows = 256;  // query rows per workgroup (64 per wave)
constexpr int kBN = 128;        // output channels per workgroup
constexpr int kThreads = 256;
constexpr int kChunkBytes = 64;   // smallest per-stage reduction slice of a row (bytes)
constexpr int kMaxTableK = 32;    // MFMA tile: kernels with at most 32 offsets

struct ConvArgs {
    const void *input;
    const int32_t *map;  // [n_q][K]; NULL only for the dense linear (K = 1, query row r reads row r)
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
    int vec_out;      // 4-channel packed output stores allowed (counts and pointers aligned)
    // Fused epilogue (order: + bias -> LayerNorm over the row -> SiLU -> + residual).
    // LayerNorm needs every channel of a row in one workgroup (groups == 1, Cout <= 128).
    int ln;
    const float *ln_w;
    const float *ln_b;
    float ln_eps;
    int silu;
    // Optional row order (a permutation of [0, n_q), padded with -1 to whole
    // tiles): tile row p computes query row perm[p].
    const int32_t *perm;
    // Weights packed by sc_conv_weight_pack (the halo-staged kernel's layout),
    // starting with their PackHeader.
    const void *wpack;
    // Header of the plan a planned launch reads (the dense kernel's linear
    // child plan checks it against the call's shape before anything else).
    const PlanHeader *plan_hdr;
    // LayerNorm over consecutive groups of ln_group channels: the row's
    // Cout, or one child's scatter_ch (64 or 128) in the C2S scatter.
    int ln_group;
    // C2S forms of the decoder's upsample block (NULL otherwise).  Child
    // scatter (conv1): query row r's channels [c*scatter_ch, (c+1)*scatter_ch)
    // go to output row scatter_rows[8r + c] (a child row; -1 or >= scatter_n:
    // dropped), pitch scatter_ch.
    const int32_t *scatter_rows;
    int64_t scatter_n;
    int scatter_ch;
    // Channel-repeated parent skip (conv2): value (r, o) += parent[li >> 3]
    // [(li & 7) * skip_S + o / skip_R], li = skip_idx[r], parent in the
    // output dtype.
    const void *skip_parent;
    const int32_t *skip_idx;
    int64_t skip_parent_rows;
    int64_t skip_parent_ch;
    int skip_S;
    int skip_R;
    int scatter_shift;  // log2(scatter_ch), or -1 when not a power of two
    int skip_shift;     // log2(skip_R), or -1 when not a power of two
    // Child plan (C2S conv1 over the active children only): the plan's tiles
    // each belong to one child c, tile_child[t], and compute its output
    // channels [c * child_ch, (c + 1) * child_ch); child_plan marks the call.
    const int32_t *tile_child;
    int child_ch;
    int child_plan;
};

// Header of a packed weight buffer (its first 256 bytes): the shape the
// weights were packed for.  The planned conv compares it with the call's
// config before it reads a fragment.
constexpr uint32_t kPackMagic = 0x31574353u;  // "SCW1"
constexpr size_t kPackHeaderBytes = 256;
struct alignas(16) PackHeader {
    uint32_t magic;
    int32_t groups;
    int32_t cout_g;
    int32_t cin_g;
    int32_t K;
    int32_t src_dtype;  // SC_DTYPE_BF16 or SC_DTYPE_I8
    int32_t n_ot;       // 128-channel output tiles per group
    int32_t pad0;
    int64_t bytes;      // whole buffer, header included
    uint32_t pad[54];
};
static_assert(sizeof(PackHeader) == kPackHeaderBytes, "pack header size");

namespace {

// A plan built for this call's map shape (n_q, n_in, K)?
__device__ inline bool plan_matches(const PlanHeader *h, const ConvArgs &a)
{
    return h->n_q == a.n_q && h->n_in == a.n_in && h->K == a.K;
}

// Records a mismatch in the plan's status (first workgroup only; the caller
// reads it with sc_conv_plan_check).
__device__ inline void flag_plan_status(const PlanHeader *h, uint32_t bits)
{
    if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x == 0)
        atomicOr(const_cast<uint32_t *>(&h->status), bits);
}

// ------------------------------------------------------------ loaders

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

// A fragments of one 32-row block for one stage: NP 16-byte pieces of the
// gathered row's CB-byte slice.  Piece q of lane half h sits at byte
// bf16: q*32 + h*16 (one MFMA k-step per piece); f32: h*CB/2 + q*16 (4
// consecutive k-elements per piece).
template <int NP>
struct APiece {
    uint4 p[NP];
};

template <bool kF32, int CB>
__device__ inline int piece_offset(int q, int half)
{
    return kF32 ? half * (CB / 2) + q * 16 : q * 32 + half * 16;
}


template <bool kF32, int CB>
__device__ inline APiece<CB / 32> load_a_pieces(__amdgpu_buffer_rsrc_t r, uint32_t row_off, int kc,
                                                 int half)
{
    APiece<CB / 32> a;
#pragma unroll
    for (int q = 0; q < CB / 32; ++q)
        a.p[q] = bload16(r, row_off + (uint32_t)(kc * CB + piece_offset<kF32, CB>(q, half)));
    return a;
}

__device__ inline float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// One piece of one 32x32 output block, computed transposed: the weight
// fragment w (32 output channels) is the MFMA A operand and the gathered
// input fragment x (32 voxel rows) the B operand, so D[o][r] = sum_k w[o][k]
// x[r][k] and a lane ends up holding 4 consecutive output channels of one
// row (packed stores in the epilogue).  bf16 -> one v_mfma_f32_32x32x16_bf16;
// f32 -> four v_mfma_f32_32x32x2_f32 (element e of each lane half's piece).
template <bool kF32>
__device__ inline void mfma_piece(f32x16 &acc, const uint4 &x, const uint4 &w)
{
    if constexpr (!kF32) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, w),
                                                      __builtin_bit_cast(bf16x8, x), acc, 0, 0, 0);
    } else {
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(u2f(w.x), u2f(x.x), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(u2f(w.y), u2f(x.y), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(u2f(w.z), u2f(x.z), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(u2f(w.w), u2f(x.w), acc, 0, 0, 0);
    }
}

// Packs / unpacks 4 consecutive output values.
template <typename TO>
struct Out4;
template <>
struct Out4<float> {
    typedef float4 V;
    static __device__ inline V pack(const float *v) { return make_float4(v[0], v[1], v[2], v[3]); }
    static __device__ inline void unpack(const V &u, float *v)
    {
        v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
    }
};
template <>
struct Out4<uint16_t> {
    typedef uint2 V;
    static __device__ inline V pack(const float *v)
    {
        return make_uint2((uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16),
                          (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16));
    }
    static __device__ inline void unpack(const V &u, float *v)
    {
        v[0] = bf16_to_f32((uint16_t)(u.x & 0xffffu));
        v[1] = bf16_to_f32((uint16_t)(u.x >> 16));
        v[2] = bf16_to_f32((uint16_t)(u.y & 0xffffu));
        v[3] = bf16_to_f32((uint16_t)(u.y >> 16));
    }
};

template <>
struct Out4<_Float16> {
    typedef uint2 V;
    static __device__ inline V pack(const float *v)
    {
        return make_uint2(pack_half2<_Float16>(v[0], v[1]), pack_half2<_Float16>(v[2], v[3]));
    }
    static __device__ inline void unpack(const V &u, float *v)
    {
        v[0] = half_lo<_Float16>(u.x);
        v[1] = half_hi<_Float16>(u.x);
        v[2] = half_lo<_Float16>(u.y);
        v[3] = half_hi<_Float16>(u.y);
    }
};

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// One 16x16x32 MFMA step on 16-bit operands: bf16 (TA = uint16_t) or f16
// (TA = _Float16), f32 accumulation either way.
template <typename TA>
__device__ inline f32x4 mfma_16x16x32(const uint4 &a, const uint4 &b, const f32x4 &c)
{
    if constexpr (__is_same(TA, _Float16))
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
}

// C2S epilogue stores (child scatter of conv1, parent skip of conv2).  Per
// output row, c2s_row reads the row's linear index once and keeps the parent
// slice it adds; c2s_store4 then writes channels [col, col + nv) (nv <= 4,
// col a multiple of 4 within the output row whenever nv == 4) with 32-bit
// index arithmetic and shifts for the power-of-two child widths and repeat
// factors of the decoder.
struct C2SRow {
    const void *skip_row;  // parent slice added to this row, or NULL
};

template <typename TO>
__device__ inline C2SRow c2s_row(const ConvArgs &a, int64_t qrow)
{
    C2SRow c{nullptr};
    if (a.skip_idx) {
        const int32_t li = a.skip_idx[qrow];
        if (li >= 0 && (int64_t)li < a.skip_parent_rows * 8)
            c.skip_row = static_cast<const TO *>(a.skip_parent) + (int64_t)(li >> 3) * a.skip_parent_ch +
                         (int64_t)(li & 7) * a.skip_S;
    }
    return c;
}

// kSharedSkip: the one-load form of repeat factors >= 4 (left out of the
// LayerNorm kernels, whose register budget it exceeds; the decoder's parent
// skip follows a conv without LayerNorm).
template <typename TO, bool kSharedSkip = true>
__device__ inline void c2s_store4(const ConvArgs &a, const C2SRow &c, int64_t qrow, int col, int nv, const float *v,
                                  bool vec)
{
    TO *out = static_cast<TO *>(a.out);
    int64_t base;
    if (a.scatter_rows) {
        const int ch = a.scatter_shift >= 0 ? col >> a.scatter_shift : col / a.scatter_ch;
        const int32_t r = a.scatter_rows[qrow * 8 + ch];
        if (r < 0 || r >= a.scatter_n) return;
        base = (int64_t)r * a.scatter_ch + (col - ch * a.scatter_ch);
    } else {
        base = qrow * a.cout + col;
    }
    float t[4] = {v[0], nv > 1 ? v[1] : 0.f, nv > 2 ? v[2] : 0.f, nv > 3 ? v[3] : 0.f};
    if (c.skip_row) {
        const TO *pp = static_cast<const TO *>(c.skip_row);
        if (kSharedSkip && nv == 4 && a.skip_shift >= 2) {
            // repeat factor >= 4: the 4 channels (col % 4 == 0) add one parent value
            const float sv = load_as_f32<TO>(pp, col >> a.skip_shift);
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) t[cc] += sv;
        } else {
#pragma unroll
            for (int cc = 0; cc < 4; ++cc)
                if (cc < nv)
                    t[cc] += load_as_f32<TO>(pp, a.skip_shift >= 0 ? (col + cc) >> a.skip_shift : (col + cc) / a.skip_R);
        }
    }
    if (vec && nv == 4) {
        *reinterpret_cast<typename Out4<TO>::V *>(out + base) = Out4<TO>::pack(t);
    } else {
#pragma unroll
        for (int cc = 0; cc < 4; ++cc)
            if (cc < nv) store_from_f32<TO>(out, base + cc, t[cc]);
    }
}

// ------------------------------------------------------------- MFMA tile

// Per-tile list of kernel offsets (K <= 32) used by at least one row of the
// tile: per-thread bit masks OR-reduced across the wave, one LDS atomic per
// wave, then a serial compaction by thread 0.
__device__ inline int build_offset_list(const int32_t *map_tile, int nrows, int K, int64_t n_in,
                                        uint32_t *s_kmask, int16_t *s_klist, int *s_nk)
{
    const int tid = threadIdx.x, lane = tid & 63;
    for (int i = tid; i < (K + 31) / 32; i += blockDim.x) s_kmask[i] = 0;
    __syncthreads();
    {
        // The tile's map block is contiguous: read it as int4, four loads in
        // flight per thread before any is inspected.
        uint32_t m = 0;
        const int total = nrows * K;
        const int4 *m4 = reinterpret_cast<const int4 *>(map_tile);
        const int n4 = total >> 2;
        for (int base = tid; base < n4; base += 4 * (int)blockDim.x) {
            int4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i4 = base + u * (int)blockDim.x;
                v[u] = i4 < n4 ? m4[i4] : make_int4(-1, -1, -1, -1);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int e = 4 * (base + u * (int)blockDim.x);
                const int32_t vv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (vv[c] >= 0 && vv[c] < n_in) m |= 1u << ((e + c) % K);
            }
        }
        for (int e = 4 * n4 + tid; e < total; e += blockDim.x) {
            const int32_t v = map_tile[e];
            if (v >= 0 && v < n_in) m |= 1u << (e % K);
        }
        uint32_t lo = (uint32_t)m;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) lo |= __shfl_xor(lo, off, 64);
        if (lane == 0 && lo) atomicOr(&s_kmask[0], lo);
    }
    __syncthreads();
    if (tid == 0) {
        int nk = 0;
        for (int k = 0; k < K; ++k)
            if (s_kmask[k >> 5] & (1u << (k & 31))) s_klist[nk++] = (int16_t)k;
        *s_nk = nk;
    }
    __syncthreads();
    return *s_nk;
}


// LDS table of the byte offsets (in the input) of the neighbour rows of the
// tile: s_aoff[ki][r] for used offset ki and tile row r (thread r fills row r);
// kOobOffset for an absent neighbour or a row past the end.
__device__ inline void fill_row_offsets(const int32_t *map_tile, int nrows, int K, int64_t n_in,
                                        uint32_t row_bytes, const int16_t *s_klist, int nk,
                                        uint32_t (*s_aoff)[kTileRows])
{
    const int r = threadIdx.x;  // kThreads == kTileRows
    const int32_t *mrow = map_tile + (int64_t)min(r, nrows - 1) * K;
    for (int k0 = 0; k0 < nk; k0 += 8) {
        int32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = k0 + u < nk ? mrow[s_klist[k0 + u]] : -1;
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (k0 + u < nk)
                s_aoff[k0 + u][r] =
                    (r < nrows && v[u] >= 0 && v[u] < n_in) ? (uint32_t)v[u] * row_bytes : kOobOffset;
    }
    __syncthreads();
}

// Tile = 256 query rows x 128 output channels of one group; 4 waves, wave w
// owns rows [64w, 64w+64) x all 128 channels (2 x 4 MFMA 32x32 blocks, 128
// f32 accumulators per lane).  CB = bytes of a row's reduction slice per
// stage (64 or 128); a stage is (used offset ki, input chunk kc).
//
// Prologue: the offsets used by the tile, then an LDS table of the byte
// offsets of every (used offset, row) neighbour row in the input (an
// out-of-range offset for absent neighbours), so the main loop issues no map
// loads.  Main loop: a two-half software pipeline with no branches -- each
// half issues the next stage's weight loads (-> LDS after the MFMAs) and A
// loads (-> the other register set), then runs this stage's MFMAs.  The
// stage count is padded to even with a zero-weight stage.
template <typename TA, typename TW, typename TO, int CB>
__global__ __launch_bounds__(kThreads, 2) void conv_mfma_kernel(ConvArgs args)
{
    constexpr bool kF32 = sizeof(TA) == 4;
    constexpr int kBK = CB / (int)sizeof(TA);  // reduction elements per stage
    constexpr bool kI8 = sizeof(TW) == 1;
    constexpr int kRows = kTileRows;
    constexpr int NP = CB / 32;                 // A/B pieces per lane per row block
    constexpr int kStride = CB + 16;            // LDS pitch of one output channel
    constexpr int kWBytes = kBK * (int)sizeof(TW);  // weight bytes per channel per stage
    constexpr int kWPieces = kWBytes / 16;      // 16-byte weight pieces per channel
    constexpr int kBPerThread = kBN * kWPieces / kThreads;
    static_assert(kBPerThread >= 1, "weight pieces per thread");

    __shared__ __attribute__((aligned(16))) unsigned char s_b[2][kBN * kStride];
    __shared__ uint32_t s_aoff[kMaxTableK][kRows];
    __shared__ uint32_t s_kmask[kMaxTableK / 32 + 1];
    __shared__ int16_t s_klist[kMaxTableK];
    __shared__ int s_nk;

    const TA *input = static_cast<const TA *>(args.input);
    const TW *weight = static_cast<const TW *>(args.weight);
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, half = lane >> 5;
    const int K = args.K;

    const int tile = tile_for_block(blockIdx.x, gridDim.x);
    const int64_t row0 = (int64_t)tile * kRows;
    const int o0 = blockIdx.y * kBN;  // within the group
    const int g = blockIdx.z;
    const int64_t in_col0 = (int64_t)g * args.cin_g;
    const int64_t out_col0 = (int64_t)g * args.cout_g;
    const int nrows = (int)min<int64_t>(kRows, args.n_q - row0);
    const int32_t *map_tile = args.map ? args.map + row0 * K : nullptr;
    const int64_t n_in = args.n_in;
    const uint32_t row_bytes = (uint32_t)(args.cin * (int64_t)sizeof(TA));

    int nk;
    if (args.map) {
        nk = build_offset_list(map_tile, nrows, K, n_in, s_kmask, s_klist, &s_nk);
        fill_row_offsets(map_tile, nrows, K, n_in, row_bytes, s_klist, nk, s_aoff);
    } else {
        // no map: the dense linear (K = 1), query row r reads input row r
        nk = 1;
        if (tid == 0) s_klist[0] = 0;
        s_aoff[0][tid] = tid < nrows && row0 + tid < n_in ? (uint32_t)(row0 + tid) * row_bytes : kOobOffset;
        __syncthreads();
    }

    const int nkc = args.cin_g / kBK;  // chunks per offset
    const int S = nk * nkc;
    const int S2 = S + (S & 1);

    f32x16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    if (S > 0) {
        const int ar0 = wave * 64 + (lane & 31), ar1 = ar0 + 32;
        const __amdgpu_buffer_rsrc_t a_rsrc =
            make_rsrc(input + in_col0, (uint32_t)(n_in * row_bytes - in_col0 * (int64_t)sizeof(TA)));
        const __amdgpu_buffer_rsrc_t w_rsrc =
            make_rsrc(weight, (uint32_t)(args.cout * (int64_t)K * args.cin_g * (int64_t)sizeof(TW)));

        // Weight pieces: index t + 256*i -> channel idx / kWPieces, piece idx % kWPieces.
        uint32_t w_base[kBPerThread];
#pragma unroll
        for (int i = 0; i < kBPerThread; ++i) {
            const int idx = tid + kThreads * i;
            const int ch = idx / kWPieces, pc = idx % kWPieces;
            w_base[i] = o0 + ch < args.cout_g
                            ? (uint32_t)((out_col0 + o0 + ch) * (int64_t)K * args.cin_g * (int64_t)sizeof(TW)) + pc * 16
                            : kOobOffset;
        }
        const uint32_t w_k_bytes = (uint32_t)(args.cin_g * (int64_t)sizeof(TW));
        uint4 rb[kBPerThread];
        // Loads of stage t (t >= S: zero weights, zero A).
        auto load_stage = [&](int t, APiece<NP> &f0, APiece<NP> &f1) {
            const bool live = t < S;
            const int tt = live ? t : 0;
            const int ki = tt / nkc, kc = tt - ki * nkc;
            const int k = s_klist[ki];
            const uint32_t wk = (uint32_t)k * w_k_bytes + (uint32_t)(kc * kWBytes);
#pragma unroll
            for (int i = 0; i < kBPerThread; ++i) rb[i] = bload16(w_rsrc, live ? w_base[i] + wk : kOobOffset);
            const uint32_t o_a0 = live ? s_aoff[ki][ar0] : kOobOffset;
            const uint32_t o_a1 = live ? s_aoff[ki][ar1] : kOobOffset;
            f0 = load_a_pieces<kF32, CB>(a_rsrc, o_a0, kc, half);
            f1 = load_a_pieces<kF32, CB>(a_rsrc, o_a1, kc, half);
        };
        auto store_b = [&](int buf) {
            unsigned char *b = s_b[buf];
#pragma unroll
            for (int i = 0; i < kBPerThread; ++i) {
                const int idx = tid + kThreads * i;
                const int ch = idx / kWPieces, pc = idx % kWPieces;
                if constexpr (kI8) {
                    uint4 w0, w1;
                    widen_i8x16(rb[i], w0, w1);
                    *reinterpret_cast<uint4 *>(b + ch * kStride + pc * 32) = w0;
                    *reinterpret_cast<uint4 *>(b + ch * kStride + pc * 32 + 16) = w1;
                } else {
                    *reinterpret_cast<uint4 *>(b + ch * kStride + pc * 16) = rb[i];
                }
            }
        };
        const int bcol = lane & 31;
        auto compute = [&](int buf, const APiece<NP> &c0, const APiece<NP> &c1) {
            const unsigned char *b = s_b[buf];
#pragma unroll
            for (int q = 0; q < NP; ++q) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint4 bq = *reinterpret_cast<const uint4 *>(
                        b + (j * 32 + bcol) * kStride + piece_offset<kF32, CB>(q, half));
                    mfma_piece<kF32>(acc[0][j], c0.p[q], bq);
                    mfma_piece<kF32>(acc[1][j], c1.p[q], bq);
                }
            }
        };

        APiece<NP> x0, x1, y0, y1;
        load_stage(0, x0, x1);
        store_b(0);
        __syncthreads();
        // sched_barrier keeps the next stage's loads ahead of this stage's
        // MFMAs (the scheduler would otherwise sink them below).
        for (int t = 0; t < S2; t += 2) {
            load_stage(t + 1, y0, y1);
            __builtin_amdgcn_sched_barrier(0);
            compute(0, x0, x1);
            store_b(1);
            __syncthreads();
            load_stage(t + 2, x0, x1);
            __builtin_amdgcn_sched_barrier(0);
            compute(1, y0, y1);
            store_b(0);
            __syncthreads();
        }
    }

    // ---- epilogue.  32x32 MFMA result layout (transposed product): lane l,
    //      element e -> output channel 8*(e/4) + 4*(l/32) + e%4 of the block,
    //      voxel row l%32.  Each run of 4 elements is 4 consecutive channels;
    //      lanes l and l^32 together hold all channels of a row.
    TO *__restrict__ out = static_cast<TO *>(args.out);
    const TO *__restrict__ res = static_cast<const TO *>(args.residual);
    const bool vec_ok = args.vec_out != 0;
    // bias / int8 scale per channel, applied to both row blocks at once
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int o = o0 + j * 32 + 8 * (e >> 2) + 4 * half + (e & 3);
            const bool ok = o < args.cout_g;
            const float bias = (args.bias && ok) ? args.bias[out_col0 + o] : 0.f;
            const float scale = (kI8 && args.w_scale && ok) ? args.w_scale[out_col0 + o] : 1.f;
#pragma unroll
            for (int i = 0; i < 2; ++i)
                acc[i][j][e] = ok ? (kI8 ? acc[i][j][e] * scale + bias : acc[i][j][e] + bias) : 0.f;
        }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = wave * 64 + i * 32 + (lane & 31);
        if (r >= nrows) continue;  // lanes l and l^32 share r: both skip together
        const int64_t rowbase = (row0 + r) * args.cout + out_col0;
        if (args.ln) {
            // Two-pass f32 statistics over the row's Cout channels (the
            // reference's layer_norm_row_stats, wgpu/ops.rs:162-187).
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) s += acc[i][j][e];
            s += __shfl_xor(s, 32, 64);
            const float inv_c = 1.0f / (float)args.cout_g;
            const float mean = s * inv_c;
            float q = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int o = o0 + j * 32 + 8 * (e >> 2) + 4 * half + (e & 3);
                    const float d = acc[i][j][e] - mean;
                    q += o < args.cout_g ? d * d : 0.f;
                }
            q += __shfl_xor(q, 32, 64);
            const float inv_std = rsqrt_f32(q * inv_c + args.ln_eps);
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int o = o0 + j * 32 + 8 * (e >> 2) + 4 * half + (e & 3);
                    const bool ok = o < args.cout_g;
                    float t = (acc[i][j][e] - mean) * inv_std;
                    if (args.ln_w && ok) t *= args.ln_w[o];
                    if (args.ln_b && ok) t += args.ln_b[o];
                    acc[i][j][e] = t;
                }
        }
        if (args.silu) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float t = acc[i][j][e];
                    acc[i][j][e] = silu_f32(t);
                }
        }
        if (args.scatter_rows || args.skip_idx) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e4 = 0; e4 < 4; ++e4) {
                    const int oc = o0 + j * 32 + 8 * e4 + 4 * half;
                    if (oc >= args.cout_g) continue;
                    float v[4];
#pragma unroll
                    for (int c = 0; c < 4; ++c) v[c] = acc[i][j][4 * e4 + c];
                    c2s_store4<TO>(args, c2s_row<TO>(args, row0 + r), row0 + r, (int)(out_col0 + oc),
                                   min(4, args.cout_g - oc), v, vec_ok);
                }
            continue;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4) {
                const int oc = o0 + j * 32 + 8 * e4 + 4 * half;  // first of 4 channels
                float v[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) v[c] = acc[i][j][4 * e4 + c];
                if (vec_ok && oc + 3 < args.cout_g) {
                    typename Out4<TO>::V *dst = reinterpret_cast<typename Out4<TO>::V *>(out + rowbase + oc);
                    if (res) {
                        float rv[4];
                        Out4<TO>::unpack(*reinterpret_cast<const typename Out4<TO>::V *>(res + rowbase + oc), rv);
#pragma unroll
                        for (int c = 0; c < 4; ++c) v[c] += rv[c];
                    }
                    *dst = Out4<TO>::pack(v);
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        if (oc + c >= args.cout_g) continue;
                        float t = v[c];
                        if (res) t += load_as_f32<TO>(res, rowbase + oc + c);
                        store_from_f32<TO>(out, rowbase + oc + c, t);
                    }
                }
            }
    }
}


// ------------------------------------------------------ bf16 tile, v2
//
// 256 rows x 128 output channels, 4 waves; wave w owns rows [64w, 64w+64) as
// 4 x 8 blocks of v_mfma_f32_16x16x32_bf16 (transposed product: lane l ends
// with channels 4*(l/16)+e of row l%16 of each block).  The neighbour rows are
// gathered from global memory per (row, offset):
//  * a stage is one used offset x CB bytes of the input row (CB = 128: two
//    MFMA k-steps, half the barriers of 64-byte stages);
//  * bf16 weights go global -> LDS by buffer_load ... lds (no staging
//    registers, no ds_write); int8 weights are widened through registers;
//  * LDS weight slices are XOR-swizzled per 16-byte piece, so the MFMA
//    operand reads (16 channels x 16 bytes per 16 lanes) hit distinct banks;
//  * offsets are walked by scalar bit cursors over the tile's offset mask,
//    and the gathered-row byte offsets of the next A stage are read from LDS
//    one stage before the loads that use them.
// The stage loop keeps a static number of vector loads per stage, so the
// explicit vmcnt waits below are exact: W(t) and A(t) have landed when
// stage t starts.

template <int N>
__device__ inline void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Physical 16-byte slot of logical piece p of channel c's CB-byte slice.
template <int CB>
__device__ inline int wslot(int c, int p)
{
    if constexpr (CB == 128)
        return p ^ (c & 7);
    else
        return p ^ (((c >> 1) ^ (c >> 2)) & 3);
}

// Scalar cursor over (used offset, input chunk) stages.
struct StageCursor {
    uint32_t rem;  // offsets not yet finished (bit k = offset k); 0 = past the end
    int k;         // current offset
    int kc;        // current input chunk
    __device__ inline void init(uint32_t mask)
    {
        rem = mask;
        k = mask ? __builtin_ctz(mask) : 0;
        kc = 0;
    }
    __device__ inline void next(int nkc)
    {
        if (++kc == nkc) {
            kc = 0;
            rem &= rem - 1u;
            k = rem ? __builtin_ctz(rem) : 0;
        }
    }
    __device__ inline bool live() const { return rem != 0u; }
};

template <typename TA, typename TW, typename TO, int CB, int DIST>
__global__ __launch_bounds__(kThreads, 2) void conv_v2_kernel(ConvArgs args)
{
    constexpr bool kI8 = sizeof(TW) == 1;
    constexpr bool kDMA = !kI8;              // bf16 weights: direct global -> LDS
    constexpr int KS = CB / 64;              // 32-element MFMA k-steps per stage
    constexpr int NP = CB / 16;              // 16-byte pieces per channel per stage
    constexpr int NSET = DIST + 1;           // register sets of gathered rows
    constexpr int NA = 4 * KS;               // A load instructions per stage
    constexpr int kRows = kTileRows;
    constexpr int kWStage = kBN * CB;        // LDS bytes of one weight stage
    constexpr int kDmaPerWave = kWStage / 1024 / 4;  // 1 KB per DMA instruction
    constexpr int kWBytesCh = kI8 ? CB / 2 : CB;     // weight bytes per channel per stage
    constexpr int kRegPieces = kBN * (kWBytesCh / 16) / kThreads;  // staged 16 B loads/thread
    constexpr int NW = kDMA ? kDmaPerWave : kRegPieces;  // weight load instructions per stage
    static_assert(!kDMA || kDmaPerWave >= 1, "DMA pieces");
    static_assert(DIST == 1 || DIST == 2, "prefetch distance");
    static_assert(kDMA || kRegPieces >= 1, "staged pieces");

    // Two weight buffers as separate LDS objects: the compiler then sees that
    // the MFMA operand reads of one buffer cannot alias the DMA into the
    // other, and does not wait for that DMA before them.
    __shared__ __attribute__((aligned(16))) unsigned char s_b0[kWStage];
    __shared__ __attribute__((aligned(16))) unsigned char s_b1[kWStage];
    __shared__ uint32_t s_aoff[kMaxTableK][kRows];
    __shared__ int32_t s_qrow[kRows];
    __shared__ uint32_t s_tmask;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, q4 = lane >> 4;
    const int K = args.K;

    const int tile = tile_for_block(blockIdx.x, gridDim.x);
    const int64_t row0 = (int64_t)tile * kRows;
    const int o0 = blockIdx.y * kBN;
    const int g = blockIdx.z;
    const int64_t in_col0 = (int64_t)g * args.cin_g;
    const int64_t out_col0 = (int64_t)g * args.cout_g;
    const int64_t n_in = args.n_in;
    const uint32_t row_bytes = (uint32_t)(args.cin * (int64_t)sizeof(TA));

    // ---- prologue: row ids, neighbour byte offsets, masks.
    if (tid == 0) s_tmask = 0u;
    uint32_t m = 0;
    {
        const int64_t qrow = row0 + tid;
        const bool rv = qrow < args.n_q;
        s_qrow[tid] = rv ? (int32_t)qrow : -1;
        // no map: the dense linear (K = 1), query row q reads input row q
        const int32_t *mrow = args.map ? args.map + (rv ? qrow : 0) * K : nullptr;
        int32_t v[kMaxTableK];
#pragma unroll
        for (int k = 0; k < kMaxTableK; ++k) v[k] = (rv && k < K) ? (mrow ? mrow[k] : (int32_t)qrow) : -1;
#pragma unroll
        for (int k = 0; k < kMaxTableK; ++k) {
            const bool ok = v[k] >= 0 && v[k] < n_in;
            if (k < K) s_aoff[k][tid] = ok ? (uint32_t)v[k] * row_bytes : kOobOffset;
            m |= (uint32_t)ok << k;
        }
    }
    // Per-16-row-block masks (wave-uniform) and the tile's offset mask.
    uint32_t bm = m;
    bm |= __shfl_xor(bm, 1, 64);
    bm |= __shfl_xor(bm, 2, 64);
    bm |= __shfl_xor(bm, 4, 64);
    bm |= __shfl_xor(bm, 8, 64);
    const uint32_t bm0 = __builtin_amdgcn_readlane(bm, 0), bm1 = __builtin_amdgcn_readlane(bm, 16);
    const uint32_t bm2 = __builtin_amdgcn_readlane(bm, 32), bm3 = __builtin_amdgcn_readlane(bm, 48);
    __syncthreads();
    if (lane == 0) atomicOr(&s_tmask, bm0 | bm1 | bm2 | bm3);
    __syncthreads();
    const uint32_t tmask = __builtin_amdgcn_readfirstlane(s_tmask);

    f32x4 acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][e] = 0.f;

    const int nkc = args.cin_g / (CB / 2);
    if (tmask != 0u) {
        const TA *input = static_cast<const TA *>(args.input);
        const __amdgpu_buffer_rsrc_t a_rsrc =
            make_rsrc(input + in_col0, (uint32_t)(n_in * row_bytes - in_col0 * (int64_t)sizeof(TA)));
        const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(
            args.weight, (uint32_t)(args.cout * (int64_t)K * args.cin_g * (int64_t)sizeof(TW)));
        const uint32_t w_k_bytes = (uint32_t)(args.cin_g * (int64_t)sizeof(TW));
        const uint32_t w_ch_bytes = (uint32_t)K * w_k_bytes;

        // Weight piece(s) this thread moves per stage: channel, logical piece, LDS slot.
        uint32_t w_gbase[NW];
        uint32_t w_lds[NW];
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            int c, p;
            if constexpr (kDMA) {
                // DMA instruction i of this wave fills LDS bytes [1 KB * (wave*NW + i), +1 KB):
                // lane l writes slot l -> channel c, physical piece l % NP.
                c = (wave * NW + i) * (1024 / CB) + lane / NP;
                const int phys = lane % NP;
                p = wslot<CB>(c, phys);  // logical piece stored at that slot
                w_lds[i] = (uint32_t)((wave * NW + i) * 1024);
            } else {
                const int idx = tid + kThreads * i;
                constexpr int pcs = kWBytesCh / 16;  // 16-byte global pieces per channel
                c = idx / pcs;
                p = idx % pcs;
                w_lds[i] = 0;
            }
            w_gbase[i] = (o0 + c < args.cout_g)
                             ? (uint32_t)((out_col0 + o0 + c) * (int64_t)w_ch_bytes) + (uint32_t)(p * 16)
                             : kOobOffset;
        }
        uint4 rb[kDMA ? 1 : NW];
        // buf is a compile-time constant wherever this is called (unrolled loops)
        auto wbuf = [&](int buf) -> unsigned char * { return buf ? s_b1 : s_b0; };

        auto load_w = [&](const StageCursor &c, int buf) {
            const bool live = c.live();
            const uint32_t wk = (uint32_t)c.k * w_k_bytes + (uint32_t)(c.kc * kWBytesCh);
#pragma unroll
            for (int i = 0; i < NW; ++i) {
                // an out-of-range base stays out of range: w_gbase + wk < 2^32
                const uint32_t off = live ? w_gbase[i] + wk : kOobOffset;
                if constexpr (kDMA) {
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        w_rsrc, (__attribute__((address_space(3))) void *)(wbuf(buf) + w_lds[i]), 16, off, 0, 0,
                        0);
                } else {
                    rb[i] = bload16(w_rsrc, off);
                }
            }
        };
        auto store_w = [&](int buf) {  // staged (int8) path only
            if constexpr (!kDMA) {
                unsigned char *b = wbuf(buf);
#pragma unroll
                for (int i = 0; i < NW; ++i) {
                    const int idx = tid + kThreads * i;
                    constexpr int pcs = kWBytesCh / 16;
                    const int c = idx / pcs, p = idx % pcs;
                    uint4 w0, w1;
                    widen_i8x16(rb[i], w0, w1);
                    *reinterpret_cast<uint4 *>(b + c * CB + wslot<CB>(c, 2 * p) * 16) = w0;
                    *reinterpret_cast<uint4 *>(b + c * CB + wslot<CB>(c, 2 * p + 1) * 16) = w1;
                }
            }
        };
        auto read_offsets = [&](const StageCursor &c, uint32_t (&ro)[4]) {
            const int k = c.live() ? c.k : 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) ro[i] = s_aoff[k][wave * 64 + i * 16 + l16];
        };
        auto load_a = [&](const StageCursor &c, const uint32_t (&ro)[4], uint4 (&f)[4][KS]) {
            const bool live = c.live();
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t base = live ? ro[i] : kOobOffset;
#pragma unroll
                for (int q = 0; q < KS; ++q)
                    f[i][q] = bload16(a_rsrc, base + (uint32_t)(c.kc * CB + q * 64 + q4 * 16));
            }
        };
        auto compute = [&](const StageCursor &c, int buf, const uint4 (&f)[4][KS]) {
            if (!c.live()) return;
            const unsigned char *b = wbuf(buf);
#pragma unroll
            for (int q = 0; q < KS; ++q) {
                uint4 w[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int ch = j * 16 + l16;
                    w[j] = *reinterpret_cast<const uint4 *>(b + ch * CB + wslot<CB>(ch, q * 4 + q4) * 16);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        acc[i][j] = mfma_16x16x32<TA>(w[j], f[i][q], acc[i][j]);
                }
            }
        };
        // LDS-only barrier: the waits above it are explicit (vmcnt for the
        // DMA'd weights, lgkmcnt for ds ops).
        auto barrier = [&]() {
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0) (vmcnt, expcnt untouched)
            __builtin_amdgcn_s_barrier();
        };

        uint4 fa[NSET][4][KS];
        uint32_t ro[4];
        StageCursor cc, ca, co;  // compute (t), A loads (t + DIST), offsets (t + DIST + 1)
        cc.init(tmask);
        ca.init(tmask);
        co.init(tmask);
        // Prologue: W(0), A(0..DIST-1), offsets of stage DIST.
        read_offsets(co, ro);
        co.next(nkc);
        load_w(cc, 0);
        store_w(0);  // staged weights only (the compiler waits for rb)
#pragma unroll
        for (int d = 0; d < DIST; ++d) {
            load_a(ca, ro, fa[d]);
            ca.next(nkc);
            read_offsets(co, ro);
            co.next(nkc);
        }

        // Stage t (weight buffer t & 1, register set t % NSET):
        //   wait until W(t) and A(t) have landed; barrier; issue W(t+1) into
        //   buffer (t+1) & 1 (its last readers finished stage t-1 before the
        //   barrier) and A(t+DIST) into set (t+DIST) % NSET; read the row
        //   offsets of stage t+DIST+1; MFMAs of stage t.
        // Loads are issued in the order W(t+1), A(t+DIST), so at the top of
        // stage t+1 only A(t+DIST) (DIST >= 2) may still be in flight.
        // The body covers lcm(2, NSET) stages so parities and sets are static.
        constexpr int kUnroll = (NSET % 2 == 0) ? NSET : 2 * NSET;
        constexpr int kInFlight = DIST >= 2 ? NA : 0;
        while (cc.live()) {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int buf = u & 1;
                wait_vmcnt<kInFlight>();
                barrier();
                __builtin_amdgcn_sched_barrier(0);
                StageCursor cn = cc;
                cn.next(nkc);
                load_w(cn, buf ^ 1);
                load_a(ca, ro, fa[(u + DIST) % NSET]);
                ca.next(nkc);
                read_offsets(co, ro);
                co.next(nkc);
                __builtin_amdgcn_sched_barrier(0);
                compute(cc, buf, fa[u % NSET]);
                // staged weights: W(t+1) registers -> buffer buf ^ 1
                store_w(buf ^ 1);
                cc = cn;
            }
        }
        wait_vmcnt<0>();
    }

    // ---- epilogue: lane l holds channels j*16 + 4*(l/16) + e (e = 0..3) of
    //      tile row i*16 + l%16; the 4 lanes of a row skip together.
    TO *__restrict__ out = static_cast<TO *>(args.out);
    const TO *__restrict__ res = static_cast<const TO *>(args.residual);
    const bool vec_ok = args.vec_out != 0;
    const bool c2s = args.scatter_rows || args.skip_idx;
    // LayerNorm groups: the row (ln_group = Cout_g <= 128, or a 128-channel
    // C2S child = the tile) or the two 64-channel halves of the tile (C2S
    // children of 64 channels).  Partial sums are kept per half either way.
    const bool halves = args.ln_group == 64 && args.cout_g > 64;
    const float inv_c = 1.0f / (float)args.ln_group;
    // bias / int8 scale per channel, applied to the 4 row blocks at once (each
    // value is then dead: no 32 + 32 registers held through the epilogue)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int o = o0 + j * 16 + 4 * q4 + e;
            const bool ok = o < args.cout_g;
            const float bias = (args.bias && ok) ? args.bias[out_col0 + o] : 0.f;
            const float scale = (kI8 && args.w_scale && ok) ? args.w_scale[out_col0 + o] : 1.f;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[i][j][e] = ok ? (kI8 ? acc[i][j][e] * scale + bias : acc[i][j][e] + bias) : 0.f;
        }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int32_t qrow = s_qrow[wave * 64 + i * 16 + l16];
        if (qrow < 0) continue;
        const int64_t rowbase = (int64_t)qrow * args.cout + out_col0;
        if (args.ln) {
            float sum[2] = {0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) sum[j >> 2] += acc[i][j][e];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                sum[h] += __shfl_xor(sum[h], 16, 64);
                sum[h] += __shfl_xor(sum[h], 32, 64);
            }
            if (!halves) sum[0] = sum[1] = sum[0] + sum[1];
            const float mean[2] = {sum[0] * inv_c, sum[1] * inv_c};
            float qv[2] = {0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int o = o0 + j * 16 + 4 * q4 + e;
                    const float d = acc[i][j][e] - mean[j >> 2];
                    qv[j >> 2] += o < args.cout_g ? d * d : 0.f;
                }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                qv[h] += __shfl_xor(qv[h], 16, 64);
                qv[h] += __shfl_xor(qv[h], 32, 64);
            }
            if (!halves) qv[0] = qv[1] = qv[0] + qv[1];
            const float inv_std[2] = {rsqrt_f32(qv[0] * inv_c + args.ln_eps), rsqrt_f32(qv[1] * inv_c + args.ln_eps)};
            // channel within the LayerNorm group: o itself for a whole row,
            // o - o0 (+ 64 for the upper half) inside a C2S child
            const int gbase = args.ln_group == args.cout_g ? 0 : o0;
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int o = o0 + j * 16 + 4 * q4 + e;
                    const bool ok = o < args.cout_g;
                    const int og = halves ? (o - o0) & 63 : o - gbase;
                    float t = (acc[i][j][e] - mean[j >> 2]) * inv_std[j >> 2];
                    if (args.ln_w && ok) t *= args.ln_w[og];
                    if (args.ln_b && ok) t += args.ln_b[og];
                    acc[i][j][e] = t;
                }
        }
        if (args.silu) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float t = acc[i][j][e];
                    acc[i][j][e] = silu_f32(t);
                }
        }
        const C2SRow crow = c2s ? c2s_row<TO>(args, qrow) : C2SRow{nullptr};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int oc = o0 + j * 16 + 4 * q4;
            float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
            if (c2s) {
                if (oc < args.cout_g)
                    c2s_store4<TO>(args, crow, qrow, (int)(out_col0 + oc), min(4, args.cout_g - oc), v, vec_ok);
                continue;
            }
            if (vec_ok && oc + 3 < args.cout_g) {
                typename Out4<TO>::V *dst = reinterpret_cast<typename Out4<TO>::V *>(out + rowbase + oc);
                if (res) {
                    float rv[4];
                    Out4<TO>::unpack(*reinterpret_cast<const typename Out4<TO>::V *>(res + rowbase + oc), rv);
#pragma unroll
                    for (int c = 0; c < 4; ++c) v[c] += rv[c];
                }
                *dst = Out4<TO>::pack(v);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    if (oc + c >= args.cout_g) continue;
                    float t = v[c];
                    if (res) t += load_as_f32<TO>(res, rowbase + oc + c);
                    store_from_f32<TO>(out, rowbase + oc + c, t);
                }
            }
        }
    }
}

// ------------------------------------------------- bf16 tile, halo-staged
//
// Reads a conv plan (sc_plan.hpp).  For 256-row tile t (rows order[t*256..]
// in brick order), the U distinct input rows its neighbours touch (the halo,
// U <= kPlanHaloMax, numbered in increasing row order) are staged into LDS
// once per 32-channel chunk by buffer_load ... lds (16 rows x 64 B per
// instruction, coalesced), and every (row, offset) operand is read from LDS
// through the local map lmap[k][row].  Global gather traffic drops from one
// row per valid (row, offset) pair (~21 per output row at config 3) to ~2.
//
// Tile = 256 rows x 128 output channels, 4 waves, two workgroups per CU;
// wave w owns rows [128 (w/2), +128) x channels [64 (w%2), +64) as 8 x 4
// blocks of v_mfma_f32_16x16x32_bf16 (transposed product: lane l ends with
// channels 4*(l/16)+e of row l%16 of each block).  Stage = (32-channel chunk
// c, used offset k), chunk-major.  Per stage a wave reads 8 operand fragments
// from the LDS halo (each feeds 4 MFMAs) and loads its 4 weight fragments
// w[o, k, 32c..32c+32) from L2 straight into registers one stage ahead (the
// two waves of a column half share them through L1), so stages need no
// barrier: the workgroup synchronises only when the halo moves to the next
// chunk, and the other workgroup on the CU computes meanwhile.  The 2 x 2
// split halves the vector-memory weight traffic of a 1 x 4 row split (the
// texture path, not the MFMAs, bounds that form) for twice the LDS operand
// reads.  Absent neighbours read a zero row.  Per-row accumulation order is
// fixed (chunk-major, offsets ascending).  A tile whose halo exceeds
// kPlanHaloMax rows (no local map or halo is built for it) keeps the byte
// offsets of its rows' neighbours where the halo would be and loads every
// operand from global memory, in the same stages and order.
//
// Tiles of 64 output channels (layers of at most 64 per group, and C2S
// children of 64) keep the 128 x 64 wave block: the two waves of a row half
// split the stages instead of the channels (in chunk c the wave of parity p
// takes the offsets at even or odd positions of the tile's offset list,
// alternating per chunk when the list is odd, so the halves differ by at
// most one stage per two chunks), and add their partial sums through LDS
// after the loop, each keeping 64 rows.  A wave of 64 rows x 64 channels
// would load a weight fragment per 4 MFMAs instead of per 8 and be bound by
// the texture path at about 0.6 PFLOP/s.  Per value the sum is (stages of
// parity 0) + (stages of parity 1), each in stage order.
//
// LDS: halo (960 + 1) x 64 B + source offsets 960 x 4 B + lmap 27 x 256 x 2 B
// = 77 KB.
constexpr int kHaloK = 27;
#ifndef SC_HALO_WS
#define SC_HALO_WS 2
#endif

__device__ inline int hslot(int j, int p) { return p ^ (((j >> 1) ^ (j >> 2)) & 3); }

template <typename TA, typename TO, bool kLN, int kNT>
__global__ __launch_bounds__(kThreads, 2) void conv_halo_kernel(ConvArgs args, PlanView plan)
{
    constexpr int CB = 64;  // bytes of an input row per chunk (32 bf16 = one MFMA k-step)
    constexpr int kWLane = 16;                  // weight bytes (8 bf16) per lane per fragment
    constexpr int kZeroRow = kPlanHaloMax;
    constexpr int kHaloPerWave = (kPlanHaloMax / 16 + 3) / 4;  // 16-row DMA instructions per wave
    static_assert(kHaloPerWave * 64 == kPlanHaloMax, "4 waves x 16 rows tile the halo exactly");
    constexpr int kWS = SC_HALO_WS;             // weight register sets: stages t .. t+kWS-1
    static_assert(kPlanTileRows == kTileRows, "plan tile = 256 rows");
    // kNT = 128: waves 2 x 2 (128 rows x 64 channels each); kNT = 64 (layers
    // of at most 64 output channels): waves 2 (row halves) x 2 (stage
    // parity) in the loop, 64 rows x 64 channels each in the epilogue.
    static_assert(kNT == 128 || kNT == 64, "output tile of 128 or 64 channels");
    constexpr bool kKS = kNT == 64;             // stages split between the waves of a row half
    constexpr int kIM = 8;                      // 16-row MFMA blocks per wave in the loop
    constexpr int kI = kNT == 128 ? 8 : 4;      // ... and in the epilogue

    __shared__ __attribute__((aligned(16))) unsigned char s_halo[(kPlanHaloMax + 1) * CB];
    // s_lmap[k][rh][l16][i]: LDS byte offset of the halo row feeding tile row
    // 128 rh + 16 i + l16 at offset k, pre-swizzled (j*64 + 16*s(j), so that
    // XOR with 16 q4 gives the lane's piece); absent -> the zero row.  One
    // 16-byte read hands a lane its 8 operand rows of a stage.
    __shared__ __attribute__((aligned(16))) uint16_t s_lmap[kHaloK][2][16][8];
    __shared__ uint32_t s_hoff[kPlanHaloMax];
    __shared__ uint32_t s_wmask[kThreads / 64];
    // fetched in the prologue's round trip for the epilogue: the tile's
    // output rows (the plan order) and its channels' bias and int8 scale
    __shared__ int32_t s_order[kPlanTileRows];
    __shared__ float s_bias[kNT], s_scale[kNT];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, q4 = lane >> 4;
    const int rh = wave >> 1;                              // lmap half of the wave's rows
    const int ch = kNT == 128 ? (wave & 1) : 0;            // channel half
    const int row0 = kNT == 128 ? 128 * rh : 64 * wave;    // first tile row of the wave (epilogue)
    const int K = args.K;

    // The plan must be the one built for this map shape and the packed
    // weights the ones packed for this config: otherwise nothing past the two
    // headers is read, nothing is written, and the plan's status records it.
    {
        const PackHeader *wh = static_cast<const PackHeader *>(args.wpack);
        const bool plan_ok = plan_matches(plan.hdr, args);
        // f16 fragments for f16 activations, bf16 fragments (from bf16 or int8) otherwise
        const bool w_f16 = wh->src_dtype == SC_DTYPE_F16;
        const bool w_ok = wh->magic == kPackMagic && wh->groups == (int)gridDim.z && wh->cout_g == args.cout_g &&
                          wh->cin_g == args.cin_g && wh->K == K && w_f16 == __is_same(TA, _Float16);
        if (!plan_ok || !w_ok) {
            flag_plan_status(plan.hdr, (plan_ok ? 0u : kPlanStatusMapMismatch) | (w_ok ? 0u : kPlanStatusWeightMismatch));
            return;
        }
        // a plan flagged by an earlier call stays flagged until it is
        // rebuilt: nothing is written meanwhile
        if (plan.hdr->status != 0u) return;
    }
    int tile;
    if (plan.tile_child) {
        // a child plan: its list tiles in use, then its split spares, dealt
        // to the XCDs as one range (the grid covers the layout's bound; the
        // other workgroups exit on every XCD alike)
        const int n_used = plan.hdr->n_unique, n_real = n_used + plan.hdr->n_extras;
        if ((int)blockIdx.x >= n_real) return;
        const int l = tile_for_block(blockIdx.x, n_real);
        tile = l < n_used ? l : plan.hdr->list_tiles + (l - n_used);
    } else {
        tile = tile_for_block(blockIdx.x, gridDim.x);
    }
    const int U = plan.tile_u[tile];
    // A tile whose halo exceeds the LDS budget (listed in plan.overflow; its
    // local map and halo are not built) gathers its operands straight from
    // global memory, through the byte offsets of its rows' neighbours held
    // where the halo would be.
    const bool direct = U > kPlanHaloMax;
    // a child plan's tile computes its child's channel block (an unused tile nothing)
    const int child = plan.tile_child ? plan.tile_child[tile] : 0;
    if (child < 0) return;
    const int o0 = child * args.child_ch + blockIdx.y * kNT;
    const int g = blockIdx.z;
    const int64_t in_col0 = (int64_t)g * args.cin_g;
    const int64_t out_col0 = (int64_t)g * args.cout_g;
    const uint32_t row_bytes = (uint32_t)(args.cin * (int64_t)sizeof(uint16_t));

    // ---- prologue: local map (as LDS offsets, thread = tile row), zero
    //      row, halo source offsets, mask of the offsets the tile uses.
    {
        // Every load first -- the row's K local-map entries and this
        // thread's halo rows -- so the prologue costs one memory round trip
        // (a loop over k waits once per few offsets: ~10 round trips a tile).
        const int32_t ord = plan.order[(int64_t)tile * kPlanTileRows + tid];
        float bv = 0.f, sv = 1.f;
        if (tid < kNT) {
            const int o = o0 + tid;
            const bool ok = o < args.cout_g;
            if (args.bias && ok) bv = args.bias[out_col0 + o];
            if (args.w_scale && ok) sv = args.w_scale[out_col0 + o];  // int8 weights
        }
        uint32_t m = 0;
        if (direct) {
            // the row's map entries -> byte offsets of its neighbours' input
            // rows, dof[k][tile row] (absent: an offset past the input)
            uint32_t *dof = reinterpret_cast<uint32_t *>(s_halo);
            const bool live = ord >= 0 && ord < args.n_q;
            int32_t e[kHaloK];
#pragma unroll
            for (int k = 0; k < kHaloK; ++k) e[k] = (k < K && live) ? args.map[(int64_t)ord * K + k] : -1;
#pragma unroll
            for (int k = 0; k < kHaloK; ++k) {
                if (k >= K) break;
                const bool ok = e[k] >= 0 && e[k] < args.n_in;
                m |= (uint32_t)ok << k;
                dof[k * kPlanTileRows + tid] = ok ? (uint32_t)e[k] * row_bytes : kOobOffset;
            }
        } else {
            const uint16_t *src = plan.lmap + (int64_t)tile * K * kPlanTileRows + tid;
            const int32_t *hrows = plan.halo + (int64_t)tile * kPlanHaloMax;
            constexpr int kHPer = (kPlanHaloMax + kThreads - 1) / kThreads;  // halo rows per thread
            uint32_t jv[kHaloK];
            int32_t hv[kHPer];
#pragma unroll
            for (int k = 0; k < kHaloK; ++k) jv[k] = k < K ? src[k * kPlanTileRows] : (uint32_t)kPlanAbsent;
#pragma unroll
            for (int u = 0; u < kHPer; ++u) hv[u] = tid + u * kThreads < U ? hrows[tid + u * kThreads] : 0;
            uint16_t *dst = &s_lmap[0][tid >> 7][tid & 15][(tid >> 4) & 7];
#pragma unroll
            for (int k = 0; k < kHaloK; ++k) {
                if (k >= K) break;
                const int j = (int)jv[k];
                m |= (uint32_t)(j != kPlanAbsent) << k;
                dst[k * kPlanTileRows] =
                    (uint16_t)(j == kPlanAbsent ? kZeroRow * CB : j * CB + 16 * (((j >> 1) ^ (j >> 2)) & 3));
            }
            if (tid < CB / 16) reinterpret_cast<uint4 *>(s_halo + kZeroRow * CB)[tid] = make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int u = 0; u < kHPer; ++u)
                if (tid + u * kThreads < U) s_hoff[tid + u * kThreads] = (uint32_t)hv[u] * row_bytes;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m |= __shfl_xor(m, off, 64);
        if (lane == 0) s_wmask[wave] = m;
        s_order[tid] = ord;
        if (tid < kNT) {
            s_bias[tid] = bv;
            s_scale[tid] = sv;
        }
    }
    __syncthreads();
    const uint32_t tmask = __builtin_amdgcn_readfirstlane(s_wmask[0] | s_wmask[1] | s_wmask[2] | s_wmask[3]);
    // The wave's offsets in even and odd chunks (all of them without the
    // stage split; a tile with one offset leaves the parity-1 waves idle).
    uint32_t m_even = tmask, m_odd = tmask;
    const int kpar = kKS ? (__builtin_amdgcn_readfirstlane(wave) & 1) : 0;
    if constexpr (kKS) {
        uint32_t ev = 0u, r = tmask;
        for (bool take = true; r != 0u; take = !take) {
            const uint32_t b = r & (0u - r);
            if (take) ev |= b;
            r ^= b;
        }
        const uint32_t od = tmask ^ ev;
        if (od == 0u) {
            m_even = m_odd = kpar ? 0u : tmask;
        } else if ((__builtin_popcount(tmask) & 1) == 0) {
            m_even = m_odd = kpar ? od : ev;
        } else {
            m_even = kpar ? od : ev;
            m_odd = kpar ? ev : od;
        }
    }

    f32x4 acc[kIM][4];
#pragma unroll
    for (int i = 0; i < kIM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][e] = 0.f;

    const int nkc = args.cin_g / (CB / 2);
    if (tmask != 0u && nkc > 0) {
        const uint16_t *input = static_cast<const uint16_t *>(args.input);
        const i32x4_rsrc a_rsrc =
            rsrc_words(input + in_col0, (uint32_t)(args.n_in * row_bytes - in_col0 * (int64_t)sizeof(uint16_t)));
        const uint32_t halo_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)s_halo;
        const int wave_u = __builtin_amdgcn_readfirstlane(wave);  // uniform: scalar DMA branches
        const int n_ot = (args.cout_g + kBN - 1) / kBN;  // 128-channel tiles of the packing
        // Packed weights (sc_conv_weight_pack): per (group, 128-channel tile)
        // a block of K x nkc x 8 fragments; fragment (k, c, jj) is 64 lanes x
        // kWLane bytes, lane (l16, q4) holding w[tile*128 + 16 jj + l16, k,
        // 32c + 8 q4 .. +8]: one contiguous load per fragment and wave.
        constexpr uint32_t kFrag = 64u * kWLane;
        const uint32_t w_tile_bytes = (uint32_t)K * (uint32_t)nkc * 8u * kFrag;
        const __amdgpu_buffer_rsrc_t w_rsrc =
            make_rsrc(static_cast<const char *>(args.wpack) + kPackHeaderBytes,
                      (uint32_t)((int64_t)args.cin / args.cin_g * n_ot) * w_tile_bytes);
        const uint32_t w_lane = (uint32_t)(g * n_ot + (o0 >> 7)) * w_tile_bytes +
                                (uint32_t)((o0 & 127) / 16 + 4 * ch) * kFrag + (uint32_t)(lane * kWLane);
        const int n_halo_instr = (U + 15) >> 4;

        struct Cursor {
            uint32_t rem;
            int k, c;
        };
        auto cur_init = [&](Cursor &u) {
            u.rem = m_even;
            u.k = __builtin_ctz(m_even);
            u.c = 0;
        };
        auto cur_next = [&](Cursor &u) {
            u.rem &= u.rem - 1u;
            if (u.rem == 0u) {
                ++u.c;
                if constexpr (kKS) {
                    // bit arithmetic, not a select: the compiler would make a
                    // two-entry table of the masks in scratch memory
                    u.rem = m_even ^ ((m_even ^ m_odd) & (0u - (uint32_t)(u.c & 1)));
                } else {
                    u.rem = tmask;
                }
            }
            u.k = __builtin_ctz(u.rem);
        };
        uint4 wf[kWS][4];
        auto load_w = [&](const Cursor &u, uint4(&f)[4]) {
            const bool live = u.c < nkc;
            const uint32_t wk = w_lane + (uint32_t)((u.k * nkc + u.c) * 8) * kFrag;
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) f[jj] = bload16(w_rsrc, live ? wk + (uint32_t)jj * kFrag : kOobOffset);
        };
        // Halo DMA: instruction wave + 4*ii fills halo rows 16*(wave + 4*ii) + lane/4;
        // the lane moves logical piece hslot(j, lane%4) of row j.  Issued as
        // lds_dma16 (the compiler does not count it): the caller's
        // wait_vmcnt<0> is the wait, and no other vector-memory load is
        // issued between a halo load and that wait.
        auto load_halo = [&](int c) {
            const uint32_t cb = (uint32_t)(c * CB) + (uint32_t)(hslot(lane >> 2, lane & 3) * 16);
            // All source offsets first (rows < kPlanHaloMax, in bounds; those
            // past U are not used), so the LDS reads overlap.
            uint32_t hv[kHaloPerWave];
#pragma unroll
            for (int ii = 0; ii < kHaloPerWave; ++ii) hv[ii] = s_hoff[16 * (wave + 4 * ii) + (lane >> 2)];
#pragma unroll
            for (int ii = 0; ii < kHaloPerWave; ++ii) {
                const int instr = wave_u + 4 * ii;
                if (instr < n_halo_instr) {
                    const int j = 16 * instr + (lane >> 2);
                    const uint32_t off = j < U ? hv[ii] + cb : kOobOffset;
                    lds_dma16(a_rsrc, off, halo_lds + (uint32_t)instr * 1024u);
                }
            }
        };
        auto barrier = [&]() {
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            __builtin_amdgcn_s_barrier();
        };
        auto read_lm = [&](int k) { return *reinterpret_cast<const uint4 *>(&s_lmap[k][rh][l16][0]); };
        auto mfma_all = [&](const uint4(&x)[kIM], const uint4(&f)[4]) {
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const uint4 w = f[jj];
#pragma unroll
                for (int i = 0; i < kIM; ++i)
                    acc[i][jj] = mfma_16x16x32<TA>(w, x[i], acc[i][jj]);
            }
        };
        auto compute = [&](const uint4 &lm, const uint4(&f)[4]) {
            const uint32_t lw[4] = {lm.x, lm.y, lm.z, lm.w};
            const uint32_t qx = (uint32_t)q4 << 4;
            uint4 x[kIM];
#pragma unroll
            for (int i = 0; i < kIM; ++i) {
                const uint32_t off = ((i & 1) ? (lw[i >> 1] >> 16) : (lw[i >> 1] & 0xFFFFu)) ^ qx;
                x[i] = *reinterpret_cast<const uint4 *>(s_halo + off);
            }
            mfma_all(x, f);
        };

        if (direct) {
            // Operands from global memory, stage by stage (the same stage
            // order and accumulation as the halo path; no barrier, the
            // neighbour offsets are only read).
            if (m_even != 0u) {
                const uint32_t *dof = reinterpret_cast<const uint32_t *>(s_halo) + 128 * rh + l16;
                const __amdgpu_buffer_rsrc_t x_rsrc =
                    make_rsrc(input + in_col0, (uint32_t)(args.n_in * row_bytes - in_col0 * (int64_t)sizeof(uint16_t)));
                Cursor cur;
                cur_init(cur);
                while (cur.c < nkc) {
                    uint4 f[4];
                    load_w(cur, f);
                    const uint32_t cb = (uint32_t)(cur.c * CB + q4 * 16);
                    uint4 x[kIM];
#pragma unroll
                    for (int i = 0; i < kIM; ++i) x[i] = bload16(x_rsrc, dof[cur.k * kPlanTileRows + 16 * i] + cb);
                    mfma_all(x, f);
                    cur_next(cur);
                }
            }
        } else if (m_even == 0u) {
            // idle wave (stage split, one offset): its share of every halo
            // load and the same barriers as the others
            for (int c = 0; c < nkc; ++c) {
                if (c > 0) barrier();
                load_halo(c);
                wait_vmcnt<0>();
                barrier();
            }
        } else {
            Cursor cur, pre;
            cur_init(cur);
            cur_init(pre);
            uint4 lm[kWS];
#pragma unroll
            for (int s0 = 0; s0 < kWS - 1; ++s0) {
                load_w(pre, wf[s0]);
                lm[s0] = read_lm(pre.k);
                cur_next(pre);
            }
            load_halo(0);
            wait_vmcnt<0>();
            barrier();
            // Stage t uses weight set t % 2 and issues the loads of stage t + 1
            // into the other set; the body covers two stages so the sets are
            // compile-time constants.
            int prev_c = 0;
            while (true) {
                bool done = false;
#pragma unroll
                for (int u = 0; u < kWS; ++u) {
                    if (!done && cur.c >= nkc) done = true;
                    if (!done) {
                        if (cur.c != prev_c) {  // next chunk: every wave is done with the halo
                            barrier();
                            load_halo(cur.c);
                            wait_vmcnt<0>();
                            barrier();
                        }
                        load_w(pre, wf[(u + kWS - 1) % kWS]);
                        lm[(u + kWS - 1) % kWS] = read_lm(pre.k);
                        cur_next(pre);
                        compute(lm[u], wf[u]);
                        prev_c = cur.c;
                        cur_next(cur);
                    }
                }
                if (done) break;
            }
            wait_vmcnt<0>();
        }
    }
    if constexpr (kKS) {
        // The two waves of a row half add their partial sums: the wave of
        // parity p keeps row blocks [4p, 4p + 4) (tile rows 128 rh + 64 p ..,
        // its epilogue rows) and hands the other four to its partner, two
        // 16-channel blocks per round (32 KB of the halo's LDS).
        f32x4 *xb = reinterpret_cast<f32x4 *>(s_halo);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            __syncthreads();
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                for (int ii = 0; ii < 4; ++ii)
                    xb[((wave * 2 + jj) * 4 + ii) * 64 + lane] = kpar ? acc[ii][2 * r + jj] : acc[ii + 4][2 * r + jj];
            __syncthreads();
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    const f32x4 v = xb[(((wave ^ 1) * 2 + jj) * 4 + ii) * 64 + lane];
                    const f32x4 own = kpar ? acc[ii + 4][2 * r + jj] : acc[ii][2 * r + jj];
                    acc[ii][2 * r + jj] = own + v;
                    // computed here: sunk into the epilogue's branches, the
                    // sum would keep both halves and v live there
                    asm volatile("" : "+v"(acc[ii][2 * r + jj]));
                }
        }
        // nothing of the epilogue moves above the exchange (its loads would
        // be live beside the whole accumulator)
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- epilogue: lane l holds channels oc0 + 16 j + 4 q4 + e of tile row
    //      row0 + 16 i + l16; the lanes l16 + 16 m of the wave (kNT = 64) or
    //      of the two waves of a row half (kNT = 128) hold the whole row.
    TO *__restrict__ out = static_cast<TO *>(args.out);
    const TO *__restrict__ res = static_cast<const TO *>(args.residual);
    const bool vec_ok = args.vec_out != 0;
    const int oc0 = o0 + 64 * ch;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int o = oc0 + j * 16 + 4 * q4 + e;
            const bool ok = o < args.cout_g;
            const float bias = s_bias[o - o0], scale = s_scale[o - o0];
#pragma unroll
            for (int i = 0; i < kI; ++i)
                acc[i][j][e] = ok ? acc[i][j][e] * scale + bias : 0.f;
            __builtin_amdgcn_sched_barrier(0);
        }
    if constexpr (kLN) {
        // Two-pass f32 statistics over the row's Cout channels (the
        // reference's layer_norm_row_stats, wgpu/ops.rs:162-187).  Each wave
        // reduces its 64 channels over the 4 lanes of a row; with 128-channel
        // tiles the two channel halves meet in LDS (the halo's first 2 KB,
        // free once every wave has left the main loop) and are added in a
        // fixed order, so both waves hold the same statistics.
        float *red = reinterpret_cast<float *>(s_halo);  // [channel half][256 tile rows]
        auto row_total = [&](float(&part)[kI]) {
            if constexpr (kNT == 128) {
                __syncthreads();
#pragma unroll
                for (int i = 0; i < kI; ++i)
                    if (q4 == 0) red[ch * kPlanTileRows + row0 + 16 * i + l16] = part[i];
                __syncthreads();
#pragma unroll
                for (int i = 0; i < kI; ++i) {
                    const int r = row0 + 16 * i + l16;
                    part[i] = red[r] + red[kPlanTileRows + r];
                }
            }
        };
        // LayerNorm groups of 64 channels in a 128-channel tile (one C2S child
        // per wave half): each wave's statistics are its group's, no exchange.
        const bool half_groups = kNT == 128 && args.ln_group == 64;
        const float inv_c = 1.0f / (float)args.ln_group;
        float mean[kI], inv_std[kI], part[kI];
#pragma unroll
        for (int i = 0; i < kI; ++i) {
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) sum += acc[i][j][e];
            sum += __shfl_xor(sum, 16, 64);
            sum += __shfl_xor(sum, 32, 64);
            part[i] = sum;
        }
        if (!half_groups) row_total(part);
#pragma unroll
        for (int i = 0; i < kI; ++i) mean[i] = part[i] * inv_c;
#pragma unroll
        for (int i = 0; i < kI; ++i) {
            float qv = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int o = oc0 + j * 16 + 4 * q4 + e;
                    const float d = acc[i][j][e] - mean[i];
                    qv += o < args.cout_g ? d * d : 0.f;
                }
            qv += __shfl_xor(qv, 16, 64);
            qv += __shfl_xor(qv, 32, 64);
            part[i] = qv;
        }
        if (!half_groups) row_total(part);
#pragma unroll
        for (int i = 0; i < kI; ++i) inv_std[i] = rsqrt_f32(part[i] * inv_c + args.ln_eps);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int o = oc0 + j * 16 + 4 * q4 + e;
                const bool ok = o < args.cout_g;
                const int og = o % args.ln_group;  // channel within the LayerNorm group
                const float lw = (args.ln_w && ok) ? args.ln_w[og] : 1.f;
                const float lb = (args.ln_b && ok) ? args.ln_b[og] : 0.f;
#pragma unroll
                for (int i = 0; i < kI; ++i) acc[i][j][e] = (acc[i][j][e] - mean[i]) * inv_std[i] * lw + lb;
                __builtin_amdgcn_sched_barrier(0);
            }
    }
    // Stores: the residual of kRG row blocks (4 for bf16, 2 for f32 outputs)
    // is fetched before any of them is written, so its latency overlaps
    // instead of serialising per block.
    constexpr int kRG = sizeof(TO) == 2 ? 4 : 2;
    int32_t qrow[kI];
#pragma unroll
    for (int i = 0; i < kI; ++i) {
        const int32_t q = s_order[row0 + 16 * i + l16];
        qrow[i] = q < args.n_q ? q : -1;  // -1 pads the order; nothing past n_q is written
    }
    if (args.scatter_rows || args.skip_idx) {
#pragma unroll
        for (int i = 0; i < kI; ++i) {
            if (qrow[i] < 0) continue;
            const C2SRow crow = c2s_row<TO>(args, qrow[i]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int oc = oc0 + j * 16 + 4 * q4;
                if (oc >= args.cout_g) continue;
                float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
                if (args.silu) {
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc) v[cc] = silu_f32(v[cc]);
                }
                c2s_store4<TO, !kLN>(args, crow, qrow[i], (int)(out_col0 + oc), min(4, args.cout_g - oc), v, vec_ok);
            }
            // one row block at a time: loads hoisted across blocks would
            // hold their registers beside the whole accumulator
            __builtin_amdgcn_sched_barrier(0);
        }
        return;
    }
#pragma unroll
    for (int ih = 0; ih < kI; ih += kRG) {
        typename Out4<TO>::V rv[kRG][4];
        if (res && vec_ok) {
#pragma unroll
            for (int ii = 0; ii < kRG; ++ii)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int oc = oc0 + j * 16 + 4 * q4;
                    if (qrow[ih + ii] >= 0 && oc + 3 < args.cout_g)
                        rv[ii][j] = *reinterpret_cast<const typename Out4<TO>::V *>(
                            res + (int64_t)qrow[ih + ii] * args.cout + out_col0 + oc);
                }
        }
#pragma unroll
        for (int ii = 0; ii < kRG; ++ii) {
            const int i = ih + ii;
            if (qrow[i] < 0) continue;
            const int64_t rowbase = (int64_t)qrow[i] * args.cout + out_col0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int oc = oc0 + j * 16 + 4 * q4;
                float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
                if (args.silu) {
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc) v[cc] = silu_f32(v[cc]);
                }
                if (vec_ok && oc + 3 < args.cout_g) {
                    if (res) {
                        float r4[4];
                        Out4<TO>::unpack(rv[ii][j], r4);
#pragma unroll
                        for (int cc = 0; cc < 4; ++cc) v[cc] += r4[cc];
                    }
                    *reinterpret_cast<typename Out4<TO>::V *>(out + rowbase + oc) = Out4<TO>::pack(v);
                } else {
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc) {
                        if (oc + cc >= args.cout_g) continue;
                        float t = v[cc];
                        if (res) t += load_as_f32<TO>(res, rowbase + oc + cc);
                        store_from_f32<TO>(out, rowbase + oc + cc, t);
                    }
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// ----------------------------------------------------------- dense linear
//
// The dense layer out = x W^T + b (the decoder's linear layers, and the 2x2x2
// transposed upsample as a linear Cin -> 8 Cout with the child scatter: a
// 1x1x1 conv without a map, query row r reading input row r) as an
// LDS-pipelined GEMM.
// A tile of 256 rows x 64 kQ output channels steps through the input
// channels 32 at a time: each k-step's rows (256 x 64 B) and weights (64 kQ
// channels x 64 B of W [Cout][Cin], the reference layout) are DMA'd into one
// of kBuf LDS buffers kBuf - 1 k-steps ahead, one barrier per k-step; waves
// 2 x kQ (128 rows x 64 channels each) read their MFMA fragments from LDS,
// 16-byte pieces XOR-swizzled per row (wslot) so that the reads of 8
// consecutive rows hit distinct banks.  kQ = 2: 128-channel tiles, 3
// buffers (72 KB), two workgroups per CU; kQ = 4 (129-256 output channels,
// no LayerNorm): one 256-channel tile per row, 4 buffers (128 KB), one
// workgroup of 8 waves per CU.  Same epilogue layout as the halo kernel:
// lane (l16, q4) holds channels oc0 + 16 j + 4 q4 .. +4 of row
// row0 + 16 i + l16.
template <int kQ>
struct DenseShape {
    static constexpr int kThreads = 128 * kQ;
    static constexpr int kWaves = 2 * kQ;
    static constexpr int kCols = 64 * kQ;         // output channels per tile
    static constexpr int kBuf = kQ == 2 ? 3 : 4;  // LDS stage buffers
    static constexpr int kBlocksPerCU = kQ == 2 ? 2 : 1;
};

// kListed: the rows come from a linear child plan (sc_linear_child_plan_build):
// tile t holds up to 256 parents whose child tile_child[t] is active (perm, -1
// pads), and computes only that child's channels, so inactive children cost
// nothing; a row's values are the same sums as without the plan.
template <typename TA, typename TO, bool kLN, int kQ, bool kStaged, bool kListed = false>
__global__ __launch_bounds__(DenseShape<kQ>::kThreads, DenseShape<kQ>::kBlocksPerCU) void dense_gemm_kernel(
    ConvArgs args)
{
    using S = DenseShape<kQ>;
    constexpr int kI = 8;                             // 16-row MFMA blocks per wave
    constexpr int kBuf = S::kBuf;
    constexpr int kRowsBytes = kTileRows * 64;        // one k-step of rows
    constexpr int kWBytes = S::kCols * 64;            // one k-step of weights
    constexpr int kStage = kRowsBytes + kWBytes;      // 24 or 32 KB
    constexpr int kAInstr = kRowsBytes / 1024 / S::kWaves;  // 1 KB DMA instructions per wave and k-step
    constexpr int kWInstr = kWBytes / 1024 / S::kWaves;
    constexpr int kPerStep = kAInstr + kWInstr;
    static_assert(kAInstr * 1024 * S::kWaves == kRowsBytes && kWInstr * 1024 * S::kWaves == kWBytes, "DMA split");
    __shared__ __attribute__((aligned(16))) unsigned char s_buf[kBuf * kStage];  // stages; then the output tile
    __shared__ float s_red[kQ][kTileRows];            // LayerNorm: per channel quarter, per tile row
    __shared__ int32_t s_rows[kListed ? kTileRows : 1];  // listed: the tile's parents (-1: none)
    auto stage = [&](int u) -> unsigned char * { return s_buf + u * kStage; };

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, q4 = lane >> 4;
    const int rh = wave / kQ, qc = wave % kQ;         // row half, channel quarter
    // Block b (dealt to the XCDs in contiguous ranges) is column tile b % n_ct
    // of row tile b / n_ct: a row tile's column tiles run together on one
    // XCD, so its rows come from HBM once and from L2 for the other columns
    // (otherwise each column tile re-reads every row from HBM).
    int64_t trow0 = 0;  // the tile's first row (unlisted)
    int o0;             // the tile's first channel
    if constexpr (kListed) {
        // the plan's list tiles in use, each with child_ch / kCols column
        // tiles of its child, dealt to the XCDs as one range; the plan must
        // be the one built for these parents
        if (!plan_matches(args.plan_hdr, args) || args.plan_hdr->status != 0u) return;
        const int n_ct = args.child_ch / S::kCols;
        const int n_real = args.plan_hdr->n_unique * n_ct;
        if ((int)blockIdx.x >= n_real) return;
        const int b = tile_for_block(blockIdx.x, n_real);
        const int lt = b / n_ct;
        const int child = args.tile_child[lt];
        if (child < 0) return;
        o0 = child * args.child_ch + (b % n_ct) * S::kCols;
        if (tid < kTileRows) {
            const int32_t p = args.perm[(int64_t)lt * kTileRows + tid];
            s_rows[tid] = p >= 0 && p < args.n_q ? p : -1;
        }
        __syncthreads();
    } else {
        const int n_ct = (args.cout_g + S::kCols - 1) / S::kCols;
        const int b = tile_for_block(blockIdx.x, gridDim.x);
        trow0 = (int64_t)(b / n_ct) * kTileRows;
        o0 = (b % n_ct) * S::kCols;
    }
    // input row of tile row rl (-1: none)
    auto tile_row = [&](int rl) -> int64_t {
        if constexpr (kListed) return s_rows[rl];
        const int64_t r = trow0 + rl;
        return r < args.n_q ? r : -1;
    };
    const int cin = (int)args.cin;
    const int nk = cin / 32;
    const i32x4_rsrc a_rsrc = rsrc_words(args.input, (uint32_t)(args.n_q * (int64_t)cin * (int64_t)sizeof(TA)));
    const i32x4_rsrc w_rsrc = rsrc_words(args.weight, (uint32_t)((int64_t)args.cout_g * cin * (int64_t)sizeof(TA)));

    // DMA sources: instruction t of this wave fills LDS bytes [1 KB * (wave +
    // kWaves t), +1 KB) of the rows (or weights) region: 16 rows (channels) x
    // 4 slots; lane L writes row 16 (wave + kWaves t) + L / 4, slot L % 4, and
    // loads the logical piece stored there.  Rows past n_q and channels past
    // Cout read zero.
    uint32_t a_src[kAInstr], w_src[kWInstr];
#pragma unroll
    for (int t = 0; t < kAInstr; ++t) {
        const int r = 16 * (wave + S::kWaves * t) + (lane >> 2);
        const int piece = wslot<64>(r, lane & 3);
        const int64_t row = tile_row(r);
        a_src[t] = row >= 0 ? (uint32_t)((row * cin + 8 * piece) * (int64_t)sizeof(TA)) : kOobOffset;
    }
#pragma unroll
    for (int t = 0; t < kWInstr; ++t) {
        const int c = 16 * (wave + S::kWaves * t) + (lane >> 2);
        const int piece = wslot<64>(c, lane & 3);
        const int o = o0 + c;
        w_src[t] = o < args.cout_g ? (uint32_t)(((int64_t)o * cin + 8 * piece) * (int64_t)sizeof(TA)) : kOobOffset;
    }
    const uint32_t wave_kb = (uint32_t)__builtin_amdgcn_readfirstlane(1024 * wave);  // uniform
    auto dma = [&](int k, int buf) {
        const uint32_t step = (uint32_t)(k * 32 * (int)sizeof(TA));  // an out-of-range offset stays out of range
        const uint32_t lds =
            (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)stage(buf) + wave_kb;
#pragma unroll
        for (int t = 0; t < kAInstr; ++t) lds_dma16(a_rsrc, a_src[t] + step, lds + 1024 * S::kWaves * t);
#pragma unroll
        for (int t = 0; t < kWInstr; ++t)
            lds_dma16(w_rsrc, w_src[t] + step, lds + kRowsBytes + 1024 * S::kWaves * t);
    };

    f32x4 acc[kI][4];
#pragma unroll
    for (int i = 0; i < kI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][e] = 0.f;

    // This lane's fragment offsets in a stage: row 128 rh + 16 i + l16 and
    // weight channel 64 qc + 16 j + l16 sit 1 KB apart per i (j), their
    // swizzled slot fixed (wslot reads bits 1-3 of the row).  Kept opaque,
    // so each fragment address is this offset plus a constant (otherwise the
    // compiler holds every buffer's addresses in registers, and spills).
    int xoff = (128 * rh + l16) * 64 + wslot<64>(128 * rh + l16, q4) * 16;
    int woff = kRowsBytes + (64 * qc + l16) * 64 + wslot<64>(64 * qc + l16, q4) * 16;
    asm("" : "+v"(xoff));
    asm("" : "+v"(woff));
    // k-step k on buffer u: read its fragments, start the DMA of k + kBuf - 1
    // (into the buffer every wave finished at k - 1), then the MFMAs.
    auto step = [&](int u, int k) {
        const unsigned char *base = stage(u);
        uint4 x[kI], w[4];
#pragma unroll
        for (int i = 0; i < kI; ++i) x[i] = *reinterpret_cast<const uint4 *>(base + xoff + 1024 * i);
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = *reinterpret_cast<const uint4 *>(base + woff + 1024 * j);
        __builtin_amdgcn_sched_barrier(0);
        if (k + kBuf - 1 < nk) dma(k + kBuf - 1, (u + kBuf - 1) % kBuf);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < kI; ++i) acc[i][j] = mfma_16x16x32<TA>(w[j], x[i], acc[i][j]);
    };
    // k-step k uses buffer k % kBuf.  At its top, steps k .. min(k + kBuf -
    // 2, nk - 1) are in flight: wait until only the younger ones are (the
    // DMAs complete in issue order; no other vector memory operation is
    // outstanding in the loop), barrier (every wave's DMA of k has landed and
    // every wave is done with k - 1's buffer), then step.  The DMAs are inline
    // asm, which the compiler does not track: these waits are the only ones.
    // The main loop runs the k-steps that have kBuf - 2 younger steps in
    // flight, unrolled by kBuf so the buffers are constants; the tail (fewer
    // than 2 kBuf - 2 steps) waits for what is left.
    for (int k = 0; k < kBuf - 1; ++k)
        if (k < nk) dma(k, k);
    int k0 = 0;
    for (; k0 + 2 * kBuf - 2 <= nk; k0 += kBuf) {
#pragma unroll
        for (int u = 0; u < kBuf; ++u) {
            wait_vmcnt<(kBuf - 2) * kPerStep>();
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            __builtin_amdgcn_s_barrier();
            step(u, k0 + u);
        }
    }
#pragma unroll
    for (int u = 0; u < 2 * kBuf - 2; ++u) {
        const int k = k0 + u;
        if (k >= nk) break;
        const int younger = min(kBuf - 2, nk - 1 - k);  // steps after k already issued
        if (younger >= 2)
            wait_vmcnt<2 * kPerStep>();
        else if (younger == 1)
            wait_vmcnt<kPerStep>();
        else
            wait_vmcnt<0>();
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        step(u % kBuf, k);
    }

    // ---- epilogue: bias, LayerNorm (over the row or one child; the channel
    //      quarters of a group meet in LDS), SiLU, residual, stores
    //      (row-major, or each child's slice to its row in the child scatter).
    const int oc0 = o0 + 64 * qc;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int o = oc0 + j * 16 + 4 * q4 + e;
            const bool ok = o < args.cout_g;
            const float bias = (args.bias && ok) ? args.bias[o] : 0.f;
#pragma unroll
            for (int i = 0; i < kI; ++i) acc[i][j][e] = ok ? acc[i][j][e] + bias : 0.f;
        }
    if constexpr (kLN) {
        // ln_group channels per normalised row: the whole row (<= 128), or in
        // the child scatter one child's 64 (one wave's quarter) or 128 (two
        // quarters); the gq quarters of a group add their partial sums in a
        // fixed order, so they all hold the same statistics.
        const int gq = (args.ln_group + 63) / 64;
        const int g0 = qc - qc % gq;                 // first quarter of this wave's group
        const int trow = 128 * rh + l16;             // tile row of block 0
        auto row_total = [&](float(&part)[kI]) {
            __syncthreads();
#pragma unroll
            for (int i = 0; i < kI; ++i)
                if (q4 == 0) s_red[qc][trow + 16 * i] = part[i];
            __syncthreads();
#pragma unroll
            for (int i = 0; i < kI; ++i) {
                float t = 0.f;
                for (int q = 0; q < gq; ++q) t += s_red[g0 + q][trow + 16 * i];
                part[i] = t;
            }
        };
        const float inv_c = 1.0f / (float)args.ln_group;
        float mean[kI], inv_std[kI], part[kI];
#pragma unroll
        for (int i = 0; i < kI; ++i) {
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) sum += acc[i][j][e];
            sum += __shfl_xor(sum, 16, 64);
            sum += __shfl_xor(sum, 32, 64);
            part[i] = sum;
        }
        if (gq > 1) row_total(part);
#pragma unroll
        for (int i = 0; i < kI; ++i) mean[i] = part[i] * inv_c;
#pragma unroll
        for (int i = 0; i < kI; ++i) {
            float qv = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int o = oc0 + j * 16 + 4 * q4 + e;
                    const float d = acc[i][j][e] - mean[i];
                    qv += o < args.cout_g ? d * d : 0.f;
                }
            qv += __shfl_xor(qv, 16, 64);
            qv += __shfl_xor(qv, 32, 64);
            part[i] = qv;
        }
        if (gq > 1) row_total(part);
#pragma unroll
        for (int i = 0; i < kI; ++i) inv_std[i] = rsqrt_f32(part[i] * inv_c + args.ln_eps);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int o = oc0 + j * 16 + 4 * q4 + e;
                const bool ok = o < args.cout_g;
                const int og = o % args.ln_group;  // channel within the LayerNorm group
                const float lw = (args.ln_w && ok) ? args.ln_w[og] : 1.f;
                const float lb = (args.ln_b && ok) ? args.ln_b[og] : 0.f;
#pragma unroll
                for (int i = 0; i < kI; ++i) acc[i][j][e] = (acc[i][j][e] - mean[i]) * inv_std[i] * lw + lb;
            }
    }
    TO *__restrict__ out = static_cast<TO *>(args.out);
    if constexpr (kStaged) {
        // 16-bit output, counts and pointers 16-byte aligned (host): the
        // tile goes through the idle stage buffers, rounded once (after the
        // residual, added here in f32), so that every store instruction
        // writes whole 16-byte pieces of consecutive rows (a lane's own
        // layout scatters 8-byte pieces over 16 rows per store, which costs
        // the store path several times the bytes' time).  Tile row rl sits at
        // rl * kRB, its 16-byte piece c in slot c ^ (rl % kNC), so neither
        // phase has more bank conflicts than its bytes need.
        static_assert(sizeof(TO) == 2, "16-bit output");
        constexpr int kRB = S::kCols * 2;  // bytes of a tile row
        constexpr int kNC = kRB / 16;      // 16-byte pieces per tile row
        static_assert(kTileRows * kRB <= kBuf * kStage, "output tile fits the stage buffers");
        const TO *__restrict__ res = static_cast<const TO *>(args.residual);
        __syncthreads();  // every wave is done with the last stage's fragments
#pragma unroll
        for (int i = 0; i < kI; ++i) {
            const int rl = 128 * rh + 16 * i + l16;
            const int64_t r = tile_row(rl);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
                if (args.silu) {
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc) v[cc] = silu_f32(v[cc]);
                }
                const int oc = oc0 + j * 16 + 4 * q4;
                if (res && r >= 0 && oc < args.cout_g) {
                    float r4[4];
                    Out4<TO>::unpack(*reinterpret_cast<const typename Out4<TO>::V *>(res + r * args.cout + oc), r4);
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc) v[cc] += r4[cc];
                }
                const int c = 8 * qc + 2 * j + (q4 >> 1);
                *reinterpret_cast<typename Out4<TO>::V *>(s_buf + rl * kRB + ((c ^ (rl & (kNC - 1))) << 4) +
                                                          8 * (q4 & 1)) = Out4<TO>::pack(v);
            }
        }
        __syncthreads();
#pragma unroll 4
        for (int it = 0; it < kTileRows * kNC / S::kThreads; ++it) {
            const int idx = it * S::kThreads + tid;
            const int rl = idx / kNC, c = idx % kNC;
            const int64_t r = tile_row(rl);
            const int col = o0 + 8 * c;  // first of the piece's 8 channels
            if (r < 0 || col >= args.cout_g) continue;
            const uint4 val = *reinterpret_cast<const uint4 *>(s_buf + rl * kRB + ((c ^ (rl & (kNC - 1))) << 4));
            int64_t off;
            if (args.scatter_rows) {
                const int child = args.scatter_shift >= 0 ? col >> args.scatter_shift : col / args.scatter_ch;
                const int32_t cr = args.scatter_rows[r * 8 + child];
                if (cr < 0 || cr >= args.scatter_n) continue;
                off = (int64_t)cr * args.scatter_ch + (col - child * args.scatter_ch);
            } else {
                off = r * args.cout + col;
            }
            *reinterpret_cast<uint4 *>(out + off) = val;
        }
        return;
    }
    const TO *__restrict__ res = static_cast<const TO *>(args.residual);
    const bool vec_ok = args.vec_out != 0;
#pragma unroll
    for (int i = 0; i < kI; ++i) {
        const int64_t r = tile_row(128 * rh + 16 * i + l16);
        if (r < 0) continue;
        const int64_t rowbase = r * args.cout;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int oc = oc0 + j * 16 + 4 * q4;
            if (oc >= args.cout_g) continue;
            float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
            if (args.silu) {
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) v[cc] = silu_f32(v[cc]);
            }
            if (args.scatter_rows) {
                c2s_store4<TO, false>(args, C2SRow{nullptr}, r, oc, min(4, args.cout_g - oc), v, vec_ok);
            } else if (vec_ok && oc + 3 < args.cout_g) {
                if (res) {
                    float r4[4];
                    Out4<TO>::unpack(*reinterpret_cast<const typename Out4<TO>::V *>(res + rowbase + oc), r4);
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc) v[cc] += r4[cc];
                }
                *reinterpret_cast<typename Out4<TO>::V *>(out + rowbase + oc) = Out4<TO>::pack(v);
            } else {
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    if (oc + cc >= args.cout_g) continue;
                    float t = v[cc];
                    if (res) t += load_as_f32<TO>(res, rowbase + oc + cc);
                    store_from_f32<TO>(out, rowbase + oc + cc, t);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// --------------------------------------------------------- weight packing
//
// The halo-staged kernel's weight layout: per (group g, 128-channel output
// tile ot, offset k, 32-channel input chunk c, 16-channel block jj) one
// fragment of 64 lanes; lane (l16, q4) holds the 8 weights
// w[g, ot*128 + 16 jj + l16, k, 32c + 8 q4 .. +8] as bf16 (16 B; int8 weights
// are widened exactly, their per-channel scales stay [Cout] f32 and are
// applied in the conv's epilogue), zero for channels beyond Cout_g.  Same role as the reference's
// pack_flex_weight (crates/burn_flex_gmm/src/lib.rs:377-426): a one-time
// per-layer reorder so that the conv's weight reads are contiguous.
template <typename TS>
__global__ void pack_weights_kernel(const TS *__restrict__ w, unsigned char *__restrict__ buf, int groups,
                                    int cout_g, int cin_g, int K, int src_dtype, int64_t bytes)
{
    const int nkc = cin_g / 32, n_ot = (cout_g + kBN - 1) / kBN;
    const int64_t pieces = (int64_t)groups * n_ot * K * nkc * 8 * 64;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        PackHeader *h = reinterpret_cast<PackHeader *>(buf);
        h->magic = kPackMagic;
        h->groups = groups;
        h->cout_g = cout_g;
        h->cin_g = cin_g;
        h->K = K;
        h->src_dtype = src_dtype;
        h->n_ot = n_ot;
        h->pad0 = 0;
        h->bytes = bytes;
    }
    uint16_t *dst = reinterpret_cast<uint16_t *>(buf + kPackHeaderBytes);
    for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < pieces;
         p += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(p & 63);
        int64_t r = p >> 6;
        const int jj = (int)(r % 8);
        r /= 8;
        const int c = (int)(r % nkc);
        r /= nkc;
        const int k = (int)(r % K);
        r /= K;
        const int ot = (int)(r % n_ot);
        const int g = (int)(r / n_ot);
        const int o = ot * kBN + 16 * jj + (lane & 15);
        const int i0 = 32 * c + 8 * (lane >> 4);
        uint16_t *d = dst + p * 8;
        if (o < cout_g) {
            const TS *s = w + (((int64_t)g * cout_g + o) * K + k) * cin_g + i0;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if constexpr (sizeof(TS) == 1)
                    d[e] = f32_to_bf16((float)s[e]);  // exact: |q| <= 128
                else
                    d[e] = __builtin_bit_cast(uint16_t, s[e]);  // bf16 or f16 bits, unchanged
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) d[e] = 0;
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
            const int32_t nb = args.map ? args.map[r * args.K + k] : (int32_t)r;  // no map: dense linear
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
        if (args.silu) v = silu_f32(v);
        if (args.scatter_rows || args.skip_idx) {
            const float v4[4] = {v, 0.f, 0.f, 0.f};
            c2s_store4<TO>(args, c2s_row<TO>(args, r), r, (int)o, 1, v4, false);
            continue;
        }
        if (res) v += load_as_f32<TO>(res, e);
        store_from_f32<TO>(out, e, v);
    }
}

// 16-bit activations through the v2 tile: 128-byte stages when the group's
// input channels allow it, else 64-byte stages with a deeper A prefetch.
// int8 weights always take the 64-byte stages: their register staging of the
// widened pieces does not fit beside the 128-byte stage's operands (the
// 128-byte int8 variant spilled), so it is not instantiated.
template <typename TA, typename TW, typename TO>
void launch_v2(const ConvArgs &a, dim3 grid, hipStream_t s)
{
    if constexpr (sizeof(TW) == 2) {
        if (a.cin_g % 64 == 0) {
            conv_v2_kernel<TA, TW, TO, 128, 1><<<grid, kThreads, 0, s>>>(a);
            return;
        }
    }
    conv_v2_kernel<TA, TW, TO, 64, 2><<<grid, kThreads, 0, s>>>(a);
}

template <typename TA, typename TW, typename TO>
int launch_conv(const ConvArgs &a, int groups, bool mfma, const void *plan, hipStream_t s)
{
    if (mfma) {
        const bool wide = a.cin_g % (128 / (int)sizeof(TA)) == 0;
        const int64_t tiles = (a.n_q + kTileRows - 1) / kTileRows;
        const int64_t ntile = (a.cout_g + kBN - 1) / kBN;
        if (tiles > INT32_MAX || ntile > 65535 || groups > 65535)
            return fail(SC_ERR_OVERFLOW, "sparse conv grid overflow");
        dim3 grid((unsigned)tiles, (unsigned)ntile, (unsigned)groups);
        if constexpr (sizeof(TA) == 2) {
            if (plan && a.wpack) {
                // Halo-staged tiles (a tile whose halo overflowed gathers
                // its operands from global memory in the same launch).
                // Packed weights are bf16 for either weight type; int8
                // weights keep their per-channel scales for the epilogue.
                // A child plan (C2S conv1 over the active children): its own
                // tile count, and one tile per child and column block of the
                // child's channels.
                PlanView pv;
                int64_t n_tiles;
                if (a.child_plan) {
                    const ChildPlanLayout CL = child_plan_layout(a.n_q, a.scatter_n, a.K);
                    pv = child_plan_view(plan, CL);
                    n_tiles = CL.n_tiles;
                } else {
                    const PlanLayout L = plan_layout(a.n_q, a.K);
                    pv = plan_view(plan, L);
                    n_tiles = L.n_tiles;
                }
                const int64_t cols = a.child_plan ? a.child_ch : a.cout_g;  // channels one tile row spans
                dim3 hgrid((unsigned)n_tiles, (unsigned)((cols + kBN - 1) / kBN), (unsigned)groups);
                ConvArgs h = a;
                h.plan_hdr = pv.hdr;
                h.tile_child = pv.tile_child;
                if (sizeof(TW) != 1) h.w_scale = nullptr;
                if (cols <= 64) {  // 64-channel tiles: no half-empty MFMA tile
                    hgrid.y = (unsigned)((cols + 63) / 64);
                    if (a.ln)
                        conv_halo_kernel<TA, TO, true, 64><<<hgrid, kThreads, 0, s>>>(h, pv);
                    else
                        conv_halo_kernel<TA, TO, false, 64><<<hgrid, kThreads, 0, s>>>(h, pv);
                } else if (a.ln) {
                    conv_halo_kernel<TA, TO, true, 128><<<hgrid, kThreads, 0, s>>>(h, pv);
                } else {
                    conv_halo_kernel<TA, TO, false, 128><<<hgrid, kThreads, 0, s>>>(h, pv);
                }
                SC_LAUNCH_CHECK("conv_halo_kernel launch");
            } else if (sizeof(TW) == 2 && !a.map && a.K == 1 && groups == 1 && a.cin % 32 == 0 && !a.skip_idx) {
                // the dense linear: contiguous rows, reference-layout weights;
                // row tile x column tile flattened, column tile fastest;
                // one 256-channel tile for 129-256 output channels (the rows
                // are read once); 128-channel tiles otherwise, two workgroups
                // per CU, so one's epilogue stores overlap the other's
                // MFMAs (measured faster once a row spans several column
                // tiles); never with LayerNorm, whose statistics do not fit
                // the wide tile's registers
                const bool wide_tile = a.cout_g > 128 && a.cout_g <= 256 && !a.ln;
                const int64_t ncol = (a.cout_g + (wide_tile ? 255 : 127)) / (wide_tile ? 256 : 128);
                if (tiles * ncol > INT32_MAX) return fail(SC_ERR_OVERFLOW, "dense linear grid overflow");
                const dim3 dgrid((unsigned)(tiles * ncol), 1, 1);
                // row-contiguous stores through LDS: 16-bit output, 8-channel
                // pieces aligned in the output rows, residual aligned
                const bool staged = sizeof(TO) == 2 && a.cout % 8 == 0 && (uintptr_t)a.out % 16 == 0 &&
                                    (uintptr_t)a.residual % 16 == 0 && (!a.scatter_rows || a.scatter_ch % 8 == 0);
                if (plan && a.child_plan) {
                    // the transposed upsample over the active children only: a
                    // linear child plan's list tiles (sc_linear_child_plan_build),
                    // 128-channel column tiles of each tile's child
                    const ChildPlanLayout CL = child_plan_layout(a.n_q, a.scatter_n, 1);
                    const PlanView pv = child_plan_view(plan, CL);
                    ConvArgs h = a;
                    h.plan_hdr = pv.hdr;
                    h.perm = pv.order;
                    h.tile_child = pv.tile_child;
                    const int64_t lgrid = CL.n_main * (a.child_ch / 128);
                    if (lgrid > INT32_MAX) return fail(SC_ERR_OVERFLOW, "dense linear grid overflow");
                    const dim3 lg((unsigned)lgrid, 1, 1);
                    if (a.ln) {
                        if (staged)
                            dense_gemm_kernel<TA, TO, true, 2, sizeof(TO) == 2, true><<<lg, DenseShape<2>::kThreads, 0, s>>>(h);
                        else
                            dense_gemm_kernel<TA, TO, true, 2, false, true><<<lg, DenseShape<2>::kThreads, 0, s>>>(h);
                    } else {
                        if (staged)
                            dense_gemm_kernel<TA, TO, false, 2, sizeof(TO) == 2, true><<<lg, DenseShape<2>::kThreads, 0, s>>>(h);
                        else
                            dense_gemm_kernel<TA, TO, false, 2, false, true><<<lg, DenseShape<2>::kThreads, 0, s>>>(h);
                    }
                    SC_LAUNCH_CHECK("dense_gemm_kernel launch (child plan)");
                    return SC_OK;
                }
                if (wide_tile) {
                    if (staged)
                        dense_gemm_kernel<TA, TO, false, 4, sizeof(TO) == 2><<<dgrid, DenseShape<4>::kThreads, 0, s>>>(a);
                    else
                        dense_gemm_kernel<TA, TO, false, 4, false><<<dgrid, DenseShape<4>::kThreads, 0, s>>>(a);
                } else if (a.ln) {
                    if (staged)
                        dense_gemm_kernel<TA, TO, true, 2, sizeof(TO) == 2><<<dgrid, DenseShape<2>::kThreads, 0, s>>>(a);
                    else
                        dense_gemm_kernel<TA, TO, true, 2, false><<<dgrid, DenseShape<2>::kThreads, 0, s>>>(a);
                } else {
                    if (staged)
                        dense_gemm_kernel<TA, TO, false, 2, sizeof(TO) == 2><<<dgrid, DenseShape<2>::kThreads, 0, s>>>(a);
                    else
                        dense_gemm_kernel<TA, TO, false, 2, false><<<dgrid, DenseShape<2>::kThreads, 0, s>>>(a);
                }
                SC_LAUNCH_CHECK("dense_gemm_kernel launch");
            } else {
                launch_v2<TA, TW, TO>(a, grid, s);
            }
        } else {
            if (wide)
                conv_mfma_kernel<TA, TW, TO, 128><<<grid, kThreads, 0, s>>>(a);
            else
                conv_mfma_kernel<TA, TW, TO, 64><<<grid, kThreads, 0, s>>>(a);
        }
        SC_LAUNCH_CHECK("conv_mfma_kernel launch");
    } else {
        conv_scalar_kernel<TA, TW, TO><<<grid_for(a.n_q * a.cout, 256, 65536), 256, 0, s>>>(a);
        SC_LAUNCH_CHECK("conv_scalar_kernel launch");
    }
    return SC_OK;
}

}  // namespace

// The f16 instantiations (sc_conv_f16.hip): f16 activations and weights,
// output f16 or f32.
int launch_conv_f16(const ConvArgs &a, int out_dtype, int groups, bool mfma, const void *plan, hipStream_t s);
// The int8-weight instantiations (sc_conv_i8.hip): bf16 activations, int8
// weights with per-output-channel scales, output bf16 or f32.
int launch_conv_i8(const ConvArgs &a, int out_dtype, int groups, bool mfma, const void *plan, hipStream_t s);

}  // namespace sc
