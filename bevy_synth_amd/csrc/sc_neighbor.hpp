// Layout of the neighbour-map workspace (header, bbox partials, offset table,
// cell table) and the dense-grid / rank-bitmap lookups of the map build.
#pragma once

#include "sc_common.hpp"

namespace sc {
namespace nbr {

constexpr size_t kHeaderBytes = 256;
constexpr uint64_t kEmpty64 = ~0ull;
constexpr uint32_t kStatusNegative = 1u;
// Dense grid: some cell received more than one row (duplicate coords). Not an
// error; the query then maps row by row, since the grid names one row per cell.
constexpr uint32_t kStatusDupCell = 2u;
constexpr int kMaxStagedOffsets = 512;

// Table budgets, in bbox cells, that the workspace affords: the dense grid
// (4 B per cell, at most 32 cells per row) and the rank bitmap (8 B per 32 cells).
struct Limits {
    uint64_t dense_cells;
    uint64_t bitmap_cells;
};

struct Plan {
    int mode;  // 0: no table (error), 1: 32-bit keys packed with rows, 2: 64-bit keys,
               // 3: row-only table compared through the coords, 4: dense grid,
               // 5: rank bitmap (rows strictly increasing in rank_key)
    int levels;      // mode 5: octree levels of the key (0: the plain (b, x, y, z) order)
    uint64_t total;  // table cells (valid for modes 1, 2, 4, 5)
    int32_t lo[4];
    int32_t hi[4];
    uint64_t ext[4];
    int32_t rlo[4];   // mode 5: the root cells' bbox (lo >> levels; batch unchanged)
    uint64_t rext[4]; //         and its extents
};

struct alignas(16) NbrHeader {
    int32_t bmin[4];
    int32_t bmax[4];
    uint32_t status;
    uint32_t unsorted;  // bit L set unless the rows are strictly increasing in the L-level key
    int32_t mode;       // the table mode chosen (Plan::mode), a diagnostic for callers
    uint32_t pad0;
    Plan plan;          // derived once from the fields above, read by every later kernel
    uint8_t pad[kHeaderBytes - 48 - sizeof(Plan)];
};
static_assert(sizeof(NbrHeader) == kHeaderBytes, "header size");

constexpr size_t kPartialBytes = 1024 * 10 * 4;  // bbox partials (kBboxBlocks x 10 ints)
constexpr size_t kOffsetTableBytes = kMaxStagedOffsets * 16;  // per offset {dx, dy, dz, cell delta}
constexpr size_t kFixedBytes = kHeaderBytes + kPartialBytes + kOffsetTableBytes;

__device__ inline uint64_t pack_key(const Plan &p, int32_t b, int32_t x, int32_t y, int32_t z)
{
    uint64_t k = (uint64_t)(b - p.lo[0]);
    k = k * p.ext[1] + (uint64_t)(x - p.lo[1]);
    k = k * p.ext[2] + (uint64_t)(y - p.lo[2]);
    k = k * p.ext[3] + (uint64_t)(z - p.lo[3]);
    return k;
}

// Bits 0..9 of v spread to every third bit (bit i -> bit 3i).
__device__ inline uint32_t spread3(uint32_t v)
{
    v &= 0x3FFu;
    v = (v | (v << 16)) & 0x030000FFu;
    v = (v | (v << 8)) & 0x0300F00Fu;
    v = (v | (v << 4)) & 0x030C30C3u;
    v = (v | (v << 2)) & 0x09249249u;
    return v;
}

// Octree digits of the low `levels` bits of (x, y, z): per level one 3-bit
// digit x | y << 1 | z << 2 (a C2S child index), the coarsest level most
// significant.
__device__ inline uint32_t octree_digits(int32_t x, int32_t y, int32_t z, int levels)
{
    const uint32_t m = (1u << levels) - 1u;
    return spread3((uint32_t)x & m) | spread3((uint32_t)y & m) << 1 | spread3((uint32_t)z & m) << 2;
}

// The rank bitmap's cell key with L = p.levels octree levels: the
// lexicographic index of the root cell (coords >> L, inside the root bbox)
// times 8^L plus the octree digits of the low L bits.  Children that C2S
// subdivision emits (parent-major, child index ascending) L times below a
// lexicographically sorted set are strictly increasing in this key, so a
// decoder stage after an upsample keeps the rank bitmap.  L = 0 is pack_key.
__device__ inline uint64_t rank_key(const Plan &p, int32_t b, int32_t x, int32_t y, int32_t z)
{
    const int L = p.levels;
    if (L == 0) return pack_key(p, b, x, y, z);
    uint64_t k = (uint64_t)(b - p.rlo[0]);
    k = k * p.rext[1] + (uint64_t)((x >> L) - p.rlo[1]);
    k = k * p.rext[2] + (uint64_t)((y >> L) - p.rlo[2]);
    k = k * p.rext[3] + (uint64_t)((z >> L) - p.rlo[3]);
    return (k << (3 * L)) | octree_digits(x, y, z, L);
}

// The 3x3x3 kernel with unit axis signs (the decoder's submanifold conv):
// offset k = (kd*3 + kh)*3 + kw is known at compile time, so its cell delta
// is a signed sum of three per-launch strides and its bbox test an AND of
// per-row "one step up / down along kernel axis j stays inside" flags.
struct Cube3 {
    uint32_t D[3];  // cell delta of +1 along kernel axis j (wraps)
    int a[3];       // spatial axis (0 x, 1 y, 2 z) of kernel axis j
    int s[3];       // its sign
    int lo[3], hi[3];  // bbox bounds of that spatial axis
};

// Uniform int through a scalar register.
__device__ inline int uniform_i32(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Selections by axis pick among register values (never a computed address
// into a local struct, which would put the struct in scratch memory).
__device__ inline Cube3 cube3_of(const KernelShape &ks, const Plan &p)
{
    Cube3 q;
    const uint32_t sx = (uint32_t)uniform_i32((int)(uint32_t)(p.ext[2] * p.ext[3]));
    const uint32_t sy = (uint32_t)uniform_i32((int)(uint32_t)p.ext[3]);
    const int lx = uniform_i32(p.lo[1]), ly = uniform_i32(p.lo[2]), lz = uniform_i32(p.lo[3]);
    const int hx = uniform_i32(p.hi[1]), hy = uniform_i32(p.hi[2]), hz = uniform_i32(p.hi[3]);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int a = uniform_i32(ks.order[j]);
        q.a[j] = a;
        q.s[j] = uniform_i32(ks.sign[j]);
        const uint32_t st = a == 0 ? sx : (a == 1 ? sy : 1u);
        q.D[j] = q.s[j] > 0 ? st : 0u - st;
        q.lo[j] = a == 0 ? lx : (a == 1 ? ly : lz);
        q.hi[j] = a == 0 ? hx : (a == 1 ? hy : hz);
    }
    return q;
}

// Per-row flags of the 3x3x3 path: one step up / down along kernel axis j
// stays inside the bbox.
__device__ inline void cube3_flags(const int4 c, const Cube3 &cube, bool up[3], bool dn[3])
{
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int a = cube.a[j];
        const int ca = a == 0 ? c.y : (a == 1 ? c.z : c.w);
        up[j] = cube.s[j] > 0 ? ca < cube.hi[j] : ca > cube.lo[j];
        dn[j] = cube.s[j] > 0 ? ca > cube.lo[j] : ca < cube.hi[j];
    }
}

// Cell of the neighbour of a row (coord c, cell base) at offset k; `inside`
// tells whether it lies in the bbox (and the row is valid). k is a
// compile-time constant on the 3x3x3 path; otherwise the offset comes from
// the offset table (uniform loads).
template <bool kCube3>
__device__ inline uint32_t neighbour_cell(int k, const int4 c, bool valid, uint32_t base,
                                          const bool up[3], const bool dn[3], const Cube3 &cube,
                                          const Plan &p, const int4 *__restrict__ otab, bool &inside)
{
    uint32_t delta = 0;
    if (kCube3) {
        const int e[3] = {k / 9 - 1, (k / 3) % 3 - 1, k % 3 - 1};
        inside = valid;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            if (e[j] > 0) inside = inside && up[j];
            if (e[j] < 0) inside = inside && dn[j];
            delta += e[j] > 0 ? cube.D[j] : (e[j] < 0 ? 0u - cube.D[j] : 0u);
        }
    } else {
        const int4 o = otab[k];
        const int nx = c.y + o.x, ny = c.z + o.y, nz = c.w + o.z;
        inside = valid && nx >= p.lo[1] && nx <= p.hi[1] && ny >= p.lo[2] && ny <= p.hi[2] &&
                 nz >= p.lo[3] && nz <= p.hi[3];
        delta = (uint32_t)o.w;
    }
    return base + delta;
}

// Cell tables of modes 4 (dense grid of ~row, 0 = empty) and 5 (rank bitmap:
// per 32 cells a u32 of occupancy bits and the u32 row of the first occupied
// cell), read through a buffer descriptor: a cell outside the bbox gets an
// offset beyond it and reads 0, which decodes to -1 in both tables.
__device__ inline uint64_t cell_table_bytes(const Plan &p)
{
    return p.mode == 5 ? (p.total + 31) / 32 * 8 : p.total * 4;
}

__device__ inline __amdgpu_buffer_rsrc_t cell_table_rsrc(const void *table, uint32_t bytes)
{
    // The descriptor must live in scalar registers (its inputs are uniform).
    // readfirstlane returns a signed int: each half goes through uint32_t
    // before widening, or a low half with bit 31 set would sign-extend into
    // the high half of the address.
    const uint64_t tp = (uint64_t)(uintptr_t)table;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)tp);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(tp >> 32));
    const uint32_t nb = (uint32_t)__builtin_amdgcn_readfirstlane((int)bytes);
    return make_rsrc((const void *)(uintptr_t)(((uint64_t)hi << 32) | lo), nb);
}

template <bool kRank>
__device__ inline uint32_t cell_offset(uint32_t q, bool inside)
{
    return inside ? (kRank ? (q >> 5) << 3 : q << 2) : kOobOffset;
}

// Rank word -> row: first row of the word + occupied cells below bit b; -1
// unless bit b is set (the all-ones mask t selects the rank).
__device__ inline int32_t decode_rank(uint2 raw, uint32_t q)
{
    const uint32_t bits = raw.x, b = q & 31u;
    const int32_t t = __builtin_amdgcn_sbfe((int32_t)bits, b, 1);
    const int32_t rank = (int32_t)(__builtin_popcount(__builtin_amdgcn_ubfe(bits, 0, b)) + raw.y);
    return (rank & t) | ~t;
}

__device__ inline int32_t decode_grid(uint32_t raw) { return (int32_t)~raw; }

// The 3x3x3 path applies: kernel 3x3x3 with unit axis signs.
__device__ inline bool is_cube3(const KernelShape &ks)
{
    return ks.KD == 3 && ks.KH == 3 && ks.KW == 3 && abs(ks.sign[0]) == 1 && abs(ks.sign[1]) == 1 &&
           abs(ks.sign[2]) == 1;
}

}  // namespace nbr
}  // namespace sc
