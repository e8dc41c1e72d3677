// Voxel hash table + K-offset neighbour-map builder for gfx950.
//
// Replaces the reference's device map builders (crates/burn_flex_gmm/src/
// wgpu/neighbor_kernels.rs K1-K8 and their routing in wgpu/neighbor.rs:9-57,
// 777-936) with one order-independent algorithm:
//
//   1. bbox   : coalesced int4 coord loads, per-block min/max partials
//               (wave64/LDS reductions, no atomics); negative coords and rows
//               out of (b, x, y, z) order flagged
//   2. init   : every block reduces the partials and derives the table
//               plan; block 0 writes the header and the per-offset table;
//               all blocks fill the table region
//   3. insert : key = mixed-radix index of (b,x,y,z) inside the bbox; a
//               32-bit key packs with the row into one 64-bit slot (single
//               atomicCAS, atomicMin on the slot keeps the LOWEST row of
//               duplicates); wider keys use a u64 key array + u32 row array;
//               a bbox beyond 2^64-1 cells uses a row-only table whose slots
//               are compared through the coords themselves
//   4. query  : one row per lane for the dense tables (below), else R rows
//               per block staged in LDS, one (row, k) entry per lane;
//               coalesced map writes; neighbours outside the bbox (including
//               negative ones) are rejected before probing. A dense grid
//               over rows in no particular order is swept in cell order
//               instead (sweep_grid)
//
// Linear probing over a power-of-two table with >= 2 slots per row; every
// probe loop is bounded by the table capacity.
//
// When the bbox holds at most 32 cells per row (and the workspace has room),
// the "table" is a dense bbox-indexed grid of rows instead: the slot of a key
// is the key itself, so insertion is one atomicMax of ~row on a distinct word
// (empty cells are 0, the lowest row of duplicates wins) and a
// query one load, and the neighbours of nearby voxels share cache lines.
//
// When the rows are strictly increasing in (b, x, y, z) (checked by the bbox
// pass: sorted and unique, the order an argwhere over a grid produces), a
// row's index is the rank of its cell among the occupied cells. The table is
// then a rank bitmap: per 32 cells, 32 occupancy bits and the row of the first
// occupied cell (8 B per 32 cells, 1/16 of the dense grid, small enough to stay
// in L2), built by one writer per word with no atomics; a query is one 8-byte
// load and a popcount. The same holds for rows in the order C2S subdivision
// emits children (parent-major, child index ascending) L times below such a
// set: they are strictly increasing in a key with L octree levels (rank_key),
// which the bbox pass also checks, for L < 8. Any other row order takes the
// modes above.
#include <climits>

#include "sc_common.hpp"
#include "sc_neighbor.hpp"

namespace sc {
namespace {

using namespace nbr;
constexpr int kMaxStagedRows = 256;

inline uint64_t table_capacity(int64_t n)
{
    uint64_t want = (uint64_t)(n > 32 ? n : 32) * 2u;
    uint64_t cap = 64;
    while (cap < want) cap <<= 1;
    return cap;
}

inline uint64_t dense_cells_for(int64_t n);

// Slots the hash modes use: at least table_capacity, and as many as the
// table region of the minimal workspace holds at 12 bytes per slot (5-10 per
// row), which keeps the brick-local probe runs short.
inline uint64_t table_slots(int64_t n)
{
    uint64_t cap = table_capacity(n);
    const uint64_t room = dense_cells_for(n) * 4u / 12u;
    while (cap * 2 <= room) cap <<= 1;
    return cap;
}

// Dense-grid budget: 32 cells per row (at least 2^16 cells).
inline uint64_t dense_cells_for(int64_t n)
{
    const uint64_t c = (uint64_t)(n > 0 ? n : 0) * 32u;
    return c < (1u << 16) ? (1u << 16) : c;
}

inline size_t workspace_bytes_for(int64_t n)
{
    const size_t hash_bytes = (size_t)table_capacity(n) * 12u;
    const size_t dense_bytes = (size_t)dense_cells_for(n) * 4u;
    return kFixedBytes + (hash_bytes > dense_bytes ? hash_bytes : dense_bytes);
}

// splitmix64 finaliser (Steele, Lea & Flood, OOPSLA 2014).
__device__ inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__device__ inline Plan make_plan(const NbrHeader *h, Limits lim)
{
    Plan p;
    p.mode = 0;
    p.levels = 0;
    p.total = 0;
    for (int j = 0; j < 4; ++j) {
        p.lo[j] = h->bmin[j];
        p.hi[j] = h->bmax[j];
        p.ext[j] = (uint64_t)((int64_t)h->bmax[j] - (int64_t)h->bmin[j] + 1);
        p.rlo[j] = p.lo[j];
        p.rext[j] = p.ext[j];
    }
    if (h->status & kStatusNegative) return p;
    uint64_t total = 1;
    bool ovf = false;
    for (int j = 0; j < 4; ++j) {
        if (total != 0 && p.ext[j] > kEmpty64 / total) ovf = true;
        total *= p.ext[j];
    }
    p.total = total;
    if (ovf) {
        p.mode = 3;
        return p;
    }
    if (!(h->unsorted & 1u) && total <= lim.bitmap_cells) {
        p.mode = 5;
        return p;
    }
    // Rows in C2S order below a sorted root set: the rank bitmap over the
    // fewest octree levels whose key they follow (coords are non-negative
    // here, so >> is the parent index).
    for (int L = 1; L < kRankLevels; ++L) {
        if ((h->unsorted >> L) & 1u) continue;
        uint64_t t = p.ext[0];
        uint64_t re[4] = {p.ext[0], 0, 0, 0};
        int32_t rl[4] = {p.lo[0], 0, 0, 0};
        for (int j = 1; j < 4; ++j) {
            rl[j] = p.lo[j] >> L;
            re[j] = (uint64_t)((p.hi[j] >> L) - rl[j] + 1);
            t = t * re[j];  // <= ext product, no overflow
        }
        if (t > (lim.bitmap_cells >> (3 * L))) continue;
        p.mode = 5;
        p.levels = L;
        p.total = t << (3 * L);
        for (int j = 0; j < 4; ++j) {
            p.rlo[j] = rl[j];
            p.rext[j] = re[j];
        }
        return p;
    }
    p.mode = total <= lim.dense_cells ? 4 : (total <= 0xffffffffull ? 1 : 2);
    return p;
}

__device__ inline uint64_t hash_coord(int32_t b, int32_t x, int32_t y, int32_t z)
{
    return mix64((uint64_t)(uint32_t)b ^ mix64(((uint64_t)(uint32_t)x << 32 | (uint32_t)y) ^
                                               mix64((uint64_t)(uint32_t)z)));
}

__device__ inline bool same_coord(const int4 a, const int4 b)
{
    return a.x == b.x && a.y == b.y && a.z == b.z && a.w == b.w;
}

__global__ void nm_header_init_kernel(NbrHeader *h)
{
    for (int j = 0; j < 4; ++j) {
        h->bmin[j] = INT_MAX;
        h->bmax[j] = INT_MIN;
    }
    h->status = 0;
    h->unsorted = 0;
    h->mode = 0;
}

// Rank bitmap lookup: word w of the bitmap holds the occupancy bits of cells
// 32w..32w+31 (low half) and the row of its first occupied cell (high half).
// With rows strictly increasing in key order, a cell's row is its rank among
// the occupied cells: that first row plus the occupied cells below it in the word.
__device__ inline int32_t rank_lookup(const uint64_t *__restrict__ words, uint64_t q)
{
    const uint64_t w = words[q >> 5];
    const uint32_t bits = (uint32_t)w, b = (uint32_t)q & 31u;
    if (!((bits >> b) & 1u)) return SC_INVALID_NEIGHBOR_ROW;
    return (int32_t)(uint32_t)(w >> 32) + __builtin_popcount(bits & ((1u << b) - 1u));
}

__device__ inline uint32_t wave_or_u32(uint32_t v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v |= __shfl_xor(v, off, 64);
    return v;
}

// Combines entry j of two bbox partials: min of the lower corner, max of the
// upper corner and of the negative flag, OR of the order bits.
__device__ inline int reduce_partial(int j, int a, int b)
{
    return j < 4 ? min(a, b) : (j < 9 ? max(a, b) : (a | b));
}

// Per-block bbox partials (4 min, 4 max, negative flag, order bits), no atomics;
// at most 256 blocks of 1024 threads, so that every block of the next launch
// can reduce the partials.
constexpr int kBboxBlocks = 256;
constexpr int kBboxThreads = 1024;
constexpr int kPartialInts = 10;

__global__ __launch_bounds__(kBboxThreads) void nm_bbox_partial_kernel(const int4 *__restrict__ coords, int64_t n,
                                                              int32_t *__restrict__ partials)
{
    int mn[4] = {INT_MAX, INT_MAX, INT_MAX, INT_MAX};
    int mx[4] = {INT_MIN, INT_MIN, INT_MIN, INT_MIN};
    int neg = 0, uns = 0;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    // Wave-uniform loop, four rows per lane in flight: in each of them lane
    // l holds row w0 + u * stride + l, so lane l - 1 holds its predecessor.
    for (int64_t w0 = (int64_t)blockIdx.x * blockDim.x + wave * 64; w0 < n; w0 += 4 * stride) {
        int4 c[4], pl[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t i = w0 + u * stride + lane;
            c[u] = i < n ? coords[i] : make_int4(0, 0, 0, 0);
            pl[u] = lane == 0 && i < n && i > 0 ? coords[i - 1] : make_int4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t i = w0 + u * stride + lane;
            const int4 cu = c[u];
            int4 prev = make_int4(__shfl_up(cu.x, 1), __shfl_up(cu.y, 1), __shfl_up(cu.z, 1), __shfl_up(cu.w, 1));
            if (lane == 0) prev = pl[u];
            if (i < n) {
                const int v[4] = {cu.x, cu.y, cu.z, cu.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    mn[j] = min(mn[j], v[j]);
                    mx[j] = max(mx[j], v[j]);
                    neg |= v[j] < 0;
                }
                if (i > 0) uns |= (int)unsorted_levels(prev, cu);
            }
        }
    }
    __shared__ int s_red[kBboxThreads / 64][kPartialInts];  // per wave: 4 min, 4 max, neg, unsorted
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        mn[j] = wave_min_i32(mn[j]);
        mx[j] = wave_max_i32(mx[j]);
    }
    neg = wave_max_i32(neg);
    uns = (int)wave_or_u32((uint32_t)uns);
    if (lane == 0) {
        for (int j = 0; j < 4; ++j) {
            s_red[wave][j] = mn[j];
            s_red[wave][4 + j] = mx[j];
        }
        s_red[wave][8] = neg;
        s_red[wave][9] = uns;
    }
    __syncthreads();
    if (threadIdx.x < kPartialInts) {
        const int j = threadIdx.x;
        const int nw = blockDim.x >> 6;
        int v = s_red[0][j];
        for (int w = 1; w < nw; ++w) v = reduce_partial(j, v, s_red[w][j]);
        partials[blockIdx.x * kPartialInts + j] = v;
    }
}

// Every block reduces the partials (at most kBboxBlocks x 10 ints, a few KB
// from L2) and derives the table plan from them, then fills its share of the
// table region: all-ones (EMPTY keys, EMPTY rows) over cap*12 bytes for the
// hash modes; zero (no cell occupied) over the grid's total*4 bytes and the
// rank bitmap's ceil(total/32) words.  Block 0 also writes the header (bbox,
// status, order flag, plan) and the offset table {dx, dy, dz, cell delta}
// that the insert and query kernels read.
__global__ __launch_bounds__(256) void nm_plan_init_kernel(const int32_t *__restrict__ partials, int nblocks,
                                                           NbrHeader *__restrict__ h, Limits lim, KernelShape ks,
                                                           int4 *__restrict__ otab, uint64_t *__restrict__ words,
                                                           uint64_t cap)
{
    __shared__ int s_red[4][kPartialInts];
    __shared__ NbrHeader s_h;
    int mn[4] = {INT_MAX, INT_MAX, INT_MAX, INT_MAX};
    int mx[4] = {INT_MIN, INT_MIN, INT_MIN, INT_MIN};
    int neg = 0, uns = 0;
    for (int b = threadIdx.x; b < nblocks; b += blockDim.x) {
        const int32_t *pb = partials + b * kPartialInts;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            mn[j] = min(mn[j], pb[j]);
            mx[j] = max(mx[j], pb[4 + j]);
        }
        neg |= pb[8];
        uns |= pb[9];
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        mn[j] = wave_min_i32(mn[j]);
        mx[j] = wave_max_i32(mx[j]);
    }
    neg = wave_max_i32(neg);
    uns = (int)wave_or_u32((uint32_t)uns);
    if (lane == 0) {
        for (int j = 0; j < 4; ++j) {
            s_red[wave][j] = mn[j];
            s_red[wave][4 + j] = mx[j];
        }
        s_red[wave][8] = neg;
        s_red[wave][9] = uns;
    }
    __syncthreads();
    if (threadIdx.x < kPartialInts) {
        const int j = threadIdx.x;
        int v = s_red[0][j];
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) v = reduce_partial(j, v, s_red[w][j]);
        if (j < 4)
            s_h.bmin[j] = v;
        else if (j < 8)
            s_h.bmax[j - 4] = v;
        else if (j == 8)
            s_h.status = v ? kStatusNegative : 0u;
        else
            s_h.unsorted = (uint32_t)v;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const Plan p = make_plan(&s_h, lim);
        s_h.plan = p;
        s_h.mode = p.mode;
        s_h.pad0 = 0;
    }
    __syncthreads();
    const Plan p = s_h.plan;
    if (blockIdx.x == 0) {
        static_assert(sizeof(NbrHeader) % 16 == 0, "header copies in 16-byte pieces");
        if (threadIdx.x < sizeof(NbrHeader) / 16)
            reinterpret_cast<uint4 *>(h)[threadIdx.x] = reinterpret_cast<const uint4 *>(&s_h)[threadIdx.x];
        // 32-bit cell delta of each offset (wraps; only used for neighbours inside the bbox)
        const uint32_t sy = (uint32_t)p.ext[3], sx = (uint32_t)(p.ext[2] * p.ext[3]);
        for (int k = threadIdx.x; k < ks.K && k < kMaxStagedOffsets; k += blockDim.x) {
            int o[3];
            offset_of(ks, k, o);
            otab[k] = make_int4(o[0], o[1], o[2], (int)((uint32_t)o[0] * sx + (uint32_t)o[1] * sy + (uint32_t)o[2]));
        }
    }
    if (p.mode == 0) return;
    // hash modes: mode 1 uses the packed key slots [0, cap), mode 3 the row
    // slots (words [cap, cap + cap / 2)), mode 2 both
    uint64_t w0 = p.mode == 3 ? cap : 0;
    uint64_t n_words = p.mode == 1 ? cap : cap + cap / 2, fill = kEmpty64;
    if (p.mode == 4) {
        n_words = (p.total + 1) / 2;
        fill = 0;
    }
    if (p.mode == 5) {
        n_words = (p.total + 31) / 32;
        fill = 0;
    }
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    if (p.mode == 4 || p.mode == 5) w0 = 0;
    for (uint64_t i = w0 + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_words; i += stride) words[i] = fill;
}

__global__ __launch_bounds__(256) void nm_insert_kernel(const int4 *__restrict__ coords, int64_t n,
                                                        NbrHeader *h, uint64_t *keys, uint32_t *rows,
                                                        uint64_t mask)
{
    const Plan p = h->plan;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p.mode == 0) return;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    if (p.mode == 5) {
        // Rank bitmap (words start at zero): a word receives its occupancy bits
        // and the row of its first occupied cell. The keys strictly increase,
        // so the rows of a word are consecutive (at most 32). Lane l of a wave
        // holds row w0 + l: a segmented suffix OR over the lanes of one word
        // collects their bits, and the word's first lane in this wave ORs them
        // in (with its row when it is the word's first row). A word split
        // across two waves gets one OR from each; ORs commute.
        const int lane = threadIdx.x & 63;
        for (int64_t w0 = tid - lane; w0 < n; w0 += stride) {
            const int64_t r = w0 + lane;
            const bool valid = r < n;
            uint32_t q = 0, w = 0xffffffffu;  // total <= 2^32 - 1 cells: 32-bit keys
            if (valid) {
                const int4 c = coords[r];
                q = (uint32_t)rank_key(p, c.x, c.y, c.z, c.w);
                w = q >> 5;
            }
            uint32_t wp = __shfl_up(w, 1);
            if (lane == 0) {
                wp = 0xfffffffeu;  // no predecessor: differs from every word
                if (r > 0) {
                    const int4 cp = coords[r - 1];
                    wp = (uint32_t)rank_key(p, cp.x, cp.y, cp.z, cp.w) >> 5;
                }
            }
            uint32_t bits = valid ? 1u << (q & 31u) : 0u;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const uint32_t ob = __shfl_down(bits, d), ow = __shfl_down(w, d);
                if (lane + d < 64 && ow == w) bits |= ob;
            }
            const bool head = wp != w;  // the word's first row
            if (valid && (head || lane == 0))
                atomicOr((unsigned long long *)&keys[w],
                         (head ? (unsigned long long)(uint32_t)r << 32 : 0ull) | bits);
        }
        return;
    }
    uint32_t *grid = reinterpret_cast<uint32_t *>(keys);
    for (int64_t r = tid; r < n; r += stride) {
        const int4 c = coords[r];
        if (p.mode == 4) {
            // cells hold ~row and start at 0 (empty): the unsigned maximum keeps
            // the lowest row, and an empty cell decodes as ~0 = -1
            const uint32_t old = atomicMax(&grid[pack_key(p, c.x, c.y, c.z, c.w)], ~(uint32_t)r);
            if (old != 0u) atomicOr(&h->status, kStatusDupCell);
            continue;
        }
        if (p.mode == 3) {
            uint64_t s = hash_coord(c.x, c.y, c.z, c.w) & mask;
            for (uint64_t probe = 0; probe <= mask; ++probe) {
                const uint32_t old = atomicCAS(&rows[s], 0xffffffffu, (uint32_t)r);
                if (old == 0xffffffffu) break;
                if (same_coord(coords[old], c)) {
                    atomicMin(&rows[s], (uint32_t)r);
                    break;
                }
                s = (s + 1) & mask;
            }
            continue;
        }
        const uint64_t key = pack_key(p, c.x, c.y, c.z, c.w);
        uint64_t s = mix64(key) & mask;
        if (p.mode == 1) {
            const uint64_t mine = (key << 32) | (uint64_t)(uint32_t)r;
            for (uint64_t probe = 0; probe <= mask; ++probe) {
                const uint64_t old = atomicCAS((unsigned long long *)&keys[s], kEmpty64, mine);
                if (old == kEmpty64) break;
                if ((old >> 32) == key) {
                    atomicMin((unsigned long long *)&keys[s], (unsigned long long)mine);
                    break;
                }
                s = (s + 1) & mask;
            }
        } else {
            for (uint64_t probe = 0; probe <= mask; ++probe) {
                const uint64_t old = atomicCAS((unsigned long long *)&keys[s], kEmpty64, key);
                if (old == kEmpty64 || old == key) {
                    atomicMin(&rows[s], (uint32_t)r);
                    break;
                }
                s = (s + 1) & mask;
            }
        }
    }
}

// Dense-grid and rank-bitmap query: a row's neighbour at offset k is cell
// base[r] + delta[k] (32-bit mixed-radix strides), valid when the neighbour
// lies in the bbox. Entries (r, k) are walked incrementally (no division),
// four loads in flight per lane before their stores.
template <bool kRank>
__device__ inline void query_dense(const int4 *s_coord, const int *s_off, const uint32_t *s_base,
                                   const int *s_delta, int nrows, int K, const Plan &p,
                                   const uint64_t *__restrict__ table, int32_t *__restrict__ out)
{
    const uint32_t *grid = reinterpret_cast<const uint32_t *>(table);
    const int total = nrows * K;
    const int step_r = (int)blockDim.x / K, step_k = (int)blockDim.x % K;
    int r = (int)threadIdx.x / K, k = (int)threadIdx.x % K;
    for (int e0 = threadIdx.x; e0 < total; e0 += 4 * (int)blockDim.x) {
        // all four loads issue before any result is used
        uint64_t raw[4];
        uint32_t bit[4];
        int idx[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = e0 + u * (int)blockDim.x;
            idx[u] = e;
            raw[u] = 0;  // decodes to -1 in both tables
            bit[u] = 0;
            if (e < total) {
                const int4 c = s_coord[r];
                const int nx = c.y + s_off[3 * k], ny = c.z + s_off[3 * k + 1], nz = c.w + s_off[3 * k + 2];
                if (nx >= p.lo[1] && nx <= p.hi[1] && ny >= p.lo[2] && ny <= p.hi[2] && nz >= p.lo[3] &&
                    nz <= p.hi[3]) {
                    const uint32_t q = s_base[r] + (uint32_t)s_delta[k];
                    if (kRank) {
                        raw[u] = table[q >> 5];
                        bit[u] = q & 31u;
                    } else {
                        raw[u] = grid[q];
                    }
                }
            }
            r += step_r;
            k += step_k;
            if (k >= K) {
                k -= K;
                ++r;
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            int32_t v = (int32_t)~(uint32_t)raw[u];  // grid cells hold ~row
            if (kRank) {
                // empty word or cell: no bit set -> -1
                const uint32_t bits = (uint32_t)raw[u];
                v = (bits >> bit[u]) & 1u
                        ? (int32_t)(uint32_t)(raw[u] >> 32) + __builtin_popcount(bits & ((1u << bit[u]) - 1u))
                        : SC_INVALID_NEIGHBOR_ROW;
            }
            if (idx[u] < total) out[idx[u]] = v;
        }
    }
}

// Dense-grid and rank-bitmap query with one row per lane (rows_per_block ==
// 256, K <= kCellwiseMaxK): the row's coord and base cell stay in registers,
// the offset loop is uniform across the wave (offsets and cell deltas come
// from the table the bbox pass writes, through scalar loads),
// up to 27 lookups are in flight per lane, and the results pass through LDS
// ([row][k], conflict-free for odd K) so that the block's rows*K map entries
// leave as coalesced 16-byte stores.
constexpr int kCellwiseMaxK = 32;
constexpr int kCellChunk = 27;

// Grid sweep (below): per wave, a ring of (cell, row) entries (< 64 left
// over + 64 appended) and results for 64 entries.
constexpr int kSweepRing = 128;

// LDS of the sweep (3x3x3 kernels), in ints: per wave, [entry][27] results,
// then the ring's cells and rows.
constexpr int kSweepLdsInts = 4 * (64 * 27 + 2 * kSweepRing);

// Dynamic LDS of the query kernel, in ints: the larger of the row-wise
// results (rows x K, or the grid sweep's) and the entry-wise staging (3 + 1
// ints per offset, then 4 + 1 ints per row).
inline int query_lds_ints(int64_t K, int rows_per_block)
{
    const int kst = K <= kMaxStagedOffsets ? (int)K : 0;
    const int staged = 4 * kst + 5 * kMaxStagedRows;
    int rowwise = K <= kCellwiseMaxK ? rows_per_block * (int)K : 0;
    if (K == 27 && rows_per_block == 256 && kSweepLdsInts > rowwise) rowwise = kSweepLdsInts;
    return staged > rowwise ? staged : rowwise;
}

// Dense grid over rows in no particular order (sorted rows take the rank
// bitmap), 3x3x3 kernels. Row by row, the lookups would go to random cells,
// a few cache lines per row, so the query sweeps the grid in cell order
// instead. Each wave takes a contiguous range of cells (XCD-aware, so an
// XCD's waves cover one region of the grid) in units of 64 cells, one per
// lane, four units per step with the next four in flight; the occupied cells
// of query rows are appended, in cell order, to the wave's ring of (cell,
// row) entries in LDS. Each time it holds 64 entries, one per lane, they are
// mapped: an entry's 27 neighbour lookups fall in the cache lines of nearby
// entries' lookups; the results go through LDS ([entry][27]) and leave as
// runs of 27 consecutive ints, the rows' map rows. Waves need no barrier,
// only their own LDS order. A cell names one row, so duplicate coords
// (flagged by the insert) take the row-wise query instead.
__device__ inline void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The 3x3x3 path: each entry's 27 neighbour cells come from its coord's
// per-axis up / down flags and the kernel axes' cell deltas (no offset table
// reads), and all 27 lookups are in flight together.
__device__ inline void sweep_map_entries(const Plan &p, const Cube3 &cube, const __amdgpu_buffer_rsrc_t rt,
                                         const int *s_cell, const int *s_rrow, int *s_val, uint32_t head,
                                         int cnt, int32_t *__restrict__ map)
{
    constexpr int K = 27;
    const int lane = (int)threadIdx.x & 63;
    if (lane < cnt) {
        const uint32_t ez = (uint32_t)p.ext[3], ey = (uint32_t)p.ext[2], ex = (uint32_t)p.ext[1];
        const uint32_t cell = (uint32_t)s_cell[(head + lane) & (kSweepRing - 1)];
        const uint32_t line = cell / ez, cz = cell - line * ez;
        const uint32_t xy = line / ey, cy = line - xy * ey, cx = xy % ex;
        const int4 c = make_int4(0, p.lo[1] + (int)cx, p.lo[2] + (int)cy, p.lo[3] + (int)cz);
        bool up[3], dn[3];
        cube3_flags(c, cube, up, dn);
        uint32_t raw[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            bool inside;
            const uint32_t q = neighbour_cell<true>(k, c, true, cell, up, dn, cube, p, nullptr, inside);
            raw[k] = bload4(rt, cell_offset<false>(q, inside));
        }
#pragma unroll
        for (int k = 0; k < K; ++k) s_val[lane * K + k] = decode_grid(raw[k]);
    }
    wave_lds_sync();
    const int n_ent = cnt * K;
    int r = lane / K, k = lane % K;
    constexpr int step_r = 64 / K, step_k = 64 % K;
#pragma unroll 4
    for (int i = lane; i < n_ent; i += 64) {
        map[(int64_t)s_rrow[(head + r) & (kSweepRing - 1)] * K + k] = s_val[i];
        r += step_r;
        k += step_k;
        if (k >= K) {
            k -= K;
            ++r;
        }
    }
    wave_lds_sync();
}

__device__ inline void sweep_grid(const Plan &p, const Cube3 &cube, int64_t q_rows,
                                  const uint64_t *__restrict__ table, uint32_t table_bytes, int *s_dyn,
                                  int32_t *__restrict__ map)
{
    const __amdgpu_buffer_rsrc_t rt = cell_table_rsrc(table, table_bytes);
    const int lane = (int)threadIdx.x & 63, wave = uniform_i32((int)threadIdx.x >> 6);
    int *s_val = s_dyn + wave * (64 * 27 + 2 * kSweepRing);
    int *s_cell = s_val + 64 * 27;
    int *s_rrow = s_cell + kSweepRing;
    // total <= 2^32 - 2 cells (dense-grid budget), and table_bytes < 3 GiB
    // keeps every cell's byte offset in 32 bits
    const uint64_t total = p.total, n_waves = (uint64_t)gridDim.x * 4;
    const uint64_t per = (total + n_waves - 1) / n_waves;
    const uint64_t gw = (uint64_t)tile_for_block((int)blockIdx.x, (int)gridDim.x) * 4 + wave;
    const uint32_t c0 = (uint32_t)min(gw * per, total), c1 = (uint32_t)min(gw * per + per, total);
    // Units go in groups of four: a group's cells are read (waited for)
    // before the next group's loads issue, and the next group's loads are in
    // flight while this group's entries are mapped. (A wait for a load issued
    // before the map stores would also wait for those stores.)
    constexpr int kGroup = 4;
    uint32_t g[kGroup];
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
        const uint32_t c = c0 + 64u * u + lane;
        g[u] = bload4(rt, c < c1 ? c << 2 : kOobOffset);
    }
    uint32_t head = 0, tail = 0;
    for (uint32_t base = c0; base < c1; base += 64u * kGroup) {
        int32_t row[kGroup];
        bool occ[kGroup];
        uint64_t m[kGroup];
#pragma unroll
        for (int u = 0; u < kGroup; ++u) {
            row[u] = decode_grid(g[u]);
            occ[u] = g[u] != 0u && (int64_t)row[u] < q_rows;  // 0 beyond the range
            m[u] = __ballot(occ[u]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < kGroup; ++u) {
            const uint64_t c = (uint64_t)base + 64u * (kGroup + u) + lane;
            g[u] = bload4(rt, c < c1 ? (uint32_t)c << 2 : kOobOffset);
        }
        __builtin_amdgcn_sched_barrier(0);
        // one unit per step, its values in slot 0 (the others move down), so
        // that the mapping step appears once in the code
#pragma unroll 1
        for (int u = 0; u < kGroup; ++u) {
            const uint32_t ub = base + 64u * u;
            if (ub >= c1) break;
            const bool o = occ[0];
            const int32_t r0 = row[0];
            const uint64_t mu = m[0];
#pragma unroll
            for (int i = 0; i + 1 < kGroup; ++i) {
                occ[i] = occ[i + 1];
                row[i] = row[i + 1];
                m[i] = m[i + 1];
            }
            if (o) {
                const uint32_t e = (tail + __builtin_amdgcn_mbcnt_hi((uint32_t)(mu >> 32),
                                                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mu, 0u))) &
                                   (kSweepRing - 1);
                s_cell[e] = (int)(ub + lane);
                s_rrow[e] = r0;
            }
            tail += (uint32_t)__popcll(mu);
            wave_lds_sync();
            // map 64 entries at a time; after the range's last cells, the rest
            const bool last = (uint64_t)ub + 64u >= c1;
            while (tail - head >= 64u || (last && tail != head)) {
                const int cnt = (int)min(tail - head, 64u);
                sweep_map_entries(p, cube, rt, s_cell, s_rrow, s_val, head, cnt, map);
                head += (uint32_t)cnt;
            }
        }
    }
}

// Rank bitmap with octree levels on the 3x3x3 path: the key (rank_key) is
// not linear in the coords, but it is a sum of per-axis terms, so each row
// keeps, per kernel axis j and step e in {-1, 0, +1}, the term T[j][e + 1]
// of its neighbour's coordinate along that axis (root index times its stride,
// shifted past the digits, plus the axis's octree digits), and base the
// batch term; a neighbour's key is base + three terms.
__device__ inline void levels_terms(const int4 c, const Cube3 &cube, const Plan &p, uint32_t &base,
                                    uint32_t (&T)[3][3])
{
    const int L = uniform_i32(p.levels);
    const uint32_t e1 = (uint32_t)uniform_i32((int)(uint32_t)p.rext[1]);
    const uint32_t e2 = (uint32_t)uniform_i32((int)(uint32_t)p.rext[2]);
    const uint32_t e3 = (uint32_t)uniform_i32((int)(uint32_t)p.rext[3]);
    const int l0 = uniform_i32(p.rlo[0]), l1 = uniform_i32(p.rlo[1]), l2 = uniform_i32(p.rlo[2]),
              l3 = uniform_i32(p.rlo[3]);
    const uint32_t sx = e2 * e3, sy = e3;  // root strides of x, y (z: 1)
    base = ((uint32_t)(c.x - l0) * (e1 * sx)) << (3 * L);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int a = cube.a[j];
        const int ca = a == 0 ? c.y : (a == 1 ? c.z : c.w);
        const int rl = a == 0 ? l1 : (a == 1 ? l2 : l3);
        const uint32_t st = a == 0 ? sx : (a == 1 ? sy : 1u);
        const uint32_t m = (1u << L) - 1u;
#pragma unroll
        for (int e = 0; e < 3; ++e) {
            const int v = ca + (e - 1) * cube.s[j];
            T[j][e] = (((uint32_t)((v >> L) - rl) * st) << (3 * L)) + (spread3((uint32_t)v & m) << a);
        }
    }
}

template <bool kRank, bool kCube3, bool kLevels = false>
__device__ inline void query_cells(const int4 *__restrict__ coords, int64_t row0, int nrows, int K,
                                   const int4 *__restrict__ otab, const Cube3 &cube, const Plan &p,
                                   const uint64_t *__restrict__ table, uint32_t table_bytes, int *s_out,
                                   int32_t *__restrict__ out)
{
    static_assert(!kLevels || (kRank && kCube3), "octree levels: rank bitmap, 3x3x3 path");
    const __amdgpu_buffer_rsrc_t rt = cell_table_rsrc(table, table_bytes);
    const int rw = (int)threadIdx.x;  // row within the block
    const bool valid = rw < nrows;
    int4 c = make_int4(0, 0, 0, 0);
    uint32_t base = 0;
    if (valid) {
        c = coords[row0 + rw];
        if (!kLevels) base = (uint32_t)pack_key(p, c.x, c.y, c.z, c.w);
    }
    bool up[3] = {false, false, false}, dn[3] = {false, false, false};
    if (kCube3) cube3_flags(c, cube, up, dn);
    uint32_t T[3][3];
    if (kLevels) levels_terms(c, cube, p, base, T);
    const int KK = kCube3 ? 27 : K;
    int *so = s_out + rw * KK;
    for (int k0 = 0; k0 < KK; k0 += kCellChunk) {
        uint2 raw[kCellChunk];
        uint32_t q[kCellChunk];
#pragma unroll
        for (int u = 0; u < kCellChunk; ++u) {
            const int k = k0 + u;
            if (k >= KK) break;
            bool inside;
            if (kLevels) {
                const int e[3] = {k / 9, (k / 3) % 3, k % 3};  // step + 1 along kernel axis j
                inside = valid;
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    if (e[j] == 2) inside = inside && up[j];
                    if (e[j] == 0) inside = inside && dn[j];
                }
                q[u] = base + T[0][e[0]] + T[1][e[1]] + T[2][e[2]];
            } else {
                q[u] = neighbour_cell<kCube3>(k, c, valid, base, up, dn, cube, p, otab, inside);
            }
            if (kRank)
                raw[u] = bload8(rt, cell_offset<true>(q[u], inside));
            else
                raw[u].x = bload4(rt, cell_offset<false>(q[u], inside));
        }
#pragma unroll
        for (int u = 0; u < kCellChunk; ++u) {
            const int k = k0 + u;
            if (k >= KK) break;
            const int32_t v = kRank ? decode_rank(raw[u], q[u]) : decode_grid(raw[u].x);
            if (valid) so[k] = v;
        }
    }
    __syncthreads();
    const int n_ints = nrows * K;
    if (((uintptr_t)out & 15u) == 0) {
        const int n4 = n_ints >> 2;
        int4 *dst4 = reinterpret_cast<int4 *>(out);
        const int4 *src4 = reinterpret_cast<const int4 *>(s_out);
        // Ordinary stores: the conv plan reads the map next, and finds part of
        // it still in L2 (nontemporal stores speed this kernel up and slow that one down).
        for (int i = threadIdx.x; i < n4; i += blockDim.x) dst4[i] = src4[i];
        for (int i = (n4 << 2) + threadIdx.x; i < n_ints; i += blockDim.x) out[i] = s_out[i];
    } else {
        for (int i = threadIdx.x; i < n_ints; i += blockDim.x) out[i] = s_out[i];
    }
}

__global__ __launch_bounds__(256) void nm_query_kernel(const int4 *__restrict__ coords, int64_t n_rows,
                                                       int64_t q_rows, KernelShape ks,
                                                       int rows_per_block,
                                                       const NbrHeader *__restrict__ h,
                                                       const uint64_t *__restrict__ keys,
                                                       const uint32_t *__restrict__ rows,
                                                       uint64_t mask, const int4 *__restrict__ otab,
                                                       int32_t *__restrict__ map)
{
    // Row-wise path: the [row][k] results. Entry-wise paths: [staged offsets:
    // 3 ints each][their cell deltas][staged rows: coords, base cells].
    // Sized by query_lds_ints.
    extern __shared__ __align__(16) int s_dyn[];
    const int kst = ks.K <= kMaxStagedOffsets ? ks.K : 0;
    int *s_off = s_dyn;
    int *s_delta = s_dyn + 3 * kst;
    int *s_mem = s_dyn + 4 * kst;
    int4 *s_coord = reinterpret_cast<int4 *>(s_mem);
    uint32_t *s_base = reinterpret_cast<uint32_t *>(s_mem + 4 * kMaxStagedRows);
    // Each XCD takes a contiguous range of row blocks, so its L2 holds the
    // part of the cell table those rows' neighbours fall in.
    const int64_t row0 = (int64_t)tile_for_block((int)blockIdx.x, (int)gridDim.x) * rows_per_block;
    const int nrows = (int)min<int64_t>(rows_per_block, q_rows - row0);
    const Plan p = h->plan;
    const bool staged = ks.K <= kMaxStagedOffsets;
    const bool cellwise = p.mode == 4 || p.mode == 5;
    // octree-level keys are not linear in the coords: only the 3x3x3 row-wise
    // path handles them specially, other shapes take the per-entry path below
    const bool levels = p.mode == 5 && p.levels > 0;
    // table bytes, addressed through a buffer descriptor on the row-wise path
    const uint64_t tbytes = cell_table_bytes(p);
    const bool cube3 = is_cube3(ks);
    const bool rowwise = cellwise && ks.K <= kCellwiseMaxK && rows_per_block == (int)blockDim.x &&
                         tbytes <= kOobOffset && (!levels || cube3);
    int32_t *out = map + row0 * ks.K;
    // the sweep covers every cell, so it pays when most rows are queried
    if (rowwise && cube3 && p.mode == 4 && !(h->status & kStatusDupCell) && 2 * q_rows >= n_rows) {
        sweep_grid(p, cube3_of(ks, p), q_rows, keys, (uint32_t)tbytes, s_dyn, map);
        return;
    }
    if (rowwise) {
        const Cube3 cube = cube3_of(ks, p);
        if (levels)
            query_cells<true, true, true>(coords, row0, nrows, ks.K, otab, cube, p, keys, (uint32_t)tbytes, s_dyn,
                                          out);
        else if (p.mode == 5 && cube3)
            query_cells<true, true>(coords, row0, nrows, ks.K, otab, cube, p, keys, (uint32_t)tbytes, s_dyn,
                                     out);
        else if (p.mode == 5)
            query_cells<true, false>(coords, row0, nrows, ks.K, otab, cube, p, keys, (uint32_t)tbytes, s_dyn,
                                     out);
        else if (cube3)
            query_cells<false, true>(coords, row0, nrows, ks.K, otab, cube, p, keys, (uint32_t)tbytes, s_dyn,
                                     out);
        else
            query_cells<false, false>(coords, row0, nrows, ks.K, otab, cube, p, keys, (uint32_t)tbytes, s_dyn,
                                     out);
        return;
    }
    for (int i = threadIdx.x; i < nrows; i += blockDim.x) {
        const int4 c = coords[row0 + i];
        s_coord[i] = c;
        if (cellwise) s_base[i] = (uint32_t)pack_key(p, c.x, c.y, c.z, c.w);
    }
    if (staged)
        for (int k = threadIdx.x; k < ks.K; k += blockDim.x) {
            const int4 o = otab[k];
            s_off[3 * k] = o.x;
            s_off[3 * k + 1] = o.y;
            s_off[3 * k + 2] = o.z;
            s_delta[k] = o.w;
        }
    __syncthreads();
    if (cellwise && staged && !levels) {
        if (p.mode == 5)
            query_dense<true>(s_coord, s_off, s_base, s_delta, nrows, ks.K, p, keys, out);
        else
            query_dense<false>(s_coord, s_off, s_base, s_delta, nrows, ks.K, p, keys, out);
        return;
    }
    const uint32_t *grid = reinterpret_cast<const uint32_t *>(keys);
    const int total = nrows * ks.K;
    for (int e = threadIdx.x; e < total; e += blockDim.x) {
        const int r = e / ks.K, k = e - r * ks.K;
        int o[3];
        if (staged) {
            o[0] = s_off[3 * k];
            o[1] = s_off[3 * k + 1];
            o[2] = s_off[3 * k + 2];
        } else {
            offset_of(ks, k, o);
        }
        const int4 c = s_coord[r];
        // int64 so that coord + offset cannot wrap.
        const int64_t nx = (int64_t)c.y + o[0], ny = (int64_t)c.z + o[1], nz = (int64_t)c.w + o[2];
        int32_t found = SC_INVALID_NEIGHBOR_ROW;
        // A negative neighbour is absent (crates/burn_flex_gmm/src/lib.rs:98-100);
        // so is any neighbour outside the bbox of the coord set.
        const bool inside = p.mode != 0 && nx >= p.lo[1] && nx <= p.hi[1] && ny >= p.lo[2] &&
                            ny <= p.hi[2] && nz >= p.lo[3] && nz <= p.hi[3];
        if (inside && p.mode == 5) {
            found = rank_lookup(keys, rank_key(p, c.x, (int32_t)nx, (int32_t)ny, (int32_t)nz));
        } else if (inside && p.mode == 4) {
            found = (int32_t)~grid[pack_key(p, c.x, (int32_t)nx, (int32_t)ny, (int32_t)nz)];
        } else if (inside && p.mode == 3) {
            const int4 q = make_int4(c.x, (int32_t)nx, (int32_t)ny, (int32_t)nz);
            uint64_t s = hash_coord(q.x, q.y, q.z, q.w) & mask;
            for (uint64_t probe = 0; probe <= mask; ++probe) {
                const uint32_t v = rows[s];
                if (v == 0xffffffffu) break;
                if (same_coord(coords[v], q)) {
                    found = (int32_t)v;
                    break;
                }
                s = (s + 1) & mask;
            }
        } else if (inside) {
            const uint64_t key = pack_key(p, c.x, (int32_t)nx, (int32_t)ny, (int32_t)nz);
            uint64_t s = mix64(key) & mask;
            if (p.mode == 1) {
                for (uint64_t probe = 0; probe <= mask; ++probe) {
                    const uint64_t v = keys[s];
                    if (v == kEmpty64) break;
                    if ((v >> 32) == key) {
                        found = (int32_t)(uint32_t)v;
                        break;
                    }
                    s = (s + 1) & mask;
                }
            } else {
                for (uint64_t probe = 0; probe <= mask; ++probe) {
                    const uint64_t v = keys[s];
                    if (v == kEmpty64) break;
                    if (v == key) {
                        found = (int32_t)rows[s];
                        break;
                    }
                    s = (s + 1) & mask;
                }
            }
        }
        out[e] = found;
    }
}

}  // namespace
}  // namespace sc

using namespace sc;

extern "C" {

int sc_neighbor_map_workspace_size(int64_t n_rows, size_t *bytes)
{
    clear_error();
    if (!bytes) return fail(SC_ERR_NULL, "bytes out-pointer is NULL");
    if (n_rows < 0 || n_rows > INT32_MAX)
        return fail(SC_ERR_SHAPE, "sparse conv coord row count exceeds i32::MAX");
    *bytes = workspace_bytes_for(n_rows);
    return SC_OK;
}

int sc_neighbor_map_build(const sc_conv_config *cfg, const int32_t *d_coords, int64_t n_rows,
                          int64_t query_rows, int32_t *d_map, void *d_workspace,
                          size_t workspace_bytes, sc_stream stream)
{
    clear_error();
    int rc = validate_config(cfg);
    if (rc) return rc;
    if (n_rows < 0 || n_rows > INT32_MAX)
        return fail(SC_ERR_SHAPE, "sparse conv coord row count exceeds i32::MAX");
    if (query_rows < 0 || query_rows > n_rows)
        return fail(SC_ERR_SHAPE, "neighbor map query rows must be in [0, n_rows]");
    if (!d_workspace) return fail(SC_ERR_NULL, "neighbor map workspace is NULL");
    if ((uintptr_t)d_workspace % 16 != 0)
        return fail(SC_ERR_WORKSPACE, "neighbor map workspace must be 16-byte aligned");
    const size_t need = workspace_bytes_for(n_rows);
    if (workspace_bytes < need)
        return fail(SC_ERR_WORKSPACE, "neighbor map workspace too small: got " +
                                          std::to_string(workspace_bytes) + " need " +
                                          std::to_string(need));
    if (n_rows > 0 && !d_coords) return fail(SC_ERR_NULL, "coords pointer is NULL");
    if (query_rows > 0 && !d_map) return fail(SC_ERR_NULL, "map pointer is NULL");
    if ((uintptr_t)d_coords % 16 != 0) return fail(SC_ERR_SHAPE, "coords must be 16-byte aligned");
    const int64_t K = cfg->kernel_d * cfg->kernel_h * cfg->kernel_w;
    int64_t map_elems;
    if (!mul_ok(query_rows, K, &map_elems)) return fail(SC_ERR_OVERFLOW, "neighbor map size overflow");

    hipStream_t s = as_stream(stream);
    // Workspace: [header 256 B][bbox partials][offset table][hash table, grid or bitmap].
    NbrHeader *h = (NbrHeader *)d_workspace;
    int32_t *partials = (int32_t *)((char *)d_workspace + kHeaderBytes);
    const uint64_t cap = table_slots(n_rows);
    int4 *otab = (int4 *)((char *)d_workspace + kHeaderBytes + kPartialBytes);
    uint64_t *keys = (uint64_t *)((char *)d_workspace + kFixedBytes);
    uint32_t *rows = (uint32_t *)(keys + cap);
    // Dense grid when the bbox fits the workspace's grid budget (decided on the
    // device from the bbox; the budget never exceeds 32 cells per row).
    uint64_t dense_cells = (workspace_bytes - kFixedBytes) / 4u;
    if (dense_cells > dense_cells_for(n_rows)) dense_cells = dense_cells_for(n_rows);
    dense_cells &= ~1ull;  // even: the 8-byte fill of an odd cell count stays inside
    if (dense_cells > 0xffffffffull) dense_cells = 0xfffffffeull;  // 32-bit grid keys
    // Rank bitmap (sorted, unique rows): 8 B per 32 cells, 32-bit cell keys,
    // at most 512 cells per row (what the default workspace holds; a larger
    // workspace does not make a sparser bbox take the bitmap).
    uint64_t bitmap_cells = (workspace_bytes - kFixedBytes) / 8u * 32u;
    const uint64_t bitmap_cap = 16u * dense_cells_for(n_rows);
    if (bitmap_cells > bitmap_cap) bitmap_cells = bitmap_cap;
    if (bitmap_cells > 0xffffffffull) bitmap_cells = 0xffffffffull;
    const Limits lim{dense_cells, bitmap_cells};
    if (n_rows == 0) {
        nm_header_init_kernel<<<1, 1, 0, s>>>(h);
        SC_LAUNCH_CHECK("nm_header_init_kernel launch");
        return SC_OK;
    }
    const int4 *c4 = (const int4 *)d_coords;
    const unsigned bb = grid_for(n_rows, kBboxThreads, kBboxBlocks);
    nm_bbox_partial_kernel<<<bb, kBboxThreads, 0, s>>>(c4, n_rows, partials);
    SC_LAUNCH_CHECK("nm_bbox_partial_kernel launch");
    nm_plan_init_kernel<<<512, 256, 0, s>>>(partials, (int)bb, h, lim, kernel_shape(cfg), otab, keys, cap);
    SC_LAUNCH_CHECK("nm_plan_init_kernel launch");
    nm_insert_kernel<<<grid_for(n_rows, 256, 65536), 256, 0, s>>>(c4, n_rows, h, keys, rows, cap - 1);
    SC_LAUNCH_CHECK("nm_insert_kernel launch");
    if (query_rows == 0) return SC_OK;
    const KernelShape ks = kernel_shape(cfg);
    // 256 rows per block (one per lane on the row-wise path) for K <= 32,
    // else about 2048 (row, offset) entries per block.
    int rpb = K <= kCellwiseMaxK ? 256 : (int)(2048 / K);
    if (rpb < 1) rpb = 1;
    if (rpb > kMaxStagedRows) rpb = kMaxStagedRows;
    const int64_t blocks = (query_rows + rpb - 1) / rpb;
    if (blocks > INT32_MAX) return fail(SC_ERR_OVERFLOW, "neighbor map grid overflow");
    const size_t lds = (size_t)query_lds_ints(K, rpb) * sizeof(int);
    nm_query_kernel<<<(unsigned)blocks, 256, lds, s>>>(c4, n_rows, query_rows, ks, rpb, h, keys, rows, cap - 1,
                                                       otab, d_map);
    SC_LAUNCH_CHECK("nm_query_kernel launch");
    return SC_OK;
}

int sc_neighbor_map_check(const void *d_workspace, sc_stream stream)
{
    clear_error();
    if (!d_workspace) return fail(SC_ERR_NULL, "neighbor map workspace is NULL");
    hipStream_t s = as_stream(stream);
    uint32_t status = 0;
    SC_HIP_CHECK(hipMemcpyAsync(&status, &((const NbrHeader *)d_workspace)->status, sizeof(status),
                                hipMemcpyDeviceToHost, s),
                 "neighbor map status readback");
    SC_HIP_CHECK(hipStreamSynchronize(s), "neighbor map status sync");
    if (status & kStatusNegative)
        return fail(SC_ERR_COORD, "coord value exceeds i32::MAX (negative i32) for device neighbor kernel");
    return SC_OK;
}

}  // extern "C"
