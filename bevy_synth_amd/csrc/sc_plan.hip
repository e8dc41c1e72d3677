// Conv plan builder (layout in sc_plan.hpp).
//
// The halo-staged conv stages, per 256-row tile, every distinct input row the
// tile's neighbours touch into LDS once, instead of gathering a row from
// global memory for every (row, offset) pair: at config 3 each input row is
// gathered ~21 times by the direct kernel, but a tile of spatially compact
// rows touches only ~2 distinct input rows per output row.  The plan holds
// what that kernel needs and is built once per neighbour map.
//
// Row order (tiles of 256 consecutive entries of `order`):
//   1. init    : header, padding entries of `order` := -1
//   2. bbox    : min/max of the query coords (per-block partials, which
//                every prep block reduces; no atomics)
//   3. prep    : grid mode when the bounding box, cut into 8^3 bricks, has
//                at most grid_cap cells: the occupancy grid := EMPTY
//   4. place   : each row atomicMin's its row index into its cell (cells in
//                brick-major order, lexicographic inside a brick) and flags
//                the cell's 2048-cell block; the row displaced from a cell
//                (a duplicated coord) goes to a list
//   5. scan1/2 : occupied cells per flagged 2048-cell block (unflagged
//                blocks count 0 unread), then one block scans the totals
//   6. emit    : the occupied cells' rows compacted in cell order -> order
//                (blocks without occupied cells unread)
//   7. fix     : rows of duplicated coords appended after the distinct ones
// The order is a pure function of the coords (no sort, no atomics whose
// interleaving shows): bricks in (batch, x, y, z) order, lexicographic inside
// a brick.  Rows that already come in the order of 3 or more C2S
// subdivisions below a sorted set (the bbox pass tests it, as the map build
// does) keep their own order: they are grouped by aligned 8^3 root cells,
// Morton order inside, which is as compact, so steps 3-7 are skipped.
// Rows sorted and unique in (b, x, y, z) (no duplicate to place) take one
// occupancy bit per cell instead of the grid's row per cell: the bitmap
// stays in L2, and each row finds its own position by popcounts.
// A bounding box too large for the grid falls back to a counting
// sort by brick (brick edge 2^s, the smallest s >= 3 with at most brick_cap
// bricks): count, scan, scatter with wave-aggregated atomics, then each
// brick's segment sorted by row index so that the order is deterministic.
//
// Halo tables:
//   8. tiles   : one workgroup per tile, one thread per tile row; the
//                distinct neighbour rows are numbered in increasing row
//                order -> halo[] and the u16 local map lmap[k][row], through
//                an LDS bitmap over the tile's neighbour row range (the usual
//                case) or, for a wide range, an LDS hash table and a bitonic
//                sort.  Tiles whose halo exceeds kPlanHaloMax are listed in
//                `overflow` (the conv gathers their operands from global
//                memory; the list is a diagnostic).
#include <climits>

#include "sc_common.hpp"
#include "sc_plan.hpp"

namespace sc {
namespace {

constexpr int kThreads = 256;
constexpr int kTileThreads = kPlanTileRows;  // plan_tiles_kernel: one thread per tile row
// Tile hash table: a tile with more than kPlanHaloMax distinct neighbours
// gets no halo (the conv gathers its operands), so insertion stops past that many keys and
// 2048 slots (load factor < 1/2 for a tile that fits) suffice.
constexpr int kHashBits = 11;
constexpr int kHashSlots = 1 << kHashBits;

struct PlanArgs {
    const int4 *coords;
    const int32_t *map;
    int64_t n_q;
    int64_t n_in;
    int K;
    PlanHeader *hdr;
    int32_t *order;
    int32_t *tile_u;
    int32_t *overflow;
    int32_t *halo;
    uint16_t *lmap;
    uint32_t *grid;
    int32_t *gsum;
    int32_t *counts;
    int32_t *offsets;
    int32_t *bsum;
    int64_t n_tiles;
    int64_t brick_cap;
    int64_t n_bsum;
    int64_t grid_cap;
    // plan_tiles_kernel on listed tiles only (a child plan's split tiles):
    // workgroup b takes tile_list[b] when b < *tile_list_n; the overflow
    // list is then not appended to (the caller rebuilds it)
    const int32_t *tile_list;
    const int32_t *tile_list_n;
};

constexpr uint32_t kGridEmpty = 0xFFFFFFFFu;

__device__ inline void plan_init(const PlanArgs &a)
{
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    if (tid == 0) {
        PlanHeader *h = a.hdr;
        h->n_q = a.n_q;
        h->n_in = a.n_in;
        h->n_tiles = (int32_t)a.n_tiles;
        h->K = a.K;
        h->brick_shift = -1;
        h->n_overflow = 0;
        for (int j = 0; j < 4; ++j) {
            h->bmin[j] = INT_MAX;
            h->bmax[j] = INT_MIN;
        }
        h->n_bricks = 0;
        h->status = 0;
        h->grid_mode = 0;
        h->n_unique = 0;
        h->n_extras = 0;
        h->list_tiles = 0;
    }
    for (int64_t i = a.n_q + tid; i < a.n_tiles * kPlanTileRows; i += stride) a.order[i] = -1;
}

// Header and padding entries of `order` (only launched without query rows;
// otherwise plan_bbox_kernel does it).
__global__ void plan_init_kernel(PlanArgs a) { plan_init(a); }

// Per-block min/max of the query coords and the octree-order bits
// (unsorted_levels of each row against its predecessor, ORed) -> partials of
// kPartial ints (in the brick-offset array, which the scan overwrites later:
// kBboxBlocks * kPartial <= 4096 <= brick_cap); every block of
// plan_prep_kernel reduces them (atomic-free, and no launch of its own).
constexpr int kBboxBlocks = 448;
constexpr int kPartial = 9;
static_assert(kBboxBlocks * kPartial <= 4096, "partials fit the smallest brick-offset array");
// Rows in octree order over at least this many levels keep their order.
constexpr int kOwnOrderLevels = 3;

__global__ __launch_bounds__(kThreads) void plan_bbox_kernel(PlanArgs a)
{
    __shared__ int s_mn[4][4], s_mx[4][4];
    __shared__ uint32_t s_uns[4];
    plan_init(a);  // header and order padding (read by no kernel before the next launch)
    int mn[4] = {INT_MAX, INT_MAX, INT_MAX, INT_MAX}, mx[4] = {INT_MIN, INT_MIN, INT_MIN, INT_MIN};
    uint32_t uns = 0;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // Wave-uniform loop, four rows per lane in flight: in each of them lane l
    // holds row w0 + u * stride + l, so lane l - 1 holds its predecessor
    // (lane 0 loads its own).
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t w0 = (int64_t)blockIdx.x * blockDim.x + wave * 64; w0 < a.n_q; w0 += 4 * stride) {
        int4 c[4], pl[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t i = w0 + u * stride + lane;
            c[u] = i < a.n_q ? a.coords[i] : make_int4(0, 0, 0, 0);
            pl[u] = lane == 0 && i < a.n_q && i > 0 ? a.coords[i - 1] : make_int4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t i = w0 + u * stride + lane;
            const int4 cu = c[u];
            int4 prev = make_int4(__shfl_up(cu.x, 1), __shfl_up(cu.y, 1), __shfl_up(cu.z, 1), __shfl_up(cu.w, 1));
            if (lane == 0) prev = pl[u];
            if (i < a.n_q) {
                const int v[4] = {cu.x, cu.y, cu.z, cu.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    mn[j] = min(mn[j], v[j]);
                    mx[j] = max(mx[j], v[j]);
                }
                if (i > 0) uns |= unsorted_levels(prev, cu);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        mn[j] = wave_min_i32(mn[j]);
        mx[j] = wave_max_i32(mx[j]);
        if (lane == 0) {
            s_mn[wave][j] = mn[j];
            s_mx[wave][j] = mx[j];
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) uns |= __shfl_xor(uns, off, 64);
    if (lane == 0) s_uns[wave] = uns;
    __syncthreads();
    if (threadIdx.x < 4) {
        const int j = threadIdx.x;
        int lo = INT_MAX, hi = INT_MIN;
        for (int w = 0; w < (int)blockDim.x / 64; ++w) {
            lo = min(lo, s_mn[w][j]);
            hi = max(hi, s_mx[w][j]);
        }
        a.offsets[blockIdx.x * kPartial + j] = lo;
        a.offsets[blockIdx.x * kPartial + 4 + j] = hi;
    }
    if (threadIdx.x == 0) {
        uint32_t u = 0;
        for (int w = 0; w < (int)blockDim.x / 64; ++w) u |= s_uns[w];
        a.offsets[blockIdx.x * kPartial + 8] = (int32_t)u;
    }
}

// Groups the active lanes of a wave by key: for each distinct key the lowest
// lane calls fn(key, count, lane) once; every lane of the group receives the
// leader's return value plus its rank among the group's lanes (lane order).
template <typename F>
__device__ inline int wave_runs(bool active, uint32_t key, F fn)
{
    const int lane = threadIdx.x & 63;
    uint64_t pending = __ballot(active);
    int mine = 0;
    while (pending) {
        const int leader = __builtin_ctzll(pending);
        const uint32_t k = __builtin_amdgcn_readlane(key, leader);
        const uint64_t same = __ballot(active && key == k) & pending;
        int r = 0;
        if (lane == leader) r = fn(k, __builtin_popcountll(same), lane);
        r = __builtin_amdgcn_readlane(r, leader);
        if ((same >> lane) & 1ull) mine = r + __builtin_popcountll(same & ((1ull << lane) - 1ull));
        pending &= ~same;
    }
    return mine;
}

struct BrickGrid {
    int shift;  // -1: no brick order fits the budget
    int64_t lo[4];
    int64_t nb[4];  // bricks per dimension (batch: one per batch index)
    uint64_t total;
};

__device__ inline BrickGrid brick_grid(const PlanHeader *h, int64_t cap)
{
    BrickGrid g;
    g.shift = -1;
    g.total = 0;
    int64_t ext[4];
    for (int j = 0; j < 4; ++j) {
        g.lo[j] = h->bmin[j];
        ext[j] = (int64_t)h->bmax[j] - (int64_t)h->bmin[j] + 1;
        g.nb[j] = 1;
    }
    if (ext[0] <= 0) return g;  // no rows
    for (int s = 3; s < 32; ++s) {
        double tot = (double)ext[0];
        int64_t nb[4] = {ext[0], 0, 0, 0};
        for (int j = 1; j < 4; ++j) {
            nb[j] = ((ext[j] - 1) >> s) + 1;
            tot *= (double)nb[j];
        }
        if (tot <= (double)cap) {
            g.shift = s;
            g.total = (uint64_t)nb[0] * (uint64_t)nb[1] * (uint64_t)nb[2] * (uint64_t)nb[3];
            for (int j = 0; j < 4; ++j) g.nb[j] = nb[j];
            return g;
        }
    }
    return g;
}

__device__ inline int64_t brick_of(const BrickGrid &g, int4 c)
{
    const int64_t b = (int64_t)c.x - g.lo[0];
    const int64_t x = ((int64_t)c.y - g.lo[1]) >> g.shift;
    const int64_t y = ((int64_t)c.z - g.lo[2]) >> g.shift;
    const int64_t z = ((int64_t)c.w - g.lo[3]) >> g.shift;
    return ((b * g.nb[1] + x) * g.nb[2] + y) * g.nb[3] + z;
}

// Occupancy-grid geometry: 8^3 bricks over the bounding box; a cell's index
// is brick * 512 + its lexicographic position inside the brick, bricks in
// (batch, x, y, z) order.  Valid when the cells fit the plan's grid.
struct GridGeom {
    bool ok;
    int64_t lo[4];
    int64_t nb[4];
    int64_t cells;
    int64_t blocks;  // 2048-cell blocks holding cells
};

// grid_cap: the most cells the layout holds (the u32 grid's capacity, or
// bitmap_cells below for the occupancy bitmap).
__device__ inline GridGeom grid_geom(const PlanHeader *h, int64_t grid_cap)
{
    GridGeom g;
    g.ok = false;
    g.cells = 0;
    g.blocks = 0;
    double tot = 512.0;
    for (int j = 0; j < 4; ++j) {
        g.lo[j] = h->bmin[j];
        const int64_t ext = (int64_t)h->bmax[j] - (int64_t)h->bmin[j] + 1;
        if (ext <= 0) return g;
        g.nb[j] = j == 0 ? ext : ((ext - 1) >> 3) + 1;
        tot *= (double)g.nb[j];
    }
    if (tot > (double)grid_cap) return g;
    g.ok = true;
    g.cells = g.nb[0] * g.nb[1] * g.nb[2] * g.nb[3] * 512;
    g.blocks = (g.cells + kPlanGridBlock - 1) / kPlanGridBlock;
    return g;
}

// Occupancy-bitmap order (rows sorted and unique in (b, x, y, z)): one bit
// per cell of the same brick-major layout, in the grid's words; a row's
// position in the order is the number of occupied cells before its own,
// from a prefix per 256-cell block (in the brick-count array) and one per
// 65,536-cell group (gsum).  It holds 32 cells per grid word, as far as the
// block prefixes fit the brick-count array.
constexpr int kBitBlock = 256;      // cells per block prefix (8 words)
constexpr int kBitGroup = 65536;    // cells per group prefix (256 blocks, one scan1 workgroup)

__device__ inline int64_t bitmap_cells(const PlanArgs &a)
{
    const int64_t by_words = 32 * a.grid_cap, by_prefix = kBitBlock * a.brick_cap;
    return by_words < by_prefix ? by_words : by_prefix;
}

__device__ inline int64_t grid_cell(const GridGeom &g, int4 c)
{
    const int64_t b = (int64_t)c.x - g.lo[0];
    const int64_t x = (int64_t)c.y - g.lo[1], y = (int64_t)c.z - g.lo[2], z = (int64_t)c.w - g.lo[3];
    const int64_t brick = ((b * g.nb[1] + (x >> 3)) * g.nb[2] + (y >> 3)) * g.nb[3] + (z >> 3);
    return brick * 512 + ((x & 7) * 64 + (y & 7) * 8 + (z & 7));
}

// Every block reduces the bbox partials of plan_bbox_kernel (nbb blocks x kPartial
// ints, from L2; block 0 writes the bbox to the header) and chooses the
// ordering mode; grid mode: grid := EMPTY, block flags := 0; fallback: brick
// counts := 0.
__global__ __launch_bounds__(kThreads) void plan_prep_kernel(PlanArgs a, int nbb)
{
    __shared__ PlanHeader s_h;  // only bmin / bmax are set
    __shared__ int s_v[8][kThreads / 64];
    __shared__ uint32_t s_uns[kThreads / 64];
    uint32_t uns = 0;
    {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        int v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = j < 4 ? INT_MAX : INT_MIN;
        for (int b = threadIdx.x; b < nbb; b += blockDim.x) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[j] = min(v[j], a.offsets[b * kPartial + j]);
                v[4 + j] = max(v[4 + j], a.offsets[b * kPartial + 4 + j]);
            }
            uns |= (uint32_t)a.offsets[b * kPartial + 8];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[j] = j < 4 ? wave_min_i32(v[j]) : wave_max_i32(v[j]);
            if (lane == 0) s_v[j][wave] = v[j];
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) uns |= __shfl_xor(uns, off, 64);
        if (lane == 0) s_uns[wave] = uns;
        __syncthreads();
        uns = 0;
        for (int w = 0; w < kThreads / 64; ++w) uns |= s_uns[w];
        if (threadIdx.x < 8) {
            const int j = threadIdx.x;
            int r = s_v[j][0];
            for (int w = 1; w < (int)blockDim.x / 64; ++w) r = j < 4 ? min(r, s_v[j][w]) : max(r, s_v[j][w]);
            if (j < 4) {
                s_h.bmin[j] = r;
                if (blockIdx.x == 0) a.hdr->bmin[j] = r;
            } else {
                s_h.bmax[j - 4] = r;
                if (blockIdx.x == 0) a.hdr->bmax[j - 4] = r;
            }
        }
        __syncthreads();
    }
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    // Rows in octree order over kOwnOrderLevels or more levels keep their
    // order (no grid, no sort): grid_mode 2, and the later order kernels exit.
    const uint32_t deep = ((1u << kRankLevels) - 1u) & ~((1u << kOwnOrderLevels) - 1u);
    if ((~uns & deep) != 0u && a.n_q > 0) {
        if (tid == 0) {
            a.hdr->grid_mode = 2;
            a.hdr->brick_shift = -1;
            a.hdr->n_bricks = 0;
            a.hdr->n_unique = (int32_t)a.n_q;
        }
        for (int64_t i = tid; i < a.n_q; i += stride) a.order[i] = (int32_t)i;
        return;
    }
    if (!(uns & 1u)) {
        // sorted, unique rows: the occupancy bitmap (bits := 0, group flags := 0)
        const GridGeom bg = grid_geom(&s_h, bitmap_cells(a));
        if (bg.ok) {
            if (tid == 0) {
                a.hdr->grid_mode = 3;
                a.hdr->brick_shift = 3;
                a.hdr->n_bricks = (uint64_t)(bg.cells / 512);
            }
            uint4 *w4 = reinterpret_cast<uint4 *>(a.grid);  // cells / 32 words, a multiple of 16
            for (int64_t i = tid; i < bg.cells / 128; i += stride) w4[i] = make_uint4(0, 0, 0, 0);
            for (int64_t i = tid; i < (bg.cells + kBitGroup - 1) / kBitGroup; i += stride) a.gsum[i] = 0;
            return;
        }
    }
    const GridGeom gg = grid_geom(&s_h, a.grid_cap);
    if (gg.ok) {
        if (tid == 0) {
            a.hdr->grid_mode = 1;
            a.hdr->brick_shift = 3;
            a.hdr->n_bricks = (uint64_t)(gg.cells / 512);
        }
        // cells: a multiple of 512; the grid is 256-byte aligned
        uint4 *g4 = reinterpret_cast<uint4 *>(a.grid);
        const uint4 empty4 = make_uint4(kGridEmpty, kGridEmpty, kGridEmpty, kGridEmpty);
        for (int64_t i = tid; i < gg.cells / 4; i += stride) g4[i] = empty4;
        // per 2048-cell block: touched flag (set by place, read by scan1)
        for (int64_t i = tid; i < gg.blocks; i += stride) a.gsum[i] = 0;
        return;
    }
    const BrickGrid g = brick_grid(&s_h, a.brick_cap);
    if (tid == 0) {
        a.hdr->brick_shift = g.shift;
        a.hdr->n_bricks = g.total;
    }
    for (int64_t i = tid; i < a.brick_cap; i += stride) a.counts[i] = 0;
}

// Grid mode: each query row claims its cell (the lowest row of a duplicated
// coord keeps it, the others go to the extras list); fallback: brick counts.
__global__ __launch_bounds__(kThreads) void plan_place_kernel(PlanArgs a)
{
    if (a.hdr->grid_mode == 2) return;  // rows keep their own order
    if (a.hdr->grid_mode == 3) {
        // Sorted rows put runs of consecutive lanes on one word (a z-run
        // inside a brick): a segmented OR over the lanes of each run, then
        // one atomic per run (same-address atomics serialise).  A word seen
        // again in a later run of the wave gets a second OR; ORs commute.
        const GridGeom bg = grid_geom(a.hdr, bitmap_cells(a));
        const int lane = threadIdx.x & 63;
        const int64_t stride = (int64_t)gridDim.x * blockDim.x;
        for (int64_t w0 = (int64_t)blockIdx.x * blockDim.x + (threadIdx.x & ~63); w0 < a.n_q; w0 += stride) {
            const int64_t i = w0 + lane;
            const bool valid = i < a.n_q;
            const int64_t cell = valid ? grid_cell(bg, a.coords[i]) : -1;
            const int64_t w = valid ? cell >> 5 : -2 - lane;  // invalid lanes match nothing
            uint32_t bits = valid ? 1u << (cell & 31) : 0u;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const uint32_t ob = __shfl_down(bits, d, 64);
                const int64_t ow = __shfl_down(w, d, 64);
                if (lane + d < 64 && ow == w) bits |= ob;
            }
            const int64_t wp = __shfl_up(w, 1, 64);
            if (valid && (lane == 0 || wp != w)) {
                atomicOr(&a.grid[w], bits);
                a.gsum[cell / kBitGroup] = 1;  // the group holds a cell: scan1 reads it
            }
        }
        return;
    }
    if (a.hdr->grid_mode == 1) {
        const GridGeom gg = grid_geom(a.hdr, a.grid_cap);
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n_q;
             i += (int64_t)gridDim.x * blockDim.x) {
            const int64_t cell = grid_cell(gg, a.coords[i]);
            const uint32_t old = atomicMin(&a.grid[cell], (uint32_t)i);
            if (old != kGridEmpty) atomicAdd(&a.hdr->n_extras, 1);
            a.gsum[cell / kPlanGridBlock] = 1;  // the block holds a cell: scan1 and emit read it
        }
        return;
    }
    const int shift = a.hdr->brick_shift;
    if (shift < 0) return;
    const BrickGrid g = brick_grid(a.hdr, a.brick_cap);
    for (int64_t base = (int64_t)blockIdx.x * blockDim.x; base < a.n_q; base += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = base + threadIdx.x;
        const bool act = i < a.n_q;
        const uint32_t br = act ? (uint32_t)brick_of(g, a.coords[i]) : 0u;
        wave_runs(act, br, [&](uint32_t key, int n, int) {
            atomicAdd(&a.counts[key], n);
            return 0;
        });
    }
}

// Block-wide exclusive scan of one int per thread (256 threads).
__device__ inline int block_scan_excl(int x, int *s_wave, int &total)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int inc = x;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(inc, off, 64);
        if (lane >= off) inc += y;
    }
    __syncthreads();
    if (lane == 63) s_wave[wave] = inc;
    __syncthreads();
    int before = 0;
    total = 0;
    for (int w = 0; w < kThreads / 64; ++w) {
        if (w < wave) before += s_wave[w];
        total += s_wave[w];
    }
    return before + inc - x;
}

// Grid mode, duplicated coords: query rows whose cell holds a lower row.
// 2048-row blocks, 8 consecutive rows per thread; returns the thread's count
// and (optionally) its rows as bits.
__device__ inline int64_t row_blocks(const PlanArgs &a) { return (a.n_q + kPlanGridBlock - 1) / kPlanGridBlock; }

__device__ inline int extras_in(const PlanArgs &a, const GridGeom &gg, int64_t rb, uint32_t *flags = nullptr)
{
    const int64_t r0 = rb * kPlanGridBlock + threadIdx.x * 8;
    uint32_t f = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int64_t i = r0 + u;
        if (i < a.n_q && a.grid[grid_cell(gg, a.coords[i])] != (uint32_t)i) f |= 1u << u;
    }
    if (flags) *flags = f;
    return __builtin_popcount(f);
}

// Grid mode: occupied cells per 2048-cell block -> gsum (in place of the
// block's flag; an unflagged block holds no cell and is not read), and with duplicated
// coords the extra rows per 2048-row block -> bsum; fallback: exclusive
// scan of the brick counts within 1024-entry blocks, block totals -> bsum.
__global__ __launch_bounds__(kThreads) void plan_scan1_kernel(PlanArgs a)
{
    __shared__ int s_wave[kThreads / 64];
    if (a.hdr->grid_mode == 2) return;
    if (a.hdr->grid_mode == 3) {
        // group g (one workgroup): thread t counts block 256 g + t (8 words),
        // block prefixes within the group -> counts, the group total -> gsum
        static_assert(kBitGroup == kBitBlock * kThreads, "one block per thread");
        const GridGeom bg = grid_geom(a.hdr, bitmap_cells(a));
        const int64_t g = blockIdx.x;
        if (g * kBitGroup >= bg.cells || a.gsum[g] == 0) return;  // no cell placed: stays 0
        const int64_t b = g * kThreads + threadIdx.x;
        int cnt = 0;
        if (b * kBitBlock < bg.cells) {
            const uint4 *w4 = reinterpret_cast<const uint4 *>(a.grid + b * (kBitBlock / 32));
            const uint4 u0 = w4[0], u1 = w4[1];
            cnt = __builtin_popcount(u0.x) + __builtin_popcount(u0.y) + __builtin_popcount(u0.z) +
                  __builtin_popcount(u0.w) + __builtin_popcount(u1.x) + __builtin_popcount(u1.y) +
                  __builtin_popcount(u1.z) + __builtin_popcount(u1.w);
        }
        int total;
        const int ex = block_scan_excl(cnt, s_wave, total);
        if (b * kBitBlock < bg.cells) a.counts[b] = ex;
        if (threadIdx.x == 0) a.gsum[g] = total;
        return;
    }
    if (a.hdr->grid_mode == 1) {
        const int64_t nblk = a.grid_cap / kPlanGridBlock;
        const GridGeom gg = grid_geom(a.hdr, a.grid_cap);
        if ((int64_t)blockIdx.x >= nblk) {  // rows of duplicated coords per 2048-row block
            const int64_t rb = (int64_t)blockIdx.x - nblk;
            if (a.hdr->n_extras == 0 || rb >= row_blocks(a)) return;
            int total;
            block_scan_excl(extras_in(a, gg, rb), s_wave, total);
            if (threadIdx.x == 0) a.bsum[rb] = total;
            return;
        }
        if ((int64_t)blockIdx.x >= gg.blocks) return;  // beyond the cells in use
        if (a.gsum[blockIdx.x] == 0) return;           // no cell placed: the count stays 0
        const int64_t base = (int64_t)blockIdx.x * kPlanGridBlock + threadIdx.x * 8;
        int cnt = 0;
        if (base < gg.cells) {
            const uint4 *g4 = reinterpret_cast<const uint4 *>(a.grid + base);
            const uint4 u0 = g4[0], u1 = g4[1];
            cnt = (u0.x != kGridEmpty) + (u0.y != kGridEmpty) + (u0.z != kGridEmpty) + (u0.w != kGridEmpty) +
                  (u1.x != kGridEmpty) + (u1.y != kGridEmpty) + (u1.z != kGridEmpty) + (u1.w != kGridEmpty);
        }
        int total;
        block_scan_excl(cnt, s_wave, total);
        if (threadIdx.x == 0) a.gsum[blockIdx.x] = total;
        return;
    }
    if ((int64_t)blockIdx.x >= a.n_bsum || a.hdr->brick_shift < 0) return;
    const int64_t base = (int64_t)blockIdx.x * kPlanScanBlock + threadIdx.x * 4;
    const int4 c = *reinterpret_cast<const int4 *>(a.counts + base);
    int total;
    const int ex = block_scan_excl(c.x + c.y + c.z + c.w, s_wave, total);
    int4 o;
    o.x = ex;
    o.y = ex + c.x;
    o.z = o.y + c.y;
    o.w = o.z + c.z;
    *reinterpret_cast<int4 *>(a.offsets + base) = o;
    if (threadIdx.x == 0) a.bsum[blockIdx.x] = total;
}

// In-place exclusive scan of arr[0, n) by one block in a single pass: thread
// p sums a contiguous segment of ceil(n / 256) entries (rounded up to 4), one
// block-wide scan of the sums, then each thread writes its segment's
// prefixes.  Returns the total.
__device__ inline int block_scan_array(int32_t *arr, int64_t n, int *s_wave)
{
    const int64_t seg = ((n + kThreads - 1) / kThreads + 3) & ~(int64_t)3;
    const int64_t b0 = min((int64_t)threadIdx.x * seg, n), b1 = min(b0 + seg, n);
    int sum = 0;
#pragma unroll 8
    for (int64_t i = b0; i < b1; ++i) sum += arr[i];
    int total;
    int run = block_scan_excl(sum, s_wave, total);
#pragma unroll 8
    for (int64_t i = b0; i < b1; ++i) {
        const int v = arr[i];
        arr[i] = run;
        run += v;
    }
    return total;
}

// Exclusive scan of the block totals (gsum or bsum, one block).  Grid mode:
// the total (distinct coords) -> n_unique.
__global__ __launch_bounds__(kThreads) void plan_scan2_kernel(PlanArgs a)
{
    __shared__ int s_wave[kThreads / 64];
    if (a.hdr->grid_mode == 2) return;
    if (a.hdr->grid_mode == 3) {
        const GridGeom bg = grid_geom(a.hdr, bitmap_cells(a));
        const int total = block_scan_array(a.gsum, (bg.cells + kBitGroup - 1) / kBitGroup, s_wave);
        if (threadIdx.x == 0) a.hdr->n_unique = total;
        return;
    }
    const bool grid = a.hdr->grid_mode == 1;
    if (!grid && a.hdr->brick_shift < 0) return;
    int32_t *arr = grid ? a.gsum : a.bsum;
    const int64_t n = grid ? grid_geom(a.hdr, a.grid_cap).blocks : a.n_bsum;
    const int total = block_scan_array(arr, n, s_wave);
    if (grid && threadIdx.x == 0) a.hdr->n_unique = total;
    if (grid && a.hdr->n_extras > 0) block_scan_array(a.bsum, row_blocks(a), s_wave);
}

__device__ inline int64_t brick_start(const PlanArgs &a, uint32_t br)
{
    return (int64_t)a.offsets[br] + a.bsum[br / kPlanScanBlock];
}

// Grid mode: the rows of the occupied cells in cell order -> order (brick
// order, lexicographic within a brick).  Fallback: rows to their brick's
// segment (ranks from wave-aggregated atomics), or row order when no brick
// grid fits.
__global__ __launch_bounds__(kThreads) void plan_emit_kernel(PlanArgs a)
{
    __shared__ int s_wave[kThreads / 64];
    if (a.hdr->grid_mode == 2) return;
    if (a.hdr->grid_mode == 3) {
        // each row's position: group prefix + block prefix + the occupied
        // cells before its own in the block (at most 8 words)
        const GridGeom bg = grid_geom(a.hdr, bitmap_cells(a));
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n_q;
             i += (int64_t)gridDim.x * blockDim.x) {
            const int64_t cell = grid_cell(bg, a.coords[i]);
            const int64_t b = cell / kBitBlock;
            // the block's 8 words (32 aligned bytes) and both prefixes in one
            // round trip (word-by-word conditional loads waited one by one)
            static_assert(kBitBlock == 256, "a block is two 16-byte loads");
            const uint4 *bw4 = reinterpret_cast<const uint4 *>(a.grid + b * (kBitBlock / 32));
            const uint4 lo = bw4[0], hi = bw4[1];
            const int32_t gp = a.gsum[cell / kBitGroup], bp = a.counts[b];
            const uint32_t bw[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            const int wi = (int)((cell >> 5) & (kBitBlock / 32 - 1));
            int before = 0;
#pragma unroll
            for (int w = 0; w < kBitBlock / 32; ++w) {
                const uint32_t m = w < wi ? 0xFFFFFFFFu : (w == wi ? (1u << (cell & 31)) - 1u : 0u);
                before += __builtin_popcount(bw[w] & m);
            }
            a.order[(int64_t)gp + bp + before] = (int32_t)i;
        }
        return;
    }
    if (a.hdr->grid_mode == 1) {
        const int64_t nblk = a.grid_cap / kPlanGridBlock;
        const GridGeom gg = grid_geom(a.hdr, a.grid_cap);
        if ((int64_t)blockIdx.x >= nblk) {  // rows of duplicated coords, in row order
            const int64_t rb = (int64_t)blockIdx.x - nblk;
            if (a.hdr->n_extras == 0 || rb >= row_blocks(a)) return;
            uint32_t flags;
            const int cnt = extras_in(a, gg, rb, &flags);
            int total;
            int64_t pos = (int64_t)a.hdr->n_unique + a.bsum[rb] + block_scan_excl(cnt, s_wave, total);
            const int64_t r0 = rb * kPlanGridBlock + threadIdx.x * 8;
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if ((flags >> u) & 1u) a.order[pos++] = (int32_t)(r0 + u);
            return;
        }
        if ((int64_t)blockIdx.x >= gg.blocks) return;  // beyond the cells in use
        const int64_t next = (int64_t)blockIdx.x + 1 < gg.blocks ? (int64_t)a.gsum[blockIdx.x + 1]
                                                                  : (int64_t)a.hdr->n_unique;
        if (next == (int64_t)a.gsum[blockIdx.x]) return;  // no occupied cell in the block
        const int64_t base = (int64_t)blockIdx.x * kPlanGridBlock + threadIdx.x * 8;
        uint32_t r[8];
        int cnt = 0;
#pragma unroll
        for (int u = 0; u < 8; ++u) r[u] = kGridEmpty;
        if (base < gg.cells) {
            const uint4 *g4 = reinterpret_cast<const uint4 *>(a.grid + base);
            const uint4 u0 = g4[0], u1 = g4[1];
            r[0] = u0.x; r[1] = u0.y; r[2] = u0.z; r[3] = u0.w;
            r[4] = u1.x; r[5] = u1.y; r[6] = u1.z; r[7] = u1.w;
#pragma unroll
            for (int u = 0; u < 8; ++u) cnt += r[u] != kGridEmpty;
        }
        int total;
        int pos = a.gsum[blockIdx.x] + block_scan_excl(cnt, s_wave, total);
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (r[u] != kGridEmpty) a.order[pos++] = (int32_t)r[u];
        return;
    }
    const int shift = a.hdr->brick_shift;
    BrickGrid g;
    if (shift >= 0) g = brick_grid(a.hdr, a.brick_cap);
    for (int64_t base = (int64_t)blockIdx.x * blockDim.x; base < a.n_q; base += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = base + threadIdx.x;
        const bool act = i < a.n_q;
        if (shift < 0) {
            if (act) a.order[i] = (int32_t)i;
            continue;
        }
        const uint32_t br = act ? (uint32_t)brick_of(g, a.coords[i]) : 0u;
        // counts[br] counts down: the group takes ranks [old - n, old)
        const int rank = wave_runs(act, br, [&](uint32_t key, int n, int) { return atomicSub(&a.counts[key], n) - n; });
        if (act) a.order[brick_start(a, br) + rank] = (int32_t)i;
    }
}

// Fallback mode: each brick's segment sorted by row index (one wave per
// brick, rank = number of smaller rows), so the order is deterministic;
// segments longer than kSegWave (only with duplicated coords) keep the
// scatter's order.  (Grid mode needs no fix-up: emit places everything.)
constexpr int kSegWave = 512;

__global__ __launch_bounds__(kThreads) void plan_fix_kernel(PlanArgs a)
{
    __shared__ __attribute__((aligned(16))) int32_t s_seg[kThreads / 64][kSegWave];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (a.hdr->grid_mode) return;  // grid mode places everything; own order needs nothing
    if (a.hdr->brick_shift < 0) return;
    const uint64_t nb = a.hdr->n_bricks;
    int32_t *seg_lds = s_seg[wave];
    for (uint64_t br = (uint64_t)blockIdx.x * (kThreads / 64) + wave; br < nb;
         br += (uint64_t)gridDim.x * (kThreads / 64)) {
        const int64_t start = brick_start(a, (uint32_t)br);
        const int64_t end = br + 1 < nb ? brick_start(a, (uint32_t)(br + 1)) : a.n_q;
        const int n = (int)(end - start);
        if (n <= 1 || n > kSegWave) continue;
        int32_t *seg = a.order + start;
        const int n4 = (n + 3) & ~3;
        constexpr int kPer = kSegWave / 64;
        int32_t mine[kPer];
        int rank[kPer];
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int e = lane + 64 * u;
            mine[u] = e < n ? seg[e] : INT_MAX;
            rank[u] = 0;
            if (e < n4) seg_lds[e] = mine[u];
        }
        // the wave's own LDS writes are visible to its later reads once lgkmcnt drains
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
        const int4 *s4 = reinterpret_cast<const int4 *>(seg_lds);
        for (int f = 0; f < n4 / 4; ++f) {
            const int4 v = s4[f];
#pragma unroll
            for (int u = 0; u < kPer; ++u)
                rank[u] += (v.x < mine[u]) + (v.y < mine[u]) + (v.z < mine[u]) + (v.w < mine[u]);
        }
#pragma unroll
        for (int u = 0; u < kPer; ++u)
            if (lane + 64 * u < n) seg[rank[u]] = mine[u];
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    }
}

__device__ inline uint32_t slot_hash(int32_t v)
{
    return ((uint32_t)v * 0x9E3779B1u) >> (32 - kHashBits);
}

// Block-wide exclusive scan for plan_tiles_kernel (kTileThreads threads).
__device__ inline int tile_scan_excl(int x, int *s_wave, int &total)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int inc = x;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(inc, off, 64);
        if (lane >= off) inc += y;
    }
    __syncthreads();
    if (lane == 63) s_wave[wave] = inc;
    __syncthreads();
    int before = 0;
    total = 0;
    for (int w = 0; w < kTileThreads / 64; ++w) {
        if (w < wave) before += s_wave[w];
        total += s_wave[w];
    }
    return before + inc - x;
}

// Halo numbering: the rank of a row among the tile's distinct neighbour rows.
//  * bitmap path (the neighbours span at most kBitmapBits row indices, the
//    usual case for brick-ordered rows): one bit per row index in LDS, then
//    a per-word prefix of popcounts; rank = prefix + popcount below the bit.
//  * paged bitmap (a wider span, but within kPages pages of kPageRows rows):
//    the same over the tile's pages laid side by side in page order.
//  * otherwise: an LDS hash table of the distinct rows, sorted (bitonic).
constexpr int kBitmapWords = 4096;  // 131072 row indices
constexpr int kBitmapBits = kBitmapWords * 32;
// Paged bitmap: neighbour rows wider apart than kBitmapBits (rows in octree
// or coarse-brick order put the x-adjacent neighbours ~100,000 rows away)
// but inside at most kPages pages of kPageRows rows get those pages of the
// bitmap side by side in page order instead of one contiguous window.  The
// tile's pages are found as bits of a page bitmap over its neighbour range
// (at most kPageBits pages, 4 M rows), and a page's rank is the number of
// set bits below its own.
constexpr int kPageShift = 12;
constexpr int kPageRows = 1 << kPageShift;               // 128 bitmap words
constexpr int kPages = kBitmapBits / kPageRows;          // 32
constexpr int kPageWords = 32;                           // page bitmap words
constexpr int kPageBits = kPageWords * 32;               // 1024 pages

__global__ __launch_bounds__(kTileThreads) void plan_tiles_kernel(PlanArgs a)
{
    // 28 KB in all, so that five workgroups fit a CU
    __shared__ uint32_t s_bits[kBitmapWords];      // bitmap, or the hash table's keys
    __shared__ __attribute__((aligned(16))) uint16_t s_pre[kBitmapWords];  // word prefix (bitmap path)
    __shared__ int s_nkeys;                         // keys inserted (hash path)
    __shared__ int32_t s_halo[kPlanHaloMax];        // the halo rows (bitmap path)
    __shared__ int s_wave[kTileThreads / 64];
    __shared__ int s_mm[2][kTileThreads / 64];
    __shared__ uint32_t s_pbits[kPageWords]; // paged: the tile's pages (ids relative to lo)
    __shared__ int32_t s_ppre[kPageWords];   // set bits in the words before each word
    __shared__ int32_t s_pid[kPages];        // page id of rank r
    __shared__ int s_npages;
    int32_t *s_key = reinterpret_cast<int32_t *>(s_bits);
    uint64_t *s_list = reinterpret_cast<uint64_t *>(s_pre);  // up to 1024 sorted entries
    static_assert(kHashSlots <= kBitmapWords, "hash table fits the bitmap array");
    static_assert(kPlanHaloMax <= 1024 && 1024 * 8 <= kBitmapWords * 2, "sort list fits the prefix array");
    // XCD-contiguous tiles: neighbouring tiles read neighbouring map rows.
    // Rows in their own (octree) order take the tiles round-robin instead:
    // there the tiles whose neighbours span several pages (the slower paged
    // path) come in long runs, and contiguous ranges left half the XCDs idle
    // for the last third of the launch (config 5's last level).
    int64_t t;
    if (a.tile_list) {
        if ((int)blockIdx.x >= *a.tile_list_n) return;
        t = a.tile_list[blockIdx.x];
    } else if (a.hdr->grid_mode == kPlanModeChild) {
        // a child plan's list tiles in use (the grid covers the layout's
        // bound): dealt to the XCDs like any tile range, the rest exit
        const int n_used = a.hdr->n_unique;
        if ((int)blockIdx.x >= n_used) return;
        t = tile_for_block((int)blockIdx.x, n_used);
    } else if (a.hdr->grid_mode == 2) {
        t = blockIdx.x;
    } else {
        t = tile_for_block((int)blockIdx.x, (int)gridDim.x);
    }
    const int p = threadIdx.x;
    const int lane = p & 63, wave = p >> 6;
    const int K = a.K;
    const int32_t n_in = (int32_t)a.n_in;  // <= INT32_MAX
    // rows that keep their own order (grid_mode 2): order[i] = i, so the
    // tile's rows need no read before their map rows
    const int64_t slot = t * kPlanTileRows + p;
    const int32_t q = a.hdr->grid_mode == 2 ? (slot < a.n_q ? (int32_t)slot : -1) : a.order[slot];
    // A tile of padding only (a child plan's unused list and spare tiles)
    // records an empty halo and writes nothing else: no conv reads the
    // other tables of such a tile.
    if (!__syncthreads_or(q >= 0)) {
        if (p == 0) a.tile_u[t] = 0;
        return;
    }

    int32_t v[32];
    if (a.n_q * (int64_t)K * 4 + 256 <= (int64_t)kOobOffset) {
        // The thread's map row (K dwords at dword K*q, rows in brick order,
        // so scattered across lanes): 16-byte loads from the aligned-down
        // address, then a shift by the row's dword offset within 16 bytes
        // (s).  Maps of 3 GiB or more take one 4-byte load per entry.
        const int64_t map_bytes = a.n_q * (int64_t)K * 4;
        const __amdgpu_buffer_rsrc_t r = make_rsrc(a.map, (uint32_t)map_bytes);
        const int64_t d0 = q >= 0 ? (int64_t)q * K : 0;
        const int s = (int)(d0 & 3);
        const uint32_t base = q >= 0 ? (uint32_t)((d0 & ~(int64_t)3) * 4) : kOobOffset;
        const int nl = (K + 6) >> 2;  // loads covering s + K dwords for every s
        uint32_t w[36];
#pragma unroll
        for (int i = 0; i < 9; ++i) {
            uint4 x = make_uint4(0u, 0u, 0u, 0u);
            if (i < nl) x = bload16(r, base + 16u * i);
            w[4 * i] = x.x;
            w[4 * i + 1] = x.y;
            w[4 * i + 2] = x.z;
            w[4 * i + 3] = x.w;
        }
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            const int32_t x = (int32_t)(s == 0 ? w[k] : s == 1 ? w[k + 1] : s == 2 ? w[k + 2] : w[k + 3]);
            v[k] = (k < K && q >= 0 && x >= 0 && x < n_in) ? x : -1;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            int32_t x = -1;
            if (k < K && q >= 0) x = a.map[(int64_t)q * K + k];
            v[k] = (x >= 0 && x < n_in) ? x : -1;
        }
    }
    int lo = INT_MAX, hi = INT_MIN;
#pragma unroll
    for (int k = 0; k < 32; ++k)
        if (v[k] >= 0) {
            lo = min(lo, v[k]);
            hi = max(hi, v[k]);
        }
    lo = wave_min_i32(lo);
    hi = wave_max_i32(hi);
    if (lane == 0) {
        s_mm[0][wave] = lo;
        s_mm[1][wave] = hi;
    }
    __syncthreads();
    for (int w = 0; w < kTileThreads / 64; ++w) {
        lo = min(lo, s_mm[0][w]);
        hi = max(hi, s_mm[1][w]);
    }
    int32_t *halo = a.halo + t * kPlanHaloMax;
    uint16_t *lm = a.lmap + t * K * kPlanTileRows + p;
    const bool window = hi < lo || (int64_t)hi - lo < (int64_t)kBitmapBits;
    bool paged = false;
    int np = 0;
    if (!window && (int64_t)hi - lo < (int64_t)kPageBits * kPageRows) {
        // The tile's distinct pages as bits (a wider range takes the hash
        // path).
        if (p < kPageWords) s_pbits[p] = 0u;
        __syncthreads();
        // A row's neighbours come in offset order, z fastest, so runs of
        // them share a page: each run sets its bit once.
        int32_t last_pg = -1;
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            if (v[k] < 0) continue;
            const int32_t pg = (int32_t)((uint32_t)(v[k] - lo) >> kPageShift);
            if (pg == last_pg) continue;
            last_pg = pg;
            atomicOr(&s_pbits[pg >> 5], 1u << (pg & 31));
        }
        __syncthreads();
        if (p < kPageWords) {
            // lanes 0..31 of wave 0: the words' exclusive prefix of set bits,
            // and the page ids in rank order (while they fit kPages)
            const uint32_t w = s_pbits[p];
            const int c = __builtin_popcount(w);
            int pre = c;
#pragma unroll
            for (int off = 1; off < kPageWords; off <<= 1) {
                const int y = __shfl_up(pre, off, kPageWords);
                if (p >= off) pre += y;
            }
            pre -= c;
            s_ppre[p] = pre;
            uint32_t rest = w;
            for (int r = pre; rest != 0u; ++r) {
                const int b = __builtin_ctz(rest);
                rest &= rest - 1u;
                if (r < kPages) s_pid[r] = p * 32 + b;
            }
            if (p == kPageWords - 1) s_npages = pre + c;
        }
        __syncthreads();
        np = s_npages;
        paged = np <= kPages;
        if (paged) {
            // position: page rank * kPageRows + the row's offset in its page
            int32_t run_pg = -1, run_rank = 0;
#pragma unroll
            for (int k = 0; k < 32; ++k) {
                if (v[k] < 0) continue;
                const uint32_t d = (uint32_t)(v[k] - lo);
                const int32_t pg = (int32_t)(d >> kPageShift);
                if (pg != run_pg) {
                    run_pg = pg;
                    run_rank = s_ppre[pg >> 5] + __builtin_popcount(s_pbits[pg >> 5] & ((1u << (pg & 31)) - 1u));
                }
                v[k] = (run_rank << kPageShift) | (int32_t)(d & (kPageRows - 1));
            }
        }
    }

    if (window || paged) {
        // v[k] := the neighbour's position in the bitmap (row - lo in one
        // window; the paged position already); row_of inverts it.
        if (window) {
#pragma unroll
            for (int k = 0; k < 32; ++k)
                if (v[k] >= 0) v[k] -= lo;
        }
        auto row_of = [&](int32_t pos) {
            return paged ? lo + (s_pid[pos >> kPageShift] << kPageShift) + (pos & (kPageRows - 1)) : lo + pos;
        };
        // Only words [0, nw) can hold bits.
        const int nw = paged ? np * (kPageRows / 32) : (hi < lo ? 0 : (int)(((int64_t)hi - lo) >> 5) + 1);
        for (int i = p; i < nw; i += kTileThreads) s_bits[i] = 0u;
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 32; ++k)
            if (v[k] >= 0) atomicOr(&s_bits[v[k] >> 5], 1u << (v[k] & 31));
        __syncthreads();
        // Thread p owns `chunk` consecutive words, chunk odd so that the lanes
        // of a wave (stride chunk words) hit distinct LDS banks; first the
        // popcounts, then, after the scan, each word's prefix.
        int chunk = (nw + kTileThreads - 1) / kTileThreads;
        chunk |= 1;
        const int w0 = p * chunk, w1 = min(w0 + chunk, nw);
        int cnt = 0;
        for (int w = w0; w < w1; ++w) cnt += __builtin_popcount(s_bits[w]);
        int U;
        int run = tile_scan_excl(cnt, s_wave, U);
        for (int w = w0; w < w1; ++w) {
            s_pre[w] = (uint16_t)run;
            run += __builtin_popcount(s_bits[w]);
        }
        if (p == 0) {
            a.tile_u[t] = U;
            if (U > kPlanHaloMax && !a.tile_list) a.overflow[atomicAdd(&a.hdr->n_overflow, 1)] = (int32_t)t;
        }
        if (U > kPlanHaloMax) return;  // no halo: the conv gathers this tile's operands
        __syncthreads();
        // Each neighbour's rank is its local index; its row goes to that
        // halo slot (neighbours shared by several rows write the same row).
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            if (k >= K) break;
            uint16_t out = kPlanAbsent;
            if (v[k] >= 0) {
                const int d = v[k], w = d >> 5;
                out = (uint16_t)(s_pre[w] + __builtin_popcount(s_bits[w] & ((1u << (d & 31)) - 1u)));
                s_halo[out] = row_of(d);
            }
            lm[k * kPlanTileRows] = out;
        }
        __syncthreads();
        for (int i = p; i < U; i += kTileThreads) halo[i] = s_halo[i];  // coalesced
        return;
    }

    // ---- wide neighbour range: LDS hash table of the distinct rows (linear
    // probing, every probe loop bounded by the slot count).  A slot is read
    // before it is claimed; each neighbour's slot is kept.  Once more than
    // kPlanHaloMax keys are in, the tile overflows whatever follows, and
    // insertion stops (the count of occupied slots then exceeds kPlanHaloMax).
    for (int i = p; i < kHashSlots; i += kTileThreads) s_key[i] = -1;
    if (p == 0) s_nkeys = 0;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        if (v[k] < 0) continue;
        uint32_t h = slot_hash(v[k]);
        for (int probe = 0; probe < kHashSlots; ++probe) {
            if (*(volatile int *)&s_nkeys > kPlanHaloMax) break;
            int32_t cur = s_key[h];
            if (cur == -1) {
                cur = atomicCAS(&s_key[h], -1, v[k]);
                if (cur == -1) atomicAdd(&s_nkeys, 1);
            }
            if (cur == -1 || cur == v[k]) break;
            h = (h + 1) & (kHashSlots - 1);
        }
        v[k] = (int32_t)h;  // present neighbour: its slot (absent stays -1)
    }
    __syncthreads();
    constexpr int kPer = kHashSlots / kTileThreads;
    int cnt = 0;
    for (int i = 0; i < kPer; ++i) cnt += s_key[p * kPer + i] >= 0;
    int U;
    int id = tile_scan_excl(cnt, s_wave, U);
    if (p == 0) {
        a.tile_u[t] = U;
        if (U > kPlanHaloMax && !a.tile_list) a.overflow[atomicAdd(&a.hdr->n_overflow, 1)] = (int32_t)t;
    }
    if (U > kPlanHaloMax) return;
    for (int i = 0; i < kPer; ++i) {
        const int slot = p * kPer + i;
        const int32_t key = s_key[slot];
        if (key >= 0) s_list[id++] = ((uint64_t)(uint32_t)key << 32) | (uint32_t)slot;
    }
    // Pad to a power of two and sort by row (bitonic); the rank is the halo index.
    int n2 = 1;
    while (n2 < U) n2 <<= 1;
    for (int i = U + p; i < n2; i += kTileThreads) s_list[i] = ~0ull;
    __syncthreads();
    for (int size = 2; size <= n2; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int e = p; e < n2; e += kTileThreads) {
                const int partner = e ^ stride;
                if (partner > e) {
                    const bool up = (e & size) == 0;
                    const uint64_t x = s_list[e], y = s_list[partner];
                    if ((x > y) == up) {
                        s_list[e] = y;
                        s_list[partner] = x;
                    }
                }
            }
            __syncthreads();
        }
    for (int e = p; e < U; e += kTileThreads) {
        const uint64_t kv = s_list[e];
        halo[e] = (int32_t)(kv >> 32);
        s_key[(uint32_t)kv & (kHashSlots - 1)] = e;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        if (k >= K) break;
        lm[k * kPlanTileRows] = v[k] >= 0 ? (uint16_t)s_key[v[k] & (kHashSlots - 1)] : kPlanAbsent;
    }
}

// ------------------------------------------------------------ child plans
//
// For C2S conv1 over the active children only (sc_conv_child_plan_build):
// per child index c, the entries of the parent plan's order whose child c is
// active, in that order, compacted into tiles of their own (sc_plan.hpp,
// ChildPlanLayout):
//   count  : one workgroup per parent-plan tile, a ballot per child
//   chunk  : per 256 parent tiles, the counts scanned per child (exclusive)
//   layout : one workgroup: the chunk totals scanned, the children's tile
//            ranges, the header and tile_child
//   emit   : every entry to its slot (chunk offset + in-chunk offset + the
//            wave's ballot prefix)
//   pad    : -1 in every slot no entry takes
//   tiles  : plan_tiles_kernel on the child order (the parents' map rows)
//   split  : each list tile whose halo overflows gives its rows 128..255 to
//            a spare tile (in tile order), then both are rebuilt, and the
//            overflow list is rebuilt in tile order
// The plan is a pure function of the inputs (no atomics whose order shows).

struct ChildArgs {
    const PlanHeader *phdr;     // the parent plan (NULL: parents in row order, a linear child plan)
    const int32_t *porder;      // its order [n_ptiles * 256] (NULL: row order)
    const int32_t *child_rows;  // [P][8]: row of child (p, c), or -1
    int64_t n_parents;
    int64_t n_children;
    int64_t n_ptiles;
    int64_t n_chunks;
    int64_t n_main;
    int64_t n_tiles;
    int K;
    PlanHeader *hdr;  // the child plan
    int32_t *order;
    int32_t *tile_child;
    int32_t *tile_u;
    int32_t *overflow;
    int32_t *counts;  // [n_ptiles][8]: count, then in-chunk exclusive offset
    int32_t *chunks;  // [n_chunks][8]: chunk total, then chunk exclusive offset
    int32_t *child_n;
    int32_t *child_base;
    int32_t *split;   // [n_extra][2]: (split tile, spare tile)
    int32_t *split_n; // 2 x splits: the rebuild's tile count
};

// Parent-order entry e: its parent row (-1 for padding) and its active
// children as bits (a row outside [0, n_children) counts as inactive).
__device__ inline uint32_t child_bits(const ChildArgs &a, int64_t e, int32_t &p)
{
    p = a.porder ? a.porder[e] : (int32_t)e;  // no parent plan: parents in row order
    if (p < 0 || p >= a.n_parents) {
        p = -1;
        return 0u;
    }
    const int4 *r = reinterpret_cast<const int4 *>(a.child_rows + (int64_t)p * 8);
    const int4 x = r[0], y = r[1];
    const int32_t v[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
    uint32_t b = 0;
#pragma unroll
    for (int c = 0; c < 8; ++c) b |= (uint32_t)(v[c] >= 0 && v[c] < a.n_children) << c;
    return b;
}

__global__ __launch_bounds__(kThreads) void child_count_kernel(ChildArgs a)
{
    __shared__ int s_c[kThreads / 64][8];
    int32_t p;
    const uint32_t bits = child_bits(a, (int64_t)blockIdx.x * kPlanTileRows + threadIdx.x, p);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const uint64_t m = __ballot((bits >> c) & 1u);
        if (lane == 0) s_c[wave][c] = __popcll(m);
    }
    __syncthreads();
    if (threadIdx.x < 8) {
        int t = 0;
        for (int w = 0; w < kThreads / 64; ++w) t += s_c[w][threadIdx.x];
        a.counts[(int64_t)blockIdx.x * 8 + threadIdx.x] = t;
    }
}

// Exclusive scan of 256 per-thread values of 8 children at once (LDS
// Hillis-Steele over [256][8]); returns the thread's exclusive prefixes and
// the totals.
__device__ inline void scan8(int (&v)[8], int (*s)[8], int (&tot)[8])
{
    const int tid = threadIdx.x;
#pragma unroll
    for (int c = 0; c < 8; ++c) s[tid][c] = v[c];
    __syncthreads();
    for (int off = 1; off < kThreads; off <<= 1) {
        int add[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) add[c] = tid >= off ? s[tid - off][c] : 0;
        __syncthreads();
#pragma unroll
        for (int c = 0; c < 8; ++c) s[tid][c] += add[c];
        __syncthreads();
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        tot[c] = s[kThreads - 1][c];
        v[c] = s[tid][c] - v[c];
    }
    __syncthreads();
}

// Per group of 256 parent tiles: counts -> in-group exclusive offsets, and
// the group's totals.
__global__ __launch_bounds__(kThreads) void child_chunk_kernel(ChildArgs a)
{
    __shared__ int s[kThreads][8];
    const int64_t b = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    int v[8], tot[8];
    if (b < a.n_ptiles) {
        const int4 *q = reinterpret_cast<const int4 *>(a.counts + b * 8);
        const int4 x = q[0], y = q[1];
        v[0] = x.x, v[1] = x.y, v[2] = x.z, v[3] = x.w, v[4] = y.x, v[5] = y.y, v[6] = y.z, v[7] = y.w;
    } else {
#pragma unroll
        for (int c = 0; c < 8; ++c) v[c] = 0;
    }
    scan8(v, s, tot);
    if (b < a.n_ptiles) {
        int4 *q = reinterpret_cast<int4 *>(a.counts + b * 8);
        q[0] = make_int4(v[0], v[1], v[2], v[3]);
        q[1] = make_int4(v[4], v[5], v[6], v[7]);
    }
    if (threadIdx.x < 8) a.chunks[(int64_t)blockIdx.x * 8 + threadIdx.x] = tot[threadIdx.x];
}

// One workgroup: the group totals scanned (loops of 256 groups), the
// children's tile ranges and the header (tile_child is the pad pass's).  A parent plan of
// another size or more active children than the list tiles hold flags the
// status; every tile is then empty.
__global__ __launch_bounds__(kThreads) void child_layout_kernel(ChildArgs a)
{
    __shared__ int s[kThreads][8];
    __shared__ int64_t s_base[9];
    int run[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t k0 = 0; k0 < a.n_chunks; k0 += kThreads) {
        const int64_t k = k0 + threadIdx.x;
        int v[8], tot[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) v[c] = k < a.n_chunks ? a.chunks[k * 8 + c] : 0;
        scan8(v, s, tot);
        if (k < a.n_chunks)
#pragma unroll
            for (int c = 0; c < 8; ++c) a.chunks[k * 8 + c] = v[c] + run[c];
#pragma unroll
        for (int c = 0; c < 8; ++c) run[c] += tot[c];
    }
    if (threadIdx.x == 0) {
        int64_t base = 0;
        for (int c = 0; c < 8; ++c) {
            s_base[c] = base;
            base += (run[c] + kPlanTileRows - 1) / kPlanTileRows;
        }
        s_base[8] = base;
        const bool ok = base <= a.n_main && (!a.phdr || (a.phdr->n_q == a.n_parents && a.phdr->K == a.K));
        for (int c = 0; c < 8; ++c) {
            a.child_n[c] = ok ? run[c] : 0;
            a.child_base[c] = ok ? (int32_t)s_base[c] : 0;
        }
        PlanHeader *h = a.hdr;
        h->n_q = a.n_parents;
        h->n_in = a.n_parents;
        h->n_tiles = (int32_t)a.n_tiles;
        h->K = a.K;
        h->brick_shift = -1;
        h->n_overflow = 0;
        for (int j = 0; j < 4; ++j) h->bmin[j] = h->bmax[j] = 0;
        h->n_bricks = 0;
        h->status = ok ? 0u : kPlanStatusChildRows;
        h->grid_mode = kPlanModeChild;
        h->n_unique = ok ? (int32_t)base : 0;  // list tiles in use
        h->n_extras = 0;                       // splits (the split pass sets it)
        h->list_tiles = (int32_t)a.n_main;     // spare tiles from here
        *a.split_n = 0;
    }
}

__global__ __launch_bounds__(kThreads) void child_emit_kernel(ChildArgs a)
{
    __shared__ int s_c[kThreads / 64][8];
    if (a.hdr->status != 0u) return;  // refused by the layout (uniform)
    int32_t p;
    const uint32_t bits = child_bits(a, (int64_t)blockIdx.x * kPlanTileRows + threadIdx.x, p);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t below = (1ull << lane) - 1ull;
    int pos[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const uint64_t m = __ballot((bits >> c) & 1u);
        pos[c] = __popcll(m & below);
        if (lane == 0) s_c[wave][c] = __popcll(m);
    }
    __syncthreads();
    const int64_t chunk = (int64_t)blockIdx.x / kThreads;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        if (!((bits >> c) & 1u)) continue;
        int off = a.chunks[chunk * 8 + c] + a.counts[(int64_t)blockIdx.x * 8 + c] + pos[c];
        for (int w = 0; w < wave; ++w) off += s_c[w][c];
        a.order[(int64_t)a.child_base[c] * kPlanTileRows + off] = p;
    }
}

// Per tile: its child (tile_child; -1 past the list tiles in use, and for
// every tile when the build was refused), and -1 in every order slot no entry
// takes: past a child's entries in its last tile, and every unused tile.
__global__ __launch_bounds__(kThreads) void child_pad_kernel(ChildArgs a)
{
    const int64_t t = blockIdx.x;
    int c = -1;
    if (a.hdr->status == 0u) {
        const int64_t n_used = a.hdr->n_unique;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int64_t hi = k < 7 ? (int64_t)a.child_base[k + 1] : n_used;
            if (t >= a.child_base[k] && t < hi) c = k;
        }
    }
    if (threadIdx.x == 0) a.tile_child[t] = c;
    const int64_t i = t * kPlanTileRows + threadIdx.x;
    bool pad = c < 0;
    if (!pad) pad = i >= (int64_t)a.child_base[c] * kPlanTileRows + a.child_n[c];
    if (pad) a.order[i] = -1;
}

// The two passes over the tile list below run in one workgroup of
// kListThreads threads, kListPer consecutive tiles per thread: a block scan
// per kListThreads * kListPer tiles (4 rounds for config 5's 14,000 tiles).
constexpr int kListThreads = 1024;
constexpr int kListPer = 4;

__device__ inline int list_scan_excl(int x, int *s_wave, int &total)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int inc = x;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(inc, off, 64);
        if (lane >= off) inc += y;
    }
    __syncthreads();
    if (lane == 63) s_wave[wave] = inc;
    __syncthreads();
    int before = 0;
    total = 0;
    for (int w = 0; w < kListThreads / 64; ++w) {
        if (w < wave) before += s_wave[w];
        total += s_wave[w];
    }
    return before + inc - x;
}

// After the first tables: list tiles whose halo overflows, in tile order,
// each paired with the next spare tile while spares last; the spare takes
// the tile's child.
__global__ __launch_bounds__(kListThreads) void child_split_kernel(ChildArgs a)
{
    __shared__ int s_wave[kListThreads / 64];
    if (a.hdr->status != 0u) return;
    const int64_t n_used = a.hdr->n_unique;
    const int64_t n_extra = a.n_tiles - a.n_main;
    int64_t done = 0;
    for (int64_t t0 = 0; t0 < n_used; t0 += kListThreads * kListPer) {
        const int64_t tb = t0 + (int64_t)threadIdx.x * kListPer;
        bool f[kListPer];
        int cnt = 0;
#pragma unroll
        for (int u = 0; u < kListPer; ++u) {
            f[u] = tb + u < n_used && a.tile_u[tb + u] > kPlanHaloMax;
            cnt += f[u];
        }
        int total;
        int64_t j = done + list_scan_excl(cnt, s_wave, total);
#pragma unroll
        for (int u = 0; u < kListPer; ++u) {
            if (!f[u]) continue;
            if (j < n_extra) {
                const int64_t t = tb + u, spare = a.n_main + j;
                a.split[2 * j] = (int32_t)t;
                a.split[2 * j + 1] = (int32_t)spare;
                a.tile_child[spare] = a.tile_child[t];
            }
            ++j;
        }
        done += total;
    }
    if (threadIdx.x == 0) {
        const int64_t ns = done < n_extra ? done : n_extra;
        *a.split_n = (int32_t)(2 * ns);
        a.hdr->n_extras = (int32_t)ns;
    }
}

// One workgroup per split: rows 128..255 of the tile go to its spare (whose
// slots are all -1 from the pad pass).
__global__ __launch_bounds__(kPlanTileRows / 2) void child_move_kernel(ChildArgs a)
{
    const int j = blockIdx.x;
    if (2 * j >= *a.split_n) return;
    const int64_t t = a.split[2 * j], spare = a.split[2 * j + 1];
    const int i = threadIdx.x;
    a.order[spare * kPlanTileRows + i] = a.order[t * kPlanTileRows + kPlanTileRows / 2 + i];
    a.order[t * kPlanTileRows + kPlanTileRows / 2 + i] = -1;
}

// The overflow list rebuilt in tile order (tiles whose halo still overflows
// after the splits, or that found no spare). Only the tiles in use can: the
// list tiles [0, n_unique) and the spares taken, [n_main, n_main + n_extras)
// (none when the build was refused), walked as one index range.
__global__ __launch_bounds__(kListThreads) void child_overflow_kernel(ChildArgs a)
{
    __shared__ int s_wave[kListThreads / 64];
    const int64_t n_used = a.hdr->status == 0u ? a.hdr->n_unique : 0;
    const int64_t n_live = n_used + (a.hdr->status == 0u ? a.hdr->n_extras : 0);
    int64_t done = 0;
    for (int64_t v0 = 0; v0 < n_live; v0 += kListThreads * kListPer) {
        const int64_t vb = v0 + (int64_t)threadIdx.x * kListPer;
        bool f[kListPer];
        int64_t tt[kListPer];
        int cnt = 0;
#pragma unroll
        for (int u = 0; u < kListPer; ++u) {
            const int64_t v = vb + u;
            tt[u] = v < n_used ? v : a.n_main + (v - n_used);
            f[u] = v < n_live && a.tile_child[tt[u]] >= 0 && a.tile_u[tt[u]] > kPlanHaloMax;
            cnt += f[u];
        }
        int total;
        int64_t j = done + list_scan_excl(cnt, s_wave, total);
#pragma unroll
        for (int u = 0; u < kListPer; ++u)
            if (f[u]) a.overflow[j++] = (int32_t)tt[u];
        done += total;
    }
    if (threadIdx.x == 0) a.hdr->n_overflow = (int32_t)done;
}

}  // namespace
}  // namespace sc

using namespace sc;

extern "C" int sc_conv_plan_size(int64_t n_q, int64_t kernel_rows, size_t *bytes)
{
    clear_error();
    if (!bytes) return fail(SC_ERR_NULL, "bytes out-pointer is NULL");
    if (n_q < 0 || n_q > INT32_MAX) return fail(SC_ERR_SHAPE, "conv plan row count must be in [0, i32::MAX]");
    if (kernel_rows < 1 || kernel_rows > 32)
        return fail(SC_ERR_UNSUPPORTED, "conv plan supports kernels of 1..32 offsets");
    *bytes = plan_layout(n_q, kernel_rows).total;
    return SC_OK;
}

namespace {

// Validates a plan call and fills the kernel arguments (the map may be NULL
// for the ordering half).
int plan_args(const sc_conv_config *cfg, const int32_t *d_coords, int64_t n_in, const int32_t *d_map,
              int64_t n_q, void *d_plan, size_t plan_bytes, bool need_coords, bool need_map, PlanArgs &a,
              PlanLayout &L)
{
    int rc = validate_config(cfg);
    if (rc) return rc;
    const int64_t K = cfg->kernel_d * cfg->kernel_h * cfg->kernel_w;
    if (K > 32) return fail(SC_ERR_UNSUPPORTED, "conv plan supports kernels of 1..32 offsets");
    if (n_in < 0 || n_in > INT32_MAX || n_q < 0 || n_q > n_in)
        return fail(SC_ERR_SHAPE, "conv plan needs 0 <= n_q <= n_in <= i32::MAX");
    if (!d_plan) return fail(SC_ERR_NULL, "conv plan buffer is NULL");
    if ((uintptr_t)d_plan % 256 != 0) return fail(SC_ERR_WORKSPACE, "conv plan buffer must be 256-byte aligned");
    L = plan_layout(n_q, K);
    if (plan_bytes < L.total)
        return fail(SC_ERR_WORKSPACE, "conv plan buffer too small: got " + std::to_string(plan_bytes) + " need " +
                                          std::to_string(L.total));
    if (n_q > 0 && need_coords && !d_coords) return fail(SC_ERR_NULL, "conv plan: coords is NULL");
    if (n_q > 0 && need_map && !d_map) return fail(SC_ERR_NULL, "conv plan: map is NULL");
    if ((uintptr_t)d_coords % 16 != 0) return fail(SC_ERR_SHAPE, "coords must be 16-byte aligned");
    if (L.n_tiles > INT32_MAX) return fail(SC_ERR_OVERFLOW, "conv plan tile count overflow");
    if (L.grid_cap / kPlanGridBlock + (n_q + kPlanGridBlock - 1) / kPlanGridBlock > INT32_MAX)
        return fail(SC_ERR_OVERFLOW, "conv plan grid overflow");

    char *b = static_cast<char *>(d_plan);
    a.coords = reinterpret_cast<const int4 *>(d_coords);
    a.map = d_map;

    a.n_q = n_q;
    a.n_in = n_in;
    a.K = (int)K;
    a.hdr = reinterpret_cast<PlanHeader *>(b);
    a.order = reinterpret_cast<int32_t *>(b + L.order);
    a.tile_u = reinterpret_cast<int32_t *>(b + L.tile_u);
    a.overflow = reinterpret_cast<int32_t *>(b + L.overflow);
    a.halo = reinterpret_cast<int32_t *>(b + L.halo);
    a.lmap = reinterpret_cast<uint16_t *>(b + L.lmap);
    a.grid = reinterpret_cast<uint32_t *>(b + L.grid);
    a.gsum = reinterpret_cast<int32_t *>(b + L.gsum);
    a.counts = reinterpret_cast<int32_t *>(b + L.counts);
    a.offsets = reinterpret_cast<int32_t *>(b + L.offsets);
    a.bsum = reinterpret_cast<int32_t *>(b + L.bsum);
    a.n_tiles = L.n_tiles;
    a.brick_cap = L.brick_cap;
    a.n_bsum = L.n_bsum;
    a.grid_cap = L.grid_cap;
    a.tile_list = nullptr;
    a.tile_list_n = nullptr;
    return SC_OK;
}

int launch_plan_order(const PlanArgs &a, const PlanLayout &L, hipStream_t s)
{
    const int64_t n_q = a.n_q;
    if (n_q == 0) {
        plan_init_kernel<<<grid_for(L.n_tiles * kPlanTileRows, kThreads, 1024), kThreads, 0, s>>>(a);
        SC_LAUNCH_CHECK("plan_init_kernel launch");
        return SC_OK;
    }
    const unsigned nbb = grid_for(n_q, kThreads, kBboxBlocks);
    plan_bbox_kernel<<<nbb, kThreads, 0, s>>>(a);
    SC_LAUNCH_CHECK("plan_bbox_kernel launch");
    // The ordering mode (occupancy grid or counting sort) is chosen on the
    // device from the bounding box; every launch below covers both.
    const int64_t grid_blocks = L.grid_cap / kPlanGridBlock;
    plan_prep_kernel<<<grid_for(L.grid_cap > L.brick_cap ? L.grid_cap : L.brick_cap, kThreads, 1024), kThreads, 0,
                       s>>>(a, (int)nbb);
    SC_LAUNCH_CHECK("plan_prep_kernel launch");
    plan_place_kernel<<<grid_for(n_q, kThreads, 8192), kThreads, 0, s>>>(a);
    SC_LAUNCH_CHECK("plan_place_kernel launch");
    // grid mode uses grid_blocks cell blocks + row_blocks duplicate-row blocks
    const int64_t row_blocks = (n_q + kPlanGridBlock - 1) / kPlanGridBlock;
    const int64_t scan_blocks = grid_blocks + row_blocks > L.n_bsum ? grid_blocks + row_blocks : L.n_bsum;
    plan_scan1_kernel<<<(unsigned)scan_blocks, kThreads, 0, s>>>(a);
    SC_LAUNCH_CHECK("plan_scan1_kernel launch");
    plan_scan2_kernel<<<1, kThreads, 0, s>>>(a);
    SC_LAUNCH_CHECK("plan_scan2_kernel launch");
    const unsigned emit_blocks = grid_for(n_q, kThreads, 8192);
    plan_emit_kernel<<<(unsigned)(grid_blocks + row_blocks) > emit_blocks ? (unsigned)(grid_blocks + row_blocks)
                                                                          : emit_blocks,
                       kThreads, 0, s>>>(a);
    SC_LAUNCH_CHECK("plan_emit_kernel launch");
    plan_fix_kernel<<<grid_for(L.brick_cap, kThreads / 64, 512), kThreads, 0, s>>>(a);
    SC_LAUNCH_CHECK("plan_fix_kernel launch");
    return SC_OK;
}

int launch_plan_tables(const PlanArgs &a, const PlanLayout &L, hipStream_t s)
{
    if (a.n_q == 0) return SC_OK;
    plan_tiles_kernel<<<(unsigned)L.n_tiles, kTileThreads, 0, s>>>(a);
    SC_LAUNCH_CHECK("plan_tiles_kernel launch");
    return SC_OK;
}

}  // namespace

extern "C" int sc_conv_plan_build(const sc_conv_config *cfg, const int32_t *d_coords, int64_t n_in,
                                  const int32_t *d_map, int64_t n_q, void *d_plan, size_t plan_bytes,
                                  sc_stream stream)
{
    clear_error();
    PlanArgs a;
    PlanLayout L;
    int rc = plan_args(cfg, d_coords, n_in, d_map, n_q, d_plan, plan_bytes, true, true, a, L);
    if (rc) return rc;
    hipStream_t s = as_stream(stream);
    rc = launch_plan_order(a, L, s);
    if (rc) return rc;
    return launch_plan_tables(a, L, s);
}

extern "C" int sc_conv_plan_order(const sc_conv_config *cfg, const int32_t *d_coords, int64_t n_in, int64_t n_q,
                                  void *d_plan, size_t plan_bytes, sc_stream stream)
{
    clear_error();
    PlanArgs a;
    PlanLayout L;
    int rc = plan_args(cfg, d_coords, n_in, nullptr, n_q, d_plan, plan_bytes, true, false, a, L);
    if (rc) return rc;
    return launch_plan_order(a, L, as_stream(stream));
}

extern "C" int sc_conv_plan_tables(const sc_conv_config *cfg, const int32_t *d_map, int64_t n_in, int64_t n_q,
                                   void *d_plan, size_t plan_bytes, sc_stream stream)
{
    clear_error();
    PlanArgs a;
    PlanLayout L;
    int rc = plan_args(cfg, nullptr, n_in, d_map, n_q, d_plan, plan_bytes, false, true, a, L);
    if (rc) return rc;
    return launch_plan_tables(a, L, as_stream(stream));
}

extern "C" int sc_conv_child_plan_size(int64_t n_parents, int64_t n_children, int64_t kernel_rows, size_t *bytes)
{
    clear_error();
    if (!bytes) return fail(SC_ERR_NULL, "bytes out-pointer is NULL");
    if (n_parents < 0 || n_parents > INT32_MAX)
        return fail(SC_ERR_SHAPE, "child plan parent count must be in [0, i32::MAX]");
    if (n_children < 0 || n_children > 8 * n_parents)
        return fail(SC_ERR_SHAPE, "child plan child count must be in [0, 8 * parents]");
    if (kernel_rows < 1 || kernel_rows > 32)
        return fail(SC_ERR_UNSUPPORTED, "conv plan supports kernels of 1..32 offsets");
    *bytes = child_plan_layout(n_parents, n_children, kernel_rows).total;
    return SC_OK;
}

extern "C" int sc_linear_child_plan_build(int64_t n_parents, const int32_t *d_child_rows, int64_t n_children,
                                          void *d_child_plan, size_t child_plan_bytes, sc_stream stream)
{
    clear_error();
    if (n_parents < 0 || n_parents > INT32_MAX)
        return fail(SC_ERR_SHAPE, "child plan parent count must be in [0, i32::MAX]");
    if (n_children < 0 || n_children > 8 * n_parents)
        return fail(SC_ERR_SHAPE, "child plan child count must be in [0, 8 * parents]");
    if (!d_child_plan || (n_parents > 0 && !d_child_rows)) return fail(SC_ERR_NULL, "linear child plan: NULL pointer");
    if ((uintptr_t)d_child_plan % 256 != 0) return fail(SC_ERR_WORKSPACE, "conv plans must be 256-byte aligned");
    if ((uintptr_t)d_child_rows % 16 != 0) return fail(SC_ERR_SHAPE, "child rows must be 16-byte aligned");
    const ChildPlanLayout CL = child_plan_layout(n_parents, n_children, 1);
    if (child_plan_bytes < CL.total)
        return fail(SC_ERR_WORKSPACE, "child plan buffer too small: got " + std::to_string(child_plan_bytes) +
                                          " need " + std::to_string(CL.total));
    if (CL.n_tiles > INT32_MAX) return fail(SC_ERR_OVERFLOW, "child plan tile count overflow");
    char *b = static_cast<char *>(d_child_plan);
    ChildArgs c;
    c.phdr = nullptr;  // parents in row order: no parent plan
    c.porder = nullptr;
    c.child_rows = d_child_rows;
    c.n_parents = n_parents;
    c.n_children = n_children;
    c.n_ptiles = CL.n_ptiles;
    c.n_chunks = CL.n_chunks;
    c.n_main = CL.n_main;
    c.n_tiles = CL.n_tiles;
    c.K = 1;
    c.hdr = reinterpret_cast<PlanHeader *>(b);
    c.order = reinterpret_cast<int32_t *>(b + CL.order);
    c.tile_child = reinterpret_cast<int32_t *>(b + CL.tile_child);
    c.tile_u = reinterpret_cast<int32_t *>(b + CL.tile_u);
    c.overflow = reinterpret_cast<int32_t *>(b + CL.overflow);
    c.counts = reinterpret_cast<int32_t *>(b + CL.counts);
    c.chunks = reinterpret_cast<int32_t *>(b + CL.chunks);
    c.child_n = reinterpret_cast<int32_t *>(b + CL.child_n);
    c.child_base = reinterpret_cast<int32_t *>(b + CL.child_base);
    c.split = reinterpret_cast<int32_t *>(b + CL.split);
    c.split_n = reinterpret_cast<int32_t *>(b + CL.split_n);
    hipStream_t s = as_stream(stream);
    // the child plan's lists and tile_child, without halo tables: the linear
    // reads each parent's own row
    if (CL.n_ptiles > 0) {
        child_count_kernel<<<(unsigned)CL.n_ptiles, kThreads, 0, s>>>(c);
        SC_LAUNCH_CHECK("child_count_kernel launch");
        child_chunk_kernel<<<(unsigned)CL.n_chunks, kThreads, 0, s>>>(c);
        SC_LAUNCH_CHECK("child_chunk_kernel launch");
    }
    child_layout_kernel<<<1, kThreads, 0, s>>>(c);
    SC_LAUNCH_CHECK("child_layout_kernel launch");
    if (CL.n_ptiles > 0) {
        child_emit_kernel<<<(unsigned)CL.n_ptiles, kThreads, 0, s>>>(c);
        SC_LAUNCH_CHECK("child_emit_kernel launch");
    }
    child_pad_kernel<<<(unsigned)CL.n_tiles, kThreads, 0, s>>>(c);
    SC_LAUNCH_CHECK("child_pad_kernel launch");
    return SC_OK;
}

extern "C" int sc_conv_child_plan_build(const sc_conv_config *cfg, const void *d_parent_plan, const int32_t *d_map,
                                        int64_t n_parents, const int32_t *d_child_rows, int64_t n_children,
                                        void *d_child_plan, size_t child_plan_bytes, sc_stream stream)
{
    clear_error();
    int rc = validate_config(cfg);
    if (rc) return rc;
    const int64_t K = cfg->kernel_d * cfg->kernel_h * cfg->kernel_w;
    if (K > 32) return fail(SC_ERR_UNSUPPORTED, "conv plan supports kernels of 1..32 offsets");
    if (n_parents < 0 || n_parents > INT32_MAX)
        return fail(SC_ERR_SHAPE, "child plan parent count must be in [0, i32::MAX]");
    if (n_children < 0 || n_children > 8 * n_parents)
        return fail(SC_ERR_SHAPE, "child plan child count must be in [0, 8 * parents]");
    if (!d_parent_plan || !d_child_plan || (n_parents > 0 && (!d_map || !d_child_rows)))
        return fail(SC_ERR_NULL, "child plan: NULL pointer");
    if ((uintptr_t)d_parent_plan % 256 != 0 || (uintptr_t)d_child_plan % 256 != 0)
        return fail(SC_ERR_WORKSPACE, "conv plans must be 256-byte aligned");
    if ((uintptr_t)d_child_rows % 16 != 0) return fail(SC_ERR_SHAPE, "child rows must be 16-byte aligned");
    const ChildPlanLayout CL = child_plan_layout(n_parents, n_children, K);
    if (child_plan_bytes < CL.total)
        return fail(SC_ERR_WORKSPACE, "child plan buffer too small: got " + std::to_string(child_plan_bytes) +
                                          " need " + std::to_string(CL.total));
    if (CL.n_tiles > INT32_MAX) return fail(SC_ERR_OVERFLOW, "child plan tile count overflow");
    const PlanLayout PL = plan_layout(n_parents, K);
    const char *pb = static_cast<const char *>(d_parent_plan);
    char *b = static_cast<char *>(d_child_plan);
    ChildArgs c;
    c.phdr = reinterpret_cast<const PlanHeader *>(pb);
    c.porder = reinterpret_cast<const int32_t *>(pb + PL.order);
    c.child_rows = d_child_rows;
    c.n_parents = n_parents;
    c.n_children = n_children;
    c.n_ptiles = CL.n_ptiles;
    c.n_chunks = CL.n_chunks;
    c.n_main = CL.n_main;
    c.n_tiles = CL.n_tiles;
    c.K = (int)K;
    c.hdr = reinterpret_cast<PlanHeader *>(b);
    c.order = reinterpret_cast<int32_t *>(b + CL.order);
    c.tile_child = reinterpret_cast<int32_t *>(b + CL.tile_child);
    c.tile_u = reinterpret_cast<int32_t *>(b + CL.tile_u);
    c.overflow = reinterpret_cast<int32_t *>(b + CL.overflow);
    c.counts = reinterpret_cast<int32_t *>(b + CL.counts);
    c.chunks = reinterpret_cast<int32_t *>(b + CL.chunks);
    c.child_n = reinterpret_cast<int32_t *>(b + CL.child_n);
    c.child_base = reinterpret_cast<int32_t *>(b + CL.child_base);
    c.split = reinterpret_cast<int32_t *>(b + CL.split);
    c.split_n = reinterpret_cast<int32_t *>(b + CL.split_n);
    hipStream_t s = as_stream(stream);
    if (CL.n_ptiles > 0) {
        child_count_kernel<<<(unsigned)CL.n_ptiles, kThreads, 0, s>>>(c);
        SC_LAUNCH_CHECK("child_count_kernel launch");
        child_chunk_kernel<<<(unsigned)CL.n_chunks, kThreads, 0, s>>>(c);
        SC_LAUNCH_CHECK("child_chunk_kernel launch");
    }
    child_layout_kernel<<<1, kThreads, 0, s>>>(c);
    SC_LAUNCH_CHECK("child_layout_kernel launch");
    if (CL.n_ptiles > 0) {
        child_emit_kernel<<<(unsigned)CL.n_ptiles, kThreads, 0, s>>>(c);
        SC_LAUNCH_CHECK("child_emit_kernel launch");
    }
    child_pad_kernel<<<(unsigned)CL.n_tiles, kThreads, 0, s>>>(c);
    SC_LAUNCH_CHECK("child_pad_kernel launch");
    // the halo tables of the child tiles, from the parents' map rows
    PlanArgs a{};
    a.map = d_map;
    a.n_q = n_parents;
    a.n_in = n_parents;
    a.K = (int)K;
    a.hdr = c.hdr;
    a.order = c.order;
    a.tile_u = c.tile_u;
    a.overflow = c.overflow;
    a.halo = reinterpret_cast<int32_t *>(b + CL.halo);
    a.lmap = reinterpret_cast<uint16_t *>(b + CL.lmap);
    a.n_tiles = CL.n_tiles;
    a.tile_list = nullptr;
    a.tile_list_n = nullptr;
    plan_tiles_kernel<<<(unsigned)CL.n_tiles, kTileThreads, 0, s>>>(a);
    SC_LAUNCH_CHECK("plan_tiles_kernel launch (child plan)");
    // overflowing tiles split in two, both rebuilt; the overflow list in tile order
    child_split_kernel<<<1, kListThreads, 0, s>>>(c);
    SC_LAUNCH_CHECK("child_split_kernel launch");
    const int64_t n_extra = CL.n_tiles - CL.n_main;
    child_move_kernel<<<(unsigned)n_extra, kPlanTileRows / 2, 0, s>>>(c);
    SC_LAUNCH_CHECK("child_move_kernel launch");
    a.tile_list = c.split;
    a.tile_list_n = c.split_n;
    plan_tiles_kernel<<<(unsigned)(2 * n_extra), kTileThreads, 0, s>>>(a);
    SC_LAUNCH_CHECK("plan_tiles_kernel launch (child plan splits)");
    child_overflow_kernel<<<1, kListThreads, 0, s>>>(c);
    SC_LAUNCH_CHECK("child_overflow_kernel launch");
    return SC_OK;
}
