// Conv plan: the row order and per-tile halo tables that the halo-staged
// submanifold conv (conv_halo_kernel) reads.  Built on the device from the
// coords and the neighbour map by sc_conv_plan_build (sc_plan.hip); shared by
// every conv that uses the same map.
//
//   order   [n_tiles * 256] i32   tile row p of tile t computes query row
//                                 order[t*256 + p] (-1 = padding)
//   tile_u  [n_tiles]       i32   number of distinct input rows (the halo)
//                                 the tile's neighbours touch
//   overflow[n_tiles]       i32   tiles whose halo exceeds kPlanHaloMax
//                                 (first header.n_overflow entries)
//   halo    [n_tiles][kPlanHaloMax] i32  input row of local index u, increasing
//   lmap    [n_tiles][K][256] u16  local index of neighbour (p, k), or
//                                 kPlanAbsent
//   grid    [grid_cap] u32        row of each cell of the coords' bounding
//                                 box, cells in brick-major order (8^3
//                                 bricks, lexicographic inside a brick)
//   gsum    [grid_cap / 2048] i32 occupied cells per compaction block
//   brick counts / offsets / block sums: scratch of the counting-sort
//                                 fallback (bounding box too large for the
//                                 grid); counts also hold the rows of
//                                 duplicated coords in grid mode
#pragma once

#include <cstddef>
#include <cstdint>

namespace sc {

constexpr int kPlanTileRows = 256;
// Halo rows of one tile held in LDS at 64 bytes each (one 32-channel bf16
// slice) plus a 4-byte source offset: 960 x 68 B = 64 KB, so that two
// workgroups fit a CU's 160 KB.
constexpr int kPlanHaloMax = 960;
constexpr uint16_t kPlanAbsent = 0xFFFFu;
constexpr int kPlanScanBlock = 1024;  // entries per block of the brick-count scan
constexpr int kPlanGridBlock = 2048;  // grid cells per compaction block
constexpr int kPlanGridPerRow = 16;   // grid budget: cells per query row

// PlanHeader::status bits.  The build clears them; the planned conv sets
// them (and writes nothing) when the plan or the packed weights it is given
// were built for another shape; sc_conv_plan_check reads them back.
constexpr uint32_t kPlanStatusMapMismatch = 1u;     // plan's n_q / n_in / K differ from the call's
constexpr uint32_t kPlanStatusWeightMismatch = 2u;  // packed weights packed for another config
constexpr uint32_t kPlanStatusChildRows = 4u;       // child plan: parent plan of another size, or more
                                                    // active children than the call's child count

struct alignas(16) PlanHeader {
    int64_t n_q;
    int64_t n_in;
    int32_t n_tiles;
    int32_t K;
    int32_t brick_shift;  // log2 of the brick edge used for the row order
    int32_t n_overflow;   // tiles listed in `overflow`
    int32_t bmin[4];
    int32_t bmax[4];
    uint64_t n_bricks;
    uint32_t status;
    int32_t grid_mode;  // 1: occupancy-grid order, 0: counting-sort fallback,
                        // 2: the rows' own order (octree order of >= 3 levels),
                        // 3: occupancy-bitmap order (sorted, unique rows),
                        // 4: a child plan (tiles grouped by C2S child index)
    int32_t n_unique;   // grid mode: occupied cells (distinct coords); child plan: list tiles in use
    int32_t n_extras;   // grid mode: rows of duplicated coords; child plan: splits
    int32_t list_tiles; // child plan: list tiles laid out (the first spare tile); 0 otherwise
    uint32_t pad[41];
};
static_assert(sizeof(PlanHeader) == 256, "plan header size");

struct PlanLayout {
    int64_t n_tiles;
    int64_t brick_cap;  // brick-count entries (multiple of kPlanScanBlock)
    int64_t n_bsum;     // scan block sums
    int64_t grid_cap;   // grid cells (multiple of kPlanGridBlock)
    size_t order, tile_u, overflow, halo, lmap, grid, gsum, counts, offsets, bsum, total;
};

inline size_t plan_align(size_t x) { return (x + 255) & ~(size_t)255; }

inline PlanLayout plan_layout(int64_t n_q, int64_t K)
{
    PlanLayout L;
    L.n_tiles = (n_q + kPlanTileRows - 1) / kPlanTileRows;
    int64_t cap = 2 * n_q;
    if (cap < 4096) cap = 4096;
    L.brick_cap = (cap + kPlanScanBlock - 1) / kPlanScanBlock * kPlanScanBlock;
    L.n_bsum = L.brick_cap / kPlanScanBlock;
    int64_t gcap = kPlanGridPerRow * n_q;
    if (gcap < (1 << 20)) gcap = 1 << 20;
    L.grid_cap = (gcap + kPlanGridBlock - 1) / kPlanGridBlock * kPlanGridBlock;
    size_t o = plan_align(sizeof(PlanHeader));
    L.order = o;
    o = plan_align(o + (size_t)L.n_tiles * kPlanTileRows * 4);
    L.tile_u = o;
    o = plan_align(o + (size_t)L.n_tiles * 4);
    L.overflow = o;
    o = plan_align(o + (size_t)L.n_tiles * 4);
    L.halo = o;
    o = plan_align(o + (size_t)L.n_tiles * kPlanHaloMax * 4);
    L.lmap = o;
    o = plan_align(o + (size_t)L.n_tiles * (size_t)K * kPlanTileRows * 2);
    L.grid = o;
    o = plan_align(o + (size_t)L.grid_cap * 4);
    L.gsum = o;
    o = plan_align(o + (size_t)(L.grid_cap / kPlanGridBlock) * 4);
    L.counts = o;
    o = plan_align(o + (size_t)L.brick_cap * 4);
    L.offsets = o;
    o = plan_align(o + (size_t)L.brick_cap * 4);
    L.bsum = o;
    o = plan_align(o + (size_t)L.n_bsum * 4);
    L.total = o;
    return L;
}

// Device view of a built plan (tile_child: a child plan's per-tile child
// index, NULL for a plan of the query rows themselves).
struct PlanView {
    const PlanHeader *hdr;
    const int32_t *order;
    const int32_t *tile_u;
    const int32_t *overflow;
    const int32_t *halo;
    const uint16_t *lmap;
    const int32_t *tile_child;
};

inline PlanView plan_view(const void *plan, const PlanLayout &L)
{
    const char *b = static_cast<const char *>(plan);
    PlanView v;
    v.hdr = reinterpret_cast<const PlanHeader *>(b);
    v.order = reinterpret_cast<const int32_t *>(b + L.order);
    v.tile_u = reinterpret_cast<const int32_t *>(b + L.tile_u);
    v.overflow = reinterpret_cast<const int32_t *>(b + L.overflow);
    v.halo = reinterpret_cast<const int32_t *>(b + L.halo);
    v.lmap = reinterpret_cast<const uint16_t *>(b + L.lmap);
    v.tile_child = nullptr;
    return v;
}

// Child plan (C2S conv1 over the active children only).  For each child
// index c, the parents whose child c is active, in the parent plan's order,
// in 256-row tiles of their own; tile t computes child tile_child[t]'s
// channel block for its parents.  Same tables as a plan (order holds parent
// rows), plus tile_child and the build's scratch.  The first n_main tiles
// take the children's lists (every list but its last tile fills whole
// tiles, so ceil(A / 256) + 8 suffice for A active children); a tile whose
// halo overflows is then split, its second 128 rows moved to one of the
// n_extra spare tiles, so both halves take the halo-staged kernel.  The
// header's n_unique holds the tiles the lists use, n_extras the splits.
constexpr int32_t kPlanModeChild = 4;

struct ChildPlanLayout {
    int64_t n_main, n_extra, n_tiles;  // list tiles, spare tiles for splits, all
    int64_t n_ptiles;                  // tiles of the parent plan (compaction blocks)
    int64_t n_chunks;                  // groups of 256 parent tiles (the scan's first level)
    size_t order, tile_u, overflow, halo, lmap, tile_child, counts, chunks, child_n, child_base, split, split_n,
        total;
};

inline ChildPlanLayout child_plan_layout(int64_t n_parents, int64_t n_children, int64_t K)
{
    ChildPlanLayout L;
    L.n_main = (n_children + kPlanTileRows - 1) / kPlanTileRows + 8;
    L.n_extra = L.n_main / 8 + 16;  // splits measured at 3-5 % of the list tiles
    L.n_tiles = L.n_main + L.n_extra;
    L.n_ptiles = (n_parents + kPlanTileRows - 1) / kPlanTileRows;
    L.n_chunks = (L.n_ptiles + 255) / 256;
    size_t o = plan_align(sizeof(PlanHeader));
    L.order = o;
    o = plan_align(o + (size_t)L.n_tiles * kPlanTileRows * 4);
    L.tile_u = o;
    o = plan_align(o + (size_t)L.n_tiles * 4);
    L.overflow = o;
    o = plan_align(o + (size_t)L.n_tiles * 4);
    L.halo = o;
    o = plan_align(o + (size_t)L.n_tiles * kPlanHaloMax * 4);
    L.lmap = o;
    o = plan_align(o + (size_t)L.n_tiles * (size_t)K * kPlanTileRows * 2);
    L.tile_child = o;
    o = plan_align(o + (size_t)L.n_tiles * 4);
    L.counts = o;
    o = plan_align(o + (size_t)L.n_ptiles * 8 * 4);
    L.chunks = o;
    o = plan_align(o + (size_t)L.n_chunks * 8 * 4);
    L.child_n = o;
    o = plan_align(o + 8 * 4);
    L.child_base = o;
    o = plan_align(o + 8 * 4);
    L.split = o;
    o = plan_align(o + (size_t)L.n_extra * 2 * 4);
    L.split_n = o;
    o = plan_align(o + 4);
    L.total = o;
    return L;
}

inline PlanView child_plan_view(const void *plan, const ChildPlanLayout &L)
{
    const char *b = static_cast<const char *>(plan);
    PlanView v;
    v.hdr = reinterpret_cast<const PlanHeader *>(b);
    v.order = reinterpret_cast<const int32_t *>(b + L.order);
    v.tile_u = reinterpret_cast<const int32_t *>(b + L.tile_u);
    v.overflow = reinterpret_cast<const int32_t *>(b + L.overflow);
    v.halo = reinterpret_cast<const int32_t *>(b + L.halo);
    v.lmap = reinterpret_cast<const uint16_t *>(b + L.lmap);
    v.tile_child = reinterpret_cast<const int32_t *>(b + L.tile_child);
    return v;
}

}  // namespace sc
