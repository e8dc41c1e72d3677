// Voxel hash table + K-offset neighbour-map builder for gfx950.
//
// Replaces the reference's device map builders (crates/burn_flex_gmm/src/
// wgpu/neighbor_kernels.rs K1-K8 and their routing in wgpu/neighbor.rs:9-57,
// 777-936) with one order-independent algorithm:
//
//   1. init   : header (bbox accumulators, status) + table slots := EMPTY
//   2. bbox   : coalesced int4 coord loads, wave64/LDS min-max reduction,
//               one atomic per block and component; negative coords flagged
//   3. insert : key = mixed-radix index of (b,x,y,z) inside the bbox; a
//               32-bit key packs with the row into one 64-bit slot (single
//               atomicCAS, atomicMin on the slot keeps the LOWEST row of
//               duplicates); wider keys use a u64 key array + u32 row array;
//               a bbox beyond 2^64-1 cells uses a row-only table whose slots
//               are compared through the coords themselves
//   4. query  : R rows per block staged in LDS, one (row, k) entry per lane,
//               coalesced map writes; neighbours outside the bbox (including
//               negative ones) are rejected before probing
//
// Linear probing over a power-of-two table with >= 2 slots per row; every
// probe loop is bounded by the table capacity.
//
// When the bbox holds at most 32 cells per row (and the workspace has room),
// the "table" is a dense bbox-indexed grid of rows instead: the slot of a key
// is the key itself, so insertion is one atomicMin on a distinct word and a
// query one load, and the neighbours of nearby voxels share cache lines.
#include <climits>

#include "sc_common.hpp"

namespace sc {
namespace {

constexpr size_t kHeaderBytes = 256;
constexpr uint64_t kEmpty64 = ~0ull;
constexpr uint32_t kStatusNegative = 1u;
constexpr int kMaxStagedRows = 256;
constexpr int kMaxStagedOffsets = 512;

struct alignas(16) NbrHeader {
    int32_t bmin[4];
    int32_t bmax[4];
    uint32_t status;
    uint32_t pad[55];
};
static_assert(sizeof(NbrHeader) == kHeaderBytes, "header size");

inline uint64_t table_capacity(int64_t n)
{
    uint64_t want = (uint64_t)(n > 32 ? n : 32) * 2u;
    uint64_t cap = 64;
    while (cap < want) cap <<= 1;
    return cap;
}

// Dense-grid budget: 32 cells per row (at least 2^16 cells).
inline uint64_t dense_cells_for(int64_t n)
{
    const uint64_t c = (uint64_t)(n > 0 ? n : 0) * 32u;
    return c < (1u << 16) ? (1u << 16) : c;
}

constexpr size_t kPartialBytes = 1024 * 9 * 4;  // bbox partials (kBboxBlocks x 9 ints)

inline size_t workspace_bytes_for(int64_t n)
{
    const size_t hash_bytes = (size_t)table_capacity(n) * 12u;
    const size_t dense_bytes = (size_t)dense_cells_for(n) * 4u;
    return kHeaderBytes + kPartialBytes + (hash_bytes > dense_bytes ? hash_bytes : dense_bytes);
}

// splitmix64 finaliser (Steele, Lea & Flood, OOPSLA 2014).
__device__ inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

struct Plan {
    int mode;  // 0: no table (error), 1: 32-bit keys packed with rows, 2: 64-bit keys,
               // 3: row-only table compared through the coords, 4: dense grid
    uint64_t total;  // bbox cells (valid for modes 1, 2, 4)
    int32_t lo[4];
    int32_t hi[4];
    uint64_t ext[4];
};

__device__ inline Plan make_plan(const NbrHeader *h, uint64_t dense_cells)
{
    Plan p;
    p.mode = 0;
    p.total = 0;
    for (int j = 0; j < 4; ++j) {
        p.lo[j] = h->bmin[j];
        p.hi[j] = h->bmax[j];
        p.ext[j] = (uint64_t)((int64_t)h->bmax[j] - (int64_t)h->bmin[j] + 1);
    }
    if (h->status & kStatusNegative) return p;
    uint64_t total = 1;
    bool ovf = false;
    for (int j = 0; j < 4; ++j) {
        if (total != 0 && p.ext[j] > kEmpty64 / total) ovf = true;
        total *= p.ext[j];
    }
    p.total = total;
    p.mode = ovf ? 3 : (total <= dense_cells ? 4 : (total <= 0xffffffffull ? 1 : 2));
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

__device__ inline uint64_t pack_key(const Plan &p, int32_t b, int32_t x, int32_t y, int32_t z)
{
    uint64_t k = (uint64_t)(b - p.lo[0]);
    k = k * p.ext[1] + (uint64_t)(x - p.lo[1]);
    k = k * p.ext[2] + (uint64_t)(y - p.lo[2]);
    k = k * p.ext[3] + (uint64_t)(z - p.lo[3]);
    return k;
}

__global__ void nm_header_init_kernel(NbrHeader *h)
{
    for (int j = 0; j < 4; ++j) {
        h->bmin[j] = INT_MAX;
        h->bmax[j] = INT_MIN;
    }
    h->status = 0;
}

// Fills the table region the plan uses with all-ones (EMPTY keys, EMPTY rows,
// or -1 grid cells): cap*12 bytes for the hash modes, total*4 for the grid.
__global__ void nm_table_init_kernel(const NbrHeader *h, uint64_t *words, uint64_t cap,
                                     uint64_t dense_cells)
{
    const Plan p = make_plan(h, dense_cells);
    if (p.mode == 0) return;
    const uint64_t n_words = p.mode == 4 ? (p.total + 1) / 2 : cap + cap / 2;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_words; i += stride)
        words[i] = kEmpty64;
}

// Per-block bbox partials (4 min, 4 max, negative flag), no atomics.
constexpr int kBboxBlocks = 1024;

__global__ __launch_bounds__(256) void nm_bbox_partial_kernel(const int4 *__restrict__ coords, int64_t n,
                                                              int32_t *__restrict__ partials)
{
    int mn[4] = {INT_MAX, INT_MAX, INT_MAX, INT_MAX};
    int mx[4] = {INT_MIN, INT_MIN, INT_MIN, INT_MIN};
    int neg = 0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const int4 c = coords[i];
        const int v[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            mn[j] = min(mn[j], v[j]);
            mx[j] = max(mx[j], v[j]);
            neg |= v[j] < 0;
        }
    }
    __shared__ int s_red[4][9];  // per wave: 4 min, 4 max, neg
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        mn[j] = wave_min_i32(mn[j]);
        mx[j] = wave_max_i32(mx[j]);
    }
    neg = wave_max_i32(neg);
    if (lane == 0) {
        for (int j = 0; j < 4; ++j) {
            s_red[wave][j] = mn[j];
            s_red[wave][4 + j] = mx[j];
        }
        s_red[wave][8] = neg;
    }
    __syncthreads();
    if (threadIdx.x < 9) {
        const int j = threadIdx.x;
        const int nw = blockDim.x >> 6;
        int v = s_red[0][j];
        for (int w = 1; w < nw; ++w) v = j < 4 ? min(v, s_red[w][j]) : max(v, s_red[w][j]);
        partials[blockIdx.x * 9 + j] = v;
    }
}

// One block: reduces the partials and writes the header (bbox + status).
__global__ __launch_bounds__(256) void nm_bbox_final_kernel(const int32_t *__restrict__ partials,
                                                            int nblocks, NbrHeader *h)
{
    int mn[4] = {INT_MAX, INT_MAX, INT_MAX, INT_MAX};
    int mx[4] = {INT_MIN, INT_MIN, INT_MIN, INT_MIN};
    int neg = 0;
    for (int b = threadIdx.x; b < nblocks; b += blockDim.x) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            mn[j] = min(mn[j], partials[b * 9 + j]);
            mx[j] = max(mx[j], partials[b * 9 + 4 + j]);
        }
        neg |= partials[b * 9 + 8];
    }
    __shared__ int s_red[4][9];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        mn[j] = wave_min_i32(mn[j]);
        mx[j] = wave_max_i32(mx[j]);
    }
    neg = wave_max_i32(neg);
    if (lane == 0) {
        for (int j = 0; j < 4; ++j) {
            s_red[wave][j] = mn[j];
            s_red[wave][4 + j] = mx[j];
        }
        s_red[wave][8] = neg;
    }
    __syncthreads();
    if (threadIdx.x < 9) {
        const int j = threadIdx.x;
        int v = s_red[0][j];
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) v = j < 4 ? min(v, s_red[w][j]) : max(v, s_red[w][j]);
        if (j < 4)
            h->bmin[j] = v;
        else if (j < 8)
            h->bmax[j - 4] = v;
        else
            h->status = v ? kStatusNegative : 0u;
    }
}

__global__ __launch_bounds__(256) void nm_insert_kernel(const int4 *__restrict__ coords, int64_t n,
                                                        NbrHeader *h, uint64_t *keys, uint32_t *rows,
                                                        uint64_t mask, uint64_t dense_cells)
{
    const Plan p = make_plan(h, dense_cells);
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p.mode == 0) return;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    uint32_t *grid = reinterpret_cast<uint32_t *>(keys);
    for (int64_t r = tid; r < n; r += stride) {
        const int4 c = coords[r];
        if (p.mode == 4) {
            // cells start at 0xffffffff: the unsigned minimum keeps the lowest row
            atomicMin(&grid[pack_key(p, c.x, c.y, c.z, c.w)], (uint32_t)r);
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

// Dense-grid query: a row's neighbour at offset k is cell base[r] + delta[k]
// (32-bit mixed-radix strides), valid when the neighbour lies in the bbox.
// Entries (r, k) are walked incrementally (no division), four loads in
// flight per lane before their stores.
__device__ inline void query_dense(const int4 *s_coord, const int *s_off, const uint32_t *s_base,
                                   const int *s_delta, int nrows, int K, const Plan &p,
                                   const uint32_t *__restrict__ grid, int32_t *__restrict__ out)
{
    const int total = nrows * K;
    const int step_r = (int)blockDim.x / K, step_k = (int)blockDim.x % K;
    int r = (int)threadIdx.x / K, k = (int)threadIdx.x % K;
    for (int e0 = threadIdx.x; e0 < total; e0 += 4 * (int)blockDim.x) {
        int32_t v[4];
        int idx[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = e0 + u * (int)blockDim.x;
            idx[u] = e;
            v[u] = SC_INVALID_NEIGHBOR_ROW;
            if (e < total) {
                const int4 c = s_coord[r];
                const int nx = c.y + s_off[3 * k], ny = c.z + s_off[3 * k + 1], nz = c.w + s_off[3 * k + 2];
                if (nx >= p.lo[1] && nx <= p.hi[1] && ny >= p.lo[2] && ny <= p.hi[2] && nz >= p.lo[3] &&
                    nz <= p.hi[3])
                    v[u] = (int32_t)grid[s_base[r] + (uint32_t)s_delta[k]];
            }
            r += step_r;
            k += step_k;
            if (k >= K) {
                k -= K;
                ++r;
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (idx[u] < total) out[idx[u]] = v[u];
    }
}

__global__ __launch_bounds__(256) void nm_query_kernel(const int4 *__restrict__ coords,
                                                       int64_t q_rows, KernelShape ks,
                                                       int rows_per_block,
                                                       const NbrHeader *__restrict__ h,
                                                       const uint64_t *__restrict__ keys,
                                                       const uint32_t *__restrict__ rows,
                                                       uint64_t mask, uint64_t dense_cells,
                                                       int32_t *__restrict__ map)
{
    __shared__ int4 s_coord[kMaxStagedRows];
    __shared__ uint32_t s_base[kMaxStagedRows];
    __shared__ int s_off[kMaxStagedOffsets * 3];
    __shared__ int s_delta[kMaxStagedOffsets];
    const int64_t row0 = (int64_t)blockIdx.x * rows_per_block;
    const int nrows = (int)min<int64_t>(rows_per_block, q_rows - row0);
    const Plan p = make_plan(h, dense_cells);
    const bool staged = ks.K <= kMaxStagedOffsets;
    for (int i = threadIdx.x; i < nrows; i += blockDim.x) {
        const int4 c = coords[row0 + i];
        s_coord[i] = c;
        if (p.mode == 4) s_base[i] = (uint32_t)pack_key(p, c.x, c.y, c.z, c.w);
    }
    if (staged)
        for (int k = threadIdx.x; k < ks.K; k += blockDim.x) {
            offset_of(ks, k, &s_off[3 * k]);
            // 32-bit cell delta of the offset (wraps; only used inside the bbox)
            s_delta[k] = (int)((uint32_t)s_off[3 * k] * (uint32_t)(p.ext[2] * p.ext[3]) +
                               (uint32_t)s_off[3 * k + 1] * (uint32_t)p.ext[3] + (uint32_t)s_off[3 * k + 2]);
        }
    __syncthreads();
    int32_t *out = map + row0 * ks.K;
    if (p.mode == 4 && staged) {
        query_dense(s_coord, s_off, s_base, s_delta, nrows, ks.K, p,
                    reinterpret_cast<const uint32_t *>(keys), out);
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
        if (inside && p.mode == 4) {
            found = (int32_t)grid[pack_key(p, c.x, (int32_t)nx, (int32_t)ny, (int32_t)nz)];
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
    // Workspace: [header 256 B][bbox partials][table or grid].
    NbrHeader *h = (NbrHeader *)d_workspace;
    int32_t *partials = (int32_t *)((char *)d_workspace + kHeaderBytes);
    const uint64_t cap = table_capacity(n_rows);
    uint64_t *keys = (uint64_t *)((char *)d_workspace + kHeaderBytes + kPartialBytes);
    uint32_t *rows = (uint32_t *)(keys + cap);
    // Dense grid when the bbox fits the workspace's grid budget (decided on the
    // device from the bbox; the budget never exceeds 32 cells per row).
    uint64_t dense_cells = (workspace_bytes - kHeaderBytes - kPartialBytes) / 4u;
    if (dense_cells > dense_cells_for(n_rows)) dense_cells = dense_cells_for(n_rows);
    dense_cells &= ~1ull;  // even: the 8-byte fill of an odd cell count stays inside
    if (dense_cells > 0xffffffffull) dense_cells = 0xfffffffeull;  // 32-bit grid keys
    if (n_rows == 0) {
        nm_header_init_kernel<<<1, 1, 0, s>>>(h);
        SC_LAUNCH_CHECK("nm_header_init_kernel launch");
        return SC_OK;
    }
    const int4 *c4 = (const int4 *)d_coords;
    const unsigned bb = grid_for(n_rows, 256, kBboxBlocks);
    nm_bbox_partial_kernel<<<bb, 256, 0, s>>>(c4, n_rows, partials);
    SC_LAUNCH_CHECK("nm_bbox_partial_kernel launch");
    nm_bbox_final_kernel<<<1, 256, 0, s>>>(partials, (int)bb, h);
    SC_LAUNCH_CHECK("nm_bbox_final_kernel launch");
    nm_table_init_kernel<<<4096, 256, 0, s>>>(h, keys, cap, dense_cells);
    SC_LAUNCH_CHECK("nm_table_init_kernel launch");
    nm_insert_kernel<<<grid_for(n_rows, 256, 65536), 256, 0, s>>>(c4, n_rows, h, keys, rows, cap - 1,
                                                                  dense_cells);
    SC_LAUNCH_CHECK("nm_insert_kernel launch");
    if (query_rows == 0) return SC_OK;
    const KernelShape ks = kernel_shape(cfg);
    int rpb = (int)(2048 / K);
    if (rpb < 1) rpb = 1;
    if (rpb > kMaxStagedRows) rpb = kMaxStagedRows;
    const int64_t blocks = (query_rows + rpb - 1) / rpb;
    if (blocks > INT32_MAX) return fail(SC_ERR_OVERFLOW, "neighbor map grid overflow");
    nm_query_kernel<<<(unsigned)blocks, 256, 0, s>>>(c4, query_rows, ks, rpb, h, keys, rows, cap - 1,
                                                     dense_cells, d_map);
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
