// C2S subdivision: active-child compaction and child coordinate expansion.
//
// Replaces subdivision_active_indices_wgpu (argwhere of (logits - thr) > 0
// on [P,8]) and expand_subdivision_coords_and_linear_indices_wgpu
// (sparse_decoder_wgpu_ops.rs:885-1054) with a two-launch stream compaction.
// A block takes `rounds` rounds of 256 consecutive parents (rounds chosen so
// that there are at most kMaxBlocks blocks):
//   count : per block, the popcount of each parent's 8-bit child mask,
//           summed
//   emit  : the block's output offset = the counts of the blocks before it
//           (at most kMaxBlocks values, read by the whole block); per
//           round, a block scan of the parents' child counts, child_rows per
//           parent, then the round's children written one per thread in
//           output order (the thread finds its parent by binary search of
//           the round's prefix), so consecutive lanes write consecutive
//           rows -> parent-major, child-ascending output, identical to
//           argwhere's row-major order.  The last block writes the count.
#include "sc_common.hpp"

#include <mutex>

namespace sc {
namespace {

constexpr int kThreads = 256;               // parents per round
constexpr int64_t kMaxBlocks = 4096;         // blocks while rounds stay under kMaxRounds
constexpr int64_t kMaxRounds = 64;

struct Thresholds {
    float t[8];
};

__device__ inline unsigned child_mask(const float *logits, const uint8_t *mask, const Thresholds &th,
                                      int64_t p)
{
    unsigned m = 0;
    if (mask) {
        const uint2 v = *reinterpret_cast<const uint2 *>(mask + p * 8);
        const uint32_t w[2] = {v.x, v.y};
#pragma unroll
        for (int c = 0; c < 8; ++c) m |= (((w[c >> 2] >> (8 * (c & 3))) & 0xffu) != 0) << c;
    } else {
        const float4 *q = reinterpret_cast<const float4 *>(logits + p * 8);
        const float4 a = q[0], b = q[1];
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        // logits_to_mask compares logit > threshold (sparse_decoder_wgpu_ops.rs:1783);
        // the device path's (logit - thr) > 0 is the same test for finite values.
#pragma unroll
        for (int c = 0; c < 8; ++c) m |= (unsigned)(v[c] > th.t[c]) << c;
    }
    return m;
}

__device__ inline int block_exclusive_scan(int x, int *s_wave, int &total)
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

__global__ __launch_bounds__(kThreads) void subdiv_count_kernel(const float *logits, const uint8_t *mask,
                                                                Thresholds th, int64_t P, int rounds,
                                                                int32_t *block_counts)
{
    __shared__ int s_wave[kThreads / 64];
    const int64_t base = (int64_t)blockIdx.x * kThreads * rounds + threadIdx.x;
    int cnt = 0;
    for (int r = 0; r < rounds; ++r) {
        const int64_t p = base + (int64_t)r * kThreads;
        if (p < P) cnt += __popc(child_mask(logits, mask, th, p));
    }
    int total;
    block_exclusive_scan(cnt, s_wave, total);
    if (threadIdx.x == 0) block_counts[blockIdx.x] = total;
}

__global__ __launch_bounds__(kThreads) void subdiv_emit_kernel(const float *logits, const uint8_t *mask,
                                                               Thresholds th, int64_t P, int rounds,
                                                               const int4 *__restrict__ parent_coords,
                                                               const int32_t *block_counts,
                                                               int4 *child_coords, int32_t *linear_idx,
                                                               int2 *pairs, int32_t *child_rows,
                                                               int64_t *count)
{
    __shared__ int s_wave[kThreads / 64];
    __shared__ int s_pre[kThreads];
    __shared__ uint8_t s_m[kThreads];
    __shared__ int4 s_pc[kThreads];
    __shared__ int64_t s_sum[kThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // the block's first output row: the counts of the blocks before it
    int64_t part = 0;
    for (int64_t i = tid; i < (int64_t)blockIdx.x; i += kThreads) part += block_counts[i];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off, 64);
    if (lane == 0) s_sum[wave] = part;
    __syncthreads();
    int64_t out = 0;
    for (int w = 0; w < kThreads / 64; ++w) out += s_sum[w];
    const int64_t base = (int64_t)blockIdx.x * kThreads * rounds;
    for (int r = 0; r < rounds; ++r) {
        const int64_t p0 = base + (int64_t)r * kThreads;
        const int64_t p = p0 + tid;
        const unsigned m = p < P ? child_mask(logits, mask, th, p) : 0u;
        // the round's parent coords, fetched with the masks (the emit loop
        // then reads them from LDS, not through a dependent global load)
        s_pc[tid] = p < P ? parent_coords[p] : make_int4(0, 0, 0, 0);
        int total;
        const int ex = block_exclusive_scan(__popc(m), s_wave, total);
        if (child_rows && p < P) {
            // the inverse of linear_idx: child row of (parent, c), -1 if inactive
            int32_t cr[8];
            int32_t o = (int32_t)(out + ex);
#pragma unroll
            for (int c = 0; c < 8; ++c) cr[c] = (m >> c) & 1u ? o++ : -1;
            int4 *dst = reinterpret_cast<int4 *>(child_rows + p * 8);
            dst[0] = make_int4(cr[0], cr[1], cr[2], cr[3]);
            dst[1] = make_int4(cr[4], cr[5], cr[6], cr[7]);
        }
        s_pre[tid] = ex;
        s_m[tid] = (uint8_t)m;
        __syncthreads();
        for (int j = tid; j < total; j += kThreads) {
            // the last parent of the round whose prefix is <= j (parents with
            // no children share the next one's prefix, so it is the owner)
            int lo = 0, hi = kThreads - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (s_pre[mid] <= j) lo = mid;
                else hi = mid - 1;
            }
            const unsigned pm = s_m[lo];
            int k = j - s_pre[lo], c = 0;
            for (; c < 8; ++c)
                if ((pm >> c) & 1u) {
                    if (k == 0) break;
                    --k;
                }
            const int64_t pp = p0 + lo, row = out + j;
            const int4 pc = s_pc[lo];
            child_coords[row] = make_int4(pc.x, 2 * pc.y + (c & 1), 2 * pc.z + ((c >> 1) & 1),
                                          2 * pc.w + ((c >> 2) & 1));
            linear_idx[row] = (int32_t)(pp * 8 + c);
            if (pairs) pairs[row] = make_int2((int32_t)pp, c);
        }
        out += total;
        __syncthreads();  // s_pre / s_m / s_pc are rewritten by the next round
    }
    if (blockIdx.x == gridDim.x - 1 && tid == 0) *count = out;
}

__global__ void write_zero_count(int64_t *count) { *count = 0; }

inline int rounds_for(int64_t P)
{
    const int64_t r = (P + kThreads * kMaxBlocks - 1) / (kThreads * kMaxBlocks);
    return (int)(r < 1 ? 1 : (r > kMaxRounds ? kMaxRounds : r));
}
inline int64_t n_blocks(int64_t P)
{
    const int64_t per = (int64_t)kThreads * rounds_for(P);
    return (P + per - 1) / per;
}

// Bytes of block counts for P parents.
inline size_t workspace_bytes_for(int64_t P) { return (size_t)(n_blocks(P) + 4) * sizeof(int32_t); }

// Argument checks shared by both entry points (the workspace is checked by
// the caller).
int check_args(const float *d_logits, const uint8_t *d_mask, const float *thresholds,
               const int32_t *d_parent_coords, int64_t parent_rows, int32_t *d_child_coords,
               int32_t *d_linear_idx, int32_t *d_pairs, int64_t *d_count)
{
    if (parent_rows < 0 || parent_rows > INT32_MAX / 8)
        return fail(SC_ERR_SHAPE, "subdivision parent rows out of range");
    if (!d_count) return fail(SC_ERR_NULL, "subdivision count pointer is NULL");
    if (parent_rows == 0) return SC_OK;
    if ((d_logits == nullptr) == (d_mask == nullptr))
        return fail(SC_ERR_NULL, "subdivision needs exactly one of logits or mask");
    if (d_logits && !thresholds) return fail(SC_ERR_NULL, "subdivision thresholds are NULL");
    if (!d_parent_coords || !d_child_coords || !d_linear_idx)
        return fail(SC_ERR_NULL, "subdivision: NULL pointer");
    const uintptr_t al = (uintptr_t)d_parent_coords | (uintptr_t)d_child_coords |
                         (uintptr_t)(d_logits ? (const void *)d_logits : (const void *)d_mask);
    if (al % 16 != 0 || (d_pairs && (uintptr_t)d_pairs % 8 != 0))
        return fail(SC_ERR_SHAPE, "subdivision buffers must be 16-byte aligned");
    return SC_OK;
}

// The two launches over a workspace of workspace_bytes_for(parent_rows)
// bytes (the caller's, or the library's static scratch).  count writes every
// block total before emit reads them, so nothing in the workspace needs to
// start at zero.
int launch_subdivision(const float *d_logits, const uint8_t *d_mask, const float *thresholds,
                       const int32_t *d_parent_coords, int64_t parent_rows, int32_t *d_child_coords,
                       int32_t *d_linear_idx, int32_t *d_pairs, int32_t *d_child_rows, int64_t *d_count,
                       int32_t *ws, hipStream_t s)
{
    if (parent_rows == 0) {
        write_zero_count<<<1, 1, 0, s>>>(d_count);
        SC_LAUNCH_CHECK("write_zero_count launch");
        return SC_OK;
    }
    Thresholds th;
    for (int c = 0; c < 8; ++c) th.t[c] = thresholds ? thresholds[c] : 0.f;
    const int rounds = rounds_for(parent_rows);
    const int64_t nb = n_blocks(parent_rows);
    int32_t *counts = ws;
    subdiv_count_kernel<<<(unsigned)nb, kThreads, 0, s>>>(d_logits, d_mask, th, parent_rows, rounds, counts);
    SC_LAUNCH_CHECK("subdiv_count_kernel launch");
    subdiv_emit_kernel<<<(unsigned)nb, kThreads, 0, s>>>(d_logits, d_mask, th, parent_rows, rounds,
                                                         (const int4 *)d_parent_coords, counts,
                                                         (int4 *)d_child_coords, d_linear_idx,
                                                         (int2 *)d_pairs, d_child_rows, d_count);
    SC_LAUNCH_CHECK("subdiv_emit_kernel launch");
    return SC_OK;
}

// ------------------------------------------------------ static scratch
// The workspace of sc_subdivision_build_static: block counts for up to
// kStaticMaxParents parents (4,096 blocks, 16 KiB + 16 B), one copy per GPU,
// held until the process ends.  In host code `scratch` names a host-side stand-in,
// never the device array: every host use goes through the per-device
// address from hipGetSymbolAddress (static_scratch_for).
constexpr int64_t kStaticMaxParents = (int64_t)1 << 26;
constexpr int64_t kStaticMaxBlocks = kStaticMaxParents / (kThreads * kMaxRounds);
static __device__ __align__(256) int32_t scratch[kStaticMaxBlocks + 4];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
int32_t *g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device that stream s belongs to (the
// current device for the NULL stream), looked up once per device with that
// device current.
int static_scratch_for(hipStream_t s, int32_t **out)
{
    int dev = 0;
    if (s)
        SC_HIP_CHECK(hipStreamGetDevice(s, &dev), "hipStreamGetDevice");
    else
        SC_HIP_CHECK(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(SC_ERR_UNSUPPORTED, "device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        int cur = 0;
        SC_HIP_CHECK(hipGetDevice(&cur), "hipGetDevice");
        if (cur != dev) SC_HIP_CHECK(hipSetDevice(dev), "hipSetDevice");
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) SC_HIP_CHECK(hipSetDevice(cur), "hipSetDevice");
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p || (uintptr_t)p % 256 != 0) return fail(SC_ERR_HIP, "static subdivision scratch is misaligned");
        g_scratch_ptr[dev] = static_cast<int32_t *>(p);
    }
    *out = g_scratch_ptr[dev];
    return SC_OK;
}

}  // namespace
}  // namespace sc

using namespace sc;

extern "C" {

int sc_subdivision_workspace_size(int64_t parent_rows, size_t *bytes)
{
    clear_error();
    if (!bytes) return fail(SC_ERR_NULL, "bytes out-pointer is NULL");
    if (parent_rows < 0 || parent_rows > INT32_MAX / 8)
        return fail(SC_ERR_SHAPE, "subdivision parent rows out of range");
    *bytes = workspace_bytes_for(parent_rows);
    return SC_OK;
}

int sc_subdivision_build(const float *d_logits, const uint8_t *d_mask, const float *thresholds,
                         const int32_t *d_parent_coords, int64_t parent_rows,
                         int32_t *d_child_coords, int32_t *d_linear_idx, int32_t *d_pairs,
                         int64_t *d_count, void *d_workspace, size_t workspace_bytes,
                         sc_stream stream)
{
    clear_error();
    int rc = check_args(d_logits, d_mask, thresholds, d_parent_coords, parent_rows, d_child_coords, d_linear_idx,
                        d_pairs, d_count);
    if (rc) return rc;
    if (parent_rows > 0) {
        if (!d_workspace) return fail(SC_ERR_NULL, "subdivision: NULL pointer");
        if ((uintptr_t)d_workspace % 8 != 0) return fail(SC_ERR_SHAPE, "subdivision buffers must be 16-byte aligned");
        if (workspace_bytes < workspace_bytes_for(parent_rows))
            return fail(SC_ERR_WORKSPACE, "subdivision workspace too small");
    }
    return launch_subdivision(d_logits, d_mask, thresholds, d_parent_coords, parent_rows, d_child_coords,
                              d_linear_idx, d_pairs, nullptr, d_count, static_cast<int32_t *>(d_workspace),
                              as_stream(stream));
}

int sc_subdivision_build_indexed(const float *d_logits, const uint8_t *d_mask, const float *thresholds,
                                 const int32_t *d_parent_coords, int64_t parent_rows,
                                 int32_t *d_child_coords, int32_t *d_linear_idx, int32_t *d_pairs,
                                 int32_t *d_child_rows, int64_t *d_count, void *d_workspace,
                                 size_t workspace_bytes, sc_stream stream)
{
    clear_error();
    int rc = check_args(d_logits, d_mask, thresholds, d_parent_coords, parent_rows, d_child_coords, d_linear_idx,
                        d_pairs, d_count);
    if (rc) return rc;
    if (parent_rows > 0) {
        if (!d_workspace || !d_child_rows) return fail(SC_ERR_NULL, "subdivision: NULL pointer");
        if ((uintptr_t)d_workspace % 8 != 0 || (uintptr_t)d_child_rows % 16 != 0)
            return fail(SC_ERR_SHAPE, "subdivision buffers must be 16-byte aligned");
        if (workspace_bytes < workspace_bytes_for(parent_rows))
            return fail(SC_ERR_WORKSPACE, "subdivision workspace too small");
    }
    return launch_subdivision(d_logits, d_mask, thresholds, d_parent_coords, parent_rows, d_child_coords,
                              d_linear_idx, d_pairs, d_child_rows, d_count, static_cast<int32_t *>(d_workspace),
                              as_stream(stream));
}

int sc_subdivision_build_static(const float *d_logits, const uint8_t *d_mask, const float *thresholds,
                                const int32_t *d_parent_coords, int64_t parent_rows,
                                int32_t *d_child_coords, int32_t *d_linear_idx, int32_t *d_pairs,
                                int64_t *d_count, sc_stream stream)
{
    clear_error();
    int rc = check_args(d_logits, d_mask, thresholds, d_parent_coords, parent_rows, d_child_coords, d_linear_idx,
                        d_pairs, d_count);
    if (rc) return rc;
    if (parent_rows > kStaticMaxParents)
        return fail(SC_ERR_WORKSPACE, "sc_subdivision_build_static takes at most " +
                                          std::to_string(kStaticMaxParents) + " parent rows, got " +
                                          std::to_string(parent_rows) + " (use sc_subdivision_build)");
    hipStream_t s = as_stream(stream);
    int32_t *ws = nullptr;
    if (parent_rows > 0) {
        rc = static_scratch_for(s, &ws);
        if (rc) return rc;
    }
    return launch_subdivision(d_logits, d_mask, thresholds, d_parent_coords, parent_rows, d_child_coords,
                              d_linear_idx, d_pairs, nullptr, d_count, ws, s);
}

}  // extern "C"
