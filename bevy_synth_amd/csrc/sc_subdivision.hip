// C2S subdivision: active-child compaction and child coordinate expansion.
//
// Replaces subdivision_active_indices_wgpu (argwhere of (logits - thr) > 0
// on [P,8]) and expand_subdivision_coords_and_linear_indices_wgpu
// (sparse_decoder_wgpu_ops.rs:885-1054) with a three-launch stream compaction:
//   count : 1024 parents per block, popcount of each parent's 8-bit child
//           mask, block total via wave64 reduction
//   scan  : one block scans the block totals (exclusive) and writes the
//           child count
//   emit  : block-exclusive prefix (wave64 shfl scan + LDS wave totals) of
//           per-thread counts; each thread writes the children of its 4
//           consecutive parents in child order -> parent-major,
//           child-ascending output, identical to argwhere's row-major order.
#include "sc_common.hpp"

namespace sc {
namespace {

constexpr int kThreads = 256;
constexpr int kParentsPerThread = 4;
constexpr int kParentsPerBlock = kThreads * kParentsPerThread;

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
                                                                Thresholds th, int64_t P,
                                                                int64_t *block_counts)
{
    __shared__ int s_wave[kThreads / 64];
    const int64_t p0 = (int64_t)blockIdx.x * kParentsPerBlock + (int64_t)threadIdx.x * kParentsPerThread;
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < kParentsPerThread; ++i)
        if (p0 + i < P) cnt += __popc(child_mask(logits, mask, th, p0 + i));
    int total;
    block_exclusive_scan(cnt, s_wave, total);
    if (threadIdx.x == 0) block_counts[blockIdx.x] = total;
}

__global__ __launch_bounds__(1024) void subdiv_scan_kernel(const int64_t *block_counts, int64_t nblocks,
                                                           int64_t *block_offsets, int64_t *count)
{
    __shared__ int64_t s_part[1024];
    int64_t carry = 0;
    for (int64_t base = 0; base < nblocks; base += 1024) {
        const int64_t i = base + threadIdx.x;
        const int64_t v = i < nblocks ? block_counts[i] : 0;
        s_part[threadIdx.x] = v;
        __syncthreads();
        // Hillis-Steele inclusive scan over 1024 entries.
        for (int off = 1; off < 1024; off <<= 1) {
            const int64_t y = threadIdx.x >= (unsigned)off ? s_part[threadIdx.x - off] : 0;
            __syncthreads();
            s_part[threadIdx.x] += y;
            __syncthreads();
        }
        if (i < nblocks) block_offsets[i] = carry + s_part[threadIdx.x] - v;
        const int64_t chunk_total = s_part[1023];
        __syncthreads();
        carry += chunk_total;
    }
    if (threadIdx.x == 0) *count = carry;
}

__global__ __launch_bounds__(kThreads) void subdiv_emit_kernel(const float *logits, const uint8_t *mask,
                                                               Thresholds th, int64_t P,
                                                               const int4 *__restrict__ parent_coords,
                                                               const int64_t *block_offsets,
                                                               int4 *child_coords, int32_t *linear_idx,
                                                               int2 *pairs)
{
    __shared__ int s_wave[kThreads / 64];
    const int64_t p0 = (int64_t)blockIdx.x * kParentsPerBlock + (int64_t)threadIdx.x * kParentsPerThread;
    unsigned m[kParentsPerThread];
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < kParentsPerThread; ++i) {
        m[i] = p0 + i < P ? child_mask(logits, mask, th, p0 + i) : 0u;
        cnt += __popc(m[i]);
    }
    int total;
    int64_t out = block_offsets[blockIdx.x] + block_exclusive_scan(cnt, s_wave, total);
#pragma unroll
    for (int i = 0; i < kParentsPerThread; ++i) {
        if (!m[i]) continue;
        const int64_t p = p0 + i;
        const int4 pc = parent_coords[p];
        for (int c = 0; c < 8; ++c) {
            if (!(m[i] & (1u << c))) continue;
            child_coords[out] = make_int4(pc.x, 2 * pc.y + (c & 1), 2 * pc.z + ((c >> 1) & 1),
                                          2 * pc.w + ((c >> 2) & 1));
            linear_idx[out] = (int32_t)(p * 8 + c);
            if (pairs) pairs[out] = make_int2((int32_t)p, c);
            ++out;
        }
    }
}

__global__ void write_zero_count(int64_t *count) { *count = 0; }

inline int64_t n_blocks(int64_t P) { return (P + kParentsPerBlock - 1) / kParentsPerBlock; }

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
    *bytes = (size_t)(2 * n_blocks(parent_rows) + 2) * sizeof(int64_t);
    return SC_OK;
}

int sc_subdivision_build(const float *d_logits, const uint8_t *d_mask, const float *thresholds,
                         const int32_t *d_parent_coords, int64_t parent_rows,
                         int32_t *d_child_coords, int32_t *d_linear_idx, int32_t *d_pairs,
                         int64_t *d_count, void *d_workspace, size_t workspace_bytes,
                         sc_stream stream)
{
    clear_error();
    if (parent_rows < 0 || parent_rows > INT32_MAX / 8)
        return fail(SC_ERR_SHAPE, "subdivision parent rows out of range");
    if (!d_count) return fail(SC_ERR_NULL, "subdivision count pointer is NULL");
    hipStream_t s = as_stream(stream);
    if (parent_rows == 0) {
        write_zero_count<<<1, 1, 0, s>>>(d_count);
        SC_LAUNCH_CHECK("write_zero_count launch");
        return SC_OK;
    }
    if ((d_logits == nullptr) == (d_mask == nullptr))
        return fail(SC_ERR_NULL, "subdivision needs exactly one of logits or mask");
    if (d_logits && !thresholds) return fail(SC_ERR_NULL, "subdivision thresholds are NULL");
    if (!d_parent_coords || !d_child_coords || !d_linear_idx || !d_workspace)
        return fail(SC_ERR_NULL, "subdivision: NULL pointer");
    const uintptr_t al = (uintptr_t)d_parent_coords | (uintptr_t)d_child_coords |
                         (uintptr_t)(d_logits ? (const void *)d_logits : (const void *)d_mask);
    if (al % 16 != 0 || (uintptr_t)d_workspace % 8 != 0 || (d_pairs && (uintptr_t)d_pairs % 8 != 0))
        return fail(SC_ERR_SHAPE, "subdivision buffers must be 16-byte aligned");
    const int64_t nb = n_blocks(parent_rows);
    const size_t need = (size_t)(2 * nb + 2) * sizeof(int64_t);
    if (workspace_bytes < need) return fail(SC_ERR_WORKSPACE, "subdivision workspace too small");
    Thresholds th;
    for (int c = 0; c < 8; ++c) th.t[c] = thresholds ? thresholds[c] : 0.f;
    int64_t *counts = (int64_t *)d_workspace;
    int64_t *offsets = counts + nb;
    subdiv_count_kernel<<<(unsigned)nb, kThreads, 0, s>>>(d_logits, d_mask, th, parent_rows, counts);
    SC_LAUNCH_CHECK("subdiv_count_kernel launch");
    subdiv_scan_kernel<<<1, 1024, 0, s>>>(counts, nb, offsets, d_count);
    SC_LAUNCH_CHECK("subdiv_scan_kernel launch");
    subdiv_emit_kernel<<<(unsigned)nb, kThreads, 0, s>>>(d_logits, d_mask, th, parent_rows,
                                                         (const int4 *)d_parent_coords, offsets,
                                                         (int4 *)d_child_coords, d_linear_idx,
                                                         (int2 *)d_pairs);
    SC_LAUNCH_CHECK("subdiv_emit_kernel launch");
    return SC_OK;
}

}  // extern "C"
