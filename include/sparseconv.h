/*
 * sparseconv.h -- C ABI of the MI355X (gfx950) sparse 3D convolution path.
 *
 * Drop-in boundary for burn_flex_gmm's device operator API and the
 * TRELLIS2 sparse decoder's conv seam (mosure/bevy_synth):
 *   - neighbour map   : neighbor_rows_tensor_from_coords_tensor
 *                       (crates/burn_flex_gmm/src/wgpu/neighbor.rs:977-1006)
 *   - submanifold conv: sparse_subm_conv_forward_wgpu[_with_config]
 *                       (crates/burn_flex_gmm/src/wgpu/sparse_conv.rs:310-367)
 *   - C2S subdivision : subdivision_active_indices_wgpu / expand_subdivision_
 *                       coords_and_linear_indices_wgpu / conv1 child select /
 *                       skip add (crates/burn_trellis/src/runtime_model/
 *                       sparse_decoder_wgpu_ops.rs:885-1054,
 *                       sparse_decoder_runtime_impl.rs:1009-1144,2180-2426)
 *   - block ops       : layer_norm[_silu], residual add
 *                       (crates/burn_flex_gmm/src/wgpu/ops.rs:162-446)
 *
 * Rules: every device pointer is caller-allocated; calls are stream-ordered
 * on the given hipStream_t (NULL = the default stream) and never synchronise
 * unless documented ("syncs"); no call allocates device memory except the
 * ones documented to (none in this header); the library keeps no mutable
 * global state except the per-thread error message.  Every function returns
 * an sc_status; on failure sc_last_error() holds a message on the calling
 * thread (the reference returns Result<_, String>).
 *
 * Tensors are dense row-major.  bf16 is the upper 16 bits of an IEEE f32
 * (uint16_t storage, same as torch.bfloat16).
 */
#ifndef SPARSECONV_H
#define SPARSECONV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SC_ABI_VERSION 2
#define SC_INVALID_NEIGHBOR_ROW (-1) /* crates/burn_flex_gmm/src/lib.rs:3 */

/* Mirror of SparseSubmConvConfig, crates/burn_flex_gmm/src/lib.rs:5-17. */
typedef struct sc_conv_config {
    int64_t in_channels;
    int64_t out_channels;
    int64_t kernel_d;
    int64_t kernel_h;
    int64_t kernel_w;
    int64_t in_channels_per_group;
    int64_t out_channels_per_group;
    int64_t groups;
    int32_t axis_order[3];
    int32_t axis_sign[3];
} sc_conv_config;

typedef enum sc_status {
    SC_OK = 0,
    SC_ERR_CONFIG = 1,      /* validate_config failures (lib.rs:698-725) */
    SC_ERR_SHAPE = 2,       /* shape / length mismatch */
    SC_ERR_DTYPE = 3,       /* unsupported dtype combination */
    SC_ERR_OVERFLOW = 4,    /* size arithmetic overflow */
    SC_ERR_WORKSPACE = 5,   /* workspace too small or misaligned */
    SC_ERR_COORD = 6,       /* negative coordinate or coordinate span too wide */
    SC_ERR_HIP = 7,         /* HIP runtime error (launch / copy) */
    SC_ERR_NULL = 8,        /* required pointer is NULL */
    SC_ERR_UNSUPPORTED = 9  /* valid request this build does not implement */
} sc_status;

typedef enum sc_dtype {
    SC_DTYPE_F32 = 0,
    SC_DTYPE_BF16 = 1,
    SC_DTYPE_I8 = 2,
    SC_DTYPE_F16 = 3  /* IEEE binary16: the decoder's compute_fp16 mode */
} sc_dtype;

/* hipStream_t, passed through untyped so that the header needs no HIP. */
typedef void *sc_stream;

int sc_abi_version(void);
const char *sc_status_string(int status);
/* Message of the last failing call on this thread ("" if none). */
const char *sc_last_error(void);

/* ---------------------------------------------------------------- config */

/* validate_config, crates/burn_flex_gmm/src/lib.rs:698-725. */
int sc_validate_config(const sc_conv_config *cfg);
/* kernel_rows, crates/burn_flex_gmm/src/lib.rs:59-67. */
int sc_kernel_rows(const sc_conv_config *cfg, int64_t *rows);
/* kernel_layout / kernel_offsets, crates/burn_flex_gmm/src/lib.rs:727-752 and
 * crates/burn_flex_gmm/src/wgpu/neighbor.rs:190-217.  Host only: writes
 * [K][3] (dx,dy,dz) into offsets; capacity_rows must be >= K. */
int sc_kernel_offsets(const sc_conv_config *cfg, int32_t *offsets, int64_t capacity_rows);

/* --------------------------------------------------------- neighbour map */

/* Bytes of device workspace sc_neighbor_map_build needs for n_rows coords
 * (a 256-byte header, bbox partials, and the larger of a hash table of 2..4
 * slots per row and a dense grid of 32 cells per row). */
int sc_neighbor_map_workspace_size(int64_t n_rows, size_t *bytes);

/*
 * Replaces neighbor_rows_tensor_from_coords_tensor
 * (crates/burn_flex_gmm/src/wgpu/neighbor.rs:977-1006) and the CPU
 * build_neighbor_rows (crates/burn_flex_gmm/src/lib.rs:69-109).
 *
 * d_coords: [n_rows][4] int32 (batch, x, y, z), all >= 0.
 * d_map   : [query_rows][K] int32 out; entry (r,k) is the row whose coord
 *           equals coord[r] + offset[k] (same batch), or -1.  Duplicated
 *           coords resolve to the LOWEST row, as every device algorithm of
 *           the reference does (neighbor_kernels.rs:30-40,249-256,419-422).
 *           query_rows <= n_rows maps the first query_rows coords against
 *           the full coord set (sparse_decoder_tests.rs:239-292).
 * Stream-ordered, no sync.  A negative coordinate component (a u32 coord
 * above i32::MAX, rejected by the reference at crates/burn_flex_gmm/src/
 * wgpu/neighbor.rs:252-263) is detected on the device: the map is then all
 * -1 and sc_neighbor_map_check reports SC_ERR_COORD.
 * The table is chosen on the device from the coords' bbox and order; the
 * int32 at byte 40 of d_workspace records it after the build (a diagnostic):
 * 1/2 hash table with 32/64-bit keys, 3 hash table over the coords, 4 dense
 * bbox grid, 5 rank bitmap (rows strictly increasing in (b, x, y, z)).
 */
int sc_neighbor_map_build(const sc_conv_config *cfg, const int32_t *d_coords, int64_t n_rows,
                          int64_t query_rows, int32_t *d_map, void *d_workspace,
                          size_t workspace_bytes, sc_stream stream);

/* Syncs `stream` and returns the device-side status of the last build that
 * used d_workspace (the reference reads its overflow counter back the same
 * way, crates/burn_flex_gmm/src/wgpu/neighbor.rs:859-879). */
int sc_neighbor_map_check(const void *d_workspace, sc_stream stream);

/* ---------------------------------------------------- submanifold conv */

/*
 * Replaces sparse_subm_conv_forward_wgpu[_with_config]
 * (crates/burn_flex_gmm/src/wgpu/sparse_conv.rs:310-367) and the CPU
 * sparse_subm_conv_forward_flex_precomputed (crates/burn_flex_gmm/src/
 * lib.rs:242-375):
 *   out[r, o] = bias[o] + scale[o] * sum_{k : map[r,k] != -1}
 *               sum_i in[map[r,k], g*Cin_g + i] * w[o, k, i],  g = o / Cout_g
 *   (+ residual[r, o] when d_residual is not NULL).
 *
 * d_input    : [n_in][Cin], act_dtype f32 or bf16.
 * d_map      : [n_q][K] int32 from sc_neighbor_map_build; n_q <= n_in.
 * d_weight   : [Cout][KD][KH][KW][Cin_g] (the reference layout),
 *              w_dtype f32 (act f32), bf16 (act bf16) or i8 (act bf16, with
 *              d_w_scale [Cout] f32 per-output-channel scales).
 * d_bias     : [Cout] f32 (may be NULL = zeros).
 * d_residual : [n_q][Cout] in out_dtype, or NULL.
 * d_out      : [n_q][Cout], out_dtype f32 or bf16 (bf16 is rounded to nearest
 *              even from the f32 accumulator).
 * Map entries outside [0, n_in) are treated as absent (-1).
 * Accumulation is fp32 in a fixed order: results are bit-identical run to run.
 */
int sc_subm_conv_forward(const sc_conv_config *cfg, int act_dtype, const void *d_input,
                         int64_t n_in, const int32_t *d_map, int64_t n_q, int w_dtype,
                         const void *d_weight, const float *d_w_scale, const float *d_bias,
                         const void *d_residual, int out_dtype, void *d_out, sc_stream stream);

/*
 * Epilogue fused into the conv (the block patterns of the decoder: conv ->
 * LayerNorm -> SiLU, sparse_decoder_wgpu_ops.rs:1091-1161, and conv -> + x):
 *   y = conv + bias;  if layer_norm: y = LN(y over the row's Cout channels)
 *   [*ln_weight][+ln_bias] (two-pass f32, biased variance, ln_eps);  if silu:
 *   y = y / (1 + exp(-y));  if residual: y += residual.
 */
typedef struct sc_conv_epilogue {
    const void *residual;    /* [n_q][Cout] in out_dtype, or NULL */
    int layer_norm;          /* 0 / 1 */
    const float *ln_weight;  /* [Cout] or NULL */
    const float *ln_bias;    /* [Cout] or NULL */
    float ln_eps;
    int silu;                /* 0 / 1 */
    /* f32 staging for a LayerNorm the conv tile cannot hold (below), 16-byte
     * aligned, or NULL; sc_conv_epilogue_workspace_size gives the size. */
    void *workspace;
    size_t workspace_bytes;
    /* C2S forms of the decoder's upsample block (all NULL / 0 otherwise;
     * groups == 1, no residual; the two are exclusive):
     *  - child scatter, conv1 on the parents (Cout = 8 * C, C a multiple of
     *    4): parent row r's channels [c*C, (c+1)*C) are child c's features
     *    and go to row child_rows[8r + c] of d_out ([n_child_rows][C]); -1
     *    (inactive child) drops them.  LayerNorm then runs over each child's
     *    C channels.  With n_child_rows == 0 the call writes nothing and
     *    d_out may be NULL.  This is conv1 + reshape [P, 8C] -> [8P, C] + select
     *    (sparse_decoder_runtime_impl.rs:2240-2255) without the [P, 8C]
     *    tensor; child_rows comes from sc_subdivision_build_indexed.
     *  - parent skip, conv2 on the children: with S = skip_parent_channels/8
     *    and R = Cout/S, y[a, o] += parent[li / 8][(li % 8)*S + o / R],
     *    li = skip_index[a] (the children's linear_idx), parent in out_dtype
     *    (sparse_decoder_runtime_impl.rs:1054-1076,1123-1133). */
    const int32_t *child_rows;
    int64_t n_child_rows;
    const void *skip_parent;
    const int32_t *skip_index;
    int64_t skip_parent_rows;
    int64_t skip_parent_channels;
    /* Child scatter with n_child_rows an upper bound (8P, so that conv1 can
     * be enqueued before the child count reaches the host): the device int64
     * count sc_subdivision_build_indexed wrote, or NULL.  A LayerNorm staged
     * through `workspace` then stops at that row; rows past it are neither
     * written by the conv nor read.  (Last field: a zero-initialised
     * epilogue leaves it NULL.) */
    const int64_t *child_count;
} sc_conv_epilogue;

/* sc_subm_conv_forward with a fused epilogue (same arguments, epi replaces
 * d_residual; epi may be NULL).  Every value is rounded to out_dtype once,
 * at the end.  SiLU without LayerNorm and the residual run inside the conv
 * kernel, on the f32 accumulators, for every shape; so does LayerNorm when
 * one workgroup holds whole rows (groups == 1, Cout <= 128, the MFMA tile:
 * Cin_g a multiple of 32 (bf16) / 16 (f32), K <= 32, 16-byte aligned
 * pointers).  Otherwise the conv stores its f32 accumulators -- into d_out
 * for an f32 output, else into epi->workspace (n_q * Cout * 4 bytes; without
 * it the call fails with SC_ERR_WORKSPACE) -- and one stream-ordered row
 * kernel applies LayerNorm -> SiLU -> + residual to them (the reference
 * normalises its f32 conv output the same way, sparse_decoder_wgpu_ops.rs
 * :1642-1711). */
int sc_subm_conv_forward_fused(const sc_conv_config *cfg, int act_dtype, const void *d_input,
                               int64_t n_in, const int32_t *d_map, int64_t n_q, int w_dtype,
                               const void *d_weight, const float *d_w_scale, const float *d_bias,
                               const sc_conv_epilogue *epi, int out_dtype, void *d_out,
                               sc_stream stream);

/* Bytes of epi->workspace a fused or planned conv with this epilogue needs:
 * n_q * Cout * 4 when epi asks for LayerNorm with a bf16 output and the
 * shape keeps the row out of one conv tile (groups > 1, Cout > 128, Cin_g
 * not a multiple of 32, K > 32), else 0.  (Misaligned pointers or tensors of
 * 2 GiB and more also keep the row out of the tile; the conv then reports
 * the size it needs.)  Host only. */
int sc_conv_epilogue_workspace_size(const sc_conv_config *cfg, int act_dtype, int64_t n_q, int out_dtype,
                                    const sc_conv_epilogue *epi, size_t *bytes);

/*
 * Dense linear layer out = x W^T + b with the conv's epilogue (SiLU,
 * residual, LayerNorm over the row): linear_forward_wgpu
 * (sparse_decoder_wgpu_ops.rs:79-160) as used by the ConvNeXt block's MLP
 * (convnext_block_mlp_forward_wgpu, :356-489: mlp_0 -> SiLU -> mlp_2 + x).
 * x [rows][in_channels], W [out_channels][in_channels] (the reference's
 * LinearLayer layout), b [out_channels] f32 or NULL; dtypes as for
 * sc_subm_conv_forward_fused (bf16 / f16 / f32 activations; int8 weights
 * with d_w_scale).  It is that conv with a 1x1x1 kernel and no map (row r
 * reads row r), on the same MFMA tiles.  epi may be NULL.  epi->child_rows
 * (no residual) makes it the 2x2x2 transposed upsample: rows are parents,
 * out_channels = 8 x C, and slice c of row r lands in row child_rows[r * 8 +
 * c] of an [n_child_rows][C] output (LayerNorm, when asked, per child);
 * epi->skip_index, the conv2 form, is refused.
 */
int sc_linear_forward(int act_dtype, const void *d_input, int64_t rows, int64_t in_channels,
                      int64_t out_channels, int w_dtype, const void *d_weight, const float *d_w_scale,
                      const float *d_bias, const sc_conv_epilogue *epi, int out_dtype, void *d_out,
                      sc_stream stream);

/* ----------------------------------------------------------- conv plan */

/*
 * Conv plan: a row order and per-tile halo tables derived from one
 * neighbour map, which the planned conv reads.  It has no counterpart in the
 * reference's API: it plays the role of the reference's neighbour cache
 * (the decoder reuses one map for every conv at a resolution,
 * crates/burn_flex_gmm/src/wgpu.rs:349-382, sparse_decoder.rs:1057-1136):
 * build it once per map, right after sc_neighbor_map_build, and pass it to
 * every sc_subm_conv_forward_planned call on that map.
 *
 * Rows are ordered by 8^3 bricks of the coords' bounding box (bricks in
 * (batch, x, y, z) order, lexicographic inside a brick; coarser bricks when
 * the box is too large for the plan's occupancy grid) and cut into tiles of
 * 256 rows; for each tile the plan lists the distinct input rows its
 * neighbours touch (at most 960, else the tile is listed for the direct
 * kernel) and a 16-bit local index per (row, offset).  The row order and
 * the tables are a pure function of the coords and the map: a rebuild gives
 * the same plan.
 *
 * sc_conv_plan_size: bytes of the plan buffer for n_q query rows and a kernel
 * of kernel_rows offsets (1..32).
 * sc_conv_plan_build: d_coords [n_in][4] i32 (the coords the map was built
 * from), d_map [n_q][K] i32 (sc_neighbor_map_build's output for query rows
 * [0, n_q)); d_plan 256-byte aligned, plan_bytes >= sc_conv_plan_size.
 * Stream-ordered, no sync, no allocation.  The plan is valid for that map
 * (same n_in, n_q, K) until the map changes.
 */
int sc_conv_plan_size(int64_t n_q, int64_t kernel_rows, size_t *bytes);
int sc_conv_plan_build(const sc_conv_config *cfg, const int32_t *d_coords, int64_t n_in,
                       const int32_t *d_map, int64_t n_q, void *d_plan, size_t plan_bytes,
                       sc_stream stream);

/*
 * sc_conv_plan_build in two halves, so that the first can overlap the map
 * build on another stream: sc_conv_plan_order reads only the coords (the row
 * order: query rows [0, n_q) of d_coords [n_in][4]); sc_conv_plan_tables then
 * reads the map (the per-tile halo tables) and must run after both the
 * order (same plan buffer) and the map build are complete -- stream order or
 * an event.  Same arguments as sc_conv_plan_build; together they write the
 * same plan.
 */
int sc_conv_plan_order(const sc_conv_config *cfg, const int32_t *d_coords, int64_t n_in, int64_t n_q,
                       void *d_plan, size_t plan_bytes, sc_stream stream);
int sc_conv_plan_tables(const sc_conv_config *cfg, const int32_t *d_map, int64_t n_in, int64_t n_q,
                        void *d_plan, size_t plan_bytes, sc_stream stream);


/*
 * Weights packed for the planned conv: per (group, 128-output-channel tile,
 * offset k, 32-input-channel chunk, 16-channel block) one contiguous
 * fragment in MFMA operand order.  It has no counterpart in the reference's
 * device API; it plays the role of pack_flex_weight
 * (crates/burn_flex_gmm/src/lib.rs:377-426), a one-time per-layer reorder
 * (the decoder caches its weights per layer, sparse_decoder.rs:757-844).
 * w_dtype bf16 or i8; the fragments are bf16 either way (int8 weights are
 * widened exactly, |q| <= 127, and their [Cout] f32 scales, passed to the
 * conv as usual, are applied in its epilogue).  Cin per group must be a
 * multiple of 32.  d_weight is the reference layout [Cout][KD][KH][KW]
 * [Cin_g]; d_packed is 16-byte aligned, sc_conv_weight_pack_size bytes: a
 * 256-byte header recording the config the weights were packed for (groups,
 * Cout_g, Cin_g, K), then 2 bytes per weight of each 128-channel output tile.
 */
int sc_conv_weight_pack_size(const sc_conv_config *cfg, int w_dtype, size_t *bytes);
int sc_conv_weight_pack(const sc_conv_config *cfg, int w_dtype, const void *d_weight, void *d_packed,
                        sc_stream stream);

/*
 * sc_subm_conv_forward_fused reading a plan of the same map and the packed
 * copy of the weights (both may be NULL).  With both, bf16 activations and at
 * most 27 offsets take the halo-staged kernel (a tile whose halo exceeds its
 * LDS budget reads its operands from global memory, in the same order);
 * d_weight (reference layout) is still required for shapes the halo kernel
 * does not take.  Same result as
 * sc_subm_conv_forward_fused up to f32 summation order: the halo kernel sums
 * each row's (32-channel chunk, offset) products chunk-major instead of
 * offset-major, in a fixed order, so results are bit-identical run to run.
 * The kernels compare the plan's header (n_q, n_in, K) and the packed
 * weights' header (groups, Cout_g, Cin_g, K) with this call before they
 * read anything else from either buffer: on a mismatch d_out is left
 * untouched (the epilogue workspace of a LayerNorm wider than one tile too
 * is then not normalised into d_out) and the plan's status records it
 * (sc_conv_plan_check).  A flagged plan stays flagged until it is rebuilt:
 * every planned conv on it leaves d_out untouched meanwhile.  A plan from
 * another map of the same n_q / n_in / K is not detected.
 */
int sc_subm_conv_forward_planned(const sc_conv_config *cfg, int act_dtype, const void *d_input,
                                 int64_t n_in, const int32_t *d_map, int64_t n_q, int w_dtype,
                                 const void *d_weight, const void *d_packed_weight,
                                 const float *d_w_scale, const float *d_bias,
                                 const sc_conv_epilogue *epi, int out_dtype, void *d_out,
                                 const void *d_plan, sc_stream stream);

/*
 * Child plan: C2S conv1 over the active children only.  conv1 of the
 * decoder's upsample block maps Cin -> 8 * Cout_child on the parents and
 * keeps, per parent, only its active children's slices (the reference
 * computes all eight and selects, sparse_decoder_runtime_impl.rs:2180-2255).
 * A child plan groups, per child index c, the parents whose child c is
 * active (d_child_rows [P][8] from sc_subdivision_build_indexed, 16-byte
 * aligned; rows outside [0, n_children) count as inactive), in the parent
 * plan's order (d_parent_plan: sc_conv_plan_build on the parents' map
 * d_map [P][K]), into 256-row tiles of their own with halo tables; a tile
 * then computes only its child's Cout_child channels.  Size it with
 * sc_conv_child_plan_size (it depends on the child count); the build
 * launches four kernels, stream-ordered, no sync.  A parent plan built for
 * another row count or K, or more active children than n_children, leaves
 * the plan empty and flagged (sc_conv_plan_check).  No reference
 * counterpart: it replaces the [P, 8 * Cout_child] tensor and its select.
 */
int sc_conv_child_plan_size(int64_t n_parents, int64_t n_children, int64_t kernel_rows, size_t *bytes);
int sc_conv_child_plan_build(const sc_conv_config *cfg, const void *d_parent_plan, const int32_t *d_map,
                             int64_t n_parents, const int32_t *d_child_rows, int64_t n_children,
                             void *d_child_plan, size_t child_plan_bytes, sc_stream stream);

/*
 * A child plan for the dense linear's child scatter (the 2x2x2 transposed
 * upsample: sc_linear_forward with epi->child_rows): per child index c, the
 * parents whose child c is active (d_child_rows[p * 8 + c] in
 * [0, n_children)), in row order, in 256-row tiles of their own, so that
 * sc_linear_forward_child_planned computes only the active children.  The
 * buffer is sized by sc_conv_child_plan_size(n_parents, n_children, 1); the
 * build launches five kernels, stream-ordered, no sync, and has no halo
 * tables (the linear reads each parent's own row).  More active children
 * than n_children leaves the plan empty and flagged (sc_conv_plan_check).
 * No reference counterpart: the reference's transposed upsample computes
 * every child of every parent.
 */
int sc_linear_child_plan_build(int64_t n_parents, const int32_t *d_child_rows, int64_t n_children,
                               void *d_child_plan, size_t child_plan_bytes, sc_stream stream);

/*
 * sc_linear_forward with the child scatter (epi->child_rows and
 * epi->n_child_rows required, the table and count the plan was built from)
 * over a linear child plan: each tile's parents, one child's channels, so
 * inactive children cost nothing.  Every stored value is the same sum as
 * sc_linear_forward's.  Needs 16-bit activations and weights, in_channels a
 * multiple of 32 and children of a multiple of 128 channels (out_channels /
 * 8); other shapes fail with SC_ERR_UNSUPPORTED.
 */
int sc_linear_forward_child_planned(int act_dtype, const void *d_input, int64_t rows, int64_t in_channels,
                                    int64_t out_channels, int w_dtype, const void *d_weight,
                                    const float *d_w_scale, const float *d_bias, const sc_conv_epilogue *epi,
                                    int out_dtype, void *d_out, const void *d_child_plan, sc_stream stream);

/*
 * sc_subm_conv_forward_planned on a child plan: conv1 of the C2S block with
 * the child scatter (epi->child_rows and epi->n_child_rows required, the same
 * table and count the child plan was built from), only the active children
 * computed.  Same results as sc_subm_conv_forward_planned with the parent
 * plan and the same epilogue (each stored value is the same sum in the same
 * order), except for children of 64 channels: their tiles split the stages
 * between two waves by the tile's offsets, another fixed order.  Needs 16-bit
 * activations, packed weights, one group, at most 27
 * offsets, and children of 64 channels or a multiple of 128 (Cout 512 or a
 * multiple of 1024); other shapes fail with SC_ERR_UNSUPPORTED.
 */
int sc_subm_conv_forward_child_planned(const sc_conv_config *cfg, int act_dtype, const void *d_input,
                                       int64_t n_in, const int32_t *d_map, int64_t n_q, int w_dtype,
                                       const void *d_weight, const void *d_packed_weight,
                                       const float *d_w_scale, const float *d_bias,
                                       const sc_conv_epilogue *epi, int out_dtype, void *d_out,
                                       const void *d_child_plan, sc_stream stream);

/* Syncs `stream` and reports whether a planned conv on d_plan found the plan
 * or the packed weights built for another shape (SC_ERR_SHAPE; the conv then
 * wrote nothing).  The status is cleared when the plan is rebuilt (the
 * reference checks shapes before every launch, crates/burn_flex_gmm/src/
 * wgpu/sparse_conv.rs:369-473; here the plan lives on the device, so the
 * check runs there). */
int sc_conv_plan_check(const void *d_plan, sc_stream stream);

/* ------------------------------------------------------------ block ops */

/*
 * Row LayerNorm with optional affine and SiLU: layer_norm_row_stats +
 * layer_norm_affine[_silu] (crates/burn_flex_gmm/src/wgpu/ops.rs:162-446),
 * host form layer_norm_inplace + silu_inplace (sparse_decoder_wgpu_ops.rs
 * :1642-1720): two-pass f32 mean / biased variance, (x-mean)/sqrt(var+eps)
 * [*w][+b], then x/(1+exp(-x)) if apply_silu.  d_w / d_b may be NULL.
 * d_in may equal d_out when the dtypes match.
 */
int sc_layer_norm(int in_dtype, const void *d_in, int64_t rows, int64_t channels,
                  const float *d_w, const float *d_b, float eps, int apply_silu, int out_dtype,
                  void *d_out, sc_stream stream);

/* Skinny linear for the C2S to_subdiv head: out[r, o] = b[o] + sum_i x[r, i]
 * w[o, i] (linear_skinny_forward_wgpu, crates/burn_flex_gmm/src/wgpu/
 * ops.rs:1390-1410; kernel :135-160).  x [rows][in_channels] f32 or bf16
 * (16-byte aligned), w [out_channels][in_channels] f32, b [out_channels] f32
 * or NULL, out [rows][out_channels] f32; out_channels 1..8.  f32
 * accumulation in a fixed order. */
int sc_linear_skinny(int in_dtype, const void *d_x, int64_t rows, int64_t in_channels, const float *d_w,
                     const float *d_b, int64_t out_channels, float *d_out, sc_stream stream);

/* Post-processing of the to_subdiv logits [rows][8] f32 in place (16-byte
 * aligned), in the reference's order: with round_f16, each logit is rounded
 * to f16 and back (quantize_f16 under compute_fp16,
 * sparse_decoder_runtime_impl.rs:871-873); with center, the row's mean (f32
 * sum in child order / 8) is subtracted (center_subdivision_logits,
 * row_center_logits, sparse_decoder_wgpu_ops.rs:1728-1745).  Both off: no
 * launch. */
int sc_subdivision_logits_finish(float *d_logits, int64_t rows, int round_f16, int center, sc_stream stream);

/* out = a + b elementwise over n values (add_inplace, sparse_decoder_wgpu_ops.rs
 * :1747-1757).  All three share `dtype`; d_out may alias d_a. */
int sc_add(int dtype, const void *d_a, const void *d_b, int64_t n, void *d_out, sc_stream stream);

/* ------------------------------------------------- C2S subdivision path */

/* Workspace bytes for sc_subdivision_build with parent_rows parents. */
int sc_subdivision_workspace_size(int64_t parent_rows, size_t *bytes);

/*
 * subdivision_active_indices_wgpu + expand_subdivision_coords_and_linear_
 * indices_wgpu (sparse_decoder_wgpu_ops.rs:885-1054): child c of parent p is
 * active when logits[p][c] > thresholds[c] (d_logits given) or mask[p][c] != 0
 * (d_mask given; exactly one of the two).  Children are emitted parent-major,
 * child-ascending (the argwhere order on [P,8]); for child a:
 *   child_coords[a] = (b, 2x + (c&1), 2y + (c>>1 & 1), 2z + (c>>2 & 1))
 *   linear_idx[a]   = 8*p + c
 *   pairs[a]        = (p, c)          (d_pairs may be NULL)
 * d_child_coords [8P][4], d_linear_idx [8P] and d_pairs [8P][2] are sized for
 * the worst case.  The child count is written to d_count (int64, device).
 * thresholds is a host array of 8 floats (ignored with a mask).
 */
int sc_subdivision_build(const float *d_logits, const uint8_t *d_mask, const float *thresholds,
                         const int32_t *d_parent_coords, int64_t parent_rows,
                         int32_t *d_child_coords, int32_t *d_linear_idx, int32_t *d_pairs,
                         int64_t *d_count, void *d_workspace, size_t workspace_bytes,
                         sc_stream stream);

/*
 * sc_subdivision_build that also writes the inverse of linear_idx:
 * d_child_rows [P][8] int32 (16-byte aligned) holds, for child c of parent p,
 * its row a in the outputs above (linear_idx[a] == 8p + c), or -1 when the
 * child is inactive.  That is the table the conv1 child scatter
 * (sc_conv_epilogue.child_rows) reads.
 */
int sc_subdivision_build_indexed(const float *d_logits, const uint8_t *d_mask, const float *thresholds,
                                 const int32_t *d_parent_coords, int64_t parent_rows,
                                 int32_t *d_child_coords, int32_t *d_linear_idx, int32_t *d_pairs,
                                 int32_t *d_child_rows, int64_t *d_count, void *d_workspace,
                                 size_t workspace_bytes, sc_stream stream);

/*
 * sc_subdivision_build without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid hipMalloc).  It has no counterpart in the reference.  Same
 * arguments and results as sc_subdivision_build; its scratch (block counts,
 * 16 KiB + 16 B) is a static device array inside the library,
 * one copy per GPU, held until the process ends.  parent_rows is limited to
 * 2^26 (67,108,864; larger counts fail with SC_ERR_WORKSPACE and
 * launch nothing).  It calls no allocator.  Every call on one GPU shares that
 * array: calls that overlap on one GPU (different streams, or threads without
 * stream ordering between them) race and must not be issued; calls ordered
 * on one stream are fine.  The first call on a device looks up the array's
 * address there (hipGetSymbolAddress), which is not capturable: make one
 * call on each device before capturing.
 */
int sc_subdivision_build_static(const float *d_logits, const uint8_t *d_mask, const float *thresholds,
                                const int32_t *d_parent_coords, int64_t parent_rows,
                                int32_t *d_child_coords, int32_t *d_linear_idx, int32_t *d_pairs,
                                int64_t *d_count, sc_stream stream);

/*
 * Row gather from a [src_rows*split][width] view of src ([src_rows][split*width]):
 *   out[a, :] = view[idx[a], :]      for a < n_out
 * This is conv1's child selection (reshape [P, 8*Cout] -> [8P, Cout], then
 * select(linear_idx); sparse_decoder_runtime_impl.rs:2249-2255) with split=8.
 */
int sc_gather_rows(int dtype, const void *d_src, int64_t src_rows, int64_t split, int64_t width,
                   const int32_t *d_idx, int64_t n_out, void *d_out, sc_stream stream);

/*
 * C2S channel-repeated skip (sparse_decoder_runtime_impl.rs:1054-1076,
 * 1123-1133): with S = parent_channels/8 and R = out_channels/S,
 *   h[a, j] += parent[idx[a] / 8, (idx[a] % 8)*S + j / R]
 * h is [n][out_channels] (f32 or bf16, = dtype), parent [P][parent_channels]
 * in parent_dtype.
 */
int sc_c2s_skip_add(int dtype, void *d_h, int64_t n, int64_t out_channels, int parent_dtype,
                    const void *d_parent, int64_t parent_rows, int64_t parent_channels,
                    const int32_t *d_idx, sc_stream stream);

/* Element conversions (f32 <-> bf16 with round-to-nearest-even, the rule of
 * bf16_round_to_f32, crates/burn_flex_gmm/src/wgpu.rs:57-67). */
int sc_convert(int in_dtype, const void *d_in, int out_dtype, void *d_out, int64_t n,
               sc_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* SPARSECONV_H */
