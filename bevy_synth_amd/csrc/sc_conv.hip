// Submanifold sparse convolution for gfx950: output-stationary implicit
// gather-GEMM on MFMA.
//
// Replaces the scalar gather-dot kernels of the reference
// (crates/burn_flex_gmm/src/wgpu/sparse_conv_kernels.rs K9-K17: one lane per
// output value re-reading K*Cin inputs and weights from global memory).
//
// Every MFMA kernel here computes a tile of 256 query rows x 128 output
// channels of one group with 4 waves, reduces over (used kernel offset,
// input-channel chunk) stages, skips offsets no row of the tile uses, and
// fuses the epilogue (* int8 scale + bias, optional LayerNorm / SiLU over the
// row, optional residual).  Kernels, by the path that takes them:
//   conv_halo_kernel  bf16 activations with a conv plan (sc_plan.hpp) and
//                     packed weights: the tile's distinct neighbour rows are
//                     staged in LDS once per 32-channel chunk and every
//                     operand is read from there (v_mfma_f32_16x16x32_bf16);
//                     a tile whose halo exceeds the LDS budget gathers its
//                     operands from global memory in the same stage order;
//   conv_v2_kernel    bf16 activations without a plan: neighbour rows
//                     gathered from global memory per (row, offset), weights
//                     staged in LDS;
//   conv_mfma_kernel  f32 activations (v_mfma_f32_32x32x2_f32);
//   conv_scalar_kernel  shapes no tile takes (channel counts that are not
//                     multiples of the chunk, K > 32, unaligned pointers,
//                     tensors of 2 GiB or more): one lane per output value.
// All accumulate in f32 in a fixed order, so results are bit-identical run to
// run.
#include "sc_conv_kernels.hpp"

using namespace sc;

static int launch_conv_typed(const ConvArgs &a, bool act_f32, int w_dtype, int out_dtype, int groups,
                             bool mfma, const void *plan, hipStream_t s)
{
    if (act_f32) {
        if (out_dtype == SC_DTYPE_F32) return launch_conv<float, float, float>(a, groups, mfma, nullptr, s);
        return launch_conv<float, float, uint16_t>(a, groups, mfma, nullptr, s);
    }
    if (w_dtype == SC_DTYPE_F16)  // f16 activations and weights (the decoder's compute_fp16 mode)
        return launch_conv_f16(a, out_dtype, groups, mfma, plan, s);
    if (w_dtype == SC_DTYPE_BF16) {
        if (out_dtype == SC_DTYPE_F32) return launch_conv<uint16_t, uint16_t, float>(a, groups, mfma, plan, s);
        return launch_conv<uint16_t, uint16_t, uint16_t>(a, groups, mfma, plan, s);
    }
    return launch_conv_i8(a, out_dtype, groups, mfma, plan, s);
}

// Shapes the MFMA tiles take (pointer alignment and tensor sizes aside):
// Cin per group a multiple of the 64-byte reduction chunk, at most 32 offsets.
static bool mfma_shape_ok(const sc_conv_config *cfg, int act_dtype)
{
    const int bk = kChunkBytes / (int)dtype_size(act_dtype);
    const int64_t K = cfg->kernel_d * cfg->kernel_h * cfg->kernel_w;
    return bk > 0 && cfg->in_channels_per_group % bk == 0 && K <= kMaxTableK;
}

// The C2S epilogue forms of an epilogue (child scatter of conv1, parent skip
// of conv2), checked against the config.
struct C2SForms {
    bool scatter = false, skip = false;
    int64_t scatter_ch = 0, scatter_n = 0;
    int64_t skip_S = 0, skip_R = 0;
};

static int c2s_forms(const sc_conv_config *cfg, const sc_conv_epilogue *epi, C2SForms &f)
{
    f = C2SForms{};
    if (!epi) return SC_OK;
    f.scatter = epi->child_rows != nullptr;
    f.skip = epi->skip_index != nullptr;
    if (!f.scatter && !f.skip) return SC_OK;
    if (f.scatter && f.skip) return fail(SC_ERR_UNSUPPORTED, "sparse conv: child scatter and parent skip are exclusive");
    if (epi->residual) return fail(SC_ERR_UNSUPPORTED, "sparse conv: the C2S forms take no residual");
    if (cfg->groups != 1) return fail(SC_ERR_UNSUPPORTED, "sparse conv: the C2S forms need groups == 1");
    if (f.scatter) {
        if (cfg->out_channels % 32 != 0)
            return fail(SC_ERR_SHAPE, "sparse conv child scatter: Cout must be 8 children x a multiple of 4 channels");
        if (epi->n_child_rows < 0) return fail(SC_ERR_SHAPE, "sparse conv child scatter: negative child row count");
        f.scatter_ch = cfg->out_channels / 8;
        f.scatter_n = epi->n_child_rows;
    } else {
        const int64_t pc = epi->skip_parent_channels;
        if (!epi->skip_parent) return fail(SC_ERR_NULL, "sparse conv parent skip: parent features are NULL");
        if (epi->skip_parent_rows < 0 || pc <= 0 || pc % 8 != 0 || cfg->out_channels % (pc / 8) != 0)
            return fail(SC_ERR_SHAPE, "decoder invalid skip channel ratio (in=" + std::to_string(pc) +
                                          ", out=" + std::to_string(cfg->out_channels) + ")");
        if (epi->skip_parent_rows > INT32_MAX / 8)
            return fail(SC_ERR_SHAPE, "sparse conv parent skip: too many parent rows");
        f.skip_S = pc / 8;
        f.skip_R = cfg->out_channels / f.skip_S;
    }
    return SC_OK;
}

// Whether LayerNorm runs in the conv tile's epilogue: the whole row (or, in
// the child scatter, one child's 64 or 128 channels inside a 128-channel
// tile of the bf16 kernels) in one workgroup.
static bool ln_in_tile(const sc_conv_config *cfg, int act_dtype, const C2SForms &f)
{
    if (!mfma_shape_ok(cfg, act_dtype) || cfg->groups != 1) return false;
    if (f.scatter)
        return act_dtype != SC_DTYPE_F32 && (f.scatter_ch == 64 || f.scatter_ch == 128);
    return cfg->out_channels_per_group <= kBN;
}

// dense: the linear layer (a 1x1x1 kernel without a map: query row r reads
// input row r).
static int conv_forward_impl(const sc_conv_config *cfg, int act_dtype, const void *d_input,
                             int64_t n_in, const int32_t *d_map, int64_t n_q, int w_dtype,
                             const void *d_weight, const float *d_w_scale, const float *d_bias,
                             const sc_conv_epilogue *epi, int out_dtype, void *d_out,
                             const void *d_plan, const void *d_wpack, sc_stream stream, bool dense = false,
                             bool child_plan = false)
{
    clear_error();
    const void *d_residual = epi ? epi->residual : nullptr;
    int rc = validate_config(cfg);
    if (rc) return rc;
    if (n_in < 0 || n_q < 0) return fail(SC_ERR_SHAPE, "negative row count");
    if (n_q > n_in)
        return fail(SC_ERR_SHAPE, "sparse conv neighbor row count exceeds input rows: got " +
                                      std::to_string(n_q) + " input rows " + std::to_string(n_in));
    const bool act_bf16 = act_dtype == SC_DTYPE_BF16, act_f32 = act_dtype == SC_DTYPE_F32,
               act_f16 = act_dtype == SC_DTYPE_F16;
    if (!(act_bf16 || act_f32 || act_f16))
        return fail(SC_ERR_DTYPE, "sparse conv input dtype must be f32, bf16 or f16");
    if (act_f32 && w_dtype != SC_DTYPE_F32)
        return fail(SC_ERR_DTYPE, "sparse conv f32 input needs f32 weights");
    if (act_bf16 && w_dtype != SC_DTYPE_BF16 && w_dtype != SC_DTYPE_I8)
        return fail(SC_ERR_DTYPE, "sparse conv bf16 input needs bf16 or int8 weights");
    if (act_f16 && w_dtype != SC_DTYPE_F16)
        return fail(SC_ERR_DTYPE, "sparse conv f16 input needs f16 weights");
    if (act_f16 ? (out_dtype != SC_DTYPE_F32 && out_dtype != SC_DTYPE_F16)
                : (out_dtype != SC_DTYPE_F32 && out_dtype != SC_DTYPE_BF16))
        return fail(SC_ERR_DTYPE, "sparse conv output dtype must be f32 or the input's 16-bit type");
    if (w_dtype == SC_DTYPE_I8 && !d_w_scale)
        return fail(SC_ERR_NULL, "int8 weights need per-output-channel scales");
    const int64_t K = cfg->kernel_d * cfg->kernel_h * cfg->kernel_w;
    int64_t t;
    if (!mul_ok(n_q, K, &t) || !mul_ok(n_q, cfg->out_channels, &t) ||
        !mul_ok(n_in, cfg->in_channels, &t) || !mul_ok(cfg->out_channels, K, &t) ||
        !mul_ok(t, cfg->in_channels_per_group, &t))
        return fail(SC_ERR_OVERFLOW, "sparse conv size overflow");
    if (cfg->in_channels_per_group > INT32_MAX || cfg->out_channels_per_group > INT32_MAX)
        return fail(SC_ERR_OVERFLOW, "sparse conv channel count overflow");
    C2SForms c2s;
    rc = c2s_forms(cfg, epi, c2s);
    if (rc) return rc;
    if (n_q == 0) return SC_OK;
    // A child scatter with no active child writes nothing (the reference's
    // select of an empty index); its output may be an empty (NULL) buffer.
    if (c2s.scatter && c2s.scatter_n == 0) return SC_OK;
    if (!d_input || (!d_map && !dense) || !d_weight || !d_out) return fail(SC_ERR_NULL, "sparse conv: NULL pointer");

    ConvArgs a;
    a.input = d_input;
    a.map = d_map;
    a.weight = d_weight;
    a.w_scale = d_w_scale;
    a.bias = d_bias;
    a.residual = d_residual;
    a.out = d_out;
    a.n_q = n_q;
    a.n_in = n_in;
    a.cin = cfg->in_channels;
    a.cout = cfg->out_channels;
    a.cin_g = (int)cfg->in_channels_per_group;
    a.cout_g = (int)cfg->out_channels_per_group;
    a.K = (int)K;
    a.ln = 0;
    a.ln_w = a.ln_b = nullptr;
    a.ln_eps = 0.f;
    a.silu = 0;
    a.perm = nullptr;
    a.wpack = d_wpack;
    a.plan_hdr = nullptr;
    a.ln_group = (int)cfg->out_channels_per_group;
    a.scatter_rows = c2s.scatter ? epi->child_rows : nullptr;
    a.scatter_n = c2s.scatter_n;
    a.scatter_ch = (int)c2s.scatter_ch;
    a.skip_parent = c2s.skip ? epi->skip_parent : nullptr;
    a.skip_idx = c2s.skip ? epi->skip_index : nullptr;
    a.skip_parent_rows = c2s.skip ? epi->skip_parent_rows : 0;
    a.skip_parent_ch = c2s.skip ? epi->skip_parent_channels : 0;
    a.skip_S = (int)c2s.skip_S;
    a.skip_R = (int)c2s.skip_R;
    auto log2_or_neg = [](int64_t v) {
        if (v <= 0 || (v & (v - 1)) != 0) return -1;
        int sh = 0;
        while (((int64_t)1 << sh) < v) ++sh;
        return sh;
    };
    a.scatter_shift = log2_or_neg(c2s.scatter_ch);
    a.skip_shift = log2_or_neg(c2s.skip_R);
    a.tile_child = nullptr;
    a.child_ch = (int)c2s.scatter_ch;
    a.child_plan = child_plan ? 1 : 0;
    if (c2s.scatter) a.ln_group = a.scatter_ch;

    const size_t asz = dtype_size(act_dtype);
    const uintptr_t align = (uintptr_t)d_input | (uintptr_t)d_weight | (uintptr_t)d_map;
    const int64_t in_bytes = n_in * cfg->in_channels * (int64_t)asz;
    const int64_t w_bytes = cfg->out_channels * K * cfg->in_channels_per_group * (int64_t)dtype_size(w_dtype);
    const bool mfma = mfma_shape_ok(cfg, act_dtype) && (align % 16 == 0) && in_bytes < (int64_t)1 << 31 &&
                      w_bytes < (int64_t)1 << 31;
    const int groups = (int)cfg->groups;
    hipStream_t s = as_stream(stream);
    const bool want_ln = epi && epi->layer_norm, want_silu = epi && epi->silu;
    // LayerNorm needs every channel of a row in one workgroup: it is fused
    // into the MFMA tile's epilogue when groups == 1 and Cout <= 128.  SiLU
    // without LayerNorm and the residual are per element and fuse into every
    // conv kernel.  Otherwise the conv stores its f32 accumulators (into
    // d_out for an f32 output, else into the caller's workspace) and one row
    // kernel applies LayerNorm -> SiLU -> + residual and rounds once.
    const bool row_fuse = mfma && ln_in_tile(cfg, act_dtype, c2s);
    const bool split_ln = want_ln && !row_fuse;
    if (split_ln && c2s.skip)
        return fail(SC_ERR_UNSUPPORTED, "sparse conv: LayerNorm before the parent skip needs the row in one tile");
    // rows and channels the row kernel normalises (the children in a scatter)
    const int64_t ln_rows = c2s.scatter ? c2s.scatter_n : n_q;
    const int64_t ln_ch = c2s.scatter ? c2s.scatter_ch : cfg->out_channels;
    void *conv_out = d_out;
    int conv_out_dtype = out_dtype;
    if (!split_ln) {
        a.ln = want_ln;
        a.ln_w = want_ln ? epi->ln_weight : nullptr;
        a.ln_b = want_ln ? epi->ln_bias : nullptr;
        a.ln_eps = want_ln ? epi->ln_eps : 0.f;
        a.silu = want_silu;
    } else {
        a.residual = nullptr;
        if (out_dtype != SC_DTYPE_F32) {
            int64_t need;
            if (!mul_ok(ln_rows, ln_ch, &need) || !mul_ok(need, 4, &need))
                return fail(SC_ERR_OVERFLOW, "sparse conv size overflow");
            if (!epi->workspace || epi->workspace_bytes < (size_t)need)
                return fail(SC_ERR_WORKSPACE,
                            "sparse conv: LayerNorm over " + std::to_string(ln_ch) +
                                " channels cannot run in the conv tile; a bf16 output then needs an f32 "
                                "workspace of " + std::to_string(need) + " bytes (sc_conv_epilogue_workspace_size)");
            if ((uintptr_t)epi->workspace % 16 != 0)
                return fail(SC_ERR_WORKSPACE, "sparse conv epilogue workspace must be 16-byte aligned");
            conv_out = epi->workspace;
            conv_out_dtype = SC_DTYPE_F32;
        }
    }
    a.out = conv_out;
    a.vec_out = (a.cout_g % 4 == 0) && (a.cout % 4 == 0) && ((uintptr_t)conv_out % 16 == 0) &&
                ((uintptr_t)a.residual % 16 == 0) && (a.scatter_ch % 4 == 0);
    // The halo-staged path (bf16 activations, up to 27 offsets) reads the
    // plan; other shapes ignore it.
    if (d_plan && (uintptr_t)d_plan % 256 != 0)
        return fail(SC_ERR_WORKSPACE, "conv plan must be 256-byte aligned");
    if (d_wpack && (uintptr_t)d_wpack % 16 != 0)
        return fail(SC_ERR_SHAPE, "packed weights must be 16-byte aligned");
    const void *plan = (d_plan && (act_bf16 || act_f16) && mfma && K <= kHaloK) ? d_plan : nullptr;
    if (child_plan && !dense) {
        // a child plan's tiles hold parents, not query rows: only the
        // halo-staged kernel on packed weights can run it
        if (!plan || !d_wpack || groups != 1)
            return fail(SC_ERR_UNSUPPORTED, "sparse conv child plan needs 16-bit activations, packed weights, "
                                            "one group and a kernel of at most 27 offsets");
    }
    if (child_plan && dense) {
        // a linear child plan: only the dense MFMA tile on 16-bit weights runs it
        if (!plan || w_dtype == SC_DTYPE_I8 || cfg->in_channels % 32 != 0 || c2s.scatter_ch % 128 != 0)
            return fail(SC_ERR_UNSUPPORTED, "linear child plan needs 16-bit activations and weights, input channels "
                                            "a multiple of 32 and children of a multiple of 128 channels");
    }
    int rc2 = launch_conv_typed(a, act_f32, w_dtype, conv_out_dtype, groups, mfma, plan, s);
    if (rc2 != SC_OK || !split_ln) return rc2;
    // After a planned conv, the row kernel is gated on the plan's status: a
    // conv that found a mismatch stored nothing to normalise, and nothing
    // may reach d_out.
    // With the child scatter, rows at or past the device child count (when
    // given) were never written: the row kernel stops there.
    return layer_norm_rows(SC_DTYPE_F32, conv_out, ln_rows, ln_ch, epi->ln_weight, epi->ln_bias, epi->ln_eps,
                           want_silu, out_dtype, d_residual, d_out, s,
                           plan ? &static_cast<const PlanHeader *>(plan)->status : nullptr,
                           c2s.scatter ? epi->child_count : nullptr);
}


extern "C" int sc_subm_conv_forward(const sc_conv_config *cfg, int act_dtype, const void *d_input,
                                    int64_t n_in, const int32_t *d_map, int64_t n_q, int w_dtype,
                                    const void *d_weight, const float *d_w_scale,
                                    const float *d_bias, const void *d_residual, int out_dtype,
                                    void *d_out, sc_stream stream)
{
    sc_conv_epilogue epi{};
    epi.residual = d_residual;
    return conv_forward_impl(cfg, act_dtype, d_input, n_in, d_map, n_q, w_dtype, d_weight, d_w_scale,
                             d_bias, &epi, out_dtype, d_out, nullptr, nullptr, stream);
}

extern "C" int sc_subm_conv_forward_fused(const sc_conv_config *cfg, int act_dtype,
                                          const void *d_input, int64_t n_in, const int32_t *d_map,
                                          int64_t n_q, int w_dtype, const void *d_weight,
                                          const float *d_w_scale, const float *d_bias,
                                          const sc_conv_epilogue *epi, int out_dtype, void *d_out,
                                          sc_stream stream)
{
    return conv_forward_impl(cfg, act_dtype, d_input, n_in, d_map, n_q, w_dtype, d_weight, d_w_scale,
                             d_bias, epi, out_dtype, d_out, nullptr, nullptr, stream);
}

extern "C" int sc_linear_forward(int act_dtype, const void *d_input, int64_t rows, int64_t in_channels,
                                 int64_t out_channels, int w_dtype, const void *d_weight, const float *d_w_scale,
                                 const float *d_bias, const sc_conv_epilogue *epi, int out_dtype, void *d_out,
                                 sc_stream stream)
{
    clear_error();
    if (epi && epi->skip_index)
        return fail(SC_ERR_UNSUPPORTED, "linear: the parent skip belongs to the sparse conv");
    sc_conv_config c{};
    c.in_channels = in_channels;
    c.out_channels = out_channels;
    c.kernel_d = c.kernel_h = c.kernel_w = 1;
    c.in_channels_per_group = in_channels;
    c.out_channels_per_group = out_channels;
    c.groups = 1;
    c.axis_order[0] = 0;
    c.axis_order[1] = 1;
    c.axis_order[2] = 2;
    c.axis_sign[0] = c.axis_sign[1] = c.axis_sign[2] = 1;
    return conv_forward_impl(&c, act_dtype, d_input, rows, nullptr, rows, w_dtype, d_weight, d_w_scale, d_bias,
                             epi, out_dtype, d_out, nullptr, nullptr, stream, true);
}

extern "C" int sc_linear_forward_child_planned(int act_dtype, const void *d_input, int64_t rows,
                                               int64_t in_channels, int64_t out_channels, int w_dtype,
                                               const void *d_weight, const float *d_w_scale, const float *d_bias,
                                               const sc_conv_epilogue *epi, int out_dtype, void *d_out,
                                               const void *d_child_plan, sc_stream stream)
{
    clear_error();
    if (!epi || !epi->child_rows)
        return fail(SC_ERR_NULL, "linear child plan: the epilogue's child_rows (the child scatter) is required");
    if (epi->skip_index)
        return fail(SC_ERR_UNSUPPORTED, "linear: the parent skip belongs to the sparse conv");
    if (!d_child_plan) return fail(SC_ERR_NULL, "linear child plan: NULL plan");
    if ((uintptr_t)d_child_plan % 256 != 0) return fail(SC_ERR_WORKSPACE, "conv plans must be 256-byte aligned");
    sc_conv_config c{};
    c.in_channels = in_channels;
    c.out_channels = out_channels;
    c.kernel_d = c.kernel_h = c.kernel_w = 1;
    c.in_channels_per_group = in_channels;
    c.out_channels_per_group = out_channels;
    c.groups = 1;
    c.axis_order[0] = 0;
    c.axis_order[1] = 1;
    c.axis_order[2] = 2;
    c.axis_sign[0] = c.axis_sign[1] = c.axis_sign[2] = 1;
    return conv_forward_impl(&c, act_dtype, d_input, rows, nullptr, rows, w_dtype, d_weight, d_w_scale, d_bias,
                             epi, out_dtype, d_out, d_child_plan, nullptr, stream, true, true);
}

extern "C" int sc_subm_conv_forward_planned(const sc_conv_config *cfg, int act_dtype,
                                            const void *d_input, int64_t n_in, const int32_t *d_map,
                                            int64_t n_q, int w_dtype, const void *d_weight,
                                            const void *d_packed_weight, const float *d_w_scale,
                                            const float *d_bias, const sc_conv_epilogue *epi,
                                            int out_dtype, void *d_out, const void *d_plan,
                                            sc_stream stream)
{
    return conv_forward_impl(cfg, act_dtype, d_input, n_in, d_map, n_q, w_dtype, d_weight, d_w_scale,
                             d_bias, epi, out_dtype, d_out, d_plan, d_packed_weight, stream);
}

extern "C" int sc_subm_conv_forward_child_planned(const sc_conv_config *cfg, int act_dtype,
                                                  const void *d_input, int64_t n_in, const int32_t *d_map,
                                                  int64_t n_q, int w_dtype, const void *d_weight,
                                                  const void *d_packed_weight, const float *d_w_scale,
                                                  const float *d_bias, const sc_conv_epilogue *epi,
                                                  int out_dtype, void *d_out, const void *d_child_plan,
                                                  sc_stream stream)
{
    clear_error();
    if (!epi || !epi->child_rows)
        return fail(SC_ERR_NULL, "sparse conv child plan: the epilogue's child_rows (the child scatter) is required");
    if (!d_child_plan || !d_packed_weight) return fail(SC_ERR_NULL, "sparse conv child plan: NULL plan or weights");
    // children of 64 channels or a multiple of 128: the halo tiles then cover
    // one child each
    if (cfg && cfg->out_channels != 512 && cfg->out_channels % 1024 != 0)
        return fail(SC_ERR_UNSUPPORTED, "sparse conv child plan needs children of 64 channels or a multiple of 128 "
                                        "(Cout 512 or a multiple of 1024)");
    return conv_forward_impl(cfg, act_dtype, d_input, n_in, d_map, n_q, w_dtype, d_weight, d_w_scale, d_bias, epi,
                             out_dtype, d_out, d_child_plan, d_packed_weight, stream, false, true);
}

static int weight_pack_bytes(const sc_conv_config *cfg, int w_dtype, size_t *bytes)
{
    int rc = validate_config(cfg);
    if (rc) return rc;
    if (w_dtype != SC_DTYPE_BF16 && w_dtype != SC_DTYPE_I8 && w_dtype != SC_DTYPE_F16)
        return fail(SC_ERR_DTYPE, "weight packing takes bf16, f16 or int8 weights");
    if (cfg->in_channels_per_group % 32 != 0)
        return fail(SC_ERR_UNSUPPORTED, "weight packing needs input channels per group divisible by 32");
    const int64_t K = cfg->kernel_d * cfg->kernel_h * cfg->kernel_w;
    const int64_t n_ot = (cfg->out_channels_per_group + kBN - 1) / kBN;
    const long double b = (long double)cfg->groups * n_ot * kBN * K * cfg->in_channels_per_group * 2.0L;
    if (b >= (long double)((int64_t)1 << 31))
        return fail(SC_ERR_OVERFLOW, "packed weights must stay below 2 GiB");
    *bytes = (size_t)b + kPackHeaderBytes;
    return SC_OK;
}

extern "C" int sc_conv_weight_pack_size(const sc_conv_config *cfg, int w_dtype, size_t *bytes)
{
    clear_error();
    if (!bytes) return fail(SC_ERR_NULL, "bytes out-pointer is NULL");
    return weight_pack_bytes(cfg, w_dtype, bytes);
}

extern "C" int sc_conv_weight_pack(const sc_conv_config *cfg, int w_dtype, const void *d_weight,
                                   void *d_packed, sc_stream stream)
{
    clear_error();
    size_t bytes = 0;
    int rc = weight_pack_bytes(cfg, w_dtype, &bytes);
    if (rc) return rc;
    if (!d_packed) return fail(SC_ERR_NULL, "weight packing: NULL pointer");
    if (bytes > kPackHeaderBytes && !d_weight) return fail(SC_ERR_NULL, "weight packing: NULL pointer");
    if ((uintptr_t)d_packed % 16 != 0) return fail(SC_ERR_SHAPE, "packed weights must be 16-byte aligned");
    const int groups = (int)cfg->groups, cout_g = (int)cfg->out_channels_per_group,
              cin_g = (int)cfg->in_channels_per_group;
    const int K = (int)(cfg->kernel_d * cfg->kernel_h * cfg->kernel_w);
    const int64_t pieces = (int64_t)((bytes - kPackHeaderBytes) / 16);  // 8 bf16 per lane and fragment
    hipStream_t s = as_stream(stream);
    unsigned char *buf = static_cast<unsigned char *>(d_packed);
    if (w_dtype == SC_DTYPE_F16)
        pack_weights_kernel<_Float16><<<grid_for(pieces, 256, 16384), 256, 0, s>>>(
            static_cast<const _Float16 *>(d_weight), buf, groups, cout_g, cin_g, K, w_dtype, (int64_t)bytes);
    else if (w_dtype == SC_DTYPE_BF16)
        pack_weights_kernel<uint16_t><<<grid_for(pieces, 256, 16384), 256, 0, s>>>(
            static_cast<const uint16_t *>(d_weight), buf, groups, cout_g, cin_g, K, w_dtype, (int64_t)bytes);
    else
        pack_weights_kernel<int8_t><<<grid_for(pieces, 256, 16384), 256, 0, s>>>(
            static_cast<const int8_t *>(d_weight), buf, groups, cout_g, cin_g, K, w_dtype, (int64_t)bytes);
    SC_LAUNCH_CHECK("pack_weights_kernel launch");
    return SC_OK;
}

extern "C" int sc_conv_plan_check(const void *d_plan, sc_stream stream)
{
    clear_error();
    if (!d_plan) return fail(SC_ERR_NULL, "conv plan buffer is NULL");
    hipStream_t s = as_stream(stream);
    uint32_t status = 0;
    SC_HIP_CHECK(hipMemcpyAsync(&status, &static_cast<const PlanHeader *>(d_plan)->status, sizeof(status),
                                hipMemcpyDeviceToHost, s),
                 "conv plan status readback");
    SC_HIP_CHECK(hipStreamSynchronize(s), "conv plan status sync");
    if (status & kPlanStatusMapMismatch)
        return fail(SC_ERR_SHAPE, "sparse conv: the conv plan was built for another map (n_q, n_in or K differ); "
                                  "the conv wrote nothing");
    if (status & kPlanStatusWeightMismatch)
        return fail(SC_ERR_SHAPE, "sparse conv: the packed weights were packed for another config; "
                                  "the conv wrote nothing");
    if (status & kPlanStatusChildRows)
        return fail(SC_ERR_SHAPE, "child plan: the parent plan was built for another row count, or the child "
                                  "rows name more active children than n_children; the plan is empty");
    return SC_OK;
}

extern "C" int sc_conv_epilogue_workspace_size(const sc_conv_config *cfg, int act_dtype, int64_t n_q,
                                               int out_dtype, const sc_conv_epilogue *epi, size_t *bytes)
{
    clear_error();
    if (!bytes) return fail(SC_ERR_NULL, "bytes out-pointer is NULL");
    int rc = validate_config(cfg);
    if (rc) return rc;
    if (n_q < 0) return fail(SC_ERR_SHAPE, "negative row count");
    if (act_dtype != SC_DTYPE_F32 && act_dtype != SC_DTYPE_BF16 && act_dtype != SC_DTYPE_F16)
        return fail(SC_ERR_DTYPE, "sparse conv input dtype must be f32, bf16 or f16");
    *bytes = 0;
    C2SForms c2s;
    rc = c2s_forms(cfg, epi, c2s);
    if (rc) return rc;
    if (epi && epi->layer_norm && out_dtype != SC_DTYPE_F32 && !ln_in_tile(cfg, act_dtype, c2s)) {
        int64_t need;
        if (!mul_ok(c2s.scatter ? c2s.scatter_n : n_q, c2s.scatter ? c2s.scatter_ch : cfg->out_channels, &need) ||
            !mul_ok(need, 4, &need))
            return fail(SC_ERR_OVERFLOW, "sparse conv size overflow");
        *bytes = (size_t)need;
    }
    return SC_OK;
}
