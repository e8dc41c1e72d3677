// f16 instantiations of the submanifold conv kernels (sc_conv_kernels.hpp):
// f16 activations and weights with f32 accumulation on
// v_mfma_f32_16x16x32_f16, output f16 or f32 -- the decoder's compute_fp16
// mode (sparse_decoder_runtime_impl.rs:195,219-221), where the reference
// computes in f32 on f16-rounded operands (f16 x f16 products are exact in
// f32).  A translation unit of its own so that both halves of the conv
// compile in parallel.
#include "sc_conv_kernels.hpp"

namespace sc {

int launch_conv_f16(const ConvArgs &a, int out_dtype, int groups, bool mfma, const void *plan, hipStream_t s)
{
    if (out_dtype == SC_DTYPE_F32) return launch_conv<_Float16, _Float16, float>(a, groups, mfma, plan, s);
    return launch_conv<_Float16, _Float16, _Float16>(a, groups, mfma, plan, s);
}

}  // namespace sc
