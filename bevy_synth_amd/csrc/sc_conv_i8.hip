// int8-weight instantiations of the submanifold conv kernels
// (sc_conv_kernels.hpp): bf16 activations, per-output-channel symmetric int8
// weights (W8A16; scales applied in the epilogue), output bf16 or f32.  A
// translation unit of its own so that the conv's forms compile in parallel.
#include "sc_conv_kernels.hpp"

namespace sc {

int launch_conv_i8(const ConvArgs &a, int out_dtype, int groups, bool mfma, const void *plan, hipStream_t s)
{
    if (out_dtype == SC_DTYPE_F32) return launch_conv<uint16_t, int8_t, float>(a, groups, mfma, plan, s);
    return launch_conv<uint16_t, int8_t, uint16_t>(a, groups, mfma, plan, s);
}

}  // namespace sc
