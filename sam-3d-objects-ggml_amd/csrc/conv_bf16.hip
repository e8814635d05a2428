// conv_bf16.hip -- instantiations of the sparse-conv kernel (conv_kernel.h)
// for one operand type, compiled as a separate unit to parallelise the build.
#include "conv_kernel.h"

namespace spc {

hipError_t conv_bf16(hipStream_t s, const ConvArgs& a) { return dispatch_conv<__bf16, false>(s, a); }

}  // namespace spc
