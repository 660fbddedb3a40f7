// Kernel instances, part 2a: bf16 tiles and skinny kernels, bf16 output.
#include "gemm_registry.h"

namespace aiter_amd {

#include "gemm_reg_bf16.inc"

template void RegBuilder::part_bf16<false>();

}  // namespace aiter_amd
