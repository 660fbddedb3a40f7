// Kernel instances, part 2b: bf16 tiles and skinny kernels, f32 output.
#include "gemm_registry.h"

namespace aiter_amd {

#include "gemm_reg_bf16.inc"

template void RegBuilder::part_bf16<true>();

}  // namespace aiter_amd
