// Instantiations of the forward kernel for head dim 16 (fp16 and bf16).
#include "fa_fwd_kernel.hpp"
#include "kernel_table.hpp"

using namespace rsfa;

RSFA_DEFINE_KERNEL_LIST(kernels_d16,
    RSFA_TILE_ENTRIES(TypeF16, 0, 16, 64, 4, 2), RSFA_TILE_ENTRIES(TypeBF16, 1, 16, 64, 4, 2))
