// Instantiations of the forward kernel for head dim 16 (fp16, bf16, and fp16 with a float8 e5m2 V).
#include "fa_fwd_kernel.hpp"
#include "kernel_table.hpp"

using namespace rsfa;

// (BN, NW, OCC) of the compiled tile shapes; overridable for tile sweeps.
#ifndef RSFA_D16_TILES
#define RSFA_D16_TILES(T, DTYPE) RSFA_TILE_ENTRIES(T, DTYPE, 16, 64, 4, 2)
#endif

RSFA_DEFINE_KERNEL_LIST(kernels_d16, RSFA_D16_TILES(TypeF16, 0), RSFA_D16_TILES(TypeBF16, 1),
                        RSFA_D16_TILES(TypeF16V8, 2))
