// Instantiations of the forward kernel for head dim 64 (fp16, bf16, and fp16 with a float8 e5m2 V).
#include "fa_fwd_kernel.hpp"
#include "kernel_table.hpp"

using namespace rsfa;

// (BN, NW, OCC) of the compiled tile shapes; overridable for tile sweeps.
#ifndef RSFA_D64_TILES
#define RSFA_D64_TILES(T, DTYPE) RSFA_TILE_ENTRIES(T, DTYPE, 64, 128, 8, 2), RSFA_TILE_ENTRIES(T, DTYPE, 64, 64, 4, 2)
#endif

// float8 V: V's bytes go into LDS as they are (TypeF16V8)
RSFA_DEFINE_KERNEL_LIST(kernels_d64, RSFA_D64_TILES(TypeF16, 0), RSFA_D64_TILES(TypeBF16, 1),
                        RSFA_D64_TILES(TypeF16V8, 2))
