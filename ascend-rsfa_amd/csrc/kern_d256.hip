// Instantiations of the forward kernel for head dim 256 (fp16, bf16, and fp16 with a float8 e5m2 V).
#include "fa_fwd_kernel.hpp"
#include "kernel_table.hpp"

using namespace rsfa;

// (BN, NW, OCC) of the compiled tile shapes; overridable for tile sweeps.
#ifndef RSFA_D256_TILES
#define RSFA_D256_TILES(T, DTYPE) RSFA_TILE_ENTRIES(T, DTYPE, 256, 32, 8, 2), RSFA_TILE_ENTRIES(T, DTYPE, 256, 32, 4, 2)
#endif

// float8 V at head dim 256: V's bytes go into LDS as they are (TypeF16V8);
// each 32-key tile's P.V is one 64-key float8 MFMA with P = 0 for its upper
// half.  Its 4-wave tile is built for one wave per SIMD: the 8-register
// operands of the float8 MFMA do not fit beside O^T and Q^T in the 256
// VGPRs of two waves per SIMD without spills inside the key loop.
#ifndef RSFA_D256_V8_TILES
#define RSFA_D256_V8_TILES(T, DTYPE) RSFA_TILE_ENTRIES(T, DTYPE, 256, 32, 8, 2), RSFA_TILE_ENTRIES(T, DTYPE, 256, 32, 4, 1)
#endif

RSFA_DEFINE_KERNEL_LIST(kernels_d256, RSFA_D256_TILES(TypeF16, 0), RSFA_D256_TILES(TypeBF16, 1),
                        RSFA_D256_V8_TILES(TypeF16V8, 2))
