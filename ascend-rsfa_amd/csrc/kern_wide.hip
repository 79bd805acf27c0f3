// Instantiations of the one-wave-per-SIMD forward kernel (fa_fwd_wide.hpp):
// head dim 128, non-causal, fp16 and bf16 (a float8 V at head dim 128 is read
// as bytes, which only fa_fwd_kernel's TypeF16V8 tiles do).
//
// Built with -mllvm -amdgpu-mfma-vgpr-form=1 (build_native.py): with 512
// registers per wave the compiler would otherwise give every MFMA an AGPR
// accumulator, and the softmax would copy each score out of the AGPRs; in the
// VGPR form O, S and P stay in VGPRs and the register allocator places the
// Q^T operands (read only by MFMAs) in AGPRs.
#include "fa_fwd_wide.hpp"
#include "kernel_table.hpp"

using namespace rsfa;

// (BN, LDS ring of tiles); overridable for sweeps
#ifndef RSFA_WIDE_TILES
#define RSFA_WIDE_TILES(T, DTYPE) RSFA_WIDE_ENTRY(T, DTYPE, 128, 32, 8, 1)
#endif

#if RSFA_WIDE
RSFA_DEFINE_KERNEL_LIST(kernels_wide, RSFA_WIDE_TILES(TypeF16, 0), RSFA_WIDE_TILES(TypeBF16, 1))
#else
namespace rsfa {
KernelList kernels_wide() { return KernelList{nullptr, 0}; }
}
#endif
