// Registry of the compiled kernel instantiations.  Each kern_d*.hip unit
// instantiates fa_fwd_kernel for one head dim and lists the results here; the
// launcher (rsfa_api.hip) dispatches on (dtype, head dim, tile, causal, mode).
#pragma once

#include <stdint.h>

namespace rsfa {

struct KernelEntry {
    int dtype;   // rsfa_dtype
    int d;       // head dim
    int bn;      // keys per LDS tile (BLOCK_N)
    int nw;      // waves per workgroup; BLOCK_M = 32 * nw
    int causal;  // 0 / 1
    int mode;    // MODE_FUSED / MODE_PREFIX / MODE_DIAG
    int occ;     // waves per SIMD the kernel was register-budgeted for
    int pp;      // 1: ping-pong schedule (three K/V buffers)
    const void* fn;
    int bm;      // BLOCK_M: query rows per workgroup (32 * nw)
};

struct KernelList {
    const KernelEntry* entries;
    int count;
};

KernelList kernels_d16();
KernelList kernels_d32();
KernelList kernels_d64();
KernelList kernels_d128();
KernelList kernels_d256();

}  // namespace rsfa

// One tile configuration: non-causal fused, causal fused, causal prefix, causal diagonal.
#define RSFA_TILE_ENTRIES(T, DTYPE, D, BN, NW, OCC)                                                  \
    {DTYPE, D, BN, NW, 0, MODE_FUSED, OCC, uses_pingpong(D, BN, NW, false, MODE_FUSED),                   \
     (const void*)&fa_fwd_kernel<T, D, BN, NW, false, MODE_FUSED, OCC>, 32 * NW},                         \
    {DTYPE, D, BN, NW, 1, MODE_FUSED, OCC, uses_pingpong(D, BN, NW, true, MODE_FUSED),                    \
     (const void*)&fa_fwd_kernel<T, D, BN, NW, true, MODE_FUSED, OCC>, 32 * NW},                          \
    {DTYPE, D, BN, NW, 1, MODE_PREFIX, OCC, 0, (const void*)&fa_fwd_kernel<T, D, BN, NW, true, MODE_PREFIX, OCC>, \
     32 * NW},                                                                                            \
    {DTYPE, D, BN, NW, 1, MODE_DIAG, OCC, 0, (const void*)&fa_fwd_kernel<T, D, BN, NW, true, MODE_DIAG, OCC>, \
     32 * NW}


#define RSFA_DEFINE_KERNEL_LIST(NAME, ...)                                   \
    namespace rsfa {                                                         \
    static const KernelEntry NAME##_table[] = {__VA_ARGS__};                 \
    KernelList NAME() {                                                      \
        return KernelList{NAME##_table, (int)(sizeof(NAME##_table) / sizeof(NAME##_table[0]))}; \
    }                                                                        \
    }
