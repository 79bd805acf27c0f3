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
    int bm;      // BLOCK_M: query rows per workgroup (32 * nw, or 64 * nw for wide)
    int wide;    // fa_fwd_wide_kernel: its 32-row blocks per wave (1 or 2), 0 for fa_fwd_kernel
    int nbuf;
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
KernelList kernels_wide();

}  // namespace rsfa

// One tile configuration: non-causal fused, causal fused, causal prefix, causal diagonal.
#define RSFA_TILE_ENTRIES(T, DTYPE, D, BN, NW, OCC)                                                  \
    {DTYPE, D, BN, NW, 0, MODE_FUSED, OCC, uses_pingpong(D, BN, NW, false, MODE_FUSED),                   \
     (const void*)&fa_fwd_kernel<T, D, BN, NW, false, MODE_FUSED, OCC>, 32 * NW, 0, 0},                   \
    {DTYPE, D, BN, NW, 1, MODE_FUSED, OCC, uses_pingpong(D, BN, NW, true, MODE_FUSED),                    \
     (const void*)&fa_fwd_kernel<T, D, BN, NW, true, MODE_FUSED, OCC>, 32 * NW, 0, 0},                    \
    {DTYPE, D, BN, NW, 1, MODE_PREFIX, OCC, 0, (const void*)&fa_fwd_kernel<T, D, BN, NW, true, MODE_PREFIX, OCC>, \
     32 * NW, 0, 0},                                                                                      \
    {DTYPE, D, BN, NW, 1, MODE_DIAG, OCC, 0, (const void*)&fa_fwd_kernel<T, D, BN, NW, true, MODE_DIAG, OCC>, \
     32 * NW, 0, 0}

// The software-pipelined kernel (non-causal), BLOCK_M 256: RB = 2 runs 4 waves
// of 64 rows (one per SIMD), RB = 1 runs 8 waves of 32 rows (two per SIMD).
#define RSFA_WIDE_ENTRY(T, DTYPE, D, BN, NBUF, RB) \
    {DTYPE, D, BN, 8 / RB, 0, MODE_FUSED, 3 - RB, 0, (const void*)&fa_fwd_wide_kernel<T, D, BN, NBUF, RB>, 256, RB, NBUF}

#define RSFA_DEFINE_KERNEL_LIST(NAME, ...)                                   \
    namespace rsfa {                                                         \
    static const KernelEntry NAME##_table[] = {__VA_ARGS__};                 \
    KernelList NAME() {                                                      \
        return KernelList{NAME##_table, (int)(sizeof(NAME##_table) / sizeof(NAME##_table[0]))}; \
    }                                                                        \
    }
