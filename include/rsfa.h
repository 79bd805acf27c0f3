/*
 * rsfa.h - C ABI of the MI355X (gfx950) FlashAttention-2 forward library.
 *
 * This is the only native boundary of the package.  The Python module
 * ascend_rsfa.flash_attention_forward binds it with ctypes; any other host
 * language can bind the same symbols (plain pointers, sizes and ints, no
 * torch or C++ types in any signature).
 *
 * Every entry point below replaces one piece of the reference operator
 * (Dell710000/ascend-rsfa, file ascend_rsfa/flash_attention_forward.py):
 *
 *   rsfa_attention_fwd        -> _attention.forward, lines 547-616, i.e. the
 *                                kernel launches at 565, 574, 599 and the causal
 *                                two-launch split _run_causal_split (493-541)
 *   rsfa_get_tiling           -> get_tiling(Z, H, N_CTX, HEAD_DIM, causal), 624-665
 *   rsfa_resolve_tiling       -> the (BLOCK_M, BLOCK_N) meta-parameters the
 *                                reference passes to _attn_fwd[grid] (518-519, 606-607)
 *   rsfa_get_num_compute_cores-> get_num_compute_cores(), 19-21
 *   rsfa_v8_workspace_bytes   -> (no counterpart: workspace a float8 V needs,
 *                                for the fp8_v branch of _attn_fwd_inner,
 *                                208-211; zero, the kernels read V's bytes;
 *                                kept so that callers of ABI version 5 link)
 *   rsfa_strerror             -> (no counterpart: the reference raises Python
 *                                exceptions; codes map to them in the wrapper)
 *
 * Conventions
 *   - All tensor pointers are device pointers owned by the caller; the library
 *     never frees them.  Strides are in elements.  The last (head-dim) stride
 *     of q/k/v/o must be 1, every other stride a multiple of 8 elements (16
 *     for a float8 V) and every base pointer 16-byte aligned.  The K and V
 *     row strides (and at D = 64 and 128 the Q row stride, whose rows the
 *     8-wave tiles load the same way) must also keep BLOCK_N rows inside
 *     4 GiB: ((BLOCK_N - 1) * row_stride + max(D, 32)) * 2 < 2^32 bytes for
 *     every tile the call could run (BLOCK_N <= 128: row strides below
 *     ~16.9 M elements always pass).  RSFA_E_ALIGN otherwise.
 *   - Work is enqueued asynchronously on `stream` (a hipStream_t, NULL = the
 *     null stream).  The call returns after the launch, not after completion.
 *   - Return codes: 0 on success, a negative rsfa_status otherwise.  Invalid
 *     arguments are rejected before anything is launched.
 */
#ifndef RSFA_H_
#define RSFA_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RSFA_ABI_VERSION 6

typedef enum rsfa_status {
    RSFA_OK          = 0,
    RSFA_E_NULL      = -1,  /* a required pointer is NULL                      */
    RSFA_E_SHAPE     = -2,  /* Z, H or N_CTX not >= 1, or too large             */
    RSFA_E_HEADDIM   = -3,  /* head_dim not in {16, 32, 64, 128, 256}           */
    RSFA_E_DTYPE     = -4,  /* dtype not one of rsfa_dtype                      */
    RSFA_E_TILE      = -5,  /* block_m/block_n invalid (see rsfa_resolve_tiling)*/
    RSFA_E_ALIGN     = -6,  /* stride / alignment contract violated             */
    RSFA_E_DEVICE    = -7,  /* HIP runtime error while querying or preparing    */
    RSFA_E_LAUNCH    = -8,  /* kernel launch failed                             */
    RSFA_E_ABI       = -9,  /* struct_size does not match this library          */
    RSFA_E_WORKSPACE = -10, /* split mode without a large enough workspace       */
    RSFA_E_SCRATCH   = -11  /* rsfa_attention_fwd_noalloc: the problem needs
                               more workspace than RSFA_NOALLOC_WORKSPACE_BYTES */
} rsfa_status;

typedef enum rsfa_dtype {
    RSFA_DTYPE_F16  = 0,         /* q, k, v, o float16                         */
    RSFA_DTYPE_BF16 = 1,         /* q, k, v, o bfloat16                        */
    RSFA_DTYPE_F16_V8E5M2 = 2    /* q, k, o float16; v float8 e5m2 (OCP: sign,
                                    5 exponent bits, bias 15, 2 mantissa bits).
                                    P is rounded to e5m2 for P.V and the row
                                    sums add the unrounded P, as the reference's
                                    fp8_v branch does (208-211, 217).  The
                                    kernels read V's bytes and run P.V on the
                                    e5m2 MFMA at every head dim (no
                                    workspace) */
} rsfa_dtype;

/* flags (bit set) */
#define RSFA_FLAG_STATIC_SCHEDULE 0x1u /* grid-stride task order instead of the
                                          dynamic atomic-ticket queue            */
#define RSFA_FLAG_CAUSAL_SPLIT    0x2u /* causal only: two launches, mask-free
                                          prefix then masked diagonal, with the
                                          (m, l, acc) state handed over in fp32
                                          through `workspace` (reference
                                          493-541)                              */
#define RSFA_FLAG_EXACT_TILE      0x4u /* a request (block_m, block_n) runs the
                                          compiled tile nearest to it: the
                                          default, kept for callers of ABI
                                          version 4; overrides TILE_HINT        */
#define RSFA_FLAG_TILE_HINT       0x8u /* a valid request is only checked, and
                                          the tile rsfa_get_tiling picks for
                                          the shape runs                        */
#define RSFA_FLAG_SINGLE_BLOCKS   0x10u /* causal: one query block per task
                                          instead of the pairs (nmb-1-i, i) the
                                          library uses when they fill whole
                                          rounds of the grid; same results,
                                          bit for bit (a scheduling knob)       */

typedef struct rsfa_fwd_args {
    uint32_t    struct_size;  /* = sizeof(rsfa_fwd_args)                        */
    int32_t     dtype;        /* rsfa_dtype of q, k, v and o                    */
    const void *q;            /* [Z, H, N_CTX, D]                               */
    const void *k;            /* [Z, H, N_CTX, D]                               */
    const void *v;            /* [Z, H, N_CTX, D]                               */
    void       *o;            /* [Z, H, N_CTX, D], same dtype as q              */
    float      *lse;          /* optional [Z, H, N_CTX] fp32, natural-log
                                 logsumexp of the scaled scores (the reference's
                                 M = m + ln(l), 400-403); NULL = not written    */
    void       *workspace;    /* split mode: the split state
                                 (rsfa_split_workspace_bytes)                  */
    uint64_t    workspace_bytes;
    int64_t     z, h, n_ctx, head_dim;
    int64_t     q_stride[4];  /* element strides of dims (Z, H, N_CTX, D)       */
    int64_t     k_stride[4];
    int64_t     v_stride[4];
    int64_t     o_stride[4];
    float       sm_scale;     /* multiplies q.k before the softmax              */
    int32_t     causal;       /* 0/1: key n visible to query m iff n <= m       */
    int32_t     block_m;      /* requested BLOCK_M; 0 (with block_n 0) = no
                                 request, the tile rsfa_get_tiling picks runs.
                                 A request is checked against the reference's
                                 rules (RSFA_E_TILE otherwise) and, like the
                                 reference's BLOCK_M/BLOCK_N meta-parameters,
                                 selects the tile: the compiled one nearest to
                                 it runs (rsfa_resolve_tiling), unless
                                 RSFA_FLAG_TILE_HINT.  Split mode sizes its
                                 workspace with the BLOCK_M that runs        */
    int32_t     block_n;      /* requested BLOCK_N (see block_m)                */
    uint32_t    flags;        /* RSFA_FLAG_*                                    */
} rsfa_fwd_args;

/* Fused FlashAttention-2 forward: o = softmax(q k^T * sm_scale [+ causal mask]) v.
 * Replaces _attention.forward (flash_attention_forward.py:547-616). */
int rsfa_attention_fwd(const rsfa_fwd_args *args, void *stream);

/* Workspace rsfa_attention_fwd_noalloc has for the split state (its fixed
 * per-device buffer holds 4 KiB of queue counters besides). */
#define RSFA_NOALLOC_WORKSPACE_BYTES (16u << 20)

/* rsfa_attention_fwd without any allocation.  It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, kernels and results as rsfa_attention_fwd, except that
 * `workspace`/`workspace_bytes` are ignored: the queue counters and the
 * workspace (the split state) live in one fixed
 * buffer per device, a static device array of RSFA_NOALLOC_WORKSPACE_BYTES
 * + 4 KiB that the device holds until the process ends.  Problems that need
 * more workspace fail with RSFA_E_SCRATCH before any device work.  The first
 * call on a device looks the buffer up (hipGetSymbolAddress); every call
 * clears its counters with a small kernel on `stream` first.  All calls on one
 * device share the buffer: calls that overlap in time on one device (other
 * streams, concurrent graph replays) race and must be serialised by the
 * caller. */
int rsfa_attention_fwd_noalloc(const rsfa_fwd_args *args, void *stream);

/* Bytes of fp32 workspace RSFA_FLAG_CAUSAL_SPLIT needs for this problem and
 * the BLOCK_M that runs (rsfa_resolve_tiling of the request, or
 * rsfa_get_tiling's without one / under RSFA_FLAG_TILE_HINT): state[2, Z, H,
 * NBM, BM] (row max in exp2 units, row sum), as the reference allocates at
 * 501, then the un-normalised accumulator [Z, H, NBM, BM, head_dim] in fp32,
 * which the reference instead rounds to the input dtype into O (353).
 * 0 for invalid sizes. */
uint64_t rsfa_split_workspace_bytes(int64_t z, int64_t h, int64_t n_ctx,
                                    int64_t head_dim, int32_t block_m);

/* Bytes of workspace a float8 V (RSFA_DTYPE_F16_V8E5M2) needs: 0 (the kernels
 * read the float8 bytes at every head dim).  ABI version 5 placed an fp16
 * copy of V at head dims 16 and 32 here, before the split state; version 6
 * has none, and the split state starts at the workspace's first byte. */
uint64_t rsfa_v8_workspace_bytes(int64_t z, int64_t h, int64_t n_ctx,
                                 int64_t head_dim);

/* Tile search for gfx950 (replaces the lookup table get_tiling, 624-665):
 * writes the (BLOCK_M, BLOCK_N) rsfa_attention_fwd runs for the shape on the
 * current device (planned for its CU count; for a 256-CU MI355X where no
 * device is visible).  Never fails for a valid shape. */
int rsfa_get_tiling(int64_t z, int64_t h, int64_t n_ctx, int64_t head_dim,
                    int32_t causal, int32_t dtype, int32_t *block_m,
                    int32_t *block_n);

/* Maps a caller-requested (BLOCK_M, BLOCK_N) to the compiled instantiation
 * a launch with that request runs (the nearest compiled tile; log distance
 * in BLOCK_M and BLOCK_N, ties to the larger BLOCK_N).
 * Requests follow the reference's rules (powers of two,
 * 16 <= BLOCK <= 512, BLOCK_M*BLOCK_N <= 65536, causal needs
 * BLOCK_N <= BLOCK_M, which the reference silently breaks on, see
 * benchmarks/run_correctness_test.py:24-25).  Returns RSFA_E_TILE otherwise. */
int rsfa_resolve_tiling(int64_t head_dim, int32_t causal, int32_t dtype,
                        int32_t req_block_m, int32_t req_block_n,
                        int32_t *block_m, int32_t *block_n);

/* Number of compute units of `device` (-1 = current device); replaces
 * get_num_compute_cores (19-21).  Negative rsfa_status on error. */
int rsfa_get_num_compute_cores(int device);

/* Static string for a status code. */
const char *rsfa_strerror(int status);

/* RSFA_ABI_VERSION the library was built with. */
int rsfa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* RSFA_H_ */
