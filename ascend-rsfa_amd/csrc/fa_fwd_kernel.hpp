// FlashAttention-2 forward for MI355X (gfx950 / CDNA4), hand-written HIP.
//
// Reference algorithm: Dell710000/ascend-rsfa ascend_rsfa/flash_attention_forward.py
//   _attn_fwd (271-404), _attn_fwd_inner (163-226), _attn_fwd_split_inner
//   (408-489), causal prefix/diagonal split (338-368, 493-541).
//
// Work decomposition
//   One task = (batch b, head h, query block mb) of BM = 32*NW query rows.
//   A workgroup of NW wave64s runs tasks from a persistent queue; wave w owns
//   the 32 query rows [mb*BM + 32w, +32).  K and V stream through LDS in tiles
//   of BN keys with direct global->LDS loads (global_load_lds_dwordx4): double
//   buffered in the one-phase body (tile j+1 arrives while tile j is computed),
//   triple buffered in the two-phase ping-pong schedule of 8-wave workgroups,
//   where one wave of each SIMD runs its MFMAs while the other runs its softmax.
//
// Contractions (v_mfma_f32_32x32x16_{f16,bf16}, fp32 accumulation)
//   S^T = K Q^T : A = K rows from LDS (ds_read_b128), B = Q^T kept in VGPRs for
//                 the whole task.  In the 32x32 accumulator layout lane l holds
//                 query column l%32 and keys 8*(r/4) + 4*(l/32) + r%4 in its 16
//                 registers r, so every query row lives in one lane pair
//                 (l, l^32): the row max needs one permlane32 swap, the row sum
//                 none until the end of the task.
//   O^T = V^T P^T : B = P^T converted in registers straight from the S^T
//                 accumulator (no LDS round trip); A = V^T read with the gfx950
//                 transposing LDS load ds_read_b64_tr_b16 from the same
//                 row-major V tile, with keys ordered to match P^T's registers.
//                 O^T's layout puts each query in one lane too, so the online
//                 softmax rescale is a per-lane multiply.
//
// Online softmax (exp2 domain, c = |sm_scale| * log2 e)
//   m_tile = c * rowmax(S); the running max is only moved when the tile max
//   exceeds it by more than RESCALE_SLACK (log2 units), so most tiles skip the
//   O rescale entirely (the reference's FA4-style skip, 466-487, uses slack 0;
//   any slack gives the same softmax, it only bounds P <= 2^slack).  P is
//   rounded to the input dtype before the PV product, as the reference does
//   (211, 456); the row sum adds the rounded values (v_dot2 with ones).
//
// LDS layout of one K or V tile (BN rows x DP cols, 2-byte elements)
//   rows are grouped in blocks of 16; inside a block the 16-byte chunk c of row
//   r sits at  c*256 + ((r%16) ^ (4*(c%4)))*16.  Each 256-byte chunk plane holds
//   16 rows, so a half-wave's 16-byte K reads and the 16-lane groups of the
//   transposing V reads both touch 64 distinct banks, and one wave's direct
//   load instruction fills 1 KB of consecutive LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace rsfa {

#define RSFA_LDS __attribute__((address_space(3)))
#define RSFA_GLOBAL __attribute__((address_space(1)))

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

// How far (in log2 units) the running row max may lag the true max before the
// accumulator is rescaled.  P = 2^(s*c - m) stays <= 2^15, inside the normal
// range of fp16 (65504), bf16 and e5m2 (57344) with the same relative
// precision as P <= 1; the final normalisation divides it out.  A larger
// slack means fewer rescales of O where the scores spread widely (sm_scale
// 0.5 at D = 128: +1.9 % over a slack of 8).
constexpr float RESCALE_SLACK = 15.0f;

struct TypeF16 {
    static constexpr bool v8 = false;  // V tiles in LDS as float8 bytes
    typedef _Float16 elem;
    typedef _Float16 velem;  // element of V in global memory
    typedef _Float16 x8 __attribute__((ext_vector_type(8)));
    typedef _Float16 x4 __attribute__((ext_vector_type(4)));
    typedef _Float16 x2 __attribute__((ext_vector_type(2)));
    typedef decltype(__builtin_amdgcn_ds_read_tr16_b64_v4f16(nullptr)) tr4;
    static __device__ __forceinline__ f32x16 mfma(x8 a, x8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ tr4 tr_read(const RSFA_LDS char* p) {
        return __builtin_amdgcn_ds_read_tr16_b64_v4f16((RSFA_LDS tr4*)p);
    }
    static __device__ __forceinline__ x2 cvt2(float a, float b) {
        return __builtin_convertvector((f32x2){a, b}, x2);
    }
    static __device__ __forceinline__ float dot2(x2 a, x2 b, float c) {
        return __builtin_amdgcn_fdot2(a, b, c, false);
    }
    static __device__ __forceinline__ x2 ones2() { return (x2){(elem)1.0f, (elem)1.0f}; }
};

struct TypeBF16 {
    static constexpr bool v8 = false;
    typedef __bf16 elem;
    typedef __bf16 velem;
    typedef __bf16 x8 __attribute__((ext_vector_type(8)));
    typedef __bf16 x4 __attribute__((ext_vector_type(4)));
    typedef __bf16 x2 __attribute__((ext_vector_type(2)));
    typedef decltype(__builtin_amdgcn_ds_read_tr16_b64_v4bf16(nullptr)) tr4;
    static __device__ __forceinline__ f32x16 mfma(x8 a, x8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ tr4 tr_read(const RSFA_LDS char* p) {
        return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((RSFA_LDS tr4*)p);
    }
    static __device__ __forceinline__ x2 cvt2(float a, float b) {
        return __builtin_convertvector((f32x2){a, b}, x2);
    }
    static __device__ __forceinline__ float dot2(x2 a, x2 b, float c) {
        return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
    }
    static __device__ __forceinline__ x2 ones2() { return (x2){(elem)1.0f, (elem)1.0f}; }
};

// fp16 Q, K, O with a float8 e5m2 V (reference flash_attention_forward.py:
// 208-211, 253-256, 453-456: when V is float8e5, P is cast to float8e5 for
// P.V, while the row sum l adds the unrounded P, 217 and 466).  V's tiles go
// into LDS as the e5m2 bytes themselves, P is rounded to e5m2 bytes, and P.V
// runs on the float8 MFMA (e5m2 x e5m2, 64 keys per MFMA, twice the fp16
// rate); its products are exact in fp32, and it accumulates in fp32.
struct TypeF16V8 : TypeF16 {
    static constexpr bool v8 = true;
    typedef uint8_t velem;
    static __device__ __forceinline__ f32x16 mfma8(i32x8 a, i32x8 b, f32x16 c) {
        // cbsz = blgp = 1: both operands bf8 (e5m2); no block scale
        return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 1, 1, 0, 0, 0, 0);
    }
};

// Kernel modes.  MODE_FUSED runs every key tile of a task in one launch (the
// causal prefix with the mask-free body, the diagonal with the masked body).
// MODE_PREFIX / MODE_DIAG are the reference's two-launch causal split
// (STAGE 4 / STAGE 5, flash_attention_forward.py:338-368).
enum { MODE_FUSED = 0, MODE_PREFIX = 1, MODE_DIAG = 2 };

struct FwdParams {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* lse;      // optional [Z*H, n_ctx]
    float* state;    // split mode: [2][Z*H*nmb*BM] (m, l) per query row
    float* acc;      // split mode: [Z*H*nmb*BM][D] un-normalised fp32 accumulator per query row
    int64_t q_sz, q_sh, q_sm;
    int64_t k_sz, k_sh, k_sn;
    int64_t v_sz, v_sh, v_sn;
    int64_t o_sz, o_sh, o_sm;
    int32_t H;
    int32_t n_ctx;
    int32_t nmb;        // query blocks per head = ceil(n_ctx / BM)
    int32_t num_heads;  // Z * H
    int32_t num_tasks;  // num_heads * nmb
    int32_t nq;         // task queues (1 or 8): queue x holds the heads bh % nq == x
    int32_t pairs;      // causal, fused mode: a ticket runs query blocks nmb-1-i and i
    float c;            // |sm_scale| * log2(e)
    uint32_t neg;       // 1 when sm_scale < 0: q is negated (exact) and c = |c|
    uint32_t* ticket;   // dynamic queue counters (nq of them, 16 words apart; each returns
                        // to 0 at kernel end) or null for the static schedule
};

// Queues.  Workgroups are dispatched to the 8 XCDs of an MI355X round robin,
// so workgroup b runs on XCD b % 8 and serves queue b % nq: with nq = 8 all
// query blocks of a head run on one XCD and its K/V are fetched into that
// XCD's L2 once, instead of once per XCD.
struct Queue {
    int x;        // queue index
    int nh;       // heads in the queue
    int ntask;    // task indices of the queue: nh * nmb, or 2 * nh * pph with pairs
    int nwg;      // workgroups serving the queue
    int rank;     // this workgroup's rank among them
    int tail;     // causal: heads at the queue's end served heavy-first across heads
    int pph;      // causal pairs per head (0: no pairs): ticket k runs tasks 2k, 2k+1
};

template <bool PAIRS>
__device__ __forceinline__ Queue make_queue(const FwdParams& p) {
    Queue q;
    q.x = (int)blockIdx.x % p.nq;
    q.rank = (int)blockIdx.x / p.nq;
    q.nwg = ((int)gridDim.x - q.x + p.nq - 1) / p.nq;
    q.nh = (p.num_heads - q.x + p.nq - 1) / p.nq;
    q.pph = PAIRS && p.pairs ? (p.nmb + 1) / 2 : 0;
    q.ntask = q.pph ? 2 * q.nh * q.pph : q.nh * p.nmb;
    // the tail spans about two rounds of the queue's workgroups
    q.tail = max(1, min(q.nh, 2 * (q.nwg / p.nmb)));
    return q;
}

// Pairs: the first task of ticket k is 2k; the second, 2k + 1, follows
// without a ticket unless the pair is a head's middle block alone.
__device__ __forceinline__ int task_of_ticket(const Queue& q, int k) { return q.pph ? 2 * k : k; }
__device__ __forceinline__ int ticket_of_task(const Queue& q, int t) { return q.pph ? t >> 1 : t; }
__device__ __forceinline__ bool pair_continues(const FwdParams& p, const Queue& q, int t) {
    if (!q.pph || (t & 1)) return false;
    return !((p.nmb & 1) && (t >> 1) % q.pph == q.pph - 1);
}

__device__ __forceinline__ float swap_max(float x) {
    // {x[l%32], x[l%32 + 32]} in some order for every lane l
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __builtin_elementwise_maximum(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float swap_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Task order inside a queue.  Head-major, so the tasks of a head start close
// together in time and walk its K/V in the same order: the first fetches a
// key tile into the XCD's L2 and the others hit it (causal tasks of one head
// all start at key tile 0).
// Causal with pairs (the host's choice when the pairs fill whole rounds of
// the queue's workgroups): ticket k of a head runs its query block nmb-1-i,
// then block i, so every ticket carries nmb + 1 block-lengths of key tiles.
// The workgroups then run in lockstep rounds, as in the non-causal case, and
// a head's heavy halves walk its K/V together (key tiles fetched past L2 at
// B=128 H=8 S=2048 D=128: 1.42x Q+K+V against 1.88x single blocks; at
// B=4 H=16 S=8192 D=64 1.21x against 1.87x, 3 % faster).  Light block first
// instead: 2.26x and 1.00x.
// Causal single blocks: inside a head the heaviest query block first, and the
// last q.tail heads are served heavy-first across heads (longest-processing-
// time first), which bounds the persistent grid's tail.  Grouping heads
// heavy-first over the whole queue balances as well but spreads a head's
// tasks over several rounds of tickets, and their K/V are evicted between
// them (B=128 H=8 S=2048 D=128: 2.09x the Q+K+V bytes fetched past L2,
// against 1.84x head-major; 4 % slower at B=4 H=16 S=8192 D=64 and 10 % at
// B=16 H=8 S=1024).
template <bool CAUSAL>
__device__ __forceinline__ void decode_task(const FwdParams& p, const Queue& q, int t, int& bh, int& mb) {
    int lh;  // head index inside the queue
    if (q.pph) {
        const int k = t >> 1;
        lh = k / q.pph;
        const int i = k - lh * q.pph;
        mb = (t & 1) ? i : p.nmb - 1 - i;
    } else if (!CAUSAL) {
        lh = t / p.nmb;
        mb = t - lh * p.nmb;
    } else {
        const int bulk = (q.nh - q.tail) * p.nmb;
        if (t < bulk) {
            lh = t / p.nmb;
            mb = p.nmb - 1 - (t - lh * p.nmb);
        } else {
            const int w = t - bulk;
            const int i = w / q.tail;
            mb = p.nmb - 1 - i;
            lh = q.nh - q.tail + (w - i * q.tail);
        }
    }
    bh = lh * p.nq + q.x;
}

// One wave's direct global->LDS load: each lane fetches 16 bytes from
// sbase + voff_bytes and the hardware writes lane i's data to
// lds_addr + 16*i (1 KB of consecutive LDS per instruction).  It is issued from
// inline asm so the compiler does not make later LDS reads wait for it; the
// kernel itself waits (vmcnt(0) + barrier) before reading a buffer a load
// targets, and only ever loads into the buffer nobody is reading.
// The compiler's hazard recognizer does not see this asm as a vector-memory
// instruction, so it adds no wait states for its scalar operands: when the
// SGPR base was just written by a VALU instruction (e.g. a v_readlane reload of
// a spilled SGPR), the load would read the stale base.  s_nop 4 supplies the 5
// wait states "VALU writes SGPR -> VMEM reads that SGPR" needs (and covers the
// one "write M0 -> LDS DMA" needs).
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff_bytes, uint32_t lds_addr) {
    asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff_bytes), "s"(sbase), "{m0}"(lds_addr)
                 : "memory");
}

// Compile-time loop: f(std::integral_constant<int, I>) for I = 0 .. N-1.
template <int... I, class F>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, I...>, F&& f) {
    (f(std::integral_constant<int, I>()), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(std::make_integer_sequence<int, N>(), f);
}

// MFMA operands read from LDS ahead of use.  The compiler's scheduler places
// each LDS read right before its MFMA and waits for it, exposing the LDS
// latency once per MFMA; here the reads are issued PF MFMAs ahead from inline
// asm and each MFMA first waits (s_waitcnt lgkmcnt) for its own operand only.
// The wait takes the operand as an in/out register so the MFMA that consumes
// it cannot be scheduled before the wait.  LDS operations complete in order,
// so a wait for "at most N outstanding" (N = reads issued after the one needed)
// is exact for these reads and only conservative for any LDS or scalar-memory
// operation the compiler interleaves.
#ifndef RSFA_QK_PREFETCH
#define RSFA_QK_PREFETCH 4
#endif
#ifndef RSFA_PV_PREFETCH
#define RSFA_PV_PREFETCH 4
#endif
#ifndef RSFA_PINGPONG
#define RSFA_PINGPONG 1
#endif
constexpr int QK_PREFETCH = RSFA_QK_PREFETCH;
constexpr int PV_PREFETCH = RSFA_PV_PREFETCH;

template <int OFF>
__device__ __forceinline__ i32x4 lds_read_b128(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "DS offset is 16 bits");
    i32x4 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
    return r;
}

template <int OFF>
__device__ __forceinline__ i32x2 lds_read_tr16(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "DS offset is 16 bits");
    i32x2 r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
    return r;
}

template <int OFF>
__device__ __forceinline__ i32x2 lds_read_tr8(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "DS offset is 16 bits");
    i32x2 r;
    asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
    return r;
}

// The float8 P.V MFMA's operands: A from four byte-transposing reads (8
// bytes each), B from the P bytes of two 32-key sub-tiles (16 each).
__device__ __forceinline__ i32x8 cat4(i32x2 r0, i32x2 r1, i32x2 r2, i32x2 r3) {
    return (i32x8){r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
}
template <class X8>
__device__ __forceinline__ i32x8 cat2(X8 p0, X8 p1) {
    const i32x4 b0 = __builtin_bit_cast(i32x4, p0), b1 = __builtin_bit_cast(i32x4, p1);
    return (i32x8){b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
}

template <int N, class V>
__device__ __forceinline__ void lgkm_wait(V& v) {
    static_assert(N >= 0 && N < 16, "lgkmcnt is 4 bits");
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "n"(N));
}

template <int N, class V>
__device__ __forceinline__ void lgkm_wait4(V& a, V& b, V& c, V& d) {
    static_assert(N >= 0 && N < 16, "lgkmcnt is 4 bits");
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "n"(N));
}

template <int N, class V>
__device__ __forceinline__ void lgkm_wait2(V& a, V& b) {
    static_assert(N >= 0 && N < 16, "lgkmcnt is 4 bits");
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N));
}

// A workgroup barrier that the compiler's scheduler does not move work across
// (the ping-pong phases must not leak into each other).  No memory fence: the
// LDS reads before it have all been waited for, and the direct loads are
// tracked with explicit vmcnt waits.
__device__ __forceinline__ void phase_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
}

// An operand stream of nops ops: ops below npv (P.V) take pvr reads each and
// are read pfv ops ahead, the others (QK) one read, pf ops ahead (pfv >= pf,
// so reads go out in op order): op x's reads are issued after op
// x_issue_after(x) (-1: before the stream).  x_reads_pending: LDS reads still
// outstanding once op m's have completed, at op m's wait.
constexpr int x_issue_after(int npv, int pf, int pfv, int x) {
    const int a = x - (x < npv ? pfv : pf);
    return a < -1 ? -1 : a;
}
constexpr int x_reads_pending(int npv, int nops, int pf, int pfv, int pvr, int m) {
    int n = 0;
    for (int x = m + 1; x < nops; ++x)
        if (x_issue_after(npv, pf, pfv, x) <= m - 1) n += x < npv ? pvr : 1;
    return n;
}

__device__ __forceinline__ void wait_loads_and_sync() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
}

// Whether an instantiation runs the ping-pong schedule (8-wave workgroups,
// three K/V buffers within the 160 KB of LDS of a CU).  At D = 256 (32-key
// tiles) O^T and Q^T take 192 of the 256 VGPRs: the loop still fits (+2 %
// non-causal against the one-phase loop); causal
// D = 256 runs its diagonal tiles in the loop too, masked by VALU selects
// (bias blocks there spilled 164 bytes per lane inside the loop): +3 % on
// B=64 S=1024 against the one-phase loop.
constexpr bool uses_pingpong(int d, int bn, int nw, bool causal, int mode) {
    return RSFA_PINGPONG && nw == 8 && mode == MODE_FUSED && (d <= 128 || d == 256) &&
           3 * (2 * bn * (d < 32 ? 32 : d) * 2) <= 160 * 1024 - 64;
}

// Whether a ping-pong instantiation stages Q through a Q buffer in LDS (the
// BM = 32*NW query rows of a task beside the three K/V buffers, D = 64 and
// 128).  Its Q loads use the K/V loader's per-lane 32-bit offsets, which span
// BN rows of Q.
constexpr bool uses_q_buffer(int d, int bn, int nw, bool causal, int mode) {
    return uses_pingpong(d, bn, nw, causal, mode) && d >= 64 && d <= 128 && (32 * nw) % bn == 0 &&
           3 * (2 * bn * d * 2) + 32 * nw * d * 2 <= 160 * 1024;
}

template <class T, int D, int BN, int NW, bool CAUSAL, int MODE, int OCC>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(OCC, OCC)))
fa_fwd_kernel(FwdParams p) {
    typedef typename T::elem elem;
    typedef typename T::velem velem;
    typedef typename T::x8 x8;
    typedef typename T::x4 x4;
    typedef typename T::x2 x2;

    constexpr int DP = D < 32 ? 32 : D;  // LDS row width / PV output rows
    constexpr int KST = D / 16;          // 16-wide k-steps of QK^T
    constexpr int DT = DP / 32;          // 32-row tiles of O^T
    constexpr int CPR = DP / 8;          // 16-byte chunks per LDS row
    constexpr int CPRV = D / 8;          // chunks that hold data
    constexpr int NKT = BN / 32;         // 32-key sub-tiles of a key tile
    constexpr int BM = NW * 32;
    constexpr int BLK = 32 * DP;          // bytes of a 16-row block
    constexpr int TILE = BN * DP * 2;     // bytes of one K (or fp16 V) tile
    constexpr int NINST = BN * CPR / 64;  // 1-KB direct loads per tile
    // V8: V tiles of e5m2 bytes, BN rows of DP bytes (D = 16: the row's
    // second 16-byte chunk is filler, its head dims are never stored); the
    // 1-KB slice s holds rows V8RPS*s.. whole, and row R keeps its 16-byte
    // chunk c at column c ^ v8_swz(R), so the eight rows one transposing read
    // of P.V gathers (below), and the sixteen (row, chunk) pairs of 32 lanes,
    // fall in distinct banks: R % 4 + 4 ((R / 8) % 2) for 128-byte rows (rows
    // 2 apart share banks), 2 ((R / 8) % 2) for 64-byte rows (rows 4 apart
    // do), and twice the 128-byte value for 256-byte rows (every row spans
    // all banks, so the two chunk columns c, c ^ 1 one read takes from each of
    // its eight rows must land on sixteen distinct columns).  32-byte rows
    // keep their chunks in place (a chunk swap stays inside the row's banks).
    constexpr bool V8 = T::v8;
    static_assert(!V8 || (BN % 64 == 0 || BN == 32),
                  "byte V tiles: 64-key groups or one 32-key tile");
    constexpr int TILEV = V8 ? BN * DP : TILE;  // bytes of one V tile
    constexpr int BUF = TILE + TILEV;          // K + V
    constexpr int NINSTV = V8 ? TILEV / 1024 : NINST;
    constexpr int V8RPS = 1024 / DP;           // rows per 1-KB slice of a byte V tile
    constexpr int V8CPR = DP / 16;             // 16-byte chunks per row of it
    // (rq = R % 4, rh = (R / 8) % 2 of the row)
    auto v8_swz = [](int rq, int rh) {
        return D <= 32 ? 0 : D == 64 ? 2 * rh : D == 128 ? rq + 4 * rh : 2 * (rq + 4 * rh);
    };
    // V8: transposing reads per float8 MFMA (64 keys): four, or two for a
    // 32-key tile, whose MFMA takes P = 0 for its upper 32 keys (and the same
    // two reads again as their finite V)
    constexpr int V8RPM = 2 * NKT < 4 ? 2 * NKT : 4;
    static_assert(BN % 32 == 0 && BN >= 32, "BN must be a multiple of 32");
    static_assert(D % 16 == 0, "D must be a multiple of 16");
    static_assert((BN * CPR) % 64 == 0, "tile must be whole 1-KB load slices");
    static_assert(MODE == MODE_FUSED || CAUSAL, "split modes are causal only");
    // Ping-pong schedule for 8-wave workgroups (two waves per SIMD): the key
    // tiles every row of the workgroup sees unmasked run with waves 4-7 one
    // phase behind waves 0-3, so one wave of each SIMD runs its softmax (VALU)
    // while the other runs its matrix products.  K/V are triple buffered.
    constexpr bool PP = uses_pingpong(D, BN, NW, CAUSAL, MODE);
    constexpr int NBUF = PP ? 3 : 2;
    // Causal ping-pong tiles also cover the diagonal key tiles of a whole
    // query block: the first S^T MFMA of each 32-key sub-tile accumulates onto
    // a per-wave bias block (0 below the wave's rows, -inf above, triangular
    // on its diagonal), so masking costs no VALU work per score.  Two
    // sub-tiles per tile (32 VGPRs); at D <= 128 only (register budget).
    constexpr bool DIAG_PP = CAUSAL && PP && NKT <= 2 && D <= 128;
    // At D = 256 the diagonal tiles run in the ping-pong loop too, masked by
    // VALU selects in the softmax phase (no bias registers; at D = 256 the
    // softmax phase is the short one).
    constexpr bool DIAG_VM = CAUSAL && PP && !DIAG_PP;
    // Q through LDS (ping-pong tiles, D = 64 and 128): a Q buffer after the
    // K/V buffers takes a task's BM query rows in the K tile layout, filled by
    // the same coalesced direct loads as K and read into the Q^T registers with
    // the K operand's reads.  Loaded straight into registers, every load
    // instruction of Q touches 32 rows (measured: ~5k of the ~9k cycles from a
    // task's start to its first MFMA).  A task that runs its key loop in
    // ping-pong also loads the next task's Q into the buffer during two of its
    // MFMA phases, so that task starts with its Q in LDS.
    constexpr int QTILE = BM * DP * 2;  // bytes of the Q buffer
    constexpr bool QPF = uses_q_buffer(D, BN, NW, CAUSAL, MODE);
    static_assert(!QPF || (NBUF == 3 && NBUF * BUF + QTILE <= 160 * 1024), "Q buffer past the LDS");

    __shared__ __attribute__((aligned(1024))) char smem_raw[NBUF * BUF + (QPF ? QTILE : 0)];
    RSFA_LDS char* const smem = (RSFA_LDS char*)smem_raw;
    const uint32_t smem_addr = (uint32_t)(uintptr_t)smem;
    // Ticket broadcast slot.  With the Q buffer the LDS is full: the slot is
    // then the last word of the third K/V buffer (its V tile), which the
    // epilogue's staging does not reach, the tiles past the ping-pong loop do
    // not use, and the loop first loads two barriers after its first phase.
    RSFA_LDS int* tslot;
    if constexpr (QPF) {
        tslot = (RSFA_LDS int*)(smem + NBUF * BUF - 4);
    } else {
        __shared__ int s_ticket;
        tslot = (RSFA_LDS int*)&s_ticket;
    }

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int hh = lane >> 5;  // which 8-key half of a 16-key MFMA step
    const int l32 = lane & 31;
    const int l16 = lane & 15;

    // LDS read offsets (bytes, relative to a K or V tile).
    // K (A operand of S^T): row l32 (+32 per sub-tile), chunk 2s+hh.
    uint32_t koff[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) koff[e] = (l32 >> 4) * BLK + hh * 256 + ((l16 ^ (8 * e + 4 * hh)) * 16);
    // At D = 256 (O^T and Q^T hold 192 of the 256 VGPRs) values the compiler
    // hoists out of the task loop are spilled, and each reload from scratch
    // makes it wait for every load in flight (vmcnt(0)): at a task's start the
    // K/V loads, then Q's, went out one latency at a time.  REG_TIGHT kernels
    // recompute what the start needs per task instead (+1.2 to +3.8 % on
    // D = 256 shapes); the lane id is then taken from asm (v_mbcnt), which
    // the compiler cannot hoist.
    constexpr bool REG_TIGHT = D > 128;
    auto fresh_lane = []() {
        int ln;
        asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
        return ln;
    };
    // V (A operand of O^T via transposing reads): lane l16 of a 16-lane group
    // addresses row (l16/4) of the group's 4 keys and columns 4*(l16%4)..+3 of
    // its 16 head dims; the hardware hands lane j column j of the 4 rows.
    const int vg = (lane >> 4) & 1;
    const int vcc = 2 * vg + ((l16 >> 1) & 1);
    uint32_t voff[2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
        voff[u] = vcc * 256 + (((8 * u + 4 * hh + (l16 >> 2)) ^ (4 * vcc)) * 16) + 8 * (l16 & 1);
    // V8 (ds_read_b64_tr_b8): in a 16-lane group lanes 2r and 2r+1 address
    // bytes 0-7 and 8-15 of row r of eight rows, and the hardware hands lane j
    // column j of the eight rows.  The read of 16-key group q' (keys 16q'.. of
    // the tile) and head-dim block db gives bytes 8 (q' % 4) .. +7 of the A
    // operand (V^T) of the 64-key float8 MFMA of keys 64 (q' / 4).. ; its byte
    // e must be key 16q' + 4hh + e % 4 + 8 (e / 4) for lane (d + 32 hh), the
    // key whose rounded P that lane holds in the same byte of its B operand
    // (P^T, in the S^T accumulator layout); so row r of the group is that key
    // for e = r, and the group's 16 columns are head dims 32db + 16((lane /
    // 16) % 2) ...  Offset from the tile at q' = 0 (q' adds 16q' rows), per db.
    // At D = 256 (eight head-dim blocks, O^T and Q^T in 192 VGPRs) only the
    // row base and swizzle are kept (v8_rb, v8_sw) and each block's offset is
    // formed where it is read (v8_off).
    constexpr bool V8_INLINE = V8 && DT > 4;
    uint32_t vo8[V8 && !V8_INLINE ? DT : 1];
    int v8_rb = 0, v8_sw = 0;
    if constexpr (V8) {
        const int tr = l16 >> 1;  // row r of the group: R % 4 = r % 4, (R / 8) % 2 = r / 4
        const int rowb = DP * (4 * hh + (tr & 3) + 8 * (tr >> 2)) + 8 * (l16 & 1);
        const int swz = v8_swz(tr & 3, tr >> 2);
        if constexpr (V8_INLINE) {
            v8_rb = rowb;
            v8_sw = swz ^ ((lane >> 4) & 1);  // (2 db + g) ^ swz = 2 db ^ (swz ^ g)
        } else {
#pragma unroll
            for (int db = 0; db < DT; ++db) vo8[db] = (uint32_t)(rowb + 16 * ((2 * db + ((lane >> 4) & 1)) ^ swz));
        }
    }
    // byte offset of head-dim block db's transposing reads from a V tile
    auto v8_off = [&](int db) -> uint32_t {
        if constexpr (V8_INLINE) {
            int sw = v8_sw;
            asm volatile("" : "+v"(sw));  // formed here, not hoisted out of the loops
            return (uint32_t)(v8_rb + 16 * ((2 * db) ^ sw));
        } else {
            return vo8[db];
        }
    };

    // Loader: in every 1-KB slice lane i fills chunk 4*cg + i/16 of the 16-row
    // block's row (i%16) ^ 4*((i/16)%4), so its global offset inside the block
    // is the same for every slice.
    const int ld_rib = l16 ^ (4 * ((lane >> 4) & 3));
    const int ld_chl = lane >> 4;
    // Byte offsets of this wave's slices (slice w = sl*NW + wave) from the first
    // row of a whole tile, for K and V; the tile loop only adds a uniform base.
    constexpr int NSL = (NINST + NW - 1) / NW;
    constexpr int NSLV = (NINSTV + NW - 1) / NW;  // V slices per wave
    uint32_t kgo[NSL], vgo[NSLV];
#pragma unroll
    for (int sl = 0; sl < NSL; ++sl) {
        const int w = sl * NW + wave;
        const int blk = (w * 64) / (16 * CPR);
        const int cg = ((w * 64) % (16 * CPR)) / 64;
        kgo[sl] = (uint32_t)(((16 * blk + ld_rib) * p.k_sn + cg * 32 + ld_chl * 8) * 2);
        if constexpr (!V8) vgo[sl] = (uint32_t)(((16 * blk + ld_rib) * p.v_sn + cg * 32 + ld_chl * 8) * 2);
    }
    // V8: lane i of slice s fills position i of the slice, i.e. chunk column
    // i % V8CPR of row V8RPS*s + i / V8CPR, with that row's chunk
    // (i % V8CPR) ^ v8_swz(row); at D = 16 the filler chunk re-reads chunk 0
    // (a row has no second chunk to read)
    auto v8_chunk = [&](int s) {
        const int row = V8RPS * s + lane / V8CPR;
        return D < 32 ? 0 : (lane % V8CPR) ^ v8_swz(row & 3, (row >> 3) & 1);
    };
    if constexpr (V8) {
#pragma unroll
        for (int sl = 0; sl < NSLV; ++sl) {
            const int s = sl * NW + wave;
            vgo[sl] = (uint32_t)((V8RPS * s + lane / V8CPR) * p.v_sn + 16 * v8_chunk(s));
        }
    }
    // Q rows (QPF): each wave loads its own 32 rows, i.e. the slices of the two
    // 16-row blocks 2*wave, 2*wave+1 of the Q buffer; the lane's offset inside a
    // slice is the same for all of them.
    constexpr int QSPB = CPR / 4;   // 1-KB slices per 16-row block
    constexpr int NQD = 2 * QSPB;   // Q direct loads per wave
    const uint32_t qlo = QPF ? (uint32_t)((ld_rib * p.q_sm + ld_chl * 8) * 2) : 0u;

    const float c = p.c;
    const int qsign = p.neg ? (int)0x80008000u : 0;
    const elem* const qg = (const elem*)p.q;
    const elem* const kg = (const elem*)p.k;
    const velem* const vgp = (const velem*)p.v;
    elem* const og = (elem*)p.o;

    constexpr bool PAIRS = CAUSAL && MODE == MODE_FUSED;
    const Queue qu = make_queue<PAIRS>(p);
    uint32_t* const ctr = p.ticket ? p.ticket + 16 * qu.x : nullptr;
    int t;
    if (ctr) {
        if (tid == 0) *tslot = (int)atomicAdd(ctr, 1u);
        __syncthreads();
        t = task_of_ticket(qu, *tslot);
        if constexpr (QPF) __syncthreads();  // read before the first task writes the slot again
    } else {
        t = task_of_ticket(qu, qu.rank);
    }
    bool qready = false;  // QPF: the previous task loaded this task's Q into the Q buffer

    while (t < qu.ntask) {
        int nxt = 0;
        // the next task needs no ticket when it is the second of a pair
        // (recomputed where needed: a flag kept live across the task costs a
        // register of the tight causal kernels)
        if (ctr && tid == 0 && !pair_continues(p, qu, t)) {
            if constexpr (QPF) {
                // from asm, so the compiler adds no wait for it before its use
                // (the ticket slot write after the first phase's partial load
                // wait, which covers it: it is the task's oldest vector memory
                // operation; the epilogue waits for every load)
                asm volatile("s_nop 4\n\tglobal_atomic_add %0, %1, %2, %3 sc0"
                             : "=v"(nxt)
                             : "v"(0u), "v"(1u), "s"(ctr)
                             : "memory");
            } else {
                nxt = (int)atomicAdd(ctr, 1u);
            }
        }

        int bh, mb;
        decode_task<CAUSAL>(p, qu, t, bh, mb);
        const int b = bh / p.H;
        const int h = bh - b * p.H;
        // REG_TIGHT: opaque per task, so values derived from n stay inside the
        // task instead of being hoisted out of the task loop and spilled
        int n = p.n_ctx;
        if constexpr (REG_TIGHT) asm volatile("" : "+s"(n));
        const int m0 = mb * BM;
        const int qrow = m0 + wave * 32 + l32;

        const elem* qb = qg + b * p.q_sz + h * p.q_sh;
        const elem* kh = kg + b * p.k_sz + h * p.k_sh;
        const velem* vh = vgp + b * p.v_sz + h * p.v_sh;
        elem* ob = og + b * p.o_sz + h * p.o_sh;

        // key tiles of this task
        const int kv_end = CAUSAL ? min(n, m0 + BM) : n;
        int j0 = 0, j1 = (kv_end + BN - 1) / BN;
        if (MODE == MODE_PREFIX) j1 = m0 / BN;
        if (MODE == MODE_DIAG) j0 = m0 / BN;

        auto load_tile = [&](int j, int buf) {
            const int kbase = j * BN;
            const elem* kt0 = kh + (int64_t)kbase * p.k_sn;
            const velem* vt0 = vh + (int64_t)kbase * p.v_sn;
            const uint32_t dst0 = smem_addr + buf * BUF;
            if (kbase + BN <= n) {
                // whole tile: one uniform base per tensor, per-slice offsets precomputed
#pragma unroll
                for (int sl = 0; sl < NSL; ++sl) {
                    const int w = sl * NW + wave;
                    if (NINST % NW == 0 || w < NINST) {
                        const int cg = ((w * 64) % (16 * CPR)) / 64;
                        if (CPRV == CPR || 4 * cg + ld_chl < CPRV) {
                            dma16(kt0, kgo[sl], dst0 + w * 1024);
                            if constexpr (!V8) dma16(vt0, vgo[sl], dst0 + w * 1024 + TILE);
                        }
                    }
                }
                if constexpr (V8) {
#pragma unroll
                    for (int sl = 0; sl < NSLV; ++sl) {
                        const int s = sl * NW + wave;
                        if (NINSTV % NW == 0 || s < NINSTV) dma16(vt0, vgo[sl], dst0 + TILE + s * 1024);
                    }
                }
                return;
            }
            const int last = n - 1 - kbase;  // last row of the tile inside the sequence
            if constexpr (V8) {
                // rows past the sequence re-read its last row (masked later)
#pragma unroll
                for (int sl = 0; sl < NSLV; ++sl) {
                    const int s = sl * NW + wave;
                    if (NINSTV % NW == 0 || s < NINSTV) {
                        const int row0 = min(V8RPS * s, last);
                        const int rr = min(V8RPS * s + lane / V8CPR, last) - row0;
                        const uint32_t vo = (uint32_t)(rr * p.v_sn + 16 * v8_chunk(s));
                        dma16(vt0 + (int64_t)row0 * p.v_sn, vo, dst0 + TILE + s * 1024);
                    }
                }
            }
#pragma unroll
            for (int sl = 0; sl < NSL; ++sl) {
                const int w = sl * NW + wave;
                if (NINST % NW == 0 || w < NINST) {
                    const int blk = (w * 64) / (16 * CPR);
                    const int cg = ((w * 64) % (16 * CPR)) / 64;
                    // rows past the sequence re-read its last row (masked later)
                    const int row0 = min(16 * blk, last);
                    const int rr = min(16 * blk + ld_rib, last) - row0;
                    const uint32_t ko = (uint32_t)((rr * p.k_sn + ld_chl * 8) * 2);
                    const elem* ks = kt0 + (int64_t)row0 * p.k_sn + cg * 32;
                    if (CPRV == CPR || 4 * cg + ld_chl < CPRV) {
                        dma16(ks, ko, dst0 + w * 1024);
                        if constexpr (!V8) {
                            const uint32_t vo = (uint32_t)((rr * p.v_sn + ld_chl * 8) * 2);
                            dma16(vt0 + (int64_t)row0 * p.v_sn + cg * 32, vo, dst0 + w * 1024 + TILE);
                        }
                    }
                }
            }
        };

        // Ping-pong buffers: tile jj of K and V in buffer jj % NBUF.
        auto bofs = [&](int jj) { return (uint32_t)((jj % NBUF) * BUF); };
        // slice sl of this wave's share of tile jj of K (or V)
        // (the tile's first row at tp)
        auto pp_dma_at = [&](const elem* tp, const uint32_t(&go)[NSL], uint32_t dst0, int sl) {
            const int w = sl * NW + wave;
            if (NINST % NW == 0 || w < NINST) {
                const int cg = ((w * 64) % (16 * CPR)) / 64;
                if (CPRV == CPR || 4 * cg + ld_chl < CPRV) dma16(tp, go[sl], dst0 + w * 1024);
            }
        };
        // the same for V (dst0: the V tile)
        auto pp_dma_v_at = [&](const velem* tp, uint32_t dst0, int sl) {
            const int w = sl * NW + wave;
            if constexpr (V8) {
                if (NINSTV % NW == 0 || w < NINSTV) dma16(tp, vgo[sl], dst0 + w * 1024);
            } else {
                if (NINST % NW == 0 || w < NINST) {
                    const int cg = ((w * 64) % (16 * CPR)) / 64;
                    if (CPRV == CPR || 4 * cg + ld_chl < CPRV) dma16(tp, vgo[sl], dst0 + w * 1024);
                }
            }
        };
        auto dma_k = [&](int jj, int sl) { pp_dma_at(kh + (int64_t)(jj * BN) * p.k_sn, kgo, smem_addr + bofs(jj), sl); };
        auto dma_v = [&](int jj, int sl) { pp_dma_v_at(vh + (int64_t)(jj * BN) * p.v_sn, smem_addr + bofs(jj) + TILE, sl); };
        auto load_k = [&](int jj) { for (int sl = 0; sl < NSL; ++sl) dma_k(jj, sl); };
        auto load_v = [&](int jj) { for (int sl = 0; sl < NSLV; ++sl) dma_v(jj, sl); };

        // [j0, jpp): ping-pong tiles (whole tiles no row of the workgroup masks).
        // The first loads go out before the Q loads, so their latencies overlap.
        int jpp = j0;
        if constexpr (PP) jpp = min(j1, (CAUSAL ? m0 : n) / BN);
        if constexpr (DIAG_PP || DIAG_VM) {
            if (m0 + BM <= n) jpp = j1;  // the diagonal tiles too (whole tiles only)
        }
        // QPF: direct load q (< NQD) of this wave's rows into the Q buffer, for
        // the BM rows from qsrc on: block 2*wave + q / QSPB, chunk group q % QSPB.
        // Only this wave reads what it loads there (read_q).
        auto dma_q = [&](const elem* qsrc, int q) {
            const int bb = q / QSPB, cg = q % QSPB;
            // wave-uniform by construction; made explicit for the SGPR operand
            const uint64_t a = (uint64_t)(uintptr_t)(qsrc + (int64_t)(32 * wave + 16 * bb) * p.q_sm + cg * 32);
            const uint64_t ua = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(a >> 32)) << 32) |
                                (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
            dma16((const void*)(uintptr_t)ua, qlo, smem_addr + NBUF * BUF + (2 * wave + bb) * BLK + cg * 1024);
        };
        // Where this task's Q comes from (QPF): the Q buffer, filled by the
        // previous task (qready) or by loads issued here for a ping-pong task
        // of a whole query block (q_dma, read after the first phase's load
        // wait), else global memory.
        const bool q_dma = QPF && !qready && jpp > j0 && m0 + BM <= n;
        int t_next = -1;         // QPF, ticket queue: the next ticket, read at the first barrier
        bool qpf_do = false;     // QPF: this task loads the next task's Q into the Q buffer
        const elem* qnext = qg;  // its first row
        if (jpp > j0) {
            load_k(j0);
            if (q_dma)
                for (int q = 0; q < NQD; ++q) dma_q(qb + (int64_t)m0 * p.q_sm, q);
            load_v(j0);
            if (j0 + 1 < jpp) load_k(j0 + 1);
        } else if (j0 < j1) {
            load_tile(j0, 0);
        }

        // first element of this lane's Q fragments, q[qrow][8hh]
        auto q_lane = [&]() {
            if constexpr (REG_TIGHT) {
                const int ln = fresh_lane();
                return qb + (int64_t)min(m0 + wave * 32 + (ln & 31), n - 1) * p.q_sm + ((ln >> 5) & 1) * 8;
            } else {
                return qb + (int64_t)min(qrow, n - 1) * p.q_sm + hh * 8;
            }
        };
        // Q^T fragments (B operand of S^T): lane holds q[qrow][16s + 8hh .. +7]
        // (sign flip for a negative sm_scale: xor with a uniform mask, 0 otherwise)
        x8 qf[KST];
        auto q_sign = [&]() {
            int qs = qsign;
            // REG_TIGHT: tested here, in an SGPR (hoisted out of the task loop,
            // the test was kept in a VGPR and spilled)
            if constexpr (REG_TIGHT) asm volatile("" : "+s"(qs));
            if (qs) {
                // a real branch (the asm keeps it from being flattened into an
                // xor with 0), so positive scales do not wait for Q here
                asm volatile("");
#pragma unroll
                for (int s = 0; s < KST; ++s) qf[s] = __builtin_bit_cast(x8, __builtin_bit_cast(i32x4, qf[s]) ^ qs);
            }
        };
        // QPF: this wave's 32 rows of the Q buffer (32-row sub-tile `wave`),
        // with the K operand's read pattern
        auto read_q = [&]() {
            const uint32_t qa0 = smem_addr + NBUF * BUF + wave * 2 * BLK + koff[0];
            const uint32_t qa1 = smem_addr + NBUF * BUF + wave * 2 * BLK + koff[1];
            i32x4 r[KST];
            static_for<KST>([&](auto sc) {
                constexpr int s = decltype(sc)::value;
                r[s] = lds_read_b128<s * 512>((s & 1) ? qa1 : qa0);
            });
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int s = 0; s < KST; ++s) {
                asm volatile("" : "+v"(r[s]));
                qf[s] = __builtin_bit_cast(x8, r[s]);
            }
            q_sign();
        };
        if (QPF && qready) {
            read_q();
        } else if (!q_dma) {
            const elem* const ql = q_lane();
#pragma unroll
            for (int s = 0; s < KST; ++s) qf[s] = *(const x8*)(ql + 16 * s);
            // Q has arrived here as far as the compiler knows (the tile loops
            // wait for the first tile's loads, issued before Q's, anyway):
            // without this it would wait for Q, i.e. for the newest direct
            // loads, at every use of qf inside the loops.  Kept on this path:
            // where the paths join it would make the others wait too.
#pragma unroll
            for (int s = 0; s < KST; ++s) asm volatile("" : "+v"(qf[s]));
            q_sign();
        }

        f32x16 o[DT];
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[d][r] = 0.0f;
        float m_use = -INFINITY;  // running max (exp2 domain) of this lane's query row
        float l_sum = 0.0f;       // this lane's half of the row sum
        // Bias blocks of the diagonal ping-pong tiles: sub-tile kt of tile tt
        // lies below (<0), on (0) or above (>0) this wave's 32 rows.
        f32x16 cb[DIAG_PP ? NKT : 1];
        auto cb_rel = [&](int tt, int kt) { return tt * NKT + kt - (m0 / 32 + wave); };
        auto cb_fill = [&](int kt, int rel) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int kk = 8 * (i >> 2) + 4 * hh + (i & 3);  // key of register i in the sub-tile
                cb[kt][i] = rel < 0 ? 0.0f : (rel > 0 || kk > l32) ? -INFINITY : 0.0f;
            }
        };
        if constexpr (DIAG_PP) {
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) cb_fill(kt, cb_rel(j0, kt));
        }
        // DIAG_VM: scores of tile tt a wave's row does not see become -inf
        // (sub-tiles past the diagonal whole, the diagonal one triangular)
        auto vmask = [&](f32x16 (&sacc)[NKT], int tt) {
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                const int rel = cb_rel(tt, kt);
                if (rel >= 0) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int kk = 8 * (i >> 2) + 4 * hh + (i & 3);  // key of register i in the sub-tile
                        if (rel > 0 || kk > l32) sacc[kt][i] = -INFINITY;
                    }
                }
            }
        };

        const int srow = bh * p.nmb * BM + m0 + wave * 32 + l32;  // split-state row
        // split mode: this row's fp32 accumulator in the workspace (every
        // row of every task has one, rows past n included)
        float* const acc_row = MODE == MODE_FUSED ? nullptr : p.acc + (int64_t)srow * D;
        if (MODE == MODE_DIAG) {
            // resume from the prefix launch: its (m, l) and un-normalised
            // accumulator, all fp32
            m_use = p.state[srow];
            l_sum = hh == 0 ? p.state[(int64_t)p.num_tasks * BM + srow] : 0.0f;
#pragma unroll
            for (int d = 0; d < DT; ++d)
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    const int col = 32 * d + 8 * a + 4 * hh;
                    if (col < D) {
                        const float4 v4 = *(const float4*)(acc_row + col);
                        o[d][4 * a + 0] = v4.x;
                        o[d][4 * a + 1] = v4.y;
                        o[d][4 * a + 2] = v4.z;
                        o[d][4 * a + 3] = v4.w;
                    }
                }
        }

        const int wq_lo = m0 + wave * 32;  // smallest query row of this wave
        const int wq_hi = wq_lo + 31;      // largest
        const int lim = CAUSAL ? min(qrow, n - 1) : n - 1;     // last key this lane sees
        const int vis_lo = CAUSAL ? min(wq_lo, n - 1) : n - 1;  // last key every lane of the wave sees
        const int vis_hi = CAUSAL ? min(wq_hi, n - 1) : n - 1;  // last key any lane of the wave sees

        // S^T = K Q^T for the key tile whose K sits at LDS byte offset kofs.
        // Masked: keys past each row's last visible key become -inf, and 32-key
        // sub-tiles at or past nkt_act (no row of the wave sees them) are skipped.
        auto qk_part = [&](uint32_t kofs, int kbase, int nkt_act, f32x16 (&sacc)[NKT], auto masked, auto use_cb) {
            constexpr bool MASK = decltype(masked)::value;
            const RSFA_LDS char* kt_lds = smem + kofs;
            const f32x16 zero = {};  // the first k-step adds to an inline-constant 0
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) sacc[kt] = zero;
            if (!MASK) {
                // MFMA i = (k-step s, sub-tile kt), i = s*NKT + kt; operand ring of PF+1
                constexpr int NM = KST * NKT;
                constexpr int PF = QK_PREFETCH < NM ? QK_PREFETCH : NM;
                constexpr int NB = PF + 1;
                const uint32_t kb0 = smem_addr + kofs + koff[0];
                const uint32_t kb1 = smem_addr + kofs + koff[1];
                i32x4 ring[NB];
                auto issue = [&](auto ic) {
                    constexpr int i = decltype(ic)::value;
                    constexpr int ss = i / NKT, kt = i % NKT;
                    ring[i % NB] = lds_read_b128<kt * 2 * BLK + ss * 512>((ss & 1) ? kb1 : kb0);
                };
                static_for<PF>(issue);
                static_for<NM>([&](auto ic) {
                    constexpr int i = decltype(ic)::value;
                    constexpr int ss = i / NKT, kt = i % NKT;
                    constexpr int ahead = (NM - 1 - i) < (PF - 1) ? (NM - 1 - i) : (PF - 1);
                    lgkm_wait<ahead>(ring[i % NB]);
                    sacc[kt] = T::mfma(__builtin_bit_cast(x8, ring[i % NB]), qf[ss],
                                       ss == 0 ? (DIAG_PP && decltype(use_cb)::value ? cb[DIAG_PP ? kt : 0] : zero) : sacc[kt]);
                    if constexpr (i + PF < NM) issue(std::integral_constant<int, i + PF>());
                });
            } else {
#pragma unroll
                for (int s = 0; s < KST; ++s) {
#pragma unroll
                    for (int kt = 0; kt < NKT; ++kt) {
                        if (kt < nkt_act) {
                            const x8 a = *(const RSFA_LDS x8*)(kt_lds + koff[s & 1] + kt * 2 * BLK + s * 512);
                            sacc[kt] = T::mfma(a, qf[s], s == 0 ? zero : sacc[kt]);
                        }
                    }
                }
            }
            if (MASK) {
                const int rel = lim - kbase - 4 * hh;
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int kk = 32 * kt + 8 * (r >> 2) + (r & 3);
                        if (kk > rel || kt >= nkt_act) sacc[kt][r] = -INFINITY;
                    }
            }
        };
        // Row max of the tile folded into m_use (rescaling O and l when it
        // moves); returns the value to subtract before exp2.  NaN-propagating
        // (v_maximum3_f32) as the reference's max is (flash_attention_forward.py:
        // 200-203), which also spares the operand canonicalisation of maxNum.
        auto softmax_max = [&](f32x16 (&sacc)[NKT], auto masked) {
            constexpr bool MASK = decltype(masked)::value;
            float mx = sacc[0][0];
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (kt + r > 0) mx = __builtin_elementwise_maximum(mx, sacc[kt][r]);
            mx = swap_max(mx);
            const float m_tile = mx * c;
            const bool need = m_tile > m_use + RESCALE_SLACK;
            if (__builtin_amdgcn_ballot_w64(need)) {
                const float m_new = need ? m_tile : m_use;
                const float alpha = need ? __builtin_amdgcn_exp2f(m_use - m_new) : 1.0f;
                l_sum *= alpha;
#pragma unroll
                for (int d = 0; d < DT; ++d)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[d][r] *= alpha;
                m_use = m_new;
            }
            return (MASK && m_use == -INFINITY) ? 0.0f : m_use;
        };
        // P for one pair of scores, unit u = (kt, h2, i) = ((kt*2 + h2)*4 + i):
        // pk[kt][h2] elements 2i, 2i+1, and their rounded sum into l_sum.
        auto softmax_unit = [&](auto uc, const f32x16 (&sacc)[NKT], x8 (&pk)[NKT][2], float msub) {
            constexpr int u = decltype(uc)::value;
            constexpr int kt = u / 8, h2 = (u / 4) % 2, i = u % 4;
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt][8 * h2 + 2 * i], c, -msub));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt][8 * h2 + 2 * i + 1], c, -msub));
            if constexpr (V8) {
                // e5m2 bytes of the float8 P.V MFMA's B operand: the pair's
                // accumulator registers rho = 8h2 + 2i, +1 of sub-tile kt go to
                // bytes 16kt + rho (pk[kt][0] holds sub-tile kt's 16 bytes)
                constexpr int dw = 2 * h2 + (i >> 1);
                i32x4 w = __builtin_bit_cast(i32x4, pk[kt][0]);
                w[dw] = __builtin_amdgcn_cvt_pk_bf8_f32(p0, p1, (i & 1) ? w[dw] : 0, (i & 1) != 0);
                pk[kt][0] = __builtin_bit_cast(x8, w);
                l_sum += p0 + p1;  // the reference sums the unrounded P for an e5m2 V
            } else {
                const x2 pr = T::cvt2(p0, p1);
                l_sum = T::dot2(pr, T::ones2(), l_sum);
                pk[kt][h2][2 * i] = pr[0];
                pk[kt][h2][2 * i + 1] = pr[1];
            }
        };
        // Online softmax of one S^T tile: row max (softmax_max), then
        // P = exp2(S c - m) rounded to the input type into pk and the row sum
        // of the rounded P into l_sum.
        auto softmax_part = [&](f32x16 (&sacc)[NKT], x8 (&pk)[NKT][2], auto masked) {
            const float msub = softmax_max(sacc, masked);
            static_for<NKT * 8>([&](auto uc) { softmax_unit(uc, sacc, pk, msub); });
        };
        // O^T += V^T P^T for the value tile at LDS byte offset vofs.
        auto pv_part = [&](uint32_t vofs, int nkt_act, const x8 (&pk)[NKT][2], auto masked) {
            constexpr bool MASK = decltype(masked)::value;
            const RSFA_LDS char* vt_lds = smem + vofs;
            if constexpr (V8) {
                // read i = (d*NKT + kt)*2 + h2 fetches keys 16(2kt + h2).. of
                // head-dim block d (byte-transposing, 8 bytes per lane); every
                // V8RPM-th completes the A operand of a 64-key float8 MFMA, whose
                // B operand is sub-tiles 2kk, 2kk+1 of the P bytes (P = 0 past
                // a 32-key tile)
                constexpr int NM = DT * NKT * 2;
                constexpr int PF = V8RPM == 2 ? 4 : 8;  // two float8 MFMAs ahead
                constexpr int NB = PF + V8RPM;  // the reads of an MFMA stay live to it
                const uint32_t vb = smem_addr + vofs;
                if (!MASK) {
                    i32x2 rv[NB];
                    auto issue = [&](auto ic) {
                        constexpr int i = decltype(ic)::value;
                        constexpr int d = i / (2 * NKT), kt = (i / 2) % NKT, h2 = i % 2;
                        rv[i % NB] = lds_read_tr8<(2 * kt + h2) * 16 * DP>(vb + v8_off(d));
                    };
                    static_for<PF>(issue);
                    static_for<NM>([&](auto ic) {
                        constexpr int i = decltype(ic)::value;
                        constexpr int d = i / (2 * NKT), qq = i % (2 * NKT);
                        constexpr int ahead = (NM - 1 - i) < (PF - 1) ? (NM - 1 - i) : (PF - 1);
                        if constexpr (V8RPM == 4 && qq % 4 == 3) {
                            i32x2 &r0 = rv[(i - 3) % NB], &r1 = rv[(i - 2) % NB], &r2 = rv[(i - 1) % NB], &r3 = rv[i % NB];
                            lgkm_wait4<ahead>(r0, r1, r2, r3);
                            o[d] = T::mfma8(cat4(r0, r1, r2, r3), cat2(pk[qq / 2 - 1][0], pk[qq / 2][0]), o[d]);
                            __builtin_amdgcn_sched_barrier(0);  // issued here, not sunk below the next reads
                        } else if constexpr (V8RPM == 2 && qq == 1) {
                            i32x2 &r0 = rv[(i - 1) % NB], &r1 = rv[i % NB];
                            lgkm_wait2<ahead>(r0, r1);
                            o[d] = T::mfma8(cat4(r0, r1, r0, r1), cat2(pk[0][0], x8{}), o[d]);
                            __builtin_amdgcn_sched_barrier(0);
                        }
                        if constexpr (i + PF < NM) issue(std::integral_constant<int, i + PF>());
                    });
                } else {
                    // sub-tiles no row of the wave sees (kt >= nkt_act) hold
                    // P = 0; their V is not read (zeros), as the fp16 path skips them
#pragma unroll
                    for (int d = 0; d < DT; ++d)
#pragma unroll
                        for (int kk = 0; kk < (NKT + 1) / 2; ++kk)
                            if (2 * kk < nkt_act) {
                                i32x2 r[4];
#pragma unroll
                                for (int qq = 0; qq < 4; ++qq) {
                                    r[qq] = (i32x2){0, 0};
                                    if (2 * kk + qq / 2 < nkt_act && 2 * kk + qq / 2 < NKT)
                                        r[qq] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                                            (RSFA_LDS i32x2*)(vt_lds + (4 * kk + qq) * 16 * DP + v8_off(d)));
                                }
                                o[d] = T::mfma8(cat4(r[0], r[1], r[2], r[3]),
                                                cat2(pk[2 * kk][0], 2 * kk + 1 < NKT ? pk[(2 * kk + 1) % NKT][0] : x8{}), o[d]);
                            }
                }
            } else if (!MASK) {
                // MFMA i = (d, kt, h2), i = (d*NKT + kt)*2 + h2, two transposing reads each
                constexpr int NM = DT * NKT * 2;
                constexpr int PF = PV_PREFETCH < NM ? PV_PREFETCH : NM;
                constexpr int NB = PF + 1;
                const uint32_t vb0 = smem_addr + vofs + voff[0];
                const uint32_t vb1 = smem_addr + vofs + voff[1];
                // the two halves stay separate registers until their wait: a
                // copy into one 4-register operand before it would read them early
                i32x2 rlo[NB], rhi[NB];
                auto issue = [&](auto ic) {
                    constexpr int i = decltype(ic)::value;
                    constexpr int d = i / (2 * NKT), kt = (i / 2) % NKT, h2 = i % 2;
                    constexpr int off = (2 * kt + h2) * BLK + d * 1024;
                    rlo[i % NB] = lds_read_tr16<off>(vb0);
                    rhi[i % NB] = lds_read_tr16<off>(vb1);
                };
                static_for<PF>(issue);
                static_for<NM>([&](auto ic) {
                    constexpr int i = decltype(ic)::value;
                    constexpr int d = i / (2 * NKT), kt = (i / 2) % NKT, h2 = i % 2;
                    constexpr int ahead = 2 * ((NM - 1 - i) < (PF - 1) ? (NM - 1 - i) : (PF - 1));
                    lgkm_wait2<ahead>(rlo[i % NB], rhi[i % NB]);
                    const i32x2 lo = rlo[i % NB], hi = rhi[i % NB];
                    o[d] = T::mfma(__builtin_bit_cast(x8, (i32x4){lo[0], lo[1], hi[0], hi[1]}), pk[kt][h2], o[d]);
                    if constexpr (i + PF < NM) issue(std::integral_constant<int, i + PF>());
                });
            } else {
#pragma unroll
            for (int d = 0; d < DT; ++d) {
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt) {
#pragma unroll
                    for (int h2 = 0; h2 < 2; ++h2) {
                        if (kt < nkt_act) {
                            const RSFA_LDS char* vp = vt_lds + (2 * kt + h2) * BLK + d * 1024;
                            const i32x2 lo = __builtin_bit_cast(i32x2, T::tr_read(vp + voff[0]));
                            const i32x2 hi = __builtin_bit_cast(i32x2, T::tr_read(vp + voff[1]));
                            const x8 a = __builtin_bit_cast(x8, (i32x4){lo[0], lo[1], hi[0], hi[1]});
                            o[d] = T::mfma(a, pk[kt][h2], o[d]);
                        }
                    }
                }
            }
            }
        };
        // one key tile in LDS buffer buf: S^T, softmax update, O^T += V^T P^T
        auto tile_step = [&](int buf, int kbase, int nkt_act, auto masked) {
            f32x16 sacc[NKT];
            x8 pk[NKT][2];
            qk_part((uint32_t)(buf * BUF), kbase, nkt_act, sacc, masked, std::false_type());
            softmax_part(sacc, pk, masked);
            pv_part((uint32_t)(buf * BUF + TILE), nkt_act, pk, masked);
        };


        int j = j0;
        if constexpr (PP) {
            if (jpp > j0) {
                // Phases are cut by barriers.  Every wave runs the same code:
                //   X_t: PV(t-1) then QK(t), and the loads of K_{t+2}, V_{t+1}
                //   Y_t: softmax(t)
                // and waves 4-7 pass one extra barrier first, so while waves
                // 0-3 run X_t the others run Y_{t-1}, and while 0-3 run Y_t the
                // others run X_t.  Because of that one-phase lag, data waited
                // for (vmcnt) at some point of the code is read only after two
                // more barriers of the code, and a buffer is refilled only two
                // barriers after its last read.  With three buffers: X_t waits
                // for the loads of X_{t-1} and then refills the buffers of
                // K_{t-1} and V_{t-2}, last read in X_{t-1}; X_{t+1} reads V_t
                // and K_{t+1}.  The loads sit among the last MFMAs of the phase,
                // where they do not hold up the softmax of the other waves.
                const int grp = wave >= NW / 2 ? 1 : 0;
                // the MFMA phase's wave is issued first when both waves of a SIMD are ready
                auto prio_mfma = [&]() { __builtin_amdgcn_s_setprio(1); };
                auto prio_valu = [&]() { __builtin_amdgcn_s_setprio(0); };
                const std::false_type mask_free;

                // One X phase is a single stream of MFMAs, op m < NPV being
                // PV MFMA m (two transposing reads) and op NPV + i QK MFMA i
                // (one read); each op's reads are issued XPF ops ahead.
                constexpr int NPV = DT * NKT * 2;
                constexpr int NQK = KST * NKT;
                constexpr int XPF = PV_PREFETCH;
                constexpr int XNB = XPF + 1;
                // The row sums of P (one dependent chain of VALU adds) are left
                // to the compiler, which sinks them to the end of the next X
                // phase, unless the softmax phase is the shorter one: the MFMA
                // work of a phase grows with D, the softmax work does not.  At
                // D = 128 the softmax waves wait ~500 cycles at each barrier for
                // the MFMA waves, so the sums are pinned there (an empty asm that
                // uses l_sum before the barrier); at D = 64 the softmax phase is
                // the longer one (measured: +2 % at D = 128, -5 % at D = 64).
                constexpr bool LSUM_IN_Y = D >= 128;
                constexpr int NDMA = NSL + NSLV;  // direct loads per wave per X phase
                constexpr int DSTEP = 2;       // MFMAs between them
                // V8: rlo only, read PFV ahead (two float8 MFMAs; one is
                // shorter than an LDS read's latency), and the four reads of
                // a float8 MFMA stay live to it
                constexpr int PFV = V8 ? (V8RPM == 2 ? 4 : 8) : XPF;
                constexpr int XNBV = V8 ? PFV + V8RPM : XNB;
                i32x2 rlo[XNBV], rhi[XNB];
                i32x4 kr[XNB];
                uint32_t xa[4];  // V reads (two halves), K reads (even / odd k-steps)
                uint32_t xv[V8 && !V8_INLINE ? DT : 1];  // V8: V reads per head-dim block (V8_INLINE: the tile)
                auto x_issue = [&](auto mc) {
                    constexpr int m = decltype(mc)::value;
                    if constexpr (m < NPV) {
                        constexpr int d = m / (2 * NKT), kt = (m / 2) % NKT, h2 = m % 2;
                        if constexpr (V8) {
                            if constexpr (V8_INLINE)
                                rlo[m % XNBV] = lds_read_tr8<(2 * kt + h2) * 16 * DP>(xv[0] + v8_off(d));
                            else
                                rlo[m % XNBV] = lds_read_tr8<(2 * kt + h2) * 16 * DP>(xv[d]);
                        } else {
                            constexpr int off = (2 * kt + h2) * BLK + d * 1024;
                            rlo[m % XNB] = lds_read_tr16<off>(xa[0]);
                            rhi[m % XNB] = lds_read_tr16<off>(xa[1]);
                        }
                    } else {
                        constexpr int i = m - NPV, ss = i / NKT, kt = i % NKT;
                        kr[i % XNB] = lds_read_b128<kt * 2 * BLK + ss * 512>(xa[2 + (ss & 1)]);
                    }
                };
                // X phase of PV(tv) and, when M > NPV, QK(tv + 1); with tl >= 0 it
                // first waits for the loads of the previous X phase, then loads
                // K_{tl+1} (if tl + 1 < jpp) and V_tl (if tl < jpp).
                // LDS byte addresses of the buffers of tiles tv, tv + 1, tv + 2
                // (rotated once per tile instead of computing jj % NBUF)
                uint32_t b_tv = smem_addr + bofs(j0), b_t1 = smem_addr + bofs(j0 + 1), b_t2 = smem_addr + bofs(j0 + 2);
                // first rows of the tiles the next X phase loads (K_{tl+1}, V_tl for
                // tl = t + 2 at step t), advanced by one tile per step: left to
                // the compiler, the causal kernels rebuilt them with 64-bit
                // multiplies at every load, inside the MFMA stream
                const int64_t kstep = (int64_t)BN * p.k_sn, vstep = (int64_t)BN * p.v_sn;
                const elem* kld = kh + (j0 + 3) * kstep;
                const velem* vld = vh + (j0 + 2) * vstep;
                auto x_phase = [&](auto nm, int tv, int tl, const x8(&pk)[NKT][2], f32x16(&sacc)[NKT], auto wq, int qi, auto use_cb) {
                    constexpr int M = decltype(nm)::value;
                    constexpr int D0 = M - NDMA * DSTEP;
                    static_assert(D0 >= 0 && D0 + NDMA * DSTEP <= M, "operand stream shorter than its loads");
                    if constexpr (V8) {
#pragma unroll
                        for (int d = 0; d < (V8_INLINE ? 1 : DT); ++d) xv[d] = b_tv + TILE + (V8_INLINE ? 0u : vo8[d]);
                    } else {
                        xa[0] = b_tv + TILE + voff[0];
                        xa[1] = b_tv + TILE + voff[1];
                    }
                    xa[2] = b_t1 + koff[0];
                    xa[3] = b_t1 + koff[1];
                    static_for<M>([&](auto xc) {
                        constexpr int x = decltype(xc)::value;
                        if constexpr (x_issue_after(NPV, XPF, PFV, x) == -1) x_issue(xc);
                    });
                    const f32x16 zero = {};
                    static_for<M>([&](auto mc) {
                        constexpr int m = decltype(mc)::value;
                        constexpr int N = x_reads_pending(NPV, M, XPF, PFV, V8 ? 1 : 2, m);
                        if constexpr (m < NPV) {
                            if constexpr (V8) {
                                // read m = (d*NKT + kt)*2 + h2; every fourth ends
                                // a 64-key float8 MFMA (as in pv_part), which
                                // waits for its four reads
                                constexpr int d = m / (2 * NKT), qq = m % (2 * NKT);
                                if constexpr (V8RPM == 2 && qq == 1) {
                                    // a 32-key tile: the MFMA's upper 32 keys have P = 0
                                    i32x2 &r0 = rlo[(m - 1) % XNBV], &r1 = rlo[m % XNBV];
                                    lgkm_wait2<N>(r0, r1);
                                    o[d] = T::mfma8(cat4(r0, r1, r0, r1), cat2(pk[0][0], x8{}), o[d]);
                                    __builtin_amdgcn_sched_barrier(0);
                                } else if constexpr (V8RPM == 4 && qq % 4 == 3) {
                                    i32x2 &r0 = rlo[(m - 3) % XNBV], &r1 = rlo[(m - 2) % XNBV], &r2 = rlo[(m - 1) % XNBV],
                                          &r3 = rlo[m % XNBV];
                                    lgkm_wait4<N>(r0, r1, r2, r3);
                                    o[d] = T::mfma8(cat4(r0, r1, r2, r3), cat2(pk[qq / 2 - 1][0], pk[qq / 2][0]), o[d]);
                                    // issued here, not sunk below the next reads and waits
                                    __builtin_amdgcn_sched_barrier(0);
                                }
                            } else {
                                constexpr int d = m / (2 * NKT), kt = (m / 2) % NKT, h2 = m % 2;
                                lgkm_wait2<N>(rlo[m % XNB], rhi[m % XNB]);
                                const i32x2 lo = rlo[m % XNB], hi = rhi[m % XNB];
                                o[d] = T::mfma(__builtin_bit_cast(x8, (i32x4){lo[0], lo[1], hi[0], hi[1]}), pk[kt][h2], o[d]);
                            }
                        } else {
                            constexpr int i = m - NPV, ss = i / NKT, kt = i % NKT;
                            lgkm_wait<N>(kr[i % XNB]);
                            sacc[kt] = T::mfma(__builtin_bit_cast(x8, kr[i % XNB]), qf[ss],
                                               ss == 0 ? (DIAG_PP && decltype(use_cb)::value ? cb[DIAG_PP ? kt : 0] : zero) : sacc[kt]);
                        }
                        // the next reads: a P.V op PFV ahead, or a QK op XPF ahead
                        if constexpr (m + PFV < NPV) x_issue(std::integral_constant<int, m + PFV>());
                        if constexpr (m + XPF >= NPV && m + XPF < M) x_issue(std::integral_constant<int, m + XPF>());
                        // load q of NDMA at op D0 + q * DSTEP (q < NDMA: the wave's K
                        // slices, then its V slices)
                        if constexpr (m >= D0 && m < D0 + NDMA * DSTEP && (m - D0) % DSTEP == 0) {
                            constexpr int q = (m - D0) / DSTEP;
                            static_assert(q < NDMA, "load slot past the wave's slices");
                            if (tl >= 0) {
                                if constexpr (q == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                                // tl = tv + 2: K_{tv+3} into the buffer of tile tv, V_{tv+2}
                                if constexpr (q < NSL) {
                                    if (tl + 1 < jpp) pp_dma_at(kld, kgo, b_tv, q);
                                } else {
                                    if (tl < jpp) pp_dma_v_at(vld, b_t2 + TILE, q - NSL);
                                }
                            }
                        }
                        // QPF: half of the next task's Q loads (from load qi on),
                        // right after the phase's wait for the previous loads
                        if constexpr (decltype(wq)::value && m == D0 + 1) {
                            if (qi >= 0) static_for<NQD / 2>([&](auto qc) { dma_q(qnext, qi + decltype(qc)::value); });
                        }
                    });
                };

                // K_j0 (and Q): the first phase reads only these; V_j0 and K_j0+1
                // are waited for at the end of X_j0 (each load_k / load_v is
                // NSL (NSLV) direct loads per wave, issued in order K_j0, Q, V_j0, K_j0+1)
                static_assert(NINST % NW == 0 && NINSTV % NW == 0, "every wave issues NSL (NSLV) loads per tile");
                if (j0 + 1 < jpp)
                    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NSLV + NSL) : "memory");
                else
                    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NSLV) : "memory");
                if constexpr (QPF) {
                    // the next ticket (its atomic is done), published by the barrier
                    if (ctr && tid == 0) {
                        asm volatile("" : "+v"(nxt));  // after the wait above
                        *tslot = nxt;
                    }
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                }
                if constexpr (QPF) {
                    if (q_dma) read_q();  // this wave's own loads, waited for above
                }
                phase_barrier();  // waves 0-3: X_j0; waves 4-7 wait one phase more
                if constexpr (QPF) {
                    // the next task; when this task has at least four ping-pong
                    // tiles and the next one a whole query block, its Q is loaded
                    // in the phases X_{j0+2} and X_{j0+3}
                    const int tn = pair_continues(p, qu, t) ? t + 1
                                   : task_of_ticket(qu, ctr ? __builtin_amdgcn_readfirstlane(*tslot)
                                                            : ticket_of_task(qu, t) + qu.nwg);
                    if (ctr) t_next = tn;
                    if (tn < qu.ntask && jpp - j0 >= 4) {
                        int nbh, nmb;
                        decode_task<CAUSAL>(p, qu, tn, nbh, nmb);
                        if ((nmb + 1) * BM <= n) {
                            const int nb = nbh / p.H, nh = nbh - nb * p.H;
                            qpf_do = true;
                            qnext = qg + nb * p.q_sz + nh * p.q_sh + (int64_t)nmb * BM * p.q_sm;
                        }
                    }
                }
                if (grp) phase_barrier();  // X_j0: QK only, then the loads of K_{j0+2}, V_{j0+1}
                prio_mfma();
                f32x16 sacc[NKT];
                qk_part(bofs(j0), j0 * BN, NKT, sacc, mask_free, std::true_type());
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // V_j0, K_j0+1, published by the next barrier
                if (j0 + 2 < jpp) load_k(j0 + 2);
                if (j0 + 1 < jpp) load_v(j0 + 1);
                int t = j0;
                // one step: Y_t, then X_{t+1} (WQ: with the slots of the Q loads
                // of the next task, from load qi on when qi >= 0)
                // the loads of an X phase without its MFMAs (tl = t + 2)
                auto x_loads = [&](int tl) {
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
                    for (int q = 0; q < NSL; ++q)
                        if (tl + 1 < jpp) pp_dma_at(kld, kgo, b_tv, q);
#pragma unroll
                    for (int q = 0; q < NSLV; ++q)
                        if (tl < jpp) pp_dma_v_at(vld, b_t2 + TILE, q);
                };
                // DIAG_VM: steps that may reach the diagonal block (diag) mask
                // the scores a wave's rows do not see.  A key tile wholly above
                // this wave's rows has P = 0: from the first such tile on (but
                // the last tile, whose masked softmax is harmless) the wave
                // runs steps without its softmax, P.V and the next tile's S^T
                // (above its rows too), keeping only the loads; when the four
                // waves of a group skip, the phase lasts as long as the other
                // group's work.
                auto tile_hidden = [&](int tt) { return tt * BN > wq_hi; };
                auto pp_advance = [&]() {
                    kld += kstep;
                    vld += vstep;
                    const uint32_t b_old = b_tv;
                    b_tv = b_t1;
                    b_t1 = b_t2;
                    b_t2 = b_old;
                };
                auto pp_step = [&](auto wq, int qi, auto use_cb, auto diag) {
                    phase_barrier();  // Y_t
                    prio_valu();
                    x8 pk[NKT][2];
                    if constexpr (DIAG_VM && decltype(diag)::value) vmask(sacc, t);
                    softmax_part(sacc, pk, mask_free);
                    if constexpr (LSUM_IN_Y) asm volatile("" : "+v"(l_sum));
                    if constexpr (DIAG_PP && decltype(use_cb)::value) {
                        // bias of tile t+1 where it changes: onto the diagonal, or past it
#pragma unroll
                        for (int kt = 0; kt < NKT; ++kt) {
                            const int rel = cb_rel(t + 1, kt);
                            if (rel == 0 || (rel > 0 && rel - NKT <= 0)) cb_fill(kt, rel);
                        }
                    }
                    phase_barrier();  // X_{t+1}
                    prio_mfma();
                    x_phase(std::integral_constant<int, NPV + NQK>(), t, t + 2, pk, sacc, wq, qi, use_cb);
                    pp_advance();
                };
                // a step of a tile hidden from this wave: the barriers and loads only
                auto pp_skip_step = [&]() {
                    phase_barrier();  // Y_t
                    prio_valu();
                    phase_barrier();  // X_{t+1}
                    prio_mfma();
                    x_loads(t + 2);
                    pp_advance();
                };
                if constexpr (QPF) {
                    // a task that loads the next task's Q (in X_{j0+2} and
                    // X_{j0+3}) runs its first three steps in a copy with the
                    // load slots; the loop below carries no check for them
                    // (a check in every MFMA phase cost more than the loads save)
                    if (qpf_do)
                        for (; t < j0 + 3; ++t)
                            pp_step(std::true_type(), t == j0 ? -1 : (t - j0 - 1) * (NQD / 2), std::true_type(),
                                    std::bool_constant<DIAG_VM>());  // (may reach the diagonal block: masked)
                }
                if constexpr (DIAG_PP) {
                    // steps whose key tile lies below the whole query block run
                    // a copy without the bias blocks (their bias is 0): with
                    // the 32 bias VGPRs free the softmax phase is ~70 cycles
                    // shorter; the bias of the next tile is then filled whole
                    const int jd = m0 / BN;  // first key tile of the diagonal block
                    for (; t + 1 < jpp && t + 1 < jd; ++t) pp_step(std::false_type(), -1, std::false_type(), std::false_type());
#pragma unroll
                    for (int kt = 0; kt < NKT; ++kt) cb_fill(kt, cb_rel(t + 1, kt));
                }
                if constexpr (DIAG_VM) {
                    // steps below the diagonal block need no mask and skip nothing
                    // (separate loops: a skip branch inside the step made the
                    // register allocator spill ~400 VGPRs; whether a tile is
                    // hidden changes once per wave, so every wave still runs
                    // the same steps and barriers)
                    const int jd = m0 / BN;
                    for (; t + 1 < jpp && t < jd; ++t) pp_step(std::false_type(), -1, std::true_type(), std::false_type());
                    for (; t + 1 < jpp && !tile_hidden(t); ++t) pp_step(std::false_type(), -1, std::true_type(), std::true_type());
                    for (; t + 1 < jpp; ++t) pp_skip_step();
                } else if constexpr (DIAG_PP) {
                    // the same skip of hidden diagonal tiles (bias blocks mask the others)
                    for (; t + 1 < jpp && !tile_hidden(t); ++t) pp_step(std::false_type(), -1, std::true_type(), std::false_type());
                    for (; t + 1 < jpp; ++t) pp_skip_step();
                } else {
                    for (; t + 1 < jpp; ++t) pp_step(std::false_type(), -1, std::true_type(), std::false_type());
                }
                {
                    phase_barrier();  // Y of the last tile
                    prio_valu();
                    x8 pk[NKT][2];
                    if constexpr (DIAG_VM) vmask(sacc, t);
                    if constexpr (DIAG_PP) {
                        // a last tile hidden from this wave: its S^T was not
                        // formed (skipped steps), and its P must be 0
                        const bool hid = tile_hidden(t);
#pragma unroll
                        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                            for (int i = 0; i < 16; ++i) sacc[kt][i] = hid ? -INFINITY : sacc[kt][i];
                    }
                    softmax_part(sacc, pk, mask_free);
                    if constexpr (LSUM_IN_Y) asm volatile("" : "+v"(l_sum));
                    phase_barrier();  // its PV
                    prio_mfma();
                    x_phase(std::integral_constant<int, NPV>(), t, -1, pk, sacc, std::false_type(), -1, std::true_type());
                    prio_valu();
                }
                if (!grp) phase_barrier();
                // realigned; the remaining tiles use buffers 0 and 1
                __syncthreads();
                j = jpp;
                if (j < j1) load_tile(j, 0);
            }
        }

        // Key tiles [jr, ju) are visible to every row of this wave (mask-free
        // body); [ju, j1) straddle the causal diagonal or the sequence end.
        // Both loops run the same barrier sequence in every wave.
        const int jr = j;
        int ju = min(j1, (vis_lo + 1) / BN);
        ju = max(ju, jr);
        for (; j < ju; ++j) {
            const int buf = (j - jr) & 1;
            wait_loads_and_sync();
            if (j + 1 < j1) load_tile(j + 1, buf ^ 1);
            tile_step(buf, j * BN, NKT, std::integral_constant<bool, false>());
        }
        for (; j < j1; ++j) {
            const int buf = (j - jr) & 1;
            wait_loads_and_sync();
            if (j + 1 < j1) load_tile(j + 1, buf ^ 1);
            const int kbase = j * BN;
            if (kbase <= vis_hi) {
                const int nkt_act = min(NKT, (vis_hi - kbase) / 32 + 1);
                tile_step(buf, kbase, nkt_act, std::integral_constant<bool, true>());
            }
        }

        // epilogue
        // (QPF: the next task's Q loads are waited for here, the barrier below
        // publishes them)
        if constexpr (QPF) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const float lt = swap_sum(l_sum);
        const float inv = 1.0f / lt;
        // O leaves through LDS: in the accumulator layout a lane holds 8 bytes
        // of a row per (d, a), so a direct store instruction writes 32 rows x
        // 16 bytes, and a CU needs ~64 cycles per such instruction (measured:
        // the second group of waves waited ~4k cycles per task behind the
        // first group's stores); staged row-major, each store instruction
        // writes whole 16-byte chunks of 64 / (OCOLS / 8) consecutive rows
        // (+2.5 to +3.6 % on C2, B=128, C3 and D=64).  OCOLS columns of the
        // workgroup's rows go through the K/V buffers per round: all D when
        // they fit, else half or a quarter of them (D = 256).
        constexpr int OCOLS = NW * 32 * (2 * D + 16) <= NBUF * BUF ? D
                              : NW * 32 * (D + 16) <= NBUF * BUF ? D / 2 : D / 4;
        constexpr int OROW = 2 * OCOLS + 16;  // bytes per staged row (16-byte pad)
        constexpr bool OSTAGE = NW * 32 * OROW <= NBUF * BUF && OCOLS >= 16;
        if constexpr (MODE == MODE_PREFIX) {
            // hand (m, l) and the un-normalised accumulator to the diagonal
            // launch in fp32 (the reference rounds acc to the input dtype
            // into O, 353)
            if (hh == 0) {
                p.state[srow] = m_use;
                p.state[(int64_t)p.num_tasks * BM + srow] = lt;
            }
#pragma unroll
            for (int d = 0; d < DT; ++d)
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    const int col = 32 * d + 8 * a + 4 * hh;
                    if (col < D)
                        *(float4*)(acc_row + col) =
                            make_float4(o[d][4 * a + 0], o[d][4 * a + 1], o[d][4 * a + 2], o[d][4 * a + 3]);
                }
        } else if constexpr (OSTAGE) {
            __syncthreads();  // every wave is done with the K/V tiles
            // a wave's own region: its reads of one round precede (in LDS
            // order) its writes of the next, so rounds need no barrier
            RSFA_LDS char* const ow = smem + wave * (32 * OROW);
            constexpr int CH = OCOLS / 8;  // 16-byte chunks per staged row
            constexpr int RPI = 64 / CH;   // rows per store instruction
            const int rr = lane / CH, cc = (lane % CH) * 8;
            const int row0 = m0 + wave * 32;
#pragma unroll
            for (int hf = 0; hf < D / OCOLS; ++hf) {
#pragma unroll
                for (int d = 0; d < DT; ++d)
#pragma unroll
                    for (int a = 0; a < 4; ++a) {
                        const int col = 32 * d + 8 * a + 4 * hh;
                        if (col < D && col / OCOLS == hf) {
                            x4 v4;
#pragma unroll
                            for (int e = 0; e < 4; ++e) v4[e] = (elem)(o[d][4 * a + e] * inv);
                            *(RSFA_LDS x4*)(ow + l32 * OROW + (col - hf * OCOLS) * 2) = v4;
                        }
                    }
#pragma unroll
                for (int it = 0; it < 32 / RPI; ++it) {
                    const int r = it * RPI + rr;
                    const x8 v = *(const RSFA_LDS x8*)(ow + r * OROW + cc * 2);
                    if (row0 + r < n) *(x8*)(ob + (int64_t)(row0 + r) * p.o_sm + hf * OCOLS + cc) = v;
                }
            }
            if (p.lse && hh == 0 && qrow < n)
                p.lse[(int64_t)bh * n + qrow] = (m_use + __log2f(lt)) * 0.69314718055994530942f;
        } else if (qrow < n) {
#pragma unroll
            for (int d = 0; d < DT; ++d)
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    const int col = 32 * d + 8 * a + 4 * hh;
                    if (col < D) {
                        x4 v4;
#pragma unroll
                        for (int e = 0; e < 4; ++e) v4[e] = (elem)(o[d][4 * a + e] * inv);
                        *(x4*)(ob + (int64_t)qrow * p.o_sm + col) = v4;
                    }
                }
            if (p.lse && hh == 0)
                p.lse[(int64_t)bh * n + qrow] = (m_use + __log2f(lt)) * 0.69314718055994530942f;
        }

        if (ctr) {
            __syncthreads();
            if (QPF && t_next >= 0) {
                t = t_next;
            } else if (pair_continues(p, qu, t)) {
                t = t + 1;
            } else {
                if (tid == 0) *tslot = nxt;
                __syncthreads();
                t = task_of_ticket(qu, *tslot);
                if constexpr (QPF) __syncthreads();  // read before the next task writes the slot
            }
        } else {
            __syncthreads();
            t = pair_continues(p, qu, t) ? t + 1 : task_of_ticket(qu, ticket_of_task(qu, t) + qu.nwg);
        }
        qready = qpf_do;
    }

    // The workgroup holding the last ticket handed out by its queue returns the
    // counter to zero for the next launch on this stream: every workgroup of
    // the queue draws exactly one ticket >= ntask, so that ticket is
    // ntask + nwg - 1.
    if (ctr && tid == 0 && ticket_of_task(qu, t) == ticket_of_task(qu, qu.ntask) + qu.nwg - 1) atomicExch(ctr, 0u);
}

}  // namespace rsfa
