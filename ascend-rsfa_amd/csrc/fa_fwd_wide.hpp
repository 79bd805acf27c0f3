// FlashAttention-2 forward for MI355X (gfx950): the one-wave-per-SIMD kernel.
//
// Reference algorithm: Dell710000/ascend-rsfa ascend_rsfa/flash_attention_forward.py
//   _attn_fwd (271-404) and _attn_fwd_inner (163-226), non-causal.
//
// Work decomposition
//   One task = (batch b, head h, query block mb) of BM = 256 query rows, run by
//   a workgroup of 4 waves, one per SIMD of a CU (occupancy 1: each wave has
//   the whole register file of its SIMD, 512 registers).  Wave w owns the 64
//   rows [mb*BM + 64w, +64) as two 32-row MFMA row blocks that share every K
//   and V operand read from LDS, which halves the LDS operand traffic per MFMA
//   against 32 rows per wave.
//
// Software pipeline (one wave, no partner wave to hide latency)
//   Key tiles of BN keys.  Step t issues the MFMAs of S(t+2) = Q K(t+2)^T and
//   then of O += P(t) V(t) (each K/V operand read feeding two MFMAs) and,
//   interleaved one slot per MFMA, the VALU work of the online softmax of
//   S(t+1) into P(t+1), so the matrix cores and the VALU run side by side in
//   one instruction stream.  A wave issues MFMAs faster than they run; the
//   softmax at the start of step t reads S(t+1), which the first half of step
//   t - 1 produced, so it never waits for the MFMA queue to drain.  The rare rescale of O (a row max that grows by
//   more than RESCALE_SLACK) is applied after the step's PV MFMAs.
//   K and V tiles sit in four LDS buffers (tile j in buffer j % 4); step t
//   loads tile t + 3 into the buffer of tile t - 1, which step t - 1 finished.
//   One barrier per step (after each wave waited for its own loads of the
//   previous step) publishes the loads and frees the buffer.
//
// Operand layouts are those of fa_fwd_kernel.hpp (S^T = K Q^T and
// O^T = V^T P^T with v_mfma_f32_32x32x16, the same swizzled LDS tiles and
// direct global->LDS loads).
#pragma once

#include "fa_fwd_kernel.hpp"

namespace rsfa {

#ifndef RSFA_WIDE
#define RSFA_WIDE 1
#endif
// LDS operand reads issued this many operands (two MFMAs each) ahead
#ifndef RSFA_WIDE_PF
#define RSFA_WIDE_PF 3
#endif
// first slot of the step's direct loads, and slots between them
#ifndef RSFA_WIDE_DMA0
#define RSFA_WIDE_DMA0 2
#endif
#ifndef RSFA_WIDE_DMAS
#define RSFA_WIDE_DMAS 4
#endif

// Whether the one-wave kernel exists for a head dim (non-causal, key tiles of
// 64 whole keys).
constexpr bool wide_supported(int d) { return RSFA_WIDE && d == 128; }

// A pipeline step's work, as template flags: bit 0 PV, bit 1 QK, bit 2
// softmax, bits 3-4 the loads (0 none, 1 always, 2 when `tl` is a tile).
// bit 5 set: the step starts without the wait and barrier (the second step
// of a pair in the steady loop).
constexpr int wide_step(bool pv, bool qk, bool sm, int load, bool nosync = false) {
    return (pv ? 1 : 0) | (qk ? 2 : 0) | (sm ? 4 : 0) | (load << 3) | (nosync ? 32 : 0);
}
struct WideStep {
    bool pv, qk, sm, sync;
    int load;
    constexpr explicit WideStep(int f) : pv(f & 1), qk(f & 2), sm(f & 4), sync(!(f & 32)), load((f >> 3) & 3) {}
};

// VALU work units of one softmax of a BN = 32 * NKT key tile, in issue order,
// and the slot (MFMA) each is issued after.  Units: 8 * NKT max3 steps per row
// block (the two row blocks' chains interleaved), a lane-pair max swap per row
// block, the running-max update per row block, then 8 * NKT units per row
// block of two exp2s, one conversion pair and the row-sum update (interleaved
// across row blocks).
template <int NKT, int RB>
struct SmUnits {
    static constexpr int NMAX = 8 * NKT, NEXP = 8 * NKT;
    static constexpr int COUNT = RB * NMAX + RB + RB + RB * NEXP;
    static constexpr int weight(int u) { return u < RB * NMAX ? 1 : u < RB * NMAX + RB ? 2 : 6; }
    static constexpr int total() {
        int w = 0;
        for (int u = 0; u < COUNT; ++u) w += weight(u);
        return w;
    }
    // slot of unit u when the step has `slots` MFMAs (units spread by weight)
    static constexpr int slot(int u, int slots) {
        int w = 0;
        for (int v = 0; v < u; ++v) w += weight(v);
        const int s = slots > 0 ? (w * slots) / total() : 0;
        return s < slots ? s : (slots > 0 ? slots - 1 : 0);
    }
};

// 16 bytes from global memory into VGPRs, or straight into AGPRs (the Q^T
// fragments only ever feed MFMAs).  Issued from asm so the compiler does not
// wait for them before the direct tile loads issued after them (vmcnt counts
// in issue order); the caller waits (wait_tiles) before the first use.
template <class X8>
__device__ __forceinline__ X8 load_vgpr(const void* ptr) {
    X8 r;
    asm volatile("s_nop 4\n\tglobal_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(ptr) : "memory");
    return r;
}
template <class X8>
__device__ __forceinline__ X8 load_agpr(const void* ptr) {
    X8 r;
    // s_nop 4: the same guard as dma16 (the compiler adds no wait states for asm)
    asm volatile("s_nop 4\n\tglobal_load_dwordx4 %0, %1, off" : "=a"(r) : "v"(ptr) : "memory");
    return r;
}
template <class T, int D, int BN, int NBUF, int RB>
__global__ void __launch_bounds__(256 * (3 - RB)) __attribute__((amdgpu_waves_per_eu(3 - RB, 3 - RB)))
fa_fwd_wide_kernel(FwdParams p) {
    typedef typename T::elem elem;
    typedef typename T::x8 x8;
    typedef typename T::x2 x2;
    typedef typename T::x4 x4;

    static_assert(RB == 1 || RB == 2, "32 or 64 query rows per wave");
    constexpr int NW = 8 / RB;          // waves: 1 (RB 2) or 2 (RB 1) per SIMD
    constexpr int NKT = BN / 32;        // 32-key sub-tiles
    constexpr int BM = NW * RB * 32;    // query rows per task
    constexpr int KST = D / 16;         // k-steps of S
    constexpr int DT = D / 32;          // 32-row tiles of O^T
    constexpr int CPR = D / 8;          // 16-byte chunks per row
    constexpr int BLK = 32 * D;         // bytes of a 16-row block
    constexpr int TILE = BN * D * 2;    // bytes of a K (or V) tile
    constexpr int BUF = 2 * TILE;       // K + V
    typedef SmUnits<NKT, RB> SU;
    constexpr int WR = 32 * RB;         // query rows per wave
    static_assert(BN == 32 || BN == 64, "key tiles of 32 or 64 keys");
    static_assert(NBUF >= 8 && (NBUF & (NBUF - 1)) == 0, "a power-of-two ring of at least eight tiles");
    constexpr int NINST = BN * CPR / 64;  // 1-KB direct loads per K (or V) tile
    constexpr int NSL = NINST / NW;       // of them per wave
    static_assert(NINST % NW == 0, "a tile must split evenly over the waves");
    static_assert(D == 128, "the one-wave kernel is instantiated for head dim 128");

    __shared__ __attribute__((aligned(1024))) char smem_raw[NBUF * BUF];
    __shared__ int s_ticket;
    RSFA_LDS char* const smem = (RSFA_LDS char*)smem_raw;
    const uint32_t smem_addr = (uint32_t)(uintptr_t)smem;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int hh = lane >> 5;
    const int l32 = lane & 31;
    const int l16 = lane & 15;

    // LDS read offsets of the K (A of S^T) and V (A of O^T, transposing) operands
    uint32_t koff[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) koff[e] = (l32 >> 4) * BLK + hh * 256 + ((l16 ^ (8 * e + 4 * hh)) * 16);
    const int vg = (lane >> 4) & 1;
    const int vcc = 2 * vg + ((l16 >> 1) & 1);
    uint32_t voff[2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
        voff[u] = vcc * 256 + (((8 * u + 4 * hh + (l16 >> 2)) ^ (4 * vcc)) * 16) + 8 * (l16 & 1);

    // loader: per-lane byte offsets of this wave's slices of a tile
    const int ld_rib = l16 ^ (4 * ((lane >> 4) & 3));
    const int ld_chl = lane >> 4;
    uint32_t kgo[NSL], vgo[NSL];
#pragma unroll
    for (int sl = 0; sl < NSL; ++sl) {
        const int w = sl * NW + wave;
        const int blk = (w * 64) / (16 * CPR);
        const int cg = ((w * 64) % (16 * CPR)) / 64;
        kgo[sl] = (uint32_t)(((16 * blk + ld_rib) * p.k_sn + cg * 32 + ld_chl * 8) * 2);
        vgo[sl] = (uint32_t)(((16 * blk + ld_rib) * p.v_sn + cg * 32 + ld_chl * 8) * 2);
    }

    const float c = p.c;
    const int qsign = p.neg ? (int)0x80008000u : 0;
    const elem* const qg = (const elem*)p.q;
    const elem* const kg = (const elem*)p.k;
    const elem* const vgp = (const elem*)p.v;
    elem* const og = (elem*)p.o;

    const Queue qu = make_queue<false>(p);
    uint32_t* const ctr = p.ticket ? p.ticket + 16 * qu.x : nullptr;
    int t;
    if (ctr) {
        if (tid == 0) s_ticket = (int)atomicAdd(ctr, 1u);
        __syncthreads();
        t = s_ticket;
    } else {
        t = qu.rank;
    }

    while (t < qu.ntask) {
        int nxt = 0;
        if (ctr && tid == 0) nxt = (int)atomicAdd(ctr, 1u);

        int bh, mb;
        decode_task<false>(p, qu, t, bh, mb);
        const int b = bh / p.H;
        const int h = bh - b * p.H;
        const int n = p.n_ctx;
        const int m0 = mb * BM;
        const int nt = n / BN;  // key tiles (the launcher guarantees n % BN == 0)

        const elem* qb = qg + b * p.q_sz + h * p.q_sh;
        const elem* kh = kg + b * p.k_sz + h * p.k_sh;
        const elem* vh = vgp + b * p.v_sz + h * p.v_sh;
        elem* ob = og + b * p.o_sz + h * p.o_sh;

        // slice sl of this wave's share of tile j (K and V) into the buffer at dst
        auto load_tile = [&](int j, uint32_t dst) {
            const elem* kt0 = kh + (int64_t)(j * BN) * p.k_sn;
            const elem* vt0 = vh + (int64_t)(j * BN) * p.v_sn;
#pragma unroll
            for (int sl = 0; sl < NSL; ++sl) {
                const int w = sl * NW + wave;
                dma16(kt0, kgo[sl], dst + w * 1024);
                dma16(vt0, vgo[sl], dst + w * 1024 + TILE);
            }
        };
        // Q^T fragments of both row blocks (B operands of S^T), loaded first
        x8 qf[RB][KST];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int row = min(m0 + wave * WR + rb * 32 + l32, n - 1);
#pragma unroll
            for (int s = 0; s < KST; ++s) {
                const elem* src = qb + (int64_t)row * p.q_sm + (2 * s + hh) * 8;
                // 64 rows per wave: Q^T in AGPRs (no room in the VGPRs); 32
                // rows: VGPRs, so the compiler needs no AGPR share
                if constexpr (RB == 2)
                    qf[rb][s] = load_agpr<x8>(src);
                else
                    qf[rb][s] = load_vgpr<x8>(src);
            }
        }
        // LDS buffer of tile j.  Step s loads tile s + LD into the buffer of
        // tile s - 2 (LD = NBUF - 2); the first LD tiles are loaded here.
        // Loading two tiles behind lets the steady loop synchronise once per
        // pair of steps: the barrier before step s frees the buffers of the
        // tiles s - 2 and s - 1 that steps s and s + 1 refill.
        constexpr int LD = NBUF - 2;
        auto buf = [&](int j) { return smem_addr + (uint32_t)((j & (NBUF - 1)) * BUF); };
        const int nt0 = min(nt, LD);
        for (int j = 0; j < nt0; ++j) load_tile(j, buf(j));
        // Waits until this wave's loads of a tile are done while the loads of
        // the `newer` tiles issued after it may still be in flight (vmcnt
        // counts loads in issue order; every tile is 2 * NSL loads per wave).
        auto wait_tiles = [&](int newer) {
            bool done = false;
            static_for<LD>([&](auto kc) {
                constexpr int k = LD - 1 - decltype(kc)::value;
                if (!done && newer >= k) {
                    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(k * 2 * NSL) : "memory");
                    done = true;
                }
            });
        };
        // Q (issued before the tiles) and tile 0.  The loads are asm: the
        // empty asm after the wait takes every fragment as an operand, so no
        // read of Q can be placed before the wait.
        wait_tiles(nt0 - 1);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            if constexpr (RB == 2)
                asm volatile(""
                             : "+a"(qf[rb][0]), "+a"(qf[rb][1]), "+a"(qf[rb][2]), "+a"(qf[rb][3]), "+a"(qf[rb][4]),
                               "+a"(qf[rb][5]), "+a"(qf[rb][6]), "+a"(qf[rb][7]));
            else
                asm volatile(""
                             : "+v"(qf[rb][0]), "+v"(qf[rb][1]), "+v"(qf[rb][2]), "+v"(qf[rb][3]), "+v"(qf[rb][4]),
                               "+v"(qf[rb][5]), "+v"(qf[rb][6]), "+v"(qf[rb][7]));
        }
        if (qsign) {
            // a negative sm_scale: q negated (exact), once per task
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int s = 0; s < KST; ++s) {
                    qf[rb][s] = __builtin_bit_cast(x8, __builtin_bit_cast(i32x4, qf[rb][s]) ^ qsign);
                }
        }

        f32x16 o[RB][DT];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int d = 0; d < DT; ++d) o[rb][d] = f32x16{};
        float m_use[RB], l_sum[RB], alpha[RB], mx[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            m_use[rb] = -INFINITY;
            l_sum[rb] = 0.0f;
            alpha[rb] = 1.0f;
            mx[rb] = 0.0f;
        }


        // One pipeline step (see the file comment).  bv: buffer of the V tile
        // of PV, bk: buffer of the K tile of QK, bl: where tile tl goes.
        // newer: tiles loaded after the newest one the step reads (wait_tiles).
        auto step = [&](auto cfg, auto newer, uint32_t bv, uint32_t bk, const x8(&ppv)[RB][NKT][2],
                        f32x16(&sqk)[RB][NKT], f32x16(&ssm)[RB][NKT], x8(&psm)[RB][NKT][2], int tl,
                        uint32_t bl) -> bool {
            constexpr WideStep C(decltype(cfg)::value);
            constexpr int NPV = C.pv ? DT * NKT * 2 : 0;  // V operands (two transposing reads each)
            constexpr int NQK = C.qk ? KST * NKT : 0;     // K operands (one read each)
            constexpr int NOPS = NPV + NQK;
            constexpr int NSLOT = RB * NOPS;              // MFMAs: each operand feeds every row block
            constexpr int PF = RSFA_WIDE_PF < NOPS ? RSFA_WIDE_PF : NOPS;
            constexpr int NB = PF + 1;
            const uint32_t va0 = bv + TILE + voff[0], va1 = bv + TILE + voff[1];
            const uint32_t ka0 = bk + koff[0], ka1 = bk + koff[1];
            i32x2 rlo[NB], rhi[NB];
            i32x4 kr[NB];
            bool need_any = false;
            float msub[RB];
            // Operand i: QK operands (one read each) first, then PV operands
            // (two transposing reads each).  The reads are ordinary LDS loads
            // the compiler sees (not asm): it then inserts the lgkmcnt waits
            // itself and, when it reuses the registers of an operand the
            // MFMA just issued for a new read, the wait states an in-flight
            // MFMA needs before its source registers are overwritten.
            const RSFA_LDS char* const kp0 = smem + (ka0 - smem_addr);
            const RSFA_LDS char* const kp1 = smem + (ka1 - smem_addr);
            const RSFA_LDS char* const vp0 = smem + (va0 - smem_addr);
            const RSFA_LDS char* const vp1 = smem + (va1 - smem_addr);
            auto issue = [&](auto ic) {
                constexpr int i = decltype(ic)::value;
                if constexpr (i < NQK) {
                    constexpr int s = i / NKT, kt = i % NKT;
                    kr[i % NB] = *(const RSFA_LDS i32x4*)(((s & 1) ? kp1 : kp0) + kt * 2 * BLK + s * 512);
                } else {
                    constexpr int j = i - NQK, d = j / (2 * NKT), kt = (j / 2) % NKT, h2 = j % 2;
                    constexpr int off = (2 * kt + h2) * BLK + d * 1024;
                    rlo[i % NB] = __builtin_bit_cast(i32x2, T::tr_read(vp0 + off));
                    rhi[i % NB] = __builtin_bit_cast(i32x2, T::tr_read(vp1 + off));
                }
            };
            // softmax unit u of S = ssm into P = psm
            auto unit = [&](auto uc) {
                constexpr int u = decltype(uc)::value;
                constexpr int NMX = SU::NMAX;
                if constexpr (u < RB * NMX) {
                    constexpr int rb = u % RB, i = u / RB, kt = i / 8, r = 2 * (i % 8);
                    if constexpr (i == 0)
                        mx[rb] = __builtin_elementwise_maximum(ssm[rb][0][0], ssm[rb][0][1]);
                    else
                        mx[rb] = __builtin_elementwise_maximum(
                            __builtin_elementwise_maximum(mx[rb], ssm[rb][kt][r]), ssm[rb][kt][r + 1]);
                } else if constexpr (u < RB * NMX + RB) {
                    constexpr int rb = u - RB * NMX;
                    mx[rb] = swap_max(mx[rb]);
                } else if constexpr (u < RB * NMX + 2 * RB) {
                    constexpr int rb = u - RB * NMX - RB;
                    const float m_tile = mx[rb] * c;
                    const bool need = m_tile > m_use[rb] + RESCALE_SLACK;
                    const float m_new = need ? m_tile : m_use[rb];
                    alpha[rb] = __builtin_amdgcn_exp2f(m_use[rb] - m_new);
                    l_sum[rb] *= alpha[rb];
                    need_any |= __builtin_amdgcn_ballot_w64(need) != 0;
                    m_use[rb] = m_new;
                    msub[rb] = m_new;
                } else {
                    constexpr int v = u - RB * NMX - 2 * RB, rb = v % RB, i = v / RB;
                    constexpr int kt = i / 8, h2 = (i / 4) % 2, e = i % 4;
                    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(ssm[rb][kt][8 * h2 + 2 * e], c, -msub[rb]));
                    const float p1 =
                        __builtin_amdgcn_exp2f(__builtin_fmaf(ssm[rb][kt][8 * h2 + 2 * e + 1], c, -msub[rb]));
                    x2 pr = T::cvt2(p0, p1);
                    if constexpr (T::p8)
                        l_sum[rb] += p0 + p1;
                    else
                        l_sum[rb] = T::dot2(pr, T::ones2(), l_sum[rb]);
                    // P and the row sum are first read in the next step, past
                    // the rescale branch; the empty asm keeps the compiler from
                    // sinking this unit's VALU work out of its MFMA slot.
                    asm volatile("" : "+v"(pr), "+v"(l_sum[rb]));
                    psm[rb][kt][h2][2 * e] = pr[0];
                    psm[rb][kt][h2][2 * e + 1] = pr[1];
                }
            };
            auto units_of_slot = [&](auto sc) {
                constexpr int sl = decltype(sc)::value;
                if constexpr (C.sm) {
                    static_for<SU::COUNT>([&](auto uc) {
                        constexpr int u = decltype(uc)::value;
                        if constexpr (SU::slot(u, NSLOT) == sl) unit(uc);
                    });
                }
            };

            if constexpr (C.sync) {
                if constexpr (std::is_same<decltype(newer), int>::value)
                    wait_tiles(newer);
                else
                    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(decltype(newer)::value * 2 * NSL) : "memory");
                phase_barrier();
            }
            if constexpr (NOPS > 0) {
                static_for<PF>(issue);
                static_for<NSLOT>([&](auto sc) {
                    constexpr int sl = decltype(sc)::value;
                    constexpr int i = sl / RB, rb = sl % RB;
                    if constexpr (i < NQK) {
                        constexpr int s = i / NKT, kt = i % NKT;
                        sqk[rb][kt] = T::mfma(__builtin_bit_cast(x8, kr[i % NB]), qf[rb][s],
                                              s == 0 ? f32x16{} : sqk[rb][kt]);
                    } else {
                        constexpr int j = i - NQK, d = j / (2 * NKT), kt = (j / 2) % NKT, h2 = j % 2;
                        const i32x2 lo = rlo[i % NB], hi = rhi[i % NB];
                        o[rb][d] = T::mfma(__builtin_bit_cast(x8, (i32x4){lo[0], lo[1], hi[0], hi[1]}),
                                           ppv[rb][kt][h2], o[rb][d]);
                    }
                    if constexpr (rb == RB - 1 && i + PF < NOPS) issue(std::integral_constant<int, i + PF>());
                    units_of_slot(sc);
                    if constexpr (C.load != 0 && sl >= RSFA_WIDE_DMA0 && (sl - RSFA_WIDE_DMA0) % RSFA_WIDE_DMAS == 0 &&
                                  (sl - RSFA_WIDE_DMA0) / RSFA_WIDE_DMAS < 2 * NSL) {
                        constexpr int q = (sl - RSFA_WIDE_DMA0) / RSFA_WIDE_DMAS;
                        if (C.load == 1 || tl < nt) {
                            const int64_t row0 = (int64_t)tl * BN;
                            if constexpr (q < NSL)
                                dma16(kh + row0 * p.k_sn, kgo[q], bl + (q * NW + wave) * 1024);
                            else
                                dma16(vh + row0 * p.v_sn, vgo[q - NSL], bl + ((q - NSL) * NW + wave) * 1024 + TILE);
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                });
            } else if constexpr (C.sm) {
                static_for<SU::COUNT>(unit);
            }
            return need_any;
        };
        auto rescale_o = [&]() {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int d = 0; d < DT; ++d)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[rb][d][r] *= alpha[rb];
        };
#define RSFA_STEP(PV_, QK_, SM_, LD_) std::integral_constant<int, wide_step(PV_, QK_, SM_, LD_)>()

        f32x16 sA[RB][NKT], sB[RB][NKT];
        x8 pA[RB][NKT][2], pB[RB][NKT][2];
        // prologue: S(0) = QK(0); then S(1) = QK(1) beside the softmax of S(0)
        // (the first running max never rescales O, which is still zero)
        step(RSFA_STEP(false, true, false, 0), nt0 - 1, 0, buf(0), pA, sA, sB, pB, 0, 0);
        if (nt > 1) {
            step(RSFA_STEP(false, true, true, 0), nt0 - 2, 0, buf(1), pA, sB, sA, pA, 0, 0);
            // state: P(s) in pA, S(s+1) in sB.  Step s: PV(s) from pA, QK(s+2)
            // into sA, softmax of S(s+1) in sB into pB, load of tile s+LD;
            // then the same with A and B swapped.  Before step s the tiles
            // 0 .. min(nt, s + LD) - 1 have been loaded; a step with QK reads
            // K(s+2), one without reads V(s) last.
            auto newer_qk = [&](int s) { return min(nt, s + LD) - 1 - (s + 2); };
            auto newer_pv = [&](int s) { return min(nt, s + LD) - 1 - s; };
            int s = 0;
            // Steady pairs (both steps load a tile): one wait and barrier
            // before the pair, for the tiles up to s + 3 (K(s+3) is read by
            // the second step); LD - 4 newer tiles stay in flight.
            const std::integral_constant<int, LD - 4> steady_newer;
            for (; s + NBUF <= nt; s += 2) {
                if (step(RSFA_STEP(true, true, true, 1), steady_newer, buf(s), buf(s + 2), pA, sA, sB, pB, s + LD,
                         buf(s + LD)))
                    rescale_o();
                if (step(std::integral_constant<int, wide_step(true, true, true, 1, true)>(), 0, buf(s + 1),
                         buf(s + 3), pB, sB, sA, pA, s + LD + 1, buf(s + LD + 1)))
                    rescale_o();
            }
            for (; s + 3 < nt; s += 2) {
                if (step(RSFA_STEP(true, true, true, 2), newer_qk(s), buf(s), buf(s + 2), pA, sA, sB, pB, s + LD,
                         buf(s + LD)))
                    rescale_o();
                if (step(RSFA_STEP(true, true, true, 2), newer_qk(s + 1), buf(s + 1), buf(s + 3), pB, sB, sA, pA,
                         s + LD + 1, buf(s + LD + 1)))
                    rescale_o();
            }
            // the last 2 or 3 steps
            if (nt - s == 3) {
                if (step(RSFA_STEP(true, true, true, 2), newer_qk(s), buf(s), buf(s + 2), pA, sA, sB, pB, s + LD,
                         buf(s + LD)))
                    rescale_o();
                if (step(RSFA_STEP(true, false, true, 0), newer_pv(s + 1), buf(s + 1), 0, pB, sB, sA, pA, 0, 0))
                    rescale_o();
                step(RSFA_STEP(true, false, false, 0), newer_pv(s + 2), buf(s + 2), 0, pA, sA, sB, pB, 0, 0);
            } else {
                if (step(RSFA_STEP(true, false, true, 0), newer_pv(s), buf(s), 0, pA, sA, sB, pB, 0, 0))
                    rescale_o();
                step(RSFA_STEP(true, false, false, 0), newer_pv(s + 1), buf(s + 1), 0, pB, sB, sA, pA, 0, 0);
            }
        } else {
            step(RSFA_STEP(false, false, true, 0), 0, 0, 0, pB, sB, sA, pA, 0, 0);
            step(RSFA_STEP(true, false, false, 0), 0, buf(0), 0, pA, sA, sB, pB, 0, 0);
        }
#undef RSFA_STEP

        // epilogue: O / l through LDS, row-major 16-byte chunks to global
        constexpr int OROW = 2 * D + 16;  // bytes per staged row (16-byte pad)
        static_assert(NW * WR * OROW <= NBUF * BUF, "O staging must fit the K/V buffers");
        __syncthreads();  // every wave is done with the K/V tiles
        RSFA_LDS char* const ow = smem + wave * (WR * OROW);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const float lt = swap_sum(l_sum[rb]);
            const float inv = 1.0f / lt;
#pragma unroll
            for (int d = 0; d < DT; ++d)
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    const int col = 32 * d + 8 * a + 4 * hh;
                    x4 v4;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v4[e] = (elem)(o[rb][d][4 * a + e] * inv);
                    *(RSFA_LDS x4*)(ow + (rb * 32 + l32) * OROW + col * 2) = v4;
                }
            const int qrow = m0 + wave * WR + rb * 32 + l32;
            if (p.lse && hh == 0 && qrow < n)
                p.lse[(int64_t)bh * n + qrow] = (m_use[rb] + __log2f(lt)) * 0.69314718055994530942f;
        }
        {
            constexpr int CH = D / 8;     // 16-byte chunks per row
            constexpr int RPI = 64 / CH;  // rows per store instruction
            const int rr = lane / CH, cc = (lane % CH) * 8;
            const int row0 = m0 + wave * WR;
#pragma unroll
            for (int it = 0; it < WR / RPI; ++it) {
                const int r = it * RPI + rr;
                const x8 v = *(const RSFA_LDS x8*)(ow + r * OROW + cc * 2);
                if (row0 + r < n) *(x8*)(ob + (int64_t)(row0 + r) * p.o_sm + cc) = v;
            }
        }

        if (ctr) {
            __syncthreads();
            if (tid == 0) s_ticket = nxt;
            __syncthreads();
            t = s_ticket;
        } else {
            __syncthreads();
            t += qu.nwg;
        }
    }

    if (ctr && tid == 0 && t == qu.ntask + qu.nwg - 1) atomicExch(ctr, 0u);
}

}  // namespace rsfa
