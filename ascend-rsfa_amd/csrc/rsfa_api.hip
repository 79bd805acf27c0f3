// C ABI of the gfx950 FlashAttention-2 forward library (declared in include/rsfa.h).
//
// Replaces the host half of the reference operator
// (ascend_rsfa/flash_attention_forward.py): argument checks of
// _attention.forward (551-556), the dispatch to the small / causal-split /
// persistent kernels (564-610), _run_causal_split (493-541), get_tiling
// (624-665) and get_num_compute_cores (19-21).
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <cfloat>
#include <cmath>
#include <mutex>
#include <unordered_map>

#include "../../include/rsfa.h"
#include "fa_fwd_kernel.hpp"
#include "kernel_table.hpp"

namespace rsfa {

// The no-allocation entry point's buffer: queue counters in the first 4 KiB,
// then the workspace.  Host code never uses this name as an address (on the
// host it only stands for the symbol): rsfa_attention_fwd_noalloc looks the
// device address up once per device with hipGetSymbolAddress.
constexpr size_t kScratchCounterBytes = 4096;
static __device__ __align__(256) char scratch[kScratchCounterBytes + RSFA_NOALLOC_WORKSPACE_BYTES];

namespace {

constexpr int kMaxDevices = 64;
constexpr int kTicketSlots = 256;       // concurrent streams with a dynamic queue
constexpr int kQueues = 8;              // task queues per launch (one per XCD)
constexpr int kTicketStrideWords = 16;  // one 64-byte line per counter
constexpr int kSlotWords = kQueues * kTicketStrideWords;
static_assert(kSlotWords * sizeof(uint32_t) <= kScratchCounterBytes, "the counters fit the scratch head");
constexpr int kLdsPerCu = 160 * 1024;   // gfx950
constexpr int kMaxKernels = 512;        // instantiations in all kernel lists

KernelList all_lists[] = {kernels_d16(), kernels_d32(), kernels_d64(), kernels_d128(), kernels_d256()};

template <class F>
void for_each_kernel(F&& f) {
    for (const KernelList& l : all_lists)
        for (int i = 0; i < l.count; ++i) f(l.entries[i]);
}

const KernelEntry* find_kernel(int dtype, int d, int bn, int bm, int causal, int mode) {
    const KernelEntry* hit = nullptr;
    for_each_kernel([&](const KernelEntry& e) {
        if (e.dtype == dtype && e.d == d && e.bn == bn && e.bm == bm && e.causal == causal && e.mode == mode)
            hit = &e;
    });
    return hit;
}

bool valid_head_dim(int64_t d) { return d == 16 || d == 32 || d == 64 || d == 128 || d == 256; }
bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

struct DeviceState {
    std::mutex mu;
    int num_cus = 0;              // 0 until queried
    uint32_t* tickets = nullptr;  // kTicketSlots counters, allocated by the first dynamic launch
    std::unordered_map<void*, int> stream_slot;
    std::atomic<int> occupancy[kMaxKernels] = {};  // by kernel_index: resident workgroups per CU, 0 = not yet queried
    void* scratch = nullptr;                        // this device's address of `scratch` (no-allocation entry point)
};

DeviceState g_dev[kMaxDevices];

int current_device(int* dev) {
    if (hipGetDevice(dev) != hipSuccess) return RSFA_E_DEVICE;
    if (*dev < 0 || *dev >= kMaxDevices) return RSFA_E_DEVICE;
    return RSFA_OK;
}

// Compute units of `dev`, queried once.  A failed query is not remembered, so
// a later call retries it.
int device_cus(DeviceState& ds, int dev, int* cus) {
    std::lock_guard<std::mutex> lock(ds.mu);
    if (ds.num_cus <= 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            return RSFA_E_DEVICE;
        ds.num_cus = n;
    }
    *cus = ds.num_cus;
    return RSFA_OK;
}

// CU count the tile search plans for: the current device's, or a whole
// MI355X (256) where no device is visible, so get_tiling answers the same as
// the launcher on a GPU and still answers without one.
int planning_cus() {
    int dev = 0, cus = 0;
    if (current_device(&dev) == RSFA_OK && device_cus(g_dev[dev], dev, &cus) == RSFA_OK) return cus;
    return 256;
}

// Whether a launch on `stream` may use a dynamic ticket counter.  The counter
// is found by the stream handle and relies on the stream running its launches
// one after another, which fails for launches recorded into a graph (replays
// of graphs captured on one stream may run concurrently on other streams) and
// for hipStreamPerThread (one handle for every thread's stream): those use the
// static schedule, which gives bitwise the same results.
bool dynamic_schedule_allowed(void* stream) {
    if ((hipStream_t)stream == hipStreamPerThread) return false;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess) return false;
    return cs == hipStreamCaptureStatusNone;
}

// Counter for launches on `stream`.  Launches on one stream run in order, and
// each launch leaves its counter at 0 when it ends, so a stream can reuse its
// counter; distinct streams get distinct counters.  The counters are allocated
// (and zeroed) by the first call; returns null when that fails or all counters
// are taken (the launch then uses the static schedule; a failed allocation is
// retried by the next call).
uint32_t* stream_ticket(DeviceState& ds, void* stream) {
    std::lock_guard<std::mutex> lock(ds.mu);
    if (!ds.tickets) {
        void* buf = nullptr;
        const size_t bytes = sizeof(uint32_t) * kTicketSlots * kSlotWords;
        if (hipMalloc(&buf, bytes) != hipSuccess) return nullptr;
        if (hipMemset(buf, 0, bytes) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
            (void)hipFree(buf);
            return nullptr;
        }
        ds.tickets = (uint32_t*)buf;
    }
    auto it = ds.stream_slot.find(stream);
    int slot;
    if (it != ds.stream_slot.end()) {
        slot = it->second;
    } else {
        if ((int)ds.stream_slot.size() >= kTicketSlots) return nullptr;
        slot = (int)ds.stream_slot.size();
        ds.stream_slot.emplace(stream, slot);
    }
    return ds.tickets + (size_t)slot * kSlotWords;
}

// Task queues of a launch: one per XCD (8) when every queue gets whole heads
// in near-equal numbers, else a single queue.  The kernel's queue x holds the
// heads bh % nq == x and is served by workgroups b % nq == x.
int32_t queue_count(int64_t num_heads, int64_t grid) {
    if (grid < kQueues || num_heads < kQueues) return 1;
    if (num_heads % kQueues != 0 && num_heads < 8 * kQueues) return 1;
    return kQueues;
}

// Whether a causal fused launch hands out its query blocks in pairs (nmb-1-i,
// then i, as one ticket: every ticket the same length, nmb + 1 block-lengths
// of key tiles).  Pairs run in lockstep rounds and fetch fewer K/V bytes past
// L2, but a last round that the pairs fill only partly idles workgroups for a
// whole pair, where single blocks served longest-first end closer together.
// Makespans per queue in block-lengths, with Wq workgroups: pairs
// ceil(heads * nmb / 2 / Wq) * (nmb + 1), single blocks about their total
// work / Wq + 1/2; pairs win ties within 3 %.  Every tile takes them: at head
// dim 256, whose tasks load Q at their start, interleaved against single
// blocks: B=64 H=8 S=1024 +1.2 % (8 % fewer bytes fetched past L2), B=128
// S=2048 +2.0 %, B=16 S=2048 +4.3 %, B=8 S=4096 +5.5 %.  Only for an even
// nmb, whose pairs are all whole (B=64 H=8 S=1792 D=128: 1.5 % slower with
// the middle blocks alone).
int32_t use_pairs(int64_t num_heads, int32_t nmb, int64_t grid, int32_t nq) {
    if (nmb < 2 || (nmb & 1)) return 0;
    const int64_t wq = grid / nq;                  // workgroups per queue
    const int64_t hq = (num_heads + nq - 1) / nq;  // heads of the fullest queue
    if (wq < 1) return 0;
    const double rounds = (double)hq * nmb / 2.0 / (double)wq;
    if (rounds < 1.0) return 0;
    const double len = nmb + 1.0;
    const double paired = std::ceil(rounds - 1e-9) * len;
    const double single = rounds * len + 0.5;
    return paired <= 1.03 * single ? 1 : 0;
}

// Position of an instantiation in the kernel lists (a fixed-size cache index).
int kernel_index(const KernelEntry& e) {
    int base = 0;
    for (const KernelList& l : all_lists) {
        if (&e >= l.entries && &e < l.entries + l.count) return base + (int)(&e - l.entries);
        base += l.count;
    }
    return -1;
}

// Resident workgroups per CU of an instantiation, queried once per device
// (a fixed array, so launches allocate no host memory either).
int resident_wgs(DeviceState& ds, const KernelEntry& e) {
    const int idx = kernel_index(e);
    if (idx >= 0 && idx < kMaxKernels) {
        const int cached = ds.occupancy[idx].load(std::memory_order_relaxed);
        if (cached > 0) return cached;
    }
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, e.fn, e.nw * 64, 0) != hipSuccess || nb <= 0) nb = 1;
    if (idx >= 0 && idx < kMaxKernels) ds.occupancy[idx].store(nb, std::memory_order_relaxed);
    return nb;
}

// ---------------------------------------------------------------------------
// Tile search.  The reference's get_tiling is a table of Ascend UB tilings
// (flash_attention_forward.py:628-664) and its search tool times every
// (BM, BN) pair (tiling/search_optimal_tiling.py:47-81).  Here the candidates
// are the compiled instantiations for (dtype, head dim), each built for a
// stated number of waves per SIMD; each is checked against gfx950's per-CU LDS
// and scored with a
// cost model: the persistent grid's makespan in key-tile steps, where a step of
// a BM x BN tile costs its MFMA cycles plus a fixed per-tile synchronisation
// overhead, and workgroups sharing a CU share its four SIMDs.
// ---------------------------------------------------------------------------
struct TileCost {
    bool feasible;
    double cycles;
};

// SIMD-cycle model of one wave's key-tile step, measured on MI355X: the two
// contractions (32 x BN x D each at 1024 flop/cycle) plus the softmax VALU work
// (~9.5 cycles per score of the lane's 32 x BN tile share) plus workgroup
// synchronisation, which costs an 8-wave workgroup (one per CU, two waves of
// it per SIMD) about a third of what two 4-wave workgroups per CU pay.  The
// ping-pong schedule hides about a quarter of the softmax work behind the
// other wave's MFMAs.
double wave_tile_cycles(const KernelEntry& e) {
    const int dp = e.d < 32 ? 32 : e.d;
    const double mfma = 2.0 * 2.0 * 32.0 * e.bn * dp / 1024.0;
    const double valu = (9.5 * e.bn / 2.0 + 300.0 * e.bn / 64.0) * (e.pp ? 0.75 : 1.0);
    const double sync = e.nw >= 8 ? 100.0 : 300.0;
    return mfma + valu + sync;
}

TileCost tile_cost(const KernelEntry& e, int64_t z, int64_t h, int64_t n, int num_cus) {
    TileCost tc{false, 0.0};
    const int dp = e.d < 32 ? 32 : e.d;
    // Each instantiation was compiled for `occ` waves per SIMD (the compiler
    // fits its registers to that), so only the LDS budget is checked here.
    const int lds = (e.pp ? 3 : 2) * 2 * e.bn * dp * 2;
    if (lds > kLdsPerCu) return tc;
    const int wg_by_waves = (4 * e.occ) / e.nw;
    const int wg_by_lds = kLdsPerCu / lds;
    const int wg_per_cu = std::max(1, std::min(wg_by_waves, wg_by_lds));
    const int bm = e.bm;
    const int64_t nmb = (n + bm - 1) / bm;
    // workgroups that actually share a CU: fewer tasks than CUs leave each alone
    const int64_t ntask = z * h * nmb;
    const int64_t conc = std::min<int64_t>(wg_per_cu, (ntask + num_cus - 1) / num_cus);
    const int waves_per_simd = (int)std::max<int64_t>(1, conc * e.nw / 4);
    const int64_t tiles_full = (n + e.bn - 1) / e.bn;
    const double step = wave_tile_cycles(e);
    // Makespan of the persistent grid: total wave work over the 4 SIMDs of
    // every CU, but no shorter than the longest task, whose waves each share
    // a SIMD with waves_per_simd - 1 others.
    double work = 0.0, longest = 0.0;
    for (int64_t mb = 0; mb < nmb; ++mb) {
        const int64_t tiles = e.causal ? std::min<int64_t>(tiles_full, ((mb + 1) * bm + e.bn - 1) / e.bn) : tiles_full;
        const double c = tiles * step + 600.0;  // + task setup / epilogue
        work += c * e.nw;
        longest = std::max(longest, c * waves_per_simd);
    }
    work *= (double)(z * h);
    // SIMDs with work: each wave of a running task sits on its own SIMD
    // until all 4 * num_cus are taken
    const double busy_simds = std::min<double>(4.0 * num_cus, (double)ntask * e.nw);
    tc.feasible = true;
    tc.cycles = std::max(work / busy_simds, longest);
    return tc;
}

int choose_tiling(int64_t z, int64_t h, int64_t n, int64_t d, int causal, int dtype, int num_cus,
                  const KernelEntry** out) {
    const KernelEntry* best = nullptr;
    double best_cycles = 0.0;
    for_each_kernel([&](const KernelEntry& e) {
        if (e.dtype != dtype || e.d != d || e.causal != (causal ? 1 : 0) || e.mode != MODE_FUSED) return;
        const TileCost tc = tile_cost(e, z, h, n, num_cus);
        if (!tc.feasible) return;
        if (!best || tc.cycles < best_cycles - 1e-6 ||
            (std::fabs(tc.cycles - best_cycles) <= 1e-6 && e.bn > best->bn)) {
            best = &e;
            best_cycles = tc.cycles;
        }
    });
    if (!best) return RSFA_E_TILE;
    *out = best;
    return RSFA_OK;
}

// A requested (BLOCK_M, BLOCK_N) must follow the reference's rules (powers of
// two in [16, 512], BLOCK_M * BLOCK_N <= 65536, tiling/search_optimal_tiling.py:
// 47-81) and, when causal, BLOCK_N <= BLOCK_M, which the reference silently
// breaks on (NaN, benchmarks/run_correctness_test.py:24-25).
int validate_request(int causal, int req_bm, int req_bn) {
    if (!is_pow2(req_bm) || !is_pow2(req_bn) || req_bm < 16 || req_bn < 16 || req_bm > 512 || req_bn > 512 ||
        (int64_t)req_bm * req_bn > 65536)
        return RSFA_E_TILE;
    if (causal && req_bn > req_bm) return RSFA_E_TILE;
    return RSFA_OK;
}

// The compiled instantiation nearest to a valid request (log distance in BM
// and BN; ties go to the larger BN).  This is what a launch with a request runs.
int resolve_exact(int64_t d, int causal, int dtype, int req_bm, int req_bn, const KernelEntry** out) {
    const int st = validate_request(causal, req_bm, req_bn);
    if (st != RSFA_OK) return st;
    const KernelEntry* best = nullptr;
    double best_dist = 0.0;
    for_each_kernel([&](const KernelEntry& e) {
        if (e.dtype != dtype || e.d != d || e.causal != (causal ? 1 : 0) || e.mode != MODE_FUSED) return;
        const double dist = std::fabs(std::log2((double)e.bm / req_bm)) + std::fabs(std::log2((double)e.bn / req_bn));
        if (!best || dist < best_dist - 1e-9 || (std::fabs(dist - best_dist) <= 1e-9 && e.bn > best->bn)) {
            best = &e;
            best_dist = dist;
        }
    });
    if (!best) return RSFA_E_TILE;
    *out = best;
    return RSFA_OK;
}

bool valid_dtype(int dt) {
    return dt == RSFA_DTYPE_F16 || dt == RSFA_DTYPE_BF16 || dt == RSFA_DTYPE_F16_V8E5M2;
}

// `mult`: required multiple (elements) of the outer strides: 8 for 2-byte
// elements, 16 for a float8 V, i.e. 16-byte rows either way.
int check_tensor(const void* ptr, const int64_t st[4], int mult = 8) {
    if (((uintptr_t)ptr & 15) != 0) return RSFA_E_ALIGN;
    if (st[3] != 1) return RSFA_E_ALIGN;
    for (int i = 0; i < 3; ++i)
        if (st[i] < 0 || (st[i] % mult) != 0) return RSFA_E_ALIGN;
    return RSFA_OK;
}

// The K/V loader of a tile (and the Q loader of the ping-pong tiles that stage
// Q through LDS) keeps one uniform 64-bit base per tile and per-lane 32-bit
// byte offsets that span the tile's BN rows: ((BN - 1) * row stride +
// row width) * 2 bytes must stay below 2^32, or the offsets would wrap.
bool loader_offsets_fit(const KernelEntry& e, int64_t row_stride) {
    const int64_t dp = e.d < 32 ? 32 : e.d;
    return ((int64_t)(e.bn - 1) * row_stride + dp) * 2 < (int64_t(1) << 32);
}

// Zeroes `words` 32-bit words (the no-allocation entry point's queue
// counters) in stream order; a kernel rather than a memset so that graph
// capture records a kernel node.
__global__ void __launch_bounds__(64) clear_words(uint32_t* __restrict__ p, int words) {
    for (int i = threadIdx.x; i < words; i += blockDim.x) p[i] = 0u;
}

}  // namespace
}  // namespace rsfa

using namespace rsfa;

extern "C" {

int rsfa_abi_version(void) { return RSFA_ABI_VERSION; }

const char* rsfa_strerror(int status) {
    switch (status) {
        case RSFA_OK: return "success";
        case RSFA_E_NULL: return "a required pointer is NULL";
        case RSFA_E_SHAPE: return "invalid shape: Z, H and N_CTX must be >= 1 and fit the 32-bit task index "
                                  "(split mode: Z*H*N_CTX below 2^31 rows)";
        case RSFA_E_HEADDIM: return "head_dim must be one of 16, 32, 64, 128, 256";
        case RSFA_E_DTYPE: return "dtype must be float16 or bfloat16 (q, k, v, o), or float16 q, k, o with a float8_e5m2 v";
        case RSFA_E_TILE: return "invalid BLOCK_M/BLOCK_N: powers of two in [16, 512], BLOCK_M*BLOCK_N <= 65536, "
                                 "and BLOCK_N <= BLOCK_M when causal";
        case RSFA_E_ALIGN: return "tensors need a unit last-dim stride, other strides multiple of 8 elements, "
                                  "16-byte aligned base pointers, and K/V row strides that keep a key tile "
                                  "within 4 GiB";
        case RSFA_E_DEVICE: return "HIP runtime error while preparing the device";
        case RSFA_E_LAUNCH: return "kernel launch failed";
        case RSFA_E_ABI: return "rsfa_fwd_args.struct_size does not match this library";
        case RSFA_E_SCRATCH:
            return "the problem needs more workspace (split state) than the no-allocation "
                   "entry point's fixed buffer (RSFA_NOALLOC_WORKSPACE_BYTES)";
        case RSFA_E_WORKSPACE:
            return "workspace missing or smaller than rsfa_split_workspace_bytes() (causal split mode)";
        default: return "unknown rsfa status";
    }
}

int rsfa_get_num_compute_cores(int device) {
    int dev = device;
    if (dev < 0) {
        const int st = current_device(&dev);
        if (st != RSFA_OK) return st;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return RSFA_E_DEVICE;
    return cus;
}

int rsfa_resolve_tiling(int64_t head_dim, int32_t causal, int32_t dtype, int32_t req_block_m, int32_t req_block_n,
                        int32_t* block_m, int32_t* block_n) {
    if (!block_m || !block_n) return RSFA_E_NULL;
    if (!valid_head_dim(head_dim)) return RSFA_E_HEADDIM;
    if (!valid_dtype(dtype)) return RSFA_E_DTYPE;
    const KernelEntry* e = nullptr;
    const int st = resolve_exact(head_dim, causal, dtype, req_block_m, req_block_n, &e);
    if (st != RSFA_OK) return st;
    *block_m = e->bm;
    *block_n = e->bn;
    return RSFA_OK;
}

int rsfa_get_tiling(int64_t z, int64_t h, int64_t n_ctx, int64_t head_dim, int32_t causal, int32_t dtype,
                    int32_t* block_m, int32_t* block_n) {
    if (!block_m || !block_n) return RSFA_E_NULL;
    if (z < 1 || h < 1 || n_ctx < 1) return RSFA_E_SHAPE;
    if (!valid_head_dim(head_dim)) return RSFA_E_HEADDIM;
    if (!valid_dtype(dtype)) return RSFA_E_DTYPE;
    // the same CU count the launcher plans with (256 where no device is visible)
    const KernelEntry* e = nullptr;
    const int st = choose_tiling(z, h, n_ctx, head_dim, causal, dtype, planning_cus(), &e);
    if (st != RSFA_OK) return st;
    *block_m = e->bm;
    *block_n = e->bn;
    return RSFA_OK;
}

// The kernels read a float8 V's bytes at every head dim: no copy, no workspace.
uint64_t rsfa_v8_workspace_bytes(int64_t, int64_t, int64_t, int64_t) { return 0; }

uint64_t rsfa_split_workspace_bytes(int64_t z, int64_t h, int64_t n_ctx, int64_t head_dim, int32_t block_m) {
    if (z < 1 || h < 1 || n_ctx < 1 || block_m < 1 || !valid_head_dim(head_dim)) return 0;
    const int64_t nmb = (n_ctx + block_m - 1) / block_m;
    // per query row: m and l, then the un-normalised accumulator (head_dim floats)
    return (uint64_t)(z * h * nmb * block_m) * (uint64_t)(2 + head_dim) * sizeof(float);
}

// The tile a launch runs: for a request (block_m, block_n), the nearest
// compiled one, as the reference's BLOCK_M / BLOCK_N select its kernel's
// tile; under RSFA_FLAG_TILE_HINT (unless RSFA_FLAG_EXACT_TILE) and without a
// request, the tile search's choice for `num_cus` CUs (fwd_launch).
static int launch_tile(const rsfa_fwd_args* a, int num_cus, const KernelEntry** e) {
    const bool causal = a->causal != 0;
    const bool hint = (a->flags & RSFA_FLAG_TILE_HINT) && !(a->flags & RSFA_FLAG_EXACT_TILE);
    if ((a->block_m != 0 || a->block_n != 0) && !hint)
        return resolve_exact(a->head_dim, causal, a->dtype, a->block_m, a->block_n, e);
    return choose_tiling(a->z, a->h, a->n_ctx, a->head_dim, causal, a->dtype, num_cus, e);
}

// Shared body of the launch entry points.  `ws` / `ws_bytes` is the
// workspace the launch may use (float8 V copy, split state).  With
// `tickets_given`, `tickets` holds the dynamic queue counters (kSlotWords
// words, cleared here on `stream` before use) and the dynamic schedule is
// used even under graph capture; otherwise the launch takes this stream's
// counter from the library's allocation when the stream allows it.
static int fwd_launch(const rsfa_fwd_args* a, void* stream, void* ws, uint64_t ws_bytes, uint32_t* tickets,
                      bool tickets_given) {
    if (!a) return RSFA_E_NULL;
    if (a->struct_size != sizeof(rsfa_fwd_args)) return RSFA_E_ABI;
    if (!a->q || !a->k || !a->v || !a->o) return RSFA_E_NULL;
    if (!valid_dtype(a->dtype)) return RSFA_E_DTYPE;
    const bool v8 = a->dtype == RSFA_DTYPE_F16_V8E5M2;
    if (!valid_head_dim(a->head_dim)) return RSFA_E_HEADDIM;
    if (a->z < 1 || a->h < 1 || a->n_ctx < 1 || a->n_ctx > (1 << 30) || a->z * a->h > (1 << 30))
        return RSFA_E_SHAPE;
    int st;
    if ((st = check_tensor(a->q, a->q_stride)) != RSFA_OK) return st;
    if ((st = check_tensor(a->k, a->k_stride)) != RSFA_OK) return st;
    if ((st = check_tensor(a->v, a->v_stride, v8 ? 16 : 8)) != RSFA_OK) return st;
    if ((st = check_tensor(a->o, a->o_stride)) != RSFA_OK) return st;
    if (((uintptr_t)a->lse & 3) != 0) return RSFA_E_ALIGN;
    const bool causal = a->causal != 0;
    const bool split = causal && (a->flags & RSFA_FLAG_CAUSAL_SPLIT);
    if ((a->block_m != 0 || a->block_n != 0) &&
        (st = validate_request(causal ? 1 : 0, a->block_m, a->block_n)) != RSFA_OK)
        return st;
    // Limits of the kernels' index arithmetic, checked for every tile the
    // launch could pick (before any device work): the K/V loader's per-lane
    // 32-bit offsets, and the split state's 32-bit rows (task * BLOCK_M + row
    // <= Z*H*N_CTX rounded up to the largest BLOCK_M, 256).
    // (a float8 V's byte offsets are half those of the two-byte check)
    for_each_kernel([&](const KernelEntry& e) {
        const bool q_loader = uses_q_buffer(e.d, e.bn, e.nw, e.causal != 0, e.mode);  // Q through LDS
        if (st == RSFA_OK && e.dtype == a->dtype && e.d == a->head_dim &&
            (!loader_offsets_fit(e, a->k_stride[2]) || !loader_offsets_fit(e, a->v_stride[2]) ||
             (q_loader && !loader_offsets_fit(e, a->q_stride[2]))))
            st = RSFA_E_ALIGN;
    });
    if (st != RSFA_OK) return st;
    if (split && a->z * a->h * ((a->n_ctx + 255) / 256 * 256) >= (int64_t(1) << 31)) return RSFA_E_SHAPE;

    int dev = 0;
    if ((st = current_device(&dev)) != RSFA_OK) return st;
    DeviceState& ds = g_dev[dev];
    int num_cus = 0;
    if ((st = device_cus(ds, dev, &num_cus)) != RSFA_OK) return st;

    // A valid (BLOCK_M, BLOCK_N) request runs the nearest compiled tile, a
    // hint (RSFA_FLAG_TILE_HINT) or no request the tile the search picks.
    const KernelEntry* e = nullptr;
    if ((st = launch_tile(a, num_cus, &e)) != RSFA_OK) return st;
    const int bm = e->bm;

    FwdParams p{};
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.o = a->o;
    p.lse = a->lse;
    p.q_sz = a->q_stride[0], p.q_sh = a->q_stride[1], p.q_sm = a->q_stride[2];
    p.k_sz = a->k_stride[0], p.k_sh = a->k_stride[1], p.k_sn = a->k_stride[2];
    p.v_sz = a->v_stride[0], p.v_sh = a->v_stride[1], p.v_sn = a->v_stride[2];
    p.o_sz = a->o_stride[0], p.o_sh = a->o_stride[1], p.o_sm = a->o_stride[2];
    p.H = (int32_t)a->h;
    p.n_ctx = (int32_t)a->n_ctx;
    p.nmb = (int32_t)((a->n_ctx + bm - 1) / bm);
    p.num_heads = (int32_t)(a->z * a->h);
    if ((int64_t)p.num_heads * p.nmb > (int64_t(1) << 30)) return RSFA_E_SHAPE;
    p.num_tasks = p.num_heads * p.nmb;
    const float sc = a->sm_scale;
    p.c = std::fabs(sc) * 1.4426950408889634f;
    // Masked scores are -inf and the kernel forms exp2(s * c - m): with c == 0
    // that is -inf * 0 = NaN.  FLT_MIN scales every finite fp16/bf16 score
    // product (|s| < 2^40) below 2^-86, so exp2 of it is exactly 1.0f, the
    // value sm_scale == 0 gives, while masked keys still get exp2(-inf) = 0.
    if (p.c < FLT_MIN) p.c = FLT_MIN;
    p.neg = sc < 0.0f ? 1u : 0u;

    // workspace: the split state
    if (split) {
        const uint64_t need = rsfa_split_workspace_bytes(a->z, a->h, a->n_ctx, a->head_dim, bm);
        if (!ws || ws_bytes < need) return RSFA_E_WORKSPACE;
        if (((uintptr_t)ws & 3) != 0) return RSFA_E_ALIGN;
        // (m, l) of every row, then the rows' fp32 accumulators
        p.state = (float*)ws;
        p.acc = p.state + 2 * (int64_t)p.num_tasks * bm;
    }

    const bool dynamic = !(a->flags & RSFA_FLAG_STATIC_SCHEDULE) && (tickets_given || dynamic_schedule_allowed(stream));
    if (dynamic && tickets_given) {
        // caller-placed counters start each call at zero (a launch leaves
        // them at zero, but the caller's buffer may hold anything)
        hipLaunchKernelGGL(clear_words, dim3(1), dim3(64), 0, (hipStream_t)stream, tickets, kSlotWords);
        if (hipGetLastError() != hipSuccess) return RSFA_E_LAUNCH;
    }
    const int modes[2] = {split ? MODE_PREFIX : MODE_FUSED, MODE_DIAG};
    const int launches = split ? 2 : 1;
    for (int li = 0; li < launches; ++li) {
        const KernelEntry* k = modes[li] == MODE_FUSED ? e
                               : find_kernel(a->dtype, (int)a->head_dim, e->bn, e->bm, causal ? 1 : 0, modes[li]);
        if (!k) return RSFA_E_TILE;
        const int wgs = resident_wgs(ds, *k);
        int64_t grid = (int64_t)num_cus * wgs;
        grid = std::min<int64_t>(grid, p.num_tasks);
        grid = std::max<int64_t>(grid, 1);
        p.nq = queue_count(p.num_heads, grid);
        p.pairs = causal && modes[li] == MODE_FUSED && !(a->flags & RSFA_FLAG_SINGLE_BLOCKS)
                      ? use_pairs(p.num_heads, p.nmb, grid, p.nq)
                      : 0;
        p.ticket = !dynamic ? nullptr : tickets_given ? tickets : stream_ticket(ds, stream);
        void* args[] = {&p};
        if (hipLaunchKernel(k->fn, dim3((unsigned)grid), dim3((unsigned)(k->nw * 64)), args, 0,
                            (hipStream_t)stream) != hipSuccess)
            return RSFA_E_LAUNCH;
    }
    return RSFA_OK;
}

int rsfa_attention_fwd_noalloc(const rsfa_fwd_args* a, void* stream) {
    if (!a) return RSFA_E_NULL;
    if (a->struct_size != sizeof(rsfa_fwd_args)) return RSFA_E_ABI;
    // Workspace this call needs, checked before any device work (fwd_launch
    // repeats every other check).
    if (valid_dtype(a->dtype) && valid_head_dim(a->head_dim) && a->z >= 1 && a->h >= 1 && a->n_ctx >= 1) {
        const bool split = a->causal != 0 && (a->flags & RSFA_FLAG_CAUSAL_SPLIT);
        uint64_t need = 0;
        if (split) {
            const KernelEntry* e = nullptr;
            if (launch_tile(a, planning_cus(), &e) == RSFA_OK)
                need += rsfa_split_workspace_bytes(a->z, a->h, a->n_ctx, a->head_dim, e->bm);
        }
        if (need > RSFA_NOALLOC_WORKSPACE_BYTES) return RSFA_E_SCRATCH;
    }
    int dev = 0, st;
    if ((st = current_device(&dev)) != RSFA_OK) return st;
    DeviceState& ds = g_dev[dev];
    {
        // set-up, once per device, with that device current
        std::lock_guard<std::mutex> lock(ds.mu);
        if (!ds.scratch) {
            void* ptr = nullptr;
            if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return RSFA_E_DEVICE;
            ds.scratch = ptr;
        }
    }
    char* const base = (char*)ds.scratch;
    return fwd_launch(a, stream, base + kScratchCounterBytes, RSFA_NOALLOC_WORKSPACE_BYTES, (uint32_t*)base, true);
}

int rsfa_attention_fwd(const rsfa_fwd_args* a, void* stream) {
    if (!a) return RSFA_E_NULL;
    if (a->struct_size != sizeof(rsfa_fwd_args)) return RSFA_E_ABI;
    return fwd_launch(a, stream, a->workspace, a->workspace_bytes, nullptr, false);
}

}  // extern "C"
