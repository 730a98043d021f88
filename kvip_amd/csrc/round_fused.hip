// One decode round — LI scoring -> TopK-2048 -> Fetch gather — as a single persistent
// launch for fp8 Q/K with one query row per request.
//
// Why one launch: as two launches the round leaves HBM idle while every row selects
// (TopK is a latency chain) and at each kernel's start-up and tail. Here the selection of
// a row overlaps the scoring of later rows and the gathers of earlier ones.
//
// Requests are XCD-local. MI355X's L2 is split over its XCDs and the L2s are not coherent
// with each other: device-scope atomics and loads must go past the L2 to memory, at a
// latency that stalls every wave waiting on them. So each request is owned by one XCD and
// all the waves exchange about it stays in that XCD's L2: work counters and completion
// counts are L2 atomics (workgroup scope); keys, histograms and the TopK row are plain
// stores and atomics, read back by other CUs of the XCD with sc1 loads (an sc0 load may
// be served from the reader's stale L1 copy; an sc1 load is not). Requests are dealt to the
// XCDs in decreasing order of length, boustrophedon, so the XCDs get near-equal scoring
// work. A workgroup reads its XCD from the XCC_ID register; the dispatcher deals the
// workgroups round-robin over the XCDs (from a varying first XCD), so each XCD runs
// grid / xcds of them. Each wave takes its index within the XCD from an arrival counter;
// a wave beyond the expected count reports KVIP_STATUS_STALLED.
//
// Within an XCD:
//  * Scoring items are (request, 8-tile chunk) pairs, requests in the XCD's order. Each
//    wave takes its first two items from the XCD's counter and then one more at a time,
//    two items ahead of use. It streams the items' 32-token tiles through a wave-private
//    4-slot LDS ring exactly as the streaming decode kernel does (direct-to-LDS loads with
//    the fragment swizzle, fp8 MFMA, ReLU-weight-reduce epilogue, sortable bf16 keys) and
//    counts the keys' high bytes in an LDS histogram that is added to the request's 256-bin
//    histogram at the item's end. Every ring iteration issues the same vector memory
//    instructions (5 ring loads, one key store; the next item's 12*MT Q / weight / query
//    scale loads on the first) and every item boundary the same 6 (4 histogram adds, a
//    block-table load, a counter grab), so the waits are exact counts of the operations
//    still in flight (vmcnt completes in order).
//  * Four tiles into the next item (in-order completion has then covered the item's key
//    stores and histogram adds) the wave adds the item's tile count to the request's
//    completion count, and reads the old value at that item's end. The wave that completes
//    a request drains its ring and selects the row: the threshold bin from the histogram,
//    a low-byte histogram of that bin over the keys, then one emission pass in token order
//    (keys above the threshold, then the first keys equal to it) — the TopK contract of
//    kvip_hip_topk — and publishes the row.
//  * When no scoring item is left a wave turns to gather items: 64 selected KV rows of a
//    published row (32 items per row), copied from the paged KV cache into the contiguous
//    output. Rows shorter than 2048 need no scores: they are published at start with TopK
//    = their positions, then -1.
//  * Waits on other waves are bounded (KVIP_STATUS_STALLED on expiry); the last wave of an
//    XCD to leave restores that XCD's part of the work memory, which is zero between
//    launches.
//
// Reference: the round of kvip_lifetch_streaming_forward (op_kernel/streaming.cpp:
// 103-274, 365-500) with LI (indexer_cube.h:161-322, indexer_score.h:384-426,
// score_common.h:66-97), TopK (indexer_vector.h:799-973, topk_common.h:1000-1067) and
// Fetch (KvafBatchGetDevice, streaming.cpp:445).
#include "indexer_tile.h"
#include "lds_async.h"

namespace kvip {
namespace {

constexpr int kRfWaves = 4;
constexpr int kRfThreads = kRfWaves * 64;
constexpr int kRfSlots = 4;
constexpr int kRfTileBytes = 32 * kIndexDim;
constexpr int kRfSlotBytes = kRfTileBytes + 64 * 4;  // + key scales (both lane halves load them)
constexpr int kRfItemTiles = 8;                    // tiles per scoring item
constexpr int kRfMaxRows = KVIP_ROUND_MAX_ROWS;
constexpr int kRfMaxXcds = KVIP_ROUND_MAX_XCDS;
constexpr int kRfOps = 5;                          // ring loads per tile
constexpr int kRfBoundaryOps = 6;                  // histogram adds (4), block-table load, grab
constexpr int kRfGatherRows = 64;                  // selected rows per gather item
constexpr int kRfGatherItems = kTopK / kRfGatherRows;
constexpr int kRfPieces = KVIP_KV_ROW_BYTES / 16;  // 41
constexpr uint32_t kRfSpin = 1u << 16;             // bounded waits (polls of an L2 word)
constexpr int kVmcntZero = 0x0F70;
constexpr int kRsrcFlags = 0x00020000;             // raw buffer resource, 32-bit data format
constexpr int kSc1 = 16;                           // cache policy sc1: not served from the CU's L1
static_assert(kRfMaxRows <= kRfThreads, "one request per thread in the prologue");

// Work memory (32-bit words): per XCD a 128-byte line of counters, then per request a
// 128-byte completion record, per publication slot a 128-byte record (request + 1, 0 =
// not yet) and per request a 256-bin histogram.
constexpr int kXcdWords = KVIP_ROUND_LINE_WORDS;
constexpr int kWNext = 0, kWGather = 1, kWTail = 2, kWExited = 3, kWSpare = 4, kWArrive = 5;
static_assert(KVIP_ROUND_WORK_WORDS(1) == kRfMaxXcds * kXcdWords + 2 * kXcdWords + 256, "work memory layout");

// s_waitcnt immediate waiting for at most N vector-memory operations in flight (gfx9
// layout: vmcnt bits 3:0 and 15:14, expcnt and lgkmcnt left at their maxima). Issued
// through the builtin, so the compiler's own wait tracking knows what has completed.
template <int N>
KVIP_DEVICE void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
    __builtin_amdgcn_s_waitcnt(kVmcntZero | (N & 15) | ((N >> 4) << 14));
}

template <int V>
struct IntC {
    static constexpr int value = V;
};
template <int U, int END, typename F>
KVIP_DEVICE void static_for(F&& f) {
    if constexpr (U < END) {
        f(IntC<U>{});
        static_for<U + 1, END>(f);
    }
}

__device__ __align__(16) float kRfUnitScale[kBlockTokens] = {
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};

// Atomic add performed in the XCD's L2 (every participant runs on that XCD).
KVIP_DEVICE uint32_t add_l2(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// One L2 atomic add for the whole wave, issued by lane 0 alone. The old value is meaningful
// in lane 0 only and is read with readlane where it is used (the waits before that use are
// the caller's). The address goes through a VGPR: with a wave-uniform address and value the
// compiler would turn the add into a reduction plus an immediate broadcast of the result,
// which waits for it at once.
typedef __attribute__((address_space(1))) uint32_t global_u32;
KVIP_DEVICE uint32_t wave_add_l2(uint32_t* p, uint32_t v) {
    uint32_t old = 0;
    if (lane_id() == 0) {
        global_u32* q = (global_u32*)p;
        asm volatile("" : "+v"(q));
        old = __hip_atomic_fetch_add(q, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    return old;
}
// Buffer resource over `bytes` bytes at `base`: loads through it read 0 past the end.
KVIP_DEVICE __amdgpu_buffer_rsrc_t rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kRsrcFlags);
}

KVIP_DEVICE int rf_valid(const KvipIndexerArgs& p, int b) {
    int v = max(p.seq_lens[b], 0);
    if (p.query_ends != nullptr) v = min(v, p.query_ends[b]);
    return min(max(v, 0), p.max_blocks * kBlockTokens);
}

// Tiles scored for a request of `valid` positions: rows shorter than 2048 need no scores.
KVIP_DEVICE int rf_tiles_of(int valid) { return valid >= kTopK ? (valid + 31) / 32 : 0; }

// Inclusive prefix sum over the wave's lanes (lane order).
KVIP_DEVICE uint32_t wave_scan(uint32_t v) {
    const int lane = lane_id();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = __shfl_up(v, d);
        if (lane >= d) v += o;
    }
    return v;
}

// In a 256-bin histogram spread 4 bins per lane (bins 4l..4l+3 in h[0..3]), the highest
// bin `sel` whose count of keys at or above it reaches `target`, and the count strictly
// above it. Whole wave.
KVIP_DEVICE void wave_select_bin(const uint32_t (&h)[4], uint32_t target, int& sel, uint32_t& above) {
    const int lane = lane_id();
    const uint32_t mine = h[0] + h[1] + h[2] + h[3];
    // Suffix sums over lanes: scan the reversed lane order.
    const uint32_t rev = __shfl(mine, 63 - lane);
    const uint32_t inc = wave_scan(rev);
    const uint32_t suffix_incl = __shfl(inc, 63 - lane);      // sum over lanes >= lane
    uint32_t ge = suffix_incl - mine;                          // lanes > lane
    int best = -1;
    uint32_t best_above = 0;
#pragma unroll
    for (int i = 3; i >= 0; --i) {
        const uint32_t at_or_above = ge + h[i];
        if (best < 0 && at_or_above >= target) {
            best = lane * 4 + i;
            best_above = ge;
        }
        ge = at_or_above;
    }
    // Highest lane with a candidate.
    const unsigned long long cand = __ballot(best >= 0);
    const int top = cand ? 63 - __clzll(cand) : 0;
    sel = __shfl(best, top);
    above = __shfl(best_above, top);
}

// Requests of XCD x when `rows` requests are dealt boustrophedon over `nx` XCDs.
KVIP_DEVICE int xcd_rows(int rows, int nx, int x) {
    const int full = rows / nx, rem = rows - full * nx;
    return full + ((rem > 0 && ((full & 1) ? x >= nx - rem : x < rem)) ? 1 : 0);
}

struct RfPlan {
    int xcds;           // XCDs of the device
    int waves_per_xcd;  // waves of the grid on each XCD
};

template <int HEADS, bool W_BF16>
__global__ __launch_bounds__(kRfThreads, 2) void round_fused_kernel(const KvipIndexerArgs p, const KvipFetchArgs f,
                                                                    uint32_t* work, const RfPlan plan) {
    constexpr int MT = HEADS / 32;
    __shared__ __align__(16) uint8_t s_ring[kRfWaves][kRfSlots][kRfSlotBytes];
    __shared__ __align__(16) uint32_t s_hist[kRfWaves][2][256];
    __shared__ int s_xrow[kRfMaxRows];          // the XCD's requests in its order
    __shared__ int s_xvalid[kRfMaxRows];        // their valid positions
    __shared__ int s_iprefix[kRfMaxRows + 1];   // items before the XCD's i-th request
    __shared__ uint32_t s_scan[kRfWaves];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31;
    const int g = lane >> 5;
    const int rows = p.batch;
    const int nx = plan.xcds;
    const int nw = plan.waves_per_xcd;
    uint32_t err = 0;
    int x;
    {
        uint32_t xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        x = static_cast<int>(xcc & 15u) % nx;
    }
    uint32_t* ctr = work + x * kXcdWords;
    const uint32_t arrival = wave_add_l2(ctr + kWArrive, 1u);  // read after the prologue
    uint32_t* done_rec = work + kRfMaxXcds * kXcdWords;     // [rows][32]
    uint32_t* slot_rec = done_rec + rows * kXcdWords;        // [rows][32]
    uint32_t* hist_g = slot_rec + rows * kXcdWords;          // [rows][256]
    int32_t* topk = const_cast<int32_t*>(f.topk);

    // ---- deal the requests to the XCDs ----------------------------------------------------
    // Rank by scored tiles (descending, ties by index); rank r goes to XCD r % nx in even
    // rounds and nx - 1 - r % nx in odd ones, at position r / nx of that XCD's order.
    uint32_t* s_tiles = &s_hist[0][0][0];  // prologue scratch
    const int my_valid = tid < rows ? rf_valid(p, tid) : 0;
    if (tid < rows) s_tiles[tid] = static_cast<uint32_t>(rf_tiles_of(my_valid));
    __syncthreads();
    if (tid < rows) {
        const uint32_t tb = s_tiles[tid];
        int rank = 0;
        for (int u = 0; u < rows; ++u) {
            const uint32_t tu = s_tiles[u];
            rank += (tu > tb || (tu == tb && u < tid)) ? 1 : 0;
        }
        const int round = rank / nx, k = rank - round * nx;
        if (((round & 1) ? nx - 1 - k : k) == x) {
            s_xrow[round] = tid;
            s_xvalid[round] = my_valid;
        }
    }
    const int rows_x = xcd_rows(rows, nx, x);
    int xoff = 0;  // publication slots of the XCDs before x
    for (int y = 0; y < x; ++y) xoff += xcd_rows(rows, nx, y);
    __syncthreads();
    int n_scored;  // the XCD's requests that need scores (they come first)
    {
        const int v = tid < rows_x ? s_xvalid[tid] : 0;
        const uint32_t ti = static_cast<uint32_t>(rf_tiles_of(v));
        uint32_t tot_i, tot_s;
        const uint32_t ex_i = block_exclusive_scan((ti + kRfItemTiles - 1) / kRfItemTiles, s_scan, &tot_i);
        block_exclusive_scan(ti > 0 ? 1u : 0u, s_scan, &tot_s);
        if (tid < rows_x) s_iprefix[tid] = static_cast<int>(ex_i);
        if (tid == 0) s_iprefix[rows_x] = static_cast<int>(tot_i);
        n_scored = __builtin_amdgcn_readfirstlane(static_cast<int>(tot_s));
    }
    __syncthreads();
    const int items = s_iprefix[rows_x];
    const int lw = static_cast<int>(__builtin_amdgcn_readlane(arrival, 0));  // wave index within the XCD
    if (lw >= nw) err |= KVIP_STATUS_STALLED;
    const uint32_t hist_lds = lds_addr(&s_hist[wave][0][0]);
    lds_write_b128(hist_lds + lane * 16, v4i{0, 0, 0, 0});

    // Publishes request r's TopK row (in memory once this wave's stores are done).
    auto publish = [&](int r) {
        __builtin_amdgcn_s_waitcnt(kVmcntZero);
        const uint32_t slot = __builtin_amdgcn_readlane(wave_add_l2(ctr + kWTail, 1u), 0);
        if (slot < static_cast<uint32_t>(rows_x)) {
            if (lane == 0) slot_rec[(xoff + static_cast<int>(slot)) * kXcdWords] = static_cast<uint32_t>(r) + 1u;
        } else {
            err |= KVIP_STATUS_STALLED;
        }
    };

    // Rows shorter than 2048: TopK = positions then -1, published at once.
    for (int k = lw; k < rows_x - n_scored; k += nw) {
        const int r = s_xrow[n_scored + k];
        const int v = s_xvalid[n_scored + k];
        int32_t* out = topk + static_cast<size_t>(r) * kTopK;
        for (int e = lane; e < kTopK; e += 64) out[e] = e < v ? e : -1;
        publish(r);
    }

    uint8_t* ring = &s_ring[wave][0][0];
    const uint32_t ring_lds = lds_addr(ring);
    uint32_t ka[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) ka[u] = ring_lds + n * kIndexDim + (((g * 4 + u) ^ (n & 7)) * 16);
    const uint32_t ksa = ring_lds + kRfTileBytes + n * 4;
    const int src_lane = (lane >> 3) * kIndexDim + (((lane & 7) ^ (lane >> 3)) * 16);
    const uint8_t* kbase = static_cast<const uint8_t*>(p.keys);
    const float* kscale = p.key_scale != nullptr ? p.key_scale : kRfUnitScale;
    const int64_t kscale_stride = p.key_scale != nullptr ? p.scale_block_stride : 0;
    const bool qscale = p.query_scale != nullptr;
    const float* qsc = qscale ? p.query_scale : kRfUnitScale;

    // ---- item bookkeeping --------------------------------------------------------------
    // Wave item m occupies stream slots [8m, 8m + 8), lanes (8m) % 64 + u of the
    // descriptor registers: d_k (tile within the request, -1 for padding), d_page, d_ok.
    // d_raw holds the block-table entries of the item described last until finish() has
    // checked them (one item later, so the load is long complete by then).
    int d_k = -1, d_page = 0, d_raw = 0;
    float d_ok = 0.0f;
    auto lds_int = [&](const int* a) { return __builtin_amdgcn_readfirstlane(static_cast<int>(lds_read_b32(lds_addr(a)))); };
    auto item_row = [&](int item) {  // largest i < n_scored with s_iprefix[i] <= item
        int lo = 0, hi = n_scored - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (lds_int(&s_iprefix[mid]) <= item) lo = mid; else hi = mid - 1;
        }
        return lo;
    };
    // Describes wave item m = XCD item `item` of the XCD's i-th request (request b, valid
    // positions v): tile ids now, block-table entries loaded into d_raw (every lane loads, a
    // clamped entry outside the item, so the load instruction is unconditional); finish(m)
    // must run before the item's first ring load. Returns the item's real tiles.
    auto describe = [&](int m, int item, int i, int& b, int& v) {
        const int c = item - lds_int(&s_iprefix[i]);
        b = lds_int(&s_xrow[i]);
        v = lds_int(&s_xvalid[i]);
        const int tb = rf_tiles_of(v);
        const int l0 = (m * kRfItemTiles) & 63;
        const bool mine = lane >= l0 && lane < l0 + kRfItemTiles;
        const int k = c * kRfItemTiles + (lane - l0);
        const bool real = mine && k < tb;
        if (mine) d_k = real ? k : -1;
        d_raw = p.block_table[static_cast<size_t>(b) * p.max_blocks + (real ? (k >> 2) : 0)];
        return min(kRfItemTiles, tb - c * kRfItemTiles);
    };
    auto finish = [&](int m) {
        const int l0 = (m * kRfItemTiles) & 63;
        const bool mine = lane >= l0 && lane < l0 + kRfItemTiles;
        const bool real = mine && d_k >= 0;
        const bool ok = static_cast<unsigned>(d_raw) < static_cast<unsigned>(p.num_blocks);
        if (real && !ok) err |= KVIP_STATUS_BAD_BLOCK;
        if (mine) {
            d_page = real && ok ? d_raw : 0;
            d_ok = real && ok ? 1.0f : 0.0f;
        }
    };

    // ---- Q / weights of the current and the next item ----------------------------------
    v4i qa[MT][4], qn[MT][4];
    float wr[MT * 16], wrn[MT * 16];
    v4f wn[MT * 4], sn[MT * 4];
    // Next-item piece i (0..12*MT-1): Q fragment (4*MT), weights (4*MT), query scales (4*MT).
    auto load_next_piece = [&](int b, int i) {
        if (i < 4 * MT) {
            const int mt = i >> 2, v = i & 3;
            qn[mt][v] = reinterpret_cast<const v4i*>(static_cast<const uint8_t*>(p.query) +
                                                     (static_cast<size_t>(b) * HEADS + mt * 32 + n) * kIndexDim +
                                                     g * (kIndexDim / 2))[v];
        } else if (i < 8 * MT) {
            const int e = i - 4 * MT;  // mt * 4 + r4
            const size_t idx = static_cast<size_t>(b) * HEADS + (e >> 2) * 32 + (e & 3) * 8 + g * 4;
            if constexpr (W_BF16) {
                const v2i raw = *reinterpret_cast<const v2i*>(static_cast<const uint16_t*>(p.weights) + idx);
                wn[e] = v4f{__uint_as_float(static_cast<uint32_t>(raw[0]) << 16),
                            __uint_as_float(static_cast<uint32_t>(raw[0]) & 0xFFFF0000u),
                            __uint_as_float(static_cast<uint32_t>(raw[1]) << 16),
                            __uint_as_float(static_cast<uint32_t>(raw[1]) & 0xFFFF0000u)};
            } else {
                wn[e] = *reinterpret_cast<const v4f*>(static_cast<const float*>(p.weights) + idx);
            }
        } else {
            const int e = i - 8 * MT;
            const size_t idx = static_cast<size_t>(b) * HEADS + (e >> 2) * 32 + (e & 3) * 8 + g * 4;
            sn[e] = *reinterpret_cast<const v4f*>(qsc + (qscale ? idx : (idx & 127)));
        }
    };
    // w' = w * qscale of the next item, once its pieces have landed.
    auto fold_next = [&]() {
#pragma unroll
        for (int e = 0; e < MT * 4; ++e) {
#pragma unroll
            for (int j = 0; j < 4; ++j) wrn[e * 4 + j] = wn[e][j] * sn[e][j];
        }
    };
    auto take_next = [&]() {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int v = 0; v < 4; ++v) qa[mt][v] = qn[mt][v];
        }
#pragma unroll
        for (int e = 0; e < MT * 16; ++e) wr[e] = wrn[e];
    };

    // ---- ring ----------------------------------------------------------------------------
    auto issue = [&](int j, int jj) {  // stream slot j's ring slot, loads tile of slot jj
        const int page = __builtin_amdgcn_readlane(d_page, jj & 63);
        const int k = __builtin_amdgcn_readlane(d_k, jj & 63);
        uint8_t* dst = ring + (j & (kRfSlots - 1)) * kRfSlotBytes;
        const uint8_t* src = kbase + static_cast<size_t>(page) * p.key_block_stride + (k & 3) * kRfTileBytes + src_lane;
#pragma unroll
        for (int v = 0; v < 4; ++v) __builtin_amdgcn_global_load_lds(src + v * 1024, LDS_PTR(dst + v * 1024), 16, 0, 0);
        // Key scales: 4 bytes per lane, lanes 32-63 repeat lanes 0-31 (unconditional).
        const float* ssrc = kscale + static_cast<size_t>(page) * kscale_stride + (k & 3) * 32 + n;
        __builtin_amdgcn_global_load_lds(ssrc, LDS_PTR(dst + kRfTileBytes), 4, 0, 0);
    };
    // Scores stream slot j of request b (v valid positions), stores its keys (one store
    // instruction) and counts their high bytes in the wave's LDS histogram.
    auto score = [&](int j, int b, int v) {
        const uint32_t so = (j & (kRfSlots - 1)) * kRfSlotBytes;
        v4i kb[4];
        float ks_raw;
        lds_read_tile(ka[0] + so, ka[1] + so, ka[2] + so, ka[3] + so, ksa + so, kb, ks_raw);
        float pj[4] = {0.f, 0.f, 0.f, 0.f};
        v16f acc[2];
        acc[0] = v16f{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        Mma<1>::step(0, qa[0], kb, acc[0]);
        Mma<1>::step(1, qa[0], kb, acc[0]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            v16f& cur = acc[mt & 1];
            if (mt + 1 < MT) {
                v16f& nxt = acc[(mt + 1) & 1];
                nxt = v16f{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                Mma<1>::step(0, qa[mt + 1], kb, nxt);
                Mma<1>::step(1, qa[mt + 1], kb, nxt);
            }
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const float relu = __int_as_float(max(__float_as_int(cur[r4 * 4 + jj]), 0));
                    pj[jj] = fmaf(relu, wr[mt * 16 + r4 * 4 + jj], pj[jj]);
                }
            }
            if (mt + 1 < MT) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        float part = (pj[0] + pj[1]) + (pj[2] + pj[3]);
        const auto swapped = __builtin_amdgcn_permlane32_swap(__float_as_int(part), __float_as_int(part), false, false);
        part += __int_as_float(g == 0 ? swapped[1] : swapped[0]);
        const float ks = ks_raw * __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, d_ok), j & 63));
        const uint32_t key = sortable_key(bf16_bits_half_away(part * ks));
        const int tok = __builtin_amdgcn_readlane(d_k, j & 63) * 32 + n;
        // Both lane halves hold token n's key: one unconditional store instruction.
        p.score_keys[static_cast<size_t>(b) * p.key_stride + tok] = static_cast<uint16_t>(key);
        if (lane < 32 && tok < v) lds_add_u32(hist_lds + ((key >> 8) << 2), 1u);
    };
    // Adds the wave's LDS histogram to request b's (4 L2 atomics per lane, also for empty
    // bins) and clears it.
    auto flush = [&](int b) {
        const v4i c = lds_read_b128(hist_lds + lane * 16);
        uint32_t* hg = hist_g + static_cast<size_t>(b) * 256 + lane * 4;
#pragma unroll
        for (int k = 0; k < 4; ++k) add_l2(hg + k, static_cast<uint32_t>(c[k]));
        lds_write_b128(hist_lds + lane * 16, v4i{0, 0, 0, 0});
    };

    // ---- selection of a completed request (whole wave; no ring load in flight) ------------
    uint32_t* hl = &s_hist[wave][1][0];
    auto select_row = [&](int i) {
        const int b = lds_int(&s_xrow[i]);
        const int valid = lds_int(&s_xvalid[i]);
        // Threshold bin from the request's histogram, which is then cleared for the next launch.
        uint32_t* hg = hist_g + static_cast<size_t>(b) * 256;
        const v4i hv = __builtin_amdgcn_raw_buffer_load_b128(rsrc(hg, 1024), lane * 16, 0, kSc1);
        uint32_t h[4] = {static_cast<uint32_t>(hv[0]), static_cast<uint32_t>(hv[1]), static_cast<uint32_t>(hv[2]),
                         static_cast<uint32_t>(hv[3])};
        int hb;
        uint32_t gt_hi;
        wave_select_bin(h, kTopK, hb, gt_hi);
        const uint32_t total = __shfl(wave_scan(h[0] + h[1] + h[2] + h[3]), 63);
        if (total != static_cast<uint32_t>(valid)) err |= KVIP_STATUS_HISTOGRAM;
        *reinterpret_cast<v4i*>(hg + lane * 4) = v4i{0, 0, 0, 0};  // after the counts are in registers
        // Keys of the request: 8 per lane per 512-key chunk (lane l holds keys 8l..8l+7), two
        // chunks per load batch, the next batch in flight while one is processed (loads past
        // the row read 0 and are masked by `valid`).
        const auto rk = rsrc(p.score_keys + static_cast<size_t>(b) * p.key_stride, p.key_stride * 2);
        const int chunks = (valid + 511) / 512;
        auto load2 = [&](int c, v4i (&w)[2]) {
            w[0] = __builtin_amdgcn_raw_buffer_load_b128(rk, (c * 512 + lane * 8) * 2, 0, kSc1);
            w[1] = __builtin_amdgcn_raw_buffer_load_b128(rk, ((c + 1) * 512 + lane * 8) * 2, 0, kSc1);
        };
        auto key_of = [](const v4i& w, int e) { return (static_cast<uint32_t>(w[e >> 1]) >> (16 * (e & 1))) & 0xFFFFu; };
        // Runs f(c, w) over every chunk c of the row.
        auto each_chunk = [&](auto&& f) {
            v4i wa[2], wb[2];
            load2(0, wa);
            for (int c0 = 0; c0 < chunks; c0 += 4) {
                load2(c0 + 2, wb);
                f(c0, wa[0]);
                f(c0 + 1, wa[1]);
                load2(c0 + 4, wa);
                f(c0 + 2, wb[0]);
                f(c0 + 3, wb[1]);
            }
        };
        // Pass 1: low-byte histogram of the threshold bin.
#pragma unroll
        for (int k = 0; k < 4; ++k) hl[lane * 4 + k] = 0u;
        each_chunk([&](int c, const v4i& w) {
            const int k0 = c * 512 + lane * 8;
            uint32_t in_bin = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                in_bin |= (k0 + e < valid && static_cast<int>(key_of(w, e) >> 8) == hb) ? (1u << e) : 0u;
            }
            for (uint32_t mask = in_bin; mask != 0; mask &= mask - 1) {
                atomicAdd(&hl[key_of(w, __builtin_ctz(mask)) & 255u], 1u);
            }
        });
#pragma unroll
        for (int k = 0; k < 4; ++k) h[k] = hl[lane * 4 + k];
        int lb;
        uint32_t gt_lo;
        wave_select_bin(h, kTopK - gt_hi, lb, gt_lo);
        const uint32_t kth = (static_cast<uint32_t>(hb) << 8) | static_cast<uint32_t>(lb);
        const uint32_t n_gt = gt_hi + gt_lo;
        // Pass 2: emission in token order — keys above kth, then the first keys equal to it.
        // A lane's position among the chunk's selected keys is the count over lower lanes
        // (bitwise ballots of the per-lane counts, mbcnt) plus the count within the lane.
        int32_t* out = topk + static_cast<size_t>(b) * kTopK;
        uint32_t run_gt = 0, run_eq = 0;
        auto lower_lanes = [](uint32_t cnt, uint32_t& total) {  // cnt <= 8
            uint32_t before = 0;
            total = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const unsigned long long bal = __ballot((cnt >> k) & 1u);
                before += static_cast<uint32_t>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u))) << k;
                total += static_cast<uint32_t>(__popcll(bal)) << k;
            }
            return before;
        };
        each_chunk([&](int c, const v4i& w) {
            const int k0 = c * 512 + lane * 8;
            uint32_t gtm = 0, eqm = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t key = key_of(w, e);
                const bool live = k0 + e < valid;
                gtm |= (live && key > kth) ? (1u << e) : 0u;
                eqm |= (live && key == kth) ? (1u << e) : 0u;
            }
            if (__ballot(gtm != 0) != 0) {
                uint32_t total;
                uint32_t pos = run_gt + lower_lanes(static_cast<uint32_t>(__popc(gtm)), total);
                for (uint32_t mask = gtm; mask != 0; mask &= mask - 1, ++pos) {
                    if (pos < static_cast<uint32_t>(kTopK)) out[pos] = k0 + __builtin_ctz(mask);
                }
                run_gt += total;
            }
            if (__ballot(eqm != 0) != 0) {
                uint32_t total;
                uint32_t pos = n_gt + run_eq + lower_lanes(static_cast<uint32_t>(__popc(eqm)), total);
                for (uint32_t mask = eqm; mask != 0; mask &= mask - 1, ++pos) {
                    if (pos < static_cast<uint32_t>(kTopK)) out[pos] = k0 + __builtin_ctz(mask);
                }
                run_eq += total;
            }
        });
        if (run_gt != n_gt) err |= KVIP_STATUS_HISTOGRAM;
        if (lane == 0) done_rec[static_cast<size_t>(b) * kXcdWords] = 0u;  // ready for the next launch
        publish(b);
    };

    // ---- scoring stream ------------------------------------------------------------------
    // cur/nxt: wave items m and m+1 (XCD item, request index in the XCD order, request,
    // valid positions, real tiles); grab: the XCD counter value fetched for item m+2.
    // Pending completion: the previous item's request and tile count, and the counter's
    // old value once fetched.
    const int first = static_cast<int>(__builtin_amdgcn_readlane(wave_add_l2(ctr + kWNext, 2u), 0));
    int it_cur = first < items ? first : -1;
    int it_nxt = first + 1 < items ? first + 1 : -1;
    uint32_t grab = 0;
    int i_cur = 0, b_cur = 0, v_cur = 0, t_cur = 0;
    int i_nxt = 0, b_nxt = 0, v_nxt = 0, t_nxt = 0;
    bool desc_pending = false;  // the next item's block-table entries await finish()
    if (it_cur >= 0) {
        i_cur = item_row(it_cur);
        t_cur = describe(0, it_cur, i_cur, b_cur, v_cur);
        finish(0);
        i_nxt = item_row(it_nxt >= 0 ? it_nxt : it_cur);
        t_nxt = describe(1, it_nxt >= 0 ? it_nxt : it_cur, i_nxt, b_nxt, v_nxt);
        desc_pending = it_nxt >= 0;
        grab = wave_add_l2(ctr + kWNext, 1u);
        // Q of the first item, then the first three ring loads; the wait leaves only them in
        // flight.
#pragma unroll
        for (int q = 0; q < 12 * MT; ++q) load_next_piece(b_cur, q);
        const int lr = max(t_cur, 1) - 1;
        issue(0, 0);
        issue(1, min(1, lr));
        issue(2, min(2, lr));
        wait_vm<3 * kRfOps>();
        fold_next();
        take_next();
    }
    int pend_i = -1, pend_b = 0, pend_v = 0, pend_n = 0;
    uint32_t pend_old = 0;
    int last_real = 0;  // stream slot repeated by loads past the end
    constexpr int P = 12 * MT;
    for (int m = 0; it_cur >= 0; ++m) {
        const int s0 = m * kRfItemTiles;
        last_real = s0 + max(t_cur, 1) - 1;
        static_for<0, kRfItemTiles>([&](auto U) {
            constexpr int u = decltype(U)::value;
            const int j = s0 + u;
            // Ring load for slot j + 3 (next item, or a repeat past the stream end).
            {
                const int jn = j + 3;
                int jj;
                if (jn < s0 + kRfItemTiles) {
                    jj = jn < s0 + t_cur ? jn : last_real;
                } else if (it_nxt >= 0) {
                    const int un = jn - (s0 + kRfItemTiles);
                    jj = un < t_nxt ? jn : s0 + kRfItemTiles + max(t_nxt, 1) - 1;
                } else {
                    jj = last_real;
                }
                issue(jn, jj);
            }
            // The next item's Q / weight / scale pieces (the current request again when
            // there is no next item), landed long before the item boundary uses them.
            if constexpr (u == 0) {
                const int bq = it_nxt >= 0 ? b_nxt : b_cur;
#pragma unroll
                for (int q = 0; q < P; ++q) load_next_piece(bq, q);
            }
            // Exact wait for slot j: the operations issued after its 5 ring loads.
            if constexpr (u < 3) {
                if (m == 0) {
                    wait_vm<3 * kRfOps + P + u>();
                } else {
                    wait_vm<3 * kRfOps + 3 + kRfBoundaryOps + P>();
                }
            } else if constexpr (u == 3) {
                wait_vm<3 * kRfOps + 3 + P>();
            } else if constexpr (u < 7) {
                wait_vm<3 * kRfOps + 4>();
            } else {
                wait_vm<3 * kRfOps + 3>();
            }
            if (u < t_cur) {
                score(j, b_cur, v_cur);
            } else {
                ctr[kWSpare] = 0u;  // keeps one store per iteration
            }
            // Completion of the previous item (0 to a spare word when there is none, so the
            // atomic is unconditional); its old value is read at this item's end.
            if constexpr (u == 3) {
                pend_old = wave_add_l2(pend_i >= 0 ? done_rec + static_cast<size_t>(pend_b) * kXcdWords : ctr + kWSpare,
                                       pend_i >= 0 ? static_cast<uint32_t>(pend_n) : 0u);
            }
            // The next item's first ring load is at u == 5; its pieces have landed.
            if constexpr (u == 4) {
                fold_next();
                if (desc_pending) {
                    finish(m + 1);
                    desc_pending = false;
                }
            }
        });
        // Item boundary: the item's histogram, then the previous item's completion.
        flush(b_cur);
        if (pend_i >= 0 && static_cast<int>(__builtin_amdgcn_readlane(pend_old, 0)) + pend_n == rf_tiles_of(pend_v)) {
            __builtin_amdgcn_s_waitcnt(kVmcntZero);
            select_row(pend_i);
        }
        pend_i = i_cur;
        pend_b = b_cur;
        pend_v = v_cur;
        pend_n = t_cur;
        // Advance: the next item becomes current; describe the grabbed one (a repeat of the
        // current one when nothing is left, so the boundary's operations stay the same).
        it_cur = it_nxt;
        i_cur = i_nxt;
        b_cur = b_nxt;
        v_cur = v_nxt;
        t_cur = t_nxt;
        take_next();
        const int id = static_cast<int>(__builtin_amdgcn_readlane(grab, 0));
        it_nxt = (it_cur >= 0 && id < items) ? id : -1;
        const int dsc = it_nxt >= 0 ? it_nxt : max(it_cur, 0);
        i_nxt = item_row(dsc);
        t_nxt = describe(m + 2, dsc, i_nxt, b_nxt, v_nxt);
        desc_pending = it_nxt >= 0;
        grab = wave_add_l2(ctr + kWNext, 1u);
    }
    __builtin_amdgcn_s_waitcnt(kVmcntZero);
    if (pend_i >= 0) {
        const uint32_t old = wave_add_l2(done_rec + static_cast<size_t>(pend_b) * kXcdWords, static_cast<uint32_t>(pend_n));
        if (static_cast<int>(__builtin_amdgcn_readlane(old, 0)) + pend_n == rf_tiles_of(pend_v)) select_row(pend_i);
    }

    // ---- gathers ---------------------------------------------------------------------------
    const int total_gather = rows_x * kRfGatherItems;
    for (;;) {
        const int gi = static_cast<int>(__builtin_amdgcn_readlane(wave_add_l2(ctr + kWGather, 1u), 0));
        if (gi >= total_gather) break;
        const int slot = gi / kRfGatherItems;
        const int piece = gi % kRfGatherItems;
        const auto srs = rsrc(slot_rec + static_cast<size_t>(xoff + slot) * kXcdWords, 4);
        int r = 0;
        for (uint32_t spin = 0; spin < kRfSpin; ++spin) {
            r = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_raw_buffer_load_b32(srs, 0, 0, kSc1));
            if (r > 0) break;
            __builtin_amdgcn_s_sleep(4);
        }
        r -= 1;
        if (r < 0 || r >= rows) {
            err |= KVIP_STATUS_STALLED;
            continue;
        }
        const int e0 = piece * kRfGatherRows;
        const int token = __builtin_amdgcn_raw_buffer_load_b32(
            rsrc(topk + static_cast<size_t>(r) * kTopK + e0, kRfGatherRows * 4), lane * 4, 0, kSc1);
        int64_t src = -1;
        if (token >= 0) {
            if (token >= f.max_blocks * kBlockTokens) {
                err |= KVIP_STATUS_BAD_TOKEN;
            } else {
                const int blk = f.block_table[static_cast<size_t>(r) * f.max_blocks + (token >> 7)];
                if (static_cast<unsigned>(blk) >= static_cast<unsigned>(f.num_blocks)) {
                    err |= KVIP_STATUS_BAD_BLOCK;
                } else {
                    src = static_cast<int64_t>(blk) * f.kv_block_stride + static_cast<int64_t>(token & 127) * f.row_stride;
                }
            }
        }
        uint8_t* dst = f.output + (static_cast<size_t>(r) * kTopK + e0) * KVIP_KV_ROW_BYTES;
        // 4 passes of 16 rows: 16 x 41 pieces per pass over the 64 lanes.
#pragma unroll 1
        for (int pass = 0; pass < 4; ++pass) {
            constexpr int kIters = (16 * kRfPieces + 63) / 64;
            v4i val[kIters];
#pragma unroll
            for (int it = 0; it < kIters; ++it) {
                const int idx = it * 64 + lane;
                const int rr = idx / kRfPieces;
                const int pc = idx - rr * kRfPieces;
                const int64_t base = __shfl(src, pass * 16 + min(rr, 15));
                val[it] = v4i{0, 0, 0, 0};
                if (idx < 16 * kRfPieces && base >= 0) {
                    val[it] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(f.kv_cache + base + pc * 16));
                }
            }
#pragma unroll
            for (int it = 0; it < kIters; ++it) {
                const int idx = it * 64 + lane;
                if (idx < 16 * kRfPieces) {
                    *reinterpret_cast<v4i*>(dst + (static_cast<size_t>(pass) * 16 * kRfPieces + idx) * 16) = val[it];
                }
            }
        }
    }

    // ---- leave: the XCD's last wave restores its part of the work memory -------------------
    __builtin_amdgcn_s_waitcnt(kVmcntZero);
    const uint32_t exited = __builtin_amdgcn_readlane(wave_add_l2(ctr + kWExited, 1u), 0);
    if (exited == static_cast<uint32_t>(nw - 1)) {
        for (int i = lane; i < rows_x; i += 64) slot_rec[static_cast<size_t>(xoff + i) * kXcdWords] = 0u;
        if (lane == 0) {
            ctr[kWNext] = 0u;
            ctr[kWGather] = 0u;
            ctr[kWTail] = 0u;
            ctr[kWExited] = 0u;
            ctr[kWSpare] = 0u;
            ctr[kWArrive] = 0u;
        }
    }
    report(p.status, err);
}

struct FusedGeometry {
    int grid = 0;
    int xcds = 0;
};

// Grid (every CU at its occupancy) and XCD count of the current device, or grid 0 when the
// single-launch round cannot run there (the grid must split evenly over the XCDs).
template <typename K>
FusedGeometry fused_geometry(K kernel) {
    constexpr int kMaxDevices = 64;
    static FusedGeometry cache[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return {};
    FusedGeometry& c = cache[dev];
    if (c.grid == 0) {
        int cus = 0, per_cu = 0, xcds = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kRfThreads, 0) != hipSuccess) {
            return {};
        }
        const int grid = cus * max(per_cu, 1);
        if (xcds < 1 || xcds > kRfMaxXcds || grid % xcds != 0) return {};
        c.xcds = xcds;
        c.grid = grid;
    }
    return c;
}

template <int HEADS, bool W_BF16>
hipError_t launch_fused(const KvipIndexerArgs& a, const KvipFetchArgs& f, uint32_t* work, hipStream_t stream) {
    auto kernel = round_fused_kernel<HEADS, W_BF16>;
    const FusedGeometry geo = fused_geometry(kernel);
    if (geo.grid == 0) return hipErrorInvalidDevice;
    const RfPlan plan{geo.xcds, geo.grid / geo.xcds * kRfWaves};
    hipLaunchKernelGGL(kernel, dim3(geo.grid), dim3(kRfThreads), 0, stream, a, f, work, plan);
    return hipGetLastError();
}

}  // namespace

bool round_fused_eligible(const KvipIndexerArgs& a, const KvipTopkArgs& t, const KvipFetchArgs& f,
                          const uint32_t* work) {
    const uintptr_t wal = a.weight_dtype == KVIP_DTYPE_BF16 ? 7u : 15u;
    const bool shape =
        work != nullptr && a.qk_dtype == KVIP_DTYPE_FP8_E4M3 && a.rows_per_request == 1 && a.batch <= kRfMaxRows &&
        f.row_bytes == KVIP_KV_ROW_BYTES && f.topk == t.topk && (reinterpret_cast<uintptr_t>(a.weights) & wal) == 0 &&
        (reinterpret_cast<uintptr_t>(work) & 127u) == 0 &&
        (a.query_scale == nullptr || (reinterpret_cast<uintptr_t>(a.query_scale) & 15u) == 0) &&
        (a.key_scale == nullptr ||
         ((reinterpret_cast<uintptr_t>(a.key_scale) & 15u) == 0 && a.scale_block_stride % 4 == 0)) &&
        (reinterpret_cast<uintptr_t>(a.score_keys) & 15u) == 0 && a.key_stride % 8 == 0 &&
        (reinterpret_cast<uintptr_t>(f.topk) & 15u) == 0 && (reinterpret_cast<uintptr_t>(f.output) & 15u) == 0 &&
        f.kv_block_stride % 16 == 0 && f.row_stride % 16 == 0;
    if (!shape) return false;
    return fused_geometry(round_fused_kernel<64, false>).grid != 0;
}

hipError_t launch_round_fused(const KvipIndexerArgs& a, const KvipFetchArgs& f, uint32_t* work, hipStream_t stream) {
    if (a.heads == 64) {
        return a.weight_dtype == KVIP_DTYPE_BF16 ? launch_fused<64, true>(a, f, work, stream)
                                                 : launch_fused<64, false>(a, f, work, stream);
    }
    return a.weight_dtype == KVIP_DTYPE_BF16 ? launch_fused<32, true>(a, f, work, stream)
                                             : launch_fused<32, false>(a, f, work, stream);
}

}  // namespace kvip
