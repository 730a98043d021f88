// Decode round, launch 1 of 2, for fp8 Q/K with one query row per request: lightning-
// indexer scoring of every request and the TopK-2048 selection of each request by the
// workgroup that finishes scoring it. Launch 2 is the Fetch gather (fetch_gather.hip),
// which also checks and clears this launch's work memory.
//
// Why selection lives here: as its own launch TopK is a latency chain (key loads, two
// histograms, a scan) during which HBM idles. Here a request is selected as soon as its
// last tile is scored, while other workgroups are still streaming index-K, so only the
// selections of the last requests to finish add to the round.
//
// Requests are XCD-local. MI355X's L2 is split over its XCDs and the L2s are not coherent
// with each other inside a launch, so a request's keys, histogram and completion count are
// only ever touched by the CUs of one XCD: there plain stores and L2 atomics (workgroup
// scope: the CU sends every global atomic to the L2) are visible to the other CUs of the
// XCD, which read them with sc1 loads (not served from their own L1). The dispatcher deals
// workgroups round-robin over the XCDs, so workgroups j, j + X, j + 2X, ... (X XCDs) share
// one XCD: that group is "virtual XCD" j % X. Each workgroup ORs its physical XCD into the
// group's mask at exit; the gather launch reports KVIP_STATUS_STALLED if a group spanned
// two XCDs or a request went unselected, so a dispatcher that breaks the assumption is
// detected instead of read past.
//
// Within a virtual XCD:
//  * its requests (dealt to the XCDs by decreasing tile count, boustrophedon, so the XCDs
//    get near-equal scoring work) are flattened into one list of 32-token tiles, and each
//    of the XCD's waves streams one balanced contiguous range of it exactly as the
//    streaming decode kernel does: a wave-private 4-slot LDS ring filled by direct-to-LDS
//    loads with the fragment swizzle, fp8 MFMA, ReLU / head weights / head reduction /
//    key scale, bf16 half-away rounding, sortable keys, a per-run LDS histogram of the
//    keys' high bytes added to the request's 256-bin histogram (L2 atomics, non-zero bins
//    only);
//  * when its range is done the wave adds its tile count to each request it covered (L2
//    atomic, after all its key stores and histogram adds have completed); the wave that
//    brings a request to its tile total has completed it;
//  * after the workgroup's four waves have finished, the workgroup selects every request
//    its waves completed: the threshold bin from the histogram, a low-byte histogram of
//    that bin over the request's keys (held in registers, 128 per thread at most), one
//    workgroup scan of (keys above the threshold, keys equal to it) in token order, and
//    the GT-then-EQ emission of kvip_hip_topk into the TopK row. It then clears the
//    request's histogram for the next launch and marks the request selected.
// Rows shorter than 2048 tokens are not scored: their TopK row is their positions, then -1.
//
// Work memory (32-bit words, 128-byte lines): line v < 16 word 0 = physical-XCD mask of
// virtual XCD v; line 16 + b = request b's record (word 0 completion count, word 1
// selected flag); then one word per request: 1 if the request is scored. The gather launch
// of the same round zeroes all of it.
//
// Reference: QLIMatmul::ComputeMm1 (op_kernel/indexer/indexer_cube.h:161-322),
// MulWeightAndReduceSum (indexer_score.h:384-426, loop :60-103, finalize :105-140),
// FloatToSortableKey (score_common.h:66-97), QLIVector::ProcessTopK with LITopk's
// GT-then-EQ emission (indexer_vector.h:799-973, topk.h:155-187, topk_common.h:1000-1067).
#include "indexer_tile.h"
#include "lds_async.h"
#include "select_row.h"

namespace kvip {
namespace {

constexpr int kSsWaves = 4;
constexpr int kSsThreads = kSsWaves * 64;
constexpr int kSsSlots = 4;                          // ring slots per wave
constexpr int kSsTileBytes = 32 * kIndexDim;         // 32 fp8 rows
constexpr int kSsSlotBytes = kSsTileBytes + 32 * 4;  // + 32 key scales
constexpr int kSsPass = 64;                          // tiles described per pass (one per lane)
constexpr int kSsMaxRows = KVIP_ROUND_MAX_ROWS;
constexpr int kSsOps = 5;                            // vector memory instructions per tile load
constexpr int kLineWords = KVIP_ROUND_LINE_WORDS;
constexpr int kVmcntZero = 0x0F70;
constexpr int kVmcnt15 = 0x0F7F;
constexpr int kRsrcFlags = 0x00020000;  // raw buffer resource, 32-bit data format
constexpr int kSc1 = 16;                // cache policy sc1: not served from the CU's L1
static_assert(kSsMaxRows <= kSsThreads, "one request per thread in the prologue");
static_assert(kTopK * 4 <= kSsWaves * kSsSlots * kSsSlotBytes, "TopK row staging fits the ring");

__device__ __align__(16) float kSsUnitScale[kBlockTokens] = {
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};

struct SsPlan {
    int xcds;  // XCDs of the device (virtual XCDs of the grid)
};

// Atomic add performed in the XCD's L2 (every participant runs on that XCD).
KVIP_DEVICE uint32_t add_l2(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Buffer resource over `bytes` bytes at `base`: loads through it read 0 past the end.
KVIP_DEVICE __amdgpu_buffer_rsrc_t ss_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kRsrcFlags);
}

// Weights w'_h = w_h * qscale_h of heads [h, h + 4) of row `row` (h a multiple of 4).
template <int HEADS, bool W_BF16>
KVIP_DEVICE v4f ss_weights4(const KvipIndexerArgs& p, int row, int h, bool qscale) {
    const size_t idx = static_cast<size_t>(row) * HEADS + h;
    v4f w;
    if constexpr (W_BF16) {
        const v2i raw = *reinterpret_cast<const v2i*>(static_cast<const uint16_t*>(p.weights) + idx);
        w = v4f{__uint_as_float(static_cast<uint32_t>(raw[0]) << 16),
                __uint_as_float(static_cast<uint32_t>(raw[0]) & 0xFFFF0000u),
                __uint_as_float(static_cast<uint32_t>(raw[1]) << 16),
                __uint_as_float(static_cast<uint32_t>(raw[1]) & 0xFFFF0000u)};
    } else {
        w = *reinterpret_cast<const v4f*>(static_cast<const float*>(p.weights) + idx);
    }
    if (qscale) w *= *reinterpret_cast<const v4f*>(p.query_scale + idx);
    return w;
}

// Visible tokens of request b's single query row (clamped to the block table and the key
// row).
KVIP_DEVICE int ss_valid(const KvipIndexerArgs& p, int b) {
    int v = max(p.seq_lens[b], 0);
    if (p.query_ends != nullptr) v = min(v, p.query_ends[b]);
    return min(max(v, 0), min(p.max_blocks * kBlockTokens, p.key_stride));
}

KVIP_DEVICE int ss_tiles_of(int valid) { return valid >= kTopK ? (valid + 31) / 32 : 0; }

// Requests of virtual XCD x when `n` requests are dealt boustrophedon over `nx` XCDs.
KVIP_DEVICE int ss_xcd_rows(int n, int nx, int x) {
    const int full = n / nx, rem = n - full * nx;
    return full + ((rem > 0 && ((full & 1) ? x >= nx - rem : x < rem)) ? 1 : 0);
}

// TopK-2048 of request b (v >= 2048 valid keys, scored by waves of this XCD) by the whole
// workgroup, into t.topk row b; then clears the request's histogram and sets its selected
// flag. s_lo: 256 words, s_wave: kSsWaves words, s_out: 2048 words of LDS.
template <int KPT>
KVIP_DEVICE void ss_select(const KvipTopkArgs& t, int b, int v, uint32_t* rec, uint32_t* s_lo, uint32_t* s_wave,
                           int32_t* s_out, uint32_t& err) {
    constexpr int W = KPT / 2;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    uint32_t* hg = t.histogram + static_cast<size_t>(b) * 256;
    // Every wave reads the whole high-byte histogram (4 bins per lane).
    const v4i hv = __builtin_amdgcn_raw_buffer_load_b128(ss_rsrc(hg, 1024), lane * 16, 0, kSc1);
    // Keys [first, first + KPT) of this thread, two per register (0 past the row's stride;
    // keys at or past v are excluded by `count`).
    const int first = tid * KPT;
    const int count = max(0, min(KPT, v - first));
    const auto rk = ss_rsrc(t.score_keys + static_cast<size_t>(b) * t.key_stride, t.key_stride * 2);
    uint32_t kk[W];
#pragma unroll
    for (int q = 0; q < W / 4; ++q) {
        const v4i x = __builtin_amdgcn_raw_buffer_load_b128(rk, (first + q * 8) * 2, 0, kSc1);
#pragma unroll
        for (int w = 0; w < 4; ++w) kk[4 * q + w] = static_cast<uint32_t>(x[w]);
    }

    s_lo[tid] = 0u;  // 256 threads, 256 bins
    for (int i = tid; i < kTopK; i += kSsThreads) s_out[i] = -1;
    const uint32_t h[4] = {static_cast<uint32_t>(hv[0]), static_cast<uint32_t>(hv[1]), static_cast<uint32_t>(hv[2]),
                           static_cast<uint32_t>(hv[3])};
    int hb;
    uint32_t gt_hi;
    wave_select_bin(h, kTopK, hb, gt_hi);
    const uint32_t hist_total =
        static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(wave_inclusive_scan(h[0] + h[1] + h[2] + h[3])), 63));
    if (tid == 0 && hist_total != static_cast<uint32_t>(v)) err |= KVIP_STATUS_HISTOGRAM;
    __syncthreads();
    const RowSelection sel =
        select_row<KPT>(kk, count, first, hb, gt_hi, s_lo, s_wave, [&](int pos, int tok) { s_out[pos] = tok; });
    if (tid == 0 && !sel.ok) err |= KVIP_STATUS_HISTOGRAM;
    __syncthreads();
    // The row (8 KB) with two coalesced 16-byte stores per thread, the histogram cleared for
    // the next launch, the request marked selected.
    static_assert(kTopK == 8 * kSsThreads, "two 16-byte pieces per thread");
    int32_t* out = t.topk + static_cast<size_t>(b) * kTopK;
    reinterpret_cast<v4i*>(out)[tid] = reinterpret_cast<const v4i*>(s_out)[tid];
    reinterpret_cast<v4i*>(out)[tid + kSsThreads] = reinterpret_cast<const v4i*>(s_out)[tid + kSsThreads];
    if (tid < 64) reinterpret_cast<v4i*>(hg)[tid] = v4i{0, 0, 0, 0};
    if (tid == 0) rec[1] = 1u;
    __syncthreads();  // s_lo / s_out are reused by the next selection
}

template <int HEADS, bool W_BF16, int KPT>
__global__ __launch_bounds__(kSsThreads, 2) void score_select_kernel(const KvipIndexerArgs p, const KvipTopkArgs t,
                                                                     uint32_t* work, const SsPlan plan) {
    constexpr int MT = HEADS / 32;
    __shared__ __align__(16) uint8_t s_ring[kSsWaves][kSsSlots][kSsSlotBytes];
    __shared__ __align__(16) uint32_t s_hist[kSsWaves][256];
    __shared__ int s_xrow[kSsMaxRows];          // the XCD's requests in its order
    __shared__ int s_prefix[kSsMaxRows + 1];    // tiles before the XCD's i-th request
    __shared__ int s_tiles[kSsMaxRows];         // tiles per request; then the completed list
    __shared__ uint32_t s_scan[kSsWaves];
    __shared__ int s_ndone;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31;
    const int g = lane >> 5;
    const int nx = plan.xcds;
    const int vx = static_cast<int>(blockIdx.x) % nx;            // virtual XCD
    const int wgs = static_cast<int>(gridDim.x) / nx;           // its workgroups
    const int rows = p.batch;
    uint32_t err = 0;
    uint32_t* records = work + 16 * kLineWords;
    uint32_t* scored_flags = records + rows * kLineWords;

    // ---- deal the scored requests to the XCDs -----------------------------------------
    // Rank by tile count (descending, ties by index); rank r goes to XCD r % nx in even
    // rounds and nx - 1 - r % nx in odd ones, at position r / nx of that XCD's order.
    const int my_valid = tid < rows ? ss_valid(p, tid) : 0;
    const int my_tiles = ss_tiles_of(my_valid);
    if (tid < rows) s_tiles[tid] = my_tiles;
    if (tid == 0) s_ndone = 0;
    for (int i = tid; i < kSsWaves * 256; i += kSsThreads) (&s_hist[0][0])[i] = 0u;
    if (blockIdx.x == 0 && tid < rows) scored_flags[tid] = my_tiles > 0 ? 1u : 0u;
    __syncthreads();
    if (tid < rows && my_tiles > 0) {
        int rank = 0;
        for (int u = 0; u < rows; ++u) {
            const int tu = s_tiles[u];
            rank += (tu > my_tiles || (tu == my_tiles && u < tid)) ? 1 : 0;
        }
        const int round = rank / nx, k = rank - round * nx;
        if (((round & 1) ? nx - 1 - k : k) == vx) s_xrow[round] = tid;
    }
    uint32_t n_scored;
    block_exclusive_scan(tid < rows && my_tiles > 0 ? 1u : 0u, s_scan, &n_scored);
    const int rows_x = ss_xcd_rows(static_cast<int>(n_scored), nx, vx);
    {
        const uint32_t c = tid < rows_x ? static_cast<uint32_t>(s_tiles[s_xrow[tid]]) : 0u;
        uint32_t tot;
        const uint32_t ex = block_exclusive_scan(c, s_scan, &tot);
        if (tid < rows_x) s_prefix[tid] = static_cast<int>(ex);
        if (tid == 0) s_prefix[rows_x] = static_cast<int>(tot);
    }
    __syncthreads();

    // This wave's balanced share [t, t_end) of the XCD's tile list.
    const int total_tiles = s_prefix[rows_x];
    const int64_t nw = static_cast<int64_t>(wgs) * kSsWaves;
    const int64_t w = static_cast<int64_t>(blockIdx.x / nx) * kSsWaves + wave;
    const int t_begin = static_cast<int>(total_tiles * w / nw);
    const int t_end = static_cast<int>(total_tiles * (w + 1) / nw);
    auto row_of = [&](int tt) {  // largest i with s_prefix[i] <= tt
        int lo = 0, hi = rows_x - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_prefix[mid] <= tt) lo = mid; else hi = mid - 1;
        }
        return lo;
    };

    uint8_t* ring = &s_ring[wave][0][0];
    const uint32_t ring_lds = lds_addr(ring);
    // Fragment reads (slot 0): lane (n, g) reads pieces g*4 + u of row n.
    uint32_t ka[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) ka[u] = ring_lds + n * kIndexDim + (((g * 4 + u) ^ (n & 7)) * 16);
    const uint32_t ksa = ring_lds + kSsTileBytes + n * 4;
    const uint32_t hist_lds = lds_addr(&s_hist[wave][0]);
    // Ring loads: in the v-th 1 KiB of a slot, lane L fills LDS row 8v + L/8, slot L%8, with
    // piece (L%8) ^ (L/8) of that token's row (rows 8v + L/8 have swizzle L/8).
    const int src_lane = (lane >> 3) * kIndexDim + (((lane & 7) ^ (lane >> 3)) * 16);
    const uint8_t* kbase = static_cast<const uint8_t*>(p.keys);
    const float* kscale = p.key_scale != nullptr ? p.key_scale : kSsUnitScale;
    const int64_t kscale_stride = p.key_scale != nullptr ? p.scale_block_stride : 0;

    v4i qa[MT][4];
    float wr[MT * 16];
    int qb = -1;  // request whose Q fragments and weights are loaded
    const bool qscale = p.query_scale != nullptr;
    auto load_q = [&](int b) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const v4i* src = reinterpret_cast<const v4i*>(static_cast<const uint8_t*>(p.query) +
                                                          (static_cast<size_t>(b) * HEADS + mt * 32 + n) * kIndexDim +
                                                          g * (kIndexDim / 2));
#pragma unroll
            for (int v = 0; v < 4; ++v) qa[mt][v] = src[v];
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const v4f w4 = ss_weights4<HEADS, W_BF16>(p, b, mt * 32 + r4 * 8 + g * 4, qscale);
#pragma unroll
                for (int j = 0; j < 4; ++j) wr[mt * 16 + r4 * 4 + j] = w4[j];
            }
        }
    };
    // The run's histogram (one request) in LDS, added to the request's row in the XCD's L2
    // at the run's end (non-zero bins only).
    auto flush = [&](int req) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t a = hist_lds + (k * 64 + lane) * 4;
            const uint32_t c = lds_read_b32(a);
            if (c != 0u) {
                add_l2(&p.histogram[static_cast<size_t>(req) * 256 + k * 64 + lane], c);
                lds_write_b32(a, 0u);
            }
        }
    };

    for (int tt0 = t_begin; tt0 < t_end;) {
        const int cnt = min(t_end - tt0, kSsPass);
        // Lane i describes tile tt0 + i: request, tile within the request, page, validity.
        int d_b = 0, d_k = 0, d_page = 0, d_valid = 0;
        float d_ok = 0.0f;
        if (lane < cnt) {
            const int i = row_of(tt0 + lane);
            d_b = s_xrow[i];
            d_k = tt0 + lane - s_prefix[i];
            const int id = p.block_table[static_cast<size_t>(d_b) * p.max_blocks + (d_k >> 2)];
            const bool ok = static_cast<unsigned>(id) < static_cast<unsigned>(p.num_blocks);
            d_page = ok ? id : 0;
            d_ok = ok ? 1.0f : 0.0f;
            if (!ok) err |= KVIP_STATUS_BAD_BLOCK;
            d_valid = ss_valid(p, d_b);
        }
        // Tiles whose request differs from the next tile's end a run (lane cnt - 1 always).
        const int next_b = __shfl_down(d_b, 1);
        const uint64_t run_ends = __ballot(lane < cnt && (lane == cnt - 1 || next_b != d_b));

        auto issue = [&](int j) {
            const int jj = min(j, cnt - 1);
            const int page = __builtin_amdgcn_readlane(d_page, jj);
            const int k = __builtin_amdgcn_readlane(d_k, jj);
            uint8_t* dst = ring + (j & (kSsSlots - 1)) * kSsSlotBytes;
            const uint8_t* src = kbase + static_cast<size_t>(page) * p.key_block_stride + (k & 3) * kSsTileBytes + src_lane;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                __builtin_amdgcn_global_load_lds(src + v * 1024, LDS_PTR(dst + v * 1024), 16, 0, 0);
            }
            if (lane < 8) {
                const float* ssrc = kscale + static_cast<size_t>(page) * kscale_stride + (k & 3) * 32 + lane * 4;
                __builtin_amdgcn_global_load_lds(ssrc, LDS_PTR(dst + kSsTileBytes), 16, 0, 0);
            }
        };

        // Scores tile i with the current Q and stores its keys (one store instruction).
        auto score = [&](int i) {
            const uint32_t so = (i & (kSsSlots - 1)) * kSsSlotBytes;
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
                    for (int j = 0; j < 4; ++j) {
                        // ReLU as an integer max: negative floats (sign bit set) map to +0.
                        const float relu = __int_as_float(max(__float_as_int(cur[r4 * 4 + j]), 0));
                        pj[j] = fmaf(relu, wr[mt * 16 + r4 * 4 + j], pj[j]);
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
            // Add the other lane half's heads (v_permlane32_swap: lane l <-> lane l ^ 32).
            const auto swapped =
                __builtin_amdgcn_permlane32_swap(__float_as_int(part), __float_as_int(part), false, false);
            part += __int_as_float(g == 0 ? swapped[1] : swapped[0]);
            const float ks = ks_raw * __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, d_ok), i));
            const uint32_t key = sortable_key(bf16_bits_half_away(part * ks));
            const int b = __builtin_amdgcn_readlane(d_b, i);
            const int tok = __builtin_amdgcn_readlane(d_k, i) * 32 + n;
            if (g == 0) {  // lanes 0-31: one store instruction per tile
                p.score_keys[static_cast<size_t>(b) * p.key_stride + tok] = static_cast<uint16_t>(key);
                if (tok < __builtin_amdgcn_readlane(d_valid, i)) lds_add_u32(hist_lds + (key >> 8) * 4, 1u);
            }
        };

        // Q of the pass's first request is loaded ahead of the ring loads and waited for
        // with them in flight (loads complete in order: at most the 15 ring-load
        // instructions issued after it may remain).
        const int b_first = __builtin_amdgcn_readlane(d_b, 0);
        if (b_first != qb) {
            load_q(b_first);
            qb = b_first;
        }
        issue(0);
        issue(1);
        issue(2);
        __builtin_amdgcn_s_waitcnt(kVmcnt15);
        // Pipeline: loads of tiles i+1..i+3 stay in flight while tile i is scored. The
        // vmcnt of each wait counts the vector memory instructions issued after tile i's
        // loads (3 tile loads of kSsOps instructions plus the key stores in between);
        // a Q reload or histogram flush in between only makes a wait longer.
        int i = 0;
        while (i < cnt) {  // runs of one request
            const int b = __builtin_amdgcn_readlane(d_b, i);
            if (b != qb) {
                load_q(b);
                qb = b;
                __builtin_amdgcn_s_waitcnt(kVmcntZero);  // after the ring loads in flight
            }
            const uint64_t later = run_ends >> i;
            const int run_end = i + static_cast<int>(__builtin_ctzll(later)) + 1;
            for (; i < run_end; ++i) {
                issue(i + 3);
                if (i >= 3) {
                    wait_vmcnt<3 * kSsOps + 3>();
                } else if (i == 2) {
                    wait_vmcnt<3 * kSsOps + 2>();
                } else if (i == 1) {
                    wait_vmcnt<3 * kSsOps + 1>();
                } else {
                    wait_vmcnt<3 * kSsOps>();
                }
                score(i);
            }
            flush(b);
        }
        wait_vmcnt<0>();  // repeated tail loads land before the ring is reused
        tt0 += cnt;
    }

    // ---- completion ------------------------------------------------------------------------
    // Every key store and histogram add of this wave has completed in the L2 (waited just
    // above, or nothing was issued): add the wave's tile count to each request it covered.
    __builtin_amdgcn_s_waitcnt(kVmcntZero);
    if (t_begin < t_end) {
        const int i_first = row_of(t_begin);
        const int i_last = row_of(t_end - 1);
        for (int base = i_first; base <= i_last; base += 64) {
            const int i = base + lane;
            if (i <= i_last) {
                const int b = s_xrow[i];
                const int lo = max(t_begin, s_prefix[i]);
                const int hi = min(t_end, s_prefix[i + 1]);
                const uint32_t cnt = static_cast<uint32_t>(hi - lo);
                const uint32_t old = add_l2(records + static_cast<size_t>(b) * kLineWords, cnt);
                if (old + cnt == static_cast<uint32_t>(s_prefix[i + 1] - s_prefix[i])) {
                    s_tiles[atomicAdd(&s_ndone, 1)] = b;  // this wave completed request b
                }
            }
        }
    }
    __syncthreads();

    // ---- selection of the requests this workgroup completed --------------------------------
    const int ndone = s_ndone;
    for (int q = 0; q < ndone; ++q) {
        const int b = s_tiles[q];
        ss_select<KPT>(t, b, ss_valid(p, b), records + static_cast<size_t>(b) * kLineWords, &s_hist[0][0], s_scan,
                       reinterpret_cast<int32_t*>(&s_ring[0][0][0]), err);
    }

    // Rows shorter than 2048: every position in order, then -1 (one wave per row).
    const int gw = static_cast<int>(blockIdx.x) * kSsWaves + wave;
    for (int r = gw; r < rows; r += static_cast<int>(gridDim.x) * kSsWaves) {
        const int v = ss_valid(p, r);
        if (v < kTopK) {
            int32_t* out = t.topk + static_cast<size_t>(r) * kTopK;
            for (int e = lane; e < kTopK; e += 64) out[e] = e < v ? e : -1;
        }
    }
    // The physical XCD of this workgroup, for the gather launch's dispatch check.
    if (tid == 0) {
        uint32_t xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        __hip_atomic_fetch_or(work + vx * kLineWords, 1u << (xcc & 31u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    report(p.status, err);
}

struct SsGeometry {
    int grid = 0;
    int xcds = 0;
};

// Grid (every CU at the kernel's occupancy) and XCD count of the current device, or grid 0
// when the launch cannot run there (the grid must split evenly over the XCDs).
template <typename K>
SsGeometry ss_geometry(K kernel) {
    constexpr int kMaxDevices = 64;
    static SsGeometry cache[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return {};
    SsGeometry& c = cache[dev];
    if (c.grid == 0) {
        int cus = 0, per_cu = 0, xcds = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kSsThreads, 0) != hipSuccess) {
            return {};
        }
        const int grid = cus * max(per_cu, 1);
        if (xcds < 1 || xcds > 16 || grid % xcds != 0) return {};
        c.xcds = xcds;
        c.grid = grid;
    }
    return c;
}

template <int HEADS, bool W_BF16, int KPT>
hipError_t launch_ss(const KvipIndexerArgs& a, const KvipTopkArgs& t, uint32_t* work, hipStream_t stream) {
    auto kernel = score_select_kernel<HEADS, W_BF16, KPT>;
    const SsGeometry geo = ss_geometry(kernel);
    if (geo.grid == 0) return hipErrorInvalidDevice;
    hipLaunchKernelGGL(kernel, dim3(geo.grid), dim3(kSsThreads), 0, stream, a, t, work, SsPlan{geo.xcds});
    return hipGetLastError();
}

template <int HEADS, bool W_BF16>
hipError_t launch_ss_keys(const KvipIndexerArgs& a, const KvipTopkArgs& t, uint32_t* work, hipStream_t stream) {
    if (t.key_stride <= kSsThreads * 32) return launch_ss<HEADS, W_BF16, 32>(a, t, work, stream);
    if (t.key_stride <= kSsThreads * 64) return launch_ss<HEADS, W_BF16, 64>(a, t, work, stream);
    return launch_ss<HEADS, W_BF16, 128>(a, t, work, stream);
}

}  // namespace

// fp8, one row per request, at most KVIP_ROUND_MAX_ROWS requests, rows of at most
// 256*128 keys starting on 128-byte boundaries (key rows of two requests never share an
// L2 line), the scoring histogram, and the alignments of the streaming decode kernel.
bool score_select_eligible(const KvipIndexerArgs& a, const KvipTopkArgs& t, const uint32_t* work) {
    const uintptr_t wal = a.weight_dtype == KVIP_DTYPE_BF16 ? 7u : 15u;
    const bool shape =
        work != nullptr && (reinterpret_cast<uintptr_t>(work) & 127u) == 0 && a.qk_dtype == KVIP_DTYPE_FP8_E4M3 &&
        a.rows_per_request == 1 && a.batch <= kSsMaxRows && t.histogram != nullptr && t.histogram == a.histogram &&
        t.score_keys == a.score_keys && t.key_stride == a.key_stride && t.limit == 0 &&
        a.key_stride <= kSsThreads * 128 && a.key_stride % 64 == 0 &&
        (reinterpret_cast<uintptr_t>(a.score_keys) & 127u) == 0 &&
        (reinterpret_cast<uintptr_t>(a.histogram) & 127u) == 0 && (reinterpret_cast<uintptr_t>(t.topk) & 15u) == 0 &&
        (a.heads == 64 || a.heads == 32) && (reinterpret_cast<uintptr_t>(a.weights) & wal) == 0 &&
        (a.query_scale == nullptr || (reinterpret_cast<uintptr_t>(a.query_scale) & 15u) == 0) &&
        (a.key_scale == nullptr ||
         ((reinterpret_cast<uintptr_t>(a.key_scale) & 15u) == 0 && a.scale_block_stride % 4 == 0));
    if (!shape) return false;
    return ss_geometry(score_select_kernel<64, false, 128>).grid != 0;
}

hipError_t launch_score_select(const KvipIndexerArgs& a, const KvipTopkArgs& t, uint32_t* work, hipStream_t stream) {
    if (a.heads == 64) {
        return a.weight_dtype == KVIP_DTYPE_BF16 ? launch_ss_keys<64, true>(a, t, work, stream)
                                                 : launch_ss_keys<64, false>(a, t, work, stream);
    }
    return a.weight_dtype == KVIP_DTYPE_BF16 ? launch_ss_keys<32, true>(a, t, work, stream)
                                             : launch_ss_keys<32, false>(a, t, work, stream);
}

}  // namespace kvip
