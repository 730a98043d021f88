// Decode lightning-indexer scoring for fp8 Q/K with one query row per request (the plain
// decode step): a streaming kernel that feeds MFMA straight from a per-wave LDS ring.
//
// Work split: the (request, 32-token tile) pairs of the batch are flattened and every
// wave of a grid that fills the GPU once takes one contiguous range of them (weighted by
// dispatch round, see kRgLeadWeight). Each wave owns a 4-slot LDS ring (4 KiB of K rows +
// 128 bytes of key scales per slot): direct-to-LDS loads (global_load_lds_dwordx4) bring
// the next kRgDepth tiles while tile i is scored.
// The loads apply the fragment swizzle on the global side (LDS row r, 16-byte slot s
// holds piece s ^ (r & 7) of token r's row), so the MFMA B fragments are read straight
// from the ring, bank-conflict free, with no transposition and no barrier (the ring is
// private to the wave). The wave waits for its own loads with an exact vmcnt: every
// iteration issues the same vector memory instructions (tiles past the range end repeat
// its last tile into their own slot).
//
// Q fragments and per-lane head weights (w'_h = w_h * qscale_h) of the current request
// stay in registers and are reloaded when the range crosses a request boundary. Scoring
// is the decode formula: fp8 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4), ReLU, head
// weights, head reduction, key scale, bf16 half-away rounding, sortable key. Each lane
// half holds half of the heads of the tile's 32 tokens; after the per-lane-half head
// reduction a v_permlane32_swap adds the other half's heads, and lanes 0-31 scale, round,
// store the tile's keys and count them. The 256-bin high-byte histogram of the current
// request is kept per wave in LDS (one buffer: a run covers one request) and added to the
// global row at the run's end. LDS per workgroup stays under 80 KB so that two scoring
// workgroups leave room on a CU for a 1024-thread TopK workgroup of another row group.
//
// Reference: QLIMatmul::ComputeMm1 (op_kernel/indexer/indexer_cube.h:161-322),
// MulWeightAndReduceSum (indexer_score.h:384-426, loop :60-103, finalize :105-140),
// FloatToSortableKey (score_common.h:66-97).
#include "indexer_tile.h"
#include "lds_async.h"

namespace kvip {
namespace {

constexpr int kRgWaves = 4;
constexpr int kRgThreads = kRgWaves * 64;
constexpr int kRgSlots = 4;                          // ring slots per wave
constexpr int kRgTileBytes = 32 * kIndexDim;         // 32 fp8 rows
constexpr int kRgSlotBytes = kRgTileBytes + 32 * 4;  // + 32 key scales
constexpr int kRgPass = 64;                          // tiles described per pass (one per lane)
constexpr int kRgMaxBatch = 512;
// Vector memory instructions per tile load: 4 K pieces + 1 key-scale piece.
constexpr int kRgOps = 5;
// s_waitcnt immediate (gfx9 encoding) for vmcnt(0), expcnt and lgkmcnt unconstrained.
constexpr int kVmcntZero = 0x0F70;
// Cache policy of the K-tile loads: nt (each index-K byte is read once per step; streamed
// past the caches, reads run at ~7.0 TB/s on MI355X against ~6.3 TB/s with the default policy).
constexpr int kNonTemporal = 2;
// Tiles in flight per wave while one is scored (at most kRgSlots - 1). One: with ~2000
// waves the HBM queues stay full, and deeper rings only delay the first tiles of the
// workgroups dispatched last (their waves then finish last).
constexpr int kRgDepth = 1;
// Relative tile shares of the waves of the first dispatch round (the first workgroup on
// each CU) and of the later rounds: the later workgroups' first tiles queue behind the
// first round's and land ~2 us later at config-2 sizes, so they get ~18 % fewer tiles.
constexpr int kRgLeadWeight = 22;
constexpr int kRgLagWeight = 18;

// Stands in for a missing key-scale array (stride 0): 128 unit scales.
__device__ __align__(16) float kRingUnitScale[kBlockTokens] = {
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};

// Weights w'_h = w_h * qscale_h of heads [h, h + 4) of row `row` (h a multiple of 4).
template <int HEADS, bool W_BF16>
KVIP_DEVICE v4f rg_weights4(const KvipIndexerArgs& p, int row, int h, bool qscale) {
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

// Visible tokens of query row `row` of request b.
KVIP_DEVICE int rg_valid(const KvipIndexerArgs& p, int b, int row) {
    int v = max(p.seq_lens[b], 0);
    if (p.query_ends != nullptr) v = min(v, p.query_ends[row]);
    return min(max(v, 0), p.max_blocks * kBlockTokens);
}

// Q fragments (A operand: head mt*32 + n, bytes [64*g, +64)) and per-lane weights of
// query row `row`, in the MFMA output layout (wr[mt*16 + r] weighs head
// mt*32 + 8*(r/4) + 4*g + r%4).
template <int HEADS, bool W_BF16>
KVIP_DEVICE void rg_load_q(const KvipIndexerArgs& p, int row, int n, int g, bool qscale,
                           v4i (&qa)[HEADS / 32][4], float (&wr)[HEADS / 2]) {
#pragma unroll
    for (int mt = 0; mt < HEADS / 32; ++mt) {
        const v4i* src = reinterpret_cast<const v4i*>(static_cast<const uint8_t*>(p.query) +
                                                      (static_cast<size_t>(row) * HEADS + mt * 32 + n) * kIndexDim +
                                                      g * (kIndexDim / 2));
#pragma unroll
        for (int v = 0; v < 4; ++v) qa[mt][v] = src[v];
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const v4f w4 = rg_weights4<HEADS, W_BF16>(p, row, mt * 32 + r4 * 8 + g * 4, qscale);
#pragma unroll
            for (int j = 0; j < 4; ++j) wr[mt * 16 + r4 * 4 + j] = w4[j];
        }
    }
}

// Sortable key of token n for one query row from the tile's B fragments kb and the
// token's key scale ks (same value in both lane halves): fp8 MFMA over the heads, ReLU
// (integer max: negative floats map to +0), head weights, head reduction (4 FMA chains,
// then v_permlane32_swap adds the other lane half's heads), key scale, bf16 half-away
// rounding, sortable transform. The next head tile's MFMAs are interleaved with the
// current tile's epilogue.
template <int MT>
KVIP_DEVICE uint32_t rg_key(const v4i (&qa)[MT][4], const float (&wr)[MT * 16], const v4i (&kb)[4], float ks,
                            int g) {
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
    const auto swapped = __builtin_amdgcn_permlane32_swap(__float_as_int(part), __float_as_int(part), false, false);
    part += __int_as_float(g == 0 ? swapped[1] : swapped[0]);
    return sortable_key(bf16_bits_half_away(part * ks));
}

template <int HEADS, bool W_BF16>
__global__ __launch_bounds__(kRgThreads, 2) void indexer_ring_kernel(const KvipIndexerArgs p, int lead_blocks,
                                                                     int tile_lo, int tile_hi) {
    constexpr int MT = HEADS / 32;
    __shared__ __align__(16) uint8_t s_ring[kRgWaves][kRgSlots][kRgSlotBytes];
    __shared__ __align__(16) uint32_t s_hist[kRgWaves][256];
    __shared__ int s_prefix[kRgMaxBatch + 1];
    __shared__ uint32_t s_scan[kRgWaves];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31;
    const int g = lane >> 5;

    // Tile counts per request inside the window [tile_lo, tile_hi) of 32-token tiles ->
    // prefix sums (whole workgroup, before any ring load).
    int running = 0;
    for (int base = 0; base < p.batch; base += kRgThreads) {
        const int b = base + tid;
        const int c = b < p.batch ? max(0, min((rg_valid(p, b, b) + 31) / 32, tile_hi) - tile_lo) : 0;
        uint32_t total;
        const uint32_t excl = block_exclusive_scan(static_cast<uint32_t>(c), s_scan, &total);
        if (b < p.batch) s_prefix[b] = running + static_cast<int>(excl);
        running += static_cast<int>(total);
    }
    if (tid == 0) s_prefix[p.batch] = running;
    for (int i = tid; i < kRgWaves * 256; i += kRgThreads) (&s_hist[0][0])[i] = 0u;
    __syncthreads();

    // This wave's share [t, t_end) of the flattened tile list: the waves of the first
    // lead_blocks workgroups weigh kRgLeadWeight, the others kRgLagWeight.
    const int total_tiles = s_prefix[p.batch];
    const int64_t lead = static_cast<int64_t>(min(lead_blocks, static_cast<int>(gridDim.x))) * kRgWaves;
    auto weight_before = [&](int64_t v) {
        return kRgLeadWeight * min(v, lead) + kRgLagWeight * max(v - lead, static_cast<int64_t>(0));
    };
    const int64_t nw = static_cast<int64_t>(gridDim.x) * kRgWaves;
    const int64_t w = static_cast<int64_t>(blockIdx.x) * kRgWaves + wave;
    const int64_t weight_total = weight_before(nw);
    int t = static_cast<int>(total_tiles * weight_before(w) / weight_total);
    const int t_end = static_cast<int>(total_tiles * weight_before(w + 1) / weight_total);
    if (t >= t_end) return;  // no barrier follows: waves run independently from here

    uint8_t* ring = &s_ring[wave][0][0];
    const uint32_t ring_lds = lds_addr(ring);
    // Fragment reads (slot 0): lane (n, g) reads pieces g*4 + u of row n.
    uint32_t ka[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) ka[u] = ring_lds + n * kIndexDim + (((g * 4 + u) ^ (n & 7)) * 16);
    const uint32_t ksa = ring_lds + kRgTileBytes + n * 4;
    const uint32_t hist_lds = lds_addr(&s_hist[wave][0]);
    // Ring loads: in the v-th 1 KiB of a slot, lane L fills LDS row 8v + L/8, slot L%8, with
    // piece (L%8) ^ (L/8) of that token's row (rows 8v + L/8 have swizzle L/8).
    const int src_lane = (lane >> 3) * kIndexDim + (((lane & 7) ^ (lane >> 3)) * 16);
    const uint8_t* kbase = static_cast<const uint8_t*>(p.keys);
    const float* kscale = p.key_scale != nullptr ? p.key_scale : kRingUnitScale;
    const int64_t kscale_stride = p.key_scale != nullptr ? p.scale_block_stride : 0;
    uint32_t err = 0;

    v4i qa[MT][4];
    float wr[MT * 16];
    int qb = -1;  // request whose Q fragments and weights are loaded
    const bool qscale = p.query_scale != nullptr;
    auto load_q = [&](int b) { rg_load_q<HEADS, W_BF16>(p, b, n, g, qscale, qa, wr); };

    // The run's histogram (one request) in LDS, added to the global row at the run's end.
    auto flush = [&](int req) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t a = hist_lds + (k * 64 + lane) * 4;
            const uint32_t c = lds_read_b32(a);
            if (c != 0u) {
                atomicAdd(&p.histogram[static_cast<size_t>(req) * 256 + k * 64 + lane], c);
                lds_write_b32(a, 0u);
            }
        }
    };

    while (t < t_end) {
        const int cnt = min(t_end - t, kRgPass);
        // Lane i describes tile t + i: request, tile within the request, page, validity.
        int d_b = 0, d_k = 0, d_page = 0, d_valid = 0;
        float d_ok = 0.0f;
        if (lane < cnt) {
            const int tt = t + lane;
            int lo = 0, hi = p.batch - 1;  // largest b with s_prefix[b] <= tt
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (s_prefix[mid] <= tt) lo = mid; else hi = mid - 1;
            }
            d_b = lo;
            d_k = tt - s_prefix[lo] + tile_lo;
            const int id = p.block_table[static_cast<size_t>(d_b) * p.max_blocks + (d_k >> 2)];
            const bool ok = static_cast<unsigned>(id) < static_cast<unsigned>(p.num_blocks);
            d_page = ok ? id : 0;
            d_ok = ok ? 1.0f : 0.0f;
            if (!ok) err |= KVIP_STATUS_BAD_BLOCK;
            d_valid = rg_valid(p, d_b, d_b);
        }
        // Tiles whose request differs from the next tile's end a run (lane cnt - 1 always).
        const int next_b = __shfl_down(d_b, 1);
        const uint64_t run_ends = __ballot(lane < cnt && (lane == cnt - 1 || next_b != d_b));

        auto issue = [&](int j) {
            const int jj = min(j, cnt - 1);
            const int page = __builtin_amdgcn_readlane(d_page, jj);
            const int k = __builtin_amdgcn_readlane(d_k, jj);
            uint8_t* dst = ring + (j & (kRgSlots - 1)) * kRgSlotBytes;
            const uint8_t* src = kbase + static_cast<size_t>(page) * p.key_block_stride + (k & 3) * kRgTileBytes + src_lane;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                __builtin_amdgcn_global_load_lds(src + v * 1024, LDS_PTR(dst + v * 1024), 16, 0, kNonTemporal);
            }
            if (lane < 8) {
                const float* ssrc = kscale + static_cast<size_t>(page) * kscale_stride + (k & 3) * 32 + lane * 4;
                __builtin_amdgcn_global_load_lds(ssrc, LDS_PTR(dst + kRgTileBytes), 16, 0, kNonTemporal);
            }
        };

        // Scores tile i with the current Q and stores its keys (one store instruction).
        auto score = [&](int i) {
            const uint32_t so = (i & (kRgSlots - 1)) * kRgSlotBytes;
            v4i kb[4];
            float ks_raw;
            lds_read_tile(ka[0] + so, ka[1] + so, ka[2] + so, ka[3] + so, ksa + so, kb, ks_raw);
            const float ks = ks_raw * __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, d_ok), i));
            const uint32_t key = rg_key<MT>(qa, wr, kb, ks, g);
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
#pragma unroll
        for (int j = 0; j < kRgDepth; ++j) issue(j);
        wait_vmcnt<kRgDepth * kRgOps>();
        // Pipeline: loads of tiles i+1..i+kRgDepth stay in flight while tile i is scored.
        // The vmcnt of each wait counts the vector memory instructions issued after tile
        // i's loads (kRgDepth tile loads of kRgOps instructions plus the key stores in
        // between); a Q reload or histogram flush in between only makes a wait longer.
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
                issue(i + kRgDepth);
                if (i >= kRgDepth) {
                    wait_vmcnt<kRgDepth * kRgOps + kRgDepth>();
                } else if (i == 2) {
                    wait_vmcnt<kRgDepth * kRgOps + 2>();
                } else if (i == 1) {
                    wait_vmcnt<kRgDepth * kRgOps + 1>();
                } else {
                    wait_vmcnt<kRgDepth * kRgOps>();
                }
                score(i);
            }
            flush(b);
        }
        wait_vmcnt<0>();  // repeated tail loads land before the ring is reused
        t += cnt;
    }
    report(p.status, err);
}

// Keys of two 32-token tiles A and B for one query row: the same arithmetic as rg_key per
// tile (MFMA over the heads, ReLU, head weights, four FMA chains per lane half in head
// order), with one v_permlane32_swap joining the lane halves of both tiles, so that lanes
// 0-31 finish token n of A and lanes 32-63 token n of B (ks: that token's key scale).
template <int MT>
KVIP_DEVICE uint32_t rg_key2(const v4i (&qa)[MT][4], const float (&wr)[MT * 16], const v4i (&ka)[4],
                             const v4i (&kbb)[4], float ks) {
    float pa[4] = {0.f, 0.f, 0.f, 0.f};
    float pb[4] = {0.f, 0.f, 0.f, 0.f};
    v16f acc[2];
    acc[0] = v16f{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    Mma<1>::step(0, qa[0], ka, acc[0]);
    Mma<1>::step(1, qa[0], ka, acc[0]);
    __builtin_amdgcn_sched_barrier(0);
    // Groups j = 2 mt + t: head tile mt of tile t (t = 0: A, 1: B).
#pragma unroll
    for (int j = 0; j < 2 * MT; ++j) {
        v16f& cur = acc[j & 1];
        if (j + 1 < 2 * MT) {
            const int mn = (j + 1) >> 1;
            v16f& nxt = acc[(j + 1) & 1];
            nxt = v16f{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if ((j + 1) & 1) {
                Mma<1>::step(0, qa[mn], kbb, nxt);
                Mma<1>::step(1, qa[mn], kbb, nxt);
            } else {
                Mma<1>::step(0, qa[mn], ka, nxt);
                Mma<1>::step(1, qa[mn], ka, nxt);
            }
        }
        const int mt = j >> 1;
        float (&pj)[4] = (j & 1) ? pb : pa;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float relu = __int_as_float(max(__float_as_int(cur[r4 * 4 + q]), 0));
                pj[q] = fmaf(relu, wr[mt * 16 + r4 * 4 + q], pj[q]);
            }
        }
        if (j + 1 < 2 * MT) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const float part_a = (pa[0] + pa[1]) + (pa[2] + pa[3]);
    const float part_b = (pb[0] + pb[1]) + (pb[2] + pb[3]);
    // [A lanes 0-31, B lanes 0-31] and [A lanes 32-63, B lanes 32-63].
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(part_a), __float_as_int(part_b), false, false);
    const float part = __int_as_float(sw[0]) + __int_as_float(sw[1]);
    return sortable_key(bf16_bits_half_away(part * ks));
}

// The eight 16-byte K fragment pieces of token rows n (A) and 32 + n (B, 4 KiB further) and
// one 4-byte value (the lane's key scale), then wait for them.
KVIP_DEVICE void lds_read_tile2(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, uint32_t as, v4i (&ka)[4],
                                v4i (&kbb)[4], float& ks) {
    asm volatile(
        "ds_read_b128 %0, %9\n"
        "ds_read_b128 %1, %10\n"
        "ds_read_b128 %2, %11\n"
        "ds_read_b128 %3, %12\n"
        "ds_read_b128 %4, %9 offset:4096\n"
        "ds_read_b128 %5, %10 offset:4096\n"
        "ds_read_b128 %6, %11 offset:4096\n"
        "ds_read_b128 %7, %12 offset:4096\n"
        "ds_read_b32 %8, %13\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(ka[0]), "=&v"(ka[1]), "=&v"(ka[2]), "=&v"(ka[3]), "=&v"(kbb[0]), "=&v"(kbb[1]), "=&v"(kbb[2]),
          "=&v"(kbb[3]), "=&v"(ks)
        : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "v"(as));
}

// Decode with ROWS = 2 or 4 query rows per request (the MTP rows): one workgroup of ROWS
// waves per tile stream, wave w scoring row w of each tile's request, over 64-token tiles
// (half an index-K block). The workgroup shares one LDS ring: every wave loads its share of
// each tile (8 / ROWS KiB of K rows and 256 / ROWS bytes of key scales, same fragment
// swizzle as the one-row kernel), waits for its own loads with an exact vmcnt and meets the
// others at a barrier, after which every wave reads the whole tile. A tile is thus read from
// HBM once for all rows of its request; each wave keeps the Q fragments and weights of one
// row in registers and finishes the keys of 64 tokens at once (lanes 0-31 the first 32,
// lanes 32-63 the next 32: one key store and one histogram add per lane and tile).
// Slots: kRrDepth tiles are in flight while tile i is scored, and the loads of tile
// i + kRrDepth are issued while slow waves may still read tile i - 1, so the ring needs
// kRrDepth + 2 slots (rounded up to a power of two; a full pass of kRgPass tiles then ends
// on the last slot and the next pass starts on slot 0, away from the one still read).
// Every wave of a workgroup walks the same tiles, runs and passes, so all of them reach
// the same barriers.
constexpr int kRrDepth = 1;
constexpr int kRrSlots = kRrDepth + 2 <= 4 ? 4 : 8;
constexpr int kRrTile = 64;                                // tokens per tile
constexpr int kRrTileBytes = kRrTile * kIndexDim;          // 8 KiB of fp8 K rows
constexpr int kRrSlotBytes = kRrTileBytes + kRrTile * 4;   // + 64 key scales
static_assert(kRgPass % kRrSlots == 0, "a full pass ends on the last slot");
static_assert(kRrDepth >= 1 && kRrDepth <= 4, "the waits below cover up to 4 tiles in flight");

template <int ROWS, int HEADS, bool W_BF16>
__global__ __launch_bounds__(ROWS * 64, 3) void indexer_rows_kernel(const KvipIndexerArgs p, int lead_blocks) {
    constexpr int MT = HEADS / 32;
    constexpr int kThreads = ROWS * 64;
    constexpr int kChunks = 8 / ROWS;  // KiB of K rows each wave loads per tile
    constexpr int kScaleLanes = 16 / ROWS;
    constexpr int kOps = kChunks + 1;  // vector memory instructions per tile and wave
    __shared__ __align__(16) uint8_t s_ring[kRrSlots][kRrSlotBytes];
    __shared__ __align__(16) uint32_t s_hist[ROWS][256];
    __shared__ int s_prefix[kRgMaxBatch + 1];
    __shared__ uint32_t s_scan[ROWS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31;
    const int g = lane >> 5;

    // 64-token tiles per request (the longest of its rows) -> prefix sums.
    int running = 0;
    for (int base = 0; base < p.batch; base += kThreads) {
        const int b = base + tid;
        int c = 0;
        if (b < p.batch) {
            int vmax = 0;
#pragma unroll
            for (int q = 0; q < ROWS; ++q) vmax = max(vmax, rg_valid(p, b, b * ROWS + q));
            c = (vmax + kRrTile - 1) / kRrTile;
        }
        uint32_t total;
        const uint32_t excl = block_exclusive_scan(static_cast<uint32_t>(c), s_scan, &total);
        if (b < p.batch) s_prefix[b] = running + static_cast<int>(excl);
        running += static_cast<int>(total);
    }
    if (tid == 0) s_prefix[p.batch] = running;
    for (int i = tid; i < ROWS * 256; i += kThreads) (&s_hist[0][0])[i] = 0u;
    __syncthreads();

    // The workgroup's share [t, t_end) of the flattened tile list (first dispatch round
    // weighted kRgLeadWeight, later ones kRgLagWeight).
    const int total_tiles = s_prefix[p.batch];
    const int64_t lead = min(lead_blocks, static_cast<int>(gridDim.x));
    auto weight_before = [&](int64_t v) {
        return kRgLeadWeight * min(v, lead) + kRgLagWeight * max(v - lead, static_cast<int64_t>(0));
    };
    const int64_t weight_total = weight_before(gridDim.x);
    int t = static_cast<int>(total_tiles * weight_before(blockIdx.x) / weight_total);
    const int t_end = static_cast<int>(total_tiles * weight_before(blockIdx.x + 1) / weight_total);
    if (t >= t_end) return;  // uniform for the workgroup

    uint8_t* ring = &s_ring[0][0];
    const uint32_t ring_lds = lds_addr(ring);
    // Fragment reads of token row n (the B rows 32 + n sit 4 KiB further, same swizzle).
    uint32_t ka[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) ka[u] = ring_lds + n * kIndexDim + (((g * 4 + u) ^ (n & 7)) * 16);
    const uint32_t ksa = ring_lds + kRrTileBytes + lane * 4;  // key scale of token `lane`
    const uint32_t hist_lds = lds_addr(&s_hist[wave][0]);
    const int src_lane = (lane >> 3) * kIndexDim + (((lane & 7) ^ (lane >> 3)) * 16);
    const uint8_t* kbase = static_cast<const uint8_t*>(p.keys);
    const float* kscale = p.key_scale != nullptr ? p.key_scale : kRingUnitScale;
    const int64_t kscale_stride = p.key_scale != nullptr ? p.scale_block_stride : 0;
    uint32_t err = 0;

    v4i qa[MT][4];
    float wr[MT * 16];
    int qb = -1;
    const bool qscale = p.query_scale != nullptr;

    auto flush = [&](int row) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t a = hist_lds + (k * 64 + lane) * 4;
            const uint32_t c = lds_read_b32(a);
            if (c != 0u) {
                atomicAdd(&p.histogram[static_cast<size_t>(row) * 256 + k * 64 + lane], c);
                lds_write_b32(a, 0u);
            }
        }
    };

    while (t < t_end) {
        const int cnt = min(t_end - t, kRgPass);
        // Lane i describes tile t + i (every wave computes the same descriptors).
        int d_b = 0, d_k = 0, d_page = 0, d_valid = 0;
        float d_ok = 0.0f;
        if (lane < cnt) {
            const int tt = t + lane;
            int lo = 0, hi = p.batch - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (s_prefix[mid] <= tt) lo = mid; else hi = mid - 1;
            }
            d_b = lo;
            d_k = tt - s_prefix[lo];
            const int id = p.block_table[static_cast<size_t>(d_b) * p.max_blocks + (d_k >> 1)];
            const bool ok = static_cast<unsigned>(id) < static_cast<unsigned>(p.num_blocks);
            d_page = ok ? id : 0;
            d_ok = ok ? 1.0f : 0.0f;
            if (!ok && wave == 0) err |= KVIP_STATUS_BAD_BLOCK;
            d_valid = rg_valid(p, d_b, d_b * ROWS + wave);
        }
        const int next_b = __shfl_down(d_b, 1);
        const uint64_t run_ends = __ballot(lane < cnt && (lane == cnt - 1 || next_b != d_b));

        // This wave's share of tile j's loads (tiles past the pass end repeat its last tile).
        auto issue = [&](int j) {
            const int jj = min(j, cnt - 1);
            const int page = __builtin_amdgcn_readlane(d_page, jj);
            const int k = __builtin_amdgcn_readlane(d_k, jj);
            uint8_t* dst = ring + (j & (kRrSlots - 1)) * kRrSlotBytes;
            const uint8_t* src = kbase + static_cast<size_t>(page) * p.key_block_stride + (k & 1) * kRrTileBytes + src_lane;
#pragma unroll
            for (int c = 0; c < kChunks; ++c) {
                const int v = wave * kChunks + c;
                __builtin_amdgcn_global_load_lds(src + v * 1024, LDS_PTR(dst + v * 1024), 16, 0, kNonTemporal);
            }
            if (lane < kScaleLanes) {
                const float* ssrc = kscale + static_cast<size_t>(page) * kscale_stride + (k & 1) * kRrTile +
                                    (wave * kScaleLanes + lane) * 4;
                __builtin_amdgcn_global_load_lds(ssrc, LDS_PTR(dst + kRrTileBytes + wave * kScaleLanes * 16), 16, 0,
                                                 kNonTemporal);
            }
        };

        auto score = [&](int i) {
            const uint32_t so = (i & (kRrSlots - 1)) * kRrSlotBytes;
            v4i kba[4], kbb[4];
            float ks_raw;
            lds_read_tile2(ka[0] + so, ka[1] + so, ka[2] + so, ka[3] + so, ksa + so, kba, kbb, ks_raw);
            const float ks = ks_raw * __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, d_ok), i));
            const uint32_t key = rg_key2<MT>(qa, wr, kba, kbb, ks);
            const int row = __builtin_amdgcn_readlane(d_b, i) * ROWS + wave;
            const int tok = __builtin_amdgcn_readlane(d_k, i) * kRrTile + lane;
            p.score_keys[static_cast<size_t>(row) * p.key_stride + tok] = static_cast<uint16_t>(key);
            if (tok < __builtin_amdgcn_readlane(d_valid, i)) lds_add_u32(hist_lds + (key >> 8) * 4, 1u);
        };

        const int b_first = __builtin_amdgcn_readlane(d_b, 0);
        if (b_first != qb) {
            rg_load_q<HEADS, W_BF16>(p, b_first * ROWS + wave, n, g, qscale, qa, wr);
            qb = b_first;
        }
#pragma unroll
        for (int j = 0; j < kRrDepth; ++j) issue(j);
        int i = 0;
        while (i < cnt) {  // runs of one request
            const int b = __builtin_amdgcn_readlane(d_b, i);
            if (b != qb) {
                rg_load_q<HEADS, W_BF16>(p, b * ROWS + wave, n, g, qscale, qa, wr);
                qb = b;
                __builtin_amdgcn_s_waitcnt(kVmcntZero);
            }
            const uint64_t later = run_ends >> i;
            const int run_end = i + static_cast<int>(__builtin_ctzll(later)) + 1;
            for (; i < run_end; ++i) {
                issue(i + kRrDepth);
                // Own share of tile i landed: after its loads come those of the next
                // kRrDepth tiles and the key stores of the (at most kRrDepth) tiles before i.
                if (i >= kRrDepth) {
                    wait_vmcnt<kRrDepth * kOps + kRrDepth>();
                } else if (kRrDepth > 3 && i == 3) {
                    wait_vmcnt<kRrDepth * kOps + (kRrDepth > 3 ? 3 : 0)>();
                } else if (kRrDepth > 2 && i == 2) {
                    wait_vmcnt<kRrDepth * kOps + (kRrDepth > 2 ? 2 : 0)>();
                } else if (kRrDepth > 1 && i == 1) {
                    wait_vmcnt<kRrDepth * kOps + (kRrDepth > 1 ? 1 : 0)>();
                } else {
                    wait_vmcnt<kRrDepth * kOps>();
                }
                __builtin_amdgcn_s_barrier();  // every wave's share of tile i landed
                score(i);
            }
            flush(b * ROWS + wave);
        }
        wait_vmcnt<0>();  // the repeated tail load lands before the ring is reused
        t += cnt;
    }
    report(p.status, err);
}

// Grid = workgroups per CU the kernel keeps resident times the CU count; the first
// dispatch round is one workgroup per CU.
struct RingGrid {
    int blocks;
    int lead_blocks;
};

template <typename K>
RingGrid ring_grid(K kernel) {
    static RingGrid grid{0, 0};
    if (grid.blocks == 0) {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kRgThreads, 0) != hipSuccess) {
            return grid;
        }
        grid = RingGrid{max(1, cus * max(per_cu, 1)), max(1, cus)};
    }
    return grid;
}

template <int HEADS, bool W_BF16>
hipError_t launch_ring_kernel(const KvipIndexerArgs& a, int tile_lo, int tile_hi, hipStream_t stream) {
    auto kernel = indexer_ring_kernel<HEADS, W_BF16>;
    const RingGrid grid = ring_grid(kernel);
    if (grid.blocks == 0) return hipErrorInvalidDevice;
    hipLaunchKernelGGL(kernel, dim3(grid.blocks), dim3(kRgThreads), 0, stream, a, grid.lead_blocks, tile_lo, tile_hi);
    return hipGetLastError();
}

template <int ROWS, int HEADS, bool W_BF16>
hipError_t launch_rows_kernel(const KvipIndexerArgs& a, hipStream_t stream) {
    auto kernel = indexer_rows_kernel<ROWS, HEADS, W_BF16>;
    static RingGrid grid{0, 0};
    if (grid.blocks == 0) {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, ROWS * 64, 0) != hipSuccess) {
            return hipErrorInvalidDevice;
        }
        grid = RingGrid{max(1, cus * max(per_cu, 1)), max(1, cus)};
    }
    hipLaunchKernelGGL(kernel, dim3(grid.blocks), dim3(ROWS * 64), 0, stream, a, grid.lead_blocks);
    return hipGetLastError();
}

template <int ROWS>
hipError_t launch_rows(const KvipIndexerArgs& a, hipStream_t stream) {
    if (a.heads == 64) {
        return a.weight_dtype == KVIP_DTYPE_BF16 ? launch_rows_kernel<ROWS, 64, true>(a, stream)
                                                 : launch_rows_kernel<ROWS, 64, false>(a, stream);
    }
    return a.weight_dtype == KVIP_DTYPE_BF16 ? launch_rows_kernel<ROWS, 32, true>(a, stream)
                                             : launch_rows_kernel<ROWS, 32, false>(a, stream);
}

}  // namespace

// fp8, one row per request, batch within the LDS prefix table, 16-byte aligned key-scale
// rows (direct-to-LDS loads move 16 bytes per lane) and 16-byte (8-byte for bf16) aligned
// weight and query-scale rows (vector loads of 4 heads).
bool ring_eligible(const KvipIndexerArgs& a) {
    const uintptr_t wal = a.weight_dtype == KVIP_DTYPE_BF16 ? 7u : 15u;
    return a.qk_dtype == KVIP_DTYPE_FP8_E4M3 && a.rows_per_request == 1 && a.batch <= kRgMaxBatch &&
           (reinterpret_cast<uintptr_t>(a.weights) & wal) == 0 &&
           (a.query_scale == nullptr || (reinterpret_cast<uintptr_t>(a.query_scale) & 15u) == 0) &&
           (a.key_scale == nullptr ||
            ((reinterpret_cast<uintptr_t>(a.key_scale) & 15u) == 0 && a.scale_block_stride % 4 == 0));
}

// fp8 with 2 or 4 rows per request, same batch and alignment limits as the one-row kernel.
bool ring_rows_eligible(const KvipIndexerArgs& a) {
    const uintptr_t wal = a.weight_dtype == KVIP_DTYPE_BF16 ? 7u : 15u;
    return a.qk_dtype == KVIP_DTYPE_FP8_E4M3 && (a.rows_per_request == 2 || a.rows_per_request == 4) &&
           a.batch <= kRgMaxBatch && (reinterpret_cast<uintptr_t>(a.weights) & wal) == 0 &&
           (a.query_scale == nullptr || (reinterpret_cast<uintptr_t>(a.query_scale) & 15u) == 0) &&
           (a.key_scale == nullptr ||
            ((reinterpret_cast<uintptr_t>(a.key_scale) & 15u) == 0 && a.scale_block_stride % 4 == 0));
}

hipError_t launch_indexer_ring_rows(const KvipIndexerArgs& a, hipStream_t stream) {
    return a.rows_per_request == 2 ? launch_rows<2>(a, stream) : launch_rows<4>(a, stream);
}

// Scores the 32-token tiles [tile_lo, tile_hi) of every row's visible positions.
hipError_t launch_indexer_ring(const KvipIndexerArgs& a, hipStream_t stream, int tile_lo, int tile_hi) {
    if (a.heads == 64) {
        return a.weight_dtype == KVIP_DTYPE_BF16 ? launch_ring_kernel<64, true>(a, tile_lo, tile_hi, stream)
                                                 : launch_ring_kernel<64, false>(a, tile_lo, tile_hi, stream);
    }
    return a.weight_dtype == KVIP_DTYPE_BF16 ? launch_ring_kernel<32, true>(a, tile_lo, tile_hi, stream)
                                             : launch_ring_kernel<32, false>(a, tile_lo, tile_hi, stream);
}

}  // namespace kvip
