// Decode lightning-indexer scoring on gfx950 MFMA.
//
// Per request b the contraction Q_b[heads x 128] x K[128 x tokens] runs as 32x32
// MFMA tiles (fp8: v_mfma_scale_f32_32x32x64_f8f6f4 with unit scales; bf16:
// v_mfma_f32_32x32x16_bf16). Rows of the tile are heads, columns are 32 tokens of
// one 128-token page. The epilogue fuses ReLU, the per-head weight w'_h =
// w_h * qscale_h, the head reduction, the per-token key scale, the bf16 rounding
// (half away from zero) and the sortable-key transform, so only 2 bytes per
// (row, token) leave the kernel, plus a 256-bin histogram of the key's high byte
// that lets TopK skip one pass over the keys.
//
// Work split (streaming kernel): the (request, 32-token tile) pairs of the whole batch
// are flattened and every wave of a persistent grid streams one contiguous, balanced
// range of them through a three-deep register pipeline, reloading Q only when its
// range crosses into the next request. Batches larger than kStreamMaxBatch use the
// chunked kernel (one workgroup per 512-token chunk of one request). Tile loads are fully coalesced (lane L reads the L-th 16 bytes
// of each KiB) and are transposed into MFMA B fragments through a swizzled per-wave
// LDS tile; lane (n = lane%32, g = lane/32) then holds 64*elem contiguous bytes of
// token n's row at byte offset 64*elem*g, and the Q fragments (A operand) use the
// same lane->byte assignment, so the contraction pairs identical dims in both
// operands. Every load and key store of the tile loop is unconditional (tiles past a
// range end repeat its last tile), which keeps LLVM's vmcnt waits exact.
//
// Reference: QLIMatmul::ComputeMm1 (op_kernel/indexer/indexer_cube.h:161-322),
// MulWeightAndReduceSum bf16-weight variant (indexer_score.h:384-426, loop :60-103,
// finalize :105-140), FloatToSortableKey (score_common.h:66-97).
#include "indexer_tile.h"

namespace kvip {

// fp8 decode with one row per request: the LDS-ring kernel (indexer_ring.hip).
bool ring_eligible(const KvipIndexerArgs& a);
hipError_t launch_indexer_ring(const KvipIndexerArgs& a, hipStream_t stream, int tile_lo = 0,
                               int tile_hi = 1 << 30);
// fp8 decode with 2 or 4 rows per request: the shared-ring kernel (indexer_ring.hip).
bool ring_rows_eligible(const KvipIndexerArgs& a);
hipError_t launch_indexer_ring_rows(const KvipIndexerArgs& a, hipStream_t stream);

namespace {

constexpr int kLiWaves = 4;
constexpr int kLiThreads = kLiWaves * 64;
constexpr int kTileTokens = 32;
constexpr int kTilesPerWave = 4;                                        // chunked kernel
constexpr int kChunkTokens = kLiWaves * kTilesPerWave * kTileTokens;    // 512
constexpr int kStreamMaxBatch = 2048;
// Tiles per streaming sub-segment: its keys fit the wave's 4 KiB LDS key strip (and
// its page ids one register per lane).
template <int RPR>
constexpr int kSegmentTiles = 64 / RPR;

// Stands in for a missing per-token key-scale array, so that the scale load of every
// tile is unconditional (stride 0 keeps the index inside this table). Not const: it
// must share the global address space with the kernel arguments, or the select of
// the two pointers becomes a flat load.
__device__ float kUnitScale[kBlockTokens] = {
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f,
    1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};

template <int ELEM, int HEADS, int RPR>
struct Tile {
    static constexpr int MT = HEADS / 32;
    static constexpr int NV = Mma<ELEM>::NV;
    static constexpr int ROW_BYTES = kIndexDim * ELEM;
    static constexpr int BYTES = kTileTokens * ROW_BYTES;

    // Coalesced load of a 32-token tile: lane L reads the L-th 16 bytes of every KiB.
    KVIP_DEVICE static void load(const uint8_t* tile_base, int lane, v4i (&staged)[NV]) {
        const v4i* src = reinterpret_cast<const v4i*>(tile_base);
#pragma unroll
        for (int v = 0; v < NV; ++v) staged[v] = src[v * 64 + lane];
    }

    // Q fragments (A operand) of query row `row`: head mt*32 + n, bytes [64*ELEM*g, +64*ELEM).
    KVIP_DEVICE static void load_q(const uint8_t* query, int row, int lane, v4i (&qa)[MT][NV]) {
        const int n = lane & 31, g = lane >> 5;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const v4i* src = reinterpret_cast<const v4i*>(
                query + (static_cast<size_t>(row) * HEADS + mt * 32 + n) * ROW_BYTES + g * (ROW_BYTES / 2));
#pragma unroll
            for (int v = 0; v < NV; ++v) qa[mt][v] = src[v];
        }
    }

    // Transposes a staged tile into B fragments through the wave's LDS tile. Row r's
    // 16-byte piece j lives at r*ROW_BYTES + (j ^ swizzle(r))*16, so the 16 lanes of each
    // ds_*_b128 pass touch 16 distinct bank groups.
    KVIP_DEVICE static void fragments(const v4i (&staged)[NV], uint8_t* lds, int lane, v4i (&kb)[NV]) {
        const int n = lane & 31, g = lane >> 5;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int d = v * 1024 + lane * 16;
            const int r = d / ROW_BYTES;
            const int j = (d % ROW_BYTES) / 16;
            *reinterpret_cast<v4i*>(lds + r * ROW_BYTES + ((j ^ swizzle<ELEM>(r)) * 16)) = staged[v];
        }
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            const int j = g * NV + u;
            kb[u] = *reinterpret_cast<const v4i*>(lds + n * ROW_BYTES + ((j ^ swizzle<ELEM>(n)) * 16));
        }
    }

    // Sortable key of token n (= lane % 32, same value in both lane halves) for one query
    // row: MFMA over 64*ELEM... bytes, then ReLU, weights, head reduction, key scale,
    // bf16 half-away rounding, sortable transform.
    KVIP_DEVICE static uint32_t key(const v4i (&qa)[MT][NV], const v4i (&kb)[NV], const float* w_row, float ks,
                                    int lane) {
        const int g = lane >> 5;
        v16f acc[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            acc[mt] = v16f{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int s = 0; s < Mma<ELEM>::STEPS; ++s) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) Mma<ELEM>::step(s, qa[mt], kb, acc[mt]);
        }
        // acc[mt][r] holds head mt*32 + 8*(r/4) + 4*g + r%4 for token n. Four independent
        // FMA chains (one per r%4) keep the reduction off the critical path.
        float pj[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const v4f w = *reinterpret_cast<const v4f*>(&w_row[mt * 32 + r4 * 8 + g * 4]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // ReLU as an integer max: every negative float (sign bit set) maps to +0,
                    // one instruction without NaN canonicalisation.
                    const float relu = __int_as_float(max(__float_as_int(acc[mt][r4 * 4 + j]), 0));
                    pj[j] = fmaf(relu, w[j], pj[j]);
                }
            }
        }
        float part = (pj[0] + pj[1]) + (pj[2] + pj[3]);
        // Add the other lane half's heads (v_permlane32_swap: lane l <-> lane l^32).
        const auto swapped = __builtin_amdgcn_permlane32_swap(__float_as_int(part), __float_as_int(part), false, false);
        part += __int_as_float(g == 0 ? swapped[1] : swapped[0]);
        return sortable_key(bf16_bits_half_away(part * ks));
    }
};

template <bool W_BF16>
KVIP_DEVICE float weight_at(const KvipIndexerArgs& p, int idx) {
    float w;
    if constexpr (W_BF16) {
        w = bf16_to_float(static_cast<const uint16_t*>(p.weights)[idx]);
    } else {
        w = static_cast<const float*>(p.weights)[idx];
    }
    return w * (p.query_scale != nullptr ? p.query_scale[idx] : 1.0f);
}

KVIP_DEVICE int row_valid(const KvipIndexerArgs& p, int b, int row) {
    int v = max(p.seq_lens[b], 0);
    if (p.query_ends != nullptr) v = min(v, p.query_ends[row]);
    return min(max(v, 0), p.max_blocks * kBlockTokens);
}

// ---------------------------------------------------------------------------------
// Streaming kernel (batch <= kStreamMaxBatch).
// ---------------------------------------------------------------------------------
template <int ELEM, int HEADS, int RPR, bool W_BF16>
__global__ __launch_bounds__(kLiThreads) void indexer_stream_kernel(const KvipIndexerArgs p) {
    using T = Tile<ELEM, HEADS, RPR>;
    constexpr int MT = T::MT;
    constexpr int NV = T::NV;
    __shared__ int s_prefix[kStreamMaxBatch + 1];
    __shared__ uint32_t s_scan[kLiWaves];
    __shared__ __align__(16) float s_w[kLiWaves][RPR * HEADS];
    __shared__ uint32_t s_hist[kLiWaves][RPR * 256];
    __shared__ __align__(16) uint8_t s_tile[kLiWaves][T::BYTES];
    constexpr int SEG = kSegmentTiles<RPR>;
    __shared__ __align__(16) uint16_t s_keys[kLiWaves][RPR * SEG * kTileTokens];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = lane & 31;
    const int g = lane >> 5;

    // Tile counts per request -> prefix sums (whole workgroup, once).
    int running = 0;
    for (int base = 0; base < p.batch; base += kLiThreads) {
        const int b = base + tid;
        int c = 0;
        if (b < p.batch) {
            int vmax = 0;
#pragma unroll
            for (int q = 0; q < RPR; ++q) vmax = max(vmax, row_valid(p, b, b * RPR + q));
            c = (vmax + kTileTokens - 1) / kTileTokens;
        }
        uint32_t total;
        const uint32_t excl = block_exclusive_scan(static_cast<uint32_t>(c), s_scan, &total);
        if (b < p.batch) s_prefix[b] = running + static_cast<int>(excl);
        running += static_cast<int>(total);
    }
    if (tid == 0) s_prefix[p.batch] = running;
    for (int i = lane; i < RPR * 256; i += 64) s_hist[wave][i] = 0u;
    __syncthreads();

    // This wave's balanced share [t, t_end) of the flattened tile list.
    const int total_tiles = s_prefix[p.batch];
    const int64_t nw = static_cast<int64_t>(gridDim.x) * kLiWaves;
    const int64_t w = static_cast<int64_t>(blockIdx.x) * kLiWaves + __builtin_amdgcn_readfirstlane(wave);
    int t = static_cast<int>(total_tiles * w / nw);
    const int t_end = static_cast<int>(total_tiles * (w + 1) / nw);
    if (t >= t_end) return;  // no barriers follow: waves run independently from here
    int lo = 0, hi = p.batch - 1;  // largest b with s_prefix[b] <= t
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_prefix[mid] <= t) lo = mid; else hi = mid - 1;
    }
    int b = lo;

    const uint8_t* kbase = static_cast<const uint8_t*>(p.keys);
    const float* kscale = p.key_scale != nullptr ? p.key_scale : kUnitScale;
    const int64_t kscale_stride = p.key_scale != nullptr ? p.scale_block_stride : 0;
    uint8_t* lds_tile = s_tile[wave];
    uint16_t* keys_lds = s_keys[wave];
    float* w_rows = s_w[wave];
    uint32_t* hist = s_hist[wave];
    uint32_t err = 0;

    while (t < t_end) {  // one segment = this wave's tiles of request b
        while (s_prefix[b + 1] <= t) ++b;
        const int req_first = s_prefix[b];
        const int seg_end = min(t_end, s_prefix[b + 1]);
        int valid[RPR];
#pragma unroll
        for (int q = 0; q < RPR; ++q) valid[q] = row_valid(p, b, b * RPR + q);
        v4i qa[RPR][MT][NV];
#pragma unroll
        for (int q = 0; q < RPR; ++q) T::load_q(static_cast<const uint8_t*>(p.query), b * RPR + q, lane, qa[q]);
        for (int i = lane; i < RPR * HEADS; i += 64) w_rows[i] = weight_at<W_BF16>(p, b * RPR * HEADS + i);
        const int32_t* table = p.block_table + static_cast<size_t>(b) * p.max_blocks;

        while (t < seg_end) {  // sub-segments: page ids in one register per lane, keys in LDS
            const int f = t - req_first;                  // first tile (within the request)
            const int cnt = min(seg_end - t, SEG);
            const int page0 = f >> 2;
            const int npages = ((f + cnt - 1) >> 2) - page0 + 1;
            int my_page = 0;
            float my_ok = 0.0f;
            if (lane < npages) {
                const int id = table[page0 + lane];
                const bool ok = static_cast<unsigned>(id) < static_cast<unsigned>(p.num_blocks);
                my_page = ok ? id : 0;
                my_ok = ok ? 1.0f : 0.0f;
                if (!ok) err |= KVIP_STATUS_BAD_BLOCK;
            }
            // Loaded values are only consumed in compute(), never next to their load.
            auto issue = [&](int i, v4i (&staged)[NV], float& ks) {
                const int k = f + min(i, cnt - 1);
                const int slot = __builtin_amdgcn_readlane(my_page, (k >> 2) - page0);
                const int first = (k & 3) * kTileTokens;
                T::load(kbase + static_cast<size_t>(slot) * p.key_block_stride + first * T::ROW_BYTES, lane, staged);
                ks = kscale[static_cast<size_t>(slot) * kscale_stride + first + n];
            };
            // The tile loop's only vector-memory operations are its loads: keys go to the
            // wave's LDS strip (a repeated last tile rewrites identical keys).
            auto compute = [&](int i, const v4i (&staged)[NV], float ks_raw) {
                const int li = min(i, cnt - 1);
                const int tok = (f + li) * kTileTokens + n;
                const float ks = ks_raw * __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                    __builtin_bit_cast(int, my_ok), ((f + li) >> 2) - page0));  // bad block id -> 0
                v4i kb[NV];
                T::fragments(staged, lds_tile, lane, kb);
#pragma unroll
                for (int q = 0; q < RPR; ++q) {
                    const uint32_t key = T::key(qa[q], kb, w_rows + q * HEADS, ks, lane);
                    if (g == 0) {
                        keys_lds[q * SEG * kTileTokens + li * kTileTokens + n] = static_cast<uint16_t>(key);
                        if (i < cnt && tok < valid[q]) atomicAdd(&hist[q * 256 + (key >> 8)], 1u);
                    }
                }
            };
            // The scheduling barriers keep the loads in issue order, so the wait state is the
            // same on entry and around the back edge (exact vmcnt waits in the loop).
            v4i b0[NV], b1[NV], b2[NV];
            float k0, k1, k2;
            issue(0, b0, k0);
            __builtin_amdgcn_sched_barrier(0);
            issue(1, b1, k1);
            __builtin_amdgcn_sched_barrier(0);
            for (int i = 0; i < cnt; i += 3) {
                issue(i + 2, b2, k2);
                __builtin_amdgcn_sched_barrier(0);
                compute(i, b0, k0);
                issue(i + 3, b0, k0);
                __builtin_amdgcn_sched_barrier(0);
                compute(i + 1, b1, k1);
                issue(i + 4, b1, k1);
                __builtin_amdgcn_sched_barrier(0);
                compute(i + 2, b2, k2);
            }
            // Flush the sub-segment's keys: 8 bytes per lane per store, coalesced. Keys past
            // `valid` stay inside the row and are never read.
#pragma unroll
            for (int q = 0; q < RPR; ++q) {
                uint16_t* dst = p.score_keys + static_cast<size_t>(b * RPR + q) * p.key_stride + f * kTileTokens;
                const uint16_t* src = keys_lds + q * SEG * kTileTokens;
                for (int o = lane * 4; o < cnt * kTileTokens; o += 256) {
                    *reinterpret_cast<uint2*>(dst + o) = *reinterpret_cast<const uint2*>(src + o);
                }
            }
            t += cnt;
        }
        // Flush the request's histogram.
        for (int i = lane; i < RPR * 256; i += 64) {
            const uint32_t c = hist[i];
            if (c != 0u) {
                atomicAdd(&p.histogram[static_cast<size_t>(b) * RPR * 256 + i], c);
                hist[i] = 0u;
            }
        }
    }
    report(p.status, err);
}

// ---------------------------------------------------------------------------------
// Chunked kernel (any batch): one workgroup per 512-token chunk of one request.
// ---------------------------------------------------------------------------------
template <int ELEM, int HEADS, int RPR, bool W_BF16>
__global__ __launch_bounds__(kLiThreads) void indexer_chunk_kernel(const KvipIndexerArgs p) {
    using T = Tile<ELEM, HEADS, RPR>;
    constexpr int MT = T::MT;
    constexpr int NV = T::NV;
    __shared__ __align__(16) float s_w[RPR * HEADS];
    __shared__ uint32_t s_hist[RPR * 256];
    __shared__ __align__(16) uint16_t s_keys[RPR * kChunkTokens];
    __shared__ __align__(16) uint8_t s_tile[kLiWaves][T::BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = lane & 31;
    const int g = lane >> 5;
    const int b = blockIdx.y;

    int valid[RPR];
    int vmax = 0;
#pragma unroll
    for (int q = 0; q < RPR; ++q) {
        valid[q] = row_valid(p, b, b * RPR + q);
        vmax = max(vmax, valid[q]);
    }
    const int chunk0 = blockIdx.x * kChunkTokens;
    if (chunk0 >= vmax) return;  // uniform for the workgroup

    for (int i = tid; i < RPR * HEADS; i += kLiThreads) s_w[i] = weight_at<W_BF16>(p, b * RPR * HEADS + i);
    for (int i = tid; i < RPR * 256; i += kLiThreads) s_hist[i] = 0u;
    v4i qa[RPR][MT][NV];
#pragma unroll
    for (int q = 0; q < RPR; ++q) T::load_q(static_cast<const uint8_t*>(p.query), b * RPR + q, lane, qa[q]);
    __syncthreads();

    const uint8_t* kbase = static_cast<const uint8_t*>(p.keys);
    const float* kscale = p.key_scale != nullptr ? p.key_scale : kUnitScale;
    const int64_t kscale_stride = p.key_scale != nullptr ? p.scale_block_stride : 0;
    const int32_t* table = p.block_table + static_cast<size_t>(b) * p.max_blocks;
    uint32_t err = 0;

    // The wave's 128 tokens are one page, read once (scalar). Tiles past the row end
    // reload the wave's last live tile so that every load is unconditional.
    const int wave_t0 = chunk0 + __builtin_amdgcn_readfirstlane(wave) * (kTilesPerWave * kTileTokens);
    const int ntiles = min(max((vmax - wave_t0 + kTileTokens - 1) / kTileTokens, 0), kTilesPerWave);
    const int id = table[min(wave_t0 >> 7, p.max_blocks - 1)];
    const bool ok = static_cast<unsigned>(id) < static_cast<unsigned>(p.num_blocks);
    if (!ok && ntiles > 0) err |= KVIP_STATUS_BAD_BLOCK;
    const int page = ok ? id : 0;

    auto issue = [&](int i, v4i (&staged)[NV], float& ks) {
        const int first = min(i, max(ntiles - 1, 0)) * kTileTokens;
        T::load(kbase + static_cast<size_t>(page) * p.key_block_stride + first * T::ROW_BYTES, lane, staged);
        ks = kscale[static_cast<size_t>(page) * kscale_stride + first + n] * (ok ? 1.0f : 0.0f);
    };
    // Keys of the chunk are staged in LDS and written out once.
    auto compute = [&](int i, const v4i (&staged)[NV], float ks) {
        const int local = wave * (kTilesPerWave * kTileTokens) + i * kTileTokens + n;
        const int tok = chunk0 + local;
        v4i kb[NV];
        T::fragments(staged, s_tile[wave], lane, kb);
#pragma unroll
        for (int q = 0; q < RPR; ++q) {
            const uint32_t key = T::key(qa[q], kb, s_w + q * HEADS, ks, lane);
            if (g == 0) {
                s_keys[q * kChunkTokens + local] = static_cast<uint16_t>(key);
                if (tok < valid[q]) atomicAdd(&s_hist[q * 256 + (key >> 8)], 1u);
            }
        }
    };
    static_assert(kTilesPerWave * kTileTokens == kBlockTokens, "a chunk wave covers one page");
    v4i buf[3][NV];
    float ksb[3];
    issue(0, buf[0], ksb[0]);
    issue(1, buf[1], ksb[1]);
#pragma unroll
    for (int i = 0; i < kTilesPerWave; ++i) {
        if (i + 2 < kTilesPerWave) issue(i + 2, buf[(i + 2) % 3], ksb[(i + 2) % 3]);
        if (i < ntiles) compute(i, buf[i % 3], ksb[i % 3]);
    }
    __syncthreads();

    // Write the chunk's keys (8 bytes per thread per store) and histogram.
#pragma unroll
    for (int q = 0; q < RPR; ++q) {
        const int live = min(valid[q] - chunk0, kChunkTokens);
        uint16_t* dst = p.score_keys + static_cast<size_t>(b * RPR + q) * p.key_stride + chunk0;
        for (int t = tid * 4; t < live; t += kLiThreads * 4) {
            if (t + 4 <= live) {
                *reinterpret_cast<uint2*>(dst + t) = *reinterpret_cast<const uint2*>(&s_keys[q * kChunkTokens + t]);
            } else {
                for (int u = t; u < live; ++u) dst[u] = s_keys[q * kChunkTokens + u];
            }
        }
    }
    for (int i = tid; i < RPR * 256; i += kLiThreads) {
        const uint32_t c = s_hist[i];
        if (c != 0u) atomicAdd(&p.histogram[static_cast<size_t>(b) * RPR * 256 + i], c);
    }
    report(p.status, err);
}

// Workgroups per CU the streaming kernel can keep resident (queried once per
// instantiation) times the CU count: a grid that fills the GPU exactly once.
template <typename K>
int stream_grid(K kernel) {
    static int grid = 0;
    if (grid == 0) {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kLiThreads, 0) != hipSuccess) {
            return 0;
        }
        grid = max(1, cus * max(per_cu, 1));
    }
    return grid;
}

template <int ELEM, int HEADS, int RPR, bool W_BF16>
hipError_t launch_kernel(const KvipIndexerArgs& a, hipStream_t stream) {
    if (ring_eligible(a)) return launch_indexer_ring(a, stream);
    if (ring_rows_eligible(a)) return launch_indexer_ring_rows(a, stream);
    if (a.batch <= kStreamMaxBatch) {
        auto kernel = indexer_stream_kernel<ELEM, HEADS, RPR, W_BF16>;
        const int grid = stream_grid(kernel);
        if (grid == 0) return hipErrorInvalidDevice;
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(kLiThreads), 0, stream, a);
    } else {
        const dim3 grid((a.max_blocks * kBlockTokens + kChunkTokens - 1) / kChunkTokens, a.batch);
        hipLaunchKernelGGL((indexer_chunk_kernel<ELEM, HEADS, RPR, W_BF16>), grid, dim3(kLiThreads), 0, stream, a);
    }
    return hipGetLastError();
}

template <int ELEM, int HEADS, int RPR>
hipError_t launch_rpr(const KvipIndexerArgs& a, hipStream_t stream) {
    return a.weight_dtype == KVIP_DTYPE_BF16 ? launch_kernel<ELEM, HEADS, RPR, true>(a, stream)
                                             : launch_kernel<ELEM, HEADS, RPR, false>(a, stream);
}

template <int ELEM, int HEADS>
hipError_t launch_heads(const KvipIndexerArgs& a, hipStream_t stream) {
    switch (a.rows_per_request) {
        case 1: return launch_rpr<ELEM, HEADS, 1>(a, stream);
        case 2: return launch_rpr<ELEM, HEADS, 2>(a, stream);
        default: return launch_rpr<ELEM, HEADS, 4>(a, stream);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

uint32_t validate_indexer(const KvipIndexerArgs* a) {
    if (a == nullptr) return KVIP_ERR_INVALID;
    const int elem = a->qk_dtype == KVIP_DTYPE_FP8_E4M3 ? 1 : 2;
    const bool ok =
        a->query != nullptr && a->weights != nullptr && a->keys != nullptr && a->block_table != nullptr &&
        a->seq_lens != nullptr && a->score_keys != nullptr && a->histogram != nullptr &&
        (a->qk_dtype == KVIP_DTYPE_FP8_E4M3 || a->qk_dtype == KVIP_DTYPE_BF16) &&
        (a->weight_dtype == KVIP_DTYPE_FP32 || a->weight_dtype == KVIP_DTYPE_BF16) &&
        (a->heads == 32 || a->heads == 64) &&
        (a->rows_per_request == 1 || a->rows_per_request == 2 || a->rows_per_request == 4) &&
        a->batch >= 1 && a->batch <= 65535 && a->max_blocks >= 1 && a->num_blocks >= 1 &&
        a->max_blocks <= (1 << 24) / kBlockTokens &&
        static_cast<int64_t>(a->key_stride) >= static_cast<int64_t>(a->max_blocks) * kBlockTokens &&
        a->key_stride % 8 == 0 && a->key_block_stride % 16 == 0 &&
        a->key_block_stride >= static_cast<int64_t>(kBlockTokens) * kIndexDim * elem &&
        (a->key_scale == nullptr || a->scale_block_stride >= kBlockTokens) &&
        aligned16(a->query) && aligned16(a->keys) && aligned16(a->score_keys);
    return ok ? KVIP_OK : KVIP_ERR_INVALID;
}

hipError_t launch_indexer(const KvipIndexerArgs& a, hipStream_t stream) {
    if (a.qk_dtype == KVIP_DTYPE_FP8_E4M3) {
        return a.heads == 64 ? launch_heads<1, 64>(a, stream) : launch_heads<1, 32>(a, stream);
    }
    return a.heads == 64 ? launch_heads<2, 64>(a, stream) : launch_heads<2, 32>(a, stream);
}

}  // namespace kvip

extern "C" uint32_t kvip_hip_indexer_decode(const KvipIndexerArgs* args, void* stream) {
    const uint32_t rc = kvip::validate_indexer(args);
    if (rc != KVIP_OK) return rc;
    return static_cast<uint32_t>(kvip::launch_indexer(*args, static_cast<hipStream_t>(stream)));
}

extern "C" uint32_t kvip_hip_indexer_decode_window(const KvipIndexerArgs* args, int32_t token_begin,
                                                   int32_t token_end, void* stream) {
    const uint32_t rc = kvip::validate_indexer(args);
    if (rc != KVIP_OK) return rc;
    if (!kvip::ring_eligible(*args) || token_begin < 0 || token_end <= token_begin || token_begin % 128 != 0 ||
        (token_end % 128 != 0 && token_end < args->key_stride)) {
        return KVIP_ERR_INVALID;
    }
    const int end = static_cast<int>(std::min<int64_t>(token_end, args->key_stride));
    return static_cast<uint32_t>(
        kvip::launch_indexer_ring(*args, static_cast<hipStream_t>(stream), token_begin / 32, (end + 31) / 32));
}
