// Prefill (and mixed-batch) lightning-indexer scoring on gfx950 MFMA: packed query rows of
// several sequences against their paged index-K under a right-down causal mask, fp8 e4m3
// or bf16 Q/K.
//
// Work unit = (query block, context segment): 8 consecutive query rows of one sequence
// against 4096 key positions (one unit per workgroup, or a bounded grid whose workgroups
// stride over the units, kvip_hip_indexer_prefill_grid). fp8: 4 waves own 2 query rows
// each; bf16 (Q fragments twice as large): 8 waves own one row each. A wave keeps its rows'
// Q fragments and per-lane head weights (w'_h = w_h * qscale_h for the 32 heads a lane
// reduces) in registers. The segment streams through LDS in 32 KiB chunks (256 fp8 or 128
// bf16 tokens), double buffered: every wave issues direct-to-LDS 16-byte loads
// (global_load_lds_dwordx4) for its share of the next chunk, with the XOR swizzle applied
// on the global side so that the fragment reads (lane n of a 32-token tile reads row n)
// hit distinct bank groups. Each chunk tile (32 tokens) is one B fragment set read once
// from LDS and reused by the wave's rows x 2 head tiles: 2 K slices each of
// v_mfma_scale_f32_32x32x64_f8f6f4 (fp8) or 8 of v_mfma_f32_32x32x16_bf16 (bf16). The
// epilogue is the decode kernel's: ReLU, head weights, head reduction, key scale, bf16
// half-away rounding, sortable key; keys go through a per-wave LDS strip to coalesced
// stores, and a per-workgroup 256-bin histogram of the key high byte (two 16-bit counters
// per word: bins b and b + 128; bf16, whose 64 lanes add to one row, keeps four copies per
// row) is added to the row histograms at the end. fp8 runs two workgroups per CU, bf16 one
// (two waves per SIMD either way).
//
// Reference: the native prefill LI (torch_npu.npu_quant_lightning_indexer, TND layout,
// sparse_mode 3) that the vLLM selector runs for prefill rows (python/kvip/adapters/vllm/
// selector.py:126-154); the score formula is the decode one (op_kernel/indexer/
// indexer_cube.h:161-322, indexer_score.h:384-426, score_common.h:66-97).
#include <algorithm>

#include "indexer_tile.h"
#include "lds_async.h"

namespace kvip {
namespace {

constexpr int kPfBlockRows = 8;                             // query rows per workgroup
// Waves per workgroup and query rows per wave: fp8 runs 4 waves of 2 rows (one row per lane
// half at the finish) and two workgroups per CU; bf16 Q fragments are twice as large, so it
// runs 8 waves of 1 row, which keeps a wave under 256 registers and gives two waves per SIMD
// in the one workgroup per CU.
template <int ELEM>
struct PfShape {
    static constexpr int kWaves = ELEM == 1 ? 4 : 8;
    static constexpr int kRows = kPfBlockRows / kWaves;
    static constexpr int kThreads = kWaves * 64;
};
constexpr int kPfChunkBytes = 256 * kIndexDim;             // 32 KiB of K rows per LDS chunk
constexpr int kPfSegment = 4096;                            // key positions per workgroup
constexpr int kPfPages = kPfSegment / kBlockTokens;         // 32
constexpr int kPfMaxSeq = KVIP_PREFILL_MAX_SEQUENCES;
// LDS piece swizzle of a staged K row of 8 (fp8) or 16 (bf16) 16-byte pieces: piece j of
// row r sits at slot j ^ (r & 15) (j ^ (r & 7) for 8 pieces). A fragment read (lane n
// reads piece j of row n) then touches distinct 16-byte slots in every group of 8 (16)
// consecutive lanes, i.e. every bank once per phase.
template <int ELEM>
KVIP_DEVICE int pf_swizzle(int row) { return row & (8 * ELEM - 1); }

template <bool W_BF16>
KVIP_DEVICE float pf_weight(const KvipPrefillArgs& p, size_t idx) {
    float w;
    if constexpr (W_BF16) {
        w = bf16_to_float(static_cast<const uint16_t*>(p.weights)[idx]);
    } else {
        w = static_cast<const float*>(p.weights)[idx];
    }
    return w * (p.query_scale != nullptr ? p.query_scale[idx] : 1.0f);
}

template <int ELEM, int HEADS, bool W_BF16>
__global__ __launch_bounds__(PfShape<ELEM>::kThreads, 3 - ELEM) void indexer_prefill_kernel(const KvipPrefillArgs p) {
    constexpr int kPfWaves = PfShape<ELEM>::kWaves;
    constexpr int kPfRowsPerWave = PfShape<ELEM>::kRows;
    constexpr int kPfThreads = PfShape<ELEM>::kThreads;
    constexpr int MT = HEADS / 32;
    constexpr int NV = Mma<ELEM>::NV;              // 16-byte pieces of a half row per lane
    constexpr int STEPS = Mma<ELEM>::STEPS;        // MFMAs per 128-dim contraction
    constexpr int kRowBytes = kIndexDim * ELEM;
    constexpr int kPieces = kRowBytes / 16;        // 16-byte pieces per K row
    constexpr int kPfChunk = kPfChunkBytes / kRowBytes;  // tokens per LDS chunk (256 or 128)
    constexpr int kPfTiles = kPfChunk / 32;
    constexpr int kChunkPages = kPfChunk / kBlockTokens;  // pages per chunk (2 or 1)
    constexpr int kRowsPerLoad = 64 / kPieces;     // K rows one 64-lane 16-byte load fills
    static_assert(kPfRowsPerWave == 1 || kPfRowsPerWave == 2, "the finish maps row q to lane half q");
    constexpr int kStageLoads = (kPfChunk / kPfWaves) / kRowsPerLoad;  // staging loads per wave and chunk
    static_assert(kStageLoads * kRowsPerLoad * kPfWaves == kPfChunk, "whole staging loads");
    __shared__ __align__(16) uint8_t s_k[2][kPfChunkBytes];
    __shared__ __align__(16) float s_ks[2][kPfChunk];
    __shared__ __align__(16) uint16_t s_keys[kPfWaves][kPfRowsPerWave][kPfChunk];
    // Row histograms: bins b (low half) and b + 128 (high half) of a word. bf16 (one row per
    // wave, all 64 lanes adding to one row) keeps kHistCopies copies per row, lane l adding to
    // copy l % kHistCopies, so that lanes whose keys share a bin do not serialise on one word;
    // the copies sit 144 words apart, i.e. 16 banks apart.
    constexpr int kHistCopies = kPfRowsPerWave == 1 ? 4 : 1;
    constexpr int kHistStride = kHistCopies > 1 ? 144 : 128;
    constexpr int kHistWords = kHistCopies * kHistStride;
    __shared__ uint32_t s_hist[kPfBlockRows][kHistWords];
    __shared__ int s_prefix[kPfMaxSeq + 1];
    __shared__ uint32_t s_scan[kPfWaves];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: row data stays scalar
    const int n = lane & 31;
    const int g = lane >> 5;

    // Query blocks per sequence -> prefix sums; this workgroup's sequence and rows.
    int running = 0;
    for (int base = 0; base < p.sequences; base += kPfThreads) {
        const int s = base + tid;
        const int c = s < p.sequences ? (p.cu_seqlens_q[s + 1] - p.cu_seqlens_q[s] + kPfBlockRows - 1) / kPfBlockRows : 0;
        uint32_t total;
        const uint32_t excl = block_exclusive_scan(static_cast<uint32_t>(max(c, 0)), s_scan, &total);
        if (s < p.sequences) s_prefix[s] = running + static_cast<int>(excl);
        running += static_cast<int>(total);
    }
    if (tid == 0) s_prefix[p.sequences] = running;
    for (int i = tid; i < kPfBlockRows * kHistWords; i += kPfThreads) (&s_hist[0][0])[i] = 0u;
    __syncthreads();
    // Work items (query block, segment), block-fastest: the launch holds one workgroup per
    // item, or fewer that stride over them (a bounded grid, for callers that run other
    // kernels beside the prefill: workgroups that run out of items free their CU instead
    // of queueing more items behind the other kernels).
    const int nb_items = p.rows / kPfBlockRows + p.sequences;
    const int64_t n_items =
        static_cast<int64_t>(nb_items) * ((p.max_blocks * kBlockTokens + kPfSegment - 1) / kPfSegment);
    uint32_t err = 0;
    for (int64_t item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int block = static_cast<int>(item) % nb_items;  // n_items <= 2^31 - 1 (validated)
    const int segi = static_cast<int>(item) / nb_items;
    if (block >= s_prefix[p.sequences]) continue;  // uniform
    int lo = 0, hi = p.sequences - 1;            // largest s with s_prefix[s] <= block
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_prefix[mid] <= block) lo = mid; else hi = mid - 1;
    }
    const int seq = lo;
    const int q0 = p.cu_seqlens_q[seq];
    const int q_len = p.cu_seqlens_q[seq + 1] - q0;
    const int k_len = min(max(p.seq_lens_k[seq], 0), p.max_blocks * kBlockTokens);
    const int j0 = (block - s_prefix[seq]) * kPfBlockRows;

    // The wave's two rows: visibility (right-down causal) and row_valid.
    int vis[kPfRowsPerWave];
    int rowi[kPfRowsPerWave];
#pragma unroll
    for (int q = 0; q < kPfRowsPerWave; ++q) {
        const int j = j0 + wave * kPfRowsPerWave + q;
        const bool live = j < q_len;
        rowi[q] = q0 + min(j, q_len - 1);
        vis[q] = live ? min(max(k_len - q_len + j + 1, 0), k_len) : 0;
        if (live && segi == 0 && lane == 0) p.row_valid[q0 + j] = vis[q];
    }
    const int last = min(j0 + kPfBlockRows, q_len) - 1;
    const int vis_max = min(max(k_len - q_len + last + 1, 0), k_len);
    const int seg0 = segi * kPfSegment;
    const int seg_end = min(seg0 + kPfSegment, vis_max);
    if (seg0 >= seg_end) continue;  // uniform: nothing visible in this segment
    const int nchunks = (seg_end - seg0 + kPfChunk - 1) / kPfChunk;

    // Q fragments and head weights of the wave's rows.
    v4i qa[kPfRowsPerWave][MT][NV];
    float wr[kPfRowsPerWave][MT * 16];
#pragma unroll
    for (int q = 0; q < kPfRowsPerWave; ++q) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const v4i* src = reinterpret_cast<const v4i*>(static_cast<const uint8_t*>(p.query) +
                                                          (static_cast<size_t>(rowi[q]) * HEADS + mt * 32 + n) * kRowBytes +
                                                          g * (kRowBytes / 2));
#pragma unroll
            for (int v = 0; v < NV; ++v) qa[q][mt][v] = src[v];
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    wr[q][mt * 16 + r4 * 4 + j] =
                        pf_weight<W_BF16>(p, static_cast<size_t>(rowi[q]) * HEADS + mt * 32 + r4 * 8 + g * 4 + j);
                }
            }
        }
    }

    // Page ids of the segment (lane i < 32 holds page seg0/128 + i, clamped to the
    // sequence's last page; out-of-range ids read block 0 with zero key scale).
    const int pages_k = (k_len + kBlockTokens - 1) / kBlockTokens;
    int my_page = 0;
    float my_ok = 0.0f;
    if (lane < kPfPages) {
        const int pi = min(seg0 / kBlockTokens + lane, max(pages_k - 1, 0));
        const int id = p.block_table[static_cast<size_t>(seq) * p.max_blocks + pi];
        const bool ok = static_cast<unsigned>(id) < static_cast<unsigned>(p.num_blocks);
        my_page = ok ? id : 0;
        my_ok = ok ? 1.0f : 0.0f;
        if (!ok) err |= KVIP_STATUS_BAD_BLOCK;
    }
    const uint8_t* kbase = static_cast<const uint8_t*>(p.keys);

    // Wave w stages rows [w * chunk/4, (w + 1) * chunk/4) of a chunk (one page's rows):
    // 8 direct-to-LDS loads of kRowsPerLoad rows each.
    constexpr int kWaveRows = kPfChunk / kPfWaves;
    auto stage = [&](int c, int buf) {
        const int pg = __builtin_amdgcn_readlane(my_page, c * kChunkPages + (wave * kWaveRows) / kBlockTokens);
#pragma unroll
        for (int v = 0; v < kStageLoads; ++v) {
            const int row = wave * kWaveRows + v * kRowsPerLoad + lane / kPieces;
            const int piece = (lane % kPieces) ^ pf_swizzle<ELEM>(row);
            const uint8_t* src = kbase + static_cast<size_t>(pg) * p.key_block_stride +
                                 (row & (kBlockTokens - 1)) * kRowBytes + piece * 16;
            __builtin_amdgcn_global_load_lds(src, LDS_PTR(&s_k[buf][(wave * kWaveRows + v * kRowsPerLoad) * kRowBytes]),
                                             16, 0, 0);
        }
        if (wave == 0 && p.key_scale != nullptr && lane < kPfChunk / 4) {
            const int row = lane * 4;  // 4 consecutive scales of one page
            // readlane takes a wave-uniform lane index: read both pages, pick per half-wave.
            const int pg0 = __builtin_amdgcn_readlane(my_page, c * kChunkPages);
            const int pg1 = __builtin_amdgcn_readlane(my_page, c * kChunkPages + kChunkPages - 1);
            const int pg = lane < 32 ? pg0 : pg1;
            const float* src = p.key_scale + static_cast<size_t>(pg) * p.scale_block_stride + (row & 127);
            __builtin_amdgcn_global_load_lds(src, LDS_PTR(&s_ks[buf][0]), 16, 0, 0);
        }
    };
    if (p.key_scale == nullptr) {  // unit key scales, written once before the loop
        for (int i = tid; i < 2 * kPfChunk; i += kPfThreads) (&s_ks[0][0])[i] = 1.0f;
        __syncthreads();
    }

    // This lane half's row (one row per wave: the row of both halves; its keys and
    // histogram come from lanes 0-31).
    int vis_mine, vis_max_wave;
    if constexpr (kPfRowsPerWave == 2) {
        vis_mine = g == 0 ? vis[0] : vis[1];
        vis_max_wave = max(vis[0], vis[1]);
    } else {
        vis_mine = g == 0 ? vis[0] : 0;
        vis_max_wave = vis[0];
    }
    const int hist_row = wave * kPfRowsPerWave + (kPfRowsPerWave == 2 ? g : 0);
    // Per-lane LDS addresses: the tile row's four swizzled K pieces (the swizzle of row
    // k*32 + n does not depend on k), its key scale, and the key strip slots.
    uint32_t ka[NV];
#pragma unroll
    for (int u = 0; u < NV; ++u) ka[u] = lds_addr(&s_k[0][n * kRowBytes + (((g * NV + u) ^ pf_swizzle<ELEM>(n)) * 16)]);
    const uint32_t ksa = lds_addr(&s_ks[0][n]);
    const uint32_t keya = lds_addr(&s_keys[wave][kPfRowsPerWave == 2 ? g : 0][n]);
    const uint32_t hista = lds_addr(&s_hist[hist_row][(lane % kHistCopies) * kHistStride]);
    constexpr uint32_t kKBuf = kPfChunkBytes;          // bytes between the two K buffers
    constexpr uint32_t kSBuf = kPfChunk * 4;           // bytes between the two scale buffers

    stage(0, 0);
    int stores = 0;  // key stores this wave issued after the latest staging loads
    for (int c = 0; c < nchunks; ++c) {
        const int buf = c & 1;
        lds_barrier(stores);  // chunk c landed and is visible; buffer c+1 is free again
        if (c + 1 < nchunks) stage(c + 1, buf ^ 1);
        const int cstart = seg0 + c * kPfChunk;
        const float page_ok0 =
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_ok), c * kChunkPages));
        const float page_ok1 = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_ok), c * kChunkPages + kChunkPages - 1));
        if constexpr (kPfRowsPerWave == 1) {
            // One row per wave (bf16): two tiles per step, finished together. Lane half g
            // finishes tile k + g: one lane-half swap joins both tiles' head halves, so every
            // lane stores a key and counts it (the same sums, in the same order, as one tile
            // at a time).
#pragma unroll 1
            for (int k = 0; k < kPfTiles; k += 2) {
                const int t0 = cstart + k * 32;
                if (t0 >= vis_max_wave) break;  // uniform per wave: later tiles are masked too
                float part2[2];
                float ks = 0.f;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int kt = k + h;
                    v4i kb[NV];
                    float ks_raw;
                    const uint32_t toff = buf * kKBuf + kt * 32 * kRowBytes;
                    lds_read_tile8(ka, toff, ksa + buf * kSBuf + kt * 128, kb, ks_raw);
                    if (g == h) ks = ks_raw * (kt < kPfTiles / 2 ? page_ok0 : page_ok1);
                // Units u = (row q = u / MT, head tile mt = u % MT), two dependent K-slice MFMAs
                // each. Unit u+1's MFMAs are issued between the 32 VALU ops (ReLU, weight FMA) of
                // unit u's epilogue so that the matrix core and the VALU work side by side.
                constexpr int U = kPfRowsPerWave * MT;
                float pj[kPfRowsPerWave][4];
#pragma unroll
                for (int q = 0; q < kPfRowsPerWave; ++q) pj[q][0] = pj[q][1] = pj[q][2] = pj[q][3] = 0.f;
                v16f acc[2];
                acc[0] = v16f{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int st = 0; st < STEPS; ++st) Mma<ELEM>::step(st, qa[0][0], kb, acc[0]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int q = u / MT, mt = u % MT;
                    v16f& cur = acc[u & 1];
                    v16f& nxt = acc[(u + 1) & 1];
                    if (u + 1 < U) {
                        nxt = v16f{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int st = 0; st < STEPS; ++st) Mma<ELEM>::step(st, qa[(u + 1) / MT][(u + 1) % MT], kb, nxt);
                    }
#pragma unroll
                    for (int r4 = 0; r4 < 4; ++r4) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                                const float relu = __int_as_float(max(__float_as_int(cur[r4 * 4 + j]), 0));
                                pj[q][j] = fmaf(relu, wr[q][mt * 16 + r4 * 4 + j], pj[q][j]);
                        }
                    }
                    if (u + 1 < U) {
                        // The next unit's STEPS MFMAs spread over this unit's 32 VALU ops (fp8:
                        // 1 MFMA, 16 VALU, 1 MFMA, 16 VALU; bf16: 1 MFMA, 4 VALU, ...); nothing
                        // crosses into the next unit.
#pragma unroll
                        for (int st = 0; st < STEPS; ++st) {
                                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                                __builtin_amdgcn_sched_group_barrier(0x002, 32 / STEPS, 0);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                    part2[h] = (pj[0][0] + pj[0][1]) + (pj[0][2] + pj[0][3]);
                }
                // [tile k lanes 0-31, tile k + 1 lanes 0-31] + [tile k lanes 32-63, tile k + 1 lanes 32-63].
                const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(part2[0]), __float_as_int(part2[1]),
                                                                 false, false);
                const float total = __int_as_float(sw[0]) + __int_as_float(sw[1]);
                const uint32_t key = sortable_key(bf16_bits_half_away(total * ks));
                lds_write_b16(keya + (k + g) * 64, key);
                if (t0 + 32 * g + n < vis[0]) {
                    const uint32_t bin = key >> 8;
                    lds_add_u32(hista + (bin & 127) * 4, 1u << (16 * (bin >> 7)));
                }
            }
        } else {
    #pragma unroll 1
            for (int k = 0; k < kPfTiles; ++k) {
                const int t0 = cstart + k * 32;
                if (t0 >= vis_max_wave) break;  // uniform per wave: later tiles are masked too
                v4i kb[NV];
                float ks_raw;
                const uint32_t toff = buf * kKBuf + k * 32 * kRowBytes;
                if constexpr (ELEM == 1) {
                    lds_read_tile(ka[0] + toff, ka[1] + toff, ka[2] + toff, ka[3] + toff, ksa + buf * kSBuf + k * 128, kb,
                                  ks_raw);
                } else {
                    lds_read_tile8(ka, toff, ksa + buf * kSBuf + k * 128, kb, ks_raw);
                }
                const float ks = ks_raw * (k < kPfTiles / 2 ? page_ok0 : page_ok1);
                // Units u = (row q = u / MT, head tile mt = u % MT), two dependent K-slice MFMAs
                // each. Unit u+1's MFMAs are issued between the 32 VALU ops (ReLU, weight FMA) of
                // unit u's epilogue so that the matrix core and the VALU work side by side.
                constexpr int U = kPfRowsPerWave * MT;
                float pj[kPfRowsPerWave][4];
    #pragma unroll
                for (int q = 0; q < kPfRowsPerWave; ++q) pj[q][0] = pj[q][1] = pj[q][2] = pj[q][3] = 0.f;
                v16f acc[2];
                acc[0] = v16f{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    #pragma unroll
                for (int st = 0; st < STEPS; ++st) Mma<ELEM>::step(st, qa[0][0], kb, acc[0]);
                __builtin_amdgcn_sched_barrier(0);
    #pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int q = u / MT, mt = u % MT;
                    v16f& cur = acc[u & 1];
                    v16f& nxt = acc[(u + 1) & 1];
                    if (u + 1 < U) {
                        nxt = v16f{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    #pragma unroll
                        for (int st = 0; st < STEPS; ++st) Mma<ELEM>::step(st, qa[(u + 1) / MT][(u + 1) % MT], kb, nxt);
                    }
    #pragma unroll
                    for (int r4 = 0; r4 < 4; ++r4) {
    #pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const float relu = __int_as_float(max(__float_as_int(cur[r4 * 4 + j]), 0));
                            pj[q][j] = fmaf(relu, wr[q][mt * 16 + r4 * 4 + j], pj[q][j]);
                        }
                    }
                    if (u + 1 < U) {
                        // The next unit's STEPS MFMAs spread over this unit's 32 VALU ops (fp8:
                        // 1 MFMA, 16 VALU, 1 MFMA, 16 VALU; bf16: 1 MFMA, 4 VALU, ...); nothing
                        // crosses into the next unit.
    #pragma unroll
                        for (int st = 0; st < STEPS; ++st) {
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                            __builtin_amdgcn_sched_group_barrier(0x002, 32 / STEPS, 0);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                // Two rows finish together: after the swap, lanes 0-31 hold row 0's total for
                // token n and lanes 32-63 row 1's (each the sum of the two lane halves' heads).
                // One row: both halves hold its total.
                const float part0 = (pj[0][0] + pj[0][1]) + (pj[0][2] + pj[0][3]);
                float mine = part0, other = part0;
                if constexpr (kPfRowsPerWave == 2) {
                    const float part1 = (pj[1][0] + pj[1][1]) + (pj[1][2] + pj[1][3]);
                    mine = g == 0 ? part0 : part1;
                    other = g == 0 ? part1 : part0;
                }
                const auto swapped =
                    __builtin_amdgcn_permlane32_swap(__float_as_int(other), __float_as_int(other), false, false);
                const float total = mine + __int_as_float(g == 0 ? swapped[1] : swapped[0]);
                const uint32_t key = sortable_key(bf16_bits_half_away(total * ks));
                if (kPfRowsPerWave == 2 || g == 0) lds_write_b16(keya + k * 64, key);
                if (t0 + n < vis_mine) {
                    // Bins b and b ^ 128 share a word: the populated bins of a row are adjacent
                    // and would otherwise serialise on one word's atomics.
                    const uint32_t bin = key >> 8;
                    lds_add_u32(hista + (bin & 127) * 4, 1u << (16 * (bin >> 7)));
                }
            }
        }
        // Flush the chunk's keys of the wave's rows (8-byte stores, inside the row stride).
        // Lane 0's store is always in range (cstart < key_stride, both multiples of 8), so
        // each live row issues exactly one store instruction.
        stores = 0;
#pragma unroll
        for (int q = 0; q < kPfRowsPerWave; ++q) {
            if (cstart >= vis[q]) continue;  // uniform
            const int o = min(lane * 4, kPfChunk - 4);
            const v2i v = lds_read_b64(lds_addr(&s_keys[wave][q][o]));
            if (lane * 4 < kPfChunk && cstart + o + 4 <= p.key_stride) {
                *reinterpret_cast<v2i*>(p.score_keys + static_cast<size_t>(rowi[q]) * p.key_stride + cstart + o) = v;
            }
            ++stores;
        }
    }
    lds_barrier(0);
    // Histogram of the workgroup's rows.
    for (int i = tid; i < kPfBlockRows * 256; i += kPfThreads) {
        const int rq = i >> 8;
        const int bin = i & 255;
        const int j = j0 + rq;
        uint32_t c = 0u;
#pragma unroll
        for (int cp = 0; cp < kHistCopies; ++cp) c += (s_hist[rq][cp * kHistStride + (bin & 127)] >> (16 * (bin >> 7))) & 0xFFFFu;
        if (j < q_len && c != 0u) atomicAdd(&p.histogram[static_cast<size_t>(q0 + j) * 256 + bin], c);
    }
    if (item + gridDim.x < n_items) {  // uniform: clear the row histograms for the next item
        __syncthreads();
        for (int i = tid; i < kPfBlockRows * kHistWords; i += kPfThreads) (&s_hist[0][0])[i] = 0u;
        __syncthreads();
    }
    }
    report(p.status, err);
}

// Work items: (query blocks bound) x (segments of the bound context).
int64_t prefill_items(const KvipPrefillArgs& a) {
    const int64_t blocks = a.rows / kPfBlockRows + a.sequences;  // bound on the per-sequence blocks
    return blocks * ((static_cast<int64_t>(a.max_blocks) * kBlockTokens + kPfSegment - 1) / kPfSegment);
}

template <int ELEM, int HEADS>
hipError_t launch_heads(const KvipPrefillArgs& a, int workgroups, hipStream_t stream) {
    const int64_t items = prefill_items(a);
    const dim3 grid(static_cast<unsigned>(workgroups > 0 ? std::min<int64_t>(items, workgroups) : items));
    if (a.weight_dtype == KVIP_DTYPE_BF16) {
        hipLaunchKernelGGL((indexer_prefill_kernel<ELEM, HEADS, true>), grid, dim3(PfShape<ELEM>::kThreads), 0, stream,
                           a);
    } else {
        hipLaunchKernelGGL((indexer_prefill_kernel<ELEM, HEADS, false>), grid, dim3(PfShape<ELEM>::kThreads), 0, stream,
                           a);
    }
    return hipGetLastError();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

uint32_t validate_prefill(const KvipPrefillArgs* a) {
    if (a == nullptr) return KVIP_ERR_INVALID;
    const bool ok =
        a->query != nullptr && a->weights != nullptr && a->keys != nullptr && a->block_table != nullptr &&
        a->cu_seqlens_q != nullptr && a->seq_lens_k != nullptr && a->score_keys != nullptr &&
        a->histogram != nullptr && a->row_valid != nullptr &&
        (a->qk_dtype == KVIP_DTYPE_FP8_E4M3 || a->qk_dtype == KVIP_DTYPE_BF16) &&
        (a->weight_dtype == KVIP_DTYPE_FP32 || a->weight_dtype == KVIP_DTYPE_BF16) &&
        (a->heads == 32 || a->heads == 64) && a->sequences >= 1 && a->sequences <= kPfMaxSeq && a->rows >= 1 &&
        a->rows <= (1 << 24) && a->max_blocks >= 1 && a->num_blocks >= 1 &&
        a->max_blocks <= (1 << 24) / kBlockTokens &&
        static_cast<int64_t>(a->key_stride) >= static_cast<int64_t>(a->max_blocks) * kBlockTokens &&
        a->key_stride % 8 == 0 && a->key_block_stride % 16 == 0 &&
        a->key_block_stride >=
            static_cast<int64_t>(kBlockTokens) * kIndexDim * (a->qk_dtype == KVIP_DTYPE_BF16 ? 2 : 1) &&
        (a->key_scale == nullptr || (a->scale_block_stride >= kBlockTokens && a->scale_block_stride % 4 == 0 &&
                                     (reinterpret_cast<uintptr_t>(a->key_scale) & 15u) == 0)) &&
        aligned16(a->query) && aligned16(a->keys) && aligned16(a->score_keys) &&
        prefill_items(*a) <= 0x7FFFFFFF;
    return ok ? KVIP_OK : KVIP_ERR_INVALID;
}

hipError_t launch_prefill(const KvipPrefillArgs& a, hipStream_t stream, int workgroups) {
    if (a.qk_dtype == KVIP_DTYPE_BF16) {
        return a.heads == 64 ? launch_heads<2, 64>(a, workgroups, stream) : launch_heads<2, 32>(a, workgroups, stream);
    }
    return a.heads == 64 ? launch_heads<1, 64>(a, workgroups, stream) : launch_heads<1, 32>(a, workgroups, stream);
}

}  // namespace kvip

extern "C" uint32_t kvip_hip_indexer_prefill(const KvipPrefillArgs* args, void* stream) {
    const uint32_t rc = kvip::validate_prefill(args);
    if (rc != KVIP_OK) return rc;
    return static_cast<uint32_t>(kvip::launch_prefill(*args, static_cast<hipStream_t>(stream), 0));
}

extern "C" uint32_t kvip_hip_indexer_prefill_grid(const KvipPrefillArgs* args, int32_t workgroups, void* stream) {
    const uint32_t rc = kvip::validate_prefill(args);
    if (rc != KVIP_OK) return rc;
    if (workgroups < 0) return KVIP_ERR_INVALID;
    return static_cast<uint32_t>(kvip::launch_prefill(*args, static_cast<hipStream_t>(stream), workgroups));
}
