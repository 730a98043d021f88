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
// Work split: one workgroup = 4 waves = one 512-token chunk of one request; each
// wave streams 4 tiles of 32 tokens (4 KiB of fp8 index-K) through a three-deep
// register pipeline. Tile loads are fully coalesced (lane L reads the L-th 16 bytes
// of each KiB) and are transposed into MFMA B fragments through a swizzled per-wave
// LDS tile; lane (n = lane%32, g = lane/32) then holds 64*elem contiguous bytes of
// token n's row at byte offset 64*elem*g, and the Q fragments (A operand) use the
// same lane->byte assignment, so the contraction pairs identical dims in both
// operands. Keys are staged in LDS and written once per chunk, so the tile loop's
// only vector-memory operations are its loads (exact vmcnt waits).
//
// Reference: QLIMatmul::ComputeMm1 (op_kernel/indexer/indexer_cube.h:161-322),
// MulWeightAndReduceSum bf16-weight variant (indexer_score.h:384-426, loop :60-103,
// finalize :105-140), FloatToSortableKey (score_common.h:66-97).
#include "kvip_device.h"

namespace kvip {
namespace {

constexpr int kLiWaves = 4;
constexpr int kLiThreads = kLiWaves * 64;
constexpr int kTileTokens = 32;
constexpr int kTilesPerWave = 4;
constexpr int kChunkTokens = kLiWaves * kTilesPerWave * kTileTokens;  // 512

// ELEM = bytes per Q/K element (1: fp8 e4m3, 2: bf16). Each lane holds NV = 4*ELEM
// 16-byte vectors of one Q or K row.
template <int ELEM>
struct Mma;

template <>
struct Mma<1> {
    static constexpr int NV = 4;
    KVIP_DEVICE static void run(const v4i (&a)[NV], const v4i (&b)[NV], v16f& acc) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const v8i av = __builtin_shufflevector(a[2 * s], a[2 * s + 1], 0, 1, 2, 3, 4, 5, 6, 7);
            const v8i bv = __builtin_shufflevector(b[2 * s], b[2 * s + 1], 0, 1, 2, 3, 4, 5, 6, 7);
            // Format 0 = fp8 e4m3 for both operands; E8M0 scale 127 = 2^0.
            acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc, 0, 0, 0, 127, 0, 127);
        }
    }
};

template <>
struct Mma<2> {
    static constexpr int NV = 8;
    KVIP_DEVICE static void run(const v4i (&a)[NV], const v4i (&b)[NV], v16f& acc) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a[s]),
                                                          __builtin_bit_cast(v8bf, b[s]), acc, 0, 0, 0);
        }
    }
};

// LDS piece swizzle of a staged K row (8 or 16 pieces of 16 bytes per row).
template <int ELEM>
KVIP_DEVICE int swizzle(int row) {
    return ELEM == 1 ? ((row >> 1) & 7) : (row & 15);
}

template <int ELEM, int HEADS, int RPR, bool W_BF16>
__global__ __launch_bounds__(kLiThreads) void indexer_decode_kernel(const KvipIndexerArgs p) {
    constexpr int MT = HEADS / 32;
    constexpr int NV = Mma<ELEM>::NV;
    constexpr int ROW_BYTES = kIndexDim * ELEM;
    __shared__ __align__(16) float s_w[RPR * HEADS];
    __shared__ uint32_t s_hist[RPR * 256];
    __shared__ __align__(16) uint16_t s_keys[RPR * kChunkTokens];
    __shared__ __align__(16) uint8_t s_tile[kLiWaves * kTileTokens * ROW_BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = lane & 31;
    const int g = lane >> 5;
    const int b = blockIdx.y;
    const int capacity = p.max_blocks * kBlockTokens;

    const int seq = max(p.seq_lens[b], 0);
    int valid[RPR];
    int vmax = 0;
#pragma unroll
    for (int q = 0; q < RPR; ++q) {
        int v = seq;
        if (p.query_ends != nullptr) v = min(v, p.query_ends[b * RPR + q]);
        v = min(max(v, 0), capacity);
        valid[q] = v;
        vmax = max(vmax, v);
    }
    const int chunk0 = blockIdx.x * kChunkTokens;
    if (chunk0 >= vmax) return;  // uniform for the workgroup

    for (int i = tid; i < RPR * HEADS; i += kLiThreads) {
        const int row = b * RPR + i / HEADS;
        const int h = i % HEADS;
        float w;
        if constexpr (W_BF16) {
            w = bf16_to_float(static_cast<const uint16_t*>(p.weights)[row * HEADS + h]);
        } else {
            w = static_cast<const float*>(p.weights)[row * HEADS + h];
        }
        const float s = p.query_scale != nullptr ? p.query_scale[row * HEADS + h] : 1.0f;
        s_w[i] = w * s;
    }
    for (int i = tid; i < RPR * 256; i += kLiThreads) s_hist[i] = 0u;

    // Q fragments (A operand): row = head mt*32 + n, bytes [64*ELEM*g, 64*ELEM*(g+1)).
    v4i qa[RPR][MT][NV];
    const uint8_t* qbase = static_cast<const uint8_t*>(p.query);
#pragma unroll
    for (int q = 0; q < RPR; ++q) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const v4i* src = reinterpret_cast<const v4i*>(
                qbase + (static_cast<size_t>(b * RPR + q) * HEADS + mt * 32 + n) * ROW_BYTES + g * (ROW_BYTES / 2));
#pragma unroll
            for (int v = 0; v < NV; ++v) qa[q][mt][v] = src[v];
        }
    }
    __syncthreads();

    const uint8_t* kbase = static_cast<const uint8_t*>(p.keys);
    const int32_t* table = p.block_table + static_cast<size_t>(b) * p.max_blocks;
    uint32_t err = 0;

    // The wave's 256 tokens span two pages; their block ids are read once (scalar). Tiles
    // past the row end reload the wave's last live tile so that every load in the
    // pipeline is unconditional (exact vmcnt waits); their results are discarded.
    constexpr int kWavePages = kTilesPerWave * kTileTokens / kBlockTokens;
    constexpr int kTilesPerPage = kBlockTokens / kTileTokens;
    const int wave_t0 = chunk0 + __builtin_amdgcn_readfirstlane(wave) * (kTilesPerWave * kTileTokens);
    const int ntiles = min(max((vmax - wave_t0 + kTileTokens - 1) / kTileTokens, 0), kTilesPerWave);
    int page[kWavePages];
    float page_ok[kWavePages];
#pragma unroll
    for (int j = 0; j < kWavePages; ++j) {
        const int jj = min(j, max(ntiles - 1, 0) / kTilesPerPage);
        const int id = table[min((wave_t0 >> 7) + jj, p.max_blocks - 1)];
        const bool ok = static_cast<unsigned>(id) < static_cast<unsigned>(p.num_blocks);
        if (!ok && j * kTilesPerPage < ntiles) err |= KVIP_STATUS_BAD_BLOCK;
        page[j] = ok ? id : 0;
        page_ok[j] = ok ? 1.0f : 0.0f;
    }

    // Tile loads are fully coalesced: lane L reads 16-byte piece L of each 1 KiB of the
    // tile. They are transposed into MFMA fragments through the wave's own LDS tile.
    auto issue = [&](int i, v4i (&kb)[NV], float& ks) {
        const int ii = min(i, max(ntiles - 1, 0));
        const int pg = page[(ii * kTileTokens) / kBlockTokens];
        const int first = (ii * kTileTokens) & 127;
        const v4i* src = reinterpret_cast<const v4i*>(kbase + static_cast<size_t>(pg) * p.key_block_stride +
                                                      first * ROW_BYTES);
#pragma unroll
        for (int v = 0; v < NV; ++v) kb[v] = src[v * 64 + lane];
        ks = p.key_scale != nullptr ? p.key_scale[static_cast<size_t>(pg) * p.scale_block_stride + first + n] : 1.0f;
        ks *= page_ok[(ii * kTileTokens) / kBlockTokens];  // a bad block id scores 0
    };

    // Keys of the chunk are staged in LDS and written out once, so the tile loop's only
    // vector-memory operations are its loads.
    auto compute = [&](int i, const v4i (&staged)[NV], float ks) {
        const int local = wave * (kTilesPerWave * kTileTokens) + i * kTileTokens + n;
        const int tok = chunk0 + local;
        // Row r's 16-byte piece j lives at r*ROW_BYTES + (j ^ swz(r))*16 in the wave's LDS
        // tile: the 16 lanes of each ds_*_b128 pass then touch 16 distinct bank groups.
        uint8_t* tile = s_tile + wave * (kTileTokens * ROW_BYTES);
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int d = v * 1024 + lane * 16;
            const int r = d / ROW_BYTES;
            const int j = (d % ROW_BYTES) / 16;
            *reinterpret_cast<v4i*>(tile + r * ROW_BYTES + ((j ^ swizzle<ELEM>(r)) * 16)) = staged[v];
        }
        v4i kb[NV];
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            const int j = g * NV + u;
            kb[u] = *reinterpret_cast<const v4i*>(tile + n * ROW_BYTES + ((j ^ swizzle<ELEM>(n)) * 16));
        }
#pragma unroll
        for (int q = 0; q < RPR; ++q) {
            v16f acc[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                acc[mt] = v16f{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                Mma<ELEM>::run(qa[q][mt], kb, acc[mt]);
            }
            // acc[mt][r] holds head mt*32 + 8*(r/4) + 4*g + r%4 for token n.
            float part = 0.0f;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const v4f w = *reinterpret_cast<const v4f*>(&s_w[q * HEADS + mt * 32 + r4 * 8 + g * 4]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        // ReLU as an integer max: every negative float (sign bit set) maps to
                        // +0, one instruction without NaN canonicalisation.
                        const float relu = __int_as_float(max(__float_as_int(acc[mt][r4 * 4 + j]), 0));
                        part = fmaf(relu, w[j], part);
                    }
                }
            }
            part += __shfl_xor(part, 32);
            const float score = part * ks;
            const uint32_t key = sortable_key(bf16_bits_half_away(score));
            if (g == 0) {
                s_keys[q * kChunkTokens + local] = static_cast<uint16_t>(key);
                if (tok < valid[q]) atomicAdd(&s_hist[q * 256 + (key >> 8)], 1u);
            }
        }
    };

    // Three-deep register pipeline over the wave's tiles, fully unrolled so that the
    // buffers rotate by name (no register copies).
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

template <int ELEM, int HEADS, int RPR>
hipError_t launch_rpr(const KvipIndexerArgs& a, dim3 grid, hipStream_t stream) {
    if (a.weight_dtype == KVIP_DTYPE_BF16) {
        hipLaunchKernelGGL((indexer_decode_kernel<ELEM, HEADS, RPR, true>), grid, dim3(kLiThreads), 0, stream, a);
    } else {
        hipLaunchKernelGGL((indexer_decode_kernel<ELEM, HEADS, RPR, false>), grid, dim3(kLiThreads), 0, stream, a);
    }
    return hipGetLastError();
}

template <int ELEM, int HEADS>
hipError_t launch_heads(const KvipIndexerArgs& a, dim3 grid, hipStream_t stream) {
    switch (a.rows_per_request) {
        case 1: return launch_rpr<ELEM, HEADS, 1>(a, grid, stream);
        case 2: return launch_rpr<ELEM, HEADS, 2>(a, grid, stream);
        default: return launch_rpr<ELEM, HEADS, 4>(a, grid, stream);
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
    const int capacity = a.max_blocks * kBlockTokens;
    const dim3 grid((capacity + kChunkTokens - 1) / kChunkTokens, a.batch);
    if (a.qk_dtype == KVIP_DTYPE_FP8_E4M3) {
        return a.heads == 64 ? launch_heads<1, 64>(a, grid, stream) : launch_heads<1, 32>(a, grid, stream);
    }
    return a.heads == 64 ? launch_heads<2, 64>(a, grid, stream) : launch_heads<2, 32>(a, grid, stream);
}

}  // namespace kvip

extern "C" uint32_t kvip_hip_indexer_decode(const KvipIndexerArgs* args, void* stream) {
    const uint32_t rc = kvip::validate_indexer(args);
    if (rc != KVIP_OK) return rc;
    return static_cast<uint32_t>(kvip::launch_indexer(*args, static_cast<hipStream_t>(stream)));
}
