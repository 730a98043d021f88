// Fetch: gather the selected KV rows (656-byte MLA latent rows: 512 fp8 nope + 64 bf16
// rope + 4 fp32 scales) from a paged HBM KV cache into a contiguous [rows, 2048, row]
// buffer. Pure byte movement: each thread moves 16-byte pieces, the output side is
// fully coalesced, the input side reads whole rows (a row is row_bytes/16 consecutive
// pieces). Entries of -1 produce zero rows.
//
// Reference semantics: per descriptor, dst = output + output_index * token_bytes,
// src = the token's row, copy token_bytes (kvaf_device::KvafBatchGetDevice as called
// from FetchQueryGroup, op_kernel/streaming.cpp:365-500, :445; UBmem form
// patches/kvaf-ubmem-device-get.patch:41-90; row layout
// tests/operators/lifetch/support/workloads.py:493-515).
#include "kvip_device.h"

namespace kvip {
namespace {

constexpr int kGatherThreads = 256;
constexpr int kRowsPerWave = 32;
constexpr int kRowsPerBlock = kRowsPerWave * (kGatherThreads / 64);
// Outputs above this size are stored with the nontemporal policy: they do not fit the
// 256 MB memory-side cache, so caching the stream only evicts lines the gather still reads
// (4-row MTP decode, 344 MB: 145 -> 141 us); smaller outputs (config 2, 86 MB) stay
// cached, where the default policy is 3 us faster.
constexpr uint64_t kStreamOutputBytes = 192ull << 20;

// One wave moves 32 consecutive selected rows: lanes 0..31 translate the token ids to
// source rows (token id -> block table -> byte offset), then all 64 lanes copy the
// 32*PIECES 16-byte pieces (21 loads in flight per lane for 656-byte rows). Because the
// destination rows are consecutive, the wave's output
// is one contiguous range written with fully coalesced 16-byte stores.
template <int PIECES, bool NT_STORE>
__global__ __launch_bounds__(kGatherThreads) void fetch_gather_kernel(const KvipFetchArgs p, uint32_t selections) {
    const int pieces = PIECES > 0 ? PIECES : p.row_bytes / 16;
    const int lane = threadIdx.x & 63;
    uint32_t err = 0;
    const uint32_t sel0 = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6) * kRowsPerWave;
    if (sel0 >= selections) return;
    const int capacity = p.max_blocks * kBlockTokens;

    // Source byte offset of row (sel0 + lane), or -1 for an empty / invalid entry.
    int64_t src = -1;
    if (lane < kRowsPerWave && sel0 + lane < selections) {
        const uint32_t sel = sel0 + lane;
        const int t = p.topk[sel];
        const int b = static_cast<int>(sel / kTopK) / p.rows_per_request;
        if (t >= capacity) {
            err |= KVIP_STATUS_BAD_TOKEN;
        } else if (t >= 0) {
            const int blk = p.block_table[static_cast<size_t>(b) * p.max_blocks + (t >> 7)];
            if (static_cast<unsigned>(blk) < static_cast<unsigned>(p.num_blocks)) {
                src = static_cast<int64_t>(blk) * p.kv_block_stride + static_cast<int64_t>(t & 127) * p.row_stride;
            } else {
                err |= KVIP_STATUS_BAD_BLOCK;
            }
        }
    }
    const int rows = min(kRowsPerWave, static_cast<int>(selections - sel0));
    const int total = rows * pieces;
    uint8_t* dst = p.output + static_cast<size_t>(sel0) * p.row_bytes;
    constexpr int kMaxIters = PIECES > 0 ? (kRowsPerWave * PIECES + 63) / 64 : 1;
    if constexpr (PIECES > 0) {
        v4i val[kMaxIters];
#pragma unroll
        for (int it = 0; it < kMaxIters; ++it) {
            const int idx = it * 64 + lane;
            const int r = idx / PIECES;
            const int piece = idx - r * PIECES;
            const int64_t base = row_value<PIECES, kRowsPerWave>(src, it, r);
            val[it] = v4i{0, 0, 0, 0};
            if (idx < total && base >= 0) {
                val[it] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p.kv_cache + base + piece * 16));
            }
        }
#pragma unroll
        for (int it = 0; it < kMaxIters; ++it) {
            const int idx = it * 64 + lane;
            if (idx >= total) continue;
            v4i* out = reinterpret_cast<v4i*>(dst + static_cast<size_t>(idx) * 16);
            if constexpr (NT_STORE) {
                __builtin_nontemporal_store(val[it], out);
            } else {
                *out = val[it];
            }
        }
    } else {
        const int iters = (kRowsPerWave * pieces + 63) / 64;  // uniform: every lane joins each shuffle
        for (int it = 0; it < iters; ++it) {
            const int idx = it * 64 + lane;
            const int r = idx / pieces;
            const int piece = idx - r * pieces;
            const int64_t base = __shfl(src, min(r, kRowsPerWave - 1));
            v4i v = v4i{0, 0, 0, 0};
            if (idx < total && base >= 0) v = *reinterpret_cast<const v4i*>(p.kv_cache + base + piece * 16);
            if (idx < total) *reinterpret_cast<v4i*>(dst + static_cast<size_t>(idx) * 16) = v;
        }
    }
    report(p.status, err);
}

}  // namespace

uint32_t validate_fetch(const KvipFetchArgs* a) {
    if (a == nullptr) return KVIP_ERR_INVALID;
    const bool ok = a->topk != nullptr && a->kv_cache != nullptr && a->block_table != nullptr && a->output != nullptr &&
                    a->row_bytes >= 16 && a->row_bytes % 16 == 0 && a->row_stride >= a->row_bytes &&
                    a->row_stride % 16 == 0 && a->kv_block_stride % 16 == 0 &&
                    a->kv_block_stride >= static_cast<int64_t>(kBlockTokens) * a->row_stride &&
                    (a->rows_per_request == 1 || a->rows_per_request == 2 || a->rows_per_request == 4) &&
                    a->batch >= 1 && a->max_blocks >= 1 && a->num_blocks >= 1 &&
                    a->max_blocks <= (1 << 24) / kBlockTokens &&
                    static_cast<int64_t>(a->batch) * a->rows_per_request * kTopK * (a->row_bytes / 16) < (1ll << 40) &&
                    static_cast<int64_t>(a->batch) * a->rows_per_request * kTopK < (1ll << 31) &&
                    (reinterpret_cast<uintptr_t>(a->kv_cache) & 15u) == 0 &&
                    (reinterpret_cast<uintptr_t>(a->output) & 15u) == 0;
    return ok ? KVIP_OK : KVIP_ERR_INVALID;
}

hipError_t launch_fetch(const KvipFetchArgs& a, hipStream_t stream) {
    const uint32_t selections = static_cast<uint32_t>(a.batch) * a.rows_per_request * kTopK;
    const dim3 grid((selections + kRowsPerBlock - 1) / kRowsPerBlock);
    const bool stream_out = static_cast<uint64_t>(selections) * a.row_bytes > kStreamOutputBytes;
    if (a.row_bytes == KVIP_KV_ROW_BYTES) {
        if (stream_out) {
            hipLaunchKernelGGL((fetch_gather_kernel<KVIP_KV_ROW_BYTES / 16, true>), grid, dim3(kGatherThreads), 0,
                               stream, a, selections);
        } else {
            hipLaunchKernelGGL((fetch_gather_kernel<KVIP_KV_ROW_BYTES / 16, false>), grid, dim3(kGatherThreads), 0,
                               stream, a, selections);
        }
    } else {
        hipLaunchKernelGGL((fetch_gather_kernel<0, false>), grid, dim3(kGatherThreads), 0, stream, a, selections);
    }
    return hipGetLastError();
}

}  // namespace kvip

extern "C" uint32_t kvip_hip_fetch_gather(const KvipFetchArgs* args, void* stream) {
    const uint32_t rc = kvip::validate_fetch(args);
    if (rc != KVIP_OK) return rc;
    return static_cast<uint32_t>(kvip::launch_fetch(*args, static_cast<hipStream_t>(stream)));
}
