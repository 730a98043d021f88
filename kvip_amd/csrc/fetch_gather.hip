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
constexpr int kPiecesPerThread = 4;

template <int PIECES>
__global__ __launch_bounds__(kGatherThreads) void fetch_gather_kernel(const KvipFetchArgs p, uint64_t total) {
    const int pieces = PIECES > 0 ? PIECES : p.row_bytes / 16;
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * (kGatherThreads * kPiecesPerThread) + threadIdx.x;
    const int capacity = p.max_blocks * kBlockTokens;
    uint32_t err = 0;
    v4i val[kPiecesPerThread];
    uint64_t dst[kPiecesPerThread];
#pragma unroll
    for (int u = 0; u < kPiecesPerThread; ++u) {
        const uint64_t c = base + static_cast<uint64_t>(u) * kGatherThreads;
        val[u] = v4i{0, 0, 0, 0};
        dst[u] = ~0ull;
        if (c >= total) continue;
        const uint32_t sel = static_cast<uint32_t>(c / static_cast<uint32_t>(pieces));
        const uint32_t piece = static_cast<uint32_t>(c - static_cast<uint64_t>(sel) * pieces);
        const int row = static_cast<int>(sel / kTopK);
        const int b = row / p.rows_per_request;
        const int t = p.topk[sel];
        dst[u] = static_cast<uint64_t>(sel) * p.row_bytes + piece * 16u;
        if (t < 0) continue;
        if (t >= capacity) {
            err |= KVIP_STATUS_BAD_TOKEN;
            continue;
        }
        const int blk = p.block_table[static_cast<size_t>(b) * p.max_blocks + (t >> 7)];
        if (static_cast<unsigned>(blk) >= static_cast<unsigned>(p.num_blocks)) {
            err |= KVIP_STATUS_BAD_BLOCK;
            continue;
        }
        const uint8_t* src = p.kv_cache + static_cast<size_t>(blk) * p.kv_block_stride +
                             static_cast<size_t>(t & 127) * p.row_stride + piece * 16u;
        val[u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(src));
    }
#pragma unroll
    for (int u = 0; u < kPiecesPerThread; ++u) {
        if (dst[u] != ~0ull) *reinterpret_cast<v4i*>(p.output + dst[u]) = val[u];
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
    const uint64_t total = static_cast<uint64_t>(a.batch) * a.rows_per_request * kTopK * (a.row_bytes / 16);
    const uint64_t per_block = kGatherThreads * kPiecesPerThread;
    const dim3 grid(static_cast<unsigned>((total + per_block - 1) / per_block));
    if (a.row_bytes == KVIP_KV_ROW_BYTES) {
        hipLaunchKernelGGL(fetch_gather_kernel<KVIP_KV_ROW_BYTES / 16>, grid, dim3(kGatherThreads), 0, stream, a, total);
    } else {
        hipLaunchKernelGGL(fetch_gather_kernel<0>, grid, dim3(kGatherThreads), 0, stream, a, total);
    }
    return hipGetLastError();
}

}  // namespace kvip

extern "C" uint32_t kvip_hip_fetch_gather(const KvipFetchArgs* args, void* stream) {
    const uint32_t rc = kvip::validate_fetch(args);
    if (rc != KVIP_OK) return rc;
    return static_cast<uint32_t>(kvip::launch_fetch(*args, static_cast<hipStream_t>(stream)));
}
