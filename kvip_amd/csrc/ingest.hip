// Decode query packing and Index-K ingestion on gfx950 (the vLLM adapter's device work).
//
// kvip_hip_pack_queries: QueryInputs.bind_positions + QueryInputs.pack
// (python/kvip/adapters/vllm/inputs.py:127-152) in one launch, one workgroup per packed
// query row: query_ends[r] = (positions[gather[r]] + 1) * valid[r], and the row's fp8 Q
// bytes, bf16 head weights and fp32 head scales are copied from token gather[r].
//
// kvip_hip_ingest_index: VllmIndexCacheStorage.ingest_decode / ingest_prefill
// (python/kvip/adapters/vllm/index_import.py:18-52): 128-byte index-K rows and their
// fp32 scales copied from the paged cache into [owner, position] storage. Eight lanes
// move one row (16 bytes each), a 256-thread workgroup moves 32 rows.
#include "kvip_device.h"

namespace kvip {
namespace {

constexpr int kPackThreads = 256;
constexpr int kIngestThreads = 256;
constexpr int kIngestRowsPerBlock = kIngestThreads / 8;

__global__ __launch_bounds__(kPackThreads) void pack_queries_kernel(const KvipQueryPackArgs p) {
    const int r = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t src = p.gather_indices[r];
    const bool in_range = src >= 0 && src < p.tokens;
    if (!in_range && tid == 0) report(p.status, KVIP_STATUS_BAD_TOKEN);
    if (p.positions != nullptr && tid == 0) {
        const int64_t end = in_range ? (p.positions[src] + 1) * p.query_valid[r] : 0;
        p.query_ends[r] = static_cast<int32_t>(end);
    }
    if (p.query_in == nullptr) return;
    const int q_vecs = p.heads * kIndexDim / 16;
    const int w_vecs = p.heads * 2 / 16;
    const int s_vecs = p.heads * 4 / 16;
    const uint4 zero = make_uint4(0, 0, 0, 0);
    const uint4* qs = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(p.query_in) + src * p.heads * kIndexDim);
    const uint4* ws = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(p.weights_in) + src * p.heads * 2);
    const uint4* ss = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(p.scale_in) + src * p.heads * 4);
    uint4* qd = reinterpret_cast<uint4*>(static_cast<uint8_t*>(p.query_out) + static_cast<int64_t>(r) * p.heads * kIndexDim);
    uint4* wd = reinterpret_cast<uint4*>(static_cast<uint8_t*>(p.weights_out) + static_cast<int64_t>(r) * p.heads * 2);
    uint4* sd = reinterpret_cast<uint4*>(static_cast<uint8_t*>(p.scale_out) + static_cast<int64_t>(r) * p.heads * 4);
    for (int i = tid; i < q_vecs; i += kPackThreads) qd[i] = in_range ? qs[i] : zero;
    if (tid < w_vecs) wd[tid] = in_range ? ws[tid] : zero;
    if (tid < s_vecs) sd[tid] = in_range ? ss[tid] : zero;
}

__global__ __launch_bounds__(kIngestThreads) void ingest_index_kernel(const KvipIngestArgs p) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kIngestRowsPerBlock + threadIdx.x / 8;
    const int piece = threadIdx.x & 7;
    if (i >= p.count) return;
    int64_t s = 0, t = 0;
    if (p.mode == KVIP_INGEST_DECODE) {
        const int64_t end = p.query_ends[i];
        const bool valid = end > 0;
        const int64_t g = p.gather_indices[i];
        s = (valid && g >= 0 && g < p.slot_count) ? p.slot_mapping[g] : 0;
        t = valid ? static_cast<int64_t>(p.row_owners[i / p.queries_per_request]) * p.history + end - 1 : i;
        if (valid && (g < 0 || g >= p.slot_count)) s = -1;
    } else if (p.mode == KVIP_INGEST_LIST) {
        s = p.sources[i];
        t = p.target_base + p.targets[i];
    } else {
        const int64_t page = p.block_table[i / p.block_size];
        s = page * p.block_size + i % p.block_size;
        t = p.target_base + i;
    }
    if (s < 0 || s >= p.source_rows || t < 0 || t >= p.target_rows) {
        if (piece == 0) report(p.status, KVIP_STATUS_BAD_TOKEN);
        return;
    }
    const uint4* src = reinterpret_cast<const uint4*>(p.source_keys + s * kIndexDim);
    uint4* dst = reinterpret_cast<uint4*>(p.target_keys + t * kIndexDim);
    dst[piece] = src[piece];
    if (piece == 0) p.target_scales[t] = p.source_scales[s];
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace
}  // namespace kvip

extern "C" uint32_t kvip_hip_pack_queries(const KvipQueryPackArgs* a, void* stream) {
    if (a == nullptr || a->gather_indices == nullptr || a->query_valid == nullptr || a->rows < 1 ||
        a->rows > (1 << 24) || a->tokens < 0 || (a->heads != 32 && a->heads != 64)) {
        return KVIP_ERR_INVALID;
    }
    if (a->positions != nullptr && a->query_ends == nullptr) return KVIP_ERR_INVALID;
    if (a->query_in != nullptr) {
        const void* ptrs[] = {a->query_in, a->weights_in, a->scale_in, a->query_out, a->weights_out, a->scale_out};
        for (const void* ptr : ptrs) {
            if (ptr == nullptr || !kvip::aligned16(ptr)) return KVIP_ERR_INVALID;
        }
    }
    if (a->positions == nullptr && a->query_in == nullptr) return KVIP_OK;
    hipLaunchKernelGGL(kvip::pack_queries_kernel, dim3(a->rows), dim3(kvip::kPackThreads), 0,
                       static_cast<hipStream_t>(stream), *a);
    return static_cast<uint32_t>(hipGetLastError());
}

extern "C" uint32_t kvip_hip_ingest_index(const KvipIngestArgs* a, void* stream) {
    if (a == nullptr || a->source_keys == nullptr || a->source_scales == nullptr || a->target_keys == nullptr ||
        a->target_scales == nullptr || a->count < 0 || a->source_rows < 0 || a->target_rows < 0 ||
        !kvip::aligned16(a->source_keys) || !kvip::aligned16(a->target_keys)) {
        return KVIP_ERR_INVALID;
    }
    switch (a->mode) {
        case KVIP_INGEST_DECODE:
            if (a->query_ends == nullptr || a->gather_indices == nullptr || a->slot_mapping == nullptr ||
                a->row_owners == nullptr || a->queries_per_request < 1 || a->history < 1 || a->slot_count < 0) {
                return KVIP_ERR_INVALID;
            }
            break;
        case KVIP_INGEST_LIST:
            if (a->count > 0 && (a->sources == nullptr || a->targets == nullptr)) return KVIP_ERR_INVALID;
            break;
        case KVIP_INGEST_PREFIX:
            if (a->count > 0 && (a->block_table == nullptr || a->block_size < 1)) return KVIP_ERR_INVALID;
            break;
        default:
            return KVIP_ERR_INVALID;
    }
    if (a->count == 0) return KVIP_OK;
    const int64_t blocks = (a->count + kvip::kIngestRowsPerBlock - 1) / kvip::kIngestRowsPerBlock;
    if (blocks > 0x7FFFFFFF) return KVIP_ERR_INVALID;
    hipLaunchKernelGGL(kvip::ingest_index_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kvip::kIngestThreads), 0,
                       static_cast<hipStream_t>(stream), *a);
    return static_cast<uint32_t>(hipGetLastError());
}
