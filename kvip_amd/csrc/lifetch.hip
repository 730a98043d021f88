// One decode round of the lightning indexer with fetch: scoring -> TopK-2048 ->
// Fetch gather, enqueued back to back on one stream (no allocation, no sync, no
// memset), so the whole round can be captured into a single hipGraph. The default plan is
// three launches: scoring (indexer_ring.hip), TopK with the row's keys in registers
// (topk.hip; rows above 65536 keys take the multi-workgroup split select) and the
// gather (fetch_gather.hip). Measured at config 2 this beats TopK fused with the
// gather (select_fetch.hip, still exported as kvip_hip_select_fetch): the separate gather
// launch is balanced by the hardware dispatcher, while the fused one waits for its
// slowest workgroup.
//
// Replaces kvip_lifetch_streaming_forward (csrc/operators/lightning_indexer_with_fetch/
// include/api.h:7, op_host/launch.cpp:76-83), whose init -> LI -> resolve/update/fetch
// launch sequence it mirrors for the contiguous-destination Fetch.
#include "kvip_device.h"

namespace kvip {
uint32_t validate_indexer(const KvipIndexerArgs* a);
uint32_t validate_topk(const KvipTopkArgs* a);
uint32_t validate_fetch(const KvipFetchArgs* a);
hipError_t launch_indexer(const KvipIndexerArgs& a, hipStream_t stream);
hipError_t launch_topk(const KvipTopkArgs& a, hipStream_t stream);
hipError_t launch_fetch(const KvipFetchArgs& a, hipStream_t stream);
}  // namespace kvip

extern "C" uint32_t kvip_hip_abi_version(void) { return KVIP_HIP_ABI_VERSION; }

namespace {
// Validates the chained arguments and picks the launch plan (KVIP_LIFETCH_PLAN_*), or
// returns KVIP_ERR_INVALID.
uint32_t lifetch_plan(const KvipLIFetchArgs* args) {
    if (args == nullptr) return KVIP_ERR_INVALID;
    const KvipIndexerArgs& li = args->indexer;
    const KvipTopkArgs& tk = args->topk;
    const KvipFetchArgs& fe = args->fetch;
    if (kvip::validate_indexer(&li) != KVIP_OK || kvip::validate_topk(&tk) != KVIP_OK ||
        kvip::validate_fetch(&fe) != KVIP_OK) {
        return KVIP_ERR_INVALID;
    }
    // The three stages must describe the same rows and hand buffers to each other.
    const bool chained = tk.score_keys == li.score_keys && tk.key_stride == li.key_stride &&
                         tk.histogram == li.histogram && tk.seq_lens == li.seq_lens &&
                         tk.query_ends == li.query_ends && tk.batch == li.batch &&
                         tk.rows_per_request == li.rows_per_request && fe.topk == tk.topk &&
                         fe.batch == li.batch && fe.rows_per_request == li.rows_per_request;
    if (!chained) return KVIP_ERR_INVALID;
    return KVIP_LIFETCH_PLAN_THREE;
}
}  // namespace

extern "C" uint32_t kvip_hip_lifetch_plan(const KvipLIFetchArgs* args) { return lifetch_plan(args); }

extern "C" uint32_t kvip_hip_lifetch_forward(const KvipLIFetchArgs* args, void* stream) {
    const uint32_t plan = lifetch_plan(args);
    if (plan == KVIP_ERR_INVALID) return plan;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const KvipIndexerArgs& li = args->indexer;
    const KvipTopkArgs& tk = args->topk;
    const KvipFetchArgs& fe = args->fetch;
    hipError_t e = kvip::launch_indexer(li, s);
    if (e != hipSuccess) return static_cast<uint32_t>(e);
    // Rows that fit the register-resident TopK take it even when the split select's work
    // memory is given.
    KvipTopkArgs t = tk;
    if (t.histogram != nullptr && t.key_stride <= KVIP_TOPK_REGS_MAX_KEYS) t.segments = nullptr;
    e = kvip::launch_topk(t, s);
    if (e != hipSuccess) return static_cast<uint32_t>(e);
    return static_cast<uint32_t>(kvip::launch_fetch(fe, s));
}
