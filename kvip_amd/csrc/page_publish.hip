// Publication of appended KV pages: one launch for every page committed in a step, with no
// upload of earlier pages and no KV payload copy (python/kvip/cache/page_updates.py:27-62,
// _page_updates_kernel.py:8-37). Row k of `rows` is {flat page index, page address, clear}:
//   addresses[index] = address, valid[index] = 1;
//   clear >= 0: token_to_slot[clear .. clear + block_size) = -1 (the recycled page's slots);
//   with fused tables: owner = index / (groups * pages), group = index / pages % groups,
//   page = index % pages; fused table `group` (int64 [owners, history]) gets, for the page's
//   positions below history, address + i * token_bytes of that group.
// One workgroup per row, one thread per position of the page.
#include "kvip_device.h"

namespace kvip {
namespace {

__global__ __launch_bounds__(256) void publish_pages_kernel(const KvipPageArgs p) {
    const int k = blockIdx.x;
    const int64_t index = p.rows[3 * k], address = p.rows[3 * k + 1], clear = p.rows[3 * k + 2];
    const int i = threadIdx.x;
    if (index < 0 || index >= p.entries || clear >= p.map_entries - p.block_size + 1) {
        if (i == 0) report(p.status, KVIP_STATUS_BAD_TOKEN);
        return;
    }
    if (i == 0) {
        p.addresses[index] = address;
        p.valid[index] = 1u;
    }
    if (i < p.block_size && clear >= 0) p.token_to_slot[clear + i] = -1;
    if (p.fused != nullptr && i < p.block_size) {
        const int64_t per_owner = static_cast<int64_t>(p.groups) * p.pages;
        const int64_t owner = index / per_owner;
        const int group = static_cast<int>(index / p.pages % p.groups);
        const int64_t position = (index % p.pages) * p.block_size + i;
        int64_t* table = reinterpret_cast<int64_t*>(p.fused[2 * group]);
        const int64_t token_bytes = p.fused[2 * group + 1];
        if (position < p.history) table[owner * p.history + position] = address + i * token_bytes;
    }
}

}  // namespace
}  // namespace kvip

extern "C" uint32_t kvip_hip_publish_pages(const KvipPageArgs* a, void* stream) {
    if (a == nullptr || a->count < 0) return KVIP_ERR_INVALID;
    if (a->count == 0) return KVIP_OK;
    const bool ok = a->rows && a->addresses && a->valid && a->token_to_slot && a->groups >= 1 && a->pages >= 1 &&
                    a->block_size >= 1 && a->block_size <= 256 && a->entries >= 1 && a->map_entries >= a->block_size &&
                    (a->fused == nullptr || a->history >= 1);
    if (!ok) return KVIP_ERR_INVALID;
    hipLaunchKernelGGL(kvip::publish_pages_kernel, dim3(a->count), dim3(256), 0, static_cast<hipStream_t>(stream), *a);
    return static_cast<uint32_t>(hipGetLastError());
}
