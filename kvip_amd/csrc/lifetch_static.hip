// Allocation-free decode round: kvip_hip_lifetch_forward with its scratch (the per-row
// score keys and high-byte histograms that scoring hands to TopK) taken from a file-scope
// device array instead of caller buffers, for callers that cannot allocate device memory.
//
// The array `scratch` (KVIP_LIFETCH_STATIC_SCRATCH_BYTES) exists once per GPU, for the life
// of the process. Its device address is fetched with hipGetSymbolAddress the first time
// the entry point runs with a device current and kept per device; host code only ever
// passes that address (the array's name is a host-side stand-in). Layout of one call:
// the histograms [rows, 256] uint32 at offset 0, then the score keys [rows, key_stride]
// uint16 at the next 256-byte boundary. Each call first clears the histogram rows it uses
// with a fill kernel (no memset node, so the call may be captured), so nothing depends on
// what an earlier call left. Every call on one GPU shares the array: calls that overlap
// on one GPU (other streams, concurrent graphs) race.
#include <mutex>

#include "kvip_device.h"

static __device__ __align__(256) uint8_t scratch[KVIP_LIFETCH_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
uint8_t* g_scratch[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up once per device).
hipError_t scratch_address(uint8_t** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch[dev] = static_cast<uint8_t*>(p);
    }
    *out = g_scratch[dev];
    return hipSuccess;
}

__global__ __launch_bounds__(256) void clear_words_kernel(uint32_t* words, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        words[i] = 0u;
    }
}

}  // namespace

extern "C" uint32_t kvip_hip_lifetch_forward_static(const KvipLIFetchArgs* args, void* stream) {
    if (args == nullptr) return KVIP_ERR_INVALID;
    const KvipIndexerArgs& li = args->indexer;
    const KvipTopkArgs& tk = args->topk;
    // The library supplies the scratch; the split select (which needs more work memory) is
    // not offered here.
    if (li.score_keys != nullptr || li.histogram != nullptr || tk.score_keys != nullptr || tk.histogram != nullptr ||
        tk.segments != nullptr) {
        return KVIP_ERR_INVALID;
    }
    if (li.batch < 1 || li.rows_per_request < 1 || li.key_stride < 8) return KVIP_ERR_INVALID;
    const uint64_t rows = static_cast<uint64_t>(li.batch) * static_cast<uint64_t>(li.rows_per_request);
    const uint64_t hist_bytes = (rows * 256u * 4u + 255u) / 256u * 256u;
    const uint64_t key_bytes = rows * static_cast<uint64_t>(li.key_stride) * 2u;
    if (hist_bytes + key_bytes > KVIP_LIFETCH_STATIC_SCRATCH_BYTES) return KVIP_ERR_INVALID;
    uint8_t* base = nullptr;
    hipError_t e = scratch_address(&base);
    if (e != hipSuccess) return static_cast<uint32_t>(e);
    KvipLIFetchArgs a = *args;
    uint32_t* hist = reinterpret_cast<uint32_t*>(base);
    uint16_t* keys = reinterpret_cast<uint16_t*>(base + hist_bytes);
    a.indexer.histogram = hist;
    a.indexer.score_keys = keys;
    a.topk.histogram = hist;
    a.topk.score_keys = keys;
    if (kvip_hip_lifetch_plan(&a) != KVIP_LIFETCH_PLAN_THREE) return KVIP_ERR_INVALID;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t words = static_cast<int64_t>(rows) * 256;
    const int grid = static_cast<int>(std::min<int64_t>((words + 255) / 256, 1024));
    hipLaunchKernelGGL(clear_words_kernel, dim3(grid), dim3(256), 0, s, hist, words);
    e = hipGetLastError();
    if (e != hipSuccess) return static_cast<uint32_t>(e);
    return kvip_hip_lifetch_forward(&a, stream);
}
