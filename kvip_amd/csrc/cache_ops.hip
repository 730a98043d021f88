// Cache-state operators on gfx950: ABC ring maps and the resident-slot LRU.
//
// update_abc (reference: python/kvip/cache/abc.py:5-33, CPU golden :23-33). For every
// descriptor (layer, owner, begin, end) in group-major order, token_to_slot[layer, owner,
// t] = history + t % tail for t in [begin, end), and the ring slot_to_token[layer, owner,
// history : history+tail] is reset to -1 and refilled with the range's tokens, a later
// token overwriting an earlier one on the same ring slot. One workgroup per descriptor:
// the token_to_slot values depend only on t, so descriptors that overlap write identical
// values; the ring of a (layer, owner) is written only by the last descriptor naming it,
// with the closed form "largest t in [begin, end) with t % tail == s" per ring slot s.
//
// Slot LRU (reference: python/kvip/cache/lru.py:14-118, _lru_kernel.py:33-199). The
// doubly linked list of the reference is held as its order array: order[i] is the slot at
// LRU position i (0 = oldest). commit moves the unique committed slots (< active) to the
// end in ascending slot-id order: a stable partition of the order, done in place by one
// workgroup with LDS membership bits and block scans. The victims are
// order[0 .. min(2048, active)), with their bitmap.
#include "kvip_device.h"

namespace kvip {
namespace {

constexpr int kAbcThreads = 256;
constexpr int kLruThreads = 1024;
constexpr int kLruMaxSlots = (1 << 17) + 20 * 128;   // resident capacity bound (reference MAX_CACHE_TOKENS)
constexpr int kLruBitmapWords = (kLruMaxSlots + 31) / 32;

__global__ __launch_bounds__(kAbcThreads) void update_abc_kernel(const KvipAbcArgs p) {
    const int r = blockIdx.x;  // row within the group, < requests
    const int grp = blockIdx.y;
    const int32_t* d = p.descriptors + (static_cast<size_t>(grp) * p.rows + r) * 4;
    const int layer = d[0], owner = d[1], begin = d[2], end = d[3];
    auto in_range = [&](int l, int o) {
        return l >= 0 && l < p.layers && o >= 0 && o < p.pool;
    };
    const bool ok = in_range(layer, owner) && begin >= 0 && (end <= begin || end <= p.t2s_tokens);
    if (!ok) {
        if (threadIdx.x == 0) report(p.status, KVIP_STATUS_BAD_TOKEN);
        return;
    }
    const size_t base = (static_cast<size_t>(layer) * p.pool + owner);
    int32_t* t2s = p.token_to_slot + base * p.t2s_tokens;
    for (int t = begin + static_cast<int>(threadIdx.x); t < end; t += kAbcThreads) t2s[t] = p.history + t % p.tail;

    // Is a later (group-major) descriptor naming the same (layer, owner)? Then its ring wins.
    const int total = p.groups * p.requests;
    const int self = grp * p.requests + r;
    int later = 0;
    for (int k = self + 1 + static_cast<int>(threadIdx.x); k < total; k += kAbcThreads) {
        const int32_t* e = p.descriptors + (static_cast<size_t>(k / p.requests) * p.rows + k % p.requests) * 4;
        const bool valid = in_range(e[0], e[1]) && e[2] >= 0 && (e[3] <= e[2] || e[3] <= p.t2s_tokens);
        later |= (valid && e[0] == layer && e[1] == owner) ? 1 : 0;
    }
    if (__syncthreads_or(later)) return;

    int32_t* ring = p.slot_to_token + base * p.s2t_tokens + p.history;
    for (int s = threadIdx.x; s < p.tail; s += kAbcThreads) {
        int token = -1;
        if (end > begin) {
            const int hi = end - 1;
            const int back = ((hi - s) % p.tail + p.tail) % p.tail;
            const int t = hi - back;  // largest t <= hi with t % tail == s
            token = t >= begin ? t : -1;
        }
        ring[s] = token;
    }
}

// Chain c of a set of `chains` LRUs laid out back to back: order/scratch rows of
// `capacity`, slots rows of 2048, bitmap rows of `bitmap_words` (a single LRU is chain 0).
KVIP_DEVICE KvipLruArgs chain_of(const KvipLruArgs& p, int c) {
    KvipLruArgs q = p;
    q.order += static_cast<size_t>(c) * p.capacity;
    q.scratch += static_cast<size_t>(c) * p.capacity;
    q.slots += static_cast<size_t>(c) * kTopK;
    q.bitmap += static_cast<size_t>(c) * p.bitmap_words;
    return q;
}

// order[0, committed) = 0, 1, ..., committed-1 (a cold LRU in ascending slot order) and
// the victim list/bitmap of it; chain blockIdx.y.
__global__ __launch_bounds__(kLruThreads) void lru_reset_kernel(const KvipLruArgs args, int committed) {
    const KvipLruArgs p = chain_of(args, blockIdx.y);
    for (int i = blockIdx.x * kLruThreads + threadIdx.x; i < p.capacity; i += gridDim.x * kLruThreads) {
        p.order[i] = i < committed ? i : -1;
    }
}

// Appends slots [first, committed) at the end of the order (growth keeps LRU order).
__global__ __launch_bounds__(kLruThreads) void lru_extend_kernel(const KvipLruArgs p, int first, int committed) {
    for (int i = first + blockIdx.x * kLruThreads + threadIdx.x; i < committed; i += gridDim.x * kLruThreads) {
        p.order[i] = i;
    }
}

// One workgroup per chain (blockIdx.x): stable partition of order[0, active) into (not
// committed, committed in ascending slot order), in place, then the victims of the new
// order. Chain c commits dest[c * dest_stride, + count). The order moves through LDS in
// tiles of 16384 entries: a coalesced copy in, a block scan over each thread's 16
// consecutive entries, the kept entries compacted in LDS, a coalesced copy out (LDS index
// i sits at i + i/16, so a thread's 16 consecutive entries and 64 consecutive indices
// both spread over the banks). A kept
// entry only moves to a lower position and a tile is written after it was read, so the
// partition overwrites nothing still unread; the committed slots follow the last tile the
// same way, 16384 at a time. Victims (the first min(2048, active) positions) and their
// bitmap are taken from the values as they are written.
constexpr int kLruPer = 16;                       // entries per thread and tile
constexpr int kLruTile = kLruThreads * kLruPer;   // 16384
KVIP_DEVICE uint32_t lru_lds(uint32_t i) { return i + (i >> 4); }
__global__ __launch_bounds__(kLruThreads) void lru_commit_kernel(const KvipLruArgs args, const int32_t* dest,
                                                                 int64_t dest_stride, int count, int active,
                                                                 int commit) {
    __shared__ uint32_t s_member[kLruBitmapWords];
    __shared__ uint32_t s_victim[kLruBitmapWords];
    __shared__ int32_t s_tile[kLruTile + kLruTile / 16];
    __shared__ uint32_t s_wave[kLruThreads / 64];
    const KvipLruArgs p = chain_of(args, blockIdx.x);
    if (commit) dest += static_cast<size_t>(blockIdx.x) * dest_stride;
    const int tid = threadIdx.x;
    const int words = (active + 31) / 32;
    const int victims = min(kTopK, active);

    // The first tile's entries (coalesced), in flight together with the committed slots.
    int first[kLruPer];
#pragma unroll
    for (int m = 0; m < kLruPer; ++m) {
        const int k = m * kLruThreads + tid;
        first[m] = k < active ? p.order[k] : -1;
    }
    for (int i = tid; i < p.bitmap_words; i += kLruThreads) {
        s_member[i] = 0u;
        s_victim[i] = 0u;
    }
    __syncthreads();
    if (commit) {
        for (int i = tid; i < count; i += kLruThreads) {
            const int s = dest[i];
            if (s >= 0 && s < active) atomicOr(&s_member[s >> 5], 1u << (s & 31));
        }
    }

    // Writes s_tile[0, n) to order[base, base + n) and records the victims among them.
    auto flush = [&](uint32_t base, int n) {
        for (int k = tid; k < n; k += kLruThreads) {
            const int slot = s_tile[lru_lds(k)];
            const uint32_t pos = base + k;
            p.order[pos] = slot;
            if (pos < static_cast<uint32_t>(victims)) {
                p.slots[pos] = slot;
                atomicOr(&s_victim[slot >> 5], 1u << (slot & 31));
            }
        }
    };

    // Kept slots, in order.
    uint32_t kept_base = 0;
    for (int tile = 0; tile < active; tile += kLruTile) {
        const int n = min(active - tile, kLruTile);
        __syncthreads();  // membership bits complete; the previous tile's flush read s_tile
        if (tile == 0) {
#pragma unroll
            for (int m = 0; m < kLruPer; ++m) s_tile[lru_lds(m * kLruThreads + tid)] = first[m];
        } else {
            for (int k = tid; k < n; k += kLruThreads) s_tile[lru_lds(k)] = p.order[tile + k];
        }
        __syncthreads();
        int v[kLruPer];
        uint32_t keep = 0;
#pragma unroll
        for (int j = 0; j < kLruPer; ++j) {
            const int i = tid * kLruPer + j;
            v[j] = i < n ? s_tile[lru_lds(i)] : -1;
            const bool k = v[j] >= 0 && !((s_member[v[j] >> 5] >> (v[j] & 31)) & 1u);
            keep |= (k ? 1u : 0u) << j;
        }
        uint32_t tile_total;
        uint32_t pos = block_exclusive_scan(__popc(keep), s_wave, &tile_total);  // barriers: s_tile read
#pragma unroll
        for (int j = 0; j < kLruPer; ++j) {
            if ((keep >> j) & 1u) s_tile[lru_lds(pos++)] = v[j];
        }
        __syncthreads();
        flush(kept_base, static_cast<int>(tile_total));
        kept_base += tile_total;
    }
    // Committed slots in ascending id order, 512 membership words (<= 16384 slots) at a time.
    uint32_t moved_base = kept_base;
    for (int w0 = 0; w0 < words; w0 += kLruTile / 32) {
        const int w = w0 + tid;
        const uint32_t bits = (tid < kLruTile / 32 && w < words) ? s_member[w] : 0u;
        uint32_t total;
        uint32_t pos = block_exclusive_scan(__popc(bits), s_wave, &total);  // barriers: last flush done
        uint32_t rest = bits;
        while (rest) {
            const int b = __ffs(rest) - 1;
            s_tile[lru_lds(pos++)] = w * 32 + b;
            rest &= rest - 1;
        }
        __syncthreads();
        flush(moved_base, static_cast<int>(total));
        moved_base += total;
    }
    for (int i = victims + tid; i < kTopK; i += kLruThreads) p.slots[i] = -1;
    __syncthreads();
    for (int i = tid; i < p.bitmap_words; i += kLruThreads) p.bitmap[i] = static_cast<int32_t>(s_victim[i]);
}

}  // namespace
}  // namespace kvip

extern "C" uint32_t kvip_hip_update_abc(const KvipAbcArgs* a, void* stream) {
    if (a == nullptr || a->token_to_slot == nullptr || a->slot_to_token == nullptr || a->descriptors == nullptr ||
        a->groups < 0 || a->requests < 0 || a->rows < a->requests || a->layers < 1 || a->pool < 1 ||
        a->t2s_tokens < 1 || a->tail < 1 || a->history < 0 ||
        static_cast<int64_t>(a->history) + a->tail > a->s2t_tokens || a->groups > 65535) {
        return KVIP_ERR_INVALID;
    }
    if (a->groups == 0 || a->requests == 0) return KVIP_OK;
    hipLaunchKernelGGL(kvip::update_abc_kernel, dim3(a->requests, a->groups), dim3(kvip::kAbcThreads), 0,
                       static_cast<hipStream_t>(stream), *a);
    return static_cast<uint32_t>(hipGetLastError());
}

static bool lru_ok(const KvipLruArgs* a) {
    return a != nullptr && a->order != nullptr && a->scratch != nullptr && a->slots != nullptr &&
           a->bitmap != nullptr && a->capacity >= 1 && a->capacity <= kvip::kLruMaxSlots &&
           a->bitmap_words >= (a->capacity + 31) / 32 && a->bitmap_words <= kvip::kLruBitmapWords;
}

static uint32_t lru_reset_chains(const KvipLruArgs* a, int32_t chains, int32_t committed, void* stream) {
    if (!lru_ok(a) || chains < 1 || chains > 65535 || committed < 0 || committed > a->capacity) {
        return KVIP_ERR_INVALID;
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const int grid = (a->capacity + kvip::kLruThreads - 1) / kvip::kLruThreads;
    hipLaunchKernelGGL(kvip::lru_reset_kernel, dim3(grid, chains), dim3(kvip::kLruThreads), 0, s, *a, committed);
    hipLaunchKernelGGL(kvip::lru_commit_kernel, dim3(chains), dim3(kvip::kLruThreads), 0, s, *a, nullptr, int64_t{0},
                       0, committed, 0);
    return static_cast<uint32_t>(hipGetLastError());
}

static uint32_t lru_commit_chains(const KvipLruArgs* a, int32_t chains, const int32_t* destinations,
                                  int64_t dest_stride, int32_t count, int32_t active, void* stream) {
    if (!lru_ok(a) || chains < 1 || chains > 65535 || count < 0 || (count > 0 && destinations == nullptr) ||
        (chains > 1 && dest_stride < count) || active < 0 || active > a->capacity) {
        return KVIP_ERR_INVALID;
    }
    hipLaunchKernelGGL(kvip::lru_commit_kernel, dim3(chains), dim3(kvip::kLruThreads), 0,
                       static_cast<hipStream_t>(stream), *a, destinations, dest_stride, count, active, 1);
    return static_cast<uint32_t>(hipGetLastError());
}

extern "C" uint32_t kvip_hip_lru_reset(const KvipLruArgs* a, int32_t committed, void* stream) {
    return lru_reset_chains(a, 1, committed, stream);
}

extern "C" uint32_t kvip_hip_lru_extend(const KvipLruArgs* a, int32_t active, int32_t committed, void* stream) {
    if (!lru_ok(a) || active < 0 || committed < active || committed > a->capacity) return KVIP_ERR_INVALID;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const int grid = max(1, (committed - active + kvip::kLruThreads - 1) / kvip::kLruThreads);
    hipLaunchKernelGGL(kvip::lru_extend_kernel, dim3(grid), dim3(kvip::kLruThreads), 0, s, *a, active, committed);
    hipLaunchKernelGGL(kvip::lru_commit_kernel, dim3(1), dim3(kvip::kLruThreads), 0, s, *a, nullptr, int64_t{0}, 0,
                       committed, 0);
    return static_cast<uint32_t>(hipGetLastError());
}

extern "C" uint32_t kvip_hip_lru_commit(const KvipLruArgs* a, const int32_t* destinations, int32_t count,
                                        int32_t active, void* stream) {
    return lru_commit_chains(a, 1, destinations, 0, count, active, stream);
}

extern "C" uint32_t kvip_hip_lru_reset_chains(const KvipLruArgs* a, int32_t chains, int32_t committed, void* stream) {
    return lru_reset_chains(a, chains, committed, stream);
}

extern "C" uint32_t kvip_hip_lru_commit_chains(const KvipLruArgs* a, int32_t chains, const int32_t* destinations,
                                               int64_t dest_stride, int32_t count, int32_t active, void* stream) {
    return lru_commit_chains(a, chains, destinations, dest_stride, count, active, stream);
}
