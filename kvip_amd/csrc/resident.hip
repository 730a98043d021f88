// Resident-cache round of the streaming LIFetch path on gfx950: hot/cold classification
// of the final TopK positions, per-query miss resolution with LRU victim slots, Fetch of
// the missed KV rows from mapped host memory into the hot cache, the Index-row
// permutation and the residency publication. Four launches per round:
//   resident_init_kernel     one workgroup per request: reserved_hot from the LRU
//                            candidates, change records and counts cleared;
//   resident_resolve_kernel  one 1024-thread workgroup per request, everything staged in
//                            LDS (TopK rows, locations, protection bitmap, rank -> slot);
//                            first occurrences are found with atomicMin on a per-request
//                            position table kept in the workspace (reset at the end);
//   resident_fetch_kernel    one wave per 32 misses, 16-byte nontemporal copies;
//   resident_update_kernel   one 1024-thread workgroup per request: each 512-change chunk
//                            is planned in LDS (membership hash sets, closure by scan),
//                            snapshotted into registers, then written; the position <->
//                            row maps live in the workspace and are restored to identity.
// Every per-request loop is bounded by the request's sizes and every workgroup reaches
// the end of its kernel (errors skip work, never wait).
//
// Reference (paths relative to the KVIP tree, op_kernel/ of
// lightning_indexer_with_fetch unless noted): lifecycle.cpp:32-81 (InitializeRound),
// staged_topk_classify.h:9-47 and resolver_staged_dma2.h:9-22 (classification),
// resolver_staged_dma2.h:98-237 (StagedQuery), streaming.cpp:16-22, :66-90 (events,
// outputs), :205-274 and shadow_exchange_parallel.h:28-85 (Consumer, ApplyBatch,
// CommitMetadata), common/lifetch/cache_metadata.h:54-73 (residency publication).
#include "kvip_device.h"

namespace kvip {
uint32_t validate_indexer(const KvipIndexerArgs* a);
uint32_t validate_topk(const KvipTopkArgs* a);
hipError_t launch_indexer(const KvipIndexerArgs& a, hipStream_t stream);
bool ring_eligible(const KvipIndexerArgs& a);
hipError_t launch_indexer_ring(const KvipIndexerArgs& a, hipStream_t stream, int tile_lo, int tile_hi);
hipError_t launch_topk(const KvipTopkArgs& a, hipStream_t stream);

namespace {

constexpr int kRsThreads = 1024;
constexpr int kMaxQ = KVIP_RESIDENT_MAX_QUERIES;
constexpr int kLru = KVIP_RESIDENT_LRU_SLOTS;
constexpr int kMaxWords = KVIP_RESIDENT_MAX_RESIDENT / 32;
constexpr int kChanges = KVIP_RESIDENT_CHANGES;
constexpr int kChunk = 512;
constexpr int kSetSize = 2048;               // membership hash set buckets (power of two)
constexpr uint32_t kNoFirst = 0xFFFFFFFFu;
constexpr uint32_t kEmpty = 0xFFFFFFFFu;
static_assert(kTopK == 2 * kRsThreads, "two TopK entries per thread");
static_assert(kLru == 2 * kRsThreads, "two candidates per thread");

struct Workspace {
    uint32_t* first;   // [batch, history] lowest index of each position in the current query
    int32_t* rank;     // [batch, history] miss rank of each position, -1 = none
    int32_t* row_at;   // [batch, history] row now at each position (identity between rounds)
    int32_t* pos_of;   // [batch, history] position of each row (identity between rounds)
    int32_t* map;      // [batch, history] prefetch ordinal of each position, -1 = none
};

KVIP_DEVICE Workspace workspace_of(const KvipResidentArgs& p) {
    const size_t n = static_cast<size_t>(p.batch) * p.history;
    uint32_t* base = static_cast<uint32_t*>(p.workspace);
    return {base, reinterpret_cast<int32_t*>(base + n), reinterpret_cast<int32_t*>(base + 2 * n),
            reinterpret_cast<int32_t*>(base + 3 * n), reinterpret_cast<int32_t*>(base + 4 * n)};
}

// ABC tail of request b: positions [begin, end), the first T = hot_stride - resident of them
// (p < mapped) in ring slot resident + p % T. ok = false for bounds outside the history.
struct Tail {
    int begin, end, mapped, ring;
    bool ok;
};
KVIP_DEVICE Tail tail_of(const KvipResidentArgs& p, int b) {
    Tail t{0, 0, 0, p.hot_stride - p.resident, true};
    if (p.tail_bounds != nullptr) {
        t.begin = p.tail_bounds[2 * b];
        t.end = p.tail_bounds[2 * b + 1];
        t.ok = 0 <= t.begin && t.begin <= t.end && t.end <= p.history;
        if (!t.ok) t.begin = t.end = 0;
        t.mapped = min(t.end, t.begin + t.ring);
    }
    return t;
}

template <typename T>
KVIP_DEVICE T load_agent(const T* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
KVIP_DEVICE void store_agent(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

KVIP_DEVICE bool owner_ok(const KvipResidentArgs& p, int o) { return o >= 0 && o < p.owners; }

// Workspace preparation: first = none, rank = none, maps = identity, no prefetch ordinal.
__global__ void resident_prepare_kernel(const KvipResidentArgs p) {
    const Workspace ws = workspace_of(p);
    const size_t n = static_cast<size_t>(p.batch) * p.history;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const int pos = static_cast<int>(i % static_cast<size_t>(p.history));
        ws.first[i] = kNoFirst;
        ws.rank[i] = -1;
        ws.row_at[i] = pos;
        ws.pos_of[i] = pos;
        ws.map[i] = -1;
    }
}

// Round initialisation of request b. A hot slot named by two candidates fails the request
// (KVIP_RESIDENT_ERR_CANDIDATE): both ordinals would otherwise see it free and receive it.
// With `table` set it also writes request b's row of the scoring block table (entry j =
// row_owners[b] * blocks_per_owner + j for j < blocks_per_owner, else 0), so that a resident
// forward initialises its round and its owner table in one launch ahead of the scoring.
__global__ __launch_bounds__(kRsThreads) void resident_init_kernel(const KvipResidentArgs p, int32_t* table,
                                                                   int max_blocks, int blocks_per_owner) {
    __shared__ uint32_t s_seen[kMaxWords];
    __shared__ uint32_t s_dup;
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    if (table != nullptr) {
        const int o = p.row_owners[b];
        for (int j = tid; j < max_blocks; j += kRsThreads) {
            table[static_cast<size_t>(b) * max_blocks + j] = j < blocks_per_owner ? o * blocks_per_owner + j : 0;
        }
    }
    const int words = (p.resident + 31) / 32;
    int32_t* reserved = p.reserved_hot + static_cast<size_t>(b) * p.resident;
    for (int s = tid; s < p.resident; s += kRsThreads) reserved[s] = -1;
    for (int w = tid; w < words; w += kRsThreads) s_seen[w] = 0u;
    if (tid == 0) s_dup = 0u;
    const int nchg = kLru + p.rows_per_request * kTopK;
    const int32_t* lru = p.lru_slots + static_cast<size_t>(b) * kLru;
    for (int i = tid; i < nchg; i += kRsThreads) {
        p.changes[static_cast<size_t>(b) * nchg + i] = -1;
        p.change_slots[static_cast<size_t>(b) * nchg + i] = i < kLru ? lru[i] : -1;
    }
    if (tid < 5) p.miss_counts[b * 5 + tid] = 0;
    if (tid == 0 && p.prefetch_counts != nullptr) p.prefetch_counts[b] = 0;
    __syncthreads();
    for (int i = tid; i < kLru; i += kRsThreads) {
        const int s = lru[i];
        if (s >= 0 && s < p.resident) {
            const uint32_t bit = 1u << (s & 31);
            if ((atomicOr(&s_seen[s >> 5], bit) & bit) != 0u) s_dup = 1u;
            reserved[s] = i;
        }
    }
    __syncthreads();
    if (tid == 0) p.status[b] = s_dup != 0u ? static_cast<int32_t>(KVIP_RESIDENT_ERR_CANDIDATE) : 0;
}

__global__ __launch_bounds__(kRsThreads) void resident_resolve_kernel(const KvipResidentArgs p) {
    __shared__ int32_t s_sel[kMaxQ * kTopK];
    __shared__ int32_t s_loc[kMaxQ * kTopK];
    __shared__ int32_t s_slots[kMaxQ * kTopK];   // slot of each miss rank
    __shared__ uint32_t s_bitmap[kMaxWords];     // protected or allocated hot slots
    __shared__ uint32_t s_wave[kRsThreads / 64];
    __shared__ uint32_t s_err;
    __shared__ int s_dest[kMaxQ];  // token-order output row of each query row

    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int Q = p.rows_per_request;
    const int R = p.resident;
    const int H = p.history;
    const int words = (R + 31) / 32;
    const int o = p.row_owners[b];
    const Workspace ws = workspace_of(p);
    uint32_t* first = ws.first + static_cast<size_t>(b) * H;
    int32_t* rank_of = ws.rank + static_cast<size_t>(b) * H;
    const int32_t* reserved = p.reserved_hot + static_cast<size_t>(b) * R;
    const int32_t* lru = p.lru_slots + static_cast<size_t>(b) * kLru;
    const int nchg = kLru + Q * kTopK;

    // ABC tail [tail.begin, tail.end); its first T positions sit in ring slot R + p % T.
    const Tail tail = tail_of(p, b);
    const bool prefetched = p.prefetch_counts != nullptr;
    const int used = prefetched ? p.prefetch_counts[b] : p.used;
    const int32_t* pmap = ws.map + static_cast<size_t>(b) * H;

    for (int i = tid; i < words; i += kRsThreads) s_bitmap[i] = 0u;
    // Errors found by the round initialisation (duplicate candidates) carry over.
    if (tid == 0) {
        s_err = static_cast<uint32_t>(p.status[b]) |
                (owner_ok(p, o) && tail.ok ? 0u : static_cast<uint32_t>(KVIP_RESIDENT_ERR_TOKEN));
    }
    if (tid < kMaxQ) s_dest[tid] = -1;
    __syncthreads();
    const bool good_owner = owner_ok(p, o);
    const int32_t* hot_valid = p.hot_valid + static_cast<size_t>(good_owner ? o : 0) * R;

    // Classification of every query row: hot hits keep their position as slot, mapped
    // tail positions take their ring slot (>= R: neither protected nor fetched), prefetched
    // positions their candidate slot (protected).
    for (int e = tid; e < Q * kTopK; e += kRsThreads) {
        const int t = p.topk[static_cast<size_t>(b) * Q * kTopK + e];
        s_sel[e] = t;
        int loc = -1;
        if (t >= H) {
            atomicOr(&s_err, KVIP_RESIDENT_ERR_TOKEN);
        } else if (good_owner && t >= 0) {
            const bool in_tail = t >= tail.begin && t < tail.end;
            if (in_tail && t < tail.mapped) {
                loc = R + t % tail.ring;
            } else if (!in_tail && t < R && hot_valid[t] != 0 && reserved[t] < 0) {
                loc = t;
                atomicOr(&s_bitmap[t >> 5], 1u << (t & 31));
            } else if (prefetched) {
                const int k = pmap[t];
                const int s = k >= 0 && k < used ? lru[k] : -1;
                if (s >= 0 && s < R) {
                    loc = s;
                    atomicOr(&s_bitmap[s >> 5], 1u << (s & 31));
                }
            }
        }
        s_loc[e] = loc;
    }
    __syncthreads();

    int old = 0;  // misses ranked by earlier query rows (uniform)
    for (int q = 0; q < Q; ++q) {
        if (s_err != 0u) break;  // uniform: read after a barrier
        const int base = q * kTopK;
        int tok[2];
        bool shortcut[2], unresolved[2], fresh[2];
        // (a) first occurrence of every unresolved position of this row.
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = 2 * tid + k;
            const int t = s_sel[base + i];
            tok[k] = t;
            shortcut[k] = q >= 2 && t == s_sel[base - 2 * kTopK + i];
            unresolved[k] = !shortcut[k] && t >= 0 && t < H && s_loc[base + i] < 0 && load_agent(&rank_of[t]) < 0;
            if (unresolved[k]) atomicMin(&first[t], static_cast<uint32_t>(i));
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        // (b) new misses in index order -> ranks.
        uint32_t nnew = 0;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            fresh[k] = unresolved[k] && load_agent(&first[tok[k]]) == static_cast<uint32_t>(2 * tid + k);
            nnew += fresh[k] ? 1u : 0u;
        }
        uint32_t need_u;
        uint32_t r = static_cast<uint32_t>(old) + block_exclusive_scan(nnew, s_wave, &need_u);
        const int need = static_cast<int>(need_u);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            if (fresh[k]) store_agent(&rank_of[tok[k]], static_cast<int32_t>(r++));
        }
        // (c) slots: free candidates in ordinal order, pass 0 = ordinals >= used.
        int allocated = 0;
        if (need > 0) {
            for (int pass = 0; pass < 2 && allocated < need; ++pass) {
                bool ok[2];
                int cand[2];
                uint32_t avail = 0;
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int ord = 2 * tid + k;
                    const int s = lru[ord];
                    cand[k] = s;
                    ok[k] = false;
                    if ((ord >= used) == (pass == 0)) {
                        if (s < 0 || s >= R) {
                            atomicOr(&s_err, KVIP_RESIDENT_ERR_CANDIDATE);
                        } else {
                            ok[k] = ((s_bitmap[s >> 5] >> (s & 31)) & 1u) == 0u;
                        }
                    }
                    avail += ok[k] ? 1u : 0u;
                }
                uint32_t n_avail;
                uint32_t rank = block_exclusive_scan(avail, s_wave, &n_avail);
                const int take = min(static_cast<int>(n_avail), need - allocated);
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    if (ok[k]) {
                        if (rank < static_cast<uint32_t>(take)) s_slots[old + allocated + rank] = cand[k];
                        ++rank;
                    }
                }
                __syncthreads();
                for (int j = tid; j < take; j += kRsThreads) {
                    const int s = s_slots[old + allocated + j];
                    atomicOr(&s_bitmap[s >> 5], 1u << (s & 31));
                }
                allocated += take;
                __syncthreads();
            }
            if (allocated < need && s_err == 0u) {
                // Fallback: every known slot of every row is protected, then the free hot
                // slots in ascending order.
                for (int e = tid; e < Q * kTopK; e += kRsThreads) {
                    const int s = s_loc[e];
                    if (s >= 0 && s < R) atomicOr(&s_bitmap[s >> 5], 1u << (s & 31));
                }
                __syncthreads();
                const int per = (words + kRsThreads - 1) / kRsThreads;
                const int w0 = min(tid * per, words);
                const int w1 = min(w0 + per, words);
                uint32_t free_bits = 0;
                for (int w = w0; w < w1; ++w) {
                    const int bits = min(32, R - 32 * w);
                    const uint32_t live = bits == 32 ? 0xFFFFFFFFu : ((1u << bits) - 1u);
                    free_bits += __popc(~s_bitmap[w] & live);
                }
                uint32_t n_free;
                uint32_t rank = block_exclusive_scan(free_bits, s_wave, &n_free);
                const int want = need - allocated;
                if (n_free < static_cast<uint32_t>(want)) {
                    if (tid == 0) atomicOr(&s_err, KVIP_RESIDENT_ERR_CANDIDATE);
                } else {
                    for (int w = w0; w < w1 && rank < static_cast<uint32_t>(want); ++w) {
                        const int bits = min(32, R - 32 * w);
                        const uint32_t live = bits == 32 ? 0xFFFFFFFFu : ((1u << bits) - 1u);
                        uint32_t m = ~s_bitmap[w] & live;
                        while (m != 0u && rank < static_cast<uint32_t>(want)) {
                            const int bit = __ffs(m) - 1;
                            s_slots[old + allocated + rank] = 32 * w + bit;
                            ++rank;
                            m &= m - 1u;
                        }
                    }
                }
                __syncthreads();
                if (s_err == 0u) {
                    for (int j = tid; j < want; j += kRsThreads) {
                        const int s = s_slots[old + allocated + j];
                        atomicOr(&s_bitmap[s >> 5], 1u << (s & 31));
                    }
                    allocated = need;
                }
                __syncthreads();
            }
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (s_err != 0u) break;
        // (d) locations of the row, change records and Fetch descriptors of its misses.
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = 2 * tid + k;
            const int t = tok[k];
            if (shortcut[k]) {
                s_loc[base + i] = s_loc[base - 2 * kTopK + i];
            } else if (t >= 0 && t < H && s_loc[base + i] < 0) {
                s_loc[base + i] = s_slots[load_agent(&rank_of[t])];
            }
            if (fresh[k]) {
                const int rk = load_agent(&rank_of[t]);
                const int s = s_slots[rk];
                const int ord = reserved[s];
                const int rec = ord >= 0 ? ord : kLru + rk;
                p.change_slots[static_cast<size_t>(b) * nchg + rec] = s;
                p.changes[static_cast<size_t>(b) * nchg + rec] = t;
                const size_t d = static_cast<size_t>(b) * Q * kTopK + rk;
                const int64_t off = p.addresses[static_cast<size_t>(o) * H + t];
                // Every source is checked here, before anything is fetched.
                if (off < 0 || off > p.host_pool_bytes - p.row_bytes || (off & 15) != 0) {
                    atomicOr(&s_err, KVIP_RESIDENT_ERR_SOURCE);
                }
                p.fetch_slots[d] = s;
                p.fetch_positions[d] = t;
                p.fetch_sources[d] = off;
            }
        }
        if (tid == 0) p.miss_counts[b * 5 + q] = need;
        old += need;
        __syncthreads();
    }

    // Outputs of every row (-1 throughout for a failed request) and the total. In token
    // order, output row s_dest[q] holds query row q (-1: no output row names it) and this
    // request's four output rows that hold no query are filled with -1.
    const bool failed = s_err != 0u;
    const bool tnd = p.unpack_indices != nullptr;
    if (tnd) {
        const int rows = p.batch * kMaxQ;
        for (int r = tid; r < rows; r += kRsThreads) {
            const bool active = p.output_valid[r] != 0;
            const int64_t src = active ? p.unpack_indices[r] : -1;
            if (active && src >= static_cast<int64_t>(b) * kMaxQ && src < static_cast<int64_t>(b + 1) * kMaxQ) {
                s_dest[src - static_cast<int64_t>(b) * kMaxQ] = r;
            }
        }
        for (int e = tid; e < kMaxQ * kTopK; e += kRsThreads) {
            const int r = b * kMaxQ + e / kTopK;
            if (p.output_valid[r] == 0) {
                const size_t at = static_cast<size_t>(r) * kTopK + e % kTopK;
                p.slot_output[at] = -1;
                p.logical_output[at] = -1;
            }
        }
        __syncthreads();
    }
    for (int e = tid; e < Q * kTopK; e += kRsThreads) {
        const int q = e / kTopK;
        const int dest = tnd ? s_dest[q] : b * Q + q;
        if (dest < 0) continue;
        const size_t at = static_cast<size_t>(dest) * kTopK + e % kTopK;
        const int t = s_sel[e];
        const bool live = !failed && t >= 0 && t < H;
        p.slot_output[at] = live ? s_loc[e] : -1;
        p.logical_output[at] = live ? static_cast<int32_t>(p.logical_ids[static_cast<size_t>(o) * H + t]) : -1;
    }
    if (tid == 0) {
        p.miss_counts[b * 5 + 4] = failed ? 0 : old;
        p.status[b] = static_cast<int32_t>(s_err);
    }
    // Workspace back to its prepared state for the positions this request touched.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int e = tid; e < Q * kTopK; e += kRsThreads) {
        const int t = s_sel[e];
        if (t >= 0 && t < H) {
            store_agent(&first[t], kNoFirst);
            store_agent(&rank_of[t], -1);
        }
    }
}

// The resolve of a request with one query row (the plain decode step): the same outcome
// as resident_resolve_kernel, with the row's first occurrences and miss ranks kept in an
// LDS hash set of its tokens instead of the workspace tables, and every global value the
// resolve needs (hot_valid, reserved, the LRU candidates, the tokens' KV addresses and
// logical ids) requested together at the start: one round trip to memory instead of a chain
// of them.
constexpr int kHashSlots = 2 * kTopK;  // at most kTopK keys: load factor <= 1/2

KVIP_DEVICE uint32_t token_hash(int t) { return (static_cast<uint32_t>(t) * 0x9E3779B9u) >> 20; }  // 12 bits

__global__ __launch_bounds__(kRsThreads) void resident_resolve_one_kernel(const KvipResidentArgs p) {
    static_assert(kHashSlots == 4096, "12-bit token hash");
    __shared__ int32_t s_slots[kTopK];             // slot of each miss rank
    __shared__ int32_t s_ord[kTopK];               // its candidate ordinal (reserved_hot of the slot), or -1
    __shared__ uint32_t s_bitmap[kMaxWords];       // protected or allocated hot slots
    __shared__ int32_t s_hkey[kHashSlots];         // tokens of the row's unresolved entries
    __shared__ uint32_t s_hfirst[kHashSlots];      // lowest entry index of each token
    __shared__ int32_t s_hrank[kHashSlots];        // miss rank of each token
    __shared__ uint32_t s_wave[kRsThreads / 64];
    __shared__ uint32_t s_err;
    __shared__ int s_dest;

    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int R = p.resident;
    const int H = p.history;
    const int words = (R + 31) / 32;
    const int o = p.row_owners[b];
    const bool good_owner = owner_ok(p, o);
    const int oo = good_owner ? o : 0;
    const int32_t* reserved = p.reserved_hot + static_cast<size_t>(b) * R;
    const int32_t* lru = p.lru_slots + static_cast<size_t>(b) * kLru;
    const int32_t* hot_valid = p.hot_valid + static_cast<size_t>(oo) * R;
    const Tail tail = tail_of(p, b);
    const bool prefetched = p.prefetch_counts != nullptr;
    const int used = prefetched ? p.prefetch_counts[b] : p.used;
    const int32_t* pmap = workspace_of(p).map + static_cast<size_t>(b) * H;
    const int nchg = kLru + kTopK;

    // Entries i = 2 tid + k, and every global value they need, requested at once.
    int tok[2], cand[2], hv[2], rsv[2], pk[2];
    int64_t addr[2], logical[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = 2 * tid + k;
        const int t = p.topk[static_cast<size_t>(b) * kTopK + i];
        tok[k] = t;
        cand[k] = lru[i];
        const bool in = good_owner && t >= 0 && t < H;
        const int tc = in ? t : 0;
        const int th = in && t < R ? t : 0;
        hv[k] = hot_valid[th];
        rsv[k] = reserved[th];
        pk[k] = prefetched ? pmap[tc] : -1;
        addr[k] = p.addresses[static_cast<size_t>(oo) * H + tc];
        logical[k] = p.logical_ids[static_cast<size_t>(oo) * H + tc];
    }
    for (int w = tid; w < words; w += kRsThreads) s_bitmap[w] = 0u;
    for (int h = tid; h < kHashSlots; h += kRsThreads) {
        s_hkey[h] = -1;
        s_hfirst[h] = kNoFirst;
    }
    if (tid == 0) {
        s_err = static_cast<uint32_t>(p.status[b]) | (good_owner && tail.ok ? 0u : static_cast<uint32_t>(KVIP_RESIDENT_ERR_TOKEN));
        s_dest = -1;
    }
    __syncthreads();

    // Classification (as resident_resolve_kernel's, one row).
    int loc[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int t = tok[k];
        loc[k] = -1;
        if (t >= H) {
            atomicOr(&s_err, KVIP_RESIDENT_ERR_TOKEN);
        } else if (good_owner && t >= 0) {
            const bool in_tail = t >= tail.begin && t < tail.end;
            if (in_tail && t < tail.mapped) {
                loc[k] = R + t % tail.ring;
            } else if (!in_tail && t < R && hv[k] != 0 && rsv[k] < 0) {
                loc[k] = t;
                atomicOr(&s_bitmap[t >> 5], 1u << (t & 31));
            } else if (prefetched) {
                const int s = pk[k] >= 0 && pk[k] < used ? lru[pk[k]] : -1;
                if (s >= 0 && s < R) {
                    loc[k] = s;
                    atomicOr(&s_bitmap[s >> 5], 1u << (s & 31));
                }
            }
        }
    }
    // (a) first occurrence of every unresolved token (LDS hash set, linear probing).
    bool unresolved[2];
    int slot_of[2] = {0, 0};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int t = tok[k];
        unresolved[k] = t >= 0 && t < H && loc[k] < 0;
        if (unresolved[k]) {
            uint32_t h = token_hash(t);
            for (int probe = 0; probe < kHashSlots; ++probe) {
                const int prev = atomicCAS(&s_hkey[h], -1, t);
                if (prev == -1 || prev == t) break;
                h = (h + 1) & (kHashSlots - 1);
            }
            slot_of[k] = static_cast<int>(h);
            atomicMin(&s_hfirst[h], static_cast<uint32_t>(2 * tid + k));
        }
    }
    __syncthreads();
    const bool run = s_err == 0u;  // uniform: read after a barrier
    int need = 0;
    bool fresh[2] = {false, false};
    if (run) {
        // (b) new misses in index order -> ranks.
        uint32_t nnew = 0;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            fresh[k] = unresolved[k] && s_hfirst[slot_of[k]] == static_cast<uint32_t>(2 * tid + k);
            nnew += fresh[k] ? 1u : 0u;
        }
        uint32_t need_u;
        uint32_t r = block_exclusive_scan(nnew, s_wave, &need_u);
        need = static_cast<int>(need_u);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            if (fresh[k]) s_hrank[slot_of[k]] = static_cast<int32_t>(r++);
        }
        // (c) slots: free candidates in ordinal order, pass 0 = ordinals >= used.
        int allocated = 0;
        if (need > 0) {
            for (int pass = 0; pass < 2 && allocated < need; ++pass) {
                bool ok[2];
                uint32_t avail = 0;
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int ord = 2 * tid + k;
                    const int s = cand[k];
                    ok[k] = false;
                    if ((ord >= used) == (pass == 0)) {
                        if (s < 0 || s >= R) {
                            atomicOr(&s_err, KVIP_RESIDENT_ERR_CANDIDATE);
                        } else {
                            ok[k] = ((s_bitmap[s >> 5] >> (s & 31)) & 1u) == 0u;
                        }
                    }
                    avail += ok[k] ? 1u : 0u;
                }
                uint32_t n_avail;
                uint32_t rank = block_exclusive_scan(avail, s_wave, &n_avail);
                const int take = min(static_cast<int>(n_avail), need - allocated);
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    if (ok[k]) {
                        if (rank < static_cast<uint32_t>(take)) {
                            // reserved_hot of a candidate's slot is its ordinal (round init)
                            s_slots[allocated + rank] = cand[k];
                            s_ord[allocated + rank] = 2 * tid + k;
                        }
                        ++rank;
                    }
                }
                __syncthreads();
                for (int j = tid; j < take; j += kRsThreads) {
                    const int s = s_slots[allocated + j];
                    atomicOr(&s_bitmap[s >> 5], 1u << (s & 31));
                }
                allocated += take;
                __syncthreads();
            }
            if (allocated < need && s_err == 0u) {
                // Fallback: every known slot is protected, then the free hot slots in
                // ascending order (none is a candidate's: every free candidate was taken).
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    if (loc[k] >= 0 && loc[k] < R) atomicOr(&s_bitmap[loc[k] >> 5], 1u << (loc[k] & 31));
                }
                __syncthreads();
                const int per = (words + kRsThreads - 1) / kRsThreads;
                const int w0 = min(tid * per, words);
                const int w1 = min(w0 + per, words);
                uint32_t free_bits = 0;
                for (int w = w0; w < w1; ++w) {
                    const int bits = min(32, R - 32 * w);
                    const uint32_t live = bits == 32 ? 0xFFFFFFFFu : ((1u << bits) - 1u);
                    free_bits += __popc(~s_bitmap[w] & live);
                }
                uint32_t n_free;
                uint32_t rank = block_exclusive_scan(free_bits, s_wave, &n_free);
                const int want = need - allocated;
                if (n_free < static_cast<uint32_t>(want)) {
                    if (tid == 0) atomicOr(&s_err, KVIP_RESIDENT_ERR_CANDIDATE);
                } else {
                    for (int w = w0; w < w1 && rank < static_cast<uint32_t>(want); ++w) {
                        const int bits = min(32, R - 32 * w);
                        const uint32_t live = bits == 32 ? 0xFFFFFFFFu : ((1u << bits) - 1u);
                        uint32_t m = ~s_bitmap[w] & live;
                        while (m != 0u && rank < static_cast<uint32_t>(want)) {
                            const int bit = __ffs(m) - 1;
                            s_slots[allocated + rank] = 32 * w + bit;
                            s_ord[allocated + rank] = -1;
                            ++rank;
                            m &= m - 1u;
                        }
                    }
                }
                __syncthreads();
                if (s_err == 0u) {
                    for (int j = tid; j < want; j += kRsThreads) {
                        const int s = s_slots[allocated + j];
                        atomicOr(&s_bitmap[s >> 5], 1u << (s & 31));
                    }
                    allocated = need;
                }
                __syncthreads();
            }
        }
        __syncthreads();
        if (s_err == 0u) {
            // (d) locations, change records and Fetch descriptors of the misses.
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                if (unresolved[k]) loc[k] = s_slots[s_hrank[slot_of[k]]];
                if (fresh[k]) {
                    const int rk = s_hrank[slot_of[k]];
                    const int s = s_slots[rk];
                    const int ord = s_ord[rk];
                    const int rec = ord >= 0 ? ord : kLru + rk;
                    p.change_slots[static_cast<size_t>(b) * nchg + rec] = s;
                    p.changes[static_cast<size_t>(b) * nchg + rec] = tok[k];
                    const size_t d = static_cast<size_t>(b) * kTopK + rk;
                    const int64_t off = addr[k];
                    if (off < 0 || off > p.host_pool_bytes - p.row_bytes || (off & 15) != 0) {
                        atomicOr(&s_err, KVIP_RESIDENT_ERR_SOURCE);
                    }
                    p.fetch_slots[d] = s;
                    p.fetch_positions[d] = tok[k];
                    p.fetch_sources[d] = off;
                }
            }
            if (tid == 0) p.miss_counts[b * 5] = need;
        }
        __syncthreads();
    }

    // Outputs (-1 throughout for a failed request) and the miss total; in token order as in
    // resident_resolve_kernel.
    const bool failed = s_err != 0u;
    const bool tnd = p.unpack_indices != nullptr;
    int dest = b;
    if (tnd) {
        const int rows = p.batch * kMaxQ;
        for (int r = tid; r < rows; r += kRsThreads) {
            const bool active = p.output_valid[r] != 0;
            if (active && p.unpack_indices[r] == static_cast<int64_t>(b) * kMaxQ) s_dest = r;
        }
        for (int e = tid; e < kMaxQ * kTopK; e += kRsThreads) {
            const int r = b * kMaxQ + e / kTopK;
            if (p.output_valid[r] == 0) {
                const size_t at = static_cast<size_t>(r) * kTopK + e % kTopK;
                p.slot_output[at] = -1;
                p.logical_output[at] = -1;
            }
        }
        __syncthreads();
        dest = s_dest;
    }
    if (dest >= 0) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const size_t at = static_cast<size_t>(dest) * kTopK + 2 * tid + k;
            const int t = tok[k];
            const bool live = !failed && t >= 0 && t < H;
            p.slot_output[at] = live ? loc[k] : -1;
            p.logical_output[at] = live ? static_cast<int32_t>(logical[k]) : -1;
        }
    }
    if (tid == 0) {
        p.miss_counts[b * 5 + 4] = failed ? 0 : need;
        p.status[b] = static_cast<int32_t>(s_err);
    }
}

// Speculative windowed prefetch of request b (one 1024-thread workgroup): the window
// candidates in order, the first `available` of each window taken as the next ordinals.
// Records go to prefetch_tokens / the ordinal change records / the workspace map; the
// rows are copied by resident_fetch_kernel<., true>.
__global__ __launch_bounds__(kRsThreads) void resident_prefetch_kernel(const KvipResidentArgs p,
                                                                       const KvipPrefetchArgs f, int e_begin,
                                                                       int e_end) {
    __shared__ uint32_t s_wave[kRsThreads / 64];
    __shared__ uint32_t s_err;
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int Q = p.rows_per_request;
    const int R = p.resident;
    const int H = p.history;
    if (p.status[b] != 0) return;  // uniform: the round already failed (count stays 0)
    if (!owner_ok(p, p.row_owners[b])) {  // uniform; the prefetch Fetch then skips the request
        if (tid == 0) atomicOr(&p.status[b], static_cast<int32_t>(KVIP_RESIDENT_ERR_TOKEN));
        return;
    }
    const Tail tail = tail_of(p, b);
    const int o = p.row_owners[b];
    const int32_t* lru = p.lru_slots + static_cast<size_t>(b) * kLru;
    int32_t* map = workspace_of(p).map + static_cast<size_t>(b) * H;
    int32_t* tokens = p.prefetch_tokens + static_cast<size_t>(b) * kLru;
    const int nchg = kLru + Q * kTopK;
    int32_t* changes = p.changes + static_cast<size_t>(b) * nchg;
    if (tid == 0) s_err = 0u;
    __syncthreads();
    auto mapped_tail = [&](int t) { return t >= tail.begin && t < tail.mapped; };
    // Takes ordinal k for token t. The row's host source is checked here, so that a bad
    // source is in the status word before the round's resolve whenever the copy runs.
    auto take = [&](int k, int t) {
        const int s = lru[k];
        if (s < 0 || s >= R) atomicOr(&s_err, KVIP_RESIDENT_ERR_CANDIDATE);
        const int64_t off = p.addresses[static_cast<size_t>(o) * H + t];
        if (off < 0 || off > p.host_pool_bytes - p.row_bytes || (off & 15) != 0) {
            atomicOr(&s_err, KVIP_RESIDENT_ERR_SOURCE);
        }
        tokens[k] = t;
        map[t] = k;
        changes[k] = t;
    };
    // Windows [e_begin, e_end) continue from the count the earlier windows left.
    int used = e_begin == 0 ? 0 : p.prefetch_counts[b];  // uniform
    const int cold_tiles = (H - R) / kBlockTokens;
    auto window_end = [&](int e) {
        return R + kBlockTokens * static_cast<int>(static_cast<int64_t>(cold_tiles) * e / max(1, f.windows - 1));
    };
    int lo = e_begin <= 1 ? R : window_end(e_begin - 1);
    int32_t* counts = f.window_counts != nullptr ? f.window_counts + static_cast<size_t>(b) * KVIP_PREFETCH_MAX_WINDOWS
                                                 : nullptr;
    for (int e = e_begin; e < e_end; ++e) {
        const int available = min(f.window_limit, min(kLru - used, f.prefetch_limit - used));
        const int hi = window_end(e);
        if (available <= 0) {
            if (counts != nullptr && tid == 0) counts[e] = used;
            if (e > 0) lo = hi;
            continue;
        }
        int taken = 0;
        if (e == 0) {
            // Victim coordinates i = 2 tid + k, in ordinal order; candidate token lru[i].
            uint32_t mine = 0;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int i = 2 * tid + k;
                uint32_t hit = 0;
                for (int q = 0; q < Q; ++q) {
                    hit |= (f.victim_hits[static_cast<size_t>(b * Q + q) * (kLru / 32) + i / 32] >> (i % 32)) & 1u;
                }
                const int t = lru[i];
                if (hit != 0u && t >= 0 && t < H && !mapped_tail(t)) mine |= 1u << k;
            }
            uint32_t total;
            uint32_t r = block_exclusive_scan(__popc(mine), s_wave, &total);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                if ((mine >> k) & 1u) {
                    if (r < static_cast<uint32_t>(available)) take(used + static_cast<int>(r), lru[2 * tid + k]);
                    ++r;
                }
            }
            taken = min(static_cast<int>(total), available);
        } else {
            // Cold positions [lo, hi) (128-aligned offsets from R), 32 per hit word.
            const int w_lo = (lo - R) / 32, w_hi = min((hi - R) / 32, f.cold_words);
            for (int w0 = w_lo; w0 < w_hi && taken < available; w0 += kRsThreads) {
                const int w = w0 + tid;
                uint32_t bits = 0u;
                if (w < w_hi) {
                    for (int q = 0; q < Q; ++q) bits |= f.cold_hits[static_cast<size_t>(b * Q + q) * f.cold_words + w];
                    const int base = R + 32 * w;
                    if (tail.mapped > tail.begin && base < tail.mapped && base + 32 > tail.begin) {
                        for (int j = 0; j < 32; ++j) {
                            if (mapped_tail(base + j)) bits &= ~(1u << j);
                        }
                    }
                    if (base + 32 > H) bits &= H - base >= 32 ? 0xFFFFFFFFu : ((1u << max(H - base, 0)) - 1u);
                }
                uint32_t total;
                uint32_t r = static_cast<uint32_t>(taken) + block_exclusive_scan(__popc(bits), s_wave, &total);
                while (bits != 0u && r < static_cast<uint32_t>(available)) {
                    const int j = __ffs(bits) - 1;
                    take(used + static_cast<int>(r), R + 32 * w + j);
                    ++r;
                    bits &= bits - 1u;
                }
                taken = min(taken + static_cast<int>(total), available);
            }
            lo = hi;
        }
        used += taken;
        if (counts != nullptr && tid == 0) counts[e] = used;
        __syncthreads();
    }
    if (tid == 0) {
        p.prefetch_counts[b] = used;
        if (s_err != 0u) atomicOr(&p.status[b], static_cast<int32_t>(s_err));
    }
}

// Fetch of the missed rows (PREFETCH: of the prefetched rows, source = the token's KV
// address, slot = its candidate slot). Rows go in groups of 32, one group per wave at a
// time: the wave issues the group's loads from the host pool (21 16-byte loads per lane),
// then stores them to the hot cache, and moves on by the grid's wave count. The grid is
// bounded (kFetchWaves waves in all): a few MB of host reads in flight at once fill the
// L2 / fabric miss queues that the Index update's HBM accesses share, which then wait
// for the whole Fetch; ~1 MB in flight already covers the host link's latency-bandwidth
// product (57 GB/s x ~2 us).
constexpr int kFetchRows = 32;
constexpr int kFetchWaves = 64;
template <int PIECES, bool PREFETCH>
__global__ __launch_bounds__(256) void resident_fetch_kernel(const KvipResidentArgs p, const int32_t* window_counts,
                                                             int e_begin, int e_end) {
    const int b = blockIdx.y;
    const int lane = threadIdx.x & 63;
    // The prefetch copy runs before the resolve and skips a failed round. The miss copy
    // reads only the resolve's outputs (a failed request's miss total is 0, every source
    // was checked by the resolve), never the status words that a concurrent Index update
    // may set: the copy and the update can run side by side.
    if (PREFETCH && p.status[b] != 0) return;
    // Rows [first, total): the prefetch rows of windows [e_begin, e_end) with window counts,
    // else every prefetched row or every miss.
    int first = 0, total;
    if (PREFETCH && window_counts != nullptr) {
        const int32_t* counts = window_counts + static_cast<size_t>(b) * KVIP_PREFETCH_MAX_WINDOWS;
        first = e_begin > 0 ? counts[e_begin - 1] : 0;
        total = counts[e_end - 1];
    } else {
        total = PREFETCH ? p.prefetch_counts[b] : p.miss_counts[b * 5 + 4];
    }
    const int o = p.row_owners[b];
    const int pieces = PIECES > 0 ? PIECES : p.row_bytes / 16;
    uint32_t err = 0;
    for (int r0 = first + (blockIdx.x * 4 + (threadIdx.x >> 6)) * kFetchRows; r0 < total;
         r0 += gridDim.x * 4 * kFetchRows) {
        const int rows = min(kFetchRows, total - r0);
        int64_t src = -1, dst = -1;
        if (lane < rows) {
            int64_t off;
            int slot;
            if constexpr (PREFETCH) {
                const int k = r0 + lane;
                const int t = p.prefetch_tokens[static_cast<size_t>(b) * kLru + k];
                slot = p.lru_slots[static_cast<size_t>(b) * kLru + k];
                off = t >= 0 && t < p.history ? p.addresses[static_cast<size_t>(o) * p.history + t] : -1;
                if (slot < 0 || slot >= p.resident) off = -1;
            } else {
                const size_t d = static_cast<size_t>(b) * p.rows_per_request * kTopK + r0 + lane;
                off = p.fetch_sources[d];
                slot = p.fetch_slots[d];
            }
            if (off >= 0 && off <= p.host_pool_bytes - p.row_bytes && (off & 15) == 0) {
                src = off;
                dst = (static_cast<int64_t>(o) * p.hot_stride + slot) * p.row_bytes;
            } else {
                err = KVIP_RESIDENT_ERR_SOURCE;
            }
        }
        const int n = rows * pieces;
        if constexpr (PIECES > 0) {
            constexpr int kIters = (kFetchRows * PIECES + 63) / 64;
            v4i val[kIters];
#pragma unroll
            for (int it = 0; it < kIters; ++it) {
                const int idx = it * 64 + lane;
                const int r = idx / PIECES;
                const int piece = idx - r * PIECES;
                const int64_t s = row_value<PIECES, kFetchRows>(src, it, r);
                val[it] = v4i{0, 0, 0, 0};
                if (idx < n && s >= 0) {
                    val[it] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p.host_pool + s + piece * 16));
                }
            }
#pragma unroll
            for (int it = 0; it < kIters; ++it) {
                const int idx = it * 64 + lane;
                const int r = idx / PIECES;
                const int piece = idx - r * PIECES;
                const int64_t d = row_value<PIECES, kFetchRows>(dst, it, r);
                if (idx < n && d >= 0) *reinterpret_cast<v4i*>(p.hot_cache + d + piece * 16) = val[it];
            }
        } else {
            const int iters = (kFetchRows * pieces + 63) / 64;
            for (int it = 0; it < iters; ++it) {
                const int idx = it * 64 + lane;
                const int r = idx / pieces;
                const int piece = idx - r * pieces;
                const int64_t s = __shfl(src, min(r, kFetchRows - 1));
                const int64_t d = __shfl(dst, min(r, kFetchRows - 1));
                if (idx < n && s >= 0 && d >= 0) {
                    *reinterpret_cast<v4i*>(p.hot_cache + d + piece * 16) =
                        *reinterpret_cast<const v4i*>(p.host_pool + s + piece * 16);
                }
            }
        }
    }
    if (err != 0u) atomicOr(&p.status[b], static_cast<int32_t>(err));
}

KVIP_DEVICE uint32_t set_hash(uint32_t k) { return (k * 0x9E3779B9u) >> 21; }  // 11 bits: kSetSize

// Inserts k; false when it is already present (or the set is full).
KVIP_DEVICE bool set_insert(uint32_t* set, uint32_t k) {
    uint32_t h = set_hash(k);
    for (int i = 0; i < kSetSize; ++i) {
        const uint32_t prev = atomicCAS(&set[h], kEmpty, k);
        if (prev == kEmpty) return true;
        if (prev == k) return false;
        h = (h + 1) & (kSetSize - 1);
    }
    return false;
}

KVIP_DEVICE bool set_contains(const uint32_t* set, uint32_t k) {
    uint32_t h = set_hash(k);
    for (int i = 0; i < kSetSize; ++i) {
        const uint32_t v = set[h];
        if (v == k) return true;
        if (v == kEmpty) return false;
        h = (h + 1) & (kSetSize - 1);
    }
    return false;
}

// Index update of request b (the prefetch batch first, then each query's misses), then
// residency of its prefetch and miss slots.
constexpr int kMaxLog = 2 * (kLru + kMaxQ * kTopK);  // destinations written this round
__global__ __launch_bounds__(kRsThreads) void resident_update_kernel(const KvipResidentArgs p) {
    __shared__ uint32_t s_src_set[kSetSize];
    __shared__ uint32_t s_dst_set[kSetSize];
    __shared__ int32_t s_ps[2 * kChunk];
    __shared__ int32_t s_pd[2 * kChunk];
    __shared__ int32_t s_log[kMaxLog];
    __shared__ uint32_t s_wave[kRsThreads / 64];
    __shared__ uint32_t s_err;
    __shared__ int s_nlog;

    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int Q = p.rows_per_request;
    const int R = p.resident;
    const int H = p.history;
    const int o = p.row_owners[b];
    const bool prefetched = p.prefetch_counts != nullptr;
    const int used = prefetched ? p.prefetch_counts[b] : 0;
    const int32_t* pf_tokens = prefetched ? p.prefetch_tokens + static_cast<size_t>(b) * kLru : nullptr;
    const int32_t* lru = p.lru_slots + static_cast<size_t>(b) * kLru;
    if (prefetched) {
        // The prefetch map back to its prepared state (the resolve has read it).
        int32_t* map = workspace_of(p).map + static_cast<size_t>(b) * H;
        for (int k = tid; k < used; k += kRsThreads) {
            const int t = pf_tokens[k];
            if (t >= 0 && t < H) map[t] = -1;
        }
    }
    if (p.status[b] != 0) {  // uniform
        // A failed request's owner loses all residency: nothing it holds is trusted, so
        // its next round reads every position cold.
        if (owner_ok(p, o)) {
            int32_t* hv = p.hot_valid + static_cast<size_t>(o) * R;
            for (int s = tid; s < R; s += kRsThreads) hv[s] = 0;
        }
        return;
    }
    const Workspace ws = workspace_of(p);
    int32_t* row_at = ws.row_at + static_cast<size_t>(b) * H;
    int32_t* pos_of = ws.pos_of + static_cast<size_t>(b) * H;
    uint8_t* keys = p.index_keys + static_cast<size_t>(o) * H * kIndexDim;
    float* scales = p.index_scales + static_cast<size_t>(o) * H;
    int64_t* addresses = p.addresses + static_cast<size_t>(o) * H;
    int64_t* logical = p.logical_ids + static_cast<size_t>(o) * H;
    int32_t* hot_valid = p.hot_valid + static_cast<size_t>(o) * R;
    const size_t dbase = static_cast<size_t>(b) * Q * kTopK;
    if (tid == 0) {
        s_err = 0u;
        s_nlog = 0;
    }
    __syncthreads();

    int r0 = 0;
    for (int q = prefetched ? -1 : 0; q < Q; ++q) {  // q = -1: the prefetch batch, in ordinal order
        const int count = q < 0 ? used : p.miss_counts[b * 5 + q];
        for (int c0 = 0; c0 < count; c0 += kChunk) {
            if (s_err != 0u) break;  // uniform
            const int n = min(kChunk, count - c0);
            for (int i = tid; i < kSetSize; i += kRsThreads) {
                s_src_set[i] = kEmpty;
                s_dst_set[i] = kEmpty;
            }
            __syncthreads();
            int src = -1, dst = -1;
            if (tid < n) {
                const int orig = q < 0 ? pf_tokens[c0 + tid] : p.fetch_positions[dbase + r0 + c0 + tid];
                dst = q < 0 ? lru[c0 + tid] : p.fetch_slots[dbase + r0 + c0 + tid];
                const bool in_range = orig >= 0 && orig < H && dst >= 0 && dst < R;
                src = in_range ? pos_of[orig] : -1;
                if (!in_range || !set_insert(s_src_set, static_cast<uint32_t>(src)) ||
                    !set_insert(s_dst_set, static_cast<uint32_t>(dst))) {
                    atomicOr(&s_err, KVIP_RESIDENT_ERR_UPDATE);
                }
            }
            __syncthreads();
            if (s_err != 0u) break;
            // Closure: displaced destination rows fill the freed source positions in order.
            const bool out = tid < n && !set_contains(s_src_set, static_cast<uint32_t>(dst));
            const bool freed = tid < n && !set_contains(s_dst_set, static_cast<uint32_t>(src));
            uint32_t totals;
            const uint32_t pre = block_exclusive_scan((out ? 1u : 0u) | ((freed ? 1u : 0u) << 16), s_wave, &totals);
            if (tid < n) {
                s_ps[tid] = src;
                s_pd[tid] = dst;
            }
            if (out) s_ps[kChunk + (pre & 0xFFFFu)] = dst;
            if (freed) s_pd[kChunk + (pre >> 16)] = src;
            __syncthreads();
            const int extras = static_cast<int>(totals & 0xFFFFu);
            const int moves = n + extras;
            // Snapshot every moving row, then write (a permutation of the moved positions).
            const int m = tid;
            const int j = m < n ? m : kChunk + m - n;
            int ps = 0, pd = 0, row = 0;
            v4i kv[kIndexDim / 16];
            float sc = 0.f;
            int64_t ad = 0, lg = 0;
            if (m < moves) {
                ps = s_ps[j];
                pd = s_pd[j];
                const v4i* kr = reinterpret_cast<const v4i*>(keys + static_cast<size_t>(ps) * kIndexDim);
#pragma unroll
                for (int v = 0; v < kIndexDim / 16; ++v) kv[v] = kr[v];
                sc = scales[ps];
                ad = addresses[ps];
                lg = logical[ps];
                row = row_at[ps];
            }
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (m < moves) {
                v4i* kw = reinterpret_cast<v4i*>(keys + static_cast<size_t>(pd) * kIndexDim);
#pragma unroll
                for (int v = 0; v < kIndexDim / 16; ++v) kw[v] = kv[v];
                scales[pd] = sc;
                addresses[pd] = ad;
                logical[pd] = lg;
                row_at[pd] = row;
                pos_of[row] = pd;
                if (m >= n && pd < R) hot_valid[pd] = 0;  // freed hot position: its KV did not move
                const int at = atomicAdd(&s_nlog, 1);
                if (at < kMaxLog) s_log[at] = pd;
            }
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
        if (q >= 0) r0 += count;
    }
    // Residency of every fetched slot (after the freed positions were invalidated). A
    // permutation rejected in a later chunk leaves the earlier chunks applied (each one a
    // complete permutation of the Index rows, addresses and logical ids moving together),
    // so the owner then loses all residency instead.
    const int total = p.miss_counts[b * 5 + 4];
    if (s_err == 0u) {
        for (int i = tid; i < total; i += kRsThreads) hot_valid[p.fetch_slots[dbase + i]] = 1;
        for (int k = tid; k < used; k += kRsThreads) hot_valid[lru[k]] = 1;
    } else {
        for (int s = tid; s < R; s += kRsThreads) hot_valid[s] = 0;
    }
    // Maps back to identity: read every logged position's row, then reset both maps.
    const int nlog = min(s_nlog, kMaxLog);
    int rows[kMaxLog / kRsThreads];
#pragma unroll
    for (int k = 0; k < kMaxLog / kRsThreads; ++k) {
        const int i = tid + k * kRsThreads;
        rows[k] = i < nlog ? row_at[s_log[i]] : -1;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kMaxLog / kRsThreads; ++k) {
        const int i = tid + k * kRsThreads;
        if (i < nlog) {
            row_at[s_log[i]] = s_log[i];
            pos_of[rows[k]] = rows[k];
        }
    }
    if (tid == 0 && s_err != 0u) atomicOr(&p.status[b], static_cast<int32_t>(s_err));
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace

uint32_t validate_resident(const KvipResidentArgs* a) {
    if (a == nullptr) return KVIP_ERR_INVALID;
    const bool ptrs = a->topk && a->row_owners && a->lru_slots && a->reserved_hot && a->hot_valid && a->index_keys &&
                      a->index_scales && a->addresses && a->logical_ids && a->host_pool && a->hot_cache &&
                      a->logical_output && a->slot_output && a->changes && a->change_slots && a->miss_counts &&
                      a->fetch_sources && a->fetch_slots && a->fetch_positions && a->status && a->workspace;
    if (!ptrs) return KVIP_ERR_INVALID;
    const bool ok = a->batch >= 1 && a->batch <= 65535 && a->rows_per_request >= 1 &&
                    a->rows_per_request <= kMaxQ && a->owners >= 1 && a->history >= 128 && a->history % 128 == 0 &&
                    a->history <= (1 << 24) && a->resident >= kLru && a->resident <= KVIP_RESIDENT_MAX_RESIDENT &&
                    a->resident <= a->history && a->hot_stride >= a->resident && a->row_bytes >= 16 &&
                    a->row_bytes % 16 == 0 && a->used >= 0 && a->used <= kLru && a->host_pool_bytes >= a->row_bytes &&
                    aligned(a->index_keys, 16) && aligned(a->host_pool, 16) && aligned(a->hot_cache, 16) &&
                    aligned(a->workspace, 16) && (a->unpack_indices == nullptr) == (a->output_valid == nullptr) &&
                    (a->unpack_indices == nullptr || a->rows_per_request == kMaxQ) &&
                    (a->tail_bounds == nullptr ||
                     ((a->hot_stride - a->resident) % 128 == 0 && a->hot_stride - a->resident >= 384)) &&
                    (a->prefetch_tokens == nullptr) == (a->prefetch_counts == nullptr);
    return ok ? KVIP_OK : KVIP_ERR_INVALID;
}

template <bool PREFETCH>
void launch_resident_fetch(const KvipResidentArgs& a, hipStream_t s, const int32_t* window_counts = nullptr,
                           int e_begin = 0, int e_end = 0) {
    // Up to kFetchWaves waves in all (at least one workgroup per request).
    const int rows = PREFETCH ? kLru : a.rows_per_request * kTopK;
    const int per_request = max(1, kFetchWaves / (4 * a.batch));
    const dim3 fgrid(min((rows + 4 * kFetchRows - 1) / (4 * kFetchRows), per_request), a.batch);
    if (a.row_bytes == KVIP_KV_ROW_BYTES) {
        hipLaunchKernelGGL((resident_fetch_kernel<KVIP_KV_ROW_BYTES / 16, PREFETCH>), fgrid, dim3(256), 0, s, a,
                           window_counts, e_begin, e_end);
    } else {
        hipLaunchKernelGGL((resident_fetch_kernel<0, PREFETCH>), fgrid, dim3(256), 0, s, a, window_counts, e_begin,
                           e_end);
    }
}

hipError_t launch_resident_begin(const KvipResidentArgs& a, hipStream_t s, int32_t* table = nullptr,
                                 int max_blocks = 0) {
    hipLaunchKernelGGL(resident_init_kernel, dim3(a.batch), dim3(kRsThreads), 0, s, a, table, max_blocks,
                       a.history / kBlockTokens);
    return hipGetLastError();
}

hipError_t launch_resident_resolve(const KvipResidentArgs& a, hipStream_t s) {
    if (a.rows_per_request == 1) {
        hipLaunchKernelGGL(resident_resolve_one_kernel, dim3(a.batch), dim3(kRsThreads), 0, s, a);
    } else {
        hipLaunchKernelGGL(resident_resolve_kernel, dim3(a.batch), dim3(kRsThreads), 0, s, a);
    }
    return hipGetLastError();
}

hipError_t launch_resident_update(const KvipResidentArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(resident_update_kernel, dim3(a.batch), dim3(kRsThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_resident_finish(const KvipResidentArgs& a, hipStream_t s) {
    const hipError_t e = launch_resident_resolve(a, s);
    if (e != hipSuccess) return e;
    launch_resident_fetch<false>(a, s);
    return launch_resident_update(a, s);
}

hipError_t launch_resident_round(const KvipResidentArgs& a, hipStream_t s) {
    const hipError_t e = launch_resident_begin(a, s);
    return e != hipSuccess ? e : launch_resident_finish(a, s);
}

}  // namespace kvip

extern "C" uint64_t kvip_hip_resident_workspace_bytes(int32_t batch, int32_t history) {
    if (batch < 1 || history < 1) return 0;
    return 20ull * static_cast<uint64_t>(batch) * static_cast<uint64_t>(history);
}

extern "C" uint32_t kvip_hip_resident_prepare(const KvipResidentArgs* args, void* stream) {
    const uint32_t rc = kvip::validate_resident(args);
    if (rc != KVIP_OK) return rc;
    hipLaunchKernelGGL(kvip::resident_prepare_kernel, dim3(1024), dim3(256), 0, static_cast<hipStream_t>(stream),
                       *args);
    return static_cast<uint32_t>(hipGetLastError());
}

extern "C" uint32_t kvip_hip_resident_round(const KvipResidentArgs* args, void* stream) {
    const uint32_t rc = kvip::validate_resident(args);
    if (rc != KVIP_OK) return rc;
    return static_cast<uint32_t>(kvip::launch_resident_round(*args, static_cast<hipStream_t>(stream)));
}

extern "C" uint32_t kvip_hip_resident_begin(const KvipResidentArgs* args, void* stream) {
    const uint32_t rc = kvip::validate_resident(args);
    if (rc != KVIP_OK) return rc;
    return static_cast<uint32_t>(kvip::launch_resident_begin(*args, static_cast<hipStream_t>(stream)));
}

extern "C" uint32_t kvip_hip_resident_finish(const KvipResidentArgs* args, void* stream) {
    const uint32_t rc = kvip::validate_resident(args);
    if (rc != KVIP_OK) return rc;
    return static_cast<uint32_t>(kvip::launch_resident_finish(*args, static_cast<hipStream_t>(stream)));
}

extern "C" uint32_t kvip_hip_resident_resolve(const KvipResidentArgs* args, void* stream) {
    const uint32_t rc = kvip::validate_resident(args);
    if (rc != KVIP_OK) return rc;
    return static_cast<uint32_t>(kvip::launch_resident_resolve(*args, static_cast<hipStream_t>(stream)));
}

extern "C" uint32_t kvip_hip_resident_fetch(const KvipResidentArgs* args, void* stream) {
    const uint32_t rc = kvip::validate_resident(args);
    if (rc != KVIP_OK) return rc;
    kvip::launch_resident_fetch<false>(*args, static_cast<hipStream_t>(stream));
    return static_cast<uint32_t>(hipGetLastError());
}

extern "C" uint32_t kvip_hip_resident_update(const KvipResidentArgs* args, void* stream) {
    const uint32_t rc = kvip::validate_resident(args);
    if (rc != KVIP_OK) return rc;
    return static_cast<uint32_t>(kvip::launch_resident_update(*args, static_cast<hipStream_t>(stream)));
}

extern "C" uint32_t kvip_hip_resident_prefetch(const KvipResidentArgs* args, const KvipPrefetchArgs* f,
                                               void* stream) {
    const uint32_t rc = kvip::validate_resident(args);
    if (rc != KVIP_OK) return rc;
    if (f == nullptr || args->prefetch_tokens == nullptr) return KVIP_ERR_INVALID;
    const int cold_tiles = (args->history - args->resident) / kvip::kBlockTokens;
    const bool ok = f->victim_hits != nullptr && f->cold_hits != nullptr && args->resident % kvip::kBlockTokens == 0 &&
                    f->windows >= 1 && f->windows <= 32 && cold_tiles > f->windows && f->window_limit >= 1 &&
                    f->window_limit <= 480 && f->prefetch_limit >= 0 && f->prefetch_limit <= kvip::kLru &&
                    static_cast<int64_t>(f->cold_words) * 32 >= static_cast<int64_t>(args->history) - args->resident;
    if (!ok) return KVIP_ERR_INVALID;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(kvip::resident_prefetch_kernel, dim3(args->batch), dim3(kvip::kRsThreads), 0, s, *args, *f, 0,
                       f->windows);
    kvip::launch_resident_fetch<true>(*args, s);
    return static_cast<uint32_t>(hipGetLastError());
}

namespace kvip {
// Arguments of the windowed prefetch entry points: a valid prefetch, window counts, and a
// window range inside [0, windows).
static bool prefetch_windows_ok(const KvipResidentArgs* args, const KvipPrefetchArgs* f, int e_begin, int e_end) {
    if (validate_resident(args) != KVIP_OK || f == nullptr || args->prefetch_tokens == nullptr) return false;
    const int cold_tiles = (args->history - args->resident) / kBlockTokens;
    return f->victim_hits != nullptr && f->cold_hits != nullptr && f->window_counts != nullptr &&
           args->resident % kBlockTokens == 0 && f->windows >= 1 && f->windows <= KVIP_PREFETCH_MAX_WINDOWS &&
           cold_tiles > f->windows && f->window_limit >= 1 && f->window_limit <= 480 && f->prefetch_limit >= 0 &&
           f->prefetch_limit <= kLru &&
           static_cast<int64_t>(f->cold_words) * 32 >= static_cast<int64_t>(args->history) - args->resident &&
           e_begin >= 0 && e_end > e_begin && e_end <= f->windows;
}
}  // namespace kvip

extern "C" uint32_t kvip_hip_resident_prefetch_windows(const KvipResidentArgs* args, const KvipPrefetchArgs* f,
                                                       int32_t window_begin, int32_t window_end, void* stream) {
    if (!kvip::prefetch_windows_ok(args, f, window_begin, window_end)) return KVIP_ERR_INVALID;
    hipLaunchKernelGGL(kvip::resident_prefetch_kernel, dim3(args->batch), dim3(kvip::kRsThreads), 0,
                       static_cast<hipStream_t>(stream), *args, *f, window_begin, window_end);
    return static_cast<uint32_t>(hipGetLastError());
}

extern "C" uint32_t kvip_hip_resident_prefetch_copy(const KvipResidentArgs* args, const KvipPrefetchArgs* f,
                                                    int32_t window_begin, int32_t window_end, void* stream) {
    if (!kvip::prefetch_windows_ok(args, f, window_begin, window_end)) return KVIP_ERR_INVALID;
    kvip::launch_resident_fetch<true>(*args, static_cast<hipStream_t>(stream), f->window_counts, window_begin,
                                      window_end);
    return static_cast<uint32_t>(hipGetLastError());
}

namespace kvip {
// Round initialisation with the owner block table (one launch), then the scoring of the
// owners' Index rows (the first half of kvip_hip_resident_forward); KVIP_ERR_INVALID when
// the three argument blocks do not chain.
static uint32_t resident_score(const KvipIndexerArgs* indexer, const KvipTopkArgs* topk,
                               const KvipResidentArgs* resident, hipStream_t s, int token_begin = 0,
                               int token_end = -1);
}  // namespace kvip

extern "C" uint32_t kvip_hip_resident_score(const KvipIndexerArgs* indexer, const KvipTopkArgs* topk,
                                            const KvipResidentArgs* resident, void* stream) {
    return kvip::resident_score(indexer, topk, resident, static_cast<hipStream_t>(stream));
}

extern "C" uint32_t kvip_hip_resident_score_window(const KvipIndexerArgs* indexer, const KvipTopkArgs* topk,
                                                   const KvipResidentArgs* resident, int32_t token_begin,
                                                   int32_t token_end, void* stream) {
    if (indexer == nullptr || !kvip::ring_eligible(*indexer) || token_begin < 0 || token_end <= token_begin ||
        token_begin % 128 != 0) {
        return KVIP_ERR_INVALID;
    }
    return kvip::resident_score(indexer, topk, resident, static_cast<hipStream_t>(stream), token_begin, token_end);
}

extern "C" uint32_t kvip_hip_resident_forward(const KvipIndexerArgs* indexer, const KvipTopkArgs* topk,
                                              const KvipResidentArgs* resident, void* stream) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const uint32_t rc = kvip::resident_score(indexer, topk, resident, s);
    if (rc != KVIP_OK) return rc;
    const hipError_t e = kvip::launch_topk(*topk, s);
    if (e != hipSuccess) return static_cast<uint32_t>(e);
    return static_cast<uint32_t>(kvip::launch_resident_finish(*resident, s));
}

uint32_t kvip::resident_score(const KvipIndexerArgs* indexer, const KvipTopkArgs* topk,
                              const KvipResidentArgs* resident, hipStream_t s, int token_begin, int token_end) {
    if (indexer == nullptr || topk == nullptr || resident == nullptr) return KVIP_ERR_INVALID;
    if (kvip::validate_indexer(indexer) != KVIP_OK || kvip::validate_topk(topk) != KVIP_OK ||
        kvip::validate_resident(resident) != KVIP_OK) {
        return KVIP_ERR_INVALID;
    }
    const KvipIndexerArgs& li = *indexer;
    const KvipResidentArgs& ra = *resident;
    const int blocks_per_owner = ra.history / kvip::kBlockTokens;
    // Scoring reads the owners' Index rows through the block table; TopK feeds the round.
    const bool chained = topk->score_keys == li.score_keys && topk->batch == li.batch &&
                         topk->rows_per_request == li.rows_per_request && topk->key_stride == li.key_stride &&
                         li.batch == ra.batch && li.rows_per_request == ra.rows_per_request &&
                         topk->topk == ra.topk && li.keys == ra.index_keys && li.key_scale == ra.index_scales &&
                         li.key_block_stride == static_cast<int64_t>(kvip::kBlockTokens) * kvip::kIndexDim &&
                         li.scale_block_stride == kvip::kBlockTokens && li.max_blocks >= blocks_per_owner &&
                         li.num_blocks == ra.owners * blocks_per_owner && li.qk_dtype == KVIP_DTYPE_FP8_E4M3;
    if (!chained) return KVIP_ERR_INVALID;
    // The round's initialisation (it reads only the candidates) writes the owner table too;
    // a window that starts past position 0 continues a round already initialised.
    if (token_begin == 0) {
        const hipError_t e = kvip::launch_resident_begin(ra, s, const_cast<int32_t*>(li.block_table), li.max_blocks);
        if (e != hipSuccess) return static_cast<uint32_t>(e);
    }
    if (token_end < 0) return static_cast<uint32_t>(kvip::launch_indexer(li, s));
    const int end = static_cast<int>(std::min<int64_t>(token_end, li.key_stride));
    if (end % 128 != 0 && end < li.key_stride) return KVIP_ERR_INVALID;
    return static_cast<uint32_t>(kvip::launch_indexer_ring(li, s, token_begin / 32, (end + 31) / 32));
}

namespace kvip {
namespace {

constexpr int kPcThreads = 256;

// Threshold and victim bits of query row blockIdx.x.
__global__ __launch_bounds__(kPcThreads) void prefix_classify_kernel(const KvipPrefixClassifyArgs p) {
    __shared__ uint32_t s_min[kPcThreads / 64];
    const int row = blockIdx.x;
    const int b = row / p.rows_per_request;
    const int tid = threadIdx.x;
    int valid = max(p.seq_lens[b], 0);
    if (p.query_ends != nullptr) valid = min(valid, p.query_ends[row]);
    valid = min(max(valid, 0), p.key_stride);
    const int pv = min(valid, p.resident);
    const uint16_t* keys = p.score_keys + static_cast<size_t>(row) * p.key_stride;
    // Threshold: smallest key of a full prefix selection.
    uint32_t m = 0xFFFFu;
    if (pv >= kTopK) {
        const int32_t* sel = p.prefix_topk + static_cast<size_t>(row) * kTopK;
        for (int i = tid; i < kTopK; i += kPcThreads) {
            const int t = sel[i];
            if (t >= 0 && t < pv) m = min(m, static_cast<uint32_t>(keys[t]));
        }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) m = min(m, static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), d)));
    if ((tid & 63) == 0) s_min[tid >> 6] = m;
    __syncthreads();
    uint32_t thr = 0u;
    if (pv >= kTopK) {
        thr = s_min[0];
        for (int w = 1; w < kPcThreads / 64; ++w) thr = min(thr, s_min[w]);
    }
    if (tid == 0) p.thresholds[row] = static_cast<uint16_t>(thr);
    // Victim bits: one word (32 candidates) per thread.
    if (tid < kTopK / 32) {
        const int32_t* lru = p.lru_slots + static_cast<size_t>(b) * kTopK;
        uint32_t word = 0u;
        for (int k = 0; k < 32; ++k) {
            const int s = lru[tid * 32 + k];
            const bool hit = s >= 0 && s < pv && static_cast<uint32_t>(keys[s]) > thr;
            word |= (hit ? 1u : 0u) << k;
        }
        p.victim_hits[static_cast<size_t>(row) * (kTopK / 32) + tid] = word;
    }
}

// Cold bits of query row blockIdx.y, words [256 x, 256 x + 256): position resident + 32 w + k
// above the row's threshold. One word per thread, its 32 keys read as four 16-byte pieces
// when the word is aligned and complete.
__global__ __launch_bounds__(kPcThreads) void cold_hits_kernel(const KvipPrefixClassifyArgs p, int word_begin,
                                                               int word_end) {
    const int row = blockIdx.y;
    const int b = row / p.rows_per_request;
    const int w = word_begin + blockIdx.x * kPcThreads + threadIdx.x;
    if (w >= word_end) return;
    int valid = max(p.seq_lens[b], 0);
    if (p.query_ends != nullptr) valid = min(valid, p.query_ends[row]);
    valid = min(max(valid, 0), p.key_stride);
    const uint32_t thr = p.thresholds[row];
    const uint16_t* keys = p.score_keys + static_cast<size_t>(row) * p.key_stride;
    const int pos0 = p.resident + 32 * w;
    uint32_t word = 0u;
    if (pos0 + 32 <= valid && (pos0 & 7) == 0 && (p.key_stride & 7) == 0 &&
        (reinterpret_cast<uintptr_t>(p.score_keys) & 15) == 0) {
        const v4i* src = reinterpret_cast<const v4i*>(keys + pos0);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const v4i x = src[v];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t key = (static_cast<uint32_t>(x[k >> 1]) >> (16 * (k & 1))) & 0xFFFFu;
                word |= (key > thr ? 1u : 0u) << (8 * v + k);
            }
        }
    } else {
        for (int k = 0; k < 32; ++k) {
            const int pos = pos0 + k;
            const bool hit = pos < valid && static_cast<uint32_t>(keys[pos]) > thr;
            word |= (hit ? 1u : 0u) << k;
        }
    }
    p.cold_hits[static_cast<size_t>(row) * p.cold_words + w] = word;
}

}  // namespace
}  // namespace kvip

namespace kvip {
static bool prefix_args_ok(const KvipTopkArgs* topk, const KvipPrefixClassifyArgs* cls) {
    if (topk == nullptr || cls == nullptr || validate_topk(topk) != KVIP_OK) return false;
    const KvipPrefixClassifyArgs& c = *cls;
    return c.score_keys && c.prefix_topk && c.seq_lens && c.lru_slots && c.thresholds && c.victim_hits &&
           c.cold_hits && c.batch == topk->batch && c.rows_per_request == topk->rows_per_request &&
           c.key_stride == topk->key_stride && c.score_keys == topk->score_keys && c.prefix_topk == topk->topk &&
           c.seq_lens == topk->seq_lens && c.query_ends == topk->query_ends && topk->limit == c.resident &&
           c.resident >= 1 && c.resident <= c.key_stride &&
           static_cast<int64_t>(c.cold_words) * 32 >= static_cast<int64_t>(c.key_stride) - c.resident &&
           c.cold_words >= 0;
}
}  // namespace kvip

extern "C" uint32_t kvip_hip_resident_threshold(const KvipTopkArgs* topk, const KvipPrefixClassifyArgs* cls,
                                                void* stream) {
    if (!kvip::prefix_args_ok(topk, cls)) return KVIP_ERR_INVALID;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const hipError_t e = kvip::launch_topk(*topk, s);
    if (e != hipSuccess) return static_cast<uint32_t>(e);
    hipLaunchKernelGGL(kvip::prefix_classify_kernel, dim3(cls->batch * cls->rows_per_request), dim3(kvip::kPcThreads),
                       0, s, *cls);
    return static_cast<uint32_t>(hipGetLastError());
}

extern "C" uint32_t kvip_hip_resident_cold_hits(const KvipPrefixClassifyArgs* cls, int32_t word_begin,
                                                int32_t word_end, void* stream) {
    if (cls == nullptr || cls->cold_hits == nullptr || cls->score_keys == nullptr || cls->thresholds == nullptr ||
        cls->seq_lens == nullptr || word_begin < 0 || word_end <= word_begin || word_end > cls->cold_words) {
        return KVIP_ERR_INVALID;
    }
    const int words = word_end - word_begin;
    hipLaunchKernelGGL(kvip::cold_hits_kernel,
                       dim3((words + kvip::kPcThreads - 1) / kvip::kPcThreads, cls->batch * cls->rows_per_request),
                       dim3(kvip::kPcThreads), 0, static_cast<hipStream_t>(stream), *cls, word_begin, word_end);
    return static_cast<uint32_t>(hipGetLastError());
}

extern "C" uint32_t kvip_hip_resident_prefix(const KvipTopkArgs* topk, const KvipPrefixClassifyArgs* cls, void* stream) {
    if (!kvip::prefix_args_ok(topk, cls)) return KVIP_ERR_INVALID;
    const KvipPrefixClassifyArgs& c = *cls;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = kvip::launch_topk(*topk, s);
    if (e != hipSuccess) return static_cast<uint32_t>(e);
    hipLaunchKernelGGL(kvip::prefix_classify_kernel, dim3(c.batch * c.rows_per_request), dim3(kvip::kPcThreads), 0, s,
                       c);
    if (c.cold_words > 0) {
        hipLaunchKernelGGL(kvip::cold_hits_kernel,
                           dim3((c.cold_words + kvip::kPcThreads - 1) / kvip::kPcThreads, c.batch * c.rows_per_request),
                           dim3(kvip::kPcThreads), 0, s, c, 0, c.cold_words);
    }
    return static_cast<uint32_t>(hipGetLastError());
}
