// LIDU (kvip.lidu) on gfx950: one batch transaction that classifies every TopK token of
// every query row against the request's resident maps, compacts misses first, dedups the
// request's misses, chooses their resident slots, clears the victims, installs the new
// mappings, refills the miss prefixes and writes the BatchGet descriptors.
//
// Reference: csrc/operators/lidu/op_kernel/a5_lidu_fused_batch_get_prepare_mtp.cpp
// (batch flow :674-813, layout :1111-1149, row validity :1290-1329, classify/compact
// :195-221 + :1381-1449, dedup :223-262 + :1986-2021, slot selection :1564-1741 with
// hot_slot_selection.h, validation :264-295 + :1743-1797, clear/install/refill :350-449,
// descriptors :451-545 + :2198-2261, batch outputs :2111-2196).
//
// Three launches: lidu_lookup_kernel gathers the token_to_slot entries of every TopK token
// (16 workgroups per request), then one 1024-thread workgroup per request in each of:
//   lidu_prepare_kernel reads the maps only. It checks the request's query range and
//     whether its pool row aliases an earlier request's, classifies its 1-4 TopK rows
//     (token_to_slot values from the lookup launch, membership bits in LDS), compacts them
//     with block scans, dedups the misses with LDS bitmaps over 2^18-token source tiles,
//     selects slots
//     (miss_slots, then a ring scan of the unprotected bitmap), validates them, writes the
//     hit suffixes, and leaves unique tokens, slots, miss prefixes and a control block in
//     the workspace.
//   lidu_commit_kernel forms the batch-wide layout verdict and the compact-descriptor
//     prefix from the per-request words, then clear -> install -> refill on the request's
//     own pool row, its descriptors and its per-row outputs.
// The reference separates clear from install with a launch-wide barrier so that two
// requests aliasing one pool row stay ordered. The layout check rejects every batch in
// which two non-padding requests share a pool row, and padding rows never touch the maps,
// so every request that installs owns its pool row and a workgroup barrier orders its
// phases.
//
// Dedup order: per source tile, per query, each query's new tokens in ascending token
// order. The reference assigns ordinals inside one query with atomics (its order there
// is not fixed); this is one of the orders it can produce.
#include "kvip_device.h"

namespace kvip {
namespace {

constexpr int kThreads = 1024;
constexpr int kMaxQueries = KVIP_LIDU_MAX_QUERIES;
constexpr int kMissCap = KVIP_LIDU_MISS_CAPACITY;
constexpr int kMaxCacheTokens = KVIP_LIDU_MAX_CACHE_TOKENS;
constexpr int kMaxSourceTokens = KVIP_LIDU_MAX_SOURCE_TOKENS;
constexpr int kBitmapWords = KVIP_LIDU_BITMAP_WORDS;
constexpr int kSourceTile = 1 << 18;
constexpr int kTileWords = kSourceTile / 32;
constexpr int kTileWordsPerThread = kTileWords / kThreads;  // 8
constexpr int kPackedRowBytes = KVIP_KV_ROW_BYTES;
constexpr int kProfileGraphDummy = 2;
constexpr int kProfileEnabled = 1;

constexpr int kOk = 0;
constexpr int kErrRowMetadata = -101;
constexpr int kErrTopkToken = -103;
constexpr int kErrUniqueCapacity = -106;
constexpr int kErrInsufficientSlots = -107;
constexpr int kErrDestinationSlot = -110;
constexpr int kErrResidentBlock = -111;

// Per-request workspace (int32 words): unique tokens, their slots, the compacted miss
// tokens of each query, then the control block.
constexpr int kWsUnique = 0;
constexpr int kWsSlots = kWsUnique + kMissCap;
constexpr int kWsMiss = kWsSlots + kMissCap;
constexpr int kWsCtrl = kWsMiss + kMaxQueries * kTopK;
constexpr int kWsWords = (kWsCtrl + 16 + 63) / 64 * 64;
enum Ctrl { kCtrlStatus, kCtrlUnique, kCtrlResolved, kCtrlCursor, kCtrlQ0, kCtrlQn, kCtrlMiss };

// Head: {layout_bad, live unique count} per request, ahead of the request blocks.
__host__ __device__ constexpr int64_t head_words(int batch) { return (2 * static_cast<int64_t>(batch) + 63) / 64 * 64; }

KVIP_DEVICE int32_t* request_ws(const KvipLiduArgs& p, int b) {
    return static_cast<int32_t*>(p.workspace) + head_words(p.batch) + static_cast<int64_t>(b) * kWsWords;
}

// Slot-table lookups of request b after the request blocks: token_to_slot of every TopK
// entry of its query rows [kMaxQueries][2048] (kNoLookup where the entry is not looked up).
constexpr int kNoLookup = INT32_MIN;
constexpr int kLookupThreads = 256;
constexpr int kLookupParts = kMaxQueries * kTopK / (2 * kLookupThreads);  // workgroups per request
KVIP_DEVICE int32_t* request_lookups(const KvipLiduArgs& p, int b) {
    return static_cast<int32_t*>(p.workspace) + head_words(p.batch) + static_cast<int64_t>(p.batch) * kWsWords +
           static_cast<int64_t>(b) * kMaxQueries * kTopK;
}

// Graph padding rows (:1303-1320): reserved pool entry, no resident budget, no source.
KVIP_DEVICE bool padding_row(const KvipLiduArgs& p, int r) {
    return p.cache_tokens[r] == 0 && p.candidate_lens[r] == 0 && p.logical_seq_lengths[r] == 1 &&
           p.req_pool_entries[r] == p.max_num_reqs;
}

KVIP_DEVICE void fill_rows(int32_t* dest, int64_t first_row, int64_t rows) {
    int4* d = reinterpret_cast<int4*>(dest + first_row * kTopK);
    const int64_t n = rows * (kTopK / 4);
    for (int64_t i = threadIdx.x; i < n; i += kThreads) d[i] = make_int4(-1, -1, -1, -1);
}

KVIP_DEVICE void stamp(const KvipLiduArgs& p, bool on, int b, int field) {
    if (on && threadIdx.x == 0) p.profiling[static_cast<int64_t>(b) * 8 * 32 + field] = static_cast<int64_t>(wall_clock64());
}

// Available slots of ordered word `o` of the ring scan [begin, budget) ++ [0, begin).
KVIP_DEVICE uint32_t ring_word(const uint32_t* protect, uint32_t o, uint32_t first_count, uint32_t begin,
                               uint32_t budget, uint32_t* word) {
    uint32_t w, seg_begin, seg_end;
    if (o < first_count) {
        w = begin / 32 + o;
        seg_begin = begin;
        seg_end = budget;
    } else {
        w = o - first_count;
        seg_begin = 0;
        seg_end = begin;
    }
    const uint32_t base = w * 32;
    uint32_t mask = ~0u;
    if (seg_begin > base) mask &= ~0u << (seg_begin - base);
    if (seg_end < base + 32) mask &= (1u << (seg_end - base)) - 1u;
    *word = w;
    return ~protect[w] & mask;
}

// The token_to_slot gathers of the classification, spread over kLookupParts workgroups per
// request (8192 scattered 4-byte reads per request are bound by one CU's outstanding misses
// when its prepare workgroup makes them). Workgroup L serves request
// (L / (8 * kLookupParts)) * 8 + L % 8, so that all of a request's lookups run on the XCD
// (L % 8) of its prepare and commit workgroups and leave the token_to_slot lines they read in
// that XCD's L2. Same query layout, validity and dummy-mode token substitution as the
// prepare pass, which reads the results only for requests it classifies.
__global__ __launch_bounds__(kLookupThreads) void lidu_lookup_kernel(const KvipLiduArgs p) {
    const int l = blockIdx.x;
    const int b = (l / (8 * kLookupParts)) * 8 + l % 8;
    const int part = (l / 8) % kLookupParts;
    if (b >= p.batch) return;
    const int q0 = b == 0 ? 0 : p.actual_seq_lengths_query[b - 1];
    const int q_end = p.actual_seq_lengths_query[b];
    const int qn = q_end - q0;
    if (q0 < 0 || q_end < q0 || q_end > p.packed_queries || qn < 1 || qn > kMaxQueries || padding_row(p, b)) return;
    const int pool = p.req_pool_entries[b];
    const int cand = p.candidate_lens[b];
    if (pool < 0 || pool >= p.pool_size || cand < 1 || cand > p.source_capacity) return;
    const int e = 2 * (part * kLookupThreads + static_cast<int>(threadIdx.x));  // pair of TopK entries
    if (e >= qn * kTopK) return;
    const bool dummy = p.profile_enabled[0] == kProfileGraphDummy;
    const int32_t* t2s = p.token_to_slot + static_cast<int64_t>(pool) * p.source_capacity;
    const int2 t2 = reinterpret_cast<const int2*>(p.topk + static_cast<int64_t>(q0) * kTopK)[e >> 1];
    int t[2] = {t2.x, t2.y};
    int m[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        if (dummy && (t[j] < 0 || t[j] >= cand)) t[j] = 0;
        m[j] = t[j] >= 0 && t[j] < cand ? t2s[t[j]] : kNoLookup;
    }
    reinterpret_cast<int2*>(request_lookups(p, b))[e >> 1] = make_int2(m[0], m[1]);
}

__global__ __launch_bounds__(kThreads) void lidu_prepare_kernel(const KvipLiduArgs p) {
    __shared__ uint32_t s_member[kBitmapWords];   // miss-slot membership (zero in graph-dummy mode)
    __shared__ uint32_t s_protect[kBitmapWords];  // membership | every hit slot (ring scan only)
    __shared__ int32_t s_miss[kMaxQueries][kTopK];
    __shared__ uint4 s_seen[kTileWords / 4];
    __shared__ uint4 s_cur[kTileWords / 4];       // reused as the slot list after dedup
    __shared__ uint32_t s_wave[kThreads / 64];

    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    int32_t* ws = request_ws(p, b);
    int32_t* ctrl = ws + kWsCtrl;
    int32_t* head = static_cast<int32_t*>(p.workspace) + 2 * b;
    const bool profile = p.profiling != nullptr && p.profile_enabled[0] == kProfileEnabled;
    if (profile) {
        for (int i = tid; i < 8 * 32; i += kThreads) p.profiling[static_cast<int64_t>(b) * 8 * 32 + i] = 0;
    }
    stamp(p, profile, b, 0);

    // Query layout of this row and pool-row aliasing with earlier rows (:1111-1149).
    const int q0 = b == 0 ? 0 : p.actual_seq_lengths_query[b - 1];
    const int q_end = p.actual_seq_lengths_query[b];
    const int qn = q_end - q0;
    const bool pad = padding_row(p, b);
    const int pool = p.req_pool_entries[b];
    int alias = 0;
    for (int r = tid; r < b; r += kThreads) {
        alias |= (p.req_pool_entries[r] == pool && !(pad && padding_row(p, r))) ? 1 : 0;
    }
    const bool layout_bad =
        q0 < 0 || q_end < q0 || q_end > p.packed_queries || (qn < 1 && !pad) || qn > kMaxQueries;
    if (__syncthreads_or(alias) || layout_bad) {
        if (tid == 0) {
            head[0] = 1;
            head[1] = 0;
        }
        return;
    }

    const int budget = p.cache_tokens[b];
    const int cand = p.candidate_lens[b];
    const bool valid = budget >= kTopK && budget <= kMaxCacheTokens && budget <= p.resident_capacity &&
                       cand >= kTopK && cand <= p.source_capacity && (cand + 127) / 128 <= p.qcap &&
                       (budget + 127) / 128 <= p.resident_blocks && pool >= 0 && pool < p.pool_size &&
                       pool < p.max_num_reqs;
    if (pad || !valid) {
        fill_rows(p.destination_slots, q0, qn);
        if (tid == 0) {
            ctrl[kCtrlStatus] = pad ? kOk : kErrRowMetadata;
            ctrl[kCtrlUnique] = 0;
            ctrl[kCtrlResolved] = 0;
            ctrl[kCtrlCursor] = -1;
            ctrl[kCtrlQ0] = q0;
            ctrl[kCtrlQn] = qn;
            head[0] = 0;
            head[1] = 0;
        }
        return;
    }

    // Classification (:195-221, :1381-1449).
    const bool dummy = p.profile_enabled[0] == kProfileGraphDummy;
    const uint32_t* bitmap = reinterpret_cast<const uint32_t*>(p.miss_slot_bitmap) + static_cast<int64_t>(b) * kBitmapWords;
    for (int i = tid; i < kBitmapWords; i += kThreads) {
        s_member[i] = dummy ? 0u : bitmap[i];
    }
    for (int i = tid; i < kTileWords / 4; i += kThreads) s_cur[i] = make_uint4(0, 0, 0, 0);
    __syncthreads();

    // token_to_slot values from the lookup launch (lidu_lookup_kernel).
    const int32_t* looked = request_lookups(p, b);
    int tok[kMaxQueries][2], slot[kMaxQueries][2];
    int2 lk[kMaxQueries];
#pragma unroll
    for (int q = 0; q < kMaxQueries; ++q) {
        int2 v = make_int2(0, 0);
        lk[q] = make_int2(kNoLookup, kNoLookup);
        if (q < qn) {
            v = reinterpret_cast<const int2*>(p.topk + static_cast<int64_t>(q0 + q) * kTopK)[tid];
            lk[q] = reinterpret_cast<const int2*>(looked + q * kTopK)[tid];
        }
        tok[q][0] = v.x;
        tok[q][1] = v.y;
    }
#pragma unroll
    for (int q = 0; q < kMaxQueries; ++q) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            int t = tok[q][j];
            if (dummy && (t < 0 || t >= cand)) t = 0;
            tok[q][j] = t;
            int s = -1;
            if (q < qn && t >= 0 && t < cand) {
                const int m = j == 0 ? lk[q].x : lk[q].y;
                if (m >= 0 && m < budget && !((s_member[m >> 5] >> (m & 31)) & 1u)) s = m;
            }
            slot[q][j] = s;
        }
    }
    // Miss positions: one block scan per query pair, the two queries' counts in the 16-bit
    // halves of one word (each total is at most 2048).
    int pos[kMaxQueries][2];
    int miss_count[kMaxQueries];
    int bad_token = 0;
#pragma unroll
    for (int h = 0; h < kMaxQueries / 2; ++h) {
        if (2 * h >= qn) {
            miss_count[2 * h] = miss_count[2 * h + 1] = 0;
            continue;
        }
        uint32_t packed = 0;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int q = 2 * h + k;
            const uint32_t misses = q < qn ? (slot[q][0] < 0 ? 1u : 0u) + (slot[q][1] < 0 ? 1u : 0u) : 0u;
            packed |= misses << (16 * k);
        }
        uint32_t totals;
        const uint32_t pres = block_exclusive_scan(packed, s_wave, &totals);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int q = 2 * h + k;
            const uint32_t pre = (pres >> (16 * k)) & 0xFFFFu;
            const uint32_t total = (totals >> (16 * k)) & 0xFFFFu;
            miss_count[q] = q < qn ? static_cast<int>(total) : 0;
            if (q >= qn) continue;
            const uint32_t m0 = slot[q][0] < 0 ? 1u : 0u;
            const int i0 = 2 * tid;
            pos[q][0] = m0 ? pre : total + (i0 - pre);
            pos[q][1] = slot[q][1] < 0 ? pre + m0 : total + (i0 + 1 - pre - m0);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (slot[q][j] < 0) {
                    s_miss[q][pos[q][j]] = tok[q][j];
                    bad_token |= (tok[q][j] < 0 || tok[q][j] >= cand) ? 1 : 0;
                }
            }
        }
    }
    int status = __syncthreads_or(bad_token) ? kErrTopkToken : kOk;
    stamp(p, profile, b, 1);

    // Dedup over source tiles, queries in order (:1986-2021).
    uint32_t unique = 0;
    int32_t* ws_unique = ws + kWsUnique;
    const int any_miss = miss_count[0] + miss_count[1] + miss_count[2] + miss_count[3];
    if (status == kOk && any_miss > 0) {
        for (int tile = 0; tile < cand; tile += kSourceTile) {
            int here = 0;
#pragma unroll
            for (int q = 0; q < kMaxQueries; ++q) {  // miss_count[q] == 0 for q >= qn
                for (int i = tid; i < miss_count[q]; i += kThreads) {
                    const int t = s_miss[q][i];
                    here |= (t >= tile && t - tile < kSourceTile) ? 1 : 0;
                }
            }
            if (!__syncthreads_or(here)) continue;
            s_seen[2 * tid] = make_uint4(0, 0, 0, 0);
            s_seen[2 * tid + 1] = make_uint4(0, 0, 0, 0);
            __syncthreads();
#pragma unroll
            for (int q = 0; q < kMaxQueries; ++q) {
                if (miss_count[q] == 0) continue;
                for (int i = tid; i < miss_count[q]; i += kThreads) {
                    const int t = s_miss[q][i];
                    if (t >= tile && t - tile < kSourceTile) {
                        atomicOr(reinterpret_cast<uint32_t*>(s_cur) + ((t - tile) >> 5), 1u << (t & 31));
                    }
                }
                __syncthreads();
                uint32_t fresh[kTileWordsPerThread];
                uint32_t count = 0;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint4 c = s_cur[2 * tid + h];
                    uint4 s = s_seen[2 * tid + h];
                    fresh[4 * h + 0] = c.x & ~s.x;
                    fresh[4 * h + 1] = c.y & ~s.y;
                    fresh[4 * h + 2] = c.z & ~s.z;
                    fresh[4 * h + 3] = c.w & ~s.w;
                    s.x |= c.x;
                    s.y |= c.y;
                    s.z |= c.z;
                    s.w |= c.w;
                    s_seen[2 * tid + h] = s;
                    s_cur[2 * tid + h] = make_uint4(0, 0, 0, 0);
                }
#pragma unroll
                for (int j = 0; j < kTileWordsPerThread; ++j) count += __popc(fresh[j]);
                uint32_t total;
                uint32_t o = unique + block_exclusive_scan(count, s_wave, &total);
#pragma unroll
                for (int j = 0; j < kTileWordsPerThread; ++j) {
                    uint32_t bits = fresh[j];
                    const int word_token = tile + (tid * kTileWordsPerThread + j) * 32;
                    while (bits) {
                        if (o < static_cast<uint32_t>(kMissCap)) ws_unique[o] = word_token + __ffs(bits) - 1;
                        ++o;
                        bits &= bits - 1;
                    }
                }
                unique += total;
            }
        }
    }
    if (status == kOk && unique > static_cast<uint32_t>(kMissCap)) status = kErrUniqueCapacity;
    stamp(p, profile, b, 2);

    // Slot selection (:1564-1741): miss_slots first, then the ring scan from the cursor.
    __syncthreads();  // the last dedup pass is done with s_cur
    int32_t* s_slots = reinterpret_cast<int32_t*>(s_cur);
    int resolved = 0, cursor = -1;
    if (status == kOk && unique > 0) {
        const int n_in = min(static_cast<int>(unique), kTopK);
        const int32_t* preferred = p.miss_slots + static_cast<int64_t>(b) * kTopK;
        for (int i = tid; i < n_in; i += kThreads) s_slots[i] = preferred[i];
        if (unique > static_cast<uint32_t>(kTopK)) {
            // Slots the scan must skip: membership and every hit slot.
            for (int i = tid; i < kBitmapWords; i += kThreads) s_protect[i] = s_member[i];
            __syncthreads();
#pragma unroll
            for (int q = 0; q < kMaxQueries; ++q) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    if (q < qn && slot[q][j] >= 0) atomicOr(&s_protect[slot[q][j] >> 5], 1u << (slot[q][j] & 31));
                }
            }
            __syncthreads();
            const uint32_t extra = unique - kTopK;
            const int cursor_in = p.eviction_cursors[pool];
            const uint32_t ubudget = static_cast<uint32_t>(budget);
            const uint32_t begin = cursor_in >= 0 ? static_cast<uint32_t>(cursor_in) % ubudget : 0u;
            const uint32_t first_count = (ubudget - 1) / 32 - begin / 32 + 1;
            const uint32_t second_count = begin ? (begin - 1) / 32 + 1 : 0u;
            const uint32_t ordered = first_count + second_count;
            const uint32_t per = (ordered + kThreads - 1) / kThreads;
            uint32_t count = 0, w;
            for (uint32_t k = 0; k < per; ++k) {
                const uint32_t o = tid * per + k;
                if (o < ordered) count += __popc(ring_word(s_protect, o, first_count, begin, ubudget, &w));
            }
            uint32_t total;
            uint32_t at = block_exclusive_scan(count, s_wave, &total);
            if (total >= extra) {
                for (uint32_t k = 0; k < per && at < extra; ++k) {
                    const uint32_t o = tid * per + k;
                    if (o >= ordered) break;
                    uint32_t bits = ring_word(s_protect, o, first_count, begin, ubudget, &w);
                    while (bits && at < extra) {
                        s_slots[kTopK + at] = static_cast<int>(w * 32 + __ffs(bits) - 1);
                        ++at;
                        bits &= bits - 1;
                    }
                }
                resolved = 1;
            } else {
                status = kErrInsufficientSlots;
            }
            __syncthreads();
            if (resolved) {
                const int last = s_slots[kTopK + extra - 1];
                cursor = last + 1 == budget ? 0 : last + 1;
            }
        }
    }
    __syncthreads();

    // Destination validation (:1743-1797).
    if (status == kOk && unique > 0) {
        const int32_t* blocks = p.resident_block_table + static_cast<int64_t>(b) * p.resident_blocks;
        int bad_slot = 0, bad_block = 0;
        for (int i = tid; i < static_cast<int>(unique); i += kThreads) {
            const int s = s_slots[i];
            if (s < 0 || s >= budget || (s >> 7) >= p.resident_blocks) {
                bad_slot = 1;
            } else {
                const int pb = blocks[s >> 7];
                bad_block |= (pb < 0 || pb > 0x7FFFFFFF / kBlockTokens) ? 1 : 0;
            }
        }
        bad_slot = __syncthreads_or(bad_slot);
        bad_block = __syncthreads_or(bad_block);
        status = bad_slot ? kErrDestinationSlot : (bad_block ? kErrResidentBlock : kOk);
    }

    // Outputs of the prepare pass: hit suffixes (the miss prefixes are refilled after
    // install), miss prefixes, slots and the control block for the commit pass.
    const bool live = status == kOk && unique > 0 && unique <= static_cast<uint32_t>(kMissCap);
    if (status == kOk) {
        int32_t* dest = p.destination_slots + static_cast<int64_t>(q0) * kTopK;
        int32_t* ws_miss = ws + kWsMiss;
#pragma unroll
        for (int q = 0; q < kMaxQueries; ++q) {
            if (q >= qn) continue;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (slot[q][j] >= 0) {
                    dest[q * kTopK + pos[q][j]] = slot[q][j];
                } else if (live) {
                    ws_miss[q * kTopK + pos[q][j]] = tok[q][j];
                }
            }
        }
    } else {
        fill_rows(p.destination_slots, q0, qn);
    }
    if (live) {
        int32_t* ws_slots = ws + kWsSlots;
        for (int i = tid; i < static_cast<int>(unique); i += kThreads) ws_slots[i] = s_slots[i];
    }
    if (tid == 0) {
        ctrl[kCtrlStatus] = status;
        ctrl[kCtrlUnique] = static_cast<int>(unique);
        ctrl[kCtrlResolved] = status == kOk ? resolved : 0;
        ctrl[kCtrlCursor] = cursor;
        ctrl[kCtrlQ0] = q0;
        ctrl[kCtrlQn] = qn;
        for (int q = 0; q < kMaxQueries; ++q) ctrl[kCtrlMiss + q] = miss_count[q];
        head[0] = 0;
        head[1] = live ? static_cast<int>(unique) : 0;
    }
    stamp(p, profile, b, 3);
}

__global__ __launch_bounds__(kThreads) void lidu_commit_kernel(const KvipLiduArgs p) {
    __shared__ uint32_t s_wave[kThreads / 64];
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const bool profile = p.profiling != nullptr && p.profile_enabled[0] == kProfileEnabled;
    stamp(p, profile, b, 4);
    const int2* head = static_cast<const int2*>(p.workspace);
    int bad = 0;
    uint32_t before = 0;
    for (int r = tid; r < p.batch; r += kThreads) {
        const int2 h = head[r];
        bad |= h.x;
        if (r < b) before += static_cast<uint32_t>(h.y);
    }
    bad = __syncthreads_or(bad);
    uint32_t prefix;
    block_exclusive_scan(before, s_wave, &prefix);

    if (bad) {  // the whole batch is rejected (:686-696)
        const int64_t r0 = static_cast<int64_t>(b) * p.packed_queries / p.batch;
        const int64_t r1 = static_cast<int64_t>(b + 1) * p.packed_queries / p.batch;
        fill_rows(p.destination_slots, r0, r1 - r0);
        if (tid == 0) {
            p.miss_counts[b] = -1;
            p.resident_seq_lengths[b] = 0;
            if (b == p.batch - 1) p.miss_counts[p.batch] = 0;
        }
        return;
    }

    const int32_t* ws = request_ws(p, b);
    const int32_t* ctrl = ws + kWsCtrl;
    const int status = ctrl[kCtrlStatus];
    const int unique = ctrl[kCtrlUnique];
    const int live = head[b].y;
    const int pool = p.req_pool_entries[b];
    const int budget = p.cache_tokens[b];
    const int cand = p.candidate_lens[b];
    if (live > 0) {
        int32_t* t2s = p.token_to_slot + static_cast<int64_t>(pool) * p.source_capacity;
        int32_t* s2t = p.slot_to_token + static_cast<int64_t>(pool) * p.resident_capacity;
        const int32_t* ws_unique = ws + kWsUnique;
        const int32_t* ws_slots = ws + kWsSlots;
        // Clear the victims of every destination slot (:350-386).
        for (int i = tid; i < live; i += kThreads) {
            const int s = ws_slots[i];
            if (s < 0 || s >= p.resident_capacity) continue;
            const int victim = s2t[s];
            if (victim >= 0 && victim < cand && t2s[victim] == s) t2s[victim] = -1;
        }
        __syncthreads();
        stamp(p, profile, b, 5);
        // Install (:388-424).
        for (int i = tid; i < live; i += kThreads) {
            const int t = ws_unique[i];
            const int s = ws_slots[i];
            if (s < 0 || s >= p.resident_capacity) continue;
            if (t >= 0 && t < cand) t2s[t] = s;
            if (s < budget) s2t[s] = t;
        }
        __syncthreads();
        stamp(p, profile, b, 6);
        // Refill the miss prefixes through the installed forward map (:426-449).
        const int q0 = ctrl[kCtrlQ0];
        const int qn = ctrl[kCtrlQn];
        const int32_t* ws_miss = ws + kWsMiss;
        for (int q = 0; q < qn; ++q) {
            const int n = ctrl[kCtrlMiss + q];
            int32_t* dest = p.destination_slots + static_cast<int64_t>(q0 + q) * kTopK;
            for (int i = tid; i < n; i += kThreads) dest[i] = t2s[ws_miss[q * kTopK + i]];
        }
        stamp(p, profile, b, 7);
        // Compact BatchGet descriptors at this request's prefix (:451-545).
        const uint32_t layer_base =
            static_cast<uint32_t>((static_cast<uint64_t>(pool) * p.num_layers + p.layer_id) * p.qcap);
        const int32_t* blocks = p.resident_block_table + static_cast<int64_t>(b) * p.resident_blocks;
        for (int c = tid; c < live; c += kThreads) {
            const int64_t o = static_cast<int64_t>(prefix) + c;
            const uint32_t t = static_cast<uint32_t>(ws_unique[c]);
            const uint32_t s = static_cast<uint32_t>(ws_slots[c]);
            p.indices[o] = static_cast<int32_t>(layer_base + (t >> 7));
            p.offsets[o] = static_cast<int32_t>((t & 127u) * kPackedRowBytes);
            int out = -1;
            if (s < static_cast<uint32_t>(p.resident_capacity) && (s >> 7) < static_cast<uint32_t>(p.resident_blocks)) {
                const int pb = blocks[s >> 7];
                if (pb >= 0 && pb <= 0x7FFFFFFF / kBlockTokens) out = pb * kBlockTokens + static_cast<int>(s & 127u);
            }
            p.output_indices[o] = out;
        }
    }
    if (tid == 0) {
        const bool ok = status == kOk;
        p.miss_counts[b] = ok ? unique : -1;
        int resident = 0;
        if (ok) {
            const int logical = p.logical_seq_lengths[b];
            if (budget >= kTopK && cand >= kTopK && logical >= cand) {
                resident = static_cast<int>(static_cast<uint32_t>(budget) + static_cast<uint32_t>(logical) -
                                            static_cast<uint32_t>(cand));
            } else if (budget == 0 && logical >= 0) {
                resident = logical;
            }
        }
        p.resident_seq_lengths[b] = resident;
        if (ok && ctrl[kCtrlResolved] && pool >= 0 && ctrl[kCtrlCursor] >= 0) p.eviction_cursors[pool] = ctrl[kCtrlCursor];
        if (b == p.batch - 1) p.miss_counts[p.batch] = static_cast<int>(prefix) + live;
    }
    stamp(p, profile, b, 8);
}

}  // namespace
}  // namespace kvip

extern "C" uint64_t kvip_hip_lidu_workspace_bytes(int32_t batch) {
    if (batch < 1) return 0;
    return static_cast<uint64_t>(kvip::head_words(batch) +
                                 static_cast<int64_t>(batch) * (kvip::kWsWords + kvip::kMaxQueries * kvip::kTopK)) *
           4u;
}

extern "C" uint32_t kvip_hip_lidu(const KvipLiduArgs* a, void* stream) {
    if (a == nullptr || a->topk == nullptr || a->actual_seq_lengths_query == nullptr ||
        a->req_pool_entries == nullptr || a->token_to_slot == nullptr || a->slot_to_token == nullptr ||
        a->eviction_cursors == nullptr || a->cache_tokens == nullptr || a->candidate_lens == nullptr ||
        a->miss_slots == nullptr || a->miss_slot_bitmap == nullptr || a->resident_block_table == nullptr ||
        a->logical_seq_lengths == nullptr || a->profile_enabled == nullptr || a->destination_slots == nullptr ||
        a->miss_counts == nullptr || a->indices == nullptr || a->offsets == nullptr ||
        a->output_indices == nullptr || a->resident_seq_lengths == nullptr || a->workspace == nullptr) {
        return KVIP_ERR_INVALID;
    }
    // Shape and geometry checks of the reference host op
    // (torch_extension/csrc/lidu_fused_batch_get_prepare_mtp_ops.cpp:41-130).
    const int64_t batch = a->batch;
    if (batch < 1 || batch > 65535 || a->packed_queries < batch ||
        a->packed_queries > batch * kvip::kMaxQueries || a->pool_size < 1 || a->source_capacity < 1 ||
        a->source_capacity > kvip::kMaxSourceTokens || a->resident_capacity < kvip::kTopK ||
        a->resident_blocks < 1 || a->layer_id < 0 || a->num_layers < 1 || a->layer_id >= a->num_layers ||
        a->max_num_reqs < batch || a->qcap < 1 ||
        static_cast<uint64_t>(a->max_num_reqs) * static_cast<uint64_t>(a->num_layers) *
                static_cast<uint64_t>(a->qcap) > 0x7FFFFFFFull ||
        static_cast<uint64_t>(a->resident_blocks) * kvip::kBlockTokens > 0x7FFFFFFFull ||
        a->workspace_bytes < static_cast<int64_t>(kvip_hip_lidu_workspace_bytes(a->batch))) {
        return KVIP_ERR_INVALID;
    }
    // Vector accesses: int2 TopK loads, int4 row fills, int2 workspace head reads.
    if ((reinterpret_cast<uintptr_t>(a->topk) & 7) || (reinterpret_cast<uintptr_t>(a->destination_slots) & 15) ||
        (reinterpret_cast<uintptr_t>(a->workspace) & 15)) {
        return KVIP_ERR_INVALID;
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(kvip::lidu_lookup_kernel, dim3((a->batch + 7) / 8 * 8 * kvip::kLookupParts),
                       dim3(kvip::kLookupThreads), 0, s, *a);
    hipLaunchKernelGGL(kvip::lidu_prepare_kernel, dim3(a->batch), dim3(kvip::kThreads), 0, s, *a);
    hipLaunchKernelGGL(kvip::lidu_commit_kernel, dim3(a->batch), dim3(kvip::kThreads), 0, s, *a);
    return static_cast<uint32_t>(hipGetLastError());
}
