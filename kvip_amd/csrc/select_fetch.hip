// TopK-2048 fused with the Fetch gather, for rows scored by kvip_hip_indexer_decode.
//
// Grid = kParts x rows of 1024-thread workgroups; every workgroup of a row computes the
// row's whole selection from register-resident keys and then gathers only its quarter of
// the output positions:
//   1. the row's keys are loaded once (KPT consecutive keys per thread) together with
//      the scoring kernel's high-byte histogram, which gives the high byte hb of the
//      2048th largest key;
//   2. a low-byte histogram of the keys in bin hb gives the kth key and n_gt (keys above
//      it);
//   3. per-32-key bitmasks of (keys > kth, keys == kth), their popcounts scanned over the
//      workgroup in token order, place every selected token: keys > kth at [0, n_gt) in
//      token order, then the first 2048 - n_gt keys == kth in token order (select_row.h);
//   4. the tokens whose positions fall in this workgroup's quarter go to an LDS list
//      indexed by position, are written to the TopK output and their KV rows gathered
//      into output[row, position, :].
// The selection is the one kvip_hip_topk computes. The parts of a row never wait for one
// another: the only shared state is a per-row ticket, taken at the end by each part; the
// part holding the last ticket clears the histogram (read by every part at its start) for
// the next scoring launch and resets the ticket.
//
// Reference: QLIVector::ProcessTopK (op_kernel/indexer/indexer_vector.h:799-973) with
// LITopk's GT-then-EQ emission (topk.h:155-187, topk_common.h:1000-1067) followed by
// the Fetch gather (FetchQueryGroup, op_kernel/streaming.cpp:365-500; KV row layout
// tests/operators/lifetch/support/workloads.py:493-515).
#include "kvip_device.h"
#include "select_row.h"

namespace kvip {
uint32_t validate_topk(const KvipTopkArgs* a);
uint32_t validate_fetch(const KvipFetchArgs* a);

namespace {

constexpr int kSgThreads = 1024;
constexpr int kSgWaves = kSgThreads / 64;
constexpr int kParts = 4;                          // workgroups per row
constexpr int kPartRows = kTopK / kParts;          // 512 output positions per part
constexpr int kGatherRows = 16;                    // rows per wave and pass
constexpr int kTicketWord = KVIP_TOPK_SEGMENT_WORDS - 1;  // of the row's first segment record
constexpr int kMaxFusedKeys = kSgThreads * 32;     // 32768
static_assert(kPartRows % (kSgWaves * kGatherRows) == 0, "whole gather passes");

KVIP_DEVICE int sg_row_valid(const KvipTopkArgs& p, int row) { return topk_row_valid(p, row); }

// Byte offset of the KV row of `token` of request b in the paged cache, or -1 for an
// empty entry or an id outside the block table / cache (reported in err).
KVIP_DEVICE int64_t kv_source(const KvipFetchArgs& f, int b, int token, uint32_t& err) {
    if (token < 0) return -1;
    if (token >= f.max_blocks * kBlockTokens) {
        err |= KVIP_STATUS_BAD_TOKEN;
        return -1;
    }
    const int blk = f.block_table[static_cast<size_t>(b) * f.max_blocks + (token >> 7)];
    if (static_cast<unsigned>(blk) >= static_cast<unsigned>(f.num_blocks)) {
        err |= KVIP_STATUS_BAD_BLOCK;
        return -1;
    }
    return static_cast<int64_t>(blk) * f.kv_block_stride + static_cast<int64_t>(token & 127) * f.row_stride;
}

// One wave moves list entries [e0, e0 + 16): the KV row of token s_tok[e] goes to
// out_rows + e * row_bytes (zeros for token -1). Lanes 0..15 translate the entries,
// then all 64 lanes move the 16-byte pieces with every load of the pass in flight
// before the first store. Called by whole waves.
template <int PIECES>
KVIP_DEVICE void gather_pass(const KvipFetchArgs& f, int b, uint8_t* out_rows, const int32_t* s_tok, int e0,
                             uint32_t& err) {
    const int lane = lane_id();
    const int pieces = PIECES > 0 ? PIECES : f.row_bytes / 16;
    int64_t src = -1;
    if (lane < kGatherRows) src = kv_source(f, b, s_tok[e0 + lane], err);
    uint8_t* dst = out_rows + static_cast<size_t>(e0) * f.row_bytes;  // 16 consecutive output rows
    const int total = kGatherRows * pieces;
    if constexpr (PIECES > 0) {
        constexpr int kIters = (kGatherRows * PIECES + 63) / 64;
        v4i val[kIters];
#pragma unroll
        for (int it = 0; it < kIters; ++it) {
            const int idx = it * 64 + lane;
            const int r = idx / PIECES;
            const int piece = idx - r * PIECES;
            const int64_t base = __shfl(src, min(r, kGatherRows - 1));
            val[it] = v4i{0, 0, 0, 0};
            if (idx < total && base >= 0) {
                val[it] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(f.kv_cache + base + piece * 16));
            }
        }
#pragma unroll
        for (int it = 0; it < kIters; ++it) {
            const int idx = it * 64 + lane;
            if (idx < total) *reinterpret_cast<v4i*>(dst + static_cast<size_t>(idx) * 16) = val[it];
        }
    } else {
        const int iters = (total + 63) / 64;  // uniform: every lane joins each shuffle
        for (int it = 0; it < iters; ++it) {
            const int idx = it * 64 + lane;
            const int r = idx / pieces;
            const int piece = idx - r * pieces;
            const int64_t base = __shfl(src, min(r, kGatherRows - 1));
            v4i v = v4i{0, 0, 0, 0};
            if (idx < total && base >= 0) v = *reinterpret_cast<const v4i*>(f.kv_cache + base + piece * 16);
            if (idx < total) *reinterpret_cast<v4i*>(dst + static_cast<size_t>(idx) * 16) = v;
        }
    }
}

template <int KPT, int PIECES>
__global__ __launch_bounds__(kSgThreads) void select_gather_kernel(const KvipTopkArgs p, const KvipFetchArgs f) {
    constexpr int W = KPT / 2;  // packed key registers per thread
    __shared__ __align__(16) uint32_t s_hist[256];
    __shared__ uint32_t s_wave[kSgWaves];
    __shared__ int s_last;
    __shared__ __align__(16) int32_t s_tok[kPartRows];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int part = blockIdx.x;
    const int row = blockIdx.y;
    const int b = row / p.rows_per_request;
    const int valid = min(sg_row_valid(p, row), kSgThreads * KPT);
    const int pos0 = part * kPartRows;
    int32_t* out = p.topk + static_cast<size_t>(row) * kTopK;
    uint8_t* out_rows = f.output + (static_cast<size_t>(row) * kTopK + pos0) * f.row_bytes;
    uint32_t* hist_g = p.histogram + static_cast<size_t>(row) * 256;
    uint32_t err = 0;

    if (valid < kTopK) {
        // Short row: every token in order, then -1 (zero rows).
        if (part == 0 && tid < 256) hist_g[tid] = 0u;  // no other part reads it
        for (int i = tid; i < kPartRows; i += kSgThreads) s_tok[i] = pos0 + i < valid ? pos0 + i : -1;
    } else {
        // Step 1: keys (unconditional 16-byte loads clamped into the row; keys past
        // `valid` are masked by `count`) and the high-byte bin.
        const int first = tid * KPT;
        const int count = max(0, min(KPT, valid - first));
        const uint16_t* keys = p.score_keys + static_cast<size_t>(row) * p.key_stride;
        uint32_t kk[W];
#pragma unroll
        for (int v = 0; v < W / 4; ++v) {
            const v4i x = *reinterpret_cast<const v4i*>(keys + min(first + v * 8, p.key_stride - 8));
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                // Keys past `valid` read as 0 (mask from the word's count of live keys).
                const int live = min(max(count - (v * 8 + w * 2), 0), 2);
                kk[4 * v + w] = static_cast<uint32_t>(x[w]) & static_cast<uint32_t>((1ull << (16 * live)) - 1ull);
            }
        }
        // Every wave reads the whole high-byte histogram (4 bins per lane) and finds the bin
        // of the 2048th largest key on its own.
        const v4i hv = *reinterpret_cast<const v4i*>(hist_g + lane_id() * 4);
        if (tid < 256) s_hist[tid] = 0u;
        for (int i = tid; i < kPartRows; i += kSgThreads) s_tok[i] = -1;  // positions nobody claims stay empty
        const uint32_t h[4] = {static_cast<uint32_t>(hv[0]), static_cast<uint32_t>(hv[1]),
                               static_cast<uint32_t>(hv[2]), static_cast<uint32_t>(hv[3])};
        int hb;
        uint32_t gt_hi;
        wave_select_bin(h, kTopK, hb, gt_hi);
        __syncthreads();
        // Steps 2-4: the tokens whose positions fall in this part's quarter go to s_tok.
        const RowSelection sel = select_row<KPT>(kk, count, first, hb, gt_hi, s_hist, s_wave, [&](int pos, int tok) {
            const uint32_t rel = static_cast<uint32_t>(pos - pos0);
            if (rel < static_cast<uint32_t>(kPartRows)) s_tok[rel] = tok;
        });
        if (part == 0 && tid == 0 && !sel.ok) err |= KVIP_STATUS_HISTOGRAM;
    }
    __syncthreads();
    // TopK output of this part (coalesced), then the gather.
    for (int i = tid; i < kPartRows; i += kSgThreads) out[pos0 + i] = s_tok[i];
#pragma unroll
    for (int pass = 0; pass < kPartRows / (kSgWaves * kGatherRows); ++pass) {
        gather_pass<PIECES>(f, b, out_rows, s_tok, pass * kSgWaves * kGatherRows + wave * kGatherRows, err);
    }
    report(p.status, err);
    // Ticket, off the critical path: every part read the histogram at its start; the part
    // holding the last ticket clears it for the next scoring launch.
    if (valid >= kTopK) {
        if (tid == 0) {
            const size_t segs = (static_cast<size_t>(p.key_stride) + KVIP_TOPK_SEGMENT_KEYS - 1) / KVIP_TOPK_SEGMENT_KEYS;
            uint32_t* ticket = p.segments + static_cast<size_t>(row) * segs * KVIP_TOPK_SEGMENT_WORDS + kTicketWord;
            const uint32_t old = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = old == kParts - 1 ? 1 : 0;
            if (old == kParts - 1) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (s_last && tid < 256) hist_g[tid] = 0u;
    }
}

template <int PIECES>
hipError_t launch_pieces(const KvipTopkArgs& t, const KvipFetchArgs& f, hipStream_t stream) {
    const dim3 grid(kParts, t.batch * t.rows_per_request);
    const dim3 block(kSgThreads);
    if (t.key_stride <= kSgThreads * 8) {
        hipLaunchKernelGGL((select_gather_kernel<8, PIECES>), grid, block, 0, stream, t, f);
    } else if (t.key_stride <= kSgThreads * 16) {
        hipLaunchKernelGGL((select_gather_kernel<16, PIECES>), grid, block, 0, stream, t, f);
    } else {
        hipLaunchKernelGGL((select_gather_kernel<32, PIECES>), grid, block, 0, stream, t, f);
    }
    return hipGetLastError();
}

}  // namespace

uint32_t validate_select_fetch(const KvipTopkArgs* t, const KvipFetchArgs* f) {
    if (validate_topk(t) != KVIP_OK || validate_fetch(f) != KVIP_OK) return KVIP_ERR_INVALID;
    const int64_t rows = static_cast<int64_t>(t->batch) * t->rows_per_request;
    const bool ok = t->histogram != nullptr && t->segments != nullptr && rows <= 65535 && t->limit == 0 &&
                    t->key_stride <= kMaxFusedKeys && f->topk == t->topk && f->batch == t->batch &&
                    f->rows_per_request == t->rows_per_request &&
                    (reinterpret_cast<uintptr_t>(t->segments) & 3u) == 0;
    return ok ? KVIP_OK : KVIP_ERR_INVALID;
}

hipError_t launch_select_fetch(const KvipTopkArgs& t, const KvipFetchArgs& f, hipStream_t stream) {
    return f.row_bytes == KVIP_KV_ROW_BYTES ? launch_pieces<KVIP_KV_ROW_BYTES / 16>(t, f, stream)
                                            : launch_pieces<0>(t, f, stream);
}

}  // namespace kvip

extern "C" uint32_t kvip_hip_select_fetch(const KvipTopkArgs* topk, const KvipFetchArgs* fetch, void* stream) {
    if (topk == nullptr || fetch == nullptr) return KVIP_ERR_INVALID;
    const uint32_t rc = kvip::validate_select_fetch(topk, fetch);
    if (rc != KVIP_OK) return rc;
    return static_cast<uint32_t>(kvip::launch_select_fetch(*topk, *fetch, static_cast<hipStream_t>(stream)));
}
