// Exact TopK-2048 over sortable uint16 score keys, one 1024-thread workgroup per
// query row, as a two-level radix select:
//   1. high-byte histogram (taken from the scoring kernel, or built here) -> the bin
//      that holds the 2048th largest key;
//   2. low-byte histogram of the keys in that bin -> the kth key K and the number of
//      keys strictly above it (n_gt);
//   3. one ordered emission pass: keys > K in ascending token order, then the first
//      2048 - n_gt keys == K in ascending token order.
// The selected set equals the first 2048 entries of the order (key desc, token asc),
// which is what the reference's trunked GT-then-EQ select with prior-winner-first
// merging produces (op_kernel/indexer/topk.h:155-187, topk_common.h:1000-1067,
// :1094-1122). Row bounds follow QLIVector::ProcessTopK
// (op_kernel/indexer/indexer_vector.h:849-873, :943-957): valid <= 0 -> all -1,
// valid < 2048 -> [0..valid-1, -1...].
#include "kvip_device.h"
#include "select_row.h"

namespace kvip {
namespace {

constexpr int kTopkThreads = 1024;
constexpr int kKeysPerThread = 8;
constexpr int kTileKeys = kTopkThreads * kKeysPerThread;
static_assert(KVIP_TOPK_REGS_MAX_KEYS == kTopkThreads * 64, "largest register-resident row");

struct Keys8 {
    uint32_t k[kKeysPerThread];
    int count;  // keys of this thread below `valid`
};

// Keys [idx0, idx0+8) of a row with `stride` keys; positions >= valid are masked by
// `count`. The 16-byte load is unconditional with its start clamped into the row.
KVIP_DEVICE Keys8 load_keys(const uint16_t* keys, int idx0, int valid, int stride) {
    Keys8 r;
    const v4i v = *reinterpret_cast<const v4i*>(keys + min(idx0, stride - kKeysPerThread));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        r.k[2 * j] = static_cast<uint32_t>(v[j]) & 0xFFFFu;
        r.k[2 * j + 1] = static_cast<uint32_t>(v[j]) >> 16;
    }
    r.count = max(0, min(kKeysPerThread, valid - idx0));
    return r;
}

__global__ __launch_bounds__(kTopkThreads) void topk_kernel(const KvipTopkArgs p) {
    __shared__ uint32_t s_hist[256];
    __shared__ uint32_t s_wave[kTopkThreads / 64];
    __shared__ int s_sel[4];

    const int tid = threadIdx.x;
    const int row = blockIdx.x;
    const int b = row / p.rows_per_request;
    const int valid = topk_row_valid(p, row);
    int32_t* out = p.topk + static_cast<size_t>(row) * kTopK;
    const uint16_t* keys = p.score_keys + static_cast<size_t>(row) * p.key_stride;
    uint32_t* ghist = p.histogram != nullptr ? p.histogram + static_cast<size_t>(row) * 256 : nullptr;

    if (valid < kTopK) {
        for (int i = tid; i < kTopK; i += kTopkThreads) out[i] = i < valid ? i : -1;
        if (ghist != nullptr && tid < 256) ghist[tid] = 0u;
        return;
    }

    // Level 1: high byte.
    if (tid < 256) s_hist[tid] = ghist != nullptr ? ghist[tid] : 0u;
    if (tid == 0) {
        s_sel[0] = -1;
        s_sel[2] = -1;
    }
    __syncthreads();
    if (ghist != nullptr) {
        if (tid < 256) ghist[tid] = 0u;  // ready for the next scoring launch
    } else {
        for (int base = tid * kKeysPerThread; base < valid; base += kTileKeys) {
            const Keys8 r = load_keys(keys, base, valid, p.key_stride);
#pragma unroll
            for (int j = 0; j < kKeysPerThread; ++j) {
                wave_hist_add(s_hist, r.k[j] >> 8, j < r.count);
            }
        }
    }
    __syncthreads();
    select_bin(s_hist, kTopK, s_sel, s_wave);
    const int hb = s_sel[0];
    const uint32_t gt_hi = static_cast<uint32_t>(s_sel[1]);
    if (hb < 0) {
        for (int i = tid; i < kTopK; i += kTopkThreads) out[i] = -1;
        if (tid == 0) report(p.status, KVIP_STATUS_HISTOGRAM);
        return;
    }

    // Level 2: low byte among keys whose high byte is hb.
    if (tid < 256) s_hist[tid] = 0u;
    __syncthreads();
    for (int base = tid * kKeysPerThread; base < valid; base += kTileKeys) {
        const Keys8 r = load_keys(keys, base, valid, p.key_stride);
#pragma unroll
        for (int j = 0; j < kKeysPerThread; ++j) {
            if (j < r.count && static_cast<int>(r.k[j] >> 8) == hb) atomicAdd(&s_hist[r.k[j] & 0xFFu], 1u);
        }
    }
    __syncthreads();
    select_bin(s_hist, kTopK - gt_hi, s_sel + 2, s_wave);
    if (s_sel[2] < 0) {
        for (int i = tid; i < kTopK; i += kTopkThreads) out[i] = -1;
        if (tid == 0) report(p.status, KVIP_STATUS_HISTOGRAM);
        return;
    }
    const uint32_t kth = (static_cast<uint32_t>(hb) << 8) | static_cast<uint32_t>(s_sel[2]);
    const uint32_t n_gt = gt_hi + static_cast<uint32_t>(s_sel[3]);
    const uint32_t need = kTopK - n_gt;

    // Level 3: ordered emission. gt_base/eq_base are identical in every thread.
    uint32_t gt_base = 0, eq_base = 0;
    uint32_t err = 0;
    for (int tile = 0; tile < valid; tile += kTileKeys) {
        const int idx0 = tile + tid * kKeysPerThread;
        const Keys8 r = load_keys(keys, idx0, valid, p.key_stride);
        uint32_t ngt = 0, neq = 0;
#pragma unroll
        for (int j = 0; j < kKeysPerThread; ++j) {
            const bool in = j < r.count;
            ngt += (in && r.k[j] > kth) ? 1u : 0u;
            neq += (in && r.k[j] == kth) ? 1u : 0u;
        }
        uint32_t total;
        const uint32_t excl = block_exclusive_scan((ngt << 16) | neq, s_wave, &total);
        uint32_t pg = gt_base + (excl >> 16);
        uint32_t pe = eq_base + (excl & 0xFFFFu);
#pragma unroll
        for (int j = 0; j < kKeysPerThread; ++j) {
            if (j < r.count) {
                if (r.k[j] > kth) {
                    // pg < n_gt whenever the histogram matches the keys; the guard keeps a
                    // stale histogram from writing past the row.
                    if (pg < n_gt) out[pg] = idx0 + j;
                    else err = KVIP_STATUS_HISTOGRAM;
                    ++pg;
                } else if (r.k[j] == kth) {
                    if (pe < need) out[n_gt + pe] = idx0 + j;
                    ++pe;
                }
            }
        }
        gt_base += total >> 16;
        eq_base += total & 0xFFFFu;
        if (gt_base >= n_gt && eq_base >= need) break;  // uniform
    }
    report(p.status, err);
}


// Register-resident variant for rows of at most THREADS*KPT keys (KPT <= 64): thread t
// holds keys [t*KPT, (t+1)*KPT) (packed two per register), loaded in one batch; the high-byte
// bin comes from the scoring histogram (each wave reads it) or a histogram built here, and
// the rest is select_row.h (low-byte histogram, bitmask counts, one workgroup scan,
// emission of the selected keys only). Rows of at most 8192 keys take 256-thread workgroups
// (32 keys each), so that a batch of short rows keeps several rows per CU in flight.
template <int KPT, int THREADS = kTopkThreads>
__global__ __launch_bounds__(THREADS) void topk_regs_kernel(const KvipTopkArgs p) {
    constexpr int W = KPT / 2;  // packed registers per thread
    static_assert(THREADS >= 256 && THREADS % 64 == 0 && kTopK % (2 * THREADS) == 0, "whole int2 output pairs");
    __shared__ __align__(16) uint32_t s_hist[256];
    __shared__ uint32_t s_wave[THREADS / 64];
    __shared__ __align__(16) int32_t s_out[kTopK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int row = blockIdx.x;
    const int valid = min(topk_row_valid(p, row), THREADS * KPT);
    int32_t* out = p.topk + static_cast<size_t>(row) * kTopK;
    const uint16_t* keys = p.score_keys + static_cast<size_t>(row) * p.key_stride;
    uint32_t* ghist = p.histogram != nullptr ? p.histogram + static_cast<size_t>(row) * 256 : nullptr;

    if (valid < kTopK) {
        for (int i = tid; i < kTopK; i += THREADS) out[i] = i < valid ? i : -1;
        if (ghist != nullptr && tid < 256) ghist[tid] = 0u;
        return;
    }

    // Keys of this thread; positions >= valid are excluded by `count`, and threads whose
    // keys all lie past the row's end load nothing (a row's valid length is often well
    // below the stride the kernel is sized for). A load's start is clamped into the row
    // (the row stride is a multiple of 8 keys).
    const int first = tid * KPT;
    const int count = max(0, min(KPT, valid - first));
    uint32_t kk[W];
#pragma unroll
    for (int v = 0; v < W; ++v) kk[v] = 0u;
    if (count > 0) {
#pragma unroll
        for (int v = 0; v < W / 4; ++v) {
            const int at = min(first + v * 8, p.key_stride - 8);
            const v4i x = *reinterpret_cast<const v4i*>(keys + at);
            kk[4 * v] = x[0];
            kk[4 * v + 1] = x[1];
            kk[4 * v + 2] = x[2];
            kk[4 * v + 3] = x[3];
        }
    }

    // High-byte bin of the 2048th largest key: wave 0 reads the 256 bins (from the
    // scoring histogram, or one built here) and shares the bin through LDS.
    __shared__ uint32_t s_bin[3];
    if (ghist == nullptr) {
        if (tid < 256) s_hist[tid] = 0u;
        __syncthreads();
        if (count > 0) {
#pragma unroll
            for (int j = 0; j < KPT; ++j) {
                const uint32_t k = (j & 1) ? (kk[j >> 1] >> 16) : (kk[j >> 1] & 0xFFFFu);
                wave_hist_add(s_hist, k >> 8, j < count);
            }
        }
        __syncthreads();
    }
    if (tid < 64) {
        const v4i hv = *reinterpret_cast<const v4i*>((ghist != nullptr ? ghist : s_hist) + lane * 4);
        const uint32_t h[4] = {static_cast<uint32_t>(hv[0]), static_cast<uint32_t>(hv[1]),
                               static_cast<uint32_t>(hv[2]), static_cast<uint32_t>(hv[3])};
        int hb0;
        uint32_t gt0;
        wave_select_bin(h, kTopK, hb0, gt0);
        // The scoring histogram counts every visible key once: a total other than
        // `valid` means the scoring launch skipped or repeated tiles.
        const uint32_t hist_total = static_cast<uint32_t>(
            __builtin_amdgcn_readlane(static_cast<int>(wave_inclusive_scan(h[0] + h[1] + h[2] + h[3])), 63));
        if (lane == 0) {
            s_bin[0] = static_cast<uint32_t>(hb0);
            s_bin[1] = gt0;
            s_bin[2] = hist_total == static_cast<uint32_t>(valid) ? 1u : 0u;
        }
    }
    if (ghist == nullptr) __syncthreads();  // wave 0 has read the bins before they are cleared
    if (tid < 256) s_hist[tid] = 0u;
    for (int i = tid; i < kTopK / 2; i += THREADS) reinterpret_cast<int2*>(s_out)[i] = int2{-1, -1};
    __syncthreads();
    if (ghist != nullptr && tid < 256) ghist[tid] = 0u;  // read by wave 0: ready for the next scoring launch
    const int hb = static_cast<int>(s_bin[0]);
    const uint32_t gt_hi = s_bin[1];
    const bool counted = s_bin[2] != 0u;

    const RowSelection sel =
        select_row<KPT>(kk, count, first, hb, gt_hi, s_hist, s_wave, [&](int pos, int tok) { s_out[pos] = tok; });
    __syncthreads();
    for (int i = tid; i < kTopK / 2; i += THREADS) reinterpret_cast<int2*>(out)[i] = reinterpret_cast<const int2*>(s_out)[i];
    if (tid == 0 && !(sel.ok && counted)) report(p.status, KVIP_STATUS_HISTOGRAM);
}

// Split select for rows scored by kvip_hip_indexer_decode (the high-byte histogram is
// given): the row is cut into 2048-key segments, one 256-thread workgroup each, in two
// launches, so a batch of long rows spreads over many CUs instead of one workgroup per
// row.
//   topk_segment_kernel: every segment workgroup derives the high-byte bin hb from the
//     row histogram and writes its own low-byte histogram of the keys in hb and its count
//     of keys above hb.
//   topk_emit_kernel: every segment workgroup sums those records into the row's kth key
//     and its own segment prefix (keys > kth and keys == kth in earlier segments), then
//     emits its segment's selected tokens at their final positions.
// Record of segment s of a row: words [0, 256) low-byte histogram, [256] keys above hb;
// segment 0 also holds [257] hb (-1: inconsistent histogram) and [258] keys above hb in
// the row.
constexpr int kSplitThreads = 256;
constexpr int kSplitKeys = KVIP_TOPK_SEGMENT_KEYS / kSplitThreads;  // 8 per thread
constexpr int kSegWords = KVIP_TOPK_SEGMENT_WORDS;

KVIP_DEVICE int row_valid(const KvipTopkArgs& p, int row) { return topk_row_valid(p, row); }

KVIP_DEVICE void load_segment(const uint16_t* keys, int first, int stride, uint32_t* kk) {
#pragma unroll
    for (int v = 0; v < kSplitKeys / 8; ++v) {
        const v4i x = *reinterpret_cast<const v4i*>(keys + min(first + v * 8, stride - 8));
        kk[4 * v] = x[0];
        kk[4 * v + 1] = x[1];
        kk[4 * v + 2] = x[2];
        kk[4 * v + 3] = x[3];
    }
}

__global__ __launch_bounds__(kSplitThreads) void topk_segment_kernel(const KvipTopkArgs p) {
    __shared__ uint32_t s_hist[256];
    __shared__ uint32_t s_wave[kSplitThreads / 64];
    __shared__ int s_sel[2];
    const int tid = threadIdx.x;
    const int seg = blockIdx.x;
    const int row = blockIdx.y;
    const int valid = row_valid(p, row);
    const int nseg = (valid + KVIP_TOPK_SEGMENT_KEYS - 1) / KVIP_TOPK_SEGMENT_KEYS;
    if (valid < kTopK || seg >= nseg) return;
    int32_t* out = p.topk + static_cast<size_t>(row) * kTopK;
    uint32_t* rec = p.segments + (static_cast<size_t>(row) * gridDim.x + seg) * kSegWords;
    // The segment's keys are requested first so that their latency overlaps the bin select.
    const int first = seg * KVIP_TOPK_SEGMENT_KEYS + tid * kSplitKeys;
    const int count = max(0, min(kSplitKeys, valid - first));
    uint32_t kk[kSplitKeys / 2];
    load_segment(p.score_keys + static_cast<size_t>(row) * p.key_stride, first, p.key_stride, kk);
    // Positions a stale histogram would leave unwritten read -1.
    for (int i = seg * kTopK / nseg + tid; i < (seg + 1) * kTopK / nseg; i += kSplitThreads) out[i] = -1;

    s_hist[tid] = p.histogram[static_cast<size_t>(row) * 256 + tid];
    if (tid == 0) s_sel[0] = -1;
    __syncthreads();
    select_bin(s_hist, kTopK, s_sel, s_wave);
    const int hb = s_sel[0];
    if (hb < 0) {
        if (seg == 0 && tid == 0) rec[257] = 0xFFFFFFFFu;
        return;
    }
    s_hist[tid] = 0u;
    __syncthreads();
    uint32_t above = 0;
#pragma unroll
    for (int j = 0; j < kSplitKeys; ++j) {
        const uint32_t k = (j & 1) ? (kk[j >> 1] >> 16) : (kk[j >> 1] & 0xFFFFu);
        const int high = static_cast<int>(k >> 8);
        if (j < count) {
            above += high > hb ? 1u : 0u;
            if (high == hb) atomicAdd(&s_hist[k & 0xFFu], 1u);
        }
    }
    uint32_t total;
    block_exclusive_scan(above, s_wave, &total);  // its barriers also complete the histogram
    rec[tid] = s_hist[tid];
    if (tid == 0) {
        rec[256] = total;
        if (seg == 0) {
            rec[257] = static_cast<uint32_t>(hb);
            rec[258] = static_cast<uint32_t>(s_sel[1]);
        }
    }
}

__global__ __launch_bounds__(kSplitThreads) void topk_emit_kernel(const KvipTopkArgs p) {
    __shared__ uint32_t s_hist[256];
    __shared__ uint32_t s_wave[kSplitThreads / 64];
    __shared__ int s_sel[2];
    __shared__ uint32_t s_eq_before;
    const int tid = threadIdx.x;
    const int seg = blockIdx.x;
    const int row = blockIdx.y;
    const int valid = row_valid(p, row);
    int32_t* out = p.topk + static_cast<size_t>(row) * kTopK;
    if (seg == 0) p.histogram[static_cast<size_t>(row) * 256 + tid] = 0u;  // ready for the next scoring launch
    if (valid < kTopK) {
        if (seg == 0) {
            for (int i = tid; i < kTopK; i += kSplitThreads) out[i] = i < valid ? i : -1;
        }
        return;
    }
    const int nseg = (valid + KVIP_TOPK_SEGMENT_KEYS - 1) / KVIP_TOPK_SEGMENT_KEYS;
    if (seg >= nseg) return;
    const int first = seg * KVIP_TOPK_SEGMENT_KEYS + tid * kSplitKeys;
    const int count = max(0, min(kSplitKeys, valid - first));
    uint32_t kk[kSplitKeys / 2];
    load_segment(p.score_keys + static_cast<size_t>(row) * p.key_stride, first, p.key_stride, kk);
    const uint32_t* recs = p.segments + static_cast<size_t>(row) * gridDim.x * kSegWords;
    const int hb = static_cast<int>(recs[257]);
    if (hb < 0) {
        if (seg == 0 && tid == 0) report(p.status, KVIP_STATUS_HISTOGRAM);
        return;
    }
    const uint32_t gt_hi = recs[258];
    // Row histogram of the low byte within hb, and this segment's share of earlier counts
    // (8 records requested per round trip).
    uint32_t all = 0, before = 0;
#pragma unroll 8
    for (int s = 0; s < nseg; ++s) {
        const uint32_t c = recs[s * kSegWords + tid];
        all += c;
        before += s < seg ? c : 0u;
    }
    uint32_t above_before = 0;
    for (int s = tid; s < seg; s += kSplitThreads) above_before += recs[s * kSegWords + 256];
    s_hist[tid] = all;
    if (tid == 0) s_sel[0] = -1;
    __syncthreads();
    select_bin(s_hist, kTopK - gt_hi, s_sel, s_wave);
    const int lo = s_sel[0];
    if (lo < 0) {
        if (seg == 0 && tid == 0) report(p.status, KVIP_STATUS_HISTOGRAM);
        return;
    }
    const uint32_t kth = (static_cast<uint32_t>(hb) << 8) | static_cast<uint32_t>(lo);
    const uint32_t n_gt = gt_hi + static_cast<uint32_t>(s_sel[1]);
    const uint32_t need = kTopK - n_gt;
    if (tid == lo) s_eq_before = before;
    uint32_t gt_before;
    block_exclusive_scan(above_before + (tid > lo ? before : 0u), s_wave, &gt_before);
    const uint32_t eq_before = s_eq_before;
    uint32_t ngt = 0, neq = 0;
#pragma unroll
    for (int j = 0; j < kSplitKeys; ++j) {
        const uint32_t k = (j & 1) ? (kk[j >> 1] >> 16) : (kk[j >> 1] & 0xFFFFu);
        ngt += (j < count && k > kth) ? 1u : 0u;
        neq += (j < count && k == kth) ? 1u : 0u;
    }
    uint32_t total;
    const uint32_t excl = block_exclusive_scan((ngt << 16) | neq, s_wave, &total);
    uint32_t pg = gt_before + (excl >> 16);
    uint32_t pe = eq_before + (excl & 0xFFFFu);
    uint32_t err = 0;
    if (ngt != 0u || (neq != 0u && pe < need)) {
#pragma unroll
        for (int j = 0; j < kSplitKeys; ++j) {
            const uint32_t k = (j & 1) ? (kk[j >> 1] >> 16) : (kk[j >> 1] & 0xFFFFu);
            if (j < count) {
                if (k > kth) {
                    if (pg < n_gt) out[pg] = first + j;
                    else err = KVIP_STATUS_HISTOGRAM;
                    ++pg;
                } else if (k == kth) {
                    if (pe < need) out[n_gt + pe] = first + j;
                    ++pe;
                }
            }
        }
    }
    report(p.status, err);
}

}  // namespace

uint32_t validate_topk(const KvipTopkArgs* a) {
    if (a == nullptr) return KVIP_ERR_INVALID;
    const bool ok = a->score_keys != nullptr && a->seq_lens != nullptr && a->topk != nullptr &&
                    (a->rows_per_request == 1 || a->rows_per_request == 2 || a->rows_per_request == 4) &&
                    a->batch >= 1 && static_cast<int64_t>(a->batch) * a->rows_per_request <= (1 << 24) &&
                    a->key_stride >= 8 && a->key_stride % 8 == 0 && a->key_stride <= (1 << 24) &&
                    a->limit >= 0 && (a->limit == 0 || a->histogram == nullptr) &&
                    (a->segments == nullptr || static_cast<int64_t>(a->batch) * a->rows_per_request <= 65535) &&
                    (reinterpret_cast<uintptr_t>(a->score_keys) & 15u) == 0;
    return ok ? KVIP_OK : KVIP_ERR_INVALID;
}

hipError_t launch_topk(const KvipTopkArgs& a, hipStream_t stream) {
    const dim3 grid(a.batch * a.rows_per_request);
    const dim3 block(kTopkThreads);
    if (a.segments != nullptr && a.histogram != nullptr) {
        const dim3 split((a.key_stride + KVIP_TOPK_SEGMENT_KEYS - 1) / KVIP_TOPK_SEGMENT_KEYS,
                         a.batch * a.rows_per_request);
        hipLaunchKernelGGL(topk_segment_kernel, split, dim3(kSplitThreads), 0, stream, a);
        hipLaunchKernelGGL(topk_emit_kernel, split, dim3(kSplitThreads), 0, stream, a);
        return hipGetLastError();
    }
    // Rows that fit 1024*KPT keys use the register-resident select; a limit (the resident
    // prefix of a longer row) bounds the keys a row can have.
    const int64_t span = a.limit > 0 ? std::min<int64_t>(a.key_stride, (a.limit + 7) / 8 * 8) : a.key_stride;
    if (span <= 256 * 32) {
        hipLaunchKernelGGL((topk_regs_kernel<32, 256>), grid, dim3(256), 0, stream, a);
    } else if (span <= kTopkThreads * 16) {
        hipLaunchKernelGGL(topk_regs_kernel<16>, grid, block, 0, stream, a);
    } else if (span <= kTopkThreads * 32) {
        hipLaunchKernelGGL(topk_regs_kernel<32>, grid, block, 0, stream, a);
    } else if (span <= kTopkThreads * 64) {
        hipLaunchKernelGGL(topk_regs_kernel<64>, grid, block, 0, stream, a);
    } else {
        hipLaunchKernelGGL(topk_kernel, grid, block, 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace kvip

extern "C" uint32_t kvip_hip_topk(const KvipTopkArgs* args, void* stream) {
    const uint32_t rc = kvip::validate_topk(args);
    if (rc != KVIP_OK) return rc;
    return static_cast<uint32_t>(kvip::launch_topk(*args, static_cast<hipStream_t>(stream)));
}
