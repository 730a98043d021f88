// Device helpers shared by the gfx950 kernels of libkvip_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kvip_hip.h"

#define KVIP_DEVICE __device__ __forceinline__

namespace kvip {

constexpr int kTopK = KVIP_TOPK;
constexpr int kBlockTokens = KVIP_BLOCK_TOKENS;
constexpr int kIndexDim = KVIP_INDEX_DIM;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

KVIP_DEVICE int lane_id() { return __lane_id(); }

// fp32 -> bf16 bits, rounding half away from zero on the magnitude (the Ascend
// CAST_ROUND mode the reference scores use: tests/operators/lifetch/support/
// workloads.py:233-235, op_kernel/indexer/indexer_score.h:105-140).
KVIP_DEVICE uint32_t bf16_bits_half_away(float x) {
    return (__float_as_uint(x) + 0x8000u) >> 16;
}

// bf16 bits -> order-preserving uint16 key (op_kernel/indexer/score_common.h:66-97):
// the canonical NaN 0x7FC0 becomes 0xFFFF first; negative values are inverted,
// non-negative values get the sign bit flipped.
KVIP_DEVICE uint32_t sortable_key(uint32_t bits) {
    bits = (bits == 0x7FC0u) ? 0xFFFFu : bits;
    return (bits & 0x8000u) ? (~bits & 0xFFFFu) : (bits ^ 0x8000u);
}

KVIP_DEVICE float bf16_to_float(uint16_t bits) { return __uint_as_float(static_cast<uint32_t>(bits) << 16); }

KVIP_DEVICE void report(uint32_t* status, uint32_t bits) {
    if (status != nullptr && bits != 0) atomicOr(status, bits);
}

// Histogram add where the 64 lanes of a wave often share a bin: one LDS atomic per
// distinct bin present in the wave. Must be called by the whole wave.
KVIP_DEVICE void wave_hist_add(uint32_t* hist, uint32_t bin, bool live) {
    unsigned long long pending = __ballot(live);
    while (pending) {
        const int leader = __ffsll(pending) - 1;
        const uint32_t lead_bin = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(bin), leader));
        const bool same = live && bin == lead_bin;
        const unsigned long long group = __ballot(same);
        if (lane_id() == leader) atomicAdd(&hist[lead_bin], static_cast<uint32_t>(__popcll(group)));
        live = live && !same;
        pending &= ~group;
    }
}

// 64-bit value of lane l (l uniform).
KVIP_DEVICE int64_t readlane64(int64_t v, int l) {
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), l));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v >> 32), l));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Row copies with a wave-wide 16-byte piece index: piece idx = it * 64 + lane of a list of
// rows of PIECES pieces belongs to row idx / PIECES. For a compile-time `it` that row is one
// of at most three consecutive rows, so the row's value (held by lane `row` of v) is picked
// from three readlanes instead of an LDS shuffle.
template <int PIECES, int ROWS>
KVIP_DEVICE int64_t row_value(int64_t v, int it, int row) {
    const int lo = min((it * 64) / PIECES, ROWS - 1);
    const int hi = min((it * 64 + 63) / PIECES, ROWS - 1);
    int64_t out = readlane64(v, lo);
#pragma unroll
    for (int q = 1; q <= 2; ++q) {
        if (lo + q <= hi && row == lo + q) out = readlane64(v, lo + q);
    }
    return out;
}

// Value of the lane `CTRL` selects within each row of 16 lanes (a DPP row shift); lanes
// whose source falls outside their row read 0.
template <int CTRL>
KVIP_DEVICE uint32_t dpp_row(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, true));
}

// Inclusive prefix sum over the 64 lanes: Hillis-Steele inside each 16-lane row by DPP row
// shifts (no LDS round trip), then the totals of the lower rows by readlane.
KVIP_DEVICE uint32_t wave_inclusive_scan(uint32_t v) {
    v += dpp_row<0x111>(v);  // row_shr:1
    v += dpp_row<0x112>(v);  // row_shr:2
    v += dpp_row<0x114>(v);  // row_shr:4
    v += dpp_row<0x118>(v);  // row_shr:8
    const uint32_t r0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 15));
    const uint32_t r1 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 31));
    const uint32_t r2 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 47));
    const int row = lane_id() >> 4;
    return v + (row >= 1 ? r0 : 0u) + (row >= 2 ? r1 : 0u) + (row >= 3 ? r2 : 0u);
}

// Inclusive suffix sum over the 64 lanes (lane l gets the sum of lanes l..63).
KVIP_DEVICE uint32_t wave_inclusive_suffix_scan(uint32_t v) {
    v += dpp_row<0x101>(v);  // row_shl:1
    v += dpp_row<0x102>(v);  // row_shl:2
    v += dpp_row<0x104>(v);  // row_shl:4
    v += dpp_row<0x108>(v);  // row_shl:8
    const uint32_t r1 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 16));
    const uint32_t r2 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 32));
    const uint32_t r3 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 48));
    const int row = lane_id() >> 4;
    return v + (row <= 0 ? r1 : 0u) + (row <= 1 ? r2 : 0u) + (row <= 2 ? r3 : 0u);
}

// Exclusive prefix sum over the whole workgroup (blockDim.x a multiple of 64, at most
// 1024). `wave_sums` is __shared__ scratch of blockDim.x/64 words. Returns the
// exclusive prefix of this thread and writes the workgroup total into *total.
// Contains two __syncthreads and must be reached by every thread.
KVIP_DEVICE uint32_t block_exclusive_scan(uint32_t v, uint32_t* wave_sums, uint32_t* total) {
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int waves = blockDim.x >> 6;
    const uint32_t incl = wave_inclusive_scan(v);
    __syncthreads();  // previous users of wave_sums are done
    if (lane == 63) wave_sums[wave] = incl;
    __syncthreads();
    uint32_t before = 0, all = 0;
    for (int w = 0; w < waves; ++w) {
        const uint32_t s = wave_sums[w];
        before += (w < wave) ? s : 0u;
        all += s;
    }
    *total = all;
    return before + incl - v;
}

// Finds the bin holding the target-th largest element of a 256-bin histogram
// (bin 255 = largest keys). Writes {bin, count strictly above the bin} to sel[0..1]
// (sel[0] stays -1 when the histogram holds fewer than `target` elements).
KVIP_DEVICE void select_bin(const uint32_t* hist, uint32_t target, int* sel, uint32_t* wave_sums) {
    const int tid = threadIdx.x;
    const uint32_t c = tid < 256 ? hist[255 - tid] : 0u;
    uint32_t total;
    const uint32_t excl = block_exclusive_scan(c, wave_sums, &total);
    if (tid < 256 && c != 0u && excl < target && excl + c >= target) {
        sel[0] = 255 - tid;
        sel[1] = static_cast<int>(excl);
    }
    __syncthreads();
}

// Valid positions of TopK row `row`: min(seq_lens[b], query_ends[row], limit when > 0),
// clamped to [0, key_stride].
KVIP_DEVICE int topk_row_valid(const KvipTopkArgs& p, int row) {
    int valid = max(p.seq_lens[row / p.rows_per_request], 0);
    if (p.query_ends != nullptr) valid = min(valid, p.query_ends[row]);
    if (p.limit > 0) valid = min(valid, p.limit);
    return min(max(valid, 0), p.key_stride);
}

}  // namespace kvip
