// TopK-2048 selection of one row of sortable uint16 keys held in registers by a whole
// workgroup, shared by the fused TopK + gather launch and the XCD-local round.
//
// Thread t holds keys [first, first + KPT) of the row (first = t * KPT), two per 32-bit
// register, of which the first `count` are live. Given the high-byte bin hb of the 2048th
// largest key and the number of keys above that bin (from the row's 256-bin histogram):
//   1. a low-byte histogram of the live keys in bin hb (LDS atomics) gives the kth key
//      and n_gt, the number of keys above it;
//   2. one pass builds, per 32 keys, a bitmask of the keys above kth and one of the keys
//      equal to it; their popcounts, scanned over the workgroup in token order, place
//      every selected key: keys above kth at [0, n_gt) in token order, then the first
//      2048 - n_gt keys equal to kth in token order (GT-then-EQ, ties to the lower token);
//   3. each thread emits only its selected keys by walking the set bits of its masks.
// Only about one key in ten is selected, so step 3 costs a few iterations per thread
// instead of a compare-and-branch chain over every key.
//
// Reference: LITopk's GT-then-EQ emission (op_kernel/topk.h:155-187, topk_common.h:
// 1000-1067) as QLIVector::ProcessTopK applies it (indexer_vector.h:799-973).
#pragma once

#include "kvip_device.h"

namespace kvip {

// In a 256-bin histogram spread 4 bins per lane (bins 4l..4l+3 in h[0..3]), the highest
// bin `sel` whose count of keys at or above it reaches `target` (-1 if none), and the
// count strictly above it. Whole wave; no LDS.
KVIP_DEVICE void wave_select_bin(const uint32_t (&h)[4], uint32_t target, int& sel, uint32_t& above) {
    const int lane = lane_id();
    const uint32_t mine = h[0] + h[1] + h[2] + h[3];
    const uint32_t suffix_incl = wave_inclusive_suffix_scan(mine);
    uint32_t ge = suffix_incl - mine;  // keys in bins of higher lanes
    int best = -1;
    uint32_t best_above = 0;
#pragma unroll
    for (int i = 3; i >= 0; --i) {
        const uint32_t at_or_above = ge + h[i];
        if (best < 0 && at_or_above >= target) {
            best = lane * 4 + i;
            best_above = ge;
        }
        ge = at_or_above;
    }
    const unsigned long long cand = __ballot(best >= 0);
    const int top = cand ? 63 - __clzll(cand) : 0;
    sel = cand ? __builtin_amdgcn_readlane(best, top) : -1;
    above = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(best_above), top));
}

// Packed 16-bit integer operations on the two halves of a register (v_pk_sub_u16 with
// clamp: saturating subtraction; v_pk_min_u16), written out because the compiler turns the
// saturate-and-min idiom into two compares and selects per half.
KVIP_DEVICE uint32_t pk_sub_sat_u16(uint32_t a, uint32_t b) {
    uint32_t d;
    asm("v_pk_sub_u16 %0, %1, %2 clamp" : "=v"(d) : "v"(a), "v"(b));
    return d;
}
KVIP_DEVICE uint32_t pk_min_u16(uint32_t a, uint32_t b) {
    uint32_t d;
    asm("v_pk_min_u16 %0, %1, %2" : "=v"(d) : "v"(a), "v"(b));
    return d;
}

struct RowSelection {
    uint32_t kth;   // the 2048th largest key
    uint32_t n_gt;  // keys above it
    bool ok;        // false: the histogram does not match the keys
};

// Steps 1-3 above for the whole workgroup. s_lo: 256 words of LDS, zero on entry (and
// visible to every thread); s_wave: blockDim.x / 64 words. emit(pos, token) is called once
// per selected key with its position in [0, 2048). Contains three workgroup barriers.
template <int KPT, typename Emit>
KVIP_DEVICE RowSelection select_row(const uint32_t (&kk)[KPT / 2], int count, int first, int hb, uint32_t gt_hi,
                                    uint32_t* s_lo, uint32_t* s_wave, Emit&& emit) {
    constexpr int M = (KPT + 31) / 32;  // 32-key mask words per thread
    const int lane = lane_id();
    auto key_at = [&](int j) -> uint32_t { return (j & 1) ? (kk[j >> 1] >> 16) : (kk[j >> 1] & 0xFFFFu); };
    // 1. Low-byte histogram of the live keys in bin hb (threads past the row's end skip
    // their key loops).
    if (hb >= 0 && count > 0) {
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            const uint32_t k = key_at(j);
            if (j < count && static_cast<int>(k >> 8) == hb) atomicAdd(&s_lo[k & 0xFFu], 1u);
        }
    }
    __syncthreads();
    const v4i lv = *reinterpret_cast<const v4i*>(s_lo + lane * 4);
    const uint32_t l4[4] = {static_cast<uint32_t>(lv[0]), static_cast<uint32_t>(lv[1]), static_cast<uint32_t>(lv[2]),
                            static_cast<uint32_t>(lv[3])};
    int lb = -1;
    uint32_t gt_lo = 0;
    if (hb >= 0) wave_select_bin(l4, kTopK - gt_hi, lb, gt_lo);
    RowSelection r;
    r.ok = hb >= 0 && lb >= 0;
    r.kth = r.ok ? ((static_cast<uint32_t>(hb) << 8) | static_cast<uint32_t>(lb)) : 0x10000u;
    r.n_gt = r.ok ? gt_hi + gt_lo : 0u;
    // Live keys equal to kth, counted exactly by the low-byte histogram (same key set as
    // the eq masks below).
    const uint32_t n_eq = r.ok ? s_lo[lb] : 0u;
    const uint32_t need = r.ok ? kTopK - r.n_gt : 0u;
    // 2. Masks of the keys above and equal to kth, per 32 keys.
    uint32_t gtm[M], eqm[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        gtm[m] = 0u;
        eqm[m] = 0u;
    }
    if constexpr (KPT % 32 == 0) {
        // Two keys per instruction: register i of a 32-key group is repacked to hold keys i
        // (low half) and 16 + i (high half), so that (x - kth) saturated at 0 and then
        // min(., 1) per half put key i's bit at bit i and key 16 + i's at bit 16 + i of the
        // shifted result; the same with x ^ kth marks the keys that differ from kth. Without a
        // valid kth (r.ok false: kth = 0x10000, which matches no key) the masks stay empty.
        if (count > 0 && r.ok) {
            const uint32_t kth2 = r.kth * 0x00010001u, one2 = 0x00010001u;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                uint32_t gt = 0u, ne = 0u;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t wa = kk[16 * m + i / 2], wb = kk[16 * m + 8 + i / 2];
                    const uint32_t x = __builtin_amdgcn_perm(wb, wa, (i & 1) ? 0x07060302u : 0x05040100u);
                    gt |= pk_min_u16(pk_sub_sat_u16(x, kth2), one2) << i;
                    ne |= pk_min_u16(x ^ kth2, one2) << i;
                }
                const int live = count - 32 * m;  // live keys of this group
                const uint32_t lmask = live >= 32 ? 0xFFFFFFFFu : (live <= 0 ? 0u : (1u << live) - 1u);
                gtm[m] = gt & lmask;
                eqm[m] = ~ne & lmask;
            }
        }
    } else if (count > 0) {
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            const uint32_t k = key_at(j);
            const bool live = j < count;
            gtm[j >> 5] |= (live && k > r.kth) ? (1u << (j & 31)) : 0u;
            eqm[j >> 5] |= (live && k == r.kth) ? (1u << (j & 31)) : 0u;
        }
    }
    uint32_t ngt = 0, neq = 0;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        ngt += static_cast<uint32_t>(__popc(gtm[m]));
        neq += static_cast<uint32_t>(__popc(eqm[m]));
    }
    // Packed gt << 16 | eq. Per-thread counts are <= KPT and every exclusive prefix of the
    // eq counts stays below 65536 (a row holds at most 65536 keys and the thread's own
    // keys are not in its prefix), so both fields of `excl` are exact. Only the row total
    // of eq can reach 65536 (every key of a full row equal) and carry into the gt field:
    // the gt total is therefore taken as (total - n_eq) >> 16.
    uint32_t total;
    const uint32_t excl = block_exclusive_scan((ngt << 16) | neq, s_wave, &total);
    if (r.ok && ((total - n_eq) >> 16) != r.n_gt) r.ok = false;
    // 3. Emission of this thread's selected keys.
    uint32_t pg = excl >> 16;
    const uint32_t pe = excl & 0xFFFFu;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        for (uint32_t bits = gtm[m]; bits != 0u; bits &= bits - 1u) {
            if (pg < r.n_gt) emit(static_cast<int>(pg), first + m * 32 + __builtin_ctz(bits));
            ++pg;
        }
    }
    uint32_t allowed = pe < need ? min(neq, need - pe) : 0u;
    uint32_t at = r.n_gt + pe;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        for (uint32_t bits = eqm[m]; bits != 0u && allowed != 0u; bits &= bits - 1u) {
            emit(static_cast<int>(at), first + m * 32 + __builtin_ctz(bits));
            ++at;
            --allowed;
        }
    }
    return r;
}

}  // namespace kvip
