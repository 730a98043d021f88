// MFMA building blocks shared by the decode and prefill lightning-indexer kernels:
// the K-slice steps of the 128-dim Q.K contraction on gfx950 and the LDS swizzle of a
// staged K row. Lane (n = lane % 32, g = lane / 32) of a wave holds 64*ELEM contiguous
// bytes (NV 16-byte vectors) of row n at byte offset 64*ELEM*g, for both operands, so
// the contraction pairs identical dims.
#pragma once

#include "kvip_device.h"

namespace kvip {

// ELEM = bytes per Q/K element (1: fp8 e4m3, 2: bf16). Each lane holds NV = 4*ELEM
// 16-byte vectors of one Q or K row.
template <int ELEM>
struct Mma;

// step(s) adds the s-th K slice of the 128-dim contraction; MT head tiles interleave
// their slices (tile 0 slice 0, tile 1 slice 0, tile 0 slice 1, ...) so consecutive
// MFMAs are independent.
template <>
struct Mma<1> {
    static constexpr int NV = 4;
    static constexpr int STEPS = 2;
    KVIP_DEVICE static void step(int s, const v4i (&a)[NV], const v4i (&b)[NV], v16f& acc) {
        const v8i av = __builtin_shufflevector(a[2 * s], a[2 * s + 1], 0, 1, 2, 3, 4, 5, 6, 7);
        const v8i bv = __builtin_shufflevector(b[2 * s], b[2 * s + 1], 0, 1, 2, 3, 4, 5, 6, 7);
        // Format 0 = fp8 e4m3 for both operands; E8M0 scale 127 = 2^0.
        acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc, 0, 0, 0, 127, 0, 127);
    }
};

template <>
struct Mma<2> {
    static constexpr int NV = 8;
    static constexpr int STEPS = 8;
    KVIP_DEVICE static void step(int s, const v4i (&a)[NV], const v4i (&b)[NV], v16f& acc) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a[s]), __builtin_bit_cast(v8bf, b[s]),
                                                      acc, 0, 0, 0);
    }
};

// LDS piece swizzle of a staged K row (8 or 16 pieces of 16 bytes per row).
template <int ELEM>
KVIP_DEVICE int swizzle(int row) {
    return ELEM == 1 ? ((row >> 1) & 7) : (row & 15);
}

}  // namespace kvip
