// MFMA / VALU co-issue probe (measurement only; no reference counterpart): the rate at
// which one SIMD retires fp8 v_mfma_scale_f32_32x32x64_f8f6f4 when every MFMA is
// interleaved with V/4 independent fp32 VALU ops, for V = 0, 32, 64, 88 or 96 VALU ops per
// 4 MFMAs. bench.py --coissue times it to price a scoring epilogue of a given VALU density
// (the prefill indexer issues 22 VALU instructions per MFMA) against the MFMA-only rate.
//
// Each wave keeps 4 independent accumulators; the VALU ops are FMA chains on registers of
// their own (no dependency on the MFMAs), placed between the MFMAs by sched_group_barrier.
// The only memory access is one float per thread written at the end (the sum of every
// register, so that nothing is optimised away).
#include "kvip_device.h"

namespace kvip {
namespace {

template <int V>
__global__ __launch_bounds__(256) void coissue_probe_kernel(float* out, int iters, float y, float z) {
    const int t = threadIdx.x;
    v8i a = v8i{t, t + 1, t + 2, t + 3, t + 4, t + 5, t + 6, t + 7} & 0x37373737;
    const v8i b = a ^ 0x11111111;
    v16f acc[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) acc[m] = v16f{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    constexpr int kRegs = V > 0 ? V : 1;
    float x[kRegs];
#pragma unroll
    for (int j = 0; j < kRegs; ++j) x[j] = t * 0.001f + j;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            acc[m] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc[m], 0, 0, 0, 127, 0, 127);
#pragma unroll
            for (int j = m * (V / 4); j < (m + 1) * (V / 4); ++j) x[j] = fmaf(x[j], y, z);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, V / 4, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kRegs; ++j) s += x[j];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
        for (int i = 0; i < 16; ++i) s += acc[m][i];
    }
    out[static_cast<size_t>(blockIdx.x) * 256 + t] = s;
}

}  // namespace
}  // namespace kvip

// Launches the probe with `blocks` workgroups of 256 threads (one wave per SIMD per
// workgroup; 256 x waves_per_simd blocks fill an MI355X with that many waves per SIMD);
// out holds blocks * 256 floats. KVIP_ERR_INVALID for other V or sizes.
extern "C" uint32_t kvip_hip_probe_coissue(int32_t valu_per_4_mfma, int32_t blocks, int32_t iters, float* out,
                                           void* stream) {
    if (out == nullptr || blocks < 1 || blocks > 65536 || iters < 1) return KVIP_ERR_INVALID;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    switch (valu_per_4_mfma) {
        case 0: hipLaunchKernelGGL(kvip::coissue_probe_kernel<0>, dim3(blocks), dim3(256), 0, s, out, iters, 1.0001f, 0.5f); break;
        case 32: hipLaunchKernelGGL(kvip::coissue_probe_kernel<32>, dim3(blocks), dim3(256), 0, s, out, iters, 1.0001f, 0.5f); break;
        case 64: hipLaunchKernelGGL(kvip::coissue_probe_kernel<64>, dim3(blocks), dim3(256), 0, s, out, iters, 1.0001f, 0.5f); break;
        case 88: hipLaunchKernelGGL(kvip::coissue_probe_kernel<88>, dim3(blocks), dim3(256), 0, s, out, iters, 1.0001f, 0.5f); break;
        case 96: hipLaunchKernelGGL(kvip::coissue_probe_kernel<96>, dim3(blocks), dim3(256), 0, s, out, iters, 1.0001f, 0.5f); break;
        default: return KVIP_ERR_INVALID;
    }
    return static_cast<uint32_t>(hipGetLastError());
}
