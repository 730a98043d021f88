// Sparse attention over the 2048 selected KV rows of each query row: the consumer of the
// LIFetch outputs (the sparse flash attention the reference's service runs on the hot
// cache, tests/operators/lifetch/support/correctness.py:261-339; row format
// workloads.py:493-515).
//
// A 656-byte row holds 512 fp8 e4m3 "nope" features, 64 bf16 rope features and four fp32
// scales (one per 128 nope features). key = [nope * scale, rope] (576 features), value =
// nope * scale (512). For query row r and head h:
//   out[r, h] = sum_j bf16(p_j) value_j / sum_j p_j,  p_j = exp(s_j - max_j s_j),
//   s_j = scale * <q[r, h], key_j>  over the row's indices j >= 0,
// i.e. softmax attention with bf16 probabilities in the value product (the reference rounds
// the normalised probabilities to bf16; here the unnormalised ones, divided once at the end).
//
// One workgroup per (query row, group of 16 heads, split of the 2048 indices) streams its
// indices in tiles of 64 tokens: the rows are gathered (all loads of a tile in flight at once)
// and dequantised to bf16 in LDS with the hardware conversions (v_cvt_pk_f32_fp8, OCP e4m3 on
// gfx950, and v_cvt_pk_bf16_f32), the logits of the tile come from bf16 MFMA
// (v_mfma_f32_16x16x32_bf16: 16 heads x 16 tokens x 32 features), an online softmax keeps the
// running maximum and sum per head, and the value product is a second MFMA (16 heads x 16
// features x 32 tokens) accumulated in registers. Splits (up to 8, enough workgroups to fill
// the chip) leave (max, sum, unnormalised output) per head in the workspace and a second
// launch merges them. HBM traffic is one read of each selected row plus the partials.
#include "kvip_device.h"

namespace kvip {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

constexpr int kSaThreads = 256;
constexpr int kSaTile = 64;                 // tokens per tile
constexpr int kSaHeads = 16;                // heads per workgroup (MFMA M)
constexpr int kKeyDim = 576;                // 512 nope + 64 rope
constexpr int kValueDim = 512;
constexpr int kPieces = KVIP_KV_ROW_BYTES / 16;  // 41 pieces of a row, the last holds the scales
constexpr int kPitch = kKeyDim + 8;         // bf16 per LDS key row (16 bytes of padding)
constexpr int kPPitch = kSaTile + 8;        // bf16 per LDS probability row
constexpr int kStageIters = (kSaTile * (kPieces - 1) + kSaThreads - 1) / kSaThreads;
constexpr int kPartial = 2 * kSaHeads + kSaHeads * kValueDim;  // floats per split: max, sum, output
constexpr int kMaxSplits = 8;

// Index splits per (row, head group): doubled up to 8 while the launch has fewer than 512
// workgroups.
__host__ __device__ inline int sa_splits(int rows, int groups) {
    int s = 1;
    while (s < kMaxSplits && static_cast<int64_t>(rows) * groups * s < 512) s *= 2;
    return s;
}

KVIP_DEVICE uint32_t pack_bf16(float a, float b) {  // hardware round to nearest even
    const bf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
    uint32_t u;
    __builtin_memcpy(&u, &v, 4);
    return u;
}

KVIP_DEVICE uint16_t bf16_bits(float f) {  // round to nearest even (finite inputs)
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

KVIP_DEVICE bf16x8 as_bf16x8(v4i v) {
    bf16x8 r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

__global__ __launch_bounds__(kSaThreads) void sparse_attention_kernel(const KvipSparseAttnArgs p) {
    __shared__ __align__(16) uint16_t s_k[kSaTile * kPitch];
    __shared__ __align__(16) uint16_t s_p[kSaHeads * kPPitch];
    __shared__ float s_red[4][kSaHeads];
    __shared__ int64_t s_src[kSaTile];

    // XCD-aware order: the workgroups of a query row (head groups x splits) share
    // blockIdx % 8, so they run on one XCD, whose L2 then serves the row's KV rows and query to
    // every head group after the first read.
    const int groups = (p.heads + kSaHeads - 1) / kSaHeads;
    const int splits = sa_splits(p.rows, groups);
    const int units = groups * splits;
    const int chunk = blockIdx.x / (8 * units), within = blockIdx.x % (8 * units);
    const int r = chunk * 8 + within % 8;
    const int unit = within / 8, hg = unit % groups, sp = unit / groups;
    const int h0 = hg * kSaHeads;
    if (r >= p.rows) return;
    const int b = r / p.rows_per_request;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;  // MFMA lane row / group
    uint32_t err = 0;

    // Query fragments (A operand of the logits): head h0 + lr, features 32 s + 8 lg .. + 8.
    bf16x8 qf[kKeyDim / 32];
    {
        const bool live = h0 + lr < p.heads;
        const uint16_t* q = p.query + (static_cast<size_t>(r) * p.heads + (live ? h0 + lr : 0)) * kKeyDim;
#pragma unroll
        for (int s = 0; s < kKeyDim / 32; ++s) {
            const v4i v = live ? *reinterpret_cast<const v4i*>(q + s * 32 + lg * 8) : v4i{0, 0, 0, 0};
            qf[s] = as_bf16x8(v);
        }
    }
    f32x4 acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run[4], l_part[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m_run[i] = -INFINITY;
        l_part[i] = 0.f;
    }
    const int* idx_row = p.indices + static_cast<size_t>(r) * kTopK;
    const int capacity = p.max_blocks * kBlockTokens;

    const int span = kTopK / splits;
    for (int t0 = sp * span; t0 < (sp + 1) * span; t0 += kSaTile) {
        // Source rows of the tile.
        if (tid < kSaTile) {
            const int t = idx_row[t0 + tid];
            int64_t src = -1;
            if (t >= capacity) {
                err |= KVIP_STATUS_BAD_TOKEN;
            } else if (t >= 0) {
                const int blk = p.block_table[static_cast<size_t>(b) * p.max_blocks + (t >> 7)];
                if (static_cast<unsigned>(blk) < static_cast<unsigned>(p.num_blocks)) {
                    src = static_cast<int64_t>(blk) * p.kv_block_stride + static_cast<int64_t>(t & 127) * p.row_stride;
                } else {
                    err |= KVIP_STATUS_BAD_BLOCK;
                }
            }
            s_src[tid] = src;
        }
        __syncthreads();
        // Gather + dequantise: pieces 0..31 are 16 nope bytes, 32..39 8 rope values; the loads
        // of half a tile are issued before their conversions (a whole tile's would cost the
        // registers of a second wave per SIMD).
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            constexpr int kHalf = (kStageIters + 1) / 2;
            v4i raw[kHalf];
            float sc[kHalf];
#pragma unroll
            for (int j = 0; j < kHalf; ++j) {
                const int q = (half * kHalf + j) * kSaThreads + tid;
                raw[j] = v4i{0, 0, 0, 0};
                sc[j] = 0.f;
                if (half * kHalf + j < kStageIters && q < kSaTile * (kPieces - 1)) {
                    const int i = q / (kPieces - 1), pc = q - i * (kPieces - 1);
                    const int64_t src = s_src[i];
                    if (src >= 0) {
                        const uint8_t* row = p.kv_cache + src;
                        raw[j] = *reinterpret_cast<const v4i*>(row + (pc < 32 ? pc * 16 : 512 + (pc - 32) * 16));
                        if (pc < 32) sc[j] = *reinterpret_cast<const float*>(row + 640 + (pc >> 3) * 4);
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < kHalf; ++j) {
                const int q = (half * kHalf + j) * kSaThreads + tid;
                if (half * kHalf + j < kStageIters && q < kSaTile * (kPieces - 1)) {
                    const int i = q / (kPieces - 1), pc = q - i * (kPieces - 1);
                    uint16_t* dst = s_k + i * kPitch;
                    if (pc < 32) {
                        uint32_t out[8];
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(raw[j][k], false);
                            const f32x2 c = __builtin_amdgcn_cvt_pk_f32_fp8(raw[j][k], true);
                            out[2 * k] = pack_bf16(a[0] * sc[j], a[1] * sc[j]);
                            out[2 * k + 1] = pack_bf16(c[0] * sc[j], c[1] * sc[j]);
                        }
                        v4i* d = reinterpret_cast<v4i*>(dst + pc * 16);
                        d[0] = v4i{static_cast<int>(out[0]), static_cast<int>(out[1]), static_cast<int>(out[2]),
                                   static_cast<int>(out[3])};
                        d[1] = v4i{static_cast<int>(out[4]), static_cast<int>(out[5]), static_cast<int>(out[6]),
                                   static_cast<int>(out[7])};
                    } else {
                        *reinterpret_cast<v4i*>(dst + 512 + (pc - 32) * 8) = raw[j];
                    }
                }
            }
        }
        __syncthreads();

        // Logits of tokens 16 w .. 16 w + 15: lane holds heads 4 lg + i of token 16 w + lr.
        f32x4 sv = f32x4{0.f, 0.f, 0.f, 0.f};
        {
            const uint16_t* kr = s_k + (w * 16 + lr) * kPitch + lg * 8;
#pragma unroll
            for (int s = 0; s < kKeyDim / 32; ++s) {
                const bf16x8 kv = as_bf16x8(*reinterpret_cast<const v4i*>(kr + s * 32));
                sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qf[s], kv, sv, 0, 0, 0);
            }
        }
        const bool tok_live = s_src[w * 16 + lr] >= 0;
        float lg_v[4], mx[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lg_v[i] = tok_live ? sv[i] * p.scale : -INFINITY;
            float m = lg_v[i];
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
            mx[i] = m;
        }
        if (lr == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) s_red[w][lg * 4 + i] = mx[i];
        }
        __syncthreads();
        float alpha[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int h = lg * 4 + i;
            const float tile_max = fmaxf(fmaxf(s_red[0][h], s_red[1][h]), fmaxf(s_red[2][h], s_red[3][h]));
            const float m_new = fmaxf(m_run[i], tile_max);
            alpha[i] = m_new == -INFINITY ? 1.f : __expf(m_run[i] - m_new);
            m_run[i] = m_new;
            const float pr = m_new == -INFINITY ? 0.f : __expf(lg_v[i] - m_new);
            const uint16_t pb = bf16_bits(pr);
            l_part[i] = l_part[i] * alpha[i] + pr;
            s_p[h * kPPitch + w * 16 + lr] = pb;
        }
        __syncthreads();

        // Value product for features 128 w .. 128 w + 127 (8 MFMA columns of 16).
#pragma unroll
        for (int t = 0; t < 8; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][i] *= alpha[i];
        }
#pragma unroll
        for (int ks = 0; ks < kSaTile / 32; ++ks) {
            const bf16x8 pa = as_bf16x8(*reinterpret_cast<const v4i*>(s_p + lr * kPPitch + ks * 32 + lg * 8));
            const uint16_t* vr = s_k + (ks * 32 + lg * 8) * kPitch + w * 128 + lr;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                uint32_t pk[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    pk[j] = static_cast<uint32_t>(vr[(2 * j) * kPitch + t * 16]) |
                            (static_cast<uint32_t>(vr[(2 * j + 1) * kPitch + t * 16]) << 16);
                }
                const v4i vb = v4i{static_cast<int>(pk[0]), static_cast<int>(pk[1]), static_cast<int>(pk[2]),
                                   static_cast<int>(pk[3])};
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, as_bf16x8(vb), acc[t], 0, 0, 0);
            }
        }
        __syncthreads();  // s_k, s_p and s_red are rewritten by the next tile
    }

    // Row sums: over the 16 lanes of a group, then over the waves.
    float l_tot[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float l = l_part[i];
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) l += __shfl_xor(l, o);
        if (lr == 0) s_red[w][lg * 4 + i] = l;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int h = lg * 4 + i;
        l_tot[i] = s_red[0][h] + s_red[1][h] + s_red[2][h] + s_red[3][h];
    }
    if (splits > 1) {  // partial of this split: max and sum per head, unnormalised output
        float* ws = p.workspace + ((static_cast<size_t>(r) * groups + hg) * splits + sp) * kPartial;
        if (w == 0 && lr == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                ws[lg * 4 + i] = m_run[i];
                ws[kSaHeads + lg * 4 + i] = l_tot[i];
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float* o = ws + 2 * kSaHeads + (lg * 4 + i) * kValueDim + w * 128 + lr;
#pragma unroll
            for (int t = 0; t < 8; ++t) o[t * 16] = acc[t][i];
        }
        report(p.status, err);
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int h = h0 + lg * 4 + i;
        if (h >= p.heads) continue;
        const float inv = l_tot[i] > 0.f ? 1.f / l_tot[i] : 0.f;
        float* o = p.output + (static_cast<size_t>(r) * p.heads + h) * kValueDim + w * 128 + lr;
#pragma unroll
        for (int t = 0; t < 8; ++t) o[t * 16] = acc[t][i] * inv;
    }
    report(p.status, err);
}

// Merge of the splits: workgroup (row, head group, 64-feature chunk).
__global__ __launch_bounds__(kSaThreads) void sparse_attention_merge_kernel(const KvipSparseAttnArgs p) {
    __shared__ float s_w[kMaxSplits][kSaHeads];
    __shared__ float s_inv[kSaHeads];
    const int groups = (p.heads + kSaHeads - 1) / kSaHeads;
    const int splits = sa_splits(p.rows, groups);
    const int unit = blockIdx.x / 8, part = blockIdx.x % 8;
    const int r = unit / groups, h0 = (unit % groups) * kSaHeads;
    const float* ws = p.workspace + static_cast<size_t>(unit) * splits * kPartial;
    const int tid = threadIdx.x;
    if (tid < kSaHeads) {
        float m = -INFINITY;
        for (int s = 0; s < splits; ++s) m = fmaxf(m, ws[s * kPartial + tid]);
        float l = 0.f;
        for (int s = 0; s < splits; ++s) {
            const float wgt = m == -INFINITY ? 0.f : __expf(ws[s * kPartial + tid] - m);
            s_w[s][tid] = wgt;
            l += wgt * ws[s * kPartial + kSaHeads + tid];
        }
        s_inv[tid] = l > 0.f ? 1.f / l : 0.f;
    }
    __syncthreads();
    // One thread per 4 features of one head (16 heads x 64 features = 256 float4).
    const int h = tid / 16, col = part * 64 + (tid % 16) * 4;
    if (h0 + h < p.heads) {
        f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < splits; ++s) {
            const f32x4 o = *reinterpret_cast<const f32x4*>(ws + s * kPartial + 2 * kSaHeads + h * kValueDim + col);
            v += s_w[s][h] * o;
        }
        *reinterpret_cast<f32x4*>(p.output + (static_cast<size_t>(r) * p.heads + h0 + h) * kValueDim + col) =
            v * s_inv[h];
    }
}

}  // namespace

uint64_t sparse_attention_workspace_bytes(int rows, int heads) {
    if (rows < 1 || heads < 1) return 0;
    const int groups = (heads + kSaHeads - 1) / kSaHeads;
    const int splits = sa_splits(rows, groups);
    return splits > 1 ? static_cast<uint64_t>(rows) * groups * splits * kPartial * sizeof(float) : 0;
}

uint32_t validate_sparse_attention(const KvipSparseAttnArgs* a) {
    if (a == nullptr) return KVIP_ERR_INVALID;
    const bool ok = a->query && a->kv_cache && a->block_table && a->indices && a->output && a->rows >= 1 &&
                    a->rows_per_request >= 1 && a->rows % a->rows_per_request == 0 && a->heads >= 1 &&
                    a->heads <= 128 && a->max_blocks >= 1 && a->max_blocks <= (1 << 24) / kBlockTokens &&
                    a->num_blocks >= 1 && a->row_stride >= KVIP_KV_ROW_BYTES && a->row_stride % 16 == 0 &&
                    a->kv_block_stride % 16 == 0 &&
                    a->kv_block_stride >= static_cast<int64_t>(kBlockTokens) * a->row_stride &&
                    (reinterpret_cast<uintptr_t>(a->kv_cache) & 15u) == 0 &&
                    (reinterpret_cast<uintptr_t>(a->query) & 15u) == 0 && a->rows <= 65535 * 64 &&
                    (a->workspace != nullptr || sparse_attention_workspace_bytes(a->rows, a->heads) == 0);
    return ok ? KVIP_OK : KVIP_ERR_INVALID;
}

}  // namespace kvip

extern "C" uint32_t kvip_hip_sparse_attention(const KvipSparseAttnArgs* args, void* stream) {
    const uint32_t rc = kvip::validate_sparse_attention(args);
    if (rc != KVIP_OK) return rc;
    const int groups = (args->heads + kvip::kSaHeads - 1) / kvip::kSaHeads;
    const int splits = kvip::sa_splits(args->rows, groups);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(kvip::sparse_attention_kernel, dim3(((args->rows + 7) / 8) * 8 * groups * splits),
                       dim3(kvip::kSaThreads), 0, s, *args);
    if (splits > 1) {
        hipLaunchKernelGGL(kvip::sparse_attention_merge_kernel, dim3(args->rows * groups * 8), dim3(kvip::kSaThreads),
                           0, s, *args);
    }
    return static_cast<uint32_t>(hipGetLastError());
}

extern "C" uint64_t kvip_hip_sparse_attention_workspace_bytes(int32_t rows, int32_t heads) {
    return kvip::sparse_attention_workspace_bytes(rows, heads);
}
