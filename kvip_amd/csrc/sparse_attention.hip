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
// Up to 32 heads, one workgroup per (query row, set of one or two groups of 16 heads, split
// of the 2048 indices) resolves its indices to cache rows once (block table), then streams them
// in tiles of 64 tokens: a tile's rows are gathered into registers two tiles ahead,
// dequantised to bf16 with the hardware conversions (v_cvt_pk_f32_fp8, OCP e4m3 on gfx950,
// and v_cvt_pk_bf16_f32) into one of two token-major LDS tile buffers once for every head
// group of the set, the logits of the tile come from bf16 MFMA
// (v_mfma_f32_16x16x32_bf16: 16 heads x 16 tokens x 32 features), an online softmax keeps the
// running maximum and sum per head, and the value product is a second MFMA (16 heads x 16
// features x 32 tokens) accumulated in registers, its value fragments (8 tokens of one
// feature per lane) read from the same key tile by gfx950's transpose loads
// (ds_read_b64_tr_b16); the next tile is staged beside it. Splits (up to 8, enough workgroups to fill
// the chip) leave (max, sum, unnormalised output) per head in the workspace and a second
// launch merges them. HBM traffic is one read of each selected row plus the partials.
// More than 32 heads run on sparse_attention_pair_kernel (groups of four waves per 32 heads,
// 32x32x16 MFMAs, described there), which leaves the same partial records.
#include "kvip_device.h"

namespace kvip {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef short v4s __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));

constexpr int kSaThreads = 256;
constexpr int kSaTile = 64;                 // tokens per tile
constexpr int kSaHeads = 16;                // heads per workgroup (MFMA M)
constexpr int kKeyDim = 576;                // 512 nope + 64 rope
constexpr int kValueDim = 512;
constexpr int kPieces = KVIP_KV_ROW_BYTES / 16;  // 41 pieces of a row, the last holds the scales
constexpr int kPitch = kKeyDim + 8;         // bf16 per LDS key row (16 bytes of padding)
constexpr int kPPitch = kSaTile + 8;        // bf16 per LDS probability row
constexpr int kTokGroup = 8;  // tokens staged per thread
constexpr int kPartial = 2 * kSaHeads + kSaHeads * kValueDim;  // floats per split: max, sum, output
constexpr int kMaxSplits = 8;

// Index splits per (row, head-group set): doubled up to 8 while the launch has fewer than 256
// workgroups (one per CU: the kernel holds one workgroup per CU).
__host__ __device__ inline int sa_splits(int rows, int sets) {
    int s = 1;
    while (s < kMaxSplits && static_cast<int64_t>(rows) * sets * s < 256) s *= 2;
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

// Value of the lane chosen by a DPP control within each row of 16 lanes.
template <int CTRL>
KVIP_DEVICE float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
// Max / sum over the 16 lanes of a row, in every lane of it: row mirror, half-row mirror,
// then the two quad swaps; every lane's value enters each result exactly once.
KVIP_DEVICE float row_max16(float x) {
    x = fmaxf(x, dpp<0x140>(x));  // row_mirror
    x = fmaxf(x, dpp<0x141>(x));  // row_half_mirror
    x = fmaxf(x, dpp<0xB1>(x));   // quad_perm [1, 0, 3, 2]
    return fmaxf(x, dpp<0x4E>(x));  // quad_perm [2, 3, 0, 1]
}
KVIP_DEVICE float row_sum16(float x) {
    x += dpp<0x140>(x);
    x += dpp<0x141>(x);
    x += dpp<0xB1>(x);
    return x + dpp<0x4E>(x);
}

KVIP_DEVICE bf16x8 as_bf16x8(v4i v) {
    bf16x8 r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

// Head groups of 16 handled by one workgroup: G share every staged tile (its gather and
// dequantisation); group g runs on waves 4 g .. 4 g + 3, which keep its Q fragments,
// online-softmax state and value accumulators in registers (G waves per SIMD).
__host__ __device__ inline int sa_group_set(int heads) { return heads > kSaHeads ? 2 : 1; }
// Workgroups per row before index splits: more than 32 heads run on
// sparse_attention_pair_kernel, kPrGroups groups of 32 heads per workgroup, kPrSplit waves
// per group.
constexpr int kPrGroups = 2;
constexpr int kPrSplit = 4;
__host__ __device__ inline bool sa_pairs(int heads) { return heads > 2 * kSaHeads; }
__host__ __device__ inline int sa_sets(int heads) {
    if (sa_pairs(heads)) return ((heads + 31) / 32 + kPrGroups - 1) / kPrGroups;
    const int groups = (heads + kSaHeads - 1) / kSaHeads;
    return (groups + sa_group_set(heads) - 1) / sa_group_set(heads);
}

template <int G>
__global__ __launch_bounds__(kSaThreads * G, 1) void sparse_attention_kernel(const KvipSparseAttnArgs p) {
    constexpr int kThreads = kSaThreads * G;
    constexpr int kFeat = 16 / G;  // nope features per thread and token (16-byte or 8-byte pieces)
    __shared__ __align__(16) uint16_t s_k[2][kSaTile * kPitch];      // keys, token-major, two tiles
    __shared__ __align__(16) uint16_t s_p[G][kSaHeads * kPPitch];
    __shared__ float s_red[G][4][kSaHeads];
    __shared__ int32_t s_row[kTopK];  // cache row (block * 128 + offset) of each index, -1 = none

    // XCD-aware order: the workgroups of a query row (head-group sets x splits) share
    // blockIdx % 8, so they run on one XCD, whose L2 then serves the row's KV rows and query to
    // every set after the first read.
    const int groups = (p.heads + kSaHeads - 1) / kSaHeads;
    const int sets = (groups + G - 1) / G;
    const int splits = sa_splits(p.rows, sets);
    const int units = sets * splits;
    const int chunk = blockIdx.x / (8 * units), within = blockIdx.x % (8 * units);
    const int r = chunk * 8 + within % 8;
    const int unit = within / 8, hs = unit % sets, sp = unit / sets;
    if (r >= p.rows) return;
    const int b = r / p.rows_per_request;
    const int tid = threadIdx.x, lane = tid & 63;
    const int gw = tid >> 8;           // head group of this wave within the set
    const int w = (tid >> 6) & 3;      // quarter: logits of tokens 16 w .., values of features 128 w ..
    const int lr = lane & 15, lg = lane >> 4;  // MFMA lane row / group
    const int grp = hs * G + gw;
    const bool live = grp < groups;    // uniform per wave: a set's last group may hold no heads
    uint32_t err = 0;

    // Cache rows of the split's indices, resolved once through the block table.
    const int span = kTopK / splits;
    const int* idx_row = p.indices + static_cast<size_t>(r) * kTopK + sp * span;
    const int capacity = p.max_blocks * kBlockTokens;
    for (int i = tid; i < span; i += kThreads) {
        const int t = idx_row[i];
        int row = -1;
        if (t >= capacity) {
            err |= KVIP_STATUS_BAD_TOKEN;
        } else if (t >= 0) {
            const int blk = p.block_table[static_cast<size_t>(b) * p.max_blocks + (t >> 7)];
            if (static_cast<unsigned>(blk) < static_cast<unsigned>(p.num_blocks)) {
                row = blk * kBlockTokens + (t & 127);
            } else {
                err |= KVIP_STATUS_BAD_BLOCK;
            }
        }
        s_row[i] = row;
    }

    // Query fragments (A operand of the logits) of the wave's group: head 16 grp + lr,
    // features 32 s + 8 lg .. + 8; heads past p.heads read as zero.
    bf16x8 qf[kKeyDim / 32];
    {
        const int h = grp * kSaHeads + lr;
        const bool hl = h < p.heads;
        const uint16_t* q = p.query + (static_cast<size_t>(r) * p.heads + (hl ? h : 0)) * kKeyDim;
#pragma unroll
        for (int s = 0; s < kKeyDim / 32; ++s) {
            const v4i v = hl ? *reinterpret_cast<const v4i*>(q + s * 32 + lg * 8) : v4i{0, 0, 0, 0};
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
    __syncthreads();

    // Staging map: thread (token group tg, nope slice pc) holds kFeat nope features
    // [16 pc' + kFeat h, + kFeat) of the 8 tokens 8 tg .. 8 tg + 7 (pc' = pc % 32, h = the
    // thread's half of the piece when two workgroup halves share it), and the tile's 512
    // rope pieces are dealt over every thread. Tile k + 2's pieces are requested right after
    // tile k + 1 is staged (during tile k), so that their latency passes under a whole tile.
    const int tg = (tid >> 5) & 7, pc = tid & 31, half = tid >> 8;
    const int f0 = pc * 16 + half * kFeat;  // first nope feature of the thread
    constexpr int kRope = kSaTile * 8 / kThreads;
    typedef int vfi __attribute__((ext_vector_type(kFeat / 4)));
    vfi nope[kTokGroup];
    v4i rope[kRope];
    float sc[kTokGroup];
    auto row_base = [&](int row) {
        return p.kv_cache + static_cast<int64_t>(row >> 7) * p.kv_block_stride +
               static_cast<int64_t>(row & 127) * p.row_stride;
    };
    auto load_tile = [&](int k) {
#pragma unroll
        for (int u = 0; u < kTokGroup; ++u) {
            const int row = s_row[k * kSaTile + tg * kTokGroup + u];
            nope[u] = vfi{};
            sc[u] = 0.f;
            if (row >= 0) {
                const uint8_t* base = row_base(row);
                nope[u] = *reinterpret_cast<const vfi*>(base + f0);
                sc[u] = *reinterpret_cast<const float*>(base + 640 + (pc >> 3) * 4);
            }
        }
#pragma unroll
        for (int j = 0; j < kRope; ++j) {
            const int q = j * kThreads + tid;
            const int row = s_row[k * kSaTile + (q >> 3)];
            rope[j] = row >= 0 ? *reinterpret_cast<const v4i*>(row_base(row) + 512 + (q & 7) * 16) : v4i{0, 0, 0, 0};
        }
    };
    // Dequantisation to bf16: keys [nope * scale, rope] token-major into tile buffer kb. The
    // values are the same nope * scale features, read feature-wise by the transpose loads.
    auto stage_tile = [&](uint16_t* kb) {
#pragma unroll
        for (int u = 0; u < kTokGroup; ++u) {
            uint32_t out[kFeat / 2];  // features f0 + 2k, 2k + 1
#pragma unroll
            for (int k = 0; k < kFeat / 4; ++k) {
                const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(nope[u][k], false);
                const f32x2 c = __builtin_amdgcn_cvt_pk_f32_fp8(nope[u][k], true);
                out[2 * k] = pack_bf16(a[0] * sc[u], a[1] * sc[u]);
                out[2 * k + 1] = pack_bf16(c[0] * sc[u], c[1] * sc[u]);
            }
            uint16_t* d = kb + (tg * kTokGroup + u) * kPitch + f0;
            if constexpr (kFeat == 16) {
                reinterpret_cast<v4i*>(d)[0] = v4i{static_cast<int>(out[0]), static_cast<int>(out[1]),
                                                   static_cast<int>(out[2]), static_cast<int>(out[3])};
                reinterpret_cast<v4i*>(d)[1] = v4i{static_cast<int>(out[4]), static_cast<int>(out[5]),
                                                   static_cast<int>(out[6]), static_cast<int>(out[7])};
            } else {
                *reinterpret_cast<v4i*>(d) = v4i{static_cast<int>(out[0]), static_cast<int>(out[1]),
                                                 static_cast<int>(out[2]), static_cast<int>(out[3])};
            }
        }
#pragma unroll
        for (int j = 0; j < kRope; ++j) {
            const int q = j * kThreads + tid;
            *reinterpret_cast<v4i*>(kb + (q >> 3) * kPitch + 512 + (q & 7) * 8) = rope[j];
        }
    };
    // Transpose-load address of this lane within a tile: in 16-lane block lg, lane lr reads 4
    // features of one token and receives one feature (lr) of 4 consecutive tokens, i.e. block lg
    // covers tokens 8 lg + 4 j .. + 4 (j = 0, 1: two loads) of 16 features: the B operand lane
    // (feature lr, tokens 8 lg .. + 8) of the value MFMA.
    const int tr_off = (8 * lg + (lr >> 2)) * kPitch + 4 * (lr & 3);

    const int tiles = span / kSaTile;
    load_tile(0);
    stage_tile(s_k[0]);
    if (tiles > 1) load_tile(1);
    __syncthreads();  // s_k[0] holds tile 0
    for (int k = 0; k < tiles; ++k) {
        const uint16_t* kt = s_k[k & 1];
        const bool more = k + 1 < tiles;
        const bool tok_live = s_row[k * kSaTile + w * 16 + lr] >= 0;
        // Logits of tokens 16 w .. 16 w + 15: lane holds heads 4 lg + i of token 16 w + lr.
        float lg_v[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        if (live) {
            f32x4 sv = f32x4{0.f, 0.f, 0.f, 0.f};
            const uint16_t* kr = kt + (w * 16 + lr) * kPitch + lg * 8;
#pragma unroll
            for (int s = 0; s < kKeyDim / 32; ++s) {
                const bf16x8 kv = as_bf16x8(*reinterpret_cast<const v4i*>(kr + s * 32));
                sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qf[s], kv, sv, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lg_v[i] = tok_live ? sv[i] * p.scale : -INFINITY;
                const float mx = row_max16(lg_v[i]);
                if (lr == 0) s_red[gw][w][lg * 4 + i] = mx;
            }
        }
        __syncthreads();
        float alpha[4] = {1.f, 1.f, 1.f, 1.f};
        if (live) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int h = lg * 4 + i;
                const float tile_max =
                    fmaxf(fmaxf(s_red[gw][0][h], s_red[gw][1][h]), fmaxf(s_red[gw][2][h], s_red[gw][3][h]));
                const float m_new = fmaxf(m_run[i], tile_max);
                alpha[i] = m_new == -INFINITY ? 1.f : __expf(m_run[i] - m_new);
                m_run[i] = m_new;
                const float pr = m_new == -INFINITY ? 0.f : __expf(lg_v[i] - m_new);
                l_part[i] = l_part[i] * alpha[i] + pr;
                s_p[gw][h * kPPitch + w * 16 + lr] = bf16_bits(pr);
            }
        }
        __syncthreads();  // s_p complete; s_red free for the next tile
        if (live) {
            // Value product for features 128 w .. 128 w + 127 (8 MFMA columns of 16).
#pragma unroll
            for (int t = 0; t < 8; ++t) {
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][i] *= alpha[i];
            }
#pragma unroll
            for (int ks = 0; ks < kSaTile / 32; ++ks) {
                const bf16x8 pa = as_bf16x8(*reinterpret_cast<const v4i*>(&s_p[gw][lr * kPPitch + ks * 32 + lg * 8]));
                // B fragment: tokens ks * 32 + 8 lg .. + 8 of feature 128 w + 16 t + lr.
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const uint16_t* vr = kt + tr_off + ks * 32 * kPitch + w * 128 + t * 16;
                    const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(vr));
                    const v4s hi =
                        __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(vr + 4 * kPitch));
                    const bf16x8 vb = __builtin_bit_cast(bf16x8, v8s{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, vb, acc[t], 0, 0, 0);
                }
            }
            // The next tile's staging beside this tile's value MFMAs, then the loads of the
            // tile after it.
            if (more) {
                stage_tile(s_k[(k + 1) & 1]);
                if (k + 2 < tiles) load_tile(k + 2);
            }
        } else if (more) {
            stage_tile(s_k[(k + 1) & 1]);
            if (k + 2 < tiles) load_tile(k + 2);
        }
        __syncthreads();  // tile k + 1 staged; tile k's buffer and s_p free
    }

    // Row sums: over the 16 lanes of a group, then over the group's waves; then this split's
    // partial (max, sum, unnormalised output per head) or the normalised output.
    float l_tot[4];
    if (live) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float l = row_sum16(l_part[i]);
            if (lr == 0) s_red[gw][w][lg * 4 + i] = l;
        }
    }
    __syncthreads();
    if (live) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int h = lg * 4 + i;
            l_tot[i] = s_red[gw][0][h] + s_red[gw][1][h] + s_red[gw][2][h] + s_red[gw][3][h];
        }
        if (splits > 1) {
            float* ws = p.workspace + ((static_cast<size_t>(r) * groups + grp) * splits + sp) * kPartial;
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
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int h = grp * kSaHeads + lg * 4 + i;
                if (h >= p.heads) continue;
                const float inv = l_tot[i] > 0.f ? 1.f / l_tot[i] : 0.f;
                float* o = p.output + (static_cast<size_t>(r) * p.heads + h) * kValueDim + w * 128 + lr;
#pragma unroll
                for (int t = 0; t < 8; ++t) o[t * 16] = acc[t][i] * inv;
            }
        }
    }
    report(p.status, err);
}

// More than 32 heads: groups of SPLIT = 4 waves per 32 heads. A workgroup (row, index split)
// holds GROUPS such groups (GROUPS x 32 heads), so a staged tile of 32 rows serves all of
// them once. Wave (th, hh) of a group computes the logits of the tile's tokens 16 th .. + 16
// for heads 16 hh .. + 16 over all 576 features (v_mfma_f32_16x16x32_bf16, tokens as M, its 16
// heads' query fragments as N), so no partial logits are exchanged and each logit is
// exponentiated once: the two token halves exchange only their per-head maxima (LDS), every
// wave of the group derives the same reference maxima for all 32 heads from them, and each
// writes its 16 x 16 block of bf16 probabilities to LDS. For the value product each wave then
// takes all 32 heads (v_mfma_f32_32x32x16_bf16, heads as M, probabilities read from LDS as the
// A operand) and accumulates 512 / SPLIT of the value features (blocks of 32). The values are
// the key tile's nope features: the value MFMA's B operand (8 tokens of one feature per lane)
// comes from the token-major key tile by gfx950's transpose loads (ds_read_b64_tr_b16), so a
// tile is dequantised and written to LDS once, and two tile buffers let the next tile be
// staged beside this tile's value MFMAs (three barriers per tile). The running maximum is
// rescaled lazily: only when a tile's maximum exceeds it by kPrMargin (the probabilities are
// then at most e^kPrMargin, well inside bf16 and fp32), which after the first tiles of a row
// is rare, so the 128 accumulators per lane are seldom touched outside the MFMAs.
constexpr int kPrTile = 32;                  // tokens per tile
constexpr int kPrKPitch = kKeyDim + 8;       // bf16 per K row: an odd number of 16-byte units
constexpr int kPrPPitch = kPrTile + 8;       // bf16 per probability row
typedef int i32x2 __attribute__((ext_vector_type(2)));
constexpr float kPrLog2e = 1.44269504088896341f;
constexpr float kPrMargin = 8.0f;            // natural-log units

KVIP_DEVICE float lane_half_other(float x, int g) {  // x of lane l ^ 32
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
    return __int_as_float(g == 0 ? sw[1] : sw[0]);
}

KVIP_DEVICE float rows4_max(float x) {  // max over lanes l, l ^ 16, l ^ 32, l ^ 48
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
KVIP_DEVICE float rows4_sum(float x) {  // sum over lanes l, l ^ 16, l ^ 32, l ^ 48
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <int GROUPS, int SPLIT>
__global__ __launch_bounds__(GROUPS * SPLIT * 64, 1) void sparse_attention_pair_kernel(const KvipSparseAttnArgs p) {
    static_assert(SPLIT == 4, "four waves per 32 heads");
    constexpr int kThreads = GROUPS * SPLIT * 64;
    constexpr int kKSteps = kKeyDim / 32;          // logit MFMA steps (16x16x32)
    constexpr int kVPart = kValueDim / SPLIT;      // value features per wave
    constexpr int kBlocks = kVPart / 32;           // value blocks of 32 features per wave
    constexpr int kTokPer = kPrTile * 32 / kThreads;  // tokens each thread stages (2 or 4)
    static_assert(kTokPer == 2 || kTokPer == 4, "staging map");
    __shared__ __align__(16) uint16_t s_k[2][kPrTile * kPrKPitch];  // keys, token-major, two tiles
    __shared__ __align__(16) uint16_t s_p[GROUPS][32 * kPrPPitch];  // probabilities, [head][token]
    __shared__ float s_m[GROUPS][2][32];                             // per token half: head maxima / sums
    __shared__ __align__(16) float s_h[GROUPS * SPLIT][32];          // per-head values for the O layout
    __shared__ int32_t s_row[kTopK];

    const int pairs_needed = (p.heads + 31) / 32;
    const int sets = (pairs_needed + GROUPS - 1) / GROUPS;
    const int splits = sa_splits(p.rows, sets);
    const int units = sets * splits;
    // XCD-aware order as in the 16-head kernel: a row's workgroups share blockIdx % 8.
    const int chunk = blockIdx.x / (8 * units), within = blockIdx.x % (8 * units);
    const int r = chunk * 8 + within % 8;
    const int unit = within / 8, hs = unit % sets, sp = unit / sets;
    if (r >= p.rows) return;
    const int b = r / p.rows_per_request;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gi = w / SPLIT, hf = w % SPLIT;        // group in the workgroup, wave in the group
    const int pair = hs * GROUPS + gi;               // 32-head group
    const int th = hf & 1, hh = hf >> 1;             // logits of tokens 16 th .., heads 16 hh ..
    const bool live = pair < pairs_needed;           // uniform per wave
    const int n = lane & 31, g = lane >> 5;          // value product: head / feature n, half g
    const int c = lane & 15, qd = lane >> 4;         // logits: head 16 hh + c, tokens 16 th + 4 qd + i
    uint32_t err = 0;

    // Cache rows of the split's indices, resolved once through the block table.
    const int span = kTopK / splits;
    const int* idx_row = p.indices + static_cast<size_t>(r) * kTopK + sp * span;
    const int capacity = p.max_blocks * kBlockTokens;
    for (int i = tid; i < span; i += kThreads) {
        const int t = idx_row[i];
        int row = -1;
        if (t >= capacity) {
            err |= KVIP_STATUS_BAD_TOKEN;
        } else if (t >= 0) {
            const int blk = p.block_table[static_cast<size_t>(b) * p.max_blocks + (t >> 7)];
            if (static_cast<unsigned>(blk) < static_cast<unsigned>(p.num_blocks)) {
                row = blk * kBlockTokens + (t & 127);
            } else {
                err |= KVIP_STATUS_BAD_BLOCK;
            }
        }
        s_row[i] = row;
    }

    // Query fragments (B operand of the logits): head 32 pair + 16 hh + c, features
    // 32 s + 8 qd .. + 8; heads past p.heads read as zero.
    bf16x8 qf[kKSteps];
    {
        const int h = pair * 32 + 16 * hh + c;
        const bool hl = live && h < p.heads;
        const uint16_t* q = p.query + (static_cast<size_t>(r) * p.heads + (hl ? h : 0)) * kKeyDim + qd * 8;
#pragma unroll
        for (int s = 0; s < kKSteps; ++s) {
            const v4i v = hl ? *reinterpret_cast<const v4i*>(q + s * 32) : v4i{0, 0, 0, 0};
            qf[s] = as_bf16x8(v);
        }
    }
    v16f o[kBlocks];
#pragma unroll
    for (int t = 0; t < kBlocks; ++t) {
#pragma unroll
        for (int i = 0; i < 16; ++i) o[t][i] = 0.f;
    }
    // Reference maxima (natural-log units) of head 16 hh + c ("own") and 16 (1 - hh) + c:
    // every wave of the group follows all 32 heads, from the same tile maxima in the same order.
    float m_own = -INFINITY, m_oth = -INFINITY;
    float l_sum = 0.f;        // this lane's share of the own head's probability sum
    bool o_zero = true;       // no tile has been accumulated yet (uniform)
    __syncthreads();

    // Staging map: thread (token group tg, nope slice pc) holds the 16 nope features
    // 16 pc .. of kTokPer consecutive tokens; the tile's 256 rope pieces go to threads 0-255.
    const int tg = tid >> 5, pc = tid & 31;
    const int f0 = pc * 16;
    v4i nope[kTokPer];
    float sc[kTokPer];
    v4i rope = v4i{0, 0, 0, 0};
    auto row_base = [&](int row) {
        return p.kv_cache + static_cast<int64_t>(row >> 7) * p.kv_block_stride +
               static_cast<int64_t>(row & 127) * p.row_stride;
    };
    auto load_tile = [&](int k) {
#pragma unroll
        for (int u = 0; u < kTokPer; ++u) {
            const int row = s_row[k * kPrTile + tg * kTokPer + u];
            nope[u] = v4i{0, 0, 0, 0};
            sc[u] = 0.f;
            if (row >= 0) {
                const uint8_t* base = row_base(row);
                nope[u] = *reinterpret_cast<const v4i*>(base + f0);
                sc[u] = *reinterpret_cast<const float*>(base + 640 + (pc >> 3) * 4);
            }
        }
        if (tid < kPrTile * 8) {
            const int row = s_row[k * kPrTile + (tid >> 3)];
            rope = row >= 0 ? *reinterpret_cast<const v4i*>(row_base(row) + 512 + (tid & 7) * 16) : v4i{0, 0, 0, 0};
        }
    };
    // Dequantisation to bf16: keys [nope * scale, rope] token-major into tile buffer kb. The
    // values are the same nope * scale features, read feature-wise by the transpose loads.
    auto stage_tile = [&](uint16_t* kb) {
#pragma unroll
        for (int u = 0; u < kTokPer; ++u) {
            uint32_t out[8];  // features f0 + 2k, 2k + 1
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(nope[u][k], false);
                const f32x2 cc = __builtin_amdgcn_cvt_pk_f32_fp8(nope[u][k], true);
                out[2 * k] = pack_bf16(a[0] * sc[u], a[1] * sc[u]);
                out[2 * k + 1] = pack_bf16(cc[0] * sc[u], cc[1] * sc[u]);
            }
            uint16_t* d = kb + (tg * kTokPer + u) * kPrKPitch + f0;
            reinterpret_cast<v4i*>(d)[0] = v4i{static_cast<int>(out[0]), static_cast<int>(out[1]),
                                               static_cast<int>(out[2]), static_cast<int>(out[3])};
            reinterpret_cast<v4i*>(d)[1] = v4i{static_cast<int>(out[4]), static_cast<int>(out[5]),
                                               static_cast<int>(out[6]), static_cast<int>(out[7])};
        }
        if (tid < kPrTile * 8) {
            *reinterpret_cast<v4i*>(kb + (tid >> 3) * kPrKPitch + 512 + (tid & 7) * 8) = rope;
        }
    };
    // Transpose-load address of this lane within a tile: in each 16-lane block (j = lane % 16)
    // lane j reads 4 features of one token, and lane j of the result holds one feature of 4
    // consecutive tokens: block G = lane / 16 covers features 16 (G % 2) .. + 16 of tokens
    // 8 (G / 2) .. + 4 (and + 4 .. + 8 by a second load), i.e. the B operand lane (feature n,
    // tokens 8 g .. + 8) of the value MFMA.
    const int tr_off = (8 * g + ((lane & 15) >> 2)) * kPrKPitch + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

    const int tiles = span / kPrTile;
    load_tile(0);
    stage_tile(s_k[0]);
    if (tiles > 1) load_tile(1);
    __syncthreads();  // s_k[0] holds tile 0
    for (int k = 0; k < tiles; ++k) {
        const uint16_t* kt = s_k[k & 1];
        const bool more = k + 1 < tiles;
        // Tokens of the tile that have a row (bit t: token t).
        const uint32_t vmask =
            static_cast<uint32_t>(__ballot(lane < kPrTile && s_row[k * kPrTile + (lane & 31)] >= 0));
        float sv[4];
        if (live) {
            // Logits of tokens 16 th .. + 16 (M) and heads 16 hh .. + 16 (N) over all 576
            // features: lane (head 16 hh + c) gets tokens 16 th + 4 qd + i.
            f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
            const uint16_t* kr = kt + (16 * th + c) * kPrKPitch + 8 * qd;
#pragma unroll
            for (int s = 0; s < kKSteps; ++s) {
                const bf16x8 kv = as_bf16x8(*reinterpret_cast<const v4i*>(kr + s * 32));
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, qf[s], acc, 0, 0, 0);
            }
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float v = acc[i] * p.scale;
                if (!((vmask >> (16 * th + 4 * qd + i)) & 1u)) v = -INFINITY;
                sv[i] = v;
                mx = fmaxf(mx, v);
            }
            mx = rows4_max(mx);  // the head's maximum over this wave's 16 tokens
            if (qd == 0) s_m[gi][th][16 * hh + c] = mx;
        }
        __syncthreads();  // both token halves' maxima of every head in s_m
        if (live) {
            const float t_own = fmaxf(s_m[gi][0][16 * hh + c], s_m[gi][1][16 * hh + c]);
            const float t_oth = fmaxf(s_m[gi][0][16 * (1 - hh) + c], s_m[gi][1][16 * (1 - hh) + c]);
            const bool n_own = t_own > m_own + kPrMargin;  // also the first finite maximum
            const bool n_oth = t_oth > m_oth + kPrMargin;
            if (__ballot(n_own || n_oth) != 0ull) {  // the same decision in every wave of the group
                const float new_own = n_own ? t_own : m_own, new_oth = n_oth ? t_oth : m_oth;
                const float a_own = (m_own == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f((m_own - new_own) * kPrLog2e);
                const float a_oth = (m_oth == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f((m_oth - new_oth) * kPrLog2e);
                l_sum *= n_own ? a_own : 1.f;
                if (!o_zero) {
                    if (qd == 0) {
                        s_h[w][16 * hh + c] = n_own ? a_own : 1.f;
                        s_h[w][16 * (1 - hh) + c] = n_oth ? a_oth : 1.f;
                    }
                    // Wave-local: this wave's LDS writes precede its reads.
                    f32x4 a4[4];
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) a4[qq] = *reinterpret_cast<const f32x4*>(&s_h[w][8 * qq + 4 * g]);
#pragma unroll
                    for (int t = 0; t < kBlocks; ++t) {
#pragma unroll
                        for (int i = 0; i < 16; ++i) o[t][i] *= a4[i >> 2][i & 3];
                    }
                }
                m_own = new_own;
                m_oth = new_oth;
            }
            const float bias = m_own == -INFINITY ? 0.f : -m_own * kPrLog2e;
            const float p0 = __builtin_amdgcn_exp2f(fmaf(sv[0], kPrLog2e, bias));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(sv[1], kPrLog2e, bias));
            const float p2 = __builtin_amdgcn_exp2f(fmaf(sv[2], kPrLog2e, bias));
            const float p3 = __builtin_amdgcn_exp2f(fmaf(sv[3], kPrLog2e, bias));
            l_sum += (p0 + p1) + (p2 + p3);
            *reinterpret_cast<i32x2*>(s_p[gi] + (16 * hh + c) * kPrPPitch + 16 * th + 4 * qd) =
                i32x2{static_cast<int>(pack_bf16(p0, p1)), static_cast<int>(pack_bf16(p2, p3))};
        }
        __syncthreads();  // the group's probabilities in s_p
        if (live) {
            // Value product: features kVPart hf + 32 t + n; K step s2 covers tokens 16 s2 + 8 g
            // .. + 8 of head n (A: probabilities, B: transpose loads of the key tile).
            bf16x8 pa[2];
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                pa[s2] = as_bf16x8(*reinterpret_cast<const v4i*>(s_p[gi] + n * kPrPPitch + 16 * s2 + 8 * g));
            }
#pragma unroll
            for (int t = 0; t < kBlocks; ++t) {
                const uint16_t* vr = kt + tr_off + hf * kVPart + t * 32;
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2) {
                    const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) v4s*)(vr + 16 * s2 * kPrKPitch));
                    const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) v4s*)(vr + (16 * s2 + 4) * kPrKPitch));
                    const bf16x8 vb = __builtin_bit_cast(bf16x8, v8s{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
                    o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa[s2], vb, o[t], 0, 0, 0);
                }
            }
            o_zero = false;
            // The next tile's staging beside this tile's value MFMAs (inside the branch, so
            // the scheduler can interleave them), then the loads of the tile after it.
            if (more) {
                stage_tile(s_k[(k + 1) & 1]);
                if (k + 2 < tiles) load_tile(k + 2);
            }
        } else if (more) {
            stage_tile(s_k[(k + 1) & 1]);
            if (k + 2 < tiles) load_tile(k + 2);
        }
        __syncthreads();  // tile k + 1 staged; tile k's buffer, s_m and s_p free
    }

    // Probability sums: over the lane's four token rows, then the two token halves; then the
    // split's partial record (max, sum, unnormalised output per head) or the normalised
    // output. Output lane (feature kVPart hf + 32 t + n) holds heads 32 pair + 8 (i / 4) +
    // 4 g + i % 4 of o[t][i].
    if (live) {
        const float l = rows4_sum(l_sum);
        if (qd == 0) s_m[gi][th][16 * hh + c] = l;
    }
    __syncthreads();
    if (live) {
        const float l_n = s_m[gi][0][n] + s_m[gi][1][n];  // head n of the group
        const int groups = (p.heads + kSaHeads - 1) / kSaHeads;
        if (splits > 1) {
            if (hf == 0 && g == 0) {
                // Wave 0 (hh = 0) holds head c as its own and 16 + c as the other.
                const int h = pair * 32 + n;
                if (h < p.heads) {
                    float* ws = p.workspace + ((static_cast<size_t>(r) * groups + h / kSaHeads) * splits + sp) * kPartial;
                    ws[h % kSaHeads] = n < 16 ? m_own : m_oth;
                    ws[kSaHeads + h % kSaHeads] = l_n;
                }
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int h = pair * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
                if (h >= p.heads) continue;
                float* ws = p.workspace + ((static_cast<size_t>(r) * groups + h / kSaHeads) * splits + sp) * kPartial +
                            2 * kSaHeads + (h % kSaHeads) * kValueDim + hf * kVPart + n;
#pragma unroll
                for (int t = 0; t < kBlocks; ++t) ws[t * 32] = o[t][i];
            }
        } else {
            if (g == 0) s_h[w][n] = l_n > 0.f ? 1.f / l_n : 0.f;
            f32x4 inv[4];
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) inv[qq] = *reinterpret_cast<const f32x4*>(&s_h[w][8 * qq + 4 * g]);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int h = pair * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
                if (h >= p.heads) continue;
                float* out = p.output + (static_cast<size_t>(r) * p.heads + h) * kValueDim + hf * kVPart + n;
#pragma unroll
                for (int t = 0; t < kBlocks; ++t) out[t * 32] = o[t][i] * inv[i >> 2][i & 3];
            }
        }
    }
    report(p.status, err);
}

// Merge of the splits: workgroup (row, head group, 64-feature chunk).
__global__ __launch_bounds__(kSaThreads) void sparse_attention_merge_kernel(const KvipSparseAttnArgs p) {
    __shared__ float s_w[kMaxSplits][kSaHeads];
    __shared__ float s_inv[kSaHeads];
    const int groups = (p.heads + kSaHeads - 1) / kSaHeads;
    const int splits = sa_splits(p.rows, sa_sets(p.heads));
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
    const int splits = sa_splits(rows, sa_sets(heads));
    return splits > 1 ? static_cast<uint64_t>(rows) * groups * splits * kPartial * sizeof(float) : 0;
}

uint32_t validate_sparse_attention(const KvipSparseAttnArgs* a) {
    if (a == nullptr) return KVIP_ERR_INVALID;
    const bool ok = a->query && a->kv_cache && a->block_table && a->indices && a->output && a->rows >= 1 &&
                    a->rows_per_request >= 1 && a->rows % a->rows_per_request == 0 && a->heads >= 1 &&
                    a->heads <= 128 && a->max_blocks >= 1 && a->max_blocks <= (1 << 24) / kBlockTokens &&
                    a->num_blocks >= 1 && a->num_blocks < (1 << 24) && a->row_stride >= KVIP_KV_ROW_BYTES &&
                    a->row_stride % 16 == 0 &&
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
    const int sets = kvip::sa_sets(args->heads);
    const int splits = kvip::sa_splits(args->rows, sets);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(((args->rows + 7) / 8) * 8 * sets * splits);
    if (kvip::sa_pairs(args->heads)) {
        hipLaunchKernelGGL((kvip::sparse_attention_pair_kernel<kvip::kPrGroups, kvip::kPrSplit>), grid,
                           dim3(kvip::kPrGroups * kvip::kPrSplit * 64), 0, s, *args);
    } else if (kvip::sa_group_set(args->heads) == 2) {
        hipLaunchKernelGGL(kvip::sparse_attention_kernel<2>, grid, dim3(2 * kvip::kSaThreads), 0, s, *args);
    } else {
        hipLaunchKernelGGL(kvip::sparse_attention_kernel<1>, grid, dim3(kvip::kSaThreads), 0, s, *args);
    }
    if (splits > 1) {
        hipLaunchKernelGGL(kvip::sparse_attention_merge_kernel, dim3(args->rows * groups * 8), dim3(kvip::kSaThreads),
                           0, s, *args);
    }
    return static_cast<uint32_t>(hipGetLastError());
}

extern "C" uint64_t kvip_hip_sparse_attention_workspace_bytes(int32_t rows, int32_t heads) {
    return kvip::sparse_attention_workspace_bytes(rows, heads);
}
