/*
 * kvip_hip.h - C ABI of the MI355X (gfx950) lightning-indexer-with-fetch library
 * (libkvip_hip.so).
 *
 * Plain pointers, sizes and a hipStream_t passed as void*. Every entry point only
 * enqueues work on the given stream: no allocation, no host synchronisation, no
 * device-to-host read, so each one can be captured into a hipGraph. Device-side
 * problems (out-of-range block ids or tokens, inconsistent histograms) are reported
 * by OR-ing KVIP_STATUS_* bits into an optional device status word; host-side
 * argument errors return KVIP_ERR_INVALID before anything is launched.
 *
 * Reference interfaces replaced (paths relative to the KVIP reference tree):
 *   kvip_hip_lifetch_forward  <- kvip_lifetch_streaming_forward
 *                                (csrc/operators/lightning_indexer_with_fetch/include/api.h:7,
 *                                 op_host/launch.cpp:76-83)
 *   kvip_hip_indexer_decode   <- v9_li / QuantLightningIndexerKernel scoring
 *                                (op_host/launch.cpp:16; op_kernel/indexer.cpp:23-86;
 *                                 op_kernel/indexer/indexer_score.h:384-426)
 *   kvip_hip_indexer_prefill  <- the native prefill LI the vLLM selector runs for prefill rows
 *                                (python/kvip/adapters/vllm/selector.py:126-154 ->
 *                                 torch_npu.npu_quant_lightning_indexer, TND / sparse_mode 3,
 *                                 tests/operators/lifetch/support/execution.py:126-145)
 *   kvip_hip_topk             <- LITopk<uint16_t> inside QLIVector::ProcessTopK
 *                                (op_kernel/indexer/indexer_vector.h:799-973; topk.h:122-197)
 *   kvip_hip_fetch_gather     <- kvaf_device::KvafBatchGetDevice as called by FetchQueryGroup
 *                                (op_kernel/streaming.cpp:365-500, :445;
 *                                 patches/kvaf-ubmem-device-get.patch:41-90)
 *   kvip_hip_select_fetch     <- ProcessTopK followed by the FetchQueryGroup gather
 *                                (indexer_vector.h:799-973; streaming.cpp:365-500)
 *   kvip_hip_update_abc       <- kvip.update_abc (python/kvip/cache/abc.py:5-33; the NPU launch
 *                                of cache/_abc_kernel.py:9-34)
 *   kvip_hip_lru_reset/extend/commit
 *                             <- SlotLRU.resize / SlotLRU.commit (python/kvip/cache/lru.py:33-118)
 *                                and their numba kernels (cache/_lru_kernel.py:33-199)
 *   kvip_hip_lidu             <- kvip.lidu = lidu_fused_batch_get_prepare_mtp_out
 *                                (python/kvip/operators/lidu.py:4-8; torch_extension/csrc/
 *                                 lidu_fused_batch_get_prepare_mtp_ops.cpp:195-270, schema :386-399;
 *                                 op_kernel/a5_lidu_fused_batch_get_prepare_mtp.cpp)
 *   kvip_hip_lidu_workspace_bytes
 *                             <- the op's workspace sizing (op_host/a5_lidu_fused_batch_get_prepare_mtp.cpp:101, :282-288)
 *   kvip_hip_pack_queries     <- QueryInputs.bind_positions + QueryInputs.pack
 *                                (python/kvip/adapters/vllm/inputs.py:127-152)
 *   kvip_hip_ingest_index     <- VllmIndexCacheStorage.ingest_prefill / ingest_decode
 *                                (python/kvip/adapters/vllm/index_import.py:18-52)
 *   kvip_hip_resident_round   <- the streaming resolver round after LI: InitializeRound
 *                                (op_kernel/lifecycle.cpp:32-81), EmitFinalClassification /
 *                                ClassifyTopkHalf (indexer_vector.h:679-795,
 *                                staged_topk_classify.h:9-47), Producer + StagedQuery
 *                                (streaming.cpp:103-204, resolver_staged_dma2.h:98-237),
 *                                PublishQueryOutputs (streaming.cpp:66-90), the Fetch of
 *                                FetchQueryGroup (streaming.cpp:365-500), Consumer + ApplyBatch
 *                                (streaming.cpp:205-274, shadow_exchange_parallel.h:28-85),
 *                                PublishDestinationResidency (common/lifetch/cache_metadata.h:54-73)
 *   kvip_hip_resident_prefix  <- ProcessResidentTopK + SaveResident (indexer_vector.h:100-105,
 *                                :162-234), ClassifyScore / ClassifyResidentScores
 *                                (indexer_score.h:784-792, :1018-1048), GatherVictimScores
 *                                (common/lifetch/victim_ops.h:3-12), the cold-tile hit bits
 *                                (indexer_vector.h:584-593, :626-638)
 *   kvip_hip_resident_forward <- kvip_lifetch_streaming_forward in resident mode
 *                                (include/api.h:7, op_host/launch.cpp:76-83)
 *   kvip_hip_resident_begin / _prefetch / _finish
 *                             <- the same round split around the speculative windowed
 *                                prefetch: InitializeRound + InitializeTailMappings
 *                                (prefetch.h:25-43), FastService (prefetch.h:578-832) with
 *                                the window scan of common/lifetch/sequence_candidates.h and
 *                                PrefetchAllowance (common/lifetch/prefetch_budget.h:7-17),
 *                                then the final round with PublishPrefetch (streaming.cpp:
 *                                23-27, :119-121) and PublishPrefetchResidency (:330-339)
 *   kvip_hip_resident_resolve / _fetch / _update
 *                             <- kvip_hip_resident_finish in its three stages, so that the
 *                                Fetch (FetchQueryGroup, streaming.cpp:365-500) and the Index
 *                                update (Consumer + ApplyBatch, streaming.cpp:205-274) of one
 *                                round can run on two streams, as the reference's producer and
 *                                consumer run beside each other
 *   kvip_hip_resident_workspace_bytes / kvip_hip_resident_prepare
 *                             <- the rotation scratch allocated and reset at bind time
 *                                (python/kvip/operators/lifetch/workspace.py:9-31,
 *                                 binding.py:113-130)
 */
#ifndef KVIP_HIP_H
#define KVIP_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVIP_HIP_ABI_VERSION 15u

#define KVIP_TOPK 2048
#define KVIP_BLOCK_TOKENS 128
#define KVIP_INDEX_DIM 128
#define KVIP_KV_ROW_BYTES 656

/* Return codes: 0 on success, KVIP_ERR_INVALID when the arguments are rejected
 * (nothing launched), otherwise the hipError_t reported by the launch. Same
 * convention as the reference's kvip_lifetch_streaming_forward (launch.cpp:76-83). */
#define KVIP_OK 0u
#define KVIP_ERR_INVALID 100000u

/* Element types. */
#define KVIP_DTYPE_FP8_E4M3 0
#define KVIP_DTYPE_BF16 1
#define KVIP_DTYPE_FP32 2

/* Device status bits, OR-ed into *status when status is not NULL. */
#define KVIP_STATUS_BAD_BLOCK 1u     /* a block-table entry outside [0, num_blocks) */
#define KVIP_STATUS_HISTOGRAM 2u     /* TopK histogram inconsistent with the row length */
#define KVIP_STATUS_BAD_TOKEN 4u     /* a TopK token id outside the block table */

/* Lightning-indexer scoring over a paged index-K cache.
 *
 * For query row r of request b = r / rows_per_request and token t < valid(r):
 *   w'_h      = float(weights[r,h]) * query_scale[r,h]
 *   qk_h      = sum_d q[r,h,d] * k[t,d]                (fp32 accumulation)
 *   score     = key_scale[t] * sum_h max(qk_h, 0) * w'_h
 *   key[r,t]  = sortable(bf16_round_half_away(score))
 * valid(r) = min(seq_lens[b], query_ends[r]) (query_ends NULL: seq_lens[b]).
 * The kernel also adds the 256-bin histogram of key>>8 over t < valid(r) into
 * histogram[r, :]; that buffer must be zero before the first launch and is
 * re-zeroed by kvip_hip_topk when it consumes it. */
typedef struct KvipIndexerArgs {
    const void* query;           /* [rows, heads, 128], fp8 e4m3 or bf16 (qk_dtype) */
    const void* weights;         /* [rows, heads], fp32 or bf16 (weight_dtype) */
    const float* query_scale;    /* [rows, heads], or NULL for 1.0 */
    const void* keys;            /* index-K row t of block k: keys + k*key_block_stride + (t%128)*128*elem */
    const float* key_scale;      /* per-token scale key_scale[k*scale_block_stride + t%128], or NULL for 1.0 */
    const int32_t* block_table;  /* [batch, max_blocks] block ids */
    const int32_t* seq_lens;     /* [batch] context tokens per request */
    const int32_t* query_ends;   /* [rows] per-row visible bound (<= 0: padding row), or NULL */
    uint16_t* score_keys;        /* [rows, key_stride] sortable bf16 keys */
    uint32_t* histogram;         /* [rows, 256] high-byte counts */
    uint32_t* status;            /* device status word, or NULL */
    int64_t key_block_stride;    /* bytes between index-K blocks (multiple of 16) */
    int64_t scale_block_stride;  /* floats between key-scale blocks */
    int32_t batch;               /* requests */
    int32_t rows_per_request;    /* 1, 2 or 4 query rows per request (decode + MTP) */
    int32_t heads;               /* 32 or 64 index heads */
    int32_t max_blocks;          /* block_table row length */
    int32_t num_blocks;          /* valid block ids are [0, num_blocks) */
    int32_t key_stride;          /* score_keys row stride: multiple of 8, >= max_blocks*128 */
    int32_t qk_dtype;            /* KVIP_DTYPE_FP8_E4M3 or KVIP_DTYPE_BF16 */
    int32_t weight_dtype;        /* KVIP_DTYPE_FP32 or KVIP_DTYPE_BF16 */
} KvipIndexerArgs;

/* Prefill and mixed-batch lightning-indexer scoring over packed query rows (TND layout):
 * sequence s owns query rows [cu_seqlens_q[s], cu_seqlens_q[s+1]) and key positions
 * [0, seq_lens_k[s]) of block_table[s]; local row j of sequence s (q_len rows) sees the
 * positions t < vis = clamp(seq_lens_k[s] - q_len + j + 1, 0, seq_lens_k[s]) (right-down
 * causal). Keys and the high-byte histogram are those of kvip_hip_indexer_decode for each
 * (row, t < vis); row_valid[r] = vis is written for TopK (kvip_hip_topk with batch = rows,
 * rows_per_request = 1, seq_lens = row_valid). fp8 Q/K only; 32 or 64 heads; at most 1024
 * sequences. */
#define KVIP_PREFILL_MAX_SEQUENCES 1024
typedef struct KvipPrefillArgs {
    const void* query;           /* [rows, heads, 128] fp8 e4m3 or bf16 (qk_dtype) */
    const void* weights;         /* [rows, heads] fp32 or bf16 (weight_dtype) */
    const float* query_scale;    /* [rows, heads], or NULL for 1.0 */
    const void* keys;            /* paged index-K of qk_dtype, as KvipIndexerArgs */
    const float* key_scale;      /* per-token scales, as KvipIndexerArgs, or NULL */
    const int32_t* block_table;  /* [sequences, max_blocks] */
    const int32_t* cu_seqlens_q; /* [sequences + 1] cumulative query rows, cu[0] = 0 */
    const int32_t* seq_lens_k;   /* [sequences] key positions of each sequence */
    uint16_t* score_keys;        /* [rows, key_stride] */
    uint32_t* histogram;         /* [rows, 256], zero before the launch */
    int32_t* row_valid;          /* [rows] out */
    uint32_t* status;            /* device status word, or NULL */
    int64_t key_block_stride;    /* bytes between index-K blocks (multiple of 16, >= 16 KiB fp8, 32 KiB bf16) */
    int64_t scale_block_stride;  /* floats between key-scale blocks */
    int32_t sequences;
    int32_t rows;                /* = cu_seqlens_q[sequences] */
    int32_t heads;               /* 32 or 64 */
    int32_t max_blocks;
    int32_t num_blocks;
    int32_t key_stride;          /* multiple of 8, >= max_blocks * 128 */
    int32_t qk_dtype;            /* KVIP_DTYPE_FP8_E4M3 or KVIP_DTYPE_BF16 */
    int32_t weight_dtype;        /* KVIP_DTYPE_FP32 or KVIP_DTYPE_BF16 */
} KvipPrefillArgs;

/* Exact TopK-2048 of sortable uint16 keys per query row, over the row's valid
 * positions valid = min(seq_lens[b], query_ends[r], limit if limit > 0).
 * valid < 2048: out = [0, 1, ..., valid-1, -1, ...].
 * valid >= 2048: the 2048 tokens that come first in the order (key desc, index asc),
 * written as the tokens with key > kth in ascending index order followed by the
 * tokens with key == kth in ascending index order. */
#define KVIP_TOPK_SEGMENT_KEYS 2048
#define KVIP_TOPK_SEGMENT_WORDS 260
typedef struct KvipTopkArgs {
    const uint16_t* score_keys;  /* [rows, key_stride] */
    uint32_t* histogram;         /* [rows, 256] from kvip_hip_indexer_decode (re-zeroed here), or NULL */
    uint32_t* segments;          /* with a histogram: work memory of rows * ceil(key_stride / 2048) * 260
                                    words for the multi-workgroup select, zero before the first call
                                    (every call leaves it reusable); NULL: one workgroup per row */
    const int32_t* seq_lens;     /* [batch] */
    const int32_t* query_ends;   /* [rows] or NULL */
    int32_t* topk;               /* [rows, 2048] token ids, -1 = empty */
    uint32_t* status;            /* device status word, or NULL */
    int32_t batch;
    int32_t rows_per_request;
    int32_t key_stride;          /* multiple of 8 */
    int32_t limit;               /* > 0: only positions below limit take part (the resident prefix) */
} KvipTopkArgs;

/* Gather of the selected KV rows from a paged KV cache into a contiguous buffer:
 *   output[r, i, :] = kv row topk[r, i] of request r / rows_per_request, or zeros for -1. */
typedef struct KvipFetchArgs {
    const int32_t* topk;         /* [rows, 2048] */
    const uint8_t* kv_cache;     /* KV row t of block k: kv_cache + k*kv_block_stride + (t%128)*row_stride */
    const int32_t* block_table;  /* [batch, max_blocks] */
    uint8_t* output;             /* [rows, 2048, row_bytes] */
    uint32_t* status;            /* device status word, or NULL */
    int64_t kv_block_stride;     /* bytes, multiple of 16 */
    int32_t row_stride;          /* bytes between rows of one block, multiple of 16 */
    int32_t row_bytes;           /* bytes per KV row, multiple of 16 (656 for MLA latent rows) */
    int32_t batch;
    int32_t rows_per_request;
    int32_t max_blocks;
    int32_t num_blocks;
} KvipFetchArgs;

/* One decode round: scoring -> TopK-2048 -> Fetch gather, stream-ordered (three
 * launches; the stages must be chained: TopK reads the scoring's keys and histogram, the
 * gather the TopK's ids). */
typedef struct KvipLIFetchArgs {
    KvipIndexerArgs indexer;
    KvipTopkArgs topk;
    KvipFetchArgs fetch;
} KvipLIFetchArgs;

/* ABC ring maps: token_to_slot / slot_to_token are int32 [layers, pool, tokens];
 * descriptors int32 [groups, rows, 4] of (layer, owner, begin, end); the first `requests`
 * rows of every group are applied in group-major order. Descriptors naming an out-of-range
 * layer/owner/token are skipped and reported with KVIP_STATUS_BAD_TOKEN. */
typedef struct KvipAbcArgs {
    int32_t* token_to_slot;
    int32_t* slot_to_token;
    const int32_t* descriptors;
    uint32_t* status;            /* device status word, or NULL */
    int32_t groups;
    int32_t rows;                /* descriptors.shape[1] */
    int32_t requests;            /* rows applied per group, <= rows */
    int32_t layers;
    int32_t pool;
    int32_t t2s_tokens;          /* token_to_slot.shape[2] */
    int32_t s2t_tokens;          /* slot_to_token.shape[2], >= history + tail */
    int32_t history;
    int32_t tail;
} KvipAbcArgs;

/* Slot LRU of one request/layer chain on the device. order[i] is the slot at LRU position
 * i (0 = least recently used) for i < active; slots [2048] = the min(2048, active) oldest
 * slots (-1 padded); bitmap [bitmap_words] = their membership bits; scratch [capacity] is
 * reserved work memory (required non-NULL; the commit partitions the order in place and
 * leaves it untouched). capacity <= 133632 slots. */
typedef struct KvipLruArgs {
    int32_t* order;
    int32_t* scratch;
    int32_t* slots;
    int32_t* bitmap;
    int32_t capacity;
    int32_t bitmap_words;
} KvipLruArgs;

/* LIDU limits (a5_lidu_fused_batch_get_prepare_mtp.cpp:36-57). */
#define KVIP_LIDU_MAX_QUERIES 4
#define KVIP_LIDU_MISS_CAPACITY (KVIP_TOPK * KVIP_LIDU_MAX_QUERIES)
#define KVIP_LIDU_MAX_SOURCE_TOKENS ((1 << 20) + 20 * 128)
#define KVIP_LIDU_MAX_CACHE_TOKENS ((1 << 17) + 20 * 128)
#define KVIP_LIDU_BITMAP_WORDS 4176 /* miss_slot_bitmap words per request */

/* LIDU transaction over a batch of requests, each with 1-4 packed query rows. Tensors are
 * int32 and contiguous, named and shaped as in the reference out-variant op. Per request:
 * the TopK tokens of each query row are classified (hit = token_to_slot maps it to a slot
 * below the resident budget whose miss_slot_bitmap bit is clear), each row of
 * destination_slots becomes [miss prefix, hit slots], the request's distinct misses get
 * miss_slots[0..2047] and then slots scanned from eviction_cursors[pool] over the slots
 * neither in the bitmap nor hit, victims are cleared, maps installed, the miss prefixes
 * refilled with the new slots, and the compact descriptors (indices, offsets,
 * output_indices) written at the request's prefix of miss_counts. A rejected batch
 * (query layout, aliased pool rows) gives -1 rows and miss_counts -1; a rejected request
 * gives -1 rows and miss_counts[b] = -1 and leaves the maps untouched.
 * profile_enabled[0] is read on the device: 2 = graph-dummy mode (membership ignored,
 * out-of-range tokens read as token 0), 1 = write wall-clock stamps (100 MHz ticks) into
 * profiling[b][0][0..8] at the phase boundaries when profiling is not NULL.
 * The workspace holds kvip_hip_lidu_workspace_bytes(batch) bytes (no initialisation
 * needed); calls that share a workspace must be stream-ordered. */
typedef struct KvipLiduArgs {
    const int32_t* topk;                      /* [packed_queries, 2048] (8-byte aligned) */
    const int32_t* actual_seq_lengths_query;  /* [batch] cumulative query ends */
    const int32_t* req_pool_entries;          /* [batch] pool row of each request */
    int32_t* token_to_slot;                   /* [pool_size, source_capacity] */
    int32_t* slot_to_token;                   /* [pool_size, resident_capacity] */
    int32_t* eviction_cursors;                /* [pool_size] */
    const int32_t* cache_tokens;              /* [batch] resident budget */
    const int32_t* candidate_lens;            /* [batch] */
    const int32_t* miss_slots;                /* [batch, 2048] */
    const int32_t* miss_slot_bitmap;          /* [batch, 4176] */
    const int32_t* resident_block_table;      /* [batch, resident_blocks] */
    const int32_t* logical_seq_lengths;       /* [batch] */
    const int32_t* profile_enabled;           /* [1] */
    int32_t* destination_slots;               /* [packed_queries, 2048] (16-byte aligned) */
    int32_t* miss_counts;                     /* [batch + 1], last = total */
    int32_t* indices;                         /* [batch * 8192] */
    int32_t* offsets;                         /* [batch * 8192] */
    int32_t* output_indices;                  /* [batch * 8192] */
    int32_t* resident_seq_lengths;            /* [batch] */
    int64_t* profiling;                       /* [batch, 8, 32], or NULL */
    void* workspace;                          /* 16-byte aligned */
    int64_t workspace_bytes;
    int32_t batch;
    int32_t packed_queries;
    int32_t pool_size;
    int32_t source_capacity;
    int32_t resident_capacity;
    int32_t resident_blocks;
    int32_t layer_id;
    int32_t num_layers;
    int32_t max_num_reqs;
    int32_t qcap;
} KvipLiduArgs;

/* Decode query packing for the LIFetch query buffers, one packed row r < rows at a time
 * (rows = batch * 4):
 *   positions != NULL: query_ends[r] = (positions[gather_indices[r]] + 1) * query_valid[r]
 *   query_in  != NULL: query_out[r] = query_in[gather_indices[r]] (heads * 128 fp8 bytes),
 *                      weights_out[r] = weights_in[...] (heads bf16), scale_out[r] = scale_in[...]
 *                      (heads fp32); the six row arrays 16-byte aligned.
 * A gather index outside [0, tokens) yields query_ends 0 and zero rows and sets
 * KVIP_STATUS_BAD_TOKEN. */
typedef struct KvipQueryPackArgs {
    const int64_t* gather_indices;  /* [rows] source token of each packed row */
    const int64_t* query_valid;     /* [rows] 1 = live row, 0 = padding */
    const int64_t* positions;       /* [tokens] token positions, or NULL */
    int32_t* query_ends;            /* [rows] out (with positions) */
    const void* query_in;           /* [tokens, heads, 128] fp8, or NULL */
    const void* weights_in;         /* [tokens, heads] bf16 */
    const void* scale_in;           /* [tokens, heads] fp32 */
    void* query_out;                /* [rows, heads, 128] */
    void* weights_out;              /* [rows, heads] */
    void* scale_out;                /* [rows, heads] */
    uint32_t* status;               /* device status word, or NULL */
    int64_t tokens;
    int32_t rows;
    int32_t heads;                  /* 32 or 64 */
} KvipQueryPackArgs;

/* Index-K ingestion: `count` rows of 128 bytes (+ one fp32 scale) copied from the paged
 * source cache (source_rows rows = blocks * block_size) into target storage
 * (target_rows rows = owners * history), row i taking source s_i and target t_i:
 *   KVIP_INGEST_DECODE: rows of a packed decode batch, i < batch * queries_per_request:
 *       live (query_ends[i] > 0): s = slot_mapping[gather_indices[i]],
 *                                 t = row_owners[i / queries_per_request] * history + query_ends[i] - 1
 *       padding:                  s = 0, t = i (distinct positions of owner 0)
 *   KVIP_INGEST_LIST:   s = sources[i], t = target_base + targets[i]
 *   KVIP_INGEST_PREFIX: t = target_base + i, s = block_table[i / block_size] * block_size + i % block_size
 * Rows whose s or t falls outside the arrays are skipped and set KVIP_STATUS_BAD_TOKEN. */
#define KVIP_INGEST_DECODE 0
#define KVIP_INGEST_LIST 1
#define KVIP_INGEST_PREFIX 2
typedef struct KvipIngestArgs {
    const uint8_t* source_keys;     /* [source_rows, 128] */
    const float* source_scales;     /* [source_rows] */
    uint8_t* target_keys;           /* [target_rows, 128] */
    float* target_scales;           /* [target_rows] */
    const int32_t* query_ends;      /* DECODE: [count] */
    const int64_t* gather_indices;  /* DECODE: [count] */
    const int64_t* slot_mapping;    /* DECODE: [slot_count] */
    const int32_t* row_owners;      /* DECODE: [count / queries_per_request] */
    const int64_t* sources;         /* LIST: [count] */
    const int64_t* targets;         /* LIST: [count] */
    const int32_t* block_table;     /* PREFIX: [ceil(count / block_size)] */
    uint32_t* status;               /* device status word, or NULL */
    int64_t source_rows;
    int64_t target_rows;
    int64_t count;
    int64_t history;                /* DECODE: positions per owner */
    int64_t target_base;            /* LIST, PREFIX */
    int64_t slot_count;             /* DECODE: slot_mapping length */
    int32_t mode;
    int32_t queries_per_request;    /* DECODE */
    int32_t block_size;             /* PREFIX */
    int32_t reserved;
} KvipIngestArgs;

/* Resident-cache round of one LIFetch step (hot/cold split of the TopK positions):
 * every request b owns the Index rows [row_owners[b], 0..history) (keys, scales, KV
 * addresses in host_pool, logical ids); position p < resident is hot, its KV row living
 * in hot_cache[owner, p] when hot_valid[owner, p] != 0. With tail_bounds, positions
 * [begin_b, end_b) of request b are its ABC tail (the recent tokens whose KV the serving
 * step keeps in the ABC ring, the hot_stride - resident = T slots after the hot ones):
 * they are never hot hits; the first T of them, p < begin_b + T, sit in ring slot
 * resident + p % T and resolve to it without a Fetch; the rest are ordinary misses
 * (the reference's tail mapping, op_kernel/prefetch.h:25-43, resolved by
 * ResolvePhysicalSlot, common/lifetch/cache_metadata.h:102-106, in the final
 * classification, staged_topk_classify.h:9-36). After TopK over positions:
 *   init     reserved_hot[b] = LRU ordinal of each candidate slot of lru_slots[b] (-1
 *            otherwise); changes = -1; change_slots = candidates then -1; counts zero;
 *   resolve  per request, query rows in order: hot hits (p < resident, hot_valid, not a
 *            candidate, not in the tail) keep slot p, mapped tail positions take their
 *            ring slot; rows q >= 2 reuse row q-2's slot for the same position
 *            at the same index; the other positions' first occurrences become misses
 *            ranked in index order over the rows, each given the next free candidate in
 *            ordinal order (pass 0 ordinals >= used, pass 1 < used; slots holding this
 *            step's hits or earlier misses are skipped), then the lowest free hot slots;
 *            slot_output = hot slot of every selected position, logical_output = its
 *            logical id before the update; change records at (candidate ordinal or 2048 +
 *            rank); Fetch descriptors (host_pool offset, slot) per miss;
 *   fetch    hot_cache[owner, slot] = host_pool[offset .. offset + row_bytes) per miss;
 *   update   per query, misses in rank order in 512-change chunks: the row of each
 *            missed position moves to its slot, rows displaced from destinations fill
 *            the chunk's freed positions in order (those below resident lose residency);
 *            keys, scales, addresses and logical ids move with their rows; finally every
 *            miss slot becomes valid.
 * Device errors (bits of KVIP_RESIDENT_ERR_*) go to status[b]; a failed request's later
 * phases are skipped and its owner's whole hot_valid row is cleared (the reference's
 * CompleteEarlyUpdate, op_kernel/index_cache_update.h:5-21), so its next round reads every
 * position cold. A request that fails before the Fetch (bad token, owner or candidate, an
 * in-range hot slot named by two candidates, a source outside host_pool) publishes -1 in
 * both outputs and moves nothing; one whose Index update is rejected keeps its published
 * outputs (their slots hold the fetched rows) and the chunks applied before the rejected
 * one (each a complete permutation). The workspace (kvip_hip_resident_workspace_bytes) is prepared once
 * by kvip_hip_resident_prepare and left prepared by every round; rounds sharing it must
 * be stream-ordered. */
#define KVIP_RESIDENT_MAX_QUERIES 4
#define KVIP_RESIDENT_MAX_RESIDENT 131072
#define KVIP_RESIDENT_LRU_SLOTS 2048
#define KVIP_RESIDENT_CHANGES (KVIP_RESIDENT_LRU_SLOTS + KVIP_RESIDENT_MAX_QUERIES * KVIP_TOPK)
#define KVIP_RESIDENT_ERR_TOKEN 1u       /* a TopK position >= history, a bad owner row, or tail
                                            bounds outside 0 <= begin <= end <= history */
#define KVIP_RESIDENT_ERR_CANDIDATE 4u   /* a candidate outside [0, resident), or no free hot slot */
#define KVIP_RESIDENT_ERR_SOURCE 8u      /* a Fetch source outside host_pool */
#define KVIP_RESIDENT_ERR_UPDATE 16u     /* the changes are not a partial permutation */
typedef struct KvipResidentArgs {
    const int32_t* topk;          /* [batch * rows_per_request, 2048] selected positions, -1 = empty */
    const int32_t* row_owners;    /* [batch] */
    const int32_t* lru_slots;     /* [batch, 2048] victim candidates, oldest first */
    int32_t* reserved_hot;        /* [batch, resident] (written by the round) */
    int32_t* hot_valid;           /* [owners, resident] */
    uint8_t* index_keys;          /* [owners, history, 128] */
    float* index_scales;          /* [owners, history] */
    int64_t* addresses;           /* [owners, history] byte offset of each row's KV in host_pool */
    int64_t* logical_ids;         /* [owners, history] */
    const uint8_t* host_pool;     /* device-accessible host memory (mapped pinned) */
    uint8_t* hot_cache;           /* [owners, hot_stride, row_bytes] */
    int32_t* logical_output;      /* [batch * rows_per_request, 2048] */
    int32_t* slot_output;         /* [batch * rows_per_request, 2048] */
    int32_t* changes;             /* [batch, 2048 + rows_per_request * 2048] */
    int32_t* change_slots;        /* [batch, 2048 + rows_per_request * 2048] */
    int32_t* miss_counts;         /* [batch, 5]: new misses of each query row, then the total */
    int64_t* fetch_sources;       /* [batch, rows_per_request * 2048] host_pool offsets by rank */
    int32_t* fetch_slots;         /* [batch, rows_per_request * 2048] */
    int32_t* fetch_positions;     /* [batch, rows_per_request * 2048] missed position by rank */
    int32_t* status;              /* [batch] KVIP_RESIDENT_ERR_* bits */
    void* workspace;              /* kvip_hip_resident_workspace_bytes(batch, history), 16-byte aligned */
    int64_t host_pool_bytes;
    int32_t batch;
    int32_t rows_per_request;     /* 1..4 */
    int32_t owners;
    int32_t history;              /* Index rows per owner, multiple of 128 */
    int32_t resident;             /* hot positions per owner, 2048..131072 */
    int32_t hot_stride;           /* hot_cache rows per owner, >= resident */
    int32_t row_bytes;            /* KV row bytes, multiple of 16 */
    int32_t used;                 /* candidates consumed before this step (0 without prefetch) */
    /* Token-order (TND) outputs, both null or both set (then rows_per_request == 4): output
     * row t < batch * 4 holds query row unpack_indices[t] when output_valid[t] != 0, and -1
     * throughout when output_valid[t] == 0; query rows that no output row names are not
     * published. Null: output row r is query row r. (QueryInputs' unpack indices and output
     * validity, python/kvip/operators/lifetch/index_update.py:18-21; publication
     * op_kernel/streaming.cpp:31-44, :66-89.) */
    const int64_t* unpack_indices;  /* [batch * 4] */
    const int64_t* output_valid;    /* [batch * 4] */
    /* ABC tail of each request, {begin, end} Index positions, or NULL (then no position is a
     * tail position). Set: hot_stride - resident (the ring slots) is a multiple of 128 and at
     * least 384 (python/kvip/operators/lifetch/binding.py:159-164). */
    const int32_t* tail_bounds;     /* [batch, 2] */
    /* Speculative prefetch of the round, both NULL or both set: kvip_hip_resident_prefetch
     * writes the token of every prefetch ordinal and the count per request (which then
     * replaces `used`); kvip_hip_resident_finish resolves selected prefetched tokens to
     * their candidate slot, applies the prefetch as the first Index-update batch and makes
     * every prefetch slot resident. */
    int32_t* prefetch_tokens;       /* [batch, 2048] */
    int32_t* prefetch_counts;       /* [batch] */
} KvipResidentArgs;

/* Speculative windowed prefetch after the prefix classification (kvip_hip_resident_prefix
 * of the same scores and candidates), for each request b: window 0 takes the victim
 * coordinates i (candidate lru_slots[b][i] above its row's prefix threshold, any query
 * row) in ordinal order, window e >= 1 the cold positions of [end_{e-1}, end_e), end_e =
 * resident + 128 * floor(cold_tiles * e / max(1, windows - 1)), cold_tiles = (history -
 * resident) / 128 (trigger_tokens, python/kvip/operators/lifetch/geometry.py:55-61), hit
 * in any query row, in ascending order; mapped ABC tail positions are skipped; each window
 * takes the first min(window_limit, 2048 - used, prefetch_limit - used) of its candidates
 * as ordinals used, used + 1, ...: token -> candidate slot lru_slots[b][ordinal], its
 * change record at the ordinal, its KV row fetched from host_pool into the hot cache.
 * This is the reference's service when every window is serviced after scoring has passed
 * the window's end (it caps each progress snapshot at the window boundary,
 * op_kernel/prefetch.h:609-627); the final round repairs whatever was not prefetched. */
#define KVIP_PREFETCH_MAX_WINDOWS 32
typedef struct KvipPrefetchArgs {
    const uint32_t* victim_hits;  /* [batch * rows_per_request, 64], kvip_hip_resident_prefix */
    const uint32_t* cold_hits;    /* [batch * rows_per_request, cold_words] */
    int32_t* window_counts;       /* [batch, KVIP_PREFETCH_MAX_WINDOWS] prefetch count after each window
                                     (windowed entry points), or NULL */
    int32_t cold_words;           /* >= (history - resident) / 32 */
    int32_t windows;              /* 1..KVIP_PREFETCH_MAX_WINDOWS, fewer than cold_tiles */
    int32_t window_limit;         /* 1..480 */
    int32_t prefetch_limit;       /* 0..2048 */
} KvipPrefetchArgs;

/* Publication of appended KV pages (PageUpdates.submit, python/kvip/cache/page_updates.py:
 * 27-62; kernel _page_updates_kernel.py:8-37): for each of `count` rows {flat page index,
 * address, clear} of `rows`: addresses[index] = address; valid[index] = 1; clear >= 0:
 * token_to_slot[clear .. clear + block_size) = -1; with fused tables, owner = index /
 * (groups * pages), group = index / pages % groups, page = index % pages and fused[2g] the
 * int64 [owners, history] table of group g, fused[2g + 1] its token bytes:
 * table[owner][page * block_size + i] = address + i * token bytes, for positions < history.
 * A row whose index or clear range is out of bounds is skipped and sets
 * KVIP_STATUS_BAD_TOKEN. */
typedef struct KvipPageArgs {
    const int64_t* rows;          /* [count, 3] */
    int64_t* addresses;           /* [entries] = [owners, groups, pages] */
    uint8_t* valid;               /* [entries] */
    int32_t* token_to_slot;       /* [map_entries] */
    const int64_t* fused;         /* [groups, 2] {table pointer, token bytes}, or null */
    uint32_t* status;             /* optional */
    int64_t entries;
    int64_t map_entries;
    int32_t count;
    int32_t groups;
    int32_t pages;
    int32_t block_size;           /* 1..256 */
    int32_t history;              /* positions per owner in the fused tables */
    int32_t reserved;
} KvipPageArgs;

/* Sparse attention over the selected KV rows (the consumer of the LIFetch outputs: the
 * service's sparse flash attention, tests/operators/lifetch/support/correctness.py:261-339;
 * row format workloads.py:493-515). A 656-byte row is 512 fp8 e4m3 nope features, 64 bf16
 * rope features and 4 fp32 scales (scale k covers nope features 128k..128k+127):
 * key = [nope * scale, rope] (576), value = nope * scale (512). For query row r (request
 * b = r / rows_per_request) and head h, over j with indices[r][j] >= 0 (position t lives in
 * block block_table[b][t / 128], row t % 128, of kv_cache):
 *   s_j = scale * <query[r][h], key_j>, p_j = exp(s_j - max s),
 *   output[r][h] = sum_j bf16(p_j) * value_j / sum_j p_j   (0 when no index is valid).
 * Bad positions or blocks set KVIP_STATUS_BAD_TOKEN / _BAD_BLOCK and count as absent. */
typedef struct KvipSparseAttnArgs {
    const uint16_t* query;        /* [rows, heads, 576] bf16, 16-byte aligned */
    const uint8_t* kv_cache;      /* [num_blocks] blocks of 128 rows, 16-byte aligned */
    const int32_t* block_table;   /* [rows / rows_per_request, max_blocks] */
    const int32_t* indices;       /* [rows, 2048] positions, -1 = none */
    float* output;                /* [rows, heads, 512] */
    uint32_t* status;             /* optional */
    float* workspace;             /* kvip_hip_sparse_attention_workspace_bytes(rows, heads) bytes
                                     (null allowed when that is 0); partials of the index splits */
    int64_t kv_block_stride;      /* bytes between blocks, >= 128 * row_stride */
    int32_t row_stride;           /* bytes between rows, >= 656, multiple of 16 */
    int32_t rows;
    int32_t rows_per_request;
    int32_t heads;                /* 1..128 */
    int32_t max_blocks;
    int32_t num_blocks;
    float scale;                  /* softmax scale, e.g. 576^-0.5 */
    int32_t reserved;
} KvipSparseAttnArgs;

/* Resident-prefix classification of one step (the resident TopK, its threshold and the
 * hit bits the speculative prefetch reads): for query row r with valid positions
 * v = min(seq_lens[b], query_ends[r]) and prefix p = min(v, resident), given prefix_topk =
 * the TopK-2048 of positions [0, p) (kvip_hip_topk with limit = resident):
 *   thresholds[r]   = the smallest key of that selection when p >= 2048, else 0;
 *   victim_hits[r]  bit i (word i / 32) = lru_slots[b][i] in [0, p) and its key > threshold;
 *   cold_hits[r]    bit j (word j / 32) = position resident + j < v and its key > threshold. */
typedef struct KvipPrefixClassifyArgs {
    const uint16_t* score_keys;   /* [rows, key_stride] */
    const int32_t* prefix_topk;   /* [rows, 2048] */
    const int32_t* seq_lens;      /* [batch] */
    const int32_t* query_ends;    /* [rows], or NULL */
    const int32_t* lru_slots;     /* [batch, 2048] */
    uint16_t* thresholds;         /* [rows] */
    uint32_t* victim_hits;        /* [rows, 64] */
    uint32_t* cold_hits;          /* [rows, cold_words] */
    int32_t batch;
    int32_t rows_per_request;
    int32_t key_stride;
    int32_t resident;
    int32_t cold_words;           /* >= ceil((key_stride - resident) / 32) */
    int32_t reserved;
} KvipPrefixClassifyArgs;

uint32_t kvip_hip_abi_version(void);
uint32_t kvip_hip_indexer_decode(const KvipIndexerArgs* args, void* stream);
/* kvip_hip_indexer_decode of the token positions [token_begin, token_end) only (token_begin
 * a multiple of 128; token_end a multiple of 128 or at least key_stride; the histogram
 * accumulates, so windows covering the row give the whole row's keys and histogram). fp8
 * Q/K with one row per request (others: KVIP_ERR_INVALID). No reference counterpart: it
 * lets a caller start on the first positions' scores while later ones are scored. */
uint32_t kvip_hip_indexer_decode_window(const KvipIndexerArgs* args, int32_t token_begin, int32_t token_end,
                                        void* stream);
uint32_t kvip_hip_topk(const KvipTopkArgs* args, void* stream);
uint32_t kvip_hip_fetch_gather(const KvipFetchArgs* args, void* stream);
uint32_t kvip_hip_indexer_prefill(const KvipPrefillArgs* args, void* stream);
/* kvip_hip_indexer_prefill on a grid of at most `workgroups` workgroups (0: one per work unit
 * of 8 query rows x 4096 key positions, as kvip_hip_indexer_prefill) that stride over the
 * units; same results. No reference counterpart: a launch shape for callers that run the
 * prefill beside other kernels (a mixed decode + prefill round), where a grid of twice the
 * CU count leaves the CUs that finish their units to the other kernels. */
uint32_t kvip_hip_indexer_prefill_grid(const KvipPrefillArgs* args, int32_t workgroups, void* stream);
uint32_t kvip_hip_lifetch_forward(const KvipLIFetchArgs* args, void* stream);
/* The launch plan kvip_hip_lifetch_forward takes for these arguments (no launch, no device
 * access): KVIP_LIFETCH_PLAN_THREE (scoring, TopK, gather; rows of at most
 * KVIP_TOPK_REGS_MAX_KEYS keys use the register-resident TopK), or KVIP_ERR_INVALID when
 * the forward would reject them. A host query with no counterpart in the reference, for
 * callers and tests that need to know which kernels a round runs. */
#define KVIP_LIFETCH_PLAN_THREE 0u
#define KVIP_TOPK_REGS_MAX_KEYS 65536
uint32_t kvip_hip_lifetch_plan(const KvipLIFetchArgs* args);
/* kvip_hip_lifetch_forward without caller scratch, for callers that cannot allocate device
 * memory (code under hipGraph capture, serving loops or harnesses that forbid hipMalloc).
 * No counterpart in the reference. The score keys and histograms come from one
 * library-owned array of KVIP_LIFETCH_STATIC_SCRATCH_BYTES per GPU (held until the process
 * ends): indexer.score_keys, indexer.histogram, topk.score_keys, topk.histogram,
 * and topk.segments must be NULL, and rows * 1024 (rounded up to 256) + rows *
 * key_stride * 2 bytes must fit the array (rows = batch * rows_per_request), else
 * KVIP_ERR_INVALID and nothing is launched. Same outputs as kvip_hip_lifetch_forward's
 * three-launch plan (plus one small fill launch that clears the histograms first); no
 * hipMalloc, hipFree or memset. Calls that overlap on one GPU share the array and race. */
#define KVIP_LIFETCH_STATIC_SCRATCH_BYTES (16u << 20)
uint32_t kvip_hip_lifetch_forward_static(const KvipLIFetchArgs* args, void* stream);
/* TopK-2048 of rows scored by kvip_hip_indexer_decode fused with the Fetch gather of the
 * selected rows: same outputs as kvip_hip_topk followed by kvip_hip_fetch_gather. Needs
 * topk->histogram and topk->segments; fetch->topk must be topk->topk. */
uint32_t kvip_hip_select_fetch(const KvipTopkArgs* topk, const KvipFetchArgs* fetch, void* stream);
uint32_t kvip_hip_update_abc(const KvipAbcArgs* args, void* stream);
uint32_t kvip_hip_lru_reset(const KvipLruArgs* args, int32_t committed, void* stream);
uint32_t kvip_hip_lru_extend(const KvipLruArgs* args, int32_t active, int32_t committed, void* stream);
uint32_t kvip_hip_lru_commit(const KvipLruArgs* args, const int32_t* destinations, int32_t count, int32_t active,
                             void* stream);
/* The same over `chains` LRUs laid out back to back (one per request of a batch; no
 * reference counterpart: the reference keeps one SlotLRU object per request and commits
 * each from the host, python/kvip/cache/lru.py:96-118). Chain c uses order/scratch +
 * c * capacity, slots + c * 2048, bitmap + c * bitmap_words, and commits destinations
 * [c * dest_stride, + count). One launch for the whole set, so a serving round can commit
 * its slots inside a captured hipGraph. */
uint32_t kvip_hip_lru_reset_chains(const KvipLruArgs* args, int32_t chains, int32_t committed, void* stream);
uint32_t kvip_hip_lru_commit_chains(const KvipLruArgs* args, int32_t chains, const int32_t* destinations,
                                    int64_t dest_stride, int32_t count, int32_t active, void* stream);
uint64_t kvip_hip_lidu_workspace_bytes(int32_t batch);
uint32_t kvip_hip_lidu(const KvipLiduArgs* args, void* stream);
uint32_t kvip_hip_pack_queries(const KvipQueryPackArgs* args, void* stream);
uint32_t kvip_hip_ingest_index(const KvipIngestArgs* args, void* stream);
/* Resident TopK (kvip_hip_topk of `topk`, whose limit must equal cls->resident and whose
 * output must be cls->prefix_topk) followed by the prefix classification. */
uint32_t kvip_hip_resident_prefix(const KvipTopkArgs* topk, const KvipPrefixClassifyArgs* cls, void* stream);
/* kvip_hip_resident_prefix in parts, for a prefetch that follows the scoring window by
 * window: the resident TopK and classification (thresholds, victim bits), then the cold
 * hit bits of the cold words [word_begin, word_end) once those positions are scored. */
uint32_t kvip_hip_resident_threshold(const KvipTopkArgs* topk, const KvipPrefixClassifyArgs* cls, void* stream);
uint32_t kvip_hip_resident_cold_hits(const KvipPrefixClassifyArgs* cls, int32_t word_begin, int32_t word_end,
                                     void* stream);
uint64_t kvip_hip_resident_workspace_bytes(int32_t batch, int32_t history);
uint32_t kvip_hip_resident_prepare(const KvipResidentArgs* args, void* stream);
uint32_t kvip_hip_resident_round(const KvipResidentArgs* args, void* stream);
/* kvip_hip_resident_round in two halves (round = begin then finish) with the prefetch in
 * between: begin = initialisation (and the prefetch counts zeroed), finish = resolve,
 * Fetch, Index update. The prefetch may run on another stream after begin and after the
 * prefix classification; finish must follow both. */
uint32_t kvip_hip_resident_begin(const KvipResidentArgs* args, void* stream);
uint32_t kvip_hip_resident_prefetch(const KvipResidentArgs* args, const KvipPrefetchArgs* prefetch, void* stream);
/* kvip_hip_resident_prefetch window by window (no reference entry point: the reference's
 * service walks the windows as scoring passes them, op_kernel/prefetch.h:578-832):
 * _windows takes the candidates of windows [window_begin, window_end) (window 0 first,
 * each range continuing from the count the earlier ranges left in prefetch_counts) and
 * records the count after each window in prefetch->window_counts; _copy copies the host
 * rows of the ordinals those windows took. Calling _windows over consecutive ranges
 * covering [0, windows) and _copy for each range equals kvip_hip_resident_prefetch. A
 * range's copy may run beside later ranges' decisions (it reads only their earlier window
 * counts); resolve and Index update need only the decisions, kvip_hip_resident_fetch must
 * follow every copy (a final miss may take a slot a copy writes). */
uint32_t kvip_hip_resident_prefetch_windows(const KvipResidentArgs* args, const KvipPrefetchArgs* prefetch,
                                            int32_t window_begin, int32_t window_end, void* stream);
uint32_t kvip_hip_resident_prefetch_copy(const KvipResidentArgs* args, const KvipPrefetchArgs* prefetch,
                                         int32_t window_begin, int32_t window_end, void* stream);
uint32_t kvip_hip_resident_finish(const KvipResidentArgs* args, void* stream);
/* kvip_hip_resident_finish = resolve, then Fetch, then update. The Fetch copies the resolve's
 * misses (it reads fetch_sources/fetch_slots/miss_counts and writes hot_cache only) and the
 * update permutes the Index rows and publishes residency (it reads the resolve's outputs,
 * never hot_cache), so after the resolve the two may run on two streams, in either order or
 * concurrently, with the same results as the sequential finish; a caller joins both before
 * anything reads hot_cache, hot_valid or the Index rows. */
uint32_t kvip_hip_resident_resolve(const KvipResidentArgs* args, void* stream);
uint32_t kvip_hip_resident_fetch(const KvipResidentArgs* args, void* stream);
uint32_t kvip_hip_resident_update(const KvipResidentArgs* args, void* stream);
/* The first half of kvip_hip_resident_forward with the round's initialisation: the
 * initialisation of kvip_hip_resident_begin together with the owner block table (one
 * launch), then the scoring of the owners' Index rows. A prefetching forward follows it
 * with kvip_hip_resident_prefix + kvip_hip_resident_prefetch (possibly on a second stream),
 * the final kvip_hip_topk, then kvip_hip_resident_finish. */
uint32_t kvip_hip_resident_score(const KvipIndexerArgs* indexer, const KvipTopkArgs* topk,
                                 const KvipResidentArgs* resident, void* stream);
/* kvip_hip_resident_score over the token positions [token_begin, token_end) of every row
 * (token_begin a multiple of 128; token_end a multiple of 128 or at least key_stride); the
 * round's initialisation runs with the window that starts at 0. Windows covering
 * [0, key_stride) give the keys and histograms of kvip_hip_resident_score. fp8 indexers with
 * one row per request (others: KVIP_ERR_INVALID). */
uint32_t kvip_hip_resident_score_window(const KvipIndexerArgs* indexer, const KvipTopkArgs* topk,
                                        const KvipResidentArgs* resident, int32_t token_begin, int32_t token_end,
                                        void* stream);
/* One resident-cache LIFetch step: the round's initialisation with block_table[b][j] =
 * row_owners[b] * (history / 128) + j, scoring of the owners' Index rows, TopK-2048, then
 * kvip_hip_resident_finish (the same round as kvip_hip_resident_round). */
uint32_t kvip_hip_resident_forward(const KvipIndexerArgs* indexer, const KvipTopkArgs* topk,
                                   const KvipResidentArgs* resident, void* stream);
/* Sparse attention of the selected rows (no reference entry point: the consumer the
 * reference's tests run on its outputs, correctness.py:261-339). */
uint32_t kvip_hip_sparse_attention(const KvipSparseAttnArgs* args, void* stream);
uint64_t kvip_hip_sparse_attention_workspace_bytes(int32_t rows, int32_t heads);
/* Page publication of one step (PageUpdates.submit, python/kvip/cache/page_updates.py:27-62). */
uint32_t kvip_hip_publish_pages(const KvipPageArgs* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KVIP_HIP_H */
