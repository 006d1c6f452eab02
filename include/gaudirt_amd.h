/*
 * gaudirt_amd — C ABI of the MI355X (gfx950) paged-attention path.
 *
 * Every entry point takes plain pointers, sizes and a hipStream_t, enqueues its
 * work on that stream and returns a status code (GK_OK on success); no C++
 * exception crosses this boundary. Parameter structs begin with struct_size,
 * which the caller sets to sizeof the struct it was compiled with: a caller
 * built against another version of this header is rejected, not misread. On failure gk_last_error() returns a
 * message for the calling thread. Arguments are validated on the host before
 * anything is enqueued, so a rejected call has written nothing.
 *
 * KV pool layout (the reference's head-major combined pool, one layer):
 *   bf16 [2, kv_heads, slots, head_dim]; key row of (head h, slot s) at
 *   element (h * slots + s) * head_dim, value row at
 *   ((kv_heads + h) * slots + s) * head_dim.
 * Block tables: block_tables[request * bt_stride + j] is the pool block that
 * holds tokens [j * block_size, (j + 1) * block_size) of the request, so token
 * t lives at slot block_tables[...t / block_size] * block_size + t % block_size.
 * block_size is a power of two; block_size 1 makes the table the reference's
 * token-granular request map (mapping[request, token] = slot).
 */
#ifndef GAUDIRT_AMD_H
#define GAUDIRT_AMD_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  GK_OK = 0,
  GK_ERR_INVALID_ARGUMENT = 1,
  GK_ERR_UNSUPPORTED = 2,
  GK_ERR_HIP = 3,
  GK_ERR_OUT_OF_MEMORY = 4,
  GK_ERR_WORKSPACE = 5,
};

/* Message of the last failed call on this thread ("" if none). No counterpart
 * in the reference, which reports errors through TORCH_CHECK exceptions. */
const char* gk_last_error(void);
/* Library version string. No counterpart in the reference. */
const char* gk_version(void);

/* ---------------------------------------------------------------------------
 * KV store. Replaces the gk_kv_store_head_major_bf16_v1 launch of
 * src/bridge/paged_attention_tiles.cpp:236-260 (recipe :37-55, fused variant
 * src/bridge/paged_attention.cpp:66-76): for r < rows and every kv head, the
 * row's head slice of key/value is written to slot slot_mapping[r] of the pool.
 * A negative slot skips the row; every other pool byte is untouched.
 * key/value: bf16 [rows, kv_row_stride] (elements), kv_heads * head_dim used.
 * ------------------------------------------------------------------------- */
int gk_kv_store(const void* key, const void* value, int64_t key_row_stride, int64_t value_row_stride,
                const int32_t* slot_mapping, int32_t rows, void* pool, int64_t slots, int32_t kv_heads,
                int32_t head_dim, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Paged decode attention over block tables with split-K partitions and a
 * second-pass log-sum-exp merge. Replaces the fused single-tile recipe and the
 * multi-tile chunk chain of src/bridge/paged_attention.cpp:39-127,264-345 and
 * src/bridge/paged_attention_tiles.cpp:57-195,262-359 (tile softmax,
 * gk_attn_online_merge_f32_v1, gk_attn_online_finalize_bf16_v1).
 *
 * Each query row r attends keys [left, row_context[r]) of request
 * row_request[r], where left = max(0, row_context[r] - sliding_window) when a
 * window is set and 0 otherwise. Scores are q.k in fp32 times `scale`
 * (optionally capped: softcap * tanh(s / softcap)); output bf16.
 * ------------------------------------------------------------------------- */
typedef struct gk_decode_params {
  size_t struct_size;          /* sizeof(gk_decode_params) as the caller was built; checked */
  const void* query;           /* bf16 [rows, q_row_stride]; heads contiguous in a row */
  int64_t q_row_stride;        /* elements */
  const void* pool;            /* head-major combined KV pool of one layer */
  int64_t slots;
  const int32_t* block_tables; /* [requests, bt_stride] */
  int64_t bt_stride;
  int32_t block_size;          /* power of two */
  const int32_t* row_request;  /* [rows] block-table row of each query row; NULL = row index */
  const int32_t* row_context;  /* [rows] visible keys (query position + 1) */
  int32_t rows;
  int32_t q_heads, kv_heads, head_dim; /* head_dim in {64, 128, 256}; q_heads % kv_heads == 0 */
  float scale;
  float softcap;               /* 0 = off */
  int32_t sliding_window;      /* <= 0 = off */
  int32_t max_context;         /* host bound: row_context[r] <= max_context for every row */
  int32_t partition_tokens;    /* split-K partition (multiple of 32); 0 = library choice: a
                                  balanced split of all key tiles over one resident grid
                                  (any GQA group and block_size), or a partition sized from
                                  the batch for batches beyond the split's 32-bit tile
                                  numbering; either way a row's split points,
                                  and so its last bits, depend on the whole batch. A fixed
                                  partition (> 0) makes every row's output a function of
                                  that row alone, bit for bit (batch-invariant decode) */
  void* out;                   /* bf16 [rows, out_row_stride] */
  int64_t out_row_stride;      /* elements */
  /* Optional fused KV store of the new token rows (NULL new_key = none): written
   * with gk_kv_store semantics before any key is read. */
  const void* new_key;
  const void* new_value;
  int64_t new_kv_row_stride;
  const int32_t* slot_mapping;
  /* Optional [rows]: query/output row of work row r (NULL = r), so decode can
   * serve a subset of a batch's rows. row_request/row_context stay per work row. */
  const int32_t* row_map;
} gk_decode_params;

/* Workspace bytes gk_paged_decode needs for these parameters (0 if none). */
size_t gk_paged_decode_workspace_bytes(const gk_decode_params* params);
/* The split-K partition gk_paged_decode uses for these parameters; 0 when the
 * balanced split (partitions chosen on the device from row_context) applies. */
int32_t gk_paged_decode_partition_tokens(const gk_decode_params* params);
int gk_paged_decode(const gk_decode_params* params, void* workspace, size_t workspace_bytes,
                    hipStream_t stream);

/* Allocation-free gk_paged_decode. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Same parameters,
 * kernels and results as gk_paged_decode, whose workspace here is a static
 * device array of GK_DECODE_SCRATCH_BYTES that every GPU the library's code
 * object is loaded on holds until the process ends, whether or not this entry
 * point is ever called (the torch op path included). The first call on each
 * device looks up the array's address and the grid size; make it before any
 * graph capture, after which calls can be captured and replayed (the current
 * device must be the stream's). Parameters whose workspace
 * (gk_paged_decode_workspace_bytes) exceeds it are rejected with
 * GK_ERR_WORKSPACE before anything is enqueued. All calls on one GPU share the
 * array: calls that overlap on one GPU (on different streams, or from
 * different threads) race and must be serialised by the caller; calls on one
 * stream are ordered by it. */
#define GK_DECODE_SCRATCH_BYTES (32u << 20)
int gk_paged_decode_scratch(const gk_decode_params* params, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Chunked / prefix-shared prefill attention with bf16 MFMA. Replaces the
 * prefill blocks of src/bridge/paged_attention.cpp:264-345 (query blocks of up
 * to 256-512 rows over 512-key tiles, src/bridge/attention_plan.cpp:199-237).
 *
 * Sequence s contributes seq_rows[s] consecutive query rows starting at row
 * seq_first_row[s], at positions seq_prefix[s] + i; row i attends keys
 * [left, seq_prefix[s] + i] of block-table row seq_request[s] (causal; left =
 * position - sliding_window + 1 when a window is set, else 0). Every key,
 * including the chunk's own, must already be in the pool (store first).
 * head_dim 64, 128 or 256; GQA group at most 128; block_size any power of two up
 * to 2^20, 1 (the token-granular slot map as the block table) included.
 * query, pool and out are 16-byte aligned and the row strides multiples of 8
 * elements (GK_ERR_INVALID_ARGUMENT otherwise).
 * ------------------------------------------------------------------------- */
typedef struct gk_prefill_params {
  size_t struct_size;          /* sizeof(gk_prefill_params) as the caller was built; checked */
  const void* query;           /* bf16 [rows, q_row_stride] */
  int64_t q_row_stride;
  const void* pool;
  int64_t slots;
  const int32_t* block_tables; /* [requests, bt_stride] */
  int64_t bt_stride;
  int32_t block_size;
  const int32_t* seq_request;   /* [seqs] */
  const int32_t* seq_first_row; /* [seqs] */
  const int32_t* seq_rows;      /* [seqs] */
  const int32_t* seq_prefix;    /* [seqs] position of the chunk's first row */
  int32_t seqs;
  int32_t max_rows;             /* host bound: seq_rows[s] <= max_rows */
  int32_t q_heads, kv_heads, head_dim;
  float scale;
  float softcap;
  int32_t sliding_window;
  void* out;                    /* bf16 [rows, out_row_stride] */
  int64_t out_row_stride;
} gk_prefill_params;

int gk_paged_prefill(const gk_prefill_params* params, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Split-K merge on its own: combines `parts` fp32 partial states per (row, head)
 * into bf16 output. partial_out [rows, heads, max_parts, head_dim] holds
 * unnormalised sums sum_t 2^(s_t - m) v_t; partial_ml [rows, heads, max_parts, 2]
 * holds (m, l) with m in log2 units and l = sum_t 2^(s_t - m); part_count[r] is
 * the number of valid parts of row r. Replaces gk_attn_online_merge_f32_v1 and
 * gk_attn_online_finalize_bf16_v1 (src/bridge/paged_attention_tiles.cpp:173-188).
 * ------------------------------------------------------------------------- */
int gk_split_k_merge(const float* partial_out, const float* partial_ml, const int32_t* part_count,
                     int32_t rows, int32_t heads, int32_t max_parts, int32_t head_dim, void* out,
                     int64_t out_row_stride, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Tile gather indices in the reference's format (gk_attn_tile_indices_i32_v1,
 * src/bridge/attention_plan.cpp:36-57,337-354): task t = {first_row, first_key,
 * lanes, base} int32 x4; out[t * 64 + l] = base + mapping[requests[first_row] *
 * context + first_key + l] for l < lanes, base for the other lanes of a partial
 * task and 0 for a task with no lane.
 * ------------------------------------------------------------------------- */
int gk_attn_tile_indices(const int32_t* mapping, const int32_t* requests, const int32_t* work,
                         int32_t tasks, int32_t context, int32_t* out, hipStream_t stream);

/* Decode-length advance (src/bridge/eager_scheduler.cpp:50-82): next = seq + 1
 * (int64) and orig_next = orig + 1 (int32) in one launch. */
int gk_advance_decode_lengths(const int64_t* seq_lens, const int32_t* orig_seq_lens, int64_t count,
                              int64_t* next, int32_t* orig_next, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Rotary position embedding of the query and key rows. Replaces the
 * gk_rotary_bf16_v1 launch of src/bridge/generic_private_use1.cpp:294-405
 * (rotary_embedding, _rotary_embedding_validated) and the rotary_pos bucket
 * program of src/bridge/eager_ops.cpp:1243-1300 (rotary_embedding_positions).
 *
 * Every head_dim-wide head of a query or key row is rotated in its first
 * rotary_dim elements by the cos/sin row of its position: cos_sin is bf16
 * [cache_rows, rotary_dim], cos in the first rotary_dim / 2 columns, sin in the
 * rest. Pairs (a, b) are (x[i], x[i + rotary_dim / 2]) with is_neox, else
 * (x[2i], x[2i + 1]); each becomes (a cos_i - b sin_i, b cos_i + a sin_i),
 * computed in fp32 and rounded to bf16 (round to nearest even). Elements past
 * rotary_dim are copied. Positions are int32 (positions_int64 = 0) or int64;
 * a position outside [0, cache_rows) reads the nearest cache row (callers
 * validate positions; the reference's validated entry points check them on the
 * host against the cache).
 *
 * gk_rotary_embedding writes q_out and k_out (rows of q_width / k_width
 * elements). gk_rotary_kv_store is the fused write side of a layer: it writes
 * q_out, and instead of k_out stores the rotated key rows and the value rows
 * into the head-major KV pool at slot_mapping[r] with gk_kv_store semantics
 * (k_width = kv_heads * head_dim, head_dim 64/128/256, 16-byte aligned rows;
 * a negative slot skips the row). It replaces the rotary launch plus the KV
 * store that src/bridge/paged_attention.cpp:66-76,251-263 runs on the rotated
 * key, so the rotated key never round-trips through HBM.
 * ------------------------------------------------------------------------- */
typedef struct gk_rotary_params {
  size_t struct_size;          /* sizeof(gk_rotary_params) */
  const void* query;           /* bf16 [rows, q_width], row stride q_row_stride elements */
  int64_t q_row_stride;
  int64_t q_width;             /* a multiple of head_dim */
  const void* key;             /* bf16 [rows, k_width] */
  int64_t k_row_stride;
  int64_t k_width;
  const void* positions;       /* [rows] int32 or int64 */
  int32_t positions_int64;
  const void* cos_sin;         /* bf16 [cache_rows, rotary_dim], row-contiguous */
  int64_t cache_rows;
  int32_t rows, head_dim, rotary_dim, is_neox;
  void* q_out;                 /* bf16 [rows, q_width] */
  int64_t q_out_row_stride;
  void* k_out;                 /* bf16 [rows, k_width]; gk_rotary_embedding only */
  int64_t k_out_row_stride;
  /* gk_rotary_kv_store only: */
  const void* value;           /* bf16 [rows, kv_heads * head_dim] */
  int64_t v_row_stride;
  const int32_t* slot_mapping; /* [rows] */
  void* pool;                  /* head-major pool (see the file comment) */
  int64_t slots;
  int32_t kv_heads;
} gk_rotary_params;

int gk_rotary_embedding(const gk_rotary_params* params, hipStream_t stream);
int gk_rotary_kv_store(const gk_rotary_params* params, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Device metadata: normalisation and validation of device-resident scheduler
 * inputs. Replaces the gk_paged_metadata_i32_v1 / gk_scheduler_metadata_i32_v1
 * and gk_token_indices_i32_v1 / gk_scheduler_tokens_i32_v1 launches of
 * PagedMetadata's device constructor (src/bridge/paged_metadata.cpp:26-80,
 * 176-430).
 *
 * Sequence s owns rows [seq_first_row[s], seq_first_row[s+1]) at positions
 * seq_prefix[s] + i of block-table row batch_requests[s]; row_seq[r] is the
 * sequence of row r. Outputs are int32 [padded_rows] (zero past rows).
 *
 * With mapping and status both set, status[r] receives one code per row
 * (0 = valid), as the reference's device validation reports them:
 *   1 location outside [0, slots) or position outside [0, context) (int64
 *     values that do not fit included)
 *   2 batch_requests[s] outside [0, requests)
 *   3 mapping[request, position] != location
 *   4 the row's location is the output slot of an earlier row
 *   5 position != seq_prefix[s] + (r - seq_first_row[s])
 *   6 (first row of s) some prefix position t < prefix + length of the
 *     sequence's request has no slot (mapping < 0)
 *   7 (first row of s) a prefix slot is the output slot of another
 *     (request, position)
 * A row keeps the first code in the order 1, 2, 3, 5, 4, 6, 7. With
 * page_flags set, bit k of *page_flags is cleared iff every visible token t
 * of every sequence sits at mapping[t & ~(P-1)] + (t & (P-1)) with that page
 * start P-aligned, for P = 2 << k (k < 10). With mapping NULL nothing is
 * checked (scheduler-owned inputs) and no workspace is needed.
 * seq_visible[s] = sum over earlier sequences of (prefix + length);
 * visible_total = the sum over all.
 *
 * Staged words (optional, this library's own addition): staged_count <=
 * GK_METADATA_INLINE_WORDS host int32 words that the launch itself stores at
 * staged_device[0 .. staged_count), carried in the kernel's arguments, so a
 * caller that builds its row_seq / seq_prefix / seq_first_row / seq_visible
 * words on the host needs no separate upload (and its dependency wait) and
 * may reuse the host buffer once the call returns. row_seq, seq_prefix,
 * seq_first_row, positions and seq_visible may point into that range (they
 * are then read as staged); every other input and output must lie outside it.
 * ------------------------------------------------------------------------- */
#define GK_METADATA_INLINE_WORDS 768

typedef struct gk_metadata_params {
  size_t struct_size;           /* sizeof(gk_metadata_params) as the caller was built; checked */
  const void* locations;        /* [rows] int32 or int64 (locations_int64) */
  const void* batch_requests;   /* [batch] */
  const void* positions;        /* [rows] */
  const void* token_ids;        /* [rows] or NULL */
  int32_t locations_int64, requests_int64, positions_int64, tokens_int64;
  const int32_t* mapping;       /* [requests, context] or NULL */
  const int32_t* row_seq;       /* [rows] */
  const int32_t* seq_prefix;    /* [batch] */
  const int32_t* seq_first_row; /* [batch] */
  const int64_t* seq_visible;   /* [batch] */
  int64_t visible_total;
  int32_t rows, padded_rows, batch, requests, context, vocabulary;
  int64_t slots;
  int32_t* out_locations;       /* [padded_rows] */
  int32_t* out_requests;        /* [padded_rows] request of each row */
  int32_t* out_positions;       /* [padded_rows] */
  int32_t* out_tokens;          /* [padded_rows] when token_ids is set */
  int32_t* status;              /* [padded_rows] or NULL */
  int32_t* token_status;        /* [padded_rows] 1 = token outside [0, vocabulary), or NULL */
  int32_t* page_flags;          /* [1] or NULL */
  const int32_t* staged_words;  /* [staged_count] host words, or NULL */
  int32_t* staged_device;       /* device destination of the staged words, or NULL */
  int32_t staged_count;         /* 0, or 1 .. GK_METADATA_INLINE_WORDS */
} gk_metadata_params;

size_t gk_metadata_workspace_bytes(int32_t rows, int32_t batch);
int gk_metadata_normalize(const gk_metadata_params* params, void* workspace, size_t workspace_bytes,
                          hipStream_t stream);

/* Block tables of a request map whose visible tokens are page-aligned with
 * page size P (a power of two <= 1024): tables[r * pages + k] =
 * mapping[r, k P] / P (-1 where that slot is negative or k P >= context).
 * Replaces the per-token gather indices of gk_attn_tile_indices_i32_v1
 * (src/bridge/attention_plan.cpp:36-57) for page-aligned maps. */
int gk_block_tables(const int32_t* mapping, int32_t requests, int32_t context, int32_t page_size,
                    int32_t* tables, int32_t pages, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Paged slot allocator (gk_paged_alloc_i32_v1 / gk_paged_free_i32_v1 of
 * src/bridge/paged_slot_allocator.cpp:91-190).
 *
 * Allocation: seq_meta[4 s .. 4 s + 3] = {prefix, length, first output index,
 * first free page} (int64, device). Sequence s's first min(length,
 * (-prefix) mod P) new tokens continue at last_slots[s] + 1, + 2, ...; the rest
 * fill pages free_pages[first free page], ... in order, P tokens per page.
 * out_slots [total] int64.
 * ------------------------------------------------------------------------- */
int gk_paged_alloc_slots(const int64_t* last_slots, const int64_t* free_pages, const int64_t* seq_meta,
                         int32_t batch, int64_t page_size, int64_t total, int64_t* out_slots, hipStream_t stream);

/* Release: the distinct pages slot / P of slots[0 .. n), in order of first
 * occurrence, into out_pages; *out_count (device int32) = their number, or -1
 * when a slot's page lies outside [1, max_pages] (page 0 is reserved). */
size_t gk_paged_release_workspace_bytes(int64_t max_pages);
int gk_paged_release_slots(const int64_t* slots, int64_t n, int64_t page_size, int64_t max_pages, void* workspace,
                           size_t workspace_bytes, int64_t* out_pages, int32_t* out_count, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Stream-ordered block allocator (replaces runtime::BlockCachingAllocator,
 * include/gaudirt/runtime/block_caching_allocator.hpp:19-70, for this path).
 * HBM slabs from hipMalloc, carved into 256-byte aligned blocks by best fit.
 * A block freed after use on other streams is reused on a stream only after
 * that stream waits on events recorded on them (no host synchronisation);
 * events come from a pool, so steady state creates none.
 * ------------------------------------------------------------------------- */
typedef struct gk_allocator gk_allocator;

typedef struct gk_allocator_stats {
  uint64_t allocated_bytes;
  uint64_t peak_bytes;
  uint64_t reserved_bytes;
  uint64_t largest_free_block;
  uint64_t slabs;
  uint64_t events_created;
} gk_allocator_stats;

/* budget_bytes caps the total slab bytes; slab_bytes is the default slab size. */
int gk_allocator_create(int32_t device, uint64_t budget_bytes, uint64_t slab_bytes, gk_allocator** out);
int gk_allocator_destroy(gk_allocator* allocator);
int gk_allocator_alloc(gk_allocator* allocator, uint64_t bytes, hipStream_t stream, void** out);
int gk_allocator_record_stream(gk_allocator* allocator, void* ptr, hipStream_t stream);
int gk_allocator_free(gk_allocator* allocator, void* ptr);
/* Waits for pending reuse fences and returns fully free slabs to HIP. */
int gk_allocator_empty_cache(gk_allocator* allocator);
int gk_allocator_get_stats(gk_allocator* allocator, gk_allocator_stats* stats);

#ifdef __cplusplus
}
#endif

#endif /* GAUDIRT_AMD_H */
