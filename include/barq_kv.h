/*
 * barq_kv.h -- C ABI of the MI355X (gfx950) paged KV-cache library (libbarq_kv.so).
 *
 * Every entry point takes plain device pointers and sizes, enqueues its work on
 * the HIP stream it is given (NULL = the null stream), allocates nothing, never
 * synchronises with the host, and returns a barq_kv_status code.  Element data is
 * moved as raw bits (elem_bytes of 1, 2, 4 or 8), so bf16 / fp16 / fp32 / fp64
 * caches, NaN payloads included, come back bit-identical.
 *
 * Reference interfaces replaced (files under the BarqTrain tree):
 *   barq_kv_append_dense  <- paged_kv_append_cuda, csrc/kernels/paged_kv_cache.cu:58-128,
 *                            bound as barqtrain_cuda.paged_kv_append_ at
 *                            csrc/src/bindings.cpp:43-49,74-75
 *   barq_kv_append        <- BarqPagedKVCacheLayer.append / _python_append,
 *                            python/barqtrain/kv_cache.py:75-118 (page-pool layout)
 *   barq_kv_gather        <- BarqPagedKVCacheLayer._flatten_pages + current_tensors,
 *                            python/barqtrain/kv_cache.py:120-133 (materialised)
 *   barq_kv_update        <- BarqPagedKVCacheLayer.update, python/barqtrain/kv_cache.py:135-142
 *   barq_kv_crop          <- BarqPagedKVCacheLayer.crop, python/barqtrain/kv_cache.py:158-164
 *   barq_kv_pool_reset    <- BarqPagedKVCacheLayer.lazy_initialization / reset,
 *                            python/barqtrain/kv_cache.py:53-73,188-194
 *   barq_kv_copy_rows     <- batch_repeat_interleave / batch_select_indices / reorder_cache,
 *                            python/barqtrain/kv_cache.py:166-186
 *   barq_kv_free_rows     <- no reference counterpart: returns a finished sequence's pages
 *                            to the pool (the page allocator the reference only planned,
 *                            IMPLEMENTATION_PLAN.md:90-92).
 *   barq_kv_select_rows   <- batch_select_indices / batch_repeat_interleave / reorder_cache,
 *                            python/barqtrain/kv_cache.py:166-186, in place: rows share their
 *                            full pages (copy-on-write) instead of copying the cache.
 *   barq_kv_select_rows_layers, barq_kv_select_workspace_words
 *                         <- Cache.reorder_cache / batch_select_indices / batch_repeat_interleave
 *                            (transformers cache_utils, which the reference's BarqPagedKVCache
 *                            inherits, python/barqtrain/kv_cache.py:197-223): one selection for
 *                            every layer, in one set of launches.
 *   barq_kv_decode_attention, barq_kv_attention_workspace_bytes
 *                         <- no reference counterpart: the "gather/scatter kernels for attention
 *                            reads" the reference planned (IMPLEMENTATION_PLAN.md:90-91); it
 *                            replaces current_tensors() followed by attention over the
 *                            materialised K/V (python/barqtrain/kv_cache.py:120-142).
 *
 * Calls that name the same pool must be ordered on one stream; calls on different
 * pools are independent.
 */
#ifndef BARQ_KV_H
#define BARQ_KV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes. */
#define BARQ_KV_OK 0
#define BARQ_KV_ERR_INVALID 1 /* a pointer, size, stride or alignment the kernels cannot take */
#define BARQ_KV_ERR_LAUNCH 2  /* the HIP runtime refused a launch */
#define BARQ_KV_ERR_SCRATCH 3 /* the request needs more than the library's static scratch
                                 (BARQ_KV_SCRATCH_BYTES per GPU); use the workspace variant */

/* Words of barq_kv_pool.ctrl.  Counters sit on lines of their own; all counters are 0 between
   launches. */
#define BARQ_KV_CTRL_FREE_TOP 0 /* number of entries of free_pages that are free pages */
#define BARQ_KV_CTRL_ERRORS 1   /* sticky error bits below, set by kernels, cleared by reset */
#define BARQ_KV_CTRL_COLD_TOP 2 /* number of entries of a cold store's free_cold that are free */
#define BARQ_KV_CTRL_ARRIVED 32 /* tile arrival counter of the running launch */
#define BARQ_KV_CTRL_SUBCOUNTER0 64       /* first of the arrival sub-counters ... */
#define BARQ_KV_CTRL_SUBCOUNTER_STRIDE 64 /* ... one per 256 bytes ... */
#define BARQ_KV_CTRL_SUBCOUNTERS 16       /* ... this many */
#define BARQ_KV_CTRL_WORDS (BARQ_KV_CTRL_SUBCOUNTER0 + BARQ_KV_CTRL_SUBCOUNTERS * BARQ_KV_CTRL_SUBCOUNTER_STRIDE)
/* Arrival counts of decode attention's split (row, kv head) pairs, one word per pair q <
   BARQ_KV_CTRL_PAIR_SLOTS, in the second 128 bytes of each sub-counter's 256. */
#define BARQ_KV_CTRL_PAIR_SLOTS (BARQ_KV_CTRL_SUBCOUNTERS * 32)
#define BARQ_KV_CTRL_PAIR_WORD(q) \
  (BARQ_KV_CTRL_SUBCOUNTER0 + ((q) / 32) * BARQ_KV_CTRL_SUBCOUNTER_STRIDE + 32 + (q) % 32)

/* Sticky error bits in ctrl[BARQ_KV_CTRL_ERRORS]. */
#define BARQ_KV_ERRBIT_POOL_EXHAUSTED 1 /* a new block found no free page; its tokens were dropped */
#define BARQ_KV_ERRBIT_CAPACITY 2       /* a position fell at or beyond max_blocks * page_size */
#define BARQ_KV_ERRBIT_BAD_INDEX 4      /* a row index outside [0, max_batch) was given, or an
                                           attention read met a block naming no page */
#define BARQ_KV_ERRBIT_OUT_SHORT 8      /* an update's output extent ended before a row's new
                                           tokens; those tokens were not stored */
#define BARQ_KV_ERRBIT_ATTN_SHORT 16    /* a decode-attention launch's max_seq was below a row's
                                           length; that row attended its first max_seq tokens */

/* Flags of barq_kv_gather / barq_kv_update. */
#define BARQ_KV_SEQ_FROM_DEVICE 1 /* seq_out is the output's capacity; the positions written are
                                     [0, max over rows of seq_lens (after the append)), read on the
                                     device, so one launch (or a captured graph) serves every step */
#define BARQ_KV_SEPARATE_FINALIZE 2 /* update the pool's row metadata in a second, one-workgroup
                                       launch instead of in the last tile of the copy launch */

/*
 * One layer's page pool.  All pointers are device pointers.
 *   key_pages / value_pages : [num_pages, page_size, kv_heads, head_dim] elements of elem_bytes
 *   block_table             : int32 [max_batch, max_blocks], page id of (row, block) or -1
 *   seq_lens                : int32 [max_batch], tokens visible in each row
 *   high_water              : int32 [max_batch], slots [0, high_water) of the row have been written
 *   free_pages              : int32 [num_pages], a stack; entries [0, ctrl[FREE_TOP]) are free
 *   ctrl                    : int32 [BARQ_KV_CTRL_WORDS], 256-byte aligned
 *   page_shares             : int32 [num_pages], references to the page beyond the first (0 for
 *                             a free page and for a page one block maps), or NULL for a pool
 *                             whose rows never share pages (barq_kv_select_rows needs it)
 * Invariants kept by every entry point: block b of row r holds a page iff
 * b * page_size < high_water[r]; a page is on the free stack iff no block holds it; a page held
 * by k blocks has page_shares k - 1; only blocks wholly below their row's seq_lens are shared
 * (barq_kv_crop can break the last one; see there).
 */
typedef struct barq_kv_pool {
  void* key_pages;
  void* value_pages;
  int32_t* block_table;
  int32_t* seq_lens;
  int32_t* high_water;
  int32_t* free_pages;
  int32_t* ctrl;
  int32_t* page_shares;
  int64_t num_pages;
  int64_t max_batch;
  int64_t max_blocks;
  int64_t page_size;
  int64_t kv_heads;
  int64_t head_dim;
  int64_t elem_bytes;
} barq_kv_pool;

/* Library version string. */
const char* barq_kv_version(void);

/* Human-readable text of a return code. */
const char* barq_kv_status_string(int status);

/*
 * Dense drop-in for the reference kernel: key_cache / value_cache are contiguous
 * [cache_batch, kv_heads, max_blocks, page_size, head_dim]; key_states / value_states are
 * [batch, kv_heads, tokens, head_dim] with element strides (stride_b, stride_h, stride_t) and a
 * contiguous last dimension.  Token t of row b lands at slot seq_lens[b] + t; slots whose block
 * is >= max_blocks are skipped.  Afterwards seq_lens[0, batch) += tokens.
 * The capacity check of the reference (paged_kv_cache.cu:92-99) is the caller's, on its own
 * copy of the lengths.
 */
int barq_kv_append_dense(void* key_cache, void* value_cache, int32_t* seq_lens,
                         const void* key_states, const void* value_states, int64_t batch,
                         int64_t kv_heads, int64_t tokens, int64_t head_dim, int64_t cache_batch,
                         int64_t max_blocks, int64_t page_size, int64_t elem_bytes,
                         int64_t stride_b, int64_t stride_h, int64_t stride_t, void* stream);

/*
 * Empty the pool: every page free, every block unmapped, seq_lens = high_water = 0, errors
 * cleared.  page_order (device int32 [num_pages], a permutation, or NULL for 0, 1, 2, ...)
 * is the order in which later appends take pages.
 */
int barq_kv_pool_reset(const barq_kv_pool* pool, const int32_t* page_order, void* stream);

/*
 * Append tokens to rows [0, batch): token t of row b lands at slot seq_lens[b] + t.  Blocks
 * that become used take pages from the free stack in row order.  Afterwards
 * seq_lens[b] += tokens and high_water[b] = max(high_water[b], seq_lens[b]).
 * key_states / value_states: [batch, kv_heads, tokens, head_dim], element strides
 * (stride_b, stride_h, stride_t), contiguous last dimension.
 */
int barq_kv_append(const barq_kv_pool* pool, const void* key_states, const void* value_states,
                   int64_t batch, int64_t tokens, int64_t stride_b, int64_t stride_h,
                   int64_t stride_t, void* stream);

/*
 * Materialise rows [0, batch) into key_out / value_out, [batch, kv_heads, seq, head_dim] with
 * element strides (out_stride_b, out_stride_h, out_stride_s) and a contiguous last dimension.
 * Slot s of row b is the value last written there when s < high_water[b], else zero.  Writes
 * positions [0, seq_out), or with BARQ_KV_SEQ_FROM_DEVICE [0, max_b seq_lens[b]) within a
 * buffer of capacity seq_out.
 */
int barq_kv_gather(const barq_kv_pool* pool, void* key_out, void* value_out, int64_t batch,
                   int64_t seq_out, int64_t out_stride_b, int64_t out_stride_h,
                   int64_t out_stride_s, int64_t flags, void* stream);

/* barq_kv_append followed by barq_kv_gather, in one pass over the pool. */
int barq_kv_update(const barq_kv_pool* pool, const void* key_states, const void* value_states,
                   int64_t batch, int64_t tokens, int64_t stride_b, int64_t stride_h,
                   int64_t stride_t, void* key_out, void* value_out, int64_t seq_out,
                   int64_t out_stride_b, int64_t out_stride_h, int64_t out_stride_s,
                   int64_t flags, void* stream);

/*
 * barq_kv_update (flags 0) for a caller that holds the pool's row state: seq_lens[0 .. batch),
 * high_water[0 .. batch) (host arrays) and free_top must equal the pool's device values when the
 * launch runs (an eager caller's exact shadow of its own stream-ordered calls; a wrong value
 * gives wrong pages and lengths, as a wrong block table would).  The same results and pool state
 * as barq_kv_update, from a launch that reads none of that state on the device and commits it
 * without waiting for every tile (a small launch then ends with its copies, not after two
 * dependent counter round trips).  Launches outside the kernel's shapes (more than 64 rows, tiles
 * not all resident at once, other geometries) run barq_kv_update.  It replaces the same
 * reference path as barq_kv_update, the per-call paged_kv_append_ + current_tensors of
 * python/barqtrain/kv_cache.py:93-142, for callers that track their lengths on the host
 * (BarqPagedKVCacheLayer's shadow, kv_cache.py:150-153 read without a sync).
 */
int barq_kv_update_known(const barq_kv_pool* pool, const void* key_states, const void* value_states,
                         int64_t batch, int64_t tokens, int64_t stride_b, int64_t stride_h,
                         int64_t stride_t, void* key_out, void* value_out, int64_t seq_out,
                         int64_t out_stride_b, int64_t out_stride_h, int64_t out_stride_s,
                         const int32_t* seq_lens, const int32_t* high_water, int64_t free_top,
                         void* stream);

/*
 * seq_lens[b] = min(seq_lens[b], max_length) for rows [0, batch).  Page data is kept.  On a pool
 * whose rows share pages a crop can leave a shared block at or above its row's new length, where
 * the next append would write it for every row holding it: call barq_kv_select_rows with
 * src_rows = 0, 1, ..., max_batch - 1 before that append; it gives such blocks pages of their own
 * (and moves, rather than copies, every page only one block holds).
 */
int barq_kv_crop(const barq_kv_pool* pool, int64_t batch, int64_t max_length, void* stream);

/*
 * Drop the listed rows' references to their pages (device int32 [num_rows], distinct) and set
 * their seq_lens and high_water to 0; a page no block holds any more returns to the free stack.
 */
int barq_kv_free_rows(const barq_kv_pool* pool, const int32_t* rows, int64_t num_rows,
                      void* stream);

/*
 * In place: row i, for i in [0, num_rows), becomes row src_rows[i] as it was before the call
 * (src_rows: device int32 [num_rows], values in [0, max_batch), repeats allowed); every other
 * row becomes empty.  A row's blocks wholly below its seq_lens are shared with the source row
 * (page_shares counts the extra references).  The blocks an append or a crop can still write --
 * from the one holding position seq_lens up to high_water -- move to the first new row taking
 * the source when no other block holds their page, and are copied into pages from the free
 * stack otherwise: a permutation copies nothing, a beam step one partial page per repeated
 * source.  All or nothing: when the free stack cannot hold the copies, nothing changes and
 * BARQ_KV_ERRBIT_POOL_EXHAUSTED is set.  Pages no block holds any more return to the stack, in
 * no fixed order.  Needs page_shares, num_rows <= max_batch <= 8192, and a workspace of
 * barq_kv_select_workspace_words(pool, 1, num_rows) int32 words (also for num_rows = 0).
 * Three kernels on the stream.
 */
int barq_kv_select_rows(const barq_kv_pool* pool, const int32_t* src_rows, int64_t num_rows,
                        int32_t* workspace, int64_t workspace_words, void* stream);

/*
 * barq_kv_select_rows applied with the same src_rows to each of num_pools pools (a model's
 * layers, as Cache.reorder_cache / batch_select_indices apply one selection to every layer), in
 * one set of three launches per 32 pools, each pool all or nothing as in barq_kv_select_rows.
 * The pools must be distinct, each with page_shares,
 * and share max_batch, max_blocks, page_size, kv_heads, head_dim and elem_bytes (num_pages may
 * differ).  Workspace: int32 [barq_kv_select_workspace_words(pools, num_pools, num_rows)].
 */
int barq_kv_select_rows_layers(const barq_kv_pool* pools, int64_t num_pools, const int32_t* src_rows,
                               int64_t num_rows, int32_t* workspace, int64_t workspace_words,
                               void* stream);

/* Workspace words barq_kv_select_rows_layers needs -- min(num_pools, 32) *
 * (num_rows * (max_blocks + 3) + max_batch + 2) -- or -1 for arguments it rejects (num_pools < 1,
 * num_rows outside [0, max_batch], max_batch > 8192).  num_pools = 1 gives barq_kv_select_rows'. */
int64_t barq_kv_select_workspace_words(const barq_kv_pool* pool, int64_t num_pools, int64_t num_rows);

/*
 * Row i of dst, for i in [0, num_rows), becomes a copy of row src_rows[i] of src (device int32
 * [num_rows]; repeats allowed): lengths, high-water mark and the contents of its pages, which
 * are taken from dst's free stack.  dst must be empty (just reset), have the geometry of src,
 * num_rows <= dst->max_batch, and enough free pages.
 */
int barq_kv_copy_rows(const barq_kv_pool* src, const barq_kv_pool* dst, const int32_t* src_rows,
                      int64_t num_rows, void* stream);

/* Flags of barq_kv_decode_attention. */
#define BARQ_KV_ATTN_FP16 1    /* pages and query hold IEEE binary16; default bfloat16 */
#define BARQ_KV_ATTN_OUT_F32 2 /* out holds float32; default the pages' element type */

/*
 * Bytes of workspace barq_kv_decode_attention needs for these arguments (the same batch,
 * q_heads, tokens, max_seq and split_tokens), or -1 when it would reject them.
 */
int64_t barq_kv_attention_workspace_bytes(const barq_kv_pool* pool, int64_t batch,
                                          int64_t q_heads, int64_t tokens, int64_t max_seq,
                                          int64_t split_tokens);

/*
 * Decode attention over rows [0, batch) of a 2-byte (bf16 / fp16) pool with head_dim 64, 128 or
 * 256 (D below), reading K and V from the pages:
 *   out[b, h, i, :] = sum_t softmax_t(scale * q[b, h, i, :] . K[b, h / G, t, :]) V[b, h / G, t, :]
 * over positions t <= seq_lens[b] - tokens + i (the query tokens are the row's last `tokens`
 * positions, already appended), G = q_heads / kv_heads.  A row with no visible position gets
 * zeros.  query: [batch, q_heads, tokens, D] of the pool's type, element strides (q_stride_b,
 * q_stride_h, q_stride_t), 16-byte aligned rows; out: [batch, q_heads, tokens, D] of the
 * pool's type or float32 (BARQ_KV_ATTN_OUT_F32), element strides (out_stride_*), each a
 * multiple of 8.  G * tokens <= 16, batch <= 1024.  max_seq bounds every row's length (0 = the pool's
 * capacity; longer rows attend their first max_seq positions and are flagged).  The work is
 * cut into equal ranges of every row's positions, one per resident wave of the GPU, so ragged
 * rows cost what their positions cost; split_tokens instead fixes the positions of a range
 * (rounded up to 16; 0 = automatic).  Ranges that end inside a (row, kv head) keep partial
 * results in workspace (device memory of barq_kv_attention_workspace_bytes(...) bytes, 16-byte
 * aligned, no initialisation needed), merged by a second launch on the same stream; launches
 * that share a workspace must not overlap.  Rows of up to 44 to 2,304 chunks of 16 positions (by
 * batch and query rows) take one launch instead, one or more workgroups per (row, kv head); the
 * workgroups of a split pair pass their partial results through the workspace and count their
 * arrivals on the pool's ctrl (BARQ_KV_CTRL_PAIR_WORD), which they leave at 0, so calls on one
 * pool are ordered on one stream like every call naming it.
 */
int barq_kv_decode_attention(const barq_kv_pool* pool, const void* query, int64_t batch,
                             int64_t q_heads, int64_t tokens, int64_t q_stride_b,
                             int64_t q_stride_h, int64_t q_stride_t, void* out,
                             int64_t out_stride_b, int64_t out_stride_h, int64_t out_stride_t,
                             float scale, int64_t max_seq, int64_t split_tokens, int64_t flags,
                             void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of the static device scratch behind barq_kv_decode_attention_noalloc (per GPU). */
#define BARQ_KV_SCRATCH_BYTES (24 * 1024 * 1024)

/*
 * No counterpart in the reference.  For callers that cannot allocate device memory -- code under
 * HIP graph capture, a serving loop that forbids hipMalloc, harnesses that count allocations --:
 * barq_kv_decode_attention with the workspace taken from a static device array of the library
 * (BARQ_KV_SCRATCH_BYTES on each GPU it runs on, held until the process ends) instead of an
 * argument.  Arguments, results and errors as barq_kv_decode_attention; a launch whose workspace
 * (barq_kv_attention_workspace_bytes) exceeds BARQ_KV_SCRATCH_BYTES returns BARQ_KV_ERR_SCRATCH
 * and enqueues nothing.  With the automatic split the workspace is (2048 + batch * kv_heads)
 * records of (G * tokens) * (head_dim + 2) floats, so 24 MiB holds every batch <= 64 with 8 KV heads
 * and head_dim 128 at G * tokens <= 16 (21.3 MB at the largest); batch 1024 at that shape needs
 * 85 MB and is refused.  Head_dim 256 doubles the records: the same batches fit at
 * G * tokens <= 9 (23.8 MB), and G * tokens = 16 is refused at any batch (33.9 MB at batch 1).  The workspace needs no initialisation, so calls clear nothing.  Every call on
 * a GPU uses that GPU's one array: calls that overlap on one GPU (other streams, other host
 * threads) race on it; order them on one stream.  The first call on a device resolves the array's
 * address there; the call allocates nothing.
 */
int barq_kv_decode_attention_noalloc(const barq_kv_pool* pool, const void* query, int64_t batch,
                                     int64_t q_heads, int64_t tokens, int64_t q_stride_b,
                                     int64_t q_stride_h, int64_t q_stride_t, void* out,
                                     int64_t out_stride_b, int64_t out_stride_h,
                                     int64_t out_stride_t, float scale, int64_t max_seq,
                                     int64_t split_tokens, int64_t flags, void* stream);

/*
 * ---- Quantised KV pages (fp8), no reference counterpart: the reference plans "quantized KV-cache
 * storage", a "residual full-precision window plus compressed older pages" and "dequant-on-read"
 * (IMPLEMENTATION_PLAN.md:106-129, after KIVI) and ships none. ----
 *
 * A pool may carry a cold store.  A row's block j is "cold" once it lies wholly before the row's
 * residual window -- (j + 1) * page_size <= seq_lens - window -- and barq_kv_compress has run:
 * its K and V then live in the cold store as OCP FP8 E4M3 codes (round to nearest even) with
 * power-of-two scales stored as E8M0 bytes (2^(s - 127)): keys one scale per channel (head, dim)
 * over the page's tokens, values one per token (token, head) over head_dim, each the smallest
 * power of two 2^e with max |x| <= 448 * 2^e over the group's finite elements (e = 0 for a group
 * with none non-zero, e clamped to [-127, 127]).  Reads dequantise: code * 2^e, rounded to the
 * pool's element type.  The block table names cold page c as BARQ_KV_COLD_ENTRY(c) (<= -2).
 * Appends (barq_kv_append) only write at or after seq_lens, which stays in hot pages; a pool with
 * a cold store is read with barq_kv_gather_cold and released with barq_kv_free_rows_cold.
 * Element types: bf16, fp16, fp32.  Limits: page_size * kv_heads <= 4096, kv_heads * head_dim
 * <= 16384, num_cold < 2^31 - 2.
 */
#define BARQ_KV_COLD_ENTRY(c) (-2 - (c))

typedef struct barq_kv_cold {
  void* key_codes;     /* uint8 [num_cold, page_size, kv_heads, head_dim] */
  void* value_codes;   /* uint8 [num_cold, page_size, kv_heads, head_dim] */
  void* key_scales;    /* uint8 [num_cold, kv_heads, head_dim]: E8M0, per channel */
  void* value_scales;  /* uint8 [num_cold, page_size, kv_heads]: E8M0, per token */
  int32_t* free_cold;  /* int32 [num_cold], a stack; entries [0, ctrl[BARQ_KV_CTRL_COLD_TOP]) free */
  int32_t* cold_shares; /* int32 [num_cold], references to the cold page beyond the first (0 for a
                           free page and for a page one block maps), or NULL for a store whose
                           rows never share cold pages (barq_kv_select_rows_cold_layers needs it) */
  int64_t num_cold;
  int64_t window;      /* residual window in tokens, >= 0 */
  int64_t element_type; /* the pool's elements: BARQ_KV_BF16, BARQ_KV_FP16 or BARQ_KV_FP32 */
} barq_kv_cold;

#define BARQ_KV_BF16 0
#define BARQ_KV_FP16 1
#define BARQ_KV_FP32 2

/* Every cold page free and cold_shares zero (after barq_kv_pool_reset, which clears ctrl). */
int barq_kv_cold_reset(const barq_kv_pool* pool, const barq_kv_cold* cold, void* stream);

/*
 * Rows [0, batch): every hot block wholly before the residual window is quantised into a cold
 * page taken from free_cold and its hot page returns to free_pages (in no fixed order).  A block
 * finding no cold page stays hot and sets BARQ_KV_ERRBIT_POOL_EXHAUSTED; a hot page another
 * block shares (page_shares) stays hot.  One workgroup per row; rows without such a block exit
 * at once, so it can run after every append (and inside a captured graph).
 */
int barq_kv_compress(const barq_kv_pool* pool, const barq_kv_cold* cold, int64_t batch, void* stream);

/* barq_kv_gather for a pool with a cold store: cold blocks are dequantised on the way out. */
int barq_kv_gather_cold(const barq_kv_pool* pool, const barq_kv_cold* cold, void* key_out,
                        void* value_out, int64_t batch, int64_t seq_out, int64_t out_stride_b,
                        int64_t out_stride_h, int64_t out_stride_s, int64_t flags, void* stream);

/* barq_kv_append + barq_kv_compress + barq_kv_gather_cold.  When tokens <= window, batch <= 64
 * and the pool holds two-byte elements whose token rows are 64, 128 or 256 vectors of 16 bytes
 * (every address and stride 16-byte aligned, codes and key scales 8-byte), in two launches: the
 * compress for the lengths the rows reach, then one launch that appends and gathers; else in three
 * launches (append, compress, gather).  The two forms return the same K/V and leave the same
 * pool, with one exception: in the two-launch form, as for barq_kv_update, a row whose new end
 * passes seq_out does not store the tokens past seq_out in its pages (BARQ_KV_ERRBIT_OUT_SHORT is
 * raised), while the three-launch form stores them.  The compress of the two-launch form runs
 * before the append: if the second launch then fails (BARQ_KV_ERR_LAUNCH), the blocks that leave
 * the window at the lengths the rows would have reached are already quantised (they are whole
 * blocks at the current lengths too, so the pool stays consistent and the lengths unchanged; a
 * gather returns their dequantised values).
 * flags: BARQ_KV_SEQ_FROM_DEVICE as for the gather; BARQ_KV_NO_COMPRESS skips the compress launch
 * -- for a caller that knows no row's block leaves the window in this call (every page_size-th
 * token). */
#define BARQ_KV_NO_COMPRESS 4
int barq_kv_update_cold(const barq_kv_pool* pool, const barq_kv_cold* cold, const void* key_states,
                        const void* value_states, int64_t batch, int64_t tokens, int64_t stride_b,
                        int64_t stride_h, int64_t stride_t, void* key_out, void* value_out,
                        int64_t seq_out, int64_t out_stride_b, int64_t out_stride_h,
                        int64_t out_stride_s, int64_t flags, void* stream);

/*
 * barq_kv_decode_attention for a pool with a cold store: quantised blocks are read as their fp8
 * codes and scales (half the bytes of a bf16 page) and dequantised in registers to exactly the
 * values barq_kv_gather_cold returns, so the result equals attention over the dequantising
 * gather.  Needs page_size a multiple of 16 and the cold store's element type matching flags
 * (bf16, or fp16 with BARQ_KV_ATTN_FP16); workspace as for barq_kv_decode_attention.
 */
int barq_kv_decode_attention_cold(const barq_kv_pool* pool, const barq_kv_cold* cold, const void* query,
                                  int64_t batch, int64_t q_heads, int64_t tokens, int64_t q_stride_b,
                                  int64_t q_stride_h, int64_t q_stride_t, void* out, int64_t out_stride_b,
                                  int64_t out_stride_h, int64_t out_stride_t, float scale, int64_t max_seq,
                                  int64_t split_tokens, int64_t flags, void* workspace, int64_t workspace_bytes,
                                  void* stream);

/* barq_kv_free_rows for a pool with a cold store: a cold page returns to free_cold when no block
 * holds it any more (cold_shares counts the others). */
int barq_kv_free_rows_cold(const barq_kv_pool* pool, const barq_kv_cold* cold, const int32_t* rows,
                           int64_t num_rows, void* stream);

/*
 * barq_kv_select_rows_layers for pools with cold stores (colds[i] is pools[i]'s), replacing
 * batch_select_indices / batch_repeat_interleave / reorder_cache (python/barqtrain/kv_cache.py:
 * 166-186) on quantised caches: a quantised block never changes, so the new rows share it
 * (cold_shares counts the extra references); every hot block below the high-water mark -- the
 * residual window and the partial block, which an append, a crop or barq_kv_compress may still
 * rewrite -- moves to the first new row taking its source when no other block holds its page,
 * and is copied into a page from the free stack otherwise, so hot pages are never shared.  All
 * or nothing per pool, workspace and geometry rules as for barq_kv_select_rows_layers; needs
 * page_shares and cold_shares.
 */
int barq_kv_select_rows_cold_layers(const barq_kv_pool* pools, const barq_kv_cold* colds, int64_t num_pools,
                                    const int32_t* src_rows, int64_t num_rows, int32_t* workspace,
                                    int64_t workspace_words, void* stream);

/*
 * barq_kv_crop for a pool with a cold store (python/barqtrain/kv_cache.py:158-164): seq_lens[b] =
 * min(seq_lens[b], max_length) for rows [0, batch), and every quantised block of such a row from
 * the one holding its new length up to the high-water mark is re-opened: its dequantised
 * contents (the values barq_kv_gather_cold returns) are written into a page from the free stack,
 * which the block maps from then on, and the cold page loses the block's reference.  barq_kv_compress
 * quantises such a block again once it leaves the window.  A block finding no free page stays
 * quantised and sets BARQ_KV_ERRBIT_POOL_EXHAUSTED.  Pages are taken in no fixed order.  Needs
 * a pool whose hot pages are not shared (as barq_kv_select_rows_cold_layers leaves them).
 */
int barq_kv_crop_cold(const barq_kv_pool* pool, const barq_kv_cold* cold, int64_t batch, int64_t max_length,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BARQ_KV_H */
