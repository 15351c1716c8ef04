/*
 * pkv.h -- C ABI of libpkv, the MI355X (gfx950) paged-KV decode path.
 *
 * The reference (SSusantAchary/mlx-one) has no FFI on this path: its hot path
 * is Python calling MLX ops and one generated Metal kernel.  Each entry point
 * below replaces the reference code named in its comment; the Python host
 * package (mlx-one_amd/pkv) binds them with ctypes behind the reference's own
 * class and function names.
 *
 * Conventions
 *  - All pointers except `layout` are device pointers (HBM) unless noted; sizes
 *    are element counts.  No entry point allocates device memory: the caller
 *    owns every buffer, including the attention workspace (the one library-held
 *    buffer is pkv_paged_attention_noalloc's fixed scratch array, below).
 *  - `stream` is a hipStream_t passed as void* (NULL = default stream).  Work
 *    is enqueued asynchronously; entry points never synchronise.
 *  - Return value: PKV_OK or an error code; pkv_last_error() gives the text of
 *    the calling thread's last error.
 *  - Entry points are re-entrant; calls on different streams may overlap as
 *    long as they do not write the same pages or workspace.
 */
#ifndef PKV_H
#define PKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum pkv_status {
  PKV_OK = 0,
  PKV_INVALID_ARGUMENT = 1, /* shape, layout or mapping errors (reference: ValueError) */
  PKV_UNSUPPORTED = 2,      /* reference: ModelCapabilityUnsupported */
  PKV_OUT_OF_MEMORY = 3,    /* workspace too small (reference: CacheCapacityError) */
  PKV_LAUNCH_FAILED = 4     /* HIP runtime error */
};

/*
 * Page layout of one layer's pool.  Mirrors the reference's BlockLayout
 * (src/mlx_one/engine/block_cache.py:32-43): num_kv_heads, head_dim,
 * page_tokens, quantization_bits (16 = unquantized), quantization_group_size.
 * float_kind selects the float element type of unquantized pages, queries,
 * new K/V and outputs: 0 = bfloat16, 1 = float16 (key_dtype/value_dtype).
 */
typedef struct pkv_layout {
  int32_t num_kv_heads;
  int32_t head_dim;     /* 1..256 */
  int32_t page_tokens;  /* 16, 32, 64 or 128 */
  int32_t bits;         /* 4, 8 (affine quantized) or 16 (float pages) */
  int32_t group_size;   /* 32, 64 or 128 for quantized pages */
  int32_t float_kind;   /* 0 = bf16, 1 = f16 */
} pkv_layout;

/* Library version (increments when the page format or an ABI changes). */
int pkv_version(void);

/* Thread-local text of the last error; never NULL. */
const char *pkv_last_error(void);

/* Bytes of one page (all KV heads) in the pool; <0 when the layout is invalid.
 * Replaces the per-segment tensor shapes of SegmentedPageArena
 * (src/mlx_one/engine/arena.py:58-75). */
int64_t pkv_page_bytes(const pkv_layout *layout);

/* Head dimension as stored (padded to 64, 128 or 256); <0 when invalid. */
int32_t pkv_stored_dim(const pkv_layout *layout);

/*
 * Append `tokens` new K/V tokens per sequence into their pages, quantizing each
 * (head, token) group-wise as it is written (affine unsigned, f16 scale and
 * bias, the reference's quantize_page arithmetic).
 * Replaces PagedKVCache.append + quantize_page
 * (src/mlx_one/engine/paged.py:103-154 and :24-41) and the arena staging it
 * triggers (src/mlx_one/engine/arena.py:90-113).
 *
 *  keys, values : [batch][num_kv_heads][tokens][head_dim], float_kind elements
 *  block_table  : [batch][max_pages] int32 page ids (pages must already be
 *                 assigned for every position written)
 *  start_pos    : [batch] int32 length of each sequence before the append
 *  widths       : [batch] int32 tokens to append per sequence (<= tokens), or
 *                 NULL for `tokens` everywhere
 *  new_lens     : [batch] int32 output start_pos + width, or NULL
 */
int pkv_append_quantize(void *stream, const pkv_layout *layout, void *pool, int64_t num_pages,
                        const void *keys, const void *values, int32_t batch, int32_t tokens,
                        const int32_t *block_table, int32_t max_pages,
                        const int32_t *start_pos, const int32_t *widths, int32_t *new_lens);

/*
 * Causal GQA paged attention for decode (num_queries = 1), speculative
 * verify (num_queries = 1 + drafts) and chunked prefill (wide query blocks),
 * dequantization fused into the page load.  Replaces paged_attention and its
 * Metal kernel (src/mlx_one/engine/paged_attention.py:62-124 kernel, :127-206
 * dispatch and partition merge).  Up to 32 query rows per KV head
 * (num_queries x num_heads / num_kv_heads; 16 at head_dim > 128): the
 * reference splits each sequence into fixed token partitions; here the
 * 16-token tiles of all (sequence, KV head) pairs are shared out as equal runs
 * over `waves` waves (for 5-8 and 17-32 rows per KV head, one run per four
 * waves, which share its tiles and combine in LDS), and a pair whose tiles
 * span several runs is merged by log-sum-exp (:191-204) in a second kernel on
 * the same stream.  Wider query
 * blocks (up to 2^24 rows per KV head) run on an MFMA prefill kernel, 256
 * rows per workgroup (128 at head_dim > 128), that needs no workspace.
 * Mixed batches (the reference pads decode and prefill rows into one call,
 * engine/paged.py:345-346, :384-389): in a wide call with `widths`, the
 * sequences whose width fits the decode kernel (at most 32 / (H/HK) queries,
 * 16 / (H/HK) at head_dim > 128) are served by the split-K decode kernel and
 * the others by the prefill kernel, in the same call; `waves` and the
 * workspace then size that decode part (pkv_attention_workspace_bytes gives
 * its size for the wide call's arguments).  Without room for its partials the
 * prefill kernel serves every sequence.
 *
 *  queries      : [batch][num_heads][num_queries][head_dim], float_kind
 *  seq_lens     : [batch] tokens in each sequence's cache (after the append)
 *  q_pos        : [batch][num_queries] logical query positions, or NULL for
 *                 seq_lens[b] - widths[b] + q; token t is visible to query q
 *                 when t <= q_pos (paged_attention.py:81)
 *  widths       : [batch] real query rows (rows q >= widths[b] output 0), or NULL
 *  scale        : softmax scale
 *  waves        : work waves; <= 0 picks pkv_attention_default_waves(...)
 *  workspace    : device scratch of pkv_attention_workspace_bytes(...) bytes
 *                 (calls sharing one workspace must not overlap)
 *  out          : [batch][num_heads][num_queries][head_dim], float_kind
 */
int pkv_paged_attention(void *stream, const pkv_layout *layout, const void *pool,
                        int64_t num_pages, const void *queries, int32_t batch,
                        int32_t num_heads, int32_t num_queries, const int32_t *block_table,
                        int32_t max_pages, const int32_t *seq_lens, const int32_t *q_pos,
                        const int32_t *widths, float scale, int32_t waves, void *workspace,
                        int64_t workspace_bytes, void *out);

/*
 * One single-token step: append the new K/V token of every sequence (as
 * pkv_append_quantize with tokens = 1 at position seq_lens[b] - 1) and
 * attend its one query (as pkv_paged_attention with num_queries = 1, q_pos
 * NULL, widths NULL), in one launch where the decode kernel serves the shape
 * (quantized pages, at most 8 query rows per KV head): the wave that attends
 * a sequence's last tile quantizes the new token, stores it and uses it.
 * Other shapes run the append and the attention as two launches.  Replaces
 * the append-then-attend pair of PagedBatchCache.attend (engine/paged.py:
 * 260-263) for a decode step; pages and output equal the two separate calls'
 * bit for bit.
 *
 *  pool         : writable (the new tokens land in it)
 *  keys, values : [batch][HK][1][head_dim], float_kind
 *  seq_lens     : [batch] tokens in each sequence after the append (>= 1)
 *  other arguments as pkv_paged_attention (queries [batch][num_heads][1][head_dim])
 */
int pkv_append_paged_attention(void *stream, const pkv_layout *layout, void *pool,
                               int64_t num_pages, const void *keys, const void *values,
                               const void *queries, int32_t batch, int32_t num_heads,
                               const int32_t *block_table, int32_t max_pages,
                               const int32_t *seq_lens, float scale, int32_t waves,
                               void *workspace, int64_t workspace_bytes, void *out);

/*
 * pkv_paged_attention without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference (its
 * Metal path allocates per partition).  The split-K partials live in a fixed
 * 32 MiB device array of the library, one per GPU, held until the process
 * ends; this entry point allocates nothing.  Every call on one GPU shares that
 * GPU's array, so calls that overlap on one GPU (other streams, concurrent
 * graph replays) race: order them.  No part of the array needs clearing --
 * each launch writes every partial it reads.  waves <= 0 picks
 * pkv_attention_default_waves, lowered to what the array holds partials for;
 * an explicit `waves` whose partials exceed it is refused with
 * PKV_OUT_OF_MEMORY.  The first call on a device looks up the array's device
 * address (hipGetSymbolAddress); make it outside graph capture.  Query blocks
 * served by the prefill kernel need no scratch.  Arguments and results are
 * pkv_paged_attention's.
 */
int pkv_paged_attention_noalloc(void *stream, const pkv_layout *layout, const void *pool,
                                int64_t num_pages, const void *queries, int32_t batch,
                                int32_t num_heads, int32_t num_queries, const int32_t *block_table,
                                int32_t max_pages, const int32_t *seq_lens, const int32_t *q_pos,
                                const int32_t *widths, float scale, int32_t waves, void *out);

/*
 * Which kernel serves decode rows -- at most 4 query rows per KV head
 * (single-token decode at GQA <= 4) over quantized pages at head_dim <= 128:
 * PKV_DECODE_MFMA (the default: score and value products on the matrix
 * cores, queries in column slots) or PKV_DECODE_VALU (the same work split,
 * partials and merge, with v_dot2_f32_f16 products on the vector ALU).
 * Both compute the reference's result; they differ only in f32 summation
 * order.  No counterpart in the reference (its Metal kernel has one form):
 * kept so that the choice can be measured on the device.  Process-wide (read
 * when a call launches); returns the previous choice, or
 * PKV_INVALID_ARGUMENT.  Other shapes always run the MFMA kernels.
 */
#define PKV_DECODE_MFMA 0
#define PKV_DECODE_VALU 1
int pkv_select_decode_kernel(int kind);

/*
 * Measurement aid, no counterpart in the reference: a plain streaming read of
 * whole pages (every KV head), page_ids[0..count) in order, split into equal
 * runs over `waves` one-wave workgroups, each lane folding its loads into one
 * word of out [waves * 64] uint32.  Given the pages a decode step's sequences
 * hold, in block-table order, and the decode launch's wave count, its duration
 * is what HBM takes to deliver those bytes to a kernel that does nothing else:
 * the practical ceiling the decode launch is compared against.  Ids outside
 * [0, num_pages) are skipped.
 */
int pkv_read_probe(void *stream, const pkv_layout *layout, const void *pool, int64_t num_pages,
                   const int32_t *page_ids, int64_t count, int32_t waves, void *out);

/* Waves the attention kernel keeps resident on the current device for this
 * layout and (num_heads, num_queries) (1 for query blocks served by the
 * prefill kernel).  <0 on error. */
int32_t pkv_attention_waves(const pkv_layout *layout, int32_t num_heads, int32_t num_queries);

/* The `waves` pkv_paged_attention uses when given waves <= 0: the resident
 * waves, or half of them (one per SIMD) for decode rows (<= 4 query rows per
 * KV head) on the MFMA decode kernel when the batch has at most a quarter as
 * many (sequence, KV head) segments as resident waves.  <0 on error. */
int32_t pkv_attention_default_waves(const pkv_layout *layout, int32_t num_heads, int32_t num_queries,
                                    int32_t batch);

/* Workspace bytes pkv_paged_attention needs for `waves` work waves.  For
 * query blocks served by the prefill kernel: the partials of a mixed batch's
 * decode part (0 when the GQA ratio leaves the decode kernel no query). */
int64_t pkv_attention_workspace_bytes(const pkv_layout *layout, int32_t num_heads,
                                      int32_t num_queries, int32_t waves);

/*
 * Copy pages out of the pool into the reference's per-page tensor format
 * (paged_attention.py:31-35): quantized pages give K codes [count][HK][P][Dq]
 * u8 (Dq = Dp for 8 bit, Dp/2 for 4 bit, Dp = ceil(D/G)*G), K scale and K bias
 * [count][HK][P][Dp/G] f16, then the same for V; float pages give K and V
 * [count][HK][P][D] (the three V-side / scale pointers are then unused and may
 * be NULL).  Bit-exact copies: the block-table gather behind the reference's
 * page views (arena.py:101-106) and dequantize_page's input (paged.py:44-54).
 */
int pkv_gather_pages(void *stream, const pkv_layout *layout, const void *pool, int64_t num_pages,
                     const int32_t *page_ids, int32_t count, void *k_codes, void *k_scale,
                     void *k_bias, void *v_codes, void *v_scale, void *v_bias);

/*
 * Copy whole pages src_ids[i] -> dst_ids[i] inside the pool (copy-on-write of a
 * shared mutable tail page).  Replaces the tail copy in PagedKVCache.clone
 * (src/mlx_one/engine/paged.py:83-91).
 */
int pkv_copy_pages(void *stream, const pkv_layout *layout, void *pool, int64_t num_pages,
                   const int32_t *src_ids, const int32_t *dst_ids, int32_t count);

/*
 * Quantize `rows` rows of `dim` float_kind values into the reference's page
 * tensors: codes [rows][Dq] u8, scale and bias [rows][Dp/G] f16 bits
 * (Dp = ceil(dim/G)*G, Dq = Dp or Dp/2 for 4 bit; 4-bit packs
 * code[2i] | code[2i+1] << 4).  Replaces quantize_page
 * (src/mlx_one/engine/paged.py:24-41) with group_size as a parameter
 * (the reference hard-codes 32).
 */
int pkv_quantize_rows(void *stream, const void *values, int64_t rows, int32_t dim, int32_t bits,
                      int32_t group_size, int32_t float_kind, void *codes, void *scale, void *bias);

/*
 * x = f32(code) * f32(scale) + f32(bias), float32 out [rows][dim].  Replaces
 * dequantize_page (src/mlx_one/engine/paged.py:44-54).
 */
int pkv_dequantize_rows(void *stream, const void *codes, const void *scale, const void *bias,
                        int64_t rows, int32_t dim, int32_t bits, int32_t group_size, void *out);

/*
 * Caller side of the attend: rotate-half RoPE of a fused projection
 * qkv [batch][tokens][heads + 2*kv_heads][dim] (float_kind values) at
 * positions [batch][tokens] with inv_freq [dim/2] (float32), written
 * head-major: q [batch][heads][tokens][dim] rotated, k [batch][kv_heads][tokens][dim]
 * rotated, v [batch][kv_heads][tokens][dim] copied.  Per element:
 * angle = f32(pos) * inv_freq[i], out = (a*cos - b*sin, b*cos + a*sin) with
 * each product and sum rounded in float32, then one RNE cast.  Replaces the
 * projection split and apply_rotary_pos_emb of the reference's attention block
 * (src/mlx_one/models/shared/transformer.py:32-90, :146-184), which feeds
 * PagedBatchCache.attend.  dim even, at most 256.
 */
int pkv_rope_qkv(void *stream, const void *qkv, int32_t batch, int32_t tokens, int32_t heads,
                 int32_t kv_heads, int32_t dim, int32_t float_kind, const int32_t *positions,
                 const float *inv_freq, void *q, void *k, void *v);

/*
 * Device-side page allocation.  Page ownership -- the free pages, a reference
 * count per page, each sequence slot's page table and length -- lives in
 * device memory, so a decode step needs no host bookkeeping and can be
 * replayed as a graph.  Replaces the host BlockPool / SegmentedPageArena /
 * PersistentPageTable bookkeeping and the clone tail copy
 * (src/mlx_one/engine/block_cache.py:121-326, engine/arena.py:27-225,
 * engine/paged.py:83-91); the reference has no device-side counterpart.
 *
 * state: pkv_arena_state_bytes(capacity) bytes, set up by pkv_arena_init:
 *   int32 [0] free pages, [1] sticky error bits (PKV_ARENA_*), [16, 16+C) free
 *   stack, [16+C, 16+2C) reference counts (C = capacity_pages).
 * slot_table [num_slots][max_pages] int32 page ids (-1 = none; initialise to
 * -1), slot_lens [num_slots] int32 tokens (initialise to 0).  One page id
 * addresses the same page in every layer's pool.  The kernels run as one
 * workgroup each; calls on one state must be ordered on one stream, and the
 * slots of one call must be distinct.  Errors are reported in state[1]: a call
 * that hits one leaves the affected slots unchanged.
 */
#define PKV_ARENA_OUT_OF_PAGES 1
#define PKV_ARENA_TABLE_FULL 2
#define PKV_ARENA_BAD_ARGUMENT 4
#define PKV_ARENA_CORRUPT 8

int64_t pkv_arena_state_bytes(int32_t capacity_pages);
int pkv_arena_init(void *stream, void *state, int32_t capacity_pages);

/*
 * Grow slots[i] by widths[i] tokens: pages for the new tokens come off the free
 * stack (reference count 1); a partly filled tail page shared with another slot
 * is first copied, in each of the num_pools pools (page_bytes per page), to a
 * page of its own (copy-on-write).  Writes the batch's operands for
 * pkv_append_quantize / pkv_paged_attention: batch_table [count][max_pages]
 * (the slot's pages; entries past them are not written -- those kernels read
 * a row only up to its length), batch_starts [count] (length before),
 * batch_lens [count] (length after).  If the free pages do not cover the call,
 * no slot grows, PKV_ARENA_OUT_OF_PAGES is set, and each growing slot's batch
 * length is 0 and its batch row holds -1 from the page its first new token
 * would go to: an append positioned by batch_starts or by batch_lens (the
 * single-token pkv_append_paged_attention) then writes nothing, and no cached
 * token is overwritten.  A slot whose table is full is blocked the same way.
 */
int pkv_arena_reserve(void *stream, void *state, int32_t capacity_pages, int32_t page_tokens,
                      int32_t *slot_table, int32_t num_slots, int32_t max_pages, int32_t *slot_lens,
                      const int32_t *slots, const int32_t *widths, int32_t count,
                      void *const *pools, int32_t num_pools, int64_t page_bytes,
                      int32_t *batch_table, int32_t *batch_starts, int32_t *batch_lens);

/*
 * Cut slots[i] back to keep_tokens[i] tokens (0 releases the slot): pages past
 * the kept ones lose a reference and go back on the free stack at zero.  The
 * transaction rollback of PagedKVCache (by length) and its release/trim
 * (engine/paged.py:185-213).
 */
int pkv_arena_truncate(void *stream, void *state, int32_t capacity_pages, int32_t page_tokens,
                       int32_t *slot_table, int32_t num_slots, int32_t max_pages, int32_t *slot_lens,
                       const int32_t *slots, const int32_t *keep_tokens, int32_t count);

/*
 * dst_slots[i] (empty) becomes a copy of src_slots[i] sharing every page (one
 * more reference each): PagedKVCache.clone / prefix adoption
 * (engine/paged.py:77-101, :174-183), with the tail copied only when written.
 */
int pkv_arena_fork(void *stream, void *state, int32_t capacity_pages, int32_t page_tokens,
                   int32_t *slot_table, int32_t num_slots, int32_t max_pages, int32_t *slot_lens,
                   const int32_t *src_slots, const int32_t *dst_slots, int32_t count);

#ifdef __cplusplus
}
#endif

#endif /* PKV_H */
