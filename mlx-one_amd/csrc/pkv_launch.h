// pkv_launch.h -- kernel argument structs and host launchers of libpkv.
#pragma once
#include "pkv_device.h"

namespace pkv {

struct AppendArgs {
  Geo g;
  uint8_t *pool;
  int64_t num_pages;
  const uint16_t *keys, *values;  // [B][HK][T][D]
  int batch, tokens, max_pages;
  const int32_t *table, *start_pos, *widths;
  const int32_t *lens_after;  // start_pos NULL: start = lens_after[b] - tokens
  int32_t *new_lens;
};

struct GatherArgs {
  Geo g;
  const uint8_t *pool;
  int64_t num_pages;
  const int32_t *ids;
  int count;
  uint8_t *kc, *vc;        // codes, or float K/V (2 bytes per element)
  uint16_t *ks, *kb, *vs, *vb;
  int dq;                  // reference code bytes per row (quantized)
  int ngr;                 // reference groups per row
};

// Partial slots of the attention workspace per work wave: the first and the
// last piece of its run.
constexpr int kSlotsPerWave = 2;

struct AttnArgs {
  Geo g;
  const uint8_t *pool;
  int64_t num_pages;
  const uint16_t *q;  // [B][H][nq_stride][D]
  int batch, heads, nq, gqa, rows;
  // Q extent of queries, q_pos and out (= nq except for the decode part of a
  // mixed batch, which covers the first nq of nq_stride query rows)
  int nq_stride;
  // Mixed batches (narrow_q 0: off).  Decode kernel: serve only sequences
  // whose width w has narrow_lo < w <= narrow_q.  Prefill kernel: leave
  // sequences of width at most narrow_q to the decode kernel (their rows are
  // written as zeros first).
  int narrow_lo, narrow_q;
  const int32_t *table;
  int max_pages;
  const int32_t *seq_lens, *q_pos, *widths;
  float scale_log2;  // softmax scale * log2(e)
  int waves;         // work waves (grid size)
  int lead;          // tiles of start-up cost charged ahead of each segment in the split
  float *part_acc;   // [2*waves][rows][DP]
  float *part_ml;    // [2*waves][rows][2]
  uint16_t *out;     // [B][H][Q][D]
  // Fused single-token append (new_k non-NULL): each sequence's new K/V row
  // [B][HK][D] is quantized into slot seq_lens[b] - 1 of its pages (wpool is
  // the pool, writable) by the wave that attends the sequence's last tile.
  uint8_t *wpool = nullptr;
  const uint16_t *new_k = nullptr, *new_v = nullptr;
};

struct MergeArgs {
  int batch, hk, heads, nq, gqa, rows, dim, dp, float_kind;
  int waves, lead;  // as launched for the attention kernel
  int nq_stride, narrow_lo, narrow_q;
  const int32_t *seq_lens, *widths;
  const float *part_acc, *part_ml;
  uint16_t *out;
};

struct QuantRowsArgs {
  const uint16_t *values;  // [rows][dim], float_kind
  int64_t rows;
  int dim, bits, group, float_kind;
  uint8_t *codes;          // [rows][ceil(dim/group)*group * bits/8]
  uint16_t *scale, *bias;  // [rows][ceil(dim/group)] f16 bits
};

struct DequantRowsArgs {
  const uint8_t *codes;
  const uint16_t *scale, *bias;
  int64_t rows;
  int dim, bits, group;
  float *out;              // [rows][dim]
};

// Rotate-half RoPE of a fused projection [rows][heads + 2*kv_heads][dim]
// (rows = B*T) into head-major q [B][heads][T][dim], k and v [B][kv_heads][T][dim].
struct RopeArgs {
  const uint16_t *qkv;
  int64_t rows;
  int tokens, heads, kv_heads, dim, float_kind;
  const int32_t *positions;  // [rows]
  const float *inv_freq;     // [dim/2]
  uint16_t *q, *k, *v;
};

hipError_t launch_rope(hipStream_t stream, const RopeArgs &a);

// Device page allocator (pkv_arena.hip).  State words: [0] free pages,
// [1] error bits, header padded to kArenaHeaderWords, then the free stack
// [capacity] and the reference counts [capacity].
constexpr int kArenaHeaderWords = 16;
constexpr int kMaxArenaPools = 128;
constexpr int kArenaOutOfPages = 1, kArenaTableFull = 2, kArenaBadArgument = 4, kArenaCorrupt = 8;

enum class ArenaOp { Reserve, Release, Fork };

struct ArenaArgs {
  int32_t *state;
  int capacity, page_tokens;
  int32_t *table;   // [num_slots][max_pages]
  int max_pages, num_slots;
  int32_t *lens;    // [num_slots]
  const int32_t *slots, *arg;  // per item: slot, and width / kept tokens / fork destination
  int count;
  uint8_t *pools[kMaxArenaPools];  // reserve: copy-on-write in every layer's pool
  int num_pools;
  int64_t page_bytes;
  int32_t *batch_table, *batch_starts, *batch_lens;  // reserve outputs
};

hipError_t launch_arena_init(hipStream_t stream, int32_t *state, int capacity);
hipError_t launch_arena(hipStream_t stream, ArenaOp op, const ArenaArgs &a);
hipError_t launch_quantize_rows(hipStream_t stream, const QuantRowsArgs &a);
hipError_t launch_dequantize_rows(hipStream_t stream, const DequantRowsArgs &a);
hipError_t launch_append(hipStream_t stream, const AppendArgs &a);
hipError_t launch_gather(hipStream_t stream, const GatherArgs &a);
// Streaming read of the listed pages (all heads) by `waves` one-wave
// workgroups; out: waves * 64 words.
hipError_t launch_read_probe(hipStream_t stream, const uint8_t *pool, int64_t num_pages, int64_t page_bytes,
                             const int32_t *ids, int64_t count, int waves, uint32_t *out);
hipError_t launch_copy(hipStream_t stream, uint8_t *pool, int64_t num_pages, int64_t page_bytes,
                       const int32_t *src, const int32_t *dst, int count);
hipError_t launch_attention(hipStream_t stream, const AttnArgs &a);
hipError_t launch_merge(hipStream_t stream, const MergeArgs &a);
// Query blocks wider than the decode kernel serves (chunked prefill).
hipError_t launch_prefill(hipStream_t stream, const AttnArgs &a);
// Resident waves of the attention kernel for this layout and row count on the
// current device (CUs x workgroups per CU); <0 on error.
int attention_waves(const Geo &g, int rows);
// Waves per run of the split for `rows` query rows per KV head (`append`: the
// fused single-token form): a launch of W waves has
// max(1, W / attention_group(rows, append)) runs, each with its partials.
int attention_group(const Geo &g, int rows, bool append);
// Lead tiles the decode split charges per segment for `rows` query rows per KV
// head (more for a launch that fuses the single-token append).
int attention_lead(const Geo &g, int rows, bool append);
// Whether the split-K decode kernel serves this many rows per KV head (else
// launch_prefill does, with no workspace and no merge).
bool decode_serves(const Geo &g, int rows);
// Whether the decode kernel fuses the single-token append for this layout and
// row count (quantized pages, at most 8 rows per KV head).
bool append_fusable(const Geo &g, int rows);
// Decode kernel for <= 4 rows per KV head over quantized pages (head_dim <=
// 128): process-wide; select returns the previous choice.
constexpr int kDecodeMfma = 0, kDecodeValu = 1;
int select_decode_kernel(int kind);
int decode_kernel();

}  // namespace pkv
