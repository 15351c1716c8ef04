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

struct AttnArgs {
  Geo g;
  const uint8_t *pool;
  int64_t num_pages;
  const uint16_t *q;  // [B][H][Q][D]
  int batch, heads, nq, gqa, rows;
  const int32_t *table;
  int max_pages;
  const int32_t *seq_lens, *q_pos, *widths;
  float scale_log2;  // softmax scale * log2(e)
  int split;         // tokens per partition
  int max_units;
  float *part_acc;   // [units*HK][rows][DP]
  float *part_ml;    // [units*HK][rows][2]
  uint16_t *out;     // [B][H][Q][D]
};

struct MergeArgs {
  int batch, hk, heads, nq, gqa, rows, dim, dp, split, float_kind;
  int max_units;  // launched (sequence, partition) units
  const int32_t *seq_lens;
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

hipError_t launch_quantize_rows(hipStream_t stream, const QuantRowsArgs &a);
hipError_t launch_dequantize_rows(hipStream_t stream, const DequantRowsArgs &a);
hipError_t launch_append(hipStream_t stream, const AppendArgs &a);
hipError_t launch_gather(hipStream_t stream, const GatherArgs &a);
hipError_t launch_copy(hipStream_t stream, uint8_t *pool, int64_t num_pages, int64_t page_bytes,
                       const int32_t *src, const int32_t *dst, int count);
hipError_t launch_attention(hipStream_t stream, const AttnArgs &a, int row_blocks);
hipError_t launch_merge(hipStream_t stream, const MergeArgs &a);

}  // namespace pkv
