// pkv_abi.hip -- extern "C" entry points of libpkv (declared in include/pkv.h).
//
// Validation mirrors the reference's error behaviour: shape / mapping errors
// are PKV_INVALID_ARGUMENT (ValueError), envelopes the kernels do not cover are
// PKV_UNSUPPORTED (ModelCapabilityUnsupported), a short workspace is
// PKV_OUT_OF_MEMORY.  Nothing here allocates device memory or synchronises.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <string>

#include "pkv.h"

#include "pkv_launch.h"

namespace {

thread_local std::string g_error = "ok";

int fail(int code, const std::string &message) {
  g_error = message;
  return code;
}

int check_launch(hipError_t e, const char *what) {
  if (e != hipSuccess) return fail(PKV_LAUNCH_FAILED, std::string(what) + ": " + hipGetErrorString(e));
  return PKV_OK;
}

int geometry(const pkv_layout *layout, pkv_geometry *g) {
  if (!layout) return fail(PKV_INVALID_ARGUMENT, "layout is NULL");
  if (layout->bits != 4 && layout->bits != 8 && layout->bits != 16)
    return fail(PKV_UNSUPPORTED, "paged quantization supports 4 or 8 bits (or 16 for float pages)");
  if (layout->head_dim < 1 || layout->head_dim > 256)
    return fail(PKV_UNSUPPORTED, "paged attention supports head dimensions 1..256");
  if (pkv_make_geometry(layout->num_kv_heads, layout->head_dim, layout->page_tokens, layout->bits,
                        layout->group_size, layout->float_kind, g) != 0)
    return fail(PKV_UNSUPPORTED, "unsupported page layout (page_tokens 16/32/64/128, group 32/64/128, "
                                 "float_kind 0/1, num_kv_heads >= 1)");
  return PKV_OK;
}

constexpr int kDefaultSplit = 256;

}  // namespace

extern "C" {

int pkv_version(void) { return 1; }

const char *pkv_last_error(void) { return g_error.c_str(); }

int64_t pkv_page_bytes(const pkv_layout *layout) {
  pkv_geometry g;
  if (geometry(layout, &g) != PKV_OK) return -1;
  return g.page_bytes;
}

int32_t pkv_stored_dim(const pkv_layout *layout) {
  pkv_geometry g;
  if (geometry(layout, &g) != PKV_OK) return -1;
  return g.dp;
}

int pkv_append_quantize(void *stream, const pkv_layout *layout, void *pool, int64_t num_pages,
                        const void *keys, const void *values, int32_t batch, int32_t tokens,
                        const int32_t *block_table, int32_t max_pages, const int32_t *start_pos,
                        const int32_t *widths, int32_t *new_lens) {
  pkv_geometry geo;
  if (int rc = geometry(layout, &geo)) return rc;
  if (batch < 0 || tokens < 0) return fail(PKV_INVALID_ARGUMENT, "negative batch or token count");
  if (batch == 0 || tokens == 0) return PKV_OK;
  if (!pool || !keys || !values || !block_table || !start_pos)
    return fail(PKV_INVALID_ARGUMENT, "paged append requires pool, keys, values, block table, start_pos");
  if (num_pages < 1 || max_pages < 1) return fail(PKV_INVALID_ARGUMENT, "empty page pool or block table");
  if (new_lens && (const void *)new_lens == (const void *)start_pos)
    return fail(PKV_INVALID_ARGUMENT, "new_lens must not alias start_pos");
  pkv::AppendArgs a;
  a.g = pkv::to_geo(geo);
  a.pool = (uint8_t *)pool;
  a.num_pages = num_pages;
  a.keys = (const uint16_t *)keys;
  a.values = (const uint16_t *)values;
  a.batch = batch;
  a.tokens = tokens;
  a.max_pages = max_pages;
  a.table = block_table;
  a.start_pos = start_pos;
  a.widths = widths;
  a.new_lens = new_lens;
  return check_launch(pkv::launch_append((hipStream_t)stream, a), "append launch");
}

int64_t pkv_attention_workspace_bytes(const pkv_layout *layout, int32_t num_heads,
                                      int32_t num_queries, int32_t max_units) {
  pkv_geometry g;
  if (geometry(layout, &g) != PKV_OK || num_heads < 1 || num_queries < 1 || max_units < 0) return -1;
  const int64_t rows = (int64_t)num_queries * (num_heads / g.hk);
  const int64_t units = (int64_t)max_units * g.hk;
  const int64_t acc = units * rows * g.dp * 4;
  const int64_t ml = units * rows * 2 * 4;
  return (acc + 255) / 256 * 256 + ml;
}

int pkv_paged_attention(void *stream, const pkv_layout *layout, const void *pool, int64_t num_pages,
                        const void *queries, int32_t batch, int32_t num_heads, int32_t num_queries,
                        const int32_t *block_table, int32_t max_pages, const int32_t *seq_lens,
                        const int32_t *q_pos, const int32_t *widths, float scale,
                        int32_t split_tokens, int32_t max_units, void *workspace,
                        int64_t workspace_bytes, void *out) {
  pkv_geometry geo;
  if (int rc = geometry(layout, &geo)) return rc;
  if (batch < 0) return fail(PKV_INVALID_ARGUMENT, "negative batch");
  if (batch == 0) return PKV_OK;
  if (num_heads < 1 || num_queries < 1 || num_heads % geo.hk)
    return fail(PKV_UNSUPPORTED, "paged attention requires query heads to form valid GQA groups");
  const int gqa = num_heads / geo.hk;
  const int rows = num_queries * gqa;
  if (rows > 32)
    return fail(PKV_UNSUPPORTED, "paged attention supports at most 32 query rows per KV head "
                                 "(queries x heads per KV head)");
  if (!pool || !queries || !block_table || !seq_lens || !out)
    return fail(PKV_INVALID_ARGUMENT, "paged attention requires pool, queries, block table, lengths, out");
  if (num_pages < 1 || max_pages < 1) return fail(PKV_INVALID_ARGUMENT, "empty page pool or block table");
  if (!std::isfinite(scale)) return fail(PKV_INVALID_ARGUMENT, "softmax scale must be finite");
  int split = split_tokens > 0 ? split_tokens : (kDefaultSplit + geo.page - 1) / geo.page * geo.page;
  if (split % geo.page || split / geo.page > 64)
    return fail(PKV_INVALID_ARGUMENT, "split_tokens must be a multiple of page_tokens and at most 64 pages");
  if (max_units < batch) return fail(PKV_INVALID_ARGUMENT, "max_units is below the number of sequences");
  const int64_t need = pkv_attention_workspace_bytes(layout, num_heads, num_queries, max_units);
  if (max_units > batch && (!workspace || workspace_bytes < need))
    return fail(PKV_OUT_OF_MEMORY, "attention workspace too small: need " + std::to_string(need) + " bytes");
  if ((int64_t)max_units * geo.hk > INT32_MAX)
    return fail(PKV_INVALID_ARGUMENT, "too many partitions");

  const int64_t units = (int64_t)max_units * geo.hk;
  float *part_acc = (float *)workspace;
  float *part_ml = workspace ? (float *)((char *)workspace + (units * rows * geo.dp * 4 + 255) / 256 * 256)
                             : nullptr;
  pkv::AttnArgs a;
  a.g = pkv::to_geo(geo);
  a.pool = (const uint8_t *)pool;
  a.num_pages = num_pages;
  a.q = (const uint16_t *)queries;
  a.batch = batch;
  a.heads = num_heads;
  a.nq = num_queries;
  a.gqa = gqa;
  a.rows = rows;
  a.table = block_table;
  a.max_pages = max_pages;
  a.seq_lens = seq_lens;
  a.q_pos = q_pos;
  a.widths = widths;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.split = split;
  a.max_units = (int)units;
  a.part_acc = part_acc;
  a.part_ml = part_ml;
  a.out = (uint16_t *)out;
  const int row_blocks = rows <= 16 ? 1 : 2;
  if (int rc = check_launch(pkv::launch_attention((hipStream_t)stream, a, row_blocks), "attention launch"))
    return rc;
  if (max_units == batch) return PKV_OK;  // one partition per sequence: no merge
  pkv::MergeArgs m;
  m.batch = batch;
  m.hk = geo.hk;
  m.heads = num_heads;
  m.nq = num_queries;
  m.gqa = gqa;
  m.rows = rows;
  m.dim = geo.dim;
  m.dp = geo.dp;
  m.split = split;
  m.float_kind = geo.float_kind;
  m.max_units = max_units;
  m.seq_lens = seq_lens;
  m.part_acc = part_acc;
  m.part_ml = part_ml;
  m.out = (uint16_t *)out;
  return check_launch(pkv::launch_merge((hipStream_t)stream, m), "merge launch");
}

int pkv_gather_pages(void *stream, const pkv_layout *layout, const void *pool, int64_t num_pages,
                     const int32_t *page_ids, int32_t count, void *k_codes, void *k_scale,
                     void *k_bias, void *v_codes, void *v_scale, void *v_bias) {
  pkv_geometry geo;
  if (int rc = geometry(layout, &geo)) return rc;
  if (count < 0) return fail(PKV_INVALID_ARGUMENT, "negative page count");
  if (count == 0) return PKV_OK;
  const bool quant = geo.bits != 16;
  if (!pool || !page_ids || !k_codes || !v_codes ||
      (quant && (!k_scale || !k_bias || !v_scale || !v_bias)))
    return fail(PKV_INVALID_ARGUMENT, "gather requires pool, ids and every output tensor");
  pkv::GatherArgs a;
  a.g = pkv::to_geo(geo);
  a.pool = (const uint8_t *)pool;
  a.num_pages = num_pages;
  a.ids = page_ids;
  a.count = count;
  a.kc = (uint8_t *)k_codes;
  a.vc = (uint8_t *)v_codes;
  a.ks = (uint16_t *)k_scale;
  a.kb = (uint16_t *)k_bias;
  a.vs = (uint16_t *)v_scale;
  a.vb = (uint16_t *)v_bias;
  const int dpr = quant ? (geo.dim + geo.group - 1) / geo.group * geo.group : geo.dim;
  a.dq = quant ? dpr * geo.bits / 8 : 0;
  a.ngr = quant ? dpr / geo.group : 0;
  return check_launch(pkv::launch_gather((hipStream_t)stream, a), "gather launch");
}

int pkv_copy_pages(void *stream, const pkv_layout *layout, void *pool, int64_t num_pages,
                   const int32_t *src_ids, const int32_t *dst_ids, int32_t count) {
  pkv_geometry geo;
  if (int rc = geometry(layout, &geo)) return rc;
  if (count < 0) return fail(PKV_INVALID_ARGUMENT, "negative page count");
  if (count == 0) return PKV_OK;
  if (!pool || !src_ids || !dst_ids) return fail(PKV_INVALID_ARGUMENT, "copy requires pool and ids");
  return check_launch(pkv::launch_copy((hipStream_t)stream, (uint8_t *)pool, num_pages, geo.page_bytes,
                                       src_ids, dst_ids, count),
                      "copy launch");
}

int pkv_quantize_rows(void *stream, const void *values, int64_t rows, int32_t dim, int32_t bits,
                      int32_t group_size, int32_t float_kind, void *codes, void *scale, void *bias) {
  if (bits != 4 && bits != 8) return fail(PKV_UNSUPPORTED, "paged quantization supports 4 or 8 bits");
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(PKV_UNSUPPORTED, "quantization group size must be 32, 64 or 128");
  if (float_kind != 0 && float_kind != 1) return fail(PKV_INVALID_ARGUMENT, "float_kind must be 0 or 1");
  if (rows < 0 || dim < 1) return fail(PKV_INVALID_ARGUMENT, "invalid row count or dimension");
  if (rows == 0) return PKV_OK;
  if (!values || !codes || !scale || !bias) return fail(PKV_INVALID_ARGUMENT, "NULL tensor");
  pkv::QuantRowsArgs a;
  a.values = (const uint16_t *)values;
  a.rows = rows;
  a.dim = dim;
  a.bits = bits;
  a.group = group_size;
  a.float_kind = float_kind;
  a.codes = (uint8_t *)codes;
  a.scale = (uint16_t *)scale;
  a.bias = (uint16_t *)bias;
  return check_launch(pkv::launch_quantize_rows((hipStream_t)stream, a), "quantize launch");
}

int pkv_dequantize_rows(void *stream, const void *codes, const void *scale, const void *bias,
                        int64_t rows, int32_t dim, int32_t bits, int32_t group_size, void *out) {
  if (bits != 4 && bits != 8) return fail(PKV_UNSUPPORTED, "paged quantization supports 4 or 8 bits");
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(PKV_UNSUPPORTED, "quantization group size must be 32, 64 or 128");
  if (rows < 0 || dim < 1) return fail(PKV_INVALID_ARGUMENT, "invalid row count or dimension");
  if (rows == 0) return PKV_OK;
  if (!codes || !scale || !bias || !out) return fail(PKV_INVALID_ARGUMENT, "NULL tensor");
  pkv::DequantRowsArgs a;
  a.codes = (const uint8_t *)codes;
  a.scale = (const uint16_t *)scale;
  a.bias = (const uint16_t *)bias;
  a.rows = rows;
  a.dim = dim;
  a.bits = bits;
  a.group = group_size;
  a.out = (float *)out;
  return check_launch(pkv::launch_dequantize_rows((hipStream_t)stream, a), "dequantize launch");
}

}  // extern "C"
