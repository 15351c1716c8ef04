// pkv_abi.hip -- extern "C" entry points of libpkv (declared in include/pkv.h).
//
// Validation mirrors the reference's error behaviour: shape / mapping errors
// are PKV_INVALID_ARGUMENT (ValueError), envelopes the kernels do not cover are
// PKV_UNSUPPORTED (ModelCapabilityUnsupported), a short workspace is
// PKV_OUT_OF_MEMORY.  Nothing here allocates device memory or synchronises.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <utility>

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

// Query rows per KV head (queries x heads per KV head) one call may carry.
constexpr int64_t kMaxRows = 1 << 24;

// Attention workspace: [ml: S*rows*2 f32][acc: S*rows*DP f32] with
// S = kSlotsPerWave * runs partial slots (a run per wave, or per group of
// waves for 17-32 rows), each part 256-byte aligned.
struct WorkspaceParts {
  int64_t ml, acc, total;
};

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

// The runs of a launch of `waves` waves for `rows` query rows per KV head
// (`append`: the fused single-token form).
int64_t attention_runs(const pkv_geometry &g, int64_t rows, int64_t waves, bool append) {
  return std::max<int64_t>(1, waves / pkv::attention_group(pkv::to_geo(g), (int)rows, append));
}

// Partial space of a launch; `append` unknown (the public sizing query): the
// larger of the forms the shape has.
WorkspaceParts workspace_parts(const pkv_geometry &g, int64_t rows, int64_t waves, int append = -1) {
  int64_t runs = attention_runs(g, rows, waves, append > 0);
  if (append < 0 && pkv::append_fusable(pkv::to_geo(g), (int)rows))
    runs = std::max(runs, attention_runs(g, rows, waves, true));
  const int64_t slots = (int64_t)pkv::kSlotsPerWave * runs;
  WorkspaceParts w;
  w.ml = 0;
  w.acc = align256(slots * rows * 2 * 4);
  w.total = w.acc + slots * rows * g.dp * 4;
  return w;
}

// Resident-wave capacity per (device, layout, rows), measured once.
int cached_waves(const pkv_geometry &geo, int rows) {
  static std::mutex mu;
  static std::map<std::pair<int, std::string>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  char key[128];
  snprintf(key, sizeof key, "%d/%d/%d/%d/%d/%d/%d", geo.hk, geo.dp, geo.bits, geo.group, geo.float_kind, rows,
           pkv::decode_kernel());
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find({dev, key});
  if (it != cache.end()) return it->second;
  const int w = pkv::attention_waves(pkv::to_geo(geo), rows);
  if (w > 0) cache[{dev, key}] = w;
  return w;
}

// Most queries per sequence the split-K decode kernel serves at this GQA
// ratio (its row limit is 32 query rows per KV head, 16 at head_dim > 128);
// 0 when not even one.
int decode_queries(const pkv_geometry &geo, int gqa) {
  int q = 32 / std::max(gqa, 1);
  while (q > 0 && !pkv::decode_serves(pkv::to_geo(geo), q * gqa)) --q;
  return q;
}

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
  a.lens_after = nullptr;
  a.widths = widths;
  a.new_lens = new_lens;
  return check_launch(pkv::launch_append((hipStream_t)stream, a), "append launch");
}

int pkv_select_decode_kernel(int kind) {
  if (kind != PKV_DECODE_MFMA && kind != PKV_DECODE_VALU)
    return fail(PKV_INVALID_ARGUMENT, "decode kernel must be PKV_DECODE_MFMA or PKV_DECODE_VALU");
  return pkv::select_decode_kernel(kind);
}

int32_t pkv_attention_waves(const pkv_layout *layout, int32_t num_heads, int32_t num_queries) {
  pkv_geometry g;
  if (geometry(layout, &g) != PKV_OK) return -1;
  if (num_heads < 1 || num_queries < 1 || num_heads % g.hk) return -1;
  const int64_t rows = (int64_t)num_queries * (num_heads / g.hk);
  if (rows > kMaxRows) return -1;
  if (!pkv::decode_serves(pkv::to_geo(g), (int)rows)) return 1;  // prefill kernel: no split
  const int w = cached_waves(g, (int)rows);
  if (w <= 0) {
    fail(PKV_LAUNCH_FAILED, "could not query the attention kernel's occupancy");
    return -1;
  }
  return w;
}

int32_t pkv_attention_default_waves(const pkv_layout *layout, int32_t num_heads, int32_t num_queries,
                                    int32_t batch) {
  const int32_t resident = pkv_attention_waves(layout, num_heads, num_queries);
  if (resident <= 1 || batch < 1) return resident;
  pkv_geometry g;
  geometry(layout, &g);
  const int64_t rows = (int64_t)num_queries * (num_heads / g.hk);
  // Decode rows (<= 4 per KV head: four tiles per iteration) of a batch with
  // few (sequence, KV head) segments: one wave per SIMD streams longer runs
  // with fewer pieces to merge and measures faster; with many segments, two
  // waves per SIMD keep more of them in flight.  The VALU decode kernel
  // (issue-bound: its waves cover each other's LDS permutes) keeps two.
  const bool valu = pkv::decode_kernel() == pkv::kDecodeValu && g.bits != 16 && g.dp <= 128;
  if (rows <= 4 && !valu && (int64_t)batch * g.hk * 4 <= resident) return std::max(1, resident / 2);
  return resident;
}

int64_t pkv_attention_workspace_bytes(const pkv_layout *layout, int32_t num_heads,
                                      int32_t num_queries, int32_t waves) {
  pkv_geometry g;
  if (geometry(layout, &g) != PKV_OK || num_heads < 1 || num_queries < 1 || num_heads % g.hk ||
      waves < 1)
    return -1;
  const int64_t rows = (int64_t)num_queries * (num_heads / g.hk);
  if (rows > kMaxRows) return -1;
  if (!pkv::decode_serves(pkv::to_geo(g), (int)rows)) {
    // prefill kernel: no partials, except for the decode part of a mixed batch
    // (the tiers of paged_attention_impl run in turn over one workspace)
    const int gqa = num_heads / g.hk;
    const int hi = decode_queries(g, gqa);
    const int lo = std::min(hi, 4 / std::max(gqa, 1));
    int64_t need = 0;
    if (lo >= 1) need = workspace_parts(g, (int64_t)lo * gqa, waves).total;
    if (hi > lo) need = std::max(need, workspace_parts(g, (int64_t)hi * gqa, waves).total);
    return need;
  }
  return workspace_parts(g, rows, waves).total;
}

}  // extern "C"

namespace {

// The attention entry points' common body.  `fit_waves`: when the caller
// leaves the waves to the library, use no more than the workspace holds
// partials for (the split is correct at any wave count).
// The new token of every sequence, for pkv_append_paged_attention.
struct FusedAppend {
  void *pool;
  const void *keys, *values;  // [batch][HK][1][dim]
};

int paged_attention_impl(void *stream, const pkv_layout *layout, const void *pool, int64_t num_pages,
                         const void *queries, int32_t batch, int32_t num_heads, int32_t num_queries,
                         const int32_t *block_table, int32_t max_pages, const int32_t *seq_lens,
                         const int32_t *q_pos, const int32_t *widths, float scale, int32_t waves,
                         void *workspace, int64_t workspace_bytes, void *out, bool fit_waves,
                         const FusedAppend *fused = nullptr) {
  pkv_geometry geo;
  if (int rc = geometry(layout, &geo)) return rc;
  if (batch < 0) return fail(PKV_INVALID_ARGUMENT, "negative batch");
  if (batch == 0) return PKV_OK;
  if (num_heads < 1 || num_queries < 1 || num_heads % geo.hk)
    return fail(PKV_UNSUPPORTED, "paged attention requires query heads to form valid GQA groups");
  const int gqa = num_heads / geo.hk;
  if ((int64_t)num_queries * gqa > kMaxRows)
    return fail(PKV_UNSUPPORTED, "paged attention supports at most 2^24 query rows per KV head "
                                 "(queries x heads per KV head)");
  const int rows = num_queries * gqa;
  if (!pool || !queries || !block_table || !seq_lens || !out)
    return fail(PKV_INVALID_ARGUMENT, "paged attention requires pool, queries, block table, lengths, out");
  if (num_pages < 1 || max_pages < 1) return fail(PKV_INVALID_ARGUMENT, "empty page pool or block table");
  if (!std::isfinite(scale)) return fail(PKV_INVALID_ARGUMENT, "softmax scale must be finite");
  // the kernels number 16-token tiles in int32: bound them by the block table
  // (plus the split's lead tiles per segment)
  const int64_t tiles_per_seq = std::max<int64_t>(1, ((int64_t)max_pages * geo.page + 15) / 16) + 16;
  if ((int64_t)batch * tiles_per_seq * geo.hk > INT32_MAX / 2)
    return fail(PKV_UNSUPPORTED, "paged attention batch too large (more than 2^30 tiles)");
  const bool wide = !pkv::decode_serves(pkv::to_geo(geo), rows);
  if (wide && (int64_t)batch * geo.hk * ((rows + 127) / 128) > INT32_MAX)
    return fail(PKV_UNSUPPORTED, "paged attention grid too large");
  // The split-K decode parts: every sequence of a decode / verify call; in a
  // wide call with per-sequence widths (a mixed batch), the sequences whose
  // width fits the decode kernel -- in two tiers, those of at most 4 query
  // rows per KV head (the 4-row column-slot kernel) and the wider ones up to
  // the kernel's limit, so decode rows do not run at verify cost -- when the
  // workspace holds each tier's partials (else the prefill kernel serves
  // every sequence).  The tiers run one after the other on the stream and
  // share the workspace.
  struct Part {
    int nq, lo, hi, waves;  // queries covered; serve widths in (lo, hi] (hi 0: all)
    WorkspaceParts ws;
  };
  Part part[2];
  // the decode kernel appends the single new token itself (else an append
  // launch goes first): the fused form runs one wave per run
  const int in_kernel_append = fused && !wide && pkv::append_fusable(pkv::to_geo(geo), rows) ? 1 : 0;
  int nparts = 0;
  if (!wide) {
    part[nparts++] = Part{num_queries, 0, 0, waves, {0, 0, 0}};
  } else if (widths) {
    const int hi = decode_queries(geo, gqa);
    const int lo = std::min(hi, 4 / std::max(gqa, 1));
    if (lo >= 1) part[nparts++] = Part{lo, 0, lo, waves, {0, 0, 0}};
    if (hi > lo) part[nparts++] = Part{hi, lo, hi, waves, {0, 0, 0}};
  }
  for (int i = 0; i < nparts; ++i) {
    Part &t = part[i];
    const int trows = t.nq * gqa;
    if (t.waves <= 0) {
      t.waves = pkv_attention_default_waves(layout, num_heads, t.nq, batch);
      if (t.waves <= 0) return fail(PKV_LAUNCH_FAILED, "could not query the attention kernel's occupancy");
      if (fit_waves) {
        while (t.waves > 1 && workspace_parts(geo, trows, t.waves, in_kernel_append).total > workspace_bytes)
          t.waves = std::max<int64_t>(1, std::min<int64_t>(t.waves - 1,
              (int64_t)t.waves * workspace_bytes / workspace_parts(geo, trows, t.waves, in_kernel_append).total));
      }
    }
    if (t.waves > (1 << 24)) return fail(PKV_INVALID_ARGUMENT, "too many waves");
    t.ws = workspace_parts(geo, trows, t.waves, in_kernel_append);
    if (!workspace || workspace_bytes < t.ws.total) {
      if (!wide)
        return fail(PKV_OUT_OF_MEMORY,
                    "attention workspace too small: need " + std::to_string(t.ws.total) + " bytes");
      nparts = 0;  // no room: the prefill kernel serves every sequence
      break;
    }
  }

  // The fused append: in the decode kernel when it serves the shape, else
  // one append launch ahead of the attention.
  if (fused) {
    if (!fused->keys || !fused->values)
      return fail(PKV_INVALID_ARGUMENT, "fused append requires the new keys and values");
    if (wide || !pkv::append_fusable(pkv::to_geo(geo), rows)) {
      pkv::AppendArgs ap;
      ap.g = pkv::to_geo(geo);
      ap.pool = (uint8_t *)fused->pool;
      ap.num_pages = num_pages;
      ap.keys = (const uint16_t *)fused->keys;
      ap.values = (const uint16_t *)fused->values;
      ap.batch = batch;
      ap.tokens = 1;
      ap.max_pages = max_pages;
      ap.table = block_table;
      ap.start_pos = nullptr;
      ap.widths = nullptr;
      ap.lens_after = seq_lens;
      ap.new_lens = nullptr;
      if (int rc = check_launch(pkv::launch_append((hipStream_t)stream, ap), "append launch")) return rc;
      fused = nullptr;
    }
  }

  pkv::AttnArgs a;
  a.g = pkv::to_geo(geo);
  a.pool = (const uint8_t *)pool;
  a.num_pages = num_pages;
  a.q = (const uint16_t *)queries;
  a.batch = batch;
  a.heads = num_heads;
  a.gqa = gqa;
  a.table = block_table;
  a.max_pages = max_pages;
  a.seq_lens = seq_lens;
  a.q_pos = q_pos;
  a.widths = widths;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.nq_stride = num_queries;
  a.out = (uint16_t *)out;
  if (wide) {
    // chunked prefill: one pass per (sequence, KV head, row block), no
    // partials; sequences left to the decode parts get zeros, overwritten by them
    a.nq = num_queries;
    a.rows = rows;
    a.narrow_lo = 0;
    a.narrow_q = nparts ? part[nparts - 1].hi : 0;
    a.waves = 0;
    a.lead = 0;
    a.part_ml = nullptr;
    a.part_acc = nullptr;
    if (int rc = check_launch(pkv::launch_prefill((hipStream_t)stream, a), "prefill launch")) return rc;
  }
  for (int i = 0; i < nparts; ++i) {
    const Part &t = part[i];
    a.nq = t.nq;
    a.rows = t.nq * gqa;
    a.narrow_lo = t.lo;
    a.narrow_q = t.hi;
    a.waves = (int)attention_runs(geo, a.rows, t.waves, fused != nullptr);
    a.lead = pkv::attention_lead(a.g, a.rows, fused != nullptr);
    a.part_ml = (float *)((char *)workspace + t.ws.ml);
    a.part_acc = (float *)((char *)workspace + t.ws.acc);
    if (fused) {
      a.wpool = (uint8_t *)fused->pool;
      a.new_k = (const uint16_t *)fused->keys;
      a.new_v = (const uint16_t *)fused->values;
    }
    if (int rc = check_launch(pkv::launch_attention((hipStream_t)stream, a), "attention launch"))
      return rc;
    pkv::MergeArgs m;
    m.batch = batch;
    m.hk = geo.hk;
    m.heads = num_heads;
    m.nq = a.nq;
    m.gqa = gqa;
    m.rows = a.rows;
    m.dim = geo.dim;
    m.dp = geo.dp;
    m.float_kind = geo.float_kind;
    m.waves = a.waves;
    m.lead = a.lead;
    m.nq_stride = num_queries;
    m.narrow_lo = t.lo;
    m.narrow_q = t.hi;
    m.seq_lens = seq_lens;
    m.widths = widths;
    m.part_acc = a.part_acc;
    m.part_ml = a.part_ml;
    m.out = (uint16_t *)out;
    if (int rc = check_launch(pkv::launch_merge((hipStream_t)stream, m), "merge launch")) return rc;
  }
  return PKV_OK;
}

// ---- the allocation-free attention entry point ------------------------------------

// Split-K partials of pkv_paged_attention_noalloc: a fixed device array, one
// per GPU, held until the process ends.  Host code never uses its name as an
// address: the device address comes from hipGetSymbolAddress, once per device.
constexpr int64_t kNoAllocScratchBytes = 32ll << 20;
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

// The device address of this GPU's `scratch` (the current device), looked up on
// the first call on that device; NULL with the error text set on failure.
void *scratch_on_current_device() {
  static std::mutex mu;
  static void *ptrs[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(PKV_LAUNCH_FAILED, "no current HIP device (or more than 64 devices)");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      fail(PKV_LAUNCH_FAILED, std::string("scratch symbol lookup: ") + hipGetErrorString(e));
      return nullptr;
    }
    ptrs[dev] = ptr;
  }
  return ptrs[dev];
}

}  // namespace

extern "C" {

int pkv_paged_attention(void *stream, const pkv_layout *layout, const void *pool, int64_t num_pages,
                        const void *queries, int32_t batch, int32_t num_heads, int32_t num_queries,
                        const int32_t *block_table, int32_t max_pages, const int32_t *seq_lens,
                        const int32_t *q_pos, const int32_t *widths, float scale, int32_t waves,
                        void *workspace, int64_t workspace_bytes, void *out) {
  return paged_attention_impl(stream, layout, pool, num_pages, queries, batch, num_heads,
                              num_queries, block_table, max_pages, seq_lens, q_pos, widths, scale,
                              waves, workspace, workspace_bytes, out, false);
}

int pkv_append_paged_attention(void *stream, const pkv_layout *layout, void *pool, int64_t num_pages,
                               const void *keys, const void *values, const void *queries,
                               int32_t batch, int32_t num_heads, const int32_t *block_table,
                               int32_t max_pages, const int32_t *seq_lens, float scale,
                               int32_t waves, void *workspace, int64_t workspace_bytes, void *out) {
  const FusedAppend fused{pool, keys, values};
  return paged_attention_impl(stream, layout, pool, num_pages, queries, batch, num_heads, 1,
                              block_table, max_pages, seq_lens, nullptr, nullptr, scale, waves,
                              workspace, workspace_bytes, out, false, &fused);
}

int pkv_paged_attention_noalloc(void *stream, const pkv_layout *layout, const void *pool,
                                int64_t num_pages, const void *queries, int32_t batch,
                                int32_t num_heads, int32_t num_queries, const int32_t *block_table,
                                int32_t max_pages, const int32_t *seq_lens, const int32_t *q_pos,
                                const int32_t *widths, float scale, int32_t waves, void *out) {
  if (waves > 0) {
    pkv_geometry geo;
    if (int rc = geometry(layout, &geo)) return rc;
    // Only the split-K decode parts take scratch: a wide call without
    // per-sequence widths runs the prefill kernel alone and needs none.
    const bool shaped = num_heads >= 1 && num_queries >= 1 && num_heads % geo.hk == 0 &&
                        (int64_t)num_queries * (num_heads / geo.hk) <= kMaxRows;
    const bool prefill_only =
        shaped && !widths &&
        !pkv::decode_serves(pkv::to_geo(geo), num_queries * (num_heads / geo.hk));
    const int64_t need =
        prefill_only ? 0 : pkv_attention_workspace_bytes(layout, num_heads, num_queries, waves);
    if (need > kNoAllocScratchBytes)
      return fail(PKV_OUT_OF_MEMORY,
                  "pkv_paged_attention_noalloc: " + std::to_string(waves) + " waves need " +
                      std::to_string(need) + " bytes of split-K scratch, more than its fixed " +
                      std::to_string(kNoAllocScratchBytes) + " (pass fewer waves, or 0)");
  }
  void *ws = scratch_on_current_device();
  if (!ws) return PKV_LAUNCH_FAILED;
  return paged_attention_impl(stream, layout, pool, num_pages, queries, batch, num_heads,
                              num_queries, block_table, max_pages, seq_lens, q_pos, widths, scale,
                              waves, ws, kNoAllocScratchBytes, out, true);
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

int pkv_read_probe(void *stream, const pkv_layout *layout, const void *pool, int64_t num_pages,
                   const int32_t *page_ids, int64_t count, int32_t waves, void *out) {
  pkv_geometry geo;
  if (int rc = geometry(layout, &geo)) return rc;
  if (count < 0 || num_pages < 0) return fail(PKV_INVALID_ARGUMENT, "negative page count");
  if (waves < 1 || waves > (1 << 20)) return fail(PKV_INVALID_ARGUMENT, "waves must be in [1, 2^20]");
  if (!out) return fail(PKV_INVALID_ARGUMENT, "read probe requires an output buffer");
  if (count == 0) return PKV_OK;
  if (!pool || !page_ids) return fail(PKV_INVALID_ARGUMENT, "read probe requires pool and ids");
  return check_launch(pkv::launch_read_probe((hipStream_t)stream, (const uint8_t *)pool, num_pages,
                                             geo.page_bytes, page_ids, count, waves, (uint32_t *)out),
                      "read probe launch");
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

int pkv_rope_qkv(void *stream, const void *qkv, int32_t batch, int32_t tokens, int32_t heads,
                 int32_t kv_heads, int32_t dim, int32_t float_kind, const int32_t *positions,
                 const float *inv_freq, void *q, void *k, void *v) {
  if (float_kind != 0 && float_kind != 1) return fail(PKV_INVALID_ARGUMENT, "float_kind must be 0 or 1");
  if (batch < 0 || tokens < 0 || heads < 1 || kv_heads < 1 || dim < 2 || dim > 256 || (dim & 1))
    return fail(PKV_INVALID_ARGUMENT, "invalid RoPE shape");
  if ((int64_t)batch * tokens == 0) return PKV_OK;
  if ((int64_t)batch * tokens > 0x7fffffff) return fail(PKV_INVALID_ARGUMENT, "too many RoPE rows");
  if (!qkv || !positions || !inv_freq || !q || !k || !v)
    return fail(PKV_INVALID_ARGUMENT, "NULL tensor");
  pkv::RopeArgs a;
  a.qkv = (const uint16_t *)qkv;
  a.rows = (int64_t)batch * tokens;
  a.tokens = tokens;
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.dim = dim;
  a.float_kind = float_kind;
  a.positions = positions;
  a.inv_freq = inv_freq;
  a.q = (uint16_t *)q;
  a.k = (uint16_t *)k;
  a.v = (uint16_t *)v;
  return check_launch(pkv::launch_rope((hipStream_t)stream, a), "rope launch");
}

// ---- device page allocator ------------------------------------------------------

namespace {

int arena_common(void *state, int32_t capacity_pages, int32_t page_tokens, int32_t *slot_table,
                 int32_t num_slots, int32_t max_pages, int32_t *slot_lens, const int32_t *slots,
                 const int32_t *arg, int32_t count, pkv::ArenaArgs *a) {
  if (capacity_pages < 1 || capacity_pages > (1 << 30))
    return fail(PKV_INVALID_ARGUMENT, "arena capacity must be 1..2^30 pages");
  if (page_tokens != 16 && page_tokens != 32 && page_tokens != 64 && page_tokens != 128)
    return fail(PKV_INVALID_ARGUMENT, "page_tokens must be 16, 32, 64 or 128");
  if (num_slots < 1 || max_pages < 1 || (int64_t)max_pages * page_tokens > INT32_MAX)
    return fail(PKV_INVALID_ARGUMENT, "invalid slot table shape");
  if (count < 0) return fail(PKV_INVALID_ARGUMENT, "negative count");
  if (!state || !slot_table || !slot_lens || (count > 0 && (!slots || !arg)))
    return fail(PKV_INVALID_ARGUMENT, "NULL arena tensor");
  a->state = (int32_t *)state;
  a->capacity = capacity_pages;
  a->page_tokens = page_tokens;
  a->table = slot_table;
  a->max_pages = max_pages;
  a->num_slots = num_slots;
  a->lens = slot_lens;
  a->slots = slots;
  a->arg = arg;
  a->count = count;
  a->num_pools = 0;
  a->page_bytes = 0;
  a->batch_table = a->batch_starts = a->batch_lens = nullptr;
  return PKV_OK;
}

}  // namespace

int64_t pkv_arena_state_bytes(int32_t capacity_pages) {
  if (capacity_pages < 1 || capacity_pages > (1 << 30)) return -1;
  return ((int64_t)pkv::kArenaHeaderWords + 2 * (int64_t)capacity_pages) * 4;
}

int pkv_arena_init(void *stream, void *state, int32_t capacity_pages) {
  if (capacity_pages < 1 || capacity_pages > (1 << 30))
    return fail(PKV_INVALID_ARGUMENT, "arena capacity must be 1..2^30 pages");
  if (!state) return fail(PKV_INVALID_ARGUMENT, "NULL arena state");
  return check_launch(pkv::launch_arena_init((hipStream_t)stream, (int32_t *)state, capacity_pages),
                      "arena init launch");
}

int pkv_arena_reserve(void *stream, void *state, int32_t capacity_pages, int32_t page_tokens,
                      int32_t *slot_table, int32_t num_slots, int32_t max_pages, int32_t *slot_lens,
                      const int32_t *slots, const int32_t *widths, int32_t count,
                      void *const *pools, int32_t num_pools, int64_t page_bytes,
                      int32_t *batch_table, int32_t *batch_starts, int32_t *batch_lens) {
  pkv::ArenaArgs a;
  if (int rc = arena_common(state, capacity_pages, page_tokens, slot_table, num_slots, max_pages,
                            slot_lens, slots, widths, count, &a))
    return rc;
  if (num_pools < 0 || num_pools > pkv::kMaxArenaPools)
    return fail(PKV_INVALID_ARGUMENT, "arena pools must number 0..128");
  if (num_pools > 0 && (!pools || page_bytes < 16 || page_bytes % 16))
    return fail(PKV_INVALID_ARGUMENT, "arena pools need pointers and a page size that is a multiple of 16");
  for (int l = 0; l < num_pools; ++l) {
    if (!pools[l]) return fail(PKV_INVALID_ARGUMENT, "NULL arena pool");
    a.pools[l] = (uint8_t *)pools[l];
  }
  if (count > 0 && (!batch_table || !batch_starts || !batch_lens))
    return fail(PKV_INVALID_ARGUMENT, "reserve needs the batch table, starts and lengths outputs");
  a.num_pools = num_pools;
  a.page_bytes = page_bytes;
  a.batch_table = batch_table;
  a.batch_starts = batch_starts;
  a.batch_lens = batch_lens;
  return check_launch(pkv::launch_arena((hipStream_t)stream, pkv::ArenaOp::Reserve, a),
                      "arena reserve launch");
}

int pkv_arena_truncate(void *stream, void *state, int32_t capacity_pages, int32_t page_tokens,
                       int32_t *slot_table, int32_t num_slots, int32_t max_pages, int32_t *slot_lens,
                       const int32_t *slots, const int32_t *keep_tokens, int32_t count) {
  pkv::ArenaArgs a;
  if (int rc = arena_common(state, capacity_pages, page_tokens, slot_table, num_slots, max_pages,
                            slot_lens, slots, keep_tokens, count, &a))
    return rc;
  return check_launch(pkv::launch_arena((hipStream_t)stream, pkv::ArenaOp::Release, a),
                      "arena truncate launch");
}

int pkv_arena_fork(void *stream, void *state, int32_t capacity_pages, int32_t page_tokens,
                   int32_t *slot_table, int32_t num_slots, int32_t max_pages, int32_t *slot_lens,
                   const int32_t *src_slots, const int32_t *dst_slots, int32_t count) {
  pkv::ArenaArgs a;
  if (int rc = arena_common(state, capacity_pages, page_tokens, slot_table, num_slots, max_pages,
                            slot_lens, src_slots, dst_slots, count, &a))
    return rc;
  return check_launch(pkv::launch_arena((hipStream_t)stream, pkv::ArenaOp::Fork, a),
                      "arena fork launch");
}

