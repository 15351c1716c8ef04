// pkv_format.h -- page format of the MI355X page arena (host and device).
//
// A layer's KV lives in one device pool of fixed-size pages; page `p`, KV head
// `kh` owns a contiguous "head block" at  pool + p*page_bytes + kh*head_bytes.
// The logical content of a page is the reference's (src/mlx_one/engine/
// paged_attention.py:31-35: per (head, token) codes along the head dim plus an
// f16 scale and f16 bias per group); only the byte order differs.  The order is
// chosen so that one 64-lane wave reads a 16-token tile with fully coalesced
// 16-byte loads that land directly in MFMA operand registers:
//
//   head block = [K payload, P/16 tiles][V payload, P/16 tiles]
//                [K meta  P x NG x (f16 scale, f16 bias)]
//                [V meta  P x NG x (f16 scale, f16 bias)]     (quantized only)
//
// Tile payload: lane l of a wave owns "lane bytes" LB = DP*bits/32 bytes, kept
// as chunks of CS = min(16, LB) bytes; chunk c of lane l sits at
//   tile + c*64*CS + l*CS.
//
// K tile (S^T = K.Q^T on v_mfma_f32_16x16x32): lane l = t + 16*jj holds token t
// of the tile, head-dim elements d = 32*kb + 8*jj + e (kb < DP/32, e < 8),
// kb-major.  8-bit: one byte per element.  bf16/f16: two bytes.  4-bit: the 8
// elements of one kb form one dword; element e sits in nibble
// (e even ? e/2 : 4 + e/2), so that ((w >> 4s) & 0x000F000F) | 0x64006400 is
// the f16 pair (1024+c[2s], 1024+c[2s+1]).
//
// V tile (O += P.V on v_mfma_f32_16x16x16): lane l = col + 16*jj holds, for
// N-block n < DP/16 and r < 4, element V[t = 4*jj + r][d = 16*n + col],
// n-major.  8-bit: one byte per (n, r) -- 4 tokens per dword.  Float: 2 bytes.
// 4-bit: blocks (2m, 2m+1) share a dword: byte 0 = token r=0 (low nibble block
// 2m, high nibble 2m+1), byte 1 = r=2, byte 2 = r=1, byte 3 = r=3, so each
// byte belongs to one token (appends of different tokens never share a byte)
// and the same shift/mask extraction yields the operand pairs.
//
// Meta: token-major, (scale, bias) as one 32-bit word per (token, group).
#pragma once
#include <stdint.h>

#define PKV_TILE 16          // tokens per tile (MFMA M/K extent)
#define PKV_LANES 64

struct pkv_geometry {
  int hk, dim, page, bits, group, float_kind;
  int dp;           // stored head dim: 64, 128 or 256
  int ng;           // groups per (head, token) in storage = dp / group (quantized)
  int lane_bytes;   // payload bytes per lane per tile
  int chunk;        // bytes per lane chunk
  int64_t tile_bytes;   // payload bytes per tile (K or V)
  int64_t head_bytes;   // bytes per (page, kv head)
  int64_t page_bytes;   // bytes per page
  int64_t v_offset;     // V payload offset inside the head block
  int64_t kmeta_offset, vmeta_offset;
};

// Returns 0 on success, -1 when the layout is not representable.
static inline int pkv_make_geometry(int hk, int dim, int page, int bits, int group, int float_kind,
                                    struct pkv_geometry *g) {
  if (hk < 1 || dim < 1 || dim > 256 || page < 16 || page % 16 || page > 128) return -1;
  if (bits != 4 && bits != 8 && bits != 16) return -1;
  if (float_kind != 0 && float_kind != 1) return -1;
  int quant = bits != 16;
  if (quant && group != 32 && group != 64 && group != 128) return -1;
  int need = quant ? (dim + group - 1) / group * group : dim;
  int dp = need <= 64 ? 64 : need <= 128 ? 128 : 256;
  if (quant && dp % group) return -1;
  g->hk = hk; g->dim = dim; g->page = page; g->bits = bits; g->group = quant ? group : 0;
  g->float_kind = float_kind; g->dp = dp; g->ng = quant ? dp / group : 0;
  g->lane_bytes = dp * bits / 32;
  g->chunk = g->lane_bytes < 16 ? g->lane_bytes : 16;
  g->tile_bytes = (int64_t)g->lane_bytes * PKV_LANES;
  int64_t payload = g->tile_bytes * (page / PKV_TILE);
  g->v_offset = payload;
  g->kmeta_offset = 2 * payload;
  int64_t meta = quant ? (int64_t)page * g->ng * 4 : 0;
  g->vmeta_offset = g->kmeta_offset + meta;
  g->head_bytes = 2 * payload + 2 * meta;
  g->page_bytes = g->head_bytes * hk;
  return 0;
}
