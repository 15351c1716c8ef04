// pkv_append.hip -- append-and-quantize, reference-format gather and page copy.
//
// append: one wave per (sequence, new token, KV head) quantizes the K and V
// rows group-wise with the reference quantizer's arithmetic
// (src/mlx_one/engine/paged.py:30-40, restated):
//   bias  = f16(min(group))                         f32 -> f16, round to nearest even
//   scale = f16(max(f32(max - f32(bias)) / (2^b - 1), 1e-6))
//   code  = clamp(rint((x - f32(bias)) / f32(scale)), 0, 2^b - 1)
// with IEEE-correct f32 division and half-to-even rint, then scatters the
// codes and the (scale, bias) word into the MFMA-ordered page format of
// pkv_format.h.  Float pages store the input bits unchanged.
#include "pkv_launch.h"
#include "pkv_token.h"

namespace pkv {


template <int DP, int BITS>
__global__ __launch_bounds__(256) void append_kernel(const AppendArgs a) {
  constexpr int EPL = DP / 64;
  __shared__ uint8_t s_codes[4][2][DP];
  __shared__ uint32_t s_meta[4][2][8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const Geo &g = a.g;
  const int64_t item = (int64_t)blockIdx.x * 4 + wave;
  const int64_t items = (int64_t)a.batch * a.tokens * g.hk;
  if (item >= items) return;
  const int kh = (int)(item % g.hk);
  const int t = (int)((item / g.hk) % a.tokens);
  const int b = (int)(item / ((int64_t)g.hk * a.tokens));
  // The new rows first: every (sequence, token, KV head) row of the inputs
  // exists, and they do not depend on the position and page lookups below,
  // so both requests are in flight together.
  const int64_t row = (((int64_t)b * g.hk + kh) * a.tokens + t) * g.dim;
  const uint16_t *src[2] = {a.keys + row, a.values + row};
  uint16_t raw[2][EPL];
#pragma unroll
  for (int side = 0; side < 2; ++side)
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int d = lane * EPL + i;
      raw[side][i] = d < g.dim ? src[side][d] : (uint16_t)0;
    }
  const int width = a.widths ? a.widths[b] : a.tokens;
  // start position: given, or the sequence's length after the append less the new tokens
  const int start = a.start_pos ? a.start_pos[b] : a.lens_after[b] - a.tokens;
  if (a.new_lens && t == 0 && kh == 0 && lane == 0) a.new_lens[b] = start + width;
  if (t >= width) return;
  const int pos = start + t;
  if (pos < 0 || pos / g.page >= a.max_pages) return;
  const int page = a.table[(int64_t)b * a.max_pages + pos / g.page];
  if (page < 0 || page >= a.num_pages) return;
  const int slot = pos % g.page, tt = slot % PKV_TILE;
  uint8_t *head = a.pool + (int64_t)page * g.page_bytes + (int64_t)kh * g.head_bytes;
  const int64_t tile = (int64_t)(slot / PKV_TILE) * g.tile_bytes;
  uint8_t *ktile = head + tile, *vtile = head + g.v_offset + tile;

  if (BITS == 16) {
    // float pages: scatter the input bits
    for (int side = 0; side < 2; ++side) {
#pragma unroll
      for (int i = 0; i < EPL; ++i) {
        const int d = lane * EPL + i;
        const uint16_t v = raw[side][i];
        int64_t off;
        if (side == 0) {
          const int kb = d / 32, jj = (d % 32) / 8, e = d % 8;
          off = payload_offset(tt + 16 * jj, 2 * (8 * kb + e), g.chunk);
          *(uint16_t *)(ktile + off) = v;
        } else {
          const int n = d / 16, col = d % 16, jj = tt / 4, r = tt % 4;
          off = payload_offset(col + 16 * jj, 2 * (4 * n + r), g.chunk);
          *(uint16_t *)(vtile + off) = v;
        }
      }
    }
    return;
  }

  for (int side = 0; side < 2; ++side) {
    float x[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int d = lane * EPL + i;
      x[i] = d < g.dim ? bits_to_float(raw[side][i], g.float_kind) : 0.0f;  // zero pad
    }
    quantize_row<EPL>(x, lane, g.group, BITS, s_codes[wave][side], s_meta[wave][side]);
  }
  wave_lds_sync();
  const uint8_t *kc = s_codes[wave][0], *vc = s_codes[wave][1];

  store_token<DP, BITS>(g, head, slot, kc, vc, s_meta[wave][0], s_meta[wave][1], lane);
}

// ---- gather to the reference format ---------------------------------------


__device__ __forceinline__ int read_code(const uint8_t *tile, int side, int bits, int tt, int d,
                                         int chunk) {
  if (side == 0) {
    const int kb = d / 32, jj = (d % 32) / 8, e = d % 8, lane = tt + 16 * jj;
    if (bits == 8) return tile[payload_offset(lane, 8 * kb + e, chunk)];
    const int nib = k4_nibble(e);
    return (tile[payload_offset(lane, 4 * kb + nib / 2, chunk)] >> (4 * (nib & 1))) & 15;
  }
  const int n = d / 16, col = d % 16, jj = tt / 4, r = tt % 4, lane = col + 16 * jj;
  if (bits == 8) return tile[payload_offset(lane, 4 * n + r, chunk)];
  return (tile[payload_offset(lane, 4 * (n / 2) + v4_byte(r), chunk)] >> (4 * (n % 2))) & 15;
}

// One thread per (page, head, token, output byte); grid-stride.
__global__ __launch_bounds__(256) void gather_kernel(const GatherArgs a) {
  const Geo &g = a.g;
  const bool quant = g.bits != 16;
  const int per_row = quant ? a.dq : g.dim;  // codes bytes or float elements per row
  const int64_t rows = (int64_t)a.count * g.hk * g.page;
  const int64_t total = rows * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int x = (int)(i % per_row);
    const int64_t rowi = i / per_row;
    const int tok = (int)(rowi % g.page);
    const int kh = (int)((rowi / g.page) % g.hk);
    const int pi = (int)(rowi / ((int64_t)g.page * g.hk));
    const int page = a.ids[pi];
    if (page < 0 || page >= a.num_pages) continue;
    const uint8_t *head = a.pool + (int64_t)page * g.page_bytes + (int64_t)kh * g.head_bytes;
    const int64_t tile = (int64_t)(tok / PKV_TILE) * g.tile_bytes;
    const int tt = tok % PKV_TILE;
    for (int side = 0; side < 2; ++side) {
      const uint8_t *payload = head + (side ? g.v_offset : 0) + tile;
      if (!quant) {
        const int d = x;
        int64_t off;
        if (side == 0) {
          off = payload_offset(tt + 16 * ((d % 32) / 8), 2 * (8 * (d / 32) + d % 8), g.chunk);
        } else {
          off = payload_offset(d % 16 + 16 * (tt / 4), 2 * (4 * (d / 16) + tt % 4), g.chunk);
        }
        uint16_t *dst = (uint16_t *)(side ? a.vc : a.kc);
        dst[rowi * g.dim + d] = *(const uint16_t *)(payload + off);
        continue;
      }
      uint8_t out;
      if (g.bits == 8) {
        out = (uint8_t)read_code(payload, side, 8, tt, x, g.chunk);
      } else {
        out = (uint8_t)(read_code(payload, side, 4, tt, 2 * x, g.chunk) |
                        (read_code(payload, side, 4, tt, 2 * x + 1, g.chunk) << 4));
      }
      (side ? a.vc : a.kc)[rowi * a.dq + x] = out;
      if (x < a.ngr) {
        const uint32_t word = *(const uint32_t *)(head + (side ? g.vmeta_offset : g.kmeta_offset) +
                                                  ((int64_t)tok * g.ng + x) * 4);
        (side ? a.vs : a.ks)[rowi * a.ngr + x] = (uint16_t)(word & 0xFFFFu);
        (side ? a.vb : a.kb)[rowi * a.ngr + x] = (uint16_t)(word >> 16);
      }
    }
  }
}

// ---- page copy ---------------------------------------------------------------

__global__ __launch_bounds__(256) void copy_pages_kernel(uint8_t *pool, int64_t num_pages,
                                                         int64_t page_bytes, const int32_t *src,
                                                         const int32_t *dst, int count) {
  const int64_t vec = page_bytes / 16;
  const int64_t total = vec * count;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int pi = (int)(i / vec);
    const int64_t off = (i % vec) * 16;
    const int s = src[pi], d = dst[pi];
    if (s < 0 || s >= num_pages || d < 0 || d >= num_pages) continue;
    *(u4 *)(pool + (int64_t)d * page_bytes + off) = *(const u4 *)(pool + (int64_t)s * page_bytes + off);
  }
}

// ---- host launchers (called from pkv_abi.hip) ------------------------------

hipError_t launch_append(hipStream_t stream, const AppendArgs &a) {
  const int64_t items = (int64_t)a.batch * a.tokens * a.g.hk;
  if (items == 0) return hipSuccess;
  dim3 grid((unsigned)((items + 3) / 4)), block(256);
#define PKV_APPEND(DP_, BITS_)                                                       \
  if (a.g.dp == DP_ && a.g.bits == BITS_) {                                          \
    hipLaunchKernelGGL((append_kernel<DP_, BITS_>), grid, block, 0, stream, a);      \
    return hipGetLastError();                                                        \
  }
  PKV_APPEND(64, 4) PKV_APPEND(64, 8) PKV_APPEND(64, 16)
  PKV_APPEND(128, 4) PKV_APPEND(128, 8) PKV_APPEND(128, 16)
  PKV_APPEND(256, 4) PKV_APPEND(256, 8) PKV_APPEND(256, 16)
#undef PKV_APPEND
  return hipErrorInvalidValue;
}

hipError_t launch_gather(hipStream_t stream, const GatherArgs &a) {
  const int per_row = a.g.bits != 16 ? a.dq : a.g.dim;
  const int64_t total = (int64_t)a.count * a.g.hk * a.g.page * per_row;
  if (total == 0) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(gather_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_copy(hipStream_t stream, uint8_t *pool, int64_t num_pages, int64_t page_bytes,
                       const int32_t *src, const int32_t *dst, int count) {
  const int64_t total = page_bytes / 16 * count;
  if (total == 0) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(copy_pages_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, pool,
                     num_pages, page_bytes, src, dst, count);
  return hipGetLastError();
}

}  // namespace pkv
