// pkv_token.h -- quantize one token's K/V rows and store them into a page
// (device functions shared by the append kernel and the fused append +
// attention kernel).
//
// The reference quantizer's arithmetic (src/mlx_one/engine/paged.py:30-40,
// restated):
//   bias  = f16(min(group))                         f32 -> f16, round to nearest even
//   scale = f16(max(f32(max - f32(bias)) / (2^b - 1), 1e-6))
//   code  = clamp(rint((x - f32(bias)) / f32(scale)), 0, 2^b - 1)
// with IEEE-correct f32 division and half-to-even rint.  The codes are then
// scattered into the MFMA-ordered page format of pkv_format.h.
#pragma once
#include "pkv_device.h"

namespace pkv {

// Quantize the wave's row (EPL elements per lane, natural order d = lane*EPL + i)
// and leave the codes in `codes[d]` (LDS) and the meta word per group in `meta`.
template <int EPL>
__device__ __forceinline__ void quantize_row(const float (&x)[EPL], int lane, int group, int bits,
                                             uint8_t *codes, uint32_t *meta) {
  float lo = x[0], hi = x[0];
#pragma unroll
  for (int i = 1; i < EPL; ++i) { lo = fminf(lo, x[i]); hi = fmaxf(hi, x[i]); }
  const int lanes_per_group = group / EPL;  // 8..128
  for (int o = 1; o < lanes_per_group && o < 64; o <<= 1) {
    lo = fminf(lo, __shfl_xor(lo, o, 64));
    hi = fmaxf(hi, __shfl_xor(hi, o, 64));
  }
  const float levels = (float)((1 << bits) - 1);
  uint16_t b16 = f32_to_f16_bits(lo);
  float b = f16_bits_to_f32(b16);
  float s = __fdiv_rn(hi - b, levels);
  s = fmaxf(s, 1e-6f);
  uint16_t s16 = f32_to_f16_bits(s);
  float sf = f16_bits_to_f32(s16);
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    float c = rintf(__fdiv_rn(x[i] - b, sf));
    c = fminf(fmaxf(c, 0.0f), levels);
    codes[lane * EPL + i] = (uint8_t)c;
  }
  if ((lane * EPL) % group == 0) meta[(lane * EPL) / group] = (uint32_t)s16 | ((uint32_t)b16 << 16);
}

// Make one wave's LDS writes visible to its other lanes.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Store a quantized token (codes kc/vc in natural order, meta words km/vm per
// group, all in LDS) at page slot `slot` of head block `head`: the K payload
// (lane' = tt + 16*jj owns elements d = 32*kb + 8*jj + e), the V payload
// (lane' = col + 16*jj holds V[4*jj + r][16*n + col]) and the (scale, bias)
// words.  One wave; lanes split the work.
template <int DP, int BITS>
__device__ __forceinline__ void store_token(const Geo &g, uint8_t *head, int slot, const uint8_t *kc,
                                            const uint8_t *vc, const uint32_t *km, const uint32_t *vm,
                                            int lane) {
  constexpr int EPL = DP / 64;
  const int tt = slot % PKV_TILE;
  const int64_t tile = (int64_t)(slot / PKV_TILE) * g.tile_bytes;
  uint8_t *ktile = head + tile, *vtile = head + g.v_offset + tile;
  if constexpr (BITS == 8) {
    constexpr int WPJ = DP / 16;  // dwords per jj
    if (lane < 4 * WPJ) {
      const int jj = lane / WPJ, w = lane % WPJ;
      const int d0 = 32 * (w / 2) + 8 * jj + 4 * (w % 2);
      const uint32_t word = (uint32_t)kc[d0] | ((uint32_t)kc[d0 + 1] << 8) |
                            ((uint32_t)kc[d0 + 2] << 16) | ((uint32_t)kc[d0 + 3] << 24);
      *(uint32_t *)(ktile + payload_offset(tt + 16 * jj, 4 * w, g.chunk)) = word;
    }
  } else {
    constexpr int WPJ = DP / 32;
    if (lane < 4 * WPJ) {
      const int jj = lane / WPJ, kb = lane % WPJ;
      uint32_t word = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        word |= (uint32_t)(kc[32 * kb + 8 * jj + e] & 15) << (4 * k4_nibble(e));
      *(uint32_t *)(ktile + payload_offset(tt + 16 * jj, 4 * kb, g.chunk)) = word;
    }
  }
  const int vjj = tt / 4, r = tt % 4;
  if constexpr (BITS == 8) {
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int d = lane * EPL + i, n = d / 16, col = d % 16;
      vtile[payload_offset(col + 16 * vjj, 4 * n + r, g.chunk)] = vc[d];
    }
  } else {
    // one byte per (block pair m, col): low nibble block 2m, high nibble 2m+1
    for (int idx = lane; idx < DP / 2; idx += 64) {
      const int m = idx / 16, col = idx % 16;
      const uint8_t byte = (uint8_t)((vc[32 * m + col] & 15) | ((vc[32 * m + 16 + col] & 15) << 4));
      vtile[payload_offset(col + 16 * vjj, 4 * m + v4_byte(r), g.chunk)] = byte;
    }
  }
  if (lane < g.ng) {
    *(uint32_t *)(head + g.kmeta_offset + ((int64_t)slot * g.ng + lane) * 4) = km[lane];
    *(uint32_t *)(head + g.vmeta_offset + ((int64_t)slot * g.ng + lane) * 4) = vm[lane];
  }
}

}  // namespace pkv
