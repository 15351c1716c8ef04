// pkv_device.h -- device helpers shared by the libpkv kernels (gfx950).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pkv_format.h"

namespace pkv {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

// Geometry passed to kernels by value.
struct Geo {
  int hk, dim, page, bits, group, float_kind, dp, ng, lane_bytes, chunk;
  int64_t tile_bytes, head_bytes, page_bytes, v_offset, kmeta_offset, vmeta_offset;
};

static inline Geo to_geo(const pkv_geometry &g) {
  Geo o;
  o.hk = g.hk; o.dim = g.dim; o.page = g.page; o.bits = g.bits; o.group = g.group;
  o.float_kind = g.float_kind; o.dp = g.dp; o.ng = g.ng; o.lane_bytes = g.lane_bytes;
  o.chunk = g.chunk; o.tile_bytes = g.tile_bytes; o.head_bytes = g.head_bytes;
  o.page_bytes = g.page_bytes; o.v_offset = g.v_offset; o.kmeta_offset = g.kmeta_offset;
  o.vmeta_offset = g.vmeta_offset;
  return o;
}

// float16 / bfloat16 bit conversions (round to nearest even).
__device__ __forceinline__ float bits_to_float(uint16_t v, int float_kind) {
  if (float_kind == 0) return __uint_as_float((uint32_t)v << 16);
  _Float16 h = __builtin_bit_cast(_Float16, v);
  return (float)h;
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
  _Float16 h = (_Float16)x;  // v_cvt_f16_f32: round to nearest even
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t v) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFFu));
  return (float)h;
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ uint16_t float_to_bits(float x, int float_kind) {
  return float_kind == 0 ? f32_to_bf16_bits(x) : f32_to_f16_bits(x);
}

// Byte offset, inside one tile payload, of byte `i` of lane `l`'s payload.
__device__ __forceinline__ int64_t payload_offset(int lane, int i, int chunk) {
  return (int64_t)(i / chunk) * (PKV_LANES * chunk) + (int64_t)lane * chunk + (i % chunk);
}

// Nibble holding logical element x (< 8) of a 4-bit dword, so that
// ((w >> 4s) & 0x000F000F) | 0x64006400 yields the f16 pair of elements (2s, 2s+1).
__device__ __forceinline__ int k4_nibble(int x) { return (x & 1) ? 4 + (x >> 1) : (x >> 1); }

// Byte of a 4-bit V dword holding token r (< 4) of a token quad.
__device__ __forceinline__ int v4_byte(int r) {
  return r == 0 ? 0 : r == 1 ? 2 : r == 2 ? 1 : 3;
}

// Wave-wide inclusive prefix sum on DPP moves (no LDS round trips): prefix
// sums within each 16-lane row by row_shr 1, 2, 4, 8 (lanes shifted in from
// before the row read 0), then row 1 and row 3 add lane 15 / 47
// (row_bcast:15), rows 2 and 3 add lane 31 (row_bcast:31).  The whole wave
// calls it with every lane active (a DPP read of a disabled lane gives 0).
// `lane` is unused.
__device__ __forceinline__ int wave_scan_incl(int v, int /*lane*/) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return v;
}

// Wave-wide sum, uniform (read from the scan's last lane).
__device__ __forceinline__ int wave_sum(int v) {
  return __builtin_amdgcn_readlane(wave_scan_incl(v, 0), 63);
}

// v + v[lane ^ 16] and v + v[lane ^ 32] (and the max forms) on the gfx950
// permlane swaps, VALU only.  permlane16_swap(v, v) returns (row 0, row 0,
// row 2, row 2 | row 1, row 1, row 3, row 3) as its two halves, and
// permlane32_swap(v, v) (lanes < 32, lanes < 32 | lanes >= 32, lanes >= 32),
// so each lane adds its own value and its partner's.
__device__ __forceinline__ float xor16_add(float v) {
  const auto z = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(z[0]) + __uint_as_float(z[1]);
}
__device__ __forceinline__ float xor32_add(float v) {
  const auto z = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(z[0]) + __uint_as_float(z[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto z = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(z[0]), __uint_as_float(z[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto z = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(z[0]), __uint_as_float(z[1]));
}

// Lane exchange within 16-lane rows by a DPP pattern (every lane valid):
// 0xB1 quad_perm xor 1, 0x4E quad_perm xor 2, 0x141 row_half_mirror
// (lane i <-> 7 - i in each 8), 0x140 row_mirror (i <-> 15 - i).
template <int CTRL>
__device__ __forceinline__ float row_xchg(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Number of partitions of a sequence of `len` tokens (at least one, so that
// an empty sequence still owns a unit that writes zeros).
__device__ __forceinline__ int splits_of(int len, int split) {
  return len <= 0 ? 1 : (len + split - 1) / split;
}

// Find the (sequence, partition) of split-unit `su`: units are ordered by
// sequence, then partition.  Whole wave must call.  Returns false when `su`
// is past the last unit.
__device__ __forceinline__ bool locate_unit(const int32_t *__restrict__ lens, int batch, int split,
                                            int su, int lane, int &b, int &part, int &nsplit,
                                            int &first_unit) {
  int carry = 0;
  for (int c0 = 0; c0 < batch; c0 += 64) {
    int idx = c0 + lane;
    int ns = idx < batch ? splits_of(lens[idx], split) : 0;
    int incl = wave_scan_incl(ns, lane) + carry;
    unsigned long long hit = __ballot(idx < batch && incl > su);
    if (hit) {
      int first = __ffsll((long long)hit) - 1;
      int excl = incl - ns;
      first_unit = __shfl(excl, first, 64);
      nsplit = __shfl(ns, first, 64);
      b = c0 + first;
      part = su - first_unit;
      return true;
    }
    carry = __shfl(incl, 63, 64);
  }
  return false;
}

}  // namespace pkv
