// Rotate-half RoPE of a fused q|k|v projection, written head-major.
//
// The caller side of the paged attend (the reference's attention block,
// src/mlx_one/models/shared/transformer.py:32-90 and :146-184): q and k are
// rotated at their logical positions, v is passed through, and all three
// leave in the [B, heads, T, D] layout the append and attention kernels read.
// One launch replaces the projection split, two transposes and the ~20
// element-wise ops of the same computation in torch.
//
// Arithmetic is that of the reference's float32 composite
// value * cos(f) + rotate_half(value) * sin(f) (transformer.py:86-88):
//   angle = f32(pos) * inv_freq[i];  c = cos(angle);  s = sin(angle)
//   out[i]        = a*c - b*s,   out[i + D/2] = b*c + a*s      (a = x[i], b = x[i + D/2])
// with every product and sum rounded on its own (no fused multiply-add), then
// one round-to-nearest-even cast to the activation type.

#include "pkv_device.h"
#include "pkv_launch.h"

namespace pkv {

namespace {

// One workgroup per token row; its waves share the row's heads.  cos/sin depend
// on (position, i) only, so each wave computes them once (in registers) and
// applies them to every head it owns.
constexpr int kRopeWaves = 4;
constexpr int kMaxPairsPerLane = 2;   // dim <= 256

__global__ void __launch_bounds__(64 * kRopeWaves) rope_kernel(RopeArgs a) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;            // b * T + t
  if (row >= a.rows) return;
  const int heads = a.heads + 2 * a.kv_heads;
  const int half = a.dim >> 1;
  const int64_t b = row / a.tokens, t = row - b * a.tokens;
  const float pos = (float)a.positions[row];
  float c[kMaxPairsPerLane], s[kMaxPairsPerLane];
#pragma unroll
  for (int j = 0; j < kMaxPairsPerLane; ++j) {
    const int i = lane + 64 * j;
    const float angle = i < half ? pos * a.inv_freq[i] : 0.0f;
    c[j] = cosf(angle);
    s[j] = sinf(angle);
  }
  const uint16_t *src_row = a.qkv + row * heads * a.dim;
#pragma unroll 2
  for (int h = wave; h < heads; h += kRopeWaves) {
    const uint16_t *src = src_row + (int64_t)h * a.dim;
    uint16_t *dst;
    if (h < a.heads) {
      dst = a.q + ((b * a.heads + h) * a.tokens + t) * a.dim;
    } else if (h < a.heads + a.kv_heads) {
      dst = a.k + ((b * a.kv_heads + (h - a.heads)) * a.tokens + t) * a.dim;
    } else {
      dst = a.v + ((b * a.kv_heads + (h - a.heads - a.kv_heads)) * a.tokens + t) * a.dim;
      for (int i = lane; i < a.dim; i += 64) dst[i] = src[i];
      continue;
    }
#pragma unroll
    for (int j = 0; j < kMaxPairsPerLane; ++j) {
      const int i = lane + 64 * j;
      if (i < half) {
        const float x0 = bits_to_float(src[i], a.float_kind);
        const float x1 = bits_to_float(src[i + half], a.float_kind);
        const float lo = x0 * c[j] - x1 * s[j];
        const float hi = x1 * c[j] + x0 * s[j];
        dst[i] = float_to_bits(lo, a.float_kind);
        dst[i + half] = float_to_bits(hi, a.float_kind);
      }
    }
  }
}

// dim/2 a multiple of 8: each lane owns 8 pairs (two 16-byte loads and stores
// per head), LPH lanes cover one head and a wave moves 64/LPH heads; grid.y
// splits a row's heads over workgroups so short batches (decode) still fill
// the chip.  The row's cos/sin (dim/2 of each) are computed once per
// workgroup, one per thread, into LDS.
template <int LPH>
__global__ void __launch_bounds__(64 * kRopeWaves) rope_vec_kernel(RopeArgs a) {
#pragma clang fp contract(off)
  constexpr int kHeadsPerStep = 64 / LPH;
  constexpr int kHalf = LPH * 8;
  __shared__ float s_cos[kHalf], s_sin[kHalf];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;            // b * T + t (the grid has exactly rows)
  const float pos = (float)a.positions[row];
  for (int i = threadIdx.x; i < kHalf; i += 64 * kRopeWaves) {
    const float angle = pos * a.inv_freq[i];
    s_cos[i] = cosf(angle);
    s_sin[i] = sinf(angle);
  }
  __syncthreads();
  const int heads = a.heads + 2 * a.kv_heads;
  const int h = (blockIdx.y * kRopeWaves + wave) * kHeadsPerStep + lane / LPH;
  if (h >= heads) return;
  const int i0 = (lane % LPH) * 8;
  const int64_t b = row / a.tokens, t = row - b * a.tokens;
  const uint16_t *src = a.qkv + (row * heads + h) * (2 * kHalf);
  const uint4 u0 = *(const uint4 *)(src + i0);
  const uint4 u1 = *(const uint4 *)(src + kHalf + i0);
  uint16_t *dst;
  if (h < a.heads) {
    dst = a.q + ((b * a.heads + h) * a.tokens + t) * (2 * kHalf);
  } else if (h < a.heads + a.kv_heads) {
    dst = a.k + ((b * a.kv_heads + (h - a.heads)) * a.tokens + t) * (2 * kHalf);
  } else {
    dst = a.v + ((b * a.kv_heads + (h - a.heads - a.kv_heads)) * a.tokens + t) * (2 * kHalf);
    *(uint4 *)(dst + i0) = u0;
    *(uint4 *)(dst + kHalf + i0) = u1;
    return;
  }
  const uint16_t *x0 = (const uint16_t *)&u0, *x1 = (const uint16_t *)&u1;
  uint4 o0, o1;
  uint16_t *y0 = (uint16_t *)&o0, *y1 = (uint16_t *)&o1;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float c = s_cos[i0 + j], sn = s_sin[i0 + j];
    const float p = bits_to_float(x0[j], a.float_kind), q = bits_to_float(x1[j], a.float_kind);
    y0[j] = float_to_bits(p * c - q * sn, a.float_kind);
    y1[j] = float_to_bits(q * c + p * sn, a.float_kind);
  }
  *(uint4 *)(dst + i0) = o0;
  *(uint4 *)(dst + kHalf + i0) = o1;
}

}  // namespace

hipError_t launch_rope(hipStream_t stream, const RopeArgs &a) {
  if (a.dim > 128 * kMaxPairsPerLane) return hipErrorInvalidValue;
  const dim3 block(64 * kRopeWaves);
  dim3 grid((unsigned)a.rows);
  const int heads = a.heads + 2 * a.kv_heads;
  if (a.dim % 16 == 0 && a.dim <= 256) {
    const int per_block = kRopeWaves * (64 / (a.dim / 16));   // heads per workgroup
    grid.y = (heads + per_block - 1) / per_block;
  }
  switch (a.dim) {   // dim/2 = 8 * lanes per head
    case 16: hipLaunchKernelGGL(rope_vec_kernel<1>, grid, block, 0, stream, a); break;
    case 32: hipLaunchKernelGGL(rope_vec_kernel<2>, grid, block, 0, stream, a); break;
    case 64: hipLaunchKernelGGL(rope_vec_kernel<4>, grid, block, 0, stream, a); break;
    case 128: hipLaunchKernelGGL(rope_vec_kernel<8>, grid, block, 0, stream, a); break;
    case 256: hipLaunchKernelGGL(rope_vec_kernel<16>, grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL(rope_kernel, grid, block, 0, stream, a); break;
  }
  return hipGetLastError();
}

}  // namespace pkv
