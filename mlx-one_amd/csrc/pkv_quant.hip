// pkv_quant.hip -- row quantizer / dequantizer in the reference's page format.
//
// quantize: one wave per row of `dim` values, groups of `group` along the row
// (zero padded to whole groups), the quantize_page arithmetic of
// src/mlx_one/engine/paged.py:30-40 (see pkv_append.hip); 4-bit output packs
// code[2i] | code[2i+1] << 4 (paged.py:39-40).
// dequantize: x = f32(code) * f32(scale) + f32(bias) (paged.py:44-54), float32 out.
#include "pkv_launch.h"

namespace pkv {

__global__ __launch_bounds__(256) void quantize_rows_kernel(const QuantRowsArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= a.rows) return;
  const int padded = (a.dim + a.group - 1) / a.group * a.group;
  const int ngroups = padded / a.group;
  const int qbytes = a.bits == 4 ? padded / 2 : padded;
  const float levels = (float)((1 << a.bits) - 1);
  const uint16_t *src = a.values + row * a.dim;
  for (int gi = 0; gi < ngroups; ++gi) {
    // group elements: lane handles d = gi*group + lane + 64*i
    const int per = (a.group + 63) / 64;
    float x[2];
    float lo = INFINITY, hi = -INFINITY;
    for (int i = 0; i < per; ++i) {
      const int k = lane + 64 * i;
      const int d = gi * a.group + k;
      float v = 0.0f;
      if (k < a.group) {
        v = d < a.dim ? bits_to_float(src[d], a.float_kind) : 0.0f;
        lo = fminf(lo, v);
        hi = fmaxf(hi, v);
      }
      x[i] = v;
    }
    for (int o = 1; o < 64; o <<= 1) {
      lo = fminf(lo, __shfl_xor(lo, o, 64));
      hi = fmaxf(hi, __shfl_xor(hi, o, 64));
    }
    const uint16_t b16 = f32_to_f16_bits(lo);
    const float b = f16_bits_to_f32(b16);
    const float s = fmaxf(__fdiv_rn(hi - b, levels), 1e-6f);
    const uint16_t s16 = f32_to_f16_bits(s);
    const float sf = f16_bits_to_f32(s16);
    if (lane == 0) {
      a.scale[row * ngroups + gi] = s16;
      a.bias[row * ngroups + gi] = b16;
    }
    for (int i = 0; i < per; ++i) {
      const int k = lane + 64 * i;
      float c = rintf(__fdiv_rn(x[i] - b, sf));
      c = fminf(fmaxf(c, 0.0f), levels);
      const int code = (int)c;
      const int d = gi * a.group + k;
      if (a.bits == 8) {
        if (k < a.group) a.codes[row * qbytes + d] = (uint8_t)code;
      } else {
        const int high = __shfl_down(code, 1, 64);
        if (k < a.group && (k & 1) == 0)
          a.codes[row * qbytes + d / 2] = (uint8_t)((code & 15) | ((high & 15) << 4));
      }
    }
  }
}

__global__ __launch_bounds__(256) void dequantize_rows_kernel(const DequantRowsArgs a) {
  const int padded = (a.dim + a.group - 1) / a.group * a.group;
  const int ngroups = padded / a.group;
  const int qbytes = a.bits == 4 ? padded / 2 : padded;
  const int64_t total = a.rows * a.dim;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / a.dim;
    const int d = (int)(i % a.dim);
    int code;
    if (a.bits == 8) {
      code = a.codes[row * qbytes + d];
    } else {
      code = (a.codes[row * qbytes + d / 2] >> (4 * (d & 1))) & 15;
    }
    const int gi = d / a.group;
    const float s = f16_bits_to_f32(a.scale[row * ngroups + gi]);
    const float b = f16_bits_to_f32(a.bias[row * ngroups + gi]);
    a.out[i] = (float)code * s + b;
  }
}

hipError_t launch_quantize_rows(hipStream_t stream, const QuantRowsArgs &a) {
  if (a.rows == 0) return hipSuccess;
  hipLaunchKernelGGL(quantize_rows_kernel, dim3((unsigned)((a.rows + 3) / 4)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_dequantize_rows(hipStream_t stream, const DequantRowsArgs &a) {
  const int64_t total = a.rows * a.dim;
  if (total == 0) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(dequantize_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace pkv
