// pkv_mfma.h -- MFMA operand plumbing shared by the paged attention kernels
// (gfx950): tile geometry, lane payload/metadata loads, code->f16 operand
// conversion and the f16/bf16 MFMA wrappers.
//
// A 16-token tile of K (or V) stores lane l's MFMA operand bytes at
// tile + c*1024 + l*16 (16-byte chunks).  Codes become f16 operands as
// 1024 + c: two u8 codes per v_perm against the 0x64 exponent byte, two 4-bit
// codes per mask-and-or.  The K scale and bias are applied to the score tile
// after the MFMA, the V scale is folded into the P operand.
#pragma once
#include "pkv_launch.h"

namespace pkv {

constexpr float kTau = 8.0f;  // lazy-rescale threshold (log2 units)

__device__ __forceinline__ uint32_t perm(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

// Two u8 codes -> f16 pair (1024 + c0, 1024 + c1): bytes 0,1 (sel_lo) or 2,3 (sel_hi).
constexpr uint32_t kMagic = 0x64646464u;
constexpr uint32_t kSelLo = 0x00050004u;
constexpr uint32_t kSelHi = 0x00070006u;

template <int BITS, int DP, int G, int RB, int FK, int SLOTS>
struct Cfg {
  static constexpr bool QUANT = BITS != 16;
  static constexpr int NG = QUANT ? DP / G : 1;
  static constexpr int KB = DP / 32;
  static constexpr int NB = DP / 16;
  static constexpr int RPS = 16 / SLOTS;  // query rows (columns) per slot
  static constexpr int LB = DP * BITS / 32;  // payload bytes per lane and side
  static constexpr int LW = LB / 4;
  static constexpr int CS = LB < 16 ? LB : 16;
  static constexpr int NCH = LB / CS;
  static constexpr int MW = QUANT ? 4 * NG : 4;  // meta dwords per lane (4 tokens x NG)
  static_assert(SLOTS == 1 || RB == 1, "column slots need a single row block");
  static_assert(CS == 16 || (CS == 8 && NCH == 1), "payload chunk");
};

// A lane's K or V payload of one tile, straight from HBM.
// NT: non-temporal loads (streamed once: the decode kernels, whose pages are
// read by one wave each); the prefill kernel's row blocks share a span's
// tiles through L2 and load them plainly.
template <typename C, bool NT = false>
__device__ __forceinline__ void load_payload(uint32_t (&w)[C::LW], const uint8_t *tile, int lane) {
  if constexpr (C::CS == 16) {
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) {
      const u4 *src = (const u4 *)(tile + c * 1024 + lane * 16);
      const u4 x = NT ? __builtin_nontemporal_load(src) : *src;
      w[4 * c] = x.x; w[4 * c + 1] = x.y; w[4 * c + 2] = x.z; w[4 * c + 3] = x.w;
    }
  } else {
    const u2 *src = (const u2 *)(tile + lane * 8);
    const u2 x = NT ? __builtin_nontemporal_load(src) : *src;
    w[0] = x.x; w[1] = x.y;
  }
}

// The metadata words (all groups) of a lane's four tokens: 4*NG contiguous dwords.
template <typename C, bool NT = false>
__device__ __forceinline__ void load_meta(uint32_t (&mw)[C::MW], const uint8_t *p) {
#pragma unroll
  for (int i = 0; i < C::MW; i += 4) {
    const u4 *src = (const u4 *)(p + i * 4);
    const u4 x = NT ? __builtin_nontemporal_load(src) : *src;
    mw[i] = x.x; mw[i + 1] = x.y; mw[i + 2] = x.z; mw[i + 3] = x.w;
  }
}

template <int BITS>
struct Conv;

// bf16 pair of the codes in bytes i0 (low half) and i1 (high half) of w: a
// code c <= 255 converts to f32 exactly (v_cvt_f32_ubyte), and its upper 16
// bits are c as bf16, exact since c has at most 8 significant bits.
__device__ __forceinline__ uint32_t bf16_pair(uint32_t w, int i0, int i1) {
  const float f0 = (float)((w >> (8 * i0)) & 0xFFu), f1 = (float)((w >> (8 * i1)) & 0xFFu);
  return perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
}

template <>
struct Conv<8> {
  template <int LW>
  static __device__ __forceinline__ h8 kop(const uint32_t (&w)[LW], int kb) {
    const uint32_t w0 = w[2 * kb], w1 = w[2 * kb + 1];
    u4 r = {perm(w0, kMagic, kSelLo), perm(w0, kMagic, kSelHi), perm(w1, kMagic, kSelLo),
            perm(w1, kMagic, kSelHi)};
    return __builtin_bit_cast(h8, r);
  }
  template <int LW>
  static __device__ __forceinline__ h4 vop(const uint32_t (&w)[LW], int n) {
    const uint32_t w0 = w[n];
    u2 r = {perm(w0, kMagic, kSelLo), perm(w0, kMagic, kSelHi)};
    return __builtin_bit_cast(h4, r);
  }
  // The codes of kop (same element order) as bf16 values c.
  template <int LW>
  static __device__ __forceinline__ u4 kop_bf16(const uint32_t (&w)[LW], int kb) {
    const uint32_t w0 = w[2 * kb], w1 = w[2 * kb + 1];
    return u4{bf16_pair(w0, 0, 1), bf16_pair(w0, 2, 3), bf16_pair(w1, 0, 1), bf16_pair(w1, 2, 3)};
  }
};

// 4-bit codes: f16 pair s of a word x holds nibbles s and s + 4, i.e. the
// value ((x >> 4s) & 0x000F000F) | 0x64006400.  The even nibbles
// (x & 0x0F0F0F0F) and the odd ones ((x >> 4) & 0x0F0F0F0F) each sit one per
// byte, so one v_perm per pair places two of them beside the exponent byte:
// seven instructions per word instead of eleven.
constexpr uint32_t kNibLo = 0x00060004u;  // bytes 0 and 2 of the nibble word
constexpr uint32_t kNibHi = 0x00070005u;  // bytes 1 and 3

template <>
struct Conv<4> {
  template <int LW>
  static __device__ __forceinline__ h8 kop(const uint32_t (&w)[LW], int kb) {
    const uint32_t x = w[kb];
    const uint32_t ev = x & 0x0F0F0F0Fu, od = (x >> 4) & 0x0F0F0F0Fu;
    u4 r = {perm(ev, kMagic, kNibLo), perm(od, kMagic, kNibLo), perm(ev, kMagic, kNibHi),
            perm(od, kMagic, kNibHi)};
    return __builtin_bit_cast(h8, r);
  }
  template <int LW>
  static __device__ __forceinline__ h4 vop(const uint32_t (&w)[LW], int n) {
    const uint32_t x = w[n >> 1];
    // pairs (0, 2) from the even nibbles, (1, 3) from the odd ones
    const uint32_t nb = (n & 1) ? (x >> 4) & 0x0F0F0F0Fu : x & 0x0F0F0F0Fu;
    u2 r = {perm(nb, kMagic, kNibLo), perm(nb, kMagic, kNibHi)};
    return __builtin_bit_cast(h4, r);
  }
  // The codes of kop (same element order: nibbles 0, 4, 1, 5, 2, 6, 3, 7)
  // as bf16 values c.
  template <int LW>
  static __device__ __forceinline__ u4 kop_bf16(const uint32_t (&w)[LW], int kb) {
    const uint32_t x = w[kb];
    const uint32_t ev = x & 0x0F0F0F0Fu, od = (x >> 4) & 0x0F0F0F0Fu;
    return u4{bf16_pair(ev, 0, 2), bf16_pair(od, 0, 2), bf16_pair(ev, 1, 3), bf16_pair(od, 1, 3)};
  }
};

template <int FK>
struct FloatOps;

template <>
struct FloatOps<1> {  // f16 operands (f16 pages, and codes of quantized pages)
  typedef h8 KT;
  typedef h4 VT;
  static __device__ __forceinline__ f4 qk(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f4 pv(h4 a, h4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ h4 pack_p(float p0, float p1, float p2, float p3) {
    return h4{(_Float16)p0, (_Float16)p1, (_Float16)p2, (_Float16)p3};
  }
};

template <>
struct FloatOps<0> {  // bf16 pages
  typedef b8 KT;
  typedef s4 VT;
  static __device__ __forceinline__ f4 qk(b8 a, b8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f4 pv(s4 a, s4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ s4 pack_p(float p0, float p1, float p2, float p3) {
    return s4{(short)f32_to_bf16_bits(p0), (short)f32_to_bf16_bits(p1),
              (short)f32_to_bf16_bits(p2), (short)f32_to_bf16_bits(p3)};
  }
  // The rounding error of pack_p, itself rounded to bf16: P = hi + lo carries
  // 16 significant bits (p - hi is exact in f32).
  static __device__ __forceinline__ s4 pack_lo(float p0, float p1, float p2, float p3, s4 hi) {
    auto up = [](short h) { return __uint_as_float((uint32_t)(uint16_t)h << 16); };
    return pack_p(p0 - up(hi[0]), p1 - up(hi[1]), p2 - up(hi[2]), p3 - up(hi[3]));
  }
};


}  // namespace pkv
