// pkv_attention.hip -- paged decode / verify attention for gfx950.
//
// Semantics are the reference's (src/mlx_one/engine/paged_attention.py:62-113
// kernel, :127-206 dispatch and merge): query row (q, h) attends tokens
// t <= q_pos[q] of its sequence, KV head kh = h / (H/HK), softmax(q.k*scale).v,
// normaliser floored at 1e-20, rows q >= width give 0.
//
// Work unit = one wave = (sequence, partition of split_tokens, KV head).  All
// R = Q*(H/HK) query rows of the KV head share each K/V tile load (GQA reuse).
// Per 16-token tile:
//   S^T[t][row] = K.Q^T    v_mfma_f32_16x16x32_f16 over the codes as f16
//                          (1024 + c, built with one v_perm per two codes);
//                          one accumulator per quantization group, then
//                          s = sum_g scale_g*acc_g + qsum_g*(bias_g - 1024*scale_g)
//   softmax                exp2 domain, online with lazy rescaling: the running
//                          max moves only when a score exceeds it by > 8
//   O[row][d] += P'.V      v_mfma_f32_16x16x16_f16, P'_g = p*scale_v[g] (so V is
//                          never dequantized); bias_v enters as sum p*bias_v and
//                          the 1024 offset as 1024 * (P'.ones)
// Float (bf16/f16) pages use the same schedule without the affine terms.
// A unit that covers its whole sequence writes the normalised output; other
// units write (acc, m, l) partials merged by merge_kernel.
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

template <int BITS, int DP, int G, int RB, int FK>
struct Cfg {
  static constexpr bool QUANT = BITS != 16;
  static constexpr int NG = QUANT ? DP / G : 1;
  static constexpr int KB = DP / 32;
  static constexpr int NB = DP / 16;
  static constexpr int LB = DP * BITS / 32;
  static constexpr int LW = LB / 4;
  static constexpr int CS = LB < 16 ? LB : 16;
  static constexpr int NCH = LB / CS;
  static constexpr int MW = QUANT ? 4 * NG : 1;  // meta dwords per lane (4 tokens x NG)
  // LDS ring slot of one tile: [K payload][V payload][K meta][V meta]
  static constexpr int KP = LB * 64;
  static constexpr int META = QUANT ? 128 * NG : 0;
  static constexpr int SLOT = 2 * KP + META;
  // tiles per wave ring (NBUF - 1 in flight): about 13 KB of LDS per wave, so
  // three 4-wave workgroups fit a CU's 160 KB
  static constexpr int NBUF_RAW = 13312 / SLOT;
  static constexpr int NBUF = NBUF_RAW < 2 ? 2 : NBUF_RAW > 8 ? 8 : NBUF_RAW;
  // LDS-DMA instructions per tile (each decrements vmcnt once)
  static constexpr int PAY_INSTS = CS == 16 ? NCH : 2;
  static constexpr int META_INSTS = QUANT ? (32 * NG + 63) / 64 : 0;
  static constexpr int LPT = 2 * PAY_INSTS + META_INSTS;
  static_assert((NBUF - 1) * LPT <= 63, "vmcnt range");
};

template <typename C>
struct Tile {
  uint32_t k[C::LW];
  uint32_t v[C::LW];
  uint32_t km[C::MW];
  uint32_t vm[C::MW];
};

typedef __attribute__((address_space(3))) void lds_void;

// Global -> LDS DMA of one 16- or 4-byte piece per lane: lane l's data lands
// at dst + l*size (dst is wave-uniform).
__device__ __forceinline__ void dma16(const void *src, uint8_t *dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void *)dst, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void *src, uint8_t *dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void *)dst, 4, 0, 0);
}

// s_waitcnt immediate (gfx9 encoding) waiting for vmcnt <= VM only.
template <int VM>
__device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | (15 << 8) | ((VM >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Wait until the tile that has `younger` tiles issued after it has landed
// (DMA groups complete in issue order).
template <typename C, int K>
__device__ __forceinline__ void wait_tile_rec(int younger) {
  if constexpr (K == 0) {
    wait_vm<0>();
  } else {
    if (younger >= K) wait_vm<K * C::LPT>();
    else wait_tile_rec<C, K - 1>(younger);
  }
}
template <typename C>
__device__ __forceinline__ void wait_tile(int younger) {
  wait_tile_rec<C, C::NBUF - 1>(younger);
}

// Issue the LDS-DMA of one 16-token tile (payload chunks + metadata words).
template <typename C>
__device__ __forceinline__ void issue_tile(uint8_t *slot, const AttnArgs &a, const uint8_t *head,
                                           int tile_in_page, int lane) {
  const int64_t off = (int64_t)tile_in_page * a.g.tile_bytes;
  const uint8_t *kt = head + off, *vt = head + a.g.v_offset + off;
  if constexpr (C::CS == 16) {
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) dma16(kt + c * 1024 + lane * 16, slot + c * 1024);
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) dma16(vt + c * 1024 + lane * 16, slot + C::KP + c * 1024);
  } else {
    dma4(kt + lane * 8, slot);
    dma4(kt + lane * 8 + 4, slot + 256);
    dma4(vt + lane * 8, slot + C::KP);
    dma4(vt + lane * 8 + 4, slot + C::KP + 256);
  }
  if constexpr (C::QUANT) {
    const int base = tile_in_page * PKV_TILE * C::NG;
#pragma unroll
    for (int m = 0; m < 32 * C::NG; m += 64) {
      const int idx = m + lane;
      if (idx < 32 * C::NG) {
        const uint8_t *src = idx < 16 * C::NG
                                 ? head + a.g.kmeta_offset + (int64_t)(base + idx) * 4
                                 : head + a.g.vmeta_offset + (int64_t)(base + idx - 16 * C::NG) * 4;
        dma4(src, slot + 2 * C::KP + m * 4);
      }
    }
  }
}

// Registers of one tile from its LDS slot: lane payload and the lane's 4 tokens' meta.
template <typename C>
__device__ __forceinline__ void read_tile(Tile<C> &t, const uint8_t *slot, int lane, int jj) {
  if constexpr (C::CS == 16) {
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) {
      const u4 x = *(const u4 *)(slot + c * 1024 + lane * 16);
      const u4 y = *(const u4 *)(slot + C::KP + c * 1024 + lane * 16);
      t.k[4 * c] = x.x; t.k[4 * c + 1] = x.y; t.k[4 * c + 2] = x.z; t.k[4 * c + 3] = x.w;
      t.v[4 * c] = y.x; t.v[4 * c + 1] = y.y; t.v[4 * c + 2] = y.z; t.v[4 * c + 3] = y.w;
    }
  } else {
    t.k[0] = *(const uint32_t *)(slot + lane * 4);
    t.k[1] = *(const uint32_t *)(slot + 256 + lane * 4);
    t.v[0] = *(const uint32_t *)(slot + C::KP + lane * 4);
    t.v[1] = *(const uint32_t *)(slot + C::KP + 256 + lane * 4);
  }
  if constexpr (C::QUANT) {
    const uint32_t *km = (const uint32_t *)(slot + 2 * C::KP) + 4 * jj * C::NG;
    const uint32_t *vm = km + 16 * C::NG;
#pragma unroll
    for (int i = 0; i < C::MW; i += 4) {
      const u4 x = *(const u4 *)(km + i);
      const u4 y = *(const u4 *)(vm + i);
      t.km[i] = x.x; t.km[i + 1] = x.y; t.km[i + 2] = x.z; t.km[i + 3] = x.w;
      t.vm[i] = y.x; t.vm[i + 1] = y.y; t.vm[i + 2] = y.z; t.vm[i + 3] = y.w;
    }
  }
}

template <int BITS>
struct Conv;

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
};

__device__ __forceinline__ uint32_t nib_pair(uint32_t w, int s) {
  return ((w >> (4 * s)) & 0x000F000Fu) | 0x64006400u;
}

template <>
struct Conv<4> {
  template <int LW>
  static __device__ __forceinline__ h8 kop(const uint32_t (&w)[LW], int kb) {
    const uint32_t x = w[kb];
    u4 r = {nib_pair(x, 0), nib_pair(x, 1), nib_pair(x, 2), nib_pair(x, 3)};
    return __builtin_bit_cast(h8, r);
  }
  template <int LW>
  static __device__ __forceinline__ h4 vop(const uint32_t (&w)[LW], int n) {
    const uint32_t x = w[n >> 1];
    const int o = n & 1;
    u2 r = {nib_pair(x, o), nib_pair(x, 2 + o)};
    return __builtin_bit_cast(h4, r);
  }
};

template <int FK>
struct FloatOps;

template <>
struct FloatOps<1> {  // f16 pages
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
  static __device__ __forceinline__ uint16_t from_float(float x) { return f32_to_f16_bits(x); }
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
  static __device__ __forceinline__ uint16_t from_float(float x) { return f32_to_bf16_bits(x); }
};

template <int BITS, int DP, int G, int RB, int FK>
__global__ __launch_bounds__(256) void attn_kernel(const AttnArgs a) {
  using C = Cfg<BITS, DP, G, RB, FK>;
  constexpr bool QUANT = C::QUANT;
  constexpr int NG = C::NG, KB = C::KB, NB = C::NB;
  // MFMA operand types: quantized pages run in f16 (codes as 1024 + c).
  using FO = FloatOps<QUANT ? 1 : FK>;
  using KT = typename FO::KT;
  using VT = typename FO::VT;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, jj = lane >> 4;
  const int w = blockIdx.x * 4 + wave;
  if (w >= a.max_units) return;
  const Geo &g = a.g;
  const int kh = w % g.hk, su = w / g.hk;
  int b, part, nsplit, first_unit;
  if (!locate_unit(a.seq_lens, a.batch, a.split, su, lane, b, part, nsplit, first_unit)) return;
  // wave-uniform values live in SGPRs: scalar branches, scalar loads
  b = __builtin_amdgcn_readfirstlane(b);
  part = __builtin_amdgcn_readfirstlane(part);
  nsplit = __builtin_amdgcn_readfirstlane(nsplit);
  const int L = a.seq_lens[b];
  const int t0 = part * a.split;
  const int t1 = min(L, t0 + a.split);
  const int width = a.widths ? a.widths[b] : a.nq;

  // ---- query rows: row = rb*16 + col -> (q = row / gqa, h = kh*gqa + row % gqa)
  int lim[RB];
  KT qop[RB][KB];
  float qs[RB][NG];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = rb * 16 + col;
    const int qi = row / a.gqa, h = kh * a.gqa + row % a.gqa;
    const bool live = row < a.rows && qi < width;
    int qp = -1;
    if (live) qp = a.q_pos ? a.q_pos[(int64_t)b * a.nq + qi] : L - width + qi;
    lim[rb] = live ? min(qp, t1 - 1) : -1;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) qs[rb][gi] = 0.0f;
    const uint16_t *qrow = a.q + (((int64_t)b * a.heads + h) * a.nq + qi) * g.dim;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int d0 = 32 * kb + 8 * jj;
      uint16_t raw[8];
      if (row < a.rows && (g.dim & 7) == 0 && d0 + 8 <= g.dim) {
        u4 x = *(const u4 *)(qrow + d0);
        raw[0] = x.x & 0xFFFF; raw[1] = x.x >> 16; raw[2] = x.y & 0xFFFF; raw[3] = x.y >> 16;
        raw[4] = x.z & 0xFFFF; raw[5] = x.z >> 16; raw[6] = x.w & 0xFFFF; raw[7] = x.w >> 16;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) raw[e] = (row < a.rows && d0 + e < g.dim) ? qrow[d0 + e] : 0;
      }
      if constexpr (QUANT || FK == 1) {
        h8 v;
        float sum = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const _Float16 hv = (_Float16)bits_to_float(raw[e], g.float_kind);
          v[e] = hv;
          sum += (float)hv;
        }
        if constexpr (QUANT) qs[rb][(32 * kb) / G] += sum;
        if constexpr (FK == 1 || QUANT) qop[rb][kb] = __builtin_bit_cast(KT, v);
      } else {
        u4 packed = {(uint32_t)raw[0] | ((uint32_t)raw[1] << 16), (uint32_t)raw[2] | ((uint32_t)raw[3] << 16),
                     (uint32_t)raw[4] | ((uint32_t)raw[5] << 16), (uint32_t)raw[6] | ((uint32_t)raw[7] << 16)};
        qop[rb][kb] = __builtin_bit_cast(KT, packed);
      }
    }
    if constexpr (QUANT) {
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        qs[rb][gi] += __shfl_xor(qs[rb][gi], 16, 64);
        qs[rb][gi] += __shfl_xor(qs[rb][gi], 32, 64);
      }
    }
  }

  // ---- state
  float m[RB], lsum[RB], corr[RB][NG];
  f4 O[RB][NB], ones_acc[RB][NG];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m[rb] = -INFINITY;
    lsum[rb] = 0.0f;
#pragma unroll
    for (int n = 0; n < NB; ++n) O[rb][n] = f4{0, 0, 0, 0};
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) { corr[rb][gi] = 0.0f; ones_acc[rb][gi] = f4{0, 0, 0, 0}; }
  }

  // page ids of this partition (split <= 64 pages)
  const int first_page = t0 / g.page;
  const int npages = t1 > t0 ? (t1 - 1) / g.page - first_page + 1 : 0;
  int pid = 0;
  if (lane < npages && first_page + lane < a.max_pages) {
    pid = a.table[(int64_t)b * a.max_pages + first_page + lane];
    if (pid < 0 || pid >= a.num_pages) pid = -1;
  } else if (lane < npages) {
    pid = -1;
  }
  // partitions start on page boundaries: tile -> (page, tile in page) by shifts
  const int tpp_shift = __builtin_ctz(g.page / PKV_TILE);
  const int ntiles = t1 > t0 ? (t1 - t0 + PKV_TILE - 1) / PKV_TILE : 0;

  auto head_of = [&](int tile, int &tip) -> const uint8_t * {
    tip = tile & ((1 << tpp_shift) - 1);
    const int id = __builtin_amdgcn_readlane(pid, tile >> tpp_shift);
    if (id < 0) return nullptr;
    return a.pool + (int64_t)id * g.page_bytes + (int64_t)kh * g.head_bytes;
  };

  const h4 ones = h4{(_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f};

  // Tile body; `cur` holds the tile's payload and metadata registers.
  auto process = [&](const Tile<C> &cur, int tile) __attribute__((always_inline)) {
    {
      const int tok0 = t0 + tile * PKV_TILE;
      // ---- S^T = K.Q^T
      f4 acc[RB][NG];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) acc[rb][gi] = f4{0, 0, 0, 0};
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        KT kop;
        if constexpr (QUANT) {
          kop = Conv<BITS>::template kop<C::LW>(cur.k, kb);
        } else {
          u4 r = {cur.k[4 * kb], cur.k[4 * kb + 1], cur.k[4 * kb + 2], cur.k[4 * kb + 3]};
          kop = __builtin_bit_cast(KT, r);
        }
        const int gi = QUANT ? (32 * kb) / G : 0;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[rb][gi] = FO::qk(kop, qop[rb][kb], acc[rb][gi]);
      }
      // ---- scores (exp2 domain)
      float s[RB][4];
      float ksf[4][NG], kbf[4][NG];
      if constexpr (QUANT) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int gi = 0; gi < NG; ++gi) {
            const uint32_t word = cur.km[r * NG + gi];
            ksf[r][gi] = f16_bits_to_f32(word);
            kbf[r][gi] = f16_bits_to_f32(word >> 16) - 1024.0f * ksf[r][gi];
          }
      }
      bool need = false;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v;
          if constexpr (QUANT) {
            v = 0.0f;
#pragma unroll
            for (int gi = 0; gi < NG; ++gi) v += ksf[r][gi] * acc[rb][gi][r] + qs[rb][gi] * kbf[r][gi];
          } else {
            v = acc[rb][0][r];
          }
          const int t = tok0 + 4 * jj + r;
          v = t <= lim[rb] ? v * a.scale_log2 : -INFINITY;
          s[rb][r] = v;
          need |= v > m[rb] + kTau;
        }
      }
      if (__any(need)) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          float tm = fmaxf(fmaxf(s[rb][0], s[rb][1]), fmaxf(s[rb][2], s[rb][3]));
          tm = fmaxf(tm, __shfl_xor(tm, 16, 64));
          tm = fmaxf(tm, __shfl_xor(tm, 32, 64));
          const float mn = fmaxf(m[rb], tm);
          const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m[rb] - mn);
          m[rb] = mn;
          lsum[rb] *= alpha;
#pragma unroll
          for (int gi = 0; gi < NG; ++gi) corr[rb][gi] *= alpha;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float ar = __shfl(alpha, 4 * jj + r, 64);
#pragma unroll
            for (int n = 0; n < NB; ++n) O[rb][n][r] *= ar;
#pragma unroll
            for (int gi = 0; gi < NG; ++gi) ones_acc[rb][gi][r] *= ar;
          }
        }
      }
      // ---- probabilities and O += P'.V
      float p[RB][4];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = tok0 + 4 * jj + r;
          p[rb][r] = t <= lim[rb] ? __builtin_amdgcn_exp2f(s[rb][r] - m[rb]) : 0.0f;
        }
        lsum[rb] += (p[rb][0] + p[rb][1]) + (p[rb][2] + p[rb][3]);
      }
      if constexpr (QUANT) {
        float vsf[4][NG], vbf[4][NG];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int gi = 0; gi < NG; ++gi) {
            const uint32_t word = cur.vm[r * NG + gi];
            vsf[r][gi] = f16_bits_to_f32(word);
            vbf[r][gi] = f16_bits_to_f32(word >> 16);
          }
        h4 pv[RB][NG];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int gi = 0; gi < NG; ++gi) {
            pv[rb][gi] = h4{(_Float16)(p[rb][0] * vsf[0][gi]), (_Float16)(p[rb][1] * vsf[1][gi]),
                            (_Float16)(p[rb][2] * vsf[2][gi]), (_Float16)(p[rb][3] * vsf[3][gi])};
            corr[rb][gi] += (p[rb][0] * vbf[0][gi] + p[rb][1] * vbf[1][gi]) +
                            (p[rb][2] * vbf[2][gi] + p[rb][3] * vbf[3][gi]);
          }
#pragma unroll
        for (int n = 0; n < NB; ++n) {
          const h4 vop = Conv<BITS>::template vop<C::LW>(cur.v, n);
          const int gi = (16 * n) / G;
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) O[rb][n] = FO::pv(pv[rb][gi], vop, O[rb][n]);
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int gi = 0; gi < NG; ++gi) ones_acc[rb][gi] = FO::pv(pv[rb][gi], ones, ones_acc[rb][gi]);
      } else {
        VT pv[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) pv[rb] = FO::pack_p(p[rb][0], p[rb][1], p[rb][2], p[rb][3]);
#pragma unroll
        for (int n = 0; n < NB; ++n) {
          u2 r = {cur.v[2 * n], cur.v[2 * n + 1]};
          const VT vop = __builtin_bit_cast(VT, r);
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) O[rb][n] = FO::pv(pv[rb], vop, O[rb][n]);
        }
      }
    }
  };

  // LDS ring of NBUF tile slots per wave, filled by DMA NBUF - 1 tiles ahead.
  __shared__ __attribute__((aligned(16))) uint8_t ring[4][C::NBUF][C::SLOT];
  uint8_t(*slots)[C::SLOT] = ring[wave];
  int valid = 0;  // bit s: slot s holds a tile of a valid page
  auto issue = [&](int tile) __attribute__((always_inline)) {
    int tip;
    const uint8_t *h = head_of(tile, tip);
    const int s = tile % C::NBUF;
    if (h) {
      valid |= 1 << s;
    } else {
      // keep one DMA group per tile so vmcnt accounting stays exact
      valid &= ~(1 << s);
      h = a.pool + (int64_t)kh * g.head_bytes;
      tip = 0;
    }
    issue_tile<C>(slots[s], a, h, tip, lane);
  };
#pragma unroll
  for (int p = 0; p < C::NBUF - 1; ++p)
    if (p < ntiles) issue(p);
  for (int tile = 0; tile < ntiles; ++tile) {
    // refill the slot tile-1 used; its LDS reads have completed
    wait_lgkm0();
    __builtin_amdgcn_sched_barrier(0);
    if (tile + C::NBUF - 1 < ntiles) issue(tile + C::NBUF - 1);
    wait_tile<C>(min(ntiles - 1 - tile, C::NBUF - 1));
    __builtin_amdgcn_sched_barrier(0);
    const int s = tile % C::NBUF;
    if (valid & (1 << s)) {
      Tile<C> cur;
      read_tile<C>(cur, slots[s], lane, jj);
      process(cur, tile);
    }
  }

  // ---- epilogue: reduce l and the V-bias sums over the 4 token lanes of a row
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    lsum[rb] += __shfl_xor(lsum[rb], 16, 64);
    lsum[rb] += __shfl_xor(lsum[rb], 32, 64);
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      corr[rb][gi] += __shfl_xor(corr[rb][gi], 16, 64);
      corr[rb][gi] += __shfl_xor(corr[rb][gi], 32, 64);
    }
  }
  const bool direct = nsplit == 1;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int src = 4 * jj + r;  // lane holding row (rb*16 + src) in the score layout
      const float mr = __shfl(m[rb], src, 64);
      const float lr = __shfl(lsum[rb], src, 64);
      float cr[NG];
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) cr[gi] = __shfl(corr[rb][gi], src, 64);
      const int row = rb * 16 + src;
      if (row >= a.rows) continue;
      const int qi = row / a.gqa, h = kh * a.gqa + row % a.gqa;
      const float inv = 1.0f / fmaxf(lr, 1e-20f);
      const int64_t obase = (((int64_t)b * a.heads + h) * a.nq + qi) * g.dim;
      const int64_t pbase = ((int64_t)w * a.rows + row) * DP;
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        const int d = 16 * n + col;
        float val = O[rb][n][r];
        if constexpr (QUANT) {
          const int gi = (16 * n) / G;
          val += cr[gi] - 1024.0f * ones_acc[rb][gi][r];
        }
        if (direct) {
          if (d < g.dim) a.out[obase + d] = float_to_bits(val * inv, g.float_kind);
        } else {
          a.part_acc[pbase + d] = val;
        }
      }
      if (!direct && col == 0) {
        a.part_ml[((int64_t)w * a.rows + row) * 2] = mr;
        a.part_ml[((int64_t)w * a.rows + row) * 2 + 1] = lr;
      }
    }
  }
}

// Log-sum-exp merge of partition partials (paged_attention.py:191-204, exp2
// domain): one wave per (sequence, KV head).

__global__ __launch_bounds__(256) void merge_kernel(const MergeArgs a) {
  // one wave per (sequence, KV head, query row)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t w = (int64_t)blockIdx.x * 4 + wave;
  if (w >= (int64_t)a.batch * a.hk * a.rows) return;
  const int row = (int)(w % a.rows);
  const int kh = (int)((w / a.rows) % a.hk);
  const int b = (int)(w / ((int64_t)a.rows * a.hk));
  const int nsplit = splits_of(a.seq_lens[b], a.split);
  if (nsplit <= 1) return;
  // first unit of sequence b: prefix sum of the partition counts
  int carry = 0, first = 0;
  for (int c0 = 0; c0 < a.batch; c0 += 64) {
    const int idx = c0 + lane;
    const int ns = idx < a.batch ? splits_of(a.seq_lens[idx], a.split) : 0;
    const int incl = wave_scan_incl(ns, lane) + carry;
    if (b >= c0 && b < c0 + 64) first = __shfl(incl - ns, b - c0, 64);
    carry = __shfl(incl, 63, 64);
  }
  // partitions past the launched units were never computed: never read them
  if (first + nsplit > a.max_units) return;
  const int qi = row / a.gqa, h = kh * a.gqa + row % a.gqa;
  auto unit = [&](int s) { return ((int64_t)(first + s) * a.hk + kh) * a.rows + row; };
  // global max over live partitions (lanes stride the partitions)
  __shared__ float s_w[4][64];
  float top = -INFINITY;
  for (int s = lane; s < nsplit; s += 64) {
    const float ms = a.part_ml[unit(s) * 2], ls = a.part_ml[unit(s) * 2 + 1];
    if (ls > 0.0f) top = fmaxf(top, ms);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) top = fmaxf(top, __shfl_xor(top, o, 64));
  float norm = 0.0f;
  float acc[4] = {0, 0, 0, 0};
  const int per_lane = (a.dp + 63) / 64;
  for (int s0 = 0; s0 < nsplit; s0 += 64) {
    const int s = s0 + lane;
    float wgt = 0.0f, ls = 0.0f;
    if (s < nsplit) {
      const float ms = a.part_ml[unit(s) * 2];
      ls = a.part_ml[unit(s) * 2 + 1];
      wgt = ls > 0.0f ? exp2f(ms - top) : 0.0f;  // dead partitions hold acc = 0
    }
    norm += wgt * ls;
    s_w[wave][lane] = wgt;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int count = min(64, nsplit - s0);
    // independent loads: each lane owns per_lane consecutive d of every partition
    int j = 0;
    for (; j + 4 <= count; j += 4) {
      float v[4][4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float *pa = a.part_acc + unit(s0 + j + u) * a.dp;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[u][i] = i < per_lane ? pa[lane * per_lane + i] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float wj = s_w[wave][j + u];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] += wj * v[u][i];
      }
    }
    for (; j < count; ++j) {
      const float *pa = a.part_acc + unit(s0 + j) * a.dp;
      const float wj = s_w[wave][j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i < per_lane) acc[i] += wj * pa[lane * per_lane + i];
    }
    __builtin_amdgcn_wave_barrier();
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) norm += __shfl_xor(norm, o, 64);
  const float inv = 1.0f / fmaxf(norm, 1e-20f);
  const int64_t obase = (((int64_t)b * a.heads + h) * a.nq + qi) * a.dim;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane * per_lane + i;
    if (i < per_lane && d < a.dim) a.out[obase + d] = float_to_bits(acc[i] * inv, a.float_kind);
  }
}

// ---- host launcher ------------------------------------------------------------

template <int BITS, int DP, int G, int RB, int FK>
static hipError_t launch_one(hipStream_t stream, const AttnArgs &a) {
  dim3 grid((unsigned)((a.max_units + 3) / 4)), block(256);
  hipLaunchKernelGGL((attn_kernel<BITS, DP, G, RB, FK>), grid, block, 0, stream, a);
  return hipGetLastError();
}

template <int RB>
static hipError_t dispatch_rb(hipStream_t stream, const AttnArgs &a) {
  const Geo &g = a.g;
#define PKV_Q(BITS_, DP_, G_)                                                        \
  if (g.bits == BITS_ && g.dp == DP_ && g.group == G_)                               \
    return launch_one<BITS_, DP_, G_, RB, 1>(stream, a);
  PKV_Q(8, 64, 32) PKV_Q(8, 64, 64)
  PKV_Q(8, 128, 32) PKV_Q(8, 128, 64) PKV_Q(8, 128, 128)
  PKV_Q(8, 256, 32) PKV_Q(8, 256, 64) PKV_Q(8, 256, 128)
  PKV_Q(4, 64, 32) PKV_Q(4, 64, 64)
  PKV_Q(4, 128, 32) PKV_Q(4, 128, 64) PKV_Q(4, 128, 128)
  PKV_Q(4, 256, 32) PKV_Q(4, 256, 64) PKV_Q(4, 256, 128)
#undef PKV_Q
#define PKV_F(DP_, FK_)                                                              \
  if (g.bits == 16 && g.dp == DP_ && g.float_kind == FK_)                            \
    return launch_one<16, DP_, 32, RB, FK_>(stream, a);
  PKV_F(64, 0) PKV_F(64, 1) PKV_F(128, 0) PKV_F(128, 1) PKV_F(256, 0) PKV_F(256, 1)
#undef PKV_F
  return hipErrorInvalidValue;
}

hipError_t launch_attention(hipStream_t stream, const AttnArgs &a, int row_blocks) {
  if (a.max_units <= 0) return hipSuccess;
  if (row_blocks == 1) return dispatch_rb<1>(stream, a);
  if (row_blocks == 2) return dispatch_rb<2>(stream, a);
  return hipErrorInvalidValue;
}

hipError_t launch_merge(hipStream_t stream, const MergeArgs &a) {
  const int64_t waves = (int64_t)a.batch * a.hk * a.rows;
  if (waves == 0) return hipSuccess;
  hipLaunchKernelGGL(merge_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace pkv
