// pkv_prefill.hip -- chunked-prefill attention over paged KV for gfx950.
//
// Same semantics as the decode kernel (src/mlx_one/engine/paged_attention.py:
// 62-113 kernel, :204 normalisation): query row (q, h) attends tokens
// t <= q_pos[q] of its sequence, KV head kh = h / (H/HK), softmax(q.k*scale).v,
// normaliser floored at 1e-20, rows q >= width give 0.  It serves query blocks
// wider than the decode kernel's 32 rows per KV head (chunked prefill: e.g.
// 512 queries x 4 heads = 2048 rows per KV head), where the contraction is
// dense and MFMA-bound.
//
// Work unit = one workgroup of 4 waves = (sequence, KV head, block of 128
// query rows); wave w owns rows 32w..32w+31 of the block as two 16-column
// MFMA row tiles.  K/V tiles of 16 tokens are staged once per workgroup in LDS
// (global_load_lds_dwordx4, 4 tiles per stage, double-buffered: each wave
// DMAs one tile of the next stage while all four compute the current one) and
// read by all four waves: every byte of KV is fetched from HBM once per 128
// query rows.  Per tile and wave: S^T = K.Q^T (v_mfma_f32_16x16x32_f16 over the
// codes as f16, per-group scale/bias applied to the score tile), online
// softmax per column (exp2, lazy rescale), O^T += V^T.P' (v_mfma_f32_16x16x16).
// Causal: stages past the block's last visible token are not loaded; tiles
// every live row sees entirely skip the per-token mask.
#include "pkv_mfma.h"

namespace pkv {

constexpr int kPrefillWaves = 4;
constexpr int kPrefillRows = kPrefillWaves * 32;  // query rows per workgroup
constexpr int kStageTiles = kPrefillWaves;       // one tile DMA'd by each wave per stage

typedef __attribute__((address_space(3))) void lds_void;

// Global -> LDS DMA of one 16- or 4-byte piece per lane: lane l's data lands
// at dst + l*size (dst is wave-uniform).
__device__ __forceinline__ void dma16(const void *src, uint8_t *dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void *)dst, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void *src, uint8_t *dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void *)dst, 4, 0, 0);
}

// Workgroup barrier once all but this wave's VM youngest vector-memory
// operations (DMAs) have landed and its LDS operations have completed (s_waitcnt gfx9 encoding:
// vmcnt VM, expcnt any, lgkmcnt 0).  No memory fence: __syncthreads() would
// also drain the DMAs of the stage in flight.
template <int VM>
__device__ __forceinline__ void stage_barrier() {
  __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | ((VM >> 4) << 14));
  asm volatile("s_barrier" ::: "memory");
}

// Page-table reads through the constant address space: uniform indices give
// scalar loads, which do not count against vmcnt.
typedef const __attribute__((address_space(4))) int32_t const_i32;

template <int BITS, int DP, int G, int FK>
__global__ __launch_bounds__(256) void prefill_kernel(const AttnArgs a) {
  constexpr int RB = 2;
  using C = Cfg<BITS, DP, G, RB, FK, 1>;
  constexpr bool QUANT = C::QUANT;
  constexpr int NG = C::NG, KB = C::KB, NB = C::NB;
  using FO = FloatOps<QUANT ? 1 : FK>;
  using KT = typename FO::KT;
  using VT = typename FO::VT;
  // LDS image of one tile: [K payload][V payload][K meta][V meta], the
  // payload in the page's own lane order
  constexpr int KP = C::LB * 64;
  constexpr int META = QUANT ? 128 * NG : 0;
  constexpr int SLOT = 2 * KP + META;
  // LDS-DMA instructions per tile (each decrements vmcnt once)
  constexpr int PAY = C::CS == 16 ? C::NCH : 2;
  constexpr int METAI = QUANT ? (32 * NG + 63) / 64 : 0;
  constexpr int LPT = 2 * PAY + METAI;
  static_assert(LPT <= 63, "vmcnt range");
  __shared__ int s_valid[2][kStageTiles];
  __shared__ int s_lim[2][kPrefillWaves];
  // two stage buffers as distinct LDS objects: reads of one carry no
  // dependence on DMAs in flight into the other
  __shared__ __attribute__((aligned(16))) uint8_t stage0[kStageTiles][SLOT];
  __shared__ __attribute__((aligned(16))) uint8_t stage1[kStageTiles][SLOT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, jj = lane >> 4;
  const Geo &g = a.g;
  const int nblk = (a.rows + kPrefillRows - 1) / kPrefillRows;
  const int seg = blockIdx.x / nblk, rblk = blockIdx.x % nblk;
  const int b = seg / g.hk, kh = seg % g.hk;
  if (b >= a.batch) return;
  const int L = a.seq_lens[b];
  const int width = a.widths ? a.widths[b] : a.nq;

  // ---- the wave's 32 query rows: row = 128*rblk + 32*wv + 16*rb + col
  int lim[RB];
  KT qv[RB][KB];
  float qs[RB][NG];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = rblk * kPrefillRows + wv * 32 + rb * 16 + col;
    const bool valid = row < a.rows;
    const int rowv = valid ? row : 0;  // rows past the block load row 0, zeroed below
    const int qi = rowv / a.gqa, h = kh * a.gqa + rowv % a.gqa;
    const bool live = valid && qi < width;
    const int pos = a.q_pos ? a.q_pos[(int64_t)b * a.nq + qi] : L - width + qi;
    lim[rb] = live ? min(pos, L - 1) : -1;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) qs[rb][gi] = 0.0f;
    const uint16_t *qrow = a.q + (((int64_t)b * a.heads + h) * a.nq + qi) * g.dim;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int d0 = 32 * kb + 8 * jj;
      uint16_t e8[8];
      if ((g.dim & 7) == 0) {
        const u4 x = *(const u4 *)(qrow + (d0 < g.dim ? d0 : 0));
        e8[0] = x.x & 0xFFFF; e8[1] = x.x >> 16; e8[2] = x.y & 0xFFFF; e8[3] = x.y >> 16;
        e8[4] = x.z & 0xFFFF; e8[5] = x.z >> 16; e8[6] = x.w & 0xFFFF; e8[7] = x.w >> 16;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) e8[e] = qrow[d0 + e < g.dim ? d0 + e : 0];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (!valid || d0 + e >= g.dim) e8[e] = 0;
      if constexpr (QUANT || FK == 1) {
        h8 v;
        float sum = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const _Float16 hv = (_Float16)bits_to_float(e8[e], g.float_kind);
          v[e] = hv;
          sum += (float)hv;
        }
        if constexpr (QUANT) qs[rb][(32 * kb) / G] += sum;
        qv[rb][kb] = __builtin_bit_cast(KT, v);
      } else {
        u4 packed = {(uint32_t)e8[0] | ((uint32_t)e8[1] << 16), (uint32_t)e8[2] | ((uint32_t)e8[3] << 16),
                     (uint32_t)e8[4] | ((uint32_t)e8[5] << 16), (uint32_t)e8[6] | ((uint32_t)e8[7] << 16)};
        qv[rb][kb] = __builtin_bit_cast(KT, packed);
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

  // ---- the block's visible span: tokens up to the largest limit; tiles
  // below the smallest live limit need no per-token mask
  {
    int hi = max(lim[0], lim[1]);
    int lo = min(lim[0] < 0 ? 0x7FFFFFFF : lim[0], lim[1] < 0 ? 0x7FFFFFFF : lim[1]);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      hi = max(hi, __shfl_xor(hi, o, 64));
      lo = min(lo, __shfl_xor(lo, o, 64));
    }
    if (lane == 0) {
      s_lim[0][wv] = hi;
      s_lim[1][wv] = lo;
    }
  }
  __syncthreads();
  int tmax = -1, tmin = 0x7FFFFFFF;
#pragma unroll
  for (int i = 0; i < kPrefillWaves; ++i) {
    tmax = max(tmax, s_lim[0][i]);
    tmin = min(tmin, s_lim[1][i]);
  }
  tmax = __builtin_amdgcn_readfirstlane(tmax);
  tmin = __builtin_amdgcn_readfirstlane(tmin);
  const int ntiles = tmax >= 0 ? tmax / PKV_TILE + 1 : 0;
  const int clear_tiles = tmin == 0x7FFFFFFF ? 0 : (tmin + 1) / PKV_TILE;  // tiles every live row sees whole
  const int nstages = (ntiles + kStageTiles - 1) / kStageTiles;
  const int tpp_shift = __builtin_ctz(g.page / PKV_TILE);
  const int tpp_mask = (1 << tpp_shift) - 1;

  // Stage s, tile s*4 + wv is DMA'd by wave wv into slot wv of stage buffer
  // s&1; absent tiles (past the span, unmapped pages) read head block kh of
  // page 0 so every wave issues the same DMA count, and are flagged invalid.
  auto issue = [&](int s, uint8_t (&stage)[kStageTiles][SLOT], int buf) __attribute__((always_inline)) {
    const int t = s * kStageTiles + wv;
    int id = 0, tip = 0, ok = 0;
    if (t < ntiles) {
      const int p = t >> tpp_shift;
      const int pid = p < a.max_pages ? ((const_i32 *)(uintptr_t)a.table)[(int64_t)b * a.max_pages + p] : -1;
      if (pid >= 0 && pid < a.num_pages) {
        id = pid;
        tip = t & tpp_mask;
        ok = 1;
      }
    }
    if (lane == 0) s_valid[buf][wv] = ok;
    const uint8_t *head = a.pool + (int64_t)id * g.page_bytes + (int64_t)kh * g.head_bytes;
    const int64_t off = (int64_t)tip * g.tile_bytes;
    const uint8_t *kt = head + off, *vt = head + g.v_offset + off;
    uint8_t *dst = stage[wv];
    if constexpr (C::CS == 16) {
#pragma unroll
      for (int c = 0; c < C::NCH; ++c) dma16(kt + c * 1024 + lane * 16, dst + c * 1024);
#pragma unroll
      for (int c = 0; c < C::NCH; ++c) dma16(vt + c * 1024 + lane * 16, dst + KP + c * 1024);
    } else {
      dma4(kt + lane * 8, dst);
      dma4(kt + lane * 8 + 4, dst + 256);
      dma4(vt + lane * 8, dst + KP);
      dma4(vt + lane * 8 + 4, dst + KP + 256);
    }
    if constexpr (QUANT) {
      const int base = tip * PKV_TILE * NG;
#pragma unroll
      for (int m = 0; m < 32 * NG; m += 64) {
        const int idx = m + lane;
        if (idx < 32 * NG) {
          const uint8_t *src = idx < 16 * NG ? head + g.kmeta_offset + (int64_t)(base + idx) * 4
                                             : head + g.vmeta_offset + (int64_t)(base + idx - 16 * NG) * 4;
          dma4(src, dst + 2 * KP + m * 4);
        }
      }
    }
  };
  // A lane's K or V payload and metadata words of a staged tile.
  auto lds_payload = [&](uint32_t (&w)[C::LW], const uint8_t *p) __attribute__((always_inline)) {
    if constexpr (C::CS == 16) {
#pragma unroll
      for (int c = 0; c < C::NCH; ++c) {
        const u4 x = *(const u4 *)(p + c * 1024 + lane * 16);
        w[4 * c] = x.x; w[4 * c + 1] = x.y; w[4 * c + 2] = x.z; w[4 * c + 3] = x.w;
      }
    } else {
      w[0] = *(const uint32_t *)(p + lane * 4);
      w[1] = *(const uint32_t *)(p + 256 + lane * 4);
    }
  };

  float m[RB], lsum[RB], corr[RB][NG], osum[RB][NG];
  f4 O[RB][NB];  // O^T[d = 16n + 4jj + r][column]
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m[rb] = -INFINITY;
    lsum[rb] = 0.0f;
#pragma unroll
    for (int n = 0; n < NB; ++n) O[rb][n] = f4{0, 0, 0, 0};
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) { corr[rb][gi] = 0.0f; osum[rb][gi] = 0.0f; }
  }

  // one staged tile: scores, softmax, PV for the wave's 32 rows
  auto tile = [&](const uint8_t *slot, int t) __attribute__((always_inline)) {
    uint32_t kw[C::LW];
    lds_payload(kw, slot);
    f4 acc[RB][NG];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) acc[rb][gi] = f4{0, 0, 0, 0};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      KT kop;
      if constexpr (QUANT) {
        kop = Conv<BITS>::template kop<C::LW>(kw, kb);
      } else {
        u4 r = {kw[4 * kb], kw[4 * kb + 1], kw[4 * kb + 2], kw[4 * kb + 3]};
        kop = __builtin_bit_cast(KT, r);
      }
      const int gi = QUANT ? (32 * kb) / G : 0;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb][gi] = FO::qk(kop, qv[rb][kb], acc[rb][gi]);
    }
    uint32_t km[C::MW], vm[C::MW];
    if constexpr (QUANT) {
      load_meta<C>(km, slot + 2 * KP + 4 * jj * NG * 4);
      load_meta<C>(vm, slot + 2 * KP + 16 * NG * 4 + 4 * jj * NG * 4);
    }
    const int tok0 = t * PKV_TILE + 4 * jj;
    const bool clear = t < clear_tiles;  // uniform: every live row sees the whole tile
    float s[RB][4];
    bool vis[RB][4];
    bool need = false;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v;
        if constexpr (QUANT) {
          v = 0.0f;
#pragma unroll
          for (int gi = 0; gi < NG; ++gi) {
            const uint32_t word = km[r * NG + gi];
            const float ks = f16_bits_to_f32(word);
            const float kbias = f16_bits_to_f32(word >> 16) - 1024.0f * ks;
            v += ks * acc[rb][gi][r] + qs[rb][gi] * kbias;
          }
        } else {
          v = acc[rb][0][r];
        }
        vis[rb][r] = clear ? lim[rb] >= 0 : tok0 + r <= lim[rb];
        v = vis[rb][r] ? v * a.scale_log2 : -INFINITY;
        s[rb][r] = v;
        need |= v > m[rb] + kTau;
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
        for (int gi = 0; gi < NG; ++gi) { corr[rb][gi] *= alpha; osum[rb][gi] *= alpha; }
#pragma unroll
        for (int n = 0; n < NB; ++n) O[rb][n] *= alpha;
      }
    }
    VT pop[RB][NG];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) p[r] = vis[rb][r] ? __builtin_amdgcn_exp2f(s[rb][r] - m[rb]) : 0.0f;
      lsum[rb] += (p[0] + p[1]) + (p[2] + p[3]);
      if constexpr (QUANT) {
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
          h4 pv;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t word = vm[r * NG + gi];
            // absent tokens contribute exact zeros whatever their metadata holds
            const _Float16 ps = (_Float16)(p[r] * f16_bits_to_f32(word));
            pv[r] = vis[rb][r] ? ps : (_Float16)0.0f;
            corr[rb][gi] += vis[rb][r] ? p[r] * f16_bits_to_f32(word >> 16) : 0.0f;
            osum[rb][gi] += (float)pv[r];
          }
          pop[rb][gi] = pv;
        }
      } else {
        pop[rb][0] = FO::pack_p(p[0], p[1], p[2], p[3]);
      }
    }
    uint32_t vw[C::LW];
    lds_payload(vw, slot + KP);
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      VT vop;
      if constexpr (QUANT) {
        vop = Conv<BITS>::template vop<C::LW>(vw, n);
      } else {
        u2 r = {vw[2 * n], vw[2 * n + 1]};
        vop = __builtin_bit_cast(VT, r);
      }
      const int gi = QUANT ? (16 * n) / G : 0;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) O[rb][n] = FO::pv(vop, pop[rb][gi], O[rb][n]);
    }
  };

  // ---- stream the span: DMA stage s+1 while computing stage s
  auto run_stage = [&](int s, uint8_t (&cur)[kStageTiles][SLOT], uint8_t (&nxt)[kStageTiles][SLOT],
                       int buf) __attribute__((always_inline)) {
    if (s + 1 < nstages) {
      issue(s + 1, nxt, buf ^ 1);
      stage_barrier<LPT>();  // every wave's DMAs of stage s have landed (stage s+1's are younger)
    } else {
      stage_barrier<0>();
    }
    if (s < 0) return;
#pragma unroll 1
    for (int j = 0; j < kStageTiles; ++j) {
      const int t = s * kStageTiles + j;
      if (t >= ntiles) break;
      if (!__builtin_amdgcn_readfirstlane(s_valid[buf][j])) continue;
      tile(cur[j], t);
    }
    stage_barrier<63>();  // every wave is done reading this buffer: free for stage s+2
  };
  // rotated so that every DMA is issued from inside the loop (stage s lives
  // in buffer s&1; the first pass only issues stage 0)
  for (int s = -1; s < nstages; s += 2) {
    run_stage(s, stage1, stage0, 1);
    if (s + 1 < nstages) run_stage(s + 1, stage0, stage1, 0);
  }

  // ---- epilogue: fold the 4 jj lanes of a column, normalise, write
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    lsum[rb] += __shfl_xor(lsum[rb], 16, 64);
    lsum[rb] += __shfl_xor(lsum[rb], 32, 64);
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      corr[rb][gi] += __shfl_xor(corr[rb][gi], 16, 64);
      corr[rb][gi] += __shfl_xor(corr[rb][gi], 32, 64);
      osum[rb][gi] += __shfl_xor(osum[rb][gi], 16, 64);
      osum[rb][gi] += __shfl_xor(osum[rb][gi], 32, 64);
    }
    const int row = rblk * kPrefillRows + wv * 32 + rb * 16 + col;
    if (row >= a.rows) continue;
    const int qi = row / a.gqa, h = kh * a.gqa + row % a.gqa;
    const float inv = 1.0f / fmaxf(lsum[rb], 1e-20f);
    uint16_t *o = a.out + (((int64_t)b * a.heads + h) * a.nq + qi) * g.dim;
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      float v4[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = O[rb][n][r];
        if constexpr (QUANT) {
          const int gi = (16 * n) / G;
          v += corr[rb][gi] - 1024.0f * osum[rb][gi];
        }
        v4[r] = v * inv;
      }
      const int d = 16 * n + 4 * jj;
      if ((g.dim & 3) == 0 && d + 4 <= g.dim) {
        u2 packed = {(uint32_t)float_to_bits(v4[0], g.float_kind) |
                         ((uint32_t)float_to_bits(v4[1], g.float_kind) << 16),
                     (uint32_t)float_to_bits(v4[2], g.float_kind) |
                         ((uint32_t)float_to_bits(v4[3], g.float_kind) << 16)};
        *(u2 *)(o + d) = packed;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (d + r < g.dim) o[d + r] = float_to_bits(v4[r], g.float_kind);
      }
    }
  }
}

// ---- host launcher ------------------------------------------------------------

typedef void (*PrefillKernel)(AttnArgs);

static PrefillKernel select_prefill(const Geo &g) {
#define PKV_Q(BITS_, DP_, G_) \
  if (g.bits == BITS_ && g.dp == DP_ && g.group == G_) return prefill_kernel<BITS_, DP_, G_, 1>;
  PKV_Q(8, 64, 32) PKV_Q(8, 64, 64)
  PKV_Q(8, 128, 32) PKV_Q(8, 128, 64) PKV_Q(8, 128, 128)
  PKV_Q(8, 256, 32) PKV_Q(8, 256, 64) PKV_Q(8, 256, 128)
  PKV_Q(4, 64, 32) PKV_Q(4, 64, 64)
  PKV_Q(4, 128, 32) PKV_Q(4, 128, 64) PKV_Q(4, 128, 128)
  PKV_Q(4, 256, 32) PKV_Q(4, 256, 64) PKV_Q(4, 256, 128)
#undef PKV_Q
#define PKV_F(DP_, FK_) \
  if (g.bits == 16 && g.dp == DP_ && g.float_kind == FK_) return prefill_kernel<16, DP_, 32, FK_>;
  PKV_F(64, 0) PKV_F(64, 1) PKV_F(128, 0) PKV_F(128, 1) PKV_F(256, 0) PKV_F(256, 1)
#undef PKV_F
  return nullptr;
}

hipError_t launch_prefill(hipStream_t stream, const AttnArgs &a) {
  const PrefillKernel k = select_prefill(a.g);
  if (!k) return hipErrorInvalidValue;
  const int64_t blocks = (int64_t)a.batch * a.g.hk * ((a.rows + kPrefillRows - 1) / kPrefillRows);
  if (blocks == 0) return hipSuccess;
  if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(64 * kPrefillWaves), 0, stream, a);
  return hipGetLastError();
}

}  // namespace pkv
