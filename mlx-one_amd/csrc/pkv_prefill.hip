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
// Work unit = one workgroup of 8 waves = (sequence, KV head, block of 8*16*RB
// query rows); wave w owns 16*RB rows as RB 16-column MFMA row tiles.  The
// span is streamed in stages of 8 tiles (128 tokens).  Per stage each wave
// loads ONE tile of quantized K/V (plus its scale/bias words) from HBM into
// registers a stage ahead, converts it once and writes it into the LDS stage
// image that all eight waves read: K as [tile][token][dim], V transposed as
// [dim][token slot].  Conversion thus costs 1/8 of the span per wave, and a
// stage's four steps give the next stage's loads time to land.
//
// Scores keep the reference's float32 precision (engine/paged_attention.py:
// 82-83: the query dotted with keys dequantized in f32).  The K image holds
// the codes themselves (exact f16 integers) and the scores are assembled from
// per-group products on the MFMA pipe:
//   s = sum_g scale_g * (q_g . c_g) + sum_g bias_g * (sum of q_g)
// The group chains share one accumulator: after group g's MFMAs it is
// multiplied by scale_g / scale_{g+1} (f32, per token), so it ends as
// (sum_g scale_g * q_g.c_g) / scale_last; one FMA by scale_last*scale*log2(e)
// less the running max gives the exp2 argument, and one 16x16x16 MFMA adds
// the bias term (the f16 biases times the rows' f32 group sums, split into
// f16 parts that carry 33 bits) through its accumulator input.  V is
// dequantized into the image in packed f16 ((1024+c) - 1024, then
// c*scale + bias: one rounding, relative 2^-11, entering the output
// linearly).  The inner loop per step:
//   S^T = K.Q^T        v_mfma_f32_16x16x32_f16, two tiles per step
//   online softmax     per column, exp2 domain, lazy rescale
//   O^T += V^T.P^T     v_mfma_f32_16x16x32_f16 over the step's 32 tokens
// The PV contraction pairs the two tiles' tokens: lane group jj holds tokens
// 4jj..4jj+3 of each tile of its scores, and the V^T image stores those 8
// tokens contiguously, so P needs no cross-lane movement.
// Steps whose tiles every live row sees whole take a path without per-token
// masks; tokens past the sequence or on unmapped pages are stored as zeros
// and masked.
#include <type_traits>

#include "pkv_mfma.h"

namespace pkv {

// Waves per workgroup, = tiles per stage (each wave converts one tile per
// stage): 8, or 4 at head_dim 256 (LDS budget of the double-buffered image).
constexpr int prefill_waves(int dp) { return dp > 128 ? 4 : 8; }
constexpr int kMaxPrefillWaves = 8;

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Row blocks per wave: two 16-column blocks up to head_dim 128, one beyond
// (register budget of the O accumulators).
constexpr int prefill_rb(int dp) { return dp > 128 ? 1 : 2; }
constexpr int prefill_rows(int dp) { return prefill_waves(dp) * 16 * prefill_rb(dp); }

// LDS image of one stage (u16 elements).  The operand reads are ds_read_b128
// with lane (col, jj) at byte col*stride + 16*jj.  On gfx950 such a read runs
// without bank conflicts when the row stride is 16*k bytes with k = 2 (mod 4)
// (measured: 288, 352, 416, 480, 544 conflict-free; 272 and 304 two-way, 256
// eight-way), so rows are padded by 16 elements: strides of 2*(DP+16) bytes
// (160, 288, 544) and 2*(16*TILES+16) bytes (288 at 8 tiles, 160 at 4).
template <int DP>
struct StageImage {
  static constexpr int TILES = prefill_waves(DP);
  static constexpr int KROW = DP + 16;          // K row: one token
  static constexpr int KTILE = 16 * KROW;
  static constexpr int VROW = 16 * TILES + 16;  // V^T row: one dim, 16 token slots per tile
  static constexpr int K_ELEMS = TILES * KTILE;
  static constexpr int ELEMS = K_ELEMS + DP * VROW;
};

// Score metadata of quantized K tiles (next to the stage image), per tile:
//   mult [NG][16 tokens] f32: scale_g / scale_{g+1} for g < NG - 1, then
//        scale_last * softmax scale * log2(e); 0 for absent tokens
//   bias [4 slot quads][16 tokens][4 slots] 16-bit: the A operand of the
//        bias MFMA, slot k holding bias_{k / SPG} (SPG slots per group, one
//        per part of the query's group sum), 0 past the groups and for absent
//        tokens.  Lane (col, jj) reads quad jj of token col: each 16-lane
//        group reads 128 contiguous bytes (no bank conflicts; a token-major
//        layout, 32 bytes per lane apart, conflicted four ways)
// SPG: 3 parts (33 significant bits) while 3 * NG <= 16, else 2 (22 bits).
constexpr int bias_parts(int ng) { return 3 * ng <= 16 ? 3 : 2; }

// Workgroup barrier once this wave's LDS operations have completed.  No
// memory fence: __syncthreads() would also wait for the next stage's HBM
// loads still in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
}

// Query rows of sequence b live in this launch: 0 for a sequence of a mixed
// batch that the decode kernel serves (narrow_q > 0, width at most narrow_q).
// f32 -> bf16 bits on v_cvt_pk_bf16_f32 (round to nearest even): for the
// values an f16 holds (never f32 denormals) the bits of f32_to_bf16_bits,
// without its software NaN branch.
__device__ __forceinline__ uint16_t bf16_bits_cvt(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}

__device__ __forceinline__ int prefill_width(const AttnArgs &a, int b) {
  return a.widths ? (a.narrow_q > 0 && a.widths[b] <= a.narrow_q ? 0 : a.widths[b]) : a.nq;
}

// The k-th (from 0) sequence, in batch order, whose rows are live here
// (live) or not (!live); -1 past the last.  Uniform; the whole wave calls.
__device__ int nth_sequence(const AttnArgs &a, bool live, int k, int lane) {
  int carry = 0;
  for (int c0 = 0; c0 < a.batch; c0 += 64) {
    const int idx = c0 + lane;
    const int f = idx < a.batch && ((prefill_width(a, idx) > 0) == live) ? 1 : 0;
    const int incl = wave_scan_incl(f, lane) + carry;
    const unsigned long long hit = __ballot(f && incl == k + 1);
    if (hit) return c0 + __ffsll((long long)hit) - 1;
    carry = __builtin_amdgcn_readlane(incl, 63);
  }
  return -1;
}

// Zeros into one output row of `dim` 16-bit elements (4-byte lanes where aligned).
__device__ __forceinline__ void zero_row(uint16_t *o, int dim, int lane) {
  for (int d = 2 * lane; d < dim; d += 128) {
    if (d + 1 < dim && ((uintptr_t)(o + d) & 3) == 0) {
      *(uint32_t *)(o + d) = 0u;
    } else {
      o[d] = 0;
      if (d + 1 < dim) o[d + 1] = 0;
    }
  }
}

// A block's share [z, zend) of the dead rows of a mixed batch, in the
// flattened space z = ((n * HK + kh) * gqa + hh) * nq + qi over the sequences
// n that the decode kernel serves (in batch order): runs of consecutive qi
// are contiguous in the output, and the block's `nthreads` threads fill each
// run with 16-byte non-temporal stores (rows whose bytes are not 16-byte
// multiples: a wave per row).  Non-temporal, so that the zeros reach HBM
// while this MFMA-bound kernel leaves it idle instead of lingering in the
// memory-side cache to be written back under the decode kernel that follows
// (its launch: 88 -> 69 us in a mixed C2 + C5 batch).
__device__ __forceinline__ void zero_share(const AttnArgs &a, int64_t z, int64_t zend, int tid,
                                           int nthreads) {
  const int lane = tid & 63, wv = tid >> 6, nwaves = nthreads >> 6;
  const int64_t per_seq = (int64_t)a.g.hk * a.rows;
  int n = (int)(z / per_seq);
  const int64_t r = z % per_seq;
  int kh = (int)(r / a.rows);
  const int r2 = (int)(r % a.rows);
  int hh = r2 / a.nq, qi = r2 % a.nq;
  int b = nth_sequence(a, false, n, lane);
  const int dim = a.g.dim;
  const bool vec = (dim & 7) == 0 && ((uintptr_t)a.out & 15) == 0;
  while (z < zend && b >= 0) {
    const int run = (int)min((int64_t)(a.nq - qi), zend - z);
    uint16_t *o = a.out + (((int64_t)b * a.heads + kh * a.gqa + hh) * a.nq + qi) * dim;
    if (vec) {
      const int units = run * (dim / 8);
      for (int u = tid; u < units; u += nthreads) __builtin_nontemporal_store(u4{0, 0, 0, 0}, (u4 *)o + u);
    } else {
      for (int i = wv; i < run; i += nwaves) zero_row(o + (int64_t)i * dim, dim, lane);
    }
    z += run;
    qi += run;
    if (qi == a.nq) {
      qi = 0;
      if (++hh == a.gqa) {
        hh = 0;
        if (++kh == a.g.hk) {
          kh = 0;
          b = nth_sequence(a, false, ++n, lane);
        }
      }
    }
  }
}

template <int BITS, int DP, int G, int FK, bool SHARE>
__global__ __launch_bounds__(64 * kMaxPrefillWaves) void prefill_kernel(const AttnArgs a) {
  constexpr int kPrefillWaves = prefill_waves(DP);
  constexpr int kStageTiles = kPrefillWaves;
  constexpr int RB = prefill_rb(DP);
  constexpr int ROWS = prefill_rows(DP);
  using C = Cfg<BITS, DP, G, RB, FK, 1>;
  constexpr bool QUANT = C::QUANT;
  // Operand types.  S = K.Q^T takes the query in its own dtype (FK: bf16 0,
  // f16 1), so the query operand is the query exactly, and K in the same
  // type (codes are exact in either).  O += V.P^T runs in f16 for quantized
  // pages (V dequantized into the image) and in the page dtype otherwise.
  constexpr bool QF16 = FK == 1;
  constexpr bool PF16 = QUANT || FK == 1;
  constexpr int NG = C::NG, KB = C::KB, NB = C::NB, LW = C::LW;
  using I = StageImage<DP>;
  typedef typename std::conditional<QF16, h8, b8>::type QT;  // 8-element QK operand
  typedef typename std::conditional<PF16, h8, b8>::type PT;  // 8-element PV operand
  // The bias MFMA in bf16 (range of any query, no scaled rows) when its slots
  // fit one 16x16x16 MFMA: two parts of each bias (exact) times three of each
  // group sum, 6 per group; else in f16 (exact biases times 3 or 2 parts).
  constexpr bool BF16_BIAS = QUANT && 6 * NG <= 16;
  typedef typename std::conditional<BF16_BIAS, s4, h4>::type BT;  // bias MFMA operand

  // tile flags of a stage image, one byte each (0 or 1), read as words
  __shared__ __attribute__((aligned(16))) uint8_t s_valid[2][kStageTiles];
  __shared__ int s_lim[2][kPrefillWaves];
  __shared__ int64_t s_zero[SHARE ? 2 : 1];  // zero share: first row, end
  __shared__ __attribute__((aligned(16))) uint16_t stage[2][I::ELEMS];
  // score metadata of the stage's K tiles (quantized pages)
  constexpr int SPG = BF16_BIAS ? 6 : bias_parts(NG);
  __shared__ __attribute__((aligned(16))) float s_mult[2][QUANT ? kStageTiles * NG * 16 : 4];
  __shared__ __attribute__((aligned(16))) uint16_t s_bias[2][QUANT ? kStageTiles * 16 * 16 : 8];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, jj = lane >> 4;
  const Geo &g = a.g;
  // Work items.  Blocks of one (sequence, KV head) read the same pages: give
  // them consecutive slots of one XCD (workgroups are dealt to the 8 XCDs
  // round-robin) so the span is fetched into one L2.  XCD x runs segments
  // x, x + 8, x + 16, ...: heavy segments that sit together in the batch still
  // spread over every XCD.
  //
  // A mixed batch's sequences that the decode kernel serves (width 0 here)
  // only need zeros in their rows (the decode kernel, launched next, writes
  // the rows it serves).  Their blocks would each hold a CU (and its LDS)
  // for a few stores and delay the blocks with work behind them, so the
  // first R blocks of the grid take the R blocks of the sequences with live
  // rows, in order, and also write those zeros (an equal share each, after
  // their own rows: blocks of different causal spans end at different
  // times), and the rest of the grid exits at once.
  // (SHARE: the instantiation for mixed batches, launched when the decode
  // kernel serves some of the call's sequences; others carry none of it.)
  const int nblk = (a.rows + ROWS - 1) / ROWS;
  int bid = blockIdx.x;
  int64_t zlo = 0, zhi = 0;  // zero rows (of the flattened dead-row space) this block writes
  bool share = false;
  int R = (int)gridDim.x;
  if constexpr (SHARE) {
    int nlive = 0;
    for (int c0 = 0; c0 < a.batch; c0 += 64) {
      const int idx = c0 + lane;
      nlive += wave_sum(idx < a.batch && prefill_width(a, idx) > 0 ? 1 : 0);
    }
    share = nlive > 0 && nlive < a.batch;
    if (share) {
      R = nlive * g.hk * nblk;
      if (bid >= R) return;
      const int64_t Z = (int64_t)(a.batch - nlive) * g.hk * a.rows;
      zlo = (int64_t)bid * Z / R;
      zhi = (int64_t)(bid + 1) * Z / R;
    }
  }
  const int span = R;
  if (((span / nblk) & 7) == 0) {
    const int x = bid & 7, k = bid >> 3;
    bid = (x + 8 * (k / nblk)) * nblk + k % nblk;
  }
  const int seg = bid / nblk, rblk = bid % nblk;
  const int b = share ? nth_sequence(a, true, seg / g.hk, lane) : seg / g.hk;
  const int kh = seg % g.hk;
  if (b < 0 || b >= a.batch) return;
  const int L = a.seq_lens[b];
  const int width = prefill_width(a, b);
  if (SHARE && width <= 0) {
    // no row of this sequence is live here (every sequence of the call is
    // left to the decode kernel): the block's rows are zeros, written
    // without the query loads and the span walk (elsewhere such rows take
    // the general path: limit -1, zero output)
    const int r0 = rblk * ROWS, r1 = min(a.rows, r0 + ROWS);
    for (int row = r0 + wv; row < r1; row += kPrefillWaves) {
      const int qi = row / a.gqa, h = kh * a.gqa + row % a.gqa;
      zero_row(a.out + (((int64_t)b * a.heads + h) * a.nq + qi) * g.dim, g.dim, lane);
    }
    return;
  }

  // ---- the wave's query rows: row = ROWS*rblk + 16*RB*wv + 16*rb + col
  int lim[RB];
  QT qv[RB][KB];
  // The query operand is the query itself; scale*log2(e) is applied to the
  // f32 scores, never rounded into the operand.
  const float rsc = a.scale_log2;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = rblk * ROWS + wv * 16 * RB + rb * 16 + col;
    const bool valid = row < a.rows;
    const int rowv = valid ? row : 0;  // rows past the block load row 0, zeroed below
    const int qi = rowv / a.gqa, h = kh * a.gqa + rowv % a.gqa;
    const bool live = valid && qi < width;
    const int pos = a.q_pos ? a.q_pos[(int64_t)b * a.nq + qi] : L - width + qi;
    lim[rb] = live ? min(pos, L - 1) : -1;
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
      qv[rb][kb] = __builtin_bit_cast(QT, u4{e8[0] | ((uint32_t)e8[1] << 16), e8[2] | ((uint32_t)e8[3] << 16),
                                             e8[4] | ((uint32_t)e8[5] << 16), e8[6] | ((uint32_t)e8[7] << 16)});
    }
  }

  // Exact scores (quantized pages): per row block the B operand of the bias
  // MFMA, the row's group sums of q times scale*log2(e), Q_g, in parts (the
  // lane holds slots 4jj..4jj+3).  bf16 parts carry any magnitude.  f16
  // parts (four or more groups) hold |Q_g| < 2^15: a row whose largest |Q_g|
  // reaches it has its Q_g scaled by 2^-e, the MFMA then adds the bias term
  // scaled by 2^-e to an accumulator scaled the same way, and the result is
  // scaled back by 2^e; a wave holding such a row takes that general form of
  // the final step (`wide`, a uniform branch).
  BT qop[QUANT ? RB : 1];
  float dn[QUANT ? RB : 1], ue[QUANT ? RB : 1];
  bool wide_lane = false;
  if constexpr (QUANT) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float qs[NG];
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) qs[gi] = 0.0f;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        float t = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) t += (float)qv[rb][kb][e];
        qs[(32 * kb) / G] += t;
      }
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        qs[gi] += __shfl_xor(qs[gi], 16, 64);
        qs[gi] += __shfl_xor(qs[gi], 32, 64);
        qs[gi] *= rsc;
      }
      BT op = {0, 0, 0, 0};
      auto place = [&](int k, auto v) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if ((k & 3) == i) op[i] = (k >> 2) == jj ? v : op[i];
      };
      if constexpr (BF16_BIAS) {
        dn[rb] = ue[rb] = 1.0f;
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
          // three bf16 parts (24 bits): hi, mid, lo; each remainder is exact in f32
          const uint16_t hi = f32_to_bf16_bits(qs[gi]);
          const float r1 = qs[gi] - __uint_as_float((uint32_t)hi << 16);
          const uint16_t mid = f32_to_bf16_bits(r1);
          const uint16_t lo = f32_to_bf16_bits(r1 - __uint_as_float((uint32_t)mid << 16));
          const short part[3] = {(short)hi, (short)mid, (short)lo};
#pragma unroll
          for (int pt = 0; pt < SPG; ++pt) place(gi * SPG + pt, part[pt % 3]);
        }
      } else {
        float qmax = 0.0f;
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) qmax = fmaxf(qmax, fabsf(qs[gi]));
        int e = 0;
        if (qmax >= 32768.0f && qmax < INFINITY) {
          int ex;
          frexpf(qmax, &ex);  // qmax in [2^(ex-1), 2^ex): qmax * 2^(15-ex) < 2^15
          e = ex - 15;
        }
        dn[rb] = ldexpf(1.0f, -e);
        ue[rb] = ldexpf(1.0f, e);
        wide_lane |= e != 0;
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
          const float x = qs[gi] * dn[rb];
          const _Float16 hi = (_Float16)x;
          const float r1 = x - (float)hi;
          const _Float16 mid = (_Float16)r1;
          const _Float16 lo = (_Float16)(r1 - (float)mid);
          const _Float16 part[3] = {hi, mid, lo};
#pragma unroll
          for (int pt = 0; pt < SPG; ++pt) place(gi * SPG + pt, part[pt]);
        }
      }
      qop[rb] = op;
    }
  }
  const bool wide = QUANT && !BF16_BIAS && __any(wide_lane);

  // ---- the block's visible span: tokens up to the largest limit; tiles
  // below the smallest live limit are seen whole by every live row
  {
    int hi = lim[0], lo = lim[0] < 0 ? 0x7FFFFFFF : lim[0];
#pragma unroll
    for (int rb = 1; rb < RB; ++rb) {
      hi = max(hi, lim[rb]);
      lo = min(lo, lim[rb] < 0 ? 0x7FFFFFFF : lim[rb]);
    }
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
  if (SHARE && tid == 0) {
    s_zero[0] = zlo;
    s_zero[1] = zhi;
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
  const int clear_tiles = tmin == 0x7FFFFFFF ? 0 : (tmin + 1) / PKV_TILE;
  const int nstages = (ntiles + kStageTiles - 1) / kStageTiles;
  const int tpp_shift = __builtin_ctz(g.page / PKV_TILE);
  const int tpp_mask = (1 << tpp_shift) - 1;

  // ---- raw tile in flight: wave wv owns tile 4s + wv of stage s
  uint32_t rk[LW], rv[LW];
  uint32_t rkm[QUANT ? NG : 1], rvm[QUANT ? 4 * NG : 4];
  int k_ok = 0, k_t = 0, v_ok = 0, v_t = 0;  // tile whose K (V) half sits in rk (rv)
  // Page id of a tile: one uniform (scalar) load of the block table per
  // stage; the K and V halves of a tile share it.  (A page-id window held in
  // a VGPR and read with v_readlane made every lookup wait for all vector
  // loads in flight, the tile loads just issued included.)
  typedef __attribute__((address_space(4))) const int32_t cint32;  // read-only: scalar loads
  cint32 *trow = (cint32 *)(a.table + (int64_t)b * a.max_pages);
  int n_ok = 0, n_t = 0, n_tip = 0;  // the located tile
  const uint8_t *n_head = a.pool;
  // tile kStageTiles*s + wv of stage s -> (present, tile, head block, tile offset)
  auto locate = [&](int s) __attribute__((always_inline)) {
    n_t = s * kStageTiles + wv;
    int id = -1;
    n_tip = 0;
    if (n_t < ntiles) {
      const int p = n_t >> tpp_shift;
      const int pid = p < a.max_pages ? trow[p] : -1;
      if (pid >= 0 && pid < a.num_pages) {
        id = pid;
        n_tip = n_t & tpp_mask;
      }
    }
    n_ok = id >= 0;
    n_head = a.pool + (int64_t)(n_ok ? id : 0) * g.page_bytes + (int64_t)kh * g.head_bytes;
  };
  // Both halves of the wave's tile of stage s, issued together (so that the
  // compiler's wait counts before the conversions are exact: a path with
  // only one half issued would make it wait for every load in flight).
  auto fetch = [&](int s) __attribute__((always_inline)) {
    locate(s);
    k_ok = v_ok = n_ok;
    k_t = v_t = n_t;
    if (n_ok) {
      const uint8_t *head = n_head;
      const int tip = n_tip;
      load_payload<C>(rk, head + (int64_t)tip * g.tile_bytes, lane);
      if constexpr (QUANT) {
        const uint8_t *km = head + g.kmeta_offset + (int64_t)((tip * PKV_TILE + col) * NG) * 4;
        if constexpr (NG == 1) {
          rkm[0] = *(const uint32_t *)km;
        } else if constexpr (NG == 2) {
          const u2 x = *(const u2 *)km;
          rkm[0] = x.x; rkm[1] = x.y;
        } else {
#pragma unroll
          for (int i = 0; i < NG; i += 4) {
            const u4 x = *(const u4 *)(km + i * 4);
            rkm[i] = x.x; rkm[i + 1] = x.y; rkm[i + 2] = x.z; rkm[i + 3] = x.w;
          }
        }
      }
      load_payload<C>(rv, head + g.v_offset + (int64_t)tip * g.tile_bytes, lane);
      if constexpr (QUANT)
        load_meta<C>(rvm, head + g.vmeta_offset + (int64_t)((tip * PKV_TILE + 4 * jj) * NG) * 4);
    }
  };

  // ---- convert the raw tile into slot wv of a stage image (K half, then V
  // half: each is scheduled against one step's MFMAs)
  auto convert = [&](int dst, bool k_half) __attribute__((always_inline)) {
    uint16_t *img = stage[dst];
    const int r_ok = k_half ? k_ok : v_ok;
    const int tok0 = (k_half ? k_t : v_t) * PKV_TILE;
    const bool whole = r_ok && tok0 + PKV_TILE <= L;  // uniform
    const bool kvalid = r_ok && tok0 + col < L;
    bool vvalid[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) vvalid[e] = r_ok && tok0 + 4 * jj + e < L;
    uint16_t *kdst = img + wv * I::KTILE + col * I::KROW + 8 * jj;
    uint16_t *vdst = img + I::K_ELEMS + col * I::VROW + 32 * (wv >> 1) + 8 * jj + 4 * (wv & 1);
    if constexpr (QUANT) {
      // absent tokens: scale = bias = 0 -> exact zeros
      uint32_t km[NG], vm[4 * NG];
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) km[gi] = whole || kvalid ? rkm[gi] : 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) vm[e * NG + gi] = whole || vvalid[e] ? rvm[e * NG + gi] : 0u;
      // K: the codes as exact integers in the query dtype (f16:
      // (1024 + c) - 1024; bf16: through f32), and the token's score
      // metadata (lane (col, jj): multiplier rows g = jj, jj + 4, bias slots
      // 4jj..4jj+3)
#pragma unroll
      for (int kb = 0; kb < (k_half ? KB : 0); ++kb) {
        if constexpr (QF16) {
          const h8 c = Conv<BITS>::template kop<LW>(rk, kb) - (_Float16)1024.0f;
          *(u4 *)(kdst + 32 * kb) = __builtin_bit_cast(u4, c);
        } else {
          *(u4 *)(kdst + 32 * kb) = Conv<BITS>::template kop_bf16<LW>(rk, kb);
        }
      }
      if (k_half) {
        const bool tv = whole || kvalid;
        float scl[NG];
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) scl[gi] = f16_bits_to_f32(km[gi]);
        float *mrow = s_mult[dst] + wv * NG * 16 + col;
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
          if ((gi & 3) != jj) continue;
          // (scales are at least 1e-6: the reciprocal is within 1 ulp)
          const float mv = gi + 1 < NG ? scl[gi] * __builtin_amdgcn_rcpf(scl[gi + 1 < NG ? gi + 1 : gi])
                                       : scl[gi] * a.scale_log2;
          mrow[gi * 16] = tv ? mv : 0.0f;
        }
        // slot k of group g = k / SPG: the f16 bias, or (bf16 bias MFMA) its
        // first part (bf16 rounding, slots 0-2 of the group) and the exact
        // remainder (slots 3-5)
        s4 bo = {0, 0, 0, 0};
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
          const uint32_t bb = km[gi] >> 16;
          short part[2] = {(short)bb, (short)bb};
          if constexpr (BF16_BIAS) {
            const float bf = f16_bits_to_f32(bb);
            const uint16_t hi = bf16_bits_cvt(bf);
            part[0] = (short)hi;
            part[1] = (short)bf16_bits_cvt(bf - __uint_as_float((uint32_t)hi << 16));
          }
#pragma unroll
          for (int pt = 0; pt < SPG; ++pt) {
            const int k = gi * SPG + pt;
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if ((k & 3) == i) bo[i] = (k >> 2) == jj ? part[BF16_BIAS && pt >= 3] : bo[i];
          }
        }
        *(u2 *)(s_bias[dst] + ((wv * 4 + jj) * 16 + col) * 4) = __builtin_bit_cast(u2, bo);
      }
#pragma unroll
      for (int n = 0; n < (k_half ? 0 : NB); ++n) {
        const int gi = (16 * n) / G;
        h4 sc, bi;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const h2 sb = __builtin_bit_cast(h2, vm[e * NG + gi]);
          sc[e] = sb.x;
          bi[e] = sb.y;
        }
        const h4 c = Conv<BITS>::template vop<LW>(rv, n);
        const h4 v = __builtin_elementwise_fma(c - (_Float16)1024.0f, sc, bi);
        *(u2 *)(vdst + 16 * n * I::VROW) = __builtin_bit_cast(u2, v);
      }
    } else {
      const uint32_t kmask = whole || kvalid ? 0xFFFFFFFFu : 0u;
      const uint32_t vmask0 = whole ? 0xFFFFFFFFu : (vvalid[0] ? 0xFFFFu : 0u) | (vvalid[1] ? 0xFFFF0000u : 0u);
      const uint32_t vmask1 = whole ? 0xFFFFFFFFu : (vvalid[2] ? 0xFFFFu : 0u) | (vvalid[3] ? 0xFFFF0000u : 0u);
#pragma unroll
      for (int kb = 0; kb < (k_half ? KB : 0); ++kb) {
        const u4 v = {rk[4 * kb] & kmask, rk[4 * kb + 1] & kmask, rk[4 * kb + 2] & kmask, rk[4 * kb + 3] & kmask};
        *(u4 *)(kdst + 32 * kb) = v;
      }
#pragma unroll
      for (int n = 0; n < (k_half ? 0 : NB); ++n) {
        const u2 v = {rv[2 * n] & vmask0, rv[2 * n + 1] & vmask1};
        *(u2 *)(vdst + 16 * n * I::VROW) = v;
      }
    }
    if (!k_half && lane == 0) s_valid[dst][wv] = r_ok ? 1 : 0;
  };

  // Row sums of P: f16 P operands (quantized and f16 pages) sum on the MFMA
  // pipe, as the V^T row of a ones operand (row 0 of OS[rb], lanes jj = 0),
  // the same rounded P the output accumulates; bf16 pages (P = hi + lo) sum
  // the f32 probabilities on the VALU.
  constexpr bool MSUM = PF16;
  // m: the running maximum in the exp2 domain, 0 before the row has seen a
  // token; thr: the rescale threshold over m, -inf until then (so that the
  // first finite score sets m), kTau after.
  float m[RB], thr[RB], lsum[RB];
  f4 OS[MSUM ? RB : 1];
  f4 O[RB][NB];  // O^T[d = 16n + 4jj + r][column]
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m[rb] = 0.0f;
    thr[rb] = -INFINITY;
    lsum[rb] = 0.0f;
    if constexpr (MSUM) OS[rb] = f4{0, 0, 0, 0};
#pragma unroll
    for (int n = 0; n < NB; ++n) O[rb][n] = f4{0, 0, 0, 0};
  }

  // max of 8 values (v_maximum3_f32: no NaN canonicalisation)
  auto max8 = [](const float (&x)[8]) __attribute__((always_inline)) {
    const float a3 = __builtin_elementwise_maximum(__builtin_elementwise_maximum(x[0], x[1]), x[2]);
    const float b3 = __builtin_elementwise_maximum(__builtin_elementwise_maximum(x[3], x[4]), x[5]);
    const float c3 = __builtin_elementwise_maximum(__builtin_elementwise_maximum(x[6], x[7]), a3);
    return __builtin_elementwise_maximum(b3, c3);
  };

  // ---- one step covers tiles 2pr and 2pr + 1 of a stage image.
  // S^T = K.Q^T for both tiles; the scores then become v = s*rsc - mb in the
  // exp2 domain (mb: the running max, 0 before any token is seen).
  // Quantized pages: the group chains share the accumulator (scaled by
  // scale_g / scale_{g+1} between groups), then the exp2 argument less the
  // bias term, then the bias MFMA; S ends as the exp2 argument itself.
  auto qk = [&](const uint16_t *img, const float *mult, const uint16_t *bias, int pr,
                f4 (&S)[2][RB], float (&mb)[RB]) __attribute__((always_inline)) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      mb[rb] = m[rb];
#pragma unroll
      for (int i = 0; i < 2; ++i) S[i][rb] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const uint16_t *kbase = img + 2 * pr * I::KTILE + col * I::KROW + 8 * jj;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if constexpr (QUANT) {
        if (kb > 0 && (32 * kb) % G == 0) {  // group boundary: scale_g / scale_{g+1}
          const int gprev = (32 * kb) / G - 1;
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const f4 r = *(const f4 *)(mult + ((2 * pr + i) * NG + gprev) * 16 + 4 * jj);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) S[i][rb] *= r;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const QT kop = __builtin_bit_cast(QT, *(const u4 *)(kbase + i * I::KTILE + 32 * kb));
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          if constexpr (QF16)
            S[i][rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, qv[rb][kb], S[i][rb], 0, 0, 0);
          else
            S[i][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qv[rb][kb], S[i][rb], 0, 0, 0);
        }
      }
    }
    if constexpr (QUANT) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const f4 scr = *(const f4 *)(mult + ((2 * pr + i) * NG + NG - 1) * 16 + 4 * jj);
        const BT aop = __builtin_bit_cast(BT, *(const u2 *)(bias + (((2 * pr + i) * 4 + jj) * 16 + col) * 4));
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          f4 c;
          if constexpr (BF16_BIAS) {
#pragma unroll
            for (int r = 0; r < 4; ++r) c[r] = __builtin_fmaf(S[i][rb][r], scr[r], -mb[rb]);
            c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(aop, qop[rb], c, 0, 0, 0);
          } else if (wide) {  // uniform: rows outside f16 range in this wave (rare)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              c[r] = __builtin_fmaf(S[i][rb][r], scr[r] * dn[rb], -mb[rb] * dn[rb]);
            c = __builtin_amdgcn_mfma_f32_16x16x16f16(aop, qop[rb], c, 0, 0, 0);
            c *= ue[rb];
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) c[r] = __builtin_fmaf(S[i][rb][r], scr[r], -mb[rb]);
            c = __builtin_amdgcn_mfma_f32_16x16x16f16(aop, qop[rb], c, 0, 0, 0);
          }
          S[i][rb] = c;
        }
      }
    }
  };
  // Masks (steps not seen whole by every live row), then the lazy rescale:
  // only when a score exceeds the running max by more than kTau.
  auto scores = [&](const f4 (&S)[2][RB], const float (&mb)[RB], int s, int pr, int okv,
                    float (&v)[RB][8]) __attribute__((always_inline)) {
    const int ta = s * kStageTiles + 2 * pr;
    const bool oka = (okv >> (2 * pr)) & 1;
    const bool okb = ta + 1 < ntiles && ((okv >> (2 * pr + 1)) & 1);
    const bool fast = oka && okb && ta + 1 < clear_tiles;
    float mx[RB];
    bool need = false;
    // token (ta + i) * 16 + 4jj + r is visible to row block rb when
    // i * 16 + r <= rel
    auto mask = [&](int rb) __attribute__((always_inline)) {
      const int rel = lim[rb] - ta * PKV_TILE - 4 * jj;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool vis = (i ? okb : oka) && i * PKV_TILE + r <= rel;
          v[rb][4 * i + r] = vis ? v[rb][4 * i + r] : -INFINITY;
        }
    };
    if constexpr (QUANT) {  // the scores are S itself: one mask branch per step
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int e = 0; e < 8; ++e) v[rb][e] = S[e >> 2][rb][e & 3];
      if (!fast) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) mask(rb);
      }
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if constexpr (!QUANT) {  // (one branch per row block keeps fewer scores live)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) v[rb][4 * i + r] = __builtin_fmaf(S[i][rb][r], rsc, -mb[rb]);
        if (!fast) mask(rb);
      }
      mx[rb] = max8(v[rb]);
      // before any token is seen every finite score sets the max
      need |= mx[rb] > thr[rb];
    }
    if (__any(need)) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        float tm = mx[rb];
        tm = __builtin_elementwise_maximum(tm, __shfl_xor(tm, 16, 64));
        tm = __builtin_elementwise_maximum(tm, __shfl_xor(tm, 32, 64));
        const bool first = thr[rb] == -INFINITY;  // nothing accumulated yet
        const float mn = first ? tm + mb[rb] : fmaxf(m[rb], tm + mb[rb]);
        if (mn != -INFINITY && (first || mn != m[rb])) {
          const float shift = mn - mb[rb];
          const float alpha = first ? 0.0f : __builtin_amdgcn_exp2f(m[rb] - mn);
          thr[rb] = kTau;
#pragma unroll
          for (int e = 0; e < 8; ++e) v[rb][e] -= shift;
          m[rb] = mn;
          if constexpr (MSUM) OS[rb] *= alpha;
          else lsum[rb] *= alpha;
#pragma unroll
          for (int n = 0; n < NB; ++n) O[rb][n] *= alpha;
        }
      }
    }
  };
  // P = exp2(v) (masked: exp2(-inf) = 0), row sums, packed operand; bf16
  // pages also pack the rounding error Plo (P = hi + lo: 16 significant bits,
  // where one bf16 alone, 2^-9 relative, times values of outlier channels
  // exceeds the output tolerance on short spans)
  auto probs = [&](const float (&v)[RB][8], PT (&P)[RB], PT (&Plo)[RB]) __attribute__((always_inline)) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) p[e] = __builtin_amdgcn_exp2f(v[rb][e]);
      if constexpr (!MSUM) lsum[rb] += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
      if constexpr (PF16) {
        P[rb] = h8{(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3],
                   (_Float16)p[4], (_Float16)p[5], (_Float16)p[6], (_Float16)p[7]};
      } else {
        P[rb] = b8{(__bf16)p[0], (__bf16)p[1], (__bf16)p[2], (__bf16)p[3],
                   (__bf16)p[4], (__bf16)p[5], (__bf16)p[6], (__bf16)p[7]};
        PT lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) lo[e] = (__bf16)(p[e] - (float)P[rb][e]);
        Plo[rb] = lo;
      }
    }
  };
  // O^T += V^T.P^T over the step's 32 tokens
  auto pv = [&](const uint16_t *img, int pr, const PT (&P)[RB], const PT (&Plo)[RB]) __attribute__((always_inline)) {
    const uint16_t *vbase = img + I::K_ELEMS + col * I::VROW + 32 * pr + 8 * jj;
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      const PT vop = __builtin_bit_cast(PT, *(const u4 *)(vbase + 16 * n * I::VROW));
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        if constexpr (PF16)
          O[rb][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, P[rb], O[rb][n], 0, 0, 0);
        else {
          O[rb][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, P[rb], O[rb][n], 0, 0, 0);
          O[rb][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, Plo[rb], O[rb][n], 0, 0, 0);
        }
      }
    }
    if constexpr (MSUM) {
      const _Float16 one = col == 0 ? (_Float16)1.0f : (_Float16)0.0f;
      const h8 ones = {one, one, one, one, one, one, one, one};
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        OS[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, P[rb], OS[rb], 0, 0, 0);
    }
  };

  // ---- stream the span.  Iteration s computes stage s from image s&1,
  // converts the tile of stage s+1 (loaded during stage s-1) into image
  // (s+1)&1 -- last read in iteration s-1, before its barrier -- and, after
  // its V half, issues the loads of stage s+2.  Within a stage the second step's QK MFMAs are
  // issued before the first step's exponentials and the conversion halves
  // sit beside the PV MFMAs, so that the MFMA and VALU pipes overlap.  Both
  // run without branches: past the span the second step sees tiles flagged
  // invalid (zeros, fully masked), and the last stage converts the absent
  // tile past the span into the image nobody reads again.
  if (nstages > 0) {
    fetch(0);
    convert(0, true);
    convert(0, false);
    if (nstages > 1) fetch(1);
  }
  lds_barrier();
  for (int s = 0; s < nstages; ++s) {
    const int buf = s & 1;
    const uint16_t *img = stage[buf];
    const float *mult = s_mult[buf];
    const uint16_t *bias = s_bias[buf];
    // the stage's tile flags (uniform bit mask)
    // (bytes b0..b3 of 0/1: w * 0x01020408 puts b_i at bit 24 + i, every
    // other product term below bit 20 or past bit 31)
    int okv = 0;
#pragma unroll
    for (int q4 = 0; q4 < kStageTiles / 4; ++q4) {
      const uint32_t w = __builtin_amdgcn_readfirstlane(*(const uint32_t *)&s_valid[buf][4 * q4]);
      okv |= (int)(((w * 0x01020408u) >> 24) & 0xFu) << (4 * q4);
    }
    // steps over tile pairs; pair pr+1's QK MFMAs are issued before pair
    // pr's exponentials, the conversion halves sit beside the first two
    // pairs' PV MFMAs
    constexpr int NPAIR = kStageTiles / 2;
    f4 S[2][2][RB];
    float mb[2][RB], v[RB][8];
    PT P[RB], Plo[RB];
    qk(img, mult, bias, 0, S[0], mb[0]);
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr) {
      scores(S[pr & 1], mb[pr & 1], s, pr, okv, v);
      if (pr + 1 < NPAIR) qk(img, mult, bias, pr + 1, S[(pr + 1) & 1], mb[(pr + 1) & 1]);
      probs(v, P, Plo);
      pv(img, pr, P, Plo);
      if (pr == 0) {
        convert(buf ^ 1, true);
      } else if (pr == 1) {
        convert(buf ^ 1, false);
        fetch(s + 2);  // past the span: located as absent, no loads
      }
    }
    lds_barrier();
  }

  // ---- epilogue: fold the 4 jj lanes of a column, normalise, write
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    if constexpr (MSUM) {
      lsum[rb] = __shfl(OS[rb][0], col, 64);  // row 0 lives in lane (col, jj = 0)
    } else {
      lsum[rb] += __shfl_xor(lsum[rb], 16, 64);
      lsum[rb] += __shfl_xor(lsum[rb], 32, 64);
    }
    const int row = rblk * ROWS + wv * 16 * RB + rb * 16 + col;
    if (row >= a.rows) continue;
    const int qi = row / a.gqa, h = kh * a.gqa + row % a.gqa;
    // dead rows (past the chunk's width) ran the unmasked steps: write 0
    const float inv = lim[rb] < 0 ? 0.0f : 1.0f / fmaxf(lsum[rb], 1e-20f);
    uint16_t *o = a.out + (((int64_t)b * a.heads + h) * a.nq + qi) * g.dim;
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      float v4[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v4[r] = lim[rb] < 0 ? 0.0f : O[rb][n][r] * inv;
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
  // the block's share of the dead sequences' zero rows, after its own output
  // rows (stores issued before the stages would hold up the first tile
  // loads: vmcnt counts both, in order)
  if constexpr (SHARE) {
    if (share) zero_share(a, s_zero[0], s_zero[1], tid, 64 * kPrefillWaves);
  }
}

// ---- host launcher ------------------------------------------------------------

typedef void (*PrefillKernel)(AttnArgs);

template <bool SHARE>
static PrefillKernel select_prefill(const Geo &g) {
#define PKV_Q(BITS_, DP_, G_)                                                              \
  if (g.bits == BITS_ && g.dp == DP_ && g.group == G_)                                     \
    return g.float_kind == 1 ? prefill_kernel<BITS_, DP_, G_, 1, SHARE> : prefill_kernel<BITS_, DP_, G_, 0, SHARE>;
  PKV_Q(8, 64, 32) PKV_Q(8, 64, 64)
  PKV_Q(8, 128, 32) PKV_Q(8, 128, 64) PKV_Q(8, 128, 128)
  PKV_Q(8, 256, 32) PKV_Q(8, 256, 64) PKV_Q(8, 256, 128)
  PKV_Q(4, 64, 32) PKV_Q(4, 64, 64)
  PKV_Q(4, 128, 32) PKV_Q(4, 128, 64) PKV_Q(4, 128, 128)
  PKV_Q(4, 256, 32) PKV_Q(4, 256, 64) PKV_Q(4, 256, 128)
#undef PKV_Q
#define PKV_F(DP_, FK_) \
  if (g.bits == 16 && g.dp == DP_ && g.float_kind == FK_) return prefill_kernel<16, DP_, 32, FK_, SHARE>;
  PKV_F(64, 0) PKV_F(64, 1) PKV_F(128, 0) PKV_F(128, 1) PKV_F(256, 0) PKV_F(256, 1)
#undef PKV_F
  return nullptr;
}

hipError_t launch_prefill(hipStream_t stream, const AttnArgs &a) {
  // sequences left to the decode kernel: the instantiation that shares their zero rows out
  const PrefillKernel k = a.widths && a.narrow_q > 0 ? select_prefill<true>(a.g) : select_prefill<false>(a.g);
  if (!k) return hipErrorInvalidValue;
  const int rows_per_block = prefill_rows(a.g.dp);
  const int64_t blocks = (int64_t)a.batch * a.g.hk * ((a.rows + rows_per_block - 1) / rows_per_block);
  if (blocks == 0) return hipSuccess;
  if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(64 * prefill_waves(a.g.dp)), 0, stream, a);
  return hipGetLastError();
}

}  // namespace pkv
