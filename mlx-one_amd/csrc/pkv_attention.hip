// pkv_attention.hip -- paged decode / verify attention for gfx950.
//
// Semantics are the reference's (src/mlx_one/engine/paged_attention.py:62-113
// kernel, :127-206 dispatch and merge): query row (q, h) attends tokens
// t <= q_pos[q] of its sequence, KV head kh = h / (H/HK), softmax(q.k*scale).v,
// normaliser floored at 1e-20, rows q >= width give 0.
//
// Work split (stream-K).  The 16-token tiles of every (sequence, KV head)
// segment, in that order, are shared out as equal contiguous runs over a grid
// of resident waves (one 64-thread workgroup each): no wave waits on a ragged
// tail and each pays its start-up latency once.  The split counts `lead`
// extra tiles ahead of each segment for the cost of starting a piece, so a
// run that crosses into another segment holds fewer real tiles.  A wave
// processes the pieces of the segments its run crosses; all R = Q*(H/HK)
// query rows of the KV head share each K/V tile load (GQA reuse).
//
// Column slots.  The 16 columns of a 16x16 MFMA tile hold SLOTS = 16/RPS
// groups of RPS query rows; slot j of an iteration works on tile (SLOTS*it +
// j).  The slot-j query operand is zero outside its columns, so the score
// MFMAs of SLOTS tiles accumulate into one dense 16x16 tile, and every lane's
// softmax work is useful (decode at GQA 4 would otherwise leave 12 of 16
// columns empty).  Each column keeps its own online-softmax state, so the
// SLOTS columns of a row are independent sub-partitions (interleaved tiles)
// merged by log-sum-exp once per unit.
//
// Per iteration (SLOTS tiles of 16 tokens):
//   S^T[t][col] = K.Q^T   v_mfma_f32_16x16x32_f16 over the codes as f16
//                         (1024 + c, one v_perm per two codes); one
//                         accumulator per quantization group, then
//                         s = sum_g scale_g*acc_g + qsum_g*(bias_g - 1024*scale_g)
//   softmax               exp2 domain, online with lazy rescaling: a column's
//                         running max moves only when a score exceeds it by > 8
//   O^T[d][col] += V^T.P' v_mfma_f32_16x16x16_f16 with P'_g = p*scale_v[g]
//                         (V is never dequantized); bias_v enters as
//                         sum p*bias_v, the 1024 offset as 1024*sum P'.
// O is kept transposed (d in rows, columns in lanes): rescaling a column
// touches only the lane's own registers.
//
// Loads.  The page format stores a lane's share of a tile where its MFMA
// operand registers want it (16-byte chunks at tile + c*1024 + lane*16), so K
// and V stream from HBM straight into VGPRs (global_load_dwordx4, no LDS
// staging).  The next iteration's K and score metadata are requested as soon
// as the score MFMAs have consumed the current ones, its V and value metadata
// after the PV MFMAs; the other waves of the CU (one wave per workgroup, no
// LDS, bounded VGPRs) cover the rest of the latency.
// Float (bf16/f16) pages use the same schedule without the affine terms.
// A piece that covers its whole segment writes the normalised output; other
// pieces write (acc, m, l) partials that merge_kernel, launched next on the
// same stream, combines by log-sum-exp (the kernel boundary makes them
// visible across the XCDs' L2s without any cache maintenance in the loop).
#include <atomic>
#include <type_traits>

#include "pkv_mfma.h"
#include "pkv_token.h"

namespace pkv {

// Column slots for a layout: the count the rows allow, halved while the
// per-lane register estimate (payload of SLOTS tiles, metadata, O^T, Q) stays
// above what leaves room for three waves per SIMD.
constexpr int fit_slots(int bits, int dp, int g, int slots) {
  const int lw = dp * bits / 128;
  const int mw = bits != 16 ? 4 * (dp / g) : 0;
  while (slots > 1 && slots * 2 * lw + 2 * mw + dp / 4 + dp / 8 + 40 > 176) slots /= 2;
  return slots;
}

// Shapes whose register needs sit just above 256 VGPRs: asking for two waves
// per SIMD costs them at most a few spills outside the tile loop and doubles
// their occupancy.  Others keep the compiler's choice (heavier shapes would
// spill inside the loop: int8 D256 G128 forced to two waves spilled 98 VGPRs
// and ran 5.6% slower than at one wave per SIMD).
constexpr int min_waves_per_simd(int bits, int dp, int g, int rb, int slots) {
  return (bits == 8 && dp == 128 && g == 64 && rb == 1 && slots == 4) ||
                 (bits == 4 && dp == 128 && g == 32 && rb == 1 && slots == 4) ||
                 (bits == 4 && dp == 128 && g == 64 && rb == 2) ||
                 (bits == 8 && dp == 128 && g == 64 && rb == 2)
             ? 2
             : 1;
}

// Two-row-block kernels dequantize quantized V tiles in registers (see attn_kernel).
constexpr bool kDequantRows = true;

// Waves per run: the kernels for 5-8 rows (two column slots) and 17-32 rows
// (two row blocks) per KV head give each run of the split to a workgroup of
// this many waves, which share its iterations round robin and combine their
// states in LDS at each piece's end; the others (and the fused single-token
// append) run one wave per run.
constexpr int run_waves(int rb, int slots, bool append) { return !append && (rb == 2 || slots == 2) ? 4 : 1; }

// Tiles of a sequence: at least one, so that an empty sequence still owns a
// piece that writes its zero output.
__device__ __forceinline__ int seq_tiles(int len) {
  return len <= 0 ? 1 : (len + PKV_TILE - 1) / PKV_TILE;
}

// Work split.  Split tiles are numbered over (sequence b, KV head kh) in that
// order, T in all: each (b, kh) segment spans `lead` tiles with no data, then
// its own tiles.  Wave w of W (W <= T) owns the run [start(w), start(w+1)):
// equal runs whatever the lengths, so no wave waits on a ragged tail and each
// pays its start-up once.  A run is cut into pieces at segment boundaries; a
// run that holds lead tiles only has no piece.
struct Split {
  int T, W, q, r;  // T tiles over W waves: the first r runs have q + 1 tiles, the rest q
  __device__ __forceinline__ void init(int t, int w) {
    T = t; W = w; q = t / w; r = t - q * w;
  }
  __device__ __forceinline__ int start(int w) const { return w * q + min(w, r); }
  // the wave whose run holds tile g
  __device__ __forceinline__ int wave_of(int g) const {
    const int big = r * (q + 1);
    return g < big ? g / (q + 1) : r + (g - big) / q;
  }
};

// Partial slots: the first piece of wave w's run goes to slot 2w, a later
// (its last) one to 2w+1; pieces in between cover whole segments and write
// the output directly.  A segment starting at split tile sv has its tiles at
// [s0, s1) (s0 = sv + lead); its pieces are those of waves wa .. wa+n-1, and
// wave wa's piece is its first one unless its run started before sv.
struct SegPieces {
  int n, wa, slot0;
  __device__ __forceinline__ int slot(int i) const { return i == 0 ? slot0 : 2 * (wa + i); }
};

__device__ __forceinline__ SegPieces seg_pieces(const Split &sp, int sv, int s0, int s1) {
  SegPieces p;
  p.wa = sp.wave_of(s0);
  p.n = sp.wave_of(s1 - 1) - p.wa + 1;
  p.slot0 = sp.start(p.wa) < sv ? 2 * p.wa + 1 : 2 * p.wa;
  return p;
}

// Tiles the split gives sequence idx (< batch): seq_tiles, or none for a
// sequence of a mixed batch that the prefill kernel serves (its width is past
// narrow_q, the query rows this launch covers).  Served sequences have at
// least one tile, so "served" is "tiles > 0", and only they are charged lead
// tiles.
__device__ __forceinline__ int split_tiles(const int32_t *lens, const int32_t *widths, int narrow_lo,
                                           int narrow_q, int idx) {
  if (narrow_q > 0 && (widths[idx] > narrow_q || widths[idx] <= narrow_lo)) return 0;
  return seq_tiles(lens[idx]);
}

// The lead tiles a launch's split charges ahead of each segment: `lead`, or
// none when the lead-free split's equal runs already end on segment
// boundaries (every sequence's tile count a multiple of the run length), so
// that no run crosses one.  nt0: the lane's tile count in the first
// 64-sequence chunk; t0: the lead-free tile total over all segments.
__device__ __forceinline__ int charged_lead(const int32_t *lens, const int32_t *widths, int narrow_lo,
                                            int narrow_q, int batch, int waves, int lead, int nt0,
                                            int t0, int lane) {
  if (lead == 0 || t0 == 0) return 0;
  const int w0 = min(waves, t0);
  if (t0 % w0) return lead;
  const int q0 = t0 / w0;
  bool off = lane < batch && nt0 % q0 != 0;
  for (int c0 = 64; c0 < batch; c0 += 64) {
    const int idx = c0 + lane;
    off |= idx < batch && split_tiles(lens, widths, narrow_lo, narrow_q, idx) % q0 != 0;
  }
  return __any(off) ? lead : 0;
}

// Log-sum-exp merge of partition partials (paged_attention.py:191-204, in
// the exp2 domain): one NW-wave workgroup (1, 2 or 4 waves, as many as a
// segment's pieces need at 16 per wave) per (segment, query
// row) of a segment split over several waves' runs; whole segments were
// written by the attention kernel.  Every wave finds M = max m and
// S = sum l 2^(m - M) over the pieces (lanes stride the pieces); wave w
// weighs pieces w, w+NW, ..., whose partial rows (lanes stride the DP
// columns, up to 16 in flight) it requests before that pass, and the NW sums
// meet in LDS.  Up to 16*NW pieces the merge is one memory round trip.
template <int DP, int NW>
__global__ __launch_bounds__(64 * NW) void merge_kernel(const MergeArgs a) {
  constexpr int PER = DP / 64 > 0 ? DP / 64 : 1;  // output columns per lane
  constexpr int KW = 16;                          // pieces per wave in flight
  __shared__ float s_acc[NW > 1 ? NW - 1 : 1][64 * PER];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int unit = blockIdx.x;
  const int row = unit % a.rows, seg = unit / a.rows;
  const int b = seg / a.hk, kh = seg % a.hk;
  // tiles (and served sequences) before sequence b, and the launch's split
  // (as the attention kernel made it)
  int pre = 0, spre = 0, tiles = 0, served = 0, nt0 = 0;
  for (int c0 = 0; c0 < a.batch; c0 += 64) {
    const int idx = c0 + lane;
    const int nt = idx < a.batch ? split_tiles(a.seq_lens, a.widths, a.narrow_lo, a.narrow_q, idx) : 0;
    if (c0 == 0) nt0 = nt;
    tiles += wave_sum(nt);
    served += wave_sum(nt > 0 ? 1 : 0);
    pre += wave_sum(idx < b ? nt : 0);
    spre += wave_sum(idx < b && nt > 0 ? 1 : 0);
  }
  const int ntb = split_tiles(a.seq_lens, a.widths, a.narrow_lo, a.narrow_q, b);
  if (ntb == 0) return;  // served by the prefill kernel
  const int t0 = __builtin_amdgcn_readfirstlane(tiles) * a.hk;
  const int lead = charged_lead(a.seq_lens, a.widths, a.narrow_lo, a.narrow_q, a.batch, a.waves, a.lead, nt0,
                                t0, lane);
  const int T = t0 + __builtin_amdgcn_readfirstlane(served) * a.hk * lead;
  const int sv = (__builtin_amdgcn_readfirstlane(pre) + __builtin_amdgcn_readfirstlane(spre) * lead) *
                     a.hk + kh * (ntb + lead);
  Split sp;
  sp.init(T, min(a.waves, T));
  const SegPieces pc = seg_pieces(sp, sv, sv + lead, sv + lead + ntb);
  if (pc.n < 2) return;  // the same for every wave of the workgroup

  // this wave's partial rows of pieces k0 + wv + NW*i, all requested at once
  float x[KW][PER];
  auto request = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < KW; ++i) {
      const int k = k0 + wv + NW * i;
#pragma unroll
      for (int e = 0; e < PER; ++e) x[i][e] = 0.0f;
      if (k < pc.n) {
        const float *src = a.part_acc + ((int64_t)pc.slot(k) * a.rows + row) * DP + lane * PER;
        if constexpr (PER == 4) {
          const f4 v = *(const f4 *)src;
          x[i][0] = v[0]; x[i][1] = v[1]; x[i][2] = v[2]; x[i][3] = v[3];
        } else if constexpr (PER == 2) {
          const float2 v = *(const float2 *)src;
          x[i][0] = v.x; x[i][1] = v.y;
        } else {
          x[i][0] = src[0];
        }
      }
    }
  };
  // The first rows go out before the (m, l) pass: both in one memory round trip.
  request(0);

  // M = max m, S = sum l 2^(m - M) over the pieces (lanes stride the pieces);
  // lane l keeps piece l's (m, l)
  float mx = -INFINITY, sm = 0.0f;
  float2 mine = make_float2(-INFINITY, 0.0f);
  for (int k0 = 0; k0 < pc.n; k0 += 64) {
    const int k = k0 + lane;
    if (k < pc.n) {
      const float2 ml = *(const float2 *)(a.part_ml + ((int64_t)pc.slot(k) * a.rows + row) * 2);
      if (k0 == 0) mine = ml;
      if (ml.y > 0.0f) {  // a piece with no visible token holds l = 0
        const float nm = fmaxf(mx, ml.x);
        sm = sm * __builtin_amdgcn_exp2f(mx - nm) + ml.y * __builtin_amdgcn_exp2f(ml.x - nm);
        mx = nm;
      }
    }
  }
  // combine across lanes: within 16-lane rows by DPP exchanges (the
  // combination is symmetric, so both lanes of a pair hold the same bits),
  // then the four rows' results, read as uniform values, in row order
  auto combine = [&](float om, float os) __attribute__((always_inline)) {
    const float nm = fmaxf(mx, om);
    sm = nm == -INFINITY ? 0.0f
                         : sm * __builtin_amdgcn_exp2f(mx - nm) + os * __builtin_amdgcn_exp2f(om - nm);
    mx = nm;
  };
  combine(row_xchg<0xB1>(mx), row_xchg<0xB1>(sm));
  combine(row_xchg<0x4E>(mx), row_xchg<0x4E>(sm));
  combine(row_xchg<0x141>(mx), row_xchg<0x141>(sm));
  combine(row_xchg<0x140>(mx), row_xchg<0x140>(sm));
  {
    float rm[4], rs[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      rm[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 16 * r));
      rs[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sm), 16 * r));
    }
    mx = rm[0];
    sm = rs[0];
#pragma unroll
    for (int r = 1; r < 4; ++r) combine(rm[r], rs[r]);
  }
  const float inv = 1.0f / fmaxf(sm, 1e-20f);
  // lane l: weight 2^(m - M) / S of piece l
  const float w_first = mine.y > 0.0f ? __builtin_amdgcn_exp2f(mine.x - mx) * inv : 0.0f;
  float acc[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) acc[i] = 0.0f;
  for (int k0 = 0; k0 < pc.n; k0 += NW * KW) {
    if (k0 > 0) request(k0);
    // lane l: weight of piece k0 + l (pieces below 64 from the pass above)
    const bool held = k0 + NW * KW <= 64;
    float wl = w_first;
    if (!held) {
      wl = 0.0f;
      const int k = k0 + lane;
      if (k < pc.n) {
        const float2 ml = *(const float2 *)(a.part_ml + ((int64_t)pc.slot(k) * a.rows + row) * 2);
        wl = ml.y > 0.0f ? __builtin_amdgcn_exp2f(ml.x - mx) * inv : 0.0f;
      }
    }
#pragma unroll
    for (int i = 0; i < KW; ++i) {
      const int src_lane = held ? k0 + wv + NW * i : wv + NW * i;
      const float wk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), src_lane));
#pragma unroll
      for (int e = 0; e < PER; ++e) acc[e] += wk * x[i][e];
    }
  }
  if (wv > 0) {
#pragma unroll
    for (int e = 0; e < PER; ++e) s_acc[wv - 1][lane * PER + e] = acc[e];
  }
  __syncthreads();
  if (wv != 0) return;
  const int qi = row / a.gqa, h = kh * a.gqa + row % a.gqa;
  uint16_t *o = a.out + (((int64_t)b * a.heads + h) * a.nq_stride + qi) * a.dim;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int d = lane * PER + e;
    float v = acc[e];
#pragma unroll
    for (int k = 0; k < NW - 1; ++k) v += s_acc[k][d];
    if (d < a.dim) o[d] = float_to_bits(v, a.float_kind);
  }
}

template <int BITS, int DP, int G, int RB, int FK, int SLOTS, bool APPEND>
__global__ __launch_bounds__(64 * run_waves(RB, SLOTS, APPEND))
__attribute__((amdgpu_waves_per_eu(min_waves_per_simd(BITS, DP, G, RB, SLOTS)))) void attn_kernel(
    const AttnArgs a) {
  using C = Cfg<BITS, DP, G, RB, FK, SLOTS>;
  constexpr bool QUANT = C::QUANT;
  static_assert(!APPEND || (QUANT && RB == 1), "fused append: quantized pages, one row block");
  // Tiles stream in with non-temporal loads for one row block (decode rows:
  // C2 67.7 -> 59.9 us per fused launch); two row blocks (verify) keep plain
  // loads, which let the sequences of a shared prefix meet its pages in L2
  // (C4: 32.8 against 33.8 us with non-temporal loads).
  constexpr bool NT = RB == 1;
  // Quantized V tiles for two row blocks (17-32 query rows per KV head) are
  // dequantized once per tile in registers -- per lane its four tokens,
  // (c - 1024)*scale + bias in f16 as the prefill kernel does -- and the PV
  // contraction takes P itself: with 20 rows the per-group P' operands and
  // bias sums of the undequantized form (AFF) cost more VALU than the
  // elements' conversion.  K stays undequantized at every shape (codes exact
  // in the MFMA, scales applied to the f32 scores), which keeps queries far
  // past unit scale within the bar.
  constexpr bool DEQ = QUANT && RB == 2 && kDequantRows;
  constexpr bool AFF = QUANT && !DEQ;
  constexpr int NG = C::NG, KB = C::KB, NB = C::NB, RPS = C::RPS;
  // MFMA operand types: quantized pages run in f16 (codes as 1024 + c).
  using FO = FloatOps<QUANT ? 1 : FK>;
  using KT = typename FO::KT;
  using VT = typename FO::VT;
  // bf16 pages: P enters the PV MFMA as a bf16 pair hi + lo (16 significant
  // bits).  One bf16 alone is 2^-9 relative, which values of outlier channels
  // (|v| ~ 30) turn into more than the output tolerance on short sequences.
  constexpr bool SPLITP = !QUANT && FK == 0;

  // Lane-derived values are refreshed at every piece through an opaque copy
  // of the lane id, so the compiler recomputes per-lane addresses inside the
  // piece loop instead of hoisting them all and pinning them in registers.
  // Runs of GW waves (GW > 1): wave wk of the workgroup takes iterations wk,
  // wk + GW, ... of each piece of the run.
  constexpr int GW = run_waves(RB, SLOTS, APPEND);
  const int wk = GW > 1 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) : 0;
  int lane = threadIdx.x & 63;
  int col, jj, slot_l, rowc;  // slot_l: this lane's column slot; rowc: its row within the slot
  auto refresh_lane = [&]() __attribute__((always_inline)) {
    asm volatile("" : "+v"(lane));
    col = lane & 15;
    jj = lane >> 4;
    slot_l = col / RPS;
    rowc = col % RPS;
  };
  refresh_lane();
  const int w = blockIdx.x;
  const Geo &g = a.g;
  const int hk = g.hk;
  const int tpp_shift = __builtin_ctz(g.page / PKV_TILE);
  const int tpp_mask = (1 << tpp_shift) - 1;

  // ---- sequences: lanes hold one 64-sequence chunk (length, tiles, inclusive
  // tile prefix over all sequences); chunk_pre / chunk_end bound its prefix
  int cbase = 0, len_l = 0, nt_l = 0, incl_l = 0, chunk_pre = 0, chunk_end = 0, lead = 0;
  auto scan_chunk = [&](int base, int pre) __attribute__((always_inline)) {
    cbase = base;
    chunk_pre = pre;
    incl_l = wave_scan_incl(base + lane < a.batch && nt_l > 0 ? nt_l + lead : 0, lane) + pre;
    chunk_end = __builtin_amdgcn_readlane(incl_l, 63);
  };
  auto load_chunk = [&](int base, int pre) __attribute__((always_inline)) {
    const int idx = base + lane;
    len_l = idx < a.batch ? a.seq_lens[idx] : 0;
    nt_l = idx < a.batch ? split_tiles(a.seq_lens, a.widths, a.narrow_lo, a.narrow_q, idx) : 0;
    scan_chunk(base, pre);
  };
  len_l = lane < a.batch ? a.seq_lens[lane] : 0;
  nt_l = lane < a.batch ? split_tiles(a.seq_lens, a.widths, a.narrow_lo, a.narrow_q, lane) : 0;
  int all_tiles = wave_sum(nt_l), served = wave_sum(nt_l > 0 ? 1 : 0);
  for (int c0 = 64; c0 < a.batch; c0 += 64) {
    const int idx = c0 + lane;
    const int nt = idx < a.batch ? split_tiles(a.seq_lens, a.widths, a.narrow_lo, a.narrow_q, idx) : 0;
    all_tiles += wave_sum(nt);
    served += wave_sum(nt > 0 ? 1 : 0);
  }
  // tile counts fit in int32: the host bounds batch * (max_pages * pages' tiles + 16) * HK
  const int t0 = __builtin_amdgcn_readfirstlane(all_tiles) * hk;
  if (t0 == 0) return;  // every sequence is served by the prefill kernel
  lead = charged_lead(a.seq_lens, a.widths, a.narrow_lo, a.narrow_q, a.batch, a.waves, a.lead, nt_l, t0, lane);
  scan_chunk(0, 0);
  const int T = t0 + __builtin_amdgcn_readfirstlane(served) * hk * lead;
  const int W = min(a.waves, T);
  if (w >= W) return;
  Split sp;
  sp.init(T, W);

  // the segment holding split tile g (uniform): sequence, KV head, length,
  // tiles, and its first split tile (its own tiles start `lead` split tiles later)
  auto locate = [&](int gt, int &pb, int &pkh, int &pL, int &pnt, int &pseg0)
      __attribute__((always_inline)) {
    if (gt < chunk_pre * hk) load_chunk(0, 0);
    while (gt >= chunk_end * hk && cbase + 64 < a.batch) load_chunk(cbase + 64, chunk_end);
    const unsigned long long hit = __ballot(cbase + lane < a.batch && incl_l * hk > gt);
    const int f = hit ? __ffsll((long long)hit) - 1 : 0;
    pb = cbase + f;
    pnt = __builtin_amdgcn_readlane(nt_l, f);
    pL = __builtin_amdgcn_readlane(len_l, f);
    const int span = pnt + lead;
    const int pre = (__builtin_amdgcn_readlane(incl_l, f) - span) * hk;
    pkh = (gt - pre) / span;
    pseg0 = pre + pkh * span;
  };

  // ---- per-piece metadata, requested a piece ahead: page-id window (page
  // win + lane), raw query words and query positions
  auto fetch_window = [&](int pb, int win, int t1) __attribute__((always_inline)) -> int {
    const int p = win + lane;
    int id = -1;
    if (p < a.max_pages && (int64_t)p * g.page < t1) id = a.table[(int64_t)pb * a.max_pages + p];
    return id < a.num_pages ? id : -1;
  };
  auto fetch_q = [&](int pb, int pkh, u4 (&raw)[RB][KB], int (&qp)[RB]) __attribute__((always_inline)) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int row = SLOTS > 1 ? rowc : rb * 16 + col;
      const int rowv = row < a.rows ? row : 0;  // rows past the block load row 0, zeroed later
      const int qi = rowv / a.gqa, h = pkh * a.gqa + rowv % a.gqa;
      const uint16_t *qrow = a.q + (((int64_t)pb * a.heads + h) * a.nq_stride + qi) * g.dim;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const int d0 = 32 * kb + 8 * jj;
        if ((g.dim & 7) == 0) {
          raw[rb][kb] = *(const u4 *)(qrow + (d0 < g.dim ? d0 : 0));
        } else {
          uint16_t e8[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) e8[e] = qrow[d0 + e < g.dim ? d0 + e : 0];
          raw[rb][kb] = u4{(uint32_t)e8[0] | ((uint32_t)e8[1] << 16), (uint32_t)e8[2] | ((uint32_t)e8[3] << 16),
                           (uint32_t)e8[4] | ((uint32_t)e8[5] << 16), (uint32_t)e8[6] | ((uint32_t)e8[7] << 16)};
        }
      }
      qp[rb] = a.q_pos ? a.q_pos[(int64_t)pb * a.nq_stride + qi] : 0;
    }
  };

  // query operands, row limits and per-row score scales of the current piece
  int lim[RB];
  float rsc[RB];
  KT qv[RB][KB];
  KT qsl[SLOTS > 1 ? SLOTS : 1][KB];  // per slot: the lane's query operand in that slot's columns
  float qs[RB][NG];
  // Grouped runs over quantized pages: the GW waves convert a piece's query
  // operands together -- (row block, kb) pair i by wave i % GW -- and share
  // them, with their f16 sums, through LDS (the same values and sums each
  // wave would form); a row whose group sum overflows f16 takes the per-wave
  // scaled conversion below.
  constexpr bool QSHARE = QUANT && GW > 1;
  constexpr int QPAIRS = RB * KB;
  __shared__ u4 s_qop[QSHARE ? QPAIRS : 1][QSHARE ? 64 : 1];
  __shared__ float s_qsum[QSHARE ? QPAIRS : 1][QSHARE ? 64 : 1];
  auto set_queries = [&](int pL, int pwidth, int t1, const u4 (&raw)[RB][KB], const int (&qp)[RB])
      __attribute__((always_inline)) {
    if constexpr (QSHARE) {
#pragma unroll
      for (int i = 0; i < QPAIRS; ++i) {
        if (i % GW != wk) continue;
        const int rb = i / KB, kb = i % KB;
        const int row = SLOTS > 1 ? rowc : rb * 16 + col;
        const bool valid = row < a.rows;
        const int d0 = 32 * kb + 8 * jj;
        const u4 x = raw[rb][kb];
        uint16_t e8[8] = {(uint16_t)(x.x & 0xFFFF), (uint16_t)(x.x >> 16), (uint16_t)(x.y & 0xFFFF),
                          (uint16_t)(x.y >> 16), (uint16_t)(x.z & 0xFFFF), (uint16_t)(x.z >> 16),
                          (uint16_t)(x.w & 0xFFFF), (uint16_t)(x.w >> 16)};
        h8 v;
        float sum = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const _Float16 hv = (_Float16)(bits_to_float(!valid || d0 + e >= g.dim ? (uint16_t)0 : e8[e],
                                                       g.float_kind) * 1.0f);
          v[e] = hv;
          sum += (float)hv;
        }
        s_qop[i][lane] = __builtin_bit_cast(u4, v);
        s_qsum[i][lane] = sum;
      }
      __syncthreads();
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int row = SLOTS > 1 ? rowc : rb * 16 + col;
      const bool valid = row < a.rows;
      const int qi = row / a.gqa;
      const bool live = valid && qi < pwidth;
      const int pos = a.q_pos ? qp[rb] : pL - pwidth + qi;
      lim[rb] = live ? min(pos, t1 - 1) : -1;
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) qs[rb][gi] = 0.0f;
      // f16 operands hold at most 65504: a row of bf16 queries with a larger
      // element (seen as a non-finite group sum) is converted again, scaled by
      // a power of two sc that brings its largest element into [2^14, 2^15)
      // (exact), and the inverse is folded into its softmax scale
      float sc = 1.0f;
      auto convert = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const int d0 = 32 * kb + 8 * jj;
        u4 x = raw[rb][kb];
        uint16_t e8[8] = {(uint16_t)(x.x & 0xFFFF), (uint16_t)(x.x >> 16), (uint16_t)(x.y & 0xFFFF),
                          (uint16_t)(x.y >> 16), (uint16_t)(x.z & 0xFFFF), (uint16_t)(x.z >> 16),
                          (uint16_t)(x.w & 0xFFFF), (uint16_t)(x.w >> 16)};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (!valid || d0 + e >= g.dim) e8[e] = 0;
        if constexpr (QUANT || FK == 1) {
          h8 v;
          float sum = 0.0f;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const _Float16 hv = (_Float16)(bits_to_float(e8[e], g.float_kind) * sc);
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
      };
      if constexpr (QSHARE) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          qv[rb][kb] = __builtin_bit_cast(KT, s_qop[rb * KB + kb][lane]);
          qs[rb][(32 * kb) / G] += s_qsum[rb * KB + kb][lane];
        }
      } else {
        convert();
      }
      if constexpr (QUANT) {
        bool bad = false;
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) bad |= !__builtin_isfinite(qs[rb][gi]);
        if (__any(bad)) {  // rare: bf16 queries past the f16 range
          float mx = 0.0f;
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            const int d0 = 32 * kb + 8 * jj;
            const u4 x = raw[rb][kb];
            const uint32_t w4[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const uint16_t bits = (uint16_t)(w4[e >> 1] >> (16 * (e & 1)));
              if (valid && d0 + e < g.dim) mx = fmaxf(mx, fabsf(bits_to_float(bits, g.float_kind)));
            }
          }
          mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
          mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
          if (mx >= 32768.0f && mx < INFINITY) {
            int ex;
            frexpf(mx, &ex);  // mx in [2^(ex-1), 2^ex)
            sc = ldexpf(1.0f, 15 - ex);
          }
#pragma unroll
          for (int gi = 0; gi < NG; ++gi) qs[rb][gi] = 0.0f;
          convert();
        }
      }
      rsc[rb] = a.scale_log2 / sc;
      if constexpr (QUANT) {
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
          qs[rb][gi] = xor32_add(xor16_add(qs[rb][gi]));
        }
      }
    }
    if constexpr (SLOTS > 1) {
      // slot j's operands, masked once per piece (column slots need one row block)
      const u4 zero = {0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < SLOTS; ++j)
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) qsl[j][kb] = slot_l == j ? qv[0][kb] : __builtin_bit_cast(KT, zero);
    }
  };
  // slot j's query operand: the lane's rows in slot j's columns, zero elsewhere
  auto qop = [&](int j, int rb, int kb) __attribute__((always_inline)) -> KT {
    if constexpr (SLOTS == 1) return qv[rb][kb];
    else return qsl[j][kb];
  };

  // Tiles of iteration `it` of a piece (first tile pta, ntl tiles, page window
  // pwin held in ppid): per slot, the byte offset of its head block in the pool
  // and its tile within the page (uniform); bit j of the returned mask is set
  // when slot j's tile exists.  Loads of absent tiles (past the piece, unmapped
  // pages) read head block kh of page 0; their results are never used.
  auto plan = [&](int pta, int ntl, int pwin, int ppid, int it, int (&pg)[SLOTS], int (&tp)[SLOTS])
      __attribute__((always_inline)) {
    int mask = 0;
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) {
      const int tile = it * SLOTS + j;
      int id = 0, t = 0;
      if (tile < ntl) {
        const int st = pta + tile;
        const int pid_j = __builtin_amdgcn_readlane(ppid, (st >> tpp_shift) - pwin);
        if (pid_j >= 0) {
          id = pid_j;
          t = st & tpp_mask;
          mask |= 1 << j;
        }
      }
      pg[j] = id;
      tp[j] = t;
    }
    return mask;
  };
  // a tile's K payload in the pool (V is g.v_offset further)
  auto tile_at = [&](int pkh, int id, int t) __attribute__((always_inline)) {
    return a.pool + (int64_t)id * g.page_bytes + (int64_t)pkh * g.head_bytes + (int64_t)t * g.tile_bytes;
  };
  // the lane's metadata words: its slot's tile of an iteration as plan()
  // placed it (absent tiles: page 0, tile 0), tokens 4*jj..4*jj+3; the page
  // id comes from plan's uniform values by selects (no lane permute)
  auto meta_at = [&](int pkh, const int (&pg)[SLOTS], const int (&tp)[SLOTS], int64_t side)
      __attribute__((always_inline)) {
    int id = pg[0], t = tp[0];
#pragma unroll
    for (int j = 1; j < SLOTS; ++j) {
      id = slot_l == j ? pg[j] : id;
      t = slot_l == j ? tp[j] : t;
    }
    const int64_t h = (int64_t)pkh * g.head_bytes + (int64_t)id * g.page_bytes;
    return a.pool + h + side + (int64_t)(t * PKV_TILE + 4 * jj) * (NG * 4);
  };

  uint32_t kw[SLOTS][C::LW], vw[SLOTS][C::LW];
  uint32_t km[C::MW], vm[C::MW];
  auto load_k = [&](int pkh, const int (&pg)[SLOTS], const int (&tp)[SLOTS], const uint8_t *mp)
      __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) load_payload<C, NT>(kw[j], tile_at(pkh, pg[j], tp[j]), lane);
    if constexpr (QUANT) load_meta<C, NT>(km, mp);
  };
  auto load_v = [&](int pkh, const int (&pg)[SLOTS], const int (&tp)[SLOTS], const uint8_t *mp)
      __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) load_payload<C, NT>(vw[j], tile_at(pkh, pg[j], tp[j]) + g.v_offset, lane);
    if constexpr (QUANT) load_meta<C, NT>(vm, mp);
  };

  // ---- pieces.  Current: tiles [cta, ctb) of segment (cb, ckh) starting at
  // tile cseg0; the run ends at run_end.  Next (n*): the rest of the run.
  const int run_end = sp.start(w + 1);
  int cb, ckh, cL, cnt, cseg0;
  bool cfirst = true;
  locate(sp.start(w), cb, ckh, cL, cnt, cseg0);
  int cta = max(sp.start(w) - cseg0 - lead, 0);
  int ctb = min(cnt, run_end - cseg0 - lead);
  if (ctb <= 0) return;  // the run holds lead tiles only: no piece
  int cpid = fetch_window(cb, cta >> tpp_shift, min(cL, ctb * PKV_TILE));

  bool has_next = false;
  int nb = 0, nkh = 0, nL = 0, nnt = 1, nta = 0, ntb = 0, npid = -1, nseg0 = 0;

  // next piece: the next segment's tiles up to the run's end, and its
  // page-id window (read at the next switch)
  auto set_next = [&](int gstart) __attribute__((always_inline)) {
    locate(gstart, nb, nkh, nL, nnt, nseg0);
    nta = max(gstart - nseg0 - lead, 0);
    ntb = min(nnt, run_end - nseg0 - lead);
    npid = fetch_window(nb, nta >> tpp_shift, min(nL, ntb * PKV_TILE));
  };

  int pg[SLOTS], npg[SLOTS], tp[SLOTS], ntp[SLOTS];

  // ---- fused single-token append (APPEND).  The wave whose piece holds a
  // segment's last tile quantizes the sequence's new K/V token (it sits at
  // seq_lens - 1) into LDS, stores it into its page slot, and patches its
  // codes and (scale, bias) words into the tile registers of the iteration
  // that holds it; no other wave reads that tile in this launch, so the
  // store needs no ordering against the tile loads.
  __shared__ uint8_t s_app_codes[2][APPEND ? DP : 4];
  __shared__ uint32_t s_app_meta[2][8];
  int app_it = -1, app_j = 0, app_tt = 0;
  // the new rows are requested with the piece's queries, ahead of its tiles
  // (loads return in order)
  constexpr int AEPL = DP / 64;
  uint16_t app_raw[APPEND ? 2 : 1][APPEND ? AEPL : 1];
  int app_pid = -1;
  auto append_fetch = [&](int pb, int pkh, int pos) __attribute__((always_inline)) {
    if constexpr (APPEND) {
      app_pid = a.table[(int64_t)pb * a.max_pages + pos / g.page];
      const int64_t row = ((int64_t)pb * hk + pkh) * g.dim;
#pragma unroll
      for (int side = 0; side < 2; ++side) {
        const uint16_t *src = (side ? a.new_v : a.new_k) + row;
#pragma unroll
        for (int i = 0; i < AEPL; ++i) {
          const int d = lane * AEPL + i;
          app_raw[side][i] = d < g.dim ? src[d] : (uint16_t)0;
        }
      }
    }
  };
  auto append_token = [&](int pkh, int pos, int pta) __attribute__((always_inline)) {
    if constexpr (APPEND) {
      if (app_pid < 0 || app_pid >= a.num_pages) return;  // an unmapped page holds no tile either
#pragma unroll
      for (int side = 0; side < 2; ++side) {
        float x[AEPL];
#pragma unroll
        for (int i = 0; i < AEPL; ++i) {
          const int d = lane * AEPL + i;
          x[i] = d < g.dim ? bits_to_float(app_raw[side][i], g.float_kind) : 0.0f;  // zero pad
        }
        quantize_row<AEPL>(x, lane, G, BITS, s_app_codes[side], s_app_meta[side]);
      }
      wave_lds_sync();
      store_token<DP, BITS>(g, a.wpool + (int64_t)app_pid * g.page_bytes + (int64_t)pkh * g.head_bytes,
                            pos % g.page, s_app_codes[0], s_app_codes[1], s_app_meta[0], s_app_meta[1],
                            lane);
      const int tile = pos / PKV_TILE - pta;  // within the piece
      app_it = tile / SLOTS;
      app_j = tile % SLOTS;
      app_tt = pos % PKV_TILE;
    }
  };
  // the token's K payload (lanes col == tt hold its elements d = 32kb + 8jj + e)
  // and K meta word (lanes of its slot whose four tokens 4jj..4jj+3 hold it)
  auto patch_k = [&]() __attribute__((always_inline)) {
    if constexpr (APPEND) {
      const bool mine = col == app_tt;
#pragma unroll
      for (int j = 0; j < SLOTS; ++j) {
        if (j != app_j) continue;
#pragma unroll
        for (int x = 0; x < C::LW; ++x) {
          uint32_t word = 0;
          if constexpr (BITS == 8) {
            word = *(const uint32_t *)&s_app_codes[0][32 * (x / 2) + 8 * jj + 4 * (x % 2)];
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
              word |= (uint32_t)(s_app_codes[0][32 * x + 8 * jj + e] & 15) << (4 * k4_nibble(e));
          }
          kw[j][x] = mine ? word : kw[j][x];
        }
      }
      const bool mm = slot_l == app_j && jj == app_tt / 4;
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int gi = 0; gi < NG; ++gi)
          if (r == app_tt % 4) km[r * NG + gi] = mm ? s_app_meta[0][gi] : km[r * NG + gi];
    }
  };
  // the token's V payload (lanes jj == tt/4, byte r = tt%4 of each block) and V meta word
  auto patch_v = [&]() __attribute__((always_inline)) {
    if constexpr (APPEND) {
      const int r = app_tt % 4;
      const bool mine = jj == app_tt / 4;
#pragma unroll
      for (int j = 0; j < SLOTS; ++j) {
        if (j != app_j) continue;
        if constexpr (BITS == 8) {
#pragma unroll
          for (int n = 0; n < NB; ++n) {
            const uint32_t sh = 8 * r;
            const uint32_t word = (vw[j][n] & ~(0xFFu << sh)) | ((uint32_t)s_app_codes[1][16 * n + col] << sh);
            vw[j][n] = mine ? word : vw[j][n];
          }
        } else {
#pragma unroll
          for (int m2 = 0; m2 < NB / 2; ++m2) {
            const uint32_t sh = 8 * v4_byte(r);
            const uint32_t byte = (uint32_t)(s_app_codes[1][32 * m2 + col] & 15) |
                                  ((uint32_t)(s_app_codes[1][32 * m2 + 16 + col] & 15) << 4);
            const uint32_t word = (vw[j][m2] & ~(0xFFu << sh)) | (byte << sh);
            vw[j][m2] = mine ? word : vw[j][m2];
          }
        }
      }
      const bool mm = slot_l == app_j && jj == app_tt / 4;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
#pragma unroll
        for (int gi = 0; gi < NG; ++gi)
          if (rr == r) vm[rr * NG + gi] = mm ? s_app_meta[1][gi] : vm[rr * NG + gi];
    }
  };

  // ---- grouped runs: the GW waves' states of a piece meet in LDS (64 KB at
  // head_dim 128, two row blocks).  At the piece's end every wave publishes
  // its rows' maxima, sums and O^T values as its epilogue leaves them (jj
  // lanes and column slots folded; writer lanes); then wave wk combines
  // output columns d in [16*NB/GW*wk, 16*NB/GW*(wk+1)) by log-sum-exp (a wave
  // without a visible token holds l = 0 and weighs nothing) and writes them,
  // normalised (whole segment) or as the run's partial.  (Deferring the
  // combine until the next piece's first loads were issued measured slower:
  // C4 29.6 against 29.1 us.)
  constexpr int GWL = GW > 1 ? GW : 1;
  constexpr int RBL = GW > 1 ? RB : 1;
  constexpr int NBL = GW > 1 ? NB : 1;
  __shared__ f4 s_gO[GWL][RBL][NBL][GW > 1 ? 64 : 1];
  __shared__ float s_gm[GWL][RBL][16], s_gl[GWL][RBL][16];
  auto group_combine = [&](bool whole, int slot, int pb, int pkh) __attribute__((always_inline)) {
    if constexpr (GW > 1) {
      constexpr int NPW = NB / GW;
      static_assert(NPW * GW == NB, "output column blocks per wave");
      __syncthreads();  // every wave's state is published
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        float M = -INFINITY, mk[GW], lk[GW], wt[GW];
#pragma unroll
        for (int k = 0; k < GW; ++k) {
          mk[k] = s_gm[k][rb][col];
          lk[k] = s_gl[k][rb][col];
          if (lk[k] > 0.0f) M = fmaxf(M, mk[k]);
        }
        float L = 0.0f;
#pragma unroll
        for (int k = 0; k < GW; ++k) {
          wt[k] = lk[k] > 0.0f ? __builtin_amdgcn_exp2f(mk[k] - M) : 0.0f;
          L += wt[k] * lk[k];
        }
        const int row = SLOTS > 1 ? rowc : rb * 16 + col;
        const bool writer = slot_l == 0 && row < a.rows;
        const int qi = row / a.gqa, h = pkh * a.gqa + row % a.gqa;
        const float inv = 1.0f / fmaxf(L, 1e-20f);
        uint16_t *o = a.out + (((int64_t)pb * a.heads + h) * a.nq_stride + qi) * g.dim;
        float *pa = a.part_acc + ((int64_t)slot * a.rows + row) * DP;
#pragma unroll
        for (int i = 0; i < NPW; ++i) {
          const int n = wk * NPW + i;
          f4 v = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int k = 0; k < GW; ++k) v += wt[k] * s_gO[k][rb][n][lane];
          const int d = 16 * n + 4 * jj;
          if (!writer) continue;
          if (whole) {
            if ((g.dim & 3) == 0 && d + 4 <= g.dim) {
              u2 packed = {(uint32_t)float_to_bits(v[0] * inv, g.float_kind) |
                               ((uint32_t)float_to_bits(v[1] * inv, g.float_kind) << 16),
                           (uint32_t)float_to_bits(v[2] * inv, g.float_kind) |
                               ((uint32_t)float_to_bits(v[3] * inv, g.float_kind) << 16)};
              *(u2 *)(o + d) = packed;
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (d + r < g.dim) o[d + r] = float_to_bits(v[r] * inv, g.float_kind);
            }
          } else {
            *(f4 *)(pa + d) = v;
          }
        }
        if (wk == 0 && writer && !whole && jj == 0)
          *(float2 *)(a.part_ml + ((int64_t)slot * a.rows + row) * 2) = make_float2(M, L);
      }
      __syncthreads();  // the next piece's states are published over these
    }
  };
  for (;;) {
    refresh_lane();
    // ---- start the piece: query rows and its first tiles, in flight together
    const int width = a.widths ? a.widths[cb] : a.nq;
    const int t0 = cta * PKV_TILE;
    const int t1 = min(cL, ctb * PKV_TILE);
    const int ntl = t1 > t0 ? (t1 - t0 + PKV_TILE - 1) / PKV_TILE : 0;
    const int niters = max(1, (ntl + SLOTS - 1) / SLOTS);
    int cwin = cta >> tpp_shift;
    int cmask;
    const bool appends = APPEND && ctb == cnt && cL > 0;  // the piece holds the segment's last tile
    {
      u4 raw[RB][KB];
      int qp[RB];
      if constexpr (APPEND) {
        if (appends) append_fetch(cb, ckh, cL - 1);
      }
      fetch_q(cb, ckh, raw, qp);
      cmask = plan(cta, ntl, cwin, cpid, wk, pg, tp);
      load_k(ckh, pg, tp, meta_at(ckh, pg, tp, g.kmeta_offset));
      load_v(ckh, pg, tp, meta_at(ckh, pg, tp, g.vmeta_offset));
      set_queries(cL, width, t1, raw, qp);
      // the new token: quantized and stored while the piece's first tiles
      // are in flight (it is patched into the registers of the piece's last
      // iteration)
      if constexpr (APPEND) {
        app_it = -1;
        if (appends) append_token(ckh, cL - 1, cta);
      }
      // the rest of the run is the next piece: its page-id window now
      has_next = ctb == cnt && cseg0 + cnt + 2 * lead < run_end;
      if (has_next) set_next(cseg0 + lead + cnt);
    }

    float m[RB], lsum[RB], corr[RB][NG], osum[RB][NG];
    // Two row blocks of quantized pages take the per-column sums over tokens
    // on the MFMA pipe instead of the VALU: csum = sum p * bias_v (the V bias
    // term) and osum4 = sum P' (the 1024 offset), as 16x16x16 products of the
    // tokens' f16 biases (or ones) with p (or P'); every row of the result
    // holds the column's sum.
    constexpr bool MSUM = RB == 2 && AFF;
    f4 csum[MSUM ? RB : 1][MSUM ? NG : 1], osum4[MSUM ? RB : 1][MSUM ? NG : 1];
    f4 O[RB][NB];  // O^T[d = 16n + 4jj + r][column]
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      m[rb] = -INFINITY;
      lsum[rb] = 0.0f;
#pragma unroll
      for (int n = 0; n < NB; ++n) O[rb][n] = f4{0, 0, 0, 0};
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) { corr[rb][gi] = 0.0f; osum[rb][gi] = 0.0f; }
      if constexpr (MSUM) {
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) { csum[rb][gi] = f4{0, 0, 0, 0}; osum4[rb][gi] = f4{0, 0, 0, 0}; }
      }
    }

    // One iteration over SLOTS tiles; with `more`, the next iteration's tiles
    // are requested as soon as each half's registers are free (the last
    // iteration is peeled so nothing is in flight across the epilogue).
    auto iterate = [&](auto more, int it) __attribute__((always_inline)) {
      constexpr bool MORE = decltype(more)::value;
      refresh_lane();
      // the appended token sits in the piece's last tile, hence in its last
      // iteration (the peeled one): the loop body stays the plain kernel's
      if constexpr (APPEND && !MORE) {
        if (app_it >= 0) patch_k();
      }
      // Float pages: a page reused after another sequence may hold anything
      // past this piece's last token, and the column-slot products multiply
      // a slot's K rows by other slots' zero query columns (and every V row by
      // its P), so 0 * inf would spread.  Those rows are zeroed in registers
      // in the iteration that holds the piece's end.  (Codes are always finite.)
      const bool tail_it = t0 + (it + 1) * SLOTS * PKV_TILE > t1;
      if constexpr (!QUANT) {
        if (tail_it) {
#pragma unroll
          for (int j = 0; j < SLOTS; ++j) {
            const bool dead = t0 + (it * SLOTS + j) * PKV_TILE + col >= t1;
#pragma unroll
            for (int x = 0; x < C::LW; ++x) kw[j][x] = dead ? 0u : kw[j][x];
          }
        }
      }
      // S^T for the iteration's tiles (slot j -> columns of slot j).  Codes
      // are finite whatever a register holds, and an absent tile's columns
      // are masked by select (scores) or hold exact-zero P' operands, so
      // quantized pages with several slots run every slot's products
      // unguarded: straight-line code, no per-tile branches.
      constexpr bool UNGUARDED = QUANT && SLOTS > 1;
      // (unguarded chains start from zeros held in registers: an inline-zero
      // accumulator would let the compiler place a chain's first product over
      // part of its own operands)
      f4 zacc = f4{0, 0, 0, 0};
      if constexpr (UNGUARDED) asm volatile("" : "+v"(zacc));
      f4 acc[RB][NG];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) acc[rb][gi] = zacc;
#pragma unroll
      for (int j = 0; j < SLOTS; ++j) {
        if (UNGUARDED || (cmask & (1 << j))) {
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            KT kop;
            if constexpr (QUANT) {
              kop = Conv<BITS>::template kop<C::LW>(kw[j], kb);
            } else {
              u4 r = {kw[j][4 * kb], kw[j][4 * kb + 1], kw[j][4 * kb + 2], kw[j][4 * kb + 3]};
              kop = __builtin_bit_cast(KT, r);
            }
            const int gi = QUANT ? (32 * kb) / G : 0;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) acc[rb][gi] = FO::qk(kop, qop(j, rb, kb), acc[rb][gi]);
          }
        }
      }
      // scores of the lane's tile (its slot's tile of this iteration)
      const bool my_ok = (cmask >> slot_l) & 1;
      const int tok0 = t0 + (it * SLOTS + slot_l) * PKV_TILE + 4 * jj;
      // One slot: the tile's presence (uniform) folded into the rows'
      // limits, opaque to the compiler, which otherwise branches around every
      // score's assembly (eight branches per tile at two row blocks; C4
      // launch -3.8%).  Several slots keep the per-lane flag (the fold
      // measured 2.5% slower at C3).
      int limv[RB];
      if constexpr (SLOTS == 1) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          limv[rb] = my_ok ? lim[rb] : -1;
          asm volatile("" : "+v"(limv[rb]));
        }
      }
      float s[RB][4];
      bool vis[RB][4];
      bool need = false;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v;
          if constexpr (QUANT) {
#pragma unroll
            for (int gi = 0; gi < NG; ++gi) {
              const uint32_t word = km[r * NG + gi];
              const float ks = f16_bits_to_f32(word);
              const float kbias = f16_bits_to_f32(word >> 16) - 1024.0f * ks;
              const float term = ks * acc[rb][gi][r] + qs[rb][gi] * kbias;
              v = gi == 0 ? term : v + term;  // no 0.0f + term: the add would stay (signed zero)
            }
          } else {
            v = acc[rb][0][r];
          }
          if constexpr (SLOTS == 1) vis[rb][r] = tok0 + r <= limv[rb];
          else vis[rb][r] = my_ok && tok0 + r <= lim[rb];
          v = vis[rb][r] ? v * rsc[rb] : -INFINITY;
          s[rb][r] = v;
          need |= v > m[rb] + kTau;
        }
      // K registers and score metadata are free: request the next iteration's
      int nmask = 0;
      const uint8_t *nmv = nullptr;
      if constexpr (MORE) {
        __builtin_amdgcn_sched_barrier(0);
        const int first = cta + (it + GW) * SLOTS;
        const int last = cta + min((it + GW) * SLOTS + SLOTS, ntl) - 1;
        if ((last >> tpp_shift) - cwin > 63) {
          cwin = first >> tpp_shift;  // the iteration's tiles leave the window: slide it
          cpid = fetch_window(cb, cwin, t1);
        }
        nmask = plan(cta, ntl, cwin, cpid, it + GW, npg, ntp);
        load_k(ckh, npg, ntp, meta_at(ckh, npg, ntp, g.kmeta_offset));
        nmv = meta_at(ckh, npg, ntp, g.vmeta_offset);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (__any(need)) {
        // Until a column sees its first visible token its running max is
        // -inf and its sums and O^T are exact zeros: while that holds for
        // every column (a piece's first iteration), the max moves without
        // the rescale.
        bool fresh = true;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) fresh &= m[rb] == -INFINITY;
        const bool rescale = !__all(fresh);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          float tm = fmaxf(fmaxf(s[rb][0], s[rb][1]), fmaxf(s[rb][2], s[rb][3]));
          tm = xor32_max(xor16_max(tm));
          const float mn = fmaxf(m[rb], tm);
          if (!rescale) {
            m[rb] = mn;
            continue;
          }
          const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m[rb] - mn);
          m[rb] = mn;
          lsum[rb] *= alpha;
#pragma unroll
          for (int gi = 0; gi < NG; ++gi) {
            if constexpr (MSUM) {
              csum[rb][gi] *= alpha;
              osum4[rb][gi] *= alpha;
            } else if constexpr (AFF) {
              corr[rb][gi] *= alpha;
              osum[rb][gi] *= alpha;
            }
          }
#pragma unroll
          for (int n = 0; n < NB; ++n) O[rb][n] *= alpha;
        }
      }
      if constexpr (APPEND && !MORE) {
        if (app_it >= 0) patch_v();
      }
      // probabilities and the P operands (per group for quantized V).  Masked
      // tokens contribute exact zeros through selects, whatever their page
      // holds.  The column-sum products take the tokens' biases as an MFMA
      // operand, so for them the value metadata of tokens the piece does not
      // hold (past its end, absent tiles) is cleared as well.
      uint32_t vmw[MSUM ? C::MW : 1];
      if constexpr (MSUM) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool held = my_ok && tok0 + r < t1;
#pragma unroll
          for (int gi = 0; gi < NG; ++gi) vmw[r * NG + gi] = held ? vm[r * NG + gi] : 0u;
        }
      }
      VT pop[RB][NG];
      VT plo[SPLITP ? RB : 1];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) p[r] = vis[rb][r] ? __builtin_amdgcn_exp2f(s[rb][r] - m[rb]) : 0.0f;
        lsum[rb] += (p[0] + p[1]) + (p[2] + p[3]);
        if constexpr (AFF) {
#pragma unroll
          for (int gi = 0; gi < NG; ++gi) {
            h4 pv;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const uint32_t word = vm[r * NG + gi];
              const _Float16 ps = (_Float16)(p[r] * f16_bits_to_f32(word));
              pv[r] = vis[rb][r] ? ps : (_Float16)0.0f;
              if constexpr (!MSUM) {
                corr[rb][gi] += vis[rb][r] ? p[r] * f16_bits_to_f32(word >> 16) : 0.0f;
                osum[rb][gi] += (float)pv[r];
              }
            }
            pop[rb][gi] = pv;
            if constexpr (MSUM) {
              // A: the lane's four tokens' biases (or ones) for every row; B: p (or P')
              const h4 bias4 = __builtin_bit_cast(
                  h4, u2{perm(vmw[NG + gi], vmw[gi], 0x07060302u), perm(vmw[3 * NG + gi], vmw[2 * NG + gi], 0x07060302u)});
              const h4 p16 = {(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3]};
              const h4 ones = {(_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f};
              csum[rb][gi] = FO::pv(bias4, p16, csum[rb][gi]);
              osum4[rb][gi] = FO::pv(ones, pv, osum4[rb][gi]);
            }
          }
        } else {
          pop[rb][0] = FO::pack_p(p[0], p[1], p[2], p[3]);
          if constexpr (SPLITP) plo[rb] = FO::pack_lo(p[0], p[1], p[2], p[3], pop[rb][0]);
        }
      }
      if constexpr (!QUANT) {
        if (tail_it) {  // V rows past the piece's end (see the K rows above)
#pragma unroll
          for (int j = 0; j < SLOTS; ++j) {
            const int tb = t0 + (it * SLOTS + j) * PKV_TILE + 4 * jj;
            const uint32_t keep01 = (tb < t1 ? 0x0000FFFFu : 0u) | (tb + 1 < t1 ? 0xFFFF0000u : 0u);
            const uint32_t keep23 = (tb + 2 < t1 ? 0x0000FFFFu : 0u) | (tb + 3 < t1 ? 0xFFFF0000u : 0u);
#pragma unroll
            for (int n = 0; n < NB; ++n) {
              vw[j][2 * n] &= keep01;
              vw[j][2 * n + 1] &= keep23;
            }
          }
        }
      }
      if constexpr (DEQ) {
        static_assert(SLOTS == 1, "dequantized V rows take one column slot");
        if (tail_it) {
          // the lane's tokens past the piece's end (stale page bytes): scale
          // and bias 0, so they dequantize to exact zeros (one select per
          // word here rather than a branch per column block below)
          const int tb = t0 + it * PKV_TILE + 4 * jj;
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int gi = 0; gi < NG; ++gi) vm[r * NG + gi] = tb + r < t1 ? vm[r * NG + gi] : 0u;
        }
      }
      // O^T += V^T . P'^T for each tile
#pragma unroll
      for (int j = 0; j < SLOTS; ++j) {
        if (UNGUARDED || (cmask & (1 << j))) {
          VT bop[RB][NG], blo[SPLITP ? RB : 1];
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) {
            const u2 zero = {0, 0};
#pragma unroll
            for (int gi = 0; gi < NG; ++gi)
              bop[rb][gi] = (SLOTS == 1 || slot_l == j) ? pop[rb][gi] : __builtin_bit_cast(VT, zero);
            if constexpr (SPLITP) blo[rb] = (SLOTS == 1 || slot_l == j) ? plo[rb] : __builtin_bit_cast(VT, zero);
          }
#pragma unroll
          for (int n = 0; n < NB; ++n) {
            VT vop;
            if constexpr (DEQ) {
              // the lane's four tokens 4jj..4jj+3 of column 16n + col,
              // dequantized (tokens past the piece's end: zero metadata)
              const int gi = (16 * n) / G;
              h4 sc, bi;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const h2 sb = __builtin_bit_cast(h2, vm[r * NG + gi]);
                sc[r] = sb.x;
                bi[r] = sb.y;
              }
              const h4 c = Conv<BITS>::template vop<C::LW>(vw[j], n);
              vop = __builtin_bit_cast(VT, __builtin_elementwise_fma(c - (_Float16)1024.0f, sc, bi));
            } else if constexpr (QUANT) {
              vop = Conv<BITS>::template vop<C::LW>(vw[j], n);
            } else {
              u2 r = {vw[j][2 * n], vw[j][2 * n + 1]};
              vop = __builtin_bit_cast(VT, r);
            }
            const int gi = AFF ? (16 * n) / G : 0;
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
              O[rb][n] = FO::pv(vop, bop[rb][gi], O[rb][n]);
              if constexpr (SPLITP) O[rb][n] = FO::pv(vop, blo[rb], O[rb][n]);
            }
          }
        }
      }
      // V registers and value metadata are free: request the next iteration's
      if constexpr (MORE) {
        __builtin_amdgcn_sched_barrier(0);
        load_v(ckh, npg, ntp, nmv);
        __builtin_amdgcn_sched_barrier(0);
        cmask = nmask;
#pragma unroll
        for (int j = 0; j < SLOTS; ++j) { pg[j] = npg[j]; tp[j] = ntp[j]; }
      }
    };
    if constexpr (GW == 1) {
      for (int it = 0; it + 1 < niters; ++it) iterate(std::true_type(), it);
      iterate(std::false_type(), niters - 1);
    } else if (wk < niters) {  // (uniform per wave) a wave past the piece's iterations holds nothing
      const int last = wk + GW * ((niters - 1 - wk) / GW);
      for (int it = wk; it < last; it += GW) iterate(std::true_type(), it);
      iterate(std::false_type(), last);
    }

    // ---- piece epilogue: fold the 4 jj lanes of a column, then the slots of a
    // row, and write the output (whole segment) or the partial
    const bool whole = cta == 0 && ctb == cnt;
    const int slot = cfirst ? 2 * w : 2 * w + 1;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      lsum[rb] = xor32_add(xor16_add(lsum[rb]));
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        if constexpr (MSUM) {  // already summed over the tokens of every lane
          corr[rb][gi] = csum[rb][gi][0];
          osum[rb][gi] = osum4[rb][gi][0];
        } else if constexpr (AFF) {
          corr[rb][gi] = xor32_add(xor16_add(corr[rb][gi]));
          osum[rb][gi] = xor32_add(xor16_add(osum[rb][gi]));
        }
      }
      float mrow = m[rb], lrow = lsum[rb], wgt = 1.0f;
      if constexpr (SLOTS > 1) {
        // the row's slot columns (lanes col, col +- RPS, ...) merge by log-sum-exp
#pragma unroll
        for (int o = RPS; o < 16; o <<= 1) mrow = fmaxf(mrow, __shfl_xor(mrow, o, 64));
        wgt = lsum[rb] > 0.0f ? __builtin_amdgcn_exp2f(m[rb] - mrow) : 0.0f;
        lrow = wgt * lsum[rb];
#pragma unroll
        for (int o = RPS; o < 16; o <<= 1) lrow += __shfl_xor(lrow, o, 64);
      }
      const int row = SLOTS > 1 ? rowc : rb * 16 + col;
      const bool writer = slot_l == 0 && row < a.rows;
      const int qi = row / a.gqa, h = ckh * a.gqa + row % a.gqa;
      const float inv = 1.0f / fmaxf(lrow, 1e-20f);
      uint16_t *o = a.out + (((int64_t)cb * a.heads + h) * a.nq_stride + qi) * g.dim;
      float *pa = a.part_acc + ((int64_t)slot * a.rows + row) * DP;
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        float v4[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = O[rb][n][r];
          if constexpr (AFF) {
            const int gi = (16 * n) / G;
            v += corr[rb][gi] - 1024.0f * osum[rb][gi];
          }
          v *= wgt;
          if constexpr (SLOTS > 1) {
#pragma unroll
            for (int o2 = RPS; o2 < 16; o2 <<= 1) v += __shfl_xor(v, o2, 64);
          }
          v4[r] = v;
        }
        if constexpr (GW > 1) {  // published; the group's combine writes
          s_gO[wk][rb][n][lane] = f4{v4[0], v4[1], v4[2], v4[3]};
          continue;
        }
        if (!writer) continue;
        const int d = 16 * n + 4 * jj;
        if (whole) {
          if ((g.dim & 3) == 0 && d + 4 <= g.dim) {
            u2 packed = {(uint32_t)float_to_bits(v4[0] * inv, g.float_kind) |
                             ((uint32_t)float_to_bits(v4[1] * inv, g.float_kind) << 16),
                         (uint32_t)float_to_bits(v4[2] * inv, g.float_kind) |
                             ((uint32_t)float_to_bits(v4[3] * inv, g.float_kind) << 16)};
            *(u2 *)(o + d) = packed;
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (d + r < g.dim) o[d + r] = float_to_bits(v4[r] * inv, g.float_kind);
          }
        } else {
          *(f4 *)(pa + d) = f4{v4[0], v4[1], v4[2], v4[3]};
        }
      }
      if constexpr (GW > 1) {
        if (jj == 0) {
          s_gm[wk][rb][col] = mrow;
          s_gl[wk][rb][col] = lrow;
        }
      } else if (writer && !whole && jj == 0) {
        *(float2 *)(a.part_ml + ((int64_t)slot * a.rows + row) * 2) = make_float2(mrow, lrow);
      }
    }
    if constexpr (GW > 1) group_combine(whole, slot, cb, ckh);

    // ---- switch to the next piece
    if (!has_next) break;
    cb = nb; ckh = nkh; cL = nL; cnt = nnt; cseg0 = nseg0; cta = nta; ctb = ntb;
    cfirst = false; cpid = npid;
  }

}

// ---- VALU decode kernel --------------------------------------------------------
//
// The vector-ALU counterpart of attn_kernel for quantized pages, head_dim up
// to 128 and at most 4 query rows per KV head (single-token decode at GQA <=
// 4), chosen with pkv_select_decode_kernel.  The work split, pieces,
// partials (combined by merge_kernel), page-id windows and load schedule are
// attn_kernel's (two or four tiles per iteration); the products run as
// v_dot2_f32_f16 over f16 pairs (codes as 1024 + c, f32 accumulation)
// instead of MFMAs, with the same affine terms and the same f16 P'.
//
// Lane l = tok + 16*jj.  Scores: the K payload gives lane l token tok's
// elements d = 32kb + 8jj + e; the lane dots them with all four query rows,
// one sum per quantization group, and a butterfly over the jj lanes
// (v_permlane32_swap, then v_permlane16_swap) leaves lane l with token tok's
// sums for query row jj.  The 16 lanes of row jj share the row's running
// max.  Values: the V payload gives lane l = col + 16*jj tokens 4jj..4jj+3 at
// d = 16n + col; the lane fetches P' of those tokens for every row
// (ds_bpermute of f16 pairs that neighbouring token lanes formed) and
// accumulates O[row][d]; at the piece's end the same butterfly folds the jj
// lanes' sums and leaves lane l row jj.
template <int BITS, int DP, int G>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void valu_kernel(const AttnArgs a) {
  using C = Cfg<BITS, DP, G, 1, 1, 4>;
  constexpr int NG = C::NG, KB = C::KB, NB = C::NB, LW = C::LW;
  // tiles per iteration: four at 4-bit with up to two groups per row, else
  // two (payload and metadata registers of four tiles beside the four rows'
  // query operands would spill)
  constexpr int TPI = LW >= 8 || NG > 2 ? 2 : 4;
  constexpr int R = 4;  // query rows per KV head, one per jj lane group
  static_assert(BITS != 16 && DP <= 128, "VALU decode kernel: quantized pages, head_dim <= 128");
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  // Codes -> f16 pairs (1024 + c) as 32-bit words, the formulas of Conv<BITS>.
  // Kept as plain words: built as a half vector and taken apart again before
  // v_dot2, the high pair of a V word was dropped by this compiler (both
  // products read the low pair).
  auto kpairs = [](const uint32_t(&w)[LW], int kb, uint32_t(&o)[4]) __attribute__((always_inline)) {
    if constexpr (BITS == 8) {
      const uint32_t w0 = w[2 * kb], w1 = w[2 * kb + 1];
      o[0] = perm(w0, kMagic, kSelLo); o[1] = perm(w0, kMagic, kSelHi);
      o[2] = perm(w1, kMagic, kSelLo); o[3] = perm(w1, kMagic, kSelHi);
    } else {
      const uint32_t x = w[kb];
      const uint32_t ev = x & 0x0F0F0F0Fu, od = (x >> 4) & 0x0F0F0F0Fu;
      o[0] = perm(ev, kMagic, kNibLo); o[1] = perm(od, kMagic, kNibLo);
      o[2] = perm(ev, kMagic, kNibHi); o[3] = perm(od, kMagic, kNibHi);
    }
  };
  auto vpairs = [](const uint32_t(&w)[LW], int n, uint32_t &lo, uint32_t &hi) __attribute__((always_inline)) {
    if constexpr (BITS == 8) {
      lo = perm(w[n], kMagic, kSelLo);
      hi = perm(w[n], kMagic, kSelHi);
    } else {
      const uint32_t x = w[n >> 1];
      const uint32_t nb = (n & 1) ? (x >> 4) & 0x0F0F0F0Fu : x & 0x0F0F0F0Fu;
      lo = perm(nb, kMagic, kNibLo);
      hi = perm(nb, kMagic, kNibHi);
    }
  };

  int lane = threadIdx.x;
  int tok, jj;
  auto refresh_lane = [&]() __attribute__((always_inline)) {
    asm volatile("" : "+v"(lane));
    tok = lane & 15;
    jj = lane >> 4;
  };
  refresh_lane();
  const int w = blockIdx.x;
  const Geo &g = a.g;
  const int hk = g.hk;
  const int tpp_shift = __builtin_ctz(g.page / PKV_TILE);
  const int tpp_mask = (1 << tpp_shift) - 1;

  // ---- sequences and the split: as attn_kernel
  int cbase = 0, len_l = 0, nt_l = 0, incl_l = 0, chunk_pre = 0, chunk_end = 0, lead = 0;
  auto scan_chunk = [&](int base, int pre) __attribute__((always_inline)) {
    cbase = base;
    chunk_pre = pre;
    incl_l = wave_scan_incl(base + lane < a.batch && nt_l > 0 ? nt_l + lead : 0, lane) + pre;
    chunk_end = __builtin_amdgcn_readlane(incl_l, 63);
  };
  auto load_chunk = [&](int base, int pre) __attribute__((always_inline)) {
    const int idx = base + lane;
    len_l = idx < a.batch ? a.seq_lens[idx] : 0;
    nt_l = idx < a.batch ? split_tiles(a.seq_lens, a.widths, a.narrow_lo, a.narrow_q, idx) : 0;
    scan_chunk(base, pre);
  };
  len_l = lane < a.batch ? a.seq_lens[lane] : 0;
  nt_l = lane < a.batch ? split_tiles(a.seq_lens, a.widths, a.narrow_lo, a.narrow_q, lane) : 0;
  int all_tiles = wave_sum(nt_l), served = wave_sum(nt_l > 0 ? 1 : 0);
  for (int c0 = 64; c0 < a.batch; c0 += 64) {
    const int idx = c0 + lane;
    const int nt = idx < a.batch ? split_tiles(a.seq_lens, a.widths, a.narrow_lo, a.narrow_q, idx) : 0;
    all_tiles += wave_sum(nt);
    served += wave_sum(nt > 0 ? 1 : 0);
  }
  const int t0 = __builtin_amdgcn_readfirstlane(all_tiles) * hk;
  if (t0 == 0) return;
  lead = charged_lead(a.seq_lens, a.widths, a.narrow_lo, a.narrow_q, a.batch, a.waves, a.lead, nt_l, t0, lane);
  scan_chunk(0, 0);
  const int T = t0 + __builtin_amdgcn_readfirstlane(served) * hk * lead;
  const int W = min(a.waves, T);
  if (w >= W) return;
  Split sp;
  sp.init(T, W);

  auto locate = [&](int gt, int &pb, int &pkh, int &pL, int &pnt, int &pseg0)
      __attribute__((always_inline)) {
    if (gt < chunk_pre * hk) load_chunk(0, 0);
    while (gt >= chunk_end * hk && cbase + 64 < a.batch) load_chunk(cbase + 64, chunk_end);
    const unsigned long long hit = __ballot(cbase + lane < a.batch && incl_l * hk > gt);
    const int f = hit ? __ffsll((long long)hit) - 1 : 0;
    pb = cbase + f;
    pnt = __builtin_amdgcn_readlane(nt_l, f);
    pL = __builtin_amdgcn_readlane(len_l, f);
    const int span = pnt + lead;
    const int pre = (__builtin_amdgcn_readlane(incl_l, f) - span) * hk;
    pkh = (gt - pre) / span;
    pseg0 = pre + pkh * span;
  };
  auto fetch_window = [&](int pb, int win, int t1) __attribute__((always_inline)) -> int {
    const int p = win + lane;
    int id = -1;
    if (p < a.max_pages && (int64_t)p * g.page < t1) id = a.table[(int64_t)pb * a.max_pages + p];
    return id < a.num_pages ? id : -1;
  };

  // ---- query rows: every row's elements d = 32kb + 8jj + e, as raw words
  // in the operand registers (converted in place by set_queries)
  uint32_t qw[R][KB][4];  // plain words: see kpairs
  auto fetch_row = [&](int pb, int pkh, int r) __attribute__((always_inline)) {
    const int rowv = r < a.rows ? r : 0;  // rows past the block load row 0, zeroed later
    const int qi = rowv / a.gqa, h = pkh * a.gqa + rowv % a.gqa;
    const uint16_t *qrow = a.q + (((int64_t)pb * a.heads + h) * a.nq_stride + qi) * g.dim;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int d0 = 32 * kb + 8 * jj;
      if ((g.dim & 7) == 0) {
        const u4 x = *(const u4 *)(qrow + (d0 < g.dim ? d0 : 0));
        qw[r][kb][0] = x.x; qw[r][kb][1] = x.y; qw[r][kb][2] = x.z; qw[r][kb][3] = x.w;
      } else {
        uint16_t e8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) e8[e] = qrow[d0 + e < g.dim ? d0 + e : 0];
#pragma unroll
        for (int p = 0; p < 4; ++p) qw[r][kb][p] = (uint32_t)e8[2 * p] | ((uint32_t)e8[2 * p + 1] << 16);
      }
    }
  };
  auto fetch_q = [&](int pb, int pkh, int &qp) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < R; ++r) fetch_row(pb, pkh, r);
    const int rj = jj < a.rows ? jj : 0;
    qp = a.q_pos ? a.q_pos[(int64_t)pb * a.nq_stride + rj / a.gqa] : 0;
  };

  // f16 query operands of every row (in place); limit, group sums and score
  // scale of the lane's row jj
  int lim;
  float rsc, qsj[NG];
  auto set_queries = [&](int pb, int pkh, int pL, int pwidth, int t1, int qp) __attribute__((always_inline)) {
    float rs[R], qs[R][NG];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const bool valid = r < a.rows;
      // f16 operands hold at most 65504: a row of bf16 queries with a larger
      // element (a non-finite group sum) is read and converted again, scaled
      // by a power of two sc that brings its largest element into
      // [2^14, 2^15) (exact), and the inverse is folded into its score scale
      auto convert = [&](float sc) __attribute__((always_inline)) {
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) qs[r][gi] = 0.0f;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const int d0 = 32 * kb + 8 * jj;
          const uint32_t w4[4] = {qw[r][kb][0], qw[r][kb][1], qw[r][kb][2], qw[r][kb][3]};
          uint32_t o4[4];
          float sum = 0.0f;
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            uint32_t pair = 0;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int e = 2 * p + h;
              const uint16_t bits = (uint16_t)(w4[p] >> (16 * h));
              const bool in = valid && d0 + e < g.dim;
              const _Float16 hv = in ? (_Float16)(bits_to_float(bits, g.float_kind) * sc) : (_Float16)0.0f;
              sum += (float)hv;
              pair |= (uint32_t)__builtin_bit_cast(uint16_t, hv) << (16 * h);
            }
            o4[p] = pair;
          }
          qs[r][(32 * kb) / G] += sum;
#pragma unroll
          for (int p = 0; p < 4; ++p) qw[r][kb][p] = o4[p];
        }
      };
      convert(1.0f);
      float sc = 1.0f;
      bool bad = false;
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) bad |= !__builtin_isfinite(qs[r][gi]);
      if (__any(bad)) {  // rare: bf16 queries past the f16 range
        fetch_row(pb, pkh, r);
        float mx = 0.0f;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const int d0 = 32 * kb + 8 * jj;
          const uint32_t w4[4] = {qw[r][kb][0], qw[r][kb][1], qw[r][kb][2], qw[r][kb][3]};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint16_t bits = (uint16_t)(w4[e >> 1] >> (16 * (e & 1)));
            if (valid && d0 + e < g.dim) mx = fmaxf(mx, fabsf(bits_to_float(bits, g.float_kind)));
          }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        if (mx >= 32768.0f && mx < INFINITY) {
          int ex;
          frexpf(mx, &ex);
          sc = ldexpf(1.0f, 15 - ex);
        }
        convert(sc);
      }
      rs[r] = a.scale_log2 / sc;
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        qs[r][gi] += __shfl_xor(qs[r][gi], 16, 64);
        qs[r][gi] += __shfl_xor(qs[r][gi], 32, 64);
      }
    }
    // the lane's row jj
    const int qi = jj / a.gqa;
    const bool live = jj < a.rows && qi < pwidth;
    const int pos = a.q_pos ? qp : pL - pwidth + qi;
    lim = live ? min(pos, t1 - 1) : -1;
    rsc = jj == 0 ? rs[0] : jj == 1 ? rs[1] : jj == 2 ? rs[2] : rs[3];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi)
      qsj[gi] = jj == 0 ? qs[0][gi] : jj == 1 ? qs[1][gi] : jj == 2 ? qs[2][gi] : qs[3][gi];
  };

  // rows r0..r3 summed over the jj lanes; lane l receives row jj's sum
  auto fold_rows = [](float r0, float r1, float r2, float r3) __attribute__((always_inline)) -> float {
    const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(r0), __float_as_uint(r2), false, false);
    const auto y = __builtin_amdgcn_permlane32_swap(__float_as_uint(r1), __float_as_uint(r3), false, false);
    const float a0 = __uint_as_float(x[0]) + __uint_as_float(x[1]);  // rows 0 | 2 (lanes < 32 | >= 32)
    const float a1 = __uint_as_float(y[0]) + __uint_as_float(y[1]);  // rows 1 | 3
    const auto z = __builtin_amdgcn_permlane16_swap(__float_as_uint(a0), __float_as_uint(a1), false, false);
    return __uint_as_float(z[0]) + __uint_as_float(z[1]);
  };

  // tiles of iteration `it` (as attn_kernel's plan)
  auto plan = [&](int pta, int ntl, int pwin, int ppid, int it, int (&pg)[TPI], int (&tp)[TPI])
      __attribute__((always_inline)) {
    int mask = 0;
#pragma unroll
    for (int j = 0; j < TPI; ++j) {
      const int tile = it * TPI + j;
      int id = 0, t = 0;
      if (tile < ntl) {
        const int st = pta + tile;
        const int pid_j = __builtin_amdgcn_readlane(ppid, (st >> tpp_shift) - pwin);
        if (pid_j >= 0) {
          id = pid_j;
          t = st & tpp_mask;
          mask |= 1 << j;
        }
      }
      pg[j] = id;
      tp[j] = t;
    }
    return mask;
  };
  auto head_at = [&](int pkh, int id) __attribute__((always_inline)) {
    return a.pool + (int64_t)id * g.page_bytes + (int64_t)pkh * g.head_bytes;
  };

  uint32_t kw[TPI][LW], vw[TPI][LW];
  uint32_t km[TPI][NG], vm[TPI][NG];  // the lane's token's (scale, bias) words per group
  auto load_tok_meta = [&](uint32_t (&mw)[NG], const uint8_t *p) __attribute__((always_inline)) {
    if constexpr (NG == 1) {
      mw[0] = *(const uint32_t *)p;
    } else if constexpr (NG == 2) {
      const u2 x = *(const u2 *)p;
      mw[0] = x.x; mw[1] = x.y;
    } else {
      const u4 x = *(const u4 *)p;
      mw[0] = x.x; mw[1] = x.y; mw[2] = x.z; mw[3] = x.w;
    }
  };
  auto load_k = [&](int pkh, const int (&pg)[TPI], const int (&tp)[TPI]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < TPI; ++j) {
      const uint8_t *hb = head_at(pkh, pg[j]);
      load_payload<C>(kw[j], hb + (int64_t)tp[j] * g.tile_bytes, lane);
      load_tok_meta(km[j], hb + g.kmeta_offset + (int64_t)(tp[j] * PKV_TILE + tok) * (NG * 4));
    }
  };
  auto load_v = [&](int pkh, const int (&pg)[TPI], const int (&tp)[TPI]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < TPI; ++j) {
      const uint8_t *hb = head_at(pkh, pg[j]);
      load_payload<C>(vw[j], hb + g.v_offset + (int64_t)tp[j] * g.tile_bytes, lane);
      load_tok_meta(vm[j], hb + g.vmeta_offset + (int64_t)(tp[j] * PKV_TILE + tok) * (NG * 4));
    }
  };

  // ---- pieces (as attn_kernel)
  const int run_end = sp.start(w + 1);
  int cb, ckh, cL, cnt, cseg0;
  bool cfirst = true;
  locate(sp.start(w), cb, ckh, cL, cnt, cseg0);
  int cta = max(sp.start(w) - cseg0 - lead, 0);
  int ctb = min(cnt, run_end - cseg0 - lead);
  if (ctb <= 0) return;
  int cpid = fetch_window(cb, cta >> tpp_shift, min(cL, ctb * PKV_TILE));

  bool has_next = false;
  int nb = 0, nkh = 0, nL = 0, nnt = 1, nta = 0, ntb = 0, npid = -1, nseg0 = 0;
  auto set_next = [&](int gstart) __attribute__((always_inline)) {
    locate(gstart, nb, nkh, nL, nnt, nseg0);
    nta = max(gstart - nseg0 - lead, 0);
    ntb = min(nnt, run_end - nseg0 - lead);
    npid = fetch_window(nb, nta >> tpp_shift, min(nL, ntb * PKV_TILE));
  };

  int pg[TPI], npg[TPI], tp[TPI], ntp[TPI];

  for (;;) {
    refresh_lane();
    const int width = a.widths ? a.widths[cb] : a.nq;
    const int t0 = cta * PKV_TILE;
    const int t1 = min(cL, ctb * PKV_TILE);
    const int ntl = t1 > t0 ? (t1 - t0 + PKV_TILE - 1) / PKV_TILE : 0;
    const int niters = max(1, (ntl + TPI - 1) / TPI);
    int cwin = cta >> tpp_shift;
    int cmask;
    {
      int qp;
      fetch_q(cb, ckh, qp);
      cmask = plan(cta, ntl, cwin, cpid, 0, pg, tp);
      load_k(ckh, pg, tp);
      load_v(ckh, pg, tp);
      set_queries(cb, ckh, cL, width, t1, qp);
      has_next = ctb == cnt && cseg0 + cnt + 2 * lead < run_end;
      if (has_next) set_next(cseg0 + lead + cnt);
    }
    // P' pair sources: tokens 4jj, 4jj+1 (A) and 4jj+2, 4jj+3 (B) of row r sit
    // in lanes 16r + 4jj and 16r + 4jj + 2 (byte addresses for ds_bpermute)
    const int srcA = 4 * (4 * jj), srcB = 4 * (4 * jj + 2);

    int cmask_next = 0;
    float m = -INFINITY, lsum = 0.0f, corr[NG], osum[NG];
    float O[R][NB];  // O[row][d = 16n + col], partial over the lane's tokens
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) { corr[gi] = 0.0f; osum[gi] = 0.0f; }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int n = 0; n < NB; ++n) O[r][n] = 0.0f;

    auto iterate = [&](auto more, int it) __attribute__((always_inline)) {
      constexpr bool MORE = decltype(more)::value;
      refresh_lane();
      // scores of the lane's token in each tile, row jj
      float s[TPI];
      bool vis[TPI];
      bool need = false;
#pragma unroll
      for (int j = 0; j < TPI; ++j) {
        s[j] = -INFINITY;
        vis[j] = false;
        if (cmask & (1 << j)) {
          float acc[R][NG];
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int gi = 0; gi < NG; ++gi) acc[r][gi] = 0.0f;
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            uint32_t kx[4];
            kpairs(kw[j], kb, kx);
            const int gi = (32 * kb) / G;
#pragma unroll
            for (int r = 0; r < R; ++r) {
              float t = acc[r][gi];
#pragma unroll
              for (int p = 0; p < 4; ++p)
                t = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, qw[r][kb][p]), __builtin_bit_cast(h2, kx[p]), t,
                                           false);
              acc[r][gi] = t;
            }
          }
          float v;
#pragma unroll
          for (int gi = 0; gi < NG; ++gi) {
            const float sg = fold_rows(acc[0][gi], acc[1][gi], acc[2][gi], acc[3][gi]);
            const uint32_t word = km[j][gi];
            const float ks = f16_bits_to_f32(word);
            const float kbias = f16_bits_to_f32(word >> 16) - 1024.0f * ks;
            const float term = ks * sg + qsj[gi] * kbias;
            v = gi == 0 ? term : v + term;
          }
          vis[j] = t0 + (it * TPI + j) * PKV_TILE + tok <= lim;
          s[j] = vis[j] ? v * rsc : -INFINITY;
          need |= s[j] > m + kTau;
        }
      }
      // K registers are free: request the next iteration's
      if constexpr (MORE) {
        __builtin_amdgcn_sched_barrier(0);
        const int first = cta + (it + 1) * TPI;
        const int last = cta + min((it + 1) * TPI + TPI, ntl) - 1;
        if ((last >> tpp_shift) - cwin > 63) {
          cwin = first >> tpp_shift;
          cpid = fetch_window(cb, cwin, t1);
        }
        const int nmask = plan(cta, ntl, cwin, cpid, it + 1, npg, ntp);
#pragma unroll
        for (int j = 0; j < TPI; ++j) {
          const uint8_t *hb = head_at(ckh, npg[j]);
          load_payload<C>(kw[j], hb + (int64_t)ntp[j] * g.tile_bytes, lane);
          load_tok_meta(km[j], hb + g.kmeta_offset + (int64_t)(ntp[j] * PKV_TILE + tok) * (NG * 4));
        }
        __builtin_amdgcn_sched_barrier(0);
        cmask_next = nmask;
      }
      if (__any(need)) {
        float tm = s[0];
#pragma unroll
        for (int j = 1; j < TPI; ++j) tm = fmaxf(tm, s[j]);
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) tm = fmaxf(tm, __shfl_xor(tm, o, 64));
        const float mn = fmaxf(m, tm);
        const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
        m = mn;
        lsum *= alpha;
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) { corr[gi] *= alpha; osum[gi] *= alpha; }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float ar = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), 16 * r));
#pragma unroll
          for (int n = 0; n < NB; ++n) O[r][n] *= ar;
        }
      }
      // probabilities, P' pairs and the bias terms of the lane's token
      uint32_t pp[TPI][NG];
#pragma unroll
      for (int j = 0; j < TPI; ++j) {
        const float p = vis[j] ? __builtin_amdgcn_exp2f(s[j] - m) : 0.0f;
        lsum += p;
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
          const uint32_t word = vm[j][gi];
          const _Float16 ps = vis[j] ? (_Float16)(p * f16_bits_to_f32(word)) : (_Float16)0.0f;
          corr[gi] += vis[j] ? p * f16_bits_to_f32(word >> 16) : 0.0f;
          osum[gi] += (float)ps;
          const uint32_t own = __builtin_bit_cast(uint16_t, ps);
          const uint32_t nbr = (uint32_t)__shfl_xor((int)own, 1, 64);
          pp[j][gi] = own | (nbr << 16);  // (P'[tok], P'[tok + 1]) in even-tok lanes
        }
      }
      // O[row][d] += P'[row][t] * (1024 + c[t][d]) over the lane's 4 tokens
#pragma unroll
      for (int j = 0; j < TPI; ++j) {
        if (cmask & (1 << j)) {
          uint32_t v01[NB], v23[NB];  // f16 pairs of tokens (4jj, 4jj+1) and (4jj+2, 4jj+3)
#pragma unroll
          for (int n = 0; n < NB; ++n) vpairs(vw[j], n, v01[n], v23[n]);
#pragma unroll
          for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int gi = 0; gi < NG; ++gi) {
              const uint32_t pa = (uint32_t)__builtin_amdgcn_ds_bpermute(srcA + 64 * r, (int)pp[j][gi]);
              const uint32_t pb = (uint32_t)__builtin_amdgcn_ds_bpermute(srcB + 64 * r, (int)pp[j][gi]);
#pragma unroll
              for (int n = 0; n < NB; ++n) {
                if ((16 * n) / G != gi) continue;
                float o = O[r][n];
                o = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, pa), __builtin_bit_cast(h2, v01[n]), o, false);
                o = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, pb), __builtin_bit_cast(h2, v23[n]), o, false);
                O[r][n] = o;
              }
            }
          }
        }
      }
      // V registers are free: request the next iteration's
      if constexpr (MORE) {
        __builtin_amdgcn_sched_barrier(0);
        load_v(ckh, npg, ntp);
        __builtin_amdgcn_sched_barrier(0);
        cmask = cmask_next;
      }
    };
    for (int it = 0; it + 1 < niters; ++it) iterate(std::true_type(), it);
    iterate(std::false_type(), niters - 1);

    // ---- piece epilogue: row sums over the row's 16 token lanes, O folded
    // over the jj lanes (lane l keeps row jj), output or partial
    const bool whole = cta == 0 && ctb == cnt;
    const int slot = cfirst ? 2 * w : 2 * w + 1;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      lsum += __shfl_xor(lsum, o, 64);
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        corr[gi] += __shfl_xor(corr[gi], o, 64);
        osum[gi] += __shfl_xor(osum[gi], o, 64);
      }
    }
    const int row = jj;
    const bool writer = row < a.rows;
    const int qi = row / a.gqa, h = ckh * a.gqa + row % a.gqa;
    const float inv = 1.0f / fmaxf(lsum, 1e-20f);
    uint16_t *o = a.out + (((int64_t)cb * a.heads + h) * a.nq_stride + qi) * g.dim;
    float *pa = a.part_acc + ((int64_t)slot * a.rows + row) * DP;
    float ov[NB];
#pragma unroll
    for (int n = 0; n < NB; ++n) ov[n] = fold_rows(O[0][n], O[1][n], O[2][n], O[3][n]);
    if (writer) {
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        const int gi = (16 * n) / G;
        const float v = ov[n] + (corr[gi] - 1024.0f * osum[gi]);
        const int d = 16 * n + tok;
        if (whole) {
          if (d < g.dim) o[d] = float_to_bits(v * inv, g.float_kind);
        } else {
          pa[d] = v;
        }
      }
    }
    if (writer && !whole && tok == 0)
      *(float2 *)(a.part_ml + ((int64_t)slot * a.rows + row) * 2) = make_float2(m, lsum);

    if (!has_next) break;
    cb = nb; ckh = nkh; cL = nL; cnt = nnt; cseg0 = nseg0; cta = nta; ctb = ntb;
    cfirst = false; cpid = npid;
  }
}

// ---- host launcher ------------------------------------------------------------

typedef void (*AttnKernel)(AttnArgs);

template <int BITS, int DP, int G, int RB, int FK, int SLOTS, bool APPEND>
static AttnKernel kernel_of() {
  if constexpr (RB > 1 && DP > 128) {
    return nullptr;  // 17..32 rows at head_dim > 128 run on the prefill kernel
  } else if constexpr (APPEND && (BITS == 16 || RB > 1)) {
    return nullptr;  // the fused append serves quantized pages at one row block
  } else {
    return attn_kernel<BITS, DP, G, RB, FK, fit_slots(BITS, DP, G, SLOTS), APPEND>;
  }
}

template <int RB, int SLOTS, bool APPEND = false>
static AttnKernel select_shape(const Geo &g) {
#define PKV_Q(BITS_, DP_, G_) \
  if (g.bits == BITS_ && g.dp == DP_ && g.group == G_) return kernel_of<BITS_, DP_, G_, RB, 1, SLOTS, APPEND>();
  PKV_Q(8, 64, 32) PKV_Q(8, 64, 64)
  PKV_Q(8, 128, 32) PKV_Q(8, 128, 64) PKV_Q(8, 128, 128)
  PKV_Q(8, 256, 32) PKV_Q(8, 256, 64) PKV_Q(8, 256, 128)
  PKV_Q(4, 64, 32) PKV_Q(4, 64, 64)
  PKV_Q(4, 128, 32) PKV_Q(4, 128, 64) PKV_Q(4, 128, 128)
  PKV_Q(4, 256, 32) PKV_Q(4, 256, 64) PKV_Q(4, 256, 128)
#undef PKV_Q
#define PKV_F(DP_, FK_) \
  if (g.bits == 16 && g.dp == DP_ && g.float_kind == FK_) return kernel_of<16, DP_, 32, RB, FK_, SLOTS, false>();
  PKV_F(64, 0) PKV_F(64, 1) PKV_F(128, 0) PKV_F(128, 1) PKV_F(256, 0) PKV_F(256, 1)
#undef PKV_F
  return nullptr;
}

// The decode kernel for at most 4 rows per KV head over quantized pages at
// head_dim <= 128: attn_kernel (MFMA, the default) or valu_kernel.
static std::atomic<int> g_decode_kernel{kDecodeMfma};

int select_decode_kernel(int kind) { return g_decode_kernel.exchange(kind); }
int decode_kernel() { return g_decode_kernel.load(); }

static AttnKernel select_valu(const Geo &g) {
#define PKV_V(BITS_, DP_, G_) \
  if (g.bits == BITS_ && g.dp == DP_ && g.group == G_) return valu_kernel<BITS_, DP_, G_>;
  PKV_V(8, 64, 32) PKV_V(8, 64, 64) PKV_V(8, 128, 32) PKV_V(8, 128, 64) PKV_V(8, 128, 128)
  PKV_V(4, 64, 32) PKV_V(4, 64, 64) PKV_V(4, 128, 32) PKV_V(4, 128, 64) PKV_V(4, 128, 128)
#undef PKV_V
  return nullptr;
}

// Rows per KV head -> column slots: <= 4 rows: 4 slots, <= 8: 2, else 1
// (two row blocks past 16 rows).  With the fused single-token append: the
// MFMA kernels of up to 8 rows over quantized pages (else none).
static AttnKernel select_kernel(const Geo &g, int rows, bool append = false) {
  if (append) {
    if (g.bits == 16) return nullptr;
    if (rows <= 4) return select_shape<1, 4, true>(g);
    if (rows <= 8) return select_shape<1, 2, true>(g);
    return nullptr;
  }
  if (rows <= 4 && g_decode_kernel.load() == kDecodeValu) {
    if (const AttnKernel k = select_valu(g)) return k;
  }
  if (rows <= 4) return select_shape<1, 4>(g);
  if (rows <= 8) return select_shape<1, 2>(g);
  if (rows <= 16) return select_shape<1, 1>(g);
  if (rows <= 32) return select_shape<2, 1>(g);
  return nullptr;
}

bool decode_serves(const Geo &g, int rows) { return select_kernel(g, rows) != nullptr; }

// Waves per run of the kernel select_kernel picks for `rows`: its row blocks
// (two past 16 rows) and column slots (4, 2 or 1 up to 4, 8 and 16 rows, as
// fit_slots leaves them); the VALU decode kernel runs one wave per run.
static int group_of(const Geo &g, int rows, bool append = false) {
  if (append) return 1;
  if (rows <= 4 && g_decode_kernel.load() == kDecodeValu && select_valu(g)) return 1;
  const int req = rows <= 4 ? 4 : rows <= 8 ? 2 : 1;
  return run_waves(rows > 16 ? 2 : 1, fit_slots(g.bits, g.dp, g.bits == 16 ? 32 : g.group, req), append);
}

int attention_group(const Geo &g, int rows, bool append) { return group_of(g, rows, append); }

bool append_fusable(const Geo &g, int rows) { return select_kernel(g, rows, true) != nullptr; }

int attention_waves(const Geo &g, int rows) {
  const AttnKernel k = select_kernel(g, rows);
  if (!k) return -1;
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
  const int gw = group_of(g, rows);
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)k, 64 * gw, 0) != hipSuccess)
    return -1;
  return max(1, cus * per_cu) * gw;  // resident waves (runs of gw waves)
}

// The split charges each segment `lead` tiles ahead of its own, the cost of
// starting a piece (query rows, then its first tiles, requested after the
// previous piece's pipeline has drained and its partial is written), so that
// a wave whose run crosses into another segment gets correspondingly fewer
// tiles and ends with the others.  Eight tiles measured best, or within
// noise of it, for 1, 5 and 20 rows per KV head and contexts from 64 to
// 16K tokens (4-slot decode: about two iterations).  A launch that fuses the
// single-token append charges 16: the wave that holds a segment's last tile
// (the one whose run crosses into the next segment) also loads and quantizes
// the new token before its first tiles (C2: 67.8 us against 69.0 at 8).
// A run of a grouped kernel (GW waves) moves GW tiles in a wave's tile time,
// so its lead counts GW times as many tiles.
int attention_lead(const Geo &g, int rows, bool append) { return append ? 16 : 8 * group_of(g, rows, append); }

hipError_t launch_attention(hipStream_t stream, const AttnArgs &a) {
  const AttnKernel k = select_kernel(a.g, a.rows, a.new_k != nullptr);
  if (!k) return hipErrorInvalidValue;
  if (a.waves <= 0) return hipSuccess;
  hipLaunchKernelGGL(k, dim3((unsigned)a.waves), dim3(64 * group_of(a.g, a.rows, a.new_k != nullptr)), 0, stream, a);
  return hipGetLastError();
}

constexpr int64_t kMergeResidentWaves = 8192;

hipError_t launch_merge(hipStream_t stream, const MergeArgs &a) {
  const int64_t units = (int64_t)a.batch * a.hk * a.rows;  // one workgroup per (segment, row)
  if (units == 0 || a.waves <= 1) return hipSuccess;  // one run covers every segment whole
  if (units > 0x7FFFFFFF) return hipErrorInvalidValue;
  // Waves per workgroup: enough for a segment's pieces, about waves /
  // segments + 1, to fit one round of 16 partial rows per wave (a single wave
  // needs no LDS reduction); two instead of four when four-wave workgroups
  // would not all be resident at once (about 8,192 waves on the device).
  const int64_t segments = (int64_t)a.batch * a.hk;
  const int64_t pieces = (a.waves + segments - 1) / segments + 1;
  int nw = pieces <= 16 ? 1 : pieces <= 32 ? 2 : 4;
  if (nw == 4 && units * 4 > kMergeResidentWaves) nw = 2;
  const dim3 grid((unsigned)units), block(64 * nw);
#define PKV_M(DP_)                                                                         \
  if (a.dp == DP_) {                                                                       \
    if (nw == 1) hipLaunchKernelGGL((merge_kernel<DP_, 1>), grid, block, 0, stream, a);    \
    else if (nw == 2) hipLaunchKernelGGL((merge_kernel<DP_, 2>), grid, block, 0, stream, a); \
    else hipLaunchKernelGGL((merge_kernel<DP_, 4>), grid, block, 0, stream, a);            \
    return hipGetLastError();                                                              \
  }
  PKV_M(64) PKV_M(128) PKV_M(256)
#undef PKV_M
  return hipErrorInvalidValue;
}

}  // namespace pkv
