// Fused lm_head + softmax: token sampling with the drawn token's
// log-probability, or the log-probabilities of given target tokens, without
// materialising the [rows, vocab] logits.
//
// Reference semantics:
//   qwen3_naive.py:1387 / :1607   logits = self.lm_head(h)     (h [n, 1024] bf16)
//   qwen3_naive.py:1413-1423, :1636-1650 (top_k = None)
//       x = logits.float() / T;  tok ~ Categorical(softmax(x));  lp = log_softmax(x)[tok]
//   qwen3_grpo_train.py:46-53     lp = log_softmax(logits.float())[ids]
// The logits here are h . w accumulated in fp32 and never rounded, where the
// reference rounds its lm_head output to bf16 before the fp32 softmax.
//
// Kernel 1, lmhead_items: a work item (TVB vocabulary tiles of 128 rows, a
// tile of MT hidden-state rows) computes its logits with
// v_mfma_f32_16x16x32_bf16 and reduces them on the spot to one (max, sum of
// exp2) pair per row and 128-row vocabulary tile in the log2 domain
// (x * log2(e) / T); in target mode the lane holding a row's target also
// writes that raw logit.  The grid is persistent (one or two workgroups per
// CU), each workgroup running a contiguous range of items as one pipeline of
// (item, 64-hidden chunk) steps, so the loads never drain at item
// boundaries.  Operands are computed transposed, S^T = W H^T: A = 16
// vocabulary rows x 32 hidden of W, B = H^T (32 hidden x 16 rows), so both
// operands are 16-byte row pieces and each lane's accumulators hold 4
// consecutive vocabulary entries of one row.
//   * W and H chunks go from global memory straight into LDS (gfx950
//     global_load_lds_dwordx4, no register staging), NSTAGE stages, loads
//     issued NSTAGE - 1 steps ahead, one wait and one barrier per step.
//     16-byte piece c of staged row r sits at c ^ ((r / 2) % 8): the 16 rows
//     a 16-lane group reads then cover all 64 LDS banks.
//   * Up to 64 rows: items of 128 x 64, 4 waves of 32 vocabulary rows, three
//     stages, two workgroups per CU.  Above: items of 256 x 256, 8 waves of
//     128 x 64 (one wave per 128-row vocabulary tile), two 64 KB stages, one
//     workgroup per CU: each item re-reads its hidden-state rows from L2, so
//     256-entry items halve that traffic per FLOP (at 8,192 rows 4.07 ->
//     2.73 ms against 128-entry items staged through registers).
//   * W (311 MB for Qwen3-0.6B) is read once from HBM per row tile; H comes
//     from L2.
// Kernel 2, lmhead_sample_rows: one workgroup per row combines the row's tile
// pairs into its log-sum-exp and draws the token by inverse transform
// sampling with one Philox4x32-10 uniform per row: the first vocabulary index
// whose cumulative probability exceeds u (tile prefix sums in fp64, then the
// chosen tile's 128 logits recomputed as fp32 dot products).  This is an exact
// draw from softmax(x / T) and costs one random number per row instead of
// one per vocabulary entry.
// Kernel 2', lmhead_logprob_rows: lse and lp = x[target] - lse per row.
#include <algorithm>
#include <type_traits>

#include "qmi_common.h"

namespace {

using namespace qmi;

constexpr int kTV = 128;            // vocabulary rows per tile
constexpr int kKC = 64;             // hidden elements per staged chunk
constexpr int kRowB = kKC * 2;      // bytes per staged row
constexpr int kRowThreads = 256;    // kernel 2

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
  return __builtin_bit_cast(bf16x8_t, u32x4_t{v.x, v.y, v.z, v.w});
}

// Byte offset of 16-byte piece c of staged row r.
__device__ __forceinline__ int lds_off(int r, int c) { return r * kRowB + ((c ^ ((r >> 1) & 7)) << 4); }

// Direct global -> LDS load of 16 bytes per lane (gfx950
// global_load_lds_dwordx4): lane l's bytes at gbase + voff land at LDS byte
// lds + 16 l.  Inline asm, so that the compiler adds no wait for it; the
// caller waits with s_waitcnt vmcnt before the barrier that publishes the
// stage.
__device__ __forceinline__ void lds_load16(const void* gbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               : : "s"(lds), "v"(voff), "s"(gbase) : "memory", "m0");
}

// Kernel 1 with larger work items and direct loads: an item is TVB
// vocabulary tiles of 128 rows (TV = 128 TVB) x MT hidden-state rows; W and
// H chunks go from global memory straight into NSTAGE LDS stages (no
// register staging, no LDS write instructions), loads issued NSTAGE - 1
// steps ahead.  Wave (vq, rq) owns vocabulary rows VW vq .. +VW (VW = 128
// when TVB = NVQ: one wave per 128-row tile, whose (max, sum) pairs it
// writes itself) and hidden-state rows 64 rq .. +64.  Rows past the
// vocabulary or the batch load the last valid row (their results are
// masked or not written).  Per-item H traffic is what bounds this kernel at
// a few hundred rows and above (each item re-reads its MT x hidden rows from
// L2): 256-entry items halve it per FLOP.
template <int MT, int NW, int NSTAGE, int TVB>
__global__ __launch_bounds__(NW * 64) void lmhead_items(
    const uint16_t* __restrict__ h, int64_t h_stride, int n_rows,
    const uint16_t* __restrict__ w, int64_t w_stride, int vocab, int hidden, float c2,
    const int64_t* __restrict__ tgt, int64_t tgt_stride, int n_vtiles, int n_rtiles,
    float2* __restrict__ part, float* __restrict__ tgt_logit) {
  constexpr int TV = kTV * TVB;
  constexpr int NRQ = MT / 64;       // row blocks of 64
  constexpr int NVQ = NW / NRQ;      // waves per row block
  constexpr int VW = TV / NVQ;       // vocabulary rows per wave
  constexpr int VB = VW / 16;        // 16-row MFMA blocks per wave along the vocabulary
  constexpr int WPT = kTV / VW;      // waves per 128-row vocabulary tile
  constexpr int W_BYTES = TV * kRowB;
  constexpr int STAGE = W_BYTES + MT * kRowB;
  constexpr int WL = TV / (8 * NW);  // W wave-loads (8 rows of 128 B) per wave per chunk
  constexpr int HL = MT / (8 * NW);  // H wave-loads per wave per chunk
  constexpr int LPW = WL + HL;
  static_assert(NVQ * NRQ == NW && VB >= 1 && VW <= kTV && kTV % VW == 0, "tile shape");
  static_assert(WL >= 1 && HL >= 1 && TV % (8 * NW) == 0 && MT % (8 * NW) == 0, "loads");
  static_assert(NSTAGE >= 2 && NSTAGE * STAGE <= 160 * 1024, "LDS");
  __shared__ __align__(16) unsigned char lds[NSTAGE * STAGE];
  __shared__ float2 red[WPT > 1 ? NVQ : 1][WPT > 1 ? MT : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g4 = lane >> 4;
  const int vq = wave % NVQ, rq = wave / NVQ;
  const int n_kc = hidden / kKC;
  const int n_vitems = (n_vtiles + TVB - 1) / TVB;
  const int n_items = n_vitems * n_rtiles;
  const int i_begin = (int)((int64_t)blockIdx.x * n_items / gridDim.x);
  const int i_end = (int)((int64_t)(blockIdx.x + 1) * n_items / gridDim.x);
  const int n_steps = (i_end - i_begin) * n_kc;
  if (n_steps == 0) return;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;

  // Item positions (vocabulary item, row tile) advance incrementally.
  struct Pos {
    int vi, rt;
  };
  auto advance = [&](Pos p) -> Pos { return p.rt + 1 == n_rtiles ? Pos{p.vi + 1, 0} : Pos{p.vi, p.rt + 1}; };
  const Pos p_begin{i_begin / n_rtiles, i_begin % n_rtiles};

  // Load stream.  Wave-load j of this wave covers staged rows 8 (LPW' wave +
  // j) .. +8 of W (then of H); lane l fetches row + l / 8, physical piece
  // l % 8, i.e. logical piece (l % 8) ^ ((row / 2) % 8).
  Pos ld = p_begin;
  int ld_kc = 0, ld_step = 0;
  const char* wb0;
  const char* hb0;
  uint32_t woff[WL], hoff[HL];
  auto ld_item_setup = [&]() __attribute__((always_inline)) {
    const int v0 = ld.vi * TV, r0 = ld.rt * MT;
    const int wlast = min(TV, vocab - v0) - 1;
    const int hlast = min(MT, n_rows - r0) - 1;
    wb0 = reinterpret_cast<const char*>(w + (int64_t)v0 * w_stride);
    hb0 = reinterpret_cast<const char*>(h + (int64_t)r0 * h_stride);
#pragma unroll
    for (int j = 0; j < WL; ++j) {
      const int r = 8 * (WL * wave + j) + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      woff[j] = (uint32_t)((min(r, wlast) * w_stride + c * 8) * 2);
    }
#pragma unroll
    for (int j = 0; j < HL; ++j) {
      const int r = 8 * (HL * wave + j) + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      hoff[j] = (uint32_t)((min(r, hlast) * h_stride + c * 8) * 2);
    }
  };
  ld_item_setup();
  // Issues the next step's loads into `stage` (the stream repeats its last
  // step past the end, so every step issues the same number of loads).
  auto issue = [&](int stage) __attribute__((always_inline)) {
    const uint32_t sb = lds0 + stage * STAGE;
    const char* wk = wb0 + ld_kc * kRowB;
    const char* hk = hb0 + ld_kc * kRowB;
#pragma unroll
    for (int j = 0; j < WL; ++j) lds_load16(wk, woff[j], sb + (WL * wave + j) * 8 * kRowB);
#pragma unroll
    for (int j = 0; j < HL; ++j) lds_load16(hk, hoff[j], sb + W_BYTES + (HL * wave + j) * 8 * kRowB);
    if (ld_step + 1 < n_steps) {
      ++ld_step;
      if (++ld_kc == n_kc) {
        ld_kc = 0;
        ld = advance(ld);
        ld_item_setup();
      }
    }
  };

  // Operand reads: row VW vq + 16 vb + l16 of W, row 64 rq + 16 rb + l16 of
  // H, piece 4 ks + g4; (r / 2) % 8 of those rows is l16 / 2.
  int a_off[2], b_off[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int pc = ((4 * ks + g4) ^ (l16 >> 1)) << 4;
    a_off[ks] = (VW * vq + l16) * kRowB + pc;
    b_off[ks] = W_BYTES + (64 * rq + l16) * kRowB + pc;
  }
  f32x4_t acc[VB][4];
#pragma unroll
  for (int vb = 0; vb < VB; ++vb)
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) acc[vb][rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  int64_t tgt_id[4] = {-1, -1, -1, -1};
  auto load_targets = [&](Pos it) __attribute__((always_inline)) {
    const int r0 = it.rt * MT;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const int row = r0 + 64 * rq + 16 * rb + l16;
      tgt_id[rb] = tgt[(int64_t)(row < n_rows ? row : n_rows - 1) * tgt_stride];
    }
  };

  // Epilogue of an item: per row, (max, sum of exp2) over each 128-entry
  // vocabulary tile; acc[vb][rb][e] holds vocabulary v0 + VW vq + 16 vb +
  // 4 g4 + e of row r0 + 64 rq + 16 rb + l16.
  auto epilogue = [&](Pos it) __attribute__((always_inline)) {
    const int64_t v0 = (int64_t)it.vi * TV;
    const int64_t r0 = (int64_t)it.rt * MT;
    const int64_t vbase = v0 + VW * vq + 4 * g4;
    const int vt = (int)(v0 / kTV) + (VW * vq) / kTV;  // this wave's 128-row tile
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const int row_l = 64 * rq + 16 * rb + l16;
      const int64_t row = r0 + row_l;
      if (tgt && row < n_rows) {  // the raw logit of the target, by the lane holding it
        const int64_t tl = tgt_id[rb] - vbase;  // 16 vb + e if this lane holds it
        if (tl >= 0 && tl < VW && (tl & 12) == 0) {
#pragma unroll
          for (int vb = 0; vb < VB; ++vb)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (tl == 16 * vb + e) tgt_logit[row] = acc[vb][rb][e];
        }
      }
      float mx = kNegBig;
#pragma unroll
      for (int vb = 0; vb < VB; ++vb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool ok = vbase + 16 * vb + e < vocab;
          acc[vb][rb][e] = ok ? acc[vb][rb][e] * c2 : kNegBig;
          mx = fmaxf(mx, acc[vb][rb][e]);
        }
      float sm = 0.f;
#pragma unroll
      for (int vb = 0; vb < VB; ++vb)
#pragma unroll
        for (int e = 0; e < 4; ++e) sm += fast_exp2(acc[vb][rb][e] - mx);
      LanePair pm = lane_pair16(mx), ps = lane_pair16(sm);
      mx = pm.lo;
      sm = ps.lo;
      lse2_merge(mx, sm, pm.hi, ps.hi);
      pm = lane_pair32(mx);
      ps = lane_pair32(sm);
      mx = pm.lo;
      sm = ps.lo;
      lse2_merge(mx, sm, pm.hi, ps.hi);
      if constexpr (WPT > 1) {
        if (g4 == 0) red[vq][row_l] = make_float2(mx, sm);
      } else {
        if (g4 == 0 && row < n_rows && vt < n_vtiles) part[row * (int64_t)n_vtiles + vt] = make_float2(mx, sm);
      }
#pragma unroll
      for (int vb = 0; vb < VB; ++vb) acc[vb][rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    if constexpr (WPT > 1) {
      __syncthreads();
      for (int r = tid; r < MT; r += NW * 64) {
        if (r0 + r < n_rows) {
          float2 a = red[0][r];
#pragma unroll
          for (int j = 1; j < NVQ; ++j) lse2_merge(a.x, a.y, red[j][r].x, red[j][r].y);
          part[(r0 + r) * (int64_t)n_vtiles + (int)(v0 / kTV)] = a;
        }
      }
    }
  };

  // Step st: issue step st + NSTAGE - 1 into its stage (last read in step
  // st - 1, which ended with a barrier), multiply stage st % NSTAGE, then
  // wait for this wave's loads of step st + 1 and meet at the barrier.
  Pos it = p_begin;
  int kc = 0, stage = 0;
#pragma unroll
  for (int i = 0; i < NSTAGE - 1; ++i) issue(i);
  asm volatile("s_waitcnt vmcnt(%0)" ::"i"((NSTAGE - 2) * LPW) : "memory");
  __syncthreads();
  for (int st = 0; st < n_steps; ++st) {
    if (tgt && kc == 0) load_targets(it);
    issue(stage == 0 ? NSTAGE - 1 : stage - 1);
    const unsigned char* base = lds + stage * STAGE;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8_t a[VB], b[4];
#pragma unroll
      for (int i = 0; i < VB; ++i)
        a[i] = as_bf16x8(*reinterpret_cast<const uint4*>(base + a_off[ks] + i * 16 * kRowB));
#pragma unroll
      for (int i = 0; i < 4; ++i)
        b[i] = as_bf16x8(*reinterpret_cast<const uint4*>(base + b_off[ks] + i * 16 * kRowB));
#pragma unroll
      for (int vb = 0; vb < VB; ++vb)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
          acc[vb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[vb], b[rb], acc[vb][rb], 0, 0, 0);
    }
    if (kc + 1 == n_kc) {
      epilogue(it);
      it = advance(it);
      kc = 0;
    } else {
      ++kc;
    }
    stage = stage + 1 == NSTAGE ? 0 : stage + 1;
    asm volatile("s_waitcnt vmcnt(%0)" ::"i"((NSTAGE - 2) * LPW) : "memory");
    __syncthreads();
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Block-wide helpers for kernel 2 (256 threads).
__device__ float block_max256(float x, float* sm) {
  x = wave_max(x);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = x;
  __syncthreads();
  return fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
}

// Inclusive scan of one double per lane over the wave (fixed order).
__device__ __forceinline__ double wave_scan_f64(double x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const double y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  return x;
}

// Exclusive prefix (fp64, fixed order) of one value per thread over the 256
// threads; also returns the total.  sm holds 5 doubles.
__device__ double block_excl_scan256(double x, double* sm, double* total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const double inc = wave_scan_f64(x);
  __syncthreads();
  if (lane == 63) sm[wv] = inc;
  __syncthreads();
  double base = 0.0;
  for (int j = 0; j < wv; ++j) base += sm[j];
  *total = sm[0] + sm[1] + sm[2] + sm[3];
  return base + inc - x;
}

// Row log-sum-exp in the log2 domain from the row's tile pairs: lse2 =
// m2 + log2(s).  Each thread takes the contiguous chunk of cpt tiles
// starting at tid * cpt; *own is its fp64 mass and *excl the mass of the
// chunks before it.
struct RowLse {
  float m2;
  double s;
};

__device__ RowLse row_lse(const float2* __restrict__ pr, int n, int cpt, double* own,
                          double* excl, float* smf, double* smd) {
  const int tid = threadIdx.x;
  const int lo = min(n, tid * cpt), hi = min(n, lo + cpt);
  float mx = kNegBig;
  for (int t = lo; t < hi; ++t) mx = fmaxf(mx, pr[t].x);
  const float m2 = block_max256(mx, smf);
  double acc = 0.0;
  for (int t = lo; t < hi; ++t) acc += (double)(pr[t].y * fast_exp2(pr[t].x - m2));
  *own = acc;
  double total;
  *excl = block_excl_scan256(acc, smd, &total);
  return {m2, total};
}

__global__ __launch_bounds__(kRowThreads) void lmhead_sample_rows(
    const float2* __restrict__ part, int n_vtiles, const uint16_t* __restrict__ h,
    int64_t h_stride, const uint16_t* __restrict__ w, int64_t w_stride, int vocab, int hidden,
    float c2, uint32_t seed_lo, uint32_t seed_hi, uint32_t off_lo, uint32_t off_hi,
    int64_t* __restrict__ out_tok, float* __restrict__ out_lp) {
  __shared__ float smf[4];
  __shared__ double smd[5];
  __shared__ float xs[kTV];
  __shared__ int sel_tile;
  __shared__ double sel_resid;
  __shared__ __align__(16) uint16_t hrow[16384];
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const float2* pr = part + (int64_t)row * n_vtiles;
  const uint16_t* hr = h + (int64_t)row * h_stride;
  // The row's hidden state into LDS (read by every column below).
  for (int k = 8 * tid; k < hidden; k += 8 * kRowThreads)
    *reinterpret_cast<uint4*>(hrow + k) = load_u4(hr + k);
  const int cpt = (n_vtiles + kRowThreads - 1) / kRowThreads;
  double own, excl;
  const RowLse L = row_lse(pr, n_vtiles, cpt, &own, &excl, smf, smd);

  // u in (0, 1) with 53 bits from the first two words of the row's block.
  const uint4 r = philox4x32_10(make_uint4(0u, (uint32_t)row, off_lo, off_hi), seed_lo, seed_hi);
  const uint64_t bits = ((uint64_t)r.x << 21) | (uint64_t)(r.y >> 11);
  const double u = ((double)bits + 0.5) * 0x1p-53;
  const double target = u * L.s;

  if (tid == 0) {
    sel_tile = -1;
    sel_resid = 0.0;
  }
  __syncthreads();
  const int lo = min(n_vtiles, tid * cpt), hi = min(n_vtiles, lo + cpt);
  if (own > 0.0 && target >= excl && target < excl + own) {
    double cum = excl;
    int t = lo;
    for (; t < hi - 1; ++t) {
      const double p = (double)(pr[t].y * fast_exp2(pr[t].x - L.m2));
      if (target < cum + p) break;
      cum += p;
    }
    sel_tile = t;
    sel_resid = target - cum;
  }
  __syncthreads();
  if (sel_tile < 0) {
    // u * S rounded up to S: the last tile with mass, at its last entry.
    if (tid == 0) {
      int t = n_vtiles - 1;
      while (t > 0 && !(pr[t].y * fast_exp2(pr[t].x - L.m2) > 0.f)) --t;
      sel_tile = t;
      sel_resid = 1e300;
    }
    __syncthreads();
  }
  const int t_sel = sel_tile;

  // The chosen tile's logits for this row: thread t takes column t / 2 and
  // half t % 2 of the hidden dimension (all loads of a thread independent).
  {
    const int c = tid >> 1, half = tid & 1;
    const int64_t v = (int64_t)t_sel * kTV + c;
    float d = 0.f;
    if (v < vocab) {
      const uint16_t* wr = w + v * w_stride;
      const int k0 = half * (hidden / 2), k1 = k0 + hidden / 2;
#pragma unroll 8
      for (int k = k0; k < k1; k += 8) {
        const uint4 a = *reinterpret_cast<const uint4*>(hrow + k), b = load_u4(wr + k);
        d = dot2_bf16(a.x, b.x, d);
        d = dot2_bf16(a.y, b.y, d);
        d = dot2_bf16(a.z, b.z, d);
        d = dot2_bf16(a.w, b.w, d);
      }
    }
    d += __shfl_xor(d, 1, 64);
    if (half == 0) xs[c] = v < vocab ? d : -INFINITY;
  }
  __syncthreads();
  // Within the tile: the first column whose cumulative mass exceeds the
  // residual (wave 0, two columns per lane, fixed-order scan).
  if (tid < 64) {
    const double resid = sel_resid;
    const float x0 = xs[2 * tid], x1 = xs[2 * tid + 1];
    const double p0 = x0 == -INFINITY ? 0.0 : (double)fast_exp2(x0 * c2 - L.m2);
    const double p1 = x1 == -INFINITY ? 0.0 : (double)fast_exp2(x1 * c2 - L.m2);
    const double inc = wave_scan_f64(p0 + p1);
    const double before = inc - (p0 + p1);
    int cand = kTV;
    if (resid < before + p0) cand = 2 * tid;
    else if (resid < inc) cand = 2 * tid + 1;
    int last = p1 > 0.0 ? 2 * tid + 1 : (p0 > 0.0 ? 2 * tid : -1);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      cand = min(cand, __shfl_xor(cand, m, 64));
      last = max(last, __shfl_xor(last, m, 64));
    }
    if (tid == 0) {
      const int pick = cand < kTV ? cand : (last >= 0 ? last : 0);
      out_tok[row] = (int64_t)t_sel * kTV + pick;
      if (out_lp) {
        const double lse2 = (double)L.m2 + log2(L.s);
        out_lp[row] = (float)(((double)xs[pick] * (double)c2 - lse2) * (double)kLn2);
      }
    }
  }
}

__global__ __launch_bounds__(kRowThreads) void lmhead_logprob_rows(
    const float2* __restrict__ part, int n_vtiles, const float* __restrict__ tgt_logit,
    float c2, float* __restrict__ out_lp, float* __restrict__ out_lse) {
  __shared__ float smf[4];
  __shared__ double smd[5];
  const int row = blockIdx.x;
  const int cpt = (n_vtiles + kRowThreads - 1) / kRowThreads;
  double own, excl;
  const RowLse L = row_lse(part + (int64_t)row * n_vtiles, n_vtiles, cpt, &own, &excl, smf, smd);
  if (threadIdx.x == 0) {
    const double lse = ((double)L.m2 + log2(L.s)) * (double)kLn2;  // of x * c2 / log2(e)
    if (out_lse) out_lse[row] = (float)lse;
    out_lp[row] = (float)((double)tgt_logit[row] * (double)c2 * (double)kLn2 - lse);
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct LmWs {
  float2* part;
  float* tgt_logit;
};

inline int64_t n_vtiles_of(int64_t vocab) { return (vocab + kTV - 1) / kTV; }

inline int64_t ws_bytes(int64_t n_rows, int64_t vocab) {
  const int64_t p = n_rows * n_vtiles_of(vocab) * (int64_t)sizeof(float2);
  return ((p + 255) & ~(int64_t)255) + n_rows * (int64_t)sizeof(float);
}

inline LmWs ws_layout(void* ws, int64_t n_rows, int64_t vocab) {
  const int64_t p = n_rows * n_vtiles_of(vocab) * (int64_t)sizeof(float2);
  char* base = static_cast<char*>(ws);
  return {reinterpret_cast<float2*>(base), reinterpret_cast<float*>(base + ((p + 255) & ~(int64_t)255))};
}

int check_args(const uint16_t* h, int64_t h_stride, int64_t n_rows, const uint16_t* w,
               int64_t w_stride, int64_t vocab, int64_t hidden, void* ws, int64_t ws_size) {
  if (n_rows < 0 || vocab <= 0 || hidden <= 0) return QMI_E_BAD_SHAPE;
  if (!h || !w || !ws) return QMI_E_NULL_POINTER;
  if (hidden % kKC != 0 || hidden > 16384) return QMI_E_UNSUPPORTED;
  if (vocab > 0x7fffffffLL - kTV || n_rows > 0x7fffffffLL) return QMI_E_UNSUPPORTED;
  if (h_stride < hidden || w_stride < hidden) return QMI_E_BAD_STRIDE;
  if (h_stride % 8 || w_stride % 8 || !aligned16(h) || !aligned16(w) || !aligned16(ws))
    return QMI_E_BAD_STRIDE;
  if (ws_size < ws_bytes(n_rows, vocab)) return QMI_E_WORKSPACE_TOO_SMALL;
  return QMI_OK;
}

int launch_tiles(const uint16_t* h, int64_t h_stride, int64_t n_rows, const uint16_t* w,
                 int64_t w_stride, int64_t vocab, int64_t hidden, float c2, const int64_t* tgt,
                 int64_t tgt_stride, const LmWs& ws, hipStream_t s) {
  const int nvt = (int)n_vtiles_of(vocab);
  // Up to 64 rows: items of 128 x 64, 4 waves, three LDS stages, two 74 KB
  // workgroups per CU.  Above: items of 256 x 256, 8 waves, two LDS stages,
  // one 128 KB workgroup per CU.  A persistent grid of that many workgroups
  // per CU, or fewer when there are fewer items.
#define QMI_LMI(MT, NW, NS, TVB, PER_CU)                                                              \
  do {                                                                                            \
    const int nrt = (int)((n_rows + MT - 1) / MT);                                                \
    const int64_t items = (int64_t)((nvt + TVB - 1) / TVB) * nrt;                                 \
    const int64_t grid = std::min<int64_t>(items, (int64_t)device_cu_count() * PER_CU);           \
    hipLaunchKernelGGL((lmhead_items<MT, NW, NS, TVB>), dim3((unsigned)grid), dim3(NW * 64), 0, s, \
                       h, h_stride, (int)n_rows, w, w_stride, (int)vocab, (int)hidden, c2, tgt,   \
                       tgt_stride, nvt, nrt, ws.part, ws.tgt_logit);                              \
  } while (0)
  if (n_rows <= 64)
    QMI_LMI(64, 4, 3, 1, 2);
  else
    QMI_LMI(256, 8, 2, 2, 1);
#undef QMI_LMI
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? QMI_OK : (int)e;
}

}  // namespace

extern "C" int64_t qmi_lm_head_workspace_bytes(int64_t n_rows, int64_t vocab) {
  if (n_rows <= 0 || vocab <= 0) return 0;
  return ws_bytes(n_rows, vocab);
}

extern "C" int qmi_lm_head_sample(const uint16_t* hidden_states, int64_t h_stride, int64_t n_rows,
                                  const uint16_t* weight, int64_t w_stride, int64_t vocab,
                                  int64_t hidden, float temperature, uint64_t seed,
                                  uint64_t offset, int64_t* out_tokens, float* out_logprobs,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
  if (n_rows == 0 && vocab > 0 && hidden > 0) return QMI_OK;
  int st = check_args(hidden_states, h_stride, n_rows, weight, w_stride, vocab, hidden, workspace,
                      workspace_bytes);
  if (st != QMI_OK) return st;
  if (!out_tokens) return QMI_E_NULL_POINTER;
  if (!(temperature > 0.f) || temperature == INFINITY) return QMI_E_BAD_SHAPE;
  const float c2 = kLog2e / temperature;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const LmWs ws = ws_layout(workspace, n_rows, vocab);
  st = launch_tiles(hidden_states, h_stride, n_rows, weight, w_stride, vocab, hidden, c2, nullptr,
                    0, ws, s);
  if (st != QMI_OK) return st;
  hipLaunchKernelGGL(lmhead_sample_rows, dim3((unsigned)n_rows), dim3(kRowThreads), 0, s, ws.part,
                     (int)n_vtiles_of(vocab), hidden_states, h_stride, weight, w_stride, (int)vocab,
                     (int)hidden, c2, (uint32_t)seed, (uint32_t)(seed >> 32), (uint32_t)offset,
                     (uint32_t)(offset >> 32), out_tokens, out_logprobs);
  QMI_RETURN_LAUNCH_STATUS();
}

extern "C" int qmi_lm_head_logprob(const uint16_t* hidden_states, int64_t h_stride, int64_t n_rows,
                                   const uint16_t* weight, int64_t w_stride, int64_t vocab,
                                   int64_t hidden, const int64_t* targets, int64_t target_stride,
                                   float* out_logprobs, float* out_lse, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
  if (n_rows == 0 && vocab > 0 && hidden > 0) return QMI_OK;
  int st = check_args(hidden_states, h_stride, n_rows, weight, w_stride, vocab, hidden, workspace,
                      workspace_bytes);
  if (st != QMI_OK) return st;
  if (!targets || !out_logprobs) return QMI_E_NULL_POINTER;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const LmWs ws = ws_layout(workspace, n_rows, vocab);
  st = launch_tiles(hidden_states, h_stride, n_rows, weight, w_stride, vocab, hidden, kLog2e,
                    targets, target_stride, ws, s);
  if (st != QMI_OK) return st;
  hipLaunchKernelGGL(lmhead_logprob_rows, dim3((unsigned)n_rows), dim3(kRowThreads), 0, s, ws.part,
                     (int)n_vtiles_of(vocab), ws.tgt_logit, kLog2e, out_logprobs, out_lse);
  QMI_RETURN_LAUNCH_STATUS();
}
