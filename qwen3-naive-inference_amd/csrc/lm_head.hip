// Fused lm_head + softmax: token sampling (all entries, or the top k) with
// the drawn token's log-probability, or the log-probabilities of given target
// tokens, without materialising the [rows, vocab] logits.
//
// Reference semantics:
//   qwen3_naive.py:1387 / :1607   logits = self.lm_head(h)     (h [n, 1024] bf16)
//   qwen3_naive.py:1413-1423, :1636-1650
//       x = logits.float() / T;  [top_k: keep the k largest of x, the rest -inf]
//       tok ~ Categorical(softmax(x));  lp = log_softmax(x)[tok]
//   qwen3_grpo_train.py:46-53     lp = log_softmax(logits.float())[ids]
// Each logit is h . w accumulated in fp32 and rounded to bf16, as the
// reference's bf16 lm_head output is, before the fp32 softmax.
//
// Kernel 1, lmhead_items: a work item (TVB vocabulary tiles of 128 rows, a
// tile of MT hidden-state rows) computes its logits with
// v_mfma_f32_16x16x32_bf16 and reduces them on the spot to one (max, sum of
// exp2) pair per row and wave slice of the vocabulary (32, 64 or 128 entries
// by configuration) in the log2 domain (x * log2(e) / T), or, in top-k mode,
// to every (row, tile)'s four largest logits (value descending, index
// ascending) as packed keys.  The grid is persistent (one or two workgroups
// per CU), each workgroup running a contiguous range of items as one
// pipeline of (item, 64-hidden chunk) steps, so the loads never drain at
// item boundaries.  Operands are computed
// transposed, S^T = W H^T: A = 16 vocabulary rows x 32 hidden of W, B = H^T
// (32 hidden x 16 rows), so both operands are 16-byte row pieces and each
// lane's accumulators hold 4 consecutive vocabulary entries of one row.
//   * W and H chunks go from global memory straight into LDS (gfx950
//     global_load_lds_dwordx4, no register staging), NSTAGE stages, loads
//     issued NSTAGE - 1 steps ahead, one wait and one barrier per step.
//     16-byte piece c of staged row r sits at c ^ ((r / 2) % 8): the 16 rows
//     a 16-lane group reads then cover all 64 LDS banks.
//   * Up to 64 rows: items of 128 x 64, 4 waves of 32 vocabulary rows, three
//     stages, two workgroups per CU.  Up to 256 rows: items of 256 x 128, 8
//     waves of 64 x 64 (two per 128-row tile), three stages, one workgroup per
//     CU.  Above: items of 256 x 256, 8 waves of
//     128 x 64 (one wave per 128-row vocabulary tile), two 64 KB stages, one
//     workgroup per CU: each item re-reads its hidden-state rows from L2, so
//     256-entry items halve that traffic per FLOP (at 8,192 rows 4.07 ->
//     2.73 ms against 128-entry items staged through registers).
//   * W (311 MB for Qwen3-0.6B) is read once from HBM per row tile; H comes
//     from L2.
// Kernel 2, lmhead_sample_rows: one workgroup per row combines the row's
// pairs into its log-sum-exp and draws the token by inverse transform
// sampling with one Philox4x32-10 uniform per row: the first vocabulary index
// whose cumulative probability exceeds u (pair prefix sums in fp64, then the
// chosen slice's 32-128 logits recomputed by the same MFMA sequence as kernel
// 1, so they are bit-identical to the values its pair summarises).  This is an
// exact draw from softmax(x / T) and costs one random number per row instead
// of one per vocabulary entry.
// Kernel 2', lmhead_topk_rows: the k kept entries are found among the
// per-tile candidates (a radix select on their values, ties to the lowest
// index), then drawn from by inverse transform sampling in vocabulary order.
// The top k of a row lie in its candidates unless some tile holds four or
// more of them; such a tile is recomputed in full and the selection repeated.
// Kernel 2'', lmhead_logprob_rows: lse and lp = x[target] - lse per row, the
// target's logit recomputed from its weight row by the same MFMA sequence
// (so bit-identical; the item kernel then loads no target ids, whose waits
// would drain its load pipeline once per item).
#include <algorithm>
#include <type_traits>

#include "qmi_common.h"

namespace {

using namespace qmi;

constexpr int kTV = 128;            // vocabulary rows per tile
constexpr int kKC = 64;             // hidden elements per staged chunk
constexpr int kRowB = kKC * 2;      // bytes per staged row
constexpr int kRowThreads = 256;    // kernel 2
constexpr int kMaxFusedTopK = 64;   // largest k of the fused top-k sampler
constexpr int kMaxCandTiles = 2048; // vocabulary tiles the top-k row kernel holds in LDS
constexpr int kMaxHidden = 16384;

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
  return __builtin_bit_cast(bf16x8_t, u32x4_t{v.x, v.y, v.z, v.w});
}

// fp32 -> nearest bf16 (ties to even), returned as fp32: the value of the
// reference's bf16 lm_head output.
__device__ __forceinline__ float bf16_round(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// Candidate key of a logit: the order-preserving 16-bit key of its bf16 bits
// above the complement of its index within the 128-entry tile, so that a
// larger key is a larger value or, for equal values, a lower index.  Key 0
// is an empty slot (no finite logit maps to it).
__device__ __forceinline__ uint32_t value_key16(float xr) {
  const uint32_t b = __float_as_uint(xr) >> 16;
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}
__device__ __forceinline__ uint32_t cand_key(float xr, int local) {
  // The value key is the high half of bits ^ (sign ? ~0 : 0x80000000) (the
  // low 16 bits of a bf16-rounded value are zero).
  const uint32_t b = __float_as_uint(xr);
  const uint32_t m = (uint32_t)((int32_t)b >> 31) | 0x80000000u;
  return ((b ^ m) & 0xffff0000u) | (0xffffu ^ (uint32_t)local);
}
__device__ __forceinline__ float key_value(uint32_t key) {
  const uint32_t k = key >> 16;
  const uint32_t b = (k & 0x8000u) ? (k & 0x7fffu) : (~k & 0xffffu);
  return bf16_to_f32((uint16_t)b);
}
__device__ __forceinline__ int key_local(uint32_t key) { return (int)((key & 0xffffu) ^ 0xffffu); }

__device__ __forceinline__ uint32_t umed3(uint32_t a, uint32_t b, uint32_t c) {
  return max(min(a, b), min(max(a, b), c));  // v_med3_u32
}

// The four largest keys, c0 > c1 > c2 > c3 (0 = empty).  Inserting x keeps
// the four largest of the five: with the list sorted, max(c_i, min(c_{i-1}, x))
// is med3(c_{i-1}, c_i, x).
struct Top4 {
  uint32_t c0, c1, c2, c3;
  __device__ __forceinline__ void insert(uint32_t x) {
    const uint32_t n3 = umed3(c2, c3, x), n2 = umed3(c1, c2, x), n1 = umed3(c0, c1, x);
    c0 = max(c0, x);
    c1 = n1;
    c2 = n2;
    c3 = n3;
  }
  // Adds another list whose keys are distinct from this one's.
  __device__ __forceinline__ void merge(const Top4& o) {
    insert(o.c0);
    insert(o.c1);
    insert(o.c2);
    insert(o.c3);
  }
};

// The union of the lists of lanes l and l ^ XOR (XOR = 16 or 32), identical
// on both lanes: the lane swaps hand every lane the pair's two lists, which
// are merged from empty in the same order on both sides.
template <int XOR>
__device__ __forceinline__ Top4 top4_pair_union(const Top4& t) {
  uint32_t lo[4], hi[4];
  const uint32_t v[4] = {t.c0, t.c1, t.c2, t.c3};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto r = XOR == 16 ? __builtin_amdgcn_permlane16_swap(v[i], v[i], false, false)
                             : __builtin_amdgcn_permlane32_swap(v[i], v[i], false, false);
    lo[i] = r[0];
    hi[i] = r[1];
  }
  Top4 u{lo[0], lo[1], lo[2], lo[3]};
  u.merge(Top4{hi[0], hi[1], hi[2], hi[3]});
  return u;
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
// steps ahead.  Wave (vq, rq) owns vocabulary rows VW vq .. +VW and
// hidden-state rows 64 rq .. +64, and writes the (max, sum) pair of its VW
// entries for each of its rows (pair v0 / VW + vq).  Rows past the
// vocabulary or the batch load the last valid row (their results are
// masked or not written).  Per-item H traffic is what bounds this kernel at
// a few hundred rows and above (each item re-reads its MT x hidden rows from
// L2): 256-entry items halve it per FLOP.  TOPK also writes each (row, tile)'s
// four largest logits as candidate keys (cand[row * n_vtiles + tile]).
template <int MT, int NW, int NSTAGE, int TVB, bool TOPK, bool XO>
__global__ __launch_bounds__(NW * 64) void lmhead_items(
    const uint16_t* __restrict__ h, int64_t h_stride, int n_rows,
    const uint16_t* __restrict__ w, int64_t w_stride, int vocab, int hidden, float c2,
    int n_vtiles, int n_rtiles, float2* __restrict__ part, uint4* __restrict__ cand) {
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
  __shared__ uint4 redk[WPT > 1 && TOPK ? NVQ : 1][WPT > 1 && TOPK ? MT : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g4 = lane >> 4;
  const int vq = wave % NVQ, rq = wave / NVQ;
  const int n_kc = hidden / kKC;
  const int n_vitems = (n_vtiles + TVB - 1) / TVB;
  const int n_pairs = (vocab + VW - 1) / VW;  // (max, sum) pairs per row
  const int n_items = n_vitems * n_rtiles;
  // Item order.  With one row tile every item shares the hidden-state tile,
  // and a workgroup takes a contiguous range of items.  With several row
  // tiles (the loss step's thousands of rows) the L2 of an XCD could not
  // hold the weight tiles of 32 workgroups each walking every row tile, so
  // the order is XCD-aware (XO, grid a multiple of 8): workgroups are placed
  // on the 8 XCDs round robin by index, XCD x takes vocabulary items
  // [x V / 8, (x + 1) V / 8), and its G workgroups take that range's items
  // strided by G from a sequence that runs, per group of kGV vocabulary
  // items, row tile by row tile -- so the items an XCD has in flight at any
  // time form a block of kGV vocabulary items x G / kGV row tiles whose tiles
  // its L2 shares (at 8,192 rows 16.5 -> 3.8 GB of L2 misses per launch).
  // Any placement gives the same items and results; only the reuse depends
  // on it.
  constexpr int kGV = 8;
  constexpr bool xcd = XO;
  const int gx = blockIdx.x % 8, gj = blockIdx.x / 8, gG = gridDim.x / 8;
  const int vlo = xcd ? (int)((int64_t)gx * n_vitems / 8) : 0;
  const int nv = xcd ? (int)((int64_t)(gx + 1) * n_vitems / 8) - vlo : 0;
  const int n_local = nv * n_rtiles;
  const int i_begin = (int)((int64_t)blockIdx.x * n_items / gridDim.x);
  const int i_end = (int)((int64_t)(blockIdx.x + 1) * n_items / gridDim.x);
  const int n_mine = xcd ? (n_local > gj ? (n_local - gj + gG - 1) / gG : 0) : i_end - i_begin;
  const int n_steps = n_mine * n_kc;
  if (n_steps == 0) return;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)lds;

  // Position (vocabulary item, row tile) of this workgroup's k-th item.
  struct Pos {
    int vi, rt;
  };
  auto pos_of = [&](int k) -> Pos {
    if constexpr (xcd) {
      const int il = gj + k * gG;                  // index in the XCD's sequence
      const int g = il / (kGV * n_rtiles);         // group of kGV vocabulary items
      const int gv = min(kGV, nv - g * kGV);       // (the last group may be narrower)
      const int r = il - g * kGV * n_rtiles;
      return Pos{vlo + g * kGV + r % gv, r / gv};
    }
    const int i = i_begin + k;
    return Pos{i / n_rtiles, i % n_rtiles};
  };
  auto advance = [&](Pos p, int& k) -> Pos {
    ++k;
    if constexpr (xcd) return pos_of(k);
    return p.rt + 1 == n_rtiles ? Pos{p.vi + 1, 0} : Pos{p.vi, p.rt + 1};
  };
  const Pos p_begin = pos_of(0);

  // Load stream.  Wave-load j of this wave covers staged rows 8 (LPW' wave +
  // j) .. +8 of W (then of H); lane l fetches row + l / 8, physical piece
  // l % 8, i.e. logical piece (l % 8) ^ ((row / 2) % 8).
  Pos ld = p_begin;
  int ld_kc = 0, ld_step = 0, ld_k = 0;
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
        ld = advance(ld, ld_k);
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

  // Epilogue of an item: per row, (max, sum of exp2) over each wave's VW
  // entries of the vocabulary (pair v / VW; the top-k mode needs none);
  // acc[vb][rb][e] holds vocabulary v0 + VW vq + 16 vb + 4 g4 + e of row
  // r0 + 64 rq + 16 rb + l16.  Each logit is first rounded to bf16 (the
  // reference's lm_head output).
  auto epilogue = [&](Pos it) __attribute__((always_inline)) {
    const int64_t v0 = (int64_t)it.vi * TV;
    const int64_t r0 = (int64_t)it.rt * MT;
    const int64_t vbase = v0 + VW * vq + 4 * g4;
    const int vt = (int)(v0 / kTV) + (VW * vq) / kTV;  // this wave's 128-row tile
    const int lbase = (VW * vq) % kTV + 4 * g4;        // its first entry within the tile
    const int pidx = (int)(v0 / VW) + vq;              // this wave's (max, sum) pair
    // Only an item that reaches past the end of the vocabulary checks each
    // entry (a wave-uniform choice between two copies of the loop).
    const int vrel = vocab - (int)vbase;  // entries of this lane's columns that exist: j < vrel
    auto rows = [&](auto check) __attribute__((always_inline)) {
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const int row_l = 64 * rq + 16 * rb + l16;
      const int64_t row = r0 + row_l;
#pragma unroll
      for (int vb = 0; vb < VB; ++vb)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[vb][rb][e] = bf16_round(acc[vb][rb][e]);
      if constexpr (TOPK) {
        Top4 t{0u, 0u, 0u, 0u};
#pragma unroll
        for (int vb = 0; vb < VB; ++vb)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (!check || 16 * vb + e < vrel) t.insert(cand_key(acc[vb][rb][e], lbase + 16 * vb + e));
        t = top4_pair_union<16>(t);
        t = top4_pair_union<32>(t);
        if constexpr (WPT > 1) {
          if (g4 == 0) redk[vq][row_l] = make_uint4(t.c0, t.c1, t.c2, t.c3);
        } else {
          if (g4 == 0 && row < n_rows && vt < n_vtiles)
            cand[row * (int64_t)n_vtiles + vt] = make_uint4(t.c0, t.c1, t.c2, t.c3);
        }
      }
      if constexpr (!TOPK) {
        // (max, sum of exp2) of x c2 over the wave's slice of the row: the
        // maximum over the four lanes holding the row first (c2 > 0, so it is
        // taken on the logits and scaled once), then every lane's terms
        // against it and one cross-lane sum; entries past the vocabulary add
        // nothing.
        float mx = kNegBig;
#pragma unroll
        for (int vb = 0; vb < VB; ++vb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const bool ok = !check || 16 * vb + e < vrel;
            mx = fmaxf(mx, ok ? acc[vb][rb][e] : kNegBig);
          }
        mx = rows4_max(mx) * c2;
        float sm = 0.f;
#pragma unroll
        for (int vb = 0; vb < VB; ++vb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const bool ok = !check || 16 * vb + e < vrel;
            const float p = fast_exp2(fmaf(acc[vb][rb][e], c2, -mx));
            sm += ok ? p : 0.f;
          }
        sm = rows4_sum(sm);
        if (g4 == 0 && row < n_rows && pidx < n_pairs) part[row * (int64_t)n_pairs + pidx] = make_float2(mx, sm);
      }
#pragma unroll
      for (int vb = 0; vb < VB; ++vb) acc[vb][rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    };
    if (v0 + TV <= vocab)
      rows(std::false_type{});
    else
      rows(std::true_type{});
    if constexpr (WPT > 1 && TOPK) {
      __syncthreads();
      // Waves WPT tj .. WPT tj + WPT - 1 hold the item's tile tj.
      for (int r = tid; r < MT; r += NW * 64) {
        if (r0 + r < n_rows) {
#pragma unroll
          for (int tj = 0; tj < TVB; ++tj) {
            const int vt = (int)(v0 / kTV) + tj;
            if (vt < n_vtiles) {
              const uint4 k0 = redk[WPT * tj][r];
              Top4 t{k0.x, k0.y, k0.z, k0.w};
#pragma unroll
              for (int j = 1; j < WPT; ++j) {
                const uint4 kj = redk[WPT * tj + j][r];
                t.merge(Top4{kj.x, kj.y, kj.z, kj.w});
              }
              cand[(r0 + r) * (int64_t)n_vtiles + vt] = make_uint4(t.c0, t.c1, t.c2, t.c3);
            }
          }
        }
      }
    }
  };

  // Step st: issue step st + NSTAGE - 1 into its stage (last read in step
  // st - 1, which ended with a barrier), multiply stage st % NSTAGE, then
  // wait for this wave's loads of step st + 1 and meet at the barrier.
  Pos it = p_begin;
  int it_k = 0;
  int kc = 0, stage = 0;
#pragma unroll
  for (int i = 0; i < NSTAGE - 1; ++i) issue(i);
  asm volatile("s_waitcnt vmcnt(%0)" ::"i"((NSTAGE - 2) * LPW) : "memory");
  __syncthreads();
  for (int st = 0; st < n_steps; ++st) {
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
      it = advance(it, it_k);
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

// The Philox4x32-10 uniform of a row: u in (0, 1) with 53 bits from words 0
// and 1 of the block at counter (0, lo32(q), lo32(offset) + hi32(q),
// hi32(offset)), key (seed_lo, seed_hi), where q is the row's 64-bit counter
// value (row_ctr[row], or the row index when row_ctr is NULL).
__device__ __forceinline__ double row_uniform(int row, const uint64_t* __restrict__ row_ctr,
                                              uint32_t seed_lo, uint32_t seed_hi, uint32_t off_lo,
                                              uint32_t off_hi) {
  const uint64_t q = row_ctr ? row_ctr[row] : (uint64_t)row;
  const uint4 r = philox4x32_10(make_uint4(0u, (uint32_t)q, off_lo + (uint32_t)(q >> 32), off_hi),
                                seed_lo, seed_hi);
  const uint64_t bits = ((uint64_t)r.x << 21) | (uint64_t)(r.y >> 11);
  return ((double)bits + 0.5) * 0x1p-53;
}

// Copies a hidden-state row into LDS (read by tile_logits).
__device__ __forceinline__ void load_hrow(const uint16_t* __restrict__ hr, int hidden,
                                          uint16_t* hrow) {
  for (int k = 8 * (int)threadIdx.x; k < hidden; k += 8 * kRowThreads)
    *reinterpret_cast<uint4*>(hrow + k) = load_u4(hr + k);
}

// The bf16-rounded logits of vocabulary entries first .. first + count
// (count 32, 64 or 128) for the hidden-state row in LDS, into xs[count]
// (-inf past the vocabulary).  Wave i computes entries first + 32 i .. +32
// (waves past count skip) with the MFMA sequence of lmhead_items (the same
// operand layout, hidden elements in the same order: 32 at a time, lane group
// g4 supplying elements 8 g4 .. +8 of each 32; each 16-entry block
// accumulates on its own), every column of the B operand holding the row, so
// the values are bit-identical to the ones lmhead_items reduced.
__device__ __forceinline__ void entry_logits(const uint16_t* hrow, const uint16_t* __restrict__ w,
                                             int64_t w_stride, int vocab, int hidden, int64_t first,
                                             int count, float* xs) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  if (32 * wave >= count) return;  // wave-uniform
  const int64_t vw = first + 32 * wave;
  const uint16_t* wr0 = w + (vw + l16 < vocab ? vw + l16 : (int64_t)vocab - 1) * w_stride + 8 * g4;
  const uint16_t* wr1 = w + (vw + 16 + l16 < vocab ? vw + 16 + l16 : (int64_t)vocab - 1) * w_stride + 8 * g4;
  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  // The W pieces of 64-element steps go out kAhead steps before their MFMAs
  // (a register ring), so the 2 KB-strided rows cost a few memory round trips
  // rather than one per step.  The steady-state loop has no conditional
  // loads (a fetch past the last step re-reads the last step, unused), so
  // the compiler's waits keep the ring in flight.
  constexpr int kAhead = 8;
  const int n_it = hidden / 64;  // hidden is a multiple of 64
  uint4 ring[kAhead][4];
  auto fetch = [&](uint4* r, int it) __attribute__((always_inline)) {
    const int k = 64 * min(it, n_it - 1);
    r[0] = load_u4(wr0 + k);
    r[1] = load_u4(wr1 + k);
    r[2] = load_u4(wr0 + k + 32);
    r[3] = load_u4(wr1 + k + 32);
  };
  auto step = [&](const uint4* r, int it) __attribute__((always_inline)) {
    const int k = 64 * it;
    const bf16x8_t b0 = as_bf16x8(*reinterpret_cast<const uint4*>(hrow + k + 8 * g4));
    const bf16x8_t b1 = as_bf16x8(*reinterpret_cast<const uint4*>(hrow + k + 32 + 8 * g4));
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(r[0]), b0, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(r[1]), b0, acc1, 0, 0, 0);
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(r[2]), b1, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(r[3]), b1, acc1, 0, 0, 0);
  };
#pragma unroll
  for (int j = 0; j < kAhead; ++j) fetch(ring[j], j);
  int i0 = 0;
  for (; i0 + kAhead <= n_it; i0 += kAhead) {
#pragma unroll
    for (int j = 0; j < kAhead; ++j) {
      step(ring[j], i0 + j);
      fetch(ring[j], i0 + j + kAhead);
    }
  }
#pragma unroll
  for (int j = 0; j < kAhead; ++j)
    if (i0 + j < n_it) step(ring[j], i0 + j);
  if (l16 == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t v0 = vw + 4 * g4 + e, v1 = v0 + 16;
      xs[32 * wave + 4 * g4 + e] = v0 < vocab ? bf16_round(acc0[e]) : -INFINITY;
      xs[32 * wave + 16 + 4 * g4 + e] = v1 < vocab ? bf16_round(acc1[e]) : -INFINITY;
    }
  }
}

__global__ __launch_bounds__(kRowThreads) void lmhead_sample_rows(
    const float2* __restrict__ part, int n_pairs, int sub, const uint16_t* __restrict__ h,
    int64_t h_stride, const uint16_t* __restrict__ w, int64_t w_stride, int vocab, int hidden,
    float c2, uint32_t seed_lo, uint32_t seed_hi, uint32_t off_lo, uint32_t off_hi,
    const uint64_t* __restrict__ row_ctr, int64_t* __restrict__ out_tok, float* __restrict__ out_lp) {
  __shared__ float smf[4];
  __shared__ double smd[5];
  __shared__ float xs[kTV];
  __shared__ int sel_tile;
  __shared__ double sel_resid;
  __shared__ __align__(16) uint16_t hrow[kMaxHidden];
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  // The row's (max, sum) pairs, one per `sub` vocabulary entries.
  const float2* pr = part + (int64_t)row * n_pairs;
  const int cpt = (n_pairs + kRowThreads - 1) / kRowThreads;
  const int lo = min(n_pairs, tid * cpt), hi = min(n_pairs, lo + cpt);
  // A thread's pairs are read once into registers when they fit (up to
  // 5,120 pairs), in flight together with the hidden-state row; entries past
  // its chunk hold (-big, 0), which add exactly zero to the fp64 sums.
  constexpr int kPR = 20;
  const bool regs = cpt <= kPR;
  float2 pv[kPR];
  if (regs) {
#pragma unroll
    for (int i = 0; i < kPR; ++i) pv[i] = lo + i < hi ? pr[lo + i] : make_float2(kNegBig, 0.f);
  }
  const double u = row_uniform(row, row_ctr, seed_lo, seed_hi, off_lo, off_hi);
  load_hrow(h + (int64_t)row * h_stride, hidden, hrow);
  double own, excl;
  RowLse L;
  if (regs) {
    float mx = kNegBig;
#pragma unroll
    for (int i = 0; i < kPR; ++i) mx = fmaxf(mx, pv[i].x);
    L.m2 = block_max256(mx, smf);
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < kPR; ++i) acc += (double)(pv[i].y * fast_exp2(pv[i].x - L.m2));
    own = acc;
    excl = block_excl_scan256(acc, smd, &L.s);
  } else {
    L = row_lse(pr, n_pairs, cpt, &own, &excl, smf, smd);
  }
  const double target = u * L.s;

  if (tid == 0) {
    sel_tile = -1;
    sel_resid = 0.0;
  }
  __syncthreads();
  if (own > 0.0 && target >= excl && target < excl + own) {
    double cum = excl;
    int t = lo;
    if (regs) {
      bool found = false;
#pragma unroll
      for (int i = 0; i < kPR - 1; ++i) {
        if (!found && lo + i < hi - 1) {
          const double p = (double)(pv[i].y * fast_exp2(pv[i].x - L.m2));
          if (target < cum + p) {
            found = true;
          } else {
            cum += p;
            t = lo + i + 1;
          }
        }
      }
    } else {
      for (; t < hi - 1; ++t) {
        const double p = (double)(pr[t].y * fast_exp2(pr[t].x - L.m2));
        if (target < cum + p) break;
        cum += p;
      }
    }
    sel_tile = t;
    sel_resid = target - cum;
  }
  __syncthreads();
  if (sel_tile < 0) {
    // u * S rounded up to S: the last pair with mass, at its last entry.
    if (tid == 0) {
      int t = n_pairs - 1;
      while (t > 0 && !(pr[t].y * fast_exp2(pr[t].x - L.m2) > 0.f)) --t;
      sel_tile = t;
      sel_resid = 1e300;
    }
    __syncthreads();
  }
  const int64_t first = (int64_t)sel_tile * sub;
  entry_logits(hrow, w, w_stride, vocab, hidden, first, sub, xs);
  __syncthreads();
  // Within the pair's entries: the first whose cumulative mass exceeds the
  // residual (wave 0, two entries per lane, fixed-order scan).
  if (tid < 64) {
    const double resid = sel_resid;
    const float x0 = 2 * tid < sub ? xs[2 * tid] : -INFINITY;
    const float x1 = 2 * tid + 1 < sub ? xs[2 * tid + 1] : -INFINITY;
    const double p0 = x0 == -INFINITY ? 0.0 : (double)fast_exp2(x0 * c2 - L.m2);
    const double p1 = x1 == -INFINITY ? 0.0 : (double)fast_exp2(x1 * c2 - L.m2);
    const double inc = wave_scan_f64(p0 + p1);
    const double before = inc - (p0 + p1);
    int cand = sub;
    if (resid < before + p0) cand = 2 * tid;
    else if (resid < inc) cand = 2 * tid + 1;
    int last = p1 > 0.0 ? 2 * tid + 1 : (p0 > 0.0 ? 2 * tid : -1);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      cand = min(cand, __shfl_xor(cand, m, 64));
      last = max(last, __shfl_xor(last, m, 64));
    }
    if (tid == 0) {
      const int pick = cand < sub ? cand : (last >= 0 ? last : 0);
      out_tok[row] = first + pick;
      if (out_lp) {
        const double lse2 = (double)L.m2 + log2(L.s);
        out_lp[row] = (float)(((double)(xs[pick] * c2) - lse2) * (double)kLn2);
      }
    }
  }
}

// Exclusive prefix (fixed order) of one int per thread over the 256 threads;
// also returns the total.  sm holds 4 ints.
__device__ int block_excl_scan_i32(int x, int* sm, int* total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int inc = x;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(inc, d, 64);
    if (lane >= d) inc += y;
  }
  __syncthreads();
  if (lane == 63) sm[wv] = inc;
  __syncthreads();
  int base = 0;
  for (int j = 0; j < wv; ++j) base += sm[j];
  *total = sm[0] + sm[1] + sm[2] + sm[3];
  return base + inc - x;
}

// Top-k sampling from the per-(row, tile) candidates of lmhead_items (TOPK).
// The kept set is the k largest logits, ties at the k-th value kept in
// vocabulary order (lowest indices first).  Every entry of the kept set
// outside a tile's four candidates would need four larger ones in the same
// tile: a tile whose fourth candidate is kept ("saturated", at most k / 4 of
// them) is recomputed in full (tile_logits) and the selection repeated over
// the tiles' candidates with those tiles' 128 logits in place of their four;
// adding entries only raises the k-th value, so no further tile saturates.
// One 256-lane workgroup per row; thread t owns the contiguous tiles
// [t cpt, t cpt + cpt), which keeps every scan in vocabulary order.
__global__ __launch_bounds__(kRowThreads) void lmhead_topk_rows(
    const uint4* __restrict__ cand, int n_vtiles, const uint16_t* __restrict__ h, int64_t h_stride,
    const uint16_t* __restrict__ w, int64_t w_stride, int vocab, int hidden, int k, float c2,
    uint32_t seed_lo, uint32_t seed_hi, uint32_t off_lo, uint32_t off_hi,
    const uint64_t* __restrict__ row_ctr, int64_t* __restrict__ out_tok, float* __restrict__ out_lp) {
  constexpr int kMaxSat = kMaxFusedTopK / 4;
  __shared__ uint32_t hist[256];
  __shared__ int sel[3];  // threshold value key, entries above it, equal ones kept
  __shared__ int smi[4];
  __shared__ double smd[5];
  __shared__ float smf[4];
  __shared__ int n_sat;
  __shared__ int sat_tile[kMaxSat];
  __shared__ float sat_x[kMaxSat][kTV];
  __shared__ int kept_idx[kMaxFusedTopK];
  __shared__ float kept_x[kMaxFusedTopK];  // logit * c2
  __shared__ int pick_sm;
  __shared__ __align__(16) uint16_t hrow[kMaxHidden];
  __shared__ uint4 cr[kMaxCandTiles];  // the row's candidates, read once
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const uint4* crg = cand + (int64_t)row * n_vtiles;
  for (int t = tid; t < n_vtiles; t += kRowThreads) cr[t] = crg[t];
  const int cpt = (n_vtiles + kRowThreads - 1) / kRowThreads;
  const int lo = min(n_vtiles, tid * cpt), hi = min(n_vtiles, lo + cpt);
  if (tid == 0) n_sat = 0;

  // The candidates of tile t in descending key order (equal values in
  // vocabulary order): the expanded tile's 128 logits in index order carry
  // the same keys, so both forms feed f(key, vocabulary index).
  auto slot_of = [&](int t) {
    const int ns = min(n_sat, kMaxSat);
    for (int j = 0; j < ns; ++j)
      if (sat_tile[j] == t) return j;
    return -1;
  };
  auto for_each = [&](auto&& f) {
    for (int t = lo; t < hi; ++t) {
      const int sl = slot_of(t);
      if (sl >= 0) {
        for (int j = 0; j < kTV; ++j) {
          const float x = sat_x[sl][j];
          if (x != -INFINITY) f(cand_key(x, j), t * kTV + j);
        }
      } else {
        const uint4 c = cr[t];
        const uint32_t kk[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (kk[j]) f(kk[j], t * kTV + key_local(kk[j]));
      }
    }
  };
  // The bin of the histogram that holds the need-th largest entry, by one
  // block-wide scan (thread t takes bin 255 - t): the bin b with fewer than
  // `need` entries above it and at least `need` from it up.  Returns b and
  // the entries above it; with fewer than `need` entries in all, -1 (or, when
  // `floor0`, bin 0 with everything above it).
  auto find_bin = [&](int need, bool floor0, int* above_out) {
    const int b = 255 - tid;
    const int c = (int)hist[b];
    int tot;
    const int above = block_excl_scan_i32(c, smi, &tot);  // entries in bins > b
    const bool hit = tot >= need ? (above < need && above + c >= need) : (floor0 && b == 0);
    if (tot < need && !floor0 && tid == 0) sel[0] = -1;
    if (hit) {
      sel[0] = b;
      sel[1] = above;
    }
    __syncthreads();
    *above_out = sel[1];
    return sel[0];
  };
  // Radix select of the k-th largest value key (16 bits, high byte then low
  // byte); sel = {threshold, entries above it, entries equal to it that are
  // kept}.  Fewer than k entries in all: threshold 0, every entry kept.
  auto select = [&]() {
    hist[tid] = 0;
    __syncthreads();
    for_each([&](uint32_t key, int) { atomicAdd(&hist[key >> 24], 1u); });
    __syncthreads();
    int cum;
    const int hb = find_bin(k, false, &cum);  // high byte, or -1 when everything is kept
    __syncthreads();
    if (hb < 0) {
      if (tid == 0) {
        sel[0] = 0;
        sel[2] = 0;
      }
      __syncthreads();
      return;
    }
    hist[tid] = 0;
    __syncthreads();
    for_each([&](uint32_t key, int) {
      if ((int)(key >> 24) == hb) atomicAdd(&hist[(key >> 16) & 0xffu], 1u);
    });
    __syncthreads();
    int above;
    const int lb = find_bin(k - cum, true, &above);
    __syncthreads();
    if (tid == 0) {
      sel[0] = (hb << 8) | lb;
      sel[1] = cum + above;
      sel[2] = k - (cum + above);
    }
    __syncthreads();
  };

  // Pass 1 over the four candidates per tile.
  __syncthreads();
  select();
  {
    const uint32_t tk = (uint32_t)sel[0];
    const int need_eq = sel[2];
    int eq = 0;
    for_each([&](uint32_t key, int) { eq += (key >> 16) == tk; });
    int tot;
    int eq_at = block_excl_scan_i32(eq, smi, &tot);
    for (int t = lo; t < hi; ++t) {
      const uint4 c = cr[t];
      const uint32_t kk[4] = {c.x, c.y, c.z, c.w};
      bool kept3 = false;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t v = kk[j] >> 16;
        const bool kept = kk[j] && (v > tk || (v == tk && eq_at < need_eq));
        if (kk[j] && v == tk) ++eq_at;
        if (j == 3) kept3 = kept;
      }
      if (kept3) {
        const int sl = atomicAdd(&n_sat, 1);
        if (sl < kMaxSat) sat_tile[sl] = t;
      }
    }
  }
  __syncthreads();
  const int ns = min(n_sat, kMaxSat);
  if (ns > 0) {
    // Saturated tiles: all 128 logits, then the selection once more.
    load_hrow(h + (int64_t)row * h_stride, hidden, hrow);
    __syncthreads();
    for (int j = 0; j < ns; ++j)
      entry_logits(hrow, w, w_stride, vocab, hidden, (int64_t)sat_tile[j] * kTV, kTV, sat_x[j]);
    __syncthreads();
    select();
  }

  // The kept entries, gathered in vocabulary order.
  const uint32_t tk = (uint32_t)sel[0];
  const int need_eq = sel[2];
  int gt = 0, eq = 0;
  for_each([&](uint32_t key, int) {
    gt += (key >> 16) > tk;
    eq += (key >> 16) == tk;
  });
  int tot;
  const int eq_before = block_excl_scan_i32(eq, smi, &tot);
  const int take = max(0, min(eq, need_eq - eq_before));
  int pos = block_excl_scan_i32(gt + take, smi, &tot);
  const int nk = tot;  // k, or every entry when there are fewer
  {
    int taken = 0;
    for (int t = lo; t < hi; ++t) {
      // Kept entries of tile t in index order: at most 3 of the four
      // candidates of a tile that did not saturate, any of an expanded one.
      int ki[4];
      float kx[4];
      int nkt = 0;
      const int sl = slot_of(t);
      if (sl >= 0) {
        for (int j = 0; j < kTV; ++j) {
          const float x = sat_x[sl][j];
          if (x == -INFINITY) continue;
          const uint32_t v = value_key16(x);
          const bool keep = v > tk || (v == tk && taken < take);
          if (v == tk && keep) ++taken;
          if (keep) {
            kept_idx[pos] = t * kTV + j;
            kept_x[pos] = x * c2;
            ++pos;
          }
        }
        continue;
      }
      const uint4 c = cr[t];
      const uint32_t kk[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t v = kk[j] >> 16;
        const bool keep = kk[j] && (v > tk || (v == tk && taken < take));
        if (kk[j] && v == tk && keep) ++taken;
        if (keep) {
          ki[nkt] = t * kTV + key_local(kk[j]);
          kx[nkt] = key_value(kk[j]);
          ++nkt;
        }
      }
      // Insertion sort by index (value order -> vocabulary order).
      for (int a = 1; a < nkt; ++a)
        for (int b = a; b > 0 && ki[b - 1] > ki[b]; --b) {
          const int ti = ki[b];
          ki[b] = ki[b - 1];
          ki[b - 1] = ti;
          const float tx = kx[b];
          kx[b] = kx[b - 1];
          kx[b - 1] = tx;
        }
      for (int a = 0; a < nkt; ++a) {
        kept_idx[pos] = ki[a];
        kept_x[pos] = kx[a] * c2;
        ++pos;
      }
    }
  }
  __syncthreads();

  // Inverse transform sampling over the kept entries (x c2, rounded once when
  // stored, so that every use below sees the same value) in vocabulary order.
  float mx = kNegBig;
  for (int j = tid; j < nk; j += kRowThreads) mx = fmaxf(mx, kept_x[j]);
  const float m2 = block_max256(mx, smf);
  double p = 0.0;
  if (tid < nk) p = (double)fast_exp2(kept_x[tid] - m2);
  double s_tot;
  const double excl = block_excl_scan256(p, smd, &s_tot);
  const double target = row_uniform(row, row_ctr, seed_lo, seed_hi, off_lo, off_hi) * s_tot;
  if (tid == 0) pick_sm = nk - 1;  // u * S rounded up to S: the last entry
  __syncthreads();
  if (tid < nk && p > 0.0 && target >= excl && target < excl + p) pick_sm = tid;
  __syncthreads();
  if (tid == 0) {
    const int j = pick_sm;
    out_tok[row] = kept_idx[j];
    if (out_lp) {
      const double lse2 = (double)m2 + log2(s_tot);
      out_lp[row] = (float)(((double)kept_x[j] - lse2) * (double)kLn2);
    }
  }
}

// The bf16-rounded logit of one vocabulary entry for one hidden-state row
// (weight row wr and hidden row hr staged in LDS), by one wave: the MFMA
// sequence of lmhead_items with the entry's weight row in all 16 rows of the
// A operand and the hidden row in all 16 columns of B.  Every output element
// is then the same dot product, summed in the item kernel's order (32 hidden
// elements per MFMA, in increasing order), so the value is bit-identical to
// the one that entered the entry's (max, sum) pair.
__device__ __forceinline__ float entry_logit(const uint16_t* hr, const uint16_t* wr, int hidden) {
  const int g4 = (threadIdx.x & 63) >> 4;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int k = 8 * g4; k < hidden; k += 64) {  // hidden is a multiple of 64
    const bf16x8_t a0 = as_bf16x8(*reinterpret_cast<const uint4*>(wr + k));
    const bf16x8_t a1 = as_bf16x8(*reinterpret_cast<const uint4*>(wr + k + 32));
    const bf16x8_t b0 = as_bf16x8(*reinterpret_cast<const uint4*>(hr + k));
    const bf16x8_t b1 = as_bf16x8(*reinterpret_cast<const uint4*>(hr + k + 32));
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, acc, 0, 0, 0);
  }
  return bf16_round(acc[0]);
}

// lse and lp = x[target] - lse per row: the lse from the row's pairs, the
// target's logit recomputed (entry_logit) from its weight row and the hidden
// row, both copied into LDS by the whole workgroup (one round trip, beside
// the pair reads).  A target outside the vocabulary has no logit: NaN (the
// reference's gather would raise).  Dynamic LDS: 4 * hidden bytes.
__global__ __launch_bounds__(kRowThreads) void lmhead_logprob_rows(
    const float2* __restrict__ part, int n_pairs, const uint16_t* __restrict__ h,
    int64_t h_stride, const uint16_t* __restrict__ w, int64_t w_stride,
    const int64_t* __restrict__ tgt, int64_t tgt_stride, int vocab, int hidden, float c2,
    float* __restrict__ out_lp, float* __restrict__ out_lse) {
  __shared__ float smf[4];
  __shared__ double smd[5];
  extern __shared__ __align__(16) uint16_t rows_lds[];  // [hidden] weight row, [hidden] hidden row
  const int row = blockIdx.x;
  const int64_t t = tgt[(int64_t)row * tgt_stride];
  const bool valid = t >= 0 && t < vocab;  // uniform over the workgroup
  if (valid) {
    const uint16_t* wr = w + t * w_stride;
    const uint16_t* hr = h + (int64_t)row * h_stride;
    for (int k = 8 * (int)threadIdx.x; k < hidden; k += 8 * kRowThreads) {
      *reinterpret_cast<uint4*>(rows_lds + k) = load_u4(wr + k);
      *reinterpret_cast<uint4*>(rows_lds + hidden + k) = load_u4(hr + k);
    }
  }
  const int cpt = (n_pairs + kRowThreads - 1) / kRowThreads;
  double own, excl;
  const RowLse L = row_lse(part + (int64_t)row * n_pairs, n_pairs, cpt, &own, &excl, smf, smd);
  __syncthreads();  // the rows in LDS
  float x = 0.f;
  if (valid && threadIdx.x < 64) x = entry_logit(rows_lds + hidden, rows_lds, hidden);
  if (threadIdx.x == 0) {
    const double lse = ((double)L.m2 + log2(L.s)) * (double)kLn2;  // of x * c2 / log2(e)
    if (out_lse) out_lse[row] = (float)lse;
    out_lp[row] = valid ? (float)((double)x * (double)c2 * (double)kLn2 - lse) : __builtin_nanf("");
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct LmWs {
  float2* part;
  uint4* cand;
};

inline int64_t n_vtiles_of(int64_t vocab) { return (vocab + kTV - 1) / kTV; }
inline int64_t round256(int64_t b) { return (b + 255) & ~(int64_t)255; }

// Vocabulary entries per (max, sum) pair: what one wave of the item kernel
// covers in the configuration launch_tiles picks for n_rows (items of
// 128 x 64 with 4 waves, 256 x 128 with 8 waves of 64 x 64, 256 x 256 with
// 8 waves of 128 x 64).
inline int pair_entries(int64_t n_rows) { return n_rows <= 64 ? 32 : n_rows <= 256 ? 64 : 128; }
inline int64_t n_pairs_of(int64_t n_rows, int64_t vocab) {
  const int e = pair_entries(n_rows);
  return (vocab + e - 1) / e;
}

// Workspace: (max, sum) pairs [rows, pairs] fp32x2, then with top-k the
// candidate keys [rows, tiles] uint32x4.
inline int64_t ws_bytes(int64_t n_rows, int64_t vocab, bool topk) {
  const int64_t np = n_pairs_of(n_rows, vocab);
  const int64_t b = round256(n_rows * np * (int64_t)sizeof(float2));
  return topk ? b + n_rows * n_vtiles_of(vocab) * (int64_t)sizeof(uint4) : b;
}

inline LmWs ws_layout(void* ws, int64_t n_rows, int64_t vocab) {
  const int64_t np = n_pairs_of(n_rows, vocab);
  const int64_t p = round256(n_rows * np * (int64_t)sizeof(float2));
  char* base = static_cast<char*>(ws);
  return {reinterpret_cast<float2*>(base), reinterpret_cast<uint4*>(base + p)};
}

int check_args(const uint16_t* h, int64_t h_stride, int64_t n_rows, const uint16_t* w,
               int64_t w_stride, int64_t vocab, int64_t hidden, void* ws, int64_t ws_size,
               bool topk) {
  if (n_rows < 0 || vocab <= 0 || hidden <= 0) return QMI_E_BAD_SHAPE;
  if (!h || !w || !ws) return QMI_E_NULL_POINTER;
  if (hidden % kKC != 0 || hidden > kMaxHidden) return QMI_E_UNSUPPORTED;
  if (vocab > 0x7fffffffLL - kTV || n_rows > 0x7fffffffLL) return QMI_E_UNSUPPORTED;
  // The item kernel counts its work items and (item, chunk) steps in 32-bit
  // integers: at most n_vtiles x ceil(n_rows / 64) items of hidden / 64 steps.
  if (n_vtiles_of(vocab) * ((n_rows + 63) / 64) * (hidden / kKC) > 0x7fffffffLL)
    return QMI_E_UNSUPPORTED;
  if (h_stride < hidden || w_stride < hidden) return QMI_E_BAD_STRIDE;
  if (h_stride % 8 || w_stride % 8 || !aligned16(h) || !aligned16(w) || !aligned16(ws))
    return QMI_E_BAD_STRIDE;
  if (ws_size < ws_bytes(n_rows, vocab, topk)) return QMI_E_WORKSPACE_TOO_SMALL;
  return QMI_OK;
}

int launch_tiles(const uint16_t* h, int64_t h_stride, int64_t n_rows, const uint16_t* w,
                 int64_t w_stride, int64_t vocab, int64_t hidden, float c2, bool topk,
                 const LmWs& ws, hipStream_t s) {
  const int nvt = (int)n_vtiles_of(vocab);
  // Up to 64 rows: items of 128 x 64, 4 waves, three LDS stages, two 74 KB
  // workgroups per CU.  Up to 256 rows: items of 256 x 128 (two row tiles at
  // 256 rows, so 1,188 items for Qwen3's vocabulary instead of 594 -- 4 or 5
  // per CU, not 2 or 3), 8 waves, three 48 KB stages, one workgroup per CU.
  // Above: items of 256 x 256, 8 waves, two 64 KB stages, one workgroup per
  // CU.  A persistent grid of that many workgroups per CU, or fewer when
  // there are fewer items.
#define QMI_LMI(MT, NW, NS, TVB, PER_CU, TOPK)                                                     \
  do {                                                                                            \
    /* the kernel's (max, sum) pairs cover one wave's entries: the layout's width */            \
    if ((kTV * TVB) / (NW / (MT / 64)) != pair_entries(n_rows)) return QMI_E_UNSUPPORTED;        \
    const int nrt = (int)((n_rows + MT - 1) / MT);                                                \
    const int64_t items = (int64_t)((nvt + TVB - 1) / TVB) * nrt;                                 \
    const int64_t grid = std::min<int64_t>(items, (int64_t)device_cu_count() * PER_CU);           \
    if (nrt > 1 && grid % 8 == 0 && grid >= 64)                                                   \
      hipLaunchKernelGGL((lmhead_items<MT, NW, NS, TVB, TOPK, true>), dim3((unsigned)grid),       \
                         dim3(NW * 64), 0, s, h, h_stride, (int)n_rows, w, w_stride, (int)vocab,  \
                         (int)hidden, c2, nvt, nrt, ws.part, ws.cand);                            \
    else                                                                                          \
      hipLaunchKernelGGL((lmhead_items<MT, NW, NS, TVB, TOPK, false>), dim3((unsigned)grid),      \
                         dim3(NW * 64), 0, s, h, h_stride, (int)n_rows, w, w_stride, (int)vocab,  \
                         (int)hidden, c2, nvt, nrt, ws.part, ws.cand);                            \
  } while (0)
  if (n_rows <= 64) {
    if (topk)
      QMI_LMI(64, 4, 3, 1, 2, true);
    else
      QMI_LMI(64, 4, 3, 1, 2, false);
  } else if (n_rows <= 256) {
    if (topk)
      QMI_LMI(128, 8, 3, 2, 1, true);
    else
      QMI_LMI(128, 8, 3, 2, 1, false);
  } else {
    if (topk)
      QMI_LMI(256, 8, 2, 2, 1, true);
    else
      QMI_LMI(256, 8, 2, 2, 1, false);
  }
#undef QMI_LMI
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? QMI_OK : (int)e;
}

}  // namespace

extern "C" int64_t qmi_lm_head_workspace_bytes(int64_t n_rows, int64_t vocab, int64_t top_k) {
  if (n_rows <= 0 || vocab <= 0) return 0;
  return ws_bytes(n_rows, vocab, top_k > 0 && top_k < vocab);
}

extern "C" int qmi_lm_head_sample(const uint16_t* hidden_states, int64_t h_stride, int64_t n_rows,
                                  const uint16_t* weight, int64_t w_stride, int64_t vocab,
                                  int64_t hidden, float temperature, int64_t top_k, uint64_t seed,
                                  uint64_t offset, const uint64_t* row_counters,
                                  int64_t* out_tokens, float* out_logprobs, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  if (top_k < 0 || top_k > kMaxFusedTopK) return QMI_E_UNSUPPORTED;
  if (n_rows == 0 && vocab > 0 && hidden > 0) return QMI_OK;
  const bool topk = top_k > 0 && top_k < vocab;  // k >= vocab keeps every entry
  if (topk && n_vtiles_of(vocab) > kMaxCandTiles) return QMI_E_UNSUPPORTED;
  int st = check_args(hidden_states, h_stride, n_rows, weight, w_stride, vocab, hidden, workspace,
                      workspace_bytes, topk);
  if (st != QMI_OK) return st;
  if (!out_tokens) return QMI_E_NULL_POINTER;
  if (!(temperature > 0.f) || temperature == INFINITY) return QMI_E_BAD_SHAPE;
  const float c2 = kLog2e / temperature;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const LmWs ws = ws_layout(workspace, n_rows, vocab);
  st = launch_tiles(hidden_states, h_stride, n_rows, weight, w_stride, vocab, hidden, c2, topk, ws,
                    s);
  if (st != QMI_OK) return st;
  if (topk)
    hipLaunchKernelGGL(lmhead_topk_rows, dim3((unsigned)n_rows), dim3(kRowThreads), 0, s, ws.cand,
                       (int)n_vtiles_of(vocab), hidden_states, h_stride, weight, w_stride,
                       (int)vocab, (int)hidden, (int)top_k, c2, (uint32_t)seed,
                       (uint32_t)(seed >> 32), (uint32_t)offset, (uint32_t)(offset >> 32),
                       row_counters, out_tokens, out_logprobs);
  else
    hipLaunchKernelGGL(lmhead_sample_rows, dim3((unsigned)n_rows), dim3(kRowThreads), 0, s,
                       ws.part, (int)n_pairs_of(n_rows, vocab), pair_entries(n_rows), hidden_states,
                       h_stride, weight, w_stride,
                       (int)vocab, (int)hidden, c2, (uint32_t)seed, (uint32_t)(seed >> 32),
                       (uint32_t)offset, (uint32_t)(offset >> 32), row_counters, out_tokens,
                       out_logprobs);
  QMI_RETURN_LAUNCH_STATUS();
}

extern "C" int qmi_lm_head_logprob(const uint16_t* hidden_states, int64_t h_stride, int64_t n_rows,
                                   const uint16_t* weight, int64_t w_stride, int64_t vocab,
                                   int64_t hidden, const int64_t* targets, int64_t target_stride,
                                   float* out_logprobs, float* out_lse, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
  if (n_rows == 0 && vocab > 0 && hidden > 0) return QMI_OK;
  int st = check_args(hidden_states, h_stride, n_rows, weight, w_stride, vocab, hidden, workspace,
                      workspace_bytes, false);
  if (st != QMI_OK) return st;
  if (!targets || !out_logprobs) return QMI_E_NULL_POINTER;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const LmWs ws = ws_layout(workspace, n_rows, vocab);
  st = launch_tiles(hidden_states, h_stride, n_rows, weight, w_stride, vocab, hidden, kLog2e, false,
                    ws, s);
  if (st != QMI_OK) return st;
  hipLaunchKernelGGL(lmhead_logprob_rows, dim3((unsigned)n_rows), dim3(kRowThreads),
                     (unsigned)(4 * hidden), s, ws.part,
                     (int)n_pairs_of(n_rows, vocab), hidden_states, h_stride, weight, w_stride,
                     targets, target_stride, (int)vocab, (int)hidden, kLog2e, out_logprobs, out_lse);
  QMI_RETURN_LAUNCH_STATUS();
}
