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
// Kernel 1, lmhead_tiles: a (128-row vocabulary tile, tile of MT hidden-state
// rows) work item computes its logits with v_mfma_f32_16x16x32_bf16 and
// reduces them on the spot to one (max, sum of exp2) pair per row in the log2
// domain (x * log2(e) / T); in target mode the tile that holds a row's target
// also writes that raw logit.  The grid is persistent (one or two workgroups
// per CU), each workgroup running a contiguous range of work items as one
// pipeline of (item, 64-hidden chunk) steps, so the loads never drain at item
// boundaries.  Operands are
// computed transposed, S^T = W H^T: A = 16 vocabulary rows x 32 hidden of W,
// B = H^T (32 hidden x 16 rows), so both operands are 16-byte row pieces and
// each lane's accumulators hold 4 consecutive vocabulary entries of one row.
//   * NW waves, MT/64 per vocabulary slice: wave (vq, rq) owns vocabulary rows
//     VW vq .. +VW of the tile (VW = 128 MT / (64 NW)) and hidden-state rows
//     64 rq .. +64 (VW/16 x 4 MFMA tiles).
//   * W and H are staged through registers into LDS in chunks of 64 hidden
//     (128-byte rows), two register sets and two or three LDS stages, one
//     barrier per chunk: the global loads of chunk k+2 are issued before
//     chunk k is multiplied and written to LDS at the end of step k+1.  16-byte
//     piece c of row r sits at c ^ ((r / 2) % 8): the 16 rows a 16-lane group
//     reads then cover all 64 LDS banks.
//   * W (311 MB for Qwen3-0.6B) is read once from HBM per row tile; H comes
//     from L2.  At 256 rows the vocabulary GEMM is near the HBM / MFMA ridge.
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

// Register sets of the load stream (steps of loads in flight).
#ifndef QMI_LM_NSET_SMALL
#define QMI_LM_NSET_SMALL 2
#endif
#ifndef QMI_LM_NSET_LARGE
#define QMI_LM_NSET_LARGE 2
#endif

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
  return __builtin_bit_cast(bf16x8_t, u32x4_t{v.x, v.y, v.z, v.w});
}

// Byte offset of 16-byte piece c of staged row r.
__device__ __forceinline__ int lds_off(int r, int c) { return r * kRowB + ((c ^ ((r >> 1) & 7)) << 4); }

template <int MT, int NW, int NSTAGE, int NSET>
__global__ __launch_bounds__(NW * 64) void lmhead_tiles(
    const uint16_t* __restrict__ h, int64_t h_stride, int n_rows,
    const uint16_t* __restrict__ w, int64_t w_stride, int vocab, int hidden, float c2,
    const int64_t* __restrict__ tgt, int64_t tgt_stride, int n_vtiles, int n_rtiles,
    float2* __restrict__ part, float* __restrict__ tgt_logit) {
  constexpr int NT = NW * 64;
  constexpr int NRQ = MT / 64;       // row blocks of 64
  constexpr int NVQ = NW / NRQ;      // waves per row block, splitting the tile's vocabulary
  constexpr int VW = kTV / NVQ;      // vocabulary rows per wave
  constexpr int VB = VW / 16;        // 16-row MFMA blocks per wave along the vocabulary
  constexpr int W_BYTES = kTV * kRowB;
  constexpr int STAGE = W_BYTES + MT * kRowB;
  constexpr int WCH = kTV * 8 / NT;  // W pieces per thread per chunk
  constexpr int HCH = MT * 8 / NT;   // H pieces per thread per chunk
  static_assert(NVQ * NRQ == NW && VB >= 1 && WCH >= 1 && HCH >= 1, "tile shape");
  __shared__ __align__(16) unsigned char lds[NSTAGE * STAGE];
  __shared__ float2 red[NVQ][MT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g4 = lane >> 4;
  const int vq = wave % NVQ, rq = wave / NVQ;
  const int n_kc = hidden / kKC;
  // Persistent: this workgroup takes tiles [t_begin, t_end) of the
  // vocabulary-major order (tile i = vocabulary tile i / n_rtiles, row tile
  // i % n_rtiles, so the row tiles of one W tile run back to back and reuse
  // it from L2), as one pipelined sequence of (tile, chunk) steps.
  const int n_tiles = n_vtiles * n_rtiles;
  const int t_begin = (int)((int64_t)blockIdx.x * n_tiles / gridDim.x);
  const int t_end = (int)((int64_t)(blockIdx.x + 1) * n_tiles / gridDim.x);
  const int n_steps = (t_end - t_begin) * n_kc;
  if (n_steps == 0) return;

  // Staging: piece q = tid + i * NT of a chunk is row q / 8, piece q % 8.
  // Loads are unconditional straight-line code (the compiler then keeps two
  // steps of them in flight): rows past the vocabulary or the batch read the
  // tile's last valid row, and are zeroed when the pieces are written to LDS.
  // The load stream runs two steps ahead of the compute stream and repeats
  // its last chunk past the end.
  int wdst[WCH], hdst[HCH];
#pragma unroll
  for (int i = 0; i < WCH; ++i) {
    const int q = tid + i * NT;
    wdst[i] = lds_off(q >> 3, q & 7);
  }
#pragma unroll
  for (int i = 0; i < HCH; ++i) {
    const int q = tid + i * NT;
    hdst[i] = W_BYTES + lds_off(q >> 3, q & 7);
  }
  uint4 wreg[NSET][WCH], hreg[NSET][HCH];
  // Tile positions (vocabulary tile, row tile) advance incrementally: no
  // division per step (a runtime division is a long scalar sequence, and at
  // one instruction stream per wave it delays the MFMAs behind it).
  struct Pos {
    int vt, rt;
  };
  auto advance = [&](Pos p) -> Pos { return p.rt + 1 == n_rtiles ? Pos{p.vt + 1, 0} : Pos{p.vt, p.rt + 1}; };
  const Pos p_begin{t_begin / n_rtiles, t_begin % n_rtiles};
  // Load stream: the next step it fetches, and the current tile's bases and
  // per-lane element offsets (rows past the vocabulary or the batch clamped to
  // the tile's last valid row), set up once per tile.
  Pos ld = p_begin;
  int ld_kc = 0, ld_step = 0;
  const uint16_t* wt0;
  const uint16_t* ht0;
  int woff[WCH], hoff[HCH];
  auto ld_tile_setup = [&]() __attribute__((always_inline)) {
    const int v0 = ld.vt * kTV, r0 = ld.rt * MT;
    const int wlast = min(kTV, vocab - v0) - 1;      // last valid row of the tile
    const int hlast = min(MT, n_rows - r0) - 1;
    wt0 = w + (int64_t)v0 * w_stride;
    ht0 = h + (int64_t)r0 * h_stride;
#pragma unroll
    for (int i = 0; i < WCH; ++i) {
      const int q = tid + i * NT;
      woff[i] = min(q >> 3, wlast) * (int)w_stride + (q & 7) * 8;
    }
#pragma unroll
    for (int i = 0; i < HCH; ++i) {
      const int q = tid + i * NT;
      hoff[i] = min(q >> 3, hlast) * (int)h_stride + (q & 7) * 8;
    }
  };
  ld_tile_setup();
  auto load_next = [&](auto set_c) __attribute__((always_inline)) {
    constexpr int P = decltype(set_c)::value;
    const uint16_t* wt = wt0 + ld_kc * kKC;
    const uint16_t* ht = ht0 + ld_kc * kKC;
#pragma unroll
    for (int i = 0; i < WCH; ++i) wreg[P][i] = load_u4_stream(wt + woff[i]);
#pragma unroll
    for (int i = 0; i < HCH; ++i) hreg[P][i] = load_u4(ht + hoff[i]);
    if (ld_step + 1 < n_steps) {
      ++ld_step;
      if (++ld_kc == n_kc) {
        ld_kc = 0;
        ld = advance(ld);
        ld_tile_setup();
      }
    }
  };
  auto store_step = [&](int stage, Pos tile, auto set_c) __attribute__((always_inline)) {
    constexpr int P = decltype(set_c)::value;
    unsigned char* base = lds + stage * STAGE;
    const int wn = min(kTV, vocab - tile.vt * kTV);
    const int hn = min(MT, n_rows - tile.rt * MT);
#pragma unroll
    for (int i = 0; i < WCH; ++i) {
      const int q = tid + i * NT;
      const uint32_t keep = (q >> 3) < wn ? 0xffffffffu : 0u;
      const uint4 v = wreg[P][i];
      *reinterpret_cast<uint4*>(base + wdst[i]) = make_uint4(v.x & keep, v.y & keep, v.z & keep, v.w & keep);
    }
#pragma unroll
    for (int i = 0; i < HCH; ++i) {
      const int q = tid + i * NT;
      const uint32_t keep = (q >> 3) < hn ? 0xffffffffu : 0u;
      const uint4 v = hreg[P][i];
      *reinterpret_cast<uint4*>(base + hdst[i]) = make_uint4(v.x & keep, v.y & keep, v.z & keep, v.w & keep);
    }
  };

  // Operand read offsets: row VW vq + 16 vb + l16 of W, row 64 rq + 16 rb + l16
  // of H, piece 4 ks + g4 (hidden 32 ks + 8 g4 .. +8 of the chunk).  (r / 2) % 8
  // of those rows is l16 / 2, so the swizzled piece does not depend on vb / rb.
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

  // Epilogue of a tile: per row, (max, sum of exp2) over the tile's 128
  // entries; acc[vb][rb][e] holds vocabulary v0 + VW vq + 16 vb + 4 g4 + e of
  // row r0 + 64 rq + 16 rb + l16.
  // Target mode: the target ids of this lane's four rows, loaded when a tile
  // starts (straight-line loads, consumed by the tile's epilogue).
  int64_t tgt_id[4] = {-1, -1, -1, -1};
  auto load_targets = [&](Pos tile) __attribute__((always_inline)) {
    const int r0 = tile.rt * MT;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const int row = r0 + 64 * rq + 16 * rb + l16;
      tgt_id[rb] = tgt[(int64_t)(row < n_rows ? row : n_rows - 1) * tgt_stride];
    }
  };

  auto epilogue = [&](Pos tile) __attribute__((always_inline)) {
    const int vt = tile.vt;
    const int64_t v0 = (int64_t)vt * kTV;
    const int64_t r0 = (int64_t)tile.rt * MT;
    const int64_t vbase = v0 + VW * vq + 4 * g4;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      float x[4 * VB];
      float mx = kNegBig;
#pragma unroll
      for (int vb = 0; vb < VB; ++vb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool ok = vbase + 16 * vb + e < vocab;
          x[4 * vb + e] = ok ? acc[vb][rb][e] * c2 : kNegBig;
          mx = fmaxf(mx, x[4 * vb + e]);
        }
      float sm = 0.f;
#pragma unroll
      for (int i = 0; i < 4 * VB; ++i) sm += fast_exp2(x[i] - mx);
      LanePair pm = lane_pair16(mx), ps = lane_pair16(sm);
      mx = pm.lo;
      sm = ps.lo;
      lse2_merge(mx, sm, pm.hi, ps.hi);
      pm = lane_pair32(mx);
      ps = lane_pair32(sm);
      mx = pm.lo;
      sm = ps.lo;
      lse2_merge(mx, sm, pm.hi, ps.hi);
      const int row_l = 64 * rq + 16 * rb + l16;
      if (g4 == 0) red[vq][row_l] = make_float2(mx, sm);
      if (tgt) {
        const int64_t row = r0 + row_l;
        if (row < n_rows) {
          const int64_t tl = tgt_id[rb] - vbase;  // 16 vb + e if this lane holds it
          if (tl >= 0 && tl < VW && (tl & 12) == 0) {
#pragma unroll
            for (int vb = 0; vb < VB; ++vb)
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (tl == 16 * vb + e) tgt_logit[row] = acc[vb][rb][e];
          }
        }
      }
#pragma unroll
      for (int vb = 0; vb < VB; ++vb) acc[vb][rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();
    for (int r = tid; r < MT; r += NT) {
      if (r0 + r < n_rows) {
        float2 a = red[0][r];
#pragma unroll
        for (int j = 1; j < NVQ; ++j) lse2_merge(a.x, a.y, red[j][r].x, red[j][r].y);
        part[(r0 + r) * (int64_t)n_vtiles + vt] = a;
      }
    }
  };

  // Step st (chunk kc of tile `tile`): the loads of step st + NSET go into
  // register set st % NSET (already in LDS), the MFMAs read stage
  // st % NSTAGE, then set (st + 1) % NSET -- step st + 1, loaded NSET - 1
  // steps earlier -- is written to stage (st + 1) % NSTAGE, which no wave has
  // read since the barrier that ended step st - 1.  NSET - 1 steps of compute
  // cover each load's latency.
  Pos tile = p_begin;
  int kc = 0, stage = 0;
  auto step = [&](int st, auto set_c) __attribute__((always_inline)) {
    constexpr int P = decltype(set_c)::value;
    constexpr int PN = P + 1 == NSET ? 0 : P + 1;
    if (tgt && kc == 0) load_targets(tile);
    load_next(std::integral_constant<int, P>{});
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
    const int next_stage = stage == NSTAGE - 1 ? 0 : stage + 1;
    const Pos next_tile = kc + 1 == n_kc ? advance(tile) : tile;
    if (st + 1 < n_steps) store_step(next_stage, next_tile, std::integral_constant<int, PN>{});
    __syncthreads();
    if (kc + 1 == n_kc) epilogue(tile);
    stage = next_stage;
    tile = next_tile;
    kc = kc + 1 == n_kc ? 0 : kc + 1;
  };

  static_for<0, NSET>([&](auto i_c) __attribute__((always_inline)) { load_next(i_c); });
  store_step(0, p_begin, std::integral_constant<int, 0>{});
  __syncthreads();
  for (int st = 0; st < n_steps; st += NSET) {
    static_for<0, NSET>([&](auto i_c) __attribute__((always_inline)) {
      if (st + (int)decltype(i_c)::value < n_steps) step(st + decltype(i_c)::value, i_c);
    });
  }
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
  // Up to 64 rows: 64-row tiles, 4 waves of 32 vocabulary rows, three LDS
  // stages, two 74 KB workgroups per CU.  Above: 256-row tiles, 8 waves of
  // 64 x 64, two LDS stages, one 100 KB workgroup per CU (measured faster
  // than three stages, and than 4 waves of 128 x 64 or two 128-row
  // workgroups per CU).  A persistent grid of that many workgroups per CU, or
  // fewer when there are fewer tiles.
#define QMI_LMT(MT, NW, NS, NSET, PER_CU)                                                             \
  do {                                                                                            \
    const int nrt = (int)((n_rows + MT - 1) / MT);                                                \
    const int64_t tiles = (int64_t)nvt * nrt;                                                     \
    const int64_t grid = std::min<int64_t>(tiles, (int64_t)device_cu_count() * PER_CU);           \
    hipLaunchKernelGGL((lmhead_tiles<MT, NW, NS, NSET>), dim3((unsigned)grid), dim3(NW * 64), 0, s, \
                       h,                                                                         \
                       h_stride, (int)n_rows, w, w_stride, (int)vocab, (int)hidden, c2, tgt,      \
                       tgt_stride, nvt, nrt, ws.part, ws.tgt_logit);                              \
  } while (0)
  if (n_rows <= 64)
    QMI_LMT(64, 4, 3, QMI_LM_NSET_SMALL, 2);
  else
    QMI_LMT(256, 8, 2, QMI_LM_NSET_LARGE, 1);
#undef QMI_LMT
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
