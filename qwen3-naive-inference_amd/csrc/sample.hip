// Token sampling from bf16 logits in one streaming pass: temperature,
// softmax, the categorical draw and the drawn token's log-probability.
//
// Reference semantics (qwen3_naive.py, generate_continuous :1413-1423 and
// generate_continuous_with_logprobs :1636-1650, top_k = None):
//   x = logits.float() / T;  tok ~ Categorical(softmax(x));  lp = log_softmax(x)[tok]
//
// Method: Gumbel-max.  tok = argmax_i (x_i + G_i) with G_i iid Gumbel(0, 1)
// has exactly the softmax(x) distribution.  G_i = -ln(-ln U_i), where U_i is
// the (i % 4)-th word of Philox4x32-10 (Salmon, Moraes, Dror and Shaw,
// "Parallel random numbers: as easy as 1, 2, 3", SC 2011) at counter
// (i / 4, row, offset_lo, offset_hi) and key (seed_lo, seed_hi), mapped to
// ((w >> 8) + 0.5) / 2^24, strictly inside (0, 1).  Scores are kept in log2
// units, s_i = x_i log2(e) - log2(-log2 U_i), a positive scaling plus a
// constant shift of x_i + G_i, so the argmax is the same; E = -ln U is
// taken from 1 - U near U = 1 so the large Gumbel values keep full
// precision.  Ties go to the lowest index.  The same pass keeps the row's
// online log-sum-exp, so
// lp = (x_tok log2(e) - lse2) ln 2 needs one extra load of logits[tok].
//
// gfx950 design: one 1024-lane workgroup per row (16 waves per CU at a batch
// of 256 hide the Philox multiply chains better than 4: 56.8 -> 51.3 us for
// 256 x 151,936 logits), 16-byte non-temporal loads (8 logits), two Philox
// blocks per load; per-lane (max, sum of exp2) and (best score, index) merged
// with shuffles and one LDS exchange.
#include "qmi_common.h"

namespace {

using namespace qmi;

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

// Gumbel term in log2 units: -log2(E log2 e) with E = -ln U,
// U = ((w >> 8) + 0.5) / 2^24.  Near U = 1 (where the largest Gumbel values
// come from) E is computed from t = 1 - U, which is exact in fp32, by the
// series -ln(1 - t) = t + t^2/2 + t^3/3 (t < 2^-10: truncation < t^4/4).
__device__ __forceinline__ float gumbel2(uint32_t w) {
  const uint32_t k = w >> 8;
  const float u = ((float)k + 0.5f) * (1.0f / 16777216.0f);
  const float t = ((float)(16777216u - k) - 0.5f) * (1.0f / 16777216.0f);
  const float e_series = t * fmaf(t, fmaf(t, 1.0f / 3.0f, 0.5f), 1.0f) * kLog2e;
  const float e_log = -__builtin_amdgcn_logf(u);  // -log2 U = E log2 e
  return -__builtin_amdgcn_logf(t < (1.0f / 1024.0f) ? e_series : e_log);
}

struct RowState {
  float m2, s;     // running max and sum of exp2(xs - m2)
  float best;      // best Gumbel score
  int32_t best_i;  // its vocabulary index
};

__device__ __forceinline__ void take(RowState& st, float score, int32_t i) {
  if (score > st.best) {  // elements arrive in increasing index per lane
    st.best = score;
    st.best_i = i;
  }
}

__device__ __forceinline__ void merge(RowState& a, const RowState& b) {
  const float mn = fmaxf(a.m2, b.m2);
  a.s = a.s * fast_exp2(a.m2 - mn) + b.s * fast_exp2(b.m2 - mn);
  a.m2 = mn;
  if (b.best > a.best || (b.best == a.best && b.best_i < a.best_i)) {
    a.best = b.best;
    a.best_i = b.best_i;
  }
}

__device__ __forceinline__ RowState shfl_state(const RowState& st, int mask) {
  RowState o;
  o.m2 = __shfl_xor(st.m2, mask, 64);
  o.s = __shfl_xor(st.s, mask, 64);
  o.best = __shfl_xor(st.best, mask, 64);
  o.best_i = __shfl_xor(st.best_i, mask, 64);
  return o;
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void sample_rows(
    const uint16_t* __restrict__ logits, int64_t row_stride, int64_t vocab, float c2,
    uint32_t seed_lo, uint32_t seed_hi, uint32_t off_lo, uint32_t off_hi,
    int64_t* __restrict__ out_tok, float* __restrict__ out_lp) {
  __shared__ RowState sm[kWaves];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* rp = logits + row * row_stride;
  const uint32_t crow = (uint32_t)row;
  RowState st{kNegBig, 0.f, -INFINITY, 0};

  int64_t tail_begin = 0;
  if (VEC) {
    const int64_t nvec = vocab >> 3;
    tail_begin = nvec << 3;
    for (int64_t i = tid; i < nvec; i += kThreads) {
      const uint4 c = load_u4_stream(rp + (i << 3));
      float xs[8];
      xs[0] = bf16_lo(c.x) * c2; xs[1] = bf16_hi(c.x) * c2;
      xs[2] = bf16_lo(c.y) * c2; xs[3] = bf16_hi(c.y) * c2;
      xs[4] = bf16_lo(c.z) * c2; xs[5] = bf16_hi(c.z) * c2;
      xs[6] = bf16_lo(c.w) * c2; xs[7] = bf16_hi(c.w) * c2;
      const uint4 r0 = philox4x32_10(make_uint4((uint32_t)(2 * i), crow, off_lo, off_hi), seed_lo, seed_hi);
      const uint4 r1 = philox4x32_10(make_uint4((uint32_t)(2 * i + 1), crow, off_lo, off_hi), seed_lo, seed_hi);
      const uint32_t w[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
      float cm = xs[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) cm = fmaxf(cm, xs[e]);
      const float mn = fmaxf(st.m2, cm);
      float add = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) add += fast_exp2(xs[e] - mn);
      st.s = st.s * fast_exp2(st.m2 - mn) + add;
      st.m2 = mn;
      const int32_t e0 = (int32_t)(i << 3);
#pragma unroll
      for (int e = 0; e < 8; ++e) take(st, xs[e] + gumbel2(w[e]), e0 + e);
    }
  }
  // Scalar elements: the whole row when rows are not 16-byte aligned, else the tail.
  for (int64_t e = tail_begin + tid; e < vocab; e += kThreads) {
    const float xs = bf16_to_f32(rp[e]) * c2;
    const uint4 r = philox4x32_10(make_uint4((uint32_t)(e >> 2), crow, off_lo, off_hi), seed_lo, seed_hi);
    const int k = (int)(e & 3);
    const uint32_t w = k == 0 ? r.x : k == 1 ? r.y : k == 2 ? r.z : r.w;
    const float mn = fmaxf(st.m2, xs);
    st.s = st.s * fast_exp2(st.m2 - mn) + fast_exp2(xs - mn);
    st.m2 = mn;
    take(st, xs + gumbel2(w), (int32_t)e);
  }

  // Workgroup reduction: within each wave by shuffles, then across waves.
#pragma unroll
  for (int mask = 32; mask >= 1; mask >>= 1) merge(st, shfl_state(st, mask));
  if ((tid & 63) == 0) sm[tid >> 6] = st;
  __syncthreads();
  if (tid == 0) {
    RowState a = sm[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) merge(a, sm[w]);
    const int32_t tok = a.best_i;
    out_tok[row] = tok;
    if (out_lp) {
      const float lse2 = a.m2 + __builtin_amdgcn_logf(a.s);
      out_lp[row] = (bf16_to_f32(rp[tok]) * c2 - lse2) * kLn2;
    }
  }
}

}  // namespace

extern "C" int qmi_sample_tokens(const uint16_t* logits, int64_t row_stride, int64_t n_rows,
                                 int64_t vocab, float temperature, uint64_t seed,
                                 uint64_t offset, int64_t* out_tokens, float* out_logprobs,
                                 void* stream) {
  if (n_rows < 0 || vocab < 0) return QMI_E_BAD_SHAPE;
  if (n_rows == 0) return QMI_OK;
  if (!logits || !out_tokens) return QMI_E_NULL_POINTER;
  if (vocab == 0 || vocab > 0x7fffffff) return QMI_E_BAD_SHAPE;
  if (row_stride < vocab) return QMI_E_BAD_STRIDE;
  if (n_rows > 0x7fffffff) return QMI_E_UNSUPPORTED;
  if (!(temperature > 0.f) || temperature == INFINITY) return QMI_E_BAD_SHAPE;
  const float c2 = kLog2e / temperature;
  const uint32_t s_lo = (uint32_t)seed, s_hi = (uint32_t)(seed >> 32);
  const uint32_t o_lo = (uint32_t)offset, o_hi = (uint32_t)(offset >> 32);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool vec = (row_stride % 8 == 0) && ((reinterpret_cast<uintptr_t>(logits) & 15u) == 0);
  if (vec)
    hipLaunchKernelGGL(sample_rows<true>, dim3((unsigned)n_rows), dim3(kThreads), 0, s, logits,
                       row_stride, vocab, c2, s_lo, s_hi, o_lo, o_hi, out_tokens, out_logprobs);
  else
    hipLaunchKernelGGL(sample_rows<false>, dim3((unsigned)n_rows), dim3(kThreads), 0, s, logits,
                       row_stride, vocab, c2, s_lo, s_hi, o_lo, o_hi, out_tokens, out_logprobs);
  QMI_RETURN_LAUNCH_STATUS();
}

// ---------------------------------------------------------------------------
// Top-k sampling from bf16 logits: the reference's default generate path
// (top_k = 20, qwen3_naive.py:1413-1422 and :1641-1650):
//   x = logits.float() / T;  keep the k largest (the rest -inf);
//   tok ~ Categorical(softmax(x));  lp = log_softmax(x)[tok]
// One 256-lane workgroup per row:
//   1-2. The k-th largest logit by a two-pass radix select on the bf16 bits
//        (16-byte loads when the rows are 16-byte aligned)
//        mapped to order-preserving 16-bit keys (high byte, then low byte;
//        LDS histograms).  x / T keeps the order (T > 0), so the set is found
//        on the raw logits.
//   3.   The k kept entries gathered into LDS in vocabulary order: every
//        entry above the threshold key, and of the entries equal to it the
//        lowest-index ones up to k (each lane scans a contiguous slice;
//        slice counts are prefix-summed, so the order is fixed).
//   4.   Inverse transform sampling over the kept entries in vocabulary
//        order with one Philox4x32-10 uniform per row (53 bits of words 0 and
//        1 at counter (0, row, offset)), and the drawn token's log-prob.
namespace {

constexpr int kTopThreads = 256;
constexpr int kMaxTopK = 1024;

__device__ __forceinline__ uint32_t bf16_key(uint32_t b) {
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}

__device__ int block_excl_scan_int(int x, int* sm, int* total) {
  // sm: 4 ints.  Fixed-order inclusive scan within each wave, then the wave bases.
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

__device__ double block_excl_scan_f64(double x, double* sm, double* total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  double inc = x;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const double y = __shfl_up(inc, d, 64);
    if (lane >= d) inc += y;
  }
  __syncthreads();
  if (lane == 63) sm[wv] = inc;
  __syncthreads();
  double base = 0.0;
  for (int j = 0; j < wv; ++j) base += sm[j];
  *total = sm[0] + sm[1] + sm[2] + sm[3];
  return base + inc - x;
}

// Calls f(bits) for every 16-bit entry of the row, lane-strided (16-byte
// loads when the row is aligned for them).
template <bool VEC, class F>
__device__ __forceinline__ void for_each_bits(const uint16_t* __restrict__ rp, int vocab, F&& f) {
  const int tid = threadIdx.x;
  int tail = 0;
  if (VEC) {
    const int nvec = vocab >> 3;
    tail = nvec << 3;
    for (int i = tid; i < nvec; i += kTopThreads) {
      const uint4 c = load_u4(rp + (i << 3));
      const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f(w[e] & 0xffffu);
        f(w[e] >> 16);
      }
    }
  }
  for (int i = tail + tid; i < vocab; i += kTopThreads) f((uint32_t)rp[i]);
}

template <bool VEC>
__global__ __launch_bounds__(kTopThreads) void sample_topk_rows(
    const uint16_t* __restrict__ logits, int64_t row_stride, int vocab, int k, float c2,
    uint32_t seed_lo, uint32_t seed_hi, uint32_t off_lo, uint32_t off_hi,
    int64_t* __restrict__ out_tok, float* __restrict__ out_lp) {
  __shared__ uint32_t hist[256];
  __shared__ int sel[4];        // high byte, threshold key, entries above it, equal ones kept
  __shared__ int smi[4];
  __shared__ double smd[4];
  __shared__ float smf[4];
  __shared__ int cand_idx[kMaxTopK];
  __shared__ float cand_x[kMaxTopK];
  __shared__ int pick_sm;
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const uint16_t* rp = logits + row * row_stride;

  // ---- pass 1: histogram of the high key byte ----
  hist[tid] = 0;
  __syncthreads();
  for_each_bits<VEC>(rp, vocab, [&](uint32_t b) { atomicAdd(&hist[bf16_key(b) >> 8], 1u); });
  __syncthreads();
  if (tid == 0) {
    int cum = 0, b = 255;
    for (; b > 0; --b) {
      if (cum + (int)hist[b] >= k) break;
      cum += (int)hist[b];
    }
    sel[0] = b;
    sel[2] = cum;  // entries whose high byte is above b
  }
  __syncthreads();
  const uint32_t hb = (uint32_t)sel[0];
  // ---- pass 2: histogram of the low byte within that high byte ----
  hist[tid] = 0;
  __syncthreads();
  for_each_bits<VEC>(rp, vocab, [&](uint32_t b) {
    const uint32_t key = bf16_key(b);
    if ((key >> 8) == hb) atomicAdd(&hist[key & 0xffu], 1u);
  });
  __syncthreads();
  if (tid == 0) {
    int cum = sel[2], b = 255;
    for (; b > 0; --b) {
      if (cum + (int)hist[b] >= k) break;
      cum += (int)hist[b];
    }
    sel[1] = (int)((hb << 8) | (uint32_t)b);
    sel[2] = cum;        // entries above the threshold key (< k)
    sel[3] = k - cum;    // entries equal to it that are kept (>= 1)
  }
  __syncthreads();
  const uint32_t tkey = (uint32_t)sel[1];
  const int need_eq = sel[3];

  // ---- pass 3: gather the kept entries in vocabulary order ----
  // Lane t scans the contiguous slice [t * cpt, t * cpt + cpt), cpt a
  // multiple of 8 so that aligned rows are read 16 bytes at a time.
  const int cpt = ((vocab + kTopThreads - 1) / kTopThreads + 7) & ~7;
  const int lo = min(vocab, tid * cpt), hi = min(vocab, lo + cpt);
  int gt = 0, eq = 0;
  if (VEC) {
    const int hi8 = lo + ((hi - lo) & ~7);
    for (int i = lo; i < hi8; i += 8) {
      const uint4 c = load_u4(rp + i);
      const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t k0 = bf16_key(w[e] & 0xffffu), k1 = bf16_key(w[e] >> 16);
        gt += (k0 > tkey) + (k1 > tkey);
        eq += (k0 == tkey) + (k1 == tkey);
      }
    }
    for (int i = hi8; i < hi; ++i) {
      const uint32_t key = bf16_key(rp[i]);
      gt += key > tkey;
      eq += key == tkey;
    }
  } else {
    for (int i = lo; i < hi; ++i) {
      const uint32_t key = bf16_key(rp[i]);
      gt += key > tkey;
      eq += key == tkey;
    }
  }
  int tot;
  const int eq_before = block_excl_scan_int(eq, smi, &tot);
  const int take = max(0, min(eq, need_eq - eq_before));
  int pos = block_excl_scan_int(gt + take, smi, &tot);
  int taken = 0;
  for (int i = lo; i < hi && (gt > 0 || taken < take); ++i) {
    const uint16_t b = rp[i];
    const uint32_t key = bf16_key(b);
    const bool keep = key > tkey || (key == tkey && taken < take);
    if (key > tkey) --gt;
    if (key == tkey && taken < take) ++taken;
    if (keep) {
      cand_idx[pos] = i;
      cand_x[pos] = bf16_to_f32(b);
      ++pos;
    }
  }
  __syncthreads();

  // ---- pass 4: inverse transform sampling over the k kept entries ----
  float mx = kNegBig;
  for (int j = tid; j < k; j += kTopThreads) mx = fmaxf(mx, cand_x[j] * c2);
  mx = wave_max(mx);
  __syncthreads();
  if ((tid & 63) == 0) smf[tid >> 6] = mx;
  __syncthreads();
  const float m2 = fmaxf(fmaxf(smf[0], smf[1]), fmaxf(smf[2], smf[3]));
  // Lane t takes the contiguous entries [t * per, t * per + per).
  const int per = (k + kTopThreads - 1) / kTopThreads;
  const int jlo = min(k, tid * per), jhi = min(k, jlo + per);
  double own = 0.0;
  for (int j = jlo; j < jhi; ++j) own += (double)fast_exp2(cand_x[j] * c2 - m2);
  double s_tot;
  const double excl = block_excl_scan_f64(own, smd, &s_tot);
  const uint4 r = philox4x32_10(make_uint4(0u, (uint32_t)row, off_lo, off_hi), seed_lo, seed_hi);
  const uint64_t bits = ((uint64_t)r.x << 21) | (uint64_t)(r.y >> 11);
  const double target = (((double)bits + 0.5) * 0x1p-53) * s_tot;
  if (tid == 0) pick_sm = k - 1;  // u * S rounded up to S: the last entry
  __syncthreads();
  if (jhi > jlo && target >= excl && target < excl + own) {
    double cum = excl;
    int j = jlo;
    for (; j < jhi - 1; ++j) {
      const double p = (double)fast_exp2(cand_x[j] * c2 - m2);
      if (target < cum + p) break;
      cum += p;
    }
    pick_sm = j;
  }
  __syncthreads();
  if (tid == 0) {
    const int j = pick_sm;
    out_tok[row] = cand_idx[j];
    if (out_lp) {
      const double lse2 = (double)m2 + log2(s_tot);
      out_lp[row] = (float)(((double)cand_x[j] * (double)c2 - lse2) * (double)kLn2);
    }
  }
}

}  // namespace

extern "C" int qmi_sample_tokens_topk(const uint16_t* logits, int64_t row_stride, int64_t n_rows,
                                      int64_t vocab, int64_t top_k, float temperature,
                                      uint64_t seed, uint64_t offset, int64_t* out_tokens,
                                      float* out_logprobs, void* stream) {
  if (n_rows < 0 || vocab < 0) return QMI_E_BAD_SHAPE;
  if (n_rows == 0) return QMI_OK;
  if (!logits || !out_tokens) return QMI_E_NULL_POINTER;
  if (vocab == 0 || vocab > 0x7fffffff) return QMI_E_BAD_SHAPE;
  if (top_k < 1 || top_k > vocab) return QMI_E_BAD_SHAPE;
  if (top_k > kMaxTopK) return QMI_E_UNSUPPORTED;
  if (row_stride < vocab) return QMI_E_BAD_STRIDE;
  if (n_rows > 0x7fffffff) return QMI_E_UNSUPPORTED;
  if (!(temperature > 0.f) || temperature == INFINITY) return QMI_E_BAD_SHAPE;
  const float c2 = kLog2e / temperature;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool vec = (row_stride % 8 == 0) && ((reinterpret_cast<uintptr_t>(logits) & 15u) == 0);
  if (vec)
    hipLaunchKernelGGL(sample_topk_rows<true>, dim3((unsigned)n_rows), dim3(kTopThreads), 0, s,
                       logits, row_stride, (int)vocab, (int)top_k, c2, (uint32_t)seed,
                       (uint32_t)(seed >> 32), (uint32_t)offset, (uint32_t)(offset >> 32),
                       out_tokens, out_logprobs);
  else
    hipLaunchKernelGGL(sample_topk_rows<false>, dim3((unsigned)n_rows), dim3(kTopThreads), 0, s,
                       logits, row_stride, (int)vocab, (int)top_k, c2, (uint32_t)seed,
                       (uint32_t)(seed >> 32), (uint32_t)offset, (uint32_t)(offset >> 32),
                       out_tokens, out_logprobs);
  QMI_RETURN_LAUNCH_STATUS();
}
