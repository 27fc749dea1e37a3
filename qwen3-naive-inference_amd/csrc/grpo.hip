// GRPO loss-step kernels: streaming log-softmax gather, group advantages,
// PPO clipped masked loss, and the backward through the bf16 logits.
//
// Reference semantics (qwen3_grpo_train.py):
//   forward_logprob         :46-53   lp[b,t] = log_softmax(float(logits[b,t]))[ids[b,t]]
//   compute_grpo_advantage  :162-173 A = (r - mean_g) / (std_g + eps), unbiased std
//   token advantages        :269     A_tok = A[:, None] * mask
//   ppo_clipped_loss        :184-199 r = exp(new-old); l = -min(rA, clamp(r,1-e,1+e)A);
//                                    L = sum(l*m) / (sum(m) + 1e-8)
//
// gfx950 design.  The logits read (n_rows x vocab bf16, 4.98 GB at the
// 32x512x151936 loss step) is the whole cost, so one workgroup streams one
// row with dwordx4 non-temporal loads, four chunks in flight per lane, and
// keeps a per-lane (max, sum of exp2) pair rescaled once per 32 elements.
// The pairs are merged with shuffles and one LDS exchange.  Row workgroups
// use no fences or atomics: an agent-scope fence on gfx950 writes back and
// invalidates the L2, which costs more than the row itself when 16K
// workgroups each issue one.  The loss therefore runs as two more tiny
// launches: one workgroup per sequence computes the advantage, token losses,
// their gradients and the sequence's sums (each reads its own mask row
// once), then one workgroup per sequence applies the token-mean
// denominator (the sum of the per-sequence mask sums) to its gradients while
// workgroup 0 writes the scalar.  All sums run in a fixed order, so results
// are deterministic, and the workspace holds no state between calls.
#include "qmi_common.h"

namespace {

using namespace qmi;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kUnroll = 4;

// ---------------------------------------------------------------------------
// Block-wide log-sum-exp of one row.  Returns lse2 = log2(sum(exp(x)))
// (i.e. the natural lse times log2(e)) in every lane.
template <bool VEC>
__device__ __forceinline__ float row_lse2(const uint16_t* __restrict__ row, int64_t vocab,
                                          float* sm_m, float* sm_s) {
  const int tid = threadIdx.x;
  float m2 = kNegBig, s = 0.f;
  if (VEC) {
    const int64_t nvec = vocab >> 3;
    int64_t i = tid;
    for (; i + (kUnroll - 1) * kThreads < nvec; i += kUnroll * kThreads) {
      uint4 c[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) c[u] = load_u4_stream(row + ((i + u * kThreads) << 3));
      float x[kUnroll * 8];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        x[u * 8 + 0] = bf16_lo(c[u].x); x[u * 8 + 1] = bf16_hi(c[u].x);
        x[u * 8 + 2] = bf16_lo(c[u].y); x[u * 8 + 3] = bf16_hi(c[u].y);
        x[u * 8 + 4] = bf16_lo(c[u].z); x[u * 8 + 5] = bf16_hi(c[u].z);
        x[u * 8 + 6] = bf16_lo(c[u].w); x[u * 8 + 7] = bf16_hi(c[u].w);
      }
      float cm = x[0];
#pragma unroll
      for (int e = 1; e < kUnroll * 8; ++e) cm = fmaxf(cm, x[e]);
      const float mn = fmaxf(m2, cm * kLog2e);
      s *= fast_exp2(m2 - mn);
      m2 = mn;
#pragma unroll
      for (int e = 0; e < kUnroll * 8; ++e) s += fast_exp2(fmaf(x[e], kLog2e, -mn));
    }
    for (; i < nvec; i += kThreads) {
      const uint4 c = load_u4_stream(row + (i << 3));
      float x[8];
      x[0] = bf16_lo(c.x); x[1] = bf16_hi(c.x); x[2] = bf16_lo(c.y); x[3] = bf16_hi(c.y);
      x[4] = bf16_lo(c.z); x[5] = bf16_hi(c.z); x[6] = bf16_lo(c.w); x[7] = bf16_hi(c.w);
      float cm = x[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) cm = fmaxf(cm, x[e]);
      const float mn = fmaxf(m2, cm * kLog2e);
      s *= fast_exp2(m2 - mn);
      m2 = mn;
#pragma unroll
      for (int e = 0; e < 8; ++e) s += fast_exp2(fmaf(x[e], kLog2e, -mn));
    }
    for (int64_t j = (nvec << 3) + tid; j < vocab; j += kThreads) {
      const float x = bf16_to_f32(row[j]) * kLog2e;
      const float mn = fmaxf(m2, x);
      s = s * fast_exp2(m2 - mn) + fast_exp2(x - mn);
      m2 = mn;
    }
  } else {
    for (int64_t j = tid; j < vocab; j += kThreads) {
      const float x = bf16_to_f32(row[j]) * kLog2e;
      const float mn = fmaxf(m2, x);
      s = s * fast_exp2(m2 - mn) + fast_exp2(x - mn);
      m2 = mn;
    }
  }
  // Wave merge.
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float mo = shfl_xor_f32(m2, off);
    const float so = shfl_xor_f32(s, off);
    lse2_merge(m2, s, mo, so);
  }
  const int wave = tid >> 6;
  if ((tid & 63) == 0) {
    sm_m[wave] = m2;
    sm_s[wave] = s;
  }
  __syncthreads();
  float M = sm_m[0], S = sm_s[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) lse2_merge(M, S, sm_m[w], sm_s[w]);
  return M + log2f(S);
}

// Per-sequence group advantage (reference compute_grpo_advantage): scans the
// prompt ids; one lane computes it.
__device__ float group_advantage(const float* __restrict__ rewards,
                                 const int64_t* __restrict__ prompt_ids, int64_t n, int64_t i,
                                 float eps) {
  const int64_t pid = prompt_ids[i];
  float sum = 0.f;
  int64_t cnt = 0;
  for (int64_t j = 0; j < n; ++j)
    if (prompt_ids[j] == pid) {
      sum += rewards[j];
      ++cnt;
    }
  const float mean = sum / (float)cnt;
  float ss = 0.f;
  for (int64_t j = 0; j < n; ++j)
    if (prompt_ids[j] == pid) {
      const float d = rewards[j] - mean;
      ss += d * d;
    }
  // Unbiased estimate; cnt == 1 gives 0/0 = NaN exactly as torch.std().
  const float stdv = sqrtf(ss / (float)(cnt - 1));
  return (rewards[i] - mean) / (stdv + eps);
}

// Token term of the clipped surrogate and its derivative w.r.t. new_lp,
// following torch's subgradients: min() splits ties 1/2-1/2 and clamp()
// passes the gradient on the closed interval [lo, hi].
__device__ __forceinline__ void ppo_token(float new_lp, float old_lp, float adv, float clip,
                                          float* loss, float* dlp) {
  const float r = expf(new_lp - old_lp);
  const float lo = 1.0f - clip, hi = 1.0f + clip;
  const float rc = fminf(fmaxf(r, lo), hi);
  const float s1 = r * adv, s2 = rc * adv;
  *loss = -fminf(s1, s2);
  const float pass = (r >= lo && r <= hi) ? 1.f : 0.f;
  float w;
  if (s1 < s2) w = 1.f;
  else if (s1 > s2) w = pass;
  else w = 0.5f + 0.5f * pass;
  *dlp = -adv * r * w;
}

// ---------------------------------------------------------------------------
// Lane 0's gathered logit for the row's token.  Issued before the streaming
// loop so its latency overlaps the row read instead of trailing it.
__device__ __forceinline__ float gather_token_logit(const uint16_t* __restrict__ rp, int64_t id,
                                                    int64_t vocab) {
  return (id >= 0 && id < vocab) ? bf16_to_f32(rp[id]) : __builtin_nanf("");
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void logprob_rows(
    const uint16_t* __restrict__ logits, int64_t lss, int64_t lts,
    const int64_t* __restrict__ ids, int64_t iss, int64_t its, int64_t n_tok, int64_t vocab,
    float* __restrict__ out_lp, float* __restrict__ out_lse) {
  __shared__ float sm_m[kWaves], sm_s[kWaves];
  const int64_t row = blockIdx.x;
  const int64_t b = row / n_tok, t = row - b * n_tok;
  const uint16_t* rp = logits + b * lss + t * lts;
  float xid = 0.f;
  if (threadIdx.x == 0) xid = gather_token_logit(rp, ids[b * iss + t * its], vocab);
  const float lse2 = row_lse2<VEC>(rp, vocab, sm_m, sm_s);
  if (threadIdx.x == 0) {
    const float lse = lse2 * kLn2;
    out_lp[row] = xid - lse;
    if (out_lse) out_lse[row] = lse;
  }
}

struct FusedWs {
  float* seq_sum;        // [n_seq] sum_t l*m
  float* seq_msum;       // [n_seq] sum_t m
};

__host__ __device__ inline int64_t align16(int64_t x) { return (x + 15) & ~(int64_t)15; }

__host__ __device__ inline int64_t fused_ws_bytes(int64_t n_seq) {
  return 2 * align16(4 * n_seq);
}

__device__ inline FusedWs fused_ws(void* base, int64_t n_seq) {
  char* p = reinterpret_cast<char*>(base);
  FusedWs w;
  w.seq_sum = reinterpret_cast<float*>(p);
  p += align16(4 * n_seq);
  w.seq_msum = reinterpret_cast<float*>(p);
  return w;
}

// Block-wide fixed-order sum (every lane gets the total).
__device__ float block_sum(float x, float* sm) {
  x = wave_sum(x);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sm[wave] = x;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) t += sm[w];
  return t;
}

// Group advantage of sequence i computed by the whole block (parallel scan of
// the prompt ids; two fixed-order block reductions).
__device__ float block_group_advantage(const float* __restrict__ rewards,
                                       const int64_t* __restrict__ prompt_ids, int64_t n,
                                       int64_t i, float eps, float* sm) {
  const int64_t pid = prompt_ids[i];
  float sum = 0.f, cnt = 0.f;
  for (int64_t j = threadIdx.x; j < n; j += kThreads)
    if (prompt_ids[j] == pid) {
      sum += rewards[j];
      cnt += 1.f;
    }
  sum = block_sum(sum, sm);
  cnt = block_sum(cnt, sm);
  const float mean = sum / cnt;
  float ss = 0.f;
  for (int64_t j = threadIdx.x; j < n; j += kThreads)
    if (prompt_ids[j] == pid) {
      const float d = rewards[j] - mean;
      ss += d * d;
    }
  ss = block_sum(ss, sm);
  // Unbiased estimate; a group of one gives 0/0 = NaN exactly as torch.std().
  return (rewards[i] - mean) / (sqrtf(ss / (cnt - 1.f)) + eps);
}

// Loss epilogue of the fused step, part 1, launched right after
// logprob_rows has written lp for every row (the kernel boundary orders the
// two).  One workgroup per sequence b: the group advantage of b, the masked
// token losses and their gradients d loss / d lp for the n_tok tokens of b,
// and b's sums sum_t l*m and sum_t m.  Per-sequence mean: the gradients are
// final here (denominator n_seq * (sum_t m + 1e-8)).  Token mean: they are
// written without the denominator, which part 2 applies.
__global__ __launch_bounds__(kThreads) void grpo_loss_seqs(
    const float* __restrict__ lp, const float* __restrict__ old_lp,
    const float* __restrict__ mask, const float* __restrict__ rewards,
    const int64_t* __restrict__ prompt_ids, int64_t n_seq, int64_t n_tok, float adv_eps,
    float clip, int reduction, float* __restrict__ out_adv, float* __restrict__ out_dlp,
    void* __restrict__ ws_base) {
  __shared__ float sm_red[kWaves];
  const FusedWs ws = fused_ws(ws_base, n_seq);
  const int64_t b = blockIdx.x;
  const float adv = block_group_advantage(rewards, prompt_ids, n_seq, b, adv_eps, sm_red);
  const int64_t base = b * n_tok;
  float sl = 0.f, smk = 0.f;
  for (int64_t j = threadIdx.x; j < n_tok; j += kThreads) {
    const float m = mask[base + j];
    smk += m;
    float g = 0.f;
    if (m != 0.f) {
      float l;
      ppo_token(lp[base + j], old_lp[base + j], adv, clip, &l, &g);
      sl += l * m;
      g *= m;
    }
    out_dlp[base + j] = g;
  }
  sl = block_sum(sl, sm_red);
  smk = block_sum(smk, sm_red);
  if (reduction == QMI_REDUCE_SEQ_MEAN) {
    const float inv = 1.0f / ((float)n_seq * (smk + 1e-8f));
    for (int64_t j = threadIdx.x; j < n_tok; j += kThreads) out_dlp[base + j] *= inv;
  }
  if (threadIdx.x == 0) {
    ws.seq_sum[b] = sl;
    ws.seq_msum[b] = smk;
    out_adv[b] = adv;
  }
}

// Part 2.  Token mean: workgroup b scales sequence b's gradients by
// 1 / (sum of every sequence's mask sum + 1e-8), each workgroup forming that
// sum in the same fixed order.  Workgroup 0 also writes the scalar loss
// (sequence order).  Launched with n_seq workgroups for the token mean and
// one for the per-sequence mean.
__global__ __launch_bounds__(kThreads) void grpo_loss_finish(int64_t n_seq, int64_t n_tok,
                                                             int reduction,
                                                             float* __restrict__ out_dlp,
                                                             float* __restrict__ out_loss,
                                                             const void* __restrict__ ws_base) {
  __shared__ float sm_red[kWaves];
  const FusedWs ws = fused_ws(const_cast<void*>(ws_base), n_seq);
  const int64_t b = blockIdx.x;
  if (reduction == QMI_REDUCE_TOKEN_MEAN) {
    float part = 0.f;
    for (int64_t j = threadIdx.x; j < n_seq; j += kThreads) part += ws.seq_msum[j];
    const float den = block_sum(part, sm_red) + 1e-8f;
    const float inv = 1.0f / den;
    const int64_t base = b * n_tok;
    for (int64_t j = threadIdx.x; j < n_tok; j += kThreads) out_dlp[base + j] *= inv;
  }
  if (b == 0 && threadIdx.x == 0) {
    float loss;
    if (reduction == QMI_REDUCE_TOKEN_MEAN) {
      float num = 0.f, msum = 0.f;
      for (int64_t j = 0; j < n_seq; ++j) {
        num += ws.seq_sum[j];
        msum += ws.seq_msum[j];
      }
      loss = num / (msum + 1e-8f);
    } else {
      float acc = 0.f;
      for (int64_t j = 0; j < n_seq; ++j) acc += ws.seq_sum[j] / (ws.seq_msum[j] + 1e-8f);
      loss = acc / (float)n_seq;
    }
    *out_loss = loss;
  }
}

// ---------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(kThreads) void logprob_backward_rows(
    const uint16_t* __restrict__ logits, int64_t lss, int64_t lts,
    const int64_t* __restrict__ ids, int64_t iss, int64_t its, int64_t n_tok, int64_t vocab,
    const float* __restrict__ lse, const float* __restrict__ coef,
    const float* __restrict__ grad_scale, uint16_t* __restrict__ grad, int64_t gss, int64_t gts) {
  const int64_t row = blockIdx.x;
  const int64_t b = row / n_tok, t = row - b * n_tok;
  const uint16_t* rp = logits + b * lss + t * lts;
  uint16_t* gp = grad + b * gss + t * gts;
  const float c = coef[row] * (grad_scale ? *grad_scale : 1.0f);
  const int64_t id = ids[b * iss + t * its];
  const int tid = threadIdx.x;
  if (c == 0.f) {
    if (VEC) {
      const int64_t nvec = vocab >> 3;
      for (int64_t i = tid; i < nvec; i += kThreads)
        __builtin_nontemporal_store(u32x4_t{0u, 0u, 0u, 0u}, reinterpret_cast<u32x4_t*>(gp) + i);
      for (int64_t j = (nvec << 3) + tid; j < vocab; j += kThreads) gp[j] = 0;
    } else {
      for (int64_t j = tid; j < vocab; j += kThreads) gp[j] = 0;
    }
    return;
  }
  const float l2 = lse[row] * kLog2e;
  if (VEC) {
    const int64_t nvec = vocab >> 3;
    // kUnroll 16-byte loads in flight per lane; the gradient is streamed out
    // with non-temporal stores.
    auto grad8 = [&](const uint4 x, int64_t i) {
      const uint32_t w[4] = {x.x, x.y, x.z, x.w};
      u32x4_t o;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int64_t v0 = (i << 3) + 2 * k;
        float g0 = -c * fast_exp2(fmaf(bf16_lo(w[k]), kLog2e, -l2));
        float g1 = -c * fast_exp2(fmaf(bf16_hi(w[k]), kLog2e, -l2));
        if (v0 == id) g0 += c;
        if (v0 + 1 == id) g1 += c;
        o[k] = pack_bf16x2(g0, g1);
      }
      __builtin_nontemporal_store(o, reinterpret_cast<u32x4_t*>(gp) + i);
    };
    int64_t i = tid;
    for (; i + (kUnroll - 1) * kThreads < nvec; i += kUnroll * kThreads) {
      uint4 x[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) x[u] = load_u4_stream(rp + ((i + u * kThreads) << 3));
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) grad8(x[u], i + u * kThreads);
    }
    for (; i < nvec; i += kThreads) grad8(load_u4_stream(rp + (i << 3)), i);
    for (int64_t j = (nvec << 3) + tid; j < vocab; j += kThreads) {
      float g = -c * fast_exp2(fmaf(bf16_to_f32(rp[j]), kLog2e, -l2));
      if (j == id) g += c;
      gp[j] = f32_to_bf16(g);
    }
  } else {
    for (int64_t j = tid; j < vocab; j += kThreads) {
      float g = -c * fast_exp2(fmaf(bf16_to_f32(rp[j]), kLog2e, -l2));
      if (j == id) g += c;
      gp[j] = f32_to_bf16(g);
    }
  }
}

// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void advantage_kernel(const float* __restrict__ rewards,
                                                             const int64_t* __restrict__ pids,
                                                             int64_t n, float eps,
                                                             float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) out[i] = group_advantage(rewards, pids, n, i, eps);
}

// Single workgroup, fixed summation order (deterministic).
constexpr int kLossThreads = 1024;
__global__ __launch_bounds__(kLossThreads) void ppo_loss_kernel(
    const float* __restrict__ new_lp, const float* __restrict__ old_lp,
    const float* __restrict__ mask, const float* __restrict__ adv, int64_t ass, int64_t ats,
    int64_t n_seq, int64_t n_tok, float clip, int reduction, float* __restrict__ out_loss,
    float* __restrict__ out_dlp) {
  __shared__ float sm[kLossThreads / 64];
  const int tid = threadIdx.x;
  auto bsum = [&](float x) {
    x = wave_sum(x);
    __syncthreads();
    if ((tid & 63) == 0) sm[tid >> 6] = x;
    __syncthreads();
    float t = 0.f;
    for (int w = 0; w < kLossThreads / 64; ++w) t += sm[w];
    return t;
  };
  float all_m = 0.f;
  for (int64_t j = tid; j < n_seq * n_tok; j += kLossThreads) all_m += mask[j];
  all_m = bsum(all_m);
  float num = 0.f, acc = 0.f;
  for (int64_t b = 0; b < n_seq; ++b) {
    float sl = 0.f, smk = 0.f;
    for (int64_t t = tid; t < n_tok; t += kLossThreads) {
      const int64_t k = b * n_tok + t;
      const float m = mask[k];
      smk += m;
      if (m != 0.f) {
        float l, g;
        ppo_token(new_lp[k], old_lp[k], adv[b * ass + t * ats], clip, &l, &g);
        sl += l * m;
      }
    }
    sl = bsum(sl);
    smk = bsum(smk);
    num += sl;
    acc += sl / (smk + 1e-8f);
    if (out_dlp) {
      const float inv = reduction == QMI_REDUCE_TOKEN_MEAN ? 1.0f / (all_m + 1e-8f)
                                                           : 1.0f / ((float)n_seq * (smk + 1e-8f));
      for (int64_t t = tid; t < n_tok; t += kLossThreads) {
        const int64_t k = b * n_tok + t;
        const float m = mask[k];
        float g = 0.f;
        if (m != 0.f) {
          float l;
          ppo_token(new_lp[k], old_lp[k], adv[b * ass + t * ats], clip, &l, &g);
          g *= m * inv;
        }
        out_dlp[k] = g;
      }
    }
  }
  if (tid == 0)
    *out_loss = reduction == QMI_REDUCE_TOKEN_MEAN ? num / (all_m + 1e-8f) : acc / (float)n_seq;
}

inline bool rows_vec_ok(const uint16_t* p, int64_t s1, int64_t s2) {
  return ((reinterpret_cast<uintptr_t>(p) & 15u) == 0) && (s1 % 8 == 0) && (s2 % 8 == 0);
}

}  // namespace

extern "C" int qmi_logprob_gather(const uint16_t* logits, int64_t lss, int64_t lts,
                                  const int64_t* ids, int64_t iss, int64_t its, int64_t n_seq,
                                  int64_t n_tok, int64_t vocab, float* out_lp, float* out_lse,
                                  void* stream) {
  if (n_seq < 0 || n_tok < 0 || vocab <= 0) return QMI_E_BAD_SHAPE;
  if (n_seq * n_tok == 0) return QMI_OK;
  if (!logits || !ids || !out_lp) return QMI_E_NULL_POINTER;
  if (n_seq * n_tok > 0x7fffffffLL) return QMI_E_UNSUPPORTED;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(n_seq * n_tok));
  if (rows_vec_ok(logits, lss, lts))
    hipLaunchKernelGGL(logprob_rows<true>, grid, dim3(kThreads), 0, s, logits, lss, lts, ids, iss,
                       its, n_tok, vocab, out_lp, out_lse);
  else
    hipLaunchKernelGGL(logprob_rows<false>, grid, dim3(kThreads), 0, s, logits, lss, lts, ids,
                       iss, its, n_tok, vocab, out_lp, out_lse);
  QMI_RETURN_LAUNCH_STATUS();
}

extern "C" int qmi_grpo_advantage(const float* rewards, const int64_t* prompt_ids, int64_t n,
                                  float eps, float* out_adv, void* stream) {
  if (n < 0) return QMI_E_BAD_SHAPE;
  if (n == 0) return QMI_OK;
  if (!rewards || !prompt_ids || !out_adv) return QMI_E_NULL_POINTER;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(advantage_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, s, rewards, prompt_ids, n, eps, out_adv);
  QMI_RETURN_LAUNCH_STATUS();
}

extern "C" int qmi_ppo_clipped_loss(const float* new_lp, const float* old_lp, const float* mask,
                                    const float* adv, int64_t adv_seq_stride,
                                    int64_t adv_tok_stride, int64_t n_seq, int64_t n_tok,
                                    float clip_eps, int32_t reduction, float* out_loss,
                                    float* out_dlp, void* stream) {
  if (n_seq <= 0 || n_tok < 0) return QMI_E_BAD_SHAPE;
  if (!new_lp || !old_lp || !mask || !adv || !out_loss) return QMI_E_NULL_POINTER;
  if (reduction != QMI_REDUCE_TOKEN_MEAN && reduction != QMI_REDUCE_SEQ_MEAN)
    return QMI_E_UNSUPPORTED;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(ppo_loss_kernel, dim3(1), dim3(kLossThreads), 0, s, new_lp, old_lp, mask,
                     adv, adv_seq_stride, adv_tok_stride, n_seq, n_tok, clip_eps, (int)reduction,
                     out_loss, out_dlp);
  QMI_RETURN_LAUNCH_STATUS();
}

extern "C" int64_t qmi_grpo_fused_workspace_bytes(int64_t n_seq, int64_t n_tok) {
  if (n_seq <= 0 || n_tok <= 0) return 0;
  return fused_ws_bytes(n_seq);
}

extern "C" int qmi_grpo_fused_loss(const uint16_t* logits, int64_t lss, int64_t lts,
                                   const int64_t* ids, int64_t iss, int64_t its, int64_t n_seq,
                                   int64_t n_tok, int64_t vocab, const float* old_lp,
                                   const float* mask, const float* rewards,
                                   const int64_t* prompt_ids, float adv_eps, float clip_eps,
                                   int32_t reduction, float* out_lp, float* out_lse,
                                   float* out_adv, float* out_dlp, float* out_loss,
                                   void* workspace, int64_t workspace_bytes, void* stream) {
  if (n_seq <= 0 || n_tok <= 0 || vocab <= 0) return QMI_E_BAD_SHAPE;
  if (!logits || !ids || !old_lp || !mask || !rewards || !prompt_ids || !out_lp || !out_lse ||
      !out_adv || !out_dlp || !out_loss || !workspace)
    return QMI_E_NULL_POINTER;
  if (reduction != QMI_REDUCE_TOKEN_MEAN && reduction != QMI_REDUCE_SEQ_MEAN)
    return QMI_E_UNSUPPORTED;
  if (n_seq * n_tok > 0x7fffffffLL) return QMI_E_UNSUPPORTED;
  if (workspace_bytes < fused_ws_bytes(n_seq)) return QMI_E_WORKSPACE_TOO_SMALL;
  if (reinterpret_cast<uintptr_t>(workspace) & 15u) return QMI_E_BAD_STRIDE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(n_seq * n_tok));
  if (rows_vec_ok(logits, lss, lts))
    hipLaunchKernelGGL(logprob_rows<true>, grid, dim3(kThreads), 0, s, logits, lss, lts, ids, iss,
                       its, n_tok, vocab, out_lp, out_lse);
  else
    hipLaunchKernelGGL(logprob_rows<false>, grid, dim3(kThreads), 0, s, logits, lss, lts, ids,
                       iss, its, n_tok, vocab, out_lp, out_lse);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(grpo_loss_seqs, dim3((unsigned)n_seq), dim3(kThreads), 0, s, out_lp, old_lp,
                     mask, rewards, prompt_ids, n_seq, n_tok, adv_eps, clip_eps, (int)reduction,
                     out_adv, out_dlp, workspace);
  e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  const unsigned fin = reduction == QMI_REDUCE_TOKEN_MEAN ? (unsigned)n_seq : 1u;
  hipLaunchKernelGGL(grpo_loss_finish, dim3(fin), dim3(kThreads), 0, s, n_seq, n_tok,
                     (int)reduction, out_dlp, out_loss, workspace);
  QMI_RETURN_LAUNCH_STATUS();
}

extern "C" int qmi_logprob_gather_backward(const uint16_t* logits, int64_t lss, int64_t lts,
                                           const int64_t* ids, int64_t iss, int64_t its,
                                           int64_t n_seq, int64_t n_tok, int64_t vocab,
                                           const float* lse, const float* coef,
                                           const float* grad_scale, uint16_t* grad, int64_t gss,
                                           int64_t gts, void* stream) {
  if (n_seq < 0 || n_tok < 0 || vocab <= 0) return QMI_E_BAD_SHAPE;
  if (n_seq * n_tok == 0) return QMI_OK;
  if (!logits || !ids || !lse || !coef || !grad) return QMI_E_NULL_POINTER;
  if (n_seq * n_tok > 0x7fffffffLL) return QMI_E_UNSUPPORTED;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(n_seq * n_tok));
  if (rows_vec_ok(logits, lss, lts) && rows_vec_ok(grad, gss, gts))
    hipLaunchKernelGGL(logprob_backward_rows<true>, grid, dim3(kThreads), 0, s, logits, lss, lts,
                       ids, iss, its, n_tok, vocab, lse, coef, grad_scale, grad, gss, gts);
  else
    hipLaunchKernelGGL(logprob_backward_rows<false>, grid, dim3(kThreads), 0, s, logits, lss,
                       lts, ids, iss, its, n_tok, vocab, lse, coef, grad_scale, grad, gss, gts);
  QMI_RETURN_LAUNCH_STATUS();
}
