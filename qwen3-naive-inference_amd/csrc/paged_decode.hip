// Paged GQA decode attention with split-K online softmax (gfx950, no MFMA).
//
// Reference semantics: flash_attn_with_kvcache as called by
// Qwen3Attention.forward_decode (qwen3_naive.py:672-680): for sequence b and
// query head h, out = softmax(q_h . K^T * scale) V over keys 0..L_b-1 of KV
// head h / G, where L_b = cache_seqlens[b] and key j lives at row
// j % 256 of page block_table[b, j / 256] of the [blocks, 256, Hkv, 128]
// caches.  A single query row makes causal=True a no-op.
//
// Work decomposition (one workgroup = 256 lanes = 4 wave64):
//   grid = (Hkv, splits, B); a workgroup owns `pages_per_split` consecutive
//   pages of one (sequence, KV head).  The KV head is the fastest grid
//   index, so the 8 workgroups reading the interleaved 256-byte head rows of
//   the same 2 KB token rows run at the same time (measured: +6% HBM
//   throughput over a split-fastest grid).  Both query heads of the GQA group
//   are processed against every K/V row fetched, so K/V are read once.
//   Lane l handles head-dim slice [8*(l%16), 8*(l%16)+8): a DPP row of 16
//   lanes covers one 256-byte K (or V) head row with one dwordx4 load per
//   lane.  A page is processed in two steps of 128 tokens; row-group
//   rg = tid/16 (0..15) owns tokens rg, rg+16, ... of each step and keeps its
//   own running (max, sum, acc), so the page loop needs no barrier and no
//   LDS.  QK partial dots (v_dot2_f32_bf16 on bf16 pairs) are summed across
//   the 16 lanes with DPP adds.  Half-page steps keep the register
//   footprint small enough for >= 3 resident workgroups per CU at G = 2.
//   At the end of a split the 16 row-group states are merged (two shuffles
//   inside each wave, then LDS across the 4 waves).  A sequence that fits in
//   one split writes its output directly; otherwise the split writes
//   (acc, m, l) to the workspace and paged_decode_merge combines splits.
//
// All softmax arithmetic is fp32 in the log2 domain (exp2 with the scale
// pre-multiplied by log2(e)).
#include <atomic>
#include <mutex>

#include "qmi_common.h"

namespace {

using namespace qmi;

constexpr int kHeadDim = 128;
constexpr int kPage = 256;
constexpr int kThreads = 256;
constexpr int kRowGroups = kThreads / 16;          // 16
constexpr int kStepTokens = 128;                    // tokens per step (half a page)
constexpr int kTokPerRg = kStepTokens / kRowGroups; // 8 tokens per row-group per step
constexpr int kWsStride = kHeadDim + 4;             // acc[128], m, l, pad

// Waves per SIMD the register budget is sized for (3 => <= 168 VGPRs).
template <int G>
constexpr int decode_occupancy() { return G <= 2 ? 3 : (G == 4 ? 2 : 1); }

template <int G>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(decode_occupancy<G>())))
void paged_decode_split(
    const uint16_t* __restrict__ q, int64_t q_seq_stride, int64_t q_head_stride,
    const uint16_t* __restrict__ k_cache, const uint16_t* __restrict__ v_cache,
    int64_t num_blocks, int num_kv_heads,
    const int32_t* __restrict__ seqlens, int seqlen_bias,
    const int32_t* __restrict__ block_table, int64_t bt_stride, int bt_width,
    int pages_per_split, int num_splits, float scale_log2,
    uint16_t* __restrict__ out, int64_t out_seq_stride, int64_t out_head_stride,
    float* __restrict__ ws) {
  const int kvh = blockIdx.x;
  const int split = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane16 = tid & 15;
  const int rg = tid >> 4;

  int L = seqlens[b] + seqlen_bias;
  L = max(0, min(L, bt_width * kPage));
  const int n_pages = (L + kPage - 1) / kPage;
  const int n_split_b = (n_pages + pages_per_split - 1) / pages_per_split;

  if (split >= n_split_b) {
    // An empty sequence attends to nothing: flash-attn returns zeros.
    if (L == 0 && split == 0) {
      for (int o = tid; o < G * kHeadDim; o += kThreads) {
        const int g = o / kHeadDim, d = o % kHeadDim;
        out[b * out_seq_stride + (int64_t)(kvh * G + g) * out_head_stride + d] = 0;
      }
    }
    return;
  }
  const int page_begin = split * pages_per_split;
  const int page_end = min(n_pages, page_begin + pages_per_split);

  uint32_t qw[G][4];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint4 v = load_u4(q + b * q_seq_stride + (int64_t)(kvh * G + g) * q_head_stride + lane16 * 8);
    qw[g][0] = v.x; qw[g][1] = v.y; qw[g][2] = v.z; qw[g][3] = v.w;
  }

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegBig;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }

  const int64_t tok_stride = (int64_t)num_kv_heads * kHeadDim;
  const int n_steps = (page_end - page_begin) * (kPage / kStepTokens);
  for (int st = 0; st < n_steps; ++st) {
    const int pg = page_begin + st / (kPage / kStepTokens);
    const int half = st % (kPage / kStepTokens);
    const int64_t blk = block_table[(int64_t)b * bt_stride + pg];
    if (blk < 0 || blk >= num_blocks) continue;  // uniform over the workgroup
    const int n_valid = min(kPage, L - pg * kPage) - half * kStepTokens;
    if (n_valid <= 0) continue;
    const int64_t base = (blk * kPage * num_kv_heads + kvh) * kHeadDim + lane16 * 8 +
                         (int64_t)half * kStepTokens * tok_stride;
    const uint16_t* kp = k_cache + base;
    const uint16_t* vp = v_cache + base;

    uint4 kr[kTokPerRg], vr[kTokPerRg];
#pragma unroll
    for (int i = 0; i < kTokPerRg; ++i) {
      const int t = rg + kRowGroups * i;
      kr[i] = t < n_valid ? load_u4_stream(kp + t * tok_stride) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kTokPerRg; ++i) {
      const int t = rg + kRowGroups * i;
      vr[i] = t < n_valid ? load_u4_stream(vp + t * tok_stride) : make_uint4(0, 0, 0, 0);
    }

    float s[G][kTokPerRg];
#pragma unroll
    for (int i = 0; i < kTokPerRg; ++i) {
      const bool valid = (rg + kRowGroups * i) < n_valid;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = dot2_bf16(qw[g][0], kr[i].x, 0.f);
        d = dot2_bf16(qw[g][1], kr[i].y, d);
        d = dot2_bf16(qw[g][2], kr[i].z, d);
        d = dot2_bf16(qw[g][3], kr[i].w, d);
        d = row16_sum(d);
        s[g][i] = valid ? d * scale_log2 : -INFINITY;
      }
    }

#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = s[g][0];
#pragma unroll
      for (int i = 1; i < kTokPerRg; ++i) mx = fmaxf(mx, s[g][i]);
      const float mn = fmaxf(m[g], mx);
      const float alpha = fast_exp2(m[g] - mn);
      m[g] = mn;
      l[g] *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] *= alpha;
#pragma unroll
      for (int i = 0; i < kTokPerRg; ++i) {
        const float p = fast_exp2(s[g][i] - mn);
        s[g][i] = p;
        l[g] += p;
      }
    }

#pragma unroll
    for (int i = 0; i < kTokPerRg; ++i) {
      float v[8];
      v[0] = bf16_lo(vr[i].x); v[1] = bf16_hi(vr[i].x);
      v[2] = bf16_lo(vr[i].y); v[3] = bf16_hi(vr[i].y);
      v[4] = bf16_lo(vr[i].z); v[5] = bf16_hi(vr[i].z);
      v[6] = bf16_lo(vr[i].w); v[7] = bf16_hi(vr[i].w);
#pragma unroll
      for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(s[g][i], v[e], acc[g][e]);
      }
    }
  }

  // Merge the four row-groups of each wave (lanes differing in bits 4 and 5).
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mo = shfl_xor_f32(m[g], off);
      const float lo = shfl_xor_f32(l[g], off);
      const float mn = fmaxf(m[g], mo);
      const float a1 = fast_exp2(m[g] - mn);
      const float a2 = fast_exp2(mo - mn);
      l[g] = l[g] * a1 + lo * a2;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float ao = shfl_xor_f32(acc[g][e], off);
        acc[g][e] = acc[g][e] * a1 + ao * a2;
      }
      m[g] = mn;
    }
  }

  __shared__ float sm_acc[4][G][kHeadDim];
  __shared__ float sm_m[4][G];
  __shared__ float sm_l[4][G];
  const int wave = tid >> 6;
  if ((tid & 63) < 16) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sm_acc[wave][g][lane16 * 8 + e] = acc[g][e];
      if (lane16 == 0) {
        sm_m[wave][g] = m[g];
        sm_l[wave][g] = l[g];
      }
    }
  }
  __syncthreads();

  const bool direct = (n_split_b == 1);
  for (int o = tid; o < G * kHeadDim; o += kThreads) {
    const int g = o / kHeadDim, d = o % kHeadDim;
    float M = sm_m[0][g];
#pragma unroll
    for (int w = 1; w < 4; ++w) M = fmaxf(M, sm_m[w][g]);
    float Ls = 0.f, A = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float a = fast_exp2(sm_m[w][g] - M);
      Ls += sm_l[w][g] * a;
      A += sm_acc[w][g][d] * a;
    }
    if (direct) {
      const float r = Ls > 0.f ? A / Ls : 0.f;
      out[b * out_seq_stride + (int64_t)(kvh * G + g) * out_head_stride + d] = f32_to_bf16(r);
    } else {
      float* w = ws + ((((int64_t)b * num_kv_heads + kvh) * num_splits + split) * G + g) * kWsStride;
      w[d] = A;
      if (d == 0) {
        w[kHeadDim] = M;
        w[kHeadDim + 1] = Ls;
      }
    }
  }
}

// Combines the per-split partial states of sequences that needed > 1 split.
// grid = (Hkv, B), G*128 lanes: lane (g, d) produces out[b, kvh*G+g, d].
template <int G>
__global__ __launch_bounds__(G * kHeadDim) void paged_decode_merge(
    const int32_t* __restrict__ seqlens, int seqlen_bias, int bt_width, int num_kv_heads,
    int pages_per_split, int num_splits, const float* __restrict__ ws,
    uint16_t* __restrict__ out, int64_t out_seq_stride, int64_t out_head_stride) {
  const int kvh = blockIdx.x;
  const int b = blockIdx.y;
  const int g = threadIdx.x / kHeadDim;
  const int d = threadIdx.x % kHeadDim;
  int L = seqlens[b] + seqlen_bias;
  L = max(0, min(L, bt_width * kPage));
  const int n_pages = (L + kPage - 1) / kPage;
  const int n_split_b = (n_pages + pages_per_split - 1) / pages_per_split;
  if (n_split_b <= 1) return;
  const float* w0 = ws + ((((int64_t)b * num_kv_heads + kvh) * num_splits) * G + g) * kWsStride;
  const int64_t sstride = (int64_t)G * kWsStride;
  float M = kNegBig;
  for (int s = 0; s < n_split_b; ++s) M = fmaxf(M, w0[s * sstride + kHeadDim]);
  float Ls = 0.f, A = 0.f;
  for (int s = 0; s < n_split_b; ++s) {
    const float* w = w0 + s * sstride;
    const float a = fast_exp2(w[kHeadDim] - M);
    Ls += w[kHeadDim + 1] * a;
    A += w[d] * a;
  }
  const float r = Ls > 0.f ? A / Ls : 0.f;
  out[b * out_seq_stride + (int64_t)(kvh * G + g) * out_head_stride + d] = f32_to_bf16(r);
}

int64_t auto_pages_per_split(int64_t batch, int64_t num_kv_heads, int64_t bt_width) {
  // Small launches keep one page (128 KB of K+V per KV head) per workgroup
  // for parallelism; serving-size launches take two pages per workgroup
  // (same HBM throughput, half the partial states to merge); very wide
  // tables (graph-capture width) are folded so the grid stays near 32K
  // workgroups.
  const int64_t units = batch * num_kv_heads * bt_width;
  if (units < 4096) return 1;
  const int64_t target = 32768;
  const int64_t pps = (units + target - 1) / target;
  return pps < 2 ? 2 : pps;
}

template <int G>
int launch_decode(const uint16_t* q, int64_t q_seq_stride, int64_t q_head_stride,
                  const uint16_t* k_cache, const uint16_t* v_cache, int64_t num_blocks,
                  int64_t num_kv_heads, const int32_t* seqlens, int32_t seqlen_bias,
                  const int32_t* block_table, int64_t bt_stride, int64_t bt_width, int64_t batch,
                  float scale, uint16_t* out, int64_t out_seq_stride, int64_t out_head_stride,
                  float* ws, int64_t pps, hipStream_t s) {
  const int64_t num_splits = (bt_width + pps - 1) / pps;
  const float scale_log2 = scale * kLog2e;
  dim3 grid((unsigned)num_kv_heads, (unsigned)num_splits, (unsigned)batch);
  hipLaunchKernelGGL(paged_decode_split<G>, grid, dim3(kThreads), 0, s, q, q_seq_stride,
                     q_head_stride, k_cache, v_cache, num_blocks, (int)num_kv_heads, seqlens,
                     (int)seqlen_bias, block_table, bt_stride, (int)bt_width, (int)pps,
                     (int)num_splits, scale_log2, out, out_seq_stride, out_head_stride, ws);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  if (num_splits > 1) {
    hipLaunchKernelGGL(paged_decode_merge<G>, dim3((unsigned)num_kv_heads, (unsigned)batch),
                       dim3(G * kHeadDim), 0, s, seqlens, (int)seqlen_bias, (int)bt_width,
                       (int)num_kv_heads, (int)pps, (int)num_splits, ws, out, out_seq_stride,
                       out_head_stride);
  }
  QMI_RETURN_LAUNCH_STATUS();
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

namespace qmi {
// Balanced decode (paged_decode_streamk.hip).
int64_t streamk_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                int64_t bt_width);
bool streamk_supported(int64_t num_q_heads, int64_t num_kv_heads, int64_t batch);
int launch_streamk(const uint16_t* q, int64_t qs, int64_t qh, const uint16_t* kc,
                   const uint16_t* vc, int64_t nb, int64_t num_q_heads, int64_t num_kv_heads,
                   const int32_t* lens, int32_t bias, const int32_t* bt, int64_t bts, int64_t btw,
                   int64_t batch, float scale, uint16_t* out, int64_t os, int64_t oh, float* ws,
                   bool whole_units, hipStream_t s);
}  // namespace qmi

extern "C" int64_t qmi_paged_decode_workspace_bytes(int64_t batch, int64_t num_kv_heads,
                                                    int64_t num_q_heads, int64_t bt_width,
                                                    int64_t pages_per_split) {
  if (batch <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || bt_width <= 0) return 0;
  const int64_t pps = pages_per_split > 0 ? pages_per_split
                                          : auto_pages_per_split(batch, num_kv_heads, bt_width);
  const int64_t num_splits = (bt_width + pps - 1) / pps;
  const int64_t split_bytes =
      num_splits <= 1 ? 0 : batch * num_q_heads * num_splits * kWsStride * (int64_t)sizeof(float);
  // The automatic schedule may take either path (the balanced one needs a
  // 16-byte aligned output), so it asks for the larger of the two.
  if (pages_per_split <= 0 && num_q_heads % num_kv_heads == 0 &&
      qmi::streamk_supported(num_q_heads, num_kv_heads, batch)) {
    const int64_t sk = qmi::streamk_workspace_bytes(batch, num_q_heads, num_kv_heads, bt_width);
    return sk > split_bytes ? sk : split_bytes;
  }
  return split_bytes;
}

extern "C" int qmi_paged_decode_attention(
    const uint16_t* q, int64_t q_seq_stride, int64_t q_head_stride, const uint16_t* k_cache,
    const uint16_t* v_cache, int64_t num_blocks, int64_t block_size, int64_t num_q_heads,
    int64_t num_kv_heads, int64_t head_dim, const int32_t* seqlens, int32_t seqlen_bias,
    const int32_t* block_table, int64_t bt_stride, int64_t bt_width, int64_t batch, float scale,
    uint16_t* out, int64_t out_seq_stride, int64_t out_head_stride, float* workspace,
    int64_t workspace_bytes, int64_t pages_per_split, void* stream) {
  if (batch < 0 || num_blocks < 0 || bt_width < 0) return QMI_E_BAD_SHAPE;
  if (batch == 0) return QMI_OK;
  if (num_blocks == 0) return QMI_E_BAD_SHAPE;  // a pool without pages
  if (!q || !k_cache || !v_cache || !seqlens || !block_table || !out) return QMI_E_NULL_POINTER;
  if (head_dim != kHeadDim || block_size != kPage) return QMI_E_UNSUPPORTED;
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return QMI_E_BAD_SHAPE;
  if (bt_width == 0) return QMI_E_BAD_SHAPE;
  if (bt_stride < bt_width) return QMI_E_BAD_STRIDE;
  if (batch > 65535 || num_kv_heads > 65535) return QMI_E_UNSUPPORTED;
  if (bt_width > 65535) return QMI_E_UNSUPPORTED;
  if ((q_seq_stride % 8) || (q_head_stride % 8) || !aligned16(q) || !aligned16(k_cache) ||
      !aligned16(v_cache))
    return QMI_E_BAD_STRIDE;
  const int64_t G = num_q_heads / num_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8) return QMI_E_UNSUPPORTED;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (pages_per_split <= 0 && qmi::streamk_supported(num_q_heads, num_kv_heads, batch) &&
      aligned16(out) && out_seq_stride % 8 == 0 && out_head_stride % 8 == 0) {
    const int64_t need = qmi::streamk_workspace_bytes(batch, num_q_heads, num_kv_heads, bt_width);
    if (!workspace || workspace_bytes < need) return QMI_E_WORKSPACE_TOO_SMALL;
    return qmi::launch_streamk(q, q_seq_stride, q_head_stride, k_cache, v_cache, num_blocks,
                               num_q_heads, num_kv_heads, seqlens, seqlen_bias, block_table,
                               bt_stride, bt_width, batch, scale, out, out_seq_stride,
                               out_head_stride, workspace, pages_per_split == -1, s);
  }
  const int64_t pps = pages_per_split > 0 ? pages_per_split
                                          : auto_pages_per_split(batch, num_kv_heads, bt_width);
  const int64_t need = qmi_paged_decode_workspace_bytes(batch, num_kv_heads, num_q_heads,
                                                        bt_width, pps);
  if (need > 0 && (!workspace || workspace_bytes < need)) return QMI_E_WORKSPACE_TOO_SMALL;
#define QMI_DECODE_CASE(GG)                                                                    \
  case GG:                                                                                     \
    return launch_decode<GG>(q, q_seq_stride, q_head_stride, k_cache, v_cache, num_blocks,     \
                             num_kv_heads, seqlens, seqlen_bias, block_table, bt_stride,       \
                             bt_width, batch, scale, out, out_seq_stride, out_head_stride,     \
                             workspace, pps, s);
  switch (G) {
    QMI_DECODE_CASE(1)
    QMI_DECODE_CASE(2)
    QMI_DECODE_CASE(4)
    QMI_DECODE_CASE(8)
    default:
      return QMI_E_UNSUPPORTED;
  }
#undef QMI_DECODE_CASE
}

// ---------------------------------------------------------------------------
// No-allocation variant: the workspace is a file-scope device array instead
// of a caller buffer.  Each device that loads the library holds its own copy
// until the process ends; host code reaches it only through the address
// hipGetSymbolAddress returns for that device (the array's name is a host
// stand-in, not a device address).  Every workspace word the kernels read is
// written earlier in the same call (partial slots by the split, the step
// offsets and mode word by its workgroup 0), so nothing needs clearing
// between calls.  Calls that overlap on one device share the array and race.
namespace {

constexpr int64_t kDecodeScratchBytes = 16ll << 20;
__device__ __align__(256) float scratch[kDecodeScratchBytes / sizeof(float)];

constexpr int kMaxScratchDevices = 64;
std::atomic<float*> g_scratch_ptr[kMaxScratchDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the calling thread's current device (the
// device of the stream and of every pointer, as for all entry points),
// looked up once per device with that device current.
int decode_scratch(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxScratchDevices) return QMI_E_UNSUPPORTED;
  float* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      void* addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return (int)e;
      if (!addr) return QMI_E_NULL_POINTER;
      p = static_cast<float*>(addr);
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return QMI_OK;
}

}  // namespace

extern "C" int qmi_paged_decode_attention_noalloc(
    const uint16_t* q, int64_t q_seq_stride, int64_t q_head_stride, const uint16_t* k_cache,
    const uint16_t* v_cache, int64_t num_blocks, int64_t block_size, int64_t num_q_heads,
    int64_t num_kv_heads, int64_t head_dim, const int32_t* seqlens, int32_t seqlen_bias,
    const int32_t* block_table, int64_t bt_stride, int64_t bt_width, int64_t batch, float scale,
    uint16_t* out, int64_t out_seq_stride, int64_t out_head_stride, int64_t pages_per_split,
    void* stream) {
  // Shapes the regular entry point rejects are rejected the same way, before
  // any HIP call: it is handed a null workspace of size 0 only when nothing
  // is launched (batch 0) or an argument is invalid.
  if (batch < 0 || num_blocks < 0 || bt_width < 0) return QMI_E_BAD_SHAPE;
  if (batch == 0) return QMI_OK;
  if (num_blocks == 0 || bt_width == 0) return QMI_E_BAD_SHAPE;
  if (!q || !k_cache || !v_cache || !seqlens || !block_table || !out) return QMI_E_NULL_POINTER;
  if (head_dim != kHeadDim || block_size != kPage) return QMI_E_UNSUPPORTED;
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return QMI_E_BAD_SHAPE;
  // The workspace the call will use: the balanced schedule's when it takes
  // that path (the regular entry point's condition), else the per-split one's.
  const bool balanced = pages_per_split <= 0 &&
                        qmi::streamk_supported(num_q_heads, num_kv_heads, batch) &&
                        aligned16(out) && out_seq_stride % 8 == 0 && out_head_stride % 8 == 0;
  const int64_t pps = pages_per_split > 0 ? pages_per_split
                                          : auto_pages_per_split(batch, num_kv_heads, bt_width);
  const int64_t need =
      balanced ? qmi::streamk_workspace_bytes(batch, num_q_heads, num_kv_heads, bt_width)
               : qmi_paged_decode_workspace_bytes(batch, num_kv_heads, num_q_heads, bt_width, pps);
  if (need > kDecodeScratchBytes) return QMI_E_SCRATCH_LIMIT;
  float* ws = nullptr;
  const int st = decode_scratch(&ws);
  if (st != QMI_OK) return st;
  return qmi_paged_decode_attention(q, q_seq_stride, q_head_stride, k_cache, v_cache, num_blocks,
                                    block_size, num_q_heads, num_kv_heads, head_dim, seqlens,
                                    seqlen_bias, block_table, bt_stride, bt_width, batch, scale,
                                    out, out_seq_stride, out_head_stride, ws, kDecodeScratchBytes,
                                    pages_per_split, stream);
}
