// Varlen paged causal prefill attention on bf16 MFMA (gfx950).
//
// Reference semantics: flash_attn_varlen_func(q, k_cache, v_cache,
// cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale,
// causal=True, block_table) in Qwen3Attention.forward_prefill
// (qwen3_naive.py:631-637).  Sequence b has Lq = cu_q[b+1]-cu_q[b] new
// queries and Lk = cu_k[b+1]-cu_k[b] keys (cached prefix + earlier chunks +
// this chunk, already stored); key j is row j % 256 of page
// block_table[b, j / 256].  Causal masking is bottom-right aligned: query i
// sees keys j <= i + Lk - Lq.  Query head h reads KV head h / G.
//
// Design (FlashAttention-2 forward, reorganised for CDNA MFMA operands):
//   * Workgroup = 4 wave64 = one (sequence, KV head, block of 64/G queries);
//     wave w takes query head (w / (4/G)) of the GQA group and 16 queries, so
//     the K/V tiles staged in LDS serve all G query heads.
//   * Scores are computed transposed, S^T = K Q^T, with
//     v_mfma_f32_16x16x32_bf16 (A = 16 keys x 32 dims from LDS, B = Q^T held
//     in registers).  Its accumulator layout (lane l: keys 4*(l/16)+r,
//     query l%16) is exactly the B-operand layout of the second product
//     O^T = V^T P^T once two 16-key blocks are packed to bf16, so P never
//     leaves registers.  V^T comes from LDS, where each 64-key V tile is
//     written transposed while being staged.
//   * Online softmax in fp32 (log2 domain); per query the 4 lanes holding
//     its keys agree on the running max through two shuffles, while the
//     running sum stays lane-partial until the end.
//   * K / V^T tiles of 64 keys (one quarter page) are double-buffered in LDS:
//     the global loads for tile t+1 are in flight while tile t is computed.
//   * Grid = (Hkv, query blocks, B): with 8 KV heads the KV head maps to the
//     XCD, so all query blocks of one (sequence, KV head) share an L2.
//     Query blocks are issued last-first, so the longest (causal) blocks
//     start first.
#include "qmi_common.h"

namespace {

using namespace qmi;

constexpr int kHeadDim = 128;
constexpr int kPage = 256;
constexpr int kThreads = 256;
constexpr int kKeyTile = 64;
constexpr int kKPitch = kHeadDim + 8;   // bf16 per K row in LDS (272 B, breaks bank aliasing)
constexpr int kVtPitch = kKeyTile + 4;  // bf16 per V^T row in LDS (136 B)

typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
  return __builtin_bit_cast(bf16x8_t, u32x4_t{v.x, v.y, v.z, v.w});
}

template <int G>
__global__ __launch_bounds__(kThreads) void varlen_prefill_kernel(
    const uint16_t* __restrict__ q, int64_t q_tok_stride, int64_t q_head_stride,
    const uint16_t* __restrict__ k_cache, const uint16_t* __restrict__ v_cache,
    int64_t num_blocks, int num_kv_heads,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k,
    const int32_t* __restrict__ block_table, int64_t bt_stride, int bt_width,
    int n_qblocks, int64_t total_q, float scale_log2,
    uint16_t* __restrict__ out, int64_t out_tok_stride, int64_t out_head_stride) {
  constexpr int kWavesPerHead = 4 / G;
  constexpr int kQB = 16 * kWavesPerHead;  // queries per workgroup
  __shared__ __attribute__((aligned(16))) uint16_t sK[2][kKeyTile * kKPitch];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[2][kHeadDim * kVtPitch];

  const int kvh = blockIdx.x;
  const int qblk = n_qblocks - 1 - (int)blockIdx.y;  // late (long) blocks first
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int g4 = lane >> 4;

  // Rows outside [0, total_q) of q / out are never touched, whatever cu_q holds.
  const int q_start = max(0, cu_q[b]);
  const int Lq = (int)max((int64_t)0, min((int64_t)cu_q[b + 1], total_q) - q_start);
  int Lk = cu_k[b + 1] - cu_k[b];
  Lk = max(0, min(Lk, bt_width * kPage));
  const int q0 = qblk * kQB;
  if (q0 >= Lq) return;  // uniform over the workgroup
  const int diag = Lk - Lq;  // query i sees keys j <= i + diag

  const int qh = kvh * G + wave / kWavesPerHead;
  const int wq0 = q0 + (wave % kWavesPerHead) * 16;
  const int my_q = wq0 + l16;  // this lane's query (column of S^T)
  const bool q_valid = my_q < Lq;

  // Q^T operand: lane holds Q[my_q][32c + 8*g4 .. +8] for c = 0..3.
  bf16x8_t qop[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    uint4 v = make_uint4(0, 0, 0, 0);
    if (q_valid)
      v = load_u4(q + (int64_t)(q_start + my_q) * q_tok_stride + (int64_t)qh * q_head_stride +
                  32 * c + 8 * g4);
    qop[c] = as_bf16x8(v);
  }

  // Keys this workgroup needs: up to the last query's diagonal.
  const int kend = max(0, min(Lk, diag + min(q0 + kQB, Lq)));
  const int n_tiles = (kend + kKeyTile - 1) / kKeyTile;

  // Staging: each lane moves 4 K chunks and 4 V chunks of 16 B per tile.
  uint4 kst[4], vst[4];
  auto load_tile = [&](int t) {
    const int key0 = t * kKeyTile;
    const int64_t blk = block_table[(int64_t)b * bt_stride + key0 / kPage];
    const bool page_ok = blk >= 0 && blk < num_blocks;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + kThreads * i;
      const int key = c >> 4, dchunk = c & 15;
      const bool ok = page_ok && (key0 + key) < kend;
      const int64_t off = ((blk * kPage + (key0 % kPage) + key) * num_kv_heads + kvh) * kHeadDim +
                          8 * dchunk;
      kst[i] = ok ? load_u4(k_cache + off) : make_uint4(0, 0, 0, 0);
      vst[i] = ok ? load_u4(v_cache + off) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + kThreads * i;
      const int key = c >> 4, dchunk = c & 15;
      *reinterpret_cast<uint4*>(&sK[buf][key * kKPitch + 8 * dchunk]) = kst[i];
      const uint32_t w[4] = {vst[i].x, vst[i].y, vst[i].z, vst[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sVt[buf][(8 * dchunk + 2 * e) * kVtPitch + key] = (uint16_t)(w[e] & 0xffffu);
        sVt[buf][(8 * dchunk + 2 * e + 1) * kVtPitch + key] = (uint16_t)(w[e] >> 16);
      }
    }
  };

  float m_run = kNegBig;  // running max (log2 domain) of this lane's query
  float l_run = 0.f;      // lane-partial running sum
  f32x4_t acc_o[8];       // O^T[dim 16*db + 4*g4 + r][query l16]
#pragma unroll
  for (int db = 0; db < 8; ++db) acc_o[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int my_pos = diag + my_q;  // last key this query may see

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < n_tiles) load_tile(t + 1);

    // ---- S^T = K Q^T for 4 blocks of 16 keys ----
    f32x4_t s[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f32x4_t a = {0.f, 0.f, 0.f, 0.f};
      const uint16_t* krow = &sK[buf][(kb * 16 + l16) * kKPitch + 8 * g4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const bf16x8_t kop = as_bf16x8(*reinterpret_cast<const uint4*>(krow + 32 * c));
        a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qop[c], a, 0, 0, 0);
      }
      s[kb] = a;
    }

    // ---- scale, causal / length mask, tile max ----
    const int key_base = t * kKeyTile;
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = key_base + kb * 16 + 4 * g4 + r;
        const bool ok = q_valid && key <= my_pos && key < Lk;
        const float v = ok ? s[kb][r] * scale_log2 : -INFINITY;
        s[kb][r] = v;
        tmax = fmaxf(tmax, v);
      }
    }
    tmax = fmaxf(tmax, shfl_xor_f32(tmax, 16));
    tmax = fmaxf(tmax, shfl_xor_f32(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int db = 0; db < 8; ++db) acc_o[db] *= alpha;

    // ---- P^T as bf16 B operands: chunk c packs key blocks 2c and 2c+1 ----
    bf16x8_t pop[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      float p[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[r] = fast_exp2(s[2 * c][r] - m_new);
        p[4 + r] = fast_exp2(s[2 * c + 1][r] - m_new);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        l_run += p[e];
        pop[c][e] = (__bf16)p[e];
      }
    }

    // ---- O^T += V^T P^T over 8 blocks of 16 dims ----
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const uint16_t* vrow = &sVt[buf][(db * 16 + l16) * kVtPitch];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(vrow + 32 * c + 4 * g4);
        const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(vrow + 32 * c + 16 + 4 * g4);
        const u32x4_t w = {lo.x, lo.y, hi.x, hi.y};
        acc_o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, w),
                                                            pop[c], acc_o[db], 0, 0, 0);
      }
    }

    if (t + 1 < n_tiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- normalise and write O[query][dims] ----
  float l_tot = l_run + shfl_xor_f32(l_run, 16);
  l_tot += shfl_xor_f32(l_tot, 32);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  if (q_valid) {
    uint16_t* orow = out + (int64_t)(q_start + my_q) * out_tok_stride + (int64_t)qh * out_head_stride;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const uint32_t w0 = pack_bf16x2(acc_o[db][0] * inv, acc_o[db][1] * inv);
      const uint32_t w1 = pack_bf16x2(acc_o[db][2] * inv, acc_o[db][3] * inv);
      *reinterpret_cast<u32x2_t*>(orow + db * 16 + 4 * g4) = u32x2_t{w0, w1};
    }
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int qmi_varlen_prefill_attention(
    const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride, const uint16_t* k_cache,
    const uint16_t* v_cache, int64_t num_blocks, int64_t block_size, int64_t num_q_heads,
    int64_t num_kv_heads, int64_t head_dim, const int32_t* cu_seqlens_q,
    const int32_t* cu_seqlens_k, const int32_t* block_table, int64_t bt_stride, int64_t bt_width,
    int64_t batch, int64_t max_seqlen_q, int64_t total_q, float scale, uint16_t* out,
    int64_t out_tok_stride, int64_t out_head_stride, void* stream) {
  if (batch < 0 || max_seqlen_q < 0 || num_blocks < 0 || bt_width < 0) return QMI_E_BAD_SHAPE;
  if (total_q < 0) return QMI_E_BAD_SHAPE;
  if (batch == 0 || max_seqlen_q == 0 || total_q == 0) return QMI_OK;
  if (!q || !k_cache || !v_cache || !cu_seqlens_q || !cu_seqlens_k || !block_table || !out)
    return QMI_E_NULL_POINTER;
  if (head_dim != kHeadDim || block_size != kPage) return QMI_E_UNSUPPORTED;
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return QMI_E_BAD_SHAPE;
  const int64_t G = num_q_heads / num_kv_heads;
  if (G != 1 && G != 2 && G != 4) return QMI_E_UNSUPPORTED;
  if (bt_width == 0 || bt_stride < bt_width) return QMI_E_BAD_STRIDE;
  if ((q_tok_stride % 8) || (q_head_stride % 8) || (out_tok_stride % 4) || (out_head_stride % 4) ||
      !aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) ||
      (reinterpret_cast<uintptr_t>(out) & 7u))
    return QMI_E_BAD_STRIDE;
  const int64_t qb = 64 / G;
  const int64_t n_qblocks = (max_seqlen_q + qb - 1) / qb;
  if (n_qblocks > 65535 || batch > 65535 || num_kv_heads > 65535 || bt_width > (1 << 22))
    return QMI_E_UNSUPPORTED;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)num_kv_heads, (unsigned)n_qblocks, (unsigned)batch);
  const float scale_log2 = scale * kLog2e;
#define QMI_PREFILL_CASE(GG)                                                                      \
  case GG:                                                                                        \
    hipLaunchKernelGGL(varlen_prefill_kernel<GG>, grid, dim3(kThreads), 0, s, q, q_tok_stride,   \
                       q_head_stride, k_cache, v_cache, num_blocks, (int)num_kv_heads,            \
                       cu_seqlens_q, cu_seqlens_k, block_table, bt_stride, (int)bt_width,         \
                       (int)n_qblocks, total_q, scale_log2, out, out_tok_stride,                  \
                       out_head_stride);                                                          \
    break;
  switch (G) {
    QMI_PREFILL_CASE(1)
    QMI_PREFILL_CASE(2)
    QMI_PREFILL_CASE(4)
    default:
      return QMI_E_UNSUPPORTED;
  }
#undef QMI_PREFILL_CASE
  QMI_RETURN_LAUNCH_STATUS();
}
