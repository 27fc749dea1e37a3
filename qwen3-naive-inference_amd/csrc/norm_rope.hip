// Row-wise RMSNorm, fused residual-add + RMSNorm, fused per-head
// QK-RMSNorm + RoPE, and the SwiGLU activation product (gfx950).
//
// Reference semantics (qwen3_naive.py):
//   RMSNorm._rms_norm      :156-161  y = bf16(fp32(x) * rsqrt(mean(x^2) + eps) * w)
//   RMSNorm._add_rms_norm  :163-169  s = fp32(x) + fp32(res); res' = bf16(s);
//                                    y = bf16(s * rsqrt(mean(s^2) + eps) * w)
//   q_norm / k_norm        :431-432, :661-662  the same RMSNorm per head over D = 128
//   _apply_rope_kernel     :44-67    half-split pairs (j, j+64) with fp32 cos/sin:
//                                    o1 = x1*c - x2*s, o2 = x2*c + x1*s
//   RotaryEmbedding cache  :383-387  cache[pos] = [cos(pos*f_i), sin(pos*f_i)]
//   Qwen3MLP               :695-702  silu(gate) * up
// RMSNorm / MLP run under torch.compile in the reference, whose generated
// code keeps the elementwise chain in fp32 and rounds once at the end; these
// kernels do the same.  The reference rounds the QK-norm output to bf16 before RoPE reads it
// (separate kernels); the fused kernel keeps that rounding point so results
// match the two-step reference bit for bit up to the fp32 math order.
//
// All kernels are HBM-bound elementwise/row passes: one wave64 per row or
// head-row, 16-byte accesses where the row length allows.
#include "qmi_common.h"

namespace {

using namespace qmi;

// ---------------------------------------------------------------------------
// RMSNorm over rows of `n` elements (n % 8 == 0, n <= 8 * 64 * kMaxVec).
constexpr int kNormThreads = 128;  // 2 waves per row
constexpr int kMaxVec = 4;         // 16-byte chunks per lane -> n <= 4096

template <bool ADD>
__global__ __launch_bounds__(kNormThreads) void rms_norm_rows(
    const uint16_t* __restrict__ x, int64_t x_stride, const uint16_t* __restrict__ res_in,
    int64_t res_in_stride, uint16_t* __restrict__ res_out, int64_t res_out_stride,
    const uint16_t* __restrict__ w, uint16_t* __restrict__ y, int64_t y_stride, int64_t n_rows,
    int n, float eps) {
  __shared__ float sm[kNormThreads / 64];
  const int64_t row = blockIdx.x;
  if (row >= n_rows) return;
  const int tid = threadIdx.x;
  const int nvec = n >> 3;
  float v[kMaxVec][8];
  uint4 wv[kMaxVec];  // weight chunks, loaded with the row so the tail has no dependent load
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxVec; ++k) {
    const int c = tid + k * kNormThreads;
    if (c < nvec) {
      wv[k] = load_u4(w + 8 * c);
      const uint4 a = load_u4(x + row * x_stride + 8 * c);
      const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[k][2 * e] = bf16_lo(aw[e]);
        v[k][2 * e + 1] = bf16_hi(aw[e]);
      }
      if (ADD) {
        const uint4 r = load_u4(res_in + row * res_in_stride + 8 * c);
        const uint32_t rw[4] = {r.x, r.y, r.z, r.w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[k][2 * e] += bf16_lo(rw[e]);
          v[k][2 * e + 1] += bf16_hi(rw[e]);
          o[e] = pack_bf16x2(v[k][2 * e], v[k][2 * e + 1]);
        }
        *reinterpret_cast<uint4*>(res_out + row * res_out_stride + 8 * c) =
            make_uint4(o[0], o[1], o[2], o[3]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[k][e] * v[k][e];
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) sm[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += sm[i];
  const float inv = rsqrtf(tot / (float)n + eps);
#pragma unroll
  for (int k = 0; k < kMaxVec; ++k) {
    const int c = tid + k * kNormThreads;
    if (c < nvec) {
      const uint32_t ww[4] = {wv[k].x, wv[k].y, wv[k].z, wv[k].w};
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = pack_bf16x2(v[k][2 * e] * inv * bf16_lo(ww[e]),
                           v[k][2 * e + 1] * inv * bf16_hi(ww[e]));
      *reinterpret_cast<uint4*>(y + row * y_stride + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

// ---------------------------------------------------------------------------
// Fused per-head RMSNorm + RoPE for q and k of a fused qkv row.
// 16 lanes per (token, head) item, four items per wave: lane s of an item owns
// the RoPE pairs (4s + i, 64 + 4s + i), i < 4, read and written 8 bytes at a
// time (cos / sin 16 bytes); the sum of squares stays inside the item's DPP
// row of 16 lanes.  k goes to k_out (when given) and, with the caches given,
// the rotated k and the token's v head (16 bytes per lane) go straight to
// cache row slots[tok] (slots outside [0, n_slots) are skipped, as in the KV
// store).
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const uint16_t* __restrict__ qkv, int64_t qkv_stride, int n_q_heads, int n_kv_heads,
    const uint16_t* __restrict__ q_w, const uint16_t* __restrict__ k_w,
    const int64_t* __restrict__ positions, const float* __restrict__ cos_sin,
    int64_t max_pos, uint16_t* __restrict__ q_out, int64_t q_stride,
    uint16_t* __restrict__ k_out, int64_t k_stride, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache, const int32_t* __restrict__ slots, int64_t n_slots,
    int64_t n_tok, float eps) {
  constexpr int D = 128, HALF = 64;
  const int sub = threadIdx.x & 15;
  const int64_t item = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int heads = n_q_heads + n_kv_heads;
  if (item >= n_tok * heads) return;  // whole 16-lane rows only
  const int64_t tok = item / heads;
  const int h = (int)(item - tok * heads);
  const bool is_q = h < n_q_heads;
  // Every load is issued before the reduction: position -> cos/sin is the
  // only dependent pair.
  int64_t pos = positions[tok];
  const uint16_t* src = qkv + tok * qkv_stride + (int64_t)h * D;
  const uint16_t* w = is_q ? q_w : k_w;
  const uint2 xa = *reinterpret_cast<const uint2*>(src + 4 * sub);
  const uint2 xb = *reinterpret_cast<const uint2*>(src + HALF + 4 * sub);
  const uint2 wa = *reinterpret_cast<const uint2*>(w + 4 * sub);
  const uint2 wb = *reinterpret_cast<const uint2*>(w + HALF + 4 * sub);
  pos = pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
  const float4 c = *reinterpret_cast<const float4*>(cos_sin + pos * D + 4 * sub);
  const float4 sn = *reinterpret_cast<const float4*>(cos_sin + pos * D + HALF + 4 * sub);
  const float x1[4] = {bf16_lo(xa.x), bf16_hi(xa.x), bf16_lo(xa.y), bf16_hi(xa.y)};
  const float x2[4] = {bf16_lo(xb.x), bf16_hi(xb.x), bf16_lo(xb.y), bf16_hi(xb.y)};
  const float w1[4] = {bf16_lo(wa.x), bf16_hi(wa.x), bf16_lo(wa.y), bf16_hi(wa.y)};
  const float w2[4] = {bf16_lo(wb.x), bf16_hi(wb.x), bf16_lo(wb.y), bf16_hi(wb.y)};
  const float cc[4] = {c.x, c.y, c.z, c.w}, ss4[4] = {sn.x, sn.y, sn.z, sn.w};
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) ss += x1[i] * x1[i] + x2[i] * x2[i];
  ss = row16_sum(ss);
  const float inv = rsqrtf(ss / (float)D + eps);
  float o1[4], o2[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // QK-norm output is bf16 in the reference before RoPE reads it.
    const float n1 = bf16_to_f32(f32_to_bf16(x1[i] * inv * w1[i]));
    const float n2 = bf16_to_f32(f32_to_bf16(x2[i] * inv * w2[i]));
    o1[i] = n1 * cc[i] - n2 * ss4[i];
    o2[i] = n2 * cc[i] + n1 * ss4[i];
  }
  const uint2 ba = make_uint2(pack_bf16x2(o1[0], o1[1]), pack_bf16x2(o1[2], o1[3]));
  const uint2 bb = make_uint2(pack_bf16x2(o2[0], o2[1]), pack_bf16x2(o2[2], o2[3]));
  if (is_q) {
    uint16_t* dst = q_out + tok * q_stride + (int64_t)h * D;
    *reinterpret_cast<uint2*>(dst + 4 * sub) = ba;
    *reinterpret_cast<uint2*>(dst + HALF + 4 * sub) = bb;
    return;
  }
  const int hk = h - n_q_heads;
  if (k_out) {
    uint16_t* dst = k_out + tok * k_stride + (int64_t)hk * D;
    *reinterpret_cast<uint2*>(dst + 4 * sub) = ba;
    *reinterpret_cast<uint2*>(dst + HALF + 4 * sub) = bb;
  }
  if (k_cache) {
    const int64_t slot = slots[tok];
    if (slot >= 0 && slot < n_slots) {
      const int64_t row = slot * n_kv_heads * D + (int64_t)hk * D;
      // Cache rows are written non-temporally, as in the KV store.
      typedef __attribute__((ext_vector_type(2))) unsigned int u32x2_t;
      __builtin_nontemporal_store(u32x2_t{ba.x, ba.y}, reinterpret_cast<u32x2_t*>(k_cache + row + 4 * sub));
      __builtin_nontemporal_store(u32x2_t{bb.x, bb.y}, reinterpret_cast<u32x2_t*>(k_cache + row + HALF + 4 * sub));
      const uint16_t* vsrc = qkv + tok * qkv_stride + (int64_t)(n_q_heads + n_kv_heads + hk) * D;
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4_t*>(vsrc + 8 * sub),
                                  reinterpret_cast<u32x4_t*>(v_cache + row + 8 * sub));
    }
  }
}

// ---------------------------------------------------------------------------
// out[r, j] = silu(gu[r, j]) * gu[r, inter + j] for j < inter (bf16 in/out,
// fp32 math), the activation of Qwen3MLP on the fused gate_up output.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu,
                                                       int64_t gu_stride, int inter,
                                                       uint16_t* __restrict__ out,
                                                       int64_t out_stride, int64_t n_rows) {
  const int nvec = inter >> 3;
  const int64_t total = n_rows * nvec;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / nvec;
    const int c = (int)(i - r * nvec);
    const uint4 g = load_u4(gu + r * gu_stride + 8 * c);
    const uint4 u = load_u4(gu + r * gu_stride + inter + 8 * c);
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float g0 = bf16_lo(gw[e]), g1 = bf16_hi(gw[e]);
      const float a0 = g0 / (1.0f + __expf(-g0)) * bf16_lo(uw[e]);
      const float a1 = g1 / (1.0f + __expf(-g1)) * bf16_hi(uw[e]);
      o[e] = pack_bf16x2(a0, a1);
    }
    *reinterpret_cast<uint4*>(out + r * out_stride + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool al8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

}  // namespace

extern "C" int qmi_rms_norm(const uint16_t* x, int64_t x_stride, const uint16_t* weight, uint16_t* y,
                            int64_t y_stride, int64_t n_rows, int64_t n, float eps,
                            void* stream) {
  if (n_rows < 0 || n <= 0) return QMI_E_BAD_SHAPE;
  if (n_rows == 0) return QMI_OK;
  if (!x || !weight || !y) return QMI_E_NULL_POINTER;
  if (n % 8 || n > 8 * kNormThreads * kMaxVec || n_rows > 0x7fffffffLL) return QMI_E_UNSUPPORTED;
  if (x_stride % 8 || y_stride % 8 || !al16(x) || !al16(y)) return QMI_E_BAD_STRIDE;
  hipLaunchKernelGGL(rms_norm_rows<false>, dim3((unsigned)n_rows), dim3(kNormThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), x, x_stride, nullptr, 0, nullptr, 0,
                     weight, y, y_stride, n_rows, (int)n, eps);
  QMI_RETURN_LAUNCH_STATUS();
}

extern "C" int qmi_add_rms_norm(const uint16_t* x, int64_t x_stride, const uint16_t* residual,
                                int64_t residual_stride, uint16_t* residual_out,
                                int64_t residual_out_stride, const uint16_t* weight, uint16_t* y,
                                int64_t y_stride, int64_t n_rows, int64_t n, float eps,
                                void* stream) {
  if (n_rows < 0 || n <= 0) return QMI_E_BAD_SHAPE;
  if (n_rows == 0) return QMI_OK;
  if (!x || !residual || !residual_out || !weight || !y) return QMI_E_NULL_POINTER;
  if (n % 8 || n > 8 * kNormThreads * kMaxVec || n_rows > 0x7fffffffLL) return QMI_E_UNSUPPORTED;
  if (x_stride % 8 || y_stride % 8 || residual_stride % 8 || residual_out_stride % 8 || !al16(x) ||
      !al16(y) || !al16(residual) || !al16(residual_out))
    return QMI_E_BAD_STRIDE;
  hipLaunchKernelGGL(rms_norm_rows<true>, dim3((unsigned)n_rows), dim3(kNormThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), x, x_stride, residual, residual_stride,
                     residual_out, residual_out_stride, weight, y, y_stride, n_rows, (int)n, eps);
  QMI_RETURN_LAUNCH_STATUS();
}

extern "C" int qmi_qk_norm_rope(const uint16_t* qkv, int64_t qkv_stride, int64_t n_tok,
                                int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                const uint16_t* q_norm_weight, const uint16_t* k_norm_weight,
                                const int64_t* positions, const float* cos_sin_cache,
                                int64_t max_position, uint16_t* q_out, int64_t q_stride,
                                uint16_t* k_out, int64_t k_stride, float eps, void* stream) {
  if (n_tok < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_position <= 0)
    return QMI_E_BAD_SHAPE;
  if (n_tok == 0) return QMI_OK;
  if (!qkv || !q_norm_weight || !k_norm_weight || !positions || !cos_sin_cache || !q_out || !k_out)
    return QMI_E_NULL_POINTER;
  if (head_dim != 128) return QMI_E_UNSUPPORTED;
  if (qkv_stride < (num_q_heads + 2 * num_kv_heads) * head_dim || q_stride < num_q_heads * 128 ||
      k_stride < num_kv_heads * 128)
    return QMI_E_BAD_STRIDE;
  if (qkv_stride % 8 || q_stride % 4 || k_stride % 4 || !al16(qkv) || !al8(q_out) || !al8(k_out) ||
      !al16(cos_sin_cache) || !al8(q_norm_weight) || !al8(k_norm_weight))
    return QMI_E_BAD_STRIDE;
  const int64_t items = n_tok * (num_q_heads + num_kv_heads);
  if ((items + 15) / 16 > 0x7fffffffLL) return QMI_E_UNSUPPORTED;
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned)((items + 15) / 16)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), qkv, qkv_stride, (int)num_q_heads,
                     (int)num_kv_heads, q_norm_weight, k_norm_weight, positions, cos_sin_cache,
                     max_position, q_out, q_stride, k_out, k_stride, nullptr, nullptr, nullptr,
                     (int64_t)0, n_tok, eps);
  QMI_RETURN_LAUNCH_STATUS();
}

extern "C" int qmi_qk_norm_rope_store(
    const uint16_t* qkv, int64_t qkv_stride, int64_t n_tok, int64_t num_q_heads,
    int64_t num_kv_heads, int64_t head_dim, const uint16_t* q_norm_weight,
    const uint16_t* k_norm_weight, const int64_t* positions, const float* cos_sin_cache,
    int64_t max_position, uint16_t* q_out, int64_t q_stride, uint16_t* k_cache,
    uint16_t* v_cache, const int32_t* slot_mapping, int64_t n_slots, float eps, void* stream) {
  if (n_tok < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_position <= 0 || n_slots < 0)
    return QMI_E_BAD_SHAPE;
  if (n_tok == 0) return QMI_OK;
  if (!qkv || !q_norm_weight || !k_norm_weight || !positions || !cos_sin_cache || !q_out ||
      !k_cache || !v_cache || !slot_mapping)
    return QMI_E_NULL_POINTER;
  if (head_dim != 128) return QMI_E_UNSUPPORTED;
  if (num_q_heads > 4096 || num_kv_heads > 4096) return QMI_E_UNSUPPORTED;
  if (qkv_stride < (num_q_heads + 2 * num_kv_heads) * head_dim || q_stride < num_q_heads * 128)
    return QMI_E_BAD_STRIDE;
  if (qkv_stride % 8 || q_stride % 4 || !al16(qkv) || !al8(q_out) || !al16(cos_sin_cache) ||
      !al8(q_norm_weight) || !al8(k_norm_weight) || !al16(k_cache) || !al16(v_cache))
    return QMI_E_BAD_STRIDE;
  const int64_t items = n_tok * (num_q_heads + num_kv_heads);
  if ((items + 15) / 16 > 0x7fffffffLL) return QMI_E_UNSUPPORTED;
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned)((items + 15) / 16)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), qkv, qkv_stride, (int)num_q_heads,
                     (int)num_kv_heads, q_norm_weight, k_norm_weight, positions, cos_sin_cache,
                     max_position, q_out, q_stride, nullptr, (int64_t)0, k_cache, v_cache,
                     slot_mapping, n_slots, n_tok, eps);
  QMI_RETURN_LAUNCH_STATUS();
}

extern "C" int qmi_silu_mul(const uint16_t* gate_up, int64_t gate_up_stride, int64_t n_rows,
                            int64_t inter, uint16_t* out, int64_t out_stride, void* stream) {
  if (n_rows < 0 || inter <= 0) return QMI_E_BAD_SHAPE;
  if (n_rows == 0) return QMI_OK;
  if (!gate_up || !out) return QMI_E_NULL_POINTER;
  if (inter % 8 || gate_up_stride % 8 || out_stride % 8 || !al16(gate_up) || !al16(out) ||
      gate_up_stride < 2 * inter || out_stride < inter)
    return QMI_E_BAD_STRIDE;
  int64_t blocks = (n_rows * (inter / 8) + 255) / 256;
  if (blocks > 65535 * 8) blocks = 65535 * 8;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), gate_up, gate_up_stride, (int)inter,
                     out, out_stride, n_rows);
  QMI_RETURN_LAUNCH_STATUS();
}
