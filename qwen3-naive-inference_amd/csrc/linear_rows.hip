// Decode-batch projections on bf16 MFMA (gfx950): y = x W^T for at most 256
// rows.
//
// Reference semantics: the bf16 nn.Linear projections of a decode step —
// Qwen3Attention.qkv_proj / o_proj (qwen3_naive.py:427-428, :654, :683) and
// Qwen3MLP.gate_up_proj, silu(gate) * up, down_proj (qwen3_naive.py:692-702)
// — with fp32 accumulation and one bf16 rounding of each output, as the
// library GEMM of the reference does.
//
// At decode batch (64-256 rows) these products stream the weight matrix once
// per step and are bound by HBM and by latency: a library GEMM picks tiles for
// large M.  Here:
//   * Workgroup = 4 waves = a tile of 64 rows x NT output columns; wave w
//     takes rows 16 w .. +15 and all NT columns.  K goes through an
//     NSTAGE-deep LDS ring in 128-element chunks (256-byte rows, 16-byte
//     chunks XOR-swizzled by row % 16, conflict-free operand reads), filled
//     by gfx950 direct global->LDS loads (global_load_lds_dwordx4, issued as
//     inline asm NSTAGE-1 chunks ahead; one explicit s_waitcnt vmcnt per
//     chunk).  Rows past M load row M-1 and are never stored.
//   * v_mfma_f32_16x16x32_bf16 with the weight rows as the A operand and the
//     x rows as B, so a lane holds 4 consecutive output columns of one row
//     (8-byte bf16 / 16-byte fp32 stores).
//   * Epilogues: plain bf16; SwiGLU for the packed gate/up weight ([gate;
//     up], 2 I rows): a tile loads NT/2 gate rows and the NT/2 matching up
//     rows and writes silu(bf16(g)) * bf16(u) rounded once (the rounding
//     points of a bf16 GEMM followed by silu_mul); fp32 split-K partials
//     part[s][M][N] for the narrow projections (o_proj, down: N = hidden), so
//     that a few rows still give ~256 workgroups — the residual add + RMSNorm
//     that follows sums them (qmi_add_rms_norm_parts) instead of a separate
//     reduction.
#include <algorithm>

#include "qmi_common.h"

namespace {

using namespace qmi;

constexpr int kThreads = 256;
constexpr int kKC = 128;        // K elements per chunk
constexpr int kRowB = kKC * 2;  // bytes per staged row
constexpr int kMaxRows = 256;

typedef __attribute__((ext_vector_type(4))) unsigned int u4v_t;

__device__ __forceinline__ void lds_load16(const void* gbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               : : "s"(lds), "v"(voff), "s"(gbase) : "memory", "m0");
}

__device__ __forceinline__ u4v_t ds_read16(uint32_t addr) {
  u4v_t r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr) : "memory");
  return r;
}

enum Epi { kPlain = 0, kSwiGLU = 1, kParts = 2 };

// NT: weight rows per tile (output columns; NT / 2 for SwiGLU).
template <int NT, int NSTAGE, int EPI>
__global__ __launch_bounds__(kThreads) void linear_rows_kernel(
    const uint16_t* __restrict__ x, int64_t x_stride, const uint16_t* __restrict__ w,
    int64_t w_stride, uint16_t* __restrict__ y, int64_t y_stride, float* __restrict__ part,
    int M, int N, int K, int S) {
  constexpr int XB = 64 * kRowB, WB = NT * kRowB, SB = XB + WB;
  constexpr int WPW = NT / 16;  // weight wave-loads (4 rows each) per wave per chunk
  constexpr int LPW = 4 + WPW;  // loads per wave per chunk
  constexpr int NB = NT / 16;   // 16-column MFMA blocks
  constexpr int OUT = EPI == kSwiGLU ? NT / 2 : NT;  // output columns per tile
  __shared__ __attribute__((aligned(16))) char lds[NSTAGE * SB];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_nt = N / OUT;
  int bid = blockIdx.x;
  const int s = bid % S;
  bid /= S;
  const int nt = bid % n_nt, mt = bid / n_nt;
  const int m0 = mt * 64, n0 = nt * OUT;
  const int nkc = K / kKC;
  const int kc0 = s * nkc / S, kc1 = (s + 1) * nkc / S, nk = kc1 - kc0;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
  // Wave-load j (1 KB) covers staged rows 4j .. 4j+3: lane l fetches row
  // 4j + l/16, physical chunk l%16, i.e. logical chunk (l%16) ^ (row%16).
  const int lrow = lane >> 4, pch = lane & 15;
  uint32_t xoff[4], woff[WPW];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 16 * wave + 4 * i + lrow;
    const int row = min(m0 + r, M - 1);
    xoff[i] = (uint32_t)((row * x_stride + (pch ^ (r & 15)) * 8) * 2);
  }
#pragma unroll
  for (int i = 0; i < WPW; ++i) {
    const int r = 4 * (WPW * wave + i) + lrow;
    // SwiGLU: staged rows 0 .. NT/2-1 are gate rows, the rest the matching up rows.
    const int wrow = EPI == kSwiGLU ? (r < NT / 2 ? n0 + r : N + n0 + r - NT / 2) : n0 + r;
    woff[i] = (uint32_t)((wrow * w_stride + (pch ^ (r & 15)) * 8) * 2);
  }
  auto issue = [&](int kc, int st) {
    const uint32_t sb = lds0 + st * SB;
    const char* xb = reinterpret_cast<const char*>(x) + (int64_t)kc * kRowB;
    const char* wb = reinterpret_cast<const char*>(w) + (int64_t)kc * kRowB;
#pragma unroll
    for (int i = 0; i < 4; ++i) lds_load16(xb, xoff[i], sb + (4 * wave + i) * 1024);
#pragma unroll
    for (int i = 0; i < WPW; ++i) lds_load16(wb, woff[i], sb + XB + (WPW * wave + i) * 1024);
  };
  const int l16 = lane & 15, g4 = lane >> 4;
  // Operand (staged row r, k-step ks): logical chunk c = 4 ks + g4 at physical c ^ (r % 16).
  uint32_t x_rd[4], w_rd[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int c = 4 * ks + g4;
    x_rd[ks] = (uint32_t)((16 * wave + l16) * kRowB + 16 * (c ^ l16));
    w_rd[ks] = (uint32_t)(XB + l16 * kRowB + 16 * (c ^ l16));
  }
  f32x4_t acc[NB];  // acc[b]: weight rows 16 b + 4 g4 + r, x row 16 wave + l16
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < NSTAGE - 1; ++st) issue(kc0 + min(st, nk - 1), st);
  for (int k = 0; k < nk; ++k) {
    const int st = k % NSTAGE;
    // Chunk k has landed once at most the later NSTAGE - 2 chunks' loads are
    // outstanding; the barrier also retires every wave's reads of the slot
    // that the next issue overwrites (chunk k - 1).
    asm volatile("s_waitcnt vmcnt(%0)" ::"i"((NSTAGE - 2) * LPW) : "memory");
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue(kc0 + min(k + NSTAGE - 1, nk - 1), (k + NSTAGE - 1) % NSTAGE);
    const uint32_t base = lds0 + st * SB;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u4v_t a = ds_read16(base + x_rd[ks]);
      u4v_t bv[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) bv[b] = ds_read16(base + w_rd[ks] + b * 16 * kRowB);
      if constexpr (NB == 1)
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(bv[0]) :: "memory");
      else if constexpr (NB == 2)
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(bv[0]), "+v"(bv[1]) :: "memory");
      else
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(a), "+v"(bv[0]), "+v"(bv[1]), "+v"(bv[2]), "+v"(bv[3]) :: "memory");
#pragma unroll
      for (int b = 0; b < NB; ++b)
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, bv[b]),
                                                         __builtin_bit_cast(bf16x8_t, a), acc[b],
                                                         0, 0, 0);
    }
  }
  // The ring's last loads (re-issues of the final chunk) are drained before exit.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const int row = m0 + 16 * wave + l16;
  if (row >= M) return;
  if constexpr (EPI == kPlain) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int col = n0 + 16 * b + 4 * g4;
      *reinterpret_cast<uint2*>(y + (int64_t)row * y_stride + col) =
          make_uint2(pack_bf16x2(acc[b][0], acc[b][1]), pack_bf16x2(acc[b][2], acc[b][3]));
    }
  } else if constexpr (EPI == kSwiGLU) {
#pragma unroll
    for (int b = 0; b < NB / 2; ++b) {
      const int col = n0 + 16 * b + 4 * g4;
      float o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float g = bf16_to_f32(f32_to_bf16(acc[b][r]));
        const float u = bf16_to_f32(f32_to_bf16(acc[b + NB / 2][r]));
        o[r] = g / (1.0f + __expf(-g)) * u;
      }
      *reinterpret_cast<uint2*>(y + (int64_t)row * y_stride + col) =
          make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
    }
  } else {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int col = n0 + 16 * b + 4 * g4;
      *reinterpret_cast<f32x4_t*>(part + ((int64_t)s * M + row) * N + col) = acc[b];
    }
  }
}

// out = rms_norm(bf16(sum_s part[s]) + residual) with the residual sum
// written back, one workgroup of 128 lanes per row (as rms_norm_rows<true>).
constexpr int kNormThreads = 128;
constexpr int kNormVec = 4;  // 8-element chunks per lane: n <= 4096

template <int S>
__global__ __launch_bounds__(kNormThreads) void add_rms_norm_parts_kernel(
    const float* __restrict__ part, int64_t M, const uint16_t* __restrict__ res_in,
    int64_t res_in_stride, uint16_t* __restrict__ res_out, int64_t res_out_stride,
    const uint16_t* __restrict__ wgt, uint16_t* __restrict__ y, int64_t y_stride, int n,
    float eps) {
  __shared__ float sm[kNormThreads / 64];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int nvec = n >> 3;
  float v[kNormVec][8];
  uint4 wv[kNormVec];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kNormVec; ++k) {
    const int c = tid + k * kNormThreads;
    if (c < nvec) {
      wv[k] = load_u4(wgt + 8 * c);
      const float* p = part + row * n + 8 * c;
      // All parts' loads go out together (S is a compile-time count), then
      // they are summed in part order.
      f32x4_t pa[S], pb[S];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        pa[s] = *reinterpret_cast<const f32x4_t*>(p + (int64_t)s * M * n);
        pb[s] = *reinterpret_cast<const f32x4_t*>(p + (int64_t)s * M * n + 4);
      }
      f32x4_t a0 = pa[0], a1 = pb[0];
#pragma unroll
      for (int s = 1; s < S; ++s) {
        a0 += pa[s];
        a1 += pb[s];
      }
      const uint4 r = load_u4(res_in + row * res_in_stride + 8 * c);
      const uint32_t rw[4] = {r.x, r.y, r.z, r.w};
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // The projection's output is bf16 (one rounding), then added in fp32.
        const float x0 = bf16_to_f32(f32_to_bf16(e < 2 ? a0[2 * e] : a1[2 * e - 4]));
        const float x1 = bf16_to_f32(f32_to_bf16(e < 2 ? a0[2 * e + 1] : a1[2 * e - 3]));
        v[k][2 * e] = x0 + bf16_lo(rw[e]);
        v[k][2 * e + 1] = x1 + bf16_hi(rw[e]);
        o[e] = pack_bf16x2(v[k][2 * e], v[k][2 * e + 1]);
      }
      *reinterpret_cast<uint4*>(res_out + row * res_out_stride + 8 * c) =
          make_uint4(o[0], o[1], o[2], o[3]);
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
  for (int k = 0; k < kNormVec; ++k) {
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

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool al8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

// Tile choice, by the number of 64-row tiles (measured on the Qwen3-0.6B
// shapes in HIP graphs of 28 layers): one row tile — 16 weight rows per tile
// (32 for SwiGLU: 16 gate + 16 up), which alone gives ~256 workgroups; two —
// 32 (64); more — 64 weight rows, so that the activations are re-read
// through L2 by fewer column tiles.  The K split of the partial products
// fills ~256 workgroups (1, 2, 4 or 8 parts).
struct Cfg {
  int nt, ns, s;
};

Cfg pick(int64_t m, int64_t n, int64_t k, int epi) {
  const int64_t n_mt = (m + 63) / 64;
  Cfg c{16, 4, 1};
  if (epi == kSwiGLU) {
    c = n_mt == 1 ? Cfg{32, 3, 1} : n_mt == 2 ? Cfg{64, 3, 1} : Cfg{64, 2, 1};
    if (n % (c.nt / 2)) c = Cfg{32, 3, 1};
  } else if (epi == kPlain) {
    c = n_mt == 1 ? Cfg{16, 4, 1} : n_mt == 2 ? Cfg{32, 3, 1} : Cfg{64, 3, 1};
    if (n % c.nt) c = Cfg{16, 4, 1};
  } else {
    // Split-K partials: 32 weight rows per tile at one row tile (8 parts at
    // the Qwen3 o / down shapes, 256 workgroups), 16 at two; from three row
    // tiles 32 rows (two parts) for K <= 2048 and 64 rows (four parts) above
    // — fewer parts also mean fewer partial bytes for the norm that sums them
    // (o_proj / down at 256 rows: 6.4 -> 5.6 / 8.4 -> 7.4 us; at 64 rows
    // 3.9 -> 3.8 / 4.7 -> 4.4 us).
    c = n_mt == 2 ? Cfg{16, 4, 1} : (n_mt >= 3 && k > 2048) ? Cfg{64, 3, 1} : Cfg{32, 4, 1};
    if (n % c.nt) c = Cfg{16, 4, 1};
    const int64_t tiles = n_mt * (n / c.nt);
    const int64_t want = std::max<int64_t>(1, std::min<int64_t>({256 / tiles, 8, k / kKC}));
    c.s = want >= 8 ? 8 : want >= 4 ? 4 : want >= 2 ? 2 : 1;
  }
  return c;
}

int check_args(const void* x, int64_t x_stride, const void* w, int64_t w_stride, int64_t m,
               int64_t n, int64_t k) {
  if (m < 0 || n <= 0 || k <= 0) return QMI_E_BAD_SHAPE;
  if (!x || !w) return QMI_E_NULL_POINTER;
  if (m > kMaxRows || k % kKC || n % 16 || n > (1 << 20) || k > (1 << 20))
    return QMI_E_UNSUPPORTED;
  if (x_stride < k || w_stride < k || x_stride % 8 || w_stride % 8 || !al16(x) || !al16(w))
    return QMI_E_BAD_STRIDE;
  // Load offsets are 32-bit byte offsets from the chunk base (2 n weight rows for SwiGLU).
  if (4 * n * w_stride >= (1LL << 32) || 2 * m * x_stride >= (1LL << 32)) return QMI_E_UNSUPPORTED;
  return QMI_OK;
}

template <int EPI>
int launch(const uint16_t* x, int64_t x_stride, const uint16_t* w, int64_t w_stride, uint16_t* y,
           int64_t y_stride, float* part, int64_t m, int64_t n, int64_t k, const Cfg& c,
           hipStream_t st) {
  const int out = EPI == kSwiGLU ? c.nt / 2 : c.nt;
  if (n % out) return QMI_E_UNSUPPORTED;
  const unsigned grid = (unsigned)(((m + 63) / 64) * (n / out) * c.s);
#define QMI_LR(NT, NS)                                                                           \
  if (c.nt == NT && c.ns == NS) {                                                                \
    hipLaunchKernelGGL((linear_rows_kernel<NT, NS, EPI>), dim3(grid), dim3(kThreads), 0, st, x,  \
                       x_stride, w, w_stride, y, y_stride, part, (int)m, (int)n, (int)k, c.s);   \
    return QMI_OK;                                                                                \
  }
  if constexpr (EPI == kSwiGLU) {
    QMI_LR(32, 3)
    QMI_LR(64, 3)
    QMI_LR(64, 2)
  } else if constexpr (EPI == kPlain) {
    QMI_LR(16, 4)
    QMI_LR(32, 3)
    QMI_LR(64, 3)
  } else {
    QMI_LR(16, 4)
    QMI_LR(32, 4)
    QMI_LR(64, 3)
  }
#undef QMI_LR
  return QMI_E_UNSUPPORTED;
}

}  // namespace

extern "C" int qmi_linear_rows(const uint16_t* x, int64_t x_stride, const uint16_t* w,
                               int64_t w_stride, int64_t m, int64_t n, int64_t k,
                               int32_t activation, uint16_t* y, int64_t y_stride, void* stream) {
  int e = check_args(x, x_stride, w, w_stride, m, n, k);
  if (e != QMI_OK) return e;
  if (activation != kPlain && activation != kSwiGLU) return QMI_E_BAD_SHAPE;
  if (m == 0) return QMI_OK;
  if (!y) return QMI_E_NULL_POINTER;
  if (y_stride < n || y_stride % 4 || !al8(y)) return QMI_E_BAD_STRIDE;
  const Cfg c = pick(m, n, k, activation);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  e = activation == kSwiGLU
          ? launch<kSwiGLU>(x, x_stride, w, w_stride, y, y_stride, nullptr, m, n, k, c, st)
          : launch<kPlain>(x, x_stride, w, w_stride, y, y_stride, nullptr, m, n, k, c, st);
  if (e != QMI_OK) return e;
  QMI_RETURN_LAUNCH_STATUS();
}

extern "C" int64_t qmi_linear_rows_parts_count(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || m > kMaxRows || n <= 0 || n % 16 || k <= 0 || k % kKC) return 0;
  return pick(m, n, k, kParts).s;
}

extern "C" int qmi_linear_rows_parts(const uint16_t* x, int64_t x_stride, const uint16_t* w,
                                     int64_t w_stride, int64_t m, int64_t n, int64_t k,
                                     float* parts, int64_t n_parts, void* stream) {
  int e = check_args(x, x_stride, w, w_stride, m, n, k);
  if (e != QMI_OK) return e;
  if (m == 0) return QMI_OK;
  if (!parts) return QMI_E_NULL_POINTER;
  if (!al16(parts)) return QMI_E_BAD_STRIDE;
  const Cfg c = pick(m, n, k, kParts);
  if (n_parts != c.s) return QMI_E_BAD_SHAPE;
  e = launch<kParts>(x, x_stride, w, w_stride, nullptr, 0, parts, m, n, k, c,
                     reinterpret_cast<hipStream_t>(stream));
  if (e != QMI_OK) return e;
  QMI_RETURN_LAUNCH_STATUS();
}

extern "C" int qmi_add_rms_norm_parts(const float* parts, int64_t n_parts, int64_t m,
                                      const uint16_t* residual, int64_t residual_stride,
                                      uint16_t* residual_out, int64_t residual_out_stride,
                                      const uint16_t* weight, uint16_t* y, int64_t y_stride,
                                      int64_t n, float eps, void* stream) {
  if (m < 0 || n <= 0 || n_parts <= 0) return QMI_E_BAD_SHAPE;
  if (m == 0) return QMI_OK;
  if (!parts || !residual || !residual_out || !weight || !y) return QMI_E_NULL_POINTER;
  if (n % 8 || n > 8 * kNormThreads * kNormVec || m > 0x7fffffffLL ||
      (n_parts != 1 && n_parts != 2 && n_parts != 4 && n_parts != 8))
    return QMI_E_UNSUPPORTED;
  if (residual_stride % 8 || residual_out_stride % 8 || y_stride % 8 || !al16(parts) ||
      !al16(residual) || !al16(residual_out) || !al16(y) || !al16(weight))
    return QMI_E_BAD_STRIDE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define QMI_NP(SS)                                                                             \
  case SS:                                                                                     \
    hipLaunchKernelGGL(add_rms_norm_parts_kernel<SS>, dim3((unsigned)m), dim3(kNormThreads), 0, \
                       st, parts, m, residual, residual_stride, residual_out,                   \
                       residual_out_stride, weight, y, y_stride, (int)n, eps);                  \
    break;
  switch (n_parts) {
    QMI_NP(1)
    QMI_NP(2)
    QMI_NP(4)
    QMI_NP(8)
  }
#undef QMI_NP
  QMI_RETURN_LAUNCH_STATUS();
}
