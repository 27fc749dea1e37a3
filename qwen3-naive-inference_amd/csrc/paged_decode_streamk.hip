// Paged GQA decode attention, balanced ("stream-K") variant for gfx950.
//
// Reference semantics: as paged_decode.hip (flash_attn_with_kvcache in
// Qwen3Attention.forward_decode, qwen3_naive.py:672-680).
//
// Work decomposition.  The keys of all sequences are cut into steps of
// 4 * (16 / Hkv) tokens (8 for 8 KV heads; a divisor of the 256-token page);
// the flattened list of steps (sequence-major) is divided evenly over a fixed
// grid of two workgroups per CU, so every workgroup streams the same number
// of K/V bytes whatever the context lengths are (ragged batches leave no
// tail of idle CUs).  Two workgroups per CU with 8 dwordx4 loads per lane in
// flight read faster than more workgroups or deeper steps: on a 28-layer
// B=64 sweep, 1024 workgroups x 16 loads ran at 5.5 TB/s, 512 x 8 at 6.15.
// A workgroup handles every KV head of its tokens: lane l owns head-dim slice
// [8*(l%16), +8) of KV head (l/16) % HKV for token group l / (16*HKV), and a
// token group owns 8 consecutive tokens of the step, so each wave-wide
// dwordx4 load reads 1 KB of a contiguous token row (all KV heads of a token
// are adjacent in the [blocks, 256, Hkv, 128] cache).  Addresses are a
// per-page scalar base plus a 32-bit lane offset, and the loads of a step are
// issued unconditionally (a step never leaves its page); tokens past the
// context are masked only in a sequence's last, partial step.
// Per 16-lane DPP row the QK partial dots (v_dot2_f32_bf16) are summed with
// DPP adds; each row keeps its own online-softmax state (fp32, log2 domain)
// for the G query heads of its KV head, so the step loop needs no barrier.
// When a workgroup leaves a sequence, the token groups are merged through
// LDS; a sequence covered entirely by one workgroup is written directly,
// otherwise the segment's (acc, m, l) go to one of the workgroup's two
// partial slots (its first and its last segment) and the merge kernel
// combines the slots of the workgroups that shared the sequence.
//
// Head-group units.  For batches of 128 or more sequences the work unit is a
// (sequence, group of HG KV heads) pair instead of a whole sequence, with HG
// the fewest heads that still give two units per workgroup slot of the GPU
// (4 of 8 heads at 256 sequences).  When the units are of nearly equal length
// (a GRPO rollout: every sequence has the same prompt length and decodes in
// lockstep), each workgroup takes exactly one whole unit ("unit mode"): no
// sequence boundary inside a workgroup, no partial slots and nothing to merge.
// Every workgroup takes that decision from the same scan of the context
// lengths (unit mode iff the longest unit is at most 10% above the balanced
// share of a workgroup), so it needs no host knowledge of the lengths and
// holds inside a captured graph; otherwise the balanced split runs over the
// units.
#include <type_traits>

#include "qmi_common.h"

namespace {

using namespace qmi;

constexpr int kHeadDim = 128;
constexpr int kPage = 256;
constexpr int kThreads = 256;
constexpr int kTok = 4;                        // tokens per lane per step
// A workgroup of 256 lanes covers 16 lanes x HG heads per token group.
template <int HG> constexpr int kTokGroups = 16 / HG;
template <int HG> constexpr int kStepTokens = kTokGroups<HG> * kTok;   // divides the page
constexpr int kSlotStride = kHeadDim + 4;      // acc[128], m, l, pad (per q head)
constexpr int kMaxSeqScan = 1024;              // batch limit of the in-LDS prefix scan

#ifndef QMI_QKV_WAVES_PER_EU
#define QMI_QKV_WAVES_PER_EU 3
#endif

// Workgroups that take part: the launch is sized from the block-table width,
// before the context lengths are known, so a short total would leave most
// workgroups with an empty range, which the merge would still have to walk
// past.  At most one workgroup per step takes part (the rest exit at once);
// longer pieces for small totals measured slower (the split loses more than
// the merge gains).
constexpr int64_t kMinWgSteps = 1;
__device__ __forceinline__ int64_t active_wgs(int64_t total, int64_t n_wg) {
  const int64_t want = (total + kMinWgSteps - 1) / kMinWgSteps;
  return want < 1 ? 1 : (want < n_wg ? want : n_wg);
}

__device__ __forceinline__ int64_t range_start(int64_t w, int64_t total, int64_t n_wg) {
  return w * total / n_wg;
}

// Workgroup owning global step s: the largest w with range_start(w) <= s.
__device__ __forceinline__ int64_t owner_of(int64_t s, int64_t total, int64_t n_wg) {
  int64_t w = ((s + 1) * n_wg - 1) / total;
  return w < n_wg - 1 ? w : n_wg - 1;
}

// Prefix sum of per-sequence step counts (steps of one unit of the sequence)
// into LDS (exclusive; off[B] = total), and the largest count into *max_steps.
// Each lane takes ceil(B / THREADS) consecutive sequences; lane sums are scanned
// inside each wave with shuffles and across waves through LDS.
//
// With `positions` given, each lane also copies its sequences' positions,
// clamped to [0, max_pos), into pos_out (LDS), so that a segment's RoPE row
// needs no dependent global load.
template <int THREADS, int TS>
__device__ void scan_steps(const int32_t* __restrict__ seqlens, int seqlen_bias, int bt_width,
                           int batch, int* off, int* max_steps,
                           const int64_t* __restrict__ positions = nullptr, int64_t max_pos = 0,
                           int* pos_out = nullptr) {
  __shared__ int wave_tot[THREADS / 64];
  __shared__ int wave_max[THREADS / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (batch + THREADS - 1) / THREADS;
  const int b0 = tid * per;
  int mine = 0, mx = 0;
  for (int i = 0; i < per; ++i) {
    const int b = b0 + i;
    if (b < batch) {
      int L = seqlens[b] + seqlen_bias;
      L = max(0, min(L, bt_width * kPage));
      if (positions) {
        const int64_t p = positions[b];
        pos_out[b] = (int)(p < 0 ? 0 : (p >= max_pos ? max_pos - 1 : p));
      }
      off[b] = mine;
      const int steps = (L + TS - 1) / TS;
      mine += steps;
      mx = max(mx, steps);
    }
  }
  int incl = mine;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int t = __shfl_up(incl, d, 64);
    if (lane >= d) incl += t;
    mx = max(mx, __shfl_xor(mx, d, 64));
  }
  if (lane == 63) wave_tot[wave] = incl;
  if (lane == 0) wave_max[wave] = mx;
  __syncthreads();
  int base = incl - mine;
  int total = 0, all_max = 0;
#pragma unroll
  for (int wv = 0; wv < THREADS / 64; ++wv) {
    if (wv < wave) base += wave_tot[wv];
    total += wave_tot[wv];
    all_max = max(all_max, wave_max[wv]);
  }
  for (int i = 0; i < per; ++i) {
    const int b = b0 + i;
    if (b < batch) off[b] += base;
  }
  if (tid == 0) {
    off[batch] = total;
    *max_steps = all_max;
  }
  __syncthreads();
}

// Unit mode: every unit is a whole workgroup's work when the longest unit is
// at most 10% above the balanced share (and there is a workgroup per unit).
__device__ __forceinline__ bool use_unit_mode(int64_t total, int max_steps, int64_t n_units,
                                              int64_t n_wg_grid, int64_t n_bal) {
  if (total == 0 || n_units > n_wg_grid) return false;
  const int64_t n_act = active_wgs(total, n_bal);
  const int64_t share = (total + n_act - 1) / n_act;
  return (int64_t)max_steps * 10 <= share * 11;
}

// Per-head QK-RMSNorm + RoPE of one lane's 8 consecutive dims d0 .. d0+7 of a
// head (d0 = 8 * (lane16)), the 16 lanes of a DPP row holding the head: the
// sum of squares is a row reduction and the RoPE partner of dim d (d < 64) is
// dim d + 64, i.e. lane16 ^ 8 (a row rotation by 8).  c / s: cos / sin of the
// token's position at the pair index d % 64.  Same expressions and rounding
// points as qk_norm_rope_kernel (norm output rounded to bf16 before RoPE).
__device__ __forceinline__ void norm_rope8(uint32_t x[4], const uint4 w, const float c[8],
                                           const float s[8], float eps, bool upper) {
  float xv[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    xv[2 * e] = bf16_lo(x[e]);
    xv[2 * e + 1] = bf16_hi(x[e]);
  }
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += xv[e] * xv[e];
  ss = row16_sum(ss);
  const float inv = rsqrtf(ss / (float)kHeadDim + eps);
  float n[8], p[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    n[2 * e] = bf16_to_f32(f32_to_bf16(xv[2 * e] * inv * bf16_lo(ww[e])));
    n[2 * e + 1] = bf16_to_f32(f32_to_bf16(xv[2 * e + 1] * inv * bf16_hi(ww[e])));
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) p[e] = dpp_f32<kDppRowRor8>(n[e]);
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = upper ? n[e] * c[e] + p[e] * s[e] : n[e] * c[e] - p[e] * s[e];
#pragma unroll
  for (int e = 0; e < 4; ++e) x[e] = pack_bf16x2(o[2 * e], o[2 * e + 1]);
}

// Inputs of the form with the QK-norm / RoPE / KV store folded in (the
// kernel's q pointer is then the packed qkv rows, head stride 128).
struct QkvArgs {
  const uint16_t* q_w;       // q_norm weight [128]
  const uint16_t* k_w;       // k_norm weight [128]
  const int64_t* positions;  // [batch]
  const float* cos_sin;      // [max_pos, 128]: cos(p f_i) at i, sin(p f_i) at 64 + i
  int64_t max_pos;
  const int32_t* slots;      // [batch]; outside [0, n_slots) skips the store
  int64_t n_slots;
  uint16_t* k_store;         // the caches, written at the new token's slot
  uint16_t* v_store;
  float eps;
};

// Grid: max(n_bal, units) workgroups.  n_bal = the balanced split's workgroup
// count (two per CU), which also indexes the partial slots; the step offsets
// and the mode word follow the slots of n_bal workgroups.
//
// QKV: q points at the packed [batch, (HQ + 2 HKV) * 128] qkv rows.  The q
// heads are normalised and rotated when a segment starts; the workgroup whose
// segment holds a unit's last step also normalises and rotates the new
// token's k heads of the unit, writes them and the v heads to cache row
// slots[b] (the lanes of token group 0), and, when slots[b] is the table slot
// of key L - 1, uses them in place of that key's loaded row — the result of
// storing first and attending afterwards, without a second launch.
template <int HKV, int G, int HG, bool QKV>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(G <= 2 ? (QKV ? QMI_QKV_WAVES_PER_EU : 4) : 2)))
void decode_streamk_split(
    const uint16_t* __restrict__ q, int64_t q_seq_stride, int64_t q_head_stride,
    const uint16_t* __restrict__ k_cache, const uint16_t* __restrict__ v_cache,
    int64_t num_blocks, const int32_t* __restrict__ seqlens, int seqlen_bias,
    const int32_t* __restrict__ block_table, int64_t bt_stride, int bt_width, int batch,
    int n_bal, float scale_log2, uint16_t* __restrict__ out, int64_t out_seq_stride,
    int64_t out_head_stride, float* __restrict__ ws, int force_units, QkvArgs qa) {
  constexpr int NHG = HKV / HG;                          // units (head groups) per sequence
  constexpr int TG = kTokGroups<HG>;
  constexpr int TS = kStepTokens<HG>;
  constexpr int HQ = HKV * G;
  constexpr int GQ = HG * G;                             // query heads of a unit
  constexpr int kRowBytes = HKV * kHeadDim * 2;          // one token of every KV head
  constexpr int64_t kPageElems = (int64_t)kPage * HKV * kHeadDim;
  __shared__ int off[kMaxSeqScan + 1];
  __shared__ int sm_max_steps;
  __shared__ float sm_acc[TG][HG][G][kHeadDim];
  __shared__ float sm_ml[TG][HG][G][2];

  const int tid = threadIdx.x;
  const int lane16 = tid & 15;
  const int hl = (tid >> 4) % HG;                        // head within the unit's group
  const int tg = tid / (16 * HG);
  const int64_t w = blockIdx.x;

  __shared__ int sm_pos[QKV ? kMaxSeqScan : 1];
  if constexpr (QKV)
    scan_steps<kThreads, TS>(seqlens, seqlen_bias, bt_width, batch, off, &sm_max_steps,
                             qa.positions, qa.max_pos, sm_pos);
  else
    scan_steps<kThreads, TS>(seqlens, seqlen_bias, bt_width, batch, off, &sm_max_steps);
  const int64_t total = (int64_t)NHG * off[batch];      // unit steps of the launch
  const int64_t n_units = (int64_t)batch * NHG;
  // Whole units are forced by the caller (no merge launch follows) or chosen
  // here when the lengths are near-equal.
  const bool unit_mode =
      force_units != 0 || use_unit_mode(total, sm_max_steps, n_units, gridDim.x, n_bal);
  if (w == 0) {  // publish the step offsets and the mode for the merge kernel
    int32_t* ws_off = reinterpret_cast<int32_t*>(ws + (int64_t)n_bal * 2 * HQ * kSlotStride);
    for (int i = tid; i <= batch; i += kThreads) ws_off[i] = off[i];
    if (tid == 0) ws_off[batch + 1] = unit_mode ? 1 : 0;
  }
  int64_t s_begin, s_end;
  if (unit_mode) {  // one whole unit per workgroup (grid >= units)
    if (w >= n_units) return;
    const int ub = (int)(w / NHG);
    const int64_t steps_b = off[ub + 1] - off[ub];
    if (steps_b == 0) {  // empty sequence attends to nothing: zeros, as flash-attn
      uint16_t* o_seq = out + (int64_t)ub * out_seq_stride;
      for (int i = tid; i < GQ * (kHeadDim / 8); i += kThreads) {
        const int qh = (int)(w % NHG) * GQ + i / (kHeadDim / 8);
        *reinterpret_cast<uint4*>(o_seq + (int64_t)qh * out_head_stride + (i % (kHeadDim / 8)) * 8) =
            make_uint4(0u, 0u, 0u, 0u);
      }
      return;
    }
    s_begin = (int64_t)NHG * off[ub] + (w % NHG) * steps_b;
    s_end = s_begin + steps_b;
  } else {
    if (total == 0) return;
    const int64_t n_act = active_wgs(total, n_bal);
    if (w >= n_act) return;
    s_begin = range_start(w, total, n_act);
    s_end = range_start(w + 1, total, n_act);
  }
  if (s_begin >= s_end) return;

  // First sequence of the range (binary search over the exclusive offsets).
  int lo = 0, hi = batch - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((int64_t)NHG * off[mid] <= s_begin) lo = mid; else hi = mid - 1;
  }

  int b = lo;
  int64_t s = s_begin;
  while (s < s_end) {
    while ((int64_t)NHG * off[b + 1] <= s) ++b;  // skip empty sequences
    const int64_t steps_b = off[b + 1] - off[b];
    const int64_t sq0 = (int64_t)NHG * off[b];
    const int hgi = (int)((s - sq0) / steps_b);   // head group of the unit
    const int64_t sb = sq0 + hgi * steps_b;       // the unit's steps: [sb, sb + steps_b)
    const int64_t seg_end = min(sb + steps_b, s_end);
    const int h = hgi * HG + hl;                  // this lane's KV head
    // Byte offset of this lane's 16 B inside a step: token group tg owns the
    // kTok consecutive tokens [tg*kTok, +kTok) of the step.
    const uint32_t lane_off = (uint32_t)(tg * kTok * kRowBytes + (h * kHeadDim + lane16 * 8) * 2);
    int L = seqlens[b] + seqlen_bias;
    L = max(0, min(L, bt_width * kPage));
    const int32_t* bt_row = block_table + (int64_t)b * bt_stride;

    uint32_t qw[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint4 v = load_u4(q + (int64_t)b * q_seq_stride +
                              (int64_t)(h * G + g) * q_head_stride + lane16 * 8);
      qw[g][0] = v.x; qw[g][1] = v.y; qw[g][2] = v.z; qw[g][3] = v.w;
    }
    // QKV: the new token's rotated k and its v (this lane's 8 dims of head
    // h), and whether key L - 1 is read from them.
    [[maybe_unused]] uint4 k_new = make_uint4(0u, 0u, 0u, 0u), v_new = make_uint4(0u, 0u, 0u, 0u);
    [[maybe_unused]] int32_t slot_new = -1;
    [[maybe_unused]] const bool last_seg = seg_end == sb + steps_b;
    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = kNegBig;
      l[g] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
    }

    // Page-table entry of the current page and the next one (prefetched so
    // the lookup at a page change does not wait on memory).
    int cur_page = (int)((s - sb) * TS / kPage);
    int32_t blk = bt_row[cur_page];
    int32_t blk_next = cur_page + 1 < bt_width ? bt_row[cur_page + 1] : -1;

    // One step of the segment.  In the form with the epilogue folded in, the
    // segment's first step (FIRST: the epilogue) and the unit's last step
    // (SUB: key L - 1 may be the new token) are peeled off the loop, so the
    // steps in between run the plain loop body.
    auto step = [&](int64_t st, auto first_c, auto sub_c) {
      const int tok0 = (int)(st - sb) * TS;               // first token of the step
      const int page = tok0 / kPage;
      if (page != cur_page) {                             // wave-uniform
        cur_page = page;
        blk = blk_next;
        blk_next = page + 1 < bt_width ? bt_row[page + 1] : -1;
      }
      const bool page_ok = blk >= 0 && blk < num_blocks;
      const int n_valid = page_ok ? min(TS, L - tok0) : 0;
      // Unmapped pages read page 0 (in bounds) and are masked below.
      const int64_t pg = page_ok ? blk : 0;
      const char* kp = reinterpret_cast<const char*>(k_cache + pg * kPageElems);
      const char* vp = reinterpret_cast<const char*>(v_cache + pg * kPageElems);
      const uint32_t o0 = (uint32_t)((tok0 % kPage) * kRowBytes) + lane_off;
      // Loads never leave the page (steps are page-aligned), so they are
      // issued unconditionally; tokens past the context are masked.
      uint4 kr[kTok], vr[kTok];
#pragma unroll
      for (int i = 0; i < kTok; ++i) kr[i] = load_u4_stream(kp + (o0 + (uint32_t)(i * kRowBytes)));
#pragma unroll
      for (int i = 0; i < kTok; ++i) vr[i] = load_u4_stream(vp + (o0 + (uint32_t)(i * kRowBytes)));
      if constexpr (QKV) {
        if constexpr (decltype(first_c)::value) {
          // The segment's first step: with its K/V loads on their way, load
          // the RoPE row (position from LDS) and the norm weights, then
          // normalise and rotate q (and the new token's k).
          const float* cs = qa.cos_sin + (int64_t)sm_pos[b] * kHeadDim + 8 * (lane16 & 7);
          const f32x4_t c0 = *reinterpret_cast<const f32x4_t*>(cs);
          const f32x4_t c1 = *reinterpret_cast<const f32x4_t*>(cs + 4);
          const f32x4_t s0 = *reinterpret_cast<const f32x4_t*>(cs + 64);
          const f32x4_t s1 = *reinterpret_cast<const f32x4_t*>(cs + 68);
          const uint4 wq = load_u4(qa.q_w + lane16 * 8);
          uint4 kraw = make_uint4(0u, 0u, 0u, 0u), wk = make_uint4(0u, 0u, 0u, 0u);
          if (last_seg) {  // wave-uniform
            const uint16_t* src = q + (int64_t)b * q_seq_stride + lane16 * 8;
            kraw = load_u4(src + (int64_t)(HQ + h) * kHeadDim);
            v_new = load_u4(src + (int64_t)(HQ + HKV + h) * kHeadDim);
            wk = load_u4(qa.k_w + lane16 * 8);
            slot_new = qa.slots[b];
          }
          const float c[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
          const float sn[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
          const bool upper = lane16 >= 8;
#pragma unroll
          for (int g = 0; g < G; ++g) norm_rope8(qw[g], wq, c, sn, qa.eps, upper);
          if (last_seg) {
            uint32_t kw4[4] = {kraw.x, kraw.y, kraw.z, kraw.w};
            norm_rope8(kw4, wk, c, sn, qa.eps, upper);
            k_new = make_uint4(kw4[0], kw4[1], kw4[2], kw4[3]);
            if (tg == 0 && slot_new >= 0 && slot_new < qa.n_slots) {
              // One token group writes the unit's heads (non-temporal, as the KV store).
              const int64_t row = ((int64_t)slot_new * HKV + h) * kHeadDim + lane16 * 8;
              __builtin_nontemporal_store(*reinterpret_cast<const u32x4_t*>(&k_new),
                                          reinterpret_cast<u32x4_t*>(qa.k_store + row));
              __builtin_nontemporal_store(*reinterpret_cast<const u32x4_t*>(&v_new),
                                          reinterpret_cast<u32x4_t*>(qa.v_store + row));
            }
          }
        }
        // Key L - 1 is the new token when this call stores it at the row the
        // table maps it to: use the computed rows instead of the loaded ones.
        if (decltype(sub_c)::value && last_seg && st == seg_end - 1 && page_ok &&
            (int64_t)slot_new == (int64_t)blk * kPage + (L - 1) % kPage) {  // wave-uniform
#pragma unroll
          for (int i = 0; i < kTok; ++i) {
            if (tok0 + tg * kTok + i == L - 1) {
              kr[i] = k_new;
              vr[i] = v_new;
            }
          }
        }
      }
      const bool partial = n_valid < TS;                 // wave-uniform
      if (partial) {
#pragma unroll
        for (int i = 0; i < kTok; ++i) {
          const bool valid = tg * kTok + i < n_valid;
          vr[i].x = valid ? vr[i].x : 0u;
          vr[i].y = valid ? vr[i].y : 0u;
          vr[i].z = valid ? vr[i].z : 0u;
          vr[i].w = valid ? vr[i].w : 0u;
        }
      }
      float sc[G][kTok];
#pragma unroll
      for (int i = 0; i < kTok; ++i) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float d = dot2_bf16(qw[g][0], kr[i].x, 0.f);
          d = dot2_bf16(qw[g][1], kr[i].y, d);
          d = dot2_bf16(qw[g][2], kr[i].z, d);
          d = dot2_bf16(qw[g][3], kr[i].w, d);
          sc[g][i] = row16_sum(d) * scale_log2;
        }
      }
      if (partial) {
#pragma unroll
        for (int i = 0; i < kTok; ++i) {
          const bool valid = tg * kTok + i < n_valid;
#pragma unroll
          for (int g = 0; g < G; ++g) sc[g][i] = valid ? sc[g][i] : -INFINITY;
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mx = sc[g][0];
#pragma unroll
        for (int i = 1; i < kTok; ++i) mx = fmaxf(mx, sc[g][i]);
        const float mn = fmaxf(m[g], mx);
        const float alpha = fast_exp2(m[g] - mn);
        m[g] = mn;
        l[g] *= alpha;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] *= alpha;
#pragma unroll
        for (int i = 0; i < kTok; ++i) {
          const float p = fast_exp2(sc[g][i] - mn);
          sc[g][i] = p;
          l[g] += p;
        }
      }
#pragma unroll
      for (int i = 0; i < kTok; ++i) {
        float v[8];
        v[0] = bf16_lo(vr[i].x); v[1] = bf16_hi(vr[i].x);
        v[2] = bf16_lo(vr[i].y); v[3] = bf16_hi(vr[i].y);
        v[4] = bf16_lo(vr[i].z); v[5] = bf16_hi(vr[i].z);
        v[6] = bf16_lo(vr[i].w); v[7] = bf16_hi(vr[i].w);
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(sc[g][i], v[e], acc[g][e]);
        }
      }
    };
    using yes = std::integral_constant<bool, true>;
    using no = std::integral_constant<bool, false>;
    if constexpr (QKV) {
      step(s, yes{}, yes{});
      const int64_t stop = last_seg ? seg_end - 1 : seg_end;
      for (int64_t st = s + 1; st < stop; ++st) step(st, no{}, no{});
      if (last_seg && seg_end - 1 > s) step(seg_end - 1, no{}, yes{});
    } else {
      for (int64_t st = s; st < seg_end; ++st) step(st, no{}, no{});
    }

    // ---- merge the token groups of this segment through LDS ----
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sm_acc[tg][hl][g][lane16 * 8 + e] = acc[g][e];
      if (lane16 == 0) {
        sm_ml[tg][hl][g][0] = m[g];
        sm_ml[tg][hl][g][1] = l[g];
      }
    }
    __syncthreads();
    const bool whole = (s == sb) && (seg_end == sb + steps_b);
    // A workgroup's first and last segments are the only partial ones.
    const int slot = (s == s_begin) ? 0 : 1;
    for (int o = tid; o < GQ * kHeadDim; o += kThreads) {
      const int ql = o / kHeadDim, d = o % kHeadDim;   // query head within the unit
      const int hh = ql / G, g = ql % G;
      const int qh = hgi * GQ + ql;
      float M = sm_ml[0][hh][g][0];
#pragma unroll
      for (int t = 1; t < TG; ++t) M = fmaxf(M, sm_ml[t][hh][g][0]);
      float Ls = 0.f, A = 0.f;
#pragma unroll
      for (int t = 0; t < TG; ++t) {
        const float a = fast_exp2(sm_ml[t][hh][g][0] - M);
        Ls += sm_ml[t][hh][g][1] * a;
        A += sm_acc[t][hh][g][d] * a;
      }
      if (whole) {
        out[(int64_t)b * out_seq_stride + (int64_t)qh * out_head_stride + d] =
            f32_to_bf16(Ls > 0.f ? A / Ls : 0.f);
      } else {
        float* p = ws + (((int64_t)w * 2 + slot) * HQ + ql) * kSlotStride;
        p[d] = A;
        if (d == 0) {
          p[kHeadDim] = M;
          p[kHeadDim + 1] = Ls;
        }
      }
    }
    __syncthreads();  // LDS is reused by the next segment
    s = seg_end;
  }
}

// Unit of (sequence b, query head qh) and its workgroups.  Returns false when
// the unit needs no merge (empty, written directly in unit mode, or held by one
// workgroup); otherwise sets its step range [ub, ue), the first and last
// owning workgroups and the active workgroup count.
template <int HKV, int G, int HG>
__device__ __forceinline__ bool unit_owners(const int32_t* __restrict__ ws_off, int batch, int n_bal,
                                            int b, int qh, int64_t* ub, int64_t* w0, int64_t* w1,
                                            int64_t* total, int64_t* n_act) {
  constexpr int NHG = HKV / HG;
  const int64_t steps_b = ws_off[b + 1] - ws_off[b];
  if (ws_off[batch + 1] != 0) return false;  // unit mode: every unit was written whole
  *total = (int64_t)NHG * ws_off[batch];
  *n_act = active_wgs(*total, n_bal);
  *ub = (int64_t)NHG * ws_off[b] + (qh / (HG * G)) * steps_b;
  *w0 = owner_of(*ub, *total, *n_act);
  *w1 = owner_of(*ub + steps_b - 1, *total, *n_act);
  return *w0 != *w1;
}

// Combines the partial slots of units shared by several workgroups and
// writes zeros for empty sequences, reading the step offsets and the mode the
// split kernel published after its slots.  One workgroup per (sequence, query
// head): 16 groups of 16 lanes take every 16th sharing workgroup (a lane owns
// 8 output dims), so up to 16 slots are read at once; the group states are
// combined through LDS.
template <int HKV, int G, int HG>
__global__ __launch_bounds__(kThreads) void decode_streamk_merge(
    int batch, int n_bal, const float* __restrict__ ws, uint16_t* __restrict__ out,
    int64_t out_seq_stride, int64_t out_head_stride) {
  constexpr int HQ = HKV * G;
  constexpr int GQ = HG * G;
  constexpr int kGroups = kThreads / 16;
  __shared__ float s_ml[kGroups][2];
  __shared__ float s_acc[kGroups][kHeadDim];
  const int32_t* ws_off = reinterpret_cast<const int32_t*>(ws + (int64_t)n_bal * 2 * HQ * kSlotStride);
  const int b = blockIdx.x, qh = blockIdx.y;
  const int tid = threadIdx.x, lane16 = tid & 15, grp = tid >> 4;
  uint16_t* o_row = out + (int64_t)b * out_seq_stride + (int64_t)qh * out_head_stride;
  if (ws_off[b + 1] == ws_off[b]) {  // empty sequence attends to nothing: zeros, as flash-attn
    if (tid < kHeadDim) o_row[tid] = 0;
    return;
  }
  int64_t ub, w0, w1, total, n_act;
  if (!unit_owners<HKV, G, HG>(ws_off, batch, n_bal, b, qh, &ub, &w0, &w1, &total, &n_act)) return;
  const int ql = qh % GQ;
  const int d0 = lane16 * 8;
  float M = kNegBig, Ls = 0.f, A[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) A[e] = 0.f;
  for (int64_t ww = w0 + grp; ww <= w1; ww += kGroups) {
    const int64_t r0 = range_start(ww, total, n_act);
    if (r0 == range_start(ww + 1, total, n_act)) continue;  // empty range: owns no slot
    const int slot = (r0 >= ub) ? 0 : 1;
    const float* p = ws + ((ww * 2 + slot) * HQ + ql) * kSlotStride;
    const float mw = p[kHeadDim], lw = p[kHeadDim + 1];
    const f32x4_t a0 = *reinterpret_cast<const f32x4_t*>(p + d0);
    const f32x4_t a1 = *reinterpret_cast<const f32x4_t*>(p + d0 + 4);
    const float mn = fmaxf(M, mw);
    const float s1 = fast_exp2(M - mn), s2 = fast_exp2(mw - mn);
    Ls = Ls * s1 + lw * s2;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      A[e] = A[e] * s1 + a0[e] * s2;
      A[4 + e] = A[4 + e] * s1 + a1[e] * s2;
    }
    M = mn;
  }
  if (lane16 == 0) {
    s_ml[grp][0] = M;
    s_ml[grp][1] = Ls;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) s_acc[grp][d0 + e] = A[e];
  __syncthreads();
  if (tid < kHeadDim) {
    float Mx = s_ml[0][0];
#pragma unroll
    for (int g2 = 1; g2 < kGroups; ++g2) Mx = fmaxf(Mx, s_ml[g2][0]);
    float Lt = 0.f, At = 0.f;
#pragma unroll
    for (int g2 = 0; g2 < kGroups; ++g2) {
      const float a = fast_exp2(s_ml[g2][0] - Mx);
      Lt += s_ml[g2][1] * a;
      At += s_acc[g2][tid] * a;
    }
    o_row[tid] = f32_to_bf16(Lt > 0.f ? At / Lt : 0.f);
  }
}

// The same combination for large batches (each unit shared by a few
// workgroups): one workgroup per sequence, a 16-lane group per query head
// (a lane owns 8 output dims) walking the sharing workgroups, four slots in
// flight; no LDS.
template <int HKV, int G, int HG>
__global__ __launch_bounds__(kThreads) void decode_streamk_merge_seq(
    int batch, int n_bal, const float* __restrict__ ws, uint16_t* __restrict__ out,
    int64_t out_seq_stride, int64_t out_head_stride) {
  constexpr int HQ = HKV * G;
  constexpr int GQ = HG * G;
  constexpr int kGroups = kThreads / 16;
  const int32_t* ws_off = reinterpret_cast<const int32_t*>(ws + (int64_t)n_bal * 2 * HQ * kSlotStride);
  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane16 = tid & 15, grp = tid >> 4;
  uint16_t* o_seq = out + (int64_t)b * out_seq_stride;
  const int d0 = lane16 * 8;
  if (ws_off[b + 1] == ws_off[b]) {  // empty sequence attends to nothing: zeros, as flash-attn
    for (int qh = grp; qh < HQ; qh += kGroups)
      *reinterpret_cast<uint4*>(o_seq + (int64_t)qh * out_head_stride + d0) = make_uint4(0, 0, 0, 0);
    return;
  }
  for (int qh = grp; qh < HQ; qh += kGroups) {
    int64_t ub, w0, w1, total, n_act;
    if (!unit_owners<HKV, G, HG>(ws_off, batch, n_bal, b, qh, &ub, &w0, &w1, &total, &n_act))
      continue;
    const int ql = qh % GQ;
    float M = kNegBig, Ls = 0.f, A[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) A[e] = 0.f;
    for (int64_t wb = w0; wb <= w1; wb += 4) {
      float mw[4], lw[4];
      f32x4_t a0[4], a1[4];
      bool ok[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // A workgroup with an empty step range owns no slot; w0 owns step ub,
        // so its slot 0 is always written and stands in for such entries.
        const int64_t ww = wb + j;
        const int64_t r0 = range_start(ww, total, n_act);
        ok[j] = ww <= w1 && r0 != range_start(ww + 1, total, n_act);
        const int64_t slot = ok[j] ? ww * 2 + ((r0 >= ub) ? 0 : 1) : w0 * 2;
        const float* p = ws + (slot * HQ + ql) * kSlotStride;
        mw[j] = p[kHeadDim];
        lw[j] = p[kHeadDim + 1];
        a0[j] = *reinterpret_cast<const f32x4_t*>(p + d0);
        a1[j] = *reinterpret_cast<const f32x4_t*>(p + d0 + 4);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (!ok[j]) continue;
        const float mn = fmaxf(M, mw[j]);
        const float s1 = fast_exp2(M - mn), s2 = fast_exp2(mw[j] - mn);
        Ls = Ls * s1 + lw[j] * s2;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          A[e] = A[e] * s1 + a0[j][e] * s2;
          A[4 + e] = A[4 + e] * s1 + a1[j][e] * s2;
        }
        M = mn;
      }
    }
    const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
    uint4 pk;
    pk.x = pack_bf16x2(A[0] * inv, A[1] * inv);
    pk.y = pack_bf16x2(A[2] * inv, A[3] * inv);
    pk.z = pack_bf16x2(A[4] * inv, A[5] * inv);
    pk.w = pack_bf16x2(A[6] * inv, A[7] * inv);
    *reinterpret_cast<uint4*>(o_seq + (int64_t)qh * out_head_stride + d0) = pk;
  }
}

}  // namespace

namespace qmi {

// Compute units of the current device (cached per device id).
static int64_t device_cus() {
  static int64_t cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// KV heads per work unit: all of them below 128 sequences; from 128 sequences
// the fewest (down to a quarter of the heads, at least 2) that still give two
// units per workgroup slot of the GPU.
int64_t streamk_heads_per_unit(int64_t batch, int64_t num_kv_heads) {
  const int64_t target = 2 * device_cus();
  int64_t hg = num_kv_heads;
  if (batch >= 128)
    while (hg > 2 && hg > num_kv_heads / 4 && batch * (num_kv_heads / hg) < target) hg /= 2;
  return hg;
}

// Workgroups of the balanced split: two per CU, never more than the step
// count can feed.
static int64_t streamk_balanced_wgs(int64_t batch, int64_t num_kv_heads, int64_t hg,
                                    int64_t bt_width) {
  const int64_t ts = (16 / hg) * kTok;
  const int64_t max_steps = batch * (num_kv_heads / hg) * ((bt_width * kPage + ts - 1) / ts);
  const int64_t target = 2 * device_cus();
  return max_steps < target ? (max_steps < 1 ? 1 : max_steps) : target;
}

int64_t streamk_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                int64_t bt_width) {
  // partial slots of the balanced split, then the published step offsets
  // (int32 [batch + 1]) and the mode word
  const int64_t hg = streamk_heads_per_unit(batch, num_kv_heads);
  return streamk_balanced_wgs(batch, num_kv_heads, hg, bt_width) * 2 * num_q_heads * kSlotStride *
             (int64_t)sizeof(float) +
         (batch + 2) * (int64_t)sizeof(int32_t);
}

bool streamk_supported(int64_t num_q_heads, int64_t num_kv_heads, int64_t batch) {
  if (batch > kMaxSeqScan) return false;
  const int64_t g = num_q_heads / num_kv_heads;
  const bool hkv_ok = num_kv_heads == 2 || num_kv_heads == 4 || num_kv_heads == 8 || num_kv_heads == 16;
  return hkv_ok && (g == 1 || g == 2 || g == 4) && batch <= 65535;
}

template <int HKV, int G, int HG, bool QKV>
static int launch(const uint16_t* q, int64_t qs, int64_t qh, const uint16_t* kc, const uint16_t* vc,
                  int64_t nb, const int32_t* lens, int32_t bias, const int32_t* bt, int64_t bts,
                  int64_t btw, int64_t batch, float scale_log2, uint16_t* out, int64_t os,
                  int64_t oh, float* ws, bool whole_units, const QkvArgs& qa, hipStream_t s) {
  const int64_t n_bal = streamk_balanced_wgs(batch, HKV, HG, btw);
  const int64_t n_units = batch * (HKV / HG);
  const int64_t grid = n_bal > n_units ? n_bal : n_units;
  hipLaunchKernelGGL((decode_streamk_split<HKV, G, HG, QKV>), dim3((unsigned)grid), dim3(kThreads),
                     0, s, q, qs, qh, kc, vc, nb, lens, (int)bias, bt, bts, (int)btw, (int)batch,
                     (int)n_bal, scale_log2, out, os, oh, ws, whole_units ? 1 : 0, qa);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  if (whole_units) return QMI_OK;  // every unit was written whole, empty ones as zeros
  // Small batches: units are shared by many workgroups, so one merge
  // workgroup per (sequence, head) reads 16 slots at once; large batches:
  // a few slots per unit, one workgroup per sequence.
  if (batch >= 128)
    hipLaunchKernelGGL((decode_streamk_merge_seq<HKV, G, HG>), dim3((unsigned)batch), dim3(kThreads),
                       0, s, (int)batch, (int)n_bal, ws, out, os, oh);
  else
    hipLaunchKernelGGL((decode_streamk_merge<HKV, G, HG>), dim3((unsigned)batch, (unsigned)(HKV * G)),
                       dim3(kThreads), 0, s, (int)batch, (int)n_bal, ws, out, os, oh);
  QMI_RETURN_LAUNCH_STATUS();
}

template <bool QKV>
static int launch_sk(const uint16_t* q, int64_t qs, int64_t qh, const uint16_t* kc,
                     const uint16_t* vc, int64_t nb, int64_t num_q_heads, int64_t num_kv_heads,
                     const int32_t* lens, int32_t bias, const int32_t* bt, int64_t bts,
                     int64_t btw, int64_t batch, float scale, uint16_t* out, int64_t os,
                     int64_t oh, float* ws, bool whole_units, const QkvArgs& qa, hipStream_t s) {
  const float sl = scale * kLog2e;
  const int64_t g = num_q_heads / num_kv_heads;
  const int64_t hg = streamk_heads_per_unit(batch, num_kv_heads);
#define QMI_SK(HK, GG, HGG)                                                                      \
  if (num_kv_heads == HK && g == GG && hg == HGG)                                                \
    return launch<HK, GG, HGG, QKV>(q, qs, qh, kc, vc, nb, lens, bias, bt, bts, btw, batch, sl,   \
                                    out, os, oh, ws, whole_units, qa, s);
#define QMI_SK_G(HK, HGG) QMI_SK(HK, 1, HGG) QMI_SK(HK, 2, HGG) QMI_SK(HK, 4, HGG)
  QMI_SK_G(8, 8) QMI_SK_G(8, 4) QMI_SK_G(8, 2)
  QMI_SK_G(4, 4) QMI_SK_G(4, 2)
  QMI_SK_G(2, 2)
  QMI_SK_G(16, 16) QMI_SK_G(16, 8) QMI_SK_G(16, 4)
#undef QMI_SK_G
#undef QMI_SK
  return QMI_E_UNSUPPORTED;
}

int launch_streamk(const uint16_t* q, int64_t qs, int64_t qh, const uint16_t* kc,
                   const uint16_t* vc, int64_t nb, int64_t num_q_heads, int64_t num_kv_heads,
                   const int32_t* lens, int32_t bias, const int32_t* bt, int64_t bts, int64_t btw,
                   int64_t batch, float scale, uint16_t* out, int64_t os, int64_t oh, float* ws,
                   bool whole_units, hipStream_t s) {
  return launch_sk<false>(q, qs, qh, kc, vc, nb, num_q_heads, num_kv_heads, lens, bias, bt, bts,
                          btw, batch, scale, out, os, oh, ws, whole_units, QkvArgs{}, s);
}

}  // namespace qmi

static inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

extern "C" int qmi_paged_decode_attention_qkv(
    const uint16_t* qkv, int64_t qkv_stride, int64_t num_q_heads, int64_t num_kv_heads,
    int64_t head_dim, const uint16_t* q_norm_weight, const uint16_t* k_norm_weight,
    const int64_t* positions, const float* cos_sin_cache, int64_t max_position, float eps,
    uint16_t* k_cache, uint16_t* v_cache, int64_t num_blocks, int64_t block_size,
    const int32_t* slot_mapping, const int32_t* seqlens, const int32_t* block_table,
    int64_t bt_stride, int64_t bt_width, int64_t batch, float scale, uint16_t* out,
    int64_t out_seq_stride, int64_t out_head_stride, float* workspace, int64_t workspace_bytes,
    int64_t pages_per_split, void* stream) {
  if (batch < 0 || num_blocks < 0 || bt_width < 0 || max_position <= 0) return QMI_E_BAD_SHAPE;
  if (batch == 0) return QMI_OK;
  if (num_blocks == 0 || bt_width == 0) return QMI_E_BAD_SHAPE;
  if (!qkv || !q_norm_weight || !k_norm_weight || !positions || !cos_sin_cache || !k_cache ||
      !v_cache || !slot_mapping || !seqlens || !block_table || !out)
    return QMI_E_NULL_POINTER;
  if (head_dim != kHeadDim || block_size != kPage) return QMI_E_UNSUPPORTED;
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return QMI_E_BAD_SHAPE;
  if (pages_per_split > 0 || pages_per_split < -1) return QMI_E_UNSUPPORTED;
  if (!qmi::streamk_supported(num_q_heads, num_kv_heads, batch) || bt_width > 65535)
    return QMI_E_UNSUPPORTED;
  if (bt_stride < bt_width) return QMI_E_BAD_STRIDE;
  if (qkv_stride < (num_q_heads + 2 * num_kv_heads) * kHeadDim || qkv_stride % 8 || !al16(qkv) ||
      !al16(q_norm_weight) || !al16(k_norm_weight) || !al16(cos_sin_cache) || !al16(k_cache) ||
      !al16(v_cache) || !al16(out) || out_seq_stride % 8 || out_head_stride % 8)
    return QMI_E_BAD_STRIDE;
  const int64_t need = qmi::streamk_workspace_bytes(batch, num_q_heads, num_kv_heads, bt_width);
  if (!workspace || workspace_bytes < need) return QMI_E_WORKSPACE_TOO_SMALL;
  const QkvArgs qa{q_norm_weight, k_norm_weight, positions, cos_sin_cache, max_position,
                   slot_mapping, num_blocks * kPage, k_cache, v_cache, eps};
  return qmi::launch_sk<true>(qkv, qkv_stride, kHeadDim, k_cache, v_cache, num_blocks,
                              num_q_heads, num_kv_heads, seqlens, 1, block_table, bt_stride,
                              bt_width, batch, scale, out, out_seq_stride, out_head_stride,
                              workspace, pages_per_split == -1, qa,
                              reinterpret_cast<hipStream_t>(stream));
}
