// Slot-mapped KV store into the paged cache.
//
// Reference semantics: _store_kvcache_kernel / store_kvcache
// (qwen3_naive.py:20-41): token i's K row and V row (row_elems = kv_heads *
// head_dim contiguous bf16 each) are copied to row slot_mapping[i] of the
// flat [num_blocks * block_size, row_elems] caches; slot -1 is skipped.
//
// gfx950 design: the copy is pure HBM traffic, so each lane moves 16-byte
// chunks (one global_load_dwordx4 / global_store_dwordx4 per tensor) and a
// 256-lane workgroup covers 2 tokens of a 1024-element row.  The grid
// walks the flat (token, chunk) space, so every wave issues fully
// coalesced 1 KB transactions for any token count.  A 2-byte fallback
// handles rows or strides that are not 16-byte aligned.
#include "qmi_common.h"

namespace {

using namespace qmi;

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void store_kv_vec16(
    const uint4* __restrict__ key, int64_t key_stride_v,
    const uint4* __restrict__ value, int64_t value_stride_v,
    uint4* __restrict__ k_cache, uint4* __restrict__ v_cache,
    const int32_t* __restrict__ slots, int64_t n_tokens, int64_t row_vecs, int64_t n_slots) {
  const int64_t total = n_tokens * row_vecs;
  for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * kThreads) {
    const int64_t tok = idx / row_vecs;
    const int64_t c = idx - tok * row_vecs;
    const int64_t slot = slots[tok];
    if (slot < 0 || slot >= n_slots) continue;
    const u32x4_t kv = reinterpret_cast<const u32x4_t*>(key)[tok * key_stride_v + c];
    const u32x4_t vv = reinterpret_cast<const u32x4_t*>(value)[tok * value_stride_v + c];
    // Non-temporal stores: the cache rows are not read again in this launch,
    // and keeping them out of the caches leaves room for the streamed inputs
    // (537 MB store: 5.2 -> 6.9 TB/s; non-temporal loads as well measured slower).
    __builtin_nontemporal_store(kv, reinterpret_cast<u32x4_t*>(k_cache) + slot * row_vecs + c);
    __builtin_nontemporal_store(vv, reinterpret_cast<u32x4_t*>(v_cache) + slot * row_vecs + c);
  }
}

__global__ __launch_bounds__(kThreads) void store_kv_scalar(
    const uint16_t* __restrict__ key, int64_t key_stride,
    const uint16_t* __restrict__ value, int64_t value_stride,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const int32_t* __restrict__ slots, int64_t n_tokens, int64_t row_elems, int64_t n_slots) {
  const int64_t total = n_tokens * row_elems;
  for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * kThreads) {
    const int64_t tok = idx / row_elems;
    const int64_t c = idx - tok * row_elems;
    const int64_t slot = slots[tok];
    if (slot < 0 || slot >= n_slots) continue;
    k_cache[slot * row_elems + c] = key[tok * key_stride + c];
    v_cache[slot * row_elems + c] = value[tok * value_stride + c];
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int qmi_store_kvcache(const uint16_t* key, int64_t key_row_stride,
                                 const uint16_t* value, int64_t value_row_stride,
                                 uint16_t* k_cache, uint16_t* v_cache,
                                 const int32_t* slot_mapping, int64_t n_tokens,
                                 int64_t row_elems, int64_t n_slots, void* stream) {
  if (n_tokens < 0 || row_elems <= 0 || n_slots < 0) return QMI_E_BAD_SHAPE;
  if (n_tokens == 0) return QMI_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) return QMI_E_NULL_POINTER;
  if (key_row_stride < row_elems || value_row_stride < row_elems) return QMI_E_BAD_STRIDE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);

  const bool vec = (row_elems % 8 == 0) && (key_row_stride % 8 == 0) &&
                   (value_row_stride % 8 == 0) && aligned16(key) && aligned16(value) &&
                   aligned16(k_cache) && aligned16(v_cache);
  const int64_t units = vec ? n_tokens * (row_elems / 8) : n_tokens * row_elems;
  int64_t blocks = (units + kThreads - 1) / kThreads;
  if (blocks > 65535 * 4) blocks = 65535 * 4;  // grid-stride loop covers the rest
  if (vec) {
    hipLaunchKernelGGL(store_kv_vec16, dim3((unsigned)blocks), dim3(kThreads), 0, s,
                       reinterpret_cast<const uint4*>(key), key_row_stride / 8,
                       reinterpret_cast<const uint4*>(value), value_row_stride / 8,
                       reinterpret_cast<uint4*>(k_cache), reinterpret_cast<uint4*>(v_cache),
                       slot_mapping, n_tokens, row_elems / 8, n_slots);
  } else {
    hipLaunchKernelGGL(store_kv_scalar, dim3((unsigned)blocks), dim3(kThreads), 0, s, key,
                       key_row_stride, value, value_row_stride, k_cache, v_cache, slot_mapping,
                       n_tokens, row_elems, n_slots);
  }
  QMI_RETURN_LAUNCH_STATUS();
}
