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
//   * Workgroup = 4 wave64 = one (sequence, KV head, block of 128/G queries);
//     wave w takes query head (w / (4/G)) of the GQA group and 32 queries
//     (two 16-query column blocks), so each K / V^T operand read from LDS
//     feeds two MFMAs and the K/V tiles staged in LDS serve all G heads.
//   * Scores are computed transposed, S^T = K Q^T, with
//     v_mfma_f32_16x16x32_bf16 (A = 16 keys x 32 dims from LDS, B = Q^T held
//     in registers).  The K operands of a 32-dim slice are read from LDS two
//     slices ahead of their MFMAs (inline-asm ds_read_b128 with explicit
//     LDS-counter waits; left to itself the compiler sinks each read next to
//     the MFMA that consumes it and the LDS latency shows on every slice).  Its accumulator layout (lane l: keys 4*(l/16)+r,
//     query l%16) is exactly the B-operand layout of the second product
//     O^T = V^T P^T once two 16-key blocks are packed to bf16, so P never
//     leaves registers.
//   * K and V tiles go from the page straight into LDS: gfx950's
//     global_load_lds_dwordx4 (8 per lane per tile, no registers) writes a
//     wave's 64 x 16 bytes to 1 KB of LDS, lane l at base + 16 l.  They are
//     issued as inline asm at the start of the previous tile, so a tile's
//     loads have a whole tile of compute to land, and the compiler puts no
//     wait of its own on them (it cannot tell the LDS targets apart and
//     would wait for every load in flight before each LDS access).
//     Rows are 256 bytes (one KV head of a token) with the 16-byte chunks
//     XOR-swizzled instead of padded: chunk c of K row r sits at c ^ (r % 16)
//     (16 consecutive rows then hit 16 distinct 4-bank groups for the A
//     operand reads), chunk c of V row r at c ^ (2 (r % 4) + 8 ((r / 4) % 2))
//     (the 8 rows that the two 16-lane groups of a transpose read's 32-lane
//     half address then cover all 64 banks); each lane fetches the logical
//     chunk that its physical slot holds.
//   * The V^T operand is read with gfx950's LDS transpose read
//     (ds_read_b64_tr_b16): in a 16-lane group, lane r receives 16-bit
//     element r % 4 of lane 4e + r / 4's 8 bytes as element e, so pointing
//     lane i at V[kbase + i / 4][16 db + 4 (i % 4)] hands lane r the 4 keys
//     kbase .. kbase+3 of dim 16 db + r.  Two such reads (keys 32c + 4g and
//     32c + 16 + 4g) form the 8 keys the B operand P^T packs for the lane.
//     These reads are issued as inline asm with explicit LDS-counter waits,
//     one 16-dim block ahead, with immediate offsets from per-lane bases
//     fixed for the whole loop.
//   * Online softmax in fp32 (log2 domain); per query the 4 lanes holding
//     its keys agree on the running max through two VALU lane swaps.  The running
//     sum of P is one more MFMA per 32 keys (A = a 16 x 32 block whose row 0
//     is all ones), so it sums exactly the bf16 P the O^T product uses and
//     costs no VALU adds.
//   * K / V tiles of 64 keys (one quarter page) are double-buffered in LDS:
//     the loads of tile t+1 are in flight while tile t is computed and land
//     in the buffer no wave reads during tile t; each wave waits for its own
//     loads (s_waitcnt vmcnt(0)) before the tile's closing barrier.  Keys
//     past the workgroup's last visible key are stale page rows: their
//     scores are masked and their V rows are overwritten with zeros once
//     they have landed.
//   * Work items are (query block, sequence, KV head).  Three schedules, by
//     launch size (items) on a GPU of C CUs:
//     - queue mode, 256 <= items < 4 C: a persistent grid of two workgroups
//       per CU; workgroup w serves KV head w % Hkv (with 8 KV heads a head's
//       workgroups share an XCD and its L2) and takes items from that head's
//       counter in the workspace (first ticket static, then one atomic per
//       item), late (long, causal) query blocks first.  The hardware
//       dispatcher, left to itself, packs two workgroups on some CUs while
//       others idle and holds some back when a launch has about one item per
//       slot; the queue keeps every slot busy until the items run out.  The
//       last workgroup out resets the counters to zero.
//     - thin queue launches (no more items per KV head than workgroups per
//       head, e.g. the last chunks behind a long cached prefix): every
//       workgroup builds the same plan in LDS from cu_seqlens and cuts items
//       longer than two balanced shares (total tiles / workgroups per head)
//       into equal key ranges; the pieces store normalised bf16 rows and
//       their fp32 max / sum, and varlen_prefill_queue_merge combines them
//       after the launch (stream order, no cross-workgroup synchronisation).
//     - grid mode otherwise: grid = (Hkv, B, query blocks), one item per
//       workgroup, query blocks issued last-first; launches with fewer than
//       256 items cut long key ranges into at most 16 equal tile ranges run
//       by separate workgroups (fp32 partials, varlen_prefill_merge).
#include <algorithm>
#include <type_traits>

#include "qmi_common.h"

namespace {

using namespace qmi;

constexpr int kHeadDim = 128;
constexpr int kPage = 256;
constexpr int kThreads = 256;
constexpr int kKeyTile = 64;
constexpr int kWaveQ = 32;              // queries per wave (two MFMA column blocks)
typedef __attribute__((ext_vector_type(4))) short v4s_t;
typedef __attribute__((ext_vector_type(2))) unsigned int v2u_t;

// LDS transpose read (ds_read_b64_tr_b16) at a per-lane address plus an
// immediate byte offset.  Issued as inline asm so that the compiler does not
// put a wait for every outstanding memory operation in front of it; the
// caller waits with lgkm_wait.
template <int OFF>
__device__ __forceinline__ v2u_t ds_read_tr16_b64(uint32_t addr) {
  v2u_t r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}

// Waits until at most N LDS reads are outstanding; the four registers are
// tied to the wait so that no use of them is scheduled above it.
template <int N>
__device__ __forceinline__ void lgkm_wait(v2u_t& a, v2u_t& b, v2u_t& c, v2u_t& d) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "i"(N) : "memory");
}

// LDS read of 16 bytes (ds_read_b128) at a per-lane address plus an
// immediate byte offset; as inline asm it stays where it is written instead
// of being sunk next to its use.  The caller waits with lgkm_wait_u4.
typedef __attribute__((ext_vector_type(4))) unsigned int u4v_t;
template <int OFF>
__device__ __forceinline__ u4v_t ds_read_b128_at(uint32_t addr) {
  u4v_t r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}

template <int N>
__device__ __forceinline__ void lgkm_wait_u4(u4v_t& a, u4v_t& b, u4v_t& c, u4v_t& d) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "i"(N) : "memory");
}

// Direct global -> LDS load of 16 bytes per lane (global_load_lds_dwordx4):
// lane l's bytes at gbase + voff land at LDS byte lds + 16 l.  Inline asm, so
// that the compiler adds no wait for it (it cannot tell the LDS targets
// apart and would wait for every outstanding load); the caller waits with
// s_waitcnt vmcnt.
__device__ __forceinline__ void lds_load16(const void* gbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds), "v"(voff), "s"(gbase)
               : "memory", "m0");
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
  return __builtin_bit_cast(bf16x8_t, u32x4_t{v.x, v.y, v.z, v.w});
}

// Work item geometry shared by the attention and merge kernels.
struct Item {
  int q_start, Lq, Lk, diag, n_tiles, n_parts;
};

__device__ __forceinline__ Item item_geometry(const int32_t* cu_q, const int32_t* cu_k, int b, int q0,
                                              int qb, int64_t total_q, int bt_width, int n_split,
                                              int split_tiles) {
  Item it;
  // Rows outside [0, total_q) of q / out are never touched, whatever cu_q holds.
  it.q_start = max(0, cu_q[b]);
  it.Lq = (int)max((int64_t)0, min((int64_t)cu_q[b + 1], total_q) - it.q_start);
  it.Lk = max(0, min(cu_k[b + 1] - cu_k[b], bt_width * kPage));
  it.diag = it.Lk - it.Lq;  // query i sees keys j <= i + diag
  // Keys the block needs: up to its last query's diagonal.
  const int kend = max(0, min(it.Lk, it.diag + min(q0 + qb, it.Lq)));
  it.n_tiles = (kend + kKeyTile - 1) / kKeyTile;
  it.n_parts = max(1, min(n_split, (it.n_tiles + split_tiles - 1) / split_tiles));
  return it;
}

// ---------------------------------------------------------------------------
// Split plan of a thin queue-mode launch (no more items per KV head than
// workgroups per head, e.g. a chunk after a long cached prefix), built by
// every workgroup in LDS from cu_seqlens, so all derive the same plan and no
// host knowledge of the lengths is needed.  Items keep their ticket order
// (query block n_qblocks-1 - i / batch of sequence i % batch); an item of n
// tiles is cut into ceil(n / S) parts (at most kMaxQueueSplit),
// S = max(kMinPartTiles, ceil(kSplitShare T / P)) with T the head's total
// tiles and P its workgroups.  Empty items get no unit.  A unit packs item
// (11 bits), part (4), parts of the item (5) and the item's first partial
// slot (12).  Workgroup 0 also writes the list of split items (count, then
// item | parts << 11 | first slot << 20) for varlen_prefill_queue_merge.
constexpr int kPlanMaxItems = 512;
constexpr int kPlanPer = kPlanMaxItems / kThreads;
constexpr int kPlanMaxUnits = 2048;
constexpr int kMinPartTiles = 8;
constexpr int kMaxQueueSplit = 16;
constexpr float kSplitShare = 2.0f;

__device__ __forceinline__ uint32_t pack_unit(int item, int part, int n_parts, int pbase) {
  return (uint32_t)item | ((uint32_t)part << 11) | ((uint32_t)n_parts << 15) | ((uint32_t)pbase << 20);
}

// Exclusive workgroup scan of two ints; also returns the totals.  scr: 8 ints of LDS.
__device__ __forceinline__ void block_scan2(int a, int b, int* ea, int* eb, int* ta, int* tb,
                                            int* scr) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int ia = a, ib = b;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int xa = __shfl_up(ia, d, 64), xb = __shfl_up(ib, d, 64);
    if (lane >= d) {
      ia += xa;
      ib += xb;
    }
  }
  if (lane == 63) {
    scr[wave] = ia;
    scr[4 + wave] = ib;
  }
  __syncthreads();
  int oa = 0, ob = 0;
  for (int w = 0; w < wave; ++w) {
    oa += scr[w];
    ob += scr[4 + w];
  }
  *ea = oa + ia - a;
  *eb = ob + ib - b;
  *ta = scr[0] + scr[1] + scr[2] + scr[3];
  *tb = scr[4] + scr[5] + scr[6] + scr[7];
  __syncthreads();
}

// Returns the number of units (tickets); s_units receives them.  n_items <=
// kPlanMaxItems and n_pslots <= pslot_cap hold by the host's choice of thin
// launches (a plan over the cap returns 0 parts beyond one per item).
template <int kQB>
__device__ int build_plan(const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k,
                          int batch, int n_qblocks, int64_t total_q, int bt_width, int per_head,
                          int pslot_cap, uint32_t* s_units, int* scr, uint32_t* __restrict__ splits) {
  const int n_items = n_qblocks * batch;
  const int tid = threadIdx.x;
  int nt[kPlanPer];
  int tsum = 0;
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) {
    const int i = tid * kPlanPer + k;
    nt[k] = 0;
    if (i < n_items) {
      const int q0 = (n_qblocks - 1 - i / batch) * kQB;
      const Item it = item_geometry(cu_q, cu_k, i % batch, q0, kQB, total_q, bt_width, 1, 1 << 30);
      nt[k] = q0 < it.Lq ? it.n_tiles : 0;
    }
    tsum += nt[k];
  }
  int e0, e1, tiles, unused;
  block_scan2(tsum, 0, &e0, &e1, &tiles, &unused, scr);
  int S = max(kMinPartTiles, (int)ceilf(kSplitShare * (float)tiles / (float)per_head));
  int np[kPlanPer];
  int usum = 0, psum = 0, ssum = 0;
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) {
    np[k] = nt[k] > 0 ? min(kMaxQueueSplit, (nt[k] + S - 1) / S) : 0;
    usum += np[k];
    psum += np[k] > 1 ? np[k] : 0;
    ssum += np[k] > 1 ? 1 : 0;
  }
  int ubase, pbase, sbase, n_units, n_pslots, n_splits;
  block_scan2(usum, psum, &ubase, &pbase, &n_units, &n_pslots, scr);
  block_scan2(ssum, 0, &sbase, &e1, &n_splits, &unused, scr);
  const bool split_ok = n_units <= kPlanMaxUnits && n_pslots <= pslot_cap;  // uniform
  if (!split_ok) {  // one unit per non-empty item
#pragma unroll
    for (int k = 0; k < kPlanPer; ++k) np[k] = nt[k] > 0 ? 1 : 0;
    int cnt = 0;
#pragma unroll
    for (int k = 0; k < kPlanPer; ++k) cnt += np[k];
    block_scan2(cnt, 0, &ubase, &e1, &n_units, &unused, scr);
    n_splits = 0;
  }
#pragma unroll
  for (int k = 0; k < kPlanPer; ++k) {
    const int i = tid * kPlanPer + k;
    for (int p = 0; p < np[k]; ++p) s_units[ubase + p] = pack_unit(i, p, np[k], np[k] > 1 ? pbase : 0);
    ubase += np[k];
    if (np[k] > 1) {
      if (blockIdx.x == 0) splits[1 + sbase] = (uint32_t)i | ((uint32_t)np[k] << 11) | ((uint32_t)pbase << 20);
      ++sbase;
      pbase += np[k];
    }
  }
  if (blockIdx.x == 0 && tid == 0) splits[0] = (uint32_t)n_splits;
  __syncthreads();
  return n_units;
}

// Workspace of a split launch: per (item, part) slot, 128 rows of O (fp32,
// 128 dims, unnormalised), then, after all slots, (max, sum) per row.
__device__ __forceinline__ int64_t part_slot(int kvh, int b, int qblk, int part, int n_split) {
  return (((int64_t)qblk * gridDim.y + b) * gridDim.x + kvh) * n_split + part;
}

template <int G, bool kQueue>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void varlen_prefill_kernel(
    const uint16_t* __restrict__ q, int64_t q_tok_stride, int64_t q_head_stride,
    const uint16_t* __restrict__ k_cache, const uint16_t* __restrict__ v_cache,
    int64_t num_blocks, int num_kv_heads,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k,
    const int32_t* __restrict__ block_table, int64_t bt_stride, int bt_width,
    int batch, int n_qblocks, int64_t total_q, float scale_log2,
    uint16_t* __restrict__ out, int64_t out_tok_stride, int64_t out_head_stride,
    int n_split, int split_tiles, float* __restrict__ ws, unsigned* __restrict__ queue,
    int plan_mode, int pslot_cap) {
  constexpr int kWavesPerHead = 4 / G;
  constexpr int kQB = kWaveQ * kWavesPerHead;  // queries per workgroup
  // Unpadded 256-byte rows, 16-byte chunks XOR-swizzled: K chunk c of row r
  // sits at c ^ (r % 16), V chunk c at c ^ 2 (r % 4).
  __shared__ __attribute__((aligned(16))) uint16_t sK[2][kKeyTile * kHeadDim];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][kKeyTile * kHeadDim];
  __shared__ unsigned s_ticket;
  __shared__ uint32_t s_units[kPlanMaxUnits];
  __shared__ int s_scr[8];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: an SGPR
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int g4 = lane >> 4;
  // Queue mode: workgroup w serves KV head w % Hkv (with 8 KV heads, the
  // head's workgroups share an XCD and its L2).  Ticket k is query block
  // n_qblocks-1 - k / batch of sequence k % batch, so the long (late, causal)
  // blocks go first and the short ones fill the end.  The head's P
  // workgroups take tickets 0 .. P-1 first, then P + (the head's counter,
  // post-incremented); the next ticket is taken at the start of an item and
  // used after it, so the atomic's latency overlaps the item's loads.  Grid
  // mode: one item per workgroup.
  const int kvh = kQueue ? (int)(blockIdx.x % (unsigned)num_kv_heads) : (int)blockIdx.x;
  const unsigned per_head = gridDim.x / (unsigned)num_kv_heads;
  // Thin launches take planned units (split items), others one ticket per item.
  int n_tickets = n_qblocks * batch;
  if constexpr (kQueue) {
    if (plan_mode)
      n_tickets = build_plan<kQB>(cu_q, cu_k, batch, n_qblocks, total_q, bt_width, (int)per_head,
                                  pslot_cap, s_units, s_scr, queue + num_kv_heads + 1);
  }
  unsigned ticket = blockIdx.x / (unsigned)num_kv_heads;
  auto advance = [&]() __attribute__((always_inline)) {
    if constexpr (kQueue) {
      if (tid == 0) s_ticket = per_head + atomicAdd(&queue[kvh], 1u);
      __syncthreads();
      ticket = s_ticket;
      __syncthreads();
    }
  };

  for (int iter = 0;; ++iter) {
    int b, qblk, part, q_parts = 1, q_pbase = 0;
    if constexpr (kQueue) {
      if (ticket >= (unsigned)n_tickets) break;
      int it_idx = (int)ticket;
      part = 0;
      if (plan_mode) {
        const uint32_t u = s_units[ticket];
        it_idx = (int)(u & 2047u);
        part = (int)((u >> 11) & 15u);
        q_parts = (int)((u >> 15) & 31u);
        q_pbase = (int)(u >> 20);
      }
      qblk = n_qblocks - 1 - it_idx / batch;
      b = it_idx % batch;
    } else {
      if (iter > 0) break;
      b = blockIdx.y;
      qblk = n_qblocks - 1 - (int)(blockIdx.z % n_qblocks);  // late (long) blocks first
      part = (int)(blockIdx.z / n_qblocks);
    }

    const int q0 = qblk * kQB;
    Item item = item_geometry(cu_q, cu_k, b, q0, kQB, total_q, bt_width, n_split, split_tiles);
    if constexpr (kQueue) item.n_parts = q_parts;
    // Both exits are uniform over the workgroup.
    if (q0 >= item.Lq || part >= item.n_parts) {
      advance();
      continue;
    }
    const int q_start = item.q_start, Lq = item.Lq, Lk = item.Lk, diag = item.diag;

    const int qh = kvh * G + wave / kWavesPerHead;
    const int wq0 = q0 + (wave % kWavesPerHead) * kWaveQ;

    // Q^T operands: lane holds Q[query][32c + 8*g4 .. +8] for its query in
    // column block j (query wq0 + 16j + l16) and c = 0..3.
    bf16x8_t qop[2][4];
    int my_pos[2];  // last key each of this lane's queries may see (-1: none)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int my_q = wq0 + 16 * j + l16;
      const bool ok = my_q < Lq;
      my_pos[j] = ok ? diag + my_q : -1;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (ok)
          v = load_u4(q + (int64_t)(q_start + my_q) * q_tok_stride + (int64_t)qh * q_head_stride +
                      32 * c + 8 * g4);
        qop[j][c] = as_bf16x8(v);
      }
    }

    // Keys this workgroup needs: up to the last query's diagonal; part `part`
    // of n_parts takes tiles [t_begin, t_end).
    const int kend = max(0, min(Lk, diag + min(q0 + kQB, Lq)));
    const int t_begin = (int)((int64_t)part * item.n_tiles / item.n_parts);
    const int t_end = (int)((int64_t)(part + 1) * item.n_tiles / item.n_parts);

    // Tile loads: addresses are a per-tile scalar base (the tile's first key
    // row of this KV head) plus a fixed 32-bit lane offset.  A tile never
    // leaves its page, so the loads are issued unconditionally; keys at or past
    // kend are stale page rows, masked in the scores, and their V rows are
    // zeroed.  A tile whose page-table entry is outside [0, num_blocks) is
    // skipped in the compute.
    const int64_t row_elems = (int64_t)num_kv_heads * kHeadDim;
    // Lane offsets of the tile loads: chunk i of wave w covers rows 4q .. 4q+3
    // (q = 4w + i); lane l fetches row 4q + l / 16, physical chunk l % 16 (the
    // logical chunk the swizzle maps there), which lands at byte 1024 q + 16 l
    // of the buffer.
    uint32_t k_src[4], v_src[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * (4 * wave + i) + (lane >> 4), pc = lane & 15;
      k_src[i] = (uint32_t)((row * row_elems + 8 * (pc ^ (row & 15))) * 2);
      v_src[i] = (uint32_t)((row * row_elems + 8 * (pc ^ (((row & 3) << 1) | (row & 4) << 1))) * 2);
    }
    // Page-table entries of the current segment of tiles, one per lane: lane i
    // holds the entry of page pg0 + i (-1 past the table's width), read with
    // v_readlane, so the tile loop has no memory load besides the tile's own.
    int pg0 = 0, pg_lane = -1;
    bool tile_ok[2] = {false, false};
    int st_valid[2] = {0, 0};
    // Tile t into LDS buffer buf by direct loads (M0 = the wave's 1 KB block).
    auto load_tile = [&](int t, int buf) {
      const int key0 = t * kKeyTile;
      const int32_t blk = __builtin_amdgcn_readlane(pg_lane, key0 / kPage - pg0);
      const bool page_ok = blk >= 0 && blk < num_blocks;
      const int64_t row0 = (int64_t)(page_ok ? blk : 0) * kPage + (key0 % kPage);
      const char* kb = reinterpret_cast<const char*>(k_cache + row0 * row_elems + kvh * kHeadDim);
      const char* vb = reinterpret_cast<const char*>(v_cache + row0 * row_elems + kvh * kHeadDim);
      const uint32_t lk = __builtin_amdgcn_readfirstlane(
          (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t*)&sK[buf][16 * wave * kHeadDim]);
      const uint32_t lv = __builtin_amdgcn_readfirstlane(
          (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t*)&sV[buf][16 * wave * kHeadDim]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lds_load16(kb, k_src[i], lk + i * 4 * kHeadDim * 2);
        lds_load16(vb, v_src[i], lv + i * 4 * kHeadDim * 2);
      }
      st_valid[buf] = page_ok ? min(kKeyTile, kend - key0) : 0;
      tile_ok[buf] = st_valid[buf] > 0;
    };
    // Once tile buf has landed: V rows past the valid keys become zeros (0 * a
    // stale NaN would poison O; stale K rows are masked in the scores).  Each
    // wave clears the rows it loaded.
    auto finish_tile = [&](int buf) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      const int valid = st_valid[buf];
      if (valid < kKeyTile) {  // wave-uniform: partial tiles only
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int q4 = 4 * wave + i, row = 4 * q4 + (lane >> 4);
          if (row >= valid)
            *reinterpret_cast<uint4*>(&sV[buf][q4 * 4 * kHeadDim + 8 * lane]) = make_uint4(0, 0, 0, 0);
        }
      }
    };

    // LDS operand addresses: per-lane bases fixed for the whole loop, with the
    // buffer, key block, dim block and key half as immediate offsets (the tile
    // loop is unrolled by buffer), so no address arithmetic is left per tile.
    // K operand of key block kb, dim slice c: row 16 kb + l16, logical chunk
    // 4c + g4, stored at physical chunk (4c + g4) ^ l16.
    uint32_t k_rd[4];  // LDS byte address of the lane's K chunk of slice c, buffer 0, key block 0
    {
      const uint32_t sk0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t*)&sK[0][0];
#pragma unroll
      for (int c = 0; c < 4; ++c) k_rd[c] = sk0 + (uint32_t)(l16 * kHeadDim * 2 + 16 * ((4 * c + g4) ^ l16));
    }
    // V^T transpose reads of dim block db, key half c: lane i points at row
    // R = 32c + 4 g4 + l16 / 4 (+16 for the second read), logical 8-byte piece
    // 4 db + l16 % 4, i.e. chunk 2 db + x with x = (l16 % 4) / 2, stored at
    // chunk (2 db + x) ^ (2 (R % 4) + 8 ((R / 4) % 2)) = 2 (db ^ w) + x with
    // w = (l16 / 4) % 4 + 4 (g4 % 2): byte 32 (db ^ w) + 16 x + 8 (l16 % 2) of
    // the row.  v_lane[db] holds that address for key half 0 of buffer 0.
    uint32_t v_lane[8];
    {
      const uint32_t sv0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t*)&sV[0][0];
      const int vrow = 4 * g4 + (l16 >> 2);
      const int vx = (l16 & 3) >> 1, w = ((l16 >> 2) & 3) + 4 * (g4 & 1);
#pragma unroll
      for (int d = 0; d < 8; ++d)
        v_lane[d] = sv0 + (uint32_t)(vrow * kHeadDim * 2 + 8 * (l16 & 1) + 16 * vx + 32 * (d ^ w));
    }

    float m_run[2] = {kNegBig, kNegBig};  // running max (log2 domain) per query
    f32x4_t acc_l[2];                     // row 0 (lanes 0-15): running sum of P (bf16) per query
    acc_l[0] = acc_l[1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    f32x4_t acc_o[2][8];                  // O^T[dim 16*db + 4*g4 + r][query]
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int db = 0; db < 8; ++db) acc_o[j][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // One tile: tile t sits in LDS buffer BUF (a compile-time constant).  The
    // next tile's loads are issued on every step (the last tile of a segment
    // reloads itself into the idle buffer), after the QK product when the tile
    // is computed, so every path through the loop leaves the same loads
    // outstanding and the compiler's waits stay at the LDS writes.
    auto tile_step = [&](int t, int t_last, auto buf_c) __attribute__((always_inline)) {
      constexpr int buf = decltype(buf_c)::value;
      const bool compute = tile_ok[buf];  // wave-uniform
      // The next tile's loads go out first: its buffer held tile t-1, done
      // before the last barrier.
      load_tile(min(t + 1, t_last), buf ^ 1);
      if (compute) {

      // ---- S^T = K Q^T for 4 blocks of 16 keys x 2 blocks of 16 queries ----
      // The K operands of dim slice c (4 key blocks, 16 rows = 4 KB apart) are
      // read two slices ahead of their MFMAs, three buffers in rotation.
      f32x4_t s[2][4];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) s[j][kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      {
        constexpr int kAhead = 2;
        u4v_t kop[kAhead + 1][4];
        auto kissue = [&](auto c_c) __attribute__((always_inline)) {
          constexpr int c = decltype(c_c)::value;
          constexpr int off = buf * kKeyTile * kHeadDim * 2;
          const uint32_t ad = k_rd[c];
          kop[c % (kAhead + 1)][0] = ds_read_b128_at<off>(ad);
          kop[c % (kAhead + 1)][1] = ds_read_b128_at<off + 4096>(ad);
          kop[c % (kAhead + 1)][2] = ds_read_b128_at<off + 8192>(ad);
          kop[c % (kAhead + 1)][3] = ds_read_b128_at<off + 12288>(ad);
        };
        static_for<0, kAhead>([&](auto c_c) __attribute__((always_inline)) { kissue(c_c); });
        static_for<0, 4>([&](auto c_c) __attribute__((always_inline)) {
          constexpr int c = decltype(c_c)::value, nxt = c + kAhead, st = c % (kAhead + 1);
          if constexpr (nxt < 4) kissue(std::integral_constant<int, nxt>{});
          // LDS reads still outstanding once slice c has arrived: the slices after it.
          constexpr int later = nxt < 4 ? kAhead : 3 - c;
          lgkm_wait_u4<4 * later>(kop[st][0], kop[st][1], kop[st][2], kop[st][3]);
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int j = 0; j < 2; ++j)
              s[j][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kop[st][kb]),
                                                                 qop[j][c], s[j][kb], 0, 0, 0);
        });
      }

      // ---- per query block: mask, online softmax, P^T packed to bf16 ----
      // Scores stay unscaled; p = exp2(s * scale_log2 - m).  The running max m
      // (scaled domain) is only raised when a tile's max exceeds it by more
      // than 8, so p <= 2^8 and the accumulator rescale is skipped on most
      // tiles (the final division uses the same m, so the result is exact).
      const int key_base = t * kKeyTile;
      // Whole tile visible to every query of this wave: no masking needed.
      const bool full = key_base + kKeyTile - 1 <= diag + wq0 && key_base + kKeyTile <= Lk &&
                        wq0 + kWaveQ <= Lq;
      bf16x8_t pop[2][2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (!full) {
          // key = key_base + 16 kb + 4 g4 + r is visible iff key <= min(my_pos, Lk - 1).
          const int lim = min(my_pos[j], Lk - 1) - key_base - 4 * g4;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              s[j][kb][r] = 16 * kb + r <= lim ? s[j][kb][r] : -INFINITY;
          }
        }
        // Chained so that each pair of maxima is one v_max3_f32.
        float tmax = fmaxf(fmaxf(s[j][0][0], s[j][0][1]), s[j][0][2]);
        tmax = fmaxf(fmaxf(tmax, s[j][0][3]), s[j][1][0]);
        tmax = fmaxf(fmaxf(tmax, s[j][1][1]), s[j][1][2]);
        tmax = fmaxf(fmaxf(tmax, s[j][1][3]), s[j][2][0]);
        tmax = fmaxf(fmaxf(tmax, s[j][2][1]), s[j][2][2]);
        tmax = fmaxf(fmaxf(tmax, s[j][2][3]), s[j][3][0]);
        tmax = fmaxf(fmaxf(tmax, s[j][3][1]), s[j][3][2]);
        tmax = fmaxf(tmax, s[j][3][3]);
        tmax = rows4_max(tmax);
        const float m_cand = tmax * scale_log2;
        const bool need = m_cand > m_run[j] + 8.f;
        if (__ballot(need) != 0ull) {  // wave-uniform
          const float m_new = need ? m_cand : m_run[j];
          const float alpha = fast_exp2(m_run[j] - m_new);
          m_run[j] = m_new;
          acc_l[j] *= alpha;
#pragma unroll
          for (int db = 0; db < 8; ++db) acc_o[j][db] *= alpha;
        }
        const float neg_m = -m_run[j];
        // chunk c packs key blocks 2c and 2c+1
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          float p[8];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            p[r] = fast_exp2(fmaf(s[j][2 * c][r], scale_log2, neg_m));
            p[4 + r] = fast_exp2(fmaf(s[j][2 * c + 1][r], scale_log2, neg_m));
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) pop[j][c][e] = (__bf16)p[e];
        }
      }

      // ---- O^T += V^T P^T: V^T operands by LDS transpose reads ----
      // Issued as inline asm with explicit LDS-counter waits, so the reads of
      // tile t do not wait for the global loads of tile t+1 (still in flight).
      {
        v2u_t r[2][2][2];  // [stage][c][lo/hi]
        auto issue = [&](auto db_c) __attribute__((always_inline)) {
          constexpr int db = decltype(db_c)::value, st = db & 1;
          constexpr int off0 = buf * kKeyTile * kHeadDim * 2;
          constexpr int off1 = off0 + 32 * kHeadDim * 2;  // keys 32 .. 63
          const uint32_t ad = v_lane[db];
          r[st][0][0] = ds_read_tr16_b64<off0>(ad);
          r[st][0][1] = ds_read_tr16_b64<off0 + 4096>(ad);
          r[st][1][0] = ds_read_tr16_b64<off1>(ad);
          r[st][1][1] = ds_read_tr16_b64<off1 + 4096>(ad);
        };
        issue(std::integral_constant<int, 0>{});
        static_for<0, 8>([&](auto db_c) __attribute__((always_inline)) {
          constexpr int db = decltype(db_c)::value, st = db & 1;
          if constexpr (db + 1 < 8) {
            issue(std::integral_constant<int, db + 1>{});
            lgkm_wait<4>(r[st][0][0], r[st][0][1], r[st][1][0], r[st][1][1]);
          } else {
            lgkm_wait<0>(r[st][0][0], r[st][0][1], r[st][1][0], r[st][1][1]);
          }
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const u32x4_t w4 = {r[st][c][0].x, r[st][c][0].y, r[st][c][1].x, r[st][c][1].y};
            const bf16x8_t vop = __builtin_bit_cast(bf16x8_t, w4);
#pragma unroll
            for (int j = 0; j < 2; ++j)
              acc_o[j][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[j][c], acc_o[j][db], 0, 0, 0);
          }
        });
      }
        // Row sums of P by MFMA: A = 16 x 32 with row 0 all ones.
        {
          const __bf16 one = (l16 == 0) ? (__bf16)1.0f : (__bf16)0.0f;
          const bf16x8_t ones = {one, one, one, one, one, one, one, one};
#pragma unroll
          for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int j = 0; j < 2; ++j)
              acc_l[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pop[j][c], acc_l[j], 0, 0, 0);
        }
      }
      finish_tile(buf ^ 1);
      __syncthreads();
    };
    // Segments of at most kSegTiles tiles span at most 61 pages, within the 64
    // lanes' page-table entries.
    constexpr int kSegTiles = 240;
    for (int seg = t_begin; seg < t_end; seg += kSegTiles) {
      const int seg_last = min(t_end, seg + kSegTiles) - 1;
      pg0 = seg * kKeyTile / kPage;
      pg_lane = pg0 + lane < bt_width ? block_table[(int64_t)b * bt_stride + pg0 + lane] : -1;
      // Consume the vector loads before the tile loop (page-table entries, Q
      // rows), so the compiler's wait for them is not repeated on every tile.
      asm volatile("" ::"v"(pg_lane));
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) asm volatile("" ::"v"(qop[j][c]));
      load_tile(seg, 0);
      finish_tile(0);
      __syncthreads();
      for (int t = seg; t <= seg_last; t += 2) {
        tile_step(t, seg_last, std::integral_constant<int, 0>{});
        if (t + 1 <= seg_last) tile_step(t + 1, seg_last, std::integral_constant<int, 1>{});
      }
    }

    float l_tot[2];  // row sums of P (row 0 of acc_l lives in lanes 0-15)
#pragma unroll
    for (int j = 0; j < 2; ++j) l_tot[j] = __shfl(acc_l[j][0], l16, 64);

    if (item.n_parts > 1) {
      // ---- split item: store the unnormalised rows, their max and sum ----
      int64_t slot, n_slots;
      if constexpr (kQueue) {
        slot = (int64_t)(q_pbase + part) * num_kv_heads + kvh;
        n_slots = (int64_t)pslot_cap * num_kv_heads;
      } else {
        slot = part_slot(kvh, b, qblk, part, n_split);
        n_slots = (int64_t)n_qblocks * gridDim.y * gridDim.x * n_split;
      }
      if constexpr (kQueue) {
        // Normalised rows in bf16, then (max, sum) per row in fp32.
        uint16_t* obase = reinterpret_cast<uint16_t*>(ws);
        float* ml = ws + n_slots * 128 * (kHeadDim / 2);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int row = wave * kWaveQ + 16 * j + l16;  // row of the item: head-major, then query
          if (wq0 + 16 * j + l16 < Lq) {
            const float inv = l_tot[j] > 0.f ? 1.0f / l_tot[j] : 0.f;
            uint16_t* orow = obase + (slot * 128 + row) * kHeadDim;
#pragma unroll
            for (int db = 0; db < 8; ++db)
              *reinterpret_cast<uint2*>(orow + db * 16 + 4 * g4) =
                  make_uint2(pack_bf16x2(acc_o[j][db][0] * inv, acc_o[j][db][1] * inv),
                             pack_bf16x2(acc_o[j][db][2] * inv, acc_o[j][db][3] * inv));
            if (g4 == 0)
              *reinterpret_cast<float2*>(ml + (slot * 128 + row) * 2) = make_float2(m_run[j], l_tot[j]);
          }
        }
      } else {
        float* ml = ws + n_slots * 128 * kHeadDim;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int row = wave * kWaveQ + 16 * j + l16;
          if (wq0 + 16 * j + l16 < Lq) {
            float* orow = ws + (slot * 128 + row) * kHeadDim;
#pragma unroll
            for (int db = 0; db < 8; ++db)
              *reinterpret_cast<f32x4_t*>(orow + db * 16 + 4 * g4) = acc_o[j][db];
            if (g4 == 0)
              *reinterpret_cast<float2*>(ml + (slot * 128 + row) * 2) = make_float2(m_run[j], l_tot[j]);
          }
        }
      }
      // The parts are combined by a merge kernel launched after this one.
      advance();
      continue;
    }

    // ---- normalise and write O[query][dims] ----
    // Staged through LDS (the K buffers are idle after the last tile's
    // barrier), so that the stores run along token rows: a lane's
    // accumulators hold 8-byte pieces of 16 query rows, which stored directly
    // would be 16 separate 32-byte pieces per store.  Staging row = query of
    // the block * G + head of the group; 16-byte chunk c of the row sits at
    // c ^ (query % 16), so the writes of a 16-lane group (16 queries) and the
    // row reads are free of bank conflicts.  With contiguous heads
    // (head stride 128) the G heads of a token are G x 256 contiguous bytes
    // and each lane stores 16 bytes; other strides store 8-byte halves.
    {
      uint16_t* stage = &sK[0][0];
      const int hg = wave / kWavesPerHead;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float inv = l_tot[j] > 0.f ? 1.0f / l_tot[j] : 0.f;
        const int qi = (wave % kWavesPerHead) * kWaveQ + 16 * j + l16;  // qi % 16 == l16
        uint16_t* srow = stage + (qi * G + hg) * kHeadDim;
#pragma unroll
        for (int db = 0; db < 8; ++db) {
          const uint32_t w0 = pack_bf16x2(acc_o[j][db][0] * inv, acc_o[j][db][1] * inv);
          const uint32_t w1 = pack_bf16x2(acc_o[j][db][2] * inv, acc_o[j][db][3] * inv);
          const int c16 = 2 * db + (g4 >> 1);  // chunk of dims 16 db + 4 g4 .. +3
          *reinterpret_cast<uint2*>(srow + 8 * (c16 ^ l16) + 4 * (g4 & 1)) = make_uint2(w0, w1);
        }
      }
      __syncthreads();
      // 16-byte chunks of the block's O: kQB x G x 256 bytes = 2048 chunks
      // for every G; thread t stores chunks t, t + 256, ...
      constexpr int kChunks = kQB * G * kHeadDim / 8;
      static_assert(kChunks % kThreads == 0, "output chunks per thread");
      const bool wide = out_head_stride == kHeadDim && out_tok_stride % 8 == 0 &&
                        (reinterpret_cast<uintptr_t>(out) & 15u) == 0;  // uniform
      const int rows_valid = min(kQB, Lq - q0);
      uint16_t* obase = out + (int64_t)(q_start + q0) * out_tok_stride + (int64_t)kvh * G * out_head_stride;
      // Opaque copy of the thread index: keeps the chunk addresses from being
      // hoisted out of the item loop (they would stay live across the tile
      // loop and push it over the register budget).
      int t_ep = tid;
      asm volatile("" : "+v"(t_ep));
#pragma unroll
      for (int i = 0; i < kChunks / kThreads; ++i) {
        const int id = i * kThreads + t_ep;
        const int tok = id / (G * 16), hgr = (id / 16) % G, c16 = id % 16;
        if (tok < rows_valid) {
          const uint4 v =
              *reinterpret_cast<const uint4*>(stage + (tok * G + hgr) * kHeadDim + 8 * (c16 ^ (tok & 15)));
          uint16_t* dst = obase + (int64_t)tok * out_tok_stride + (int64_t)hgr * out_head_stride + 8 * c16;
          if (wide) {
            *reinterpret_cast<uint4*>(dst) = v;
          } else {
            *reinterpret_cast<uint2*>(dst) = make_uint2(v.x, v.y);
            *reinterpret_cast<uint2*>(dst + 4) = make_uint2(v.z, v.w);
          }
        }
      }
      // The next item's first tile overwrites the staging rows only after
      // advance()'s barrier.
    }
    advance();
  }  // item loop

  if constexpr (kQueue) {
    // The last workgroup out resets the counters (every workgroup has taken
    // its final ticket by then), so the next launch finds them at zero.
    if (tid == 0 && atomicAdd(&queue[num_kv_heads], 1u) == gridDim.x - 1) {
      for (int h = 0; h <= num_kv_heads; ++h) atomicExch(&queue[h], 0u);
    }
  }
}

// Combines the parts of split items: O = sum_p 2^(m_p - M) O_p / sum_p 2^(m_p - M) l_p
// with M = max_p m_p (m in the scaled log2 domain of the attention kernel).
// Grid = (Hkv, B, 8 x query blocks): workgroup z covers rows 16 (z / n_qblocks)
// .. +15 of its item; thread t merges dims 8 (t % 16) .. +7 of row t / 16.
constexpr int kMergeRowGroups = 8;

template <int G>
__global__ __launch_bounds__(kThreads) void varlen_prefill_merge(
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k, int bt_width,
    int n_qblocks, int64_t total_q, uint16_t* __restrict__ out, int64_t out_tok_stride,
    int64_t out_head_stride, int n_split, int split_tiles, const float* __restrict__ ws) {
  constexpr int kQB = 128 / G;
  const int kvh = blockIdx.x, b = blockIdx.y;
  const int qblk = n_qblocks - 1 - (int)(blockIdx.z % n_qblocks);
  const int rgrp = (int)(blockIdx.z / n_qblocks);
  const int q0 = qblk * kQB;
  const Item item = item_geometry(cu_q, cu_k, b, q0, kQB, total_q, bt_width, n_split, split_tiles);
  if (q0 >= item.Lq || item.n_parts <= 1) return;
  const int row = rgrp * 16 + (threadIdx.x >> 4);
  const int d0 = 8 * (threadIdx.x & 15);
  const int qry = q0 + row % kQB;
  if (qry >= item.Lq) return;
  // part_slot() indexes with the attention grid's x / y, which this grid shares.
  const int64_t slot0 = part_slot(kvh, b, qblk, 0, n_split);
  const int64_t n_slots = (int64_t)n_qblocks * gridDim.y * gridDim.x * n_split;
  const float* ml = ws + n_slots * 128 * kHeadDim;
  float m_max = kNegBig;
  for (int p = 0; p < item.n_parts; ++p) m_max = fmaxf(m_max, ml[((slot0 + p) * 128 + row) * 2]);
  float l_sum = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int p = 0; p < item.n_parts; ++p) {
    const float2 mlp = *reinterpret_cast<const float2*>(ml + ((slot0 + p) * 128 + row) * 2);
    const float* op = ws + ((slot0 + p) * 128 + row) * kHeadDim + d0;
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(op);
    const f32x4_t c = *reinterpret_cast<const f32x4_t*>(op + 4);
    const float w = fast_exp2(mlp.x - m_max);
    l_sum = fmaf(w, mlp.y, l_sum);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = fmaf(w, a[e], o[e]);
      o[4 + e] = fmaf(w, c[e], o[4 + e]);
    }
  }
  const float inv = l_sum > 0.f ? 1.0f / l_sum : 0.f;
  const int qh = kvh * G + row / kQB;
  uint16_t* orow = out + (int64_t)(item.q_start + qry) * out_tok_stride + (int64_t)qh * out_head_stride + d0;
  *reinterpret_cast<uint2*>(orow) = make_uint2(pack_bf16x2(o[0] * inv, o[1] * inv), pack_bf16x2(o[2] * inv, o[3] * inv));
  *reinterpret_cast<uint2*>(orow + 4) = make_uint2(pack_bf16x2(o[4] * inv, o[5] * inv), pack_bf16x2(o[6] * inv, o[7] * inv));
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Parts per item for a launch.  split_keys == 0 (automatic): a launch with
// fewer items than kSplitMaxItems has its longest key range cut into enough
// parts to give ~kSplitTargetItems workgroups (bounded by kMaxSplit and by the
// tile count); larger launches are not split, since their workgroups already
// fill every CU and a split only adds the partial traffic and the merge.
// split_keys > 0: parts of split_keys keys whatever the launch size.
// Returns the number of parts and the tiles per part.
constexpr int64_t kSplitMaxItems = 256;
constexpr int64_t kSplitTargetItems = 512;
constexpr int64_t kMaxSplit = 16;

void prefill_splits(int64_t batch, int64_t n_qblocks, int64_t num_kv_heads, int64_t max_seqlen_k,
                    int64_t bt_width, int64_t split_keys, int64_t* n_split, int64_t* split_tiles) {
  *n_split = 1;
  *split_tiles = 1 << 30;
  const int64_t items = batch * n_qblocks * num_kv_heads;
  const int64_t max_keys = std::min(std::max<int64_t>(max_seqlen_k, 0), bt_width * kPage);
  const int64_t max_tiles = (max_keys + kKeyTile - 1) / kKeyTile;
  if (max_tiles <= 1) return;
  if (split_keys > 0) {
    *split_tiles = split_keys / kKeyTile;
    *n_split = std::min(kMaxSplit, (max_tiles + *split_tiles - 1) / *split_tiles);
  } else if (items < kSplitMaxItems) {
    const int64_t want = (kSplitTargetItems + items - 1) / items;
    *n_split = std::min({kMaxSplit, want, max_tiles});
    *split_tiles = (max_tiles + *n_split - 1) / *n_split;
  }
  if (*n_split <= 1) {
    *n_split = 1;
    *split_tiles = 1 << 30;
  }
}

int64_t split_workspace_bytes(int64_t batch, int64_t n_qblocks, int64_t num_kv_heads, int64_t n_split) {
  if (n_split <= 1) return 0;
  return batch * n_qblocks * num_kv_heads * n_split * 128 * (kHeadDim + 2) * (int64_t)sizeof(float);
}

// Queue mode: P = 2 workgroups per CU / Hkv per KV head; at most 2 P partial
// slots per head (a plan with more is run unsplit; parts are never shorter
// than T / P tiles, so the split items' parts add up to at most 2 P).
int64_t queue_per_head(int64_t num_kv_heads) {
  return std::max<int64_t>(1, 2 * (int64_t)device_cu_count() / num_kv_heads);
}
int64_t queue_pslot_cap(int64_t num_kv_heads) { return 2 * queue_per_head(num_kv_heads); }
// Start of the workspace: one ticket counter per KV head and one exit
// counter (zero between launches), then the split list of a thin launch
// (count + one word per split item); padded to 256 bytes.
int64_t queue_bytes(int64_t num_kv_heads) {
  const int64_t words = num_kv_heads + 2 + queue_pslot_cap(num_kv_heads);
  return (words * 4 + 255) / 256 * 256;
}
// Per (partial slot, KV head): 128 rows of bf16 O, then (max, sum) fp32.
int64_t queue_partial_bytes(int64_t num_kv_heads) {
  return queue_pslot_cap(num_kv_heads) * num_kv_heads * 128 * (kHeadDim * 2 + 8);
}
// Launches with at least kQueueMinItems and fewer than kQueueMaxItemsPerCu
// per CU (query block, sequence, KV head) items, and no forced split, run
// in queue mode; thicker launches fill the GPU for several rounds, and the
// hardware dispatcher balances them as well as the queue does.
constexpr int64_t kQueueMinItems = 256;
constexpr int64_t kQueueMaxItemsPerCu = 4;

// Combines the parts of the split items of a thin queue-mode launch, from
// the list the attention kernel's workgroup 0 wrote: workgroup (h, k, z)
// merges rows 64 z .. +63 of split item k for KV head h; thread t takes dims
// 32 (t % 4) .. +31 of row 64 z + t / 4.  Online over the parts (one round
// of loads per part): M = running max, O and l rescaled when it grows.
template <int G>
__global__ __launch_bounds__(kThreads) void varlen_prefill_queue_merge(
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k, int bt_width, int batch,
    int n_qblocks, int64_t total_q, uint16_t* __restrict__ out, int64_t out_tok_stride,
    int64_t out_head_stride, int pslot_cap, const uint32_t* __restrict__ splits,
    const float* __restrict__ ws) {
  constexpr int kQB = 128 / G;
  const int kvh = blockIdx.x, num_kv_heads = gridDim.x;
  const int k = blockIdx.y;
  if (k >= (int)splits[0]) return;
  const uint32_t e = splits[1 + k];
  const int i = (int)(e & 2047u), n_parts = (int)((e >> 11) & 31u), pbase = (int)(e >> 20);
  const int q0 = (n_qblocks - 1 - i / batch) * kQB;
  const Item item = item_geometry(cu_q, cu_k, i % batch, q0, kQB, total_q, bt_width, 1, 1 << 30);
  const int row = blockIdx.z * 64 + (threadIdx.x >> 2);
  const int d0 = 32 * (threadIdx.x & 3);
  const int qry = q0 + row % kQB;
  if (qry >= item.Lq) return;
  const int64_t n_slots = (int64_t)pslot_cap * num_kv_heads;
  const uint16_t* obase = reinterpret_cast<const uint16_t*>(ws);
  const float* ml = ws + n_slots * 128 * (kHeadDim / 2);
  // Part p holds o_p = O_p / l_p in bf16 and (m_p, l_p): the result is
  // sum_p w_p o_p / sum_p w_p with w_p = l_p 2^(m_p - M).
  float m = kNegBig, l = 0.f;
  float o[32];
#pragma unroll
  for (int x = 0; x < 32; ++x) o[x] = 0.f;
  for (int p = 0; p < n_parts; ++p) {
    const int64_t slot = (pbase + p) * (int64_t)num_kv_heads + kvh;
    const float2 mlp = *reinterpret_cast<const float2*>(ml + (slot * 128 + row) * 2);
    const uint4* op = reinterpret_cast<const uint4*>(obase + (slot * 128 + row) * kHeadDim + d0);
    uint4 v[4];
#pragma unroll
    for (int x = 0; x < 4; ++x) v[x] = op[x];
    const float mx = fmaxf(m, mlp.x);
    const float a = fast_exp2(m - mx), c = mlp.y * fast_exp2(mlp.x - mx);
    m = mx;
    l = fmaf(l, a, c);
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const uint32_t w[4] = {v[x].x, v[x].y, v[x].z, v[x].w};
#pragma unroll
      for (int y = 0; y < 4; ++y) {
        o[8 * x + 2 * y] = fmaf(o[8 * x + 2 * y], a, c * bf16_lo(w[y]));
        o[8 * x + 2 * y + 1] = fmaf(o[8 * x + 2 * y + 1], a, c * bf16_hi(w[y]));
      }
    }
  }
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  const int qh = kvh * G + row / kQB;
  uint16_t* orow =
      out + (int64_t)(item.q_start + qry) * out_tok_stride + (int64_t)qh * out_head_stride + d0;
#pragma unroll
  for (int x = 0; x < 4; ++x)
    *reinterpret_cast<uint4*>(orow + 8 * x) =
        make_uint4(pack_bf16x2(o[8 * x] * inv, o[8 * x + 1] * inv),
                   pack_bf16x2(o[8 * x + 2] * inv, o[8 * x + 3] * inv),
                   pack_bf16x2(o[8 * x + 4] * inv, o[8 * x + 5] * inv),
                   pack_bf16x2(o[8 * x + 6] * inv, o[8 * x + 7] * inv));
}

}  // namespace

extern "C" int64_t qmi_varlen_prefill_workspace_bytes(int64_t batch, int64_t max_seqlen_q,
                                                      int64_t max_seqlen_k, int64_t num_q_heads,
                                                      int64_t num_kv_heads, int64_t bt_width,
                                                      int64_t split_keys) {
  if (batch <= 0 || max_seqlen_q <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 ||
      num_q_heads % num_kv_heads != 0 || bt_width <= 0)
    return 0;
  if (split_keys < 0 || split_keys % kKeyTile) return 0;
  const int64_t G = num_q_heads / num_kv_heads;
  if (G != 1 && G != 2 && G != 4) return 0;
  const int64_t n_qblocks = (max_seqlen_q + 128 / G - 1) / (128 / G);
  int64_t n_split, split_tiles;
  prefill_splits(batch, n_qblocks, num_kv_heads, max_seqlen_k, bt_width, split_keys, &n_split,
                 &split_tiles);
  return queue_bytes(num_kv_heads) +
         std::max(queue_partial_bytes(num_kv_heads),
                  split_workspace_bytes(batch, n_qblocks, num_kv_heads, n_split));
}

extern "C" int qmi_varlen_prefill_attention(
    const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride, const uint16_t* k_cache,
    const uint16_t* v_cache, int64_t num_blocks, int64_t block_size, int64_t num_q_heads,
    int64_t num_kv_heads, int64_t head_dim, const int32_t* cu_seqlens_q,
    const int32_t* cu_seqlens_k, const int32_t* block_table, int64_t bt_stride, int64_t bt_width,
    int64_t batch, int64_t max_seqlen_q, int64_t max_seqlen_k, int64_t total_q, float scale,
    uint16_t* out, int64_t out_tok_stride, int64_t out_head_stride, float* workspace,
    int64_t workspace_bytes, int64_t split_keys, void* stream) {
  if (batch < 0 || max_seqlen_q < 0 || num_blocks < 0 || bt_width < 0) return QMI_E_BAD_SHAPE;
  if (total_q < 0 || workspace_bytes < 0) return QMI_E_BAD_SHAPE;
  if (split_keys < 0 || split_keys % kKeyTile) return QMI_E_BAD_SHAPE;
  if (batch == 0 || max_seqlen_q == 0 || total_q == 0) return QMI_OK;
  if (num_blocks == 0) return QMI_E_BAD_SHAPE;  // a pool without pages
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
  const int64_t qb = 128 / G;
  const int64_t n_qblocks = (max_seqlen_q + qb - 1) / qb;
  if (n_qblocks > 65535 || batch > 65535 || num_kv_heads > 65535 || bt_width > (1 << 22))
    return QMI_E_UNSUPPORTED;
  int64_t n_split, split_tiles;
  prefill_splits(batch, n_qblocks, num_kv_heads, max_seqlen_k, bt_width, split_keys, &n_split,
                 &split_tiles);
  const int64_t qbytes = queue_bytes(num_kv_heads);
  const bool ws_ok = workspace && aligned16(workspace) && workspace_bytes >= qbytes;
  // Queue mode: a persistent grid (two workgroups per CU) taking planned
  // units from per-KV-head counters, for launches of many items that do not
  // force a split.
  const int64_t n_items = batch * n_qblocks * num_kv_heads;
  const bool use_queue = ws_ok && split_keys == 0 && n_items >= kQueueMinItems &&
                         n_items < kQueueMaxItemsPerCu * device_cu_count() &&
                         workspace_bytes - qbytes >= queue_partial_bytes(num_kv_heads);
  if (use_queue) n_split = 1;
  float* part_ws = ws_ok ? workspace + qbytes / 4 : nullptr;
  // Without room for the parts the launch runs unsplit (same result).
  if (n_split > 1 && (!ws_ok || workspace_bytes - qbytes <
                                    split_workspace_bytes(batch, n_qblocks, num_kv_heads, n_split)))
    n_split = 1;
  if (n_qblocks * n_split > 65535 || n_qblocks * kMergeRowGroups > 65535) n_split = 1;
  if (n_split == 1) split_tiles = 1 << 30;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)num_kv_heads, (unsigned)batch, (unsigned)(n_qblocks * n_split));
  const dim3 merge_grid((unsigned)num_kv_heads, (unsigned)batch, (unsigned)(n_qblocks * kMergeRowGroups));
  const dim3 queue_grid((unsigned)(queue_per_head(num_kv_heads) * num_kv_heads));
  const int pslot_cap = (int)queue_pslot_cap(num_kv_heads);
  // Thin launch: no more items per KV head than workgroups per head; its
  // long items are split (and merged by a second kernel).
  const bool thin = use_queue && batch * n_qblocks <= std::min<int64_t>(queue_per_head(num_kv_heads),
                                                                         kPlanMaxItems);
  const dim3 qmerge_grid((unsigned)num_kv_heads, (unsigned)(pslot_cap / 2), 2u);
  const uint32_t* split_list = reinterpret_cast<const uint32_t*>(workspace) + num_kv_heads + 1;
  const float scale_log2 = scale * kLog2e;
  float* ws = (n_split > 1 || use_queue) ? part_ws : nullptr;
  unsigned* queue = reinterpret_cast<unsigned*>(workspace);
#define QMI_PREFILL_CASE(GG)                                                                      \
  case GG:                                                                                        \
    if (use_queue)                                                                                \
      hipLaunchKernelGGL((varlen_prefill_kernel<GG, true>), queue_grid, dim3(kThreads), 0, s, q,  \
                         q_tok_stride, q_head_stride, k_cache, v_cache, num_blocks,               \
                         (int)num_kv_heads, cu_seqlens_q, cu_seqlens_k, block_table, bt_stride,   \
                         (int)bt_width, (int)batch, (int)n_qblocks, total_q, scale_log2, out,     \
                         out_tok_stride, out_head_stride, 1, 1 << 30, ws, queue, (int)thin,       \
                         pslot_cap);                                                              \
    else                                                                                          \
      hipLaunchKernelGGL((varlen_prefill_kernel<GG, false>), grid, dim3(kThreads), 0, s, q,       \
                         q_tok_stride, q_head_stride, k_cache, v_cache, num_blocks,               \
                         (int)num_kv_heads, cu_seqlens_q, cu_seqlens_k, block_table, bt_stride,   \
                         (int)bt_width, (int)batch, (int)n_qblocks, total_q, scale_log2, out,     \
                         out_tok_stride, out_head_stride, (int)n_split, (int)split_tiles, ws,     \
                         nullptr, 0, 0);                                                          \
    if (thin)                                                                                     \
      hipLaunchKernelGGL(varlen_prefill_queue_merge<GG>, qmerge_grid, dim3(kThreads), 0, s,       \
                         cu_seqlens_q, cu_seqlens_k, (int)bt_width, (int)batch, (int)n_qblocks,   \
                         total_q, out, out_tok_stride, out_head_stride, pslot_cap, split_list,    \
                         ws);                                                                     \
    if (!use_queue && n_split > 1)                                                                \
      hipLaunchKernelGGL(varlen_prefill_merge<GG>, merge_grid, dim3(kThreads), 0, s,              \
                         cu_seqlens_q, cu_seqlens_k, (int)bt_width, (int)n_qblocks, total_q, out,  \
                         out_tok_stride, out_head_stride, (int)n_split, (int)split_tiles, ws);    \
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
