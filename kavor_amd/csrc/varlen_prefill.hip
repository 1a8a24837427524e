// Variable-length causal prefill attention (bf16 MFMA), dense or paged K/V.
//
// Restates flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
// max_seqlen_k, softmax_scale, causal=True, block_table) as called at
// kavor/layers/attention/flash_attention_kvcache.py:76-79: dense K/V for prefills with
// no cached prefix, the paged caches (block_table) when any sequence has a prefix-cache
// hit (flash_attention_kvcache.py:74-75, model_runner.py:432-433).  The causal mask is
// bottom-right aligned (flash-attn >= 2.1; the reference pins 2.8.3.post2, setup.py:10).
//
// Tiling (gfx950, wave64, v_mfma_f32_32x32x16_bf16)
//   A workgroup (4 waves, two resident per CU) owns one (sequence, kv head, query tile)
//   and all G query heads
//   of that kv head: 128 "rows" = 128/G query tokens x G heads, row rho = tok*G + g, so a
//   staged K/V tile feeds G heads.  Wave w owns rows [32w, 32w+32).
//   Per 64-key tile K and V go from memory straight into LDS with direct-to-LDS buffer
//   loads (double-buffered, one barrier per tile; the next tile's loads are in flight
//   during the MFMAs, and no register holds them),
//   then each wave computes S^T = K Q^T (M = 64 keys, N = 32 rows, K-dim = 128) and
//   O^T += V^T P^T (M = 128 dims, N = 32 rows, K-dim = 64 keys), reading the V^T operand
//   with the gfx950 LDS transpose load (ds_read_b64_tr_b16).  With the transposed
//   products every lane holds whole columns of its own query row (row = lane % 32), so
//   the online-softmax max / sum / rescale need only one exchange between the wave halves
//   (v_permlane32_swap, no LDS) and P feeds the second MFMA straight from registers.  The
//   softmax scale is folded into the exponent (exp2(fma(s, scale*log2 e, -m))).
//   Q stays in registers for the whole key loop (8 x 16 bytes per lane).
//   Work order: a one-workgroup plan kernel ranks the units of work (a pair of
//   neighbouring query tiles of one sequence and kv head) sequence by sequence, longest
//   sequence first, into a caller workspace; persistent workgroups (two per CU) then
//   claim them in that order from per-XCD counters, so the most expensive sequences start
//   first, a sequence's query tiles run together and stream its K/V through one XCD's L2,
//   and the cheap ones fill in behind them.
#include <math.h>

#include <algorithm>
#include <atomic>

#include "common.h"

namespace kvp {

constexpr int kPrefillHeadDim = 128;
constexpr int kPrefillWaves = 4;
constexpr int kPrefillThreads = 64 * kPrefillWaves;
constexpr int kPrefillRows = 32 * kPrefillWaves;  // query rows (token x head) per workgroup
constexpr int kKeyTile = 64;
constexpr int kXcdGroup = 2;  // neighbouring query tiles of one (sequence, kv head) per XCD
// Sequences per launch (the plan kernel's loop bound); larger batches run as consecutive
// launches.
constexpr int kMaxPrefillSeqs = 2048;
// Workspace of one launch: the per-XCD claim counters (each on its own 128-byte line),
// the unit count, then the unit pairs in decreasing cost, 32 bytes each.
constexpr int kClaimStride = 32;           // ints between claim counters
constexpr int kWsCountInt = 8 * kClaimStride;  // the unit count (int index)
constexpr int kWsUnitsInt = 512;           // first unit pair (int index; byte 2048)
constexpr int kUnitInts = 8;               // s, pair index, q start, q length, k start, k length, 0, 0
constexpr int kPlanThreads = 256;
constexpr int kPlanSeqsPerThread = kMaxPrefillSeqs / kPlanThreads;
constexpr int kPlanLevels = 2048;          // cost levels (64-key tiles) ranked apart; longer units tie at the top
constexpr int kPlanGroupSlots = 4096;      // first-block hash slots, more than kMaxPrefillSeqs: a probe always ends
static_assert(kPlanLevels % kPlanThreads == 0 && kMaxPrefillSeqs % kPlanThreads == 0, "plan shape");
// A tile's row sum of P above this re-bases the running max (P itself stays <= 2^16).
constexpr float kSpecSumLimit = 65536.f;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

struct PrefillParams {
  const uint16_t* q;
  int64_t q_tok_stride, q_head_stride;
  const uint16_t* k;
  int64_t k_blk_stride, k_tok_stride, k_head_stride;
  const uint16_t* v;
  int64_t v_blk_stride, v_tok_stride, v_head_stride;
  const int32_t* block_tables;
  int64_t bt_stride;
  int32_t num_cache_blocks;
  int32_t block_size;
  int32_t max_blocks;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int32_t num_seqs;
  int32_t pair_slots;
  int32_t num_kv_heads;
  float scale_log2;
  uint16_t* out;
  int64_t o_tok_stride, o_head_stride;
  int* ws;  // launch workspace: claim counters, unit count, ranked unit pairs
};

// Ranks the launch's units for the persistent attention workgroups.  A unit is a pair of
// neighbouring query tiles of one (sequence, kv head); unit j of a sequence with ntl query
// tiles starts at tile ntl - 1 - 2j (j < J; J = pair_slots covers max_seqlen_q).  Every
// unit of a sequence ranks at the sequence's key-tile count ceil(kl / 64), the cost of its
// last query tile and an upper bound on the cost of any of its tiles: the longest
// sequences go first, and a sequence's units are claimed together, so its query tiles read
// each K/V tile at about the same time and share it through one XCD's L2.  (Ranking each
// unit at its own cost spread a sequence's tiles over the whole call: on the
// prefix-cached 32-sequence workload 390 MB were read per call against 319 MB, on its dense
// form 320 MB against 164 MB, at equal or longer times.)  One workgroup histograms the
// (sequence, j) pairs by level, turns the histogram into offsets in decreasing level and
// places each pair; every kv head of a pair follows it in rank order.  It also zeroes the
// claim counters, so a workspace needs no clearing.  Pairs of one level are placed in no
// fixed order (the attention outputs do not depend on it), but the LDS atomics interleave
// the level's sequences pair index by pair index, so every sequence's longest pair is
// claimed before the shorter ones of its level (placing each sequence's pairs together
// read 250 MB instead of 279 MB but ran 1.7% slower).
// With block tables, sequences that start with the same cache block (a prefix-cache hit:
// their leading pages are shared) rank together at the level of the longest of them, so
// they run at the same time and the shared prefix passes through each XCD's L2 once for
// the group rather than once per sequence (316 -> 278 MB per call on the prefix-cached
// workload, same time).  An LDS hash table keyed by the first block id holds each group's
// largest level.
template <int G>
__global__ __launch_bounds__(kPlanThreads) void prefill_plan_kernel(const PrefillParams p) {
  constexpr int TOK = kPrefillRows / G;
  __shared__ int hist[kPlanLevels];
  __shared__ int wsum[kPlanThreads / 64];
  __shared__ int total;
  __shared__ int grp_key[kPlanGroupSlots];  // first block id, -1 for an empty slot
  __shared__ int grp_lvl[kPlanGroupSlots];  // the largest level of the sequences starting with it
  const int tid = threadIdx.x;
  const bool grouped = p.block_tables != nullptr && p.max_blocks > 0;
  // The launch's lengths and first block ids, loaded before the LDS is initialised so
  // that their round trip overlaps it.  Every sequence has a block-table row with at
  // least one entry, so the first entry is read whatever the lengths.
  int q0[kPlanSeqsPerThread], ql[kPlanSeqsPerThread], k0[kPlanSeqsPerThread], kl[kPlanSeqsPerThread];
  int b0[kPlanSeqsPerThread];
#pragma unroll
  for (int u = 0; u < kPlanSeqsPerThread; ++u) {
    const int sq = tid + kPlanThreads * u;
    q0[u] = ql[u] = k0[u] = kl[u] = 0;
    b0[u] = -1;
    if (sq < p.num_seqs) {
      q0[u] = p.cu_q[sq];
      ql[u] = p.cu_q[sq + 1];
      k0[u] = p.cu_k[sq];
      kl[u] = p.cu_k[sq + 1];
      if (grouped) b0[u] = p.block_tables[sq * p.bt_stride];
    }
  }
  for (int i = tid; i < kPlanLevels; i += kPlanThreads) hist[i] = 0;
  if (grouped) {
    for (int i = tid; i < kPlanGroupSlots; i += kPlanThreads) {
      grp_key[i] = -1;
      grp_lvl[i] = 0;
    }
  }
  if (tid < 8) p.ws[kClaimStride * tid] = 0;
  if (tid == 0) total = 0;
  __syncthreads();
  const int J = p.pair_slots;
  auto level = [&](int kl) { return min(max((kl + kKeyTile - 1) / kKeyTile, 0), kPlanLevels - 1); };
  // the hash slot of a first block id, inserted if absent (linear probing; fewer ids than
  // slots, so a free or matching slot is always found)
  auto group_slot = [&](int key) {
    int h = static_cast<int>((static_cast<uint32_t>(key) * 2654435769u) >> 20) & (kPlanGroupSlots - 1);
    for (int probe = 0; probe < kPlanGroupSlots; ++probe) {
      const int prev = atomicCAS(&grp_key[h], -1, key);
      if (prev == -1 || prev == key) return h;
      h = (h + 1) & (kPlanGroupSlots - 1);
    }
    return -1;
  };
  int gs[kPlanSeqsPerThread];  // group slot, -1 for a sequence ranked alone
  int mine = 0;
#pragma unroll
  for (int u = 0; u < kPlanSeqsPerThread; ++u) {
    ql[u] -= q0[u];
    kl[u] -= k0[u];
    gs[u] = -1;
    if (b0[u] >= 0 && kl[u] > 0 && ql[u] > 0) {
      gs[u] = group_slot(b0[u]);
      if (gs[u] >= 0) atomicMax(&grp_lvl[gs[u]], level(kl[u]));
    }
    mine += min(J, ((ql[u] + TOK - 1) / TOK + kXcdGroup - 1) / kXcdGroup);
  }
  if (mine) atomicAdd(&total, mine);
  __syncthreads();
  int lv[kPlanSeqsPerThread];
#pragma unroll
  for (int u = 0; u < kPlanSeqsPerThread; ++u) {
    lv[u] = gs[u] >= 0 ? grp_lvl[gs[u]] : level(kl[u]);
    const int nu = min(J, ((ql[u] + TOK - 1) / TOK + kXcdGroup - 1) / kXcdGroup);
    if (nu) atomicAdd(&hist[lv[u]], nu);
  }
  __syncthreads();
  // exclusive offsets in decreasing cost: thread t owns the kPlanLevels / kPlanThreads
  // levels just below the ones of thread t - 1
  constexpr int LPT = kPlanLevels / kPlanThreads;
  const int top = kPlanLevels - 1 - LPT * tid;
  int h[LPT], run = 0;
#pragma unroll
  for (int e = 0; e < LPT; ++e) {
    h[e] = hist[top - e];
    run += h[e];
  }
  const int incl = wave_incl_scan(run);
  if ((tid & 63) == 63) wsum[tid >> 6] = incl;
  __syncthreads();
  int before = incl - run;
  for (int w = 0; w < (tid >> 6); ++w) before += wsum[w];
#pragma unroll
  for (int e = 0; e < LPT; ++e) {
    hist[top - e] = before;
    before += h[e];
  }
  __syncthreads();
  int* units = p.ws + kWsUnitsInt;
#pragma unroll
  for (int u = 0; u < kPlanSeqsPerThread; ++u) {
    const int sq = tid + kPlanThreads * u;
    const int nu = min(J, ((ql[u] + TOK - 1) / TOK + kXcdGroup - 1) / kXcdGroup);
    for (int j = 0; j < nu; ++j) {
      const int pos = atomicAdd(&hist[lv[u]], 1);
      *reinterpret_cast<int4*>(units + kUnitInts * pos) = make_int4(sq, j, q0[u], ql[u]);
      *reinterpret_cast<int4*>(units + kUnitInts * pos + 4) = make_int4(k0[u], kl[u], 0, 0);
    }
  }
  if (tid == 0) p.ws[kWsCountInt] = total * p.num_kv_heads;
}

typedef short s16x4_t __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: 8 bytes per lane, transposed as 16-bit elements across each
// 16-lane group (see the V^T operand in the kernel).
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* lds_ptr) {
  const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4_t*)(lds_ptr));
  return __builtin_bit_cast(uint2, v);
}

// Max / sum of x over lanes l and l ^ 32 (v_permlane32_swap_b32 exchanges the wave halves:
// the first result holds lanes 0-31 in both halves, the second lanes 32-63).
__device__ __forceinline__ float half_swap_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_swap_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ f32x16_t mfma32(uint4 a, uint4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Two workgroups per CU (2 waves per SIMD, <= 256 registers per wave): the workgroups'
// barriers are independent, so one's MFMAs overlap the other's softmax (measured
// 1.45 -> 0.83 ms on the prefix-cached prefill workload vs one 4-wave workgroup per CU,
// 0.97 ms with one 8-wave workgroup).

template <int G, bool PAGED, bool CAUSAL>
__global__ __launch_bounds__(kPrefillThreads) __attribute__((amdgpu_waves_per_eu(2))) void varlen_prefill_kernel(const PrefillParams p) {
  constexpr int D = kPrefillHeadDim;
  constexpr int TOK = kPrefillRows / G;  // query tokens per tile

  // Work order.  The plan kernel listed the units sequence by sequence, longest first;
  // persistent workgroups claim them in that order, so the most expensive work starts
  // first and the cheap work fills in behind it (0.82 -> 0.58 ms for "last tiles first"
  // against (sequence, kv head, tile) order, then 0.457 -> 0.437 ms for a global cost
  // order, one workgroup per unit).  Claims come from one counter per XCD: workgroup b runs on
  // XCD b % 8 (the hardware deals workgroup ids round-robin to the 8 XCDs), claim c of
  // XCD x is rank 8 (c / 2) + x, and its two tiles go to two consecutive claims, so both
  // tiles of a unit, which read nearly the same K/V, run together on one XCD and share its
  // L2 (0.53 -> 0.50 ms).  Against one workgroup per unit with an in-kernel rank search:
  // prefix-cached 32-sequence prefill 365.5 -> 361.4 us, its dense form 96.1 -> 91.4 us
  // (plan kernel included; the persistent workgroups need no per-unit search, no
  // per-workgroup staging of the lengths and no empty workgroups).
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS bases and M0 stay scalar
  const int lane = tid & 63;
  const int n = lane & 31;   // this lane's query row within the wave
  const int hf = lane >> 5;  // which half of the MFMA K-dim this lane feeds

  // Two buffers of the K and V tiles (row-major, unpadded, 16-byte chunks XOR-swizzled
  // per row): tile i+1 is written while other waves may still read tile i.
  __shared__ __attribute__((aligned(16))) uint16_t s_k0[kKeyTile * kPrefillHeadDim];
  __shared__ __attribute__((aligned(16))) uint16_t s_k1[kKeyTile * kPrefillHeadDim];
  __shared__ __attribute__((aligned(16))) uint16_t s_v0[kKeyTile * kPrefillHeadDim];
  __shared__ __attribute__((aligned(16))) uint16_t s_v1[kKeyTile * kPrefillHeadDim];
  // Each unit's next claim is published in the slot of its unit count's parity: a slot is
  // rewritten two units later, after a barrier every wave has passed since reading it.
  __shared__ int s_claim[2];
  const int J = p.pair_slots;  // tile pairs per (sequence, kv head) the plan covers
  const int xcd = blockIdx.x & 7;
  int* const ctr = p.ws + kClaimStride * xcd;
  const int num_units = __builtin_amdgcn_readfirstlane(p.ws[kWsCountInt]);
  if (tid == 0) s_claim[0] = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  int claim = __builtin_amdgcn_readfirstlane(s_claim[0]);
  int cslot = 1;

  for (;;) {
  const int r = 8 * (claim / kXcdGroup) + xcd;  // rank in decreasing cost
  const int member = claim % kXcdGroup;         // which tile of the unit
  if (r >= num_units) break;             // uniform
  const int* ent = p.ws + kWsUnitsInt + kUnitInts * (r / p.num_kv_heads);
  const int kvh = r % p.num_kv_heads;
  const int s = __builtin_amdgcn_readfirstlane(ent[0]);
  const int jj = __builtin_amdgcn_readfirstlane(ent[1]);
  const int q_start = __builtin_amdgcn_readfirstlane(ent[2]);
  const int qlen = __builtin_amdgcn_readfirstlane(ent[3]);
  const int k_start = __builtin_amdgcn_readfirstlane(ent[4]);
  const int klen = __builtin_amdgcn_readfirstlane(ent[5]);
  const int diag = klen - qlen;  // bottom-right causal offset

  bool bad = false;
  if (PAGED && klen > p.max_blocks * p.block_size) bad = true;

  // Block-table entries 64 w .. 64 w + 63 of the sequence, one per lane, read with
  // readlane: a tile's block id then costs no memory round trip on the way to its K/V
  // loads.  Another window of 64 entries is loaded when the tiles move into it (once per
  // 64 blocks, i.e. 16,384 keys at block size 256).
  int bt_win = 0;
  int bt_lane = -1;
  if (PAGED && lane < p.max_blocks) bt_lane = p.block_tables[s * p.bt_stride + lane];

  // Tiles go from memory straight into LDS (lds_dma16: lane l of a wave writes 16 bytes
  // at the instruction's LDS base + 16 l), through a buffer resource over the tile's 64
  // key rows (a tile never crosses a page: block sizes are multiples of 64).  Wave w, instruction i
  // fills rows 4(4i + w) .. +3 of the unpadded [64 keys][128 dims] tile; lane l covers
  // row 4(4i + w) + l/16 and physical chunk l % 16, which holds logical chunk
  // pc ^ swz(row): K rows are swizzled by (row & 15), V rows by 4 (row & 3).  Keys past
  // the context are clamped onto its last key; their scores are masked.  Every wave of the
  // workgroup looks up the same block ids, so `bad` is uniform over the workgroup.
  // Per-lane parts of the tile load offsets.  Lane l of an instruction covers row
  // r0 + l/16 (r0 a multiple of 4) and physical chunk l % 16; its logical chunk is
  // (l % 16) ^ (r & 15) for K and (l % 16) ^ 4 (r & 3) for V, where r & 15 = (r0 + l/16) & 15
  // is the same for the 4 instructions of a wave (r0 = 4 (4 i + w)) and r & 3 = (l/16) & 3.
  const int k_row_bytes = static_cast<int>(p.k_tok_stride) * 2;
  const int v_row_bytes = static_cast<int>(p.v_tok_stride) * 2;
  const int k_lane_off = (lane >> 4) * k_row_bytes;
  const int v_lane_off = (lane >> 4) * v_row_bytes;
  const int k_chunk_off = 16 * ((lane & 15) ^ ((4 * wave + (lane >> 4)) & 15));
  const int v_chunk_off = 16 * ((lane & 15) ^ (4 * ((lane >> 4) & 3)));
  // Paged instance: full tiles load from per-lane offsets fixed for the whole kernel (row
  // 4 (4 i + w) + l/16 and the lane's swizzled chunk; only a sequence's last, partial tile
  // clamps rows onto its last key), and K and V share one block lookup per block, with the
  // tile bases advanced by additions.  Per tile this leaves about 45 scalar instructions
  // instead of 107 (two divisions by the block size, two lookups, 64-bit products) and no
  // vector ones instead of 22: 383.9 -> 377.9 us on the prefix-cached 32-sequence
  // workload, same outputs.
  // (paged instance only: the dense one keeps its clamped offsets, which measured faster
  // there under its higher register pressure)
  constexpr int NOFF = PAGED ? kKeyTile / 4 / kPrefillWaves : 1;
  int k_off[NOFF], v_off[NOFF];
#pragma unroll
  for (int i = 0; i < (PAGED ? NOFF : 0); ++i) {
    const int r0 = 4 * (kPrefillWaves * i + wave);
    k_off[i] = k_lane_off + r0 * k_row_bytes + k_chunk_off;
    v_off[i] = v_lane_off + r0 * v_row_bytes + v_chunk_off;
  }
  // Tiles are issued in key order from key 0 for each query tile, so the page position
  // advances without a division: the tile's logical block and its offset in that block,
  // with the block's K and V bases (kv head included) looked up once per block.
  int nx_lblk = 0, nx_boff = 0;
  const uint16_t* k_tile = nullptr;
  const uint16_t* v_tile = nullptr;
  const int64_t k_tile_step = PAGED ? static_cast<int64_t>(kKeyTile) * p.k_tok_stride : 0;
  const int64_t v_tile_step = PAGED ? static_cast<int64_t>(kKeyTile) * p.v_tok_stride : 0;
  auto issue_kv = [&](int kv0, uint16_t* dk, uint16_t* dv) __attribute__((always_inline)) {
    if (kv0 == 0) {  // uniform: a query tile's first key tile
      nx_lblk = 0;
      nx_boff = 0;
      if (!PAGED) {
        k_tile = p.k + static_cast<int64_t>(k_start) * p.k_tok_stride + static_cast<int64_t>(kvh) * p.k_head_stride;
        v_tile = p.v + static_cast<int64_t>(k_start) * p.v_tok_stride + static_cast<int64_t>(kvh) * p.v_head_stride;
      }
    }
    if (PAGED && nx_boff == 0) {  // uniform: the tile starts a block
      const int lblk = nx_lblk;
      const int w = lblk >> 6;
      if (w != bt_win) {  // uniform
        bt_lane = 64 * w + lane < p.max_blocks ? p.block_tables[s * p.bt_stride + 64 * w + lane] : -1;
        bt_win = w;
      }
      int blk = lblk < p.max_blocks ? __builtin_amdgcn_readlane(bt_lane, lblk & 63) : -1;
      if (blk < 0 || blk >= p.num_cache_blocks) {
        bad = true;
        blk = 0;
      }
      k_tile = p.k + static_cast<int64_t>(blk) * p.k_blk_stride + static_cast<int64_t>(kvh) * p.k_head_stride;
      v_tile = p.v + static_cast<int64_t>(blk) * p.v_blk_stride + static_cast<int64_t>(kvh) * p.v_head_stride;
    }
    const BufferRsrc krs = buffer_rsrc(k_tile, static_cast<uint32_t>(kKeyTile * k_row_bytes));
    const BufferRsrc vrs = buffer_rsrc(v_tile, static_cast<uint32_t>(kKeyTile * v_row_bytes));
    if (kv0 + kKeyTile <= klen) {  // uniform: every row of the tile is a key
#pragma unroll
      for (int i = 0; i < kKeyTile / 4 / kPrefillWaves; ++i)
        lds_dma16(krs, k_off[i % NOFF], &dk[4 * (kPrefillWaves * i + wave) * kPrefillHeadDim]);
#pragma unroll
      for (int i = 0; i < kKeyTile / 4 / kPrefillWaves; ++i)
        lds_dma16(vrs, v_off[i % NOFF], &dv[4 * (kPrefillWaves * i + wave) * kPrefillHeadDim]);
    } else {
      // byte offset of key min(r, last): min(r * stride, last * stride), r = r0 + lane / 16
      const int k_last = (klen - 1 - kv0) * k_row_bytes;
      const int v_last = (klen - 1 - kv0) * v_row_bytes;
#pragma unroll
      for (int i = 0; i < kKeyTile / 4 / kPrefillWaves; ++i) {
        const int r0 = 4 * (kPrefillWaves * i + wave);
        lds_dma16(krs, min(k_lane_off + r0 * k_row_bytes, k_last) + k_chunk_off, &dk[r0 * kPrefillHeadDim]);
      }
#pragma unroll
      for (int i = 0; i < kKeyTile / 4 / kPrefillWaves; ++i) {
        const int r0 = 4 * (kPrefillWaves * i + wave);
        lds_dma16(vrs, min(v_lane_off + r0 * v_row_bytes, v_last) + v_chunk_off, &dv[r0 * kPrefillHeadDim]);
      }
    }
    k_tile += k_tile_step;
    v_tile += v_tile_step;
    nx_boff += kKeyTile;
    if (PAGED && nx_boff == p.block_size) {
      nx_boff = 0;
      ++nx_lblk;
    }
  };

  auto issue_k = [&](int kv0, uint16_t* dk) __attribute__((always_inline)) {
    int64_t kbase = 0;
    if (PAGED) {
      const int lblk = kv0 / p.block_size;
      const int w = lblk >> 6;
      if (w != bt_win) {  // uniform
        bt_lane = 64 * w + lane < p.max_blocks ? p.block_tables[s * p.bt_stride + 64 * w + lane] : -1;
        bt_win = w;
      }
      int blk = lblk < p.max_blocks ? __builtin_amdgcn_readlane(bt_lane, lblk & 63) : -1;
      if (blk < 0 || blk >= p.num_cache_blocks) {
        bad = true;
        blk = 0;
      }
      kbase = static_cast<int64_t>(blk) * p.k_blk_stride + static_cast<int64_t>(kv0 - lblk * p.block_size) * p.k_tok_stride;
    } else {
      kbase = static_cast<int64_t>(k_start + kv0) * p.k_tok_stride;
    }
    const uint16_t* kb = p.k + kbase + static_cast<int64_t>(kvh) * p.k_head_stride;
    const BufferRsrc krs = buffer_rsrc(kb, static_cast<uint32_t>(kKeyTile * p.k_tok_stride * 2));
    // byte offset of key min(r, last): min(r * stride, last * stride) * 2, r = r0 + lane / 16
    const int last_off = (klen - 1 - kv0) * k_row_bytes;
#pragma unroll
    for (int i = 0; i < kKeyTile / 4 / kPrefillWaves; ++i) {
      const int r0 = 4 * (kPrefillWaves * i + wave);
      lds_dma16(krs, min(k_lane_off + r0 * k_row_bytes, last_off) + k_chunk_off, &dk[r0 * kPrefillHeadDim]);
    }
  };
  auto issue_v = [&](int kv0, uint16_t* dv) __attribute__((always_inline)) {
    int64_t vbase = 0;
    if (PAGED) {
      const int lblk = kv0 / p.block_size;
      const int w = lblk >> 6;
      if (w != bt_win) {  // uniform
        bt_lane = 64 * w + lane < p.max_blocks ? p.block_tables[s * p.bt_stride + 64 * w + lane] : -1;
        bt_win = w;
      }
      int blk = lblk < p.max_blocks ? __builtin_amdgcn_readlane(bt_lane, lblk & 63) : -1;
      if (blk < 0 || blk >= p.num_cache_blocks) {
        bad = true;
        blk = 0;
      }
      vbase = static_cast<int64_t>(blk) * p.v_blk_stride + static_cast<int64_t>(kv0 - lblk * p.block_size) * p.v_tok_stride;
    } else {
      vbase = static_cast<int64_t>(k_start + kv0) * p.v_tok_stride;
    }
    const uint16_t* vb = p.v + vbase + static_cast<int64_t>(kvh) * p.v_head_stride;
    const BufferRsrc vrs = buffer_rsrc(vb, static_cast<uint32_t>(kKeyTile * p.v_tok_stride * 2));
    const int last_off = (klen - 1 - kv0) * v_row_bytes;
#pragma unroll
    for (int i = 0; i < kKeyTile / 4 / kPrefillWaves; ++i) {
      const int r0 = 4 * (kPrefillWaves * i + wave);
      lds_dma16(vrs, min(v_lane_off + r0 * v_row_bytes, last_off) + v_chunk_off, &dv[r0 * kPrefillHeadDim]);
    }
  };

  // V^T operand of O^T = V^T P^T via the LDS transpose read: within each 16-lane group
  // ds_read_b64_tr_b16 hands lane i element e = element (i % 4) of the 8 bytes addressed
  // by lane 4e + i/4.  Lane L therefore addresses key 4*hf + (L%16)/4 (+16kk, +8 for the
  // upper half) at dims 32mb + 16*((L/16)%2) + 4*(L%4): it receives dim 32mb + L%32 of
  // keys 4hf + e, which is the key order of this lane's P registers.
  const int tr_key = 4 * hf + ((lane & 15) >> 2);
  const int tr_dim = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const int tr_chunk = tr_dim >> 3, tr_sub = tr_dim & 7;

  const int ntiles_seq = (qlen + TOK - 1) / TOK;
  // This unit's tile pairs jj, jj + J, jj + 2J, ... counted from the last tile (more
  // than one only when max_seqlen_q understates the sequence); member 0 takes the later
  // tile of each pair, member 1 the earlier one.
  for (int t = kXcdGroup * jj + member; t < ntiles_seq; t += kXcdGroup * J) {
    const int tile = ntiles_seq - 1 - t;
    const int q0 = tile * TOK;

    // This lane's query row.
    const int rho = 32 * wave + n;
    const int tq = rho / G;
    const int g = rho - tq * G;
    const int qi = q0 + tq;  // query index within the sequence
    // rows past the tile's TOK whole tokens (G = 5: 125 of 128) are padding
    const bool row_valid = tq < TOK && qi < qlen;

    uint4 qreg[D / 16];
    {
      const uint16_t* qp = p.q + static_cast<int64_t>(q_start + qi) * p.q_tok_stride +
                           static_cast<int64_t>(kvh * G + g) * p.q_head_stride + 8 * hf;
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks)
        qreg[ks] = row_valid ? *reinterpret_cast<const uint4*>(qp + 16 * ks) : make_uint4(0, 0, 0, 0);
    }

    const int q_last = min(qlen, q0 + TOK) - 1;
    const int kv_end = CAUSAL ? min(klen, q_last + diag + 1) : klen;
    const int nkv = kv_end > 0 ? (kv_end + kKeyTile - 1) / kKeyTile : 0;

    f32x16_t oacc[D / 32];
#pragma unroll
    for (int mb = 0; mb < D / 32; ++mb)
#pragma unroll
      for (int j = 0; j < 16; ++j) oacc[mb][j] = 0.f;
    float m_run = kMaxFloor, l_run = 0.f;
    const int row_limit = CAUSAL ? qi + diag : klen - 1;  // last key this row may see
    // smallest row_limit over this wave's rows (its first query token)
    const int wave_min_limit = CAUSAL ? q0 + (32 * wave) / G + diag : klen - 1;
    // last key any row of this wave may see; no row of the wave is a query when its first
    // token is past the sequence (padding rows of the last query tile)
    const int wave_max_limit = CAUSAL ? q0 + (32 * wave + 31) / G + diag : klen - 1;
    const bool wave_live = q0 + (32 * wave) / G < qlen;

    if (nkv > 0) {
      if constexpr (PAGED) {
        issue_kv(0, s_k0, s_v0);
      } else {
        issue_k(0, s_k0);
        issue_v(0, s_v0);
      }
    }
    auto tile_step = [&](int it, const uint16_t* sk, const uint16_t* sv, uint16_t* nk, uint16_t* nv)
                         __attribute__((always_inline)) {
      const int kv0 = it * kKeyTile;
      // this wave's share of tile `it` has landed; after the barrier every wave's has, and
      // every wave is done with tile it-1's buffers
      wait_vmem<0>();
      __syncthreads();
      if (it + 1 < nkv) {  // in flight during the MFMAs
        if constexpr (PAGED) {
          issue_kv(kv0 + kKeyTile, nk, nv);
        } else {
          issue_k(kv0 + kKeyTile, nk);
          issue_v(kv0 + kKeyTile, nv);
        }
      }
      // Nothing to compute when no row of the wave sees a key of this tile: the tile would
      // add exact zeros.  The SIMD is left to the other workgroup's wave.
      if (!wave_live || kv0 > wave_max_limit) return;

      // ---- S^T = K Q^T : two 32-key blocks, lane holds keys of its own query row
      f32x16_t sacc[2];
      // MFMA blocks run at wave priority 1 and the softmax at 0: of the two waves a SIMD
      // holds, the one with matrix work issues first and the other's VALU fills in.
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int j = 0; j < 16; ++j) sacc[mb][j] = 0.f;
      {
        // Step st = (ks = st / 2, mb = st % 2): consecutive MFMAs are independent, and a
        // ring of four K fragments keeps four LDS reads in flight ahead of the MFMAs
        // (the compiler's own order waited on a fresh read before every other MFMA;
        // 0.459 -> 0.456 ms on the prefix-cached 32-sequence workload, same bits).
        const uint16_t* krow = &sk[n * kPrefillHeadDim];
        const int ksw = n & 15;
        uint4 ka[4];
#pragma unroll
        for (int st = 0; st < 4; ++st)
          ka[st] = *reinterpret_cast<const uint4*>(krow + (st & 1) * 32 * kPrefillHeadDim + 8 * ((2 * (st >> 1) + hf) ^ ksw));
#pragma unroll
        for (int st = 0; st < 2 * (D / 16); ++st) {
          sacc[st & 1] = mfma32(ka[st & 3], qreg[st >> 1], sacc[st & 1]);
          if (st + 4 < 2 * (D / 16))
            ka[st & 3] = *reinterpret_cast<const uint4*>(krow + ((st + 4) & 1) * 32 * kPrefillHeadDim + 8 * ((2 * ((st + 4) >> 1) + hf) ^ ksw));
        }
        // Pin that order: 4 LDS reads, then (MFMA, LDS read) x 12, then the last 4 MFMAs.
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int st = 0; st < 2 * (D / 16) - 4; ++st) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
      }

      __builtin_amdgcn_s_setprio(0);
      // ---- online softmax over this tile (base 2), against the running max without
      // this tile's own maximum: only the query tile's first key tile takes its maximum.
      // P is exact enough in bf16 at any magnitude (the relative precision does not
      // depend on it), so the running max may lag the true one; a row whose tile sum
      // exceeds 2^16 (a score more than 16 above the running max, or an overflow) makes
      // the wave take the tile's maximum, rescale O and form P again.  Skipping the
      // per-tile maximum (16 v_max3, a half swap, a compare per lane): 384.2 -> 376.6 us
      // on the prefix-cached 32-sequence workload, dense 98.6 -> 95.8 us, same outputs
      // there (the maximum never moved past the first tile's by 2^8).  Interior tiles
      // (every key visible to every row of the wave) skip the mask.
      const bool interior = kv0 + kKeyTile - 1 <= min(klen - 1, wave_min_limit);
      if (!interior) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int key = kv0 + 32 * mb + 8 * (j >> 2) + 4 * hf + (j & 3);
            const bool ok = key < klen && key <= row_limit;
            sacc[mb][j] = ok ? sacc[mb][j] : -INFINITY;
          }
      }
      // the row's maximum over this tile, scaled to base 2 (raw scores: scale > 0 keeps
      // their order; a row without a visible key keeps the finite floor)
      auto tile_max = [&]() __attribute__((always_inline)) {
        float mx = kMaxFloor;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int j = 0; j < 16; ++j) mx = fmaxf(mx, sacc[mb][j]);
        return half_swap_max(mx) * p.scale_log2;
      };
      if (it == 0) m_run = tile_max();  // uniform; O and l are still zero
      float rsum = 0.f;
      u32 pk[2][8];  // P as packed bf16 pairs: [mb][pair]
      auto make_p = [&]() __attribute__((always_inline)) {
        rsum = 0.f;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int j = 0; j < 16; j += 2) {
            const float p0 = fast_exp2(fmaf(sacc[mb][j], p.scale_log2, -m_run));
            const float p1 = fast_exp2(fmaf(sacc[mb][j + 1], p.scale_log2, -m_run));
            rsum += p0 + p1;
            pk[mb][j >> 1] = pack_bf16x2(p0, p1);
          }
        rsum = half_swap_sum(rsum);
      };
      make_p();
      if (__any(!(rsum <= kSpecSumLimit))) {  // rare: the running max is re-based
        const float m_new = fmaxf(m_run, tile_max());
        const float alpha = fast_exp2(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int mb = 0; mb < D / 32; ++mb)
#pragma unroll
          for (int j = 0; j < 16; ++j) oacc[mb][j] *= alpha;
        make_p();
      }
      l_run += rsum;

      // ---- O^T += V^T P^T : K-dim step kk covers keys 16kk..16kk+15.  This lane's P
      // registers for that step hold key offsets {4hf+0..3, 8+4hf+0..3}.
      __builtin_amdgcn_s_setprio(1);
      {
        // The V^T fragments of step kk + 1 are read while the MFMAs of step kk run; the
        // schedule below pins that order (the compiler's own waited on each step's reads
        // before its first MFMA: 0.440 -> 0.431 ms on the prefix-cached 32-sequence
        // workload, same bits).
        uint4 vf[2][D / 32];
        auto read_v = [&](int kk, uint4 (&dst)[D / 32]) __attribute__((always_inline)) {
#pragma unroll
          for (int mb = 0; mb < D / 32; ++mb) {
            const uint16_t* vp = &sv[(16 * kk + tr_key) * kPrefillHeadDim + 8 * ((4 * mb + tr_chunk) ^ (lane & 12)) + tr_sub];
            const uint2 lo = lds_read_tr16(vp);
            const uint2 hi = lds_read_tr16(vp + 8 * kPrefillHeadDim);
            dst[mb] = make_uint4(lo.x, lo.y, hi.x, hi.y);
          }
        };
        read_v(0, vf[0]);
#pragma unroll
        for (int kk = 0; kk < kKeyTile / 16; ++kk) {
          if (kk + 1 < kKeyTile / 16) read_v(kk + 1, vf[(kk + 1) & 1]);
          const int mbs = kk >> 1;
          const int pj = (kk & 1) * 4;  // first packed pair of this step within pk[mbs]
          const uint4 b = make_uint4(pk[mbs][pj], pk[mbs][pj + 1], pk[mbs][pj + 2], pk[mbs][pj + 3]);
#pragma unroll
          for (int mb = 0; mb < D / 32; ++mb) oacc[mb] = mfma32(vf[kk & 1][mb], b, oacc[mb]);
        }
        // 8 LDS reads (step 0), then (2 reads of step kk + 1, 1 MFMA of step kk) x 12,
        // then the last step's 4 MFMAs.
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
        for (int i = 0; i < (kKeyTile / 16 - 1) * (D / 32); ++i) {
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, D / 32, 0);
      }
    };
    for (int it = 0; it < nkv; it += 2) {
      tile_step(it, s_k0, s_v0, s_k1, s_v1);
      if (it + 1 < nkv) tile_step(it + 1, s_k1, s_v1, s_k0, s_v0);
    }
    __builtin_amdgcn_s_setprio(0);
    __syncthreads();  // every wave is done with the tile buffers (the next unit restages them)

    // ---- write O through LDS.  The lane holds dims 32mb + 8(j/4) + 4hf + (j%4) of its
    // query row, so a direct store writes 16 bytes into each of 32 rows; staged in the
    // finished tile buffers (each wave its own 32 rows, rewritten by the next query tile's
    // second key tile only after that tile's barrier), every store instruction writes
    // whole rows.  A row's 16-byte chunk c sits at chunk c ^ (row & 15) and its 8-byte
    // halves swap for rows 16..31, so neither the 8-byte writes nor the 16-byte reads
    // share a bank.  Dense 32-sequence prefill 92.9 -> 88.1 us, prefix-cached 343.0 ->
    // 341.1 us, same outputs.
    {
      const float inv = bad ? NAN : (l_run > 0.f ? 1.f / l_run : 0.f);
      uint16_t* const stg = (wave < 2 ? s_k1 : s_v1) + (wave & 1) * 32 * kPrefillHeadDim;
      // lane index recomputed here: offsets derived from it are not hoisted out of the
      // unit loop (where they would hold 24 registers through the key loop)
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int nn = ln & 31, hh = ln >> 5;
      const int hsw = (nn >> 4) & 1;
#pragma unroll
      for (int mb = 0; mb < D / 32; ++mb)
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
          const int c = 4 * mb + jq;
          const uint2 w = make_uint2(pack_bf16x2(oacc[mb][4 * jq] * inv, oacc[mb][4 * jq + 1] * inv),
                                     pack_bf16x2(oacc[mb][4 * jq + 2] * inv, oacc[mb][4 * jq + 3] * inv));
          *reinterpret_cast<uint2*>(stg + nn * kPrefillHeadDim + 8 * (c ^ (nn & 15)) + 4 * (hh ^ hsw)) = w;
        }
      __builtin_amdgcn_wave_barrier();  // a wave's LDS accesses run in order
      const int chunk = ln & 15;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int row = 4 * i + (ln >> 4);
        uint4 v = *reinterpret_cast<const uint4*>(stg + row * kPrefillHeadDim + 8 * (chunk ^ (row & 15)));
        if ((row >> 4) & 1) v = make_uint4(v.z, v.w, v.x, v.y);
        const int rho_o = 32 * wave + row;
        const int tq_o = rho_o / G;
        const int qi_o = q0 + tq_o;
        if (tq_o < TOK && qi_o < qlen) {
          uint16_t* op = p.out + static_cast<int64_t>(q_start + qi_o) * p.o_tok_stride +
                         static_cast<int64_t>(kvh * G + rho_o - tq_o * G) * p.o_head_stride + 8 * chunk;
          *reinterpret_cast<uint4*>(op) = v;
        }
      }
    }
  }
  // The next claim is taken only now, when the workgroup is ready to start it: the two
  // tiles of a unit are consecutive claims of one XCD, so claiming when a unit ends
  // starts them close together and the second reads the shared K/V from that XCD's L2.
  // Claiming when a unit starts (to hide the atomic's latency) started them up to a unit
  // apart: prefix-cached 32-sequence prefill 360.0 -> 349.3 us, reads 521 -> 386 MB per
  // call.  The co-resident workgroup covers the atomic's round trip.
  if (tid == 0) s_claim[cslot] = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  claim = __builtin_amdgcn_readfirstlane(s_claim[cslot]);
  cslot ^= 1;
  }  // next unit
}

// Workgroups of one kernel variant resident on the current device (cached per variant and
// device), rounded down to whole groups of 16 (one pair on each XCD).
template <int G, bool PAGED, bool CAUSAL>
static int64_t prefill_resident() {
  static std::atomic<int64_t> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int64_t v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int per_cu = 0, cus = 0;
  bool ok = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, varlen_prefill_kernel<G, PAGED, CAUSAL>,
                                                         kPrefillThreads, 0) == hipSuccess && per_cu >= 1;
  if (!ok) per_cu = 1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) {
    cus = 16;
    ok = false;
  }
  v = std::max<int64_t>(16, static_cast<int64_t>(per_cu) * cus / 16 * 16);
  if (ok) cache[dev].store(v, std::memory_order_relaxed);
  return v;
}

// The plan kernel ranks the launch's units into the workspace, then the resident count of
// persistent workgroups (a multiple of 16, so each XCD holds the same number) claims them.
template <int G, bool PAGED, bool CAUSAL>
static void launch_variant(hipStream_t s, const PrefillParams& p) {
  hipLaunchKernelGGL((prefill_plan_kernel<G>), dim3(1), dim3(kPlanThreads), 0, s, p);
  const int64_t grid = prefill_resident<G, PAGED, CAUSAL>();
  hipLaunchKernelGGL((varlen_prefill_kernel<G, PAGED, CAUSAL>), dim3(static_cast<unsigned>(grid)),
                     dim3(kPrefillThreads), 0, s, p);
}

template <int G>
static void launch_prefill(bool paged, bool causal, hipStream_t s, const PrefillParams& p) {
  if (paged) {
    if (causal) launch_variant<G, true, true>(s, p);
    else launch_variant<G, true, false>(s, p);
  } else {
    if (causal) launch_variant<G, false, true>(s, p);
    else launch_variant<G, false, false>(s, p);
  }
}

// Tile pairs per (sequence, kv head) that cover max_seqlen_q query tokens at GQA ratio g.
static int64_t prefill_pair_slots(int64_t max_seqlen_q, int g) {
  const int64_t tok_per_tile = kPrefillRows / g;
  return ((max_seqlen_q + tok_per_tile - 1) / tok_per_tile + kXcdGroup - 1) / kXcdGroup;
}

// Workspace bytes of one launch over up to `seqs` sequences.
static int64_t prefill_workspace_need(int64_t seqs, int64_t pair_slots) {
  return 4 * static_cast<int64_t>(kWsUnitsInt) + 4 * kUnitInts * seqs * pair_slots;
}

}  // namespace kvp

using namespace kvp;

extern "C" int kvp_varlen_prefill_bf16(const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                                       const void* k, int64_t k_block_stride, int64_t k_tok_stride,
                                       int64_t k_head_stride,
                                       const void* v, int64_t v_block_stride, int64_t v_tok_stride,
                                       int64_t v_head_stride,
                                       const int32_t* block_tables, int64_t block_table_stride,
                                       int32_t num_cache_blocks, int32_t block_size,
                                       int32_t max_blocks_per_seq,
                                       const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                       int32_t num_seqs, int32_t max_seqlen_q,
                                       int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                       float softmax_scale, int32_t causal,
                                       void* out, int64_t out_tok_stride, int64_t out_head_stride,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (num_seqs < 0 || max_seqlen_q < 0)
    return fail(KVP_EINVAL, "kvp_varlen_prefill_bf16: num_seqs=%d max_seqlen_q=%d", num_seqs, max_seqlen_q);
  if (num_seqs == 0 || max_seqlen_q == 0) return KVP_OK;
  if (head_dim != kPrefillHeadDim)
    return fail(KVP_EUNSUPPORTED, "kvp_varlen_prefill_bf16: head_dim=%d (supported: 128)", head_dim);
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return fail(KVP_EINVAL, "kvp_varlen_prefill_bf16: num_q_heads=%d not a multiple of num_kv_heads=%d",
                num_q_heads, num_kv_heads);
  const int G = num_q_heads / num_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 5 && G != 8)
    return fail(KVP_EUNSUPPORTED, "kvp_varlen_prefill_bf16: GQA ratio %d (supported: 1, 2, 4, 5, 8)", G);
  const bool paged = block_tables != nullptr;
  if (paged) {
    if (block_size <= 0 || block_size % kKeyTile != 0)
      return fail(KVP_EINVAL, "kvp_varlen_prefill_bf16: block_size=%d must be a positive multiple of 64",
                  block_size);
    if (max_blocks_per_seq <= 0 || num_cache_blocks <= 0 || block_table_stride < max_blocks_per_seq)
      return fail(KVP_EINVAL,
                  "kvp_varlen_prefill_bf16: max_blocks_per_seq=%d num_cache_blocks=%d block_table_stride=%lld",
                  max_blocks_per_seq, num_cache_blocks, static_cast<long long>(block_table_stride));
    if (reinterpret_cast<uintptr_t>(block_tables) & 3u)
      return fail(KVP_EINVAL, "kvp_varlen_prefill_bf16: block_tables must be 4-byte aligned");
    if (!mult8(k_block_stride) || !mult8(v_block_stride))
      return fail(KVP_EINVAL, "kvp_varlen_prefill_bf16: block strides must be multiples of 8 elements");
  }
  if (!q || !k || !v || !cu_seqlens_q || !cu_seqlens_k || !out)
    return fail(KVP_EINVAL, "kvp_varlen_prefill_bf16: null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(KVP_EINVAL, "kvp_varlen_prefill_bf16: q/k/v/out must be 16-byte aligned");
  if (!mult8(q_tok_stride) || !mult8(q_head_stride) || !mult8(k_tok_stride) || !mult8(k_head_stride) ||
      !mult8(v_tok_stride) || !mult8(v_head_stride) || !mult8(out_tok_stride) || !mult8(out_head_stride))
    return fail(KVP_EINVAL, "kvp_varlen_prefill_bf16: q/k/v/out strides must be multiples of 8 elements");
  // a K/V tile's 64 rows are addressed with 32-bit byte offsets
  if (k_tok_stride <= 0 || v_tok_stride <= 0 || k_tok_stride > INT32_MAX / (2 * kKeyTile) ||
      v_tok_stride > INT32_MAX / (2 * kKeyTile))
    return fail(KVP_EINVAL, "kvp_varlen_prefill_bf16: k/v token strides %lld / %lld out of range",
                static_cast<long long>(k_tok_stride), static_cast<long long>(v_tok_stride));

  const int64_t pair_slots = prefill_pair_slots(max_seqlen_q, G);
  if (pair_slots * num_kv_heads * kMaxPrefillSeqs * kXcdGroup > (1ll << 30))
    return fail(KVP_EINVAL, "kvp_varlen_prefill_bf16: too many units of work (max_seqlen_q=%d)", max_seqlen_q);
  const int64_t need = prefill_workspace_need(std::min(num_seqs, kMaxPrefillSeqs), pair_slots);
  if (!workspace || workspace_bytes < static_cast<size_t>(need))
    return fail(KVP_EWORKSPACE, "kvp_varlen_prefill_bf16: workspace of %zu bytes, %lld needed", workspace_bytes,
                static_cast<long long>(need));
  if (reinterpret_cast<uintptr_t>(workspace) & 255u)
    return fail(KVP_EINVAL, "kvp_varlen_prefill_bf16: workspace must be 256-byte aligned");

  PrefillParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.q_tok_stride = q_tok_stride;
  p.q_head_stride = q_head_stride;
  p.k = static_cast<const uint16_t*>(k);
  p.k_blk_stride = k_block_stride;
  p.k_tok_stride = k_tok_stride;
  p.k_head_stride = k_head_stride;
  p.v = static_cast<const uint16_t*>(v);
  p.v_blk_stride = v_block_stride;
  p.v_tok_stride = v_tok_stride;
  p.v_head_stride = v_head_stride;
  p.bt_stride = block_table_stride;
  p.num_cache_blocks = num_cache_blocks;
  p.block_size = paged ? block_size : kKeyTile;
  p.max_blocks = max_blocks_per_seq;
  p.pair_slots = static_cast<int32_t>(pair_slots);
  p.num_kv_heads = num_kv_heads;
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
  p.out = static_cast<uint16_t*>(out);
  p.o_tok_stride = out_tok_stride;
  p.o_head_stride = out_head_stride;
  p.ws = static_cast<int*>(workspace);

  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool c = causal != 0;
  // cu_seqlens hold absolute offsets, so a launch over sequences [s0, s0 + n) reads
  // the same q/k/out rows through the offset pointers.  Consecutive launches share the
  // workspace: each one's plan kernel runs after the previous attention kernel.
  for (int s0 = 0; s0 < num_seqs; s0 += kMaxPrefillSeqs) {
    const int n = std::min(kMaxPrefillSeqs, num_seqs - s0);
    p.cu_q = cu_seqlens_q + s0;
    p.cu_k = cu_seqlens_k + s0;
    p.block_tables = paged ? block_tables + s0 * block_table_stride : nullptr;
    p.num_seqs = n;
    switch (G) {
      case 1: launch_prefill<1>(paged, c, s, p); break;
      case 2: launch_prefill<2>(paged, c, s, p); break;
      case 4: launch_prefill<4>(paged, c, s, p); break;
      case 5: launch_prefill<5>(paged, c, s, p); break;
      default: launch_prefill<8>(paged, c, s, p); break;
    }
    const int rc = launch_status("kvp_varlen_prefill_bf16");
    if (rc != KVP_OK) return rc;
  }
  return KVP_OK;
}

extern "C" size_t kvp_prefill_workspace_bytes(int32_t num_seqs, int32_t max_seqlen_q, int32_t num_q_heads,
                                              int32_t num_kv_heads) {
  if (num_seqs < 0 || max_seqlen_q < 0 || num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return 0;
  const int g = num_q_heads / num_kv_heads;
  if (g != 1 && g != 2 && g != 4 && g != 5 && g != 8) return 0;
  return static_cast<size_t>(
      prefill_workspace_need(std::min(num_seqs, kMaxPrefillSeqs), prefill_pair_slots(max_seqlen_q, g)));
}
