// Paged decode attention: one query token per sequence against its paged KV cache.
//
// Restates flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache, cache_seqlens,
// block_table, softmax_scale, causal=True) as used at
// kavor/layers/attention/flash_attention_kvcache.py:80-83.
//
// Work decomposition (HBM-bound: every KV byte is read exactly once)
//   grid = (num_splits, num_kv_heads, num_seqs); a workgroup owns one (sequence,
//   kv head, split) and all G = num_q_heads / num_kv_heads query heads of that kv
//   head, so GQA costs no extra KV traffic.  A split is `blocks_per_split` logical
//   blocks; workgroups past a sequence's last block exit at once.
//   Inside a workgroup the 4 waves walk the split in chunks of 128 tokens, wave w
//   taking tokens [32w, 32w+32) of the chunk.  Lane (r = lane/16, c = lane%16) owns
//   dims [8c, 8c+8) of tokens 4i+r, i = 0..7: 8 dwordx4 loads of K and 8 of V per
//   lane (8 KiB per wave in flight), each 16-lane row reading one 256-byte head row.
//   Scores: q.k with v_dot2c_f32_bf16 on packed bf16 pairs, then a 4-step DPP sum
//   across the 16-lane row.  Softmax: online, base 2, scale*log2(e) folded into the
//   scores, one running (max, sum, acc[8]) per lane row.  The 16 row states of a
//   workgroup (4 rows x 4 waves) are merged through LDS.
//   Output: a sequence that fits one split writes bf16 directly; otherwise each split
//   writes (max, sum, unnormalised acc) in fp32 to the workspace and
//   decode_merge_kernel combines the splits with the same online-softmax rule.
#include <math.h>
#include <stdlib.h>

#include "common.h"

namespace kvp {

constexpr int kDecodeHeadDim = 128;
constexpr int kDecodeWaves = 4;
constexpr int kWaveTokens = 32;
constexpr int kLoadsPerLane = kWaveTokens / 4;
constexpr int kChunkTokens = kDecodeWaves * kWaveTokens;
constexpr int kRowStates = kDecodeWaves * 4;

struct DecodeParams {
  const uint16_t* q;
  int64_t q_seq_stride, q_head_stride;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  int64_t blk_stride, slot_stride, head_stride;
  int32_t num_cache_blocks;
  const int32_t* block_tables;
  int64_t bt_stride;
  const int32_t* context_lens;
  int32_t num_q_heads;
  int32_t block_size;
  int32_t max_blocks;
  int32_t blocks_per_split;
  int32_t num_splits;
  float scale_log2;  // softmax_scale * log2(e)
  uint16_t* out;
  int64_t o_seq_stride, o_head_stride;
  float* part_o;   // [num_seqs][num_q_heads][num_splits][128]
  float* part_ml;  // [num_seqs][num_q_heads][num_splits][2] = (max, sum)
};

__device__ __forceinline__ uint4 load16(const uint16_t* ptr) {
  return *reinterpret_cast<const uint4*>(ptr);
}

template <int G>
__global__ __launch_bounds__(64 * kDecodeWaves) void paged_decode_kernel(const DecodeParams p) {
  constexpr int D = kDecodeHeadDim;
  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r = lane >> 4;
  const int c = lane & 15;

  const int bs = p.block_size;
  const int ctx = p.context_lens[b];
  const int capacity = p.max_blocks * bs;
  if (ctx <= 0 || ctx > capacity) {
    // Empty (graph padding) rows read as zeros; impossible lengths read as NaN.
    if (split == 0) {
      const uint16_t fill = ctx <= 0 ? 0 : 0x7fc0;
      for (int o = tid; o < G * D; o += 64 * kDecodeWaves) {
        const int g = o / D, d = o - g * D;
        p.out[b * p.o_seq_stride + (kvh * G + g) * p.o_head_stride + d] = fill;
      }
    }
    return;
  }
  const int nblk = (ctx + bs - 1) / bs;
  const int bps = p.blocks_per_split;
  const int blk_begin = split * bps;
  if (blk_begin >= nblk) return;
  const int blk_end = min(nblk, blk_begin + bps);
  const int nsplit_seq = (nblk + bps - 1) / bps;
  const int tok_begin = blk_begin * bs;
  const int tok_end = min(ctx, blk_end * bs);

  __shared__ int s_bad;
  __shared__ float s_m[G][kRowStates];
  __shared__ float s_l[G][kRowStates];
  __shared__ float s_acc[G][kRowStates][D];
  if (tid == 0) s_bad = 0;

  // This lane's query slice: dims [8c, 8c+8) of every query head of the group.
  uint4 qv[G];
#pragma unroll
  for (int g = 0; g < G; ++g)
    qv[g] = load16(p.q + b * p.q_seq_stride + (kvh * G + g) * p.q_head_stride + 8 * c);

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kMaxFloor;
    l[g] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = 0.f;
  }

  const int32_t* bt_row = p.block_tables + b * p.bt_stride;
  const int64_t head_off = static_cast<int64_t>(kvh) * p.head_stride + 8 * c;
  bool bad = false;

  for (int t0 = tok_begin; t0 < tok_end; t0 += kChunkTokens) {
    const int tw = t0 + kWaveTokens * wave;  // first token of this wave's slice
    if (tw >= tok_end) continue;             // wave-uniform
    const int lblk = tw / bs;
    int blk = bt_row[lblk];
    if (blk < 0 || blk >= p.num_cache_blocks) {
      bad = true;
      blk = 0;
    }
    const int64_t base = static_cast<int64_t>(blk) * p.blk_stride +
                         static_cast<int64_t>(tw - lblk * bs) * p.slot_stride + head_off;
    const int nvalid = tok_end - tw;  // tokens of this wave's slice that exist (may exceed it)

    uint4 kr[kLoadsPerLane], vr[kLoadsPerLane];
#pragma unroll
    for (int i = 0; i < kLoadsPerLane; ++i) {
      const int t = 4 * i + r;
      kr[i] = make_uint4(0, 0, 0, 0);
      if (t < nvalid) kr[i] = load16(p.k_cache + base + t * p.slot_stride);
    }
#pragma unroll
    for (int i = 0; i < kLoadsPerLane; ++i) {
      const int t = 4 * i + r;
      vr[i] = make_uint4(0, 0, 0, 0);
      if (t < nvalid) vr[i] = load16(p.v_cache + base + t * p.slot_stride);
    }

#pragma unroll
    for (int g = 0; g < G; ++g) {
      float s[kLoadsPerLane];
      float mx = kMaxFloor;
#pragma unroll
      for (int i = 0; i < kLoadsPerLane; ++i) {
        float part = dot2_bf16(qv[g].x, kr[i].x, 0.f);
        part = dot2_bf16(qv[g].y, kr[i].y, part);
        part = dot2_bf16(qv[g].z, kr[i].z, part);
        part = dot2_bf16(qv[g].w, kr[i].w, part);
        const float sc = row16_sum(part) * p.scale_log2;
        s[i] = (4 * i + r < nvalid) ? sc : -INFINITY;
        mx = fmaxf(mx, s[i]);
      }
      const float m_new = fmaxf(m[g], mx);
      const float alpha = fast_exp2(m[g] - m_new);
      m[g] = m_new;
      float lsum = l[g] * alpha;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[g][j] *= alpha;
#pragma unroll
      for (int i = 0; i < kLoadsPerLane; ++i) {
        const float pr = fast_exp2(s[i] - m_new);
        lsum += pr;
        acc[g][0] += pr * bf16_lo(vr[i].x);
        acc[g][1] += pr * bf16_hi(vr[i].x);
        acc[g][2] += pr * bf16_lo(vr[i].y);
        acc[g][3] += pr * bf16_hi(vr[i].y);
        acc[g][4] += pr * bf16_lo(vr[i].z);
        acc[g][5] += pr * bf16_hi(vr[i].z);
        acc[g][6] += pr * bf16_lo(vr[i].w);
        acc[g][7] += pr * bf16_hi(vr[i].w);
      }
      l[g] = lsum;
    }
  }

  __syncthreads();  // s_bad initialised before any wave may set it
  if (bad) s_bad = 1;
  const int rs = wave * 4 + r;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (c == 0) {
      s_m[g][rs] = m[g];
      s_l[g][rs] = l[g];
    }
    float4* dst = reinterpret_cast<float4*>(&s_acc[g][rs][8 * c]);
    dst[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
    dst[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
  }
  __syncthreads();

  const bool poisoned = s_bad != 0;
  for (int o = tid; o < G * D; o += 64 * kDecodeWaves) {
    const int g = o / D, d = o - g * D;
    float mm = kMaxFloor;
#pragma unroll
    for (int k = 0; k < kRowStates; ++k) mm = fmaxf(mm, s_m[g][k]);
    float ll = 0.f, oo = 0.f;
#pragma unroll
    for (int k = 0; k < kRowStates; ++k) {
      const float w = fast_exp2(s_m[g][k] - mm);
      ll += w * s_l[g][k];
      oo += w * s_acc[g][k][d];
    }
    if (poisoned) ll = NAN;
    const int h = kvh * G + g;
    if (nsplit_seq == 1) {
      p.out[b * p.o_seq_stride + h * p.o_head_stride + d] = f32_to_bf16(oo / ll);
    } else {
      const int64_t row = (static_cast<int64_t>(b) * p.num_q_heads + h) * p.num_splits + split;
      p.part_o[row * D + d] = oo;
      if (d == 0) {
        p.part_ml[row * 2] = mm;
        p.part_ml[row * 2 + 1] = ll;
      }
    }
  }
}

// Combines the per-split partial states of sequences that span several splits.
// grid = (num_q_heads, num_seqs), 128 threads (one per head dim).
__global__ __launch_bounds__(kDecodeHeadDim) void decode_merge_kernel(const DecodeParams p) {
  constexpr int D = kDecodeHeadDim;
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;
  const int bs = p.block_size;
  const int ctx = p.context_lens[b];
  if (ctx <= 0 || ctx > p.max_blocks * bs) return;
  const int nblk = (ctx + bs - 1) / bs;
  const int ns = (nblk + p.blocks_per_split - 1) / p.blocks_per_split;
  if (ns <= 1) return;
  const int64_t row0 = (static_cast<int64_t>(b) * p.num_q_heads + h) * p.num_splits;
  const float* ml = p.part_ml + row0 * 2;
  float mm = kMaxFloor;
  for (int s = 0; s < ns; ++s) mm = fmaxf(mm, ml[2 * s]);
  float ll = 0.f, oo = 0.f;
  for (int s = 0; s < ns; ++s) {
    const float w = fast_exp2(ml[2 * s] - mm);
    ll += w * ml[2 * s + 1];
    oo += w * p.part_o[(row0 + s) * D + d];
  }
  p.out[b * p.o_seq_stride + h * p.o_head_stride + d] = f32_to_bf16(oo / ll);
}

// Blocks per split: one 256-token block per workgroup keeps ragged batches balanced;
// very wide block tables group blocks so that no sequence needs more than 32 splits,
// which bounds the fp32 partial traffic to well under 2% of the KV bytes.
static int choose_blocks_per_split(int max_blocks) {
  static int forced = [] {
    const char* env = getenv("KVP_DECODE_BLOCKS_PER_SPLIT");
    return env ? atoi(env) : 0;
  }();
  if (forced > 0) return forced;
  return max_blocks <= 32 ? 1 : (max_blocks + 31) / 32;
}

}  // namespace kvp

using namespace kvp;

extern "C" size_t kvp_decode_workspace_bytes(int32_t max_num_seqs, int32_t num_q_heads,
                                             int32_t head_dim, int32_t max_blocks_per_seq) {
  if (max_num_seqs <= 0 || num_q_heads <= 0 || head_dim <= 0 || max_blocks_per_seq <= 0) return 0;
  // Sized for one block per split, the finest split choose_blocks_per_split can make.
  return static_cast<size_t>(max_num_seqs) * num_q_heads * max_blocks_per_seq *
         (static_cast<size_t>(head_dim) + 2) * sizeof(float);
}

extern "C" int kvp_paged_decode_bf16(const void* q, int64_t q_seq_stride, int64_t q_head_stride,
                                     const void* k_cache, const void* v_cache,
                                     int64_t cache_block_stride, int64_t cache_slot_stride,
                                     int64_t cache_head_stride, int32_t num_cache_blocks,
                                     const int32_t* block_tables, int64_t block_table_stride,
                                     const int32_t* context_lens, int32_t num_seqs,
                                     int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                     int32_t block_size, int32_t max_blocks_per_seq,
                                     float softmax_scale,
                                     void* out, int64_t out_seq_stride, int64_t out_head_stride,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (num_seqs < 0) return fail(KVP_EINVAL, "kvp_paged_decode_bf16: num_seqs=%d < 0", num_seqs);
  if (num_seqs == 0) return KVP_OK;
  if (num_seqs > 65535) return fail(KVP_EINVAL, "kvp_paged_decode_bf16: num_seqs=%d > 65535", num_seqs);
  if (head_dim != kDecodeHeadDim)
    return fail(KVP_EUNSUPPORTED, "kvp_paged_decode_bf16: head_dim=%d (supported: 128)", head_dim);
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0)
    return fail(KVP_EINVAL, "kvp_paged_decode_bf16: num_q_heads=%d not a multiple of num_kv_heads=%d",
                num_q_heads, num_kv_heads);
  if (num_kv_heads > 65535)
    return fail(KVP_EINVAL, "kvp_paged_decode_bf16: num_kv_heads=%d > 65535", num_kv_heads);
  const int G = num_q_heads / num_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return fail(KVP_EUNSUPPORTED, "kvp_paged_decode_bf16: GQA ratio %d (supported: 1, 2, 4, 8)", G);
  if (block_size <= 0 || block_size % 64 != 0)
    return fail(KVP_EINVAL, "kvp_paged_decode_bf16: block_size=%d must be a positive multiple of 64",
                block_size);
  if (max_blocks_per_seq <= 0 || num_cache_blocks <= 0)
    return fail(KVP_EINVAL, "kvp_paged_decode_bf16: max_blocks_per_seq=%d num_cache_blocks=%d",
                max_blocks_per_seq, num_cache_blocks);
  if (static_cast<int64_t>(max_blocks_per_seq) * block_size > (1ll << 30))
    return fail(KVP_EINVAL, "kvp_paged_decode_bf16: max_blocks_per_seq*block_size too large");
  if (block_table_stride < max_blocks_per_seq)
    return fail(KVP_EINVAL, "kvp_paged_decode_bf16: block_table_stride=%lld < max_blocks_per_seq=%d",
                static_cast<long long>(block_table_stride), max_blocks_per_seq);
  if (!q || !k_cache || !v_cache || !block_tables || !context_lens || !out)
    return fail(KVP_EINVAL, "kvp_paged_decode_bf16: null pointer");
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(KVP_EINVAL, "kvp_paged_decode_bf16: q and cache pointers must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(out) & 1u) || (reinterpret_cast<uintptr_t>(block_tables) & 3u) ||
      (reinterpret_cast<uintptr_t>(context_lens) & 3u))
    return fail(KVP_EINVAL, "kvp_paged_decode_bf16: misaligned out/block_tables/context_lens");
  if (!mult8(q_seq_stride) || !mult8(q_head_stride) || !mult8(cache_block_stride) ||
      !mult8(cache_slot_stride) || !mult8(cache_head_stride))
    return fail(KVP_EINVAL, "kvp_paged_decode_bf16: q and cache strides must be multiples of 8 elements");

  const int bps = choose_blocks_per_split(max_blocks_per_seq);
  const int num_splits = (max_blocks_per_seq + bps - 1) / bps;
  const size_t need = static_cast<size_t>(num_seqs) * num_q_heads * num_splits *
                      (kDecodeHeadDim + 2) * sizeof(float);
  if (num_splits > 1) {
    if (!workspace || workspace_bytes < need)
      return fail(KVP_EWORKSPACE, "kvp_paged_decode_bf16: workspace of %zu bytes, %zu needed",
                  workspace_bytes, need);
    if (reinterpret_cast<uintptr_t>(workspace) & 15u)
      return fail(KVP_EINVAL, "kvp_paged_decode_bf16: workspace must be 16-byte aligned");
  }

  DecodeParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.q_seq_stride = q_seq_stride;
  p.q_head_stride = q_head_stride;
  p.k_cache = static_cast<const uint16_t*>(k_cache);
  p.v_cache = static_cast<const uint16_t*>(v_cache);
  p.blk_stride = cache_block_stride;
  p.slot_stride = cache_slot_stride;
  p.head_stride = cache_head_stride;
  p.num_cache_blocks = num_cache_blocks;
  p.block_tables = block_tables;
  p.bt_stride = block_table_stride;
  p.context_lens = context_lens;
  p.num_q_heads = num_q_heads;
  p.block_size = block_size;
  p.max_blocks = max_blocks_per_seq;
  p.blocks_per_split = bps;
  p.num_splits = num_splits;
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
  p.out = static_cast<uint16_t*>(out);
  p.o_seq_stride = out_seq_stride;
  p.o_head_stride = out_head_stride;
  float* ws = static_cast<float*>(workspace);
  p.part_o = ws;
  p.part_ml = ws ? ws + static_cast<size_t>(num_seqs) * num_q_heads * num_splits * kDecodeHeadDim
                 : nullptr;

  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(num_splits, num_kv_heads, num_seqs);
  const dim3 block(64 * kDecodeWaves);
  switch (G) {
    case 1: hipLaunchKernelGGL(paged_decode_kernel<1>, grid, block, 0, s, p); break;
    case 2: hipLaunchKernelGGL(paged_decode_kernel<2>, grid, block, 0, s, p); break;
    case 4: hipLaunchKernelGGL(paged_decode_kernel<4>, grid, block, 0, s, p); break;
    default: hipLaunchKernelGGL(paged_decode_kernel<8>, grid, block, 0, s, p); break;
  }
  int rc = launch_status("kvp_paged_decode_bf16");
  if (rc != KVP_OK || num_splits == 1) return rc;
  hipLaunchKernelGGL(decode_merge_kernel, dim3(num_q_heads, num_seqs), dim3(kDecodeHeadDim), 0, s, p);
  return launch_status("kvp_paged_decode_bf16 (merge)");
}
