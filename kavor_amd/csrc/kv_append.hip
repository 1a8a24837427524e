// KV append: scatter each token's K and V rows into its paged-cache slot.
//
// Restates store_kvcache_kernel / store_kvcache
// (kavor/layers/attention/flash_attention_kvcache.py:10-46): a pure bit copy of
// num_kv_heads*head_dim bf16 values per tensor per token, slot -1 skipped.
//
// Mapping: one wave64 per token.  A token's K row and V row are cut into 16-byte
// chunks (8 bf16); the wave's lanes own consecutive chunks, so every load and store
// is a dwordx4 and a 16-lane group covers one 256-byte head row contiguously.  Each
// lane issues all of its loads before its first store so a wave keeps up to 4 KiB in
// flight; the token index, slot and row addresses are wave-uniform scalars.  For Qwen3
// (8 kv heads x 128) a token row is 128 chunks per tensor: 2 K + 2 V chunks per lane.
#include "common.h"

namespace kvp {

struct AppendParams {
  const uint4* key;
  const uint4* value;
  int64_t key_tok_stride, key_head_stride;      // in 16-byte chunks
  int64_t value_tok_stride, value_head_stride;  // in 16-byte chunks
  uint4* k_cache;
  uint4* v_cache;
  int64_t blk_stride, slot_stride, head_stride;  // in 16-byte chunks
  int64_t num_cache_slots;
  const int32_t* slot_mapping;
  int32_t num_tokens;
  int32_t num_kv_heads;
  int32_t block_size;
};

constexpr int kAppendWaves = 4;  // tokens per workgroup

// CPL = 16-byte chunks per lane per tensor: a token's K row and its V row are each
// Hkv * HEAD_DIM / 8 chunks; lane l owns chunks l, l + 64, ... of both.  Every lane issues
// all 2 * CPL loads before its first store; chunk indices are clamped onto the row's last
// chunk, so neither loads nor stores need a branch.
template <int HEAD_DIM, int CPL>
__global__ __launch_bounds__(64 * kAppendWaves) void kv_append_kernel(const AppendParams p) {
  constexpr int kChunksPerHead = HEAD_DIM / 8;
  // Token index and slot are wave-uniform: keep them (and the address math) scalar.  No
  // early return precedes the loads (the token index is clamped instead), so the only
  // scalar round trip before them is the kernel-argument fetch.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tok_raw = blockIdx.x * kAppendWaves + wave;
  const int tok = min(tok_raw, p.num_tokens - 1);
  const int lane = threadIdx.x & 63;
  const int cpt = p.num_kv_heads * kChunksPerHead;  // chunks per tensor row
  const uint4* key_row = p.key + static_cast<int64_t>(tok) * p.key_tok_stride;
  const uint4* value_row = p.value + static_cast<int64_t>(tok) * p.value_tok_stride;
  const int32_t slot = p.slot_mapping[tok];
  const bool store = tok_raw < p.num_tokens && slot >= 0 && static_cast<int64_t>(slot) < p.num_cache_slots;
  const int32_t blk = slot / p.block_size;  // scalar division: no branch before the loads
  const int32_t off = slot - blk * p.block_size;
  const int64_t dst_base = static_cast<int64_t>(blk) * p.blk_stride + static_cast<int64_t>(off) * p.slot_stride;

  int j0 = 0;
  do {  // every row has at least one chunk group
    uint4 kb[CPL], vb[CPL];
    int64_t dofs[CPL];
    int64_t kofs[CPL], vofs[CPL];
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
      const int j = min(j0 + 64 * u + lane, cpt - 1);
      const int head = j / kChunksPerHead;
      const int part = j - head * kChunksPerHead;
      kofs[u] = head * p.key_head_stride + part;
      vofs[u] = head * p.value_head_stride + part;
      dofs[u] = head * p.head_stride + part;
    }
    // K row then V row (each a contiguous stretch of HBM), loads and stores alike.
#pragma unroll
    for (int u = 0; u < CPL; ++u) kb[u] = key_row[kofs[u]];
#pragma unroll
    for (int u = 0; u < CPL; ++u) vb[u] = value_row[vofs[u]];
    if (!store) return;  // -1 (padding), a slot outside the pool, or past the last token
    // Cache rows are written once and read by a later kernel: nontemporal stores keep
    // them out of L2 (measured 10.0 -> 8.3 us for 4096 tokens).  A lane past the row's
    // last chunk was clamped onto that chunk and rewrites the same bytes to the same
    // place, so the stores need no mask either.
#pragma unroll
    for (int u = 0; u < CPL; ++u) store16_nt(p.k_cache + dst_base + dofs[u], kb[u]);
#pragma unroll
    for (int u = 0; u < CPL; ++u) store16_nt(p.v_cache + dst_base + dofs[u], vb[u]);
    j0 += 64 * CPL;
  } while (j0 < cpt);
}

template <int HEAD_DIM>
static void launch_append(const AppendParams& p, int chunks_per_tensor, dim3 grid, dim3 block, hipStream_t s) {
  if (chunks_per_tensor <= 64) hipLaunchKernelGGL((kv_append_kernel<HEAD_DIM, 1>), grid, block, 0, s, p);
  else if (chunks_per_tensor <= 128) hipLaunchKernelGGL((kv_append_kernel<HEAD_DIM, 2>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((kv_append_kernel<HEAD_DIM, 4>), grid, block, 0, s, p);
}

}  // namespace kvp

using namespace kvp;

extern "C" int kvp_append_bf16(const void* key, int64_t key_tok_stride, int64_t key_head_stride,
                               const void* value, int64_t value_tok_stride, int64_t value_head_stride,
                               void* k_cache, void* v_cache,
                               int64_t cache_block_stride, int64_t cache_slot_stride,
                               int64_t cache_head_stride, int64_t num_cache_slots,
                               const int32_t* slot_mapping, int32_t num_tokens,
                               int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                               void* stream) {
  clear_error();
  if (num_tokens < 0) return fail(KVP_EINVAL, "kvp_append_bf16: num_tokens=%d < 0", num_tokens);
  if (num_tokens == 0) return KVP_OK;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(KVP_EUNSUPPORTED, "kvp_append_bf16: head_dim=%d (supported: 64, 128, 256)", head_dim);
  if (num_kv_heads <= 0 || block_size <= 0 || num_cache_slots < 0)
    return fail(KVP_EINVAL, "kvp_append_bf16: num_kv_heads=%d block_size=%d num_cache_slots=%lld",
                num_kv_heads, block_size, static_cast<long long>(num_cache_slots));
  if (!key || !value || !k_cache || !v_cache || !slot_mapping)
    return fail(KVP_EINVAL, "kvp_append_bf16: null pointer");
  if (!aligned16(key) || !aligned16(value) || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(KVP_EINVAL, "kvp_append_bf16: key/value/cache pointers must be 16-byte aligned");
  if (!mult8(key_tok_stride) || !mult8(key_head_stride) || !mult8(value_tok_stride) ||
      !mult8(value_head_stride) || !mult8(cache_block_stride) || !mult8(cache_slot_stride) ||
      !mult8(cache_head_stride))
    return fail(KVP_EINVAL, "kvp_append_bf16: every stride must be a multiple of 8 elements");
  if (reinterpret_cast<uintptr_t>(slot_mapping) & 3u)
    return fail(KVP_EINVAL, "kvp_append_bf16: slot_mapping must be 4-byte aligned");

  AppendParams p;
  p.key = static_cast<const uint4*>(key);
  p.value = static_cast<const uint4*>(value);
  p.key_tok_stride = key_tok_stride / 8;
  p.key_head_stride = key_head_stride / 8;
  p.value_tok_stride = value_tok_stride / 8;
  p.value_head_stride = value_head_stride / 8;
  p.k_cache = static_cast<uint4*>(k_cache);
  p.v_cache = static_cast<uint4*>(v_cache);
  p.blk_stride = cache_block_stride / 8;
  p.slot_stride = cache_slot_stride / 8;
  p.head_stride = cache_head_stride / 8;
  p.num_cache_slots = num_cache_slots;
  p.slot_mapping = slot_mapping;
  p.num_tokens = num_tokens;
  p.num_kv_heads = num_kv_heads;
  p.block_size = block_size;

  const dim3 grid((num_tokens + kAppendWaves - 1) / kAppendWaves);
  const dim3 block(64 * kAppendWaves);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int cpt = num_kv_heads * (head_dim / 8);
  switch (head_dim) {
    case 64: launch_append<64>(p, cpt, grid, block, s); break;
    case 128: launch_append<128>(p, cpt, grid, block, s); break;
    default: launch_append<256>(p, cpt, grid, block, s); break;
  }
  return launch_status("kvp_append_bf16");
}
