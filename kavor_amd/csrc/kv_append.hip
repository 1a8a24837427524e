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
// flight; the token index, slot and row addresses are wave-uniform scalars.  For Qwen3 (8 kv heads x 128) a token is 256 chunks: 4 per lane.
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

constexpr int kAppendWaves = 4;     // tokens per workgroup
constexpr int kAppendUnroll = 4;    // 16-byte chunks in flight per lane

// Chunk j of a token (K chunks first, then V) -> source and destination offsets in
// 16-byte units.  `j` is clamped by the caller so every computed address is valid.
template <int HEAD_DIM>
__device__ __forceinline__ void chunk_offsets(const AppendParams& p, int j, int chunks_per_tensor,
                                              bool& is_v, int64_t& src, int64_t& dst) {
  constexpr int kChunksPerHead = HEAD_DIM / 8;
  is_v = j >= chunks_per_tensor;
  const int jj = is_v ? j - chunks_per_tensor : j;
  const int head = jj / kChunksPerHead;
  const int part = jj - head * kChunksPerHead;
  src = head * (is_v ? p.value_head_stride : p.key_head_stride) + part;
  dst = head * p.head_stride + part;
}

template <int HEAD_DIM>
__global__ __launch_bounds__(64 * kAppendWaves) void kv_append_kernel(const AppendParams p) {
  // Token index and slot are wave-uniform: keep them (and the address math) scalar.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tok = blockIdx.x * kAppendWaves + wave;
  const int lane = threadIdx.x & 63;
  if (tok >= p.num_tokens) return;
  const int32_t slot = p.slot_mapping[tok];
  if (slot < 0 || static_cast<int64_t>(slot) >= p.num_cache_slots) return;  // -1: padding
  const int bs = p.block_size;
  int32_t blk, off;
  if ((bs & (bs - 1)) == 0) {
    const int shift = __builtin_ctz(bs);
    blk = slot >> shift;
    off = slot & (bs - 1);
  } else {
    blk = slot / bs;
    off = slot - blk * bs;
  }
  const int64_t dst_base = static_cast<int64_t>(blk) * p.blk_stride + static_cast<int64_t>(off) * p.slot_stride;
  const int chunks_per_tensor = p.num_kv_heads * (HEAD_DIM / 8);
  const int total = 2 * chunks_per_tensor;
  const uint4* key_row = p.key + static_cast<int64_t>(tok) * p.key_tok_stride;
  const uint4* value_row = p.value + static_cast<int64_t>(tok) * p.value_tok_stride;
  uint4* k_dst = p.k_cache + dst_base;
  uint4* v_dst = p.v_cache + dst_base;

  for (int j0 = 0; j0 < total; j0 += 64 * kAppendUnroll) {
    // All loads of this group first (addresses clamped to a valid chunk, so no branch
    // guards the loads and they stay in flight together), then the guarded stores.
    uint4 b0, b1, b2, b3;
    int64_t d0, d1, d2, d3;
    bool v0, v1, v2, v3;
    {
      int64_t s0, s1, s2, s3;
      chunk_offsets<HEAD_DIM>(p, min(j0 + lane, total - 1), chunks_per_tensor, v0, s0, d0);
      chunk_offsets<HEAD_DIM>(p, min(j0 + 64 + lane, total - 1), chunks_per_tensor, v1, s1, d1);
      chunk_offsets<HEAD_DIM>(p, min(j0 + 128 + lane, total - 1), chunks_per_tensor, v2, s2, d2);
      chunk_offsets<HEAD_DIM>(p, min(j0 + 192 + lane, total - 1), chunks_per_tensor, v3, s3, d3);
      b0 = (v0 ? value_row : key_row)[s0];
      b1 = (v1 ? value_row : key_row)[s1];
      b2 = (v2 ? value_row : key_row)[s2];
      b3 = (v3 ? value_row : key_row)[s3];
    }
    if (j0 + lane < total) (v0 ? v_dst : k_dst)[d0] = b0;
    if (j0 + 64 + lane < total) (v1 ? v_dst : k_dst)[d1] = b1;
    if (j0 + 128 + lane < total) (v2 ? v_dst : k_dst)[d2] = b2;
    if (j0 + 192 + lane < total) (v3 ? v_dst : k_dst)[d3] = b3;
  }
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
  switch (head_dim) {
    case 64: hipLaunchKernelGGL(kv_append_kernel<64>, grid, block, 0, s, p); break;
    case 128: hipLaunchKernelGGL(kv_append_kernel<128>, grid, block, 0, s, p); break;
    default: hipLaunchKernelGGL(kv_append_kernel<256>, grid, block, 0, s, p); break;
  }
  return launch_status("kvp_append_bf16");
}
