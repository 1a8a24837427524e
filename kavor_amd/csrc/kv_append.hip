// KV append: scatter each token's K and V rows into its paged-cache slot.
//
// Restates store_kvcache_kernel / store_kvcache
// (kavor/layers/attention/flash_attention_kvcache.py:10-46): a pure bit copy of
// num_kv_heads*head_dim bf16 values per tensor per token, slot -1 skipped.
//
// Mapping: each wave64 moves two tokens.  A token's K row and V row are cut into
// 16-byte chunks (8 bf16); the wave's lanes own consecutive chunks, so every load and
// store is a dwordx4 and a 16-lane group covers one 256-byte head row contiguously.
// Each lane issues the loads of both its tokens before it reads a slot or stores
// anything, so a wave keeps 8 KiB in flight (Qwen3: 8 kv heads x 128 is 128 chunks per
// tensor row, 2 K + 2 V chunks per lane per token).  Source rows are read once and
// cache rows written once, so both go nontemporal.  Measured on the 4096-token append
// (graph-replayed, rotating inputs): one token per wave 8.5 us; two 7.0 us; two with
// nontemporal loads 6.6-6.7 us (60-61% of 8 TB/s); four or eight per wave 7.4 / 8.2 us
// (too few waves); workgroups of 1-8 waves alike.
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

constexpr int kAppendWaves = 4;
constexpr int kAppendTokensPerWave = 2;
constexpr int kAppendTokensPerGroup = kAppendWaves * kAppendTokensPerWave;

// CPL = 16-byte chunks per lane per tensor: a token's K row and its V row are each
// Hkv * HEAD_DIM / 8 chunks; lane l owns chunks l, l + 64, ... of both (rows longer
// than 64 * CPL chunks take several passes).  Chunk indices are clamped onto the row's
// last chunk and token indices onto the last token, so no branch guards a load; a lane
// past the row's end rewrites that chunk's bytes to the same place.
template <int HEAD_DIM, int CPL>
__global__ __launch_bounds__(64 * kAppendWaves) void kv_append_kernel(const AppendParams p) {
  constexpr int kChunksPerHead = HEAD_DIM / 8;
  constexpr int TPW = kAppendTokensPerWave;
  // Token indices, slots and row addresses are wave-uniform.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tok0 = (static_cast<int>(blockIdx.x) * kAppendWaves + wave) * TPW;
  const int lane = threadIdx.x & 63;
  const int cpt = p.num_kv_heads * kChunksPerHead;  // chunks per tensor row

  int j0 = 0;
  do {  // every row has at least one chunk group
    int64_t kofs[CPL], vofs[CPL], dofs[CPL];
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
      const int j = min(j0 + 64 * u + lane, cpt - 1);
      const int head = j / kChunksPerHead;
      const int part = j - head * kChunksPerHead;
      kofs[u] = head * p.key_head_stride + part;
      vofs[u] = head * p.value_head_stride + part;
      dofs[u] = head * p.head_stride + part;
    }
    uint4 kb[TPW][CPL], vb[TPW][CPL];
    int32_t slots[TPW];
#pragma unroll
    for (int q = 0; q < TPW; ++q) {
      const int tok = min(tok0 + q, p.num_tokens - 1);
      const uint4* key_row = p.key + static_cast<int64_t>(tok) * p.key_tok_stride;
      const uint4* value_row = p.value + static_cast<int64_t>(tok) * p.value_tok_stride;
#pragma unroll
      for (int u = 0; u < CPL; ++u) kb[q][u] = load16_nt(key_row + kofs[u]);
#pragma unroll
      for (int u = 0; u < CPL; ++u) vb[q][u] = load16_nt(value_row + vofs[u]);
      // Each token's slot is read after its rows are issued: without this fence the
      // compiler hoists the slot loads, their wait and the division ahead of the row
      // loads, and every wave pays a memory round trip before its first row load.  In
      // this order the first token's stores can start while the second token's loads
      // are still in flight.  (Reading the slots first, as scalar loads, measured 7.7 us.)
      asm volatile("" ::: "memory");
      slots[q] = p.slot_mapping[tok];
    }
#pragma unroll
    for (int q = 0; q < TPW; ++q) {
      const int tok = tok0 + q;
      const int32_t slot = slots[q];
      // -1 (padding), a slot outside the pool and tokens past the last are skipped; cache
      // rows are written once and read by a later kernel, so the stores are nontemporal
      if (tok >= p.num_tokens || slot < 0 || static_cast<int64_t>(slot) >= p.num_cache_slots) continue;
      const int32_t blk = slot / p.block_size;
      const int32_t off = slot - blk * p.block_size;
      const int64_t dst_base = static_cast<int64_t>(blk) * p.blk_stride + static_cast<int64_t>(off) * p.slot_stride;
#pragma unroll
      for (int u = 0; u < CPL; ++u) store16_nt(p.k_cache + dst_base + dofs[u], kb[q][u]);
#pragma unroll
      for (int u = 0; u < CPL; ++u) store16_nt(p.v_cache + dst_base + dofs[u], vb[q][u]);
    }
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

  const dim3 grid((num_tokens + kAppendTokensPerGroup - 1) / kAppendTokensPerGroup);
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
