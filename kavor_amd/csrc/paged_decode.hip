// Paged decode attention: one query token per sequence against its paged KV cache.
//
// Restates flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache, cache_seqlens,
// block_table, softmax_scale, causal=True) as used at
// kavor/layers/attention/flash_attention_kvcache.py:80-83.
//
// Work decomposition (HBM-bound: every KV byte is read exactly once) -- stream-K
//   Work is counted in steps of 16 tokens of one sequence; the steps of all sequences
//   are laid end to end (prefix sums of ceil(ctx / 16), built in LDS by every
//   workgroup from context_lens).  The kernel is persistent: its grid is the number of
//   workgroups the GPU holds at once, independent of the batch and of the block-table
//   width, so a captured graph never launches empty workgroups.  A workgroup is 4
//   waves = 4 kv heads; ceil(Hkv / 4) consecutive workgroups form a group that walks
//   one contiguous range of steps for all kv heads (kv heads of one token row share HBM
//   pages and are fetched together).  Every group gets the same number of steps
//   (exact balance whatever the context lengths), and at least 128 tokens: a large batch
//   is split by the grid (the range limit does not bind), while a small one is cut into
//   short ranges so that it still spreads over many CUs (measured with 8 sequences of
//   500-2000 tokens: 34.6 us per call with 512-token ranges, 19.5 us with 128).
//   A wave owns all G = Hq / Hkv query heads of its kv head, so GQA costs no extra KV
//   traffic.  Lane (r = lane/16, c = lane%16) owns dims [8c, 8c+8) of tokens 4i+r of a
//   step (i = 0..3): 4 dwordx4 loads of K and 4 of V per lane, each 16-lane row
//   reading one 256-byte head row.  The loads of step n+1 are issued before step n is
//   computed (register double buffer), so 8-16 KiB per wave stay in flight.  KV rows are
//   read with the nontemporal hint (each byte is used once; measured +12% on MI355X over
//   plain loads, which keep the stream in L2 for nothing); addresses
//   past the context are clamped onto its last token (masked in the softmax), so no
//   branch guards a load.
//   Scores: q.k with v_dot2c_f32_bf16 on packed bf16 pairs, then a 4-step DPP sum
//   across the 16-lane row.  Softmax: online, base 2, scale*log2(e) folded into the
//   scores, one running (max, sum, acc[8]) per lane row.
//   Output: where a wave's range ends or a sequence ends, the 4 lane rows are merged
//   with cross-lane shuffles; a sequence covered by one range writes bf16 directly,
//   otherwise each range writes (max, sum, unnormalised acc) in fp32 to the workspace
//   and decode_merge_kernel combines them with the same online-softmax rule.  Partial
//   traffic is about 2 states per group per sequence boundary: well under 1% of the KV
//   bytes.
//   Partial slots: the state that range r writes for sequence b goes to slot r + b.
//   Sequence b's ranges are first_b .. last_b (first_b = cum_b / spr), and the next
//   sequence with steps starts at a range >= last_b, so slots are unique, and one
//   sequence's slots are consecutive.  A launch with R ranges over B sequences uses at
//   most R + B slots of num_q_heads states each, whatever the context lengths.
#include <math.h>

#include <algorithm>
#include <atomic>
#include <type_traits>

#include "common.h"

namespace kvp {

constexpr int kDecodeHeadDim = 128;
constexpr int kDecodeWaves = 4;  // kv heads per workgroup
constexpr int kDecodeThreads = 64 * kDecodeWaves;
constexpr int kMinRangeTokens = 128;        // a range covers at least 128 tokens
constexpr int kMinStepTokens = 16;           // smallest step (G = 8); G <= 4 steps 32 tokens
constexpr int kG5Step = 32;                  // G = 5 (Qwen3-14B: 40 q heads over 8 kv heads)
constexpr int kMaxSeqsPerLaunch = 4096;      // size of the LDS prefix-sum table
constexpr int kHeaderInts = 16;              // workspace header before the prefix table
// Upper bound of the persistent grid.  The variants hold 1 or 2 workgroups per CU on
// MI355X (at most 512 in all); the cap makes the workspace bound independent of the device.
constexpr int kMaxDecodeGrid = 1024;

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
  int32_t num_seqs;  // <= kMaxSeqsPerLaunch
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t block_size;
  int32_t max_blocks;
  int32_t step_tokens;  // tokens per step (the kernel's STEP)
  float scale_log2;   // softmax_scale * log2(e)
  uint16_t* out;
  int64_t o_seq_stride, o_head_stride;
  int32_t* header;  // [0] steps per range, [kHeaderInts ..] step prefix sums (B + 1)
  float* part_o;    // [slot][num_q_heads][128], slot = range + sequence (ranges + B slots)
  float* part_ml;   // [slot][num_q_heads][2] = (max, sum)
  // Fused q/k norm + RoPE + append (FUSED kernels): row b of qkv holds the token's
  // num_q_heads q heads, then num_kv_heads k heads, then num_kv_heads v heads.
  // The token's position is context_lens[b] - 1.
  const uint16_t* qkv;
  int64_t qkv_stride;
  const float* cos_sin;  // [max_position][128] fp32: cos of the 64 frequencies, then sin
  int32_t max_position;
  const uint16_t* q_weight;
  const uint16_t* k_weight;
  float eps;
  const int32_t* slot_mapping;
  int64_t num_cache_slots;
};

__device__ __forceinline__ uint4 load16(const uint16_t* ptr) {
  return *reinterpret_cast<const uint4*>(ptr);
}

// A wave-uniform read of read-only metadata (context lengths, block tables) through the
// constant address space, so it compiles to a scalar load.  Scalar loads are counted
// apart from the vector loads of the K/V stream: waiting for a block id does not wait
// for the KV loads in flight (as a vector load's wait would, vector loads complete in
// order), and a block id loaded one block ahead is waited for only where it is used.
__device__ __forceinline__ int load_uniform(const int32_t* base, int64_t idx) {
  return ((const __attribute__((address_space(4))) int32_t*)(base))[idx];
}

// Steps of a sequence; 0 for empty or impossible contexts (written separately).
__device__ __forceinline__ int seq_steps(int ctx, const DecodeParams& p) {
  if (ctx <= 0 || ctx > p.max_blocks * p.block_size) return 0;
  return (ctx + p.step_tokens - 1) / p.step_tokens;
}

// s_cum[b] = steps of sequences 0..b-1 (b = 0..num_seqs), built by the whole workgroup:
// each thread sums a contiguous run of sequences, then the 256 run totals are scanned
// with DPP within each wave and the 4 wave totals through LDS (one barrier; a
// Hillis-Steele scan over LDS took 16: 15.0 -> 14.65 us per call for 4 sequences).
__device__ void build_step_prefix(const DecodeParams& p, int* s_cum, int* s_part) {
  const int tid = threadIdx.x;
  const int B = p.num_seqs;
  const int per = (B + kDecodeThreads - 1) / kDecodeThreads;
  const int j0 = tid * per;
  int local = 0;
  for (int i = 0; i < per; ++i) {
    const int b = j0 + i;
    if (b < B) local += seq_steps(p.context_lens[b], p);
  }
  // Rows with nothing to attend (ctx 0: graph padding) read as zeros; impossible
  // lengths read as NaN.  Neither has steps.  Workgroup w writes rows b == w (mod grid).
  for (int i = 0; i < per; ++i) {
    const int b = j0 + i;
    if (b >= B || b % static_cast<int>(gridDim.x) != static_cast<int>(blockIdx.x)) continue;
    const int ctx = p.context_lens[b];
    if (ctx > 0 && ctx <= p.max_blocks * p.block_size) continue;
    const uint16_t fill = ctx <= 0 ? 0 : 0x7fc0;
    for (int o = 0; o < p.num_q_heads * kDecodeHeadDim; o += 8) {
      const int h = o / kDecodeHeadDim, d = o - h * kDecodeHeadDim;
      const uint4 f = make_uint4(fill * 0x10001u, fill * 0x10001u, fill * 0x10001u, fill * 0x10001u);
      *reinterpret_cast<uint4*>(p.out + b * p.o_seq_stride + h * p.o_head_stride + d) = f;
    }
  }
  // Inclusive scan of the run totals within each wave (DPP and lane reads), then across
  // the 4 waves through LDS: one barrier.
  const int lane = tid & 63, wave = tid >> 6;
  const int incl = wave_incl_scan(local);
  if (lane == 63) s_part[wave] = incl;
  __syncthreads();
  int before = 0;
#pragma unroll
  for (int w = 0; w < kDecodeWaves - 1; ++w)
    if (w < wave) before += s_part[w];
  int run = before + incl - local;
  for (int i = 0; i < per; ++i) {
    const int b = j0 + i;
    if (b < B) {
      s_cum[b] = run;
      run += seq_steps(p.context_lens[b], p);
    }
  }
  if (tid == kDecodeThreads - 1) s_cum[B] = before + incl;
  __syncthreads();
}

// Ranges [part_first(b), part_last(b)] touch sequence b's steps [cum_b, cum_b1).
__device__ __forceinline__ int num_parts(int cum_b, int cum_b1, int spr) {
  return (cum_b1 - 1) / spr - cum_b / spr + 1;
}

// Per-wave cursor over the steps of one range.
struct StepCursor {
  int b;        // sequence
  int j;        // step within the sequence
  int nsteps;   // steps of sequence b
  int ctx;      // context length of sequence b
  int lblk;     // logical block whose id is cached in blk (-1: none)
  int blk;      // physical block id of lblk
  int pf_blk;   // id of block lblk + 1, loaded one block ahead (-1: not loaded)
  bool bad;     // a needed block id was out of range
};

__device__ __forceinline__ void cursor_start_seq(const DecodeParams& p, StepCursor& cur, int b, int j) {
  cur.b = b;
  cur.j = j;
  cur.ctx = load_uniform(p.context_lens, b);
  cur.nsteps = seq_steps(cur.ctx, p);
  cur.lblk = -1;
  cur.blk = 0;
  cur.pf_blk = -1;
  cur.bad = false;
}

// Address (in elements) of this lane's first token of the cursor's step, and the number
// of valid tokens of the step.  On entering a block it takes the id prefetched one
// block earlier (or loads it) and prefetches the next block's id, so the scalar load
// is off the critical path.
template <int STEP>
__device__ __forceinline__ int64_t step_base(const DecodeParams& p, StepCursor& cur, int64_t head_off,
                                            int& nvalid) {
  const int t0 = cur.j * STEP;
  const int lblk = t0 / p.block_size;
  if (lblk != cur.lblk) {
    const int32_t* row = p.block_tables + cur.b * p.bt_stride;
    int blk = (cur.lblk >= 0 && lblk == cur.lblk + 1 && cur.pf_blk != -1) ? cur.pf_blk : load_uniform(row, lblk);
    if (blk < 0 || blk >= p.num_cache_blocks) {
      cur.bad = true;
      blk = 0;
    }
    cur.blk = blk;
    cur.lblk = lblk;
    cur.pf_blk = (lblk + 1) * p.block_size < cur.ctx ? load_uniform(row, lblk + 1) : -1;
  }
  nvalid = min(STEP, cur.ctx - t0);
  return static_cast<int64_t>(cur.blk) * p.blk_stride +
         static_cast<int64_t>(t0 - lblk * p.block_size) * p.slot_stride + head_off;
}

// Token 4i + r of the step, clamped onto the last valid token so every load is in
// bounds and needs no branch; clamped tokens are masked out of the softmax.
template <int NL>
__device__ __forceinline__ void step_load(const DecodeParams& p, int64_t base, int nvalid, int r,
                                          uint4 (&kr)[NL], uint4 (&vr)[NL]) {
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int t = min(4 * i + r, nvalid - 1);
    kr[i] = load16_nt(p.k_cache + base + t * p.slot_stride);
    vr[i] = load16_nt(p.v_cache + base + t * p.slot_stride);
  }
}

template <int G, int NL>
__device__ __forceinline__ void step_compute(const DecodeParams& p, const uint4 (&qv)[G],
                                             const uint4 (&kr)[NL], const uint4 (&vr)[NL],
                                             int nvalid, int r, float (&m)[G], float (&l)[G],
                                             float (&acc)[G][8]) {
  float s[G][NL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mx = kMaxFloor;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      float part = dot2_bf16(qv[g].x, kr[i].x, 0.f);
      part = dot2_bf16(qv[g].y, kr[i].y, part);
      part = dot2_bf16(qv[g].z, kr[i].z, part);
      part = dot2_bf16(qv[g].w, kr[i].w, part);
      const float sc = row16_sum(part) * p.scale_log2;
      s[g][i] = (4 * i + r < nvalid) ? sc : -INFINITY;
      mx = fmaxf(mx, s[g][i]);
    }
    const float m_new = fmaxf(m[g], mx);
    const float alpha = fast_exp2(m[g] - m_new);
    m[g] = m_new;
    l[g] *= alpha;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] *= alpha;
  }
  // P V: each V row is widened to fp32 once and feeds all G heads.
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const float vf[8] = {bf16_lo(vr[i].x), bf16_hi(vr[i].x), bf16_lo(vr[i].y), bf16_hi(vr[i].y),
                         bf16_lo(vr[i].z), bf16_hi(vr[i].z), bf16_lo(vr[i].w), bf16_hi(vr[i].w)};
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float pr = fast_exp2(s[g][i] - m[g]);
      l[g] += pr;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[g][j] += pr * vf[j];
    }
  }
}

// Merges the 4 lane rows of the wave and writes the state of (b, kvh) for this range:
// the bf16 output when one range covers the sequence, otherwise an fp32 partial.
template <int G>
__device__ __forceinline__ void emit_state(const DecodeParams& p, int b, int kvh, int slot, bool single,
                                           bool bad, int lane, float (&m)[G], float (&l)[G],
                                           float (&acc)[G][8]) {
  const int c = lane & 15;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float mm = xor32_max(xor16_max(m[g]));
    const float sc = fast_exp2(m[g] - mm);
    const float ll0 = xor32_sum(xor16_sum(l[g] * sc));
    float a[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = xor32_sum(xor16_sum(acc[g][j] * sc));
    float ll = ll0;
    if (bad) ll = NAN;
    const int h = kvh * G + g;
    if (lane < 16) {
      if (single) {
        const float inv = 1.f / ll;
        uint4 o;
        o.x = pack_bf16x2(a[0] * inv, a[1] * inv);
        o.y = pack_bf16x2(a[2] * inv, a[3] * inv);
        o.z = pack_bf16x2(a[4] * inv, a[5] * inv);
        o.w = pack_bf16x2(a[6] * inv, a[7] * inv);
        *reinterpret_cast<uint4*>(p.out + b * p.o_seq_stride + h * p.o_head_stride + 8 * c) = o;
      } else {
        const int64_t row = static_cast<int64_t>(slot) * p.num_q_heads + h;
        float4* dst = reinterpret_cast<float4*>(p.part_o + row * kDecodeHeadDim + 8 * c);
        dst[0] = make_float4(a[0], a[1], a[2], a[3]);
        dst[1] = make_float4(a[4], a[5], a[6], a[7]);
        if (c == 0) *reinterpret_cast<float2*>(p.part_ml + row * 2) = make_float2(mm, ll);
      }
    }
  }
}

// ---- fused q/k norm + RoPE + append (FUSED kernels)
//
// The inputs of the q of a sequence (its cos/sin row and raw q heads) and of its new token
// (cos/sin row, raw k and v heads) reach a per-wave LDS scratch with direct-to-LDS buffer
// loads (buffer_load_dwordx4 ... lds: lane l writes 16 bytes at M0 + 16 l), issued one
// step before they are needed, so the wave never waits on a dependent load chain at a
// sequence boundary and no VGPR holds them meanwhile.  Each kind has two regions, one per
// copy of the unrolled step loop; a region is read by the step copy that consumes it and
// written only by the other copy.  A region read at the end of step S was filled during
// step S - 1, after the K/V loads of step S and before those of step S + 1 (2 NL loads);
// vector memory operations complete in issue order, so an explicit wait that leaves at
// most 2 NL of them in flight covers it.  The compiler's own tracking of direct-to-LDS
// loads does not order these reads, hence the explicit wait.  The token's position is
// context_lens[b] - 1.
constexpr int kFzRow = 512;  // bytes: one cos/sin row, 128 fp32
constexpr int kFzNew = 1024;  // new token: cos/sin row | raw k head | raw v head
template <int G>
struct FzSize {  // q of a sequence: cos/sin row | G raw q heads, in 1 KiB loads
  static constexpr int kLoads = (kFzRow + G * 256 + 1023) / 1024;
  static constexpr int kBytes = kLoads * 1024;
};

__device__ __forceinline__ BufferRsrc cos_sin_rsrc(const DecodeParams& p) {
  return buffer_rsrc(p.cos_sin, static_cast<uint32_t>(p.max_position) * kFzRow);
}
__device__ __forceinline__ BufferRsrc qkv_rsrc(const DecodeParams& p) {
  return buffer_rsrc(p.qkv, static_cast<uint32_t>(p.num_seqs * p.qkv_stride * 2));
}
__device__ __forceinline__ int fz_row_bytes(const DecodeParams& p, int ctx) {
  const int pos = ctx - 1;
  return (pos >= 0 && pos < p.max_position ? pos : 0) * kFzRow;
}

// Weights: lanes 0-15 the q norm weight, 16-31 the k norm weight.
__device__ __forceinline__ void fz_issue_weights(const DecodeParams& p, int lane, char* region) {
  if (lane < 16) lds_dma16(buffer_rsrc(p.q_weight, 256), 16 * lane, region);
  else if (lane < 32) lds_dma16(buffer_rsrc(p.k_weight, 256), 16 * (lane - 16), region);
}

// q inputs of sequence b (context ctx) for kv head kvh: the cos/sin row at bytes 0-511,
// then the G q heads.
template <int G>
__device__ __forceinline__ void fz_issue_q(const DecodeParams& p, int b, int ctx, int kvh, int lane, char* region) {
  if (lane < 32) lds_dma16(cos_sin_rsrc(p), fz_row_bytes(p, ctx) + 16 * lane, region);
  const int heads = (b * static_cast<int>(p.qkv_stride) + kvh * G * kRopeDim) * 2;
#pragma unroll
  for (int i = 0; i < FzSize<G>::kLoads; ++i) {
    const int byte = 1024 * i + 16 * lane;  // this lane's destination within the region
    if (byte >= kFzRow && byte < kFzRow + G * 256) lds_dma16(qkv_rsrc(p), heads + byte - kFzRow, region + 1024 * i);
  }
}

// New-token inputs of sequence b (context ctx) for kv head kvh: the cos/sin row, then the
// raw k head (bytes 512-767) and the raw v head (768-1023).
__device__ __forceinline__ void fz_issue_new(const DecodeParams& p, int b, int ctx, int kvh, int lane, char* region) {
  if (lane < 32) {
    lds_dma16(cos_sin_rsrc(p), fz_row_bytes(p, ctx) + 16 * lane, region);
  } else {
    const int head = lane < 48 ? p.num_q_heads + kvh : p.num_q_heads + p.num_kv_heads + kvh;
    lds_dma16(qkv_rsrc(p), (b * static_cast<int>(p.qkv_stride) + head * kRopeDim) * 2 + 16 * (lane & 15), region);
  }
}

__device__ __forceinline__ void fz_cos_sin(const char* row, int c, float (&cs)[8], float (&sn)[8]) {
  const float* f = reinterpret_cast<const float*>(row) + 8 * (c & 7);
  *reinterpret_cast<float4*>(cs) = *reinterpret_cast<const float4*>(f);
  *reinterpret_cast<float4*>(cs + 4) = *reinterpret_cast<const float4*>(f + 4);
  *reinterpret_cast<float4*>(sn) = *reinterpret_cast<const float4*>(f + kRopeDim / 2);
  *reinterpret_cast<float4*>(sn + 4) = *reinterpret_cast<const float4*>(f + kRopeDim / 2 + 4);
}

// q of a sequence from its q region: RMS-normalised and rotated, in the decode's q layout
// (lane c: dims 8c..8c+7 of every head).
template <int G>
__device__ __forceinline__ void fz_finish_q(const DecodeParams& p, int ctx, int c, const char* region,
                                            const char* weights, uint4 (&qv)[G]) {
  const bool pos_ok = ctx - 1 >= 0 && ctx - 1 < p.max_position;
  float w[8], cs[8], sn[8];
  unpack8(*reinterpret_cast<const uint4*>(weights + 16 * c), w);
  fz_cos_sin(region, c, cs, sn);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float x[8];
    unpack8(*reinterpret_cast<const uint4*>(region + kFzRow + 256 * g + 16 * c), x);
    norm_rope_head(x, w, cs, sn, c < 8, pos_ok, p.eps);
    qv[g] = pack8(x);
  }
}

// The new token of sequence b: k normalised and rotated, v as is; both appended at
// slot_mapping[b] (-1 or a slot outside the pool: not stored) by lanes 0-15, and folded
// into the wave's online softmax as one more key (counted in lane row 0 only; the step
// that loaded its slot masked it out).  Only the wave owning the sequence's final step of
// kv head kvh runs this, so the appended token is never read from the cache in the launch.
template <int G>
__device__ __forceinline__ void fz_finish_new(const DecodeParams& p, int b, int ctx, int kvh, int r, int c,
                                              const char* region, const char* weights, const uint4 (&qv)[G],
                                              float (&m)[G], float (&l)[G], float (&acc)[G][8]) {
  const bool pos_ok = ctx - 1 >= 0 && ctx - 1 < p.max_position;
  const int slot = load_uniform(p.slot_mapping, b);
  float w[8], cs[8], sn[8], x[8];
  unpack8(*reinterpret_cast<const uint4*>(weights + 256 + 16 * c), w);
  fz_cos_sin(region, c, cs, sn);
  unpack8(*reinterpret_cast<const uint4*>(region + kFzRow + 16 * c), x);
  const uint4 vraw = *reinterpret_cast<const uint4*>(region + kFzRow + 256 + 16 * c);
  norm_rope_head(x, w, cs, sn, c < 8, pos_ok, p.eps);
  const uint4 knew = pack8(x);
  if (r == 0 && slot >= 0 && slot < p.num_cache_slots) {
    const int blk = slot / p.block_size, off = slot - blk * p.block_size;
    const int64_t at = static_cast<int64_t>(blk) * p.blk_stride + static_cast<int64_t>(off) * p.slot_stride +
                       static_cast<int64_t>(kvh) * p.head_stride + 8 * c;
    *reinterpret_cast<uint4*>(const_cast<uint16_t*>(p.k_cache) + at) = knew;
    *reinterpret_cast<uint4*>(const_cast<uint16_t*>(p.v_cache) + at) = vraw;
  }
  const float vf[8] = {bf16_lo(vraw.x), bf16_hi(vraw.x), bf16_lo(vraw.y), bf16_hi(vraw.y),
                       bf16_lo(vraw.z), bf16_hi(vraw.z), bf16_lo(vraw.w), bf16_hi(vraw.w)};
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float part = dot2_bf16(qv[g].x, knew.x, 0.f);
    part = dot2_bf16(qv[g].y, knew.y, part);
    part = dot2_bf16(qv[g].z, knew.z, part);
    part = dot2_bf16(qv[g].w, knew.w, part);
    const float sc = r == 0 ? row16_sum(part) * p.scale_log2 : -INFINITY;
    const float m_new = fmaxf(m[g], sc);
    const float alpha = fast_exp2(m[g] - m_new);
    const float pr = fast_exp2(sc - m_new);
    m[g] = m_new;
    l[g] = l[g] * alpha + pr;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = acc[g][j] * alpha + pr * vf[j];
  }
}

template <int G, int STEP, bool FUSED>
__global__ __launch_bounds__(kDecodeThreads) void paged_decode_kernel(const DecodeParams p) {
  constexpr int NL = STEP / 4;  // dwordx4 loads per lane per tensor per step
  constexpr int kMinSteps = kMinRangeTokens / STEP;
  __shared__ int s_cum[kMaxSeqsPerLaunch + 1];
  __shared__ int s_part[kDecodeThreads];
  // fused scratch, per wave: norm weights; q inputs and new-token inputs, one region of
  // each per copy of the unrolled step loop (see the fused helpers)
  constexpr int kFzWaves = FUSED ? kDecodeWaves : 1;
  __shared__ __attribute__((aligned(16))) char s_fw[kFzWaves][1024];
  __shared__ __attribute__((aligned(16))) char s_fq0[kFzWaves][FUSED ? FzSize<G>::kBytes : 16];
  __shared__ __attribute__((aligned(16))) char s_fq1[kFzWaves][FUSED ? FzSize<G>::kBytes : 16];
  __shared__ __attribute__((aligned(16))) char s_fn0[kFzWaves][FUSED ? kFzNew : 16];
  __shared__ __attribute__((aligned(16))) char s_fn1[kFzWaves][FUSED ? kFzNew : 16];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r = lane >> 4;
  const int c = lane & 15;

  build_step_prefix(p, s_cum, s_part);
  const int B = p.num_seqs;
  const int total_steps = s_cum[B];
  const int groups_per_range = (p.num_kv_heads + kDecodeWaves - 1) / kDecodeWaves;
  const int num_ranges = max(1, static_cast<int>(gridDim.x) / groups_per_range);
  const int spr = max(kMinSteps, (total_steps + num_ranges - 1) / num_ranges);
  if (blockIdx.x == 0) {  // for the merge kernel
    if (tid == 0) p.header[0] = spr;
    for (int b = tid; b <= B; b += kDecodeThreads) p.header[kHeaderInts + b] = s_cum[b];
  }

  const int range = blockIdx.x / groups_per_range;
  const int kvh = (blockIdx.x - range * groups_per_range) * kDecodeWaves + wave;
  const int S0 = range * spr;
  const int S1 = min(total_steps, S0 + spr);
  if (kvh >= p.num_kv_heads || S0 >= S1) return;  // no barrier follows

  // Sequence holding step S0: s_cum[b] <= S0 < s_cum[b + 1].
  int lo = 0, hi = B;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (s_cum[mid] <= S0) lo = mid;
    else hi = mid;
  }
  StepCursor cur;
  lo = __builtin_amdgcn_readfirstlane(lo);  // uniform: the cursor's loads stay scalar
  cursor_start_seq(p, cur, lo, __builtin_amdgcn_readfirstlane(S0 - s_cum[lo]));
  const int64_t head_off = static_cast<int64_t>(kvh) * p.head_stride + 8 * c;

  const int fw = FUSED ? wave : 0;
  // The next sequence after the one whose steps end at step S (S < S1 - 1): the first
  // sequence with steps starting at S + 1.
  auto seq_after = [&](int b, int S) {
    int nb = b + 1;
    while (s_cum[nb + 1] == S + 1) ++nb;
    return __builtin_amdgcn_readfirstlane(nb);
  };
  uint4 qv[G];
  if (FUSED) {
    // q of the first sequence (waited for here, once per wave), and, if step S0 ends it,
    // its new token and the next sequence's q for copy 0 of the step loop
    fz_issue_weights(p, lane, s_fw[fw]);
    fz_issue_q<G>(p, cur.b, cur.ctx, kvh, lane, s_fq1[fw]);
    if (cur.j + 1 == cur.nsteps) {
      fz_issue_new(p, cur.b, cur.ctx, kvh, lane, s_fn0[fw]);
      if (S0 + 1 < S1) {
        const int nb = seq_after(cur.b, S0);
        fz_issue_q<G>(p, nb, load_uniform(p.context_lens, nb), kvh, lane, s_fq0[fw]);
      }
    }
    wait_vmem<0>();
    fz_finish_q<G>(p, cur.ctx, c, s_fq1[fw], s_fw[fw], qv);
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g)
      qv[g] = load16(p.q + cur.b * p.q_seq_stride + (kvh * G + g) * p.q_head_stride + 8 * c);
  }
  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kMaxFloor;
    l[g] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = 0.f;
  }

  // Tokens a step's loads may touch: with FUSED, a sequence's final step holds the token
  // this launch appends, whose slot is not written yet; its rows are clamped onto the
  // last cached token instead (a step with only the new token loads that slot but is
  // never computed).
  auto fused_load_count = [](const StepCursor& s, int nv) { return s.j + 1 == s.nsteps && nv > 1 ? nv - 1 : nv; };
  uint4 kA[NL], vA[NL], kB[NL], vB[NL];
  int nvA, nvB = 0;
  if constexpr (FUSED) {
    const int64_t base = step_base<STEP>(p, cur, head_off, nvA);
    step_load<NL>(p, base, fused_load_count(cur, nvA), r, kA, vA);
  } else {
    step_load<NL>(p, step_base<STEP>(p, cur, head_off, nvA), nvA, r, kA, vA);
  }

  // One step: prefetch the next step into (kN, vN), compute (kC, vC), emit at the end
  // of a sequence or of the range.  Returns false when the range is done.
  // Compute of the step held in (kC, vC), the fused new token at a sequence end, the emit
  // at the end of a sequence or of the range, and with MORE the switch to the next
  // sequence's q.  The last step of a range gets its own instance: where the path that
  // prefetched the next step met the one that did not, the compiler would keep the
  // smaller wait count of the two and stall on the prefetch.
  auto finish = [&](const uint4 (&kC)[NL], const uint4 (&vC)[NL], int nvC, bool seq_end, const StepCursor& nxt,
                    const uint4 (&qn)[G], char* fq_mine, char* fn_mine, auto more_c) {
    constexpr bool MORE = decltype(more_c)::value;
    // Fused: the sequence's last token is not read from the cache (it is appended by this
    // launch) but folded in from the qkv row after the step.  The step's loads were
    // clamped onto the last cached token (fused_load_count), so no row holds the
    // unwritten slot; a final step with no cached token is not computed at all.
    if constexpr (FUSED) {
      if (!(seq_end && nvC == 1)) step_compute<G, NL>(p, qv, kC, vC, seq_end ? nvC - 1 : nvC, r, m, l, acc);
    } else {
      step_compute<G, NL>(p, qv, kC, vC, nvC, r, m, l, acc);
    }
    if (FUSED && seq_end) {
      // this sequence's new-token region and, with MORE, the next one's q region were
      // filled before the K/V loads of the next step
      if (MORE) wait_vmem<2 * NL>();
      else wait_vmem<0>();
      fz_finish_new<G>(p, cur.b, cur.ctx, kvh, r, c, fn_mine, s_fw[fw], qv, m, l, acc);
    }
    if (!MORE || seq_end) {
      const int cb = s_cum[cur.b], cb1 = s_cum[cur.b + 1];
      const int np = num_parts(cb, cb1, spr);
      emit_state<G>(p, cur.b, kvh, range + cur.b, np == 1, cur.bad, lane, m, l, acc);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        m[g] = kMaxFloor;
        l[g] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[g][j] = 0.f;
      }
      if (MORE) {
        if (FUSED) {
          fz_finish_q<G>(p, nxt.ctx, c, fq_mine, s_fw[fw], qv);
        } else {
#pragma unroll
          for (int g = 0; g < G; ++g) qv[g] = qn[g];
        }
      }
    }
  };

  // One step: prefetch the next step into (kN, vN), then finish this one.  Returns false
  // when the range is done.
  auto advance = [&](uint4 (&kC)[NL], uint4 (&vC)[NL], int nvC,
                     uint4 (&kN)[NL], uint4 (&vN)[NL], int& nvN, int S, auto copy) -> bool {
    constexpr int X = decltype(copy)::value;  // this copy of the step loop (0 or 1)
    char* fq_mine = X == 0 ? s_fq0[fw] : s_fq1[fw];
    char* fn_mine = X == 0 ? s_fn0[fw] : s_fn1[fw];
    char* fq_other = X == 0 ? s_fq1[fw] : s_fq0[fw];
    char* fn_other = X == 0 ? s_fn1[fw] : s_fn0[fw];
    const bool seq_end = cur.j + 1 == cur.nsteps;
    if (S + 1 < S1) {
      StepCursor nxt = cur;
      uint4 qn[G];
      if (seq_end) {
        // next non-empty sequence: the one whose steps start at S + 1
        const int nb = seq_after(cur.b, S);
        cursor_start_seq(p, nxt, nb, 0);
        if (!FUSED) {
#pragma unroll
          for (int g = 0; g < G; ++g)
            qn[g] = load16(p.q + nb * p.q_seq_stride + (kvh * G + g) * p.q_head_stride + 8 * c);
        }
      } else {
        nxt.j = cur.j + 1;
      }
      if constexpr (FUSED) {
        const int64_t base = step_base<STEP>(p, nxt, head_off, nvN);
        step_load<NL>(p, base, fused_load_count(nxt, nvN), r, kN, vN);
      } else {
        step_load<NL>(p, step_base<STEP>(p, nxt, head_off, nvN), nvN, r, kN, vN);
      }
      if (FUSED && nxt.j + 1 == nxt.nsteps) {
        // step S + 1 (the other copy) ends sequence nxt.b: its new token, and the q of the
        // sequence after it, for that copy
        fz_issue_new(p, nxt.b, nxt.ctx, kvh, lane, fn_other);
        if (S + 2 < S1) {
          const int nb2 = seq_after(nxt.b, S + 1);
          fz_issue_q<G>(p, nb2, load_uniform(p.context_lens, nb2), kvh, lane, fq_other);
        }
      }
      finish(kC, vC, nvC, seq_end, nxt, qn, fq_mine, fn_mine, std::true_type{});
      cur = nxt;
      return true;
    }
    finish(kC, vC, nvC, seq_end, cur, qv, fq_mine, fn_mine, std::false_type{});
    return false;
  };

  for (int S = S0;; S += 2) {
    if (!advance(kA, vA, nvA, kB, vB, nvB, S, std::integral_constant<int, 0>{})) break;
    if (!advance(kB, vB, nvB, kA, vA, nvA, S + 1, std::integral_constant<int, 1>{})) break;
  }
}

// Combines the per-range partial states of sequences that span several ranges.
// grid = (ceil(num_q_heads / 4), num_seqs), 128 threads: 4 query heads x 32 threads,
// 4 output elements (16-byte partial rows) per thread.  A quarter of the waves of one
// thread per element: 175.0 -> 174.2 us per decode call on 256 sequences, and about
// 1 us less for small batches.
// The kernel is latency-bound: it reads the sequence's step span and the steps per range
// from the header (one round trip), then its first kSpecParts slots together (a second
// one: the slots are consecutive and start at slot first_b + b); rows past the part count
// are clamped onto the last part and ignored.
constexpr int kMergeHeads = 4;
constexpr int kSpecParts = 4;
constexpr int kMergeThreads = kMergeHeads * kDecodeHeadDim / 4;  // 4 dims per thread
__device__ __forceinline__ float4 fma4(float w, float4 o, float4 acc) {
  return make_float4(acc.x + w * o.x, acc.y + w * o.y, acc.z + w * o.z, acc.w + w * o.w);
}
__global__ __launch_bounds__(kMergeThreads) void decode_merge_kernel(const DecodeParams p) {
  constexpr int D = kDecodeHeadDim;
  const int h = blockIdx.x * kMergeHeads + static_cast<int>(threadIdx.x) / (D / 4);
  const int b = blockIdx.y;
  const int d = 4 * (threadIdx.x % (D / 4));
  if (h >= p.num_q_heads) return;
  const int cb = load_uniform(p.header, kHeaderInts + b), cb1 = load_uniform(p.header, kHeaderInts + b + 1);
  const int spr = load_uniform(p.header, 0);
  if (cb1 <= cb) return;  // no steps: written by the main kernel
  const int np = num_parts(cb, cb1, spr);
  if (np <= 1) return;  // written by the main kernel
  const int64_t row0 = static_cast<int64_t>(cb / spr + b) * p.num_q_heads + h;  // first slot's row
  const int64_t hq = p.num_q_heads;  // rows between consecutive slots
  const float* ml = p.part_ml + row0 * 2;
  const float* po = p.part_o + row0 * D + d;
  float2 st0[kSpecParts];
  float4 ov0[kSpecParts];
#pragma unroll
  for (int k = 0; k < kSpecParts; ++k) {
    const int s = min(k, np - 1);
    st0[k] = *reinterpret_cast<const float2*>(ml + 2 * s * hq);
    ov0[k] = *reinterpret_cast<const float4*>(po + s * hq * D);
  }
  float mm = kMaxFloor;
#pragma unroll
  for (int k = 0; k < kSpecParts; ++k)
    if (k < np) mm = fmaxf(mm, st0[k].x);
  float ll = 0.f;
  float4 oo = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int k = 0; k < kSpecParts; ++k) {
    if (k < np) {
      const float w = fast_exp2(st0[k].x - mm);
      ll += w * st0[k].y;
      oo = fma4(w, ov0[k], oo);
    }
  }
  // Further parts (long sequences): batches of 8, all loads of a batch issued first.
  for (int s0 = kSpecParts; s0 < np; s0 += 8) {
    float2 st[8];
    float4 ov[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int s = min(s0 + k, np - 1);
      st[k] = *reinterpret_cast<const float2*>(ml + 2 * s * hq);
      ov[k] = *reinterpret_cast<const float4*>(po + s * hq * D);
    }
    float bm = mm;
#pragma unroll
    for (int k = 0; k < 8; ++k) bm = fmaxf(bm, st[k].x);
    const float alpha = fast_exp2(mm - bm);
    ll *= alpha;
    oo = make_float4(oo.x * alpha, oo.y * alpha, oo.z * alpha, oo.w * alpha);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (s0 + k < np) {
        const float w = fast_exp2(st[k].x - bm);
        ll += w * st[k].y;
        oo = fma4(w, ov[k], oo);
      }
    }
    mm = bm;
  }
  uint16_t* o = p.out + b * p.o_seq_stride + h * p.o_head_stride + d;
  *reinterpret_cast<uint2*>(o) = make_uint2(pack_bf16x2(oo.x / ll, oo.y / ll), pack_bf16x2(oo.z / ll, oo.w / ll));
}

constexpr int64_t kHeaderBytes = ((kHeaderInts + kMaxSeqsPerLaunch + 1) * 4 + 255) / 256 * 256;
constexpr int64_t kStateBytes = (kDecodeHeadDim + 2) * 4;  // one (acc[128], max, sum) state

// Ranges of one launch: the grid's groups, and no more than minimum-size ranges over the
// largest possible work (max_tokens = sequences * table width * block_size).
static int64_t range_cap(int64_t max_tokens) {
  return std::max<int64_t>(1, (max_tokens + kMinRangeTokens - 1) / kMinRangeTokens);
}

// Workspace bytes for a launch of `seqs` sequences over `ranges` ranges.
static int64_t decode_workspace_need(int64_t seqs, int64_t q_heads, int64_t ranges) {
  return kHeaderBytes + (ranges + seqs) * q_heads * kStateBytes;
}

// Workspace bytes that cover every launch of up to `seqs` sequences, on any device:
// a launch has at most kMaxDecodeGrid ranges.
static int64_t decode_workspace_bound(int64_t seqs, int64_t q_heads, int64_t max_blocks, int64_t block_size) {
  const int64_t ranges = std::min<int64_t>(kMaxDecodeGrid, range_cap(seqs * max_blocks * block_size));
  return decode_workspace_need(seqs, q_heads, ranges);
}

// Workgroups of paged_decode_kernel<G, STEP, FUSED> resident on the whole current device
// (cached per device once the queries succeed), capped at kMaxDecodeGrid.
template <int G, int STEP, bool FUSED>
static int resident_workgroups() {
  static std::atomic<int> cached[16];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) dev = 0;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int cus = 0, per_cu = 0;
  bool ok = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0;
  if (!ok) cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, paged_decode_kernel<G, STEP, FUSED>, kDecodeThreads, 0) !=
          hipSuccess || per_cu <= 0) {
    per_cu = 1;
    ok = false;
  }
  v = std::min(cus * per_cu, kMaxDecodeGrid);
  if (ok) cached[dev].store(v, std::memory_order_relaxed);
  return v;
}

template <int G, int STEP, bool FUSED>
static int64_t decode_ranges(int num_kv_heads, int64_t max_tokens) {
  const int64_t groups_per_range = (num_kv_heads + kDecodeWaves - 1) / kDecodeWaves;
  return std::max<int64_t>(1, std::min<int64_t>(resident_workgroups<G, STEP, FUSED>() / groups_per_range,
                                                range_cap(max_tokens)));
}

template <bool FUSED>
static int64_t decode_ranges_for(int G, int num_kv_heads, int64_t max_tokens) {
  switch (G) {
    case 1: return decode_ranges<1, 32, FUSED>(num_kv_heads, max_tokens);
    case 2: return decode_ranges<2, 32, FUSED>(num_kv_heads, max_tokens);
    case 4: return decode_ranges<4, 32, FUSED>(num_kv_heads, max_tokens);
    case 5: return decode_ranges<5, kG5Step, FUSED>(num_kv_heads, max_tokens);
    default: return decode_ranges<8, kMinStepTokens, FUSED>(num_kv_heads, max_tokens);
  }
}

template <int G, int STEP, bool FUSED>
static void launch_decode(DecodeParams p, int64_t ranges, hipStream_t s) {
  const int64_t groups_per_range = (p.num_kv_heads + kDecodeWaves - 1) / kDecodeWaves;
  p.step_tokens = STEP;
  hipLaunchKernelGGL((paged_decode_kernel<G, STEP, FUSED>), dim3(static_cast<unsigned>(ranges * groups_per_range)),
                     dim3(kDecodeThreads), 0, s, p);
  hipLaunchKernelGGL(decode_merge_kernel, dim3((p.num_q_heads + kMergeHeads - 1) / kMergeHeads, p.num_seqs),
                     dim3(kMergeThreads), 0, s, p);
}

struct DecodeArgs {
  const void* q;
  int64_t q_seq_stride, q_head_stride;
  const void* k_cache;
  const void* v_cache;
  int64_t cache_block_stride, cache_slot_stride, cache_head_stride;
  int32_t num_cache_blocks;
  const int32_t* block_tables;
  int64_t block_table_stride;
  const int32_t* context_lens;
  int32_t num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq;
  float softmax_scale;
  void* out;
  int64_t out_seq_stride, out_head_stride;
};

// Host-side argument checks shared by both decode entry points (no HIP call).
static int check_decode_args(const char* fn, const DecodeArgs& a) {
  if (a.num_seqs < 0) return fail(KVP_EINVAL, "%s: num_seqs=%d < 0", fn, a.num_seqs);
  if (a.head_dim != kDecodeHeadDim)
    return fail(KVP_EUNSUPPORTED, "%s: head_dim=%d (supported: 128)", fn, a.head_dim);
  if (a.num_kv_heads <= 0 || a.num_q_heads <= 0 || a.num_q_heads % a.num_kv_heads != 0)
    return fail(KVP_EINVAL, "%s: num_q_heads=%d not a multiple of num_kv_heads=%d", fn, a.num_q_heads,
                a.num_kv_heads);
  const int G = a.num_q_heads / a.num_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 5 && G != 8)
    return fail(KVP_EUNSUPPORTED, "%s: GQA ratio %d (supported: 1, 2, 4, 5, 8)", fn, G);
  if (a.block_size <= 0 || a.block_size % 64 != 0)
    return fail(KVP_EINVAL, "%s: block_size=%d must be a positive multiple of 64", fn, a.block_size);
  if (a.max_blocks_per_seq <= 0 || a.num_cache_blocks <= 0)
    return fail(KVP_EINVAL, "%s: max_blocks_per_seq=%d num_cache_blocks=%d", fn, a.max_blocks_per_seq,
                a.num_cache_blocks);
  if (static_cast<int64_t>(a.max_blocks_per_seq) * a.block_size > (1ll << 30))
    return fail(KVP_EINVAL, "%s: max_blocks_per_seq*block_size too large", fn);
  if (a.block_table_stride < a.max_blocks_per_seq)
    return fail(KVP_EINVAL, "%s: block_table_stride=%lld < max_blocks_per_seq=%d", fn,
                static_cast<long long>(a.block_table_stride), a.max_blocks_per_seq);
  if (!a.q || !a.k_cache || !a.v_cache || !a.block_tables || !a.context_lens || !a.out)
    return fail(KVP_EINVAL, "%s: null pointer", fn);
  if (!aligned16(a.q) || !aligned16(a.k_cache) || !aligned16(a.v_cache))
    return fail(KVP_EINVAL, "%s: q and cache pointers must be 16-byte aligned", fn);
  if (!aligned16(a.out) || (reinterpret_cast<uintptr_t>(a.block_tables) & 3u) ||
      (reinterpret_cast<uintptr_t>(a.context_lens) & 3u))
    return fail(KVP_EINVAL, "%s: misaligned out/block_tables/context_lens", fn);
  if (!mult8(a.q_seq_stride) || !mult8(a.q_head_stride) || !mult8(a.cache_block_stride) ||
      !mult8(a.cache_slot_stride) || !mult8(a.cache_head_stride) || !mult8(a.out_seq_stride) ||
      !mult8(a.out_head_stride))
    return fail(KVP_EINVAL, "%s: q, cache and out strides must be multiples of 8 elements", fn);
  return KVP_OK;
}

// Enqueues the decode of a checked batch on `s` with `ws` as workspace (ws_bytes must
// cover decode_workspace_need of every launch; checked by the callers).  Batches beyond
// the LDS prefix table run as consecutive launches of up to 4096 sequences; they reuse
// the workspace in stream order.
template <bool FUSED>
static int enqueue_decode(const char* fn, const DecodeArgs& a, int64_t ranges, char* ws, hipStream_t s,
                          const DecodeParams* fused = nullptr) {
  const int G = a.num_q_heads / a.num_kv_heads;
  for (int b0 = 0; b0 < a.num_seqs; b0 += kMaxSeqsPerLaunch) {
    const int nb = std::min(kMaxSeqsPerLaunch, a.num_seqs - b0);
    DecodeParams p = fused ? *fused : DecodeParams{};
    if (FUSED) {  // this chunk's rows of the per-sequence inputs
      p.qkv += b0 * p.qkv_stride;
      p.slot_mapping += b0;
    }
    p.q = static_cast<const uint16_t*>(a.q) + b0 * a.q_seq_stride;
    p.q_seq_stride = a.q_seq_stride;
    p.q_head_stride = a.q_head_stride;
    p.k_cache = static_cast<const uint16_t*>(a.k_cache);
    p.v_cache = static_cast<const uint16_t*>(a.v_cache);
    p.blk_stride = a.cache_block_stride;
    p.slot_stride = a.cache_slot_stride;
    p.head_stride = a.cache_head_stride;
    p.num_cache_blocks = a.num_cache_blocks;
    p.block_tables = a.block_tables + b0 * a.block_table_stride;
    p.bt_stride = a.block_table_stride;
    p.context_lens = a.context_lens + b0;
    p.num_seqs = nb;
    p.num_q_heads = a.num_q_heads;
    p.num_kv_heads = a.num_kv_heads;
    p.block_size = a.block_size;
    p.max_blocks = a.max_blocks_per_seq;
    p.scale_log2 = a.softmax_scale * 1.4426950408889634f;
    p.out = static_cast<uint16_t*>(a.out) + b0 * a.out_seq_stride;
    p.o_seq_stride = a.out_seq_stride;
    p.o_head_stride = a.out_head_stride;
    p.header = reinterpret_cast<int32_t*>(ws);
    p.part_o = reinterpret_cast<float*>(ws + kHeaderBytes);
    p.part_ml = p.part_o + static_cast<size_t>(ranges + nb) * a.num_q_heads * kDecodeHeadDim;
    switch (G) {
      case 1: launch_decode<1, 32, FUSED>(p, ranges, s); break;
      case 2: launch_decode<2, 32, FUSED>(p, ranges, s); break;
      case 4: launch_decode<4, 32, FUSED>(p, ranges, s); break;
      case 5: launch_decode<5, kG5Step, FUSED>(p, ranges, s); break;
      default: launch_decode<8, kMinStepTokens, FUSED>(p, ranges, s); break;
    }
    const int rc = launch_status(fn);
    if (rc != KVP_OK) return rc;
  }
  return KVP_OK;
}

// Launch ranges for the batch's first (largest) launch.
template <bool FUSED = false>
static int64_t batch_ranges(const DecodeArgs& a) {
  const int nb = std::min(a.num_seqs, kMaxSeqsPerLaunch);
  const int64_t max_tokens = static_cast<int64_t>(nb) * a.max_blocks_per_seq * a.block_size;
  return decode_ranges_for<FUSED>(a.num_q_heads / a.num_kv_heads, a.num_kv_heads, max_tokens);
}

// ---------------------------------------------------------------- no-allocation variant

// Workspace of kvp_paged_decode_bf16_noalloc: one per device, held until the process ends.
constexpr size_t kScratchBytes = 32u << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

// Device address of this device's `scratch`, looked up once per device with that device
// current.  The host-side symbol is not a device address and is never passed to a kernel.
// The lookup may load the library's code object (and the array) on that device, which is
// not an operation to record into a graph: a first call on a device while `stream` is
// being captured is refused, and one call outside capture (any batch) sets the device up.
static int scratch_address(const char* fn, hipStream_t stream, char** out) {
  constexpr int kMaxDevices = 64;
  static std::atomic<char*> addr[kMaxDevices];
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return fail(static_cast<int>(err), "%s: hipGetDevice: %s", fn, hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxDevices) return fail(KVP_EINVAL, "%s: device %d beyond %d", fn, dev, kMaxDevices);
  char* ptr = addr[dev].load(std::memory_order_acquire);
  if (!ptr) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    err = hipStreamIsCapturing(stream, &cap);
    if (err != hipSuccess)
      return fail(static_cast<int>(err), "%s: hipStreamIsCapturing: %s", fn, hipGetErrorString(err));
    if (cap != hipStreamCaptureStatusNone)
      return fail(KVP_EINVAL,
                  "%s: first call on device %d is inside a graph capture; call it once outside capture "
                  "(any batch) to set up the device's static scratch, then capture",
                  fn, dev);
    void* sym = nullptr;
    err = hipGetSymbolAddress(&sym, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !sym)
      return fail(err != hipSuccess ? static_cast<int>(err) : KVP_EINVAL, "%s: hipGetSymbolAddress(scratch): %s",
                  fn, hipGetErrorString(err));
    ptr = static_cast<char*>(sym);
    addr[dev].store(ptr, std::memory_order_release);
  }
  *out = ptr;
  return KVP_OK;
}

}  // namespace kvp

using namespace kvp;

extern "C" size_t kvp_decode_workspace_bytes(int32_t max_num_seqs, int32_t num_q_heads, int32_t head_dim,
                                             int32_t max_blocks_per_seq, int32_t block_size) {
  if (max_num_seqs <= 0 || num_q_heads <= 0 || head_dim != kDecodeHeadDim || max_blocks_per_seq <= 0 ||
      block_size <= 0)
    return 0;
  const int64_t seqs = std::min<int64_t>(max_num_seqs, kMaxSeqsPerLaunch);
  return static_cast<size_t>(decode_workspace_bound(seqs, num_q_heads, max_blocks_per_seq, block_size));
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
  static const char fn[] = "kvp_paged_decode_bf16";
  clear_error();
  const DecodeArgs a = {q, q_seq_stride, q_head_stride, k_cache, v_cache, cache_block_stride,
                        cache_slot_stride, cache_head_stride, num_cache_blocks, block_tables,
                        block_table_stride, context_lens, num_seqs, num_q_heads, num_kv_heads,
                        head_dim, block_size, max_blocks_per_seq, softmax_scale, out,
                        out_seq_stride, out_head_stride};
  int rc = check_decode_args(fn, a);
  if (rc != KVP_OK) return rc;
  if (num_seqs == 0) return KVP_OK;
  const int chunk_seqs = std::min(num_seqs, kMaxSeqsPerLaunch);
  const size_t need =
      static_cast<size_t>(decode_workspace_bound(chunk_seqs, num_q_heads, max_blocks_per_seq, block_size));
  if (!workspace || workspace_bytes < need)
    return fail(KVP_EWORKSPACE, "%s: workspace of %zu bytes, %zu needed", fn, workspace_bytes, need);
  if (reinterpret_cast<uintptr_t>(workspace) & 255u)
    return fail(KVP_EINVAL, "%s: workspace must be 256-byte aligned", fn);
  return enqueue_decode<false>(fn, a, batch_ranges(a), static_cast<char*>(workspace),
                               static_cast<hipStream_t>(stream));
}

extern "C" int kvp_paged_decode_bf16_noalloc(const void* q, int64_t q_seq_stride, int64_t q_head_stride,
                                             const void* k_cache, const void* v_cache,
                                             int64_t cache_block_stride, int64_t cache_slot_stride,
                                             int64_t cache_head_stride, int32_t num_cache_blocks,
                                             const int32_t* block_tables, int64_t block_table_stride,
                                             const int32_t* context_lens, int32_t num_seqs,
                                             int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                             int32_t block_size, int32_t max_blocks_per_seq,
                                             float softmax_scale,
                                             void* out, int64_t out_seq_stride, int64_t out_head_stride,
                                             void* stream) {
  static const char fn[] = "kvp_paged_decode_bf16_noalloc";
  clear_error();
  const DecodeArgs a = {q, q_seq_stride, q_head_stride, k_cache, v_cache, cache_block_stride,
                        cache_slot_stride, cache_head_stride, num_cache_blocks, block_tables,
                        block_table_stride, context_lens, num_seqs, num_q_heads, num_kv_heads,
                        head_dim, block_size, max_blocks_per_seq, softmax_scale, out,
                        out_seq_stride, out_head_stride};
  int rc = check_decode_args(fn, a);
  if (rc != KVP_OK) return rc;
  if (num_seqs == 0) return KVP_OK;
  const int64_t ranges = batch_ranges(a);
  const int64_t need = decode_workspace_need(std::min(num_seqs, kMaxSeqsPerLaunch), num_q_heads, ranges);
  if (need > static_cast<int64_t>(kScratchBytes))
    return fail(KVP_EWORKSPACE,
                "%s: %d sequences x %d query heads need %lld bytes of decode scratch; the static scratch "
                "holds %zu (use kvp_paged_decode_bf16 with a caller workspace)",
                fn, std::min(num_seqs, kMaxSeqsPerLaunch), num_q_heads, static_cast<long long>(need), kScratchBytes);
  char* ws = nullptr;
  rc = scratch_address(fn, static_cast<hipStream_t>(stream), &ws);
  if (rc != KVP_OK) return rc;
  return enqueue_decode<false>(fn, a, ranges, ws, static_cast<hipStream_t>(stream));
}

extern "C" int kvp_paged_decode_fused_bf16(
    const void* qkv, int64_t qkv_tok_stride, const float* cos_sin,
    int32_t max_position, const void* q_norm_weight, const void* k_norm_weight, float eps,
    void* k_cache, void* v_cache, int64_t cache_block_stride, int64_t cache_slot_stride,
    int64_t cache_head_stride, int32_t num_cache_blocks, const int32_t* slot_mapping,
    const int32_t* block_tables, int64_t block_table_stride, const int32_t* context_lens,
    int32_t num_seqs, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t block_size, int32_t max_blocks_per_seq, float softmax_scale,
    void* out, int64_t out_seq_stride, int64_t out_head_stride,
    void* workspace, size_t workspace_bytes, void* stream) {
  static const char fn[] = "kvp_paged_decode_fused_bf16";
  clear_error();
  // q is read from the qkv rows: the q pointer and strides of the shared checks stand in
  // for them (the q heads of row b start at qkv + b * qkv_tok_stride).
  const DecodeArgs a = {qkv, qkv_tok_stride, kRopeDim, k_cache, v_cache, cache_block_stride,
                        cache_slot_stride, cache_head_stride, num_cache_blocks, block_tables,
                        block_table_stride, context_lens, num_seqs, num_q_heads, num_kv_heads,
                        head_dim, block_size, max_blocks_per_seq, softmax_scale, out,
                        out_seq_stride, out_head_stride};
  int rc = check_decode_args(fn, a);
  if (rc != KVP_OK) return rc;
  if (!cos_sin || !q_norm_weight || !k_norm_weight || !slot_mapping)
    return fail(KVP_EINVAL, "%s: null pointer", fn);
  if (max_position < 1) return fail(KVP_EINVAL, "%s: max_position=%d", fn, max_position);
  if (!aligned16(cos_sin) || !aligned16(q_norm_weight) || !aligned16(k_norm_weight) ||
      (reinterpret_cast<uintptr_t>(slot_mapping) & 3u))
    return fail(KVP_EINVAL, "%s: misaligned cos_sin / norm weights / slot_mapping", fn);
  if (qkv_tok_stride < static_cast<int64_t>(num_q_heads + 2 * num_kv_heads) * head_dim)
    return fail(KVP_EINVAL, "%s: qkv row stride %lld is shorter than (hq + 2 hkv) * head_dim", fn,
                static_cast<long long>(qkv_tok_stride));
  if (num_seqs == 0) return KVP_OK;
  const int chunk_seqs = std::min(num_seqs, kMaxSeqsPerLaunch);
  // the kernel addresses the table and one launch's qkv rows with 32-bit byte offsets
  if (static_cast<int64_t>(max_position) * kRopeDim * 4 > INT32_MAX ||
      static_cast<int64_t>(chunk_seqs) * qkv_tok_stride * 2 > INT32_MAX)
    return fail(KVP_EINVAL, "%s: the cos/sin table or %d qkv rows exceed 2 GiB", fn, chunk_seqs);
  const size_t need =
      static_cast<size_t>(decode_workspace_bound(chunk_seqs, num_q_heads, max_blocks_per_seq, block_size));
  if (!workspace || workspace_bytes < need)
    return fail(KVP_EWORKSPACE, "%s: workspace of %zu bytes, %zu needed", fn, workspace_bytes, need);
  if (reinterpret_cast<uintptr_t>(workspace) & 255u)
    return fail(KVP_EINVAL, "%s: workspace must be 256-byte aligned", fn);
  DecodeParams f{};
  f.qkv = static_cast<const uint16_t*>(qkv);
  f.qkv_stride = qkv_tok_stride;
  f.cos_sin = cos_sin;
  f.max_position = max_position;
  f.q_weight = static_cast<const uint16_t*>(q_norm_weight);
  f.k_weight = static_cast<const uint16_t*>(k_norm_weight);
  f.eps = eps;
  f.slot_mapping = slot_mapping;
  f.num_cache_slots = static_cast<int64_t>(num_cache_blocks) * block_size;
  return enqueue_decode<true>(fn, a, batch_ranges<true>(a), static_cast<char*>(workspace),
                              static_cast<hipStream_t>(stream), &f);
}
