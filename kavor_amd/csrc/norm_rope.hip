// The layer work on either side of the paged KV path, fused for gfx950:
//
//   rmsnorm_kernel            (add-)RMSNorm over rows of any 2-D or [T, H, D] strided view
//                             (kavor/layers/layernorm.py:8-40, 113-140, 235-284)
//   qk_norm_rope_append_kernel  per token: q/k RMSNorm, neox RoPE, q written out, k and v
//                             appended to the paged cache (qwen3.py:79-89,
//                             rotary_embedding.py:8-53, flash_attention_kvcache.py:10-34)
//   silu_mul_kernel           SiLU(gate) * up (kavor/layers/activation.py:6-11)
//   argmax_kernel             greedy token per logits row, or a Gumbel-max sample per row
//                             (kavor/layers/sampler.py:7-45)
//
// All are HBM / latency bound elementwise work: every thread moves 16-byte vectors of 8
// bf16, reductions stay in registers (DPP inside a 16-lane row, lane swaps across rows),
// nothing goes through LDS except the argmax's cross-wave step.  Numerics follow the
// reference's eager formulas: statistics in fp32, the normalised value rounded to bf16
// before the weight multiply (double rounding, layernorm.py:32-33), RoPE rotated in fp32
// and rounded once.

#include <algorithm>

#include "common.h"

namespace kvp {

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ uint4 load16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void store16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }

// ------------------------------------------------------------------ RMSNorm

struct NormParams {
  const uint16_t* x;
  int64_t x_s0, x_s1;          // row (t, h) starts at x + t*x_s0 + h*x_s1 (elements)
  uint16_t* residual;          // nullptr: plain RMSNorm; else read, added, rewritten in place
  int64_t r_s0, r_s1;
  const uint16_t* weight;
  uint16_t* out;
  int64_t o_s0, o_s1;
  int rows_inner;              // rows per leading index (H of a [T, H, D] view, 1 for 2-D)
  int num_rows;
  int cols;                    // multiple of 8
  float eps;
};

// LANES (16 or 64) lanes normalise one row; each lane owns up to MAXC 8-element chunks.
template <int LANES, int MAXC>
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(NormParams p) {
  const int lane = threadIdx.x % LANES;
  const int row = (blockIdx.x * kThreads + threadIdx.x) / LANES;
  if (row >= p.num_rows) return;  // uniform across the lanes of a row
  const int t = row / p.rows_inner, h = row - t * p.rows_inner;
  const uint16_t* xr = p.x + t * p.x_s0 + h * p.x_s1;
  uint16_t* rr = p.residual ? p.residual + t * p.r_s0 + h * p.r_s1 : nullptr;
  uint16_t* orow = p.out + t * p.o_s0 + h * p.o_s1;
  const int nch = p.cols >> 3;

  // The weight chunks are loaded with the row, so the output waits for one memory round
  // trip, not two (3.15 -> 2.94 us per call at 256 x 1024 with a residual, graph-replayed).
  uint4 wv[MAXC];
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = lane + i * LANES;
    wv[i] = load16(p.weight + 8 * (c < nch ? c : 0));
  }
  float v[MAXC][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = lane + i * LANES;
    const bool ok = c < nch;
    const int cc = ok ? c : 0;
    unpack8(load16(xr + 8 * cc), v[i]);
    if (rr) {
      float r[8];
      unpack8(load16(rr + 8 * cc), r);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[i][e] += r[e];
      if (ok) store16(rr + 8 * c, pack8(v[i]));
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (!ok) v[i][e] = 0.f;
      ss += v[i][e] * v[i][e];
    }
  }
  ss = row16_sum(ss);
  if (LANES == 64) ss = xor32_sum(xor16_sum(ss));
  const float rstd = rsqrtf(ss / static_cast<float>(p.cols) + p.eps);
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = lane + i * LANES;
    if (c < nch) {
      float w[8], y[8];
      unpack8(wv[i], w);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = round_bf16(v[i][e] * rstd) * w[e];
      store16(orow + 8 * c, pack8(y));
    }
  }
}

template <int LANES, int MAXC>
void launch_norm(const NormParams& p, hipStream_t stream) {
  const int rows_per_block = kThreads / LANES;
  const int grid = (p.num_rows + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL((rmsnorm_kernel<LANES, MAXC>), dim3(grid), dim3(kThreads), 0, stream, p);
}

// ------------------------------------------------------------------ q/k norm + RoPE + append


struct QkParams {
  const uint16_t* qkv;
  int64_t qkv_stride;          // token row stride; heads are consecutive D-element blocks
  const int32_t* positions;
  const float* cos_sin;        // [max_position, D] fp32: cos of the D/2 frequencies, then sin
  int max_position;
  const uint16_t* q_weight;
  const uint16_t* k_weight;
  float eps;
  uint16_t* q_out;
  int64_t q_out_stride;        // token stride of q_out; heads D apart
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t blk_stride, slot_stride, head_stride, num_cache_slots;
  const int32_t* slot_mapping;
  uint16_t* k_out;             // non-null: k goes here ([token][hkv][D]), not into the pages
  int64_t k_out_stride;        // token stride of k_out; heads D apart
  int num_tokens, hq, hkv, block_size;
  int rows;                    // head rows per token: hq + 2 hkv, or hq + hkv without v
};

// A token's hq + 2 hkv head rows ([0, hq) q, [hq, hq+hkv) k, [hq+hkv, hq+2hkv) v) are
// cut into groups of 4*NB; one wave takes one group, its four 16-lane rows taking rows
// r, r+4, ..., r+4(NB-1) of it (r = lane / 16).  Lane j of a row holds elements 8j..8j+7
// of its head, so its cos/sin values and norm weights are the same for every head: they
// are loaded once per wave, and the wave issues the loads of its NB heads per row before
// computing any of them.  The RoPE partner of element i (< 64) is i + 64, which lives in
// lane j ^ 8 (DPP row_ror:8).  NB = 4 (two waves per token for Qwen3's 32 rows) suits
// prefill-sized inputs (16384 tokens: NB = 2, 4, 8 take 50, 46-47, 48 us); decode-sized
// ones take NB = 1 (8 waves per token), so that a few tokens still spread over the GPU
// and each wave normalises one head per row instead of several in sequence (measured for
// one token: 6.3 us with NB = 8).

constexpr int kQkWideTokens = 2048;  // token count from which NB = 4 is used

template <int NB>
__global__ __launch_bounds__(kThreads) void qk_norm_rope_append_kernel(QkParams p) {
  const int lane = threadIdx.x & 63;
  const int r = lane >> 4, j = lane & 15;
  const int heads = p.rows;
  const int groups = (heads + 4 * NB - 1) / (4 * NB);  // waves per token
  const int wave = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int t = wave / groups;
  const int h0 = (wave - t * groups) * 4 * NB;  // first head row of this wave's group
  if (t >= p.num_tokens) return;  // uniform across the wave
  const uint16_t* row = p.qkv + t * p.qkv_stride + 8 * j;

  // Everything that depends only on the token index is loaded first, together: the slot,
  // the position, the norm weights and this wave's head rows.  Only the RoPE row
  // waits for the position.  (Written in the other order, the compiler waited on the slot,
  // then the position, then the RoPE row before issuing the head rows: four serial memory
  // round trips, 6.6 us for a single token.)
  const int slot_raw = p.slot_mapping ? p.slot_mapping[t] : -1;
  const int pos_raw = p.positions[t];
  uint4 raw[NB];
#pragma unroll
  for (int u = 0; u < NB; ++u) {
    const int h = min(h0 + 4 * u + r, heads - 1);  // clamped: rows past the last head idle below
    raw[u] = load16(row + h * kRopeDim);
  }
  float c[8], sn[8], wq[8], wk[8];
  unpack8(load16(p.q_weight + 8 * j), wq);
  unpack8(load16(p.k_weight + 8 * j), wk);

  const bool pos_ok = pos_raw >= 0 && pos_raw < p.max_position;
  const int pos = pos_ok ? pos_raw : 0;
  const int fi = 8 * (j & 7);  // frequency index of this lane's first element
  const float* cs = p.cos_sin + static_cast<int64_t>(pos) * kRopeDim;
  *reinterpret_cast<float4*>(c) = *reinterpret_cast<const float4*>(cs + fi);
  *reinterpret_cast<float4*>(c + 4) = *reinterpret_cast<const float4*>(cs + fi + 4);
  *reinterpret_cast<float4*>(sn) = *reinterpret_cast<const float4*>(cs + kRopeDim / 2 + fi);
  *reinterpret_cast<float4*>(sn + 4) = *reinterpret_cast<const float4*>(cs + kRopeDim / 2 + fi + 4);
  const bool store_kv = slot_raw >= 0 && slot_raw < p.num_cache_slots;
  int64_t cache_off = 0;
  if (store_kv) {
    const int blk = slot_raw / p.block_size, off = slot_raw - blk * p.block_size;
    cache_off = blk * p.blk_stride + off * p.slot_stride + 8 * j;
  }
  const bool first_half = j < 8;

#pragma unroll
  for (int u = 0; u < NB; ++u) {
    const int h = h0 + 4 * u + r;  // uniform across the 16-lane row
    if (h >= heads) continue;
    if (h >= p.hq + p.hkv) {  // v head: bit copy into the cache
      if (store_kv) store16(p.v_cache + cache_off + (h - p.hq - p.hkv) * p.head_stride, raw[u]);
      continue;
    }
    const bool is_q = h < p.hq;
    if (!is_q && !store_kv && !p.k_out) continue;  // k head of a padding token
    float x[8];
    unpack8(raw[u], x);
    norm_rope_head(x, is_q ? wq : wk, c, sn, first_half, pos_ok, p.eps);
    const uint4 packed = pack8(x);
    if (is_q) store16(p.q_out + t * p.q_out_stride + h * kRopeDim + 8 * j, packed);
    else if (p.k_out) store16(p.k_out + t * p.k_out_stride + (h - p.hq) * kRopeDim + 8 * j, packed);
    else store16(p.k_cache + cache_off + (h - p.hq) * p.head_stride, packed);
  }
}

// ------------------------------------------------------------------ SiLU * up

struct SiluParams {
  const uint16_t* gate_up;     // row t: [gate (inter) | up (inter)]
  int64_t gu_stride;
  uint16_t* out;
  int64_t out_stride;
  int num_tokens, inter;
};

__global__ __launch_bounds__(kThreads) void silu_mul_kernel(SiluParams p) {
  const int per_row = p.inter >> 3;
  const int64_t total = static_cast<int64_t>(p.num_tokens) * per_row;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int t = static_cast<int>(i / per_row);
    const int c = static_cast<int>(i - static_cast<int64_t>(t) * per_row);
    const uint16_t* row = p.gate_up + t * p.gu_stride + 8 * c;
    float g[8], u[8], o[8];
    unpack8(load16(row), g);
    unpack8(load16(row + p.inter), u);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = g[e] / (1.0f + __expf(-g[e])) * u[e];
    store16(p.out + t * p.out_stride + 8 * c, pack8(o));
  }
}

// ------------------------------------------------------------------ argmax

// Whole rows: one 1024-thread workgroup per row.  16-byte loads per thread per round:
// over 256 rows of 151936 (six rotating inputs, so HBM-resident) 3 per round 15.5 us,
// 4 15.9 us, 8 16.9 us; deeper rounds leave more of the last round's loads clamped onto
// the row's final chunk.  A plain streaming read of the same 78 MB (same grid shapes)
// takes 12.4 us: keeping the winning chunk's bits costs about 1 us and the reduction
// epilogue with the end-of-kernel write-back about 1.8 us.
constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxBatch = 3;
// Split rows: below kArgmaxSplitRows rows, each row is cut into S segments of one
// 256-thread workgroup each (S up to 16, so that rows * S reaches about 1024 workgroups);
// for a 151936-wide row at 8 or more segments every thread loads all of its chunks in
// one round.  Each workgroup writes its best as an ordered 64-bit key and
// argmax_merge_kernel takes the largest key of each row.  Measured over rotating inputs of width 151936: 1 row 9.6 -> 5.3 us,
// 16 rows 10.5 -> 6.1 us, 64 rows 11.6 -> 8.3 us, 128 rows 12.2 -> 10.9 us; at 256 rows
// the split (2 segments) is 2% slower than whole rows.
constexpr int kArgmaxSplitThreads = 256;
constexpr int kArgmaxSplitRows = 192;
constexpr int kArgmaxMaxSegments = 16;

struct ArgmaxParams {
  const uint16_t* logits;
  int64_t row_stride;
  int vocab;
  int segments;                 // workgroups per row (1: whole rows)
  int64_t* out;                 // whole rows: the index
  unsigned long long* keys;     // split rows: [row][segment] keys
  const float* temperatures;    // sampling kernels: per row, <= 0 (or NaN) for greedy
  const int32_t* seed;          // sampling kernels: the noise stream's seed (device)
};

// (v, i) beats (b, j): NaN above every number (as torch.argmax), then larger value, then
// the smaller index on ties (first occurrence).
__device__ __forceinline__ bool beats(float v, int i, float b, int j) {
  const bool vn = v != v, bn = b != b;
  if (vn || bn) return vn && (!bn || i < j);
  return v > b || (v == b && i < j);
}

__device__ __forceinline__ float max_nan(float a, float b) {
  return __builtin_elementwise_maximum(a, b);  // NaN-propagating (v_maximum3_f32)
}

// Orders (v, i) as `beats` does, as one unsigned 64-bit integer: the value's bits made
// monotonic (NaN on top, -0 folded onto +0) above the complemented index.  0 is below
// every real key and marks an empty segment.
__device__ __forceinline__ unsigned long long argmax_key(float v, int i) {
  u32 ord;
  if (v != v) {
    ord = 0xffffffffu;
  } else {
    u32 b = __float_as_uint(v);
    if (b == 0x80000000u) b = 0;
    ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  }
  return (static_cast<unsigned long long>(ord) << 32) | (0xffffffffu - static_cast<u32>(i));
}

// ---- Gumbel-max sampling noise
//
// Row r draws token argmax_i(logit_i / T_r + g_ri), g = -log(-log(u)), u uniform in
// [0, 1): a sample of softmax(logits / T_r) (the Gumbel-max trick).  u is the reference
// sampler's stream (kavor/layers/sampler.py:34-38: tl.rand(seed, i + r * V)): the first
// output word of Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers:
// as easy as 1, 2, 3", SC 2011) for counter (i + r * V mod 2^32, 0, 0, 0) and key (the
// low and high words of the sign-extended seed), turned into a float as
// triton.language.random.uint_to_uniform_float does: the word as int32 x, x < 0 folded to
// -x - 1, times 4.6566127342e-10.
constexpr u32 kPhiloxMulA = 0xD2511F53u;
constexpr u32 kPhiloxMulB = 0xCD9E8D57u;
constexpr u32 kPhiloxWeylA = 0x9E3779B9u;
constexpr u32 kPhiloxWeylB = 0xBB67AE85u;

// a ^ b ^ k in one instruction: gfx950's three-input bit operation with the XOR truth table
// (0x96); the compiler emits two v_xor_b32 here.
__device__ __forceinline__ u32 xor3(u32 a, u32 b, u32 k) {
  u32 r;
  asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0x96" : "=v"(r) : "v"(a), "v"(b), "s"(k));
  return r;
}

__device__ __forceinline__ u32 philox_word0(u32 ctr, u32 k0, u32 k1) {
  u32 c0 = ctr, c1 = 0, c2 = 0, c3 = 0;
#pragma unroll
  for (int round = 0; round < 10; ++round) {
    const unsigned long long pa = static_cast<unsigned long long>(kPhiloxMulA) * c0;
    const unsigned long long pb = static_cast<unsigned long long>(kPhiloxMulB) * c2;
    c0 = xor3(static_cast<u32>(pb >> 32), c1, k0);
    c2 = xor3(static_cast<u32>(pa >> 32), c3, k1);
    c1 = static_cast<u32>(pb);
    c3 = static_cast<u32>(pa);
    k0 += kPhiloxWeylA;
    k1 += kPhiloxWeylB;
  }
  return c0;
}

__device__ __forceinline__ float uniform_from_word(u32 w) {
  const int x = static_cast<int>(w);
  return static_cast<float>(x < 0 ? ~x : x) * 4.6566127342e-10f;
}

// The perturbed score of value f at counter ctr (the division and the logarithms are the
// IEEE ones, as in the reference's kernel).
__device__ __forceinline__ float gumbel_score(float f, float temp, u32 ctr, u32 k0, u32 k1) {
  const float u = uniform_from_word(philox_word0(ctr, k0, k1));
  return f / temp + (-logf(-logf(u)));
}

template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_key(unsigned long long k) {
  const u32 lo = static_cast<u32>(__builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<u32>(k)), CTRL, 0xf, 0xf, false));
  const u32 hi = static_cast<u32>(__builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<u32>(k >> 32)), CTRL, 0xf, 0xf, false));
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}
__device__ __forceinline__ unsigned long long max_key(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}
// Largest key over the caller's 16-lane DPP row (every lane of the row gets it).
__device__ __forceinline__ unsigned long long row16_max_key(unsigned long long k) {
  k = max_key(k, dpp_key<kDppQuadXor1>(k));
  k = max_key(k, dpp_key<kDppQuadXor2>(k));
  k = max_key(k, dpp_key<kDppRowHalfMirror>(k));
  k = max_key(k, dpp_key<kDppRowMirror>(k));
  return k;
}
// Largest key over the wave (wave-uniform result): the four rows' maxima read by lane.
__device__ __forceinline__ unsigned long long wave_max_key(unsigned long long k) {
  k = row16_max_key(k);
  unsigned long long m = 0;
#pragma unroll
  for (int row = 0; row < 4; ++row) {
    const u32 lo = static_cast<u32>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<u32>(k)), 16 * row));
    const u32 hi = static_cast<u32>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<u32>(k >> 32)), 16 * row));
    m = max_key(m, (static_cast<unsigned long long>(hi) << 32) | lo);
  }
  return m;
}

// Per chunk of 8 values a lane keeps, without branches, the NaN-propagating maximum over
// its chunks, the chunk that first reached it and that chunk's raw bits; the index inside
// the kept chunk is found once at the end.  A lane's chunks come in increasing index
// order and only a strictly greater maximum (or a first NaN) replaces the kept chunk, so
// ties keep the first occurrence.  Chunks [cbeg, cend) of the row.  The result is this
// lane's (value, index), index 0x7fffffff when it saw nothing.
template <int THREADS, int BATCH>
__device__ __forceinline__ void greedy_scan(const uint16_t* row, int cbeg, int cend, float& best, int& bi) {
  float cmax = -__builtin_inff();
  int bc = -1;
  uint4 bw = make_uint4(0, 0, 0, 0);
  // BATCH 16-byte loads per thread in flight before any is scanned; indices past the
  // segment are clamped onto its last chunk and skipped.
  for (int c0 = cbeg + threadIdx.x; c0 < cend; c0 += THREADS * BATCH) {
    uint4 w[BATCH];
#pragma unroll
    for (int u = 0; u < BATCH; ++u) w[u] = load16_nt(row + 8 * min(c0 + u * THREADS, cend - 1));
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      const int c = c0 + u * THREADS;
      float f[8];
      unpack8(w[u], f);
      const float m = max_nan(max_nan(max_nan(f[0], f[1]), max_nan(f[2], f[3])),
                              max_nan(max_nan(f[4], f[5]), max_nan(f[6], f[7])));
      const bool up = c < cend && (bc < 0 || (m != m ? cmax == cmax : m > cmax));
      cmax = up ? m : cmax;
      bc = up ? c : bc;
      bw.x = up ? w[u].x : bw.x;
      bw.y = up ? w[u].y : bw.y;
      bw.z = up ? w[u].z : bw.z;
      bw.w = up ? w[u].w : bw.w;
    }
  }
  // The first value of the kept chunk equal to its maximum (for NaN: the first NaN);
  // -0 and +0 compare equal, as in torch.argmax.
  best = -__builtin_inff();
  bi = 0x7fffffff;
  if (bc >= 0) {
    float f[8];
    unpack8(bw, f);
    int e0 = 7;
#pragma unroll
    for (int e = 7; e >= 0; --e)
      if (f[e] == cmax || (cmax != cmax && f[e] != f[e])) e0 = e;
    best = cmax;
    bi = 8 * bc + e0;
  }
}

// The sampling counterpart: every value's Gumbel score, kept per lane with the same
// order (NaN on top, then the larger score, then the smaller index).
template <int THREADS, int BATCH>
__device__ __forceinline__ void sample_scan(const uint16_t* row, int cbeg, int cend, float temp, u32 ctr0,
                                            u32 k0, u32 k1, float& best, int& bi) {
  best = -__builtin_inff();
  bi = -1;
  for (int c0 = cbeg + threadIdx.x; c0 < cend; c0 += THREADS * BATCH) {
    uint4 w[BATCH];
#pragma unroll
    for (int u = 0; u < BATCH; ++u) w[u] = load16_nt(row + 8 * min(c0 + u * THREADS, cend - 1));
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      const int c = c0 + u * THREADS;
      if (c >= cend) continue;
      float f[8];
      unpack8(w[u], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = gumbel_score(f[e], temp, ctr0 + static_cast<u32>(8 * c + e), k0, k1);
        const bool up = bi < 0 || (v != v ? best == best : v > best);
        best = up ? v : best;
        bi = up ? 8 * c + e : bi;
      }
    }
  }
  if (bi < 0) bi = 0x7fffffff;
}

// Greedy argmax (SAMPLE false), or per-row Gumbel-max sampling (SAMPLE true: rows whose
// temperature is not above 0 take the greedy scan).  Whole rows write the index; split
// rows write one ordered key per segment for argmax_merge_kernel.  The row segment is
// chunks [cbeg, cend); the (vocab % 8)-value tail goes to the last segment.
template <int THREADS, int BATCH, bool SPLIT, bool SAMPLE>
__global__ __launch_bounds__(THREADS) void argmax_kernel(ArgmaxParams p) {
  const int r = SPLIT ? static_cast<int>(blockIdx.x) / p.segments : static_cast<int>(blockIdx.x);
  const int seg = SPLIT ? static_cast<int>(blockIdx.x) - r * p.segments : 0;
  const uint16_t* row = p.logits + r * p.row_stride;
  const int nvec = p.vocab >> 3;
  const int per = SPLIT ? (nvec + p.segments - 1) / p.segments : nvec;
  const int cbeg = seg * per, cend = min(nvec, cbeg + per);
  const float temp = SAMPLE ? p.temperatures[r] : 0.f;
  const bool sampled = SAMPLE && temp > 0.f;
  u32 k0 = 0, k1 = 0, ctr0 = 0;
  float best;
  int bi;
  if (sampled) {
    const int seed = *p.seed;
    k0 = static_cast<u32>(seed);
    k1 = seed < 0 ? 0xffffffffu : 0u;
    ctr0 = static_cast<u32>(r) * static_cast<u32>(p.vocab);
    sample_scan<THREADS, BATCH>(row, cbeg, cend, temp, ctr0, k0, k1, best, bi);
  } else {
    greedy_scan<THREADS, BATCH>(row, cbeg, cend, best, bi);
  }
  const int tail = p.vocab - 8 * nvec;
  if ((!SPLIT || seg == p.segments - 1) && static_cast<int>(threadIdx.x) < tail) {
    const int i = 8 * nvec + threadIdx.x;
    float f = __uint_as_float(static_cast<u32>(row[i]) << 16);
    if (sampled) f = gumbel_score(f, temp, ctr0 + static_cast<u32>(i), k0, k1);
    if (beats(f, i, best, bi)) { best = f; bi = i; }
  }
  // The lanes' bests as ordered keys (0: saw nothing): a plain maximum over them is the
  // order of `beats`.  Within a wave by DPP and lane reads, across the waves through
  // one LDS slot each, reduced by wave 0 (no LDS-routed shuffles, no serial loop).
  const unsigned long long key = wave_max_key(bi == 0x7fffffff ? 0ull : argmax_key(best, bi));
  __shared__ unsigned long long s_key[THREADS / 64];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) s_key[wave] = key;
  __syncthreads();
  if (wave == 0) {
    static_assert(THREADS / 64 <= 16, "one DPP row holds the waves' keys");
    const int lane = threadIdx.x;
    const unsigned long long k = row16_max_key(lane < THREADS / 64 ? s_key[lane] : 0ull);
    if (lane == 0) {
      if (SPLIT) p.keys[blockIdx.x] = k;
      else p.out[blockIdx.x] = 0xffffffffu - static_cast<u32>(k & 0xffffffffu);
    }
  }
}

// One thread per row: the largest of the row's segment keys, back to its index.
__global__ __launch_bounds__(256) void argmax_merge_kernel(ArgmaxParams p, int rows) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  const unsigned long long* k = p.keys + static_cast<int64_t>(r) * p.segments;
  unsigned long long m = 0;
  for (int s = 0; s < p.segments; ++s) m = k[s] > m ? k[s] : m;
  p.out[r] = 0xffffffffu - static_cast<u32>(m & 0xffffffffu);
}

}  // namespace
}  // namespace kvp

using namespace kvp;

extern "C" int kvp_rmsnorm_bf16(const void* x, int64_t x_stride0, int64_t x_stride1,
                                void* residual, int64_t residual_stride0, int64_t residual_stride1,
                                const void* weight, float eps,
                                void* out, int64_t out_stride0, int64_t out_stride1,
                                int32_t num_tokens, int32_t rows_per_token, int32_t cols,
                                void* stream) {
  clear_error();
  if (!x || !weight || !out) return fail(KVP_EINVAL, "null pointer");
  if (num_tokens < 0 || rows_per_token < 1 || cols < 8 || cols % 8 != 0)
    return fail(KVP_EINVAL, "bad shape: num_tokens=%d rows_per_token=%d cols=%d (cols must be a "
                "positive multiple of 8)", num_tokens, rows_per_token, cols);
  if (cols > 64 * 8 * 16)
    return fail(KVP_EUNSUPPORTED, "cols=%d exceeds the supported maximum of 8192", cols);
  if (!aligned16(x) || !aligned16(weight) || !aligned16(out) || (residual && !aligned16(residual)))
    return fail(KVP_EINVAL, "pointers must be 16-byte aligned");
  if (!mult8(x_stride0) || !mult8(x_stride1) || !mult8(out_stride0) || !mult8(out_stride1) ||
      (residual && (!mult8(residual_stride0) || !mult8(residual_stride1))))
    return fail(KVP_EINVAL, "strides must be multiples of 8 elements");
  const int64_t rows = static_cast<int64_t>(num_tokens) * rows_per_token;
  if (rows > INT32_MAX / 64) return fail(KVP_EINVAL, "too many rows (%lld)", (long long)rows);
  if (rows == 0) return KVP_OK;
  NormParams p{static_cast<const uint16_t*>(x), x_stride0, x_stride1,
               static_cast<uint16_t*>(residual), residual_stride0, residual_stride1,
               static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out),
               out_stride0, out_stride1, rows_per_token, static_cast<int>(rows), cols, eps};
  auto s = static_cast<hipStream_t>(stream);
  const int nch = cols / 8;
  if (nch <= 16) launch_norm<16, 1>(p, s);
  else if (nch <= 128) launch_norm<64, 2>(p, s);
  else if (nch <= 256) launch_norm<64, 4>(p, s);
  else if (nch <= 512) launch_norm<64, 8>(p, s);
  else launch_norm<64, 16>(p, s);
  return launch_status("rmsnorm_kernel");
}

// Prefill-sized inputs: 4 head rows per 16-lane row (two waves per token for Qwen3);
// decode-sized ones: one head row per 16-lane row, several waves per token.
static int launch_qk(const QkParams& p, hipStream_t s) {
  const bool wide = p.num_tokens >= kQkWideTokens;
  const int nb = wide ? 4 : 1;
  const int64_t groups = (p.rows + 4 * nb - 1) / (4 * nb);
  const int64_t waves = static_cast<int64_t>(p.num_tokens) * groups;
  const int64_t grid = (waves + kThreads / 64 - 1) / (kThreads / 64);
  if (grid > INT32_MAX) return fail(KVP_EINVAL, "too many tokens");
  if (wide)
    hipLaunchKernelGGL(qk_norm_rope_append_kernel<4>, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s, p);
  else
    hipLaunchKernelGGL(qk_norm_rope_append_kernel<1>, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s, p);
  return launch_status("qk_norm_rope_append_kernel");
}

extern "C" int kvp_qk_norm_rope_append_bf16(
    const void* qkv, int64_t qkv_tok_stride, const int32_t* positions, const float* cos_sin,
    int32_t max_position, const void* q_norm_weight, const void* k_norm_weight, float eps,
    void* q_out, int64_t q_out_tok_stride,
    void* k_cache, void* v_cache, int64_t cache_block_stride, int64_t cache_slot_stride,
    int64_t cache_head_stride, int64_t num_cache_slots, const int32_t* slot_mapping,
    int32_t num_tokens, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t block_size, void* stream) {
  clear_error();
  if (head_dim != kRopeDim)
    return fail(KVP_EUNSUPPORTED, "head_dim=%d: the fused q/k norm + RoPE kernel handles 128", head_dim);
  if (!qkv || !positions || !cos_sin || !q_norm_weight || !k_norm_weight || !q_out)
    return fail(KVP_EINVAL, "null pointer");
  if (slot_mapping && (!k_cache || !v_cache)) return fail(KVP_EINVAL, "slot_mapping without caches");
  if (num_tokens < 0 || num_q_heads < 1 || num_kv_heads < 1 || max_position < 1)
    return fail(KVP_EINVAL, "bad shape");
  if (slot_mapping && (block_size < 1 || num_cache_slots < 0))
    return fail(KVP_EINVAL, "bad block_size / num_cache_slots");
  if (!aligned16(qkv) || !aligned16(q_out) || !aligned16(cos_sin) || !aligned16(q_norm_weight) ||
      !aligned16(k_norm_weight) || (slot_mapping && (!aligned16(k_cache) || !aligned16(v_cache))))
    return fail(KVP_EINVAL, "pointers must be 16-byte aligned");
  if (!mult8(qkv_tok_stride) || !mult8(q_out_tok_stride) ||
      (slot_mapping && (!mult8(cache_block_stride) || !mult8(cache_slot_stride) ||
                        !mult8(cache_head_stride))))
    return fail(KVP_EINVAL, "strides must be multiples of 8 elements");
  if (qkv_tok_stride < static_cast<int64_t>(num_q_heads + 2 * num_kv_heads) * head_dim)
    return fail(KVP_EINVAL, "qkv row stride %lld is shorter than (hq + 2 hkv) * head_dim",
                (long long)qkv_tok_stride);
  if (num_tokens == 0) return KVP_OK;
  QkParams p{static_cast<const uint16_t*>(qkv), qkv_tok_stride, positions, cos_sin, max_position,
             static_cast<const uint16_t*>(q_norm_weight), static_cast<const uint16_t*>(k_norm_weight),
             eps, static_cast<uint16_t*>(q_out), q_out_tok_stride,
             static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
             cache_block_stride, cache_slot_stride, cache_head_stride, num_cache_slots,
             slot_mapping, nullptr, 0, num_tokens, num_q_heads, num_kv_heads, block_size,
             num_q_heads + 2 * num_kv_heads};
  return launch_qk(p, static_cast<hipStream_t>(stream));
}

extern "C" int kvp_qk_norm_rope_bf16(const void* qkv, int64_t qkv_tok_stride, const int32_t* positions,
                                     const float* cos_sin, int32_t max_position, const void* q_norm_weight,
                                     const void* k_norm_weight, float eps, void* q_out,
                                     int64_t q_out_tok_stride, void* k_out, int64_t k_out_tok_stride,
                                     int32_t num_tokens, int32_t num_q_heads, int32_t num_kv_heads,
                                     int32_t head_dim, void* stream) {
  clear_error();
  if (head_dim != kRopeDim)
    return fail(KVP_EUNSUPPORTED, "head_dim=%d: the q/k norm + RoPE kernel handles 128", head_dim);
  if (!qkv || !positions || !cos_sin || !q_norm_weight || !k_norm_weight || !q_out || !k_out)
    return fail(KVP_EINVAL, "null pointer");
  if (num_tokens < 0 || num_q_heads < 1 || num_kv_heads < 1 || max_position < 1)
    return fail(KVP_EINVAL, "bad shape");
  if (!aligned16(qkv) || !aligned16(q_out) || !aligned16(k_out) || !aligned16(cos_sin) ||
      !aligned16(q_norm_weight) || !aligned16(k_norm_weight))
    return fail(KVP_EINVAL, "pointers must be 16-byte aligned");
  if (!mult8(qkv_tok_stride) || !mult8(q_out_tok_stride) || !mult8(k_out_tok_stride))
    return fail(KVP_EINVAL, "strides must be multiples of 8 elements");
  if (qkv_tok_stride < static_cast<int64_t>(num_q_heads + num_kv_heads) * head_dim)
    return fail(KVP_EINVAL, "qkv row stride %lld is shorter than (hq + hkv) * head_dim",
                (long long)qkv_tok_stride);
  if (num_tokens == 0) return KVP_OK;
  QkParams p{static_cast<const uint16_t*>(qkv), qkv_tok_stride, positions, cos_sin, max_position,
             static_cast<const uint16_t*>(q_norm_weight), static_cast<const uint16_t*>(k_norm_weight),
             eps, static_cast<uint16_t*>(q_out), q_out_tok_stride, nullptr, nullptr, 0, 0, 0, 0,
             nullptr, static_cast<uint16_t*>(k_out), k_out_tok_stride, num_tokens, num_q_heads, num_kv_heads,
             1, num_q_heads + num_kv_heads};
  return launch_qk(p, static_cast<hipStream_t>(stream));
}

extern "C" int kvp_silu_mul_bf16(const void* gate_up, int64_t gate_up_tok_stride, void* out,
                                 int64_t out_tok_stride, int32_t num_tokens, int32_t intermediate,
                                 void* stream) {
  clear_error();
  if (!gate_up || !out) return fail(KVP_EINVAL, "null pointer");
  if (num_tokens < 0 || intermediate < 8 || intermediate % 8 != 0)
    return fail(KVP_EINVAL, "intermediate=%d must be a positive multiple of 8", intermediate);
  if (!aligned16(gate_up) || !aligned16(out)) return fail(KVP_EINVAL, "pointers must be 16-byte aligned");
  if (!mult8(gate_up_tok_stride) || !mult8(out_tok_stride))
    return fail(KVP_EINVAL, "strides must be multiples of 8 elements");
  if (gate_up_tok_stride < 2 * static_cast<int64_t>(intermediate))
    return fail(KVP_EINVAL, "gate_up row stride shorter than 2 * intermediate");
  const int64_t total = static_cast<int64_t>(num_tokens) * (intermediate / 8);
  if (total == 0) return KVP_OK;
  const int64_t grid = std::min<int64_t>((total + kThreads - 1) / kThreads, 256 * 16);
  SiluParams p{static_cast<const uint16_t*>(gate_up), gate_up_tok_stride, static_cast<uint16_t*>(out),
               out_tok_stride, num_tokens, intermediate};
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), p);
  return launch_status("silu_mul_kernel");
}

// Segments per row for split rows (1: whole rows).
static int argmax_segments(int32_t num_rows) {
  if (num_rows >= kArgmaxSplitRows) return 1;
  return std::min(kArgmaxMaxSegments, std::max(2, 1024 / std::max(num_rows, 1)));
}

extern "C" size_t kvp_argmax_workspace_bytes(int32_t num_rows) {
  if (num_rows <= 0) return 0;
  const int s = argmax_segments(num_rows);
  return s == 1 ? 0 : static_cast<size_t>(num_rows) * s * sizeof(unsigned long long);
}

// Checks shared by the argmax and sampling entry points.
static int check_logits(const void* logits, int64_t row_stride, int32_t num_rows, int32_t vocab, const void* out,
                        const void* workspace) {
  if (!logits || !out) return fail(KVP_EINVAL, "null pointer");
  if (num_rows < 0 || vocab < 1) return fail(KVP_EINVAL, "bad shape");
  if (!aligned16(logits) || !mult8(row_stride) || row_stride < vocab)
    return fail(KVP_EINVAL, "logits must be 16-byte aligned with a row stride >= vocab that is a "
                "multiple of 8 elements");
  if (workspace && (reinterpret_cast<uintptr_t>(workspace) & 7u))
    return fail(KVP_EINVAL, "workspace must be 8-byte aligned");
  return KVP_OK;
}

template <bool SAMPLE>
static int launch_argmax(ArgmaxParams p, int32_t num_rows, void* workspace, size_t workspace_bytes,
                         hipStream_t s) {
  p.segments = argmax_segments(num_rows);
  p.keys = static_cast<unsigned long long*>(workspace);
  // Split rows need the caller's workspace; without one (or too small) rows stay whole.
  if (p.segments > 1 && workspace && workspace_bytes >= kvp_argmax_workspace_bytes(num_rows)) {
    const int per = (p.vocab / 8 + p.segments - 1) / p.segments;  // chunks per segment
    if (per > 5 * kArgmaxSplitThreads)
      hipLaunchKernelGGL((argmax_kernel<kArgmaxSplitThreads, 10, true, SAMPLE>), dim3(num_rows * p.segments),
                         dim3(kArgmaxSplitThreads), 0, s, p);
    else
      hipLaunchKernelGGL((argmax_kernel<kArgmaxSplitThreads, 5, true, SAMPLE>), dim3(num_rows * p.segments),
                         dim3(kArgmaxSplitThreads), 0, s, p);
    hipLaunchKernelGGL(argmax_merge_kernel, dim3((num_rows + 255) / 256), dim3(256), 0, s, p, num_rows);
    return launch_status(SAMPLE ? "sample kernel (split rows)" : "argmax_kernel (split rows)");
  }
  p.segments = 1;
  hipLaunchKernelGGL((argmax_kernel<kArgmaxThreads, kArgmaxBatch, false, SAMPLE>), dim3(num_rows),
                     dim3(kArgmaxThreads), 0, s, p);
  return launch_status(SAMPLE ? "sample kernel" : "argmax_kernel");
}

extern "C" int kvp_argmax_bf16(const void* logits, int64_t row_stride, int32_t num_rows,
                               int32_t vocab, int64_t* out, void* workspace, size_t workspace_bytes,
                               void* stream) {
  clear_error();
  const int rc = check_logits(logits, row_stride, num_rows, vocab, out, workspace);
  if (rc != KVP_OK || num_rows == 0) return rc;
  ArgmaxParams p{static_cast<const uint16_t*>(logits), row_stride, vocab, 1, out, nullptr, nullptr, nullptr};
  return launch_argmax<false>(p, num_rows, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int kvp_sample_bf16(const void* logits, int64_t row_stride, int32_t num_rows, int32_t vocab,
                               const float* temperatures, const int32_t* seed, int64_t* out,
                               void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  const int rc = check_logits(logits, row_stride, num_rows, vocab, out, workspace);
  if (rc != KVP_OK) return rc;
  if (!temperatures || !seed) return fail(KVP_EINVAL, "null temperatures / seed");
  if ((reinterpret_cast<uintptr_t>(temperatures) & 3u) || (reinterpret_cast<uintptr_t>(seed) & 3u))
    return fail(KVP_EINVAL, "temperatures and seed must be 4-byte aligned");
  if (num_rows == 0) return KVP_OK;
  ArgmaxParams p{static_cast<const uint16_t*>(logits), row_stride, vocab, 1, out, nullptr, temperatures, seed};
  return launch_argmax<true>(p, num_rows, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}
