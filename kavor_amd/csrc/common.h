// Shared device helpers and the host-side error channel of libkvpath.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kvpath.h"

namespace kvp {

typedef uint32_t u32;

// ---------------------------------------------------------------- host side

// Records a printf-style message for kvp_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the thread's last error (called on entry of every exported function).
void clear_error();
// Converts a launch status into the exported return convention.
int launch_status(const char* what);

inline bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }
inline bool mult8(int64_t stride) { return (stride & 7) == 0; }

// ---------------------------------------------------------------- device side

// bf16 halves of a packed 32-bit word, widened exactly to fp32.
__device__ __forceinline__ float bf16_lo(u32 w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(u32 w) { return __uint_as_float(w & 0xffff0000u); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16 pair, round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ u32 pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(u32, v);
}

// a.lo*b.lo + a.hi*b.hi + acc on packed bf16 pairs, accumulated in fp32 (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(u32 a, u32 b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc, false);
}

// DPP lane permutes inside a 16-lane row (wave64 = 4 rows).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
constexpr int kDppQuadXor1 = 0xb1;    // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4e;    // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

// Sum over the 16 lanes of the caller's DPP row; every lane of the row gets the total.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f32<kDppQuadXor1>(x);
  x += dpp_f32<kDppQuadXor2>(x);
  x += dpp_f32<kDppRowHalfMirror>(x);
  x += dpp_f32<kDppRowMirror>(x);
  return x;
}

// x(lane) + x(lane ^ 16) and x(lane) + x(lane ^ 32) for every lane, and the maxima, by
// the gfx950 row / half swaps (VALU, no LDS): v_permlane16_swap_b32 (x, x) returns the
// even rows of each row pair in both rows, then the odd rows; v_permlane32_swap_b32 (x, x)
// returns the low half in both halves, then the high half.
__device__ __forceinline__ float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Inclusive prefix sum over the 64 lanes of a wave (all lanes active): DPP right shifts by
// 1, 2, 4 and 8 inside each 16-lane row (lanes shifted in from outside the row read 0),
// then the totals of the rows below, read with readlane.  No LDS round trips.
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(x, 15);
  const int r1 = r0 + __builtin_amdgcn_readlane(x, 31);
  const int r2 = r1 + __builtin_amdgcn_readlane(x, 47);
  const int row = (threadIdx.x & 63) >> 4;
  return x + (row == 0 ? 0 : (row == 1 ? r0 : (row == 2 ? r1 : r2)));
}

typedef u32 u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte load / store with the nontemporal hint, for data touched exactly once (KV rows
// streamed by attention, cache rows written by the append): it is not kept in L2.
__device__ __forceinline__ uint4 load16_nt(const void* ptr) {
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(ptr)));
}
__device__ __forceinline__ void store16_nt(void* ptr, uint4 v) {
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, v), reinterpret_cast<u32x4_t*>(ptr));
}

// Eight bf16 values of a 16-byte chunk, widened exactly to fp32, and back (RNE).
__device__ __forceinline__ void unpack8(const uint4 w, float f[8]) {
  f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x);
  f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
  f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z);
  f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
}

__device__ __forceinline__ uint4 pack8(const float f[8]) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]),
                    pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7]));
}

// x rounded to bf16 and back to fp32, as the eager path's intermediate bf16 tensors are
// (round-to-nearest-even, the v_cvt_pk_bf16_f32 conversion).  A software rounding took
// about 7 VALU operations per value, and RMSNorm and q/k norm round twice per element:
// the fused q/k norm + RoPE + append at 16,384 tokens ran 51.4 -> 47.3 us with the
// conversion, bit-identical.
__device__ __forceinline__ float round_bf16(float x) {
  return __uint_as_float(static_cast<u32>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(x))) << 16);
}

constexpr int kRopeDim = 128;  // head_dim of the q/k norm + RoPE code: 16 lanes x 8 elements

// One head row held by a 16-lane DPP row, lane j owning elements 8j..8j+7: RMSNorm with
// fp32 statistics, the bf16 rounding of the normalised value, the weight, a second bf16
// rounding (the reference's two eager steps, kavor/layers/layernorm.py:235-258), then neox
// RoPE in fp32 (rotary_embedding.py:8-53): element i < 64 pairs with i + 64, which lives
// in lane j ^ 8 (DPP row_ror:8).  c / sn are this lane's cos / sin of frequencies
// 8 (j & 7) .. +7; a position outside the table (pos_ok false) gives NaN.

__device__ __forceinline__ void norm_rope_head(float (&x)[8], const float (&w)[8], const float (&c)[8],
                                               const float (&sn)[8], bool first_half, bool pos_ok,
                                               float eps) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
  ss = row16_sum(ss);
  const float rstd = rsqrtf(ss * (1.0f / kRopeDim) + eps);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = round_bf16(round_bf16(x[e] * rstd) * w[e]);
  const uint4 mine = pack8(x);
  uint4 other;
  other.x = static_cast<u32>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mine.x), 0x128, 0xf, 0xf, false));
  other.y = static_cast<u32>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mine.y), 0x128, 0xf, 0xf, false));
  other.z = static_cast<u32>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mine.z), 0x128, 0xf, 0xf, false));
  other.w = static_cast<u32>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mine.w), 0x128, 0xf, 0xf, false));
  float y[8];
  unpack8(other, y);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    // first half: x1*cos - x2*sin; second half: x2*cos + x1*sin
    const float o = first_half ? x[e] * c[e] - y[e] * sn[e] : x[e] * c[e] + y[e] * sn[e];
    x[e] = pos_ok ? o : __builtin_nanf("");
  }
}

// Lowest finite value used as the running-max floor of the online softmax, so that
// exp2(m_old - m_new) never evaluates (-inf) - (-inf).
constexpr float kMaxFloor = -1.0e30f;

// ---- direct-to-LDS buffer loads
//
// buffer_load_dwordx4 ... lds: lane l of the wave writes the 16 bytes it loads at the LDS
// address in M0 + 16 l; the load is counted by vmcnt like any vector load, and vector
// memory operations complete in issue order.  The global_load_lds form is not used: the
// compiler treats it as a flat access to both memories and, while one is in flight,
// waits for every outstanding load at the next use of any loaded register.  Buffer loads
// are range-checked against the resource's size (out-of-range lanes read zeros).  The
// compiler does not order later LDS reads of the destination after these loads, so the
// kernels wait explicitly (wait_vmem) before reading what they filled.
typedef int32_t BufferRsrc __attribute__((ext_vector_type(4)));
__device__ void raw_buffer_load_lds(BufferRsrc rsrc, __attribute__((address_space(3))) void* lds, int size,
                                    int voffset, int soffset, int offset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.lds");

// Buffer resource over `bytes` bytes at `base` (stride 0, raw byte offsets).
__device__ __forceinline__ BufferRsrc buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  BufferRsrc r;
  r.x = static_cast<int32_t>(static_cast<uint32_t>(a));
  r.y = static_cast<int32_t>((a >> 32) & 0xffffu);
  r.z = static_cast<int32_t>(bytes);
  r.w = 0x00020000;  // gfx9 word 3: 32-bit data format, no swizzle
  return r;
}

// 16 bytes at byte offset voffset of the resource into LDS at lds + 16 * lane.
__device__ __forceinline__ void lds_dma16(BufferRsrc rsrc, int voffset, void* lds) {
  raw_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds, 16, voffset, 0, 0, 0);
}

// Waits until at most N vector memory operations of the wave are in flight.
template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

}  // namespace kvp
