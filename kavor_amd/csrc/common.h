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

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

typedef u32 u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte load / store with the nontemporal hint, for data touched exactly once (KV rows
// streamed by attention, cache rows written by the append): it is not kept in L2.
__device__ __forceinline__ uint4 load16_nt(const void* ptr) {
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(ptr)));
}
__device__ __forceinline__ void store16_nt(void* ptr, uint4 v) {
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, v), reinterpret_cast<u32x4_t*>(ptr));
}

// Lowest finite value used as the running-max floor of the online softmax, so that
// exp2(m_old - m_new) never evaluates (-inf) - (-inf).
constexpr float kMaxFloor = -1.0e30f;

}  // namespace kvp
