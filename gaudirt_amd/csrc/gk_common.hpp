// Shared host/device helpers of the gfx950 paged-attention library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "gaudirt_amd.h"

namespace gk {

// ---------------------------------------------------------------------------
// Host-side status plumbing: every C entry point returns a code and keeps the
// message of its last failure per thread.
// ---------------------------------------------------------------------------
void set_error(const std::string& message);
void clear_error();

inline int fail(int code, const std::string& message) {
  set_error(message);
  return code;
}

inline int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return GK_OK;
  return fail(GK_ERR_HIP, std::string(what) + ": " + hipGetErrorString(err));
}

inline bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }
inline int log2_int(int64_t v) {
  int n = 0;
  while ((int64_t{1} << n) < v) ++n;
  return n;
}

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 round-to-nearest-even (NaN quieted), as the reference's rounding.
__device__ __forceinline__ uint32_t bf16_bits(float f) {
  const uint32_t b = __float_as_uint(f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return (b >> 16) | 0x40u;
  return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
}

// Two fp32 values -> packed bf16 pair (lo, hi), round-to-nearest-even.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2 v = {lo, hi};
  bf16x2 r = __builtin_convertvector(v, bf16x2);
  return __builtin_bit_cast(uint32_t, r);
}

// a.lo*b.lo + a.hi*b.hi + c on packed bf16 pairs with fp32 accumulation.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                         false);
}

// Cross-lane moves inside a row of 16 lanes (DPP).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}
constexpr int kDppQuadXor1 = 0xb1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4e;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowRor8 = 0x128;

// Sum over groups of N consecutive lanes (N in {4, 8, 16}); every lane of a
// group receives the group total.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  x += dpp<kDppQuadXor1>(x);
  x += dpp<kDppQuadXor2>(x);
  if constexpr (N >= 8) x += dpp<kDppRowHalfMirror>(x);
  if constexpr (N >= 16) x += dpp<kDppRowMirror>(x);
  return x;
}

__device__ __forceinline__ float shfl_xor(float x, int mask) {
  const int lane = __lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(x)));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;

// Launchers shared between translation units (status-returning, host side).
int launch_kv_store(const void* key, const void* value, int64_t key_stride, int64_t value_stride,
                    const int32_t* slot_mapping, int32_t rows, void* pool, int64_t slots, int32_t kv_heads,
                    int32_t head_dim, hipStream_t stream);
int paged_prefill(const gk_prefill_params* params, hipStream_t stream);

}  // namespace gk
