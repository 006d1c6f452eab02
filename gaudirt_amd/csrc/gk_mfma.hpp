// Device building blocks shared by the gfx950 attention kernels: bf16 MFMA
// tiles, buffer resources, the LDS token swizzle and the transposed LDS read.
#pragma once

#include "gk_common.hpp"

namespace gk {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;
typedef __attribute__((address_space(3))) void lds_void_t;

// Word 3 of a raw buffer resource on gfx950 (32-bit data format, offset mode).
constexpr int kBufferDword3 = 0x00020000;

__device__ __forceinline__ uint4 load16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }

// 16 bytes of a K/V row that is read once: a non-temporal load.
__device__ __forceinline__ uint4 load16_once(const uint16_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// tanh via exp2: tanh(x) = 1 - 2 / (2^(2x log2 e) + 1); saturates cleanly at +-1.
__device__ __forceinline__ float soft_tanh(float x) {
  const float e = fast_exp2(2.f * kLog2e * x);
  return 1.f - 2.f / (e + 1.f);
}

// Pool slot of key t from block ids staged in LDS: s_bt[i] is the block id of
// block b0 + i (block size 2^shift).
__device__ __forceinline__ int slot_of(const int32_t* s_bt, int b0, int shift, int t) {
  return (s_bt[(t >> shift) - b0] << shift) | (t & ((1 << shift) - 1));
}

// Token swizzle of 16-byte chunks inside an LDS row of a K or V tile: chunk c
// of token t is stored at c ^ swz(t, CPR) (CPR = 16-byte chunks per row).
// Bank behaviour measured on gfx950 with SQ_LDS_BANK_CONFLICT, rows of 256
// bytes (d 128): ds_read_b128 serves 32 lanes at a time over 128 four-byte
// banks (two tokens per 512-byte bank row), ds_read_b64_tr_b16 32 lanes at a
// time over 64 banks. The two reads of a tile therefore need:
//  - the 16-key operand reads (lanes q = 0, 1 of a 32-lane half: 16
//    consecutive tokens, logical chunks 4c + q): swz(t) >> 1 distinct among
//    the eight tokens of each parity in an aligned group of 16;
//  - the transposed 4-token reads of P.V (32 lanes, 8 consecutive tokens, an
//    aligned pair of chunks each): swz(t) >> 1 distinct over each aligned
//    group of 8 tokens.
// swz = (t0 << 1) ^ (t1 << 3) ^ (t2 << 2) ^ (t3 << 1) (bits of t) does both:
// both reads conflict-free. The previous form ((t & 7) << 1) | (t >> 3) met
// only the second and spent half the operand reads' LDS cycles in conflicts.
// With d = 64 (8 chunks, 128-byte rows) swz = t & 7 keeps the chunk inside
// the row and is conflict-free for both reads in the same measurement (the
// form ((t & 3) << 1) | ((t >> 2) & 1) used before: 2-way on both).
// (cpr is a compile-time constant at every call site, written D / 8: passing a
// static member such as MfmaShape<D>::CPR from a lambda inside a kernel template
// makes the host pass of hipcc drop the kernel's launch stub.)
__device__ __forceinline__ int swz(int t, int cpr) {
  return cpr >= 16 ? (((t & 1) << 1) ^ ((t & 2) << 2) ^ (t & 4) ^ ((t & 8) >> 2))
                   : (t & 7);
}

// Max / sum over the four lanes c, c + 16, c + 32, c + 48 of a column of the
// 16-lane rows, with gfx950's cross-row swaps instead of LDS permutes.
// permlane32_swap(x, x) leaves, in every lane l, x[l % 32] in the first result
// and x[l % 32 + 32] in the second; permlane16_swap does the same for rows
// (0, 1) and (2, 3). Both orders of each addition give the same float, so every
// lane of the column ends with the same value. The max is a bare v_max_f32:
// fmaxf would first quiet both swapped operands (two more instructions), and
// the inputs are never NaN (masked scores are -inf).
__device__ __forceinline__ float max2(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// Maximum of N >= 2 values as a tree of bare max3 (depth log3 N): a chain
// would be N / 2 dependent instructions, and fmaxf would quiet every input
// first.
template <int N>
__device__ __forceinline__ float tree_max(const float (&v)[N]) {
  static_assert(N >= 2, "at least two values");
  if constexpr (N == 2) {
    return max2(v[0], v[1]);
  } else {
    constexpr int M = (N + 2) / 3;
    float w[M];
#pragma unroll
    for (int i = 0; i < N / 3; ++i) w[i] = max3(v[3 * i], v[3 * i + 1], v[3 * i + 2]);
    if constexpr (N % 3 == 1) w[M - 1] = v[N - 1];
    if constexpr (N % 3 == 2) w[M - 1] = max2(v[N - 2], v[N - 1]);
    if constexpr (M == 1) return w[0];
    else return tree_max<M>(w);
  }
}
__device__ __forceinline__ float col4_max(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = max2(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max2(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
// col4_max of two values at once (a and b in place). permlane32_swap(a, b)
// leaves a's lower half next to b's lower half and a's upper half next to
// b's upper half, so one maximum reduces a over the 32-lane halves in lanes
// 0-31 and b in lanes 32-63; a 16-lane swap finishes both, and a last 32-lane
// swap hands every lane both results: 3 permutes and 2 maxima for the 4 and 4
// of two col4_max calls.
__device__ __forceinline__ void col4_max2(float& a, float& b) {
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  const float c = max2(__uint_as_float(h[0]), __uint_as_float(h[1]));
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(c), __float_as_uint(c), false, false);
  const float d = max2(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto e = __builtin_amdgcn_permlane32_swap(__float_as_uint(d), __float_as_uint(d), false, false);
  a = __uint_as_float(e[0]);
  b = __uint_as_float(e[1]);
}
__device__ __forceinline__ float col4_sum(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// s_waitcnt vmcnt(0) that LLVM's wait-count tracking sees (encoding: vmcnt 0,
// expcnt and lgkmcnt at their maxima). Afterwards it treats every earlier
// vector load as complete, so it inserts no wait of its own before their
// registers are read: its model does not count the asm direct loads, and a
// wait it placed after some of them would also wait for those.
__device__ __forceinline__ void wait_vmem_visible() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// Wait until at most N vector memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// D += A . B on 16x16 tiles, K = 32 (8 bf16 per lane) or K = 16 (4 per lane).
// Lane (q = lane / 16, c = lane % 16): A row c and B column c, k slots of group
// q; D rows 4q .. 4q + 3, column c.
__device__ __forceinline__ f32x4_t mfma32(const bf16x8_t& a, const bf16x8_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16(const bf16x4_t& a, const bf16x4_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4_t, a), __builtin_bit_cast(i16x4_t, b), c,
                                                   0, 0, 0);
}

// Four consecutive LDS rows (16-bit elements), transposed: lane i of each
// 16-lane group receives column i of the 4 x 16 block its group addresses
// (lane j addresses row j / 4, columns 4 (j % 4) .. + 3).
__device__ __forceinline__ bf16x4_t lds_read_tr4(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_t*)p);
}

// One 16-byte direct load per lane, HBM -> LDS: lane l's bytes land at LDS
// address lds + 16 l. Written as an asm statement so that the compiler's
// wait-count model never sees the LDS side: kernels order every read of a
// stage after that stage's loads with explicit vmcnt waits (and barriers),
// while the compiler's own tracking of direct loads either cannot tell two
// stages apart or waits for every direct load in flight before a barrier. M0
// holds the LDS base; no other code in these kernels uses M0 (the s_nop covers
// the M0-write -> direct-load hazard).
__device__ __forceinline__ void lds_dma16(uint32_t lds, __amdgpu_buffer_rsrc_t rsrc, uint32_t voffset) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds),
      "v"(voffset), "s"(rsrc)
      : "memory");
}

// A raw buffer resource (stride 0, `bytes` records) as four words made
// wave-uniform with readfirstlane, for lds_dma16_w: where the compiler cannot
// see that a resource is uniform (e.g. after unrolling a loop whose body takes
// it from a lambda capture) it keeps __amdgpu_buffer_rsrc_t in VGPRs, which
// the direct-load asm cannot take.
__device__ __forceinline__ u32x4_t buffer_words(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  u32x4_t w;
  w[0] = __builtin_amdgcn_readfirstlane((uint32_t)p);
  w[1] = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32) & 0xffffu);
  w[2] = __builtin_amdgcn_readfirstlane(bytes);
  w[3] = (uint32_t)kBufferDword3;
  return w;
}
__device__ __forceinline__ void lds_dma16_w(uint32_t lds, u32x4_t rsrc, uint32_t voffset) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds),
      "v"(voffset), "s"(rsrc)
      : "memory");
}

// The same load for K/V rows that a decode step reads exactly once, with the
// cache policy GK_KV_LOAD_POLICY: sc1 (device scope: the line is not kept in
// the CU's vector L1) and nt (non-temporal: streamed through L2 rather than
// retained). On C2 this took the step from 117.2 to 104.9 us (sc1 alone: no
// change; nt alone: 105.4 us).
#ifndef GK_KV_LOAD_POLICY
#define GK_KV_LOAD_POLICY "sc1 nt"
#endif
// The same policy as the cache-policy operand of the buffer-load builtins
// (gfx950 bits: sc0 = 1, nt = 2, sc1 = 16).
constexpr int kKvLoadPolicyBits = 16 | 2;
__device__ __forceinline__ void lds_dma16_once(uint32_t lds, __amdgpu_buffer_rsrc_t rsrc, uint32_t voffset) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen " GK_KV_LOAD_POLICY " lds" ::"s"(lds),
      "v"(voffset), "s"(rsrc)
      : "memory");
}

// Wave-uniform load through the scalar cache (s_load). The data is only read
// by the kernel; the constant address space tells the compiler so, which it
// cannot prove itself once LDS direct loads (memory writes) are in the loop.
__device__ __forceinline__ int32_t scalar_load(const int32_t* p, int64_t i) {
  return ((const __attribute__((address_space(4))) int32_t*)p)[i];
}

// LDS byte address of a __shared__ object (or a pointer into one).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

}  // namespace gk
