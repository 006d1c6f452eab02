// Head-major KV store, tile gather indices and decode-length advance (gfx950).
//
// The store scatters each new row's per-head K and V slices into the combined
// head-major pool. It is pure data movement: every lane moves one 16-byte
// piece, so a wave writes 1 KiB of contiguous head rows and the kernel runs at
// the HBM copy rate. Semantics follow gk_kv_store_head_major_bf16_v1 as the
// reference exercises it (tests/multitile_paged_attention_unit_test.cpp:455-478,
// tests/fixed_kv_descriptor_device_test.cpp:146-197).
#include "gk_common.hpp"

#include <algorithm>

namespace gk {
namespace {

// One thread per 16-byte piece of a row: workgroup (x, y) takes pieces
// 256 x .. 256 x + 255 of rows y, y + gridDim.y, ...; piece p of a row is
// chunk p % chunks of head (p / chunks) % kv_heads of K (p / chunks <
// kv_heads) or V. The row's slot is a scalar load issued with the piece's
// load: one memory round trip before the store, no 64-bit index division.
__global__ __launch_bounds__(256) void kv_store_kernel(const uint16_t* __restrict__ key,
                                                       const uint16_t* __restrict__ value,
                                                       int64_t key_stride, int64_t value_stride,
                                                       const int32_t* __restrict__ slot_mapping,
                                                       int32_t rows, uint16_t* __restrict__ pool,
                                                       int64_t slots, int32_t kv_heads, int32_t chunk_shift) {
  const int32_t p = (int32_t)blockIdx.x * 256 + (int32_t)threadIdx.x;
  if (p >= (2 * kv_heads) << chunk_shift) return;
  const int32_t chunk = p & ((1 << chunk_shift) - 1), kh = p >> chunk_shift;
  const int32_t kind = kh >= kv_heads ? 1 : 0, head = kh - kind * kv_heads;
  const int32_t head_dim = 8 << chunk_shift;
  for (int32_t row = (int32_t)blockIdx.y; row < rows; row += (int32_t)gridDim.y) {
    const int32_t slot = slot_mapping[row];
    const uint16_t* src = (kind ? value + row * value_stride : key + row * key_stride) +
                          (int64_t)head * head_dim + chunk * 8;
    const uint4 v = *reinterpret_cast<const uint4*>(src);
    if (slot < 0 || slot >= slots) continue;  // negative: no store; past the pool: never written
    uint16_t* dst = pool + (((int64_t)kind * kv_heads + head) * slots + slot) * head_dim + chunk * 8;
    // Non-temporal (streaming) store: the rows are read next by the decode's
    // own non-temporal loads, not from this XCD's L2 (C3, same box: 188.9-189.1
    // -> 188.3-188.4 us per step).
    typedef unsigned u32x4n __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4n, v), reinterpret_cast<u32x4n*>(dst));
  }
}

__global__ __launch_bounds__(256) void tile_indices_kernel(const int32_t* __restrict__ mapping,
                                                           const int32_t* __restrict__ requests,
                                                           const int32_t* __restrict__ work, int32_t tasks,
                                                           int32_t context, int32_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)tasks * 64) return;
  const int32_t t = (int32_t)(i >> 6), l = (int32_t)(i & 63);
  const int32_t first_row = work[t * 4 + 0], first_key = work[t * 4 + 1];
  const int32_t lanes = work[t * 4 + 2], base = work[t * 4 + 3];
  int32_t value = 0;
  if (lanes > 0) {
    value = base;
    if (l < lanes) value += mapping[(int64_t)requests[first_row] * context + first_key + l];
  }
  out[i] = value;
}

__global__ __launch_bounds__(256) void advance_lengths_kernel(const int64_t* __restrict__ seq,
                                                              const int32_t* __restrict__ orig, int64_t count,
                                                              int64_t* __restrict__ next,
                                                              int32_t* __restrict__ orig_next) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  next[i] = seq[i] + 1;
  orig_next[i] = orig[i] + 1;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

int launch_kv_store(const void* key, const void* value, int64_t key_stride, int64_t value_stride,
                    const int32_t* slot_mapping, int32_t rows, void* pool, int64_t slots, int32_t kv_heads,
                    int32_t head_dim, hipStream_t stream) {
  if (rows < 0 || slots <= 0 || kv_heads <= 0 || (head_dim != 64 && head_dim != 128 && head_dim != 256))
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_kv_store: invalid geometry");
  if (rows == 0) return GK_OK;
  if (!key || !value || !slot_mapping || !pool)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_kv_store: null pointer");
  if (!aligned16(key) || !aligned16(value) || !aligned16(pool) || (key_stride & 7) || (value_stride & 7) ||
      key_stride < (int64_t)kv_heads * head_dim || value_stride < (int64_t)kv_heads * head_dim)
    return fail(GK_ERR_INVALID_ARGUMENT, "gk_kv_store: K/V rows must be 16-byte aligned and hold kv_heads * head_dim");
  if (kv_heads > (1 << 20)) return fail(GK_ERR_INVALID_ARGUMENT, "gk_kv_store: invalid geometry");
  const int chunk_shift = head_dim == 64 ? 3 : head_dim == 128 ? 4 : 5;
  const dim3 grid((unsigned)(((2 * kv_heads << chunk_shift) + 255) / 256), (unsigned)std::min(rows, 65535));
  kv_store_kernel<<<grid, 256, 0, stream>>>(static_cast<const uint16_t*>(key), static_cast<const uint16_t*>(value),
                                            key_stride, value_stride, slot_mapping, rows,
                                            static_cast<uint16_t*>(pool), slots, kv_heads, chunk_shift);
  return hip_status(hipGetLastError(), "gk_kv_store launch");
}

}  // namespace gk

extern "C" int gk_kv_store(const void* key, const void* value, int64_t key_row_stride, int64_t value_row_stride,
                           const int32_t* slot_mapping, int32_t rows, void* pool, int64_t slots,
                           int32_t kv_heads, int32_t head_dim, hipStream_t stream) {
  gk::clear_error();
  return gk::launch_kv_store(key, value, key_row_stride, value_row_stride, slot_mapping, rows, pool, slots,
                             kv_heads, head_dim, stream);
}

extern "C" int gk_attn_tile_indices(const int32_t* mapping, const int32_t* requests, const int32_t* work,
                                    int32_t tasks, int32_t context, int32_t* out, hipStream_t stream) {
  gk::clear_error();
  if (tasks < 0 || context <= 0) return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_attn_tile_indices: invalid sizes");
  if (tasks == 0) return GK_OK;
  if (!mapping || !requests || !work || !out)
    return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_attn_tile_indices: null pointer");
  const int64_t total = (int64_t)tasks * 64;
  gk::tile_indices_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(mapping, requests, work, tasks,
                                                                               context, out);
  return gk::hip_status(hipGetLastError(), "gk_attn_tile_indices launch");
}

extern "C" int gk_advance_decode_lengths(const int64_t* seq_lens, const int32_t* orig_seq_lens, int64_t count,
                                         int64_t* next, int32_t* orig_next, hipStream_t stream) {
  gk::clear_error();
  if (count < 0 || count > (int64_t{1} << 30))
    return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_advance_decode_lengths: count exceeds supported range");
  if (count == 0) return GK_OK;
  if (!seq_lens || !orig_seq_lens || !next || !orig_next)
    return gk::fail(GK_ERR_INVALID_ARGUMENT, "gk_advance_decode_lengths: null pointer");
  gk::advance_lengths_kernel<<<(unsigned)((count + 255) / 256), 256, 0, stream>>>(seq_lens, orig_seq_lens, count,
                                                                                  next, orig_next);
  return gk::hip_status(hipGetLastError(), "gk_advance_decode_lengths launch");
}
