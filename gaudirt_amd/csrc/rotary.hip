// Rotary position embedding of query/key rows, and the fused rotary + KV
// store (gfx950).
//
// Streaming work with no reuse: the kernel is bound by HBM bandwidth. When the
// geometry allows (head_dim a multiple of 8, rotary_dim a multiple of 16 for
// the NeoX layout or of 8 for the interleaved one, 16-byte aligned rows) each
// lane handles whole 16-byte pieces: 8 rotation pairs (NeoX: the piece at i and
// the piece at i + rotary_dim / 2), 4 pairs (interleaved: one piece), or a
// piece copied past rotary_dim. Otherwise one lane handles one pair or one
// element. The arithmetic is the reference's (generic_private_use1.cpp:294-405
// with the gk_rotary_bf16_v1 contract as tests/rotary_runtime_smoke.py:34-48
// states it): a cos - b sin and b cos + a sin in fp32, each rounded once to
// bf16. bf16 x bf16 products are exact in fp32, so the result does not depend
// on whether the compiler fuses a multiply into the add.
//
// The fused form writes the rotated key rows and the value rows straight into
// the head-major pool at the row's slot (gk_kv_store semantics), next to the
// rotated query rows.
#include "gk_common.hpp"

#include <algorithm>

namespace gk {
namespace {

struct RotaryJob {
  const uint16_t* src;
  int64_t src_stride;
  uint16_t* dst;         // row-major output (unused when the job goes to the pool)
  int64_t dst_stride;
  int32_t heads;         // heads per row
  int32_t rotate;        // 0: copy the rows (value rows of the fused store)
  int32_t pool_kind;     // -1: row-major output; 0 / 1: pool K / V region
};

struct RotaryArgs {
  RotaryJob job[3];
  const void* positions;
  int32_t pos64;
  const uint16_t* cos_sin;
  int64_t cache_rows;
  int32_t rows, head_dim, rotary_dim, neox;
  const int32_t* slot_mapping;
  uint16_t* pool;
  int64_t slots;
  int32_t kv_heads;
};

__device__ __forceinline__ float bf(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }
__device__ __forceinline__ uint16_t to_bf(float f) { return (uint16_t)bf16_bits(f); }

// Elements per unit of work: VEC moves 16-byte pieces, else single pairs/elements.
template <bool VEC>
__device__ __forceinline__ int rotate_units(const RotaryArgs& a) {
  if (!VEC) return a.rotary_dim / 2;
  return a.neox ? a.rotary_dim / 16 : a.rotary_dim / 8;
}
template <bool VEC>
__device__ __forceinline__ int copy_units(int elements) {
  return VEC ? elements / 8 : elements;
}

template <bool VEC>
__global__ __launch_bounds__(256) void rotary_kernel(RotaryArgs a) {
  const RotaryJob& job = a.job[blockIdx.y];
  const int d = a.head_dim, rot = a.rotary_dim, half = rot / 2;
  const int ru = job.rotate ? rotate_units<VEC>(a) : 0;
  const int units = ru + copy_units<VEC>(job.rotate ? d - rot : d);
  const int64_t per_row = (int64_t)job.heads * units;
  const int64_t total = (int64_t)a.rows * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int32_t r = (int32_t)(i / per_row);
    const int64_t rest = i - (int64_t)r * per_row;
    const int32_t h = (int32_t)(rest / units);
    const int32_t u = (int32_t)(rest - (int64_t)h * units);
    uint16_t* dst;
    if (job.pool_kind >= 0) {
      const int32_t slot = a.slot_mapping[r];
      if (slot < 0 || slot >= a.slots) continue;
      dst = a.pool + (((int64_t)job.pool_kind * a.kv_heads + h) * a.slots + slot) * d;
    } else {
      dst = job.dst + (int64_t)r * job.dst_stride + (int64_t)h * d;
    }
    const uint16_t* src = job.src + (int64_t)r * job.src_stride + (int64_t)h * d;
    if (u >= ru) {
      // Copy: elements past rotary_dim, or a whole value row.
      const int e = (job.rotate ? rot : 0) + (u - ru) * (VEC ? 8 : 1);
      if constexpr (VEC) *reinterpret_cast<uint4*>(dst + e) = *reinterpret_cast<const uint4*>(src + e);
      else dst[e] = src[e];
      continue;
    }
    int64_t pos = a.pos64 ? static_cast<const int64_t*>(a.positions)[r] : static_cast<const int32_t*>(a.positions)[r];
    pos = pos < 0 ? 0 : (pos >= a.cache_rows ? a.cache_rows - 1 : pos);
    const uint16_t* cs = a.cos_sin + pos * rot;
    if constexpr (VEC) {
      if (a.neox) {
        const int e = u * 8;  // pairs e .. e + 7: elements e + k and half + e + k
        const uint4 xa = *reinterpret_cast<const uint4*>(src + e);
        const uint4 xb = *reinterpret_cast<const uint4*>(src + half + e);
        const uint4 vc = *reinterpret_cast<const uint4*>(cs + e);
        const uint4 vs = *reinterpret_cast<const uint4*>(cs + half + e);
        const uint16_t* pa = reinterpret_cast<const uint16_t*>(&xa);
        const uint16_t* pb = reinterpret_cast<const uint16_t*>(&xb);
        const uint16_t* pc = reinterpret_cast<const uint16_t*>(&vc);
        const uint16_t* ps = reinterpret_cast<const uint16_t*>(&vs);
        uint4 oa, ob;
        uint16_t* qa = reinterpret_cast<uint16_t*>(&oa);
        uint16_t* qb = reinterpret_cast<uint16_t*>(&ob);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float x0 = bf(pa[k]), x1 = bf(pb[k]), c = bf(pc[k]), s = bf(ps[k]);
          qa[k] = to_bf(x0 * c - x1 * s);
          qb[k] = to_bf(x1 * c + x0 * s);
        }
        *reinterpret_cast<uint4*>(dst + e) = oa;
        *reinterpret_cast<uint4*>(dst + half + e) = ob;
      } else {
        const int e = u * 8;  // elements e .. e + 7: pairs (e + 2k, e + 2k + 1), frequencies e / 2 + k
        const uint4 x = *reinterpret_cast<const uint4*>(src + e);
        const uint2 vc = *reinterpret_cast<const uint2*>(cs + e / 2);
        const uint2 vs = *reinterpret_cast<const uint2*>(cs + half + e / 2);
        const uint16_t* px = reinterpret_cast<const uint16_t*>(&x);
        const uint16_t* pc = reinterpret_cast<const uint16_t*>(&vc);
        const uint16_t* ps = reinterpret_cast<const uint16_t*>(&vs);
        uint4 o;
        uint16_t* qo = reinterpret_cast<uint16_t*>(&o);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float x0 = bf(px[2 * k]), x1 = bf(px[2 * k + 1]), c = bf(pc[k]), s = bf(ps[k]);
          qo[2 * k] = to_bf(x0 * c - x1 * s);
          qo[2 * k + 1] = to_bf(x1 * c + x0 * s);
        }
        *reinterpret_cast<uint4*>(dst + e) = o;
      }
    } else {
      const int i0 = a.neox ? u : 2 * u, i1 = a.neox ? u + half : 2 * u + 1;
      const float x0 = bf(src[i0]), x1 = bf(src[i1]), c = bf(cs[u]), s = bf(cs[half + u]);
      dst[i0] = to_bf(x0 * c - x1 * s);
      dst[i1] = to_bf(x1 * c + x0 * s);
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int rotary(const gk_rotary_params* p, bool fused, hipStream_t stream) {
  const char* name = fused ? "gk_rotary_kv_store" : "gk_rotary_embedding";
  auto bad = [&](const char* what) { return fail(GK_ERR_INVALID_ARGUMENT, std::string(name) + ": " + what); };
  if (!p) return bad("null parameters");
  if (p->struct_size != sizeof(gk_rotary_params))
    return bad("struct_size does not match this library's gk_rotary_params");
  if (p->head_dim <= 0 || p->rotary_dim <= 0 || p->rotary_dim > p->head_dim || (p->rotary_dim & 1))
    return bad("invalid head or rotary dimension");
  if (p->rows < 0 || p->q_width <= 0 || p->k_width <= 0 || p->q_width % p->head_dim || p->k_width % p->head_dim ||
      p->q_width / p->head_dim > 65535 || p->k_width / p->head_dim > 65535)
    return bad("invalid query or key geometry");
  if (p->cache_rows <= 0) return bad("empty cos/sin cache");
  if (p->rows == 0) return GK_OK;
  if (!p->query || !p->key || !p->positions || !p->cos_sin || !p->q_out) return bad("null pointer");
  if (p->q_row_stride < p->q_width || p->k_row_stride < p->k_width || p->q_out_row_stride < p->q_width)
    return bad("row strides shorter than the rows");
  RotaryArgs a{};
  a.positions = p->positions;
  a.pos64 = p->positions_int64 ? 1 : 0;
  a.cos_sin = static_cast<const uint16_t*>(p->cos_sin);
  a.cache_rows = p->cache_rows;
  a.rows = p->rows;
  a.head_dim = p->head_dim;
  a.rotary_dim = p->rotary_dim;
  a.neox = p->is_neox ? 1 : 0;
  a.job[0] = RotaryJob{static_cast<const uint16_t*>(p->query), p->q_row_stride, static_cast<uint16_t*>(p->q_out),
                       p->q_out_row_stride, (int32_t)(p->q_width / p->head_dim), 1, -1};
  int njobs = 2;
  bool vec_ok = p->head_dim % 8 == 0 && p->rotary_dim % (p->is_neox ? 16 : 8) == 0 && aligned16(p->cos_sin) &&
                aligned16(p->query) && aligned16(p->key) && aligned16(p->q_out) && p->q_row_stride % 8 == 0 &&
                p->k_row_stride % 8 == 0 && p->q_out_row_stride % 8 == 0;
  if (fused) {
    if (!p->value || !p->slot_mapping || !p->pool) return bad("null pointer");
    if (p->slots <= 0 || p->kv_heads <= 0 || (p->head_dim != 64 && p->head_dim != 128 && p->head_dim != 256) ||
        p->k_width != (int64_t)p->kv_heads * p->head_dim || p->v_row_stride < p->k_width)
      return bad("invalid KV pool geometry");
    if (!aligned16(p->key) || !aligned16(p->value) || !aligned16(p->pool) || (p->k_row_stride & 7) ||
        (p->v_row_stride & 7))
      return bad("K/V rows and the pool must be 16-byte aligned");
    a.slot_mapping = p->slot_mapping;
    a.pool = static_cast<uint16_t*>(p->pool);
    a.slots = p->slots;
    a.kv_heads = p->kv_heads;
    a.job[1] = RotaryJob{static_cast<const uint16_t*>(p->key), p->k_row_stride, nullptr, 0, p->kv_heads, 1, 0};
    a.job[2] = RotaryJob{static_cast<const uint16_t*>(p->value), p->v_row_stride, nullptr, 0, p->kv_heads, 0, 1};
    vec_ok = vec_ok && aligned16(p->value);
    njobs = 3;
  } else {
    if (!p->k_out) return bad("null pointer");
    if (p->k_out_row_stride < p->k_width) return bad("row strides shorter than the rows");
    a.job[1] = RotaryJob{static_cast<const uint16_t*>(p->key), p->k_row_stride, static_cast<uint16_t*>(p->k_out),
                         p->k_out_row_stride, (int32_t)(p->k_width / p->head_dim), 1, -1};
    vec_ok = vec_ok && aligned16(p->k_out) && p->k_out_row_stride % 8 == 0;
  }
  // Enough 256-thread blocks for the largest job, capped (grid-stride loops).
  const int64_t per_head = vec_ok ? p->head_dim / 8 : p->head_dim;
  const int64_t widest = (int64_t)p->rows * std::max(p->q_width, p->k_width) / p->head_dim * per_head;
  const int64_t blocks = std::min<int64_t>((widest + 255) / 256, 8192);
  const dim3 grid((unsigned)std::max<int64_t>(blocks, 1), (unsigned)njobs);
  if (vec_ok) rotary_kernel<true><<<grid, 256, 0, stream>>>(a);
  else rotary_kernel<false><<<grid, 256, 0, stream>>>(a);
  return hip_status(hipGetLastError(), fused ? "gk_rotary_kv_store launch" : "gk_rotary_embedding launch");
}

}  // namespace
}  // namespace gk

extern "C" int gk_rotary_embedding(const gk_rotary_params* params, hipStream_t stream) {
  gk::clear_error();
  return gk::rotary(params, false, stream);
}

extern "C" int gk_rotary_kv_store(const gk_rotary_params* params, hipStream_t stream) {
  gk::clear_error();
  return gk::rotary(params, true, stream);
}
