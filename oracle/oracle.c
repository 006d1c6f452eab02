/*
 * CPU oracle for the paged-attention path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the GaudiRT reference algorithms for the head-major
 * KV store, slot/tile indexing and paged attention. Only tests, the smoke entry
 * point and the benchmark's CPU-baseline leg may load it, and only as the
 * checker; the product path never routes through it.
 *
 * Citations are to files of the reference repository (tracycam/GaudiRT).
 * Built with -ffp-contract=off so every float operation rounds as written.
 *
 * Parity status of each function (how it is pinned) is listed in the header
 * comment of oracle/oracle.py, which the tests read alongside this file.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* fp32 -> bf16 round-to-nearest-even; NaN is quieted by setting bit 6.
 * Follows tests/multitile_paged_attention_unit_test.cpp:44-48. */
uint16_t orc_bf16_from_f32(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof(bits));
  if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x0040u);
  return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

float orc_bf16_to_f32(uint16_t value) {
  uint32_t bits = (uint32_t)value << 16;
  float out;
  memcpy(&out, &bits, sizeof(out));
  return out;
}

void orc_bf16_from_f32_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_from_f32(in[i]);
}

/* binary64 -> bf16 with a single round-to-nearest-even.
 * Follows tests/fp64_reference.py:7-29: normal range keeps 7 fraction bits with
 * the 45-bit tail deciding the rounding; values below the bf16 normal range are
 * scaled by 2^133 and rounded half-to-even into the subnormal payload; values
 * above it become infinity. */
static uint16_t bf16_from_f64(double value) {
  uint64_t bits;
  memcpy(&bits, &value, sizeof(bits));
  const uint16_t sign = (uint16_t)((bits >> 48) & 0x8000u);
  const uint64_t exponent = (bits >> 52) & 0x7ffu;
  const uint64_t fraction = bits & ((UINT64_C(1) << 52) - 1);
  uint16_t out;
  if (exponent >= 897 && exponent <= 1150) {
    uint64_t payload = ((exponent - 896) << 7) | (fraction >> 45);
    const uint64_t tail = fraction & ((UINT64_C(1) << 45) - 1);
    const uint64_t halfway = UINT64_C(1) << 44;
    payload += (tail > halfway) || (tail == halfway && (payload & 1u));
    out = (uint16_t)payload;
  } else if (exponent < 897) {
    out = (uint16_t)nearbyint(ldexp(fabs(value), 133));
  } else {
    out = 0x7f80u;
  }
  return (uint16_t)(out | sign);
}

int orc_bf16_from_f64_array(const double* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    if (!isfinite(in[i])) return -1;
  for (int64_t i = 0; i < n; ++i) out[i] = bf16_from_f64(in[i]);
  return 0;
}

/* Head-major KV store: for r < valid_rows and every kv head h, copy the row's
 * head slice into pool[(h * S + loc[r]) * d] (keys) and
 * pool[((Hkv + h) * S + loc[r]) * d] (values). Rows at or beyond valid_rows and
 * every other slot are left untouched.
 * Follows tests/multitile_paged_attention_unit_test.cpp:455-478 and the
 * valid_rows gating checked by tests/fixed_kv_descriptor_device_test.cpp:146-197. */
void orc_kv_store(const uint16_t* key, const uint16_t* value, int64_t row_stride,
                  const int32_t* locations, int32_t valid_rows, uint16_t* pool,
                  int64_t slots, int32_t kv_heads, int32_t head_dim) {
  for (int32_t r = 0; r < valid_rows; ++r) {
    const int64_t slot = locations[r];
    for (int32_t h = 0; h < kv_heads; ++h) {
      uint16_t* kdst = pool + ((int64_t)h * slots + slot) * head_dim;
      uint16_t* vdst = pool + ((int64_t)(kv_heads + h) * slots + slot) * head_dim;
      memcpy(kdst, key + (int64_t)r * row_stride + (int64_t)h * head_dim, (size_t)head_dim * 2);
      memcpy(vdst, value + (int64_t)r * row_stride + (int64_t)h * head_dim, (size_t)head_dim * 2);
    }
  }
}

/* Tile gather indices: task t = {first_row, first_key, lanes, base}; lane l < 64
 * gets base + mapping[req(first_row) * context + first_key + l] for l < lanes and
 * base + 0 (the safe slot) for the masked lanes of a partial task. A task with
 * no valid lane writes absolute index 0: that is what the Gaudi2 device test
 * expects (tests/attention_plan_smoke.py:37-38), where the CPU mock
 * (tests/multitile_paged_attention_unit_test.cpp:431-454) writes base + 0; the
 * index is never dereferenced for a visible key either way.
 * Task packing: src/bridge/attention_plan.cpp:241-258. */
void orc_tile_indices(const int32_t* mapping, const int32_t* requests, const int32_t* work,
                      int64_t tasks, int32_t context, int32_t* out) {
  for (int64_t t = 0; t < tasks; ++t) {
    const int32_t first_row = work[t * 4 + 0], first_key = work[t * 4 + 1];
    const int32_t lanes = work[t * 4 + 2], base = work[t * 4 + 3];
    const int32_t req = requests[first_row];
    for (int32_t l = 0; l < 64; ++l) {
      int32_t slot = 0;
      if (l < lanes) slot = mapping[(int64_t)req * context + first_key + l];
      out[t * 64 + l] = lanes > 0 ? base + slot : 0;
    }
  }
}

/* Token-granular map from a block table: slot(t) = bt[t / blk] * blk + t % blk.
 * Entries past a request's table are -1 (the reference's "no slot" marker,
 * src/bridge/paged_metadata.cpp:106). */
void orc_mapping_from_block_table(const int32_t* block_table, int64_t requests, int64_t max_blocks,
                                  int32_t block_size, int64_t context, int32_t* mapping) {
  for (int64_t r = 0; r < requests; ++r)
    for (int64_t t = 0; t < context; ++t) {
      const int64_t j = t / block_size;
      int32_t slot = -1;
      if (j < max_blocks && block_table[r * max_blocks + j] >= 0)
        slot = block_table[r * max_blocks + j] * block_size + (int32_t)(t % block_size);
      mapping[r * context + t] = slot;
    }
}

/* ---------------------------------------------------------------------------
 * Attention references. Work is fanned out over (row, kv_head) items.
 * ------------------------------------------------------------------------- */

typedef struct {
  const orc_attention_args* a;
  int kind;          /* 0 direct, 1 tiled, 2 direct_tiled, 3 fp64, 4 fp32 softmax, 5 guid */
  int32_t kv_tile;
  const int32_t* tiles_per_row;
  uint16_t* out16;
  double* out64;
  int64_t first, step;
  int status;
} worker_args;

static inline float qk(const uint16_t* q, const uint16_t* k, int32_t d) {
  float acc = 0.f;
  for (int32_t c = 0; c < d; ++c) acc += orc_bf16_to_f32(q[c]) * orc_bf16_to_f32(k[c]);
  return acc;
}

/* qk() for keys rows[0 .. n): out[t] = qk(q, rows[t], d), every key summed in
 * the same order (c = 0, 1, ...) with the same roundings. Eight keys run as
 * independent chains at a time, which only changes how fast the sums are
 * formed, not their values. */
#define ORC_KEYS 8
static void qk_keys(const uint16_t* q, const uint16_t* const* rows, int64_t n, int32_t d, float* out) {
  int64_t t = 0;
  for (; t + ORC_KEYS <= n; t += ORC_KEYS) {
    float acc[ORC_KEYS] = {0.f};
    for (int32_t c = 0; c < d; ++c) {
      const float qc = orc_bf16_to_f32(q[c]);
      for (int j = 0; j < ORC_KEYS; ++j) acc[j] += qc * orc_bf16_to_f32(rows[t + j][c]);
    }
    for (int j = 0; j < ORC_KEYS; ++j) out[t + j] = acc[j];
  }
  for (; t < n; ++t) out[t] = qk(q, rows[t], d);
}

/* The binary64 form: out[t] = sum_c (double)q[c] * (double)k[c], in order. */
static void qk_keys64(const uint16_t* q, const uint16_t* const* rows, int64_t n, int32_t d, double* out) {
  int64_t t = 0;
  for (; t + ORC_KEYS <= n; t += ORC_KEYS) {
    double acc[ORC_KEYS] = {0.0};
    for (int32_t c = 0; c < d; ++c) {
      const double qc = (double)orc_bf16_to_f32(q[c]);
      for (int j = 0; j < ORC_KEYS; ++j) acc[j] += qc * (double)orc_bf16_to_f32(rows[t + j][c]);
    }
    for (int j = 0; j < ORC_KEYS; ++j) out[t + j] = acc[j];
  }
  for (; t < n; ++t) {
    double s = 0.0;
    for (int32_t c = 0; c < d; ++c) s += (double)orc_bf16_to_f32(q[c]) * (double)orc_bf16_to_f32(rows[t][c]);
    out[t] = s;
  }
}

static inline float apply_softcap(float s, float cap) {
  return cap > 0.f ? cap * tanhf(s / cap) : s;
}

/* Visible key range of a row: [left, pos]. The sliding window keeps the last
 * `window` positions (tests/paged_attention_generalized_smoke.py:28). */
static void visible_range(const orc_attention_args* a, int64_t row, int64_t* left, int64_t* pos) {
  *pos = a->positions[row];
  *left = 0;
  if (a->sliding_window > 0 && *pos - a->sliding_window + 1 > 0) *left = *pos - a->sliding_window + 1;
}

static const uint16_t* key_row(const orc_attention_args* a, int32_t kvh, int32_t slot) {
  return a->key_pool + (int64_t)kvh * a->head_stride + (int64_t)slot * a->slot_stride;
}
static const uint16_t* value_row(const orc_attention_args* a, int32_t kvh, int32_t slot) {
  return a->value_pool + (int64_t)kvh * a->head_stride + (int64_t)slot * a->slot_stride;
}

/* direct_bf16_pv for one (row, head): tests/paged_attention_reference.py:6-20.
 * fp32 scores times scale, one fp32 softmax, probabilities rounded to bf16,
 * fp32 P.V, bf16 output. */
static void direct_row(const orc_attention_args* a, int64_t row, int32_t h, const int32_t* slots,
                       const uint16_t* const* krows, int64_t n, float* scores, float* acc, uint16_t* out) {
  const int32_t d = a->head_dim, kvh = h / (a->heads / a->kv_heads);
  const uint16_t* q = a->query + row * a->q_stride + (int64_t)h * d;
  qk_keys(q, krows, n, d, scores);
  float m = -INFINITY;
  for (int64_t t = 0; t < n; ++t) {
    scores[t] = apply_softcap(scores[t] * a->scale, a->softcap);
    if (scores[t] > m) m = scores[t];
  }
  float sum = 0.f;
  for (int64_t t = 0; t < n; ++t) {
    scores[t] = expf(scores[t] - m);
    sum += scores[t];
  }
  for (int32_t c = 0; c < d; ++c) acc[c] = 0.f;
  for (int64_t t = 0; t < n; ++t) {
    const float p = orc_bf16_to_f32(orc_bf16_from_f32(scores[t] / sum));
    const uint16_t* v = value_row(a, kvh, slots[t]);
    for (int32_t c = 0; c < d; ++c) acc[c] += p * orc_bf16_to_f32(v[c]);
  }
  for (int32_t c = 0; c < d; ++c) out[c] = orc_bf16_from_f32(acc[c]);
}

/* tiled_bf16_pv for one (row, head): tests/paged_attention_reference.py:23-57.
 * Per-tile max and sum, per-tile normalised bf16 probabilities, fp32 running
 * (max, sum, output) merge, bf16 output. */
static void tiled_row(const orc_attention_args* a, int64_t row, int32_t h, const int32_t* slots,
                      const uint16_t* const* krows, int64_t n, int32_t tile, float* dots, float* scores,
                      float* acc, float* run, uint16_t* out) {
  const int32_t d = a->head_dim, kvh = h / (a->heads / a->kv_heads);
  const uint16_t* q = a->query + row * a->q_stride + (int64_t)h * d;
  qk_keys(q, krows, n, d, dots);
  float run_max = 0.f, run_sum = 0.f;
  for (int64_t start = 0; start < n; start += tile) {
    const int64_t count = (n - start < tile) ? n - start : tile;
    float tmax = -INFINITY;
    for (int64_t t = 0; t < count; ++t) {
      scores[t] = apply_softcap(dots[start + t] * a->scale, a->softcap);
      if (scores[t] > tmax) tmax = scores[t];
    }
    float tsum = 0.f;
    for (int64_t t = 0; t < count; ++t) {
      scores[t] = expf(scores[t] - tmax);
      tsum += scores[t];
    }
    for (int32_t c = 0; c < d; ++c) acc[c] = 0.f;
    for (int64_t t = 0; t < count; ++t) {
      const float p = orc_bf16_to_f32(orc_bf16_from_f32(scores[t] / tsum));
      const uint16_t* v = value_row(a, kvh, slots[start + t]);
      for (int32_t c = 0; c < d; ++c) acc[c] += p * orc_bf16_to_f32(v[c]);
    }
    if (start == 0) {
      run_max = tmax;
      run_sum = tsum;
      for (int32_t c = 0; c < d; ++c) run[c] = acc[c] * tsum;
      continue;
    }
    const float next = run_max > tmax ? run_max : tmax;
    const float old_scale = expf(run_max - next);
    const float tile_scale = expf(tmax - next);
    const float weight = tile_scale * tsum;
    for (int32_t c = 0; c < d; ++c) run[c] = run[c] * old_scale + acc[c] * weight;
    run_sum = run_sum * old_scale + tsum * tile_scale;
    run_max = next;
  }
  for (int32_t c = 0; c < d; ++c) out[c] = orc_bf16_from_f32(run[c] / run_sum);
}

/* direct_tiled for one (row, head): tests/paged_attention_reference_test.py:8-27.
 * Global max and denominator, per-tile unnormalised bf16 probabilities scaled
 * by exp(local_max - max). */
static void direct_tiled_row(const orc_attention_args* a, int64_t row, int32_t h, const int32_t* slots,
                             const uint16_t* const* krows, int64_t n, int32_t tile, float* scores, float* acc,
                             float* num, uint16_t* out) {
  const int32_t d = a->head_dim, kvh = h / (a->heads / a->kv_heads);
  const uint16_t* q = a->query + row * a->q_stride + (int64_t)h * d;
  qk_keys(q, krows, n, d, scores);
  float m = -INFINITY;
  for (int64_t t = 0; t < n; ++t) {
    scores[t] = apply_softcap(scores[t] * a->scale, a->softcap);
    if (scores[t] > m) m = scores[t];
  }
  float den = 0.f;
  for (int64_t t = 0; t < n; ++t) den += expf(scores[t] - m);
  for (int32_t c = 0; c < d; ++c) num[c] = 0.f;
  for (int64_t start = 0; start < n; start += tile) {
    const int64_t count = (n - start < tile) ? n - start : tile;
    float lmax = -INFINITY;
    for (int64_t t = 0; t < count; ++t)
      if (scores[start + t] > lmax) lmax = scores[start + t];
    for (int32_t c = 0; c < d; ++c) acc[c] = 0.f;
    for (int64_t t = 0; t < count; ++t) {
      const float p = orc_bf16_to_f32(orc_bf16_from_f32(expf(scores[start + t] - lmax)));
      const uint16_t* v = value_row(a, kvh, slots[start + t]);
      for (int32_t c = 0; c < d; ++c) acc[c] += p * orc_bf16_to_f32(v[c]);
    }
    const float w = expf(lmax - m);
    for (int32_t c = 0; c < d; ++c) num[c] += acc[c] * w;
  }
  for (int32_t c = 0; c < d; ++c) out[c] = orc_bf16_from_f32(num[c] / den);
}

/* binary64 attention for one (row, head): the fp64 truth of
 * tests/paged_attention_smoke.py:39-50 and
 * tests/fused_paged_decode_device_test.cpp:374-440 (before direct_bf16). */
static void fp64_row(const orc_attention_args* a, int64_t row, int32_t h, const int32_t* slots,
                     const uint16_t* const* krows, int64_t n, double* scores, double* out) {
  const int32_t d = a->head_dim, kvh = h / (a->heads / a->kv_heads);
  const uint16_t* q = a->query + row * a->q_stride + (int64_t)h * d;
  qk_keys64(q, krows, n, d, scores);
  double m = -INFINITY;
  for (int64_t t = 0; t < n; ++t) {
    double s = scores[t] * (double)a->scale;
    if (a->softcap > 0.f) s = (double)a->softcap * tanh(s / (double)a->softcap);
    scores[t] = s;
    if (s > m) m = s;
  }
  double den = 0.0;
  for (int64_t t = 0; t < n; ++t) {
    scores[t] = exp(scores[t] - m);
    den += scores[t];
  }
  for (int32_t c = 0; c < d; ++c) out[c] = 0.0;
  for (int64_t t = 0; t < n; ++t) {
    const double p = scores[t] / den;
    const uint16_t* v = value_row(a, kvh, slots[t]);
    for (int32_t c = 0; c < d; ++c) out[c] += p * (double)orc_bf16_to_f32(v[c]);
  }
}

/* fp32 softmax without bf16 probabilities: the CPU reference of
 * tests/paged_attention_generalized_smoke.py:16-34 (softcap and sliding window). */
static void fp32_row(const orc_attention_args* a, int64_t row, int32_t h, const int32_t* slots,
                     const uint16_t* const* krows, int64_t n, float* scores, float* acc, uint16_t* out) {
  const int32_t d = a->head_dim, kvh = h / (a->heads / a->kv_heads);
  const uint16_t* q = a->query + row * a->q_stride + (int64_t)h * d;
  qk_keys(q, krows, n, d, scores);
  float m = -INFINITY;
  for (int64_t t = 0; t < n; ++t) {
    scores[t] = apply_softcap(scores[t] * a->scale, a->softcap);
    if (scores[t] > m) m = scores[t];
  }
  float sum = 0.f;
  for (int64_t t = 0; t < n; ++t) {
    scores[t] = expf(scores[t] - m);
    sum += scores[t];
  }
  for (int32_t c = 0; c < d; ++c) acc[c] = 0.f;
  for (int64_t t = 0; t < n; ++t) {
    const float p = scores[t] / sum;
    const uint16_t* v = value_row(a, kvh, slots[t]);
    for (int32_t c = 0; c < d; ++c) acc[c] += p * orc_bf16_to_f32(v[c]);
  }
  for (int32_t c = 0; c < d; ++c) out[c] = orc_bf16_from_f32(acc[c]);
}

/* The reference device numerics (GUID semantics) for one (row, head).
 * tiles <= 1: gk_attn_direct_softmax_bf16_v1 + bf16-output P.V
 *   (tests/multitile_paged_attention_unit_test.cpp:1396-1424);
 * tiles > 1: per-tile gk_attn_tile_softmax_bf16_v1, gk_attn_online_merge_f32_v1
 *   with prev_unscaled on the second tile, gk_attn_online_finalize_bf16_v1
 *   (same file, :1425-1480 and the emulation at :628-738). Tiles beyond the
 *   row's position are empty (m = -inf, l = 0) and merge as no-ops. */
static void guid_row(const orc_attention_args* a, int64_t row, int32_t h, const int32_t* slots,
                     const uint16_t* const* krows, int64_t n, int32_t tiles, int32_t tile, float* dots,
                     float* scores, float* acc, float* run, uint16_t* out) {
  const int32_t d = a->head_dim, kvh = h / (a->heads / a->kv_heads);
  const uint16_t* q = a->query + row * a->q_stride + (int64_t)h * d;
  qk_keys(q, krows, n, d, dots);
  if (tiles <= 1) {
    float m = -INFINITY;
    for (int64_t t = 0; t < n; ++t) {
      scores[t] = dots[t] * a->scale;
      if (scores[t] > m) m = scores[t];
    }
    const float origin = isinf(m) ? 0.f : m;
    float sum = 0.f;
    for (int64_t t = 0; t < n; ++t) {
      scores[t] = expf(scores[t] - origin);
      sum += scores[t];
    }
    const float inv = sum > 0.f ? 1.f / sum : 0.f;
    for (int32_t c = 0; c < d; ++c) acc[c] = 0.f;
    for (int64_t t = 0; t < n; ++t) {
      const float p = orc_bf16_to_f32(orc_bf16_from_f32(scores[t] * inv));
      const uint16_t* v = value_row(a, kvh, slots[t]);
      for (int32_t c = 0; c < d; ++c) acc[c] += p * orc_bf16_to_f32(v[c]);
    }
    for (int32_t c = 0; c < d; ++c) out[c] = orc_bf16_from_f32(acc[c]);
    return;
  }
  float run_m = 0.f, run_l = 0.f;
  for (int32_t c = 0; c < d; ++c) run[c] = 0.f;
  if ((int64_t)tiles * tile < n) tiles = (int32_t)((n + tile - 1) / tile); /* a block covers its rows */
  for (int32_t ti = 0; ti < tiles; ++ti) {
    const int64_t key_start = (int64_t)ti * tile;
    const int64_t last = (n - 1 - key_start < tile - 1) ? n - 1 - key_start : tile - 1;
    float tm = -INFINITY, tl = 0.f;
    for (int32_t c = 0; c < d; ++c) acc[c] = 0.f;
    if (last >= 0) {
      for (int64_t k = 0; k <= last; ++k) {
        scores[k] = dots[key_start + k] * a->scale;
        if (scores[k] > tm) tm = scores[k];
      }
      const float origin = (tm == -INFINITY) ? 0.f : tm;
      for (int64_t k = 0; k <= last; ++k) {
        scores[k] = expf(scores[k] - origin);
        tl += scores[k];
      }
      const float inv = tl > 0.f ? 1.f / tl : 0.f;
      for (int64_t k = 0; k <= last; ++k) {
        const float p = orc_bf16_to_f32(orc_bf16_from_f32(scores[k] * inv));
        const uint16_t* v = value_row(a, kvh, slots[key_start + k]);
        for (int32_t c = 0; c < d; ++c) acc[c] += p * orc_bf16_to_f32(v[c]);
      }
    }
    if (ti == 0) {
      run_m = tm;
      run_l = tl;
      for (int32_t c = 0; c < d; ++c) run[c] = acc[c];
      continue;
    }
    const float v0 = run_l > 0.f ? run_m : -INFINITY;
    const float v1 = tl > 0.f ? tm : -INFINITY;
    const float next = v0 > v1 ? v0 : v1;
    const float origin = (next == -INFINITY) ? 0.f : next;
    const float wa0 = run_l > 0.f ? expf(run_m - origin) : 0.f;
    const float wb0 = tl > 0.f ? expf(tm - origin) : 0.f;
    const float wa = (ti == 1) ? wa0 * run_l : wa0;
    const float wb = wb0 * tl;
    for (int32_t c = 0; c < d; ++c) run[c] = wa * run[c] + wb * acc[c];
    run_l = wa0 * run_l + wb0 * tl;
    run_m = next;
  }
  const float inv = run_l > 0.f ? 1.f / run_l : 0.f;
  for (int32_t c = 0; c < d; ++c) out[c] = orc_bf16_from_f32(run[c] * inv);
}

static void* attention_worker(void* opaque) {
  worker_args* w = (worker_args*)opaque;
  const orc_attention_args* a = w->a;
  const int32_t d = a->head_dim, group = a->heads / a->kv_heads;
  const int64_t max_keys = a->context;
  int32_t* slots = (int32_t*)malloc(sizeof(int32_t) * (size_t)(max_keys > 0 ? max_keys : 1));
  float* scores = (float*)malloc(sizeof(float) * (size_t)(max_keys > 0 ? max_keys : 1));
  float* dots = (float*)malloc(sizeof(float) * (size_t)(max_keys > 0 ? max_keys : 1));
  double* scores64 = (double*)malloc(sizeof(double) * (size_t)(max_keys > 0 ? max_keys : 1));
  const uint16_t** krows = (const uint16_t**)malloc(sizeof(uint16_t*) * (size_t)(max_keys > 0 ? max_keys : 1));
  float* acc = (float*)malloc(sizeof(float) * (size_t)d * 2);
  float* run = acc + d;
  if (!slots || !scores || !dots || !scores64 || !krows || !acc) {
    w->status = -2;
    free(slots); free(scores); free(dots); free(scores64); free(krows); free(acc);
    return NULL;
  }
  const int64_t items = a->rows * a->kv_heads;
  for (int64_t item = w->first; item < items; item += w->step) {
    const int64_t row = item / a->kv_heads;
    const int32_t kvh = (int32_t)(item % a->kv_heads);
    int64_t left, pos;
    visible_range(a, row, &left, &pos);
    if (pos < 0 || pos >= a->context) { w->status = -3; break; }
    const int64_t n = pos - left + 1;
    const int32_t* map_row = a->mapping + a->requests[row] * a->context;
    for (int64_t t = 0; t < n; ++t) {
      slots[t] = map_row[left + t];
      krows[t] = key_row(a, kvh, slots[t]);
    }
    for (int32_t gh = 0; gh < group; ++gh) {
      const int32_t h = kvh * group + gh;
      uint16_t* o16 = w->out16 ? w->out16 + (row * a->heads + h) * d : NULL;
      switch (w->kind) {
        case 0: direct_row(a, row, h, slots, krows, n, scores, acc, o16); break;
        case 1: tiled_row(a, row, h, slots, krows, n, w->kv_tile, dots, scores, acc, run, o16); break;
        case 2: direct_tiled_row(a, row, h, slots, krows, n, w->kv_tile, scores, acc, run, o16); break;
        case 3: fp64_row(a, row, h, slots, krows, n, scores64, w->out64 + (row * a->heads + h) * d); break;
        case 4: fp32_row(a, row, h, slots, krows, n, scores, acc, o16); break;
        default:
          guid_row(a, row, h, slots, krows, n, w->tiles_per_row[row], w->kv_tile, dots, scores, acc, run, o16);
          break;
      }
    }
  }
  free(slots); free(scores); free(dots); free(scores64); free(krows); free(acc);
  return NULL;
}

static int run_attention(const orc_attention_args* a, int kind, int32_t kv_tile, const int32_t* tiles,
                         uint16_t* out16, double* out64) {
  if (a->heads <= 0 || a->kv_heads <= 0 || a->heads % a->kv_heads || a->head_dim <= 0) return -1;
  if ((kind == 1 || kind == 2 || kind == 5) && kv_tile <= 0) return -1;
  int threads = a->threads > 0 ? a->threads : 1;
  if (threads > 256) threads = 256;
  worker_args w[256];
  pthread_t tid[256];
  for (int i = 0; i < threads; ++i) {
    w[i] = (worker_args){a, kind, kv_tile, tiles, out16, out64, i, threads, 0};
  }
  if (threads == 1) {
    attention_worker(&w[0]);
    return w[0].status;
  }
  int started = 0;
  for (; started < threads; ++started)
    if (pthread_create(&tid[started], NULL, attention_worker, &w[started])) break;
  for (int i = 0; i < started; ++i) pthread_join(tid[i], NULL);
  if (started < threads) {
    for (int i = started; i < threads; ++i) attention_worker(&w[i]);
  }
  for (int i = 0; i < threads; ++i)
    if (w[i].status) return w[i].status;
  return 0;
}

int orc_direct_bf16_pv(const orc_attention_args* a, uint16_t* out) {
  return run_attention(a, 0, 0, NULL, out, NULL);
}
int orc_tiled_bf16_pv(const orc_attention_args* a, int32_t kv_tile, uint16_t* out) {
  return run_attention(a, 1, kv_tile, NULL, out, NULL);
}
int orc_direct_tiled(const orc_attention_args* a, int32_t kv_tile, uint16_t* out) {
  return run_attention(a, 2, kv_tile, NULL, out, NULL);
}
int orc_fp64_attention(const orc_attention_args* a, double* out) {
  return run_attention(a, 3, 0, NULL, NULL, out);
}
int orc_fp32_softmax_attention(const orc_attention_args* a, uint16_t* out) {
  return run_attention(a, 4, 0, NULL, out, NULL);
}
int orc_guid_attention(const orc_attention_args* a, const int32_t* tiles_per_row, int32_t kv_tile,
                       uint16_t* out) {
  return run_attention(a, 5, kv_tile, tiles_per_row, out, NULL);
}
