/*
 * CPU oracle for the paged-attention path: a plain-C restatement of the
 * GaudiRT reference algorithms. TEST INFRASTRUCTURE ONLY — the product never
 * links, loads or calls anything declared here; only tests, the smoke entry
 * point and the benchmark's CPU-baseline leg do, and only as the checker.
 *
 * Layout conventions shared by every function:
 *   - bf16 values travel as uint16_t bit patterns.
 *   - A KV pool is addressed as pool[head * head_stride + slot * slot_stride + c]
 *     (elements). The head-major pool [2, Hkv, S, d] has slot_stride = d and
 *     head_stride = S * d; its value half starts Hkv * S * d elements later.
 *   - mapping is the token-granular request map [requests, context] int32:
 *     token t of request r lives at slot mapping[r * context + t].
 */
#ifndef GAUDIRT_AMD_ORACLE_H
#define GAUDIRT_AMD_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

uint16_t orc_bf16_from_f32(float value);
float orc_bf16_to_f32(uint16_t value);
/* Direct binary64 -> bf16 round-to-nearest-even (one rounding). Returns 0 on
 * success, -1 when an input is not finite (the reference raises). */
int orc_bf16_from_f64_array(const double* in, uint16_t* out, int64_t n);
void orc_bf16_from_f32_array(const float* in, uint16_t* out, int64_t n);

void orc_kv_store(const uint16_t* key, const uint16_t* value, int64_t row_stride,
                  const int32_t* locations, int32_t valid_rows, uint16_t* pool,
                  int64_t slots, int32_t kv_heads, int32_t head_dim);

void orc_tile_indices(const int32_t* mapping, const int32_t* requests, const int32_t* work,
                      int64_t tasks, int32_t context, int32_t* out);

void orc_mapping_from_block_table(const int32_t* block_table, int64_t requests, int64_t max_blocks,
                                  int32_t block_size, int64_t context, int32_t* mapping);

/* Attention references. Each row r attends keys mapping[requests[r], 0..positions[r]]
 * (optionally limited to a sliding window) and writes out[r, heads * head_dim]. */
typedef struct {
  const uint16_t* query;  /* [rows, q_stride] bf16 */
  int64_t q_stride;
  const uint16_t* key_pool;
  const uint16_t* value_pool;
  int64_t slot_stride, head_stride;
  const int64_t* requests;
  const int64_t* positions;
  const int32_t* mapping;
  int64_t context;
  int64_t rows;
  int32_t heads, kv_heads, head_dim;
  float scale;
  float softcap;          /* 0 = off */
  int32_t sliding_window; /* -1 = off */
  int32_t threads;
} orc_attention_args;

int orc_direct_bf16_pv(const orc_attention_args* a, uint16_t* out);
int orc_tiled_bf16_pv(const orc_attention_args* a, int32_t kv_tile, uint16_t* out);
int orc_direct_tiled(const orc_attention_args* a, int32_t kv_tile, uint16_t* out);
int orc_fp64_attention(const orc_attention_args* a, double* out);
int orc_fp32_softmax_attention(const orc_attention_args* a, uint16_t* out);
int orc_guid_attention(const orc_attention_args* a, const int32_t* tiles_per_row, int32_t kv_tile,
                       uint16_t* out);

#ifdef __cplusplus
}
#endif

#endif
