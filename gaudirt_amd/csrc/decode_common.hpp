// Definitions shared by the decode kernels (partitioned and balanced schedules).
#pragma once

#include "gk_mfma.hpp"
#include "work_order.hpp"

namespace gk {

// The MFMA kernels re-base their running max when a score exceeds it by more
// than this (log2 units), so probabilities stay <= 2^slack. At 0 every new
// maximum re-bases: the largest probability is exactly 1 and the bf16
// rounding of the others tracks the reference's normalised probabilities
// closely enough for its relative-L2 gate against the tiled reference
// (5e-3) on rows of a few keys; a slack of 8 (rarer re-bases) reached 6.4e-3
// there. GK_DECODE_RESCALE_SLACK selects another slack at build time.
#ifndef GK_DECODE_RESCALE_SLACK
#define GK_DECODE_RESCALE_SLACK 0
#endif
constexpr float kDecodeRescaleSlack = GK_DECODE_RESCALE_SLACK;

struct DecodeArgs {
  const uint16_t* query;
  int64_t q_stride;
  const uint16_t* pool;
  int64_t slots;
  const int32_t* block_tables;
  int64_t bt_stride;
  int32_t block_shift;
  const int32_t* row_request;
  const int32_t* row_context;
  const int32_t* row_map;
  int32_t rows, q_heads, kv_heads, group, head_groups, heads_per_group;
  float score_scale;  // scale * log2(e), or scale / softcap when capping
  float softcap_log2; // softcap * log2(e) when capping
  int32_t window, partition, max_parts;
  uint16_t* out;
  int64_t out_stride;
  float* part_o;
  float* part_ml;
};

template <int D>
struct MfmaShape {
  static constexpr int TS = D == 256 ? 16 : 32;   // keys per step
  static constexpr int TG = TS / 16;              // 16-key groups per step (QK tiles)
  static constexpr int NC = D / 32;               // 32-dim k chunks of Q.K
  static constexpr int CPR = D / 8;               // 16-byte chunks per head row
  static constexpr int LOADS = TS * CPR / 64;     // 16-byte loads per lane per tile
  static constexpr int NO = D / 16;               // 16-dim output chunks of P.V
  static constexpr int TILE = TS * D * 2;         // bytes of one K or V tile in LDS
};

// Balanced ("stream") decode schedule, head dims 64/128/256, GQA group >= 4,
// any block size. Workspace layout: part_o[2 * wgs][hpw][D],
// part_ml[2 * wgs][hpw][2] and unit_span[units] (int32 pairs).
int stream_decode_wgs(int head_dim, bool softcap, int block_size);
size_t stream_decode_workspace_bytes(int head_dim, int heads_per_group, int64_t units, int wgs);
int launch_stream_decode(const DecodeArgs& a, bool softcap, int head_dim, int wgs, void* workspace,
                         hipStream_t stream);

}  // namespace gk
