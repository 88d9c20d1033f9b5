// Internal declarations shared by the libpagedkv translation units.
// Everything here is gfx950-only device code plus host launchers; the public
// surface is include/pagedkv.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/pagedkv.h"

namespace pkv {

using bf16 = __bf16;
using f16 = _Float16;

// Host-side error reporting (capi.cpp). Returns `code` so callers can write
// `return fail(PKV_ERR_INVALID, "...")`.
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

inline int elem_bytes(int dtype) {
  return dtype == PKV_DTYPE_F32 ? 4 : 2;
}

// ---------------------------------------------------------------------------
// Append / gather (append.hip)
// ---------------------------------------------------------------------------
int launch_append(void* k_pool, void* v_pool, int64_t pool_slots,
                  const void* k_new, const void* v_new, const int64_t* slots,
                  int64_t n_tok, int64_t row_bytes, int* status,
                  hipStream_t stream);

int launch_append_from_table(void* k_pool, void* v_pool, int64_t num_blocks,
                             int bs_shift, const void* k_new,
                             const void* v_new, const int32_t* block_tables,
                             int max_blk, const int32_t* qloc,
                             const int32_t* start_pos, int n_seq,
                             int64_t n_tok, int64_t row_bytes, int* status,
                             hipStream_t stream);

int launch_gather(void* k_out, void* v_out, const void* k_pool,
                  const void* v_pool, int64_t num_blocks, int bs_shift,
                  const int32_t* table, int n_blocks, int seq_len,
                  int64_t row_bytes, int* status, hipStream_t stream);

// ---------------------------------------------------------------------------
// Attention (attention.hip)
// ---------------------------------------------------------------------------
struct AttnArgs {
  void* out;
  float* lse;
  const void* q;
  const void* k_pool;
  const void* v_pool;
  const int32_t* block_tables;
  const int32_t* seq_lens;
  const int32_t* qloc;  // nullable: one query per sequence
  int64_t num_blocks;
  int bs_shift;
  int max_blk;
  int n_seq;
  int hq;
  int hkv;
  int group;  // hq / hkv
  int d;
  float scale_log2;  // softmax scale * log2(e)
  int causal;
  int part_tokens;   // split-K partition length (multiple of 32)
  int parts_max;     // partitions per (sequence, kv head, row tile) in grid
  int tiles_max;     // row tiles per (sequence, kv head) in grid
  float* ws_o;       // [units][ROWS][d] unnormalised partial outputs
  float* ws_ml;      // [units][ROWS][2] (running max (log2 units), sum)
  int* status;
};

// Rows ((query token, head) pairs of one kv head) per tile of the generic
// kernel.
constexpr int kGenRows = 32;
constexpr int kChunk = 32;  // kv tokens staged per iteration

struct AttnPlan {
  int kind;        // 0 = generic rows kernel, 1 = MFMA decode kernel
  int rows;        // rows per tile of the chosen kernel
  int part_tokens;
  int parts_max;
  int tiles_max;
  size_t ws_bytes;
};

AttnPlan plan_attention(int n_seq, int max_q_len, int hq, int hkv, int d,
                        int max_blk, int block_size, int max_kv_len,
                        int part_tokens, int dtype);

int launch_attention(const AttnArgs& a, const AttnPlan& plan, int dtype,
                     hipStream_t stream);

}  // namespace pkv
