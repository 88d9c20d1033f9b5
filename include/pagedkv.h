/*
 * pagedkv.h — C ABI of libpagedkv.so, the MI355X (gfx950) paged KV-cache
 * decode path: slot-mapped K/V append into a block pool, block-table gather,
 * and paged (multi-query) attention with split-K over the context.
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers unless stated otherwise. The caller
 *     owns every buffer (outputs, workspace, status word); nothing here
 *     allocates device memory.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     Work is enqueued asynchronously; no entry point synchronises the host.
 *   - Return value: PKV_OK (0) or a negative PKV_ERR_* code; the message of
 *     the last failure on the calling thread is pkv_last_error().
 *   - `dtype` is one of PKV_DTYPE_*; K/V/Q/out share it. OR-ing PKV_KV_FP8
 *     into it declares fp8 pools: the pools hold fp8 e4m3 (OCP,
 *     torch.float8_e4m3fn; 1 byte per element) while Q, out and the rows
 *     appended keep the PKV_DTYPE_* type (KVPool with
 *     CacheConfig.kv_dtype = torch.float8_e4m3fn, models/model_config.py:49,
 *     :77-88).
 *   - Pool layout (per layer, per K or V): [num_blocks, block_size, hkv, d]
 *     contiguous, i.e. token slot `s` starts at element s * hkv * d.
 *   - `status` (nullable) is a device int32 word the kernels OR error bits
 *     into (PKV_STATUS_*) instead of touching memory out of bounds; the caller
 *     zeroes it and reads it whenever it chooses to synchronise.
 *
 * Reference interfaces replaced (paths relative to the reference repository
 * akshay919191/tiny-transformer-inference-engine):
 *   pkv_append            KVPool.write              serving/kv_pool.py:57-70
 *   pkv_append_from_table KVPool.make_slot_mapping + write, looped per
 *                         sequence in MQA_Paged.forward_paged_batched
 *                                                    serving/kv_pool.py:40-55,
 *                                                    serving/paged_mqa.py:87-99
 *   pkv_gather            KVPool.gather             serving/kv_pool.py:72-82
 *   pkv_paged_attention   pagedattn.paged_attn_fwd  kernels/pagedattn/extension.cpp:56-69
 *                         (paged_attn_fwd_cuda      kernels/pagedattn/pagedattn.cu:1052-1079)
 *   pkv_attention_workspace_bytes  no counterpart: the reference kernel has no
 *                         split-K and therefore no workspace.
 *   pkv_paged_attention_append  KVPool.write + paged_varlen_attention per
 *                         layer                      serving/paged_mqa.py:98-110
 *   pkv_rms_norm          RMSNorm.forward            models/rmsnorm.py:12-18
 *                         (with the residual add of PagedBlock.forward,
 *                         serving/paged_model.py:20-29, fused in front)
 *   pkv_rope              RoPE.forward_at / _rotate  models/rope.py:21-47
 *                         as applied to q, k in MQA_Paged.forward_paged_batched
 *                                                    serving/paged_mqa.py:80-85
 *   pkv_silu_mul          fused_swiglu               kernels/fused_swiglu/kernel.py:6-19,131-136
 *   pkv_linear            nn.Linear of the block's out / down projections
 *                                                    serving/paged_mqa.py:112-113,
 *                                                    models/mlp.py:31-32
 *   pkv_linear_swiglu     gate_proj, up_proj and fused_swiglu
 *                                                    models/mlp.py:24-30
 *   pkv_linear_rope_qkv   q/k/v projections and RoPE serving/paged_mqa.py:76-85
 *   pkv_linear_residual   x + out(attn) / x + down_proj(...) of PagedBlock.forward
 *                                                    serving/paged_model.py:20-29
 *   pkv_linear_swiglu_rmsnorm  mlp_norm + gate_proj, up_proj, fused_swiglu
 *                                                    serving/paged_model.py:28-29,
 *                                                    models/rmsnorm.py:12-18, models/mlp.py:24-30
 *   pkv_linear_rope_qkv_rmsnorm  attn_norm + q/k/v projections and RoPE
 *                                                    serving/paged_model.py:26-27,
 *                                                    models/rmsnorm.py:12-18, serving/paged_mqa.py:76-85
 *   pkv_argmax_rows       greedy token choice: logits.argmax per sequence
 *   pkv_sample_rows       sample(): temperature, top-k, top-p, one draw per
 *                         row (sampling.py:94-137; the top-k step of
 *                         kernels/cuda-kSAMPLING/ksampling_kernel.cu:61-185)
 *                                                    serving/generation.py:77,88,132,142;
 *                         greedy()                   sampling.py:5-137
 */
#ifndef PAGEDKV_H
#define PAGEDKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PKV_VERSION 1

#define PKV_DTYPE_F32 0
#define PKV_DTYPE_F16 1
#define PKV_DTYPE_BF16 2
/* Flag OR-ed into `dtype`: the K/V pools hold fp8 e4m3. Appends round each
   new value to the nearest fp8 value (ties to even; magnitudes above 464,
   those that round past 448, infinities and NaN give NaN), the bytes
   torch's conversion to float8_e4m3fn gives; attention widens pool values
   exactly. Attention with fp8 pools: bf16/f16 Q, 16 or 32 query heads per
   kv head, d = 64 or 128. */
#define PKV_KV_FP8 0x100

/* part_tokens values of pkv_paged_attention selecting a persistent decode
   kernel where it applies (bf16/f16, one query per sequence, 16 or 32
   query heads per kv head, d = 64 or 128). Each gives every workgroup an
   equal share of all sequences' chunks. PKV_PART_PERSISTENT and
   PKV_PART_STATIC take the register-staged kernel (the automatic choice
   for long context bounds); PKV_PART_STREAM takes the wavefront-specialised
   kernel, whose producer wavefronts stream K/V into LDS by LDS-DMA while
   consumer wavefronts compute, where it applies (a decode batch without the
   fused append, 16-bit pools, d = 128, block size >= 16), else the
   register-staged one. */
#define PKV_PART_PERSISTENT (-1)
#define PKV_PART_STATIC (-2)
#define PKV_PART_STREAM (-3)

#define PKV_OK 0
#define PKV_ERR_INVALID (-1)     /* bad argument (shape, null pointer, ...) */
#define PKV_ERR_UNSUPPORTED (-2) /* valid but unsupported configuration   */
#define PKV_ERR_WORKSPACE (-3)   /* workspace missing or too small         */
#define PKV_ERR_HIP (-4)         /* a HIP runtime call failed              */

/* Bits OR-ed into *status by the kernels. */
#define PKV_STATUS_BAD_SLOT 1    /* append: slot outside [-slots, slots)   */
#define PKV_STATUS_BAD_BLOCK 2   /* a block-table entry outside [0, num_blocks)
                                    (or block 0 for an append) was skipped */
#define PKV_STATUS_SHORT_TABLE 4 /* append: position beyond the table      */
#define PKV_STATUS_BAD_QLOC 8    /* attention: query range outside [0, T)  */
#define PKV_STATUS_BAD_POS 16    /* rope: position outside [0, max_pos)    */
#define PKV_STATUS_NONFINITE 32  /* sampling: a logit is NaN or infinite    */
#define PKV_STATUS_BAD_DISTRIBUTION 64 /* sampling: logit / temperature overflowed */
#define PKV_STATUS_SAMPLE_OVERFLOW 128 /* sampling: too many ties at the top-k
                                          threshold for the kernel (id -1)    */
#define PKV_STATUS_DIRTY_WORKSPACE 256 /* attention: an arrival counter of the
                                          workspace was not zero when the call
                                          started (workspace not zero-filled, or
                                          shared by overlapping calls); rows of
                                          sequences split across workgroups may
                                          be missing or wrong                 */
#define PKV_STATUS_STALLED 512  /* attention (wavefront-specialised decode
                                   kernel): a wait between its wavefronts ran
                                   out of its poll bound and the kernel left
                                   early; the outputs are not valid       */

/* Library version (PKV_VERSION). */
int pkv_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* pkv_last_error(void);

/*
 * Slot-mapped scatter: for t in [0, n_tok):
 *   k_pool[slot(t)] = k_new[t];  v_pool[slot(t)] = v_new[t]
 * where a row is `row_elems` (= hkv * d) contiguous elements and
 * slot(t) = slot_mapping[t] (int64), wrapped by pool_slots when negative
 * (index_put semantics). Slots outside [-pool_slots, pool_slots) are skipped
 * and flagged PKV_STATUS_BAD_SLOT. Bit-exact copy (with PKV_KV_FP8: each
 * value rounded to fp8 as torch's index_put into a float8_e4m3fn pool does).
 * Replaces KVPool.write (serving/kv_pool.py:57-70).
 */
int pkv_append(void* k_pool, void* v_pool, int64_t pool_slots,
               const void* k_new, const void* v_new,
               const int64_t* slot_mapping, int64_t n_tok, int64_t row_elems,
               int dtype, int* status, void* stream);

/*
 * Append with the slot computed in-kernel from device metadata. Token t of
 * sequence s (query_start_loc[s] <= t < query_start_loc[s+1]) sits at
 * position p = start_pos[s] + (t - query_start_loc[s]) and goes to slot
 *   block_tables[s * max_blk + p / block_size] * block_size + p % block_size.
 * A position beyond max_blk blocks (PKV_STATUS_SHORT_TABLE) or a physical
 * block outside [1, num_blocks) (PKV_STATUS_BAD_BLOCK; block 0 is reserved)
 * is skipped. Same result as make_slot_mapping + write per sequence.
 * Replaces serving/kv_pool.py:40-70 as looped in serving/paged_mqa.py:87-99.
 */
int pkv_append_from_table(void* k_pool, void* v_pool, int64_t num_blocks,
                          int block_size, const void* k_new, const void* v_new,
                          const int32_t* block_tables, int max_blk,
                          const int32_t* query_start_loc,
                          const int32_t* start_pos, int n_seq, int64_t n_tok,
                          int64_t row_elems, int dtype, int* status,
                          void* stream);

/*
 * Gather one sequence's first seq_len token rows out of the pool into dense
 * k_out/v_out [seq_len, row_elems] following block_table (device int32,
 * n_blocks entries), in the pool's element type (fp8 bytes with
 * PKV_KV_FP8). Replaces KVPool.gather (serving/kv_pool.py:72-82).
 */
int pkv_gather(void* k_out, void* v_out, const void* k_pool,
               const void* v_pool, int64_t num_blocks, int block_size,
               const int32_t* block_table, int n_blocks, int seq_len,
               int64_t row_elems, int dtype, int* status, void* stream);

/*
 * Bytes of workspace pkv_paged_attention needs for this problem (0 when no
 * sequence is split). `max_kv_len` <= 0 means max_blk * block_size.
 * The workspace holds partial results and, in its first 256 KiB, the
 * persistent kernel's per-sequence arrival counters: zero-fill it once
 * before its first use; every call leaves the counters zero again. Calls
 * that overlap on one workspace race.
 */
size_t pkv_attention_workspace_bytes(int n_seq, int max_q_len, int hq, int hkv,
                                     int d, int max_blk, int block_size,
                                     int max_kv_len, int part_tokens,
                                     int dtype);

/*
 * Paged attention forward, semantics of pagedattn.paged_attn_fwd
 * (kernels/pagedattn/pagedattn.cu:142-447, host side :1052-1079):
 *   q   [T, hq, d]; out [T, hq, d]; lse (nullable) float [T, hq]
 *   k_pool/v_pool [num_blocks, block_size, hkv, d]
 *   block_tables int32 [n_seq, max_blk]; seq_lens int32 [n_seq]
 *   query_start_loc int32 [n_seq + 1] (NULL = one query per sequence,
 *   token s belongs to sequence s: the decode case); n_tokens = T. A
 *   sequence whose query range falls outside [0, T) is skipped and flagged
 *   PKV_STATUS_BAD_QLOC.
 * For sequence s: kv_len = min(seq_lens[s], max_blk * block_size),
 * q_len = query_start_loc[s+1] - query_start_loc[s],
 * ctx = causal ? max(kv_len - q_len, 0) : 0; query i sees key j iff
 * j < kv_len and (!causal or j <= ctx + i). Query head h reads kv head
 * h / (hq / hkv). scale <= 0 means 1/sqrt(d). Rows with no visible key give
 * out = 0 and lse = +inf. lse = m + ln(l) in natural-log units.
 * `max_q_len` must bound every q_len; `max_kv_len` (<= 0: the table
 * capacity) must bound every kv_len; `part_tokens` is the split-K
 * partition length (0: automatic, the persistent kernel for context bounds
 * of 4096 tokens and more where it applies, else fixed partitions;
 * PKV_PART_PERSISTENT or PKV_PART_STATIC: persistent workgroups each taking
 * an equal share of all context chunks; other negative values are invalid).
 * Workspace: pkv_attention_workspace_bytes().
 */
int pkv_paged_attention(void* out, float* lse, const void* q,
                        const void* k_pool, const void* v_pool,
                        int64_t num_blocks, int block_size,
                        const int32_t* block_tables, int max_blk,
                        const int32_t* seq_lens,
                        const int32_t* query_start_loc, int n_seq,
                        int n_tokens, int max_q_len, int max_kv_len, int hq,
                        int hkv, int d,
                        float scale, int causal, int part_tokens, int dtype,
                        void* workspace, size_t workspace_bytes, int* status,
                        void* stream);

/*
 * pkv_append_from_table followed by pkv_paged_attention in one call: the
 * step's new K/V rows (k_new, v_new [n_tokens, hkv, d], row t of sequence s
 * at position start_pos[s] + t - query_start_loc[s]) are appended to the
 * pools and attended to by the same call. The append is fused into the
 * attention launch where the kernel allows: on the split-K partition decode
 * kernel (bf16/f16 queries, one query per sequence, 16 or 32 query heads per
 * kv head, d = 64 or 128, context bound below 4096 tokens; fp8 pools too)
 * the workgroup whose context range covers the new row takes it from k_new
 * / v_new and the one holding the sequence's last chunk writes it to its
 * pool slot; with 16-bit pools, the MFMA prefill kernel (at most 512
 * sequences) writes every row of its batch, a mixed batch's decode rows
 * included, and reads its own new rows from k_new / v_new, and a mixed batch
 * whose decode part runs on the persistent kernel at d = 128 runs as one
 * launch, the decode workgroups taking their new rows from k_new / v_new.
 * Elsewhere (persistent decode alone, prefill on fp8 pools, generic kernel)
 * the table append runs first. Same results, status bits and pool contents
 * as the two calls.
 * query_start_loc is required.
 * Replaces KVPool.write + paged_varlen_attention as called per layer in
 * MQA_Paged.forward_paged_batched (serving/paged_mqa.py:98-110).
 */
int pkv_paged_attention_append(void* out, float* lse, const void* q,
                               void* k_pool, void* v_pool,
                               int64_t num_blocks, int block_size,
                               const int32_t* block_tables, int max_blk,
                               const int32_t* seq_lens,
                               const int32_t* query_start_loc, int n_seq,
                               int n_tokens, int max_q_len, int max_kv_len,
                               int hq, int hkv, int d, float scale, int causal,
                               int part_tokens, int dtype, const void* k_new,
                               const void* v_new, const int32_t* start_pos,
                               void* workspace, size_t workspace_bytes,
                               int* status, void* stream);

/*
 * pkv_paged_attention without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, serving loops that forbid
 * hipMalloc): no counterpart in the reference. Same arguments, results and
 * status bits as pkv_paged_attention; its split-K partials and arrival
 * counters live in a 16 MiB scratch array the library holds on every device
 * it runs on, for the life of the process. A problem whose
 * pkv_attention_workspace_bytes() exceeds 16 MiB returns PKV_ERR_WORKSPACE.
 * The call allocates nothing. The array starts zero-filled (static storage
 * of the library's code object) and every call leaves its counter header at
 * zero; the first call on a device takes the array's address and zeroes that
 * header once more with a fill kernel on `stream` (under graph capture that
 * kernel becomes a node of the graph, run at every replay). All calls on one
 * device share that array: calls that overlap on one device (different
 * streams, or threads) race.
 */
int pkv_paged_attention_noalloc(void* out, float* lse, const void* q,
                                const void* k_pool, const void* v_pool,
                                int64_t num_blocks, int block_size,
                                const int32_t* block_tables, int max_blk,
                                const int32_t* seq_lens,
                                const int32_t* query_start_loc, int n_seq,
                                int n_tokens, int max_q_len, int max_kv_len,
                                int hq, int hkv, int d, float scale, int causal,
                                int part_tokens, int dtype, int* status,
                                void* stream);

/*
 * RMSNorm over rows of `dim` elements: y = (x * rsqrt(mean(x^2) + eps)) * w,
 * computed in fp32 and rounded once to `dtype` (weight has `dtype` too).
 * With `delta` non-null, the residual sum r = x + delta (rounded to `dtype`)
 * is written to residual_out (which may be x itself when x_stride == dim)
 * and normalised instead of x. x and delta rows are x_stride / delta_stride
 * elements apart; y and residual_out are contiguous [rows, dim].
 * Replaces RMSNorm.forward (models/rmsnorm.py:12-18) and the residual add
 * before it (serving/paged_model.py:20-29).
 */
int pkv_rms_norm(void* y, void* residual_out, const void* x, const void* delta,
                 const void* weight, int64_t rows, int dim, int64_t x_stride,
                 int64_t delta_stride, float eps, int dtype, void* stream);

/*
 * Rotary embedding of one step's token-major rows, interleaved (even, odd)
 * pairs, at absolute positions[t] (int32 [n_tokens]):
 *   out[2i]   = x[2i] * cos - x[2i+1] * sin
 *   out[2i+1] = x[2i] * sin + x[2i+1] * cos,  cos/sin = table[pos][i]
 * q rows (hq heads of d) start q_stride elements apart, k rows (hkv heads)
 * k_stride apart, so q, k and v may be column ranges of one fused
 * projection output; q_out [n_tokens, hq, d] and k_out [n_tokens, hkv, d]
 * are written contiguous. With v non-null, v's rows (v_stride apart) are
 * copied to a contiguous v_out [n_tokens, hkv, d] in the same launch.
 * cos_table / sin_table: fp32 [max_pos, d/2]; their values are rounded to
 * `dtype` and every product and sum is rounded to `dtype`, as in the
 * framework's element-wise evaluation (bit-exact in fp32: no fused
 * multiply-add). A position outside [0, max_pos) sets PKV_STATUS_BAD_POS in
 * `status` (nullable) and rotates by angle 0.
 * Replaces RoPE.forward_at / _rotate (models/rope.py:21-47) as applied in
 * MQA_Paged.forward_paged_batched (serving/paged_mqa.py:80-85).
 */
int pkv_rope(void* q_out, void* k_out, void* v_out, const void* q, const void* k,
             const void* v, int64_t q_stride, int64_t k_stride, int64_t v_stride,
             const int32_t* positions, const float* cos_table, const float* sin_table,
             int max_pos, int64_t n_tokens, int hq, int hkv, int d, int dtype,
             int* status, void* stream);

/*
 * SwiGLU gate: out = gate * sigmoid(gate) * up in fp32, rounded once to
 * `dtype`. gate / up rows are gate_stride / up_stride elements apart (they
 * may be the two halves of one fused projection output); out is contiguous
 * [rows, cols]. Replaces fused_swiglu (kernels/fused_swiglu/kernel.py:6-19,
 * :131-136).
 */
int pkv_silu_mul(void* out, const void* gate, const void* up, int64_t rows, int64_t cols,
                 int64_t gate_stride, int64_t up_stride, int dtype, void* stream);

/*
 * y = x W^T (+ bias) for few rows: x [m, k] (rows x_stride elements apart),
 * W [n, k] contiguous, bias [n] (nullable), y [m, n] contiguous; bf16 / fp16
 * / fp32 storage, fp32 accumulation, one rounding. k must be a multiple of
 * 32 and x rows 16-byte aligned (PKV_ERR_UNSUPPORTED otherwise). Built
 * for decode steps (m up to a few hundred): the workgroups split k, so the
 * weight is streamed by the whole chip. The sum order is fixed: results are
 * deterministic and identical across the pkv_linear* entry points.
 * Replaces nn.Linear for the out projection (serving/paged_mqa.py:112-113)
 * and down_proj (models/mlp.py:31-32).
 */
int pkv_linear(void* out, const void* x, const void* w, const void* bias, int64_t m, int64_t n,
               int64_t k, int64_t x_stride, int dtype, void* stream);

/*
 * SwiGLU MLP front half: W = [gate rows; up rows] [2n, k] (bias [2n],
 * nullable); out [m, n] = g * sigmoid(g) * u in fp32, rounded once, where g
 * and u are the gate / up projections rounded to dtype (bit-identical to
 * pkv_linear into [m, 2n] followed by pkv_silu_mul). Same requirements as
 * pkv_linear. Replaces gate_proj, up_proj and fused_swiglu
 * (models/mlp.py:24-30, kernels/fused_swiglu/kernel.py:6-19).
 */
int pkv_linear_swiglu(void* out, const void* x, const void* w_gate_up, const void* bias,
                      int64_t m, int64_t n, int64_t k, int64_t x_stride, int dtype,
                      void* stream);

/*
 * MQA_Paged's three projections and RoPE in one launch: W = [q rows; k rows;
 * v rows] [(hq + 2 hkv) d, k] (bias nullable); q_out [m, hq, d] and k_out
 * [m, hkv, d] receive the projections rotated at positions[m] (int32), v_out
 * [m, hkv, d] the value projection; all contiguous. Bit-identical to
 * pkv_linear into [m, (hq + 2 hkv) d] followed by pkv_rope on the three
 * column ranges (same tables, same status bit for positions outside
 * [0, max_pos)). Same requirements as pkv_linear. Replaces
 * serving/paged_mqa.py:76-85.
 */
int pkv_linear_rope_qkv(void* q_out, void* k_out, void* v_out, const void* x, const void* w_qkv,
                        const void* bias, int64_t m, int64_t k, int64_t x_stride,
                        const int32_t* positions, const float* cos_table,
                        const float* sin_table, int max_pos, int hq, int hkv, int d, int dtype,
                        int* status, void* stream);

/*
 * Residual projection: resid [m, n] (contiguous) += x W^T (+ bias), the
 * projection rounded to dtype first and the sum rounded (bit-identical to
 * pkv_linear followed by an element-wise add in dtype). Same requirements as
 * pkv_linear. Replaces the residual adds of PagedBlock.forward around the
 * out projection and down_proj (serving/paged_model.py:20-29).
 */
int pkv_linear_residual(void* resid, const void* x, const void* w, const void* bias, int64_t m,
                        int64_t n, int64_t k, int64_t x_stride, int dtype, void* stream);

/*
 * pkv_linear_swiglu of RMSNorm(x): the rows of x are normalised in the
 * kernel, (x * rsqrt(mean(x^2) + eps)) * norm_weight[k] in fp32 rounded to
 * dtype, before the products. Bit-identical to pkv_rms_norm followed by
 * pkv_linear_swiglu (both take the sum of squares in the same fixed order).
 * Needs k <= 1024 (PKV_ERR_UNSUPPORTED otherwise) and a 16-byte aligned
 * norm_weight; else as pkv_linear_swiglu. Replaces mlp_norm followed by
 * the MLP front half (serving/paged_model.py:28-29, models/rmsnorm.py:12-18,
 * models/mlp.py:24-30).
 */
int pkv_linear_swiglu_rmsnorm(void* out, const void* x, const void* norm_weight, float eps,
                              const void* w_gate_up, const void* bias, int64_t m, int64_t n,
                              int64_t k, int64_t x_stride, int dtype, void* stream);

/*
 * pkv_linear_rope_qkv of RMSNorm(x), normalised as in
 * pkv_linear_swiglu_rmsnorm (bit-identical to pkv_rms_norm followed by
 * pkv_linear_rope_qkv). Same requirements as those two. Replaces attn_norm
 * followed by serving/paged_mqa.py:76-85 (serving/paged_model.py:26-27).
 */
int pkv_linear_rope_qkv_rmsnorm(void* q_out, void* k_out, void* v_out, const void* x,
                                const void* norm_weight, float eps, const void* w_qkv,
                                const void* bias, int64_t m, int64_t k, int64_t x_stride,
                                const int32_t* positions, const float* cos_table,
                                const float* sin_table, int max_pos, int hq, int hkv, int d,
                                int dtype, int* status, void* stream);

/*
 * Greedy token choice: ids[r] (int64) = the index of the largest of the
 * `vocab` logits of row r (rows row_stride elements apart, dtype F32 / F16 /
 * BF16). Same result as the framework's argmax: the first index holding the
 * maximum, and a NaN counts as larger than any number (the first NaN
 * wins). Replaces logits.argmax as taken per sequence by the greedy loops
 * (serving/generation.py:77, :88, :132, :142) and greedy()
 * (sampling.py:5-137). With a workspace of at least
 * pkv_argmax_workspace_bytes(rows, vocab, dtype) bytes (256-byte aligned,
 * zero-filled before its first use; every call leaves it zero-filled) a
 * batch of fewer than 512 rows is split over several workgroups per row;
 * without one (NULL), one workgroup per row. Same ids either way. Calls
 * that overlap on one workspace race.
 */
int pkv_argmax_rows(int64_t* ids, const void* logits, int64_t rows, int64_t vocab,
                    int64_t row_stride, int dtype, void* workspace,
                    size_t workspace_bytes, void* stream);

/*
 * Sampling step of the scheduler (sampling.py:94-137, sample()): per row of
 * logits [rows, vocab] (row_stride elements apart, fp32 / bf16 / fp16),
 * y = logits / temperature in fp32; keep every y >= the top_k-th largest
 * (ties kept, as apply_top_k); sort the kept values descending (ties by
 * ascending index) and keep the prefix whose softmax mass before each token
 * is at most top_p (the first always, as apply_top_p); renormalise; ids[r]
 * (int64) = the first kept index, in ascending vocabulary order, whose
 * cumulative probability exceeds uniforms[r] * total (uniforms: fp32 in
 * [0, 1), one per row, the caller's random numbers). 1 <= top_k <= 64
 * (PKV_ERR_UNSUPPORTED otherwise), 0 < top_p <= 1, temperature finite > 0.
 * Status bits (ids[r] = -1 for the row): PKV_STATUS_NONFINITE (a NaN or
 * infinite logit), PKV_STATUS_BAD_DISTRIBUTION (y overflowed),
 * PKV_STATUS_SAMPLE_OVERFLOW (more than 1024 values tie or crowd at the
 * threshold's neighbourhood; sample such a row another way).
 */
int pkv_sample_rows(int64_t* ids, const void* logits, int64_t rows, int64_t vocab,
                    int64_t row_stride, float temperature, int top_k, float top_p,
                    const float* uniforms, int dtype, int* status, void* stream);

/*
 * Workspace bytes of pkv_argmax_rows for `rows` rows of `vocab` logits of
 * `dtype` (no counterpart in the reference): per-row arrival counters and
 * key words, one 128-byte line each; 0 when those rows are not split.
 */
size_t pkv_argmax_workspace_bytes(int64_t rows, int64_t vocab, int dtype);

/*
 * Measurement helper, no counterpart in the reference: reads `bytes` bytes at
 * p (16-byte aligned, a multiple of 16) once with 16-byte non-temporal loads
 * from `grid` workgroups of 256 threads and writes nothing (sink, nullable,
 * is written only on an impossible checksum). The benchmark times it on the
 * same byte counts as the attention kernels to report the device's plain
 * HBM read rate beside theirs.
 */
int pkv_stream_read(const void* p, int64_t bytes, unsigned* sink, int grid, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PAGEDKV_H */
