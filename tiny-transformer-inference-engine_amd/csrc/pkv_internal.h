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

// fp8 pools: the PKV_KV_FP8 flag of a dtype argument, and the element type
// of Q / out / appended rows without it.
inline bool dtype_kv8(int dtype) { return (dtype & PKV_KV_FP8) != 0; }
inline int dtype_base(int dtype) { return dtype & ~PKV_KV_FP8; }

// Nearest fp8 e4m3 value (OCP, torch.float8_e4m3fn: bias 7, 3 mantissa bits,
// no infinities, S.1111.111 = NaN, largest finite 448) of x: ties to even;
// magnitudes above 464 (those that round past 448: from 480 on by the first
// test, between 464 and 480 by the rounding carry into S.1111.111),
// infinities and NaN give NaN (0x7F with the sign bit); the bytes torch's
// conversion gives. Values below 2^-6 are multiples of 2^-9.
__device__ __forceinline__ unsigned f32_to_e4m3(float x) {
  unsigned b = __float_as_uint(x);
  const unsigned sign = (b >> 24) & 0x80u;
  b &= 0x7fffffffu;
  if (b >= 0x43F00000u) return sign | 0x7Fu;
  if (b < 0x3C800000u) return sign | (unsigned)(int)rintf(__uint_as_float(b) * 512.f);
  b += 0x7FFFFu + ((b >> 20) & 1u);  // 23 mantissa bits to 3, ties to even
  return sign | ((((b >> 23) - 120u) << 3) | ((b >> 20) & 7u));
}

// x as an fp32 register value the compiler must produce before using it.
// Without it the backend may fold an fp32 operation and the conversion to
// fp16 that follows into one mixed-precision instruction (v_fma_mix*) that
// rounds once, where the framework's element-wise ops round to fp32 and then
// to fp16; the two differ in rare near-tie cases.
__device__ __forceinline__ float fp32_value(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

// SwiGLU gate of (already rounded) gate / up values, g * sigmoid(g) * u in
// fp32, the arithmetic of kernels/fused_swiglu/kernel.py:17-18. Contraction
// is off so that every kernel evaluating it (the stand-alone gate and the
// projection epilogue) gives the same bits.
__device__ __forceinline__ float swiglu_gate(float g, float u) {
#pragma clang fp contract(off)
  const float sig = 1.f / (1.f + expf(-g));
  return fp32_value(g * sig * u);
}

// RMSNorm's sum of squares over a row of k elements (k a multiple of 32, at
// most kNormCanonMax) is taken in one fixed order, shared by the
// stand-alone RMSNorm kernel and the projection kernel's fused norm (whose
// K split over kNormSplit wavefronts defines it): the 32-element steps are
// cut into kNormSplit contiguous ranges of ceil(steps / kNormSplit) steps;
// in each range the four 8-element groups of a step are summed separately,
// step by step, element by element, from 0; the groups are combined as
// (g0 + g1) + (g2 + g3) and the ranges added in order, from 0.
constexpr int kNormSplit = 8;
constexpr int kNormCanonMax = 8192;

// ---------------------------------------------------------------------------
// Append / gather (append.hip)
// ---------------------------------------------------------------------------
int launch_append(void* k_pool, void* v_pool, int64_t pool_slots,
                  const void* k_new, const void* v_new, const int64_t* slots,
                  int64_t n_tok, int64_t row_bytes, int* status,
                  hipStream_t stream);
// The same into fp8 pools: rows of row_elems values of src_dtype, each
// rounded to fp8 (f32_to_e4m3).
int launch_append_fp8(void* k_pool, void* v_pool, int64_t pool_slots, const void* k_new,
                      const void* v_new, const int64_t* slots, int64_t n_tok,
                      int64_t row_elems, int src_dtype, int* status, hipStream_t stream);

int launch_append_from_table(void* k_pool, void* v_pool, int64_t num_blocks,
                             int bs_shift, const void* k_new,
                             const void* v_new, const int32_t* block_tables,
                             int max_blk, const int32_t* qloc,
                             const int32_t* start_pos, int n_seq,
                             int64_t n_tok, int64_t row_bytes, int min_qlen,
                             int* status, hipStream_t stream);

int launch_append_from_table_fp8(void* k_pool, void* v_pool, int64_t num_blocks, int bs_shift,
                                 const void* k_new, const void* v_new,
                                 const int32_t* block_tables, int max_blk, const int32_t* qloc,
                                 const int32_t* start_pos, int n_seq, int64_t n_tok,
                                 int64_t row_elems, int src_dtype, int min_qlen, int* status,
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
  int n_tokens;  // T: rows of q / out
  int hq;
  int hkv;
  int group;  // hq / hkv
  int d;
  float scale_log2;  // softmax scale * log2(e)
  int causal;
  int kv8;  // the pools hold fp8 e4m3 (q, out, k_new, v_new keep the 16-bit type)
  // which sequences this launch handles (a mixed batch is split between the
  // decode and the prefill kernels): 0 every one, 1 only those with one
  // query token, 2 only those with more
  int qfilter;
  int part_tokens;   // split-K partition length (multiple of 32)
  int parts_max;     // partitions per (sequence, kv head, row tile) in grid
  int tiles_max;     // row tiles per (sequence, kv head) in grid
  float* ws_o;       // [units][ROWS][d] unnormalised partial outputs
  float* ws_ml;      // [units][ROWS][2] (running max (log2 units), sum)
  int* status;
  // fused append (partition decode kernel, MFMA prefill kernel and the
  // decode shares of the one-launch mixed kernel; all null otherwise): the
  // K/V rows of sequence s's query tokens go to positions new_pos[s],
  // new_pos[s] + 1, ... of its table, and the attention uses them from
  // k_new / v_new
  const void* k_new;
  const void* v_new;
  const int32_t* new_pos;
  // split-K partition kernel: per-(sequence, kv head) arrival counters
  // (workspace header, zero between calls); when set, the last partition
  // of a sequence to finish merges the partials itself and no merge kernel
  // runs
  int* merge_ctr;
};

// Rows ((query token, head) pairs of one kv head) per tile of the generic
// kernel.
constexpr int kGenRows = 32;
// The MFMA prefill kernel takes the append fused for batches of at most
// this many sequences (one block of its query_start_loc scan).
constexpr int kPrefillFuseMaxSeq = 512;
constexpr int kChunk = 32;  // kv tokens staged per iteration

// Workspace layout: the first kWsCounterBytes are a header. Its first
// kWsCtrBytes hold the partition kernel's per-(sequence, kv head) arrival
// counters: they must be zero before the first call on a workspace, and
// every call leaves them zero. The rest holds the persistent kernel's
// per-(sequence, kv head) records (which workgroups hold partials of it,
// and an arrival counter with the same zero-in, zero-out rule). Partials
// start after the header.
constexpr size_t kWsCounterBytes = 256 * 1024;
constexpr size_t kWsCtrBytes = 8 * 1024;
constexpr int kMaxCounters = (int)((kWsCounterBytes - kWsCtrBytes) / sizeof(int4));
constexpr int kSkMaxWg = 512;  // workgroups of the persistent kernel, at most
// A sequence's fixed cost in the persistent kernel (Q load, table slice,
// wavefront merge, output or partial write) measured in 32-token chunks of
// a 4-wavefront workgroup's streaming time (scaled by the launch to its
// workgroup size). At head dim 128 the launch uses the measured optimum of
// its workgroup shape instead (kSkSegCost128).
constexpr int kSkSegCost = 5;
// At head dim 128, one workgroup per CU: 4 wavefronts 9 (config 5: 3 / 5 /
// 7 / 9 / 11 / 13 / 16 gave 35.7 / 33.8 / 33.0 / 32.9 / 33.2 / 33.6 / 34.2
// us), 8 wavefronts 10 (8, 12, 14 and 20 slower).
constexpr int kSkSegCost128(int waves) { return waves == 4 ? 9 : 10; }
// Context bound from which part_tokens = 0 selects the persistent kernel.
constexpr int kSkAutoKv = 4096;
// A sequence's fixed cost in the wavefront-specialised persistent kernel
// (decode_ws.hip), in 32-token chunks of a workgroup's streaming time.
constexpr int kWsSegCost = 4;

struct SkArgs {
  int n_wg;         // workgroups launched
  int seg_cost;     // overhead of one sequence in chunk units (share balance)
  int4* recs;       // [n_seq * hkv] per-pair records: .w is the arrival counter
  uint16_t* part_o; // [n_wg][2][G][D] partial outputs, normalised (O / sum),
                    // in the kernel's 16-bit element type
  float* part_ml;   // [n_wg][2][G][2] partial (max, sum)
};

// Workspace of the persistent kernel: the record header, then the fp16
// partial outputs and the fp32 (max, sum) pairs of two slots per workgroup.
inline size_t sk_workspace_bytes(int group, int d) {
  return kWsCounterBytes + (size_t)kSkMaxWg * 2 * group * ((size_t)d * 2 + 2 * 4);
}

struct AttnPlan {
  int kind;        // 0 = generic rows kernel, 1 = MFMA partition kernel,
                   // 2 = MFMA persistent kernel, 3 = MFMA prefill kernel,
                   // 4 = small-group decode kernel (decode_small.hip)
  bool ws;         // kind 2: the wavefront-specialised form where it applies
  int rows;        // rows per tile of the chosen kernel
  int part_tokens;
  int parts_max;
  int tiles_max;
  size_t ws_bytes;
};

// Per-(sequence, kv head, row tile) geometry shared by every attention kernel
// and the split-K merge; all of them must derive the same partition count.
__device__ __forceinline__ int dceil_div(int a, int b) { return (a + b - 1) / b; }

struct TileGeom {
  int q_begin, q_len, rows_here, kv_len, ctx, kv_limit, part_len, nparts;
};

// Loads through the scalar data cache: only for metadata no kernel of the
// library writes (seq_lens, query_start_loc, block tables) or that an
// earlier kernel wrote (the cache is invalidated at every launch), at an
// index uniform across the wavefront. Unlike a vector load, waiting for one
// does not wait for the wavefront's outstanding vector stores.
typedef const __attribute__((address_space(4))) int32_t scalar_i32;
__device__ __forceinline__ int ld_meta(const int32_t* p, int64_t i) {
  return ((scalar_i32*)p)[i];
}

// Device-scope coherent accesses for data exchanged between workgroups
// within one launch: relaxed agent-scope atomic stores (global_store with the
// device scope bits: written through the XCD's L2), and a relaxed fetch-add
// whose address the compiler cannot prove uniform, so it is issued as it
// stands (not rewritten into a wavefront-wide aggregate whose result is
// waited for at once) and as a global (not flat) access.
__device__ __forceinline__ void st_agent64(void* p, uint64_t x) {
  __hip_atomic_store(static_cast<uint64_t*>(p), x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
typedef __attribute__((address_space(1))) int global_i32;
__device__ __forceinline__ int fetch_add_agent(int* p, int x) {
  global_i32* g = (global_i32*)p;
  asm volatile("" : "+v"(g));
  return __hip_atomic_fetch_add(g, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The value of lane (lane ^ S) of the wavefront, by VALU data movement:
// DPP quad permutations (S = 1, 2), DPP row shifts selected by the lane bit
// (S = 4, 8), and gfx950's cross-row swaps (S = 16, 32), instead of LDS
// permutes.
template <int S>
__device__ __forceinline__ float lane_xor(float v) {
  const int x = __float_as_int(v);
  const int lane = threadIdx.x & 63;
  if constexpr (S == 1) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
  } else if constexpr (S == 2) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
  } else if constexpr (S == 4 || S == 8) {
    const int up = __builtin_amdgcn_mov_dpp(x, 0x100 + S, 0xF, 0xF, true);  // row_shl: lane + S
    const int dn = __builtin_amdgcn_mov_dpp(x, 0x110 + S, 0xF, 0xF, true);  // row_shr: lane - S
    return __int_as_float((lane & S) ? dn : up);
  } else if constexpr (S == 16) {
    const auto a = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
    return __uint_as_float(((lane >> 4) & 1) ? a[0] : a[1]);
  } else {
    static_assert(S == 32, "xor distance");
    const auto a = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
    return __uint_as_float((lane & 32) ? a[0] : a[1]);
  }
}

// Counters of the split-K partition kernel's in-kernel merge, one per
// (sequence, kv head) pair, at the start of the header.
constexpr int kMergeCtrOff = 0;
constexpr int kMergeCtrMax = (int)(kWsCtrBytes / sizeof(int)) - kMergeCtrOff;

__device__ __forceinline__ bool tile_geom(const AttnArgs& a, int s, int tile,
                                          int rows_per_tile, TileGeom& g) {
  // s is uniform (it comes from the block index) in every caller
  g.q_begin = a.qloc ? ld_meta(a.qloc, s) : s;
  g.q_len = a.qloc ? ld_meta(a.qloc, s + 1) - g.q_begin : 1;
  if (g.q_len <= 0) return false;
  if ((a.qfilter == 1 && g.q_len != 1) || (a.qfilter == 2 && g.q_len == 1)) return false;
  if (g.q_begin < 0 || g.q_begin + g.q_len > a.n_tokens) {
    // malformed query_start_loc: never index q / out outside [0, T)
    if (a.status && tile == 0) atomicOr(a.status, PKV_STATUS_BAD_QLOC);
    return false;
  }
  const int rows_total = g.q_len * a.group;
  const int r0 = tile * rows_per_tile;
  if (r0 >= rows_total) return false;
  g.rows_here = min(rows_per_tile, rows_total - r0);
  int kv_len = ld_meta(a.seq_lens, s);
  const int cap = a.max_blk << a.bs_shift;
  kv_len = kv_len < cap ? kv_len : cap;
  g.kv_len = kv_len > 0 ? kv_len : 0;
  g.ctx = a.causal ? max(g.kv_len - g.q_len, 0) : 0;
  g.kv_limit = g.kv_len;
  if (a.causal) {
    const int i_last = (r0 + g.rows_here - 1) / a.group;
    g.kv_limit = min(g.kv_limit, g.ctx + i_last + 1);
  }
  // A sequence longer than the planned bound still gets every key: its
  // partitions grow so that their count never exceeds the grid.
  int plen = a.part_tokens;
  if (dceil_div(g.kv_limit, plen) > a.parts_max)
    plen = dceil_div(dceil_div(g.kv_limit, a.parts_max), kChunk) * kChunk;
  g.part_len = plen;
  g.nparts = max(1, dceil_div(g.kv_limit, plen));
  return true;
}


// decode_small.hip: one query token per sequence, 1 / 2 / 4 / 8 query heads
// per kv head, head dim 32 / 64 / 128, fp32 / bf16 / fp16 pools.
bool decode_small_supported(int dtype, int max_q_len, int group, int d);
int launch_decode_small(const AttnArgs& a, const AttnPlan& p, int dtype, hipStream_t stream);

AttnPlan plan_attention(int n_seq, int max_q_len, int hq, int hkv, int d,
                        int max_blk, int block_size, int max_kv_len,
                        int part_tokens, int dtype);

// A batch that may mix single-token (decode) and multi-token (prefill)
// queries is split when the decode sequences can take an MFMA decode
// kernel: `dec` handles the sequences with one query token, `pre` the
// others, launched one after the other on the stream and sharing the
// workspace (ws_bytes is the larger need). Otherwise `dec` is the one plan.
struct AttnSplit {
  bool mixed;
  AttnPlan dec;
  AttnPlan pre;
  size_t ws_bytes;
};
AttnSplit plan_split(int n_seq, int max_q_len, int hq, int hkv, int d, int max_blk,
                     int block_size, int max_kv_len, int part_tokens, int dtype,
                     bool has_qloc);

int launch_attention(const AttnArgs& a, const AttnPlan& plan, int dtype,
                     hipStream_t stream);

// MFMA decode kernel (decode_mfma.hip): bf16/fp16, one query per sequence,
// group 16 or 32, head dim 64 or 128.
bool decode_mfma_supported(int dtype, int max_q_len, int group, int d);
bool pool_needs_off64(const AttnArgs& a);

// MFMA prefill / chunked-prefill kernel (prefill_mfma.hip): bf16/fp16, query
// runs of any length (query_start_loc required), group 16 or 32, head dim
// 64 or 128.
bool prefill_mfma_supported(int dtype, int group, int d);
int launch_prefill_mfma(const AttnArgs& a, int dtype, hipStream_t stream);
int launch_decode_mfma(const AttnArgs& a, const AttnPlan& plan, int dtype,
                       hipStream_t stream);
// Persistent MFMA decode kernel (decode_sk.hip), same coverage.
// Workgroups the persistent kernel launches for this head shape.
int sk_workgroups(int d, int group);
int launch_decode_sk(const AttnArgs& a, const SkArgs& k, int dtype, hipStream_t stream);
// A mixed batch in one launch (decode_sk.hip): the persistent decode shares
// (ad, qfilter 1) and the MFMA prefill pairs with the fused append (ap,
// qfilter 2) as workgroups of one grid. Supported for bf16/fp16 16-bit
// pools, head dim 128, 16 or 32 query heads per kv head, pools addressed
// with 32-bit offsets; ad and ap carry k_new / v_new / new_pos.
bool mixed_sk_supported(const AttnArgs& ap, int dtype);
int launch_mixed_sk(const AttnArgs& ad, const SkArgs& k, const AttnArgs& ap, int dtype,
                    hipStream_t stream);
// Wavefront-specialised persistent decode kernel (decode_ws.hip): producer
// wavefronts stream K/V into an LDS ring by LDS-DMA, consumer wavefronts
// compute. Decode batches (qfilter 0, no fused append) with bf16/fp16
// queries and 16-bit pools, head dim 128, 16 or 32 query heads per kv head,
// block size >= 16.
int ws_workgroups();
bool decode_ws_supported(const AttnArgs& a, int dtype);
int launch_decode_ws(const AttnArgs& a, const SkArgs& k, int dtype, hipStream_t stream);
// The persistent kernel's arguments for launch view a (workspace layout:
// arrival records after the counter header, then the partials).
SkArgs sk_args_for(const AttnArgs& a);
// launch_attention for a mixed batch whose decode part is planned on the
// persistent kernel and whose prefill part takes the fused append, when
// mixed_sk_supported(ap): one launch.
int launch_attention_mixed(const AttnArgs& ad, const AttnArgs& ap, int dtype,
                           hipStream_t stream);
// CUs of the current device (cached; 256 when no device is visible).
int device_cu_count();

}  // namespace pkv
