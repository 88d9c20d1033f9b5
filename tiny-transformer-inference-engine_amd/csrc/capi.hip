// C ABI of libpagedkv.so (declared in include/pagedkv.h): argument
// validation mirroring the reference's checks, then dispatch to the kernels.
//
// Validation follows check_paged_inputs (kernels/pagedattn/pagedattn.cu:867-895)
// and paged_varlen_attention (serving/fake_paged_attn.py:171-198): head dim a
// multiple of 8 and <= 256, hq a multiple of hkv, power-of-two block size.
// Unlike the reference, f32 and bf16 are computed natively (the reference
// casts everything to fp16, fake_paged_attn.py:208-215).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "pkv_internal.h"

namespace pkv {

static thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(PKV_ERR_HIP, "%s launch failed: %s", what, hipGetErrorString(e));
  return PKV_OK;
}

static bool valid_dtype(int dtype) {
  return dtype == PKV_DTYPE_F32 || dtype == PKV_DTYPE_F16 ||
         dtype == PKV_DTYPE_BF16;
}

// A dtype argument: one PKV_DTYPE_* value, optionally with PKV_KV_FP8.
static bool valid_dtype_arg(int dtype) { return valid_dtype(dtype_base(dtype)); }

static int log2_exact(int64_t v) {
  if (v <= 0 || (v & (v - 1)) != 0) return -1;
  int s = 0;
  while ((int64_t(1) << s) < v) ++s;
  return s;
}

}  // namespace pkv

using namespace pkv;

extern "C" {

int pkv_version(void) { return PKV_VERSION; }

const char* pkv_last_error(void) { return g_err; }

int pkv_append(void* k_pool, void* v_pool, int64_t pool_slots,
               const void* k_new, const void* v_new,
               const int64_t* slot_mapping, int64_t n_tok, int64_t row_elems,
               int dtype, int* status, void* stream) {
  g_err[0] = 0;
  if (!valid_dtype_arg(dtype)) return fail(PKV_ERR_INVALID, "unknown dtype %d", dtype);
  if (n_tok < 0 || row_elems <= 0 || pool_slots < 0)
    return fail(PKV_ERR_INVALID, "bad sizes n_tok=%lld row_elems=%lld pool_slots=%lld",
                (long long)n_tok, (long long)row_elems, (long long)pool_slots);
  if (n_tok == 0) return PKV_OK;
  if (!k_pool || !v_pool || !k_new || !v_new || !slot_mapping)
    return fail(PKV_ERR_INVALID, "null pointer argument");
  if (dtype_kv8(dtype))
    return launch_append_fp8(k_pool, v_pool, pool_slots, k_new, v_new, slot_mapping, n_tok,
                             row_elems, dtype_base(dtype), status, (hipStream_t)stream);
  return launch_append(k_pool, v_pool, pool_slots, k_new, v_new, slot_mapping,
                       n_tok, row_elems * elem_bytes(dtype), status,
                       (hipStream_t)stream);
}

int pkv_append_from_table(void* k_pool, void* v_pool, int64_t num_blocks,
                          int block_size, const void* k_new, const void* v_new,
                          const int32_t* block_tables, int max_blk,
                          const int32_t* query_start_loc,
                          const int32_t* start_pos, int n_seq, int64_t n_tok,
                          int64_t row_elems, int dtype, int* status,
                          void* stream) {
  g_err[0] = 0;
  if (!valid_dtype_arg(dtype)) return fail(PKV_ERR_INVALID, "unknown dtype %d", dtype);
  const int bs_shift = log2_exact(block_size);
  if (bs_shift < 0)
    return fail(PKV_ERR_INVALID, "blocksize %d must be a power of two", block_size);
  if (n_tok < 0 || n_seq < 0 || row_elems <= 0 || max_blk < 0 || num_blocks < 0)
    return fail(PKV_ERR_INVALID, "bad sizes");
  if (n_tok == 0 || n_seq == 0) return PKV_OK;
  if (!k_pool || !v_pool || !k_new || !v_new || !block_tables ||
      !query_start_loc || !start_pos)
    return fail(PKV_ERR_INVALID, "null pointer argument");
  if (dtype_kv8(dtype))
    return launch_append_from_table_fp8(
        k_pool, v_pool, num_blocks, bs_shift, k_new, v_new, block_tables, max_blk,
        query_start_loc, start_pos, n_seq, n_tok, row_elems, dtype_base(dtype), 0, status,
        (hipStream_t)stream);
  return launch_append_from_table(
      k_pool, v_pool, num_blocks, bs_shift, k_new, v_new, block_tables,
      max_blk, query_start_loc, start_pos, n_seq, n_tok,
      row_elems * elem_bytes(dtype), 0, status, (hipStream_t)stream);
}

int pkv_gather(void* k_out, void* v_out, const void* k_pool,
               const void* v_pool, int64_t num_blocks, int block_size,
               const int32_t* block_table, int n_blocks, int seq_len,
               int64_t row_elems, int dtype, int* status, void* stream) {
  g_err[0] = 0;
  if (!valid_dtype_arg(dtype)) return fail(PKV_ERR_INVALID, "unknown dtype %d", dtype);
  const int bs_shift = log2_exact(block_size);
  if (bs_shift < 0)
    return fail(PKV_ERR_INVALID, "blocksize %d must be a power of two", block_size);
  if (seq_len < 0 || n_blocks < 0 || row_elems <= 0)
    return fail(PKV_ERR_INVALID, "bad sizes");
  if ((int64_t)seq_len > (int64_t)n_blocks * block_size)
    return fail(PKV_ERR_INVALID,
                "seq_len=%d exceeds capacity of block_table (%lld)", seq_len,
                (long long)n_blocks * block_size);
  if (seq_len == 0) return PKV_OK;
  if (!k_out || !v_out || !k_pool || !v_pool || !block_table)
    return fail(PKV_ERR_INVALID, "null pointer argument");
  return launch_gather(k_out, v_out, k_pool, v_pool, num_blocks, bs_shift,
                       block_table, n_blocks, seq_len,
                       row_elems * (dtype_kv8(dtype) ? 1 : elem_bytes(dtype_base(dtype))), status,
                       (hipStream_t)stream);
}

size_t pkv_attention_workspace_bytes(int n_seq, int max_q_len, int hq, int hkv,
                                     int d, int max_blk, int block_size,
                                     int max_kv_len, int part_tokens,
                                     int dtype) {
  if (n_seq <= 0 || max_q_len <= 0 || hkv <= 0 || hq <= 0 || hq % hkv != 0 ||
      part_tokens < PKV_PART_STREAM)
    return 0;
  // query_start_loc is required whenever max_q_len > 1
  return plan_split(n_seq, max_q_len, hq, hkv, d, max_blk, block_size, max_kv_len,
                    part_tokens, dtype, max_q_len > 1)
      .ws_bytes;
}

}  // extern "C"

namespace {

// Shared body of pkv_paged_attention (k_new == NULL) and
// pkv_paged_attention_append.
int attention_impl(void* out, float* lse, const void* q, const void* k_pool,
                   const void* v_pool, int64_t num_blocks, int block_size,
                   const int32_t* block_tables, int max_blk, const int32_t* seq_lens,
                   const int32_t* query_start_loc, int n_seq, int n_tokens, int max_q_len,
                   int max_kv_len, int hq, int hkv, int d, float scale, int causal,
                   int part_tokens, int dtype, void* workspace, size_t workspace_bytes,
                   int* status, void* stream, const void* k_new, const void* v_new,
                   const int32_t* start_pos) {
  g_err[0] = 0;
  if (!valid_dtype_arg(dtype)) return fail(PKV_ERR_INVALID, "unknown dtype %d", dtype);
  const bool kv8 = dtype_kv8(dtype);
  const int qdtype = dtype_base(dtype);  // Q, out, k_new / v_new
  if (kv8 && qdtype == PKV_DTYPE_F32)
    return fail(PKV_ERR_UNSUPPORTED, "fp8 KV pools need bf16 or f16 queries");
  if (hkv <= 0 || hq <= 0 || hq % hkv != 0)
    return fail(PKV_ERR_INVALID, "Hq (%d) must be a multiple of Hkv (%d)", hq, hkv);
  if (d <= 0 || d % 8 != 0)
    return fail(PKV_ERR_INVALID, "head_dim %d must be a multiple of 8", d);
  if (d > 256) return fail(PKV_ERR_UNSUPPORTED, "head dim > 256 not supported");
  const int bs_shift = log2_exact(block_size);
  if (bs_shift < 0)
    return fail(PKV_ERR_INVALID, "blocksize %d must be a power of two", block_size);
  if (n_seq < 0 || max_blk < 0 || num_blocks < 0 || max_q_len < 0 || n_tokens < 0)
    return fail(PKV_ERR_INVALID, "bad sizes");
  if (part_tokens < PKV_PART_STREAM)
    return fail(PKV_ERR_INVALID, "part_tokens %d: the negative values are PKV_PART_PERSISTENT, "
                "PKV_PART_STATIC and PKV_PART_STREAM", part_tokens);
  if (!query_start_loc && n_tokens != n_seq)
    return fail(PKV_ERR_INVALID, "without query_start_loc, n_tokens (%d) must equal n_seq (%d)",
                n_tokens, n_seq);
  if (n_seq == 0 || max_q_len == 0 || n_tokens == 0) return PKV_OK;
  if (!out || !q || !k_pool || !v_pool || !seq_lens || (max_blk > 0 && !block_tables))
    return fail(PKV_ERR_INVALID, "null pointer argument");
  if (!query_start_loc && max_q_len != 1)
    return fail(PKV_ERR_INVALID, "query_start_loc may be NULL only when max_q_len == 1");
  const AttnSplit sp = plan_split(n_seq, max_q_len, hq, hkv, d, max_blk, block_size,
                                  max_kv_len, part_tokens, dtype, query_start_loc != nullptr);
  if (sp.ws_bytes > 0 && (!workspace || workspace_bytes < sp.ws_bytes))
    return fail(PKV_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given",
                sp.ws_bytes, workspace ? workspace_bytes : (size_t)0);
  const float sc = scale > 0.f ? scale : 1.f / sqrtf((float)d);
  AttnArgs base{};
  base.out = out;
  base.lse = lse;
  base.q = q;
  base.k_pool = k_pool;
  base.v_pool = v_pool;
  base.block_tables = block_tables;
  base.seq_lens = seq_lens;
  base.qloc = query_start_loc;
  base.num_blocks = num_blocks;
  base.bs_shift = bs_shift;
  base.max_blk = max_blk;
  base.n_seq = n_seq;
  base.n_tokens = n_tokens;
  base.hq = hq;
  base.hkv = hkv;
  base.group = hq / hkv;
  base.d = d;
  base.scale_log2 = sc * 1.4426950408889634f;
  base.causal = causal ? 1 : 0;
  base.kv8 = kv8 ? 1 : 0;
  base.status = status;
  // one launch's view: its plan's geometry and workspace layout (partials
  // live after the record region, see kWsCounterBytes)
  auto args_for = [&](const AttnPlan& plan, int qfilter) {
    AttnArgs a = base;
    a.qfilter = qfilter;
    a.part_tokens = plan.part_tokens;
    a.parts_max = plan.parts_max;
    a.tiles_max = plan.tiles_max;
    float* ws = plan.ws_bytes ? reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                                         kWsCounterBytes)
                              : nullptr;
    const size_t units = (size_t)n_seq * hkv * plan.tiles_max * plan.parts_max;
    a.ws_o = ws;
    a.ws_ml = ws ? ws + units * plan.rows * (size_t)d : nullptr;
    return a;
  };
  const int64_t row_bytes = (int64_t)hkv * d * elem_bytes(qdtype);
  // the table append of rows the decode kernel does not take fused
  auto append_rows = [&](int min_qlen) {
    if (kv8)
      return launch_append_from_table_fp8(
          const_cast<void*>(k_pool), const_cast<void*>(v_pool), num_blocks, bs_shift, k_new,
          v_new, block_tables, max_blk, query_start_loc, start_pos, n_seq, n_tokens,
          (int64_t)hkv * d, qdtype, min_qlen, status, (hipStream_t)stream);
    return launch_append_from_table(
        const_cast<void*>(k_pool), const_cast<void*>(v_pool), num_blocks, bs_shift, k_new,
        v_new, block_tables, max_blk, query_start_loc, start_pos, n_seq, n_tokens, row_bytes,
        min_qlen, status, (hipStream_t)stream);
  };
  // The split-K partition and small-group decode kernels and the MFMA
  // prefill kernel (16-bit pools) take the append fused: the decode kernels
  // the one row of each sequence, the prefill kernel every row of the batch (each workgroup a
  // share of the rows; its attention takes its own sequences' new rows from
  // k_new / v_new). For the persistent decode kernel the fused form measured
  // slower than a separate append launch (register pressure at 32 heads x
  // 128 dims), and the generic kernel reads every row from the pool.
  const bool fuse_pre = k_new && !kv8 && n_seq <= kPrefillFuseMaxSeq;
  if (!sp.mixed) {
    AttnArgs a = args_for(sp.dec, 0);
    if (k_new) {
      if (sp.dec.kind == 1 || sp.dec.kind == 4 || (sp.dec.kind == 3 && fuse_pre)) {
        a.k_new = k_new;
        a.v_new = v_new;
        a.new_pos = start_pos;
      } else {
        // append, then attend
        const int rc = append_rows(0);
        if (rc != PKV_OK) return rc;
      }
    }
    return launch_attention(a, sp.dec, qdtype, (hipStream_t)stream);
  }
  // mixed batch: the decode sequences on an MFMA decode kernel, the
  // prefill sequences on the prefill kernel. With the fused append and the
  // persistent decode kernel (head dim 128) both run in one launch, the
  // decode shares taking their new rows from k_new / v_new; with the fused
  // append otherwise the prefill kernel runs first and appends every row
  // (the decode kernel after it reads them from the pool); without it the
  // prefill rows (and the decode rows unless the decode kernel takes them
  // fused) are appended first and the decode kernel runs first.
  AttnArgs ad = args_for(sp.dec, 1);
  AttnArgs ap = args_for(sp.pre, 2);
  if (fuse_pre && sp.pre.kind == 3) {
    ap.k_new = k_new;
    ap.v_new = v_new;
    ap.new_pos = start_pos;
    if (sp.dec.kind == 2 && mixed_sk_supported(ap, qdtype)) {
      ad.k_new = k_new;
      ad.v_new = v_new;
      ad.new_pos = start_pos;
      return launch_attention_mixed(ad, ap, qdtype, (hipStream_t)stream);
    }
    const int rc = launch_attention(ap, sp.pre, qdtype, (hipStream_t)stream);
    if (rc != PKV_OK) return rc;
    return launch_attention(ad, sp.dec, qdtype, (hipStream_t)stream);
  }
  if (k_new) {
    const bool fuse = sp.dec.kind == 1;
    const int rc = append_rows(fuse ? 2 : 0);
    if (rc != PKV_OK) return rc;
    if (fuse) {
      ad.k_new = k_new;
      ad.v_new = v_new;
      ad.new_pos = start_pos;
    }
  }
  int rc = launch_attention(ad, sp.dec, qdtype, (hipStream_t)stream);
  if (rc != PKV_OK) return rc;
  return launch_attention(ap, sp.pre, qdtype, (hipStream_t)stream);
}

// Scratch of pkv_paged_attention_noalloc: one array per device, in the
// library's code object (no allocation at call time), zero-filled when the
// code object is loaded. Its first kWsCounterBytes are the counter header,
// which every call leaves at zero; a fill kernel clears it once more when a
// device's address is first taken (a plain kernel, so the first call may be
// under graph capture: the fill then runs at every replay of that graph).
constexpr size_t kScratchBytes = size_t(16) << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

__global__ void zero_u4_kernel(uint4* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = uint4{0u, 0u, 0u, 0u};
}

// The current device's scratch address: hipGetSymbolAddress with that device
// current, once per device (the host-side name `scratch` is not a device
// address), then the counter header zeroed by a fill kernel on `stream`,
// ahead of the call's own kernels.
int scratch_for_current_device(void** ptr, hipStream_t stream) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(PKV_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(PKV_ERR_UNSUPPORTED, "device %d beyond the %d the scratch table holds", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(PKV_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    const size_t n = kWsCounterBytes / sizeof(uint4);
    hipLaunchKernelGGL(zero_u4_kernel, dim3(64), dim3(256), 0, stream,
                       static_cast<uint4*>(p), n);
    const int rc = check_launch("zero_u4_kernel");
    if (rc != PKV_OK) return rc;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return PKV_OK;
}

}  // namespace

extern "C" {

int pkv_paged_attention_noalloc(void* out, float* lse, const void* q, const void* k_pool,
                                const void* v_pool, int64_t num_blocks, int block_size,
                                const int32_t* block_tables, int max_blk,
                                const int32_t* seq_lens, const int32_t* query_start_loc,
                                int n_seq, int n_tokens, int max_q_len, int max_kv_len, int hq,
                                int hkv, int d, float scale, int causal, int part_tokens,
                                int dtype, int* status, void* stream) {
  g_err[0] = 0;
  if (n_seq > 0 && max_q_len > 0 && hkv > 0 && hq > 0 && hq % hkv == 0 &&
      part_tokens >= PKV_PART_STREAM) {
    const size_t need = plan_split(n_seq, max_q_len, hq, hkv, d, max_blk, block_size,
                                   max_kv_len, part_tokens, dtype, query_start_loc != nullptr)
                            .ws_bytes;
    if (need > kScratchBytes)
      return fail(PKV_ERR_WORKSPACE,
                  "pkv_paged_attention_noalloc: %zu bytes of scratch needed, the library "
                  "holds %zu per device; call pkv_paged_attention with a workspace",
                  need, kScratchBytes);
  }
  void* ws = nullptr;
  const int rc = scratch_for_current_device(&ws, (hipStream_t)stream);
  if (rc != PKV_OK) return rc;
  return attention_impl(out, lse, q, k_pool, v_pool, num_blocks, block_size, block_tables,
                        max_blk, seq_lens, query_start_loc, n_seq, n_tokens, max_q_len,
                        max_kv_len, hq, hkv, d, scale, causal, part_tokens, dtype, ws,
                        kScratchBytes, status, stream, nullptr, nullptr, nullptr);
}

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
                        void* stream) {
  return attention_impl(out, lse, q, k_pool, v_pool, num_blocks, block_size, block_tables,
                        max_blk, seq_lens, query_start_loc, n_seq, n_tokens, max_q_len,
                        max_kv_len, hq, hkv, d, scale, causal, part_tokens, dtype, workspace,
                        workspace_bytes, status, stream, nullptr, nullptr, nullptr);
}

int pkv_paged_attention_append(void* out, float* lse, const void* q, void* k_pool,
                               void* v_pool, int64_t num_blocks, int block_size,
                               const int32_t* block_tables, int max_blk,
                               const int32_t* seq_lens, const int32_t* query_start_loc,
                               int n_seq, int n_tokens, int max_q_len, int max_kv_len, int hq,
                               int hkv, int d, float scale, int causal, int part_tokens,
                               int dtype, const void* k_new, const void* v_new,
                               const int32_t* start_pos, void* workspace,
                               size_t workspace_bytes, int* status, void* stream) {
  if (n_tokens > 0 && (!k_new || !v_new || !start_pos || !query_start_loc))
    return fail(PKV_ERR_INVALID, "null k_new / v_new / start_pos / query_start_loc");
  return attention_impl(out, lse, q, k_pool, v_pool, num_blocks, block_size, block_tables,
                        max_blk, seq_lens, query_start_loc, n_seq, n_tokens, max_q_len,
                        max_kv_len, hq, hkv, d, scale, causal, part_tokens, dtype, workspace,
                        workspace_bytes, status, stream, k_new, v_new, start_pos);
}

}  // extern "C"
