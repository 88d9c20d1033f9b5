// Slot-mapped K/V append and block-table gather for the paged KV pool.
//
// Both are pure byte copies between a dense [n_tok, row] buffer and the pool
// [num_blocks * block_size, row] (row = hkv * d elements), so they are
// HBM-bound: each thread moves one 16-byte piece (narrower only when the row
// or a pointer is not 16-byte aligned). Consecutive threads take consecutive
// pieces of one row, then the next row, so the dense side is read/written in
// fully coalesced 1 KiB wave transactions and the pool side row by row.
// blockIdx.y selects K (0) or V (1), so one launch moves both.
//
// Reference behaviour being replaced: KVPool.write is an index_put scatter
// `flat_k[l][slot_mapping] = k` (serving/kv_pool.py:57-70); make_slot_mapping
// computes slot = table[p // bs] * bs + p % bs (serving/kv_pool.py:40-55);
// KVPool.gather is `kv[l, 0][table].reshape(-1, ...)[:seq_len]`
// (serving/kv_pool.py:72-82).
#include "pkv_internal.h"

namespace pkv {
namespace {

template <int VEC>
struct VecT;
template <>
struct VecT<16> { using type = uint4; };
template <>
struct VecT<8> { using type = uint2; };
template <>
struct VecT<4> { using type = uint32_t; };
template <>
struct VecT<2> { using type = uint16_t; };

constexpr int kThreads = 256;

// index_put semantics for one int64 slot: negative wraps once, anything else
// outside the pool is rejected (the reference would raise IndexError).
__device__ __forceinline__ bool resolve_slot(int64_t& slot, int64_t slots) {
  if (slot < 0) slot += slots;
  return slot >= 0 && slot < slots;
}

template <int VEC>
__global__ __launch_bounds__(kThreads) void append_kernel(
    char* __restrict__ k_pool, char* __restrict__ v_pool, int64_t pool_slots,
    const char* __restrict__ k_new, const char* __restrict__ v_new,
    const int64_t* __restrict__ slots, int64_t n_tok, int64_t row_bytes,
    int* status) {
  using V = typename VecT<VEC>::type;
  const int64_t ppr = row_bytes / VEC;  // pieces per row
  const int64_t total = n_tok * ppr;
  const char* __restrict__ src = blockIdx.y ? v_new : k_new;
  char* __restrict__ dst = blockIdx.y ? v_pool : k_pool;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
       i += stride) {
    const int64_t tok = i / ppr;
    const int64_t pc = i - tok * ppr;
    int64_t slot = slots[tok];
    if (!resolve_slot(slot, pool_slots)) {
      if (status && pc == 0 && blockIdx.y == 0)
        atomicOr(status, PKV_STATUS_BAD_SLOT);
      continue;
    }
    const V v = *reinterpret_cast<const V*>(src + tok * row_bytes + pc * VEC);
    *reinterpret_cast<V*>(dst + slot * row_bytes + pc * VEC) = v;
  }
}

// Sequence owning token `t`: the largest s with qloc[s] <= t (qloc is the
// non-decreasing cumulative query count, n_seq + 1 entries).
__device__ __forceinline__ int seq_of_token(const int32_t* __restrict__ qloc,
                                            int n_seq, int64_t t) {
  int lo = 0, hi = n_seq - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((int64_t)qloc[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// query_start_loc entries a workgroup of the table append stages in LDS
// (one coalesced read instead of a chain of dependent global reads per
// binary-search step); longer batches search the global array.
constexpr int kQlocLds = 4096;

template <int VEC>
__global__ __launch_bounds__(kThreads) void append_table_kernel(
    char* __restrict__ k_pool, char* __restrict__ v_pool, int64_t num_blocks,
    int bs_shift, const char* __restrict__ k_new,
    const char* __restrict__ v_new, const int32_t* __restrict__ tables,
    int max_blk, const int32_t* __restrict__ qloc,
    const int32_t* __restrict__ start_pos, int n_seq, int64_t n_tok,
    int64_t row_bytes, int min_qlen, int* status) {
  using V = typename VecT<VEC>::type;
  __shared__ int32_t qs[kQlocLds];
  const int64_t ppr = row_bytes / VEC;
  const int64_t total = n_tok * ppr;
  const char* __restrict__ src = blockIdx.y ? v_new : k_new;
  char* __restrict__ dst = blockIdx.y ? v_pool : k_pool;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  const bool in_lds = n_seq + 1 <= kQlocLds;
  if (in_lds) {
    for (int i = threadIdx.x; i <= n_seq; i += kThreads) qs[i] = qloc[i];
    __syncthreads();
  }
  const int32_t* ql = in_lds ? qs : qloc;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
       i += stride) {
    const int64_t tok = i / ppr;
    const int64_t pc = i - tok * ppr;
    const int s = seq_of_token(ql, n_seq, tok);
    // rows of sequences with fewer than min_qlen tokens are another
    // launch's (the fused decode append of a mixed batch)
    if (min_qlen > 1 && ql[s + 1] - ql[s] < min_qlen) continue;
    const int64_t pos = (int64_t)start_pos[s] + (tok - ql[s]);
    const int64_t page = pos >> bs_shift;
    const bool flag = status && pc == 0 && blockIdx.y == 0;
    if (pos < 0 || page >= max_blk) {
      if (flag) atomicOr(status, PKV_STATUS_SHORT_TABLE);
      continue;
    }
    const int64_t phys = tables[(int64_t)s * max_blk + page];
    if (phys <= 0 || phys >= num_blocks) {
      if (flag) atomicOr(status, PKV_STATUS_BAD_BLOCK);
      continue;
    }
    const int64_t slot = (phys << bs_shift) + (pos & ((1 << bs_shift) - 1));
    const V v = *reinterpret_cast<const V*>(src + tok * row_bytes + pc * VEC);
    *reinterpret_cast<V*>(dst + slot * row_bytes + pc * VEC) = v;
  }
}

template <int VEC>
__global__ __launch_bounds__(kThreads) void gather_kernel(
    char* __restrict__ k_out, char* __restrict__ v_out,
    const char* __restrict__ k_pool, const char* __restrict__ v_pool,
    int64_t num_blocks, int bs_shift, const int32_t* __restrict__ table,
    int n_blocks, int seq_len, int64_t row_bytes, int* status) {
  using V = typename VecT<VEC>::type;
  const int64_t ppr = row_bytes / VEC;
  const int64_t total = (int64_t)seq_len * ppr;
  const char* __restrict__ src = blockIdx.y ? v_pool : k_pool;
  char* __restrict__ dst = blockIdx.y ? v_out : k_out;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
       i += stride) {
    const int64_t tok = i / ppr;
    const int64_t pc = i - tok * ppr;
    const int64_t page = tok >> bs_shift;
    int64_t phys = page < n_blocks ? (int64_t)table[page] : -1;
    V v{};
    if (phys < 0) phys += num_blocks;  // torch indexing wraps negative ids
    if (phys >= 0 && phys < num_blocks) {
      const int64_t slot = (phys << bs_shift) + (tok & ((1 << bs_shift) - 1));
      v = *reinterpret_cast<const V*>(src + slot * row_bytes + pc * VEC);
    } else if (status && pc == 0 && blockIdx.y == 0) {
      atomicOr(status, PKV_STATUS_BAD_BLOCK);
    }
    *reinterpret_cast<V*>(dst + tok * row_bytes + pc * VEC) = v;
  }
}

// ---- fp8 pools: each thread converts one piece of 8 values (8 source
// elements in, 8 bytes out) with f32_to_e4m3.
template <typename S>
__device__ __forceinline__ float elem_to_f32(S x) {
  return (float)x;
}
template <>
__device__ __forceinline__ float elem_to_f32<bf16>(bf16 x) {
  return __uint_as_float((unsigned)__builtin_bit_cast(unsigned short, x) << 16);
}

template <typename S>
__device__ __forceinline__ uint2 narrow_piece(const S* __restrict__ p) {
  S v[8];
  __builtin_memcpy(v, p, sizeof(v));  // one or two 16-byte loads (alignment checked on the host)
  unsigned w[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e) w[e >> 2] |= f32_to_e4m3(elem_to_f32(v[e])) << (8 * (e & 3));
  return uint2{w[0], w[1]};
}

template <typename S>
__global__ __launch_bounds__(kThreads) void append_fp8_kernel(
    char* __restrict__ k_pool, char* __restrict__ v_pool, int64_t pool_slots,
    const S* __restrict__ k_new, const S* __restrict__ v_new,
    const int64_t* __restrict__ slots, int64_t n_tok, int64_t row_elems, int* status) {
  const int64_t ppr = row_elems / 8;
  const int64_t total = n_tok * ppr;
  const S* __restrict__ src = blockIdx.y ? v_new : k_new;
  char* __restrict__ dst = blockIdx.y ? v_pool : k_pool;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += stride) {
    const int64_t tok = i / ppr;
    const int64_t pc = i - tok * ppr;
    int64_t slot = slots[tok];
    if (!resolve_slot(slot, pool_slots)) {
      if (status && pc == 0 && blockIdx.y == 0) atomicOr(status, PKV_STATUS_BAD_SLOT);
      continue;
    }
    *reinterpret_cast<uint2*>(dst + slot * row_elems + pc * 8) =
        narrow_piece(src + tok * row_elems + pc * 8);
  }
}

template <typename S>
__global__ __launch_bounds__(kThreads) void append_table_fp8_kernel(
    char* __restrict__ k_pool, char* __restrict__ v_pool, int64_t num_blocks, int bs_shift,
    const S* __restrict__ k_new, const S* __restrict__ v_new,
    const int32_t* __restrict__ tables, int max_blk, const int32_t* __restrict__ qloc,
    const int32_t* __restrict__ start_pos, int n_seq, int64_t n_tok, int64_t row_elems,
    int min_qlen, int* status) {
  __shared__ int32_t qs[kQlocLds];
  const int64_t ppr = row_elems / 8;
  const int64_t total = n_tok * ppr;
  const S* __restrict__ src = blockIdx.y ? v_new : k_new;
  char* __restrict__ dst = blockIdx.y ? v_pool : k_pool;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  const bool in_lds = n_seq + 1 <= kQlocLds;
  if (in_lds) {
    for (int i = threadIdx.x; i <= n_seq; i += kThreads) qs[i] = qloc[i];
    __syncthreads();
  }
  const int32_t* ql = in_lds ? qs : qloc;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total; i += stride) {
    const int64_t tok = i / ppr;
    const int64_t pc = i - tok * ppr;
    const int s = seq_of_token(ql, n_seq, tok);
    if (min_qlen > 1 && ql[s + 1] - ql[s] < min_qlen) continue;
    const int64_t pos = (int64_t)start_pos[s] + (tok - ql[s]);
    const int64_t page = pos >> bs_shift;
    const bool flag = status && pc == 0 && blockIdx.y == 0;
    if (pos < 0 || page >= max_blk) {
      if (flag) atomicOr(status, PKV_STATUS_SHORT_TABLE);
      continue;
    }
    const int64_t phys = tables[(int64_t)s * max_blk + page];
    if (phys <= 0 || phys >= num_blocks) {
      if (flag) atomicOr(status, PKV_STATUS_BAD_BLOCK);
      continue;
    }
    const int64_t slot = (phys << bs_shift) + (pos & ((1 << bs_shift) - 1));
    *reinterpret_cast<uint2*>(dst + slot * row_elems + pc * 8) =
        narrow_piece(src + tok * row_elems + pc * 8);
  }
}

// 8-byte pool pieces and 8-element source pieces must be naturally aligned.
int check_fp8_rows(int64_t row_elems, int src_dtype, std::initializer_list<const void*> pools,
                   std::initializer_list<const void*> srcs) {
  if (row_elems % 8 != 0)
    return fail(PKV_ERR_UNSUPPORTED, "fp8 append: row of %lld elements (need a multiple of 8)",
                (long long)row_elems);
  const uintptr_t sa = (uintptr_t)8 * elem_bytes(src_dtype);
  for (const void* p : pools)
    if ((uintptr_t)p % 8) return fail(PKV_ERR_UNSUPPORTED, "fp8 append: pool not 8-byte aligned");
  for (const void* p : srcs)
    if ((uintptr_t)p % (sa < 16 ? sa : 16))
      return fail(PKV_ERR_UNSUPPORTED, "fp8 append: source rows not %zu-byte aligned",
                  (size_t)(sa < 16 ? sa : 16));
  return PKV_OK;
}

// Widest piece (16/8/4/2 bytes) dividing the row and every base pointer.
int pick_vec(int64_t row_bytes, std::initializer_list<const void*> ptrs) {
  uintptr_t acc = (uintptr_t)row_bytes;
  for (const void* p : ptrs) acc |= (uintptr_t)p;
  if ((acc & 15) == 0) return 16;
  if ((acc & 7) == 0) return 8;
  if ((acc & 3) == 0) return 4;
  return 2;
}

dim3 copy_grid(int64_t pieces) {
  // Enough workgroups to cover every CU several times; each thread loops
  // when there are more pieces than threads.
  int64_t blocks = (pieces + kThreads - 1) / kThreads;
  if (blocks > 8192) blocks = 8192;
  if (blocks < 1) blocks = 1;
  return dim3((unsigned)blocks, 2, 1);
}

}  // namespace

int launch_append(void* k_pool, void* v_pool, int64_t pool_slots,
                  const void* k_new, const void* v_new, const int64_t* slots,
                  int64_t n_tok, int64_t row_bytes, int* status,
                  hipStream_t stream) {
  if (n_tok == 0) return PKV_OK;
  const int vec = pick_vec(row_bytes, {k_pool, v_pool, k_new, v_new});
  const dim3 grid = copy_grid(n_tok * (row_bytes / vec));
#define PKV_APPEND(VEC)                                                      \
  hipLaunchKernelGGL(append_kernel<VEC>, grid, dim3(kThreads), 0, stream,    \
                     (char*)k_pool, (char*)v_pool, pool_slots,               \
                     (const char*)k_new, (const char*)v_new, slots, n_tok,   \
                     row_bytes, status)
  switch (vec) {
    case 16: PKV_APPEND(16); break;
    case 8: PKV_APPEND(8); break;
    case 4: PKV_APPEND(4); break;
    default: PKV_APPEND(2); break;
  }
#undef PKV_APPEND
  return check_launch("append_kernel");
}

int launch_append_from_table(void* k_pool, void* v_pool, int64_t num_blocks,
                             int bs_shift, const void* k_new,
                             const void* v_new, const int32_t* block_tables,
                             int max_blk, const int32_t* qloc,
                             const int32_t* start_pos, int n_seq,
                             int64_t n_tok, int64_t row_bytes, int min_qlen,
                             int* status, hipStream_t stream) {
  if (n_tok == 0 || n_seq == 0) return PKV_OK;
  const int vec = pick_vec(row_bytes, {k_pool, v_pool, k_new, v_new});
  const dim3 grid = copy_grid(n_tok * (row_bytes / vec));
#define PKV_APPEND_T(VEC)                                                    \
  hipLaunchKernelGGL(append_table_kernel<VEC>, grid, dim3(kThreads), 0,      \
                     stream, (char*)k_pool, (char*)v_pool, num_blocks,       \
                     bs_shift, (const char*)k_new, (const char*)v_new,       \
                     block_tables, max_blk, qloc, start_pos, n_seq, n_tok,   \
                     row_bytes, min_qlen, status)
  switch (vec) {
    case 16: PKV_APPEND_T(16); break;
    case 8: PKV_APPEND_T(8); break;
    case 4: PKV_APPEND_T(4); break;
    default: PKV_APPEND_T(2); break;
  }
#undef PKV_APPEND_T
  return check_launch("append_table_kernel");
}

int launch_append_fp8(void* k_pool, void* v_pool, int64_t pool_slots, const void* k_new,
                      const void* v_new, const int64_t* slots, int64_t n_tok,
                      int64_t row_elems, int src_dtype, int* status, hipStream_t stream) {
  if (n_tok == 0) return PKV_OK;
  int rc = check_fp8_rows(row_elems, src_dtype, {k_pool, v_pool}, {k_new, v_new});
  if (rc != PKV_OK) return rc;
  const dim3 grid = copy_grid(n_tok * (row_elems / 8));
#define PKV_APPEND8(S)                                                                       \
  hipLaunchKernelGGL(append_fp8_kernel<S>, grid, dim3(kThreads), 0, stream, (char*)k_pool,   \
                     (char*)v_pool, pool_slots, (const S*)k_new, (const S*)v_new, slots,     \
                     n_tok, row_elems, status)
  if (src_dtype == PKV_DTYPE_BF16) PKV_APPEND8(bf16);
  else if (src_dtype == PKV_DTYPE_F16) PKV_APPEND8(f16);
  else PKV_APPEND8(float);
#undef PKV_APPEND8
  return check_launch("append_fp8_kernel");
}

int launch_append_from_table_fp8(void* k_pool, void* v_pool, int64_t num_blocks, int bs_shift,
                                 const void* k_new, const void* v_new,
                                 const int32_t* block_tables, int max_blk, const int32_t* qloc,
                                 const int32_t* start_pos, int n_seq, int64_t n_tok,
                                 int64_t row_elems, int src_dtype, int min_qlen, int* status,
                                 hipStream_t stream) {
  if (n_tok == 0 || n_seq == 0) return PKV_OK;
  int rc = check_fp8_rows(row_elems, src_dtype, {k_pool, v_pool}, {k_new, v_new});
  if (rc != PKV_OK) return rc;
  const dim3 grid = copy_grid(n_tok * (row_elems / 8));
#define PKV_APPEND8_T(S)                                                                    \
  hipLaunchKernelGGL(append_table_fp8_kernel<S>, grid, dim3(kThreads), 0, stream,           \
                     (char*)k_pool, (char*)v_pool, num_blocks, bs_shift, (const S*)k_new,   \
                     (const S*)v_new, block_tables, max_blk, qloc, start_pos, n_seq, n_tok, \
                     row_elems, min_qlen, status)
  if (src_dtype == PKV_DTYPE_BF16) PKV_APPEND8_T(bf16);
  else if (src_dtype == PKV_DTYPE_F16) PKV_APPEND8_T(f16);
  else PKV_APPEND8_T(float);
#undef PKV_APPEND8_T
  return check_launch("append_table_fp8_kernel");
}

int launch_gather(void* k_out, void* v_out, const void* k_pool,
                  const void* v_pool, int64_t num_blocks, int bs_shift,
                  const int32_t* table, int n_blocks, int seq_len,
                  int64_t row_bytes, int* status, hipStream_t stream) {
  if (seq_len == 0) return PKV_OK;
  const int vec = pick_vec(row_bytes, {k_pool, v_pool, k_out, v_out});
  const dim3 grid = copy_grid((int64_t)seq_len * (row_bytes / vec));
#define PKV_GATHER(VEC)                                                      \
  hipLaunchKernelGGL(gather_kernel<VEC>, grid, dim3(kThreads), 0, stream,    \
                     (char*)k_out, (char*)v_out, (const char*)k_pool,        \
                     (const char*)v_pool, num_blocks, bs_shift, table,       \
                     n_blocks, seq_len, row_bytes, status)
  switch (vec) {
    case 16: PKV_GATHER(16); break;
    case 8: PKV_GATHER(8); break;
    case 4: PKV_GATHER(4); break;
    default: PKV_GATHER(2); break;
  }
#undef PKV_GATHER
  return check_launch("gather_kernel");
}

}  // namespace pkv
