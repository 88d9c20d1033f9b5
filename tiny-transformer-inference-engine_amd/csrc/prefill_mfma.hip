// Stand-alone launch of the MFMA prefill / chunked-prefill kernel: one pair
// workgroup per block of a (pair slot, kv head) grid, running
// prefill_pair_body() (prefill_mfma.h). Semantics are those of
// pagedattn.forward (kernels/pagedattn/pagedattn.cu:142-447) for query runs
// longer than one token.
#include "prefill_mfma.h"

namespace pkv {
namespace {

template <typename T, int D, int WPT, bool OFF64, bool KV8>
__global__ __launch_bounds__(kPBlock, 1) void prefill_mfma_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) char buf[PrefillLds<D>::kBufBytes];
  __shared__ int tbl[kTblCap];
  __shared__ int scan_sh[kPW];
  __shared__ int sv[4];
  __shared__ int dl_seq[kPBlock], dl_tok[kPBlock];
  const PrefillLds<D> sm{buf, tbl, scan_sh, sv, dl_seq, dl_tok};
  prefill_pair_body<T, D, WPT, OFF64, KV8>(a, blockIdx.x, blockIdx.y, sm);
}

template <typename T, int WPT, bool OFF64>
int launch_wpt(const AttnArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)prefill_slots(a.n_tokens, a.n_seq, 16 * WPT), a.hkv);
  if (a.d == 64 && a.kv8)
    hipLaunchKernelGGL((prefill_mfma_kernel<T, 64, WPT, OFF64, true>), grid, dim3(kPBlock), 0,
                       stream, a);
  else if (a.d == 64)
    hipLaunchKernelGGL((prefill_mfma_kernel<T, 64, WPT, OFF64, false>), grid, dim3(kPBlock), 0,
                       stream, a);
  else if (a.d == 128 && a.kv8)
    hipLaunchKernelGGL((prefill_mfma_kernel<T, 128, WPT, OFF64, true>), grid, dim3(kPBlock), 0,
                       stream, a);
  else if (a.d == 128)
    hipLaunchKernelGGL((prefill_mfma_kernel<T, 128, WPT, OFF64, false>), grid, dim3(kPBlock), 0,
                       stream, a);
  else
    return fail(PKV_ERR_UNSUPPORTED, "prefill_mfma: d=%d", a.d);
  return check_launch("prefill_mfma_kernel");
}

template <typename T, bool OFF64>
int launch_t(const AttnArgs& a, hipStream_t stream) {
  if (a.group == 16) return launch_wpt<T, 1, OFF64>(a, stream);
  if (a.group == 32) return launch_wpt<T, 2, OFF64>(a, stream);
  return fail(PKV_ERR_UNSUPPORTED, "prefill_mfma: %d query heads per kv head", a.group);
}

}  // namespace

bool prefill_mfma_supported(int dtype, int group, int d) {
  return (dtype == PKV_DTYPE_BF16 || dtype == PKV_DTYPE_F16) && (group == 16 || group == 32) &&
         (d == 64 || d == 128);
}

int launch_prefill_mfma(const AttnArgs& a, int dtype, hipStream_t stream) {
  if (!a.qloc) return fail(PKV_ERR_INVALID, "prefill_mfma: query_start_loc required");
  if (a.max_blk < 1) return fail(PKV_ERR_INVALID, "prefill_mfma: empty block table");
  const int64_t slots = prefill_slots(a.n_tokens, a.n_seq, a.group);
  if (slots > 0x7fffffff)
    return fail(PKV_ERR_UNSUPPORTED, "prefill_mfma: %lld tile pairs", (long long)slots);
  const bool off64 = pool_needs_off64(a);
  if (dtype == PKV_DTYPE_BF16)
    return off64 ? launch_t<bf16, true>(a, stream) : launch_t<bf16, false>(a, stream);
  if (dtype == PKV_DTYPE_F16)
    return off64 ? launch_t<f16, true>(a, stream) : launch_t<f16, false>(a, stream);
  return fail(PKV_ERR_UNSUPPORTED, "prefill_mfma: dtype %d", dtype);
}

}  // namespace pkv
