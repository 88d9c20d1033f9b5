"""CPU oracle for the paged KV-cache decode path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithm of the reference
akshay919191/tiny-transformer-inference-engine for the path the HIP library
implements. It is the checker, never the thing measured or shipped: only
`tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may
import it. The product (`tiny-transformer-inference-engine_amd/`) never
imports it and fails loudly when its HIP library is missing.

Modules:
  paged_ref  numpy restatement of slot mapping, append (index_put), gather,
             metadata packing and paged attention (fp64 / fp32).
  torch_ref  the reference's own PyTorch paged path (index_select gather +
             scaled_dot_product_attention, tests/test.py:145-178) and a CPU
             fp32 restatement of the paged model (serving/paged_model.py) with
             greedy batched generation (serving/generation.py:112-148).

How each function is pinned (tests/test_oracle.py):
  make_slot_mapping  reference KAT bt=[7,3], start=14, n=4 -> [126,127,48,49]
                     (tests/test_kv_pool.py:28-30) + closed form + block-0 and
                     short-table asserts (serving/kv_pool.py:41-42, :52-53).
  append / gather    bit-exact against torch.Tensor.index_put_ / index_select
                     (library routines) and the write->gather round trip
                     (tests/test_kv_pool.py:33-67).
  pack_metadata      hand-worked KATs of serving/fake_paged_attn.py:52-100
                     and its ValueError cases.
  paged_attention    pure-Python fp64 brute force on tiny inputs; torch
                     scaled_dot_product_attention on gathered dense K/V;
                     closed forms (kv_len=1 -> v0, constant V, q=0 -> mean of
                     visible V, empty -> 0 / lse=+inf, non-causal prefill ==
                     full softmax); planted-mistake checks (top-left causal
                     alignment, missing scale, wrong kv-head mapping, dropped
                     kv_len clamp) each fail one of them.
  torch_ref model    RMSNorm / SwiGLU / RoPE KATs from their closed forms and
                     the paged == contiguous invariant of
                     tests/test_paged_mqa.py:9-71. Bit-identity of the random
                     init with the reference modules is PARITY UNPINNED (the
                     reference model cannot be imported: it needs compiled
                     CUDA extensions); it follows the reference construction
                     order (serving/paged_model.py:11-40).
"""
