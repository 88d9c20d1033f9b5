"""FusedRows (serving/fused_ops.py): the row-concatenated projection weights
behind the one-GEMM q/k/v and gate/up paths. CPU only: the concatenation
equals the separate weights, the modules' parameters become views of it
(state-dict keys, shapes and values unchanged; load_state_dict and in-place
updates reach the fused storage), and a replaced parameter (module.to, a
new Parameter) triggers a rebuild."""
import torch
import torch.nn as nn

from serving.fused_ops import FusedRows
from serving.layers import ModelConfig, SwiGLU
from serving.paged_mqa import MQA_Paged


def test_concatenation_and_views():
    torch.manual_seed(0)
    a, b, c = nn.Linear(8, 6), nn.Linear(8, 2), nn.Linear(8, 2)
    ref = torch.cat([a.weight, b.weight, c.weight]).detach().clone()
    refb = torch.cat([a.bias, b.bias, c.bias]).detach().clone()
    f = FusedRows(a, b, c)
    w, bias = f.get()
    assert torch.equal(w, ref) and torch.equal(bias, refb)
    assert a.weight.data_ptr() == w.data_ptr()
    assert b.weight.data_ptr() == w.data_ptr() + 6 * 8 * w.element_size()
    assert f.get()[0] is w  # no rebuild while the views are intact
    with torch.no_grad():
        b.weight.add_(1.0)  # in-place update reaches the fused rows
    assert torch.equal(f.get()[0][6:8], ref[6:8] + 1.0)
    x = torch.randn(3, 8)
    y = nn.functional.linear(x, *f.get())
    torch.testing.assert_close(y, torch.cat([a(x), b(x), c(x)], -1))


def test_rebuild_after_replacement_and_dtype_change():
    a, b = nn.Linear(4, 4, bias=False), nn.Linear(4, 4, bias=False)
    f = FusedRows(a, b)
    w0, b0 = f.get()
    assert b0 is None
    a.weight = nn.Parameter(torch.ones(4, 4))
    w1, _ = f.get()
    assert w1 is not w0 and torch.equal(w1[:4], torch.ones(4, 4))
    a.to(torch.float64), b.to(torch.float64)
    w2, _ = f.get()
    assert w2.dtype == torch.float64 and a.weight.data_ptr() == w2.data_ptr()


def test_state_dict_round_trip_through_views():
    cfg = ModelConfig(vocab_size=64, d_model=32, num_layers=1, num_heads=4, num_kv_heads=1,
                      max_seq_len=16)
    torch.manual_seed(1)
    m = MQA_Paged(cfg)
    keys = sorted(m.state_dict())
    m._qkv.get()
    assert sorted(m.state_dict()) == keys
    torch.manual_seed(2)
    other = MQA_Paged(cfg)
    m.load_state_dict(other.state_dict())
    w, _ = m._qkv.get()
    assert torch.equal(w, torch.cat([other.q_proj.weight, other.k_proj.weight,
                                     other.v_proj.weight]))
    mlp = SwiGLU(16, 24)
    w, _ = mlp._gate_up.get()
    assert w.shape == (48, 16) and torch.equal(w[24:], mlp.up_proj.weight)
