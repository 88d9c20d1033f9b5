"""Host wrappers of the decoder block's kernels around the paged attention in
libpagedkv.so: RMSNorm with a fused residual add, RoPE on token-major Q/K
rows, and the SwiGLU gate (csrc/layers.hip); the few-row projections with
those ops fused into their epilogues (csrc/linear.hip); the greedy argmax
(csrc/sampling.hip).

Every function requires ROCm device tensors and the library (RuntimeError
otherwise). The projections hand shapes their kernel does not take (fp32,
k not a multiple of 32, more than LINEAR_MAX_ROWS rows or LINEAR_MAX_FEATURES
features) to the library GEMM. Outputs are allocated with
torch on the input's device and the current stream, so the calls can be
captured in a HIP graph.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _native


def _rows(x: torch.Tensor, what: str):
    """x viewed as [rows, dim] with unit column stride: (tensor, rows, stride)."""
    if x.dim() == 0:
        raise ValueError(f"{what}: expected at least one dimension")
    dim = x.shape[-1]
    x2 = x.reshape(-1, dim) if x.dim() != 2 else x
    if x2.stride(-1) != 1 or (x2.shape[0] > 1 and x2.stride(0) < dim):
        x2 = x2.contiguous()
    return x2, x2.shape[0], (x2.stride(0) if x2.shape[0] > 1 else dim)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm of the last dimension: (x * rsqrt(mean(x^2) + eps)) * weight in
    fp32, rounded to x.dtype (models/rmsnorm.py:12-18)."""
    _native.require_device(x, weight, what="rms_norm")
    w = weight if weight.dtype == x.dtype else weight.to(x.dtype)
    w = w.contiguous()
    if w.numel() != x.shape[-1]:
        raise ValueError(f"rms_norm: weight has {w.numel()} elements, rows have {x.shape[-1]}")
    x2, rows, stride = _rows(x, "rms_norm")
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    rc = _native.lib().pkv_rms_norm(
        y.data_ptr(), None, x2.data_ptr(), None, w.data_ptr(), rows, x.shape[-1], stride,
        0, float(eps), _native.dtype_code(x.dtype), _native.stream_ptr(x.device))
    _native.check(rc, "rms_norm")
    return y


def add_rms_norm_(x: torch.Tensor, delta: torch.Tensor, weight: torch.Tensor,
                  eps: float) -> torch.Tensor:
    """x += delta (rounded to x.dtype, in place), then return rms_norm(x):
    the residual add of a decoder block fused with the next norm
    (serving/paged_model.py:20-29). x must be contiguous."""
    _native.require_device(x, delta, weight, what="add_rms_norm_")
    if not x.is_contiguous():
        raise ValueError("add_rms_norm_: x must be contiguous (it is updated in place)")
    if delta.shape != x.shape or delta.dtype != x.dtype:
        raise ValueError(f"add_rms_norm_: delta {tuple(delta.shape)} {delta.dtype} vs x "
                         f"{tuple(x.shape)} {x.dtype}")
    w = weight if weight.dtype == x.dtype else weight.to(x.dtype)
    w = w.contiguous()
    dim = x.shape[-1]
    if w.numel() != dim:
        raise ValueError(f"add_rms_norm_: weight has {w.numel()} elements, rows have {dim}")
    d2, rows, dstride = _rows(delta, "add_rms_norm_")
    y = torch.empty_like(x)
    rc = _native.lib().pkv_rms_norm(
        y.data_ptr(), x.data_ptr(), x.data_ptr(), d2.data_ptr(), w.data_ptr(), rows, dim, dim,
        dstride, float(eps), _native.dtype_code(x.dtype), _native.stream_ptr(x.device))
    _native.check(rc, "add_rms_norm_")
    return y


def _tok_rows(t: torch.Tensor, heads: int, d: int, what: str):
    """[T, heads, d] or [T, heads*d] rows with contiguous heads: (tensor, row stride)."""
    if t.dim() == 3:
        if t.shape[1] != heads or t.shape[2] != d:
            raise ValueError(f"{what}: expected [T, {heads}, {d}], got {tuple(t.shape)}")
        ok = t.stride(2) == 1 and t.stride(1) == d
        if not ok:
            t = t.contiguous()
        return t, (t.stride(0) if t.shape[0] > 1 else heads * d)
    if t.dim() == 2 and t.shape[1] == heads * d:
        if t.stride(1) != 1:
            t = t.contiguous()
        return t, (t.stride(0) if t.shape[0] > 1 else heads * d)
    raise ValueError(f"{what}: expected [T, {heads}, {d}], got {tuple(t.shape)}")


def rope(q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor,
         sin: torch.Tensor, v: torch.Tensor | None = None, hq: int | None = None,
         hkv: int | None = None, d: int | None = None):
    """Rotary embedding of q [T, Hq, D] and k [T, Hkv, D] at positions [T]
    with fp32 tables cos/sin [max_pos, D/2] (models/rope.py:21-47, values and
    intermediate products rounded to q.dtype). q, k (and v) may be strided
    column ranges of one projection output, given as [T, H*D] slices with
    hq/hkv/d. Returns contiguous (q_rot, k_rot) or, with v, (q_rot, k_rot,
    v_contiguous)."""
    if q.dim() == 3:
        hq, d = q.shape[1], q.shape[2]
    if k.dim() == 3:
        hkv = k.shape[1]
    if hq is None or hkv is None or d is None:
        raise ValueError("rope: pass hq, hkv and d for 2-D q / k")
    tensors = [q, k, positions, cos, sin] + ([v] if v is not None else [])
    _native.require_device(*tensors, what="rope")
    if k.dtype != q.dtype or (v is not None and v.dtype != q.dtype):
        raise ValueError("rope: q, k, v must share a dtype")
    T = q.shape[0]
    if k.shape[0] != T or (v is not None and v.shape[0] != T) or positions.numel() != T:
        raise ValueError("rope: q, k, v and positions disagree on the token count")
    cos2 = cos.reshape(-1, d // 2)
    sin2 = sin.reshape(-1, d // 2)
    if cos2.dtype != torch.float32 or sin2.dtype != torch.float32 or cos2.shape != sin2.shape:
        raise ValueError("rope: cos / sin must be fp32 tables of equal shape [max_pos, D/2]")
    cos2, sin2 = cos2.contiguous(), sin2.contiguous()
    pos = positions if positions.dtype == torch.int32 else positions.to(torch.int32)
    pos = pos.contiguous()
    qs, q_stride = _tok_rows(q, hq, d, "rope q")
    ks, k_stride = _tok_rows(k, hkv, d, "rope k")
    q_out = torch.empty((T, hq, d), dtype=q.dtype, device=q.device)
    k_out = torch.empty((T, hkv, d), dtype=q.dtype, device=q.device)
    if v is not None:
        vs, v_stride = _tok_rows(v, hkv, d, "rope v")
        v_out = torch.empty((T, hkv, d), dtype=q.dtype, device=q.device)
    else:
        vs, v_stride, v_out = None, 0, None
    rc = _native.lib().pkv_rope(
        q_out.data_ptr(), k_out.data_ptr(), _native.ptr(v_out), qs.data_ptr(), ks.data_ptr(),
        _native.ptr(vs), q_stride, k_stride, v_stride, pos.data_ptr(), cos2.data_ptr(),
        sin2.data_ptr(), cos2.shape[0], T, hq, hkv, d, _native.dtype_code(q.dtype), None,
        _native.stream_ptr(q.device))
    _native.check(rc, "rope")
    return (q_out, k_out) if v is None else (q_out, k_out, v_out)


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """gate * sigmoid(gate) * up in fp32, rounded once
    (kernels/fused_swiglu/kernel.py:6-19). gate and up may be strided column
    ranges of one [rows, 2H] projection output; the result is contiguous."""
    _native.require_device(gate, up, what="silu_mul")
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise ValueError("silu_mul: gate and up must have the same shape and dtype")
    g2, rows, gs = _rows(gate, "silu_mul")
    u2, _, us = _rows(up, "silu_mul")
    cols = gate.shape[-1]
    out = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
    rc = _native.lib().pkv_silu_mul(out.data_ptr(), g2.data_ptr(), u2.data_ptr(), rows, cols,
                                    gs, us, _native.dtype_code(gate.dtype),
                                    _native.stream_ptr(gate.device))
    _native.check(rc, "silu_mul")
    return out


# the few-row projection kernels (csrc/linear.hip) take decode-sized row
# counts; wider problems (prefill chunks, the vocabulary projection) and
# fp32 go to the library GEMM
LINEAR_MAX_ROWS = 256
LINEAR_MAX_FEATURES = 16384


def _as_rows(x: torch.Tensor) -> torch.Tensor:
    x2 = x.reshape(-1, x.shape[-1]) if x.dim() != 2 else x
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    return x2


def _linear_ok(x2: torch.Tensor, w: torch.Tensor, bias, n_features: int) -> bool:
    return (x2.is_cuda and x2.dtype in (torch.bfloat16, torch.float16, torch.float32)
            and w.dtype == x2.dtype
            and (bias is None or (bias.dtype == x2.dtype and bias.is_contiguous()))
            and 0 < x2.shape[0] <= LINEAR_MAX_ROWS and x2.shape[1] % 32 == 0
            and n_features <= LINEAR_MAX_FEATURES and w.is_contiguous()
            and (x2.shape[0] == 1 or x2.stride(0) % 8 == 0)
            and x2.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0)


def _x_stride(x2):
    return x2.stride(0) if x2.shape[0] > 1 else x2.shape[1]


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None):
    """x W^T + b. Few-row bf16/fp16/fp32 problems run on the split-K MFMA
    kernel (pkv_linear); others on the library GEMM (F.linear)."""
    x2 = _as_rows(x)
    n = weight.shape[0]
    if not _linear_ok(x2, weight, bias, n):
        return F.linear(x, weight, bias)
    out = torch.empty((x2.shape[0], n), dtype=x.dtype, device=x.device)
    rc = _native.lib().pkv_linear(out.data_ptr(), x2.data_ptr(), weight.data_ptr(),
                                  _native.ptr(bias), x2.shape[0], n, x2.shape[1], _x_stride(x2),
                                  _native.dtype_code(x.dtype), _native.stream_ptr(x.device))
    _native.check(rc, "linear")
    return out.view(*x.shape[:-1], n)


def linear_swiglu(x: torch.Tensor, w_gate_up: torch.Tensor, b_gate_up: torch.Tensor | None):
    """silu(x Wg^T + bg) * (x Wu^T + bu) with W = [Wg; Wu] (models/mlp.py:24-30
    with the reference's fused_swiglu arithmetic)."""
    x2 = _as_rows(x)
    h = w_gate_up.shape[0] // 2
    if not _linear_ok(x2, w_gate_up, b_gate_up, 2 * h):
        gu = F.linear(x, w_gate_up, b_gate_up)
        return silu_mul(gu[..., :h], gu[..., h:])
    _native.require_device(x2, w_gate_up, what="linear_swiglu")
    out = torch.empty((x2.shape[0], h), dtype=x.dtype, device=x.device)
    rc = _native.lib().pkv_linear_swiglu(
        out.data_ptr(), x2.data_ptr(), w_gate_up.data_ptr(), _native.ptr(b_gate_up),
        x2.shape[0], h, x2.shape[1], _x_stride(x2), _native.dtype_code(x.dtype),
        _native.stream_ptr(x.device))
    _native.check(rc, "linear_swiglu")
    return out.view(*x.shape[:-1], h)


def linear_rope_qkv(x: torch.Tensor, w_qkv: torch.Tensor, b_qkv: torch.Tensor | None,
                    positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, hq: int,
                    hkv: int, d: int):
    """q, k, v projections of x [T, d_model] with W = [Wq; Wk; Wv], q and k
    rotated at positions (fp32 tables cos / sin [max_pos, d/2]): contiguous
    q [T, hq, d], k [T, hkv, d], v [T, hkv, d] (serving/paged_mqa.py:76-85)."""
    x2 = _as_rows(x)
    T = x2.shape[0]
    nq, nk = hq * d, hkv * d
    if not _linear_ok(x2, w_qkv, b_qkv, nq + 2 * nk):
        qkv = F.linear(x2, w_qkv, b_qkv)
        return rope(qkv[:, :nq], qkv[:, nq:nq + nk], positions, cos, sin, v=qkv[:, nq + nk:],
                    hq=hq, hkv=hkv, d=d)
    _native.require_device(x2, w_qkv, positions, cos, sin, what="linear_rope_qkv")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise ValueError("linear_rope_qkv: cos / sin must be fp32 tables")
    cos2, sin2 = cos.reshape(-1, d // 2).contiguous(), sin.reshape(-1, d // 2).contiguous()
    pos = positions if positions.dtype == torch.int32 else positions.to(torch.int32)
    pos = pos.contiguous()
    if pos.numel() != T:
        raise ValueError("linear_rope_qkv: positions and x disagree on the token count")
    q = torch.empty((T, hq, d), dtype=x.dtype, device=x.device)
    k = torch.empty((T, hkv, d), dtype=x.dtype, device=x.device)
    v = torch.empty((T, hkv, d), dtype=x.dtype, device=x.device)
    rc = _native.lib().pkv_linear_rope_qkv(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), x2.data_ptr(), w_qkv.data_ptr(),
        _native.ptr(b_qkv), T, x2.shape[1], _x_stride(x2), pos.data_ptr(), cos2.data_ptr(),
        sin2.data_ptr(), cos2.shape[0], hq, hkv, d, _native.dtype_code(x.dtype), None,
        _native.stream_ptr(x.device))
    _native.check(rc, "linear_rope_qkv")
    return q, k, v


# the projection kernels normalise rows of at most this many features in
# their prologue (pkv_linear_*_rmsnorm); wider rows take rms_norm first
LINEAR_NORM_MAX_K = 1024


def _norm_ok(x2: torch.Tensor, norm_weight: torch.Tensor) -> bool:
    return (x2.shape[1] <= LINEAR_NORM_MAX_K and norm_weight.dtype == x2.dtype
            and norm_weight.is_contiguous() and norm_weight.numel() == x2.shape[1]
            and norm_weight.data_ptr() % 16 == 0)


def linear_residual_(resid: torch.Tensor, x: torch.Tensor, weight: torch.Tensor,
                     bias: torch.Tensor | None = None) -> torch.Tensor:
    """resid += x W^T + b in place, the projection rounded to resid.dtype
    before the add (the residual adds of serving/paged_model.py:20-29, one
    kernel for the projection and the add). resid must be contiguous with
    x's rows. Returns resid."""
    x2 = _as_rows(x)
    n = weight.shape[0]
    if (not _linear_ok(x2, weight, bias, n) or not resid.is_contiguous()
            or resid.dtype != x.dtype or resid.numel() != x2.shape[0] * n):
        return resid.add_(linear(x, weight, bias).view(resid.shape))
    rc = _native.lib().pkv_linear_residual(
        resid.data_ptr(), x2.data_ptr(), weight.data_ptr(), _native.ptr(bias), x2.shape[0], n,
        x2.shape[1], _x_stride(x2), _native.dtype_code(x.dtype), _native.stream_ptr(x.device))
    _native.check(rc, "linear_residual_")
    return resid


def linear_swiglu_rmsnorm(x: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                          w_gate_up: torch.Tensor, b_gate_up: torch.Tensor | None):
    """linear_swiglu(rms_norm(x, norm_weight, eps), ...) with the norm taken
    in the projection kernel's prologue (bit-identical to the two calls)."""
    x2 = _as_rows(x)
    h = w_gate_up.shape[0] // 2
    if not (_linear_ok(x2, w_gate_up, b_gate_up, 2 * h) and _norm_ok(x2, norm_weight)):
        return linear_swiglu(rms_norm(x, norm_weight, eps), w_gate_up, b_gate_up)
    _native.require_device(x2, norm_weight, w_gate_up, what="linear_swiglu_rmsnorm")
    out = torch.empty((x2.shape[0], h), dtype=x.dtype, device=x.device)
    rc = _native.lib().pkv_linear_swiglu_rmsnorm(
        out.data_ptr(), x2.data_ptr(), norm_weight.data_ptr(), float(eps), w_gate_up.data_ptr(),
        _native.ptr(b_gate_up), x2.shape[0], h, x2.shape[1], _x_stride(x2),
        _native.dtype_code(x.dtype), _native.stream_ptr(x.device))
    _native.check(rc, "linear_swiglu_rmsnorm")
    return out.view(*x.shape[:-1], h)


def linear_rope_qkv_rmsnorm(x: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                            w_qkv: torch.Tensor, b_qkv: torch.Tensor | None,
                            positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                            hq: int, hkv: int, d: int):
    """linear_rope_qkv(rms_norm(x, norm_weight, eps), ...) with the norm
    taken in the projection kernel's prologue (bit-identical to the two
    calls)."""
    x2 = _as_rows(x)
    T = x2.shape[0]
    nq, nk = hq * d, hkv * d
    if not (_linear_ok(x2, w_qkv, b_qkv, nq + 2 * nk) and _norm_ok(x2, norm_weight)):
        return linear_rope_qkv(rms_norm(x, norm_weight, eps), w_qkv, b_qkv, positions, cos, sin,
                               hq, hkv, d)
    _native.require_device(x2, norm_weight, w_qkv, positions, cos, sin,
                           what="linear_rope_qkv_rmsnorm")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise ValueError("linear_rope_qkv_rmsnorm: cos / sin must be fp32 tables")
    cos2, sin2 = cos.reshape(-1, d // 2).contiguous(), sin.reshape(-1, d // 2).contiguous()
    pos = positions if positions.dtype == torch.int32 else positions.to(torch.int32)
    pos = pos.contiguous()
    if pos.numel() != T:
        raise ValueError("linear_rope_qkv_rmsnorm: positions and x disagree on the token count")
    q = torch.empty((T, hq, d), dtype=x.dtype, device=x.device)
    k = torch.empty((T, hkv, d), dtype=x.dtype, device=x.device)
    v = torch.empty((T, hkv, d), dtype=x.dtype, device=x.device)
    rc = _native.lib().pkv_linear_rope_qkv_rmsnorm(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), x2.data_ptr(), norm_weight.data_ptr(),
        float(eps), w_qkv.data_ptr(), _native.ptr(b_qkv), T, x2.shape[1], _x_stride(x2),
        pos.data_ptr(), cos2.data_ptr(), sin2.data_ptr(), cos2.shape[0], hq, hkv, d,
        _native.dtype_code(x.dtype), None, _native.stream_ptr(x.device))
    _native.check(rc, "linear_rope_qkv_rmsnorm")
    return q, k, v


def argmax_rows(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Index of the largest logit of every row of [rows, vocab] logits as
    int64 [rows] (pkv_argmax_rows; the framework's argmax result: first
    maximum, NaN above every number). With `out`, the ids are written there
    (an int64 device tensor of rows elements)."""
    _native.require_device(logits, what="argmax_rows")
    if logits.dim() != 2:
        raise ValueError(f"argmax_rows: expected [rows, vocab], got {tuple(logits.shape)}")
    lg = logits if logits.stride(1) == 1 else logits.contiguous()
    rows, vocab = lg.shape
    if out is None:
        out = torch.empty(rows, dtype=torch.long, device=logits.device)
    elif (out.dtype != torch.long or out.numel() != rows or not out.is_contiguous()
          or out.device != logits.device):
        raise ValueError("argmax_rows: out must be a contiguous int64 tensor of rows elements")
    stride = lg.stride(0) if rows > 1 else vocab
    ws, wsb = _argmax_workspace(lg)
    rc = _native.lib().pkv_argmax_rows(out.data_ptr(), lg.data_ptr(), rows, vocab, stride,
                                       _native.dtype_code(lg.dtype), _native.ptr(ws), wsb,
                                       _native.stream_ptr(logits.device))
    _native.check(rc, "argmax_rows")
    return out


def _argmax_workspace(lg):
    """The split-row argmax's counters and key words: the "argmax" slot of
    the current workspace (a graph step's own workspace under its scope)."""
    rows, vocab = lg.shape
    wsb = int(_native.lib().pkv_argmax_workspace_bytes(rows, vocab, _native.dtype_code(lg.dtype)))
    if wsb == 0:
        return None, 0
    return _native.current_workspace().get(lg.device, wsb, slot="argmax"), wsb


def sample_rows(logits: torch.Tensor, temperature: float, top_k: int, top_p: float,
                uniforms: torch.Tensor):
    """One draw per row of [rows, vocab] logits with temperature, top-k
    (1..64, ties at the threshold kept) and top-p, by inverse CDF at the
    row's uniform in [0, 1) (pkv_sample_rows). Returns (ids int64 [rows],
    status int32 [1]: PKV_STATUS_* bits; a flagged row's id is -1)."""
    _native.require_device(logits, uniforms, what="sample_rows")
    if logits.dim() != 2:
        raise ValueError(f"sample_rows: expected [rows, vocab], got {tuple(logits.shape)}")
    lg = logits if logits.stride(1) == 1 else logits.contiguous()
    rows, vocab = lg.shape
    u = uniforms.to(torch.float32).contiguous()
    if u.numel() != rows:
        raise ValueError("sample_rows: one uniform per row")
    ids = torch.empty(rows, dtype=torch.long, device=logits.device)
    status = torch.zeros(1, dtype=torch.int32, device=logits.device)
    stride = lg.stride(0) if rows > 1 else vocab
    rc = _native.lib().pkv_sample_rows(ids.data_ptr(), lg.data_ptr(), rows, vocab, stride,
                                       float(temperature), int(top_k), float(top_p),
                                       u.data_ptr(), _native.dtype_code(lg.dtype),
                                       status.data_ptr(), _native.stream_ptr(logits.device))
    _native.check(rc, "sample_rows")
    return ids, status


class FusedRows:
    """Row-concatenated weights (and biases) of several nn.Linear modules
    sharing an input, so one GEMM computes all of their outputs. The
    modules' parameters are re-pointed to views of the concatenation, so
    they stay the state-dict entries, in-place updates (load_state_dict,
    optimiser steps) reach the fused storage, and no copy is kept. When a
    parameter has been replaced (module.to(...), assignment) the
    concatenation is rebuilt on the next call."""

    def __init__(self, *linears: torch.nn.Linear):
        self.linears = linears
        self.weight = None
        self.bias = None

    def _views_intact(self) -> bool:
        if self.weight is None:
            return False
        off = 0
        base = self.weight.data_ptr()
        es = self.weight.element_size()
        for lin in self.linears:
            w = lin.weight
            if (w.device != self.weight.device or w.dtype != self.weight.dtype
                    or w.data_ptr() != base + off * es or not w.is_contiguous()):
                return False
            off += w.numel()
        if self.bias is not None:
            off, base, es = 0, self.bias.data_ptr(), self.bias.element_size()
            for lin in self.linears:
                b = lin.bias
                if b is None or b.data_ptr() != base + off * es or b.dtype != self.bias.dtype:
                    return False
                off += b.numel()
        elif any(lin.bias is not None for lin in self.linears):
            return False
        return True

    def get(self):
        """(weight [sum(out), in], bias or None) of the concatenation."""
        if not self._views_intact():
            with torch.no_grad():
                w = torch.cat([lin.weight.detach() for lin in self.linears], 0)
                has_b = [lin.bias is not None for lin in self.linears]
                if any(has_b) and not all(has_b):
                    raise ValueError("FusedRows: either every linear has a bias or none")
                b = (torch.cat([lin.bias.detach() for lin in self.linears], 0)
                     if all(has_b) else None)
                off = 0
                for lin in self.linears:
                    n = lin.weight.shape[0]
                    lin.weight.data = w[off:off + n]
                    if b is not None:
                        lin.bias.data = b[off:off + n]
                    off += n
            self.weight, self.bias = w, b
        return self.weight, self.bias
