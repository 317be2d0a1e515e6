"""The kernels, with types and shapes checked on the way in (mirror of engine/h3-core/src/ops.rs).

Each call queues work on the device's stream and returns; the result is there for the next call that uses it. The
names, argument meanings and error behaviour follow ops.rs: a type or shape that does not fit raises ``Error``
before anything is queued, and a failing library call raises ``Error`` with the library's message. The fused
entry points of include/h3hip.h come after the reference's operations.
"""
from __future__ import annotations

from dataclasses import dataclass

from . import api as _api
from .device import DType, Error, Tensor


def _floats(t: Tensor, what: str, n: int) -> int:
    """ops.rs:11-16."""
    if t.dtype != DType.F32 or t.elements() < n:
        raise Error(f"{what} must be float32 with at least {n} values, got {t.dtype} {t.shape}")
    return t.ptr()


def _row_table(t: Tensor, m: int) -> int:
    """ops.rs:18-23."""
    if t.dtype != DType.I32 or t.elements() != m:
        raise Error(f"the row table must be int32 [{m}], got {t.dtype} {t.shape}")
    return t.ptr()


def _dev(t: Tensor):
    if t.dev is None:
        raise Error("the tensor has no device")
    return t.dev


@dataclass
class Int8Linear:
    """A linear layer with int8 weights (ops.rs:25-35)."""

    weight: Tensor            # int8 [N, K]
    scale: Tensor             # float32, 1 or N values
    bias: Tensor | None = None
    group: int | None = None  # ConvRot group size, when the weights were stored rotated

    def inputs(self) -> int:
        return self.weight.shape[1]

    def outputs(self) -> int:
        return self.weight.shape[0]

    def forward(self, x: Tensor, out: Tensor) -> None:
        """out = linear(x): x [M, K] in a float type, out [M, N] in out's type (ops.rs:46-83)."""
        n, k = self.outputs(), self.inputs()
        m = x.elements() // k
        if self.weight.dtype != DType.I8 or self.scale.dtype != DType.F32:
            raise Error("int8_linear: the weight must be int8 and its scale float32")
        if x.elements() != m * k or out.elements() != m * n:
            raise Error(f"int8_linear: x {x.shape} and out {out.shape} do not fit a [{n}, {k}] weight")
        ns = self.scale.elements()
        if ns != 1 and ns != n:
            raise Error(f"int8_linear: {ns} weight scales for {n} outputs")
        bias = _floats(self.bias, "the bias", n) if self.bias is not None else None
        args = (x.ptr(), x.dtype.kernel_code(), m, k, self.weight.ptr(), n, self.scale.ptr(),
                ns, bias, out.ptr(), out.dtype.kernel_code(), self.group or 0,)
        dev = _dev(x)
        dev.check(dev.api.int8_linear(dev.ctx, *args))


@dataclass
class Linear:
    """A plain linear layer (ops.rs:164-237): weight [N, K] in float32, half or bfloat16; bias float32 [N]."""

    weight: Tensor
    bias: Tensor | None = None

    def inputs(self) -> int:
        return self.weight.shape[1]

    def outputs(self) -> int:
        return self.weight.shape[0]

    def forward(self, x: Tensor, out: Tensor) -> None:
        """out = linear(x): x [M, K] in the weight's type, out [M, N] in out's type."""
        n, k = self.outputs(), self.inputs()
        m = x.elements() // k
        if x.dtype != self.weight.dtype:
            raise Error(f"linear: x is {x.dtype} and the weight {self.weight.dtype}; they must be the same type")
        if x.elements() != m * k or out.elements() != m * n:
            raise Error(f"linear: x {x.shape} and out {out.shape} do not fit a [{n}, {k}] weight")
        bias = _floats(self.bias, "the bias", n) if self.bias is not None else None
        dev = _dev(x)
        dev.check(dev.api.linear(dev.ctx, x.ptr(), x.dtype.kernel_code(), m, k, self.weight.ptr(), n, bias, out.ptr(),
                                 out.dtype.kernel_code()))

    def forward_acc(self, x: Tensor, out: Tensor) -> None:
        """out += linear(x) (bias included), x and out in the weight's type."""
        n, k = self.outputs(), self.inputs()
        m = x.elements() // k
        if x.dtype != self.weight.dtype or out.dtype != x.dtype or x.elements() != m * k or out.elements() != m * n:
            raise Error(f"linear_acc: x {x.dtype} {x.shape}, out {out.dtype} {out.shape}, weight [{n}, {k}] {self.weight.dtype}")
        bias = _floats(self.bias, "the bias", n) if self.bias is not None else None
        dev = _dev(x)
        dev.check(dev.api.linear_acc(dev.ctx, x.ptr(), x.dtype.kernel_code(), m, k, self.weight.ptr(), n, bias, out.ptr()))

    def scale_outputs(self, s: Tensor) -> None:
        """Scales output row n of the weight by s[n] (float32 [N]) in place, on the device; the bias too (on the
        host, as the reference does)."""
        n, k = self.outputs(), self.inputs()
        if s.elements() != n or s.dtype != DType.F32:
            raise Error(f"scale_outputs: {s.elements()} factors for {n} outputs")
        dev = _dev(self.weight)
        dev.check(dev.api.scale_rows(dev.ctx, self.weight.ptr(), self.weight.dtype.kernel_code(), n, k, s.ptr()))
        if self.bias is not None:
            import numpy as np

            b = self.bias.to_numpy().astype(np.float32) * s.to_numpy().astype(np.float32)
            self.bias = Tensor.from_numpy(dev, DType.F32, [n], b)
        dev.wait()


@dataclass
class Mod:
    """How a block's tokens are modulated: the row table and the scale/shift tables (ops.rs:239-245)."""

    rows: Tensor   # int32 [M]
    scale: Tensor  # float32 [R, C]
    shift: Tensor  # float32 [R, C]


def rms_norm_mod(x: Tensor, weight: Tensor, eps: float, m: Mod | None, out: Tensor) -> None:
    """Row-wise RMS norm of x [M, C], then * (1 + scale[row]) + shift[row] when m is given; out may be x (ops.rs:249-278)."""
    c = weight.elements()
    rows = x.elements() // c
    if x.elements() != rows * c or out.elements() != x.elements():
        raise Error(f"rms_norm: x {x.shape}, out {out.shape}, {c} features")
    if m is None:
        r = sc = sh = None
    else:
        r, sc, sh = _row_table(m.rows, rows), _floats(m.scale, "scale", c), _floats(m.shift, "shift", c)
    args = (x.ptr(), x.dtype.kernel_code(), rows, c, _floats(weight, "the norm weight", c),
            eps, r, sc, sh, out.ptr(), out.dtype.kernel_code(),)
    dev = _dev(x)
    dev.check(dev.api.rms_norm_mod(dev.ctx, *args))


def layer_norm(x: Tensor, c: int, weight: Tensor | None, bias: Tensor | None, eps: float, out: Tensor) -> None:
    """Layer norm of x [M, C] per row, optional weight and bias (ops.rs:281-294)."""
    rows = x.elements() // max(c, 1)
    if x.elements() != rows * c or out.elements() != x.elements():
        raise Error(f"layer_norm: x {x.shape}, out {out.shape}, {c} features")
    w = _floats(weight, "the norm weight", c) if weight is not None else None
    b = _floats(bias, "the norm bias", c) if bias is not None else None
    args = (x.ptr(), x.dtype.kernel_code(), rows, c, w, b, eps, out.ptr(), out.dtype.kernel_code(),)
    dev = _dev(x)
    dev.check(dev.api.layer_norm(dev.ctx, *args))


@dataclass
class Rows:
    """Token rows of heads x dim features inside a wider buffer: row s at element offset + s * stride (ops.rs:298-326)."""

    t: Tensor
    offset: int
    stride: int
    tokens: int
    heads: int
    dim: int

    def layout(self):
        return (self.tokens, self.heads, self.dim, self.stride)

    def ptr(self) -> int:
        last = self.offset + (max(self.tokens, 1) - 1) * self.stride + self.heads * self.dim
        if self.stride < self.heads * self.dim or last > self.t.elements():
            raise Error(f"rows of {self.heads} x {self.dim} at offset {self.offset} with stride {self.stride} do not fit {self.t.shape}")
        return self.t.ptr() + self.offset * self.t.dtype.size()


def rms_rope(x: Rows, weight: Tensor, eps: float, cs: Tensor, rot_dim: int) -> None:
    """Per-head RMS norm and the rotary rotation, in place; cs float32 [tokens, rot_dim/2, 2] (ops.rs:327-346)."""
    args = (x.ptr(), x.t.dtype.kernel_code(), x.tokens, x.heads, x.dim, x.stride,
            _floats(weight, "the norm weight", x.dim), eps,
            _floats(cs, "the rotation table", x.tokens * rot_dim), rot_dim,)
    dev = _dev(x.t)
    dev.check(dev.api.rms_rope(dev.ctx, *args))


def attention(q: Rows, k: Rows, v: Rows, out: Tensor) -> None:
    """softmax(q k^T / sqrt(D)) v per head; out [tokens, heads * dim] (ops.rs:436-461)."""
    if q.layout() != k.layout() or q.layout() != v.layout():
        raise Error("attention: q, k and v must have the same layout")
    if out.elements() != q.tokens * q.heads * q.dim:
        raise Error(f"attention: out {out.shape} for {q.tokens} tokens of {q.heads} x {q.dim}")
    dev = _dev(out)
    dev.check(dev.api.attention(dev.ctx, q.ptr(), k.ptr(), v.ptr(), q.t.dtype.kernel_code(), q.tokens, q.heads, q.dim,
                                q.stride, out.ptr(), out.dtype.kernel_code()))


def attention_causal(q: Rows, k: Rows, v: Rows, out: Tensor) -> None:
    """The text encoder's causal attention: query i sees keys 0 .. i; q has Hq heads, k and v Hkv (head h reads kv
    head h / (Hq / Hkv)); out [tokens, Hq * dim] in q's type (te.rs:342-347)."""
    if k.layout() != v.layout() or q.tokens != k.tokens or q.dim != k.dim or q.t.dtype != k.t.dtype or k.t.dtype != v.t.dtype:
        raise Error("attention_causal: k and v must share a layout, and q their tokens, head size and type")
    if out.elements() != q.tokens * q.heads * q.dim or out.dtype != q.t.dtype:
        raise Error(f"attention_causal: out {out.dtype} {out.shape} for {q.tokens} tokens of {q.heads} x {q.dim}")
    dev = _dev(out)
    dev.check(dev.api.attention_causal(dev.ctx, q.ptr(), k.ptr(), v.ptr(), q.t.dtype.kernel_code(), q.tokens, q.heads,
                                       k.heads, q.dim, q.stride, k.stride, out.ptr()))


def attention_batch(q: Rows, k: Rows, v: Rows, seqs: int, out: Tensor) -> None:
    """attention over `seqs` equal sequences of the rows, each on its own (ops.rs:405-434)."""
    if q.layout() != k.layout() or q.layout() != v.layout():
        raise Error("attention_batch: q, k and v must have the same layout")
    if seqs == 0 or q.tokens % seqs:
        raise Error(f"attention_batch: {q.tokens} tokens are not {seqs} equal sequences")
    if out.elements() != q.tokens * q.heads * q.dim:
        raise Error(f"attention_batch: out {out.shape} for {q.tokens} tokens of {q.heads} x {q.dim}")
    dev = _dev(out)
    dev.check(dev.api.attention_batch(dev.ctx, q.ptr(), k.ptr(), v.ptr(), q.t.dtype.kernel_code(), seqs, q.tokens // seqs,
                                      q.heads, q.dim, q.stride, out.ptr(), out.dtype.kernel_code()))


def adaln_tables(w: Tensor, b: Tensor, t_emb: Tensor, modalities: int, out: Tensor) -> None:
    """The six AdaLN tables of one block (dit.rs:155-174) on the device: w [6 m C, t_dim], b [6 m C], t_emb
    [R, t_dim] float32; out float32 [6, R * m, C]."""
    if not t_emb.shape or not w.shape or len(w.shape) != 2:
        raise Error("adaln_tables: w [6 m C, t_dim] and t_emb [R, t_dim]")
    t_dim = w.shape[1]
    if t_emb.shape[-1] != t_dim or w.shape[0] % (6 * modalities) or b.elements() != w.shape[0]:
        raise Error(f"adaln_tables: w {w.shape}, b {b.shape}, t_emb {t_emb.shape} for {modalities} modalities")
    c = w.shape[0] // (6 * modalities)
    r = t_emb.elements() // t_dim
    if out.elements() != 6 * r * modalities * c or any(t.dtype != DType.F32 for t in (w, b, t_emb, out)):
        raise Error(f"adaln_tables: out {out.shape} is not float32 [6, {r * modalities}, {c}]")
    dev = _dev(out)
    dev.check(dev.api.adaln_tables(dev.ctx, w.ptr(), b.ptr(), t_emb.ptr(), r, t_dim, modalities, c, out.ptr()))


def rotations(positions: Tensor, inv_freq: Tensor, cs: Tensor) -> None:
    """(cos, sin) of every token's three position axes (dit.rs:188-203) on the device: positions float64 [S, 3],
    inv_freq float32 [n], cs float32 [S, 3 n, 2]."""
    s = positions.elements() // 3
    n = inv_freq.elements()
    if positions.dtype != DType.F64 or inv_freq.dtype != DType.F32 or cs.dtype != DType.F32 or cs.elements() != s * 3 * n * 2:
        raise Error(f"rotations: positions {positions.dtype} {positions.shape}, inv_freq {inv_freq.shape}, cs {cs.shape}")
    dev = _dev(cs)
    dev.check(dev.api.rotations(dev.ctx, positions.ptr(), s, inv_freq.ptr(), n, cs.ptr()))


def swiglu(x: Tensor, out: Tensor) -> None:
    """out[r, i] = silu(x[r, i]) * x[r, C + i]: x [M, 2C], out [M, C] (ops.rs:349-360)."""
    if not out.shape:
        raise Error("swiglu: out has no shape")
    c = out.shape[-1]
    if x.elements() != out.elements() * 2 or c == 0:
        raise Error(f"swiglu: x {x.shape} is not twice out {out.shape}")
    args = (x.ptr(), x.dtype.kernel_code(), out.elements() // c, c, out.ptr(), out.dtype.kernel_code(),)
    dev = _dev(x)
    dev.check(dev.api.swiglu(dev.ctx, *args))


def gate_add(x: Tensor, other: Tensor, rows: Tensor, gate: Tensor) -> None:
    """x[r] += other[r] * gate[rows[r]], in place (ops.rs:363-385)."""
    c = x.shape[-1]
    m = x.elements() // max(c, 1)
    if other.elements() != x.elements():
        raise Error(f"gate_add: x {x.shape} and other {other.shape} differ")
    args = (x.ptr(), x.dtype.kernel_code(), m, c, other.ptr(), other.dtype.kernel_code(),
            _row_table(rows, m), _floats(gate, "the gate", c),)
    dev = _dev(x)
    dev.check(dev.api.gate_add(dev.ctx, *args))


def add(x: Tensor, other: Tensor) -> None:
    """x += other, in place (ops.rs:388-400)."""
    c = x.shape[-1]
    if other.elements() != x.elements():
        raise Error(f"add: x {x.shape} and other {other.shape} differ")
    args = (x.ptr(), x.dtype.kernel_code(), x.elements() // max(c, 1), c, other.ptr(),
            other.dtype.kernel_code(), None, None,)
    dev = _dev(x)
    dev.check(dev.api.gate_add(dev.ctx, *args))


# ---- fused entry points of include/h3hip.h ------------------------------------------------------------------------

@dataclass
class Tables:
    """Modulation tables [R, C] (float32 or bfloat16) and an optional row table (None: every token uses row 0)."""

    scale: Tensor | None = None
    shift: Tensor | None = None
    gate: Tensor | None = None
    rows: Tensor | None = None

    def dtype(self) -> int:
        ts = [t for t in (self.scale, self.shift, self.gate) if t is not None]
        if not ts:
            return _api.F32
        d = ts[0].dtype
        if any(t.dtype != d for t in ts) or d not in (DType.F32, DType.BF16):
            raise Error("tables: scale, shift and gate share one type, float32 or bfloat16")
        return d.kernel_code()

    def check(self, m: int, c: int) -> None:
        for t in (self.scale, self.shift, self.gate):
            if t is not None and (t.elements() < c or t.elements() % c):
                raise Error(f"a table of {t.shape} for {c} features")
        if self.rows is not None:
            _row_table(self.rows, m)


def _p(t: Tensor | None):
    return t.ptr() if t is not None else None


def norm_quant(x: Tensor, weight: Tensor | None, eps: float, tables: Tables | None, q: Tensor, s: Tensor,
               rot: int = _api.ROT_NONE, group: int = 0, h_dtype: DType = DType.BF16) -> None:
    """rms_norm_mod into a virtual h (h_dtype), then the int8 quantizer (optionally rotated): q int8 [M, C], s f32 [M]."""
    c = x.shape[-1]
    m = x.elements() // c
    tb = tables or Tables()
    tb.check(m, c)
    if q.dtype != DType.I8 or q.elements() != m * c or s.dtype != DType.F32 or s.elements() != m:
        raise Error(f"norm_quant: q {q.dtype} {q.shape} / s {s.dtype} {s.shape} for x {x.shape}")
    w = _floats(weight, "the norm weight", c) if weight is not None else None
    args = (x.ptr(), x.dtype.kernel_code(), m, c, w, eps, _p(tb.rows), _p(tb.scale), _p(tb.shift),
            tb.dtype(), h_dtype.kernel_code(), rot, group, q.ptr(), s.ptr(),)
    dev = _dev(x)
    dev.check(dev.api.norm_quant(dev.ctx, *args))


def swiglu_quant(x: Tensor, q: Tensor, s: Tensor, rot: int = _api.ROT_NONE, group: int = 0,
                 h_dtype: DType = DType.BF16) -> None:
    """swiglu of x [M, 2C] into a virtual act (h_dtype), then the int8 quantizer (optionally rotated): q int8 [M, C],
    s f32 [M] - swiglu (ops.rs:349-360) and the quantizer of fc2's int8 linear in one pass (dit.rs:363-364)."""
    if not q.shape or q.dtype != DType.I8:
        raise Error("swiglu_quant: q must be int8 [M, C]")
    c = q.shape[-1]
    m = q.elements() // c
    if c == 0 or x.elements() != 2 * m * c or s.dtype != DType.F32 or s.elements() != m:
        raise Error(f"swiglu_quant: x {x.shape} is not [M, 2C] for q {q.shape}, or s {s.dtype} {s.shape} is not [M]")
    dev = _dev(x)
    dev.check(dev.api.swiglu_quant(dev.ctx, x.ptr(), x.dtype.kernel_code(), m, c, h_dtype.kernel_code(), rot, group,
                                   q.ptr(), s.ptr()))


def norm_mod_act_gate(x: Tensor, norm: int, weight: Tensor | None, bias: Tensor | None, eps: float, tables: Tables | None,
                      act: int, res: Tensor | None, out: Tensor) -> None:
    """out = res + gate * act(norm(x) * (1 + scale) + shift), one pass."""
    c = x.shape[-1]
    m = x.elements() // c
    tb = tables or Tables()
    tb.check(m, c)
    if out.elements() != x.elements() or (res is not None and res.elements() != x.elements()):
        raise Error(f"norm_mod_act_gate: x {x.shape}, res {None if res is None else res.shape}, out {out.shape}")
    w = _floats(weight, "the norm weight", c) if weight is not None else None
    b = _floats(bias, "the norm bias", c) if bias is not None else None
    args = (x.ptr(), x.dtype.kernel_code(), m, c, norm, w, b, eps, _p(tb.rows), _p(tb.scale),
            _p(tb.shift), _p(tb.gate), tb.dtype(), act, _p(res),
            res.dtype.kernel_code() if res is not None else _api.BF16, out.ptr(),
            out.dtype.kernel_code(),)
    dev = _dev(x)
    dev.check(dev.api.norm_mod_act_gate(dev.ctx, *args))


def qk_rms_rope(q: Rows, k: Rows, wq: Tensor, wk: Tensor, eps: float, cs: Tensor, rot_dim: int) -> None:
    """rms_rope of q and of k in one launch (they share the layout and the rotation table)."""
    if q.layout() != k.layout() or q.t.dtype != k.t.dtype:
        raise Error("qk_rms_rope: q and k must have the same layout and type")
    dev = _dev(q.t)
    cs_p = _floats(cs, "the rotation table", q.tokens * rot_dim) if rot_dim else (cs.ptr() if cs is not None else None)
    dev.check(dev.api.qk_rms_rope(dev.ctx, q.ptr(), k.ptr(), q.t.dtype.kernel_code(), q.tokens, q.heads, q.dim, q.stride,
                                  _floats(wq, "the q norm weight", q.dim), _floats(wk, "the k norm weight", q.dim), eps,
                                  cs_p, rot_dim))


def int8_gemm_dequant(q: Tensor, s: Tensor, layer: Int8Linear, act: int, out: Tensor) -> None:
    """out = act(dequant(q . W^T) + bias) from already quantized activations q int8 [M, K], s f32 [M]."""
    n, k = layer.outputs(), layer.inputs()
    m = q.elements() // k
    if q.dtype != DType.I8 or q.elements() != m * k or s.elements() != m or out.elements() != m * n:
        raise Error(f"int8_gemm_dequant: q {q.shape}, s {s.shape}, out {out.shape} for a [{n}, {k}] weight")
    ns = layer.scale.elements()
    bias = _floats(layer.bias, "the bias", n) if layer.bias is not None else None
    args = (q.ptr(), _floats(s, "the row scales", m), m, k, layer.weight.ptr(), n,
            layer.scale.ptr(), ns, bias, act, out.ptr(), out.dtype.kernel_code(),)
    dev = _dev(q)
    dev.check(dev.api.int8_gemm_dequant(dev.ctx, *args))


def int8_quantize(x: Tensor, q: Tensor, s: Tensor, group: int = 0) -> None:
    """The int8 linear's first pass on its own: x [M, K] rotated per `group` features by the regular Hadamard (0:
    none), then per-row codes q int8 [M, K] and scales s float32 [M] (the quantizer of ops.rs:46-83's call)."""
    if not x.shape:
        raise Error("int8_quantize: x has no shape")
    k = x.shape[-1]
    m = x.elements() // max(k, 1)
    if q.dtype != DType.I8 or q.elements() != m * k or s.dtype != DType.F32 or s.elements() != m:
        raise Error(f"int8_quantize: q {q.dtype} {q.shape} / s {s.dtype} {s.shape} for x {x.shape}")
    dev = _dev(x)
    dev.check(dev.api.int8_quantize(dev.ctx, x.ptr(), x.dtype.kernel_code(), m, k, group, q.ptr(), s.ptr()))
