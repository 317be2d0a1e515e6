"""ctypes binding of the CPU oracle (oracle/libh3oracle.so).

TEST INFRASTRUCTURE ONLY: the checker. Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this module; the product (libh3hip.so, the ``sycl_minimax_h3_amd`` package) never does.

Arrays are numpy; 16-bit floats travel as ``uint16`` bit patterns (bf16 or f16 per the dtype code), as the reference
moves them (kernels/h3sycl.cpp:42-63).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

F32, F16, BF16 = 0, 1, 2
ROT_NONE, ROT_REGULAR, ROT_SYLVESTER = 0, 1, 2
ACT_NONE, ACT_GELU_TANH, ACT_SILU = 0, 1, 2
NORM_RMS, NORM_LAYER = 0, 1
SUM, SUMSQ, SUMSQ_DIFF = 0, 1, 2

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libh3oracle.so")


def build() -> str:
    """Compiles the oracle with its Makefile (gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE, "libh3oracle.so"], check=True)
    return _LIB_PATH


_lib = None
vp, i64, i32, f32, u64 = C.c_void_p, C.c_int64, C.c_int, C.c_float, C.c_uint64
_SIGS = {
    "h3o_set_threads": (None, [i32]),
    "h3o_get_threads": (i32, []),
    "h3o_bf16_to_f32": (f32, [C.c_uint16]),
    "h3o_f32_to_bf16": (C.c_uint16, [f32]),
    "h3o_f16_to_f32": (f32, [C.c_uint16]),
    "h3o_f32_to_f16": (C.c_uint16, [f32]),
    "h3o_rng_new": (None, [vp, u64]),
    "h3o_rng_from_state": (None, [vp, vp]),
    "h3o_rng_next_u64": (u64, [vp]),
    "h3o_rng_uniform": (f32, [vp]),
    "h3o_rng_normal": (f32, [vp]),
    "h3o_fill_normal": (None, [u64, f32, i64, vp, i32]),
    "h3o_fill_uniform": (None, [u64, f32, f32, i64, vp]),
    "h3o_choose": (None, [u64, i64, i64, vp]),
    "h3o_canon_sum": (f32, [vp, i64, i32, i32, i32, f32]),
    "h3o_row_lanes": (i32, [i64, i32]),
    "h3o_rms_norm_mod": (i32, [vp, i32, i64, i64, vp, f32, vp, vp, vp, vp, i32]),
    "h3o_layer_norm": (i32, [vp, i32, i64, i64, vp, vp, f32, vp, i32]),
    "h3o_rms_rope": (i32, [vp, i32, i64, i64, i64, i64, vp, f32, vp, i32]),
    "h3o_swiglu": (i32, [vp, i32, i64, i64, vp, i32]),
    "h3o_gate_add": (i32, [vp, i32, i64, i64, vp, i32, vp, vp]),
    "h3o_int8_linear": (i32, [vp, i32, i64, i64, vp, i64, vp, i64, vp, vp, i32, i32]),
    "h3o_rotate_group": (None, [vp, i32, i32]),
    "h3o_hadamard_regular": (None, [i32, vp]),
    "h3o_hadamard_sylvester": (None, [i32, vp]),
    "h3o_quantize_rows": (None, [vp, i64, i64, vp, vp]),
    "h3o_gemm_dequant": (i32, [vp, vp, i64, i64, vp, i64, vp, i64, vp, i32, vp, i32]),
    "h3o_norm_quant": (i32, [vp, i32, i64, i64, vp, f32, vp, vp, vp, i32, i32, i32, i32, vp, vp]),
    "h3o_norm_mod_act_gate": (i32, [vp, i32, i64, i64, i32, vp, vp, f32, vp, vp, vp, vp, i32, i32, vp, i32, vp, i32]),
    "h3o_swiglu_quant": (i32, [vp, i32, i64, i64, i32, i32, i32, vp, vp]),
    "h3o_quantize_act": (i32, [vp, i32, i64, i64, i32, i32, vp, vp]),
    "h3o_attention": (i32, [vp, vp, vp, i32, i64, i64, i64, i64, vp, i32, i32, vp, vp, vp, vp, vp]),
    "h3o_sage_quantize": (None, [vp, i32, i64, i64, i64, i64, vp, vp, vp]),
    "h3o_attention_causal": (i32, [vp, vp, vp, i32, i64, i64, i64, i64, i64, i64, vp]),
    "h3o_adaln_tables": (None, [vp, vp, vp, i64, i64, i64, i64, vp]),
    "h3o_linear": (None, [vp, i32, i64, i64, vp, i64, vp, vp, i32, i32]),
    "h3o_scale_rows": (None, [vp, i32, i64, i64, vp]),
    "h3o_rotations": (None, [vp, i64, vp, i64, vp]),
    "h3o_act": (f32, [f32, i32]),
    "h3o_act_n": (None, [vp, i64, i32, vp]),
    "h3o_compare": (None, [vp, vp, i64, vp, vp]),
    "h3o_layout": (i64, [i64, i64, i64, i64, i64, vp, vp, vp, i64, vp, i64, vp, vp, i64]),
    "h3o_last_error": (C.c_char_p, []),
}


def lib():
    """The loaded oracle library (built on first use when missing)."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    """Data pointer of a numpy array (None passes NULL)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _check(rc):
    if rc != 0:
        raise RuntimeError(lib().h3o_last_error().decode())


def set_threads(n: int) -> None:
    lib().h3o_set_threads(int(n))


# ---- element types -------------------------------------------------------------------------------------------
def to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even, inf/nan truncated (engine/h3-core/src/dtype.rs:59-66)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    special = (u & 0x7F800000) == 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(special, u >> 16, r)
    return r.astype(np.uint16)


def from_bf16(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_f16(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def from_f16(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


def to_dt(x: np.ndarray, dt: int) -> np.ndarray:
    if dt == BF16:
        return to_bf16(x)
    if dt == F16:
        return to_f16(x)
    return np.ascontiguousarray(x, dtype=np.float32)


def from_dt(b: np.ndarray, dt: int) -> np.ndarray:
    if dt == BF16:
        return from_bf16(b)
    if dt == F16:
        return from_f16(b)
    return np.ascontiguousarray(b, dtype=np.float32)


def np_dtype(dt: int):
    return np.float32 if dt == F32 else np.uint16


# ---- seeded inputs -------------------------------------------------------------------------------------------
class Rng:
    """engine/h3-core/src/rng.rs: xoshiro256** seeded by splitmix64, Box-Muller normals."""

    def __init__(self, seed: int | None = 0, state=None):
        self._s = (C.c_uint64 * 4)()
        if state is not None:
            st = (C.c_uint64 * 4)(*state)
            lib().h3o_rng_from_state(C.addressof(self._s), C.addressof(st))
        else:
            lib().h3o_rng_new(C.addressof(self._s), int(seed))

    @property
    def state(self):
        return [int(v) for v in self._s]

    def next_u64(self) -> int:
        return int(lib().h3o_rng_next_u64(C.addressof(self._s)))

    def uniform(self) -> float:
        return float(lib().h3o_rng_uniform(C.addressof(self._s)))

    def normal(self) -> float:
        return float(lib().h3o_rng_normal(C.addressof(self._s)))


def normal(seed: int, n: int, scale: float = 1.0, dt: int = F32) -> np.ndarray:
    out = np.empty(n, dtype=np_dtype(dt))
    lib().h3o_fill_normal(seed, scale, n, _p(out), dt)
    return out


def uniform(seed: int, n: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().h3o_fill_uniform(seed, lo, hi, n, _p(out))
    return out


def choose(seed: int, n: int, k: int) -> np.ndarray:
    out = np.empty(k, dtype=np.int64)
    lib().h3o_choose(seed, n, k, _p(out))
    return out


def canon_sum(x: np.ndarray, V: int, L: int, kind: int = SUM, mean: float = 0.0) -> float:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return float(lib().h3o_canon_sum(_p(x), x.size, V, L, kind, mean))


def row_lanes(n: int, V: int) -> int:
    """Lanes per row of the row-wise operations' canonical order."""
    return int(lib().h3o_row_lanes(n, V))


# ---- operations ----------------------------------------------------------------------------------------------
def rms_norm_mod(x, x_dt, M, C_, weight, eps, rows=None, scale=None, shift=None, out_dt=None):
    out_dt = x_dt if out_dt is None else out_dt
    out = np.empty(M * C_, dtype=np_dtype(out_dt))
    _check(lib().h3o_rms_norm_mod(_p(x), x_dt, M, C_, _p(weight), eps, _p(rows), _p(scale), _p(shift), _p(out), out_dt))
    return out


def layer_norm(x, x_dt, M, C_, weight, bias, eps, out_dt=None):
    out_dt = x_dt if out_dt is None else out_dt
    out = np.empty(M * C_, dtype=np_dtype(out_dt))
    _check(lib().h3o_layer_norm(_p(x), x_dt, M, C_, _p(weight), _p(bias), eps, _p(out), out_dt))
    return out


def rms_rope(x, x_dt, M, H, D, stride, weight, eps, cs, rot_dim):
    """In place on a copy; returns the copy."""
    y = np.array(x, copy=True)
    _check(lib().h3o_rms_rope(_p(y), x_dt, M, H, D, stride, _p(weight), eps, _p(cs), rot_dim))
    return y


def swiglu(x, x_dt, M, C_, out_dt=None):
    out_dt = x_dt if out_dt is None else out_dt
    out = np.empty(M * C_, dtype=np_dtype(out_dt))
    _check(lib().h3o_swiglu(_p(x), x_dt, M, C_, _p(out), out_dt))
    return out


def gate_add(x, x_dt, M, C_, other, other_dt, rows=None, gate=None):
    y = np.array(x, copy=True)
    _check(lib().h3o_gate_add(_p(y), x_dt, M, C_, _p(other), other_dt, _p(rows), _p(gate)))
    return y


def int8_linear(x, x_dt, M, K, w, N, wscale, bias=None, out_dt=BF16, group=0):
    out = np.empty(M * N, dtype=np_dtype(out_dt))
    _check(lib().h3o_int8_linear(_p(x), x_dt, M, K, _p(w), N, _p(wscale), wscale.size, _p(bias), _p(out), out_dt, group))
    return out


def rotate_group(y: np.ndarray, kind: int) -> np.ndarray:
    y = np.array(y, dtype=np.float32, copy=True)
    lib().h3o_rotate_group(_p(y), y.size, kind)
    return y


def hadamard(g: int, kind: int) -> np.ndarray:
    h = np.empty((g, g), dtype=np.float32)
    (lib().h3o_hadamard_regular if kind == ROT_REGULAR else lib().h3o_hadamard_sylvester)(g, _p(h))
    return h


def quantize_rows(y: np.ndarray, M: int, K: int):
    y = np.ascontiguousarray(y, dtype=np.float32)
    q = np.empty(M * K, dtype=np.int8)
    s = np.empty(M, dtype=np.float32)
    lib().h3o_quantize_rows(_p(y), M, K, _p(q), _p(s))
    return q, s


def gemm_dequant(q, s, M, K, w, N, wscale, bias=None, act=ACT_NONE, out_dt=BF16):
    out = np.empty(M * N, dtype=np_dtype(out_dt))
    _check(lib().h3o_gemm_dequant(_p(q), _p(s), M, K, _p(w), N, _p(wscale), wscale.size, _p(bias), act, _p(out), out_dt))
    return out


def norm_quant(x, x_dt, M, C_, weight, eps, rows=None, scale=None, shift=None, tab_dt=F32, h_dt=BF16,
               rot=ROT_NONE, group=0):
    q = np.empty(M * C_, dtype=np.int8)
    s = np.empty(M, dtype=np.float32)
    _check(lib().h3o_norm_quant(_p(x), x_dt, M, C_, _p(weight), eps, _p(rows), _p(scale), _p(shift), tab_dt, h_dt, rot,
                                group, _p(q), _p(s)))
    return q, s


def swiglu_quant(x, x_dt, M, C_, h_dt=BF16, rot=ROT_NONE, group=0):
    """x [M, 2C] -> (q int8 [M*C], s f32 [M]): swiglu into h_dt, then the (rotated) quantizer."""
    q = np.empty(M * C_, dtype=np.int8)
    s = np.empty(M, dtype=np.float32)
    _check(lib().h3o_swiglu_quant(_p(x), x_dt, M, C_, h_dt, rot, group, _p(q), _p(s)))
    return q, s


def quantize_act(x, x_dt, M, C_, rot=ROT_NONE, group=0):
    """x [M, C] -> (q int8 [M*C], s f32 [M]): the (rotated) quantizer on x itself."""
    q = np.empty(M * C_, dtype=np.int8)
    s = np.empty(M, dtype=np.float32)
    _check(lib().h3o_quantize_act(_p(x), x_dt, M, C_, rot, group, _p(q), _p(s)))
    return q, s


def attention(q, k, v, dt, S, H, D, stride=None, out_dt=BF16, sage=True):
    """softmax(q k^T / sqrt(D)) v per head -> out [S * H * D] in out_dt; with sage also the int8 codes, scales and
    k's mean: (out, iq [H, S, D], ik, qs [H, nb], ks, kmean [H, D])."""
    stride = H * D if stride is None else stride
    nb = (S + 63) // 64
    out = np.empty(S * H * D, dtype=np_dtype(out_dt))
    iq, ik = np.zeros(H * S * D, np.int8), np.zeros(H * S * D, np.int8)
    qs, ks = np.zeros(H * nb, np.float32), np.zeros(H * nb, np.float32)
    km = np.zeros(H * D, np.float32)
    _check(lib().h3o_attention(_p(q), _p(k), _p(v), dt, S, H, D, stride, _p(out), out_dt, int(sage), _p(iq), _p(ik),
                               _p(qs), _p(ks), _p(km)))
    return (out, iq, ik, qs, ks, km) if sage else out


def attention_causal(q, k, v, dt, L, Hq, Hkv, D, qs=None, kvs=None):
    """causal softmax(q k^T / sqrt(D)) v with kv heads shared by Hq / Hkv query heads -> out [L * Hq * D] in dt"""
    qs = Hq * D if qs is None else qs
    kvs = Hkv * D if kvs is None else kvs
    out = np.empty(L * Hq * D, dtype=np_dtype(dt))
    _check(lib().h3o_attention_causal(_p(q), _p(k), _p(v), dt, L, Hq, Hkv, D, qs, kvs, _p(out)))
    return out


def sage_quantize(src, dt, S, H, D, stride=None, mean=None):
    stride = H * D if stride is None else stride
    nb = (S + 63) // 64
    codes, scales = np.zeros(H * S * D, np.int8), np.zeros(H * nb, np.float32)
    lib().h3o_sage_quantize(_p(src), dt, S, H, D, stride, _p(mean), _p(codes), _p(scales))
    return codes, scales


def linear(x, dt, M, K, w, N, bias=None, out_dt=BF16, acc_into=None):
    """out [M*N] = x w^T + bias in out_dt; acc_into: a previous output (dt) to accumulate into (h3s_linear_acc)"""
    out = np.array(acc_into, copy=True) if acc_into is not None else np.empty(M * N, dtype=np_dtype(out_dt))
    lib().h3o_linear(_p(x), dt, M, K, _p(w), N, _p(bias), _p(out), out_dt, int(acc_into is not None))
    return out


def scale_rows(x, dt, M, C_, s):
    out = np.array(x, copy=True)
    lib().h3o_scale_rows(_p(out), dt, M, C_, _p(s))
    return out


def adaln_tables(w, b, t_emb, R, t_dim, m, C_):
    """the six AdaLN tables [6, R * m, C] of one block (dit.rs:155-174)"""
    out = np.empty(6 * R * m * C_, np.float32)
    lib().h3o_adaln_tables(_p(w), _p(b), _p(t_emb), R, t_dim, m, C_, _p(out))
    return out


def rotations(positions, S, inv_freq):
    """(cos, sin) [S, 3 n, 2] of each token's three axes (dit.rs:188-203)"""
    n = inv_freq.size
    cs = np.empty(S * 3 * n * 2, np.float32)
    lib().h3o_rotations(_p(np.ascontiguousarray(positions, np.float64)), S, _p(inv_freq), n, _p(cs))
    return cs


def norm_mod_act_gate(x, x_dt, M, C_, norm, weight, bias, eps, rows=None, scale=None, shift=None, gate=None,
                      tab_dt=F32, act=ACT_NONE, res=None, res_dt=BF16, out_dt=BF16):
    out = np.empty(M * C_, dtype=np_dtype(out_dt))
    _check(lib().h3o_norm_mod_act_gate(_p(x), x_dt, M, C_, norm, _p(weight), _p(bias), eps, _p(rows), _p(scale),
                                       _p(shift), _p(gate), tab_dt, act, _p(res), res_dt, _p(out), out_dt))
    return out


def act(v: float, kind: int) -> float:
    return float(lib().h3o_act(v, kind))


def act_n(v: np.ndarray, kind: int) -> np.ndarray:
    """h3o_act on every value of a float32 array"""
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty_like(v)
    lib().h3o_act_n(_p(v), v.size, kind, _p(out))
    return out


TOK_TEXT, TOK_COND, TOK_COND_AUDIO, TOK_REF_AUDIO, TOK_AUDIO, TOK_VIDEO = range(6)


def layout(text_len, latent_t, latent_h, latent_w, audio_t, keyframes=(), ref_audio=()):
    """positions float64 [tokens, 3] and kinds int32 [tokens] of one denoiser call (layout.rs:107-176); keyframes:
    (frame_index, video latent frames or None, audio latent frames or None)"""
    kf_i = np.array([k[0] for k in keyframes], np.float64)
    kf_v = np.array([-1 if k[1] is None else k[1] for k in keyframes], np.int64)
    kf_a = np.array([-1 if k[2] is None else k[2] for k in keyframes], np.int64)
    refs = np.array(list(ref_audio), np.int64)
    args = (text_len, latent_t, latent_h, latent_w, audio_t, _p(kf_i), _p(kf_v), _p(kf_a), len(keyframes), _p(refs),
            refs.size)
    n = lib().h3o_layout(*args, None, None, 0)
    if n < 0:
        raise RuntimeError(lib().h3o_last_error().decode())
    pos, kinds = np.empty((n, 3), np.float64), np.empty(n, np.int32)
    lib().h3o_layout(*args, _p(pos), _p(kinds), n)
    return pos, kinds


def compare(a: np.ndarray, b: np.ndarray):
    """reference::compare: (relative L2 error, cosine) of a against b, in float64."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    rel, cos = C.c_double(), C.c_double()
    lib().h3o_compare(_p(a), _p(b), a.size, C.byref(rel), C.byref(cos))
    return rel.value, cos.value
