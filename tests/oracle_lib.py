"""ctypes access to the CPU oracle (oracle/liboracle.so) and the reference-kernel shim (oracle/_ref/libdllm_ref.so),
plus the decoder configurations, tensor names and fixture weights the parity tests use.

Test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.
Names, shapes and orders follow src/etalii_dllm/architecture.py:418-468 and modelfile.py:40-47 of the reference;
fixture weights follow tests/model_fixtures.py:216-336.
"""

from __future__ import annotations

import ctypes as C
import hashlib
import math
import re
from dataclasses import dataclass, replace
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_SO = ROOT / "oracle" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libdllm_ref.so"

_f32p = C.POINTER(C.c_float)
_f64p = C.POINTER(C.c_double)
_i64p = C.POINTER(C.c_int64)
_sz = C.c_size_t


class OrcConfig(C.Structure):
    _fields_ = [(name, C.c_int64) for name in (
        "vocab", "hidden", "inter", "layers", "heads", "kv_heads", "head_dim", "attn_bias", "qk_norm", "window",
        "tied", "experts", "topk", "normalize", "expert_inter", "rotary_dim")] + [
        ("eps", C.c_double), ("rope_theta", C.c_double), ("attention_scale", C.c_double),
        ("inv_freq", C.c_void_p), ("rope_attention_factor", C.c_double), ("embedding_multiplier", C.c_double),
        ("residual_multiplier", C.c_double), ("logits_scaling", C.c_double), ("dense_layers", C.c_int64),
        ("norm_placement", C.c_int64), ("norm_unit_offset", C.c_int64), ("activation", C.c_int64),
        ("full_attention_layers", C.c_int64), ("local_rope_theta", C.c_double), ("attention_softcap", C.c_double),
        ("logits_softcap", C.c_double), ("shared_inter", C.c_int64), ("shared_gate", C.c_int64),
        ("dense_layer_flags", C.c_void_p), ("full_attention_layer_flags", C.c_void_p)]


class OrcRopeScaling(C.Structure):
    _fields_ = [("kind", C.c_int64)] + [(name, C.c_double) for name in (
        "factor", "low_freq_factor", "high_freq_factor", "original", "beta_fast", "beta_slow")] + [
        ("truncate", C.c_int64), ("factors", C.c_void_p)]


ROPE_KINDS = {"default": 0, "linear": 1, "llama3": 2, "longrope": 3, "yarn": 4}


class OrcAdamW(C.Structure):
    _fields_ = [(name, C.c_double) for name in (
        "lr", "beta1", "beta2", "eps", "weight_decay", "max_grad_norm", "router_aux_loss")] + [("step", C.c_int64)]


def ptr(a: np.ndarray | None, kind=_f32p):
    if a is None:
        return None
    assert a.flags.c_contiguous
    return a.ctypes.data_as(kind)


_libs: dict[str, C.CDLL] = {}


def oracle() -> C.CDLL:
    if "oracle" not in _libs:
        lib = C.CDLL(str(ORACLE_SO))
        for name in ("orc_exp", "orc_log", "orc_sin", "orc_cos", "orc_tanh", "orc_sigmoid"):
            getattr(lib, name).restype = C.c_double
            getattr(lib, name).argtypes = [C.c_double]
        lib.orc_cross_entropy.restype = C.c_double
        lib.orc_sum_squares.restype = C.c_double
        lib.orc_default_ops.restype = C.c_void_p
        lib.orc_silu.restype = C.c_float
        lib.orc_silu.argtypes = [C.c_float]
        lib.orc_silu_backward.restype = C.c_float
        lib.orc_silu_backward.argtypes = [C.c_float, C.c_float]
        lib.orc_gelu_tanh.restype = C.c_float
        lib.orc_gelu_tanh.argtypes = [C.c_float]
        lib.orc_gelu_tanh_backward.restype = C.c_float
        lib.orc_gelu_tanh_backward.argtypes = [C.c_float, C.c_float]
        lib.orc_softcap_backward.restype = C.c_float
        lib.orc_softcap_backward.argtypes = [C.c_float, C.c_float, C.c_double]
        lib.orc_random_next.restype = C.c_uint64
        lib.orc_window_gradients.argtypes = [C.c_void_p, C.POINTER(OrcConfig), C.POINTER(_f32p), _i64p, _i64p,
                                             C.c_int64, C.c_double, C.c_double, C.POINTER(_f32p), _f64p, _f64p]
        lib.orc_train_step.argtypes = [C.c_void_p, C.POINTER(OrcConfig), C.POINTER(_f32p), C.POINTER(_f32p),
                                       C.POINTER(_f32p), C.POINTER(_f32p), _i64p, C.c_int64, _i64p, _i64p, _i64p,
                                       C.c_int64, C.POINTER(OrcAdamW), _f64p, _f64p]
        lib.orc_logits.argtypes = [C.c_void_p, C.POINTER(OrcConfig), C.POINTER(_f32p), _i64p, C.c_int64, _f32p]
        _libs["oracle"] = lib
    return _libs["oracle"]


def reference_available() -> bool:
    return REF_SO.exists()


def ref() -> C.CDLL:
    if "ref" not in _libs:
        lib = C.CDLL(str(REF_SO))
        for name in ("ref_exp", "ref_log", "ref_sin", "ref_cos", "ref_tanh", "ref_sigmoid"):
            getattr(lib, name).restype = C.c_double
            getattr(lib, name).argtypes = [C.c_double]
        lib.ref_ops.restype = C.c_void_p
        lib.ref_silu.restype = C.c_float
        lib.ref_silu.argtypes = [C.c_float]
        lib.ref_silu_backward.restype = C.c_float
        lib.ref_silu_backward.argtypes = [C.c_float, C.c_float]
        lib.ref_gelu_tanh.restype = C.c_float
        lib.ref_gelu_tanh.argtypes = [C.c_float]
        lib.ref_gelu_tanh_backward.restype = C.c_float
        lib.ref_gelu_tanh_backward.argtypes = [C.c_float, C.c_float]
        lib.ref_softcap_backward.restype = C.c_float
        lib.ref_softcap_backward.argtypes = [C.c_float, C.c_float, C.c_double]
        lib.ref_random_first.restype = C.c_uint64
        lib.ref_random_first.argtypes = [C.c_uint64]
        lib.ref_threads.restype = C.c_size_t
        _libs["ref"] = lib
    return _libs["ref"]


# ---- the kernel table, callable from Python for either library ----

class _OpsTable(C.Structure):
    _fields_ = [(name, C.c_void_p) for name in (
        "linear", "linear_backward", "rms_norm", "rms_norm_backward", "rope", "attention", "attention_backward", "silu",
        "swiglu", "silu_backward", "cross_entropy", "embedding_backward", "sum_squares", "adamw_step", "softmax",
        "moe_route", "moe_route_backward", "column_mean", "dot")]


_SIGS = {
    "linear": (None, [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz]),
    "linear_backward": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz]),
    "rms_norm": (None, [_f32p, _f32p, _f32p, _sz, _sz, C.c_double, C.c_int]),
    "rms_norm_backward": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _sz, _sz, C.c_double, C.c_int]),
    "rope": (None, [_f32p, _i64p, _f64p, _f32p, _sz, _sz, _sz, _sz, C.c_int, C.c_int]),
    "attention": (None, [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _sz, _sz, C.c_double, C.c_int, _sz, _sz,
                         C.c_double]),
    "attention_backward": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _sz, _sz,
                                  C.c_double, C.c_int, _sz, _sz, C.c_double]),
    "silu": (None, [_f32p, _f32p, _sz]),
    "swiglu": (None, [_f32p, _f32p, _f32p, _sz]),
    "silu_backward": (None, [_f32p, _f32p, _f32p, _sz]),
    "cross_entropy": (C.c_double, [_f32p, _i64p, _f32p, _sz, _sz, C.c_double]),
    "embedding_backward": (C.c_int, [_f32p, _i64p, _f32p, _sz, _sz, _sz]),
    "sum_squares": (C.c_double, [_f32p, _sz]),
    "adamw_step": (None, [_f32p, _f32p, _f32p, _f32p, _sz] + [C.c_double] * 8),
    "softmax": (None, [_f32p, _f32p, _sz]),
    "moe_route": (None, [_f32p, _i64p, _f32p, _sz, _sz, _sz, C.c_int]),
    "moe_route_backward": (None, [_f32p, _i64p, _f32p, _f32p, _f32p, _sz, _sz, _sz, C.c_int]),
    "column_mean": (None, [_f32p, _f32p, _sz, _sz]),
    "dot": (C.c_float, [_f32p, _f32p, _sz]),
}


class Kernels:
    """NumPy-level calls of one kernel table (the oracle's or the reference's), with the reference binding's
    argument conventions (cpp/kernels.cpp)."""

    def __init__(self, table_address: int, name: str) -> None:
        self.name = name
        self.address = table_address
        table = _OpsTable.from_address(table_address)
        self._fn = {}
        for field, (restype, argtypes) in _SIGS.items():
            self._fn[field] = C.CFUNCTYPE(restype, *argtypes)(getattr(table, field))

    def linear(self, x, w, bias=None):
        rows, inf = x.shape[0], x.shape[1]
        out = np.empty((rows, w.shape[0]), np.float32)
        self._fn["linear"](ptr(x), ptr(w), ptr(bias), ptr(out), rows, inf, w.shape[0])
        return out

    def linear_backward(self, x, w, dy, with_bias=False):
        rows, inf, outf = x.shape[0], w.shape[1], w.shape[0]
        dx = np.empty((rows, inf), np.float32)
        dw = np.empty((outf, inf), np.float32)
        db = np.empty(outf, np.float32) if with_bias else None
        self._fn["linear_backward"](ptr(x), ptr(w), ptr(dy), ptr(dx), ptr(dw), ptr(db), rows, inf, outf)
        return dx, dw, db

    def rms_norm(self, x, w, eps=1e-6, unit_offset=False):
        out = np.empty_like(x)
        dim = x.shape[-1]
        self._fn["rms_norm"](ptr(x), ptr(w), ptr(out), x.size // dim, dim, eps, int(unit_offset))
        return out

    def rms_norm_backward(self, x, w, dy, eps=1e-6, unit_offset=False):
        dim = x.shape[-1]
        dx = np.empty_like(x)
        dw = np.empty(dim, np.float32)
        self._fn["rms_norm_backward"](ptr(x), ptr(w), ptr(dy), ptr(dx), ptr(dw), x.size // dim, dim, eps,
                                      int(unit_offset))
        return dx, dw

    def rope(self, x, positions, inv_freq, interleaved=False, inverse=False):
        out = np.empty_like(x)
        t, h, d = x.shape
        self._fn["rope"](ptr(x), ptr(positions, _i64p), ptr(inv_freq, _f64p), ptr(out), t, h, d, 2 * len(inv_freq),
                         int(interleaved), int(inverse))
        return out

    def attention(self, q, k, v, scale, causal=True, q_offset=0, window=0, softcap=0.0):
        out = np.empty((q.shape[0], q.shape[1], v.shape[2]), np.float32)
        self._fn["attention"](ptr(q), ptr(k), ptr(v), ptr(out), q.shape[0], k.shape[0], q.shape[1], k.shape[1],
                              q.shape[2], v.shape[2], scale, int(causal), q_offset, window, softcap)
        return out

    def attention_backward(self, q, k, v, dout, scale, causal=True, q_offset=0, window=0, softcap=0.0):
        dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
        self._fn["attention_backward"](ptr(q), ptr(k), ptr(v), ptr(dout), ptr(dq), ptr(dk), ptr(dv), q.shape[0],
                                       k.shape[0], q.shape[1], k.shape[1], q.shape[2], v.shape[2], scale,
                                       int(causal), q_offset, window, softcap)
        return dq, dk, dv

    def silu(self, x):
        out = np.empty_like(x)
        self._fn["silu"](ptr(x), ptr(out), x.size)
        return out

    def swiglu(self, gate, up):
        out = np.empty_like(gate)
        self._fn["swiglu"](ptr(gate), ptr(up), ptr(out), gate.size)
        return out

    def silu_backward(self, x, dy):
        out = np.empty_like(x)
        self._fn["silu_backward"](ptr(x), ptr(dy), ptr(out), x.size)
        return out

    def cross_entropy(self, logits, targets, scale=1.0):
        d = np.empty_like(logits)
        loss = self._fn["cross_entropy"](ptr(logits), ptr(targets, _i64p), ptr(d), logits.shape[0], logits.shape[1],
                                         scale)
        return loss, d

    def embedding_backward(self, dy, tokens, vocab):
        out = np.empty((vocab, dy.shape[1]), np.float32)
        rc = self._fn["embedding_backward"](ptr(dy), ptr(tokens, _i64p), ptr(out), dy.shape[0], dy.shape[1], vocab)
        if rc != 0:
            raise ValueError("token id out of range")
        return out

    def sum_squares(self, v):
        return self._fn["sum_squares"](ptr(v), v.size)

    def adamw_step(self, p, g, m, v, lr, b1, b2, eps, wd, bc1, bc2, gs=1.0):
        self._fn["adamw_step"](ptr(p), ptr(g), ptr(m), ptr(v), p.size, lr, b1, b2, eps, wd, bc1, bc2, gs)

    def softmax(self, x):
        out = np.empty_like(x)
        self._fn["softmax"](ptr(x), ptr(out), x.size)
        return out

    def moe_route(self, logits, k, normalize):
        rows, e = logits.shape
        idx = np.empty((rows, k), np.int64)
        w = np.empty((rows, k), np.float32)
        self._fn["moe_route"](ptr(logits), ptr(idx, _i64p), ptr(w), rows, e, k, int(normalize))
        return idx, w

    def moe_route_backward(self, logits, idx, dweights, dprob, normalize):
        rows, e = logits.shape
        out = np.empty_like(logits)
        self._fn["moe_route_backward"](ptr(logits), ptr(idx, _i64p), ptr(dweights), ptr(dprob), ptr(out), rows, e,
                                       idx.shape[1], int(normalize))
        return out

    def column_mean(self, x):
        out = np.empty(x.shape[1], np.float32)
        self._fn["column_mean"](ptr(x), ptr(out), x.shape[0], x.shape[1])
        return out

    def dot(self, a, b):
        return self._fn["dot"](ptr(a), ptr(b), a.size)


def oracle_kernels() -> Kernels:
    return Kernels(oracle().orc_default_ops(), "oracle")


def ref_kernels() -> Kernels:
    return Kernels(ref().ref_ops(), "reference")


def fill_gaussian(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    oracle().orc_fill_gaussian(C.c_uint64(seed), ptr(out), C.c_size_t(n))
    return out


def gaussian(seed: int, *shape: int, scale: float = 1.0) -> np.ndarray:
    values = fill_gaussian(seed, int(np.prod(shape))).reshape(shape)
    return values if scale == 1.0 else values * np.float32(scale)


def rope_inv_freq(rotary_dim: int, theta: float) -> np.ndarray:
    out = np.empty(rotary_dim // 2, np.float64)
    oracle().orc_rope_inv_freq(C.c_size_t(rotary_dim), C.c_double(theta), ptr(out, _f64p))
    return out


def rope_inv_freq_scaled(rotary_dim: int, theta: float, scaling: dict | None = None) -> np.ndarray:
    """The oracle's rope_inv_freq with a Hugging Face rope_scaling dict (numerics.py:267-349)."""
    sc = OrcRopeScaling()
    kind = "default" if not scaling else str(scaling.get("rope_type", scaling.get("type", "default")))
    sc.kind = ROPE_KINDS[kind]
    keep = None
    if scaling:
        sc.factor = float(scaling.get("factor", 1.0))
        sc.low_freq_factor = float(scaling.get("low_freq_factor", 1.0))
        sc.high_freq_factor = float(scaling.get("high_freq_factor", 4.0))
        default_original = 8192 if kind == "llama3" else 0
        sc.original = float(scaling.get("original_max_position_embeddings", default_original))
        sc.beta_fast = float(scaling.get("beta_fast", 32.0))
        sc.beta_slow = float(scaling.get("beta_slow", 1.0))
        sc.truncate = int(bool(scaling.get("truncate", True)))
        if kind == "longrope":
            name = "long_factor" if scaling.get("factor_set") == "long" else "short_factor"
            keep = np.ascontiguousarray(scaling[name], dtype=np.float64)
            assert keep.size == rotary_dim // 2
            sc.factors = keep.ctypes.data
    out = np.empty(rotary_dim // 2, np.float64)
    rc = oracle().orc_rope_inv_freq_scaled(C.c_size_t(rotary_dim), C.c_double(theta), C.byref(sc), ptr(out, _f64p))
    assert rc == 0
    return out


def tensor_fingerprint(values: np.ndarray) -> str:
    """Tensor.fingerprint (src/etalii_dllm/tensor.py:93-98): SHA-256 of the shape as int64 LE, '|', then the bits."""
    digest = hashlib.sha256(np.asarray(values.shape, dtype="<i8").tobytes())
    digest.update(b"|")
    digest.update(np.ascontiguousarray(values).tobytes())
    return digest.hexdigest()


def fingerprint(values: np.ndarray) -> str:
    """numerics.fingerprint (numerics.py:76-79): SHA-256 of the little-endian float32 bits."""
    return hashlib.sha256(np.ascontiguousarray(values, dtype="<f4").tobytes()).hexdigest()


# ---- decoder configurations ----

@dataclass(frozen=True)
class Decoder:
    family: str
    vocab: int
    hidden: int
    inter: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    eps: float
    rope_theta: float
    tied: bool
    attn_bias: bool = False
    qk_norm: int = 0  # 0 none, 1 per head, 2 whole projection
    window: int = 0
    experts: int = 0
    topk: int = 0
    normalize: bool = False
    expert_inter: int = 0
    rotary_dim: int = 0  # 0: head_dim (partial rotary: the first rotary_dim dimensions of each head rotate)
    inv_freq: tuple[float, ...] | None = None  # scaled inverse frequencies (rope_scaling), rotary_dim / 2 of them
    rope_attention_factor: float = 1.0  # LongRoPE / YaRN attention factor folded into the q/k rows
    # a Hugging Face rope_scaling dict as (key, value) pairs (lists as tuples); without inv_freq, the frequencies are
    # computed from it when the configuration is handed to the oracle
    rope_scaling: tuple | None = None
    # Granite's multipliers (architecture.py:95-100, importer.py:427-434); attention_multiplier replaces the
    # attention scale 1/sqrt(head_dim) (architecture.py:311-312)
    embedding_multiplier: float = 1.0
    attention_multiplier: float | None = None
    residual_multiplier: float = 1.0
    logits_scaling: float = 1.0
    dense_layers: tuple[int, ...] = ()  # layers keeping a dense MLP in a model with experts (architecture.py:128)
    norm_placement: int = 0  # architecture.py:315-320: 0 pre, 1 post (OLMo 2), 2 sandwich (Gemma 2 and 3)
    # Gemma (architecture.py, importer.py:283-345, 416-424, 438-461): norms as 1 + w, GELU-tanh MLPs, the window on
    # the layers in window_layers only (None: every layer), a RoPE base of their own for those, soft-capped scores and
    # logits
    unit_offset: bool = False
    activation: int = 0  # 0 SiLU, 1 GELU (tanh approximation)
    window_layers: tuple[int, ...] | None = None
    local_rope_theta: float | None = None
    attention_softcap: float | None = None
    logits_softcap: float | None = None
    shared_inter: int = 0  # a shared expert's intermediate size in the sparse layers (Qwen2-MoE, Granite MoE shared)
    shared_gate: bool = False  # the shared expert's output times the sigmoid of a [1, hidden] gate (Qwen2-MoE)

    def full_attention_mask(self) -> int:
        """Bit l set: layer l ignores the sliding window (not in window_layers)."""
        if self.window_layers is None:
            return 0
        return sum(1 << layer for layer in range(self.layers) if layer not in self.window_layers)

    def is_sparse(self, layer: int) -> bool:
        """architecture.py:344-346."""
        return self.experts > 0 and layer not in self.dense_layers

    def scaling(self) -> dict | None:
        if not self.rope_scaling:
            return None
        return {k: list(v) if isinstance(v, tuple) else v for k, v in self.rope_scaling}

    @property
    def attention_scale(self) -> float:
        return 1.0 / math.sqrt(self.head_dim) if self.attention_multiplier is None else self.attention_multiplier

    def c(self) -> OrcConfig:
        cfg = OrcConfig(self.vocab, self.hidden, self.inter, self.layers, self.heads, self.kv_heads, self.head_dim,
                        int(self.attn_bias), self.qk_norm, self.window, int(self.tied), self.experts, self.topk,
                        int(self.normalize), self.expert_inter or self.inter, self.rotary_dim or self.head_dim,
                        self.eps, self.rope_theta, self.attention_scale, None, self.rope_attention_factor,
                        self.embedding_multiplier, self.residual_multiplier, self.logits_scaling,
                        0, self.norm_placement, int(self.unit_offset), self.activation, 0,
                        self.local_rope_theta or 0.0, self.attention_softcap or 0.0, self.logits_softcap or 0.0,
                        self.shared_inter, int(self.shared_gate))
        # per-layer flags (any depth) instead of the 64-bit masks
        flags = np.zeros((2, max(self.layers, 1)), dtype=np.uint8)
        for layer in range(self.layers):
            flags[0, layer] = layer in self.dense_layers
            flags[1, layer] = self.window_layers is not None and layer not in self.window_layers
        cfg.dense_layer_flags = flags[0].ctypes.data
        cfg.full_attention_layer_flags = flags[1].ctypes.data
        cfg._flags = flags
        inv_freq = self.inv_freq
        if inv_freq is None and self.rope_scaling:
            inv_freq = rope_inv_freq_scaled(self.rotary_dim or self.head_dim, self.rope_theta, self.scaling())
        if inv_freq is not None:
            table = np.ascontiguousarray(inv_freq, dtype=np.float64)
            assert table.size == (self.rotary_dim or self.head_dim) // 2
            cfg.inv_freq = table.ctypes.data
            cfg._keep = table  # the table must outlive the call that reads it
        return cfg

    def tensor_shapes(self) -> dict[str, tuple[int, ...]]:
        """architecture.py:418-468 (pre-norm decoders)."""
        q, kv, H = self.heads * self.head_dim, self.kv_heads * self.head_dim, self.hidden
        shapes = {"token_embedding.weight": (self.vocab, H)}
        for i in range(self.layers):
            p = f"layers.{i}."
            if self.norm_placement != 1:
                shapes[p + "attention_norm.weight"] = (H,)
            shapes[p + "attention.q.weight"] = (q, H)
            shapes[p + "attention.k.weight"] = (kv, H)
            shapes[p + "attention.v.weight"] = (kv, H)
            if self.attn_bias:
                shapes[p + "attention.q.bias"] = (q,)
                shapes[p + "attention.k.bias"] = (kv,)
                shapes[p + "attention.v.bias"] = (kv,)
            if self.qk_norm:
                shapes[p + "attention.q_norm.weight"] = (q if self.qk_norm == 2 else self.head_dim,)
                shapes[p + "attention.k_norm.weight"] = (kv if self.qk_norm == 2 else self.head_dim,)
            shapes[p + "attention.o.weight"] = (H, q)
            if self.norm_placement != 0:
                shapes[p + "attention_post_norm.weight"] = (H,)
                shapes[p + "mlp_post_norm.weight"] = (H,)
            if self.norm_placement != 1:
                shapes[p + "mlp_norm.weight"] = (H,)
            if self.is_sparse(i):
                e_inter = self.expert_inter or self.inter
                shapes[p + "mlp.router.weight"] = (self.experts, H)
                for e in range(self.experts):
                    shapes[p + f"mlp.experts.{e}.gate.weight"] = (e_inter, H)
                    shapes[p + f"mlp.experts.{e}.up.weight"] = (e_inter, H)
                    shapes[p + f"mlp.experts.{e}.down.weight"] = (H, e_inter)
                if self.shared_inter:
                    shapes[p + "mlp.shared.gate.weight"] = (self.shared_inter, H)
                    shapes[p + "mlp.shared.up.weight"] = (self.shared_inter, H)
                    shapes[p + "mlp.shared.down.weight"] = (H, self.shared_inter)
                    if self.shared_gate:
                        shapes[p + "mlp.shared_gate.weight"] = (1, H)
            else:
                shapes[p + "mlp.gate.weight"] = (self.inter, H)
                shapes[p + "mlp.up.weight"] = (self.inter, H)
                shapes[p + "mlp.down.weight"] = (H, self.inter)
        shapes["final_norm.weight"] = (H,)
        if not self.tied:
            shapes["lm_head.weight"] = (self.vocab, H)
        return shapes

    def slot_of(self, name: str) -> int:
        """The oracle's fixed slot of a tensor name (oracle/oracle.h)."""
        fixed = {"token_embedding.weight": 0, "final_norm.weight": 1, "lm_head.weight": 2}
        if name in fixed:
            return fixed[name]
        kinds = {"attention_norm.weight": 0, "attention.q.weight": 1, "attention.k.weight": 2,
                 "attention.v.weight": 3, "attention.q.bias": 4, "attention.k.bias": 5, "attention.v.bias": 6,
                 "attention.q_norm.weight": 7, "attention.k_norm.weight": 8, "attention.o.weight": 9,
                 "mlp_norm.weight": 10, "mlp.gate.weight": 11, "mlp.up.weight": 12, "mlp.down.weight": 13,
                 "mlp.router.weight": 14, "attention_post_norm.weight": 15, "mlp_post_norm.weight": 16,
                 "mlp.shared.gate.weight": 17, "mlp.shared.up.weight": 18, "mlp.shared.down.weight": 19,
                 "mlp.shared_gate.weight": 20}
        _, layer, rest = name.split(".", 2)
        per_layer = 21 + 3 * self.experts
        base = 3 + int(layer) * per_layer
        if rest in kinds:
            return base + kinds[rest]
        _, _, expert, which, _ = rest.split(".")
        return base + 21 + 3 * int(expert) + {"gate": 0, "up": 1, "down": 2}[which]

    def slot_count(self) -> int:
        return 3 + self.layers * (21 + 3 * self.experts)


def natural_key(name: str):
    """modelfile.py:40-43: digit runs compare as numbers, the name itself breaks ties."""
    parts = re.split(r"(\d+)", name)
    return (*((0, int(p), "") if p.isdigit() else (1, 0, p) for p in parts), name)


def tensor_order(names) -> list[str]:
    return sorted(names, key=natural_key)


TINY = dict(vocab=64, hidden=16, inter=32, layers=2, heads=4, kv_heads=2, head_dim=4, eps=1e-5, rope_theta=1e5)

def frozen_scaling(scaling: dict) -> tuple:
    return tuple((k, tuple(v) if isinstance(v, list) else v) for k, v in scaling.items())


# Phi-3's tiny config (tests/model_fixtures.py tiny_config): LongRoPE as the importer reads it (_longrope_from_hf:
# the short factors unless the model file asks for the long ones, the given attention factor), half of each head
# rotated, a 3-token window, hidden 32 (so head_dim 8), untied
PHI3_SCALING = {"rope_type": "longrope", "short_factor": [4.0, 1.0], "long_factor": [2.0, 4.0],
                "original_max_position_embeddings": 64, "attention_factor": 4.0}

# tests/model_fixtures.py:38-171 and the importer's reading of them (importing/importer.py:291-343)
FIXTURES = {
    "llama": Decoder("llama", tied=True, **TINY),
    "mistral": Decoder("mistral", tied=False, window=3, **TINY),
    "qwen2": Decoder("qwen2", tied=False, attn_bias=True, **TINY),
    "qwen3": Decoder("qwen3", tied=True, qk_norm=1, **{**TINY, "head_dim": 8}),
    "mixtral": Decoder("mixtral", tied=False, experts=4, topk=2, normalize=True, **TINY),
    "olmoe": Decoder("olmoe", tied=False, qk_norm=2, experts=4, topk=2, normalize=False,
                     **{**TINY, "inter": 8}),
    "granite": Decoder("granite", tied=True, embedding_multiplier=12.0, attention_multiplier=0.125,
                       residual_multiplier=0.22, logits_scaling=8.0, **TINY),
    "granitemoe": Decoder("granitemoe", tied=True, experts=4, topk=2, normalize=True, embedding_multiplier=12.0,
                          attention_multiplier=0.125, residual_multiplier=0.22, logits_scaling=8.0,
                          **{**TINY, "inter": 8}),
    "qwen3_moe": Decoder("qwen3_moe", tied=True, qk_norm=1, experts=4, topk=2, normalize=True, expert_inter=8,
                         dense_layers=(0,), **{**TINY, "head_dim": 8}),
    "olmo2": Decoder("olmo2", tied=False, qk_norm=2, norm_placement=1, **TINY),
    "gemma2": Decoder("gemma2", tied=True, norm_placement=2, unit_offset=True, activation=1, window=3,
                      window_layers=(0,), embedding_multiplier=math.sqrt(16), attention_multiplier=12.0 ** -0.5,
                      attention_softcap=0.02, logits_softcap=0.05, **{**TINY, "head_dim": 8}),
    "gemma3": Decoder("gemma3", tied=True, qk_norm=1, norm_placement=2, unit_offset=True, activation=1, window=3,
                      window_layers=(0,), local_rope_theta=100.0, embedding_multiplier=math.sqrt(16),
                      attention_multiplier=12.0 ** -0.5, rope_scaling=(("rope_type", "linear"), ("factor", 2.0)),
                      **{**TINY, "head_dim": 8}),
    "qwen2_moe": Decoder("qwen2_moe", tied=False, attn_bias=True, experts=4, topk=2, normalize=False, expert_inter=8,
                         shared_inter=12, shared_gate=True, **TINY),
    "granitemoeshared": Decoder("granitemoeshared", tied=True, experts=4, topk=2, normalize=True,
                                embedding_multiplier=12.0, attention_multiplier=0.125, residual_multiplier=0.22,
                                logits_scaling=8.0, shared_inter=12, **{**TINY, "inter": 8}),
    "phi3": Decoder("phi3", tied=False, window=3, rotary_dim=4, rope_attention_factor=4.0,
                    rope_scaling=frozen_scaling(PHI3_SCALING), **{**TINY, "hidden": 32, "head_dim": 8}),
}


# tests/test_quantized_finetuning.py:34-37: the tiny configs with hidden size 32 and a 264-token vocabulary
QLORA_FIXTURES = {
    "llama": Decoder("llama", tied=True, **{**TINY, "hidden": 32, "vocab": 264, "head_dim": 8}),
    "qwen3": Decoder("qwen3", tied=True, qk_norm=1, **{**TINY, "hidden": 32, "vocab": 264, "head_dim": 8}),
    "granite": replace(FIXTURES["granite"], hidden=32, vocab=264, head_dim=8),
    "qwen3_moe": replace(FIXTURES["qwen3_moe"], hidden=32, vocab=264),
    "gemma2": replace(FIXTURES["gemma2"], hidden=32, vocab=264, embedding_multiplier=math.sqrt(32)),
    "qwen2_moe": replace(FIXTURES["qwen2_moe"], hidden=32, vocab=264, head_dim=8),
}


def bf16_round(values: np.ndarray) -> np.ndarray:
    """model_fixtures.py:196-204: round to bfloat16 (nearest even) and back to float32."""
    bits = np.ascontiguousarray(values, dtype="<f4").view("<u4").astype(np.uint64)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype("<u4")
    return (rounded << np.uint32(16)).view("<f4")


def fixture_weights(d: Decoder, seed: int = 11) -> dict[str, np.ndarray]:
    """model_fixtures.hf_weights in our names (the Hugging Face import maps names one to one for these families)."""
    weights = {}
    for index, (name, shape) in enumerate(sorted(d.tensor_shapes().items())):
        values = fill_gaussian(seed * 1000 + index, int(np.prod(shape))).reshape(shape) * np.float32(0.1)
        if name.endswith("mlp.router.weight"):
            values = values * np.float32(16)
        weights[name] = bf16_round(values)
    return weights


def synthetic_weights(d: Decoder, seed: int, scale: float = 0.02) -> dict[str, np.ndarray]:
    """Benchmark inputs: fill_gaussian(seed * 1000 + i) * scale per tensor in tensor order, norms at 1.0."""
    weights = {}
    for index, name in enumerate(tensor_order(d.tensor_shapes())):
        shape = d.tensor_shapes()[name]
        if name.endswith("norm.weight"):
            weights[name] = np.ones(shape, np.float32)
        else:
            weights[name] = fill_gaussian(seed * 1000 + index, int(np.prod(shape))).reshape(shape) * np.float32(scale)
    return weights


def slot_array(d: Decoder, tensors: dict[str, np.ndarray]):
    arr = (_f32p * d.slot_count())()
    for name, values in tensors.items():
        arr[d.slot_of(name)] = ptr(values)
    return arr


def window_gradients(kern: Kernels, d: Decoder, weights, tokens, targets, scale=1.0, router_scale=0.0):
    """DecoderGradients.losses_and_gradients through the oracle's orchestration and the given kernel table."""
    grads = {name: np.empty(shape, np.float32) for name, shape in d.tensor_shapes().items()}
    tok = np.ascontiguousarray(tokens, np.int64)
    tgt = np.ascontiguousarray(targets, np.int64)
    loss, rl = C.c_double(), C.c_double()
    cfg = d.c()
    rc = oracle().orc_window_gradients(kern.address, C.byref(cfg), slot_array(d, weights), ptr(tok, _i64p),
                                       ptr(tgt, _i64p), len(tok), scale, router_scale, slot_array(d, grads),
                                       C.byref(loss), C.byref(rl))
    if rc != 0:
        raise ValueError(f"window gradients failed ({rc})")
    return loss.value, rl.value, grads


def logits(kern: Kernels, d: Decoder, weights, tokens) -> np.ndarray:
    tok = np.ascontiguousarray(tokens, np.int64)
    out = np.empty((len(tok), d.vocab), np.float32)
    cfg = d.c()
    oracle().orc_logits(kern.address, C.byref(cfg), slot_array(d, weights), ptr(tok, _i64p), len(tok), ptr(out))
    return out


def concatenated(grads: dict[str, np.ndarray]) -> np.ndarray:
    return np.concatenate([grads[name].ravel() for name in tensor_order(grads)])


def data_fingerprint(tensors: dict[str, np.ndarray]) -> str:
    """modelfile.data_fingerprint (modelfile.py:228-235): float32 bytes in tensor order, each padded to 64 bytes."""
    digest = hashlib.sha256()
    for name in tensor_order(tensors):
        data = np.ascontiguousarray(tensors[name], dtype="<f4").tobytes()
        digest.update(data + b"\0" * (-len(data) % 64))
    return digest.hexdigest()


# ---- training data and schedule (training/data.py, training/optimizer.py) ----

_EPOCH_MIX = 0x9E3779B97F4A7C15
_MASK64 = (1 << 64) - 1


class Random:
    """xoshiro256** through the oracle (random.hpp)."""

    def __init__(self, seed: int) -> None:
        self._state = (C.c_uint64 * 4)()
        oracle().orc_random_init(self._state, C.c_uint64(seed & _MASK64))

    def next_u64(self) -> int:
        return oracle().orc_random_next(self._state)


def windows_from_documents(documents, encode, sequence_length, separator):
    """TrainingData.from_documents (data.py:105-124)."""
    stream = []
    for document in documents:
        stream.extend(encode(document))
        if separator is not None:
            stream.append(separator)
    windows = []
    for start in range(0, max(len(stream) - 1, 0), sequence_length):
        window = tuple(stream[start:start + sequence_length + 1])
        if len(window) >= 2:
            windows.append(window)
    return windows


def epoch_order(count: int, seed: int, epoch: int) -> list[int]:
    """data.py:38-45: Fisher-Yates driven by Random((seed + (epoch + 1) * mix) mod 2^64)."""
    random = Random((seed + (epoch + 1) * _EPOCH_MIX) & _MASK64)
    order = list(range(count))
    for i in range(len(order) - 1, 0, -1):
        j = random.next_u64() % (i + 1)
        order[i], order[j] = order[j], order[i]
    return order


def batch_indices(count: int, step: int, batch_size: int, seed: int) -> list[int]:
    """data.py:48-57."""
    orders: dict[int, list[int]] = {}
    result = []
    for sample in range(step * batch_size, (step + 1) * batch_size):
        epoch, index = divmod(sample, count)
        if epoch not in orders:
            orders[epoch] = epoch_order(count, seed, epoch)
        result.append(orders[epoch][index])
    return result


@dataclass(frozen=True)
class AdamWConfig:
    learning_rate: float = 1e-4
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    weight_decay: float = 0.01
    max_grad_norm: float = 1.0
    warmup_steps: int = 0
    schedule: str = "cosine"
    min_learning_rate: float = 0.0

    def learning_rate_at(self, step: int, total_steps: int) -> float:
        """optimizer.py:48-56 with the portable cosine."""
        if self.warmup_steps and step <= self.warmup_steps:
            return self.learning_rate * step / self.warmup_steps
        if self.schedule == "constant" or total_steps <= self.warmup_steps:
            return self.learning_rate
        progress = (step - self.warmup_steps) / (total_steps - self.warmup_steps)
        span = self.learning_rate - self.min_learning_rate
        return self.min_learning_rate + 0.5 * span * (1.0 + oracle().orc_cos(math.pi * progress))


def train_step(kern: Kernels, d: Decoder, params, m, v, windows, opt: AdamWConfig, step: int, total_steps: int,
               router_aux_loss: float = 0.0):
    """One FineTuner.train_step (trainer.py:290-335) through the oracle: updates params, m, v in place and returns
    (loss, learning rate, gradient norm, summed gradients)."""
    names = tensor_order(d.tensor_shapes())
    grads = {name: np.empty(d.tensor_shapes()[name], np.float32) for name in names}
    order = np.array([d.slot_of(n) for n in names], np.int64)
    flat = np.array([t for w in windows for t in w], np.int64)
    lengths = np.array([len(w) for w in windows], np.int64)
    offsets = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.int64)
    lr = opt.learning_rate_at(step, total_steps)
    cfg = d.c()
    adam = OrcAdamW(lr, opt.beta1, opt.beta2, opt.eps, opt.weight_decay, opt.max_grad_norm, router_aux_loss, step)
    loss, norm = C.c_double(), C.c_double()
    rc = oracle().orc_train_step(kern.address, C.byref(cfg), slot_array(d, params), slot_array(d, m),
                                 slot_array(d, v), slot_array(d, grads), ptr(order, _i64p), len(order),
                                 ptr(flat, _i64p), ptr(offsets, _i64p), ptr(lengths, _i64p), len(windows),
                                 C.byref(adam), C.byref(loss), C.byref(norm))
    if rc != 0:
        raise ValueError(f"train step failed ({rc})")
    return loss.value, lr, norm.value, grads


def with_family(d: Decoder, **changes) -> Decoder:
    return replace(d, **changes)


# ---- LoRA (src/etalii_dllm/lora.py) ----

LORA_TARGETS = ("q", "k", "v", "o", "gate", "up", "down")  # lora.py:56-65 (ALL_TARGETS)
LORA_WEIGHT_NAMES = {"q": "attention.q.weight", "k": "attention.k.weight", "v": "attention.v.weight",
                     "o": "attention.o.weight", "gate": "mlp.gate.weight", "up": "mlp.up.weight",
                     "down": "mlp.down.weight"}  # lora.py:66-74


@dataclass(frozen=True)
class Lora:
    """LoraConfig (lora.py:159-177): scale = alpha / rank (alpha / sqrt(rank) with rsLoRA)."""

    rank: int
    alpha: float
    targets: tuple[str, ...] = LORA_TARGETS
    rslora: bool = False

    @property
    def scale(self) -> float:
        return self.alpha / (math.sqrt(self.rank) if self.rslora else self.rank)


def lora_target_weights(d: Decoder, lora: Lora) -> list[str]:
    """target_weights (lora.py:211-242) for pre-norm decoders: every expert's gate/up/down in a sparse layer."""
    names = []
    for layer in range(d.layers):
        for target in lora.targets:
            if target in ("gate", "up", "down") and d.is_sparse(layer):
                names.extend(f"layers.{layer}.mlp.experts.{e}.{target}.weight" for e in range(d.experts))
                if d.shared_inter:
                    names.append(f"layers.{layer}.mlp.shared.{target}.weight")
            else:
                names.append(f"layers.{layer}.{LORA_WEIGHT_NAMES[target]}")
    return tensor_order(names)


def adapter_shapes(d: Decoder, lora: Lora) -> dict[str, tuple[int, int]]:
    """lora.py:245-255: <weight>.lora_a [rank, in] and <weight>.lora_b [out, rank], weights in tensor order."""
    shapes = d.tensor_shapes()
    result = {}
    for name in lora_target_weights(d, lora):
        out_features, in_features = shapes[name]
        result[name + ".lora_a"] = (lora.rank, in_features)
        result[name + ".lora_b"] = (out_features, lora.rank)
    return result


def init_adapters(d: Decoder, lora: Lora, seed: int) -> dict[str, np.ndarray]:
    """lora.py:258-268: A = fill_gaussian(seed * 1000003 + index) * f32(1 / rank), B = 0."""
    adapters = {}
    for index, (name, shape) in enumerate(adapter_shapes(d, lora).items()):
        if name.endswith(".lora_a"):
            values = fill_gaussian(seed * 1_000_003 + index, shape[0] * shape[1]).reshape(shape)
            adapters[name] = np.ascontiguousarray(values * np.float32(1.0 / lora.rank), dtype=np.float32)
        else:
            adapters[name] = np.zeros(shape, dtype=np.float32)
    return adapters


def lora_merge(kern: Kernels, weight, a, b, scale: float) -> np.ndarray:
    """lora.py:271-276: weight + f32(linear(b, a^T)) * f32(scale), in float32."""
    delta = kern.linear(np.ascontiguousarray(b, np.float32), np.ascontiguousarray(a.T, np.float32))
    return np.asarray(weight, np.float32) + delta * np.float32(scale)


def adapter_gradients(kern: Kernels, gradient, a, b, scale: float):
    """lora.py:374-383: dA = linear(B^T, dW^T) * s, dB = linear(dW, A) * s (float32 products with s)."""
    s = np.float32(scale)
    gradient = np.ascontiguousarray(gradient, np.float32)
    da = kern.linear(np.ascontiguousarray(b.T, np.float32), np.ascontiguousarray(gradient.T)) * s
    db = kern.linear(gradient, np.ascontiguousarray(a, np.float32)) * s
    return da, db


def merged_weights(kern: Kernels, d: Decoder, base, adapters, lora: Lora) -> dict[str, np.ndarray]:
    """lora.py:279-287."""
    merged = dict(base)
    for name in lora_target_weights(d, lora):
        merged[name] = lora_merge(kern, base[name], adapters[name + ".lora_a"], adapters[name + ".lora_b"], lora.scale)
    return merged


def _power(base: float, exponent: int) -> float:
    """optimizer.py:59-63: repeated multiplication."""
    result = 1.0
    for _ in range(exponent):
        result *= base
    return result


def lora_train_step(kern: Kernels, d: Decoder, base, adapters, m, v, windows, opt: AdamWConfig, step: int,
                    total_steps: int, lora: Lora, router_aux_loss: float = 0.0, out: dict | None = None):
    """FineTuner.train_step for a LoRA run (trainer.py:290-335, 463-474; optimizer.py:66-109): gradients of the
    merged weights summed over the windows in float32 (the first copied), the adapters' gradients, then AdamW over
    the adapters in tensor order. Updates adapters, m and v in place; returns (loss, gradient norm). With `out`, its
    "weight_grads" and "adapter_grads" receive the summed merged-weight gradients and the adapters' gradients."""
    merged = merged_weights(kern, d, base, adapters, lora)
    targets_total = sum(len(w) - 1 for w in windows)
    scale = 1.0 / targets_total
    loss_total, router_total, grads = 0.0, 0.0, {}
    for w in windows:
        loss, router_loss, g = window_gradients(kern, d, merged, w[:-1], w[1:], scale=scale,
                                                router_scale=router_aux_loss / len(windows))
        loss_total += loss
        router_total += router_loss
        for name, value in g.items():
            if name in grads:
                grads[name] += value
            else:
                grads[name] = value.copy()
    result = {}
    for name in adapters:
        if name.endswith(".lora_b"):
            weight = name[: -len(".lora_b")]
            a_name = weight + ".lora_a"
            result[a_name], result[name] = adapter_gradients(kern, grads[weight], adapters[a_name], adapters[name],
                                                             lora.scale)
    if out is not None:
        out["weight_grads"], out["adapter_grads"] = grads, result
    total = 0.0
    for name in tensor_order(result):
        total += kern.sum_squares(result[name])
    norm = math.sqrt(total)
    clip = 1.0
    if opt.max_grad_norm > 0 and norm > opt.max_grad_norm:
        clip = opt.max_grad_norm / (norm + 1e-6)
    c1, c2 = 1.0 - _power(opt.beta1, step), 1.0 - _power(opt.beta2, step)
    lr = opt.learning_rate_at(step, total_steps)
    for name in tensor_order(adapters):
        decay = opt.weight_decay if adapters[name].ndim >= 2 else 0.0
        kern.adamw_step(adapters[name], np.ascontiguousarray(result[name], np.float32), m[name], v[name], lr,
                        opt.beta1, opt.beta2, opt.eps, decay, c1, c2, clip)
    loss = loss_total / targets_total
    if router_aux_loss:
        loss += router_aux_loss * router_total / len(windows)
    return loss, norm


# ---- direct preference optimization (src/etalii_dllm/training/trainer.py:364-384, preference.py) ----

def log_sigmoid(z: float) -> float:
    """preference.py:174-179 with the portable exp and log."""
    o = oracle()
    if z >= 0.0:
        return -o.orc_log(1.0 + o.orc_exp(-z))
    return z - o.orc_log(1.0 + o.orc_exp(z))


def preference_pairs(records, encode, sequence_length: int, end: int | None):
    """PreferenceData.from_records (preference.py:110-136): (prompt, chosen, rejected) token tuples."""
    pairs = []
    for prompt_text, chosen_text, rejected_text in records:
        prompt = tuple(encode(prompt_text))
        room = sequence_length + 1 - len(prompt)
        suffix = () if end is None else (end,)
        pairs.append((prompt, (*encode(chosen_text), *suffix)[:room], (*encode(rejected_text), *suffix)[:room]))
    return pairs


def pair_sequence(pair, which: str):
    """PreferencePair.sequence (preference.py:97-102): inputs and targets, the prompt's targets -1."""
    prompt, chosen, rejected = pair
    answer = chosen if which == "chosen" else rejected
    tokens = [*prompt, *answer]
    return tokens[:-1], [-1] * (len(prompt) - 1) + list(answer)


def log_probability(kern: Kernels, d: Decoder, weights, pair, which: str) -> float:
    """FineTuner.log_probability (trainer.py:443-453): minus the answer's summed cross-entropy."""
    tokens, targets = pair_sequence(pair, which)
    loss, _, _ = window_gradients(kern, d, weights, tokens, targets)
    return -loss


def adamw_update(kern: Kernels, params, grads, m, v, opt: AdamWConfig, step: int, total_steps: int) -> float:
    """AdamW.step over `params` in tensor order (optimizer.py:66-109); returns the gradient norm."""
    total = 0.0
    for name in tensor_order(grads):
        total += kern.sum_squares(grads[name])
    norm = math.sqrt(total)
    clip = 1.0
    if opt.max_grad_norm > 0 and norm > opt.max_grad_norm:
        clip = opt.max_grad_norm / (norm + 1e-6)
    c1, c2 = 1.0 - _power(opt.beta1, step), 1.0 - _power(opt.beta2, step)
    lr = opt.learning_rate_at(step, total_steps)
    for name in tensor_order(params):
        decay = opt.weight_decay if params[name].ndim >= 2 else 0.0
        kern.adamw_step(params[name], np.ascontiguousarray(grads[name], np.float32), m[name], v[name], lr,
                        opt.beta1, opt.beta2, opt.eps, decay, c1, c2, clip)
    return norm


def dpo_train_step(kern: Kernels, d: Decoder, params, m, v, pairs, reference, beta: float, opt: AdamWConfig,
                   step: int, total_steps: int):
    """FineTuner.train_step with the DPO objective (trainer.py:290-310, 364-384): per pair the chosen and rejected
    answers' gradients times +-f32(beta (1 - sigmoid(z)) / pairs), summed in float32 (the first product taken as is);
    then AdamW. Updates params, m, v in place; returns (loss, gradient norm, summed gradients)."""
    o = oracle()
    loss_total, grads = 0.0, {}
    for pair, (reference_chosen, reference_rejected) in zip(pairs, reference):
        chosen_loss, _, chosen_grads = window_gradients(kern, d, params, *pair_sequence(pair, "chosen"))
        rejected_loss, _, rejected_grads = window_gradients(kern, d, params, *pair_sequence(pair, "rejected"))
        z = beta * ((-chosen_loss - reference_chosen) - (-rejected_loss - reference_rejected))
        loss_total += -log_sigmoid(z)
        weight = np.float32(beta * (1.0 - o.orc_sigmoid(z)) / len(pairs))
        for sign, pair_grads in ((weight, chosen_grads), (-weight, rejected_grads)):
            for name, gradient in pair_grads.items():
                grads[name] = grads[name] + gradient * sign if name in grads else gradient * sign
    norm = adamw_update(kern, params, grads, m, v, opt, step, total_steps)
    return loss_total / len(pairs), norm, grads


# ---- Q8_0 (cpp/include/dllm/quant.hpp:27-60, numerics.py:106-139) ----

def quantize_q8_0(fn, x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(values int8 [n], scales f32 [n / 32]) from a quantize_q8_0(x, q, scales, n) C function."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    assert x.size % 32 == 0
    q = np.empty(x.size, np.int8)
    s = np.empty(x.size // 32, np.float32)
    fn.argtypes = [_f32p, C.POINTER(C.c_int8), _f32p, C.c_size_t]
    fn(ptr(x), q.ctypes.data_as(C.POINTER(C.c_int8)), ptr(s), x.size)
    return q, s


def linear_q8(fn, x: np.ndarray, q: np.ndarray, scales: np.ndarray, bias=None) -> np.ndarray:
    """A linear_q8(x, wq, ws, bias, out, rows, in, out) C function on x [rows, in], q [out, in], scales [out, in/32]."""
    x = np.ascontiguousarray(x, np.float32)
    q = np.ascontiguousarray(q, np.int8)
    s = np.ascontiguousarray(scales, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    out = np.empty((x.shape[0], q.shape[0]), np.float32)
    fn(ptr(x), q.ctypes.data_as(C.c_void_p), ptr(s), ptr(b) if b is not None else None, ptr(out),
       C.c_size_t(x.shape[0]), C.c_size_t(x.shape[1]), C.c_size_t(q.shape[0]))
    return out


def quantize_q4_0(fn, x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(packed bytes [n / 2], scales [n / 32]) from a quantize_q4_0(x, packed, scales, n) C function."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    q = np.empty(x.size // 2, np.uint8)
    s = np.empty(x.size // 32, np.float32)
    fn(ptr(x), q.ctypes.data_as(C.c_void_p), ptr(s), C.c_size_t(x.size))
    return q, s


def unpack_q4_0(fn, packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, np.uint8).ravel()
    out = np.empty(packed.size * 2, np.int8)
    fn(packed.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p), C.c_size_t(out.size))
    return out


def linear_q4(fn, x: np.ndarray, packed: np.ndarray, scales: np.ndarray, bias=None) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    q = np.ascontiguousarray(packed, np.uint8)
    s = np.ascontiguousarray(scales, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    out = np.empty((x.shape[0], q.shape[0]), np.float32)
    fn(ptr(x), q.ctypes.data_as(C.c_void_p), ptr(s), ptr(b) if b is not None else None, ptr(out),
       C.c_size_t(x.shape[0]), C.c_size_t(x.shape[1]), C.c_size_t(q.shape[0]))
    return out


# ---- encoder and T5 kernels (grad.hpp:112-174, 300-389; nn.hpp:412-432, 474-478, 827-856) ----

def _declare_encoder(lib, prefix: str) -> None:
    d, f, sz, vp = C.c_double, C.c_float, C.c_size_t, C.c_void_p
    for name, res, args in (
            ("erf", d, [d]), ("erfc", d, [d]),
            ("layer_norm", None, [vp, vp, vp, vp, sz, sz, d]),
            ("layer_norm_backward", None, [vp, vp, vp, vp, vp, vp, sz, sz, d]),
            ("biased_attention", None, [vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, d]),
            ("biased_attention_weights", None, [vp, vp, vp, vp, sz, sz, sz, sz, d]),
            ("biased_attention_backward", None, [vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, d])):
        fn = getattr(lib, f"{prefix}_{name}")
        fn.restype, fn.argtypes = res, args
    if prefix == "orc":
        lib.orc_gelu.restype, lib.orc_gelu.argtypes = f, [f]
        lib.orc_gelu_backward.restype, lib.orc_gelu_backward.argtypes = f, [f, f]
    else:
        lib.ref_gelu_n.argtypes = [vp, vp, sz]
        lib.ref_gelu_backward_n.argtypes = [vp, vp, vp, sz]


class Encoder:
    """The encoder/T5 kernels of the oracle (prefix "orc") or of the compiled reference (prefix "ref")."""

    def __init__(self, lib, prefix: str) -> None:
        _declare_encoder(lib, prefix)
        self.lib, self.p = lib, prefix

    def fn(self, name):
        return getattr(self.lib, f"{self.p}_{name}")

    def erf(self, x: float) -> float:
        return self.fn("erf")(x)

    def erfc(self, x: float) -> float:
        return self.fn("erfc")(x)

    def gelu(self, x):
        x = np.ascontiguousarray(x, np.float32)
        if self.p == "orc":
            return np.array([self.lib.orc_gelu(float(v)) for v in x.ravel()], np.float32).reshape(x.shape)
        out = np.empty_like(x)
        self.lib.ref_gelu_n(ptr(x), ptr(out), x.size)
        return out

    def gelu_backward(self, x, dy):
        x, dy = np.ascontiguousarray(x, np.float32), np.ascontiguousarray(dy, np.float32)
        if self.p == "orc":
            return np.array([self.lib.orc_gelu_backward(float(a), float(b)) for a, b in zip(x.ravel(), dy.ravel())],
                            np.float32).reshape(x.shape)
        out = np.empty_like(x)
        self.lib.ref_gelu_backward_n(ptr(x), ptr(dy), ptr(out), x.size)
        return out

    def layer_norm(self, x, w, b, eps=1e-12):
        x, w, b = (np.ascontiguousarray(a, np.float32) for a in (x, w, b))
        out = np.empty_like(x)
        dim = x.shape[-1]
        self.fn("layer_norm")(ptr(x), ptr(w), ptr(b), ptr(out), x.size // dim if dim else 0, dim, eps)
        return out

    def layer_norm_backward(self, x, w, dy, eps=1e-12):
        x, w, dy = (np.ascontiguousarray(a, np.float32) for a in (x, w, dy))
        dim = x.shape[-1]
        dx, dw, db = np.empty_like(x), np.empty(dim, np.float32), np.empty(dim, np.float32)
        self.fn("layer_norm_backward")(ptr(x), ptr(w), ptr(dy), ptr(dx), ptr(dw), ptr(db),
                                       x.size // dim if dim else 0, dim, eps)
        return dx, dw, db

    def biased_attention(self, q, k, v, bias, scale):
        q, k, v, bias = (np.ascontiguousarray(a, np.float32) for a in (q, k, v, bias))
        out = np.empty((q.shape[0], q.shape[1], v.shape[2]), np.float32)
        self.fn("biased_attention")(ptr(q), ptr(k), ptr(v), ptr(bias), ptr(out), q.shape[0], k.shape[0], q.shape[1],
                                    q.shape[2], v.shape[2], scale)
        return out

    def biased_attention_weights(self, q, k, bias, scale):
        q, k, bias = (np.ascontiguousarray(a, np.float32) for a in (q, k, bias))
        out = np.zeros((q.shape[0], q.shape[1], k.shape[0]), np.float32)
        self.fn("biased_attention_weights")(ptr(q), ptr(k), ptr(bias), ptr(out), q.shape[0], k.shape[0], q.shape[1],
                                            q.shape[2], scale)
        return out

    def biased_attention_backward(self, q, k, v, bias, dout, scale):
        q, k, v, bias, dout = (np.ascontiguousarray(a, np.float32) for a in (q, k, v, bias, dout))
        dq, dk, dv, dbias = np.empty_like(q), np.empty_like(k), np.empty_like(v), np.empty_like(bias)
        self.fn("biased_attention_backward")(ptr(q), ptr(k), ptr(v), ptr(bias), ptr(dout), ptr(dq), ptr(dk), ptr(dv),
                                             ptr(dbias), q.shape[0], k.shape[0], q.shape[1], q.shape[2], v.shape[2],
                                             scale)
        return dq, dk, dv, dbias


def oracle_encoder() -> Encoder:
    return Encoder(oracle(), "orc")


def ref_encoder() -> Encoder:
    return Encoder(ref(), "ref")


QUANTIZED_MATRICES = tuple(f".{m}.weight" for m in ("q", "k", "v", "o", "gate", "up", "down"))


def quantizable(name: str, shape) -> bool:
    """lora.py:319-324: the matrices a quantised base holds quantised (rows of whole 32-value blocks)."""
    return name.endswith(QUANTIZED_MATRICES) and len(shape) == 2 and shape[1] % 32 == 0


def dequantize_q8_0(q: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """QuantizedWeight.dequantize (numerics.py:138-139): int8 -> float32 times the block's scale, in float32."""
    return q.astype(np.float32) * np.repeat(scales, 32)


def q8_0_cases() -> dict[str, np.ndarray]:
    """Blocks exercising the rounding: exact half-way products of both parities, zeros, a block of zeros, non-finite
    values (ignored for the scale, stored as 0), a value at -amax, tiny and huge magnitudes."""
    g = gaussian(31, 32 * 64)
    cases = {"gaussian": g, "scaled": g * np.float32(1e-30), "huge": g * np.float32(1e30)}
    ties = np.tile((np.arange(32, dtype=np.float32) - 16) * np.float32(0.5), 4)
    ties[0], ties[32], ties[64], ties[96] = np.float32(63.5), np.float32(-63.5), np.float32(127.0), np.float32(-8.0)
    cases["ties"] = ties  # amax 63.5 or 127: x * (127 / amax) lands on halves
    special = gaussian(32, 32 * 4)
    special[3], special[40], special[77] = np.inf, -np.inf, np.nan
    special[96:128] = 0.0
    cases["special"] = special
    return cases


def gelu_tanh(x) -> np.ndarray:
    """The oracle's gelu_tanh (nn.hpp:481-485), elementwise."""
    f = oracle().orc_gelu_tanh
    return np.array([f(float(a)) for a in np.ravel(x)], np.float32).reshape(np.shape(x))


def gelu_tanh_backward(x, dy) -> np.ndarray:
    """The oracle's gelu_tanh_backward (grad.hpp:183-191), elementwise."""
    f = oracle().orc_gelu_tanh_backward
    return np.array([f(float(a), float(b)) for a, b in zip(np.ravel(x), np.ravel(dy))], np.float32).reshape(np.shape(x))


def softcap(x, cap: float) -> np.ndarray:
    """softcap (nn.hpp:457-461): f32(cap tanh(x / cap)) in double with the oracle's tanh, elementwise."""
    t = oracle().orc_tanh
    return np.array([np.float32(cap * t(float(a) / cap)) for a in np.ravel(x)], np.float32).reshape(np.shape(x))


def sigmoid_elementwise(x) -> np.ndarray:
    """sigmoid_float (nn.hpp:464): f32(sigmoid(x)) with the oracle's sigmoid, elementwise."""
    f = oracle().orc_sigmoid
    return np.array([np.float32(f(float(a))) for a in np.ravel(x)], np.float32).reshape(np.shape(x))


def softcap_backward(x, dy, cap: float) -> np.ndarray:
    """The oracle's softcap_backward (grad.hpp:193-197), elementwise."""
    f = oracle().orc_softcap_backward
    return np.array([f(float(a), float(b), cap) for a, b in zip(np.ravel(x), np.ravel(dy))],
                    np.float32).reshape(np.shape(x))
