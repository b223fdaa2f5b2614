"""The reference's kernel module interface (etalii_dllm._kernels, cpp/kernels.cpp) over the MI355X library.

Each function takes and returns NumPy arrays with the reference binding's names, argument meaning and errors
(ValueError where the binding raises it): inputs are uploaded to the GPU, the HIP kernels run through the C ABI of
include/dllm_hip.h, and the results come back. This is the drop-in surface for parity checks and for callers that
hold host arrays; device-resident callers use the C ABI or :mod:`etalii_dllm_amd.trainer` directly.

There is no CPU fallback: importing this module without the built library (libdllm_hip.so, see build.py) raises.
"""

from __future__ import annotations

import ctypes as C
import math
from pathlib import Path

import numpy as np

LIBRARY = Path(__file__).resolve().parent / "libdllm_hip.so"

_f32p = C.POINTER(C.c_float)
_f64p = C.POINTER(C.c_double)
_i64p = C.POINTER(C.c_int64)
_sz = C.c_size_t
_vp = C.c_void_p


def _load() -> C.CDLL:
    if not LIBRARY.exists():
        raise ImportError(f"{LIBRARY} is not built; run etalii_dllm_amd/build.py (hipcc, gfx950)")
    lib = C.CDLL(str(LIBRARY))
    lib.dllm_hip_last_error.restype = C.c_char_p
    lib.dllm_hip_version.restype = C.c_char_p
    lib.dllm_hip_trainer_tensor_name.restype = C.c_char_p
    lib.dllm_hip_trainer_tensor_name.argtypes = [_vp, C.c_int64]
    for name in ("linear", "linear_backward", "rope", "attention_backward", "cross_entropy",
                 "embedding_backward", "rms_norm_backward"):
        getattr(lib, f"dllm_hip_{name}_workspace").restype = _sz
    lib.dllm_hip_attention_workspace.restype = _sz
    lib.dllm_hip_linear_workspace.argtypes = [_sz, _sz, _sz]
    lib.dllm_hip_linear_backward_workspace.argtypes = [_sz, _sz, _sz]
    lib.dllm_hip_rope_workspace.argtypes = [_sz, _sz]
    lib.dllm_hip_attention_backward_workspace.argtypes = [_sz, _sz, _sz, _sz, _sz, _sz, C.c_int, C.c_int64, _sz,
                                                          C.c_double]
    lib.dllm_hip_attention_workspace.argtypes = [_sz, _sz, _sz, _sz, _sz, _sz, C.c_int, C.c_int64, _sz, C.c_double]
    lib.dllm_hip_cross_entropy_workspace.argtypes = [_sz]
    lib.dllm_hip_embedding_backward_workspace.argtypes = [_sz]
    lib.dllm_hip_rms_norm_backward_workspace.argtypes = [_sz]
    lib.dllm_hip_alloc.argtypes = [C.POINTER(_vp), _sz]
    lib.dllm_hip_release.argtypes = [_vp]
    lib.dllm_hip_upload.argtypes = [_vp, _vp, _sz]
    lib.dllm_hip_download.argtypes = [_vp, _vp, _sz]
    lib.dllm_hip_memset.argtypes = [_vp, C.c_int, _sz]
    lib.dllm_hip_copy.argtypes = [_vp, _vp, _sz, _vp]
    lib.dllm_hip_linear.argtypes = [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp, _sz, _vp]
    lib.dllm_hip_rms_norm.argtypes = [_vp, _vp, _vp, _sz, _sz, C.c_double, C.c_int, _vp]
    lib.dllm_hip_rope.argtypes = [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, C.c_int, C.c_int, _vp, _sz, _vp]
    lib.dllm_hip_attention.argtypes = [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, C.c_double, C.c_int,
                                       C.c_int64, _sz, C.c_double, _vp, _sz, _vp]
    lib.dllm_hip_silu.argtypes = [_vp, _vp, _sz, _vp]
    lib.dllm_hip_swiglu.argtypes = [_vp, _vp, _vp, _sz, C.c_int, _vp]
    lib.dllm_hip_gelu_tanh.argtypes = [_vp, _vp, _sz, _vp]
    lib.dllm_hip_softcap.argtypes = [_vp, _vp, _sz, C.c_double, _vp]
    lib.dllm_hip_sigmoid_elementwise.argtypes = [_vp, _vp, _sz, _vp]
    lib.dllm_hip_linear_backward.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp, _sz, _vp]
    lib.dllm_hip_rms_norm_backward.argtypes = [_vp, _vp, _vp, _vp, _vp, _sz, _sz, C.c_double, C.c_int, _vp, _sz,
                                               _vp]
    lib.dllm_hip_silu_backward.argtypes = [_vp, _vp, _vp, _sz, _vp]
    lib.dllm_hip_attention_backward.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz,
                                                C.c_double, C.c_int, C.c_int64, _sz, C.c_double, _vp, _sz, _vp]
    lib.dllm_hip_cross_entropy.argtypes = [_vp, _vp, _vp, _sz, _sz, C.c_double, _f64p, _vp, _sz, _vp]
    lib.dllm_hip_embedding_backward.argtypes = [_vp, _vp, _vp, _sz, _sz, _sz, _vp, _sz, _vp]
    lib.dllm_hip_sum_squares.argtypes = [_vp, _sz, _f64p, _vp, _sz, _vp]
    lib.dllm_hip_sum_squares_workspace.restype = _sz
    lib.dllm_hip_sum_squares_workspace.argtypes = [_sz]
    lib.dllm_hip_adamw_step.argtypes = [_vp, _vp, _vp, _vp, _sz] + [C.c_double] * 8 + [_vp]
    lib.dllm_hip_gelu_tanh_backward.argtypes = [_vp, _vp, _vp, _sz, _vp]
    lib.dllm_hip_softcap_backward.argtypes = [_vp, _vp, _vp, _sz, C.c_double, _vp]
    lib.dllm_hip_softmax.argtypes = [_vp, _vp, _sz, _sz, _vp]
    lib.dllm_hip_column_mean.argtypes = [_vp, _vp, _sz, _sz, _vp]
    lib.dllm_hip_dot_workspace.restype = _sz
    lib.dllm_hip_dot_workspace.argtypes = []
    lib.dllm_hip_dot.argtypes = [_vp, _vp, _sz, C.POINTER(C.c_float), _vp, _sz, _vp]
    lib.dllm_hip_moe_route.argtypes = [_vp, _vp, _vp, _sz, _sz, _sz, C.c_int, _vp]
    lib.dllm_hip_moe_route_backward.argtypes = [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, C.c_int, _vp]
    lib.dllm_hip_quantize_q8_0.argtypes = [_vp, _vp, _vp, _sz, _vp]
    lib.dllm_hip_dequantize_q8_0.argtypes = [_vp, _vp, _vp, _sz, _vp]
    lib.dllm_hip_lora_merge_workspace.restype = _sz
    lib.dllm_hip_lora_merge_workspace.argtypes = [_sz, _sz, _sz]
    lib.dllm_hip_lora_merge.argtypes = [_vp, _vp, _vp, _vp, _sz, _sz, _sz, C.c_double, _vp, _sz, _vp]
    lib.dllm_hip_lora_adapter_gradients_workspace.restype = _sz
    lib.dllm_hip_lora_adapter_gradients_workspace.argtypes = [_sz, _sz, _sz]
    lib.dllm_hip_lora_adapter_gradients.argtypes = [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, C.c_double, _vp, _sz,
                                                    _vp]
    return lib


lib = _load()


class HipError(RuntimeError):
    """A HIP runtime failure inside the library."""


def check(status: int) -> None:
    if status == 0:
        return
    message = (lib.dllm_hip_last_error() or b"").decode()
    if status == 1:
        raise ValueError(message)
    if status == 3:
        raise MemoryError(message)
    raise HipError(message)


class Device:
    """One device allocation (freed with the object)."""

    def __init__(self, nbytes: int) -> None:
        self.nbytes = int(nbytes)
        self.ptr = _vp()
        check(lib.dllm_hip_alloc(C.byref(self.ptr), max(self.nbytes, 1)))

    @classmethod
    def of(cls, array: np.ndarray) -> Device:
        a = np.ascontiguousarray(array)
        d = cls(a.nbytes)
        if a.nbytes:
            check(lib.dllm_hip_upload(d.ptr, a.ctypes.data, a.nbytes))
        return d

    def download(self, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype)
        if out.nbytes:
            check(lib.dllm_hip_download(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def __del__(self) -> None:
        if getattr(self, "ptr", None) is not None and self.ptr.value:
            lib.dllm_hip_release(self.ptr)
            self.ptr = _vp()


def _f32(values) -> np.ndarray:
    return np.ascontiguousarray(values, dtype=np.float32)


def _rows(x: np.ndarray) -> int:
    return int(np.prod(x.shape[:-1])) if x.ndim > 1 else 1


# ---- forward kernels (cpp/kernels.cpp) ----

def linear(x, weight, bias=None) -> np.ndarray:
    """kernels.cpp:220-238: x[..., in] @ weight[out, in]^T (+ bias), k ascending in double."""
    x, w = _f32(x), _f32(weight)
    if x.ndim < 1:
        raise ValueError("x must have at least one dimension")
    if w.ndim != 2:
        raise ValueError("weight must be [out_features, in_features]")
    out_f, in_f = w.shape
    if x.shape[-1] != in_f:
        raise ValueError("weight in_features does not match the last dimension of x")
    if bias is not None and _f32(bias).shape[0] != out_f:
        raise ValueError("bias length must equal out_features")
    rows = _rows(x)
    ws = Device(lib.dllm_hip_linear_workspace(rows, in_f, out_f))
    dx, dw = Device.of(x), Device.of(w)
    db = Device.of(_f32(bias)) if bias is not None else None
    out = Device(rows * out_f * 4)
    check(lib.dllm_hip_linear(dx.ptr, dw.ptr, db.ptr if db else None, out.ptr, rows, in_f, out_f, ws.ptr, ws.nbytes,
                              None))
    return out.download((*x.shape[:-1], out_f))


def rms_norm(x, weight=None, eps=1e-6, add_unit_offset=False) -> np.ndarray:
    """kernels.cpp:598-611."""
    x = _f32(x)
    dim = x.shape[-1]
    if weight is not None and _f32(weight).shape[0] != dim:
        raise ValueError("weight length must equal the last dimension of x")
    dx = Device.of(x)
    dw = Device.of(_f32(weight)) if weight is not None else None
    out = Device(x.nbytes)
    check(lib.dllm_hip_rms_norm(dx.ptr, dw.ptr if dw else None, out.ptr, _rows(x), dim, float(eps),
                                int(add_unit_offset), None))
    return out.download(x.shape)


def rope(x, positions, inv_freq, interleaved=False, inverse=False) -> np.ndarray:
    """kernels.cpp:662-679."""
    x = _f32(x)
    pos = np.ascontiguousarray(positions, dtype=np.int64)
    freqs = np.ascontiguousarray(inv_freq, dtype=np.float64)
    if x.ndim != 3:
        raise ValueError("x must be [tokens, heads, head_dim]")
    tokens, heads, head_dim = x.shape
    rotary = 2 * len(freqs)
    if len(pos) != tokens:
        raise ValueError("positions must have one entry per token")
    if rotary > head_dim:
        raise ValueError("2 * len(inv_freq) must not exceed head_dim")
    ws = Device(lib.dllm_hip_rope_workspace(tokens, rotary))
    dx, dp, df, out = Device.of(x), Device.of(pos), Device.of(freqs), Device(x.nbytes)
    check(lib.dllm_hip_rope(dx.ptr, dp.ptr, df.ptr, out.ptr, tokens, heads, head_dim, rotary, int(interleaved),
                            int(inverse), ws.ptr, ws.nbytes, None))
    return out.download(x.shape)


def _attention_args(q, k, v, q_offset):
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError("q, k and v must be [length, heads, dim]")
    if v.shape[0] != k.shape[0] or v.shape[1] != k.shape[1]:
        raise ValueError("k and v must have the same length and heads")
    if q.shape[2] != k.shape[2]:
        raise ValueError("q and k must have the same head_dim")
    if k.shape[1] == 0 or q.shape[1] % k.shape[1]:
        raise ValueError("q heads must be a multiple of kv heads")
    if q_offset < 0:
        q_offset = k.shape[0] - q.shape[0]
    if q_offset < 0:
        raise ValueError("q_offset must be non-negative")
    return q_offset


def attention(q, k, v, scale, causal=True, q_offset=-1, window=0, softcap=0.0, reference=False) -> np.ndarray:
    """kernels.cpp:680-705 (`reference` selects the same bits on the CPU there; it has no effect here)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    q_offset = _attention_args(q, k, v, q_offset)
    out_shape = (q.shape[0], q.shape[1], v.shape[2])
    ws = Device(lib.dllm_hip_attention_workspace(q.shape[0], k.shape[0], q.shape[1], k.shape[1], q.shape[2],
                                                 v.shape[2], int(causal), int(q_offset), int(window), float(softcap)))
    dq, dk, dv, out = Device.of(q), Device.of(k), Device.of(v), Device(int(np.prod(out_shape)) * 4)
    check(lib.dllm_hip_attention(dq.ptr, dk.ptr, dv.ptr, out.ptr, q.shape[0], k.shape[0], q.shape[1], k.shape[1],
                                 q.shape[2], v.shape[2], float(scale), int(causal), int(q_offset), int(window),
                                 float(softcap), ws.ptr, ws.nbytes, None))
    return out.download(out_shape)


def silu(x) -> np.ndarray:
    x = _f32(x)
    dx, out = Device.of(x), Device(x.nbytes)
    check(lib.dllm_hip_silu(dx.ptr, out.ptr, x.size, None))
    return out.download(x.shape)


def gelu_tanh(x) -> np.ndarray:
    """kernels.cpp:632: elementwise tanh-approximated GELU."""
    x = _f32(x)
    dx, out = Device.of(x), Device(x.nbytes)
    check(lib.dllm_hip_gelu_tanh(dx.ptr, out.ptr, x.size, None))
    return out.download(x.shape)


def softcap(x, cap: float) -> np.ndarray:
    """kernels.cpp:650-660: elementwise cap * tanh(x / cap), in double; cap must be positive."""
    x = _f32(x)
    if not cap > 0.0:
        raise ValueError("cap must be positive")
    dx, out = Device.of(x), Device(x.nbytes)
    check(lib.dllm_hip_softcap(dx.ptr, out.ptr, x.size, float(cap), None))
    return out.download(x.shape)


def sigmoid_elementwise(x) -> np.ndarray:
    """kernels.cpp:629-630: elementwise logistic sigmoid, in double, rounded once."""
    x = _f32(x)
    dx, out = Device.of(x), Device(x.nbytes)
    check(lib.dllm_hip_sigmoid_elementwise(dx.ptr, out.ptr, x.size, None))
    return out.download(x.shape)


def swiglu(gate, up, kind=0) -> np.ndarray:
    """kernels.cpp:633-649: f32(act(gate)) * up, act silu (kind 0) or gelu_tanh (kind 2)."""
    gate, up = _f32(gate), _f32(up)
    if gate.size != up.size:
        raise ValueError("gate and up must have the same size")
    if kind not in (0, 2):
        raise ValueError("kind must be silu (0) or gelu_tanh (2)")
    dg, du, out = Device.of(gate), Device.of(up), Device(gate.nbytes)
    check(lib.dllm_hip_swiglu(dg.ptr, du.ptr, out.ptr, gate.size, int(kind), None))
    return out.download(gate.shape)


# ---- backward kernels ----

def linear_backward(x, weight, dy, with_bias=False):
    """kernels.cpp:811-837: (dx, dweight, dbias or None)."""
    x, w, dy = _f32(x), _f32(weight), _f32(dy)
    if w.ndim != 2:
        raise ValueError("weight must be [out_features, in_features]")
    out_f, in_f = w.shape
    if x.ndim < 1 or x.shape[-1] != in_f:
        raise ValueError("x does not match the weight")
    if dy.ndim != x.ndim or dy.shape[-1] != out_f:
        raise ValueError("dy does not match the weight")
    rows = _rows(x)
    if _rows(dy) != rows:
        raise ValueError("x and dy must have the same leading dimensions")
    ws = Device(lib.dllm_hip_linear_backward_workspace(rows, in_f, out_f))
    d_x, d_w, d_dy = Device.of(x), Device.of(w), Device.of(dy)
    gx, gw = Device(x.nbytes), Device(w.nbytes)
    gb = Device(out_f * 4) if with_bias else None
    check(lib.dllm_hip_linear_backward(d_x.ptr, d_w.ptr, d_dy.ptr, gx.ptr, gw.ptr, gb.ptr if gb else None, rows,
                                       in_f, out_f, ws.ptr, ws.nbytes, None))
    return gx.download(x.shape), gw.download(w.shape), gb.download((out_f,)) if gb else None


def rms_norm_backward(x, weight, dy, eps=1e-6, add_unit_offset=False):
    """kernels.cpp:839-856: (dx, dweight)."""
    x, dy = _f32(x), _f32(dy)
    dim = x.shape[-1]
    if dy.size != x.size or dy.shape[-1] != dim:
        raise ValueError("dy must have the shape of x")
    if weight is not None and _f32(weight).shape[0] != dim:
        raise ValueError("weight length must equal the last dimension of x")
    rows = _rows(x)
    ws = Device(lib.dllm_hip_rms_norm_backward_workspace(rows))
    d_x, d_dy = Device.of(x), Device.of(dy)
    d_w = Device.of(_f32(weight)) if weight is not None else None
    gx, gw = Device(x.nbytes), Device(dim * 4)
    check(lib.dllm_hip_rms_norm_backward(d_x.ptr, d_w.ptr if d_w else None, d_dy.ptr, gx.ptr, gw.ptr, rows, dim,
                                         float(eps), int(add_unit_offset), ws.ptr, ws.nbytes, None))
    return gx.download(x.shape), gw.download((dim,))


def silu_backward(x, dy) -> np.ndarray:
    x, dy = _f32(x), _f32(dy)
    if x.size != dy.size:
        raise ValueError("x and dy must have the same size")
    d_x, d_dy, out = Device.of(x), Device.of(dy), Device(x.nbytes)
    check(lib.dllm_hip_silu_backward(d_x.ptr, d_dy.ptr, out.ptr, x.size, None))
    return out.download(x.shape)


def attention_backward(q, k, v, dout, scale, causal=True, q_offset=-1, window=0, softcap=0.0):
    """kernels.cpp:930-959: (dq, dk, dv)."""
    q, k, v, dout = _f32(q), _f32(k), _f32(v), _f32(dout)
    q_offset = _attention_args(q, k, v, q_offset)
    if dout.ndim != 3 or dout.shape != (q.shape[0], q.shape[1], v.shape[2]):
        raise ValueError("dout must be [q_len, q_heads, value_dim]")
    ws = Device(lib.dllm_hip_attention_backward_workspace(q.shape[0], k.shape[0], q.shape[1], k.shape[1], q.shape[2],
                                                          v.shape[2], int(causal), int(q_offset), int(window),
                                                          float(softcap)))
    d = [Device.of(a) for a in (q, k, v, dout)]
    gq, gk, gv = Device(q.nbytes), Device(k.nbytes), Device(v.nbytes)
    check(lib.dllm_hip_attention_backward(d[0].ptr, d[1].ptr, d[2].ptr, d[3].ptr, gq.ptr, gk.ptr, gv.ptr, q.shape[0],
                                          k.shape[0], q.shape[1], k.shape[1], q.shape[2], v.shape[2], float(scale),
                                          int(causal), int(q_offset), int(window), float(softcap), ws.ptr, ws.nbytes,
                                          None))
    return gq.download(q.shape), gk.download(k.shape), gv.download(v.shape)


def cross_entropy(logits, targets, scale=1.0):
    """kernels.cpp:991-1003: (summed loss, dlogits * scale)."""
    logits = _f32(logits)
    targets = np.ascontiguousarray(targets, dtype=np.int64)
    if logits.ndim != 2:
        raise ValueError("logits must be [rows, vocab]")
    if targets.shape[0] != logits.shape[0]:
        raise ValueError("targets must have one entry per row")
    rows, vocab = logits.shape
    ws = Device(lib.dllm_hip_cross_entropy_workspace(rows))
    dl, dt, out = Device.of(logits), Device.of(targets), Device(logits.nbytes)
    loss = C.c_double()
    check(lib.dllm_hip_cross_entropy(dl.ptr, dt.ptr, out.ptr, rows, vocab, float(scale), C.byref(loss), ws.ptr,
                                     ws.nbytes, None))
    return loss.value, out.download(logits.shape)


def embedding_backward(dy, tokens, vocabulary_size) -> np.ndarray:
    """kernels.cpp:1029-1039."""
    dy = _f32(dy)
    tokens = np.ascontiguousarray(tokens, dtype=np.int64)
    if dy.ndim != 2 or dy.shape[0] != tokens.shape[0]:
        raise ValueError("dy must be [len(tokens), dim]")
    rows, dim = dy.shape
    ws = Device(lib.dllm_hip_embedding_backward_workspace(rows))
    d_dy, d_t, out = Device.of(dy), Device.of(tokens), Device(vocabulary_size * dim * 4)
    check(lib.dllm_hip_embedding_backward(d_dy.ptr, d_t.ptr, out.ptr, rows, dim, int(vocabulary_size), ws.ptr,
                                          ws.nbytes, None))
    return out.download((int(vocabulary_size), dim))


def sum_squares(values) -> float:
    """kernels.cpp:1041-1043."""
    v = _f32(values)
    d, ws = Device.of(v), Device(lib.dllm_hip_sum_squares_workspace(v.size))
    result = C.c_double()
    check(lib.dllm_hip_sum_squares(d.ptr, v.size, C.byref(result), ws.ptr, ws.nbytes, None))
    return result.value


def adamw_step(param, grad, m, v, lr, beta1, beta2, eps, weight_decay, bias_correction1, bias_correction2,
               grad_scale=1.0) -> None:
    """kernels.cpp:1045-1057: in place on param, m and v (float32 C-contiguous arrays)."""
    for a in (param, m, v):
        if a.dtype != np.float32 or not a.flags.c_contiguous:
            raise ValueError("param, m and v must be C-contiguous float32 arrays")
    g = _f32(grad)
    n = param.size
    if g.size != n or m.size != n or v.size != n:
        raise ValueError("param, grad, m and v must have one size")
    dp, dg, dm, dv = Device.of(param), Device.of(g), Device.of(m), Device.of(v)
    check(lib.dllm_hip_adamw_step(dp.ptr, dg.ptr, dm.ptr, dv.ptr, n, float(lr), float(beta1), float(beta2),
                                  float(eps), float(weight_decay), float(bias_correction1), float(bias_correction2),
                                  float(grad_scale), None))
    param[...] = dp.download(param.shape)
    m[...] = dm.download(m.shape)
    v[...] = dv.download(v.shape)


# ---- LoRA and Q8_0 (src/etalii_dllm/lora.py, numerics.py:106-139) ----

def gelu_tanh_backward(x, dy) -> np.ndarray:
    """kernels.cpp:903-914."""
    x, dy = _f32(x), _f32(dy)
    if x.size != dy.size:
        raise ValueError("x and dy must have the same size")
    dx, ddy, out = Device.of(x), Device.of(dy), Device(x.nbytes)
    check(lib.dllm_hip_gelu_tanh_backward(dx.ptr, ddy.ptr, out.ptr, x.size, None))
    return out.download(x.shape)


def softcap_backward(x, dy, cap: float) -> np.ndarray:
    """kernels.cpp:916-928."""
    x, dy = _f32(x), _f32(dy)
    if x.size != dy.size:
        raise ValueError("x and dy must have the same size")
    if not cap > 0.0:
        raise ValueError("cap must be positive")
    dx, ddy, out = Device.of(x), Device.of(dy), Device(x.nbytes)
    check(lib.dllm_hip_softcap_backward(dx.ptr, ddy.ptr, out.ptr, x.size, float(cap), None))
    return out.download(x.shape)


def softmax(logits) -> np.ndarray:
    """kernels.cpp:166-176 (a vector; a matrix is taken row by row)."""
    x = _f32(logits)
    if x.size == 0:
        raise ValueError("softmax needs at least one value")
    n = x.shape[-1]
    d, out = Device.of(x), Device(x.nbytes)
    check(lib.dllm_hip_softmax(d.ptr, out.ptr, x.size // n, n, None))
    return out.download(x.shape)


def column_mean(x) -> np.ndarray:
    """kernels.cpp:787-796."""
    x = _f32(x)
    if x.ndim != 2:
        raise ValueError("x must be [rows, cols]")
    d, out = Device.of(x), Device(max(x.shape[1], 1) * 4)
    check(lib.dllm_hip_column_mean(d.ptr, out.ptr, x.shape[0], x.shape[1], None))
    return out.download((x.shape[1],))


def dot(a, b) -> float:
    """kernels.cpp:153-161: a float (returned as a Python float, as the binding does)."""
    a, b = _f32(a).ravel(), _f32(b).ravel()
    if a.size != b.size:
        raise ValueError("vectors must have the same length")
    da, db, ws = Device.of(a), Device.of(b), Device(lib.dllm_hip_dot_workspace())
    result = C.c_float()
    check(lib.dllm_hip_dot(da.ptr, db.ptr, a.size, C.byref(result), ws.ptr, ws.nbytes, None))
    return float(result.value)


def moe_route(logits, k: int, normalize: bool) -> tuple[np.ndarray, np.ndarray]:
    """kernels.cpp:190-204: (indices int64 [rows, k], weights [rows, k]) in rank order."""
    x = _f32(logits)
    if x.ndim != 2:
        raise ValueError("logits must be [rows, experts]")
    rows, experts = x.shape
    if not 1 <= k <= experts:
        raise ValueError("experts per token must be between 1 and the number of experts")
    d, idx, w = Device.of(x), Device(max(rows * k, 1) * 8), Device(max(rows * k, 1) * 4)
    check(lib.dllm_hip_moe_route(d.ptr, idx.ptr, w.ptr, rows, experts, k, int(bool(normalize)), None))
    return idx.download((rows, k), np.int64), w.download((rows, k))


def moe_route_backward(logits, indices, dweights, dprobabilities, normalize: bool) -> np.ndarray:
    """kernels.cpp:1005-1027: dlogits [rows, experts]."""
    x = _f32(logits)
    idx = np.ascontiguousarray(indices, dtype=np.int64)
    dw = _f32(dweights)
    rows, experts = x.shape
    if idx.ndim != 2 or idx.shape[0] != rows or not 1 <= idx.shape[1] <= experts:
        raise ValueError("indices must be [rows, k] with k between 1 and the number of experts")
    k = idx.shape[1]
    if dw.shape != idx.shape:
        raise ValueError("dweights must have the shape of indices")
    dp = None
    if dprobabilities is not None:
        dp = _f32(dprobabilities)
        if dp.shape != x.shape:
            raise ValueError("dprobabilities must have the shape of logits")
    if np.any(idx < 0) or np.any(idx >= experts):
        raise ValueError("expert index out of range")
    d, di, ddw, out = Device.of(x), Device.of(idx), Device.of(dw), Device(max(x.size, 1) * 4)
    ddp = Device.of(dp) if dp is not None else None
    check(lib.dllm_hip_moe_route_backward(d.ptr, di.ptr, ddw.ptr, ddp.ptr if ddp else None, out.ptr, rows, experts,
                                          k, int(bool(normalize)), None))
    return out.download((rows, experts))


def quantize_q8_0(weight) -> tuple[np.ndarray, np.ndarray]:
    """kernels.cpp quantize_q8_0 as QuantizedWeight uses it: (int8 values [out, in], float scales [out, in / 32])."""
    w = _f32(weight)
    if w.ndim != 2 or w.shape[1] % 32:
        raise ValueError("q8_0 needs a [out_features, in_features] weight with in_features a multiple of 32")
    d, q, s = Device.of(w), Device(w.size), Device(w.size // 32 * 4)
    check(lib.dllm_hip_quantize_q8_0(d.ptr, q.ptr, s.ptr, w.size, None))
    return q.download(w.shape, np.int8), s.download((w.shape[0], w.shape[1] // 32))


lib.dllm_hip_linear_q8_workspace.restype = _sz
lib.dllm_hip_linear_q8_workspace.argtypes = [_sz, _sz]
lib.dllm_hip_linear_q8.argtypes = [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp, _sz, _vp]
lib.dllm_hip_linear_q4_workspace.restype = _sz
lib.dllm_hip_linear_q4_workspace.argtypes = [_sz, _sz, _sz]
lib.dllm_hip_linear_q4.argtypes = [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp, _sz, _vp]
lib.dllm_hip_quantize_q4_0.argtypes = [_vp, _vp, _vp, _sz, _vp]
lib.dllm_hip_unpack_q4_0.argtypes = [_vp, _vp, _sz, _vp]


def _quantized_linear(name, x, q, scales, bias, in_per_row):
    x, s = _f32(x), _f32(scales)
    if x.ndim < 1:
        raise ValueError("x must have at least one dimension")
    in_f = x.shape[-1]
    out_f = q.shape[0]
    if q.ndim != 2 or q.shape[1] * in_per_row != in_f:
        raise ValueError("weight in_features does not match the last dimension of x")
    if in_f % 32:
        raise ValueError(f"{name} needs in_features to be a multiple of 32")
    if s.shape != (out_f, in_f // 32):
        raise ValueError("scales must be [out_features, in_features / 32]")
    if bias is not None and _f32(bias).shape[0] != out_f:
        raise ValueError("bias length must equal out_features")
    rows = _rows(x)
    size = (lib.dllm_hip_linear_q8_workspace(rows, in_f) if name == "Q8_0"
            else lib.dllm_hip_linear_q4_workspace(rows, in_f, out_f))
    ws, dx, dq, ds = Device(size), Device.of(x), Device.of(q), Device.of(s)
    db = Device.of(_f32(bias)) if bias is not None else None
    out = Device(rows * out_f * 4)
    fn = lib.dllm_hip_linear_q8 if name == "Q8_0" else lib.dllm_hip_linear_q4
    check(fn(dx.ptr, dq.ptr, ds.ptr, db.ptr if db else None, out.ptr, rows, in_f, out_f, ws.ptr, ws.nbytes, None))
    return out.download((*x.shape[:-1], out_f))


def linear_q8(x, q, scales, bias=None) -> np.ndarray:
    """kernels.cpp:310-329: Q8_0 linear, activations quantised per 32-block, exact int32 block sums (int8 matrix
    cores), combined in double in block order."""
    return _quantized_linear("Q8_0", x, np.ascontiguousarray(q, dtype=np.int8), scales, bias, 1)


def quantize_q4_0(weight) -> tuple[np.ndarray, np.ndarray]:
    """kernels.cpp:331-348: (packed 4-bit values as bytes [out, in / 2], float32 scales [out, in / 32])."""
    w = _f32(weight)
    if w.ndim != 2 or w.shape[1] % 32:
        raise ValueError("Q4_0 needs in_features to be a multiple of 32")
    d, q, s = Device.of(w), Device(w.size // 2), Device(w.size // 32 * 4)
    check(lib.dllm_hip_quantize_q4_0(d.ptr, q.ptr, s.ptr, w.size, None))
    return q.download((w.shape[0], w.shape[1] // 2), np.int8), s.download((w.shape[0], w.shape[1] // 32))


def unpack_q4_0(q) -> np.ndarray:
    """kernels.cpp:350-363: the int8 values [out, in] of packed Q4_0 values [out, in / 2]."""
    q = np.ascontiguousarray(q, dtype=np.int8)
    if q.ndim != 2 or (q.shape[1] * 2) % 32:
        raise ValueError("Q4_0 needs in_features to be a multiple of 32")
    dq, out = Device.of(q), Device(q.size * 2)
    check(lib.dllm_hip_unpack_q4_0(dq.ptr, out.ptr, q.size * 2, None))
    return out.download((q.shape[0], q.shape[1] * 2), np.int8)


def linear_q4(x, q, scales, bias=None) -> np.ndarray:
    """kernels.cpp:365-385: the weights unpacked to int8, then exactly linear_q8."""
    return _quantized_linear("Q4_0", x, np.ascontiguousarray(q, dtype=np.int8), scales, bias, 2)


lib.dllm_hip_gelu.argtypes = [_vp, _vp, _sz, _vp]
lib.dllm_hip_gelu_backward.argtypes = [_vp, _vp, _vp, _sz, _vp]
lib.dllm_hip_layer_norm.argtypes = [_vp, _vp, _vp, _vp, _sz, _sz, C.c_double, _vp]
lib.dllm_hip_layer_norm_backward_workspace.restype = _sz
lib.dllm_hip_layer_norm_backward_workspace.argtypes = [_sz]
lib.dllm_hip_layer_norm_backward.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, C.c_double, _vp, _sz, _vp]
for _name in ("biased_attention", "biased_attention_backward"):
    getattr(lib, f"dllm_hip_{_name}_workspace").restype = _sz
    getattr(lib, f"dllm_hip_{_name}_workspace").argtypes = [_sz] * 5
lib.dllm_hip_biased_attention_weights.argtypes = [_vp] * 4 + [_sz] * 4 + [C.c_double, _vp, _sz, _vp]
lib.dllm_hip_biased_attention.argtypes = [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, C.c_double, _vp, _sz, _vp]
lib.dllm_hip_biased_attention_backward.argtypes = [_vp] * 9 + [_sz] * 5 + [C.c_double, _vp, _sz, _vp]


def gelu(x) -> np.ndarray:
    """kernels.cpp:631: elementwise exact (erf) GELU."""
    x = _f32(x)
    dx, out = Device.of(x), Device(x.nbytes)
    check(lib.dllm_hip_gelu(dx.ptr, out.ptr, x.size, None))
    return out.download(x.shape)


def gelu_backward(x, dy) -> np.ndarray:
    """kernels.cpp:877-889: dy * gelu'(x) for the exact (erf) GELU."""
    x, dy = _f32(x), _f32(dy)
    if x.size != dy.size:
        raise ValueError("x and dy must have the same size")
    dx, dd, out = Device.of(x), Device.of(dy), Device(x.nbytes)
    check(lib.dllm_hip_gelu_backward(dx.ptr, dd.ptr, out.ptr, x.size, None))
    return out.download(x.shape)


def layer_norm(x, weight, bias, eps=1e-12) -> np.ndarray:
    """kernels.cpp:612-625: LayerNorm over the last dimension, fixed order, double accumulators."""
    x, w, b = _f32(x), _f32(weight), _f32(bias)
    if x.ndim < 1:
        raise ValueError("x must have at least one dimension")
    dim = x.shape[-1]
    if w.shape[0] != dim or b.shape[0] != dim:
        raise ValueError("weight and bias lengths must equal the last dimension of x")
    dx, dw, db, out = Device.of(x), Device.of(w), Device.of(b), Device(x.nbytes)
    check(lib.dllm_hip_layer_norm(dx.ptr, dw.ptr, db.ptr, out.ptr, _rows(x), dim, eps, None))
    return out.download(x.shape)


def layer_norm_backward(x, weight, dy, eps=1e-12):
    """kernels.cpp:858-875: (dx, dweight, dbias) of layer_norm()."""
    x, w, dy = _f32(x), _f32(weight), _f32(dy)
    if x.ndim < 1:
        raise ValueError("x must have at least one dimension")
    dim = x.shape[-1]
    if dy.size != x.size or dy.shape[-1] != dim:
        raise ValueError("dy must have the shape of x")
    if w.shape[0] != dim:
        raise ValueError("weight length must equal the last dimension of x")
    rows = _rows(x)
    ws = Device(lib.dllm_hip_layer_norm_backward_workspace(rows))
    d_x, d_w, d_dy = Device.of(x), Device.of(w), Device.of(dy)
    ddx, ddw, ddb = Device(x.nbytes), Device(dim * 4), Device(dim * 4)
    check(lib.dllm_hip_layer_norm_backward(d_x.ptr, d_w.ptr, d_dy.ptr, ddx.ptr, ddw.ptr, ddb.ptr, rows, dim, eps,
                                           ws.ptr, ws.nbytes, None))
    return ddx.download(x.shape), ddw.download((dim,)), ddb.download((dim,))


def _biased_shapes(q, k, v, bias):
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError("q, k and v must be [length, heads, dim]")
    q_len, heads, kv_len = q.shape[0], q.shape[1], k.shape[0]
    if k.shape[1] != heads or v.shape[1] != heads:
        raise ValueError("q, k and v must have the same heads")
    if v.shape[0] != kv_len:
        raise ValueError("k and v must have the same length")
    if q.shape[2] != k.shape[2]:
        raise ValueError("q and k must have the same head_dim")
    if bias.shape != (heads, q_len, kv_len):
        raise ValueError("bias must be [heads, q_len, kv_len]")
    return q_len, kv_len, heads, q.shape[2], v.shape[2]


def biased_attention(q, k, v, bias, scale) -> np.ndarray:
    """kernels.cpp:707-727: T5 attention with an additive bias [heads, q_len, kv_len]."""
    q, k, v, bias = _f32(q), _f32(k), _f32(v), _f32(bias)
    q_len, kv_len, heads, hd, vd = _biased_shapes(q, k, v, bias)
    ws = Device(lib.dllm_hip_biased_attention_workspace(q_len, kv_len, heads, hd, vd))
    dq, dk, dv, db = Device.of(q), Device.of(k), Device.of(v), Device.of(bias)
    out = Device(q_len * heads * vd * 4)
    check(lib.dllm_hip_biased_attention(dq.ptr, dk.ptr, dv.ptr, db.ptr, out.ptr, q_len, kv_len, heads, hd, vd, scale,
                                        ws.ptr, ws.nbytes, None))
    return out.download((q_len, heads, vd))


def biased_attention_weights(q, k, bias, scale) -> np.ndarray:
    """kernels.cpp:753-773: the probabilities [q_len, heads, kv_len] of biased_attention()."""
    q, k, bias = _f32(q), _f32(k), _f32(bias)
    if q.ndim != 3 or k.ndim != 3:
        raise ValueError("q and k must be [length, heads, dim]")
    q_len, heads, hd, kv_len = q.shape[0], q.shape[1], q.shape[2], k.shape[0]
    if k.shape[1] != heads:
        raise ValueError("q and k must have the same heads")
    if k.shape[2] != hd:
        raise ValueError("q and k must have the same head_dim")
    if bias.shape != (heads, q_len, kv_len):
        raise ValueError("bias must be [heads, q_len, kv_len]")
    ws = Device(lib.dllm_hip_biased_attention_workspace(q_len, kv_len, heads, hd, 4))
    dq, dk, db = Device.of(q), Device.of(k), Device.of(bias)
    out = Device(q_len * heads * kv_len * 4)
    check(lib.dllm_hip_biased_attention_weights(dq.ptr, dk.ptr, db.ptr, out.ptr, q_len, kv_len, heads, hd, scale,
                                                ws.ptr, ws.nbytes, None))
    return out.download((q_len, heads, kv_len))


def biased_attention_backward(q, k, v, bias, dout, scale):
    """kernels.cpp:961-990: (dq, dk, dv, dbias) of biased_attention()."""
    q, k, v, bias, dout = _f32(q), _f32(k), _f32(v), _f32(bias), _f32(dout)
    q_len, kv_len, heads, hd, vd = _biased_shapes(q, k, v, bias)
    if dout.shape != (q_len, heads, vd):
        raise ValueError("dout must be [q_len, heads, value_dim]")
    ws = Device(lib.dllm_hip_biased_attention_backward_workspace(q_len, kv_len, heads, hd, vd))
    d = [Device.of(a) for a in (q, k, v, bias, dout)]
    outs = [Device(max(a.nbytes, 4)) for a in (q, k, v, bias)]
    check(lib.dllm_hip_biased_attention_backward(*(x.ptr for x in d), *(o.ptr for o in outs), q_len, kv_len, heads,
                                                 hd, vd, scale, ws.ptr, ws.nbytes, None))
    return tuple(o.download(a.shape) for o, a in zip(outs, (q, k, v, bias)))


def dequantize_q8_0(values, scales) -> np.ndarray:
    """QuantizedWeight.dequantize (numerics.py:138-139): the int8 values times their block's scale, float32."""
    q = np.ascontiguousarray(values, dtype=np.int8)
    s = _f32(scales)
    if q.size % 32 or s.size * 32 != q.size:
        raise ValueError("q8_0 values come in blocks of 32 with one scale each")
    dq, ds, out = Device.of(q), Device.of(s), Device(q.size * 4)
    check(lib.dllm_hip_dequantize_q8_0(dq.ptr, ds.ptr, out.ptr, q.size, None))
    return out.download(q.shape)


def lora_merge(weight, a, b, scale: float) -> np.ndarray:
    """lora.py:271-276: weight + f32(linear(b, a^T)) * f32(scale), a [rank, in], b [out, rank]."""
    w, a, b = _f32(weight), _f32(a), _f32(b)
    out_f, in_f = w.shape
    rank = a.shape[0]
    if a.shape != (rank, in_f) or b.shape != (out_f, rank):
        raise ValueError("adapters do not match the weight")
    ws = Device(lib.dllm_hip_lora_merge_workspace(out_f, in_f, rank))
    dw, da, db, out = Device.of(w), Device.of(a), Device.of(b), Device(w.nbytes)
    check(lib.dllm_hip_lora_merge(dw.ptr, da.ptr, db.ptr, out.ptr, out_f, in_f, rank, float(scale), ws.ptr, ws.nbytes,
                                  None))
    return out.download(w.shape)


def lora_adapter_gradients(gradient, a, b, scale: float) -> tuple[np.ndarray, np.ndarray]:
    """lora.py:374-383: (dA, dB) = (f32(linear(b^T, dW^T)) * s, f32(linear(dW, a)) * s)."""
    g, a, b = _f32(gradient), _f32(a), _f32(b)
    out_f, in_f = g.shape
    rank = a.shape[0]
    if a.shape != (rank, in_f) or b.shape != (out_f, rank):
        raise ValueError("adapters do not match the gradient")
    ws = Device(lib.dllm_hip_lora_adapter_gradients_workspace(out_f, in_f, rank))
    dg, da, db = Device.of(g), Device.of(a), Device.of(b)
    ga, gb = Device(a.nbytes), Device(b.nbytes)
    check(lib.dllm_hip_lora_adapter_gradients(dg.ptr, da.ptr, db.ptr, ga.ptr, gb.ptr, out_f, in_f, rank, float(scale),
                                              ws.ptr, ws.nbytes, None))
    return ga.download(a.shape), gb.download(b.shape)


class RopeScaling(C.Structure):
    """dllm_hip_rope_scaling."""

    _fields_ = [("kind", C.c_int64)] + [(name, C.c_double) for name in (
        "factor", "low_freq_factor", "high_freq_factor", "original_max_position_embeddings", "beta_fast",
        "beta_slow")] + [("truncate", C.c_int64), ("factors", C.c_void_p)]


ROPE_KINDS = {"default": 0, "linear": 1, "llama3": 2, "longrope": 3, "yarn": 4}
lib.dllm_hip_rope_inv_freq.argtypes = [_sz, C.c_double, _sz, C.POINTER(RopeScaling), _f64p]


def rope_inv_freq(head_dim: int, theta: float = 10000.0, *, rotary_dim: int | None = None, scaling=None) -> np.ndarray:
    """numerics.py:267-324: rotary inverse frequencies theta^(-2i / rotary_dim) in double from the portable exp and
    log, with a Hugging Face rope_scaling dict ("default", "linear", "llama3", "longrope" with its short or long
    factors, "yarn"); ValueError for an odd or too large rotary_dim, an unknown kind or a wrong number of factors."""
    dim = head_dim if rotary_dim is None else rotary_dim
    if dim <= 0 or dim % 2 or dim > head_dim:
        raise ValueError("rotary_dim must be even, positive and at most head_dim")
    kind = "default" if not scaling else str(scaling.get("rope_type", scaling.get("type", "default")))
    if kind not in ROPE_KINDS:
        raise ValueError(f"unsupported rope scaling {kind!r}")
    sc = RopeScaling()
    sc.kind = ROPE_KINDS[kind]
    factors = None
    if kind in ("linear", "llama3", "yarn"):
        sc.factor = float(scaling["factor"])
    if kind == "llama3":
        sc.low_freq_factor = float(scaling.get("low_freq_factor", 1.0))
        sc.high_freq_factor = float(scaling.get("high_freq_factor", 4.0))
        sc.original_max_position_embeddings = float(scaling.get("original_max_position_embeddings", 8192))
    elif kind == "longrope":
        name = "long_factor" if scaling.get("factor_set") == "long" else "short_factor"
        factors = np.ascontiguousarray([float(f) for f in scaling[name]], dtype=np.float64)
        if factors.size != dim // 2:
            raise ValueError(f"longrope {name} needs {dim // 2} values, got {factors.size}")
        sc.factors = factors.ctypes.data
    elif kind == "yarn":
        sc.original_max_position_embeddings = float(scaling["original_max_position_embeddings"])
        sc.beta_fast = float(scaling.get("beta_fast", 32.0))
        sc.beta_slow = float(scaling.get("beta_slow", 1.0))
        sc.truncate = int(bool(scaling.get("truncate", True)))
    out = np.empty(dim // 2, np.float64)
    check(lib.dllm_hip_rope_inv_freq(head_dim, float(theta), dim, C.byref(sc), out.ctypes.data_as(_f64p)))
    return out


def rope_attention_factor(scaling) -> float:
    """architecture.py:331-336: the attention_factor of LongRoPE or YaRN (1 otherwise)."""
    if not scaling or scaling.get("rope_type", scaling.get("type")) not in ("longrope", "yarn"):
        return 1.0
    return float(scaling.get("attention_factor", 1.0))


def attention_scale(head_dim: int) -> float:
    """architecture.py:311-312: 1 / sqrt(head_dim)."""
    return 1.0 / math.sqrt(head_dim)
