"""oracle.py - ctypes wrapper of liboracle.so, the CPU restatement of the
Prism block chain (oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke entry point and the
bench's cpu_baseline leg, as the parity oracle. The product never imports it.

All arrays are float32 numpy arrays holding fp16-representable values on
input (fp16 bits are widened with numpy's exact float16 -> float32 cast).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

OFFSET_FIELDS = ("ln1_g", "ln1_b", "qkv_w", "qkv_b", "out_w", "out_b",
                 "ln2_g", "ln2_b", "router_w", "router_b",
                 "exp_w1", "exp_b1", "exp_w2", "exp_b2", "exp_stride")


class Cfg(C.Structure):
    _fields_ = [(n, C.c_int) for n in
                ("dim", "n_heads", "head_dim", "n_experts", "H", "W", "window", "batch", "faithful")]


class Offs(C.Structure):
    _fields_ = [(n, C.c_int64) for n in OFFSET_FIELDS]


_lib = None
_F = C.POINTER(C.c_float)
_I = C.POINTER(C.c_int32)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `make -C {HERE}`")
        L = C.CDLL(LIB_PATH)
        L.oracle_attn_stage.argtypes = [C.POINTER(Cfg), _F, C.POINTER(Offs), _F, _F]
        L.oracle_router_stage.argtypes = [C.POINTER(Cfg), _F, C.POINTER(Offs), _F, _I, _F]
        L.oracle_expert_stage.argtypes = [C.POINTER(Cfg), _F, C.POINTER(Offs), _F, _I, _F]
        L.oracle_forward.argtypes = [C.POINTER(Cfg), _F, C.POINTER(Offs), C.c_int, _F, _F, _I, _F]
        L.oracle_layernorm.argtypes = [_F, _F, _F, C.c_int, C.c_int, C.c_int, _F]
        L.oracle_gelu.argtypes = [_F, _F, C.c_size_t]
        L.oracle_project.argtypes = [_F, _F, C.c_int, C.c_int, C.c_int, _F, C.c_int, C.c_int, _F]
        L.oracle_window_attention.argtypes = [C.POINTER(Cfg), _F, _F, _F, _F]
        L.oracle_conv3x3.argtypes = [_F, C.c_int, C.c_int, C.c_int, C.c_int, _F, _F, C.c_int, C.c_int, C.c_int, _F]
        L.oracle_conv3x3_split.argtypes = [_F, C.c_int, C.c_int, C.c_int, _F, _F, C.c_int, C.c_int, C.c_int, _F]
        L.oracle_dec_stage.argtypes = [_F, C.c_int, C.c_int, C.c_int, _F, C.c_int, C.c_int, C.c_int, _F, _F,
                                       C.c_int, C.c_int, _F]
        L.oracle_pw_conv.argtypes = [_F, C.c_int, C.c_int, C.c_int, _F, _F, C.c_int, C.c_int, C.c_int, _F]
        L.oracle_pixelshuffle_sigmoid.argtypes = [_F, C.c_int, C.c_int, C.c_int, C.c_int, _F]
        L.oracle_f16_to_f32.argtypes = [C.POINTER(C.c_uint16), _F, C.c_size_t]
        L.oracle_f32_to_f16.argtypes = [_F, C.POINTER(C.c_uint16), C.c_size_t]
        L.oracle_max_threads.restype = C.c_int
        L.oracle_set_threads.argtypes = [C.c_int]
        _lib = L
    return _lib


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_F)


def _i(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_I)


def f16bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def cfg(dim, n_heads, head_dim, n_experts, H, W, batch, faithful=True, window=8) -> Cfg:
    return Cfg(dim, n_heads, head_dim, n_experts, H, W, window, batch, int(bool(faithful)))


def offs_from(o) -> Offs:
    """Copy any object with the 15 offset fields (e.g. prism_amd.BlockOffsets)."""
    return Offs(*[getattr(o, n) for n in OFFSET_FIELDS])


def offs_array(offs_list):
    arr = (Offs * len(offs_list))()
    for i, o in enumerate(offs_list):
        arr[i] = offs_from(o)
    return arr


def _chk(rc, what):
    if rc != 0:
        raise ValueError(f"{what} rejected its arguments (rc={rc})")


def attn_stage(c: Cfg, w: np.ndarray, o, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros_like(x)
    oo = offs_from(o)
    _chk(lib().oracle_attn_stage(C.byref(c), _f(w), C.byref(oo), _f(x), _f(y)), "oracle_attn_stage")
    return y


def router_stage(c: Cfg, w: np.ndarray, o, h: np.ndarray):
    h = np.ascontiguousarray(h, dtype=np.float32)
    n = c.batch * c.H * c.W
    assign = np.zeros(n, dtype=np.int32)
    logits = np.zeros((n, c.n_experts), dtype=np.float32)
    oo = offs_from(o)
    _chk(lib().oracle_router_stage(C.byref(c), _f(w), C.byref(oo), _f(h), _i(assign), _f(logits)),
         "oracle_router_stage")
    return assign, logits


def expert_stage(c: Cfg, w: np.ndarray, o, h: np.ndarray, assign: np.ndarray | None) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.float32)
    y = np.zeros_like(h)
    oo = offs_from(o)
    a = None if assign is None else np.ascontiguousarray(assign, dtype=np.int32)
    _chk(lib().oracle_expert_stage(C.byref(c), _f(w), C.byref(oo), _f(h),
                                   None if a is None else _i(a), _f(y)), "oracle_expert_stage")
    return y


def forward(c: Cfg, w: np.ndarray, offs_list, x: np.ndarray, keep_h: bool = False):
    """(y, assign[n_blocks][n], h[n_blocks][...] or None)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    nb = len(offs_list)
    n = c.batch * c.H * c.W
    y = np.zeros_like(x)
    assign = np.zeros((nb, n), dtype=np.int32)
    h = np.zeros((nb,) + x.shape, dtype=np.float32) if keep_h else None
    arr = offs_array(offs_list)
    _chk(lib().oracle_forward(C.byref(c), _f(w), arr, nb, _f(x), _f(y), _i(assign),
                              _f(h) if keep_h else None), "oracle_forward")
    return y, assign, h


def project(W: np.ndarray, b: np.ndarray, x: np.ndarray, relu: bool, faithful: bool = True) -> np.ndarray:
    """Projection adapter: y = r16(W x + b) per token (+ ReLU for the up
    projection). W [out][in], x [n][in] (float32, fp16-representable)."""
    W = np.ascontiguousarray(W, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    out_dim, in_dim = W.shape
    assert x.shape[1] == in_dim and b.shape == (out_dim,)
    y = np.empty((x.shape[0], out_dim), np.float32)
    _chk(lib().oracle_project(_f(W), _f(b), in_dim, out_dim, int(relu), _f(x), x.shape[0], int(faithful), _f(y)),
         "oracle_project")
    return y


def layernorm(x: np.ndarray, g: np.ndarray, b: np.ndarray, round16: bool = False) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, d = x.shape
    y = np.zeros_like(x)
    lib().oracle_layernorm(_f(x), _f(np.ascontiguousarray(g, np.float32)),
                           _f(np.ascontiguousarray(b, np.float32)), n, d, int(round16), _f(y))
    return y


def gelu(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros_like(x)
    lib().oracle_gelu(_f(x), _f(y), x.size)
    return y


def window_attention(c: Cfg, q: np.ndarray, k: np.ndarray, v: np.ndarray) -> np.ndarray:
    q, k, v = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v))
    out = np.zeros_like(q)
    lib().oracle_window_attention(C.byref(c), _f(q), _f(k), _f(v), _f(out))
    return out


def f16_roundtrip(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 bits -> fp32 through the oracle's own converters."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = np.zeros(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16(_f(x), bits.ctypes.data_as(C.POINTER(C.c_uint16)), x.size)
    back = np.zeros(x.shape, dtype=np.float32)
    lib().oracle_f16_to_f32(bits.ctypes.data_as(C.POINTER(C.c_uint16)), _f(back), x.size)
    return bits, back


def max_threads() -> int:
    return lib().oracle_max_threads()


def set_threads(n: int):
    lib().oracle_set_threads(n)


# ---- conv encoder / fused decoder, CHW maps -------------------------------

def conv3x3(x: np.ndarray, W: np.ndarray, b: np.ndarray, stride: int, relu: bool = True,
            faithful: bool = True) -> np.ndarray:
    """x [cin][h][w], W [cout][cin*9] (k = ic*9 + ky*3 + kx) -> [cout][oh][ow]."""
    cin, h, w = x.shape
    cout = W.shape[0]
    oh, ow = (h - 1) // stride + 1, (w - 1) // stride + 1
    x, W, b = (np.ascontiguousarray(a, dtype=np.float32) for a in (x, W, b))
    y = np.empty((cout, oh, ow), np.float32)
    _chk(lib().oracle_conv3x3(_f(x), cin, h, w, stride, _f(W), _f(b), cout, int(relu), int(faithful), _f(y)),
         "oracle_conv3x3")
    return y


def conv3x3_split(x: np.ndarray, W: np.ndarray, b: np.ndarray, groups: int, mode: int) -> np.ndarray:
    """The reference's split stride-2 conv3x3 + ReLU with its own rounding: each
    group's partial sum r16(b + W_g . x_g), combined in fp32 (mode 0, two
    groups: strided_conv_split_64ch) or as a running fp16 sum (mode 1:
    strided_conv_split_128ch). x [cin][h][w], W [cout][cin*9]."""
    cin, h, w = x.shape
    cout = W.shape[0]
    x, W, b = (np.ascontiguousarray(a, dtype=np.float32) for a in (x, W, b))
    y = np.empty((cout, (h - 1) // 2 + 1, (w - 1) // 2 + 1), np.float32)
    _chk(lib().oracle_conv3x3_split(_f(x), cin, h, w, _f(W), _f(b), cout, groups, mode, _f(y)),
         "oracle_conv3x3_split")
    return y


def dec_stage(up: np.ndarray, skip: np.ndarray, W: np.ndarray, b: np.ndarray, faithful: bool = True) -> np.ndarray:
    """up [cup][uh][uw], skip [cskip][oh][ow], W [cout][cup+cskip] -> [cout][oh][ow] (ReLU)."""
    cup, uh, uw = up.shape
    cskip, oh, ow = skip.shape
    cout = W.shape[0]
    up, skip, W, b = (np.ascontiguousarray(a, dtype=np.float32) for a in (up, skip, W, b))
    y = np.empty((cout, oh, ow), np.float32)
    _chk(lib().oracle_dec_stage(_f(up), cup, uh, uw, _f(skip), cskip, oh, ow, _f(W), _f(b), cout, int(faithful),
                                _f(y)), "oracle_dec_stage")
    return y


def pw_conv(x: np.ndarray, W: np.ndarray, b: np.ndarray, relu: bool = False, faithful: bool = True) -> np.ndarray:
    cin, h, w = x.shape
    cout = W.shape[0]
    x, W, b = (np.ascontiguousarray(a, dtype=np.float32) for a in (x, W, b))
    y = np.empty((cout, h, w), np.float32)
    _chk(lib().oracle_pw_conv(_f(x), cin, h, w, _f(W), _f(b), cout, int(relu), int(faithful), _f(y)),
         "oracle_pw_conv")
    return y


def pixelshuffle_sigmoid(x: np.ndarray, s: int = 2, faithful: bool = True) -> np.ndarray:
    c, h, w = x.shape
    assert c == 3 * s * s
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty((3, h * s, w * s), np.float32)
    _chk(lib().oracle_pixelshuffle_sigmoid(_f(x), h, w, s, int(faithful), _f(y)), "oracle_pixelshuffle_sigmoid")
    return y
