"""prism_amd - ctypes binding of libprism.so (the C ABI in include/prism.h).

The product is the C ABI; this module is a thin mirror of it for the tests
and the bench, plus a few lines of HIP runtime plumbing (device memory,
streams, events) taken straight from libamdhip64 so no framework sits between
the caller and the kernels.

The library must be built (``make -C prism-inference_amd``); importing this
module on a machine without it raises instead of falling back to anything.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libprism.so")
CODE_OBJECT_PATH = os.path.join(HERE, "prism_kernels.hsaco")

OK = 0
ERR_INVALID = -1
ERR_UNSUPPORTED = -2
ERR_HIP = -3
ERR_STATE = -4
ERR_BLOB = -5
ERR_NOMEM = -6
ERR_CODE_OBJECT = -7

ROUTE_RANDOM = 0
ROUTE_UNIFORM = 1
ROUTE_ZIPF = 2
ROUTE_ADVERSARIAL = 3


class PrismError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"prism error {code}: {msg}")
        self.code = code


# ---------------------------------------------------------------- structs

class ModelDesc(C.Structure):
    _fields_ = [(n, C.c_int32) for n in
                ("dim", "n_blocks", "n_heads", "head_dim", "n_experts",
                 "spatial_h", "spatial_w", "window")]


OFFSET_FIELDS = ("ln1_g", "ln1_b", "qkv_w", "qkv_b", "out_w", "out_b",
                 "ln2_g", "ln2_b", "router_w", "router_b",
                 "exp_w1", "exp_b1", "exp_w2", "exp_b2", "exp_stride")


class BlockOffsets(C.Structure):
    _fields_ = [(n, C.c_int64) for n in OFFSET_FIELDS]


class AttnPush(C.Structure):
    _fields_ = [("n_tokens", C.c_int32), ("dim", C.c_int32), ("n_heads", C.c_int32),
                ("head_dim", C.c_int32), ("spatial_w", C.c_int32), ("spatial_h", C.c_int32),
                ("window_size", C.c_int32),
                ("qkv_w", C.c_int64), ("qkv_b", C.c_int64), ("out_w", C.c_int64),
                ("out_b", C.c_int64), ("input_offset", C.c_int64), ("output_offset", C.c_int64),
                ("ln1_g", C.c_int64), ("ln1_b", C.c_int64)]


class RouterPush(C.Structure):
    _fields_ = [("n_tokens", C.c_int32), ("dim", C.c_int32), ("n_experts", C.c_int32),
                ("router_w", C.c_int64), ("router_b", C.c_int64), ("input_offset", C.c_int64),
                ("assignment_offset", C.c_int64), ("count_offset", C.c_int64),
                ("ln2_g", C.c_int64), ("ln2_b", C.c_int64), ("perm_offset", C.c_int64)]


class ExpertPush(C.Structure):
    _fields_ = [("n_tokens", C.c_int32), ("dim", C.c_int32), ("n_experts", C.c_int32),
                ("w1", C.c_int64), ("b1", C.c_int64), ("w2", C.c_int64), ("b2", C.c_int64),
                ("expert_stride", C.c_int64), ("input_offset", C.c_int64),
                ("output_offset", C.c_int64), ("assignment_offset", C.c_int64),
                ("count_offset", C.c_int64), ("ln2_g", C.c_int64), ("ln2_b", C.c_int64),
                ("perm_offset", C.c_int64)]


class AdapterOffsets(C.Structure):
    _fields_ = [("in_dim", C.c_int32), ("pad_", C.c_int32), ("up_w", C.c_int64), ("up_b", C.c_int64),
                ("down_w", C.c_int64), ("down_b", C.c_int64)]


CODEC_FIELDS = ("enc0_w", "enc0_b", "enc1_w", "enc1_b", "enc2_w", "enc2_b", "enc3_w", "enc3_b",
                "dec3_w", "dec3_b", "dec2_w", "dec2_b", "dec1_w", "dec1_b", "out_w", "out_b")
# (rows, columns) of each codec weight, in the reference's layouts
CODEC_SHAPES = {"enc0": (32, 81), "enc1": (64, 288), "enc2": (128, 576), "enc3": (128, 1152),
                "dec3": (128, 256), "dec2": (64, 192), "dec1": (32, 96), "out": (12, 32)}


class CodecOffsets(C.Structure):
    _fields_ = [("render_w", C.c_int32), ("render_h", C.c_int32), ("in_channels", C.c_int32),
                ("scale", C.c_int32)] + [(f, C.c_int64) for f in CODEC_FIELDS]


class ProjectPush(C.Structure):
    _fields_ = [("n_tokens", C.c_int32), ("pad_", C.c_int32), ("w_offset", C.c_int64),
                ("b_offset", C.c_int64), ("input_offset", C.c_int64), ("output_offset", C.c_int64)]


# Every entry point the header declares: name -> (restype, argtypes)
_P = C.c_void_p
SIGNATURES = {
    "prism_layout": (C.c_int, [C.POINTER(ModelDesc), C.POINTER(BlockOffsets), C.POINTER(C.c_int64)]),
    "prism_validate": (C.c_int, [C.POINTER(ModelDesc), C.POINTER(BlockOffsets), C.c_int64]),
    "prism_synth_weights": (C.c_int, [C.POINTER(ModelDesc), C.c_uint64, C.c_int32, _P, C.c_int64,
                                      C.POINTER(BlockOffsets)]),
    "prism_synth_normal_f16": (C.c_int, [_P, C.c_int64, C.c_uint64, C.c_uint64, C.c_float]),
    "prism_histogram": (C.c_int, [_P, C.c_int64, C.c_int32, _P]),
    "prism_pack_weight": (C.c_int, [_P, C.c_int32, C.c_int32, C.c_int32, _P]),
    "prism_create": (C.c_int, [C.POINTER(_P), C.c_int32, C.c_char_p]),
    "prism_destroy": (None, [_P]),
    "prism_last_error": (C.c_char_p, [_P]),
    "prism_load_weights": (C.c_int, [_P, C.POINTER(ModelDesc), _P, C.c_size_t, C.POINTER(BlockOffsets)]),
    "prism_load_weights_file": (C.c_int, [_P, C.POINTER(ModelDesc), C.c_char_p, C.POINTER(BlockOffsets)]),
    "prism_attn": (C.c_int, [_P, C.POINTER(AttnPush), _P, C.c_int32, _P]),
    "prism_attn_route": (C.c_int, [_P, C.POINTER(AttnPush), C.POINTER(RouterPush), _P, _P, C.c_int32, _P]),
    "prism_router": (C.c_int, [_P, C.POINTER(RouterPush), _P, _P, C.c_int32, _P]),
    "prism_experts": (C.c_int, [_P, C.POINTER(ExpertPush), _P, _P, C.c_int32, _P]),
    "prism_forward": (C.c_int, [_P, _P, _P, C.c_int32, _P]),
    "prism_forward_graph": (C.c_int, [_P, _P, _P, C.c_int32, _P]),
    "prism_forward_noalloc": (C.c_int, [_P, _P, _P, C.c_int32, _P]),
    "prism_forward_assignments": (C.c_int, [_P, C.POINTER(_P), C.POINTER(C.c_int64)]),
    "prism_chain_launch_times": (C.c_int, [_P, _P, _P, C.c_int32, _P, C.POINTER(C.c_float), C.POINTER(C.c_float),
                                           C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    "prism_aux_elems": (C.c_int64, [C.c_int32, C.c_int64]),
    "prism_adapter_layout": (C.c_int, [C.POINTER(ModelDesc), C.c_int32, C.c_int64, C.POINTER(AdapterOffsets),
                                       C.POINTER(C.c_int64)]),
    "prism_load_adapters": (C.c_int, [_P, _P, C.c_size_t, C.POINTER(AdapterOffsets)]),
    "prism_project_up": (C.c_int, [_P, C.POINTER(ProjectPush), _P, C.c_int32, _P]),
    "prism_project_down": (C.c_int, [_P, C.POINTER(ProjectPush), _P, C.c_int32, _P]),
    "prism_forward_adapted": (C.c_int, [_P, _P, _P, C.c_int32, _P]),
    "prism_read_model_json": (C.c_int, [C.c_char_p, C.POINTER(ModelDesc), C.POINTER(BlockOffsets), C.c_int32,
                                        C.POINTER(AdapterOffsets), C.POINTER(C.c_int32), C.POINTER(C.c_int64)]),
    "prism_load_model_file": (C.c_int, [_P, C.c_char_p, C.c_char_p]),
    "prism_forward_adapted_graph": (C.c_int, [_P, _P, _P, C.c_int32, _P]),
    "prism_init_with_device": (C.c_int, [C.POINTER(_P), C.c_int32, _P, C.c_char_p]),
    "prism_infer_gpu": (C.c_int, [_P, _P, C.c_uint64, _P, C.c_uint64, C.c_int32, C.POINTER(C.c_float)]),
    "prism_import_external_memory": (C.c_int, [_P, C.c_int32, C.c_uint64, C.POINTER(_P), C.POINTER(_P)]),
    "prism_release_external_memory": (C.c_int, [_P, _P]),
    "prism_codec_layout": (C.c_int, [C.POINTER(ModelDesc), C.c_int32, C.c_int32, C.c_int64, C.POINTER(CodecOffsets),
                                     C.POINTER(AdapterOffsets), C.POINTER(C.c_int64)]),
    "prism_load_codec": (C.c_int, [_P, _P, C.c_size_t, C.POINTER(CodecOffsets)]),
    "prism_encode": (C.c_int, [_P, _P, _P, C.c_int32, _P]),
    "prism_decode": (C.c_int, [_P, _P, _P, C.c_int32, _P]),
    "prism_codec_stage": (C.c_int, [_P, C.c_int32, _P, _P, _P, C.c_int32, _P]),
    "prism_forward_e2e": (C.c_int, [_P, _P, _P, C.c_int32, _P]),
    "prism_forward_e2e_graph": (C.c_int, [_P, _P, _P, C.c_int32, _P]),
}

_lib = None


def lib() -> C.CDLL:
    """Load libprism.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `make -C {HERE}` "
                               "(or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _check(rc: int, ctx=None):
    if rc != OK:
        msg = lib().prism_last_error(ctx)
        raise PrismError(rc, msg.decode() if msg else "")


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---------------------------------------------------------------- configs

@dataclass(frozen=True)
class Config:
    """A workload: model shape + grid + batch + routing of the router bias."""
    name: str
    dim: int
    n_blocks: int
    n_heads: int
    head_dim: int
    n_experts: int
    H: int
    W: int
    batch: int
    routing: int
    window: int = 8

    def desc(self, n_blocks: int | None = None, H: int | None = None, W: int | None = None) -> ModelDesc:
        return ModelDesc(self.dim, self.n_blocks if n_blocks is None else n_blocks, self.n_heads,
                         self.head_dim, self.n_experts, self.H if H is None else H,
                         self.W if W is None else W, self.window)

    @property
    def tokens(self) -> int:
        return self.H * self.W

    def flops_per_token_block(self) -> int:
        """Algorithmic FLOPs per real token per block (GEMMs + attention MACs x 2)."""
        d, hd = self.dim, self.head_dim
        qkv = 3 * d * d
        attn = 2 * 64 * d            # q.k over 64 keys + p.v over 64 keys, all heads
        out = d * d
        router = d * self.n_experts if self.n_experts > 1 else 0
        ffn = 2 * d * d
        del hd
        return 2 * (qkv + attn + out + router + ffn)


# The five workloads of the path (dense baseline, standard dense, MoE-16, the
# MoE-64 headline, MoE-32 deep at 1080p-native): shape, block count, routing.
CONFIGS = {
    "dense128": Config("dense128", 128, 4, 8, 16, 1, 68, 120, 1, ROUTE_RANDOM),
    "std256": Config("std256", 256, 12, 8, 32, 1, 68, 120, 1, ROUTE_RANDOM),
    "moe16": Config("moe16", 256, 16, 8, 32, 16, 68, 120, 1, ROUTE_UNIFORM),
    "moe64": Config("moe64", 256, 16, 8, 32, 64, 68, 120, 1, ROUTE_ZIPF),
    "moe32": Config("moe32", 256, 22, 8, 32, 32, 135, 240, 4, ROUTE_ADVERSARIAL),
}


# ---------------------------------------------------------------- host helpers

def layout(desc: ModelDesc):
    n = desc.n_blocks
    offs = (BlockOffsets * n)()
    total = C.c_int64()
    _check(lib().prism_layout(C.byref(desc), offs, C.byref(total)))
    return offs, total.value


def validate(desc: ModelDesc, offs, blob_elems: int) -> int:
    return lib().prism_validate(C.byref(desc), offs, blob_elems)


def synth_weights(desc: ModelDesc, seed: int = 0, routing: int = ROUTE_RANDOM):
    """(blob uint16[total], offsets) for the synthetic model."""
    offs, total = layout(desc)
    blob = np.empty(total, dtype=np.uint16)
    _check(lib().prism_synth_weights(C.byref(desc), seed, routing, _ptr(blob), total, offs))
    return blob, offs


def synth_normal(n: int, seed: int = 0, stream: int = 0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    _check(lib().prism_synth_normal_f16(_ptr(out), n, seed, stream, std))
    return out


def synth_features(cfg: Config, batch: int | None = None, seed: int = 0, H=None, W=None) -> np.ndarray:
    """fp16 bits of activations ~N(0,1), [batch][H*W][dim]."""
    b = cfg.batch if batch is None else batch
    h = cfg.H if H is None else H
    w = cfg.W if W is None else W
    return synth_normal(b * h * w * cfg.dim, seed=seed, stream=0, std=1.0).reshape(b, h * w, cfg.dim)


ADAPTER_IN = 128  # encoder channels either side of the block chain


def adapter_layout(desc: ModelDesc, base: int = 0, in_dim: int = ADAPTER_IN):
    """(AdapterOffsets, end element) for the adapters placed from `base` on."""
    a = AdapterOffsets()
    end = C.c_int64()
    _check(lib().prism_adapter_layout(C.byref(desc), in_dim, base, C.byref(a), C.byref(end)))
    return a, end.value


def synth_adapters(desc: ModelDesc, seed: int = 0, in_dim: int = ADAPTER_IN, std: float = 0.02):
    """(blob uint16, AdapterOffsets): both projections ~N(0, std^2), weights
    and biases alike, from the same generator as the blocks (own streams)."""
    a, end = adapter_layout(desc, 0, in_dim)
    blob = np.zeros(end, dtype=np.uint16)
    D = desc.dim
    for k, (off, n) in enumerate(((a.up_w, D * in_dim), (a.up_b, D), (a.down_w, in_dim * D), (a.down_b, in_dim))):
        blob[off:off + n] = synth_normal(n, seed=seed, stream=(0xAD << 24) | k, std=std)
    return blob, a


RENDER = (960, 540)  # the reference's render resolution r0 (prism_moe_bench.cpp:359)


def codec_resolutions(render_w: int = RENDER[0], render_h: int = RENDER[1]):
    """[(w, h)] of r0..r3: each stride-2 conv gives ceil(r / 2)."""
    r = [(render_w, render_h)]
    for _ in range(3):
        w, h = r[-1]
        r.append(((w + 1) // 2, (h + 1) // 2))
    return r


def codec_layout(desc: ModelDesc, render_w: int = RENDER[0], render_h: int = RENDER[1], base: int = 0):
    """(CodecOffsets, AdapterOffsets, end): encoder, adapters, decoder from `base`."""
    c, a, end = CodecOffsets(), AdapterOffsets(), C.c_int64()
    _check(lib().prism_codec_layout(C.byref(desc), render_w, render_h, base, C.byref(c), C.byref(a), C.byref(end)))
    return c, a, end.value


def synth_codec(desc: ModelDesc, seed: int = 0, render_w: int = RENDER[0], render_h: int = RENDER[1],
                base: int = 0, adapter_std: float = 0.02):
    """(blob uint16, CodecOffsets, AdapterOffsets) of the end-to-end section from
    element `base` on (elements below it are zero): conv / pointwise weights
    ~N(0, 2/K) for K inputs per output, so activations keep their scale
    through the ReLU stack; biases ~N(0, 0.02^2); adapters as synth_adapters."""
    c, a, end = codec_layout(desc, render_w, render_h, base)
    blob = np.zeros(end, dtype=np.uint16)
    for k, (name, (rows, cols)) in enumerate(CODEC_SHAPES.items()):
        wo, bo = getattr(c, name + "_w"), getattr(c, name + "_b")
        blob[wo:wo + rows * cols] = synth_normal(rows * cols, seed=seed, stream=(0xC0 << 24) | (2 * k),
                                                 std=float(np.sqrt(2.0 / cols)))
        blob[bo:bo + rows] = synth_normal(rows, seed=seed, stream=(0xC0 << 24) | (2 * k + 1), std=0.02)
    D, I = desc.dim, a.in_dim
    for k, (off, n) in enumerate(((a.up_w, D * I), (a.up_b, D), (a.down_w, I * D), (a.down_b, I))):
        blob[off:off + n] = synth_normal(n, seed=seed, stream=(0xAD << 24) | k, std=adapter_std)
    return blob, c, a


def read_model_json(path: str):
    """(ModelDesc, offsets, AdapterOffsets | None, total fp16 values) from a sidecar."""
    desc = ModelDesc()
    _check(lib().prism_read_model_json(path.encode(), C.byref(desc), None, 0, None, None, None))
    offs = (BlockOffsets * desc.n_blocks)()
    a = AdapterOffsets()
    has = C.c_int32()
    total = C.c_int64()
    _check(lib().prism_read_model_json(path.encode(), C.byref(desc), offs, desc.n_blocks, C.byref(a), C.byref(has),
                                       C.byref(total)))
    return desc, offs, (a if has.value else None), total.value


def pack_weight(w: np.ndarray, rows_padded: int | None = None) -> np.ndarray:
    rows, k = w.shape
    rp = rows if rows_padded is None else rows_padded
    w = np.ascontiguousarray(w, dtype=np.uint16)
    out = np.empty(rp * k, dtype=np.uint16)
    _check(lib().prism_pack_weight(_ptr(w), rows, k, rp, _ptr(out)))
    return out


def histogram(assign: np.ndarray, n_experts: int) -> np.ndarray:
    a = np.ascontiguousarray(assign, dtype=np.int32)
    out = np.zeros(n_experts, dtype=np.int64)
    _check(lib().prism_histogram(_ptr(a), a.size, n_experts, _ptr(out)))
    return out


def aux_elems(n_experts: int, tokens: int) -> int:
    return int(lib().prism_aux_elems(n_experts, tokens))


# ---------------------------------------------------------------- HIP plumbing

class Hip:
    """Device memory, streams and events straight from libamdhip64."""

    H2D, D2H, D2D = 1, 2, 3

    def __init__(self):
        self.L = C.CDLL("libamdhip64.so")
        L = self.L
        L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        L.hipFree.argtypes = [C.c_void_p]
        L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        L.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        L.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        L.hipStreamDestroy.argtypes = [C.c_void_p]
        L.hipStreamSynchronize.argtypes = [C.c_void_p]
        L.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        L.hipEventDestroy.argtypes = [C.c_void_p]
        L.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        L.hipEventSynchronize.argtypes = [C.c_void_p]
        L.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        L.hipGetErrorString.restype = C.c_char_p
        L.hipGetErrorString.argtypes = [C.c_int]
        L.hipGetDeviceCount.argtypes = [C.POINTER(C.c_int)]
        L.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
        L.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
        L.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
        L.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]
        L.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
        L.hipGraphDestroy.argtypes = [C.c_void_p]
        L.hipGraphExecDestroy.argtypes = [C.c_void_p]

    def _ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {self.L.hipGetErrorString(rc).decode()}")

    def device_count(self) -> int:
        n = C.c_int(0)
        rc = self.L.hipGetDeviceCount(C.byref(n))
        return n.value if rc == 0 else 0

    def malloc(self, nbytes: int) -> int:
        p = C.c_void_p()
        self._ok(self.L.hipMalloc(C.byref(p), max(int(nbytes), 1)), "hipMalloc")
        return p.value

    def free(self, p: int):
        self._ok(self.L.hipFree(C.c_void_p(p)), "hipFree")

    def upload(self, dst: int, a: np.ndarray):
        a = np.ascontiguousarray(a)
        self._ok(self.L.hipMemcpy(C.c_void_p(dst), C.c_void_p(a.ctypes.data), a.nbytes, self.H2D), "hipMemcpy H2D")

    def download(self, a: np.ndarray, src: int) -> np.ndarray:
        assert a.flags["C_CONTIGUOUS"]
        self._ok(self.L.hipMemcpy(C.c_void_p(a.ctypes.data), C.c_void_p(src), a.nbytes, self.D2H), "hipMemcpy D2H")
        return a

    def copy(self, dst: int, src: int, nbytes: int):
        self._ok(self.L.hipMemcpy(C.c_void_p(dst), C.c_void_p(src), nbytes, self.D2D), "hipMemcpy D2D")

    def memset(self, p: int, value: int, nbytes: int):
        self._ok(self.L.hipMemset(C.c_void_p(p), value, nbytes), "hipMemset")

    def mem_free(self) -> int:
        """Free device memory in bytes (hipMemGetInfo)."""
        free, total = C.c_size_t(), C.c_size_t()
        self._ok(self.L.hipMemGetInfo(C.byref(free), C.byref(total)), "hipMemGetInfo")
        return free.value

    def sync(self):
        self._ok(self.L.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def stream(self) -> int:
        s = C.c_void_p()
        self._ok(self.L.hipStreamCreate(C.byref(s)), "hipStreamCreate")
        return s.value

    def stream_sync(self, s: int):
        self._ok(self.L.hipStreamSynchronize(C.c_void_p(s)), "hipStreamSynchronize")

    def event(self) -> int:
        e = C.c_void_p()
        self._ok(self.L.hipEventCreate(C.byref(e)), "hipEventCreate")
        return e.value

    def record(self, ev: int, stream: int | None):
        self._ok(self.L.hipEventRecord(C.c_void_p(ev), C.c_void_p(stream or 0)), "hipEventRecord")

    CAPTURE_GLOBAL = 0  # hipStreamCaptureModeGlobal

    def begin_capture(self, stream: int, mode: int = CAPTURE_GLOBAL):
        self._ok(self.L.hipStreamBeginCapture(C.c_void_p(stream), mode), "hipStreamBeginCapture")

    def end_capture(self, stream: int) -> int:
        """The captured graph (raises if the capture was invalidated)."""
        g = C.c_void_p()
        self._ok(self.L.hipStreamEndCapture(C.c_void_p(stream), C.byref(g)), "hipStreamEndCapture")
        return g.value

    def graph_instantiate(self, graph: int) -> int:
        x = C.c_void_p()
        self._ok(self.L.hipGraphInstantiate(C.byref(x), C.c_void_p(graph), None, None, 0), "hipGraphInstantiate")
        return x.value

    def graph_launch(self, graph_exec: int, stream: int):
        self._ok(self.L.hipGraphLaunch(C.c_void_p(graph_exec), C.c_void_p(stream)), "hipGraphLaunch")

    def graph_destroy(self, graph: int, graph_exec: int | None = None):
        if graph_exec:
            self._ok(self.L.hipGraphExecDestroy(C.c_void_p(graph_exec)), "hipGraphExecDestroy")
        self._ok(self.L.hipGraphDestroy(C.c_void_p(graph)), "hipGraphDestroy")

    def elapsed_ms(self, a: int, b: int) -> float:
        self._ok(self.L.hipEventSynchronize(C.c_void_p(b)), "hipEventSynchronize")
        ms = C.c_float()
        self._ok(self.L.hipEventElapsedTime(C.byref(ms), C.c_void_p(a), C.c_void_p(b)), "hipEventElapsedTime")
        return ms.value


# ---------------------------------------------------------------- engine

class Engine:
    """One prism_ctx: weights on the device and the stage / chain launches."""

    def __init__(self, device: int = 0, code_object: str | None = None, stream: int | None = None):
        """prism_create, or prism_init_with_device when a renderer stream is given."""
        self.L = lib()
        h = C.c_void_p()
        co = code_object.encode() if code_object else None
        if stream is None:
            rc = self.L.prism_create(C.byref(h), device, co)
        else:
            rc = self.L.prism_init_with_device(C.byref(h), device, stream, co)
        _check(rc, None)
        self.h = h
        self.desc = None
        self.offs = None

    def close(self):
        if self.h:
            self.L.prism_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def error(self) -> str:
        return self.L.prism_last_error(self.h).decode()

    def load_weights(self, desc: ModelDesc, blob: np.ndarray, offs):
        blob = np.ascontiguousarray(blob, dtype=np.uint16)
        _check(self.L.prism_load_weights(self.h, C.byref(desc), _ptr(blob), blob.nbytes, offs), self.h)
        self.desc = desc
        self.offs = offs

    def load_weights_file(self, desc: ModelDesc, path: str, offs):
        _check(self.L.prism_load_weights_file(self.h, C.byref(desc), path.encode(), offs), self.h)
        self.desc = desc
        self.offs = offs

    def attn(self, push: AttnPush, features: int, batch: int, stream: int | None = None) -> int:
        return self.L.prism_attn(self.h, C.byref(push), features, batch, stream)

    def attn_route(self, pa: AttnPush, pr: RouterPush, features: int, aux: int, batch: int,
                   stream: int | None = None) -> int:
        return self.L.prism_attn_route(self.h, C.byref(pa), C.byref(pr), features, aux, batch, stream)

    def router(self, push: RouterPush, features: int, aux: int, batch: int, stream: int | None = None) -> int:
        return self.L.prism_router(self.h, C.byref(push), features, aux, batch, stream)

    def experts(self, push: ExpertPush, features: int, aux: int | None, batch: int,
                stream: int | None = None) -> int:
        return self.L.prism_experts(self.h, C.byref(push), features, aux, batch, stream)

    def forward(self, x: int, y: int, batch: int, stream: int | None = None, graph: bool = False,
                adapted: bool = False):
        if adapted:
            f = self.L.prism_forward_adapted_graph if graph else self.L.prism_forward_adapted
        else:
            f = self.L.prism_forward_graph if graph else self.L.prism_forward
        _check(f(self.h, x, y, batch, stream), self.h)

    def forward_noalloc(self, x: int, y: int, batch: int, stream: int | None = None) -> int:
        """prism_forward_noalloc: the eager chain on the device's scratch array
        (no allocation); returns the status code."""
        return self.L.prism_forward_noalloc(self.h, x, y, batch, stream)

    def infer_gpu(self, in_buf: int, in_offset: int, out_buf: int, out_offset: int, batch: int) -> float:
        """prism_infer_gpu: one synchronous inference between caller buffers; returns GPU ms."""
        ms = C.c_float()
        _check(self.L.prism_infer_gpu(self.h, in_buf, in_offset, out_buf, out_offset, batch, C.byref(ms)), self.h)
        return ms.value

    def import_external_memory(self, fd: int, size: int):
        """(handle, device pointer) of an exported allocation's first `size` bytes."""
        buf, ptr = C.c_void_p(), C.c_void_p()
        _check(self.L.prism_import_external_memory(self.h, fd, size, C.byref(buf), C.byref(ptr)), self.h)
        return buf, ptr.value

    def release_external_memory(self, buf):
        _check(self.L.prism_release_external_memory(self.h, buf), self.h)

    def load_codec(self, blob: np.ndarray, coffs: CodecOffsets):
        blob = np.ascontiguousarray(blob, dtype=np.uint16)
        _check(self.L.prism_load_codec(self.h, _ptr(blob), blob.nbytes, C.byref(coffs)), self.h)
        self.coffs = coffs

    def encode(self, frame: int, bottleneck: int, batch: int, stream: int | None = None):
        _check(self.L.prism_encode(self.h, frame, bottleneck, batch, stream), self.h)

    def decode(self, bottleneck: int, display: int, batch: int, stream: int | None = None):
        _check(self.L.prism_decode(self.h, bottleneck, display, batch, stream), self.h)

    def codec_stage(self, stage: int, x: int, skip: int | None, y: int, batch: int, stream: int | None = None):
        _check(self.L.prism_codec_stage(self.h, stage, x, skip, y, batch, stream), self.h)

    def forward_e2e(self, frame: int, display: int, batch: int, stream: int | None = None, graph: bool = False):
        f = self.L.prism_forward_e2e_graph if graph else self.L.prism_forward_e2e
        _check(f(self.h, frame, display, batch, stream), self.h)

    def load_model_file(self, weights_path: str, json_path: str | None = None):
        _check(self.L.prism_load_model_file(self.h, weights_path.encode(),
                                            json_path.encode() if json_path else None), self.h)
        desc, offs, a, _ = read_model_json(json_path or weights_path[:-len(".weights")] + ".json")
        self.desc, self.offs = desc, offs
        if a is not None:
            self.aoffs = a

    def load_adapters(self, blob: np.ndarray, aoffs: AdapterOffsets):
        blob = np.ascontiguousarray(blob, dtype=np.uint16)
        _check(self.L.prism_load_adapters(self.h, _ptr(blob), blob.nbytes, C.byref(aoffs)), self.h)
        self.aoffs = aoffs

    def project(self, up: bool, push: ProjectPush, features: int, batch: int, stream: int | None = None) -> int:
        f = self.L.prism_project_up if up else self.L.prism_project_down
        return f(self.h, C.byref(push), features, batch, stream)

    def project_push(self, up: bool, n_tokens: int, in_off: int, out_off: int) -> ProjectPush:
        a = self.aoffs
        return ProjectPush(n_tokens, 0, a.up_w if up else a.down_w, a.up_b if up else a.down_b, in_off, out_off)

    def chain_launch_times(self, x: int, y: int, batch: int, stream: int | None = None):
        """prism_chain_launch_times: (attention ms, expert ms, attention grid,
        expert grid), the means over the chain's launches run one by one."""
        a, e = C.c_float(), C.c_float()
        ga, ge = C.c_int32(), C.c_int32()
        _check(self.L.prism_chain_launch_times(self.h, x, y, batch, stream, C.byref(a), C.byref(e), C.byref(ga),
                                               C.byref(ge)), self.h)
        return a.value, e.value, ga.value, ge.value

    def forward_assignments(self):
        p = C.c_void_p()
        n = C.c_int64()
        _check(self.L.prism_forward_assignments(self.h, C.byref(p), C.byref(n)), self.h)
        return p.value, n.value

    # push builders from the offset table (the reference's push-constant arrays)
    def attn_push(self, b: int, in_off: int, out_off: int, H: int | None = None, W: int | None = None) -> AttnPush:
        d, o = self.desc, self.offs[b]
        h = d.spatial_h if H is None else H
        w = d.spatial_w if W is None else W
        return AttnPush(h * w, d.dim, d.n_heads, d.head_dim, w, h, d.window,
                        o.qkv_w, o.qkv_b, o.out_w, o.out_b, in_off, out_off, o.ln1_g, o.ln1_b)

    def router_push(self, b: int, n_tokens: int, in_off: int, assign_off: int, count_off: int,
                    perm_off: int) -> RouterPush:
        d, o = self.desc, self.offs[b]
        return RouterPush(n_tokens, d.dim, d.n_experts, o.router_w, o.router_b, in_off, assign_off,
                          count_off, o.ln2_g, o.ln2_b, perm_off)

    def expert_push(self, b: int, n_tokens: int, in_off: int, out_off: int, assign_off: int = -1,
                    count_off: int = -1, perm_off: int = -1) -> ExpertPush:
        d, o = self.desc, self.offs[b]
        n_exp = d.n_experts if count_off >= 0 else 1
        return ExpertPush(n_tokens, d.dim, n_exp, o.exp_w1, o.exp_b1, o.exp_w2, o.exp_b2, o.exp_stride,
                          in_off, out_off, assign_off, count_off, o.ln2_g, o.ln2_b, perm_off)
