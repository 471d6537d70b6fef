"""Host-renderer interop through the C ABI: prism_init_with_device (the engine
bound to the caller's stream), prism_infer_gpu (caller buffers at byte
offsets, synchronous, GPU time returned) and renderer-owned memory imported
from an exported file descriptor. The renderer-stream results equal
prism_forward_graph's bit for bit and, for the plain chains, are also held to
the free-running oracle directly.

The exporter side of the last test stands in for a Vulkan renderer that
exports a VkDeviceMemory with VK_KHR_external_memory_fd: a HIP allocation made
exportable as a POSIX descriptor (hipMemCreate + hipMemExportToShareableHandle)
and mapped into the test's own address space, so the test can see what the
engine wrote through the renderer's mapping."""
import ctypes as C
import os

import numpy as np
import pytest

import oracle as O
import prism_amd as P

SENTINEL = 0x7E7E  # an fp16 NaN pattern no kernel writes


def _model(engine, name, nb, H, W, adapted, seed=2):
    cfg = P.CONFIGS[name]
    desc = cfg.desc(n_blocks=nb, H=H, W=W)
    blob, offs = P.synth_weights(desc, seed=seed, routing=cfg.routing)
    engine.load_weights(desc, blob, offs)
    ch = cfg.dim
    if adapted:
        ablob, a = P.synth_adapters(desc, seed=seed + 1)
        engine.load_adapters(ablob, a)
        ch = a.in_dim
    return cfg, ch, desc, blob, offs


def _oracle_check(cfg, desc, blob, offs, x_bits, y_bits, H, W, batch):
    """The interop output against the free-running oracle of the same model,
    with the whole-model bounds of the configuration tests (mean error 2e-3,
    at most 2 % of tokens moved by more than 2e-2 by near-tie routing flips)."""
    d = cfg.dim
    c = O.cfg(d, cfg.n_heads, cfg.head_dim, cfg.n_experts, H, W, batch, True)
    ref, _, _ = O.forward(c, O.f16bits_to_f32(blob), list(offs), O.f16bits_to_f32(x_bits).reshape(-1, d))
    y = O.f16bits_to_f32(y_bits).reshape(-1, d).astype(np.float64)
    err = np.abs(y - ref)
    moved = float((err.max(axis=1) > 2e-2).mean())
    print(f"[interop] oracle: max {err.max():.3g} mean {err.mean():.3g}, tokens moved {moved:.4f}", flush=True)
    assert np.isfinite(y).all()
    assert err.mean() <= 2e-3 and moved <= 0.02


def _reference(hip, device_arena, name, nb, H, W, batch, adapted, x):
    """The same model through prism_forward_graph on plain device buffers."""
    eng = P.Engine(0)
    try:
        _, ch, _, _, _ = _model(eng, name, nb, H, W, adapted)
        n = batch * H * W * ch
        dx, dy = device_arena(n * 2), device_arena(n * 2)
        hip.upload(dx.ptr, x)
        eng.forward(dx.ptr, dy.ptr, batch, graph=True, adapted=adapted)
        hip.sync()
        return hip.download(np.empty(n, np.uint16), dy.ptr)
    finally:
        eng.close()


@pytest.mark.gpu
@pytest.mark.parametrize("name,nb,H,W,batch,adapted", [
    ("moe16", 2, 20, 28, 3, False),   # 3 frames: one chain (sub-chains start at 4 frames)
    ("moe16", 2, 20, 28, 5, False),   # two sub-chains (2 + 3 frames)
    ("moe64", 2, 68, 120, 1, True),   # the adapted chain: 128-channel in/out
    ("dense128", 2, 68, 120, 4, False),
])
def test_infer_gpu_on_the_renderer_stream(hip, device_arena, name, nb, H, W, batch, adapted):
    cfg = P.CONFIGS[name]
    ch = 128 if adapted else cfg.dim
    n = batch * H * W * ch
    x = P.synth_normal(n, seed=11)
    ref = _reference(hip, device_arena, name, nb, H, W, batch, adapted, x)

    stream = hip.stream()
    eng = P.Engine(0, stream=stream)
    try:
        _, _, desc, blob, offs = _model(eng, name, nb, H, W, adapted)
        in_off, out_off = 4096, 272  # byte offsets into the caller's buffers (16-byte aligned)
        tail = 512
        inb, outb = device_arena(in_off + n * 2 + tail), device_arena(out_off + n * 2 + tail)
        hip.upload(inb.ptr, np.full((in_off + n * 2 + tail) // 2, SENTINEL, np.uint16))
        hip.upload(inb.ptr + in_off, x)
        hip.upload(outb.ptr, np.full((out_off + n * 2 + tail) // 2, SENTINEL, np.uint16))
        print(f"[interop] {name} batch {batch} adapted={adapted}", flush=True)
        for rep in range(2):  # capture, then replay
            ms = eng.infer_gpu(inb.ptr, in_off, outb.ptr, out_off, batch)
            assert ms > 0.0
            # synchronous: the result is there without a further wait
            got = hip.download(np.empty((out_off + n * 2 + tail) // 2, np.uint16), outb.ptr)
            assert (got[out_off // 2:out_off // 2 + n] == ref).all(), f"call {rep} differs from prism_forward_graph"
            assert (got[:out_off // 2] == SENTINEL).all() and (got[out_off // 2 + n:] == SENTINEL).all()
            print(f"[interop] call {rep}: {ms:.3f} ms", flush=True)
        x_after = hip.download(np.empty(n, np.uint16), inb.ptr + in_off)
        assert (x_after == x).all(), "the input was modified"
        if not adapted:  # the adapted chain's oracle parity: test_gpu_adapters.py
            _oracle_check(cfg, desc, blob, offs, x, got[out_off // 2:out_off // 2 + n], H, W, batch)
        # misaligned offset, overlapping ranges: refused before any launch
        with pytest.raises(P.PrismError) as ei:
            eng.infer_gpu(inb.ptr, in_off + 2, outb.ptr, out_off, batch)
        assert ei.value.code == P.ERR_INVALID
        with pytest.raises(P.PrismError) as ei:
            eng.infer_gpu(inb.ptr, in_off, inb.ptr, in_off + n, batch)
        assert ei.value.code == P.ERR_INVALID and "overlap" in eng.error()
    finally:
        eng.close()
        hip.sync()
        hip.L.hipStreamDestroy(stream)


@pytest.mark.gpu
def test_infer_gpu_needs_weights(hip, device_arena):
    eng = P.Engine(0, stream=None)
    try:
        a = device_arena(4096)
        with pytest.raises(P.PrismError) as ei:
            eng.infer_gpu(a.ptr, 0, a.ptr, 2048, 1)
        assert ei.value.code == P.ERR_STATE
    finally:
        eng.close()


class _Loc(C.Structure):
    _fields_ = [("type", C.c_int), ("id", C.c_int)]


class _AllocFlags(C.Structure):
    _fields_ = [("compressionType", C.c_ubyte), ("gpuDirectRDMACapable", C.c_ubyte), ("usage", C.c_ushort)]


class _AllocProp(C.Structure):  # hipMemAllocationProp
    _fields_ = [("type", C.c_int), ("requestedHandleType", C.c_int), ("location", _Loc),
                ("win32HandleMetaData", C.c_void_p), ("allocFlags", _AllocFlags)]


class _AccessDesc(C.Structure):  # hipMemAccessDesc
    _fields_ = [("location", _Loc), ("flags", C.c_int)]


class ExportedAllocation:
    """Device memory exported as a POSIX file descriptor and mapped here (the
    renderer's side of the interop)."""

    PINNED, POSIX_FD, DEVICE, READ_WRITE = 1, 1, 1, 3

    def __init__(self, hip, nbytes):
        L = self.L = hip.L
        prop = _AllocProp(self.PINNED, self.POSIX_FD, _Loc(self.DEVICE, 0), None, _AllocFlags(0, 0, 0))
        gran = C.c_size_t()
        rc = L.hipMemGetAllocationGranularity(C.byref(gran), C.byref(prop), 0)
        if rc != 0:
            pytest.skip(f"hipMemGetAllocationGranularity: {hip.L.hipGetErrorString(rc).decode()}")
        self.size = -(-nbytes // gran.value) * gran.value
        self.h = C.c_void_p()
        rc = L.hipMemCreate(C.byref(self.h), C.c_size_t(self.size), C.byref(prop), C.c_ulonglong(0))
        if rc != 0:
            pytest.skip(f"hipMemCreate (exportable): {hip.L.hipGetErrorString(rc).decode()}")
        fd = C.c_int(-1)
        rc = L.hipMemExportToShareableHandle(C.byref(fd), self.h, self.POSIX_FD, C.c_ulonglong(0))
        if rc != 0:
            L.hipMemRelease(self.h)
            pytest.skip(f"hipMemExportToShareableHandle: {hip.L.hipGetErrorString(rc).decode()}")
        self.fd = fd.value
        self.va = C.c_void_p()
        ok = L.hipMemAddressReserve(C.byref(self.va), C.c_size_t(self.size), C.c_size_t(0), None,
                                    C.c_ulonglong(0)) == 0
        ok = ok and L.hipMemMap(self.va, C.c_size_t(self.size), C.c_size_t(0), self.h, C.c_ulonglong(0)) == 0
        acc = _AccessDesc(_Loc(self.DEVICE, 0), self.READ_WRITE)
        ok = ok and L.hipMemSetAccess(self.va, C.c_size_t(self.size), C.byref(acc), C.c_size_t(1)) == 0
        assert ok, "mapping the exported allocation failed"

    @property
    def ptr(self) -> int:
        return self.va.value

    def close(self):
        L = self.L
        L.hipDeviceSynchronize()
        L.hipMemUnmap(self.va, C.c_size_t(self.size))
        L.hipMemAddressFree(self.va, C.c_size_t(self.size))
        L.hipMemRelease(self.h)
        os.close(self.fd)


@pytest.mark.gpu
def test_infer_gpu_on_imported_renderer_memory(hip, device_arena):
    name, nb, H, W, batch = "moe16", 2, 20, 28, 2
    cfg = P.CONFIGS[name]
    n = batch * H * W * cfg.dim
    x = P.synth_normal(n, seed=12)
    ref = _reference(hip, device_arena, name, nb, H, W, batch, False, x)

    out_off = (n * 2 + 4095) // 4096 * 4096
    ex = ExportedAllocation(hip, out_off + n * 2)
    eng = P.Engine(0, stream=None)
    buf = None
    try:
        _model(eng, name, nb, H, W, False)
        hip.upload(ex.ptr, x)  # the renderer writes its frame
        buf, ptr = eng.import_external_memory(ex.fd, ex.size)
        os.fstat(ex.fd)  # the caller's descriptor stays open and usable
        # the import aliases the renderer's memory (checked by copies before any kernel runs)
        seen = hip.download(np.empty(n, np.uint16), ptr)
        assert (seen == x).all(), "imported mapping does not alias the exported allocation"
        print("[interop] import aliases the renderer's allocation", flush=True)
        ms = eng.infer_gpu(ptr, 0, ptr, out_off, batch)
        assert ms > 0.0
        # the renderer reads the result through its own mapping
        got = hip.download(np.empty(n, np.uint16), ex.ptr + out_off)
        assert (got == ref).all(), f"{int((got != ref).sum())} values differ from prism_forward_graph"
        eng.release_external_memory(buf)
        buf = None
        os.fstat(ex.fd)
        with pytest.raises(P.PrismError) as ei:
            eng.import_external_memory(-1, ex.size)
        assert ei.value.code == P.ERR_INVALID
    finally:
        if buf is not None:
            eng.release_external_memory(buf)
        eng.close()
        ex.close()
