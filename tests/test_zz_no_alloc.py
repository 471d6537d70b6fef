"""prism_forward_noalloc (the block chain with its workspace in the device's
fixed scratch array, no allocation) against prism_forward (same launches,
workspace allocated by the context): bit-identical outputs and assignments,
on two calls in a row, the second with a smaller input; a forward whose
workspace does not fit the array is refused before any launch."""
import numpy as np
import pytest

import prism_amd as P

SCRATCH_BYTES = 16 << 20


def workspace_bytes(desc, batch):
    """The chain's workspace for `batch` frames (the engine's layout: 256-byte
    aligned regions for h, the ping-pong rows, the assignments, the counter
    rows and the buckets)."""
    def up(b):
        return (b + 255) // 256 * 256
    n = batch * desc.spatial_h * desc.spatial_w
    return (2 * up(n * desc.dim * 2) + up(desc.n_blocks * n * 4)
            + up(2 * desc.n_blocks * desc.n_experts * 64 * 4) + up(desc.n_experts * n * 4))


@pytest.mark.gpu
def test_forward_noalloc_equals_forward(hip, device_arena):
    eng = P.Engine(0)   # a fresh context: prism_forward_noalloc runs before it has any workspace
    try:
        cfg = P.CONFIGS["moe64"]
        H, W, nb = 20, 28, 3
        desc = cfg.desc(n_blocks=nb, H=H, W=W)
        blob, offs = P.synth_weights(desc, seed=4, routing=cfg.routing)
        eng.load_weights(desc, blob, offs)
        d = cfg.dim
        results = {}
        for batch in (5, 2):    # two sub-chains, then one smaller chain
            n = batch * H * W
            assert workspace_bytes(desc, batch) <= SCRATCH_BYTES
            x = P.synth_features(cfg, batch=batch, H=H, W=W, seed=20 + batch).reshape(-1)
            dx, dz = device_arena(n * d * 2), device_arena(n * d * 2)
            hip.upload(dx.ptr, x)
            hip.memset(dz.ptr, 0xFF, n * d * 2)
            hip.sync()
            free0 = hip.mem_free()
            print(f"[noalloc] moe64 {nb} blocks {H}x{W} batch {batch}", flush=True)
            assert eng.forward_noalloc(dx.ptr, dz.ptr, batch) == 0, eng.error()
            hip.sync()
            free1 = hip.mem_free()
            # a chain workspace for this call would take > 1 MiB
            assert free0 - free1 < (1 << 20), f"device memory dropped by {free0 - free1} bytes"
            z = hip.download(np.empty(n * d, np.uint16), dz.ptr)
            a_ptr, ntok = eng.forward_assignments()
            assert ntok == n
            az = hip.download(np.empty(nb * n, np.int32), a_ptr)
            results[batch] = (dx, z, az)
        for batch, (dx, z, az) in results.items():
            n = batch * H * W
            dy = device_arena(n * d * 2)
            eng.forward(dx.ptr, dy.ptr, batch)   # the allocating entry point
            hip.sync()
            y = hip.download(np.empty(n * d, np.uint16), dy.ptr)
            a_ptr, ntok = eng.forward_assignments()
            ay = hip.download(np.empty(nb * n, np.int32), a_ptr)
            print(f"[noalloc] batch {batch}: {int((z != y).sum())} output values and "
                  f"{int((az != ay).sum())} assignments differ", flush=True)
            assert (z == y).all() and (az == ay).all()
    finally:
        eng.close()


@pytest.mark.gpu
def test_forward_noalloc_headline_model_and_its_limit(hip, device_arena):
    """MoE-64 d256 x 16 blocks at 68x120: batch 1 fits the array and equals
    prism_forward; batch 2 does not fit and is refused, writing nothing."""
    eng = P.Engine(0)
    try:
        cfg = P.CONFIGS["moe64"]
        desc = cfg.desc()
        blob, offs = P.synth_weights(desc, seed=0, routing=cfg.routing)
        eng.load_weights(desc, blob, offs)
        T, d = cfg.H * cfg.W, cfg.dim
        assert workspace_bytes(desc, 1) <= SCRATCH_BYTES < workspace_bytes(desc, 2)
        x = P.synth_features(cfg, batch=2, seed=3).reshape(-1)
        dx, dy, dz = device_arena(2 * T * d * 2), device_arena(2 * T * d * 2), device_arena(2 * T * d * 2)
        hip.upload(dx.ptr, x)
        hip.memset(dz.ptr, 0xFF, 2 * T * d * 2)
        print("[noalloc] moe64 16 blocks 68x120 batch 2 (refused)", flush=True)
        assert eng.forward_noalloc(dx.ptr, dz.ptr, 2) == P.ERR_INVALID
        assert "scratch" in eng.error()
        hip.sync()
        assert (hip.download(np.empty(2 * T * d, np.uint16), dz.ptr) == 0xFFFF).all()
        print("[noalloc] moe64 16 blocks 68x120 batch 1", flush=True)
        assert eng.forward_noalloc(dx.ptr, dz.ptr, 1) == 0, eng.error()
        eng.forward(dx.ptr, dy.ptr, 1)
        hip.sync()
        z = hip.download(np.empty(T * d, np.uint16), dz.ptr)
        y = hip.download(np.empty(T * d, np.uint16), dy.ptr)
        assert (z == y).all()
    finally:
        eng.close()
