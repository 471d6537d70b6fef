"""prism_forward_noalloc (the block chain with its workspace in the device's
fixed scratch array, no allocation) against prism_forward (same launches,
workspace allocated by the context): bit-identical outputs and assignments,
on two calls in a row, the second with a smaller input; a forward whose
workspace does not fit the array is refused before any launch; calls from two
contexts on two streams, enqueued without a synchronisation between them,
run one after another on the shared array; the call captured under global
stream capture (where an allocation or synchronisation would fail the
capture) replays bit-identically; the assignments of a forward are dropped
when the context loads other weights."""
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


def _model(seed=4, nb=3, H=20, W=28):
    cfg = P.CONFIGS["moe64"]
    desc = cfg.desc(n_blocks=nb, H=H, W=W)
    blob, offs = P.synth_weights(desc, seed=seed, routing=cfg.routing)
    return cfg, desc, blob, offs


@pytest.mark.gpu
def test_forward_noalloc_two_contexts_two_streams(hip, device_arena):
    """Two contexts on one GPU, each on its own stream, enqueue four calls each
    with no synchronisation in between: the calls share the scratch array and
    must run one after another, so every output equals prism_forward's."""
    cfg, desc, blob, offs = _model()
    H, W, batch, d = desc.spatial_h, desc.spatial_w, 5, cfg.dim
    n = batch * H * W
    engs = [P.Engine(0), P.Engine(0)]
    try:
        streams = [hip.stream(), hip.stream()]
        xs, refs, outs = [], [], []
        for k, e in enumerate(engs):
            e.load_weights(desc, blob, offs)
            x = P.synth_features(cfg, batch=batch, H=H, W=W, seed=40 + k).reshape(-1)
            dx, dy = device_arena(n * d * 2), device_arena(n * d * 2)
            hip.upload(dx.ptr, x)
            e.forward(dx.ptr, dy.ptr, batch)
            hip.sync()
            xs.append(dx)
            refs.append(hip.download(np.empty(n * d, np.uint16), dy.ptr))
            outs.append([device_arena(n * d * 2) for _ in range(4)])
        print(f"[noalloc] two contexts, two streams: moe64 3 blocks {H}x{W} batch {batch}, 4 calls each",
              flush=True)
        for i in range(4):
            for k, e in enumerate(engs):
                assert e.forward_noalloc(xs[k].ptr, outs[k][i].ptr, batch, streams[k]) == 0, e.error()
        hip.sync()
        for k in range(2):
            for i in range(4):
                z = hip.download(np.empty(n * d, np.uint16), outs[k][i].ptr)
                bad = int((z != refs[k]).sum())
                print(f"[noalloc] context {k} call {i}: {bad} values differ", flush=True)
                assert bad == 0
    finally:
        for e in engs:
            e.close()


@pytest.mark.gpu
def test_forward_noalloc_under_global_capture(hip, device_arena):
    """The call inside hipStreamCaptureModeGlobal capture (an allocation or a
    device synchronisation during it would invalidate the capture): the graph
    replays three times, with eager calls of the same entry point and
    synchronisations between the replays, and every replay equals
    prism_forward."""
    cfg, desc, blob, offs = _model(seed=6)
    H, W, batch, d = desc.spatial_h, desc.spatial_w, 4, cfg.dim
    n = batch * H * W
    eng = P.Engine(0)
    try:
        eng.load_weights(desc, blob, offs)
        x = P.synth_features(cfg, batch=batch, H=H, W=W, seed=50).reshape(-1)
        dx, dy, dz, dw = (device_arena(n * d * 2) for _ in range(4))
        hip.upload(dx.ptr, x)
        eng.forward(dx.ptr, dy.ptr, batch)
        hip.sync()
        ref = hip.download(np.empty(n * d, np.uint16), dy.ptr)
        s = hip.stream()
        print(f"[noalloc] global capture: moe64 3 blocks {H}x{W} batch {batch}", flush=True)
        hip.begin_capture(s, hip.CAPTURE_GLOBAL)
        rc = eng.forward_noalloc(dx.ptr, dz.ptr, batch, s)
        g = hip.end_capture(s)
        assert rc == 0, eng.error()
        gx = hip.graph_instantiate(g)
        try:
            for rep in range(3):
                hip.memset(dz.ptr, 0xFF, n * d * 2)
                hip.sync()
                hip.graph_launch(gx, s)
                hip.stream_sync(s)
                z = hip.download(np.empty(n * d, np.uint16), dz.ptr)
                # the program's own eager work between replays, on the same array
                assert eng.forward_noalloc(dx.ptr, dw.ptr, batch) == 0, eng.error()
                hip.sync()
                w = hip.download(np.empty(n * d, np.uint16), dw.ptr)
                print(f"[noalloc] replay {rep}: {int((z != ref).sum())} values differ; eager call between: "
                      f"{int((w != ref).sum())}", flush=True)
                assert (z == ref).all() and (w == ref).all()
        finally:
            hip.graph_destroy(g, gx)
    finally:
        eng.close()


@pytest.mark.gpu
def test_assignments_dropped_when_weights_reload(hip, device_arena):
    """After prism_forward_noalloc the assignments point into the scratch
    array; loading weights of another shape forgets them (PRISM_ERR_STATE)
    instead of handing out that array with the old token count."""
    cfg, desc, blob, offs = _model(seed=8, nb=2)
    H, W, d = desc.spatial_h, desc.spatial_w, cfg.dim
    n = H * W
    eng = P.Engine(0)
    try:
        eng.load_weights(desc, blob, offs)
        dx, dz = device_arena(n * d * 2), device_arena(n * d * 2)
        hip.upload(dx.ptr, P.synth_features(cfg, batch=1, H=H, W=W, seed=9).reshape(-1))
        assert eng.forward_noalloc(dx.ptr, dz.ptr, 1) == 0, eng.error()
        hip.sync()
        _, ntok = eng.forward_assignments()
        assert ntok == n
        _, desc3, blob3, offs3 = _model(seed=8, nb=3, H=12, W=20)
        eng.load_weights(desc3, blob3, offs3)
        with pytest.raises(P.PrismError) as err:
            eng.forward_assignments()
        assert err.value.code == P.ERR_STATE
    finally:
        eng.close()
