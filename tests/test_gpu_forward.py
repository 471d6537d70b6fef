"""GPU block chain through the C ABI: prism_forward (eager launches) and
prism_forward_graph (hipGraph replay) against each other and the oracle.

- Graph replays are bit-identical to the eager chain (same kernels, same
  order), checked on several replays with eager work in between.
- Per-block parity with teacher forcing: block b's GPU stages run on the
  oracle's input to block b; the oracle's expert stage uses the GPU's routing.
  Every block must meet the stage tolerances (max 2e-2, mean 2e-3).
- End-to-end drift of the free-running GPU chain against the free-running
  oracle is reported; near-tie routing flips make it exceed the per-block
  bound on a handful of tokens, so it is bounded on the mean and on the share
  of tokens that move by more than 2e-2.
"""
import numpy as np
import pytest

import oracle as O
import prism_amd as P
from conftest import errors

MAX_ABS, MEAN_ABS, GAP = 2e-2, 2e-3, 1e-2


def f16(bits):
    return O.f16bits_to_f32(bits)


def setup(hip, engine, name, nb, H, W, seed=0):
    cfg = P.CONFIGS[name]
    desc = cfg.desc(n_blocks=nb, H=H, W=W)
    blob, offs = P.synth_weights(desc, seed=seed, routing=cfg.routing)
    engine.load_weights(desc, blob, offs)
    return cfg, desc, blob, offs, O.f16bits_to_f32(blob)


@pytest.mark.gpu
@pytest.mark.parametrize("name,nb,H,W,batch", [
    ("moe64", 3, 68, 120, 2),
    ("dense128", 4, 68, 120, 1),
    ("moe16", 2, 20, 28, 3),
    ("std256", 2, 16, 16, 1),
])
def test_graph_replay_matches_eager(hip, engine, device_arena, name, nb, H, W, batch):
    cfg, desc, blob, offs, w = setup(hip, engine, name, nb, H, W)
    n, d = batch * H * W, cfg.dim
    x = P.synth_features(cfg, batch=batch, H=H, W=W, seed=5).reshape(n, d)
    dx, dy, dz = device_arena(n * d * 2), device_arena(n * d * 2), device_arena(n * d * 2)
    hip.upload(dx.ptr, x)
    print(f"[fwd] {name} eager", flush=True)
    engine.forward(dx.ptr, dy.ptr, batch)
    hip.sync()
    ref = hip.download(np.empty(n * d, np.uint16), dy.ptr)
    x_after = hip.download(np.empty(n * d, np.uint16), dx.ptr)
    assert (x_after == x.reshape(-1)).all(), "forward modified its input"
    for rep in range(3):
        hip.memset(dz.ptr, 0, n * d * 2)
        engine.forward(dx.ptr, dz.ptr, batch, graph=True)
        hip.sync()
        got = hip.download(np.empty(n * d, np.uint16), dz.ptr)
        assert (got == ref).all(), f"graph replay {rep} differs from the eager chain"
        engine.forward(dx.ptr, dy.ptr, batch)   # eager work between replays
        hip.sync()


@pytest.mark.gpu
@pytest.mark.parametrize("name,nb,H,W,batch", [
    ("moe64", 4, 68, 120, 1),
    ("moe32", 2, 135, 240, 1),
    ("dense128", 4, 68, 120, 1),
    ("std256", 3, 68, 120, 1),
])
def test_blocks_teacher_forced(hip, engine, device_arena, name, nb, H, W, batch):
    cfg, desc, blob, offs, w = setup(hip, engine, name, nb, H, W)
    n, d, N = batch * H * W, cfg.dim, cfg.n_experts
    c = O.cfg(cfg.dim, cfg.n_heads, cfg.head_dim, N, H, W, batch, True)
    x = f16(P.synth_features(cfg, batch=batch, H=H, W=W, seed=6).reshape(n, d))
    feats = device_arena(3 * n * d * 2)
    aux_n = P.aux_elems(N, n)
    aux = device_arena(aux_n * 4)
    a_off, c_off, p_off = 0, n, n + N
    cur = x
    for b in range(nb):
        print(f"[blocks] {name} block {b}", flush=True)
        hip.upload(feats.ptr, O.f32_to_f16bits(cur))
        assert engine.attn(engine.attn_push(b, 0, n * d, H, W), feats.ptr, batch) == 0, engine.error()
        hip.sync()
        h_gpu = f16(hip.download(np.empty(n * d, np.uint16), feats.ptr + n * d * 2)).reshape(n, d)
        h_ref = O.attn_stage(c, w, offs[b], cur)
        mx, mean = errors(h_gpu, h_ref)
        assert mx <= MAX_ABS and mean <= MEAN_ABS, f"attention block {b}: {mx} {mean}"
        # experts run on the oracle's h so that only this block's error is measured
        hip.upload(feats.ptr + n * d * 2, O.f32_to_f16bits(h_ref))
        if N > 1:
            assert engine.router(engine.router_push(b, H * W, n * d, a_off, c_off, p_off), feats.ptr, aux.ptr,
                                 batch) == 0, engine.error()
            push = engine.expert_push(b, H * W, n * d, 2 * n * d, a_off, c_off, p_off)
            assert engine.experts(push, feats.ptr, aux.ptr, batch) == 0, engine.error()
            hip.sync()
            assign = hip.download(np.empty(n, np.int32), aux.ptr)
            ref_assign, logits = O.router_stage(c, w, offs[b], h_ref)
            top2 = np.sort(logits, axis=1)[:, -2:]
            sure = (top2[:, 1] - top2[:, 0]) >= GAP
            assert (assign[sure] == ref_assign[sure]).all(), f"routing block {b}"
        else:
            assign = None
            push = engine.expert_push(b, H * W, n * d, 2 * n * d)
            assert engine.experts(push, feats.ptr, None, batch) == 0, engine.error()
            hip.sync()
        y_gpu = f16(hip.download(np.empty(n * d, np.uint16), feats.ptr + 2 * n * d * 2)).reshape(n, d)
        y_ref = O.expert_stage(c, w, offs[b], h_ref, assign)
        mx, mean = errors(y_gpu, y_ref)
        print(f"[blocks] {name} block {b}: attn ok, ffn max {mx:.3g} mean {mean:.3g}")
        assert mx <= MAX_ABS and mean <= MEAN_ABS, f"ffn block {b}: {mx} {mean}"
        cur = y_ref


@pytest.mark.gpu
@pytest.mark.parametrize("name,nb,H,W,batch", [("moe64", 16, 68, 120, 1), ("std256", 12, 68, 120, 1)])
def test_end_to_end_drift(hip, engine, device_arena, name, nb, H, W, batch):
    cfg, desc, blob, offs, w = setup(hip, engine, name, nb, H, W)
    n, d = batch * H * W, cfg.dim
    x_bits = P.synth_features(cfg, batch=batch, H=H, W=W, seed=8).reshape(n, d)
    dx, dy = device_arena(n * d * 2), device_arena(n * d * 2)
    hip.upload(dx.ptr, x_bits)
    print(f"[e2e] {name} {nb} blocks", flush=True)
    engine.forward(dx.ptr, dy.ptr, batch, graph=True)
    hip.sync()
    y = f16(hip.download(np.empty(n * d, np.uint16), dy.ptr)).reshape(n, d)
    c = O.cfg(cfg.dim, cfg.n_heads, cfg.head_dim, cfg.n_experts, H, W, batch, True)
    ref, _, _ = O.forward(c, w, list(offs), f16(x_bits))
    err = np.abs(y.astype(np.float64) - ref)
    moved = float((err.max(axis=1) > MAX_ABS).mean())
    print(f"[e2e] {name}: max {err.max():.3g} mean {err.mean():.3g}, tokens moved > {MAX_ABS}: {moved:.4f}")
    assert err.mean() <= MEAN_ABS
    assert moved <= 0.02
