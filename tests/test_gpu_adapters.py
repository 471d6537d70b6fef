"""GPU parity of the projection adapters (pw_project_128to256 + ReLU,
pw_project_256to128) through the C ABI, and of the adapted chain
(up-projection -> blocks -> down-projection, prism_moe_bench.cpp:408-444).

Tolerances: the stage bound (max |err| <= 2e-2, mean <= 2e-3) against the
fp16-faithful oracle; in practice the GPU and oracle differ only where the
fp32 sums, accumulated in different orders, round to neighbouring fp16
values, which is checked as a share of differing elements. ReLU outputs are
never negative. The adapted chain is checked like the plain chain
(graph replay == eager, end-to-end drift bounded on mean and moved tokens).
"""
import numpy as np
import pytest

import oracle as O
import prism_amd as P
from conftest import errors
from test_gpu_ln_affine import with_affine

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def f16(bits):
    return O.f16bits_to_f32(bits)


def adapters_f32(desc, blob, a):
    D, I = desc.dim, a.in_dim
    w = f16(blob)
    return (w[a.up_w:a.up_w + D * I].reshape(D, I), w[a.up_b:a.up_b + D],
            w[a.down_w:a.down_w + I * D].reshape(I, D), w[a.down_b:a.down_b + I])


def setup(engine, name, nb, H, W, seed=0, affine=False):
    """Model + adapters loaded; affine: random LN gammas and betas in every
    block (LN1 beta != 0 sends windows with padded slots through the attention
    kernels' PAD bodies, also in the first block with the fused up-projection)."""
    cfg = P.CONFIGS[name]
    desc = cfg.desc(n_blocks=nb, H=H, W=W)
    blob, offs = P.synth_weights(desc, seed=seed, routing=cfg.routing)
    if affine:
        blob = with_affine(blob, offs, cfg.dim, seed=seed + 7)
    engine.load_weights(desc, blob, offs)
    ablob, a = P.synth_adapters(desc, seed=seed + 100)
    engine.load_adapters(ablob, a)
    return cfg, desc, blob, offs, ablob, a


@pytest.mark.gpu
@pytest.mark.parametrize("name,H,W,batch", [
    ("moe64", 68, 120, 1),
    ("moe64", 9, 13, 1),      # 117 tokens: one partial 64-token tile
    ("moe64", 20, 28, 3),
    ("dense128", 68, 120, 2),  # 128 <-> 128
])
def test_projection_stages(hip, engine, device_arena, name, H, W, batch):
    cfg, desc, blob, offs, ablob, a = setup(engine, name, 1, H, W)
    up_w, up_b, dn_w, dn_b = adapters_f32(desc, ablob, a)
    n, D, I = batch * H * W, cfg.dim, a.in_dim
    x = P.synth_normal(n * I, seed=11).reshape(n, I)
    feats = device_arena((n * I + n * D + n * I) * 2 + 64)
    o_x, o_h, o_y = 0, n * I, n * I + n * D
    hip.upload(feats.ptr, x)
    hip.memset(feats.ptr + o_h * 2, 0xFF, n * D * 2)  # NaN fill: every output must be written
    print(f"[proj] {name} {H}x{W} batch {batch}", flush=True)
    assert engine.project(True, engine.project_push(True, H * W, o_x, o_h), feats.ptr, batch) == 0, engine.error()
    hip.sync()
    h = f16(hip.download(np.empty(n * D, np.uint16), feats.ptr + o_h * 2)).reshape(n, D)
    ref_h = O.project(up_w, up_b, f16(x), True)
    mx, mean = errors(h, ref_h)
    diff = float((h != ref_h).mean())
    print(f"[proj] up: max {mx:.3g} mean {mean:.3g}, {diff:.2e} of values differ")
    assert np.isfinite(h).all() and (h >= 0).all()
    assert mx <= MAX_ABS and mean <= MEAN_ABS and diff < 0.01
    # down-projection of the oracle's h, so only this stage's error is measured
    hip.upload(feats.ptr + o_h * 2, O.f32_to_f16bits(ref_h))
    assert engine.project(False, engine.project_push(False, H * W, o_h, o_y), feats.ptr, batch) == 0, engine.error()
    hip.sync()
    y = f16(hip.download(np.empty(n * I, np.uint16), feats.ptr + o_y * 2)).reshape(n, I)
    ref_y = O.project(dn_w, dn_b, ref_h, False)
    mx, mean = errors(y, ref_y)
    diff = float((y != ref_y).mean())
    print(f"[proj] down: max {mx:.3g} mean {mean:.3g}, {diff:.2e} of values differ")
    assert mx <= MAX_ABS and mean <= MEAN_ABS and diff < 0.01
    # the input region is untouched
    assert (hip.download(np.empty(n * I, np.uint16), feats.ptr) == x.reshape(-1)).all()


@pytest.mark.gpu
def test_projection_rejects_wrong_weights(hip, engine, device_arena):
    cfg, desc, blob, offs, ablob, a = setup(engine, "moe64", 1, 9, 13)
    feats = device_arena(117 * 384 * 2)
    bad = engine.project_push(True, 117, 0, 117 * 128)
    bad.w_offset = a.down_w
    assert engine.project(True, bad, feats.ptr, 1) == P.ERR_INVALID
    assert "adapter" in engine.error()
    misaligned = engine.project_push(True, 117, 3, 117 * 128)
    assert engine.project(True, misaligned, feats.ptr, 1) == P.ERR_INVALID


@pytest.mark.gpu
def test_adapted_chain_needs_adapters(hip, device_arena):
    eng = P.Engine(0)
    try:
        cfg = P.CONFIGS["moe16"]
        desc = cfg.desc(n_blocks=1, H=9, W=13)
        blob, offs = P.synth_weights(desc, seed=0, routing=cfg.routing)
        eng.load_weights(desc, blob, offs)
        buf = device_arena(117 * 256 * 2)
        with pytest.raises(P.PrismError) as ei:
            eng.forward(buf.ptr, buf.ptr, 1, adapted=True)
        assert ei.value.code == P.ERR_STATE
    finally:
        eng.close()


@pytest.mark.gpu
@pytest.mark.parametrize("name,nb,H,W,batch,affine", [
    ("moe64", 4, 68, 120, 1, False), ("dense128", 3, 68, 120, 2, False),
    ("moe16", 2, 20, 28, 3, False), ("moe16", 2, 20, 28, 4, False),
    # LN affines: PAD and PAD+HALF bodies (the 68-row grid's bottom windows)
    # with the fused up-projection in block 0, 8-wave and 4-wave kernels
    ("moe64", 3, 68, 120, 1, True), ("moe64", 2, 68, 120, 4, True), ("dense128", 2, 68, 120, 2, True),
])
def test_adapted_chain(hip, engine, device_arena, name, nb, H, W, batch, affine):
    cfg, desc, blob, offs, ablob, a = setup(engine, name, nb, H, W, affine=affine)
    up_w, up_b, dn_w, dn_b = adapters_f32(desc, ablob, a)
    n, I = batch * H * W, a.in_dim
    x = P.synth_normal(n * I, seed=12).reshape(n, I)
    dx, dy, dz = device_arena(n * I * 2), device_arena(n * I * 2), device_arena(n * I * 2)
    hip.upload(dx.ptr, x)
    print(f"[adapted] {name} {nb} blocks {H}x{W} batch {batch} affine={affine}", flush=True)
    engine.forward(dx.ptr, dy.ptr, batch, adapted=True)
    hip.sync()
    y = hip.download(np.empty(n * I, np.uint16), dy.ptr)
    for rep in range(2):  # graph replays are bit-identical to the eager chain
        hip.memset(dz.ptr, 0, n * I * 2)
        engine.forward(dx.ptr, dz.ptr, batch, graph=True, adapted=True)
        hip.sync()
        assert (hip.download(np.empty(n * I, np.uint16), dz.ptr) == y).all(), f"replay {rep}"
    c = O.cfg(cfg.dim, cfg.n_heads, cfg.head_dim, cfg.n_experts, H, W, batch, True)
    h0 = O.project(up_w, up_b, f16(x), True)
    hN, _, _ = O.forward(c, f16(blob), list(offs), h0)
    ref = O.project(dn_w, dn_b, hN, False)
    err = np.abs(f16(y).reshape(n, I).astype(np.float64) - ref)
    moved = float((err.max(axis=1) > MAX_ABS).mean())
    print(f"[adapted] {name}: max {err.max():.3g} mean {err.mean():.3g}, tokens moved > {MAX_ABS}: {moved:.4f}")
    assert err.mean() <= MEAN_ABS and moved <= 0.02


@pytest.mark.gpu
@pytest.mark.parametrize("name,nb,H,W,batch,affine", [
    ("moe16", 2, 20, 28, 4, False),    # two sub-chains; ragged windows
    ("moe64", 1, 68, 120, 1, False),   # one block: up- and down-projection in the same block
    ("moe64", 3, 68, 120, 1, False),   # 8-wave kernels
    ("dense128", 3, 68, 120, 2, False),
    ("std256", 2, 16, 16, 5, False),   # dense d256, sub-chains of 2 and 3 frames
    # LN affines (LN1 beta != 0): block 0's windows with padded slots run the
    # PAD / PAD+HALF bodies with the fused up-projection; every window of
    # every block equals the separate calls bit for bit
    ("moe64", 2, 68, 120, 1, True),    # 8 waves
    ("moe64", 2, 68, 120, 4, True),    # 4 waves
    ("moe16", 1, 20, 28, 4, True),     # ragged right and bottom windows, one block
    ("dense128", 2, 68, 120, 2, True),
    ("std256", 2, 68, 120, 16, True),  # 4-wave d256 attention with the up-projection and the FFN
    ("std256", 2, 68, 120, 1, True),   # the same in 8 waves
])
def test_fused_adapters_equal_the_separate_calls(hip, engine, device_arena, name, nb, H, W, batch, affine):
    """The adapted chain fuses the up-projection into the first block's
    attention prologue and the down-projection into the last block's expert
    epilogue, with the projection kernels' arithmetic: its output is
    bit-identical to prism_project_up -> the plain chain -> prism_project_down."""
    cfg, desc, blob, offs, ablob, a = setup(engine, name, nb, H, W, affine=affine)
    n, D, I = batch * H * W, cfg.dim, a.in_dim
    x = P.synth_normal(n * I, seed=13).reshape(n, I)
    feats = device_arena((n * I + 2 * n * D + n * I) * 2 + 64)
    o_x, o_h, o_g, o_y = 0, n * I, n * I + n * D, n * I + 2 * n * D
    hip.upload(feats.ptr, x)
    print(f"[fused] {name} {nb} blocks {H}x{W} batch {batch} affine={affine}", flush=True)
    assert engine.project(True, engine.project_push(True, H * W, o_x, o_h), feats.ptr, batch) == 0, engine.error()
    engine.forward(feats.ptr + o_h * 2, feats.ptr + o_g * 2, batch)
    assert engine.project(False, engine.project_push(False, H * W, o_g, o_y), feats.ptr, batch) == 0, engine.error()
    hip.sync()
    ref = hip.download(np.empty(n * I, np.uint16), feats.ptr + o_y * 2)
    dy = device_arena(n * I * 2)
    for graph in (False, True, True):
        hip.memset(dy.ptr, 0xFF, n * I * 2)  # NaN fill: every output row must be written
        engine.forward(feats.ptr, dy.ptr, batch, graph=graph, adapted=True)
        hip.sync()
        got = hip.download(np.empty(n * I, np.uint16), dy.ptr)
        assert (got == ref).all(), f"graph={graph}: {int((got != ref).sum())} values differ"
    assert np.isfinite(f16(ref)).all()
