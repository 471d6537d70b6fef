"""prism_chain_launch_times (the measurement aid bench.py's roofline uses)
runs exactly the chain's launches: its output equals prism_forward's bit for
bit, and it reports the grids the chain launches (attention: one workgroup
per 8x8 window of a sub-chain's frames; experts: the 128-token tiles of a
d256 sub-chain of 8 frames, 64-token 8-wave tiles at batch 1; dense blocks
run their FFN inside the attention launch, so no expert launch)."""
import numpy as np
import pytest

import prism_amd as P


@pytest.mark.gpu
@pytest.mark.parametrize("name,nb,batch,attn_grid,expert_grid", [
    ("moe64", 2, 16, 1080, 576),   # two sub-chains of 8 frames: 8 x 135 windows; 510 + 64 tiles -> 576
    ("moe64", 2, 1, 135, 192),     # one frame: 8-wave kernels, 128 + 64 tiles -> 192
    ("dense128", 2, 4, 270, 0),    # two sub-chains of 2 frames; attention + FFN in one launch
    ("std256", 2, 2, 270, 0),      # one sub-chain of 2 frames: 8-wave d256 attention + FFN in one launch
    ("std256", 2, 16, 1080, 0),    # two sub-chains of 8 frames: 4-wave attention + FFN in one launch
])
def test_chain_launch_times_run_the_chain(hip, engine, device_arena, name, nb, batch, attn_grid, expert_grid):
    cfg = P.CONFIGS[name]
    desc = cfg.desc(n_blocks=nb)
    blob, offs = P.synth_weights(desc, seed=2, routing=cfg.routing)
    engine.load_weights(desc, blob, offs)
    n, d = batch * cfg.tokens, cfg.dim
    dx, dy, dz = device_arena(n * d * 2), device_arena(n * d * 2), device_arena(n * d * 2)
    hip.upload(dx.ptr, P.synth_features(cfg, batch=batch, seed=3).reshape(-1))
    print(f"[timing] {name} {nb} blocks batch {batch}", flush=True)
    engine.forward(dx.ptr, dy.ptr, batch)
    hip.sync()
    ref = hip.download(np.empty(n * d, np.uint16), dy.ptr)
    ta, te, ga, ge = engine.chain_launch_times(dx.ptr, dz.ptr, batch)
    got = hip.download(np.empty(n * d, np.uint16), dz.ptr)
    print(f"[timing] attention {ta * 1e3:.1f} us x {ga} workgroups, experts {te * 1e3:.1f} us x {ge}", flush=True)
    assert (got == ref).all()
    assert (ga, ge) == (attn_grid, expert_grid)
    assert 0 < ta < 10 and (0 < te < 10 if expert_grid else te == 0)
    # and the forward that follows is unaffected (counters left clean)
    engine.forward(dx.ptr, dz.ptr, batch)
    hip.sync()
    assert (hip.download(np.empty(n * d, np.uint16), dz.ptr) == ref).all()
