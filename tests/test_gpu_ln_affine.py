"""GPU parity with non-trivial LayerNorm affines, through the C ABI, against the oracle.

The engine folds each LayerNorm's affine into the weights that consume its
output when it loads a blob: W' = r16(W diag(gamma)), b' = b + W beta, for LN1
into W_qkv and for LN2 into W_r and every expert's W1 (the kernels then only
normalise). The synthetic models have gamma = 1, beta = 0, where that is the
identity; trained models do not. These cases write gamma ~ N(1, 0.3) and
beta ~ N(0, 0.2) into LN1 and LN2 of every block and hold the stages and the
block chain to the bounds every other parity test uses: max |err| <= 2e-2 and
mean |err| <= 2e-3 per stage, exact routing on every token whose oracle
top-1/top-2 logit gap is >= 1e-2, exact counts and buckets.

The oracle applies gamma and beta after normalising (the reference shaders'
order, moe_router.comp.glsl:24-40); the fold moves one fp16 rounding (of
W gamma instead of z gamma + beta), which these bounds cover.
"""
import numpy as np
import pytest

import oracle as O
import prism_amd as P
from conftest import errors

MAX_ABS, MEAN_ABS, GAP = 2e-2, 2e-3, 1e-2


def f16(bits):
    return O.f16bits_to_f32(bits)


def with_affine(blob, offs, dim, seed, small_gamma=False):
    """A copy of `blob` with random LN1/LN2 gamma and beta in every block:
    gamma ~ N(1, 0.3), or with small_gamma |gamma| ~ U(1e-3, 1e-2) with a
    random sign (the folded W' = r16(W gamma) then lies in fp16's subnormal
    range, ~2e-5 for W ~ N(0, 0.02), where it keeps fewer significant bits);
    beta ~ N(0, 0.2)."""
    rng = np.random.default_rng(seed)
    out = blob.copy()
    for o in offs:
        for g_off, b_off in ((o.ln1_g, o.ln1_b), (o.ln2_g, o.ln2_b)):
            if small_gamma:
                g = rng.uniform(1e-3, 1e-2, dim) * rng.choice([-1.0, 1.0], dim)
            else:
                g = rng.normal(1.0, 0.3, dim)
            out[g_off:g_off + dim] = O.f32_to_f16bits(g.astype(np.float32))
            out[b_off:b_off + dim] = O.f32_to_f16bits(rng.normal(0.0, 0.2, dim).astype(np.float32))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("name,batch,kernel,small_gamma", [
    ("moe64", 1, "prism_attn_d256_w8_r4", False),   # 135 windows: 8 waves
    ("moe64", 4, "prism_attn_d256_r4", False),      # 540 windows: 4 waves
    ("moe24d128", 2, "prism_attn_d128_w8_r2", False),
    ("moe64", 1, "prism_attn_d256_w8_r4", True),    # folded weights in fp16's subnormal range
    ("moe64", 4, "prism_attn_d256_r4", True),
])
def test_routed_block_with_affine(hip, engine, device_arena, name, batch, kernel, small_gamma):
    cfg = P.CONFIGS[name] if name in P.CONFIGS else P.Config(name, 128, 2, 8, 16, 24, 68, 120, 1, P.ROUTE_ZIPF)
    H, W, N, d = cfg.H, cfg.W, cfg.n_experts, cfg.dim
    n = batch * H * W
    desc = cfg.desc(n_blocks=1)
    blob0, offs = P.synth_weights(desc, seed=5, routing=cfg.routing)
    blob = with_affine(blob0, offs, d, seed=7, small_gamma=small_gamma)
    engine.load_weights(desc, blob, offs)
    w = f16(blob)
    c = O.cfg(d, cfg.n_heads, cfg.head_dim, N, H, W, batch, True)
    x = f16(P.synth_features(cfg, batch=batch, H=H, W=W, seed=8).reshape(n, d))
    feats = device_arena(3 * n * d * 2)
    aux_n = P.aux_elems(N, n)
    aux = device_arena(aux_n * 4)
    hip.upload(feats.ptr, O.f32_to_f16bits(x))
    print(f"[affine] {name} batch {batch} ({kernel}) small gamma {small_gamma}", flush=True)
    pa = engine.attn_push(0, 0, n * d)
    pr = engine.router_push(0, H * W, n * d, 0, n, n + N)
    assert engine.attn_route(pa, pr, feats.ptr, aux.ptr, batch) == 0, engine.error()
    hip.sync()
    h_gpu = f16(hip.download(np.empty(n * d, np.uint16), feats.ptr + n * d * 2)).reshape(n, d)
    host = hip.download(np.empty(aux_n, np.int32), aux.ptr)
    assign, counts = host[:n], host[n:n + N]
    perm = host[n + N:].reshape(N, n)
    h_ref = O.attn_stage(c, w, offs[0], x)
    mx, mean = errors(h_gpu, h_ref)
    ref_assign, logits = O.router_stage(c, w, offs[0], h_ref)
    top2 = np.sort(logits, axis=1)[:, -2:]
    sure = (top2[:, 1] - top2[:, 0]) >= GAP
    print(f"[affine] {name}: attention max {mx:.3g} mean {mean:.3g}, "
          f"{int((assign != ref_assign).sum())} of {n} experts differ, {int((~sure).sum())} near ties", flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS
    assert (assign[sure] == ref_assign[sure]).all()
    assert (counts == np.bincount(assign, minlength=N)).all()
    for e in range(N):
        assert (np.sort(perm[e, :counts[e]]) == np.nonzero(assign == e)[0]).all(), f"bucket {e}"
    # the expert launch on the oracle's h with the GPU's routing (teacher-forced)
    hip.upload(feats.ptr + n * d * 2, O.f32_to_f16bits(h_ref))
    push = engine.expert_push(0, H * W, n * d, 2 * n * d, 0, n, n + N)
    assert engine.experts(push, feats.ptr, aux.ptr, batch) == 0, engine.error()
    hip.sync()
    y_gpu = f16(hip.download(np.empty(n * d, np.uint16), feats.ptr + 2 * n * d * 2)).reshape(n, d)
    y_ref = O.expert_stage(c, w, offs[0], h_ref, assign)
    mx2, mean2 = errors(y_gpu, y_ref)
    print(f"[affine] {name}: experts max {mx2:.3g} mean {mean2:.3g}", flush=True)
    assert mx2 <= MAX_ABS and mean2 <= MEAN_ABS
    # the standalone router on the fused launch's h: the same routing
    aux2 = device_arena(aux_n * 4)
    hip.upload(feats.ptr + n * d * 2, O.f32_to_f16bits(h_gpu))
    assert engine.router(engine.router_push(0, H * W, n * d, 0, n, n + N), feats.ptr, aux2.ptr, batch) == 0, \
        engine.error()
    hip.sync()
    assert (hip.download(np.empty(n, np.int32), aux2.ptr) == assign).all()


@pytest.mark.gpu
@pytest.mark.parametrize("name,batch,small_gamma", [("std256", 1, False), ("dense128", 2, False),
                                                    ("std256", 1, True)])
def test_dense_block_with_affine(hip, engine, device_arena, name, batch, small_gamma):
    cfg = P.CONFIGS[name]
    H, W, d = cfg.H, cfg.W, cfg.dim
    n = batch * H * W
    desc = cfg.desc(n_blocks=1)
    blob0, offs = P.synth_weights(desc, seed=9, routing=cfg.routing)
    blob = with_affine(blob0, offs, d, seed=10, small_gamma=small_gamma)
    engine.load_weights(desc, blob, offs)
    w = f16(blob)
    c = O.cfg(d, cfg.n_heads, cfg.head_dim, 1, H, W, batch, True)
    x = f16(P.synth_features(cfg, batch=batch, H=H, W=W, seed=11).reshape(n, d))
    feats = device_arena(3 * n * d * 2)
    hip.upload(feats.ptr, O.f32_to_f16bits(x))
    print(f"[affine] {name} batch {batch} small gamma {small_gamma}", flush=True)
    assert engine.attn(engine.attn_push(0, 0, n * d), feats.ptr, batch) == 0, engine.error()
    hip.sync()
    h_gpu = f16(hip.download(np.empty(n * d, np.uint16), feats.ptr + n * d * 2)).reshape(n, d)
    h_ref = O.attn_stage(c, w, offs[0], x)
    mx, mean = errors(h_gpu, h_ref)
    hip.upload(feats.ptr + n * d * 2, O.f32_to_f16bits(h_ref))
    assert engine.experts(engine.expert_push(0, H * W, n * d, 2 * n * d), feats.ptr, None, batch) == 0, \
        engine.error()
    hip.sync()
    y_gpu = f16(hip.download(np.empty(n * d, np.uint16), feats.ptr + 2 * n * d * 2)).reshape(n, d)
    y_ref = O.expert_stage(c, w, offs[0], h_ref, None)
    mx2, mean2 = errors(y_gpu, y_ref)
    print(f"[affine] {name}: attention max {mx:.3g} mean {mean:.3g}, ffn max {mx2:.3g} mean {mean2:.3g}",
          flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS
    assert mx2 <= MAX_ABS and mean2 <= MEAN_ABS


@pytest.mark.gpu
def test_chain_with_affine(hip, engine, device_arena):
    """The free-running chain (two sub-chains of 2 frames) against the
    free-running oracle, as the configuration chain tests bound it."""
    cfg = P.CONFIGS["moe16"]
    H, W, nb, batch, d = cfg.H, cfg.W, 4, 4, cfg.dim
    n = batch * H * W
    desc = cfg.desc(n_blocks=nb)
    blob0, offs = P.synth_weights(desc, seed=11, routing=cfg.routing)
    blob = with_affine(blob0, offs, d, seed=12)
    engine.load_weights(desc, blob, offs)
    x_bits = P.synth_features(cfg, batch=batch, H=H, W=W, seed=13).reshape(n, d)
    dx, dy = device_arena(n * d * 2), device_arena(n * d * 2)
    hip.upload(dx.ptr, x_bits)
    print(f"[affine] chain moe16 {nb} blocks batch {batch}", flush=True)
    engine.forward(dx.ptr, dy.ptr, batch, graph=True)
    hip.sync()
    y = f16(hip.download(np.empty(n * d, np.uint16), dy.ptr)).reshape(n, d)
    a_ptr, ntok = engine.forward_assignments()
    a_gpu = hip.download(np.empty(nb * n, np.int32), a_ptr).reshape(nb, n)
    c = O.cfg(d, cfg.n_heads, cfg.head_dim, cfg.n_experts, H, W, batch, True)
    ref, a_ref, _ = O.forward(c, f16(blob), list(offs), f16(x_bits))
    err = np.abs(y.astype(np.float64) - ref)
    moved = float((err.max(axis=1) > MAX_ABS).mean())
    same = float((a_gpu == a_ref.reshape(nb, n)).mean())
    print(f"[affine] chain: max {err.max():.3g} mean {err.mean():.3g}, moved {moved:.4f}, same expert {same:.5f}")
    assert np.isfinite(y).all()
    assert err.mean() <= MEAN_ABS and moved <= 0.02 and same >= 0.98


@pytest.mark.gpu
def test_affine_overflow_is_refused(hip, engine, device_arena):
    """A gamma that pushes a folded weight past fp16's range is refused with
    PRISM_ERR_BLOB (and names the LayerNorm); the engine still loads a good
    blob afterwards."""
    cfg = P.CONFIGS["moe16"]
    desc = cfg.desc(n_blocks=1, H=20, W=28)
    blob, offs = P.synth_weights(desc, seed=1, routing=cfg.routing)
    bad = blob.copy()
    o = offs[0]
    bad[o.ln2_g + 3] = O.f32_to_f16bits(np.array([60000.0], np.float32))[0]
    bad[o.exp_w1 + 3] = O.f32_to_f16bits(np.array([2.0], np.float32))[0]   # expert 0, row 0, channel 3
    with pytest.raises(P.PrismError) as ei:
        engine.load_weights(desc, bad, offs)
    assert ei.value.code == P.ERR_BLOB
    assert "LayerNorm" in engine.error()
    engine.load_weights(desc, blob, offs)
