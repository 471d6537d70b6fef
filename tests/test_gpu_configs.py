"""GPU parity of the block chain at the configurations' own workloads, through
the C ABI, against the oracle.

- Free-running: prism_forward_graph over the whole model (MoE-32: 22 blocks at
  135x240, batch 4, adversarial routing; MoE-16: 16 blocks at 68x120; MoE-64:
  16 blocks at 68x120, batch 16 = the headline step; dense128 and std256 at
  batch 16) against the free-running oracle. Near-tie routing flips move a few tokens by more than the per-block
  bound, so the whole-model check bounds the mean error (2e-3) and the share
  of tokens moved by more than 2e-2 (2 %).
- Teacher-forced through the chain's own kernels: the chain runs a batch of 4
  or more frames as two sub-chains of half the frames each, and every MoE block
  as one routed attention launch (prism_attn_route) plus one grouped expert
  launch (prism_experts). Calling those two entry points on half the batch
  runs the chain's attention kernels (same grid, same variant) and its expert
  kernels, except that a stage call of 512 or more 128-token tiles takes
  96-token tiles of the same body where the chain keeps 128-token ones (the
  two are bit-identical: test_chain_matches_stage_calls at batch 16); each
  block's input is the oracle's, so every block is held to the per-block
  tolerances (max 2e-2, mean 2e-3) and exact routing on every token whose
  oracle top-1/top-2 logit gap is >= 1e-2. Counts and buckets are exact.

Reference: prism_moe_bench.cpp:262-291 (block sequence), README.md:13-14 (the
MoE-16 and MoE-32 configurations).
"""
import numpy as np
import pytest

import oracle as O
import prism_amd as P
from conftest import errors

MAX_ABS, MEAN_ABS, GAP = 2e-2, 2e-3, 1e-2


def f16(bits):
    return O.f16bits_to_f32(bits)


def subchain_batches(batch):
    """Frames per sub-chain, as the engine splits a batch (2 sub-chains from 4
    frames on)."""
    if batch < 4:
        return [batch]
    return [batch // 2, batch - batch // 2]


def attn_kernel(dim, n_experts, windows, chain=False):
    """The attention kernel the engine launches for a grid of `windows`
    workgroups: 8 waves below 512 windows, 4 waves from 512 on; _r<k> routes
    over 16k padded experts; _ffn: a dense block of the chain, its FFN in the
    same launch."""
    npt = (n_experts + 15) // 16 if n_experts > 1 else 0
    return (f"prism_attn_d{dim}{'_w8' if windows < 512 else ''}{f'_r{npt}' if npt else ''}"
            + ("_ffn" if chain and not npt else ""))


@pytest.mark.gpu
@pytest.mark.parametrize("name,batch,kernel", [
    ("moe32", 4, "prism_attn_d256_r2"),   # 2 x 2 frames of 510 windows: the 4-wave N=32 kernel
    ("moe16", 1, "prism_attn_d256_w8_r1"),
    ("moe64", 16, "prism_attn_d256_r4"),  # the headline step: 2 x 8 frames, 1080 windows each
    ("dense128", 16, "prism_attn_d128_ffn"),  # 2 x 8 frames of 1080 windows, FFN in the launch
    ("std256", 16, "prism_attn_d256_ffn"),    # 2 x 8 frames, FFN in the launch
])
def test_config_chain_against_oracle(hip, engine, device_arena, name, batch, kernel):
    cfg = P.CONFIGS[name]
    H, W, nb = cfg.H, cfg.W, cfg.n_blocks
    windows = ((H + 7) // 8) * ((W + 7) // 8)
    assert attn_kernel(cfg.dim, cfg.n_experts, windows * subchain_batches(batch)[0], chain=True) == kernel
    desc = cfg.desc()
    blob, offs = P.synth_weights(desc, seed=0, routing=cfg.routing)
    engine.load_weights(desc, blob, offs)
    n, d = batch * H * W, cfg.dim
    x_bits = P.synth_features(cfg, batch=batch, H=H, W=W, seed=12).reshape(n, d)
    dx, dy = device_arena(n * d * 2), device_arena(n * d * 2)
    hip.upload(dx.ptr, x_bits)
    print(f"[config] {name}: {nb} blocks {H}x{W} batch {batch} ({kernel})", flush=True)
    engine.forward(dx.ptr, dy.ptr, batch, graph=True)
    hip.sync()
    y = f16(hip.download(np.empty(n * d, np.uint16), dy.ptr)).reshape(n, d)
    routed = cfg.n_experts > 1
    if routed:
        a_ptr, ntok = engine.forward_assignments()
        assert ntok == n
        a_gpu = hip.download(np.empty(nb * n, np.int32), a_ptr).reshape(nb, n)
    print(f"[config] {name}: oracle", flush=True)
    c = O.cfg(cfg.dim, cfg.n_heads, cfg.head_dim, cfg.n_experts, H, W, batch, True)
    ref, a_ref, _ = O.forward(c, O.f16bits_to_f32(blob), list(offs), f16(x_bits))
    err = np.abs(y.astype(np.float64) - ref)
    moved = float((err.max(axis=1) > MAX_ABS).mean())
    same = float((a_gpu == a_ref.reshape(nb, n)).mean()) if routed else 1.0
    load = np.bincount(a_gpu[0], minlength=cfg.n_experts).max() / n if routed else 1.0
    print(f"[config] {name}: max {err.max():.3g} mean {err.mean():.3g}, tokens moved > {MAX_ABS}: {moved:.4f}, "
          f"same expert {same:.5f}, block-0 hottest expert share {load:.3f}")
    assert np.isfinite(y).all()
    assert err.mean() <= MEAN_ABS
    assert moved <= 0.02
    assert same >= 0.98


@pytest.mark.gpu
@pytest.mark.parametrize("name,nb,batch", [
    ("moe64", 2, 16),   # sub-chains of 8 frames: 1080-window prism_attn_d256_r4, 96-token expert tiles
    ("moe32", 2, 4),    # sub-chains of 2 frames at 135x240: 1020-window prism_attn_d256_r2
    ("moe64", 16, 1),   # every block of the headline model at batch 1 (8-wave kernels)
])
def test_chain_kernels_teacher_forced(hip, engine, device_arena, name, nb, batch):
    cfg = P.CONFIGS[name]
    H, W, N, d = cfg.H, cfg.W, cfg.n_experts, cfg.dim
    T = H * W
    desc = cfg.desc(n_blocks=nb)
    blob, offs = P.synth_weights(desc, seed=2, routing=cfg.routing)
    engine.load_weights(desc, blob, offs)
    w = O.f16bits_to_f32(blob)
    x = f16(P.synth_features(cfg, batch=batch, H=H, W=W, seed=13).reshape(batch * T, d))
    cur = x
    for b in range(nb):
        nxt = np.empty_like(cur)
        f0 = 0
        for sb in subchain_batches(batch):
            n = sb * T
            c = O.cfg(d, cfg.n_heads, cfg.head_dim, N, H, W, sb, True)
            xin = cur[f0 * T:(f0 + sb) * T]
            feats = device_arena(3 * n * d * 2)
            aux_n = P.aux_elems(N, n)
            aux = device_arena(aux_n * 4)
            hip.upload(feats.ptr, O.f32_to_f16bits(xin))
            hip.memset(aux.ptr, 0xFF, aux_n * 4)
            pa = engine.attn_push(b, 0, n * d)
            pr = engine.router_push(b, T, n * d, 0, n, n + N)
            print(f"[tf] {name} block {b} frames {f0}..{f0 + sb - 1} "
                  f"({attn_kernel(d, N, sb * ((H + 7) // 8) * ((W + 7) // 8))})", flush=True)
            assert engine.attn_route(pa, pr, feats.ptr, aux.ptr, sb) == 0, engine.error()
            hip.sync()
            h_gpu = f16(hip.download(np.empty(n * d, np.uint16), feats.ptr + n * d * 2)).reshape(n, d)
            host = hip.download(np.empty(aux_n, np.int32), aux.ptr)
            assign, counts = host[:n], host[n:n + N]
            perm = host[n + N:].reshape(N, n)
            h_ref = O.attn_stage(c, w, offs[b], xin)
            mx, mean = errors(h_gpu, h_ref)
            assert mx <= MAX_ABS and mean <= MEAN_ABS, f"attention block {b}: {mx} {mean}"
            ref_assign, logits = O.router_stage(c, w, offs[b], h_ref)
            top2 = np.sort(logits, axis=1)[:, -2:]
            sure = (top2[:, 1] - top2[:, 0]) >= GAP
            assert ((assign >= 0) & (assign < N)).all()
            assert (assign[sure] == ref_assign[sure]).all(), f"routing block {b}"
            assert (counts == np.bincount(assign, minlength=N)).all()
            for e in range(N):
                assert (np.sort(perm[e, :counts[e]]) == np.nonzero(assign == e)[0]).all(), f"bucket {e}"
            # the expert launch on the oracle's h, with the GPU's routing
            hip.upload(feats.ptr + n * d * 2, O.f32_to_f16bits(h_ref))
            push = engine.expert_push(b, T, n * d, 2 * n * d, 0, n, n + N)
            assert engine.experts(push, feats.ptr, aux.ptr, sb) == 0, engine.error()
            hip.sync()
            y_gpu = f16(hip.download(np.empty(n * d, np.uint16), feats.ptr + 2 * n * d * 2)).reshape(n, d)
            y_ref = O.expert_stage(c, w, offs[b], h_ref, assign)
            mx2, mean2 = errors(y_gpu, y_ref)
            print(f"[tf] {name} block {b}: attention max {mx:.3g} mean {mean:.3g}, experts max {mx2:.3g} "
                  f"mean {mean2:.3g}, {int((~sure).sum())} near-tie tokens", flush=True)
            assert mx2 <= MAX_ABS and mean2 <= MEAN_ABS, f"experts block {b}: {mx2} {mean2}"
            nxt[f0 * T:(f0 + sb) * T] = y_ref
            f0 += sb
        cur = nxt


@pytest.mark.gpu
def test_assignments_report_the_last_chain(hip, engine, device_arena):
    """prism_forward_assignments names the token count of the chain that ran
    last, also when that chain was a replay of a graph captured earlier."""
    cfg = P.CONFIGS["moe16"]
    H, W = 20, 28
    desc = cfg.desc(n_blocks=2, H=H, W=W)
    blob, offs = P.synth_weights(desc, seed=1, routing=cfg.routing)
    engine.load_weights(desc, blob, offs)
    x = P.synth_features(cfg, batch=4, H=H, W=W, seed=3).reshape(-1)
    dx, dy = device_arena(x.size * 2), device_arena(x.size * 2)
    hip.upload(dx.ptr, x)
    engine.forward(dx.ptr, dy.ptr, 4, graph=True)
    hip.sync()
    a_ptr, ntok = engine.forward_assignments()
    assert ntok == 4 * H * W
    a4 = hip.download(np.empty(2 * ntok, np.int32), a_ptr)
    engine.forward(dx.ptr, dy.ptr, 1)
    hip.sync()
    assert engine.forward_assignments()[1] == H * W
    engine.forward(dx.ptr, dy.ptr, 4, graph=True)   # the cached graph, replayed
    hip.sync()
    a_ptr, ntok = engine.forward_assignments()
    assert ntok == 4 * H * W
    assert (hip.download(np.empty(2 * ntok, np.int32), a_ptr) == a4).all()


@pytest.mark.gpu
def test_tiny_grids_are_refused(hip, engine, device_arena):
    """Frames of fewer than 64 tokens: the reference keys only the first
    n_tokens window slots there (split2_qkv_attn_d256.comp.glsl:33,60); the
    attention stage and the chain refuse them instead of differing."""
    cfg = P.CONFIGS["moe16"]
    H, W = 5, 7
    desc = cfg.desc(n_blocks=1, H=H, W=W)
    blob, offs = P.synth_weights(desc, seed=1, routing=cfg.routing)
    engine.load_weights(desc, blob, offs)
    n, d = H * W, cfg.dim
    feats = device_arena(3 * n * d * 2)
    assert engine.attn(engine.attn_push(0, 0, n * d), feats.ptr, 1) == P.ERR_UNSUPPORTED
    assert "64" in engine.error()
    with pytest.raises(P.PrismError) as ei:
        engine.forward(feats.ptr, feats.ptr + n * d * 2, 1)
    assert ei.value.code == P.ERR_UNSUPPORTED
