"""Pins the CPU oracle (oracle/oracle.c) without the reference running.

The reference's hot path is GLSL on NVIDIA cooperative vectors and ships no
golden vectors, so each oracle function is checked against what fixes it
independently: library implementations (numpy's fp16 cast, torch's
layer_norm / gelu / scaled_dot_product_attention / linear in fp64), closed
forms and invariants (identical keys, a dominant key, permutations, window
locality, padding, zero weights, ties), and an independent torch fp64
restatement of the whole block built from those library calls with
windows cut by reshape/permute instead of index arithmetic.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
import prism_amd as P

torch.set_grad_enabled(False)


# ------------------------------------------------------------------ fp16

def test_f16_roundtrip_all_bit_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = bits.view(np.float16)
    finite = np.isfinite(f.astype(np.float32)) | np.isinf(f.astype(np.float32))
    back_bits, back = O.f16_roundtrip(f.astype(np.float32))
    assert (back_bits[finite] == bits[finite]).all()
    assert np.isnan(back[~finite]).all()


def test_f32_to_f16_matches_numpy_rounding():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200_000).astype(np.float32) * 3,
        (rng.standard_normal(50_000) * 1e-6).astype(np.float32),           # fp16 subnormal range
        rng.uniform(6e4, 7e4, 1000).astype(np.float32),                    # overflow boundary
        (np.arange(1, 2049, dtype=np.float32) + 0.5) / 1024,               # exact ties
        np.array([65504, 65519.99, 65520, -65520, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 0, -0.0], np.float32),
    ])
    bits, _ = O.f16_roundtrip(x)
    with np.errstate(over="ignore"):
        assert (bits == x.astype(np.float16).view(np.uint16)).all()


# ------------------------------------------------------------------ LN, GELU

@pytest.mark.parametrize("d", [128, 256])
def test_layernorm_matches_torch(d):
    rng = np.random.default_rng(d)
    x = (rng.standard_normal((500, d)) * rng.uniform(0.1, 5, (500, 1)) + rng.uniform(-3, 3, (500, 1))).astype(np.float32)
    g = rng.uniform(0.5, 1.5, d).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, d).astype(np.float32)
    got = O.layernorm(x, g, b)
    ref = F.layer_norm(torch.tensor(x, dtype=torch.float64), (d,), torch.tensor(g, dtype=torch.float64),
                       torch.tensor(b, dtype=torch.float64), eps=1e-5).numpy()
    assert np.abs(got - ref).max() < 2e-5


def test_layernorm_closed_forms():
    rng = np.random.default_rng(1)
    d = 256
    x = rng.standard_normal((64, d)).astype(np.float32)
    one, zero = np.ones(d, np.float32), np.zeros(d, np.float32)
    y = O.layernorm(x, one, zero)
    assert np.abs(y.mean(1)).max() < 1e-6
    assert np.abs(y.var(1) - 1 / (1 + 1e-5 / x.var(1))).max() < 1e-5
    # invariant to a positive affine map of the row
    y2 = O.layernorm((3 * x + 7).astype(np.float32), one, zero)
    assert np.abs(y2 - y).max() < 1e-4
    # LN(0) = beta
    beta = rng.standard_normal(d).astype(np.float32)
    assert (O.layernorm(np.zeros((2, d), np.float32), one, beta) == beta).all()
    # rounding flag rounds to fp16
    r = O.layernorm(x, one, zero, round16=True)
    assert (r == r.astype(np.float16).astype(np.float32)).all()


def test_gelu_matches_torch_and_limits():
    x = np.linspace(-12, 12, 100_001).astype(np.float32)
    got = O.gelu(x)
    ref = F.gelu(torch.tensor(x, dtype=torch.float64), approximate="tanh").numpy()
    assert np.abs(got - ref).max() < 1e-5
    assert O.gelu(np.array([0.0], np.float32))[0] == 0
    big = O.gelu(np.array([30.0, -30.0], np.float32))
    assert big[0] == 30.0 and abs(big[1]) < 1e-20


# ------------------------------------------------------------------ attention core

def core_cfg(hd):
    return O.cfg(8 * hd, 8, hd, 1, 8, 8, 1, faithful=False)


@pytest.mark.parametrize("hd", [16, 32])
def test_core_matches_torch_sdpa(hd):
    rng = np.random.default_rng(hd)
    d = 8 * hd
    q, k, v = (rng.standard_normal((64, d)).astype(np.float32) for _ in range(3))
    got = O.window_attention(core_cfg(hd), q, k, v)
    scale = 0.1767766953 if hd == 32 else 0.25
    t = lambda a: torch.tensor(a, dtype=torch.float64).view(64, 8, hd).transpose(0, 1)
    ref = F.scaled_dot_product_attention(t(q), t(k), t(v), scale=scale).transpose(0, 1).reshape(64, d).numpy()
    assert np.abs(got - ref).max() < 1e-5


def test_core_identical_keys_give_mean_of_values():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((64, 256)).astype(np.float32)
    k = np.tile(rng.standard_normal((1, 256)).astype(np.float32), (64, 1))
    v = rng.standard_normal((64, 256)).astype(np.float32)
    got = O.window_attention(core_cfg(32), q, k, v)
    assert np.abs(got - v.mean(0, keepdims=True)).max() < 1e-5


def test_core_dominant_key_selects_its_value():
    rng = np.random.default_rng(3)
    q = np.ones((64, 256), np.float32)
    k = rng.standard_normal((64, 256)).astype(np.float32) * 0.01
    k[37] = 10.0  # score 32*10*0.177 = 56 above the rest in every head
    v = rng.standard_normal((64, 256)).astype(np.float32)
    got = O.window_attention(core_cfg(32), q, k, v)
    assert np.abs(got - v[37]).max() < 1e-6


def test_core_is_slot_permutation_equivariant():
    rng = np.random.default_rng(4)
    q, k, v = (rng.standard_normal((64, 128)).astype(np.float32) for _ in range(3))
    perm = rng.permutation(64)
    a = O.window_attention(core_cfg(16), q, k, v)
    b = O.window_attention(core_cfg(16), q[perm], k[perm], v[perm])
    assert np.abs(b - a[perm]).max() < 1e-6


# ------------------------------------------------------------------ stages

def small_model(name, n_blocks=1, H=12, W=20, seed=0, routing=None):
    cfg = P.CONFIGS[name]
    desc = cfg.desc(n_blocks=n_blocks, H=H, W=W)
    blob, offs = P.synth_weights(desc, seed=seed, routing=cfg.routing if routing is None else routing)
    return cfg, blob, offs, O.f16bits_to_f32(blob)


def feats(cfg, H, W, batch, seed=1):
    return O.f16bits_to_f32(P.synth_features(cfg, batch=batch, H=H, W=W, seed=seed)).reshape(-1, cfg.dim)


def torch_block(cfg, w, o, x, H, W, batch, assign=None):
    """Independent fp64 restatement of one block with library ops."""
    d, nh, hd, N = cfg.dim, cfg.n_heads, cfg.head_dim, cfg.n_experts
    wt = torch.tensor(w, dtype=torch.float64)
    seg = lambda off, n: wt[off:off + n]
    xt = torch.tensor(x, dtype=torch.float64).view(batch, H, W, d)
    xn = F.layer_norm(xt, (d,), seg(o.ln1_g, d), seg(o.ln1_b, d), eps=1e-5)
    Hp, Wp = -(-H // 8) * 8, -(-W // 8) * 8
    pad = torch.zeros(batch, Hp, Wp, d, dtype=torch.float64)
    pad[:, :H, :W] = xn                                       # padded slots feed zeros into QKV
    win = pad.view(batch, Hp // 8, 8, Wp // 8, 8, d).permute(0, 1, 3, 2, 4, 5).reshape(-1, 64, d)
    qkv = F.linear(win, seg(o.qkv_w, 3 * d * d).view(3 * d, d), seg(o.qkv_b, 3 * d))
    q, k, v = (t.reshape(-1, 64, nh, hd).transpose(1, 2) for t in qkv.split(d, dim=-1))
    scale = 0.1767766953 if hd == 32 else 1 / hd ** 0.5
    a = F.scaled_dot_product_attention(q, k, v, scale=scale).transpose(1, 2).reshape(-1, 64, d)
    po = F.linear(a, seg(o.out_w, d * d).view(d, d), seg(o.out_b, d))
    po = po.view(batch, Hp // 8, Wp // 8, 8, 8, d).permute(0, 1, 3, 2, 4, 5).reshape(batch, Hp, Wp, d)[:, :H, :W]
    h = (xt + po).reshape(-1, d)
    hn = F.layer_norm(h, (d,), seg(o.ln2_g, d), seg(o.ln2_b, d), eps=1e-5)
    if N > 1:
        logits = F.linear(hn, seg(o.router_w, N * d).view(N, d), seg(o.router_b, N))
        route = torch.argmax(logits, dim=1) if assign is None else torch.tensor(assign)
    else:
        logits, route = None, torch.zeros(h.shape[0], dtype=torch.long)
    y = h.clone()
    for e in range(N):
        m = route == e
        if not m.any():
            continue
        eo = e * o.exp_stride
        u = F.linear(hn[m], seg(o.exp_w1 + eo, d * d).view(d, d), seg(o.exp_b1 + eo, d))
        g = F.gelu(u, approximate="tanh")
        y[m] = h[m] + F.linear(g, seg(o.exp_w2 + eo, d * d).view(d, d), seg(o.exp_b2 + eo, d))
    return h.numpy(), y.numpy(), None if logits is None else logits.numpy()


@pytest.mark.parametrize("name,H,W,batch", [("moe16", 12, 20, 2), ("dense128", 9, 17, 1), ("moe64", 8, 8, 1),
                                             ("std256", 16, 24, 1)])
def test_block_matches_torch_fp64(name, H, W, batch):
    cfg, blob, offs, w = small_model(name, H=H, W=W)
    x = feats(cfg, H, W, batch)
    c = O.cfg(cfg.dim, cfg.n_heads, cfg.head_dim, cfg.n_experts, H, W, batch, faithful=False)
    h = O.attn_stage(c, w, offs[0], x)
    h_ref, _, logits_ref = torch_block(cfg, w, offs[0], x, H, W, batch)
    assert np.abs(h - h_ref).max() < 2e-4
    if cfg.n_experts > 1:
        assign, logits = O.router_stage(c, w, offs[0], h)
        assert np.abs(logits - logits_ref).max() < 2e-4
        top2 = np.sort(logits_ref, 1)[:, -2:]
        sure = top2[:, 1] - top2[:, 0] > 1e-3
        assert (assign[sure] == logits_ref.argmax(1)[sure]).all()
    else:
        assign = None
    y = O.expert_stage(c, w, offs[0], h, assign)
    _, y_ref, _ = torch_block(cfg, w, offs[0], x, H, W, batch, assign=assign)
    assert np.abs(y - y_ref).max() < 3e-4


def test_faithful_mode_rounds_to_fp16_and_stays_close():
    cfg, blob, offs, w = small_model("moe16")
    x = feats(cfg, 12, 20, 1)
    cf = O.cfg(256, 8, 32, 16, 12, 20, 1, faithful=True)
    c32 = O.cfg(256, 8, 32, 16, 12, 20, 1, faithful=False)
    hf, h32 = O.attn_stage(cf, w, offs[0], x), O.attn_stage(c32, w, offs[0], x)
    assert (hf == hf.astype(np.float16).astype(np.float32)).all()
    assert np.abs(hf - h32).max() < 1e-2 and np.abs(hf - h32).mean() < 1e-3
    af, _ = O.router_stage(cf, w, offs[0], hf)
    yf = O.expert_stage(cf, w, offs[0], hf, af)
    assert (yf == yf.astype(np.float16).astype(np.float32)).all()


def test_window_locality():
    cfg, blob, offs, w = small_model("moe16", H=20, W=28)
    x = feats(cfg, 20, 28, 1)
    c = O.cfg(256, 8, 32, 16, 20, 28, 1, faithful=True)
    y0 = O.attn_stage(c, w, offs[0], x).reshape(20, 28, 256)
    x2 = x.reshape(20, 28, 256).copy()
    x2[8:16, 16:24] += 0.5                               # window (1, 2)
    y1 = O.attn_stage(c, w, offs[0], x2.reshape(-1, 256)).reshape(20, 28, 256)
    changed = np.abs(y1 - y0).max(axis=2) > 0
    inside = np.zeros((20, 28), bool)
    inside[8:16, 16:24] = True
    assert changed[inside].all() and not changed[~inside].any()


def test_padded_slots_behave_as_zero_inputs():
    """A 12x20 grid (padded to 16x24 inside the stage) equals a 16x24 grid whose
    extra rows/columns are zero (LN(0) = beta = 0), at the 12x20 positions."""
    cfg, blob, offs, w = small_model("moe16", H=12, W=20)
    x = feats(cfg, 12, 20, 1)
    c = O.cfg(256, 8, 32, 16, 12, 20, 1, faithful=True)
    y = O.attn_stage(c, w, offs[0], x).reshape(12, 20, 256)
    xp = np.zeros((16, 24, 256), np.float32)
    xp[:12, :20] = x.reshape(12, 20, 256)
    cp = O.cfg(256, 8, 32, 16, 16, 24, 1, faithful=True)
    yp = O.attn_stage(cp, w, offs[0], xp.reshape(-1, 256)).reshape(16, 24, 256)
    assert (yp[:12, :20] == y).all()


def test_zero_weights_are_the_identity():
    cfg = P.CONFIGS["moe16"]
    desc = cfg.desc(n_blocks=2, H=12, W=20)
    offs, total = P.layout(desc)
    w = np.zeros(total, np.float32)
    for o in offs:
        w[o.ln1_g:o.ln1_g + 256] = 1
        w[o.ln2_g:o.ln2_g + 256] = 1
    x = feats(cfg, 12, 20, 1)
    c = O.cfg(256, 8, 32, 16, 12, 20, 1, faithful=True)
    y, assign, _ = O.forward(c, w, list(offs), x)
    assert (y == x).all() and (assign == 0).all()   # all-zero logits: the first expert wins


def test_router_first_max_wins_ties():
    cfg, blob, offs, w = small_model("moe16", routing=P.ROUTE_UNIFORM)
    o = offs[0]
    w = w.copy()
    wr = w[o.router_w:o.router_w + 16 * 256].reshape(16, 256)
    wr[9] = wr[4]                                     # experts 4 and 9 always tie
    wr[4] *= 0
    wr[4] += 0.05 * np.sign(wr[9] + 1e-9)             # make 4/9 strong ...
    wr[9] = wr[4]                                     # ... and identical
    w[o.router_w:o.router_w + 16 * 256] = wr.reshape(-1)
    x = feats(cfg, 12, 20, 1)
    c = O.cfg(256, 8, 32, 16, 12, 20, 1, faithful=True)
    assign, logits = O.router_stage(c, w, o, x)
    assert (assign == np.argmax(logits, axis=1)).all()          # numpy argmax = first max
    assert (logits[:, 4] == logits[:, 9]).all()
    assert (assign != 9).all() and (assign == 4).any()


def test_single_expert_moe_equals_dense():
    cfg, blob, offs, w = small_model("std256", H=12, W=20)
    x = feats(cfg, 12, 20, 1)
    c = O.cfg(256, 8, 32, 1, 12, 20, 1, faithful=True)
    h = O.attn_stage(c, w, offs[0], x)
    dense = O.expert_stage(c, w, offs[0], h, None)
    routed = O.expert_stage(c, w, offs[0], h, np.zeros(h.shape[0], np.int32))
    assert (dense == routed).all()


def test_expert_relabelling_invariance():
    """Swapping two experts' weights and their token labels changes nothing."""
    cfg, blob, offs, w = small_model("moe16", H=12, W=20)
    o = offs[0]
    x = feats(cfg, 12, 20, 1)
    c = O.cfg(256, 8, 32, 16, 12, 20, 1, faithful=True)
    h = O.attn_stage(c, w, o, x)
    assign = np.random.default_rng(5).integers(0, 16, h.shape[0]).astype(np.int32)
    y = O.expert_stage(c, w, o, h, assign)
    w2 = w.copy()
    s = o.exp_stride
    a, b = o.exp_w1 + 3 * s, o.exp_w1 + 11 * s
    w2[a:a + s], w2[b:b + s] = w[b:b + s], w[a:a + s]
    assign2 = assign.copy()
    assign2[assign == 3], assign2[assign == 11] = 11, 3
    assert (O.expert_stage(c, w2, o, h, assign2) == y).all()


def test_forward_equals_chained_stages():
    cfg, blob, offs, w = small_model("moe16", n_blocks=3, H=12, W=20)
    x = feats(cfg, 12, 20, 2)
    c = O.cfg(256, 8, 32, 16, 12, 20, 2, faithful=True)
    y, assign, hh = O.forward(c, w, list(offs), x, keep_h=True)
    cur = x
    for b in range(3):
        h = O.attn_stage(c, w, offs[b], cur)
        assert (h == hh[b]).all()
        a, _ = O.router_stage(c, w, offs[b], h)
        assert (a == assign[b]).all()
        cur = O.expert_stage(c, w, offs[b], h, a)
    assert (cur == y).all()


def test_stage_rejects_bad_config():
    cfg, blob, offs, w = small_model("moe16")
    bad = O.cfg(256, 8, 16, 16, 12, 20, 1)      # 8 x 16 != 256
    with pytest.raises(ValueError):
        O.attn_stage(bad, w, offs[0], feats(cfg, 12, 20, 1))
    with pytest.raises(ValueError):
        O.expert_stage(O.cfg(256, 8, 32, 16, 12, 20, 1), w, offs[0], feats(cfg, 12, 20, 1),
                       np.full(240, 16, np.int32))   # expert id out of range


# ------------------------------------------------------------------ projection adapters

def _f16(x):
    return x.astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("in_dim,out_dim,relu", [(128, 256, True), (256, 128, False), (128, 128, True)])
def test_project_matches_torch_linear(in_dim, out_dim, relu):
    """fp32 mode against torch's linear (+ relu) in fp64; faithful mode is the
    fp32 value rounded to fp16 once (coopVecMatMulAddNV's fp16 result)."""
    rng = np.random.default_rng(in_dim + out_dim)
    x = _f16(rng.standard_normal((300, in_dim)))
    W = _f16(rng.standard_normal((out_dim, in_dim)) * 0.05)
    b = _f16(rng.standard_normal(out_dim) * 0.05)
    ref = F.linear(torch.tensor(x, dtype=torch.float64), torch.tensor(W, dtype=torch.float64),
                   torch.tensor(b, dtype=torch.float64))
    if relu:
        ref = F.relu(ref)
    ref = ref.numpy()
    got32 = O.project(W, b, x, relu, faithful=False)
    assert np.abs(got32 - ref).max() < 1e-5
    got16 = O.project(W, b, x, relu, faithful=True)
    assert (got16 == _f16(got32)).all()
    if relu:
        assert (got16 >= 0).all() and (got16 == 0).mean() > 0.3


def test_project_closed_forms():
    """[I; -I] with ReLU gives [relu(x); relu(-x)]; [I, I] gives the fp16 of
    x[:128] + x[128:] (exact sums of fp16 values, rounded once); zero weights
    give the bias."""
    rng = np.random.default_rng(7)
    x = _f16(rng.standard_normal((64, 128)))
    up = np.vstack([np.eye(128), -np.eye(128)]).astype(np.float32)
    y = O.project(up, np.zeros(256, np.float32), x, True)
    assert (y == np.hstack([np.maximum(x, 0), np.maximum(-x, 0)])).all()
    x2 = _f16(rng.standard_normal((64, 256)))
    dn = np.hstack([np.eye(128), np.eye(128)]).astype(np.float32)
    y2 = O.project(dn, np.zeros(128, np.float32), x2, False)
    exact = x2[:, :128].astype(np.float64) + x2[:, 128:]
    assert (y2 == exact.astype(np.float16).astype(np.float32)).all()
    bias = _f16(rng.standard_normal(256))
    y3 = O.project(np.zeros((256, 128), np.float32), bias, x, True)
    assert (y3 == np.maximum(bias, 0)[None, :]).all()
