"""Pins the oracle's faithful mode: every fp16 rounding point of the parity
contract, one by one.

oracle.c's faithful mode rounds to fp16 at eleven points (xn, q/k/v, the
attention output a, po, h = po + x, hn, the logits, u, GELU(u), yy, y = yy + h;
split2_qkv_attn_d256.comp.glsl:39-78, moe_router.comp.glsl:33-45,
moe_expert_skip.comp.glsl:36-52). This file restates the attention, router and
expert stages in torch float64 from library calls (layer_norm, linear, softmax,
gelu) with `.half()` at each of those points, and holds the oracle to it:

* agreement: with every point in place, the only differences are rounding
  flips from the oracle's fp32 sums against float64 ones, so few elements
  differ (measured 0.03-0.31 %) and each by at most one fp16 ulp at the
  element's magnitude (floored at 1/8, the operands' scale: a flip in po or
  yy of one ulp at |x| ~ 1 is many ulps of a result that cancels to ~0);
* mutation: dropping any single rounding from the restatement breaks that
  agreement (measured 0.63-100 % of elements then differ), so the oracle
  cannot have lost, moved or added one at any point without failing here.

The thresholds sit at about half the smallest mutated rate and twice the
largest agreeing rate of each case.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
import prism_amd as P

torch.set_grad_enabled(False)

ATTN_POINTS = ("xn", "qkv", "a", "po", "h")
ROUTER_POINTS = ("hn", "logits")
EXPERT_POINTS = ("hn", "u", "g", "yy", "y")

# (name, H, W, batch, experts, dim, largest fraction of differing elements that
# still agrees)
CASES = [("moe8_12x20", 12, 20, 2, 8, 256, 0.006), ("dense128_9x17", 9, 17, 1, 1, 128, 0.0025)]


def r16(t):
    return t.half().double()


def _seg(w):
    wt = torch.tensor(w, dtype=torch.float64)
    return lambda off, n: wt[off:off + n]


def restate_attn(d, nh, hd, w, o, x, H, W, B, drop=()):
    """h of the attention stage, fp64 with r16 at ATTN_POINTS (except drop)."""
    R = lambda name, t: t if name in drop else r16(t)
    seg = _seg(w)
    xt = torch.tensor(x, dtype=torch.float64).view(B, H, W, d)
    xn = R("xn", F.layer_norm(xt, (d,), seg(o.ln1_g, d), seg(o.ln1_b, d), eps=1e-5))
    Hp, Wp = -(-H // 8) * 8, -(-W // 8) * 8
    pad = torch.zeros(B, Hp, Wp, d, dtype=torch.float64)
    pad[:, :H, :W] = xn                                # padded slots: zero vector into QKV
    win = pad.view(B, Hp // 8, 8, Wp // 8, 8, d).permute(0, 1, 3, 2, 4, 5).reshape(-1, 64, d)
    qkv = R("qkv", F.linear(win, seg(o.qkv_w, 3 * d * d).view(3 * d, d), seg(o.qkv_b, 3 * d)))
    q, k, v = (t.reshape(-1, 64, nh, hd).transpose(1, 2) for t in qkv.split(d, dim=-1))
    scale = float(np.float32(0.1767766953)) if hd == 32 else float(np.float32(1.0 / np.sqrt(hd)))
    s = (q @ k.transpose(-1, -2)) * scale
    a = R("a", torch.softmax(s, dim=-1) @ v).transpose(1, 2).reshape(-1, 64, d)
    po = R("po", F.linear(a, seg(o.out_w, d * d).view(d, d), seg(o.out_b, d)))
    po = po.view(B, Hp // 8, Wp // 8, 8, 8, d).permute(0, 1, 3, 2, 4, 5).reshape(B, Hp, Wp, d)[:, :H, :W]
    return R("h", xt + po).reshape(-1, d).numpy()


def restate_router(d, N, w, o, h, drop=()):
    """Logits of the router stage, r16 at ROUTER_POINTS (except drop)."""
    R = lambda name, t: t if name in drop else r16(t)
    seg = _seg(w)
    hn = R("hn", F.layer_norm(torch.tensor(h, dtype=torch.float64), (d,), seg(o.ln2_g, d), seg(o.ln2_b, d),
                              eps=1e-5))
    return R("logits", F.linear(hn, seg(o.router_w, N * d).view(N, d), seg(o.router_b, N))).numpy()


def restate_expert(d, N, w, o, h, assign, drop=()):
    """y of the expert stage, r16 at EXPERT_POINTS (except drop)."""
    R = lambda name, t: t if name in drop else r16(t)
    seg = _seg(w)
    ht = torch.tensor(h, dtype=torch.float64)
    hn = R("hn", F.layer_norm(ht, (d,), seg(o.ln2_g, d), seg(o.ln2_b, d), eps=1e-5))
    route = torch.zeros(ht.shape[0], dtype=torch.long) if assign is None else torch.tensor(assign).long()
    y = torch.full_like(ht, float("nan"))
    for e in range(N):
        m = route == e
        if not m.any():
            continue
        eo = e * o.exp_stride
        u = R("u", F.linear(hn[m], seg(o.exp_w1 + eo, d * d).view(d, d), seg(o.exp_b1 + eo, d)))
        g = R("g", F.gelu(u, approximate="tanh"))
        yy = R("yy", F.linear(g, seg(o.exp_w2 + eo, d * d).view(d, d), seg(o.exp_b2 + eo, d)))
        y[m] = R("y", ht[m] + yy)
    return y.numpy()


def disagreement(got, ref):
    """(fraction of elements that differ, elements off by more than one fp16
    ulp at max(|got|, |ref|, 1/8))."""
    a, b = got.astype(np.float64), ref.astype(np.float64)
    mag = np.maximum(np.maximum(np.abs(a), np.abs(b)), 0.125)
    ulp = 2.0 ** (np.floor(np.log2(mag)) - 10)
    diff = np.abs(a - b)
    return float((a != b).mean()), int((diff > ulp).sum())


_cache = {}


def oracle_case(name, H, W, B, N, dim):
    """Weights, input and the oracle's faithful stage outputs of one case."""
    if name not in _cache:
        hd = dim // 8
        desc = P.ModelDesc(dim, 1, 8, hd, N, H, W, 8)
        blob, offs = P.synth_weights(desc, seed=0, routing=P.ROUTE_ZIPF if N > 1 else P.ROUTE_RANDOM)
        o, w = offs[0], O.f16bits_to_f32(blob)
        x = O.f16bits_to_f32(P.synth_normal(B * H * W * dim, seed=1)).reshape(-1, dim)
        c = O.cfg(dim, 8, hd, N, H, W, B, faithful=True)
        h = O.attn_stage(c, w, o, x)
        assign, logits = O.router_stage(c, w, o, h) if N > 1 else (None, None)
        y = O.expert_stage(c, w, o, h, assign)
        _cache[name] = (w, o, x, h, assign, logits, y)
    return _cache[name]


def stage_results(case, drop=()):
    """[(stage, disagreement)] of the restatement (without `drop`) against the
    oracle, each stage fed the oracle's own inputs."""
    name, H, W, B, N, dim, _ = case
    w, o, x, h, assign, logits, y = oracle_case(name, H, W, B, N, dim)
    out = []
    if not drop or drop[0] in ATTN_POINTS:
        out.append(("attention", disagreement(h, restate_attn(dim, 8, dim // 8, w, o, x, H, W, B, drop))))
    if N > 1 and (not drop or drop[0] in ROUTER_POINTS):
        out.append(("router", disagreement(logits, restate_router(dim, N, w, o, h, drop))))
    if not drop or drop[0] in EXPERT_POINTS:
        out.append(("expert", disagreement(y, restate_expert(dim, N, w, o, h, assign, drop))))
    return out


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_faithful_mode_agrees_with_fp64_restatement(case):
    limit = case[-1]
    for stage, (frac, off_by_more) in stage_results(case):
        assert frac <= limit, (stage, frac)
        assert off_by_more == 0, (stage, off_by_more)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("point", sorted(set(ATTN_POINTS + ROUTER_POINTS + EXPERT_POINTS)))
def test_each_rounding_point_matters(case, point):
    if point == "logits" and case[4] == 1:
        pytest.skip("dense block: no router")
    limit = case[-1]
    results = stage_results(case, drop=(point,))
    assert results
    for stage, (frac, off_by_more) in results:
        # the rounding dropped, the stage no longer agrees
        assert frac > limit or off_by_more > 0, (stage, point, frac, off_by_more)
