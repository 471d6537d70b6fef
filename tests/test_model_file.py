"""The on-disk model pair (<name>.weights flat fp16 + <name>.json sidecar):
export_weights.py writes it, prism_read_model_json / prism_load_model_file
read it. CPU tests cover the round trip and the validation of a damaged
sidecar; the GPU test checks that a model loaded from files computes exactly
what the same model loaded from memory computes."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import prism_amd as P

HERE = os.path.dirname(os.path.abspath(__file__))
EXPORT = os.path.join(HERE, "..", "prism-inference_amd", "export_weights.py")
sys.path.insert(0, os.path.dirname(EXPORT))
import export_weights as X  # noqa: E402

FIELDS = P.OFFSET_FIELDS


def same_offsets(a, b, n, dense=False):
    """Dense blocks have no router: its two fields are unused (and absent from the sidecar)."""
    fields = [f for f in FIELDS if not (dense and f.startswith("router_"))]
    return all(getattr(a[i], f) == getattr(b[i], f) for i in range(n) for f in fields)


@pytest.mark.parametrize("name,adapters", [("moe16", True), ("dense128", False), ("moe64", False)])
def test_sidecar_round_trip(tmp_path, name, adapters):
    desc, blob, offs, a = X.synth_model(name, n_blocks=2, seed=3, adapters=adapters)
    w = str(tmp_path / "m.weights")
    jpath = X.write_model(w, desc, blob, offs, a)
    assert os.path.getsize(w) == blob.size * 2
    d2, o2, a2, total = P.read_model_json(jpath)
    assert total == blob.size
    assert all(getattr(d2, f) == getattr(desc, f) for f, _ in P.ModelDesc._fields_)
    assert same_offsets(offs, o2, desc.n_blocks, dense=desc.n_experts == 1)
    if adapters:
        assert a2 is not None and all(getattr(a2, f) == getattr(a, f) for f, _ in P.AdapterOffsets._fields_)
    else:
        assert a2 is None
    # the sidecar keeps the reference exporter's per-layer keys
    side = json.load(open(jpath))
    assert side["total_bytes"] == 2 * side["total_fp16_values"] == os.path.getsize(w)
    assert all("weight_offset_fp16" in L or L["kind"] == "experts" for L in side["layers"])


def test_npz_export_equals_synth_blob(tmp_path):
    """Named tensors -> blob reproduces the synthetic blob exactly (fp16 values
    pass through float32 unchanged) and the CLI writes the same pair."""
    desc, blob, offs, a = X.synth_model("moe16", n_blocks=2, seed=4, adapters=True)
    f = lambda off, n: blob[off:off + n].view(np.float16)
    D, N, I = desc.dim, desc.n_experts, a.in_dim
    t = {}
    for b in range(desc.n_blocks):
        o, p = offs[b], f"blocks.{b}."
        t[p + "ln1.gamma"], t[p + "ln1.beta"] = f(o.ln1_g, D), f(o.ln1_b, D)
        t[p + "qkv.weight"], t[p + "qkv.bias"] = f(o.qkv_w, 3 * D * D).reshape(3 * D, D), f(o.qkv_b, 3 * D)
        t[p + "out.weight"], t[p + "out.bias"] = f(o.out_w, D * D).reshape(D, D), f(o.out_b, D)
        t[p + "ln2.gamma"], t[p + "ln2.beta"] = f(o.ln2_g, D), f(o.ln2_b, D)
        t[p + "router.weight"], t[p + "router.bias"] = f(o.router_w, N * D).reshape(N, D), f(o.router_b, N)
        for e in range(N):
            eo = e * o.exp_stride
            t[p + f"experts.{e}.w1"] = f(o.exp_w1 + eo, D * D).reshape(D, D)
            t[p + f"experts.{e}.b1"] = f(o.exp_b1 + eo, D)
            t[p + f"experts.{e}.w2"] = f(o.exp_w2 + eo, D * D).reshape(D, D)
            t[p + f"experts.{e}.b2"] = f(o.exp_b2 + eo, D)
    t["proj_up.weight"], t["proj_up.bias"] = f(a.up_w, D * I).reshape(D, I), f(a.up_b, D)
    t["proj_down.weight"], t["proj_down.bias"] = f(a.down_w, I * D).reshape(I, D), f(a.down_b, I)
    d2, blob2, o2, a2 = X.from_tensors({k: v.astype(np.float32) for k, v in t.items()}, desc.spatial_h,
                                       desc.spatial_w)
    assert (blob2 == blob).all() and same_offsets(offs, o2, desc.n_blocks)
    npz = str(tmp_path / "m.npz")
    np.savez(npz, **t)
    out = str(tmp_path / "cli.weights")
    r = subprocess.run([sys.executable, EXPORT, "npz", npz, out, "--H", str(desc.spatial_h), "--W",
                        str(desc.spatial_w)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert (np.fromfile(out, np.uint16) == blob).all()


def _damaged(tmp_path, edit):
    desc, blob, offs, a = X.synth_model("moe16", n_blocks=2, seed=5, adapters=True)
    w = str(tmp_path / "m.weights")
    jpath = X.write_model(w, desc, blob, offs, a)
    side = json.load(open(jpath))
    text = edit(side)
    with open(jpath, "w") as fh:
        fh.write(text if isinstance(text, str) else json.dumps(side))
    return jpath


@pytest.mark.parametrize("what,edit,code", [
    ("truncated", lambda s: json.dumps(s)[:-40], P.ERR_BLOB),
    ("wrong format", lambda s: s.update(format="ncnn") or None, P.ERR_BLOB),
    ("size mismatch", lambda s: s.update(total_bytes=s["total_bytes"] + 2) or None, P.ERR_BLOB),
    ("missing layer", lambda s: s["layers"].pop(2) and None, P.ERR_BLOB),
    ("duplicate layer", lambda s: s["layers"].insert(0, dict(s["layers"][0])) or None, P.ERR_BLOB),
    ("offset past the end", lambda s: s["layers"][1].update(weight_offset_fp16=s["total_fp16_values"]) or None,
     P.ERR_BLOB),
    ("misaligned offset", lambda s: s["layers"][1].update(weight_offset_fp16=s["layers"][1]["weight_offset_fp16"] + 3)
     or None, P.ERR_BLOB),
    ("unknown kind", lambda s: s["layers"][0].update(kind="conv") or None, P.ERR_BLOB),
    ("block out of range", lambda s: s["layers"][0].update(block=9) or None, P.ERR_BLOB),
    ("one adapter only", lambda s: s["layers"].pop() and None, P.ERR_BLOB),
    ("unsupported shape", lambda s: s["model"].update(dim=192) or None, P.ERR_UNSUPPORTED),
])
def test_damaged_sidecar_is_rejected(tmp_path, what, edit, code):
    jpath = _damaged(tmp_path, edit)
    with pytest.raises(P.PrismError) as ei:
        P.read_model_json(jpath)
    assert ei.value.code == code, what
    assert P.lib().prism_last_error(None)


@pytest.mark.gpu
def test_model_file_loads_the_same_model(hip, engine, device_arena, tmp_path):
    desc, blob, offs, a = X.synth_model("moe16", n_blocks=2, seed=6, adapters=True, H=20, W=28)
    w = str(tmp_path / "m.weights")
    X.write_model(w, desc, blob, offs, a)
    n, d, I = 20 * 28, desc.dim, a.in_dim
    x = P.synth_normal(n * d, seed=7)
    xa = P.synth_normal(n * I, seed=8)
    dx, dy, da, db = (device_arena(n * d * 2), device_arena(n * d * 2), device_arena(n * I * 2),
                      device_arena(n * I * 2))
    hip.upload(dx.ptr, x)
    hip.upload(da.ptr, xa)
    outs = []
    for mode in ("memory", "file"):
        if mode == "memory":
            engine.load_weights(desc, blob, offs)
            engine.load_adapters(blob, a)
        else:
            engine.load_model_file(w)
        engine.forward(dx.ptr, dy.ptr, 1)
        engine.forward(da.ptr, db.ptr, 1, adapted=True)
        hip.sync()
        outs.append((hip.download(np.empty(n * d, np.uint16), dy.ptr), hip.download(np.empty(n * I, np.uint16), db.ptr)))
    assert (outs[0][0] == outs[1][0]).all() and (outs[0][1] == outs[1][1]).all()
    # a weights file whose size disagrees with its sidecar is refused
    with open(w, "ab") as fh:
        fh.write(b"\0\0")
    with pytest.raises(P.PrismError) as ei:
        engine.load_model_file(w)
    assert ei.value.code == P.ERR_BLOB
