"""The committed fixture tests/golden/moe8_12x20.npz (written by
tests/golden/make_golden.py): synthetic generator and oracle reproduce it bit
for bit on the CPU; the HIP path reproduces it within the stage tolerances."""
import os

import numpy as np
import pytest

import oracle as O
import prism_amd as P
from conftest import errors

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "moe8_12x20.npz")
H, W, B, N = 12, 20, 2, 8


def load():
    return np.load(GOLDEN, allow_pickle=False)


def test_golden_fixture_reproduced_by_oracle_and_generator():
    import importlib.util

    spec = importlib.util.spec_from_file_location(
        "make_golden", os.path.join(os.path.dirname(GOLDEN), "make_golden.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    got = mk.compute()
    g = load()
    for key in ("blob_sha256", "x_sha256", "h_sha256", "assign_sha256", "y_sha256"):
        assert str(got[key]) == str(g[key]), key
    for key in ("assign", "h_rows", "y_rows", "x_rows", "rows"):
        assert (np.asarray(got[key]) == g[key]).all(), key


@pytest.mark.gpu
def test_golden_fixture_on_gpu(hip, engine, device_arena):
    g = load()
    desc = P.ModelDesc(256, 1, 8, 32, N, H, W, 8)
    blob, offs = P.synth_weights(desc, seed=0, routing=P.ROUTE_ZIPF)
    engine.load_weights(desc, blob, offs)
    n, d = B * H * W, 256
    x = P.synth_normal(n * d, seed=1, stream=0, std=1.0)
    feats = device_arena(3 * n * d * 2)
    aux_n = P.aux_elems(N, n)
    aux = device_arena(aux_n * 4)
    hip.upload(feats.ptr, x)
    print("[golden] attention, router, experts", flush=True)
    assert engine.attn(engine.attn_push(0, 0, n * d), feats.ptr, B) == 0, engine.error()
    assert engine.router(engine.router_push(0, H * W, n * d, 0, n, n + N), feats.ptr, aux.ptr, B) == 0
    assert engine.experts(engine.expert_push(0, H * W, n * d, 2 * n * d, 0, n, n + N), feats.ptr, aux.ptr,
                          B) == 0
    hip.sync()
    h = hip.download(np.empty(n * d, np.uint16), feats.ptr + n * d * 2).reshape(n, d)
    y = hip.download(np.empty(n * d, np.uint16), feats.ptr + 2 * n * d * 2).reshape(n, d)
    assign = hip.download(np.empty(n, np.int32), aux.ptr)
    rows = g["rows"]
    mx, mean = errors(O.f16bits_to_f32(h[rows]), O.f16bits_to_f32(g["h_rows"]))
    assert mx <= 2e-2 and mean <= 2e-3
    agree = (assign == g["assign"]).mean()
    assert agree >= 0.99, agree
    same = assign[rows] == g["assign"][rows]
    mx, mean = errors(O.f16bits_to_f32(y[rows][same]), O.f16bits_to_f32(g["y_rows"][same]))
    assert mx <= 2e-2 and mean <= 2e-3
