"""Host-side tests of the C ABI (no GPU): exports, layout, validation,
fragment packing, the synthetic generator, error codes."""
import ctypes as C
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import prism_amd as P
from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "prism.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(prism_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    syms = declared_symbols()
    assert len(syms) >= 18
    lib = C.CDLL(P.LIB_PATH)
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    # and the binding knows every one of them
    assert set(syms) <= set(P.SIGNATURES), set(syms) - set(P.SIGNATURES)


def test_code_object_is_built_for_gfx950():
    path = P.CODE_OBJECT_PATH
    assert os.path.exists(path)
    out = subprocess.run(["/opt/rocm/llvm/bin/clang-offload-bundler", "--list", "--type=o", f"--input={path}"],
                         capture_output=True, text=True)
    assert "gfx950" in out.stdout


@pytest.mark.parametrize("name", list(P.CONFIGS))
def test_layout_is_the_bump_allocator_with_ln(name):
    cfg = P.CONFIGS[name]
    desc = cfg.desc()
    offs, total = P.layout(desc)
    d, N = cfg.dim, cfg.n_experts
    spans = []
    for b in range(cfg.n_blocks):
        o = offs[b]
        # reference order (prism_moe_bench.cpp:164-172): qkv_w, qkv_b, out_w, out_b, rtr_w, rtr_b, experts
        order = [o.ln1_g, o.ln1_b, o.qkv_w, o.qkv_b, o.out_w, o.out_b, o.ln2_g, o.ln2_b]
        sizes = [d, d, 3 * d * d, 3 * d, d * d, d, d, d]
        if N > 1:
            order += [o.router_w, o.router_b]
            sizes += [N * d, N]
        assert order == sorted(order)
        assert o.exp_stride == 2 * d * d + 2 * d
        assert (o.exp_b1 - o.exp_w1, o.exp_w2 - o.exp_w1, o.exp_b2 - o.exp_w1) == (d * d, d * d + d, 2 * d * d + d)
        for off, sz in zip(order, sizes):
            assert off % 8 == 0
            spans.append((off, off + sz))
        spans.append((o.exp_w1, o.exp_w1 + N * o.exp_stride))
    spans.sort()
    for (a0, a1), (b0, b1) in zip(spans, spans[1:]):
        assert a1 <= b0, "tensors overlap"
    assert spans[-1][1] == total
    assert P.validate(desc, offs, total) == P.OK


def test_moe64_parameter_count():
    offs, total = P.layout(P.CONFIGS["moe64"].desc())
    # 16 blocks x (attention 263,168 + LN 1,024 + router 16,448 + 64 experts x 131,584)
    assert total == 16 * (197376 + 65792 + 1024 + 64 * 256 + 64 + 64 * 131584)
    assert 139e6 < total < 140e6


def test_validate_rejects_bad_tables():
    cfg = P.CONFIGS["moe16"]
    desc = cfg.desc(n_blocks=2)
    offs, total = P.layout(desc)
    assert P.validate(desc, offs, total) == P.OK
    assert P.validate(desc, offs, total - 1) == P.ERR_BLOB            # truncated blob
    offs[1].qkv_w += 4
    assert P.validate(desc, offs, total) == P.ERR_BLOB                # misaligned
    offs[1].qkv_w -= 4
    offs[0].exp_w1 = total                                             # out of range
    assert P.validate(desc, offs, total) == P.ERR_BLOB
    offs, total = P.layout(desc)
    offs[0].exp_stride = 7
    assert P.validate(desc, offs, total) == P.ERR_BLOB
    assert P.validate(desc, None, total) == P.ERR_INVALID


@pytest.mark.parametrize("field,value", [("dim", 192), ("n_heads", 4), ("head_dim", 64), ("window", 16),
                                         ("n_experts", 0), ("n_experts", 65), ("n_blocks", 0),
                                         ("spatial_h", 0)])
def test_unsupported_shapes_are_rejected(field, value):
    desc = P.CONFIGS["moe64"].desc(n_blocks=1)
    setattr(desc, field, value)
    total = C.c_int64()
    rc = P.lib().prism_layout(C.byref(desc), None, C.byref(total))
    assert rc == P.ERR_UNSUPPORTED
    assert P.lib().prism_last_error(None)


def test_pack_weight_fragment_layout():
    rows, k = 40, 64
    w = np.arange(rows * k, dtype=np.uint16).reshape(rows, k)
    packed = P.pack_weight(w, rows_padded=48).reshape(48 // 16, k // 32, 64, 8)
    for rt in range(3):
        for ks in range(2):
            for lane in (0, 5, 16, 31, 47, 63):
                r = 16 * rt + lane % 16
                want = w[r, 32 * ks + 8 * (lane // 16): 32 * ks + 8 * (lane // 16) + 8] if r < rows else np.zeros(8)
                assert (packed[rt, ks, lane] == want).all()
    # every element exactly once, padding rows zero
    vals = packed.reshape(-1)
    assert np.sort(vals[vals > 0]).tolist() == list(range(1, rows * k))
    assert (vals == 0).sum() == 1 + 8 * 64  # element 0 + 8 padding rows x 64 columns


def test_pack_weight_rejects_bad_shapes():
    w = np.zeros((16, 48), np.uint16)
    rc = P.lib().prism_pack_weight(w.ctypes.data, 16, 48, 16, w.ctypes.data)
    assert rc == P.ERR_INVALID


# -------------------------------------------------------------- generator

GOLDEN = 0x9E3779B97F4A7C15


def splitmix64(z):
    z = z.astype(np.uint64)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def normals_numpy(n, seed, stream, std):
    """The generator's published definition, restated independently."""
    with np.errstate(over="ignore"):
        key = splitmix64(np.array([seed], np.uint64) ^ splitmix64(np.array([stream + GOLDEN], np.uint64)))
        idx = np.arange(n, dtype=np.uint64)
        bits = splitmix64(key + idx * np.uint64(GOLDEN))
    u1 = ((bits >> np.uint64(40)).astype(np.float64) + 0.5) / 16777216.0
    u2 = ((bits & np.uint64(0xFFFFFF)).astype(np.float64) + 0.5) / 16777216.0
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2 * np.pi * u2)
    # the ABI takes std as a float: widen float32(std) to double as the C++ does
    return (float(np.float32(std)) * z).astype(np.float32).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("seed,stream,std", [(0, 0, 1.0), (7, 3 << 24 | 9, 0.02), (123456789, 42, 2.5)])
def test_generator_matches_its_definition(seed, stream, std):
    n = 200_000
    got = P.synth_normal(n, seed=seed, stream=stream, std=std)
    ref = normals_numpy(n, seed, stream, std)
    mism = np.nonzero(got != ref)[0]
    # float64 libm last-bit differences may move a value across an fp16 midpoint
    assert mism.size <= 2, mism[:10]
    z = got.view(np.float16).astype(np.float64) / std
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01


def test_synth_weights_deterministic_and_shaped():
    cfg = P.CONFIGS["moe16"]
    desc = cfg.desc(n_blocks=2)
    b1, offs = P.synth_weights(desc, seed=3, routing=P.ROUTE_RANDOM)
    b2, _ = P.synth_weights(desc, seed=3, routing=P.ROUTE_RANDOM)
    b3, _ = P.synth_weights(desc, seed=4, routing=P.ROUTE_RANDOM)
    assert (b1 == b2).all() and not (b1 == b3).all()
    f = b1.view(np.float16).astype(np.float32)
    o = offs[1]
    assert (f[o.ln1_g:o.ln1_g + 256] == 1).all() and (f[o.ln2_b:o.ln2_b + 256] == 0).all()
    w = f[o.qkv_w:o.qkv_w + 3 * 256 * 256]
    assert abs(w.std() - 0.02) < 0.001 and abs(w.mean()) < 0.001
    e5 = f[o.exp_w2 + 5 * o.exp_stride: o.exp_w2 + 5 * o.exp_stride + 256 * 256]
    assert abs(e5.std() - 0.02) < 0.001


def test_routing_bias_modes():
    for routing, check in [(P.ROUTE_UNIFORM, "zero"), (P.ROUTE_ZIPF, "zipf"), (P.ROUTE_ADVERSARIAL, "adv")]:
        cfg = P.CONFIGS["moe64"] if check != "adv" else P.CONFIGS["moe32"]
        desc = cfg.desc(n_blocks=1)
        blob, offs = P.synth_weights(desc, seed=0, routing=routing)
        rb = blob[offs[0].router_b:offs[0].router_b + cfg.n_experts].view(np.float16).astype(np.float32)
        if check == "zero":
            assert (rb == 0).all()
        elif check == "zipf":
            # biases fall with the Zipf rank: hottest expert first
            assert rb[0] == rb.max() and rb[0] > rb[8] > rb[63]
        else:
            assert rb[0] == rb.max() and rb[0] - np.median(rb[1:]) > 0.3


def test_histogram_and_aux_size():
    a = np.array([0, 3, 3, 1, 3], np.int32)
    assert P.histogram(a, 4).tolist() == [1, 1, 0, 3]
    with pytest.raises(P.PrismError):
        P.histogram(np.array([4], np.int32), 4)
    assert P.aux_elems(64, 1000) == 1000 + 64 + 64 * 1000


def test_context_calls_fail_cleanly_without_a_context():
    L = P.lib()
    push = P.AttnPush()
    assert L.prism_attn(None, C.byref(push), None, 1, None) == P.ERR_INVALID
    assert L.prism_forward(None, None, None, 1, None) == P.ERR_INVALID
    assert L.prism_load_weights(None, None, None, 0, None) == P.ERR_INVALID
    assert L.prism_load_adapters(None, None, 0, None) == P.ERR_INVALID
    assert L.prism_project_up(None, C.byref(P.ProjectPush()), None, 1, None) == P.ERR_INVALID
    assert L.prism_project_down(None, C.byref(P.ProjectPush()), None, 1, None) == P.ERR_INVALID
    assert L.prism_forward_adapted(None, None, None, 1, None) == P.ERR_INVALID
    assert L.prism_forward_adapted_graph(None, None, None, 1, None) == P.ERR_INVALID
    ms = C.c_float()
    assert L.prism_infer_gpu(None, None, 0, None, 0, 1, C.byref(ms)) == P.ERR_INVALID
    buf, ptr = C.c_void_p(), C.c_void_p()
    assert L.prism_import_external_memory(None, 0, 1, C.byref(buf), C.byref(ptr)) == P.ERR_INVALID
    assert L.prism_release_external_memory(None, None) == P.ERR_INVALID
    L.prism_destroy(None)  # no-op


def test_init_with_device_without_a_gpu_fails_cleanly():
    """No device in this process (or a device index past the last): an error
    code and a message, no context."""
    L = P.lib()
    h = C.c_void_p(1)
    rc = L.prism_init_with_device(C.byref(h), 4096, None, None)
    assert rc in (P.ERR_HIP, P.ERR_INVALID) and h.value is None
    assert L.prism_last_error(None)


@pytest.mark.parametrize("name", ["moe64", "dense128"])
def test_adapter_layout(name):
    """The adapters follow the reference's wa() order (proj_up_w, proj_up_b,
    proj_dn_w, proj_dn_b), 8-aligned, from an arbitrary base."""
    cfg = P.CONFIGS[name]
    desc = cfg.desc(n_blocks=1)
    _, total = P.layout(desc)
    a, end = P.adapter_layout(desc, total + 3)
    D, I = cfg.dim, 128
    assert a.in_dim == I and a.up_w == (total + 3 + 7) // 8 * 8
    assert a.up_b == a.up_w + D * I and a.down_w == a.up_b + (D + 7) // 8 * 8
    assert a.down_b == a.down_w + I * D and end == a.down_b + I
    assert all(v % 8 == 0 for v in (a.up_w, a.up_b, a.down_w, a.down_b))
    with pytest.raises(P.PrismError):
        P.adapter_layout(desc, 0, in_dim=64)
    blob, a2 = P.synth_adapters(desc, seed=1)
    blob2, _ = P.synth_adapters(desc, seed=1)
    assert a2.up_w == 0 and (blob == blob2).all() and blob.size == end - a.up_w  # same span from base 0
    w = blob[a2.up_w:a2.up_w + D * I].view(np.float16).astype(np.float32)
    assert abs(w.std() - 0.02) < 0.002


def test_create_reports_missing_code_object():
    h = C.c_void_p()
    rc = P.lib().prism_create(C.byref(h), 0, b"/nonexistent/prism_kernels.hsaco")
    assert rc != P.OK and not h.value
    assert P.lib().prism_last_error(None)


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_codec_layout_follows_the_reference_order():
    """enc_ic, enc1, enc2, enc3, proj_up, proj_dn, d3, d2, d1, out
    (prism_moe_bench.cpp:347-357), 8-aligned, after the blocks."""
    desc = P.CONFIGS["moe64"].desc()
    _, total = P.layout(desc)
    c, a, end = P.codec_layout(desc, 960, 540, base=total)
    D = desc.dim
    order = [(c.enc0_w, 32 * 81), (c.enc0_b, 32), (c.enc1_w, 64 * 288), (c.enc1_b, 64), (c.enc2_w, 128 * 576),
             (c.enc2_b, 128), (c.enc3_w, 128 * 1152), (c.enc3_b, 128), (a.up_w, D * 128), (a.up_b, D),
             (a.down_w, 128 * D), (a.down_b, 128), (c.dec3_w, 128 * 256), (c.dec3_b, 128), (c.dec2_w, 64 * 192),
             (c.dec2_b, 64), (c.dec1_w, 32 * 96), (c.dec1_b, 32), (c.out_w, 12 * 32), (c.out_b, 12)]
    assert order[0][0] == (total + 7) // 8 * 8
    for (o, n), (o2, _) in zip(order, order[1:]):
        assert o % 8 == 0 and o2 == o + (n + 7) // 8 * 8
    assert end == order[-1][0] + 16  # every tensor takes a whole number of 8-element steps
    assert (c.render_w, c.render_h, c.in_channels, c.scale) == (960, 540, 9, 2)
    assert P.codec_resolutions(960, 540) == [(960, 540), (480, 270), (240, 135), (120, 68)]
    # a render size that does not encode to the 120x68 token grid
    with pytest.raises(P.PrismError) as ei:
        P.codec_layout(desc, 960, 530)
    assert ei.value.code == P.ERR_INVALID and "encodes to" in P.lib().prism_last_error(None).decode()
    # a render size whose 32-channel fp16 map would pass 2 GiB per frame (the conv stages'
    # 32-bit map offsets), on a model whose grid it encodes to: 8192 x 4200 -> 1024 x 525
    big = P.CONFIGS["moe64"].desc(H=525, W=1024)
    with pytest.raises(P.PrismError) as ei:
        P.codec_layout(big, 8192, 4200)
    assert ei.value.code == P.ERR_INVALID and "2 GiB" in P.lib().prism_last_error(None).decode()
    # 8192 x 4093 (encodes to 1024 x 512) stays under the limit: accepted
    P.codec_layout(P.CONFIGS["moe64"].desc(H=512, W=1024), 8192, 4093)

