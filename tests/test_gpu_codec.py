"""GPU encoder / decoder through the C ABI against the oracle (conv3x3,
dec_stage, pw_conv, pixelshuffle_sigmoid on CHW maps).

- Every stage, teacher-forced: the GPU stage runs on the oracle's (or a
  synthetic) input map and must meet the block tolerances (max 2e-2, mean
  2e-3) on its output. Maps between stages are NHWC on the GPU, CHW in the
  oracle; the tests transpose.
- prism_encode -> prism_decode against the oracle's free-running chain.
- The end-to-end frame (prism_forward_e2e, eager and graph, and
  prism_infer_gpu with the codec loaded) is bit-identical to the same calls
  made one by one: encode, the adapted chain, decode.
"""
import numpy as np
import pytest

import oracle as O
import prism_amd as P
from conftest import errors
from test_gpu_ln_affine import with_affine

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def chw(nhwc, h, w):
    return nhwc.reshape(h, w, -1).transpose(2, 0, 1)


def nhwc(x):
    return np.ascontiguousarray(x.transpose(1, 2, 0))


def f16(a):
    return a.astype(np.float16).astype(np.float32)


def setup(engine, render, name="moe16", nb=1, seed=4, affine=False):
    """A model whose token grid is the render size encoded three times, and its
    codec; affine: random LN gammas and betas in every block."""
    cfg = P.CONFIGS[name]
    r = P.codec_resolutions(*render)
    desc = cfg.desc(n_blocks=nb, H=r[3][1], W=r[3][0])
    blob, offs = P.synth_weights(desc, seed=seed, routing=cfg.routing)
    if affine:
        blob = with_affine(blob, offs, cfg.dim, seed=seed + 7)
    engine.load_weights(desc, blob, offs)
    cblob, c, a = P.synth_codec(desc, seed=seed + 1, render_w=render[0], render_h=render[1])
    engine.load_codec(cblob, c)
    engine.load_adapters(cblob, a)
    w = O.f16bits_to_f32(cblob)

    def W(name):
        rows, cols = P.CODEC_SHAPES[name]
        o = getattr(c, name + "_w")
        return w[o:o + rows * cols].reshape(rows, cols), w[getattr(c, name + "_b"):getattr(c, name + "_b") + rows]

    return desc, r, W, (blob, offs), (cblob, c, a)


def run_stage(hip, engine, device_arena, stage, inp, skip, out_elems, batch=1):
    dx = device_arena(inp.size * 2)
    hip.upload(dx.ptr, O.f32_to_f16bits(inp.reshape(-1)))
    ds = None
    if skip is not None:
        ds = device_arena(skip.size * 2)
        hip.upload(ds.ptr, O.f32_to_f16bits(skip.reshape(-1)))
    dy = device_arena(out_elems * 2)
    engine.codec_stage(stage, dx.ptr, ds.ptr if ds else None, dy.ptr, batch)
    hip.sync()
    return O.f16bits_to_f32(hip.download(np.empty(out_elems, np.uint16), dy.ptr))


@pytest.mark.gpu
@pytest.mark.parametrize("render", [(70, 38), (960, 540)])
def test_codec_stages_teacher_forced(hip, engine, device_arena, render):
    desc, r, W, _, _ = setup(engine, render)
    rng = np.random.default_rng(3)
    (w0, h0), (w1, h1), (w2, h2), (w3, h3) = r
    frame = f16(rng.standard_normal((9, h0, w0)))
    print(f"[codec] render {render}: maps {r}", flush=True)
    ref = {}
    # encoder: each stage on the oracle's previous map
    ref["e0"] = O.conv3x3(frame, *W("enc0"), stride=1)
    got = run_stage(hip, engine, device_arena, 0, frame, None, h0 * w0 * 32)
    checks = [("enc0", chw(got, h0, w0), ref["e0"])]
    for st, (name, src, cin, (wo, ho), cout) in enumerate([("enc1", "e0", 32, (w1, h1), 64),
                                                            ("enc2", "e1", 64, (w2, h2), 128),
                                                            ("enc3", "e2", 128, (w3, h3), 128)], start=1):
        x = ref[src]
        ref["e" + str(st)] = O.conv3x3(x, *W(name), stride=2)
        got = run_stage(hip, engine, device_arena, st, nhwc(x), None, ho * wo * cout)
        checks.append((name, chw(got, ho, wo), ref["e" + str(st)]))
        if name in ("enc2", "enc3"):
            # the reference's split convs round each 288-column partial sum
            # (strided_conv_split_{64,128}ch.comp.glsl); this build rounds the
            # whole sum once: both within the block tolerance of each other
            split = O.conv3x3_split(x, *W(name), groups=cin // 32, mode=0 if cin == 64 else 1)
            checks.append((name + " vs split rounding", chw(got, ho, wo), split))
    # decoder: coarse input = a synthetic ReLU-like map, skips = the encoder maps
    up3 = np.maximum(f16(rng.standard_normal((128, h3, w3))), 0)
    d3 = O.dec_stage(up3, ref["e2"], *W("dec3"))
    got = run_stage(hip, engine, device_arena, 4, nhwc(up3), nhwc(ref["e2"]), h2 * w2 * 128)
    checks.append(("dec3", chw(got, h2, w2), d3))
    d2 = O.dec_stage(d3, ref["e1"], *W("dec2"))
    got = run_stage(hip, engine, device_arena, 5, nhwc(d3), nhwc(ref["e1"]), h1 * w1 * 64)
    checks.append(("dec2", chw(got, h1, w1), d2))
    d1 = O.dec_stage(d2, ref["e0"], *W("dec1"))
    o12 = O.pw_conv(d1, *W("out"))
    disp = O.pixelshuffle_sigmoid(o12, 2)
    got = run_stage(hip, engine, device_arena, 6, nhwc(d2), nhwc(ref["e0"]), 3 * 4 * h0 * w0)
    checks.append(("dec1+out+shuffle", got.reshape(3, 2 * h0, 2 * w0), disp))
    for name, g, rf in checks:
        mx, mean = errors(g, rf)
        print(f"[codec] {name}: max {mx:.3g} mean {mean:.3g} (|ref| max {np.abs(rf).max():.3g})", flush=True)
        assert mx <= MAX_ABS and mean <= MEAN_ABS, name
        assert np.abs(rf).max() > 0.1, f"{name}: degenerate reference"


@pytest.mark.gpu
def test_encode_decode_against_the_oracle_chain(hip, engine, device_arena):
    render, batch = (94, 60), 2
    desc, r, W, _, _ = setup(engine, render)
    (w0, h0), _, _, (w3, h3) = r
    rng = np.random.default_rng(5)
    frames = f16(rng.standard_normal((batch, 9, h0, w0)))
    df = device_arena(frames.size * 2)
    hip.upload(df.ptr, O.f32_to_f16bits(frames.reshape(-1)))
    db = device_arena(batch * h3 * w3 * 128 * 2)
    dd = device_arena(batch * 3 * 4 * h0 * w0 * 2)
    engine.encode(df.ptr, db.ptr, batch)
    bott = O.f16bits_to_f32(hip.download(np.empty(batch * h3 * w3 * 128, np.uint16), db.ptr))
    # decode a different bottleneck than the encoder produced: the skips are the encoder's
    z = np.maximum(f16(rng.standard_normal((batch, 128, h3, w3))), 0)
    hip.upload(db.ptr, O.f32_to_f16bits(np.stack([nhwc(z[f]) for f in range(batch)]).reshape(-1)))
    engine.decode(db.ptr, dd.ptr, batch)
    hip.sync()
    disp = O.f16bits_to_f32(hip.download(np.empty(batch * 12 * h0 * w0, np.uint16), dd.ptr))
    for f in range(batch):
        e0 = O.conv3x3(frames[f], *W("enc0"), stride=1)
        e1 = O.conv3x3(e0, *W("enc1"), stride=2)
        e2 = O.conv3x3(e1, *W("enc2"), stride=2)
        e3 = O.conv3x3(e2, *W("enc3"), stride=2)
        mx, mean = errors(chw(bott[f * h3 * w3 * 128:(f + 1) * h3 * w3 * 128], h3, w3), e3)
        print(f"[codec] frame {f} bottleneck: max {mx:.3g} mean {mean:.3g}", flush=True)
        assert mx <= MAX_ABS and mean <= MEAN_ABS
        # the same chain with the reference's split-conv rounding in enc2/enc3
        s3 = O.conv3x3_split(O.conv3x3_split(e1, *W("enc2"), groups=2, mode=0), *W("enc3"), groups=4, mode=1)
        mx, mean = errors(chw(bott[f * h3 * w3 * 128:(f + 1) * h3 * w3 * 128], h3, w3), s3)
        print(f"[codec] frame {f} bottleneck vs split rounding: max {mx:.3g} mean {mean:.3g}", flush=True)
        assert mx <= MAX_ABS and mean <= MEAN_ABS
        d3 = O.dec_stage(z[f], e2, *W("dec3"))
        d2 = O.dec_stage(d3, e1, *W("dec2"))
        d1 = O.dec_stage(d2, e0, *W("dec1"))
        ref = O.pixelshuffle_sigmoid(O.pw_conv(d1, *W("out")), 2)
        g = disp[f * 12 * h0 * w0:(f + 1) * 12 * h0 * w0].reshape(3, 2 * h0, 2 * w0)
        mx, mean = errors(g, ref)
        print(f"[codec] frame {f} display: max {mx:.3g} mean {mean:.3g}", flush=True)
        assert mx <= MAX_ABS and mean <= MEAN_ABS


@pytest.mark.gpu
@pytest.mark.parametrize("name,render,nb,batch,affine", [
    ("moe16", (130, 90), 2, 1, False), ("moe64", (960, 540), 2, 1, False), ("moe16", (130, 90), 2, 4, False),
    # LN affines: the 68-row token grid's bottom windows take the PAD+HALF body
    # with the fused up-projection in block 0
    ("moe64", (960, 540), 2, 1, True), ("moe64", (960, 540), 1, 4, True),
])
def test_e2e_frame_equals_the_calls_it_chains(hip, engine, device_arena, name, render, nb, batch, affine):
    desc, r, W, _, (cblob, c, a) = setup(engine, render, name=name, nb=nb, affine=affine)
    (w0, h0), _, _, (w3, h3) = r
    rng = np.random.default_rng(9)
    n_in, n_out, n_tok = batch * 9 * h0 * w0, batch * 12 * h0 * w0, batch * h3 * w3 * 128
    frames = O.f32_to_f16bits(f16(rng.standard_normal(n_in)))
    df, dd, de = device_arena(n_in * 2), device_arena(n_out * 2), device_arena(n_out * 2)
    db, dc = device_arena(n_tok * 2), device_arena(n_tok * 2)
    hip.upload(df.ptr, frames)
    print(f"[e2e] {name} {render} batch {batch} affine={affine}", flush=True)
    engine.encode(df.ptr, db.ptr, batch)
    engine.forward(db.ptr, dc.ptr, batch, adapted=True)
    engine.decode(dc.ptr, dd.ptr, batch)
    hip.sync()
    ref = hip.download(np.empty(n_out, np.uint16), dd.ptr)
    for graph in (False, True, True):
        hip.memset(de.ptr, 0, n_out * 2)
        engine.forward_e2e(df.ptr, de.ptr, batch, graph=graph)
        hip.sync()
        got = hip.download(np.empty(n_out, np.uint16), de.ptr)
        assert (got == ref).all(), f"graph={graph}: {int((got != ref).sum())} values differ"
    disp = O.f16bits_to_f32(ref)
    assert 0.0 <= disp.min() and disp.max() <= 1.0 and disp.std() > 0.01
    # prism_infer_gpu runs the whole frame once the codec is loaded
    ms = engine.infer_gpu(df.ptr, 0, de.ptr, 0, batch)
    got = hip.download(np.empty(n_out, np.uint16), de.ptr)
    assert (got == ref).all() and ms > 0
    print(f"[e2e] infer_gpu {ms:.3f} ms", flush=True)


@pytest.mark.gpu
def test_codec_errors(hip, engine, device_arena):
    setup(engine, (70, 38))
    a = device_arena(1 << 16)
    with pytest.raises(P.PrismError) as ei:
        engine.codec_stage(7, a.ptr, None, a.ptr, 1)
    assert ei.value.code == P.ERR_INVALID
    with pytest.raises(P.PrismError) as ei:
        engine.codec_stage(4, a.ptr, None, a.ptr, 1)  # decoder stage without its skip map
    assert ei.value.code == P.ERR_INVALID
    # a render size that does not encode to the model's token grid is refused
    desc = P.CONFIGS["moe16"].desc(n_blocks=1, H=5, W=10)
    blob, offs = P.synth_weights(desc, seed=1)
    engine.load_weights(desc, blob, offs)  # another grid: the codec is dropped
    with pytest.raises(P.PrismError) as ei:
        engine.encode(a.ptr, a.ptr, 1)
    assert ei.value.code == P.ERR_STATE
    with pytest.raises(P.PrismError):
        P.codec_layout(desc, 70, 38)
