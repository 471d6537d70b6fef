"""Pins the oracle's encoder / decoder functions (CPU only): each against an
independent torch fp64 formulation of the reference shader, plus closed forms
that a wrong tap order, stride, upsample index or channel order would break."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O

rng = np.random.default_rng(7)


def f16(a):
    return a.astype(np.float16).astype(np.float32)


def r16(a):
    return np.asarray(a, np.float64).astype(np.float16).astype(np.float64)


def one_rounding(got, exact):
    """got = r16 of an fp32 evaluation of `exact`: within one fp16 ulp of
    r16(exact), plus the fp32 accumulation error (which can move a value
    across an fp16 rounding boundary, several ulps for near-zero subnormals)."""
    slack = 1e-6 * max(1.0, float(np.abs(exact).max()))
    return bool((np.abs(got - r16(exact)) <= np.maximum(np.abs(r16(exact)) * 2.0 ** -10, 2.0 ** -24) + slack).all())


def torch_conv(x, W, b, stride, relu):
    cin = x.shape[0]
    wt = torch.from_numpy(W.astype(np.float64)).reshape(W.shape[0], cin, 3, 3)  # k = ic*9 + ky*3 + kx
    y = F.conv2d(torch.from_numpy(x.astype(np.float64))[None], wt, torch.from_numpy(b.astype(np.float64)),
                 stride=stride, padding=1)[0]
    return (y.clamp_min(0) if relu else y).numpy()


@pytest.mark.parametrize("cin,cout,h,w,stride", [(9, 32, 13, 21, 1), (32, 64, 15, 22, 2), (64, 128, 9, 11, 2),
                                                  (128, 128, 7, 8, 2), (32, 64, 135, 17, 2)])
def test_conv3x3_matches_torch(cin, cout, h, w, stride):
    x = f16(rng.standard_normal((cin, h, w)))
    W = f16(rng.standard_normal((cout, cin * 9)) * 0.05)
    b = f16(rng.standard_normal(cout) * 0.05)
    ref = torch_conv(x, W, b, stride, True)
    got = O.conv3x3(x, W, b, stride, relu=True, faithful=False)
    assert got.shape == ref.shape == (cout, (h - 1) // stride + 1, (w - 1) // stride + 1)
    assert np.abs(got - ref).max() <= 2e-5 * max(1.0, np.abs(ref).max())
    # faithful = one fp16 rounding of the sum (at most one fp16 ulp from r16 of the exact value)
    gf = O.conv3x3(x, W, b, stride, relu=True, faithful=True)
    assert one_rounding(gf, ref)
    assert (gf == r16(gf)).all()


@pytest.mark.parametrize("stride", [1, 2])
def test_conv3x3_identity_and_bias(stride):
    c, h, w = 32, 11, 14
    x = f16(rng.standard_normal((c, h, w)))
    W = np.zeros((c, c * 9), np.float32)
    W[np.arange(c), np.arange(c) * 9 + 4] = 1.0  # centre tap of its own channel
    y = O.conv3x3(x, W, np.zeros(c, np.float32), stride)
    assert (y == np.maximum(x[:, ::stride, ::stride], 0)).all()
    # one off-centre tap: the map shifted by (dy, dx) = (1, -1), zero filled
    W2 = np.zeros((c, c * 9), np.float32)
    W2[np.arange(c), np.arange(c) * 9 + 2 * 3 + 0] = 1.0  # ky = 2, kx = 0 -> x[y + 1][x - 1]
    y2 = O.conv3x3(x, W2, np.zeros(c, np.float32), 1, relu=False)
    ref = np.zeros_like(x)
    ref[:, :-1, 1:] = x[:, 1:, :-1]
    assert (y2 == ref).all()
    bias = f16(rng.standard_normal(c))
    y3 = O.conv3x3(x, np.zeros_like(W), bias, stride)
    assert (y3 == np.maximum(bias, 0)[:, None, None]).all()


def torch_dec(up, skip, W, b):
    oh, ow = skip.shape[1:]
    u = torch.from_numpy(up.astype(np.float64)).repeat_interleave(2, 1).repeat_interleave(2, 2)
    uh = up.shape[1]
    ri = torch.clamp(torch.arange(oh) // 2, max=uh - 1)
    ci = torch.clamp(torch.arange(ow) // 2, max=up.shape[2] - 1)
    u = torch.from_numpy(up.astype(np.float64))[:, ri][:, :, ci]
    z = torch.cat([u, torch.from_numpy(skip.astype(np.float64))], 0)
    y = torch.einsum("ok,khw->ohw", torch.from_numpy(W.astype(np.float64)), z) + torch.from_numpy(
        b.astype(np.float64))[:, None, None]
    return y.clamp_min(0).numpy()


@pytest.mark.parametrize("cup,cskip,cout,uh,uw,oh,ow", [(128, 128, 128, 7, 9, 13, 18), (128, 64, 64, 5, 6, 10, 12),
                                                         (64, 32, 32, 68, 5, 135, 10)])
def test_dec_stage_matches_torch(cup, cskip, cout, uh, uw, oh, ow):
    up = f16(rng.standard_normal((cup, uh, uw)))
    skip = f16(rng.standard_normal((cskip, oh, ow)))
    W = f16(rng.standard_normal((cout, cup + cskip)) * 0.05)
    b = f16(rng.standard_normal(cout) * 0.05)
    ref = torch_dec(up, skip, W, b)
    got = O.dec_stage(up, skip, W, b, faithful=False)
    assert np.abs(got - ref).max() <= 2e-5 * max(1.0, np.abs(ref).max())
    gf = O.dec_stage(up, skip, W, b)
    assert one_rounding(gf, ref)


def test_dec_stage_selects_channels():
    """A one-hot row picks one input channel: the upsampled map (each coarse
    pixel covers a 2x2 block, the last row/column clamped) or the skip map."""
    up = f16(rng.standard_normal((64, 4, 5)))
    skip = f16(rng.standard_normal((32, 7, 10)))
    W = np.zeros((32, 96), np.float32)
    W[0, 3] = 1.0    # up channel 3
    W[1, 64 + 5] = 1.0  # skip channel 5
    y = O.dec_stage(up, skip, W, np.zeros(32, np.float32))
    expect_up = np.maximum(up[3][np.minimum(np.arange(7) // 2, 3)][:, np.minimum(np.arange(10) // 2, 4)], 0)
    assert (y[0] == expect_up).all()
    assert (y[1] == np.maximum(skip[5], 0)).all()
    assert (y[2:] == 0).all()


def test_pw_conv_matches_torch():
    x = f16(rng.standard_normal((32, 9, 13)))
    W = f16(rng.standard_normal((12, 32)) * 0.1)
    b = f16(rng.standard_normal(12) * 0.1)
    ref = np.einsum("ok,khw->ohw", W.astype(np.float64), x.astype(np.float64)) + b[:, None, None]
    got = O.pw_conv(x, W, b, relu=False, faithful=False)
    assert np.abs(got - ref).max() <= 1e-5
    assert (O.pw_conv(x, W, b, relu=True, faithful=False) == np.maximum(got, 0)).all()


def test_pixelshuffle_sigmoid_matches_torch():
    x = f16(rng.standard_normal((12, 9, 13)) * 3)
    ps = F.pixel_shuffle(torch.from_numpy(x.astype(np.float64))[None], 2)[0]
    ref = torch.sigmoid(ps).numpy()
    got = O.pixelshuffle_sigmoid(x, 2, faithful=False)
    assert got.shape == (3, 18, 26)
    assert np.abs(got - ref).max() <= 1e-6
    gf = O.pixelshuffle_sigmoid(x, 2)
    assert one_rounding(gf, ref)
    # closed forms: sigmoid(0) = 1/2; the shuffle is a permutation (its inverse restores x)
    assert (O.pixelshuffle_sigmoid(np.zeros((12, 3, 4), np.float32), 2) == 0.5).all()
    g64 = got.astype(np.float64)
    logit = np.log(g64 / (1 - g64))  # fp32 sigmoid near 1 keeps ~1e-4 of the logit
    back = F.pixel_unshuffle(torch.from_numpy(logit)[None], 2)[0].numpy()
    assert np.abs(back - x).max() <= 2e-3


# ---- the reference's split strided convs (their own per-group rounding) ----

def torch_split(x, W, b, groups, mode):
    """strided_conv_split_{64,128}ch restated with torch fp64 group convs: each
    group's partial rounded to fp16 with its bias, combined in fp32 (mode 0)
    or as a running fp16 sum (mode 1), then ReLU. Also returns the largest
    |partial| per element (the scale of a one-ulp flip of a partial)."""
    gc = x.shape[0] // groups
    parts = [r16(torch_conv(x[g * gc:(g + 1) * gc], W[:, g * gc * 9:(g + 1) * gc * 9], b, 2, False))
             for g in range(groups)]
    scale = np.max(np.abs(np.stack(parts)), axis=0)
    bb = b.astype(np.float32)[:, None, None]
    if mode == 0:
        v = (parts[0].astype(np.float32) + parts[1].astype(np.float32)) - bb
        return r16(np.maximum(v, 0)), scale
    acc = parts[0]
    for g in range(1, groups):
        acc = r16((acc.astype(np.float32) + parts[g].astype(np.float32)) - bb)
        scale = np.maximum(scale, np.abs(acc))
    return np.maximum(acc, 0), scale


@pytest.mark.parametrize("cin,groups,mode", [(64, 2, 0), (128, 4, 1), (64, 2, 1)])
def test_conv3x3_split_matches_torch_restatement(cin, groups, mode):
    x = f16(rng.standard_normal((cin, 11, 13)))
    W = f16(rng.standard_normal((128, cin * 9)) * 0.05)
    b = f16(rng.standard_normal(128) * 0.05)
    got = O.conv3x3_split(x, W, b, groups, mode)
    ref, scale = torch_split(x, W, b, groups, mode)
    assert got.shape == ref.shape == (128, 6, 7)
    # identical except where an fp32 (oracle) and an fp64 (torch) partial sum
    # round to neighbouring fp16 values: one ulp of that partial, rarely
    d = np.abs(got - ref)
    ulp = np.maximum(np.maximum(np.abs(ref), scale) * 2.0 ** -10, 2.0 ** -24)
    assert (d <= groups * ulp + 1e-7).all() and (d > 0).mean() < 0.01
    # and the unsplit conv (this build's single rounding) is within a few ulps
    one = O.conv3x3(x, W, b, 2, relu=True, faithful=True)
    assert (np.abs(one - got) <= (groups + 1) * np.maximum(scale, np.abs(ref)) * 2.0 ** -10 + 1e-7).all()


def test_conv3x3_split_one_group_is_the_unsplit_conv():
    x = f16(rng.standard_normal((32, 9, 10)))
    W = f16(rng.standard_normal((64, 32 * 9)) * 0.05)
    b = f16(rng.standard_normal(64) * 0.05)
    np.testing.assert_array_equal(O.conv3x3_split(x, W, b, 1, 1), O.conv3x3(x, W, b, 2, relu=True, faithful=True))


@pytest.mark.parametrize("cin,groups,mode", [(64, 2, 0), (128, 4, 1)])
def test_conv3x3_split_later_groups_zero(cin, groups, mode):
    """With zero weights in groups 1.. and zero bias, every later partial is 0
    and the result is group 0's conv with one rounding, exactly."""
    x = f16(rng.standard_normal((cin, 12, 9)))
    W = f16(rng.standard_normal((96, cin * 9)) * 0.05)
    W[:, 32 * 9:] = 0
    b = np.zeros(96, np.float32)
    got = O.conv3x3_split(x, W, b, groups, mode)
    np.testing.assert_array_equal(got, O.conv3x3(x[:32], W[:, :32 * 9], b, 2, relu=True, faithful=True))


def test_conv3x3_split_rejects_bad_shapes():
    x = np.zeros((48, 5, 5), np.float32)
    with pytest.raises(Exception):
        O.conv3x3_split(x, np.zeros((16, 48 * 9), np.float32), np.zeros(16, np.float32), 4, 0)  # mode 0: 2 groups
    with pytest.raises(Exception):
        O.conv3x3_split(x, np.zeros((16, 48 * 9), np.float32), np.zeros(16, np.float32), 5, 1)  # 48 % 5
