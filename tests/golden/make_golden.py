#!/usr/bin/env python3
"""Writes tests/golden/moe8_12x20.npz: a regression fixture for the oracle and
the synthetic generator.

Workload: one MoE block, d256, 8 heads x 32, 8 experts, Zipf(1.1)-fitted router
bias, 12x20 token grid (padded windows on both axes), 2 frames, seed 0 for the
weights and seed 1 for the activations. Stored: SHA-256 of the weight blob,
the input and the oracle's fp16-faithful outputs (attention output h, expert
assignment, block output y), and value slices of the first 16 tokens of each
frame. Regenerate with: python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "prism-inference_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402
import prism_amd as P  # noqa: E402

H, W, B, N = 12, 20, 2, 8


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def compute():
    desc = P.ModelDesc(256, 1, 8, 32, N, H, W, 8)
    blob, offs = P.synth_weights(desc, seed=0, routing=P.ROUTE_ZIPF)
    x = P.synth_normal(B * H * W * 256, seed=1, stream=0, std=1.0).reshape(B * H * W, 256)
    c = O.cfg(256, 8, 32, N, H, W, B, faithful=True)
    w = O.f16bits_to_f32(blob)
    h = O.attn_stage(c, w, offs[0], O.f16bits_to_f32(x))
    assign, logits = O.router_stage(c, w, offs[0], h)
    y = O.expert_stage(c, w, offs[0], h, assign)
    hb, yb = O.f32_to_f16bits(h), O.f32_to_f16bits(y)
    rows = np.r_[0:16, H * W:H * W + 16]
    return {
        "blob_sha256": sha(blob), "x_sha256": sha(x), "h_sha256": sha(hb), "y_sha256": sha(yb),
        "assign_sha256": sha(assign), "assign": assign, "h_rows": hb[rows], "y_rows": yb[rows],
        "x_rows": x[rows], "rows": rows,
    }


if __name__ == "__main__":
    out = os.path.join(HERE, "moe8_12x20.npz")
    np.savez(out, **compute())
    print("wrote", out, os.path.getsize(out), "bytes")
