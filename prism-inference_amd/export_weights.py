#!/usr/bin/env python3
"""Write a model as the reference's weight-file pair: <name>.weights (flat fp16
values, no header) and <name>.json (sidecar).

The reference's exporter (vulkan_engine/export_weights.py:96-120) writes the
same pair for its conv layers: fp16 via IEEE round-to-nearest-even, then per
layer `weight_offset_fp16`, `bias_offset_fp16`, `weight_count`, `bias_count`.
This one writes the transformer: the sidecar has "format":
"prism-transformer-v1", the model shape, and one entry per layer with its
`kind` (ln1, qkv, out, ln2, router, experts, proj_up, proj_down) and `block`
(-1 for the adapters), in the offsets of the engine's blob layout
(prism_layout / prism_adapter_layout). prism_load_model_file reads it back.

Unlike the reference, it does not read ncnn files: the reference treats an
ncnn .bin as one headerless fp32 array, but ncnn prefixes each weight blob
with a 4-byte type tag, so its offsets drift by one word per layer. Inputs
here are either named tensors in an .npz (read with allow_pickle=False) or
the synthetic model.

    python export_weights.py synth moe64 out.weights [--blocks N] [--adapters] [--seed S]
    python export_weights.py npz model.npz out.weights --H 68 --W 120 [--window 8]

npz tensor names (row-major [out][in] matrices, any float dtype):
    blocks.{b}.ln1.gamma / .beta, blocks.{b}.qkv.weight [3d][d] / .bias,
    blocks.{b}.out.weight [d][d] / .bias, blocks.{b}.ln2.gamma / .beta,
    blocks.{b}.router.weight [N][d] / .bias (N > 1 only),
    blocks.{b}.experts.{e}.w1 [d][d] / .b1 / .w2 / .b2,
    proj_up.weight [d][128] / .bias, proj_down.weight [128][d] / .bias (optional).
"""
import argparse
import json
import os
import re
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import prism_amd as P  # noqa: E402

FORMAT = "prism-transformer-v1"


def _layer(name, kind, block, w_off, w_n, b_off, b_n, **extra):
    d = {"name": name, "kind": kind, "block": block, "type": "linear" if kind not in ("ln1", "ln2") else "layernorm",
         "weight_offset_fp16": int(w_off), "weight_count": int(w_n),
         "bias_offset_fp16": int(b_off), "bias_count": int(b_n)}
    d.update(extra)
    return d


def sidecar(desc, offs, total, adapters=None):
    """The JSON sidecar (a dict) for a blob of `total` fp16 values laid out per offs."""
    D, N = desc.dim, desc.n_experts
    layers = []
    for b in range(desc.n_blocks):
        o = offs[b]
        layers.append(_layer(f"blocks.{b}.ln1", "ln1", b, o.ln1_g, D, o.ln1_b, D))
        layers.append(_layer(f"blocks.{b}.qkv", "qkv", b, o.qkv_w, 3 * D * D, o.qkv_b, 3 * D, out=3 * D, **{"in": D}))
        layers.append(_layer(f"blocks.{b}.out", "out", b, o.out_w, D * D, o.out_b, D, out=D, **{"in": D}))
        layers.append(_layer(f"blocks.{b}.ln2", "ln2", b, o.ln2_g, D, o.ln2_b, D))
        if N > 1:
            layers.append(_layer(f"blocks.{b}.router", "router", b, o.router_w, N * D, o.router_b, N, out=N,
                                 **{"in": D}))
        layers.append({"name": f"blocks.{b}.experts", "kind": "experts", "block": b, "type": "experts",
                       "n_experts": N, "expert_stride": int(o.exp_stride),
                       "w1_offset_fp16": int(o.exp_w1), "b1_offset_fp16": int(o.exp_b1),
                       "w2_offset_fp16": int(o.exp_w2), "b2_offset_fp16": int(o.exp_b2),
                       "weight_count": 2 * D * D * N, "bias_count": 2 * D * N})
    if adapters is not None:
        I = adapters.in_dim
        layers.append(_layer("proj_up", "proj_up", -1, adapters.up_w, D * I, adapters.up_b, D, in_dim=I, out=D,
                             **{"in": I}))
        layers.append(_layer("proj_down", "proj_down", -1, adapters.down_w, I * D, adapters.down_b, I, in_dim=I,
                             out=I, **{"in": D}))
    model = {k: int(getattr(desc, k)) for k in ("dim", "n_blocks", "n_heads", "head_dim", "n_experts",
                                                  "spatial_h", "spatial_w", "window")}
    return {"format": FORMAT, "total_fp16_values": int(total), "total_bytes": int(total) * 2,
            "model": model, "layers": layers}


def write_model(weights_path, desc, blob, offs, adapters=None):
    """Write <weights_path> (flat fp16) and its .json sidecar; returns the sidecar path."""
    if not weights_path.endswith(".weights"):
        raise ValueError("the weights file name must end in .weights")
    blob = np.ascontiguousarray(blob, dtype=np.uint16)
    blob.tofile(weights_path)
    jpath = weights_path[:-len(".weights")] + ".json"
    with open(jpath, "w") as f:
        json.dump(sidecar(desc, offs, blob.size, adapters), f, indent=1)
    return jpath


def synth_model(cfg_name, n_blocks=None, seed=0, adapters=False, H=None, W=None):
    """(desc, blob, offs, adapter offsets | None) of the synthetic model, adapters appended to the blob."""
    cfg = P.CONFIGS[cfg_name]
    desc = cfg.desc(n_blocks=n_blocks, H=H, W=W)
    blob, offs = P.synth_weights(desc, seed=seed, routing=cfg.routing)
    if not adapters:
        return desc, blob, offs, None
    a, end = P.adapter_layout(desc, blob.size)
    ablob, a0 = P.synth_adapters(desc, seed=seed + 100)
    full = np.zeros(end, dtype=np.uint16)
    full[:blob.size] = blob
    for f in ("up_w", "up_b", "down_w", "down_b"):
        n = {"up_w": desc.dim * a.in_dim, "up_b": desc.dim, "down_w": a.in_dim * desc.dim, "down_b": a.in_dim}[f]
        full[getattr(a, f):getattr(a, f) + n] = ablob[getattr(a0, f):getattr(a0, f) + n]
    return desc, full, offs, a


def _f16(x):
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16).reshape(-1))


def from_tensors(t, H, W, window=8):
    """(desc, blob, offs, adapter offsets | None) from named tensors (see the module docstring)."""
    blocks = sorted({int(m.group(1)) for k in t for m in [re.match(r"blocks\.(\d+)\.", k)] if m})
    if not blocks or blocks != list(range(len(blocks))):
        raise ValueError("blocks.{b}.* tensors must cover blocks 0..n-1")
    D = int(np.asarray(t["blocks.0.qkv.weight"]).shape[1])
    experts = sorted({int(m.group(1)) for k in t for m in [re.match(r"blocks\.0\.experts\.(\d+)\.", k)] if m})
    N = len(experts)
    n_heads = 8
    desc = P.ModelDesc(D, len(blocks), n_heads, D // n_heads, N, H, W, window)
    offs, total = P.layout(desc)
    has_ad = "proj_up.weight" in t
    a, end = P.adapter_layout(desc, total) if has_ad else (None, total)
    blob = np.zeros(end, dtype=np.uint16)

    def put(off, name, shape):
        x = np.asarray(t[name])
        if tuple(x.shape) != tuple(shape):
            raise ValueError(f"{name}: shape {tuple(x.shape)}, expected {tuple(shape)}")
        v = _f16(x)
        blob[off:off + v.size] = v

    for b in blocks:
        o, p = offs[b], f"blocks.{b}."
        put(o.ln1_g, p + "ln1.gamma", (D,))
        put(o.ln1_b, p + "ln1.beta", (D,))
        put(o.qkv_w, p + "qkv.weight", (3 * D, D))
        put(o.qkv_b, p + "qkv.bias", (3 * D,))
        put(o.out_w, p + "out.weight", (D, D))
        put(o.out_b, p + "out.bias", (D,))
        put(o.ln2_g, p + "ln2.gamma", (D,))
        put(o.ln2_b, p + "ln2.beta", (D,))
        if N > 1:
            put(o.router_w, p + "router.weight", (N, D))
            put(o.router_b, p + "router.bias", (N,))
        for e in range(N):
            eo = e * o.exp_stride
            put(o.exp_w1 + eo, p + f"experts.{e}.w1", (D, D))
            put(o.exp_b1 + eo, p + f"experts.{e}.b1", (D,))
            put(o.exp_w2 + eo, p + f"experts.{e}.w2", (D, D))
            put(o.exp_b2 + eo, p + f"experts.{e}.b2", (D,))
    if has_ad:
        I = a.in_dim
        put(a.up_w, "proj_up.weight", (D, I))
        put(a.up_b, "proj_up.bias", (D,))
        put(a.down_w, "proj_down.weight", (I, D))
        put(a.down_b, "proj_down.bias", (I,))
    return desc, blob, offs, a


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("synth")
    s.add_argument("config", choices=sorted(P.CONFIGS))
    s.add_argument("out")
    s.add_argument("--blocks", type=int)
    s.add_argument("--seed", type=int, default=0)
    s.add_argument("--adapters", action="store_true")
    n = sub.add_parser("npz")
    n.add_argument("npz")
    n.add_argument("out")
    n.add_argument("--H", type=int, required=True)
    n.add_argument("--W", type=int, required=True)
    n.add_argument("--window", type=int, default=8)
    args = ap.parse_args()
    if args.cmd == "synth":
        desc, blob, offs, a = synth_model(args.config, args.blocks, args.seed, args.adapters)
    else:
        with np.load(args.npz, allow_pickle=False) as z:
            desc, blob, offs, a = from_tensors({k: z[k] for k in z.files}, args.H, args.W, args.window)
    jpath = write_model(args.out, desc, blob, offs, a)
    print(f"wrote {args.out} ({blob.size * 2} bytes) and {jpath}")


if __name__ == "__main__":
    main()
