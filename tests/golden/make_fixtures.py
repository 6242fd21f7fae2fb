"""Writes the golden fixtures in this directory from the NumPy oracle.

    python tests/golden/make_fixtures.py

Inputs are regenerated from their seeds in the tests, so the files hold only
expected outputs (and a few input slices for self-checking).  Shapes follow
BASELINE configs[0] (Dense 512x512, per-tensor int8, batch 64) plus small
per-channel, special-value, W8A8 and MoE-routing cases.
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402


def config0():
    """seed 0; W ~ N(0, 0.05) (512, 512), b ~ N(0, 0.01),
    X ~ N(0, 1) (64, 512); per-tensor symmetric int8, dequantize, Dense (linear)."""
    rng = np.random.default_rng(0)
    w = rng.normal(0.0, 0.05, (512, 512)).astype(np.float32)
    b = rng.normal(0.0, 0.01, 512).astype(np.float32)
    x = rng.normal(0.0, 1.0, (64, 512)).astype(np.float32)
    return w, b, x


def per_channel_case():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((64, 96)) * rng.uniform(0.01, 1.0, (64, 1))).astype(np.float32)
    w[3] = 0.0
    w[5, :4] = [np.nan, 1.0, -1.0, 0.5]
    w[7, 0] = -0.0
    w[9, :3] = [1e-40, -3e-41, 2e-42]
    return w


def w8a8_case():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((48, 160)).astype(np.float32)
    w = rng.normal(0.0, 0.05, (72, 160)).astype(np.float32)
    b = rng.normal(0.0, 0.01, 72).astype(np.float32)
    return x, w, b


def moe_case():
    rng = np.random.default_rng(3)
    d, h, e = 32, 64, 8
    layer = {"type": "moe", "embed_dim": d, "num_experts": e, "top_k": 2, "activation": "gelu",
             "W1": rng.normal(0, 0.02, (e, h, d)).astype(np.float32),
             "b1": np.zeros((e, h), np.float32),
             "W2": rng.normal(0, 0.02, (e, d, h)).astype(np.float32),
             "b2": np.zeros((e, d), np.float32),
             "Wr": rng.normal(0, 0.5, (e, d)).astype(np.float32),
             "br": np.zeros(e, np.float32)}
    x = rng.standard_normal((40, d)).astype(np.float32)
    logits = rng.standard_normal((40, e)).astype(np.float32)
    return layer, x, logits


def main():
    w, b, x = config0()
    fq, scale, _ = oracle.quantize_tensor(w, 8)
    codes = oracle.quantize(w, scale, np.zeros_like(scale), 8, "symmetric").astype(np.int8)
    layer = {"type": "dense", "weights": fq, "bias": b, "activation": "linear"}
    y, _ = oracle.dense_forward(layer, x.astype(np.float64), np.float64)
    np.savez_compressed(os.path.join(HERE, "config0_dense.npz"), scale=scale,
                        codes_head=codes[:64], codes_checksum=np.int64(codes.astype(np.int64).sum()),
                        codes_weighted=np.int64((codes.astype(np.int64)
                                                 * np.arange(codes.size).reshape(codes.shape)).sum()),
                        y_head=y[:16].astype(np.float64))

    wc = per_channel_case()
    fq, scale, zp = oracle.quantize_tensor(wc, 8, per_channel=True)
    fqa, scalea, zpa = oracle.quantize_tensor(wc, 6, "asymmetric", per_channel=True)
    np.savez_compressed(os.path.join(HERE, "per_channel.npz"), w=wc, fake=fq, scale=scale, zp=zp,
                        fake_asym6=fqa, scale_asym6=scalea, zp_asym6=zpa)

    x8, w8, b8 = w8a8_case()
    codes8, s8 = oracle.int8_codes(w8, per_channel=True)
    y8, acc8, xs8, xc8 = oracle.w8a8_dense(x8, codes8, s8.reshape(-1), b8)
    np.savez_compressed(os.path.join(HERE, "w8a8.npz"), w_codes=codes8, w_scale=s8, x_codes=xc8,
                        x_scale=xs8, acc=acc8, y=y8)

    layer, xm, logits = moe_case()
    e = np.exp(logits - logits.max(axis=1, keepdims=True))
    probs = e / e.sum(axis=1, keepdims=True)
    ym = oracle.moe_forward(xm.astype(np.float64), {k: (v.astype(np.float64) if isinstance(v, np.ndarray) else v)
                                                    for k, v in layer.items()}, probs.astype(np.float64))
    np.savez_compressed(os.path.join(HERE, "moe.npz"), top=oracle.forward_top_k(probs, 2),
                        y=ym)
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
