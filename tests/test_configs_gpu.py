"""GPU parity at the BASELINE configurations' own sizes.

* the 784 -> 1024 -> 1024 -> 10 MLP (He-normal weights quantized
  per output channel, ReLU, batch 4096 of U(0, 1)), every layer's output on
  all 4096 rows within max |y - y_ref| <= 1e-4 * max |y_ref| per row of the
  float64 oracle on the fake-quantized weights.
* the pre-norm transformer block (B 8, S 512, E 1024, 16 heads,
  FFN 4096 with GELU, weights N(0, 0.02) per channel, zero biases) through
  ``Forward``; every layer's output for whole batch elements 0 and 7 within
  the same bound of the float64 oracle run on that element alone (attention
  never mixes batch elements).
* the MoE layer (8192 tokens, 8 experts, top-2, d 1024, hidden
  4096, GELU, per-row expert weights, router logits N(0, 1) given): expert
  choices of every token identical to the oracle's ``argsort``, and every
  8th token's output (1024 tokens, spread over all tile rows of every
  expert) within the Dense bound of the float64 oracle routed by the same
  probabilities.
"""

import numpy as np
import pytest

import enilnets_amd as ea
from enilnets_amd.device import DeviceArray
from enilnets_amd.nn import Model
from enilnets_amd.nn.moe import moe_forward
import oracle

pytestmark = pytest.mark.gpu


def row_rel_err(got, ref):
    ref = np.asarray(ref, np.float64).reshape(-1, np.shape(ref)[-1])
    got = np.asarray(got, np.float64).reshape(ref.shape)
    denom = np.maximum(np.max(np.abs(ref), axis=-1), 1e-30)
    return np.max(np.abs(got - ref), axis=-1) / denom


def test_config1_mlp_batch4096(gpu):
    print("[case] configs[1] MLP 784-1024-1024-10 batch 4096", flush=True)
    rng = np.random.default_rng(0)
    m = Model()
    for (n_in, n_out), act in zip([(784, 1024), (1024, 1024), (1024, 10)],
                                  ["relu", "relu", "linear"]):
        w = rng.normal(0.0, np.sqrt(2.0 / n_in), (n_out, n_in)).astype(np.float32)
        b = rng.normal(0.0, 0.01, n_out).astype(np.float32)
        m.add_dense(w, b, act)
    ea.quantize_weights(m, bits=8, per_channel=True)
    x = rng.uniform(0.0, 1.0, (4096, 784)).astype(np.float32)
    y = m.Forward(x)
    want = oracle.forward(m.layers, x.astype(np.float64), dtype=np.float64)
    assert y.shape == (4096, 10) and y.dtype == np.float32
    for i in range(1, 4):
        err = row_rel_err(m.outputs[i], want[i])
        assert np.all(err <= 1e-4), f"layer {i - 1}: max row error {err.max():.3e}"
    # the pre-activations too (a ReLU row bound is loose where it clips)
    for i in range(1, 4):
        z_ref = want[i - 1] @ m.layers[i - 1]["weights"].astype(np.float64).T + \
            m.layers[i - 1]["bias"]
        err = row_rel_err(m.pre_activations[i], z_ref)
        assert np.all(err <= 1e-4), f"layer {i - 1} z: max row error {err.max():.3e}"


def test_config3_transformer_block(gpu):
    print("[case] configs[3] block B8 S512 E1024 H16 F4096", flush=True)
    B, S, E, F, H = 8, 512, 1024, 4096, 16
    rng = np.random.default_rng(3)
    m = Model()
    m.add_residual_start()
    m.add_layernorm(E)
    ws = [rng.normal(0.0, 0.02, (E, E)).astype(np.float32) for _ in range(4)]
    m.add_multihead_attention(*ws, num_heads=H)
    m.add_residual_end()
    m.add_residual_start()
    m.add_layernorm(E)
    m.add_dense(rng.normal(0.0, 0.02, (F, E)).astype(np.float32), np.zeros(F, np.float32), "gelu")
    m.add_dense(rng.normal(0.0, 0.02, (E, F)).astype(np.float32), np.zeros(E, np.float32),
                "linear")
    m.add_residual_end()
    ea.quantize_weights(m, bits=8, per_channel=True)
    x = rng.standard_normal((B, S, E)).astype(np.float32)
    y = m.Forward(x)
    assert y.shape == (B, S, E)
    for b in (0, B - 1):
        want = oracle.forward(m.layers, x[b:b + 1].astype(np.float64), dtype=np.float64)
        for i in range(1, len(want)):
            err = row_rel_err(m.outputs[i][b:b + 1], want[i])
            assert np.all(err <= 1e-4), f"element {b} layer {i - 1}: max row error {err.max():.3e}"


def test_config4_moe_8192_tokens(gpu):
    print("[case] configs[4] MoE T8192 E8 top2 d1024 h4096", flush=True)
    T_, D, Hd, E_, K_ = 8192, 1024, 4096, 8, 2
    rng = np.random.default_rng(4)
    L = {"type": "moe", "embed_dim": D, "num_experts": E_, "hidden_dim": Hd, "top_k": K_,
         "activation": "gelu", "quant": {}}
    for name, shape in (("W1", (E_, Hd, D)), ("W2", (E_, D, Hd))):
        w = rng.normal(0.0, 0.02, shape).astype(np.float32)
        fq, sc = [], []
        for e in range(E_):
            f, s, _ = oracle.quantize_tensor(w[e], 8, per_channel=True)
            fq.append(f)
            sc.append(s)
        L[name] = np.stack(fq)
        L["quant"][name] = {"bits": 8, "scheme": "symmetric", "scale": np.stack(sc),
                            "zero_point": np.zeros_like(np.stack(sc))}
    L["b1"] = np.zeros((E_, Hd), np.float32)
    L["b2"] = np.zeros((E_, D), np.float32)
    f, s, zp = oracle.quantize_tensor(rng.normal(0.0, 0.02, (E_, D)).astype(np.float32), 8,
                                      per_channel=True)
    L["Wr"], L["br"] = f, np.zeros(E_, np.float32)
    L["quant"]["Wr"] = {"bits": 8, "scheme": "symmetric", "scale": s, "zero_point": zp}
    x = rng.standard_normal((T_, D)).astype(np.float32)
    logits = rng.standard_normal((T_, E_)).astype(np.float32)
    out, info = moe_forward(DeviceArray.from_numpy(x), L,
                            router_logits=DeviceArray.from_numpy(logits), want_routing=True)
    z = logits - logits.max(axis=-1, keepdims=True)
    e = np.exp(z)
    probs = e / e.sum(axis=-1, keepdims=True)
    top = info["top_idx"].numpy()
    assert np.array_equal(top, oracle.top_k(probs, K_))
    counts = np.bincount(top.reshape(-1), minlength=E_)
    assert counts.sum() == T_ * K_ and np.all(counts > 1800)
    pick = np.arange(0, T_, 8)
    want = oracle.moe_forward(x[pick].astype(np.float64), L, probs=probs[pick].astype(np.float64))
    err = row_rel_err(out.numpy()[pick], want)
    assert np.all(err <= 1e-4), f"max row error {err.max():.3e}"
