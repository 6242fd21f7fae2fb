"""GPU parity of KV-cache decoding (``Enilnets/nn/kvcache.py``).

The reference pins stepping by the full forward pass: a causal stack stepped
token by token through a cache gives the outputs ``Forward`` gives over the
whole sequence (``test_enilnets.py:4949-4975,7605-7628,7782-7830``).  Here:
cached GPU steps against the GPU ``Forward`` and against the float64 oracle,
with the Dense bound (max |y - y_ref| <= 1e-4 * max |y_ref| per row); a
sliding-window cache stays bounded; a non-causal layer is refused; beam
reordering gathers the cache by batch row.
"""

import numpy as np
import pytest

import enilnets_amd as ea
from enilnets_amd.nn import Model
from enilnets_amd.nn.kvcache import KVCache, cached_forward_step
import oracle

pytestmark = pytest.mark.gpu


def row_rel_err(got, ref):
    ref = np.asarray(ref, np.float64).reshape(-1, np.shape(ref)[-1])
    got = np.asarray(got, np.float64).reshape(ref.shape)
    denom = np.maximum(np.max(np.abs(ref), axis=-1), 1e-30)
    return np.max(np.abs(got - ref), axis=-1) / denom


def decoder(rng, vocab=50, E=64, H=4, Hkv=2, window=None, moe=False, causal=True):
    m = Model()
    m.layers.append({"type": "embedding",
                     "weights": (rng.standard_normal((vocab, E)) * 0.5).astype(np.float32),
                     "vocab_size": vocab, "embed_dim": E})
    pos = np.arange(128)[:, None] * np.exp(np.arange(0, E, 2) * -(np.log(10000.0) / E))[None]
    pe = np.zeros((128, E), np.float32)
    pe[:, 0::2], pe[:, 1::2] = np.sin(pos), np.cos(pos)
    m.layers.append({"type": "positional_encoding", "pe": pe, "max_seq_len": 128,
                     "embed_dim": E, "_pos_type": "sinusoidal"})
    kv = Hkv * (E // H)
    ws = [(rng.standard_normal(s) * 0.08).astype(np.float32)
          for s in ((E, E), (kv, E), (kv, E), (E, E))]
    m.add_residual_start()
    m.add_layernorm(E)
    m.add_multihead_attention(*ws, num_heads=H, num_kv_heads=Hkv, causal=causal,
                              window_size=window)
    m.add_residual_end()
    m.add_residual_start()
    m.add_layernorm(E)
    if moe:
        m.add_moe((rng.standard_normal((4, 96, E)) * 0.08).astype(np.float32),
                  (rng.standard_normal((4, E, 96)) * 0.08).astype(np.float32),
                  (rng.standard_normal((4, E)) * 0.2).astype(np.float32), top_k=2)
    else:
        m.add_dense((rng.standard_normal((128, E)) * 0.08).astype(np.float32),
                    np.zeros(128, np.float32), "gelu")
        m.add_dense((rng.standard_normal((E, 128)) * 0.08).astype(np.float32),
                    np.zeros(E, np.float32), "linear")
    m.add_residual_end()
    m.add_dense((rng.standard_normal((vocab, E)) * 0.08).astype(np.float32),
                np.zeros(vocab, np.float32), "linear")
    ea.quantize_weights(m, per_channel=True)
    return m


def step_all(m, tokens, prime):
    cache = KVCache()
    outs = [cached_forward_step(m, tokens[:, :prime], cache)]
    for t in range(prime, tokens.shape[1]):
        outs.append(cached_forward_step(m, tokens[:, t:t + 1], cache))
    return np.concatenate(outs, axis=1), cache


@pytest.mark.parametrize("window,moe", [(None, False), (4, False), (None, True)])
def test_cached_steps_match_full_forward(gpu, window, moe):
    print(f"[case] kvcache window={window} moe={moe}", flush=True)
    rng = np.random.default_rng(3 + (window or 0) + moe)
    m = decoder(rng, window=window, moe=moe)
    tokens = rng.integers(0, 50, (2, 20))
    full = m.Forward(tokens)
    stepped, cache = step_all(m, tokens, prime=7)
    assert stepped.shape == full.shape and stepped.dtype == full.dtype
    assert np.all(row_rel_err(stepped, full) <= 1e-4)
    want = oracle.forward(m.layers, tokens, dtype=np.float64)[-1]
    assert np.all(row_rel_err(stepped, want) <= 1e-4)
    assert cache.position == 20
    if window is not None:
        entry = next(iter(cache.kv.values()))
        assert entry.length <= window + 1
        assert entry.start == 20 - entry.length


def test_cached_steps_ignore_act_quant(gpu):
    # the reference's cached step (kvcache.py:84-118) never applies a layer's
    # act_quant spec: on a calibrated model the steps follow the float layers,
    # while Forward fake-quantizes every layer output
    print("[case] kvcache calibrated model", flush=True)
    rng = np.random.default_rng(21)
    m = decoder(rng)
    tokens = rng.integers(0, 50, (2, 14))
    cal = ea.ActivationCalibrator(m)
    cal.observe(tokens)
    cal.apply()
    assert sum("act_quant" in layer for layer in m.layers) >= 8
    stepped, _ = step_all(m, tokens, prime=6)
    plain = [{k: v for k, v in layer.items() if k != "act_quant"} for layer in m.layers]
    want = oracle.forward(plain, tokens, dtype=np.float64)[-1]
    assert np.all(row_rel_err(stepped, want) <= 1e-4)
    # the specs would have moved the outputs by about a grid step of each layer
    quantized = oracle.forward(m.layers, tokens, dtype=np.float64)[-1]
    assert np.max(row_rel_err(stepped, quantized)) > 1e-3


def test_non_causal_attention_is_refused(gpu):
    m = decoder(np.random.default_rng(0), causal=False)
    with pytest.raises(ValueError):
        cached_forward_step(m, np.array([[1, 2]]), KVCache())


def test_beam_reorder_gathers_rows(gpu):
    rng = np.random.default_rng(8)
    m = decoder(rng)
    prompt = rng.integers(0, 50, (1, 6))
    cache = KVCache()
    cached_forward_step(m, prompt, cache)
    cache.expand(3)
    nxt = np.array([[5], [9], [13]])
    beams = cached_forward_step(m, nxt, cache)
    for b in range(3):
        single = KVCache()
        cached_forward_step(m, prompt, single)
        one = cached_forward_step(m, nxt[b:b + 1], single)
        assert np.all(row_rel_err(beams[b:b + 1], one) <= 1e-6)
    cache.reorder([2, 2, 0])
    after = cached_forward_step(m, np.array([[1], [1], [1]]), cache)
    assert np.allclose(after[0], after[1], rtol=0, atol=0)


def test_trusted_weights_session(gpu):
    # a session that promises unchanged weights gives the same steps, and a
    # weight replaced by a new array is still picked up
    rng = np.random.default_rng(11)
    m = decoder(rng)
    tokens = rng.integers(0, 50, (2, 12))
    plain, _ = step_all(m, tokens, prime=5)
    cache = KVCache(trust_weights=True)
    outs = [cached_forward_step(m, tokens[:, :5], cache)]
    for t in range(5, 12):
        outs.append(cached_forward_step(m, tokens[:, t:t + 1], cache))
    trusted = np.concatenate(outs, axis=1)
    assert np.array_equal(trusted, plain)
    # replace the output layer's weights (a new array) in the middle of a
    # trusted session: the next step uses them.  That layer follows every
    # attention layer, so a fresh session over the changed model holds the
    # same K/V history.
    t_cache = KVCache(trust_weights=True)
    cached_forward_step(m, tokens[:, :5], t_cache)
    last = m.layers[-1]
    last["weights"] = last["weights"] * np.float32(0.5)
    ea.quantize_weights(m, per_channel=True)
    got = cached_forward_step(m, tokens[:, 5:6], t_cache)
    fresh = KVCache()
    cached_forward_step(m, tokens[:, :5], fresh)
    want = cached_forward_step(m, tokens[:, 5:6], fresh)
    assert np.array_equal(got, want)
