"""GPU parity of the transformer-block layers on the quantized path.

* LayerNorm: max |y - y_ref| <= 2e-6 * max |y_ref| per row against the
  float64 oracle (``nn/forward.py:207-254``).
* Residual add: bit-identical to NumPy's float32 sum.
* Attention core, and the KV-cache step's attention (queries at positions
  after the cached keys, enq_attention_kv): max |ctx - ctx_ref| <= 2e-5 * max |ctx_ref| per row
  against float64 attention on the same Q, K, V (head_dim 16: fp32 MFMA
  products; 32-128: each fp32 operand split into three bf16 parts, six
  bf16 MFMA part products per product; fp32 sums and exponentials).
* Multi-head attention layer and transformer block through ``Forward``:
  the Dense bound, max |y - y_ref| <= 1e-4 * max |y_ref| per row, against the
  float64 oracle on the fake-quantized weights; host dtypes follow NumPy's
  promotion in the reference.
"""

import numpy as np
import pytest

import enilnets_amd as ea
from enilnets_amd.device import DeviceArray
from enilnets_amd.nn import Model
from enilnets_amd.nn import transformer as T
from enilnets_amd import _lib
import oracle

pytestmark = pytest.mark.gpu


def row_rel_err(got, ref):
    ref = np.asarray(ref, np.float64).reshape(-1, np.shape(ref)[-1])
    got = np.asarray(got, np.float64).reshape(ref.shape)
    denom = np.maximum(np.max(np.abs(ref), axis=-1), 1e-30)
    return np.max(np.abs(got - ref), axis=-1) / denom


@pytest.mark.parametrize("rows,cols", [(4096, 1024), (7, 5), (3, 300), (33, 1000), (2, 5000),
                                       (5, 4096), (6, 2048), (5, 1540)])
def test_layernorm(gpu, rows, cols):
    print(f"[case] layernorm rows={rows} cols={cols}", flush=True)
    rng = np.random.default_rng(rows + cols)
    x = (rng.standard_normal((rows, cols)) * 2 + 0.5).astype(np.float32)
    layer = {"gamma": rng.standard_normal(cols).astype(np.float32),
             "beta": rng.standard_normal(cols).astype(np.float32), "epsilon": 1e-5}
    y = T.layernorm(DeviceArray.from_numpy(x), layer).numpy()
    want = oracle.layernorm_forward(x.astype(np.float64), layer)
    assert np.all(row_rel_err(y, want) <= 2e-6)


def test_residual_add_bit_exact(gpu):
    rng = np.random.default_rng(3)
    for n in (1, 5, 1000003):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        got = T.residual_add(DeviceArray.from_numpy(a), DeviceArray.from_numpy(b)).numpy()
        assert np.array_equal(got.view(np.uint32), (a + b).view(np.uint32))


def attention_ref(q, k, v, H, Hkv, Dh, causal, window):
    B, S, _ = q.shape
    qh = q.reshape(B, S, H, Dh).transpose(0, 2, 1, 3).astype(np.float64)
    kh = k.reshape(B, S, Hkv, Dh).transpose(0, 2, 1, 3).astype(np.float64)
    vh = v.reshape(B, S, Hkv, Dh).transpose(0, 2, 1, 3).astype(np.float64)
    kh = np.repeat(kh, H // Hkv, axis=1)
    vh = np.repeat(vh, H // Hkv, axis=1)
    s = qh @ kh.transpose(0, 1, 3, 2) / np.sqrt(Dh)
    m = oracle.window_mask(S, causal, window)
    if m is not None:
        s = s + m
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    return (p @ vh).transpose(0, 2, 1, 3).reshape(B, S, H * Dh)


ATTN_CASES = [
    # B, S, H, Hkv, Dh, causal, window
    (2, 130, 4, 2, 32, False, None),
    (1, 64, 2, 2, 64, False, None),
    (2, 77, 4, 1, 16, True, None),
    (1, 200, 2, 2, 128, False, 5),
    (1, 70, 2, 2, 64, True, 0),
    (2, 300, 4, 2, 64, True, None),
    (3, 1, 2, 1, 64, False, None),
    (8, 512, 16, 16, 64, False, None),
]


@pytest.mark.parametrize("B,S,H,Hkv,Dh,causal,window", ATTN_CASES)
def test_attention_core(gpu, B, S, H, Hkv, Dh, causal, window):
    print(f"[case] attention B={B} S={S} H={H} Hkv={Hkv} Dh={Dh} causal={causal} "
          f"window={window}", flush=True)
    rng = np.random.default_rng(B * 1000 + S + Dh)
    nq, nkv = H * Dh, Hkv * Dh
    qkv = rng.standard_normal((B, S, nq + 2 * nkv)).astype(np.float32)
    q, k, v = qkv[..., :nq], qkv[..., nq:nq + nkv], qkv[..., nq + nkv:]
    d = DeviceArray.from_numpy(qkv)
    out = DeviceArray((B, S, nq), np.float32)
    ld = nq + 2 * nkv
    _lib.call("enq_attention", d.ptr, ld, T._at(d, 4 * nq), ld, T._at(d, 4 * (nq + nkv)), ld,
              B, S, H, Hkv, Dh, int(causal), -1 if window is None else window, out.ptr, nq)
    want = attention_ref(q, k, v, H, Hkv, Dh, causal, window)
    err = row_rel_err(out.numpy(), want)
    assert np.all(err <= 2e-5), f"max row error {err.max():.3e}"


KV_CASES = [
    # B, seq_q, seq_k, H, Hkv, Dh, causal, window: the queries are the last seq_q positions
    (2, 1, 300, 4, 2, 64, True, None),
    (2, 3, 200, 4, 4, 128, True, 50),
    (1, 5, 129, 2, 1, 32, False, None),
    (3, 70, 140, 2, 2, 64, True, None),
    (2, 1, 90, 2, 2, 16, True, 10),
    # up to 8 queries take the decode kernel: a long cache under a window, a
    # window of 0 (one key per query), and 9 queries on the blocked kernel
    (2, 1, 3000, 8, 2, 64, True, 1000),
    (1, 8, 700, 4, 1, 128, False, 0),
    (2, 9, 100, 2, 2, 32, True, None),
]


@pytest.mark.parametrize("B,SQ,SK,H,Hkv,Dh,causal,window", KV_CASES)
def test_attention_kv_core(gpu, B, SQ, SK, H, Hkv, Dh, causal, window):
    # a KV-cache step: seq_q new queries at positions SK - SQ .. SK - 1 over
    # SK cached keys, against float64 attention with the same position masks
    print(f"[case] attention_kv B={B} SQ={SQ} SK={SK} H={H} Hkv={Hkv} Dh={Dh} causal={causal} "
          f"window={window}", flush=True)
    rng = np.random.default_rng(B * 100 + SQ + SK + Dh)
    q = rng.standard_normal((B, SQ, H * Dh)).astype(np.float32)
    k = rng.standard_normal((B, SK, Hkv * Dh)).astype(np.float32)
    v = rng.standard_normal((B, SK, Hkv * Dh)).astype(np.float32)
    d_q, d_k, d_v = DeviceArray.from_numpy(q), DeviceArray.from_numpy(k), DeviceArray.from_numpy(v)
    out = DeviceArray((B, SQ, H * Dh), np.float32)
    q_pos0 = SK - SQ
    _lib.call("enq_attention_kv", d_q.ptr, H * Dh, SQ, SQ, q_pos0, d_k.ptr, Hkv * Dh, d_v.ptr,
              Hkv * Dh, SK, SK, 0, B, H, Hkv, Dh, int(causal), -1 if window is None else window,
              out.ptr, H * Dh)
    qh = q.reshape(B, SQ, H, Dh).transpose(0, 2, 1, 3).astype(np.float64)
    kh = np.repeat(k.reshape(B, SK, Hkv, Dh).transpose(0, 2, 1, 3).astype(np.float64), H // Hkv, 1)
    vh = np.repeat(v.reshape(B, SK, Hkv, Dh).transpose(0, 2, 1, 3).astype(np.float64), H // Hkv, 1)
    s = qh @ kh.transpose(0, 1, 3, 2) / np.sqrt(Dh)
    qpos = q_pos0 + np.arange(SQ)[:, None]
    kpos = np.arange(SK)[None, :]
    allowed = np.ones((SQ, SK), bool)
    if causal:
        allowed &= kpos <= qpos
    if window is not None:
        allowed &= np.abs(qpos - kpos) <= window
    s = np.where(allowed, s, -np.inf)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    want = (p @ vh).transpose(0, 2, 1, 3).reshape(B, SQ, H * Dh)
    err = row_rel_err(out.numpy(), want)
    assert np.all(err <= 2e-5), f"max row error {err.max():.3e}"


def test_attention_rejects_unsupported(gpu):
    d = DeviceArray((4, 3 * 48), np.float32)
    out = DeviceArray((4, 48), np.float32)
    with pytest.raises(NotImplementedError):
        _lib.call("enq_attention", d.ptr, 144, d.ptr, 144, d.ptr, 144, 1, 4, 1, 1, 48, 0, -1,
                  out.ptr, 48)
    with pytest.raises(ValueError):
        _lib.call("enq_attention", d.ptr, 144, d.ptr, 144, d.ptr, 144, 1, 4, 3, 2, 16, 0, -1,
                  out.ptr, 48)


def mha_model(rng, E, H, Hkv=None, causal=False, window=None, std=0.05):
    m = Model()
    kv = (H if Hkv is None else Hkv) * (E // H)
    ws = [(rng.standard_normal(s) * std).astype(np.float32)
          for s in ((E, E), (kv, E), (kv, E), (E, E))]
    biases = {n: (rng.standard_normal(r) * 0.01).astype(np.float32)
              for n, r in (("bq", E), ("bk", kv), ("bv", kv), ("bo", E))}
    m.add_multihead_attention(*ws, num_heads=H, num_kv_heads=Hkv, causal=causal,
                              window_size=window, biases=biases)
    return m


@pytest.mark.parametrize("B,S,E,H,Hkv,causal,window", [
    (2, 40, 64, 4, None, False, None),
    (1, 100, 128, 4, 2, True, None),
    (2, 33, 64, 2, 1, False, 3),
])
def test_mha_layer(gpu, B, S, E, H, Hkv, causal, window):
    print(f"[case] mha B={B} S={S} E={E} H={H} Hkv={Hkv}", flush=True)
    rng = np.random.default_rng(S + E)
    m = mha_model(rng, E, H, Hkv, causal, window)
    ea.quantize_weights(m, per_channel=True)
    x = rng.standard_normal((B, S, E)).astype(np.float32)
    y = m.Forward(x)
    assert y.dtype == np.float64  # scores / np.sqrt(Dh) promote (forward.py:525)
    want = oracle.mha_forward(x.astype(np.float64), m.layers[0])
    err = row_rel_err(y, want)
    assert np.all(err <= 1e-4), f"max row error {err.max():.3e}"
    # the fused QKV cache follows a re-quantized weight
    m.layers[0]["Wv"] = (m.layers[0]["Wv"] * 2).astype(np.float32)
    m.layers[0]["quant"]["Wv"]["scale"] = m.layers[0]["quant"]["Wv"]["scale"] * 2
    y2 = m.Forward(x)
    want2 = oracle.mha_forward(x.astype(np.float64), m.layers[0])
    assert np.all(row_rel_err(y2, want2) <= 1e-4)


def test_mha_window_zero_is_value_path(gpu):
    # test_enilnets.py:7722-7733: window 0 attends to itself only.
    rng = np.random.default_rng(7)
    m = mha_model(rng, 64, 4, window=0)
    ea.quantize_weights(m, per_channel=True)
    L = m.layers[0]
    x = rng.standard_normal((2, 9, 64)).astype(np.float32)
    want = (x.astype(np.float64) @ L["Wv"].T + L["bv"]) @ L["Wo"].T + L["bo"]
    assert np.all(row_rel_err(m.Forward(x), want) <= 1e-4)


def transformer_block(rng, E=128, H=4, hidden=512, std=0.05):
    m = mha_model(rng, E, H, std=std)
    attn = m.layers.pop()
    m.add_residual_start()
    m.add_layernorm(E)
    m.layers.append(attn)
    m.add_residual_end()
    m.add_residual_start()
    m.add_layernorm(E)
    m.add_dense((rng.standard_normal((hidden, E)) * std).astype(np.float32),
                (rng.standard_normal(hidden) * 0.01).astype(np.float32), activation="gelu")
    m.add_dense((rng.standard_normal((E, hidden)) * std).astype(np.float32),
                (rng.standard_normal(E) * 0.01).astype(np.float32), activation="linear")
    m.add_residual_end()
    return m


def test_transformer_block_forward(gpu):
    rng = np.random.default_rng(11)
    m = transformer_block(rng)
    ea.quantize_weights(m, per_channel=True)
    x = rng.standard_normal((2, 64, 128)).astype(np.float32)
    y = m.Forward(x)
    # host dtypes as the reference's NumPy expressions give them
    ref32 = oracle.forward(m.layers, x, dtype=np.float32)
    assert [o.dtype for o in m.outputs] == [o.dtype for o in ref32]
    want = oracle.forward(m.layers, x.astype(np.float64), dtype=np.float64)
    for i, (g, w) in enumerate(zip(m.outputs, want)):
        err = row_rel_err(g, w)
        assert np.all(err <= 1e-4), f"layer {i}: max row error {err.max():.3e}"
    assert y is m.outputs[-1]
