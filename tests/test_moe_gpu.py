"""GPU parity of the mixture-of-experts layer (``Enilnets/nn/moe.py:52-87``).

* Routing from given logits: expert choices identical to the oracle's
  ``argsort(-probs)[:, :k]``; probabilities within 1e-6 relative (exp and
  the sum order differ from NumPy's by a few float32 ulps).
* Layer output: max |y - y_ref| <= 1e-4 * max |y_ref| per token against the
  float64 oracle on the fake-quantized expert weights, with the oracle routed
  by the same probabilities (a float64 router can order near-equal
  probabilities differently than any float32 one).
* With the int8 router (a W8 Dense, logits within delta = 1e-4 * max |logit|
  per token): each router probability p within 2.5 p delta of the oracle's;
  tokens whose k-th and (k+1)-th oracle probabilities are closer than twice
  the sum of their bounds are excluded from the output comparison, since a
  router-side rounding difference may legitimately pick the other expert
  there.
* The dense-mixture invariant of ``test_enilnets.py:8331-8353``.
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


def softmax32(logits):
    z = logits - logits.max(axis=-1, keepdims=True)
    e = np.exp(z)
    return e / e.sum(axis=-1, keepdims=True)


def moe_model(rng, d, hidden, experts, top_k, activation="gelu", std=0.05, per_row=False):
    m = Model()
    w1 = (rng.standard_normal((experts, hidden, d)) * std).astype(np.float32)
    w2 = (rng.standard_normal((experts, d, hidden)) * std).astype(np.float32)
    wr = (rng.standard_normal((experts, d)) / np.sqrt(d)).astype(np.float32)
    b1 = (rng.standard_normal((experts, hidden)) * 0.01).astype(np.float32)
    b2 = (rng.standard_normal((experts, d)) * 0.01).astype(np.float32)
    m.add_moe(w1, w2, wr, top_k=top_k, activation=activation, b1=b1, b2=b2)
    if per_row:
        # one scale per output row of every expert slice
        L = m.layers[0]
        L["quant"] = {}
        for name in ("W1", "W2"):
            fq, sc = [], []
            for e in range(experts):
                f, s, _ = oracle.quantize_tensor(L[name][e], 8, per_channel=True)
                fq.append(f)
                sc.append(s)
            L[name] = np.stack(fq)
            L["quant"][name] = {"bits": 8, "scheme": "symmetric", "scale": np.stack(sc),
                                "zero_point": np.zeros_like(np.stack(sc))}
        f, s, z = oracle.quantize_tensor(L["Wr"], 8, per_channel=True)
        L["Wr"] = f
        L["quant"]["Wr"] = {"bits": 8, "scheme": "symmetric", "scale": s, "zero_point": z}
    else:
        ea.quantize_weights(m, per_channel=True)
    return m


@pytest.mark.parametrize("tokens,experts,top_k", [(8192, 8, 2), (1000, 4, 1), (37, 16, 4),
                                                  (5, 3, 3), (300, 32, 5), (200, 40, 3),
                                                  (20000, 8, 2)])
def test_routing_from_logits(gpu, tokens, experts, top_k):
    print(f"[case] routing tokens={tokens} experts={experts} k={top_k}", flush=True)
    rng = np.random.default_rng(tokens + experts)
    m = moe_model(rng, 32, 48, experts, top_k)
    logits = rng.standard_normal((tokens, experts)).astype(np.float32)
    x = rng.standard_normal((tokens, 32)).astype(np.float32)
    out, info = moe_forward(DeviceArray.from_numpy(x), m.layers[0],
                            router_logits=DeviceArray.from_numpy(logits), want_routing=True)
    probs = softmax32(logits)
    got_p = info["probs"].numpy()
    assert np.all(np.abs(got_p - probs) <= 1e-6 * probs)
    assert np.array_equal(info["top_idx"].numpy(), oracle.top_k(probs, top_k))
    want = oracle.moe_forward(x.astype(np.float64), m.layers[0], probs=probs.astype(np.float64))
    err = row_rel_err(out.numpy(), want)
    assert np.all(err <= 1e-4), f"max row error {err.max():.3e}"


def test_routing_ties_take_lower_index(gpu):
    rng = np.random.default_rng(5)
    m = moe_model(rng, 16, 16, 4, 2)
    logits = np.zeros((3, 4), np.float32)
    logits[1] = [1.0, 2.0, 2.0, 2.0]
    logits[2] = [3.0, 0.0, 3.0, 0.0]
    x = rng.standard_normal((3, 16)).astype(np.float32)
    _, info = moe_forward(DeviceArray.from_numpy(x), m.layers[0],
                          router_logits=DeviceArray.from_numpy(logits), want_routing=True)
    assert info["top_idx"].numpy().tolist() == [[0, 1], [1, 2], [0, 2]]


@pytest.mark.parametrize("tokens,d,hidden,experts,top_k,per_row", [
    (2048, 1024, 4096, 8, 2, True),
    (700, 64, 256, 8, 2, False),
    (300, 20, 30, 4, 2, False),     # K not a multiple of 16: per-expert Dense calls
    (129, 48, 80, 5, 1, True),
])
def test_moe_layer_with_router(gpu, tokens, d, hidden, experts, top_k, per_row):
    print(f"[case] moe tokens={tokens} d={d} hidden={hidden} E={experts} k={top_k}", flush=True)
    rng = np.random.default_rng(tokens + d)
    m = moe_model(rng, d, hidden, experts, top_k, per_row=per_row)
    L = m.layers[0]
    x = rng.standard_normal((tokens, d)).astype(np.float32)
    out, info = moe_forward(DeviceArray.from_numpy(x), L, want_routing=True)
    x64 = x.astype(np.float64)
    logits_ref, p_ref = oracle.router(x64, L)
    # the router is a W8 Dense: logits within delta = 1e-4 * max |logit| per
    # token, which moves each probability p by at most about 2 p delta
    delta = 1e-4 * np.max(np.abs(logits_ref), axis=-1, keepdims=True)
    bound = 2.5 * p_ref * delta + 1e-7
    assert np.all(np.abs(info["probs"].numpy() - p_ref) <= bound)
    order = np.argsort(-p_ref, axis=-1)
    srt = np.take_along_axis(p_ref, order, axis=-1)
    b_srt = np.take_along_axis(bound, order, axis=-1)
    clear = ((srt[:, top_k - 1] - srt[:, top_k] > 2 * (b_srt[:, top_k - 1] + b_srt[:, top_k]))
             if top_k < experts else np.ones(tokens, bool))
    want = oracle.moe_forward(x64, L)
    err = row_rel_err(out.numpy()[clear], want[clear])
    assert clear.mean() > 0.95
    assert np.all(err <= 1e-4), f"max row error {err.max():.3e}"
    # load-balancing loss (moe.py:38-49) from the oracle's routing
    top = oracle.top_k(p_ref, top_k)
    f = np.bincount(top[:, 0], minlength=experts) / tokens
    want_loss = experts * np.sum(f * p_ref.mean(axis=0))
    assert abs(info["aux_loss"] - want_loss) <= 1e-4 * max(1.0, abs(want_loss))
    if d % 16 == 0:
        # the first layer's output bound computed once gives the same output
        from enilnets_amd.nn.moe import moe_biases, moe_bound
        from enilnets_amd.nn.weights import int8_weights
        bnd = moe_bound(L, int8_weights(L, "W1"), moe_biases(L)[0])
        out2, _ = moe_forward(DeviceArray.from_numpy(x), L, bound=bnd)
        assert np.array_equal(out2.numpy(), out.numpy())


def test_moe_empty_experts(gpu):
    # logits that send every token to experts 1 and 3: the other groups are
    # empty and their tiles must not write anything
    rng = np.random.default_rng(9)
    m = moe_model(rng, 64, 128, 6, 2)
    logits = np.full((500, 6), -10.0, np.float32)
    logits[:, 1] = 2.0
    logits[:, 3] = 1.0 + rng.standard_normal(500).astype(np.float32) * 0.01
    x = rng.standard_normal((500, 64)).astype(np.float32)
    out, _ = moe_forward(DeviceArray.from_numpy(x), m.layers[0],
                         router_logits=DeviceArray.from_numpy(logits))
    probs = softmax32(logits)
    want = oracle.moe_forward(x.astype(np.float64), m.layers[0], probs=probs.astype(np.float64))
    assert np.all(row_rel_err(out.numpy(), want) <= 1e-4)


@pytest.mark.parametrize("activation", ["gelu", "relu", "sigmoid", "selu"])
def test_moe_split_rows_of_every_kind(gpu, activation):
    # the fp32 layer's fp16 / e4m3 path (hidden a multiple of 64): token rows
    # of very different scales and shapes, and expert weights with one
    # 50-sigma entry per output channel (per-row scales), all within the
    # Dense bound.  The hidden rows' exponents come from a bound on them, so
    # these are the rows where a loose bound would lose the low parts.
    print(f"[case] moe split rows activation={activation}", flush=True)
    rng = np.random.default_rng(17)
    experts, d, hidden, tokens = 4, 128, 256, 600
    m = Model()
    w1 = (rng.standard_normal((experts, hidden, d)) * 0.02).astype(np.float32)
    w2 = (rng.standard_normal((experts, d, hidden)) * 0.02).astype(np.float32)
    for w in (w1, w2):
        e_i, n_i = np.meshgrid(np.arange(w.shape[0]), np.arange(w.shape[1]), indexing="ij")
        w[e_i, n_i, rng.integers(0, w.shape[2], w.shape[:2])] = 1.0
    wr = (rng.standard_normal((experts, d)) / np.sqrt(d)).astype(np.float32)
    b1 = (rng.standard_normal((experts, hidden)) * 0.01).astype(np.float32)
    b2 = (rng.standard_normal((experts, d)) * 0.01).astype(np.float32)
    m.add_moe(w1, w2, wr, top_k=2, activation=activation, b1=b1, b2=b2)
    L = m.layers[0]
    L["quant"] = {}
    for name in ("W1", "W2"):
        fq, sc = [], []
        for e in range(experts):
            f, s, _ = oracle.quantize_tensor(L[name][e], 8, per_channel=True)
            fq.append(f)
            sc.append(s)
        L[name] = np.stack(fq)
        L["quant"][name] = {"bits": 8, "scheme": "symmetric", "scale": np.stack(sc),
                            "zero_point": np.zeros_like(np.stack(sc))}
    x = rng.standard_normal((tokens, d))
    kinds = np.arange(tokens) % 6
    x[kinds == 1] *= 1e-6
    x[kinds == 2] *= 1e-30
    x[kinds == 3] = rng.standard_cauchy((int(np.sum(kinds == 3)), d))
    x[kinds == 4] *= np.exp(rng.normal(0.0, 3.0, (int(np.sum(kinds == 4)), d)))
    x[kinds == 5, :4] *= 1000.0
    x = x.astype(np.float32)
    logits = rng.standard_normal((tokens, experts)).astype(np.float32)
    out, _ = moe_forward(DeviceArray.from_numpy(x), L,
                         router_logits=DeviceArray.from_numpy(logits))
    probs = softmax32(logits)
    want = oracle.moe_forward(x.astype(np.float64), L, probs=probs.astype(np.float64))
    err = row_rel_err(out.numpy(), want)
    assert np.all(err <= 1e-4), f"max row error {err.max():.3e} (row kind {kinds[np.argmax(err)]})"


@pytest.mark.parametrize("d,hidden", [(64, 256), (48, 80)])
def test_moe_layer_bf16(gpu, d, hidden):
    # the bf16 variant (one plane per activation); hidden 256 has the first
    # GEMM write the second's plane itself, hidden 80 (padded to 96) splits
    # it in a separate pass.  Router logits are given, so the routing is the
    # oracle's; rows within the bf16 Dense bound.
    print(f"[case] moe bf16 d={d} hidden={hidden}", flush=True)
    rng = np.random.default_rng(d + hidden)
    m = moe_model(rng, d, hidden, 8, 2)
    logits = rng.standard_normal((700, 8)).astype(np.float32)
    x = rng.standard_normal((700, d)).astype(np.float32)
    out, _ = moe_forward(DeviceArray.from_numpy(x), m.layers[0], variant="bf16",
                         router_logits=DeviceArray.from_numpy(logits))
    probs = softmax32(logits)
    want = oracle.moe_forward(x.astype(np.float64), m.layers[0], probs=probs.astype(np.float64))
    err = row_rel_err(out.numpy(), want)
    assert np.all(err <= 2e-2), f"max row error {err.max():.3e}"


@pytest.mark.parametrize("top_k", [1, 2, 4])
def test_dense_mixture_invariant(gpu, top_k):
    # test_enilnets.py:8331-8353: every expert on every token densely, gated
    # by the top-k mask, equals the routed layer.
    rng = np.random.default_rng(top_k)
    m = moe_model(rng, 32, 64, 4, top_k)
    L = m.layers[0]
    x = rng.standard_normal((2, 50, 32)).astype(np.float32)
    y = m.Forward(x)
    assert y.shape == x.shape and y.dtype == np.float32
    flat = x.reshape(-1, 32).astype(np.float64)
    _, info = moe_forward(DeviceArray.from_numpy(x), L, want_routing=True)
    p = info["probs"].numpy().astype(np.float64)
    order = info["top_idx"].numpy()
    ref = np.zeros_like(flat)
    for e in range(4):
        h = oracle.activate("gelu", flat @ L["W1"][e].T.astype(np.float64) + L["b1"][e])
        ye = h @ L["W2"][e].T.astype(np.float64) + L["b2"][e]
        picked = (order == e).any(axis=-1)
        ref += (p[:, e] * picked)[:, None] * ye
    assert np.all(row_rel_err(y.reshape(-1, 32), ref) <= 1e-4)
    assert isinstance(L["_state_aux_loss"], float)


def test_moe_validation(gpu):
    rng = np.random.default_rng(1)
    m = moe_model(rng, 16, 16, 4, 2)
    x = DeviceArray.from_numpy(rng.standard_normal((4, 16)).astype(np.float32))
    L = dict(m.layers[0], activation="softmax")
    with pytest.raises(NotImplementedError):
        moe_forward(x, L)
    with pytest.raises(ValueError):
        moe_forward(DeviceArray.from_numpy(np.zeros((4, 8), np.float32)), m.layers[0])
