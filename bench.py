#!/usr/bin/env python3
"""Benchmark of Enilnets' quantized-inference hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-components] [--no-cpu]

Headline (``value``): BASELINE.json configs[2], the largest single-GPU
configuration: the W8 Dense of an 8192 x 8192 weight (N(0, 0.02), quantized
per output channel to int8) on M = 4096 fp32 activations (N(0, 1)), on the
fp32-accurate path (per row a power-of-two scale, fp16 high parts and e4m3
low parts of the activations on the fp16 and fp8 matrix cores, one fp32
accumulator).  One step is one Dense call over that batch, inputs resident
in HBM; the metric is the algorithmic TFLOP/s, 2 * M * N * K per step.

``components`` reports the other configs[2] kernels (quantize / dequantize
GB/s, the M=16 GEMV, the bf16 variant, per-token activation quantization and
the W8A8 int8 GEMM at M=4096 and 8192^3), the configs[1] MLP step, the
configs[3] transformer block and the configs[4] MoE layer.  Memory-bound
kernels rotate over enough buffers to exceed the 256 MB MALL, so their bytes
come from HBM.

``roofline`` is the headline's tile GEMM, timed with HIP events on the
library stream around launches of that kernel alone on activations split
beforehand.  ``cpu_baseline`` times the NumPy
oracle (the reference's CPU path, restated) on the host on a bounded sample
of the same workload: the fp32 Dense (BLAS sgemm on the fake-quantized
weight) and the per-channel quantize / dequantize of the 8192 x 8192 weight.
"""

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # dense bf16 MFMA
INT8_PEAK_TOPS = 5000.0        # dense int8 MFMA


def measured_traffic(name, shape, kernel=None):
    """HBM bytes per launch of a kernel, from the rocprofv3 FETCH_SIZE and
    WRITE_SIZE passes summarised in profiles/traffic.json (None if that
    kernel and shape were not profiled)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            entry = json.load(f).get(name)
    except (OSError, ValueError):
        return None
    if not entry or list(entry.get("shape", [])) != list(shape):
        return None
    if kernel is not None and not entry.get("kernel", "").startswith(kernel):
        return None
    return entry.get("bytes_per_launch")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-components", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="", help="comma list of component names (debug)")
    return ap.parse_args()


class Timer:
    """HIP events recorded on the library stream."""

    def __init__(self):
        import ctypes
        from enilnets_amd import _lib
        self._lib, self._ct = _lib, ctypes
        self.a, self.b = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.call("enq_event_create", ctypes.byref(self.a))
        _lib.call("enq_event_create", ctypes.byref(self.b))

    def time(self, fn, reps):
        """Average milliseconds per call over ``reps`` back-to-back calls."""
        self._lib.call("enq_synchronize")
        self._lib.call("enq_event_record", self.a)
        for i in range(reps):
            fn(i)
        self._lib.call("enq_event_record", self.b)
        ms = self._ct.c_float()
        self._lib.call("enq_event_elapsed_ms", self.a, self.b, self._ct.byref(ms))
        return ms.value / reps


def mlp_weights(rng):
    """He-normal weights (n_out, n_in), biases N(0, 0.01)."""
    dims = [(784, 1024), (1024, 1024), (1024, 10)]
    layers = []
    for n_in, n_out in dims:
        w = rng.normal(0.0, np.sqrt(2.0 / n_in), (n_out, n_in)).astype(np.float32)
        b = rng.normal(0.0, 0.01, n_out).astype(np.float32)
        layers.append((w, b))
    return layers


def build_mlp(rng):
    from enilnets_amd import quantize_weights
    from enilnets_amd.nn import Model
    m = Model()
    acts = ["relu", "relu", "linear"]
    for (w, b), act in zip(mlp_weights(rng), acts):
        m.add_dense(w, b, act)
    quantize_weights(m, bits=8, per_channel=True)
    return m


def host_info():
    """The host that runs the CPU baseline: CPU model, logical CPUs, NumPy
    and its BLAS (library, version, threads)."""
    info = {"cpu_model": "unknown", "host_cpus": os.cpu_count(), "numpy": np.__version__,
            "OPENBLAS_NUM_THREADS": os.environ.get("OPENBLAS_NUM_THREADS")}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    info["cpu_model"] = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        from threadpoolctl import threadpool_info
        for i in threadpool_info():
            if i.get("user_api") == "blas":
                info.update(blas=i.get("internal_api"), blas_version=i.get("version"),
                            blas_threads=i.get("num_threads"))
                break
    except Exception:
        pass
    return info


def median_time(fn, budget_s, max_runs):
    """Median seconds of ``fn()`` over up to ``max_runs`` runs within about
    ``budget_s`` seconds (at least one run)."""
    times = []
    t_start = time.perf_counter()
    while len(times) < max_runs and (not times or time.perf_counter() - t_start < budget_s):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_baseline(x, w, fq, codes, scale):
    """The NumPy oracle on the host, on the headline's own inputs: the
    reference's fp32 Dense (``np.dot(x, W.T) + b``, BLAS sgemm, on the
    fake-quantized weight ``fq``) and the reference's per-channel
    ``quantize_tensor`` of ``w`` and ``dequantize`` of its (float) codes.
    About 15 s of host work."""
    import oracle
    M, K = x.shape
    N = w.shape[0]
    layer = {"type": "dense", "weights": fq, "bias": np.zeros(N, np.float32),
             "activation": "linear"}
    oracle.dense_forward(layer, x[:256])                       # warm-up (BLAS threads)
    gemm_s, gemm_n = median_time(lambda: oracle.dense_forward(layer, x), 8.0, 40)
    q_s, q_n = median_time(lambda: oracle.quantize_tensor(w, 8, "symmetric", per_channel=True),
                           4.0, 20)
    fcodes = codes.astype(np.float32)
    zp = np.zeros_like(scale)
    dq_s, dq_n = median_time(lambda: oracle.dequantize(fcodes, scale, zp), 2.0, 40)
    fake_bytes = 8 * N * K + 8 * N          # fp32 in, fp32 out, scale + zero point
    info = host_info()
    return {
        "value": round(2.0 * M * N * K / gemm_s / 1e12, 5), "unit": "TFLOP/s",
        "cores": info.get("blas_threads") or info["host_cpus"], "kind": "port",
        "sample": f"NumPy oracle on the headline's inputs: fp32 Dense {M}x{K} @ {N}x{K}^T "
                  f"(BLAS sgemm on the fake-quantized weight), median of {gemm_n} calls; "
                  f"per-channel quantize_tensor of the {N}x{K} weight, median of {q_n}; "
                  f"dequantize of its float codes, median of {dq_n}",
        "ms_per_step": round(gemm_s * 1e3, 3),
        "quantize_per_channel": {"ms": round(q_s * 1e3, 2), "GB/s": round(fake_bytes / q_s / 1e9, 3),
                                 "bytes": fake_bytes, "threads": 1,
                                 "note": "fake-quantized floats out, as quantization.py:76-93 "
                                         "returns them; NumPy ufuncs run on one core"},
        "dequantize": {"ms": round(dq_s * 1e3, 2), "GB/s": round(fake_bytes / dq_s / 1e9, 3),
                       "bytes": fake_bytes, "threads": 1,
                       "note": "(q - zero_point) * scale on float codes (quantization.py:59-61)"},
        "host": info,
    }


def mlp_step(timer, rng, steps, warmup):
    """the three fused dequant-GEMMs of the MLP at batch
    4096 (fp32-accurate W8), inputs resident in HBM."""
    from enilnets_amd import _lib
    from enilnets_amd.device import DeviceArray
    from enilnets_amd.nn import int8_weights
    from enilnets_amd.nn.dense import dense_w8
    model = build_mlp(rng)
    M = 4096
    x = rng.uniform(0.0, 1.0, (M, 784)).astype(np.float32)
    d_x = DeviceArray.from_numpy(x)
    ws = [int8_weights(l, "weights") for l in model.layers]
    bs = [DeviceArray.from_numpy(l["bias"]) for l in model.layers]
    acts = [l["activation"] for l in model.layers]
    outs = [DeviceArray((M, w.shape[0]), np.float32) for w in ws]

    def step(_=0):
        h = d_x
        for w, b, a, o in zip(ws, bs, acts, outs):
            h = dense_w8(h, w, b, a, variant="fp32", out=o)
        return h

    flops = 2.0 * M * sum(w.shape[0] * w.shape[1] for w in ws)
    step()
    for _ in range(warmup):
        step()
    ms = timer.time(step, steps)
    # the same step captured once as a HIP graph and replayed; each checked
    # replay first clears the output and must give the eager output bit for bit
    import ctypes
    from enilnets_amd.graph import capture
    want = outs[-1].numpy()
    zeros = np.zeros(want.shape, np.float32)
    graph = capture(step)
    try:
        for _ in range(3):
            _lib.call("enq_copy_to_device", outs[-1].ptr, zeros.ctypes.data_as(ctypes.c_void_p),
                      ctypes.c_size_t(zeros.nbytes))
            graph.replay()
            if not np.array_equal(outs[-1].numpy(), want):
                raise RuntimeError("graph replay of the MLP step differs from eager")
            step()
        ms_graph = timer.time(lambda i: graph.replay(), steps)
    finally:
        graph.close()
    # the largest layer's GEMM (4096 x 1024 x 1024), one kernel, timed alone
    big = int(np.argmax([w.shape[0] * w.shape[1] for w in ws]))
    h_in = d_x if big == 0 else outs[big - 1]
    k_ms = timer.time(lambda i: dense_w8(h_in, ws[big], bs[big], acts[big], variant="fp32",
                                         out=outs[big]), max(steps, 20))
    k_flops = 2.0 * M * ws[big].shape[0] * ws[big].shape[1]
    return {"mlp_step_config1": {
        "ms": ms, "TFLOP/s": flops / ms / 1e9, "frac_bf16_peak": flops / ms / 1e9 / BF16_PEAK_TFLOPS,
        "gflop": flops / 1e9, "variant": "fp32",
        "ms_graph_replay": ms_graph, "TFLOP/s_graph_replay": flops / ms_graph / 1e9,
        "largest_layer": {"shape": [M, ws[big].shape[0], ws[big].shape[1]], "ms": k_ms,
                          "TFLOP/s": k_flops / k_ms / 1e9,
                          "frac_bf16_peak": k_flops / k_ms / 1e9 / BF16_PEAK_TFLOPS,
                          "traffic": measured_traffic("mlp_layer_gemm",
                                                      [M, ws[big].shape[0], ws[big].shape[1]])}}}


def headline(args, timer, rng):
    """BASELINE configs[2] at M = 4096: one fp32-accurate W8 Dense call per
    step on the device-resident activations."""
    from enilnets_amd.device import DeviceArray
    from enilnets_amd.nn.dense import dense_w8, quantize_weight_rows
    M, N, K = 4096, 8192, 8192
    w = rng.normal(0.0, 0.02, (N, K)).astype(np.float32)
    wq = rows = quantize_weight_rows(w)
    x = rng.standard_normal((M, K)).astype(np.float32)
    d_x = DeviceArray.from_numpy(x)
    y = DeviceArray((M, N), np.float32)

    def step(_=0):
        dense_w8(d_x, wq, None, "linear", variant="fp32", out=y)

    # correctness guard: 64 rows spread over the batch against float64 math
    # on the fake-quantized weight (the tolerance of the parity tests)
    step()
    codes, scale = rows.codes.numpy(), rows.scale.numpy().reshape(-1, 1)
    fq = codes.astype(np.float32) * scale          # dequantize: the fake-quantized weight
    pick = np.arange(0, M, M // 64)
    ref = x[pick].astype(np.float64) @ fq.astype(np.float64).T
    got = y.numpy()[pick]
    rel = np.max(np.abs(got - ref), axis=1) / np.max(np.abs(ref), axis=1)
    if not np.all(rel <= 1e-4):
        raise SystemExit(f"bench: W8 Dense differs from the oracle (max row error {rel.max():.3e})")
    for _ in range(args.warmup):
        step()
    ms = timer.time(step, args.steps)
    flops = 2.0 * M * N * K
    # the step's two kernels timed alone: the activation split pass (fp16
    # high parts, e4m3 low parts) and the tile GEMM on its output (the
    # dominant kernel)
    from enilnets_amd.nn.dense import dense_w8_split, split_f16f8
    xs = split_f16f8(d_x)
    split_ms = timer.time(lambda i: split_f16f8(d_x), args.steps)
    gemm_ms = timer.time(lambda i: dense_w8_split(xs, wq, None, "linear", out=y), args.steps)
    return {"x": x, "w": w, "fq": fq, "codes": codes, "scale": scale, "m": M, "n": N, "k": K,
            "ms": ms, "flops": flops, "split_ms": split_ms, "gemm_ms": gemm_ms}


def components(timer, rng, only):
    """BASELINE configs[2] kernels."""
    import ctypes
    from enilnets_amd import _lib
    from enilnets_amd.device import DeviceArray, null
    from enilnets_amd.nn.dense import dense_w8, gemm_w8a8, quantize_rows_i8
    from enilnets_amd.nn.weights import Int8Weights
    N = K = 8192
    out = {}
    want = set(only.split(",")) if only else None

    def on(name):
        return want is None or name in want

    # known-size copy: rocprofv3's FETCH_SIZE / WRITE_SIZE of this blit
    # calibrate the traffic counters of the kernels below
    if on("calibration_copy"):
        import ctypes
        nbytes = 256 << 20
        src_c, dst_c = DeviceArray((nbytes,), np.uint8), DeviceArray((nbytes,), np.uint8)
        f = lambda i: _lib.call("enq_copy_on_device", dst_c.ptr, src_c.ptr, ctypes.c_size_t(nbytes))
        ms = timer.time(f, 5)
        out["calibration_copy_256MiB"] = {"ms": ms, "GB/s": 2 * nbytes / ms / 1e6, "bytes": nbytes}
        del src_c, dst_c

    copies = 5   # 5 x 268 MB fp32 or 5 x 67 MB int8 > 256 MB MALL
    w_host = rng.normal(0.0, 0.02, (N, K)).astype(np.float32)
    d_ws = [DeviceArray.from_numpy(w_host) for _ in range(copies)]
    d_codes = [DeviceArray((N, K), np.int8) for _ in range(copies)]
    d_scale = [DeviceArray((N,), np.float32) for _ in range(copies)]
    d_zp = DeviceArray((N,), np.float32)
    nk = N * K

    if on("quantize"):
        def q(i):
            j = i % copies
            _lib.call("enq_quantize_tensor", _lib.F32, d_ws[j].ptr, 1, N, K, 8, _lib.SYMMETRIC,
                      null(), d_codes[j].ptr, d_scale[j].ptr, d_zp.ptr, null())
        q(0)
        ms = timer.time(q, 30)
        nbytes = 4 * nk + nk + 4 * N
        out["quantize_8192x8192_per_channel_int8"] = {
            "ms": ms, "GB/s": nbytes / ms / 1e6, "frac_hbm": nbytes / ms / 1e6 / HBM_PEAK_GBS,
            "bytes": nbytes}
    else:
        for j in range(copies):
            _lib.call("enq_quantize_tensor", _lib.F32, d_ws[j].ptr, 1, N, K, 8, _lib.SYMMETRIC,
                      null(), d_codes[j].ptr, d_scale[j].ptr, d_zp.ptr, null())

    if on("quantize_per_tensor"):
        # one absmax over the whole tensor, then the quantize pass: the
        # reference's two passes (statistics, then quantize) read W twice
        def qt(i):
            j = i % copies
            _lib.call("enq_quantize_tensor", _lib.F32, d_ws[j].ptr, 1, 1, nk, 8, _lib.SYMMETRIC,
                      null(), d_codes[j].ptr, d_scale[j].ptr, d_zp.ptr, null())
        qt(0)
        ms = timer.time(qt, 30)
        nbytes = 2 * 4 * nk + nk + 4
        out["quantize_8192x8192_per_tensor_int8"] = {
            "ms": ms, "GB/s": nbytes / ms / 1e6, "frac_hbm": nbytes / ms / 1e6 / HBM_PEAK_GBS,
            "bytes": nbytes}

    if on("fake_quantize"):
        d_fake = [DeviceArray((N, K), np.float32) for _ in range(2)]

        def fq(i):
            j = i % copies
            _lib.call("enq_quantize_tensor", _lib.F32, d_ws[j].ptr, 1, N, K, 8, _lib.SYMMETRIC,
                      d_fake[i % 2].ptr, null(), d_scale[j].ptr, d_zp.ptr, null())
        fq(0)
        ms = timer.time(fq, 20)
        nbytes = 8 * nk + 8 * N
        out["quantize_tensor_fake_8192x8192"] = {
            "ms": ms, "GB/s": nbytes / ms / 1e6, "frac_hbm": nbytes / ms / 1e6 / HBM_PEAK_GBS,
            "bytes": nbytes}
        del d_fake

    if on("dequantize"):
        def dq(i):
            j = i % copies
            _lib.call("enq_dequantize_i8", _lib.F32, d_codes[j].ptr, 1, N, K, d_scale[j].ptr,
                      d_ws[j].ptr)
        dq(0)
        ms = timer.time(dq, 30)
        nbytes = nk + 4 * N + 4 * nk
        out["dequantize_8192x8192_int8"] = {
            "ms": ms, "GB/s": nbytes / ms / 1e6, "frac_hbm": nbytes / ms / 1e6 / HBM_PEAK_GBS,
            "bytes": nbytes}

    wq = [Int8Weights(d_codes[j], d_scale[j], (N, K), 8, True, None, None) for j in range(copies)]
    del d_ws

    if on("gemv"):
        M = 16
        x = DeviceArray.from_numpy(rng.standard_normal((M, K)).astype(np.float32))
        y = DeviceArray((M, N), np.float32)
        f = lambda i: dense_w8(x, wq[i % copies], None, "linear", out=y)
        f(0)
        ms = timer.time(f, 50)
        nbytes = nk + 4 * M * K + 4 * M * N + 8 * N
        out["gemv_w8_fp32_m16"] = {
            "ms": ms, "GB/s": nbytes / ms / 1e6, "frac_hbm": nbytes / ms / 1e6 / HBM_PEAK_GBS,
            "TFLOP/s": 2 * M * nk / ms / 1e9, "bytes": nbytes}

    M = 4096
    x4 = DeviceArray.from_numpy(rng.standard_normal((M, K)).astype(np.float32))
    y4 = DeviceArray((M, N), np.float32)
    flops = 2.0 * M * nk
    # the fp32-accurate variant at this shape is the headline
    for variant in ("bf16",):
        if on("gemm_" + variant):
            f = lambda i, v=variant: dense_w8(x4, wq[i % 2], None, "linear", variant=v, out=y4)
            f(0)
            ms = timer.time(f, 10)
            tf = flops / ms / 1e9
            out[f"gemm_w8_{variant}_m4096"] = {
                "ms": ms, "TFLOP/s": tf, "frac_bf16_peak": tf / BF16_PEAK_TFLOPS}

    if on("act_quant"):
        xc, xs = quantize_rows_i8(x4)
        f = lambda i: _lib.call("enq_quantize_rows_i8", x4.ptr, M, K, xc.ptr, xs.ptr)
        ms = timer.time(f, 30)
        nbytes = 5 * M * K + 4 * M
        out["per_token_quantize_m4096"] = {
            "ms": ms, "GB/s": nbytes / ms / 1e6, "frac_hbm": nbytes / ms / 1e6 / HBM_PEAK_GBS,
            "bytes": nbytes}

    if on("w8a8"):
        xc, xs = quantize_rows_i8(x4)
        f = lambda i: gemm_w8a8(xc, xs, wq[i % 2], out=y4)
        f(0)
        ms = timer.time(f, 10)
        tops = flops / ms / 1e9
        out["gemm_w8a8_m4096"] = {"ms": ms, "TOP/s": tops, "frac_int8_peak": tops / INT8_PEAK_TOPS}
        del xc, xs
        xsq = DeviceArray.from_numpy(rng.integers(-127, 128, (8192, K), dtype=np.int8))
        ssq = DeviceArray.from_numpy(np.full(8192, 0.01, np.float32))
        ysq = DeviceArray((8192, N), np.float32)
        f = lambda i: gemm_w8a8(xsq, ssq, wq[i % 2], out=ysq)
        f(0)
        ms = timer.time(f, 10)
        tops = 2.0 * 8192 * nk / ms / 1e9
        out["gemm_w8a8_8192cubed"] = {"ms": ms, "TOP/s": tops,
                                      "frac_int8_peak": tops / INT8_PEAK_TOPS}
        del xsq, ysq
    del wq, d_codes, d_scale, x4, y4
    if on("mlp"):
        out.update(mlp_step(timer, rng, 50, 10))
    if on("transformer_block"):
        out.update(transformer_block(timer, rng))
    if on("moe"):
        out.update(moe_layer(timer, rng))
    if on("next_rows"):
        out.update(next_rows(timer, rng))
    return out


def next_rows(timer, rng):
    """The rows built beside the hot path: the activation fake-quantization
    fused into the Dense epilogue, the int8 on-disk format, KV-cache decode
    and the QAT forward.  Device-resident operations are timed with HIP
    events on the library stream; the file and the decode step, whose API
    takes and returns host arrays, with the host clock."""
    import tempfile
    from enilnets_amd import quantize_weights
    from enilnets_amd.device import DeviceArray
    from enilnets_amd.nn import LoadInt8, Model, SaveInt8, int8_weights
    from enilnets_amd.nn.dense import act_quant, dense_w8
    from enilnets_amd.nn.kvcache import KVCache, cached_forward_step
    from enilnets_amd.nn.qat import QATLinear
    out = {}

    # activation fake-quantization (a calibrated per-tensor spec, float64
    # arithmetic as the calibrator's 0-d float64 scale gives) fused into the
    # epilogue of the MLP's 4096 x 1024 x 1024 layer, against the plain layer
    # and the standalone pass over the same output
    M, K, N = 4096, 1024, 1024
    w = rng.normal(0.0, np.sqrt(2.0 / K), (N, K)).astype(np.float32)
    m = Model()
    m.add_dense(w, np.zeros(N, np.float32), "relu")
    quantize_weights(m, bits=8, per_channel=True)
    wq = int8_weights(m.layers[0], "weights")
    x = DeviceArray.from_numpy(rng.uniform(0.0, 1.0, (M, K)).astype(np.float32))
    y, y2 = DeviceArray((M, N), np.float32), DeviceArray((M, N), np.float32)
    spec = {"bits": 8, "scheme": "symmetric", "scale": np.array(0.02),
            "zero_point": np.array(0.0)}
    dense_w8(x, wq, None, "relu", out=y, act_quant=spec)
    act_quant(y, spec, np.float32, out=y2)   # warm-up: the first launch loads the kernel
    plain = timer.time(lambda i: dense_w8(x, wq, None, "relu", out=y), 20)
    fused = timer.time(lambda i: dense_w8(x, wq, None, "relu", out=y, act_quant=spec), 20)
    alone = timer.time(lambda i: act_quant(y, spec, np.float32, out=y2), 20)
    out["act_quant_epilogue_4096x1024x1024"] = {
        "dense_ms": plain, "dense_with_act_quant_ms": fused, "overhead_frac": fused / plain - 1.0,
        "standalone_pass_ms": alone, "standalone_GB/s": 8.0 * M * N / alone / 1e6}

    # QAT forward: per-step per-channel weight fake-quantization feeding the
    # W8 Dense (QATLinear.forward, training=False)
    q = QATLinear.from_weights(w, np.zeros(N, np.float32))
    q.forward(x, training=False)
    ms = timer.time(lambda i: q.forward(x, training=False), 20)
    out["qat_forward_4096x1024x1024"] = {
        "ms": ms, "TFLOP/s": 2.0 * M * N * K / ms / 1e9,
        "note": "weight fake-quant (quantize_tensor per channel) + Dense, per call"}
    del x, y, y2

    # int8 on-disk format of the 8192 x 8192 weight
    big = Model()
    big.add_dense(rng.normal(0.0, 0.02, (8192, 8192)).astype(np.float32),
                  np.zeros(8192, np.float32), "linear")
    quantize_weights(big, bits=8, per_channel=True)
    int8_weights(big.layers[0], "weights")
    with tempfile.TemporaryDirectory() as d:
        f = os.path.join(d, "w8.npz")
        t0 = time.perf_counter()
        info = SaveInt8(big, f)
        t1 = time.perf_counter()
        size = os.path.getsize(f)
        t2 = time.perf_counter()
        LoadInt8(f)
        t3 = time.perf_counter()
    out["int8_file_8192x8192"] = {
        "save_ms": (t1 - t0) * 1e3, "load_ms": (t3 - t2) * 1e3, "file_bytes": size,
        "int8_bytes": info["int8_bytes"], "float_bytes": info["float_bytes"],
        "note": "host clock: npz write / read, codes uploaded and dequantized on the device, "
                "fake-quantized floats copied back"}
    del big

    # KV-cache decode: the configs[3] block made causal, batch 8, a 512-token
    # prompt, then one token per step
    B, S, E, F, H, steps = 8, 512, 1024, 4096, 16, 32
    dec = Model()
    dec.add_residual_start()
    dec.add_layernorm(E)
    ws = [rng.normal(0.0, 0.02, (E, E)).astype(np.float32) for _ in range(4)]
    dec.add_multihead_attention(*ws, num_heads=H, causal=True)
    dec.add_residual_end()
    dec.add_residual_start()
    dec.add_layernorm(E)
    dec.add_dense(rng.normal(0.0, 0.02, (F, E)).astype(np.float32), np.zeros(F, np.float32), "gelu")
    dec.add_dense(rng.normal(0.0, 0.02, (E, F)).astype(np.float32), np.zeros(E, np.float32),
                  "linear")
    dec.add_residual_end()
    quantize_weights(dec, bits=8, per_channel=True)
    prompt = rng.standard_normal((B, S, E)).astype(np.float32)
    new = rng.standard_normal((B, steps + 2, E)).astype(np.float32)
    warm = KVCache()
    cached_forward_step(dec, prompt, warm)
    cached_forward_step(dec, new[:, :1], warm)
    cache = KVCache()
    t0 = time.perf_counter()
    cached_forward_step(dec, prompt, cache)
    t1 = time.perf_counter()
    for i in range(2):
        cached_forward_step(dec, new[:, i:i + 1], cache)
    t2 = time.perf_counter()
    for i in range(2, steps + 2):
        cached_forward_step(dec, new[:, i:i + 1], cache)
    t3 = time.perf_counter()
    step_ms = (t3 - t2) * 1e3 / steps
    # the same session with KVCache(trust_weights=True): no per-step hash of
    # every host weight, device weights, biases and buffers kept
    tcache = KVCache(trust_weights=True)
    cached_forward_step(dec, prompt, tcache)
    for i in range(2):
        cached_forward_step(dec, new[:, i:i + 1], tcache)
    t4 = time.perf_counter()
    for i in range(2, steps + 2):
        cached_forward_step(dec, new[:, i:i + 1], tcache)
    t5 = time.perf_counter()
    trusted_ms = (t5 - t4) * 1e3 / steps
    weight_bytes = 4 * E * E + 2 * E * F
    out["kv_decode_b8_ctx512_e1024"] = {
        "prefill_ms": (t1 - t0) * 1e3, "ms_per_step": step_ms, "tokens/s": B / step_ms * 1e3,
        "ms_per_step_trusted_weights": trusted_ms, "tokens/s_trusted_weights": B / trusted_ms * 1e3,
        "weight_bytes_per_step": weight_bytes,
        "kv_bytes_per_step": 2 * B * (S + steps) * E * 4,
        "note": "host clock per cached_forward_step: host dispatch of every layer, the device "
                "work and the copy of the new positions' outputs back"}
    return out


def transformer_block(timer, rng):
    """one pre-norm transformer block on x (8, 512,
    1024), 16 heads of 64, FFN 4096 with GELU, weights N(0, 0.02) quantized
    per output channel, zero biases, LayerNorm gamma 1 beta 0.  The metric
    counts the weight GEMMs only (QKV, O, FFN1, FFN2: 103.08 GFLOP); the fp32
    attention core (8.59 GFLOP) is timed on its own as well."""
    from enilnets_amd import _lib, quantize_weights
    from enilnets_amd.device import DeviceArray
    from enilnets_amd.nn import Model, int8_weights
    from enilnets_amd.nn import transformer as T
    from enilnets_amd.nn.dense import dense_w8_ffn, ffn_bound
    B, S, E, F, H = 8, 512, 1024, 4096, 16
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
    quantize_weights(m, bits=8, per_channel=True)
    L = m.layers
    x = DeviceArray.from_numpy(rng.standard_normal((B, S, E)).astype(np.float32))
    ln1, ln2 = T.layernorm_params(L[1]), T.layernorm_params(L[5])
    plan = T.MhaPlan(L[2], B, S)
    w1, w2 = int8_weights(L[6], "weights"), int8_weights(L[7], "weights")
    b1, b2 = DeviceArray.from_numpy(L[6]["bias"]), DeviceArray.from_numpy(L[7]["bias"])
    t1, a1, r1, t2, f2, y = (DeviceArray((B, S, E), np.float32) for _ in range(6))
    fb = ffn_bound(w1, b1, "gelu")

    def block(_=0):
        T.layernorm(x, L[1], out=t1, params=ln1)
        T.mha_forward(t1, L[2], plan=plan, out=a1)
        T.residual_add(a1, x, out=r1)
        T.layernorm(r1, L[5], out=t2, params=ln2)
        # the FFN pair: the first GEMM writes the second's fp16/e4m3 split,
        # with FFN1's output bound computed once, as the weights are quantized
        dense_w8_ffn(t2, w1, b1, "gelu", w2, b2, "linear", out=f2, bound=fb)
        T.residual_add(f2, r1, out=y)

    block()
    ms = timer.time(block, 10)
    flops = 2.0 * B * S * (3 * E * E + E * E + E * F + F * E)
    # the same block captured once as a HIP graph and replayed (one launch
    # instead of a host dispatch per kernel); each checked replay first
    # clears the output and must give the eager output bit for bit
    import ctypes
    from enilnets_amd.graph import capture
    want = y.numpy()
    zeros = np.zeros(want.shape, np.float32)
    graph = capture(block)
    try:
        for _ in range(3):
            _lib.call("enq_copy_to_device", y.ptr, zeros.ctypes.data_as(ctypes.c_void_p),
                      ctypes.c_size_t(zeros.nbytes))
            graph.replay()
            if not np.array_equal(y.numpy(), want):
                raise RuntimeError("graph replay of the transformer block differs from eager")
            block()
        ms_graph = timer.time(lambda i: graph.replay(), 10)
    finally:
        graph.close()
    res = {"transformer_block_b8_s512_e1024": {
        "ms": ms, "TFLOP/s": flops / ms / 1e9, "frac_bf16_peak": flops / ms / 1e9 / BF16_PEAK_TFLOPS,
        "weight_gflop": flops / 1e9, "variant": "fp32",
        "ms_graph_replay": ms_graph, "TFLOP/s_graph_replay": flops / ms_graph / 1e9,
        "note": "ms: eager calls from Python; ms_graph_replay: the same calls captured once "
                "(enq_graph_*) and replayed"}}
    n_all = plan.wqkv.shape[0]

    def core(_=0):
        _lib.call("enq_attention", plan.qkv.ptr, n_all, T._at(plan.qkv, 4 * E), n_all,
                  T._at(plan.qkv, 8 * E), n_all, B, S, H, H, E // H, 0, -1, plan.ctx.ptr, E)

    core()
    ms = timer.time(core, 20)
    aflops = 4.0 * B * H * S * S * (E // H)
    # fp32-accurate products as six bf16 part products each: the kernel's own
    # matrix ceiling is a sixth of the bf16 peak (417 TFLOP/s of fp32 work)
    res["attention_core_b8_s512_h16_d64"] = {
        "ms": ms, "TFLOP/s": aflops / ms / 1e9,
        "frac_bf16_peak": aflops / ms / 1e9 / BF16_PEAK_TFLOPS,
        "frac_of_ceiling": aflops / ms / 1e9 / (BF16_PEAK_TFLOPS / 6),
        "note": "each fp32 product as six bf16 MFMA part products (three-part bf16 split of Q, K, P, V)"}
    return res


def moe_layer(timer, rng):
    """8192 tokens x 1024, router logits (8192, 8)
    N(0, 1) given, top-2 with raw-probability gates, W1 (8, 4096, 1024) and
    W2 (8, 1024, 4096) N(0, 0.02) quantized per output channel within each
    expert slice, zero biases, GELU; 274.88 GFLOP per call."""
    from enilnets_amd.device import DeviceArray
    from enilnets_amd.nn import Int8Weights
    from enilnets_amd.nn.dense import quantize_weight_rows
    from enilnets_amd.nn.moe import moe_bound, moe_forward
    T_, D, Hd, E_, K_ = 8192, 1024, 4096, 8, 2
    layer = {"type": "moe", "embed_dim": D, "num_experts": E_, "hidden_dim": Hd, "top_k": K_,
             "activation": "gelu"}
    weights = []
    for shape in ((E_, Hd, D), (E_, D, Hd)):
        w = rng.normal(0.0, 0.02, shape).astype(np.float32)
        rows = quantize_weight_rows(w.reshape(-1, shape[2]))  # per row of each expert slice
        weights.append(Int8Weights(rows.codes, rows.scale, shape, 8, True, None, None))
        del w
    x = DeviceArray.from_numpy(rng.standard_normal((T_, D)).astype(np.float32))
    logits = DeviceArray.from_numpy(rng.standard_normal((T_, E_)).astype(np.float32))
    y = DeviceArray((T_, D), np.float32)
    # the first expert layer's output bound, computed once with the weights
    bound = moe_bound(layer, weights[0], None)
    _, info = moe_forward(x, layer, router_logits=logits, want_routing=True, out=y,
                          biases=(None, None, None), aux_loss=False,
                          weights=(weights[0], weights[1], None), bound=bound)
    counts = np.bincount(info["top_idx"].numpy().reshape(-1), minlength=E_)
    f = lambda i: moe_forward(x, layer, router_logits=logits, out=y, biases=(None, None, None),
                              aux_loss=False, weights=(weights[0], weights[1], None),
                              bound=bound)
    ms = timer.time(f, 5)
    flops = 2.0 * T_ * K_ * D * Hd * 2
    return {"moe_t8192_e8_top2_d1024_h4096": {
        "ms": ms, "TFLOP/s": flops / ms / 1e9, "frac_bf16_peak": flops / ms / 1e9 / BF16_PEAK_TFLOPS,
        "gflop": flops / 1e9, "rows_per_expert": counts.tolist(), "variant": "fp32"}}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): this build measures the "
              "one-GPU path; sharding across GPUs is described in DESIGN.md, not run.",
              file=sys.stderr)
        return 2
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from enilnets_amd import _lib
    _lib.lib()
    info = _lib.device_info()
    print(f"[bench] device {info.name.decode()} {info.arch.decode()} CUs={info.compute_units}",
          file=sys.stderr, flush=True)
    rng = np.random.default_rng(0)
    timer = Timer()
    h = headline(args, timer, rng)
    ms, flops = h["ms"], h["flops"]
    print(f"[bench] configs[2] W8 GEMM {ms:.4f} ms", file=sys.stderr, flush=True)
    value = flops / ms / 1e9
    shape = [h["m"], h["n"], h["k"]]
    result = {
        "metric": "W8 Dense GEMM TFLOP/s (BASELINE configs[2]: 4096 x 8192 x 8192, "
                  "fp32-accurate W8)",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights x fp32 activations (fp16 hi + e4m3 lo MFMA, fp32 accumulate)",
        "data": "synthetic (seeded N(0, 0.02) weight quantized per output channel, "
                "N(0, 1) activations)",
        "config": {"workload": "configs[2]: Dense 8192x8192 int8 weight (per output channel), "
                               "M=4096 fp32 activations, no bias, linear",
                   "m": h["m"], "n": h["n"], "k": h["k"], "variant": "fp32",
                   "flops_per_step": flops},
        "roofline": {"bound": "mfma",
                     "kernel": "w8_f8_ring_kernel<F8RingCfg<256,256,4,2,2>>",
                     "shape": shape,
                     "achieved": round(flops / h["gemm_ms"] / 1e9, 3), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s",
                     "frac": round(flops / h["gemm_ms"] / 1e9 / BF16_PEAK_TFLOPS, 4),
                     "kernel_ms": round(h["gemm_ms"], 5),
                     "split_pass_ms": round(h["split_ms"], 5),
                     "traffic": measured_traffic("w8_gemm_config2", shape, "w8_f8_ring_kernel<F8RingCfg<256,256,4,2,2>"),
                     "note": "algorithmic 2*M*N*K over the HIP-event time of the tile GEMM "
                             "launched alone on pre-split activations (enq_gemm_w8_f16f8); a "
                             "step is the split pass (fp32 -> fp16 hi + e4m3 lo, per-row "
                             "power-of-two exponent) plus this kernel. Per 64-deep step the "
                             "kernel issues 4 fp16 and 1 fp8 MFMAs per 32x32 block (1.5 bf16-"
                             "MFMA equivalents per product), so its own ceiling is 2/3 of the "
                             "bf16 peak"},
    }
    if not args.no_components:
        result["components"] = components(timer, rng, args.only)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(h["x"], h["w"], h["fq"], h["codes"], h["scale"])
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
