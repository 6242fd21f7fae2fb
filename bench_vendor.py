#!/usr/bin/env python3
"""The vendor library on the GEMM shapes of bench.py, as a reference point.

    python bench_vendor.py

Times, on one GPU through PyTorch (hipBLASLt underneath), the int8 x int8 ->
int32 GEMM with the weight in the same (N, K) layout the W8A8 kernel takes
(``torch._int_mm``, no scales) at 8192^3 and 4096 x 8192 x 8192, and a plain
bf16 linear at 4096 x 8192 x 8192.  Prints one JSON line.  This is not part of
the product path and does not load enilnets_amd: torch brings its own HIP
runtime, which does not initialise in a process that already holds the
library's.
"""

import json

import torch

BF16_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA
INT8_PEAK_TOPS = 5000.0    # dense int8 MFMA


def time_ms(fn, reps=20):
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def main():
    if not torch.cuda.is_available():
        raise SystemExit("bench_vendor: no GPU")
    g = torch.Generator(device="cuda").manual_seed(0)
    out = {}
    for m, n, k in ((8192, 8192, 8192), (4096, 8192, 8192)):
        a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device="cuda", generator=g)
        w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda", generator=g)
        ms = time_ms(lambda: torch._int_mm(a, w.t()))
        tops = 2.0 * m * n * k / ms / 1e9
        out[f"int8_gemm_{m}x{n}x{k}"] = {"ms": ms, "TOP/s": tops,
                                          "frac_int8_peak": tops / INT8_PEAK_TOPS}
        del a, w
    a = torch.randn(4096, 8192, dtype=torch.bfloat16, device="cuda", generator=g)
    w = torch.randn(8192, 8192, dtype=torch.bfloat16, device="cuda", generator=g)
    ms = time_ms(lambda: torch.nn.functional.linear(a, w))
    tf = 2.0 * 4096 * 8192 * 8192 / ms / 1e9
    out["bf16_linear_4096x8192x8192"] = {"ms": ms, "TFLOP/s": tf,
                                         "frac_bf16_peak": tf / BF16_PEAK_TFLOPS}
    del a, w
    # the MLP layer shapes of the headline (batch 4096), bf16 and fp32
    for dt in (torch.bfloat16, torch.float32):
        for n, k in ((1024, 784), (1024, 1024)):
            a = torch.randn(4096, k, dtype=dt, device="cuda", generator=g)
            w = torch.randn(n, k, dtype=dt, device="cuda", generator=g)
            b = torch.randn(n, dtype=dt, device="cuda", generator=g)
            ms = time_ms(lambda: torch.nn.functional.linear(a, w, b), reps=50)
            tf = 2.0 * 4096 * n * k / ms / 1e9
            name = "bf16" if dt == torch.bfloat16 else "fp32"
            out[f"{name}_linear_4096x{n}x{k}"] = {"ms": ms, "TFLOP/s": tf}
    print(json.dumps({"library": f"torch {torch.__version__} (hipBLASLt)", "results": out}))


if __name__ == "__main__":
    main()
