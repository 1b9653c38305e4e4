"""hip_gemm benchmark driver (the analogue of specializations/cpu_gemm/runner.py).

benchmark_gemm times one plan on the GPU the way runner.py:111-232 times an
emitted C kernel (warm-up, then timed runs, the numpy reference timed on the
same inputs, a correctness check) and returns the same keys (gpu_time_ms in
place of c_time_ms, cpu_time_ms in place of numpy_time_ms, speedup,
correct) plus throughput and roofline figures.

Timing protocol: HIP events recorded on the stream the kernel is launched
on, one event pair per launch; median, min and p90 over num_runs launches
after `warmup` untimed ones. With rotate=True the launches cycle through
several distinct input/output buffer sets whose total exceeds the 256 MB
Infinity Cache, so a timed launch does not find its operands cached.
"""
from __future__ import annotations

import statistics

from .backend import (HipGemmError, PEAK_HBM_BYTES, PEAK_INT8_OPS, _operand_shapes,
                      algorithmic_bytes, run, validate_plan)

MALL_BYTES = 256 * 1024 * 1024


def _device_inputs(plan, inputs, device, seed):
    import torch
    a_shape, b_shape, c_shape = _operand_shapes(plan)
    if inputs is not None:
        A = torch.as_tensor(inputs["A"]).reshape(a_shape).to(device)
        B = torch.as_tensor(inputs["B"]).reshape(b_shape).to(device)
        D = inputs.get("D")
        D = torch.as_tensor(D).reshape(c_shape).to(device) if D is not None else None
        return A, B, D
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    A = torch.randint(-128, 128, a_shape, dtype=torch.int8, device=device, generator=g)
    B = torch.randint(-128, 128, b_shape, dtype=torch.int8, device=device, generator=g)
    D = None
    if plan["has_d"]:
        lim = plan["d_max_abs"]
        D = torch.randint(-lim, lim + 1, c_shape, dtype=torch.int32, device=device, generator=g)
    return A, B, D


def _percentile(xs, q):
    xs = sorted(xs)
    idx = min(len(xs) - 1, max(0, int(round(q * (len(xs) - 1)))))
    return xs[idx]


def _cpu_reference(A, B, D, budget_s):
    """Time the numpy reference of runner.py:206-214 on this problem.

    The product is (D + A @ B) computed in int64 and cast to int32, numpy's
    integer matmul (one thread: numpy has no BLAS for integers). It runs over
    the first rows of the first batch, as many as fit the time budget (all
    of them for small problems), and the time is scaled by the share of rows
    run. Returns (ms for the whole problem, rows run, rows in total, the
    int32 output of the rows run, seconds spent).
    """
    import numpy as np
    a = A.cpu().numpy()
    b = B.cpu().numpy()
    d = None if D is None else D.cpu().numpy()
    batched = a.ndim == 3
    a0 = a[0] if batched else a
    b0 = b[0] if (b.ndim == 3) else b
    d0 = None if d is None else (d[0] if batched else d)
    m = a0.shape[0]
    total_rows = m * (a.shape[0] if batched else 1)
    b64 = b0.astype(np.int64)

    def rows(r0, r1):
        out = a0[r0:r1].astype(np.int64) @ b64
        if d0 is not None:
            out = out + d0[r0:r1]
        return out.astype(np.int32)

    import time
    t0 = time.perf_counter()
    first = rows(0, 1)
    t1 = time.perf_counter() - t0
    n = max(1, min(m, int(budget_s / max(t1, 1e-6))))
    if n > 1:
        t0 = time.perf_counter()
        out = rows(0, n)
        t = time.perf_counter() - t0
    else:
        out, t = first, t1
    ms = t * 1e3 * total_rows / n
    return ms, n, total_rows, out, t


def benchmark_gemm(plan, num_runs=20, *, warmup=3, inputs=None, seed=0, rotate=True,
                   cpu_budget_s=2.0, device=None):
    """Time `plan` on the GPU; returns timing, correctness, CPU baseline,
    throughput and roofline figures.

    Follows runner.py:111-232: warm-up and timed runs, then the numpy
    reference timed on the same inputs, and the keys of its result
    (gpu_time_ms in place of c_time_ms, cpu_time_ms in place of
    numpy_time_ms, speedup = cpu / gpu, correct). `correct` is always
    computed: the output of the first launch must pass verify.exact_check (an
    exact projection check of every element, on the GPU) and equal the numpy
    reference on every row the reference ran. The reference runs the whole
    problem when it fits `cpu_budget_s` seconds, else the first rows that
    fit, scaled to the whole problem (cpu_extrapolated True).

    inputs: optional dict(A, B, D) of numpy arrays/tensors (else seeded
    random); for the skinny_packed variant B is given row-major and packed
    once per buffer set before timing (pack_ms).
    """
    import torch
    from . import verify
    from .backend import PACKED_VARIANT, pack_b
    ok, reason = validate_plan(plan)
    if not ok:
        raise HipGemmError("invalid plan: " + reason)
    if not torch.cuda.is_available():
        raise HipGemmError("no GPU available: hip_gemm has no CPU path")
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    packed = plan["variant"] == PACKED_VARIANT
    A, B, D = _device_inputs(plan, inputs, device, seed)
    a_shape, b_shape, c_shape = _operand_shapes(plan)
    set_bytes = A.numel() + B.numel() + 4 * (2 if D is not None else 1) * \
        int(torch.Size(c_shape).numel())
    n_sets = 1
    if rotate:
        n_sets = max(1, min(16, -(-2 * MALL_BYTES // set_bytes)))
    sets = [(A, B, D, torch.empty(c_shape, dtype=torch.int32, device=device))]
    for _ in range(n_sets - 1):
        sets.append((A.clone(), B.clone(), D.clone() if D is not None else None,
                     torch.empty(c_shape, dtype=torch.int32, device=device)))
    stream = torch.cuda.current_stream(device)
    raw = stream.cuda_stream
    pack_ms = None
    if packed:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        pb = [pack_b(s[1], stream=raw) for s in sets]
        e1.record(stream)
        torch.cuda.synchronize(device)
        pack_ms = e0.elapsed_time(e1) / len(sets)
        sets = [(s[0], p, s[2], s[3]) for s, p in zip(sets, pb)]

    # Poison, run once, check: INT32_MIN everywhere first, so an output the
    # kernel fails to write cannot pass.
    sets[0][3].fill_(-2**31)
    out0 = run(plan, *sets[0][:3], out=sets[0][3], stream=raw)
    torch.cuda.synchronize(device)
    try:
        chk = verify.exact_check(A, B, out0, D)
        check_method, check_ok = chk["method"], chk["passed"]
    except verify.VerifyError as exc:
        check_method, check_ok = "not applicable: %s" % exc, True
    cpu_ms, cpu_rows, total_rows, cpu_out, _ = _cpu_reference(A, B, D, cpu_budget_s)
    import numpy as np
    gpu_rows = (out0[0] if out0.dim() == 3 else out0)[:cpu_rows].cpu().numpy()
    rows_equal = bool(np.array_equal(gpu_rows, cpu_out))
    correct = bool(check_ok and rows_equal)

    for i in range(warmup):
        s = sets[i % n_sets]
        run(plan, s[0], s[1], s[2], out=s[3], stream=raw)
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(num_runs)]
    torch.cuda.synchronize(device)
    for i, (e0, e1) in enumerate(events):
        s = sets[(warmup + i) % n_sets]
        e0.record(stream)
        run(plan, s[0], s[1], s[2], out=s[3], stream=raw)
        e1.record(stream)
    torch.cuda.synchronize(device)
    times = [e0.elapsed_time(e1) for e0, e1 in events]
    med = statistics.median(times)
    ops = 2 * plan["batch"] * plan["m"] * plan["n"] * plan["k"]
    alg = algorithmic_bytes(plan)
    sec = med / 1e3
    tops = ops / sec / 1e12
    gbps = alg / sec / 1e9
    return {
        "plan": plan,
        "gpu_time_ms": med,
        "gpu_time_ms_min": min(times),
        "gpu_time_ms_p90": _percentile(times, 0.9),
        "num_runs": num_runs,
        "warmup": warmup,
        "rotated_sets": n_sets,
        "pack_ms": pack_ms,
        "cpu_time_ms": cpu_ms,
        "cpu_reference": "numpy int64 matmul then int32 cast, 1 thread",
        "cpu_rows": cpu_rows,
        "cpu_extrapolated": cpu_rows < total_rows,
        "speedup": cpu_ms / med if med > 0 else 0.0,   # runner.py:228
        "correct": correct,
        "check": {"method": check_method, "passed": check_ok,
                  "cpu_rows_equal": rows_equal, "cpu_rows_compared": cpu_rows},
        "ops": ops,
        "bytes_algorithmic": alg,
        "tops": tops,
        "gbps": gbps,
        "roofline": {
            "int8_frac": ops / sec / PEAK_INT8_OPS,
            "hbm_frac": alg / sec / PEAK_HBM_BYTES,
            "bound": "mfma" if ops / alg > PEAK_INT8_OPS / PEAK_HBM_BYTES else "hbm",
        },
    }
