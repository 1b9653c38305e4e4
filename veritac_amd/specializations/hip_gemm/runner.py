"""hip_gemm benchmark driver (the analogue of specializations/cpu_gemm/runner.py).

benchmark_gemm times one plan on the GPU the way runner.py:111-232 times an
emitted C kernel (warm-up, then timed runs, then a correctness check against a
reference) and returns the same keys (gpu_time_ms in place of c_time_ms,
cpu_time_ms, speedup, correct) plus throughput and roofline figures.

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


def benchmark_gemm(plan, num_runs=20, *, warmup=3, inputs=None, seed=0, rotate=True,
                   reference=None, device=None):
    """Time `plan` on the GPU; returns timing, throughput and roofline figures.

    inputs: optional dict(A, B, D) of numpy arrays/tensors (else seeded random);
    reference: optional callable (A, B, D) -> C on numpy arrays, injected by the
    caller, used to check the first launch's output (`correct`).
    """
    import torch
    ok, reason = validate_plan(plan)
    if not ok:
        raise HipGemmError("invalid plan: " + reason)
    if not torch.cuda.is_available():
        raise HipGemmError("no GPU available: hip_gemm has no CPU path")
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else device
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

    correct = None
    out0 = run(plan, *sets[0][:3], out=sets[0][3], stream=raw)
    torch.cuda.synchronize(device)
    if reference is not None:
        import numpy as np
        expect = reference(A.cpu().numpy(), B.cpu().numpy(),
                           None if D is None else D.cpu().numpy())
        correct = bool(np.array_equal(out0.cpu().numpy(), expect))
    for i in range(warmup):
        s = sets[i % n_sets]
        run(plan, s[0], s[1], s[2], out=s[3], stream=raw)
    times = []
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
        "cpu_time_ms": None,
        "speedup": None,
        "correct": correct,
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
