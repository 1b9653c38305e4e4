"""Sequential interpreter of loop-nest `Stmt` JSON (TEST INFRASTRUCTURE ONLY).

Executes a loop nest exactly as the C that the reference's emitter writes
would run it (specializations/cpu_gemm/emit_c.py:83-155): loops in program
order, `for (v = lo; v < hi; v++)` with `hi` evaluated before every
iteration, integer division and modulo truncating toward zero as in C, flat
buffers indexed either with the reference's stride-1000 rule
(emit_c.py:29-44) or row-major with declared shapes. A store's value is
computed in floating point when the stored-to buffer or a buffer read in the
value (outside its indices) is floating point, else in exact Python ints
wrapped to the buffer's width on store; indices and loop bounds are ints,
and a floating value read there truncates toward zero. Buffers allocated by
the nest are float64 when any given buffer is floating point, else int64.
It walks the JSON itself and shares no code with the HIP emitter it checks.

Pinned by closed forms in tests/test_loopnest_host.py: the naive matmul nest
and its tiled / reordered forms give A @ B (and D + A @ B when C starts at
D); an index that steps outside its buffer raises IndexError here.
"""
from __future__ import annotations

import numpy as np

STRIDE = 1000
_WRAP = {"int8": 8, "int32": 32, "int64": 64}


def _trunc_div(a, b):
    q = abs(a) // abs(b)
    return q if (a >= 0) == (b >= 0) else -q


class _Ctx:
    """Buffers, their shapes, the layout and which buffers are alloc'd locals."""

    def __init__(self, bufs, shapes, layout, floating):
        self.bufs, self.shapes, self.layout, self.floating = bufs, shapes, layout, floating
        self.local = set()


def _eval(e, env, ctx, floating):
    tag = e["tag"]
    if tag == "lit":
        return float(e["val"]) if floating else e["val"]
    if tag == "var":
        return float(env[e["name"]]) if floating else env[e["name"]]
    if tag == "bufRead":
        v = ctx.bufs[e["buf"]][_flat(e, env, ctx)].item()
        return float(v) if floating else int(v)        # int() truncates toward zero
    a = _eval(e["left"], env, ctx, floating)
    b = _eval(e["right"], env, ctx, floating)
    if tag == "add":
        return a + b
    if tag == "mul":
        return a * b
    if floating:
        return a / b if tag == "div" else float(np.fmod(a, b))
    return _trunc_div(a, b) if tag == "div" else a - b * _trunc_div(a, b)


def _flat(node, env, ctx):
    buf = node["buf"]
    flat = 0
    for d, i in enumerate(node["indices"]):
        stride_1000 = ctx.layout == "reference" and buf not in ctx.local
        flat = flat * (STRIDE if stride_1000 else ctx.shapes[buf][d]) + _eval(i, env, ctx, False)
    if not 0 <= flat < ctx.bufs[buf].size:
        raise IndexError("%s index %d outside %d cells" % (buf, flat, ctx.bufs[buf].size))
    return flat


def _value_bufs(e, out):
    """Buffers read in expression e, not counting reads inside indices."""
    if e["tag"] == "bufRead":
        out.add(e["buf"])
    elif e["tag"] in ("add", "mul", "div", "mod"):
        _value_bufs(e["left"], out)
        _value_bufs(e["right"], out)
    return out


def _store(arr, flat, value):
    if arr.dtype.kind == "f":
        arr[flat] = value
    else:
        bits = arr.dtype.itemsize * 8
        v = int(value) & ((1 << bits) - 1)
        arr[flat] = v - (1 << bits) if v >= 1 << (bits - 1) else v


def _run(s, env, ctx):
    tag = s["tag"]
    if tag == "skip":
        return
    if tag == "bufWrite":
        floating = any(ctx.bufs[b].dtype.kind == "f" for b in _value_bufs(s["val"], {s["buf"]}))
        _store(ctx.bufs[s["buf"]], _flat(s, env, ctx), _eval(s["val"], env, ctx, floating))
    elif tag == "loop":
        v = _eval(s["lo"], env, ctx, False)
        while v < _eval(s["hi"], env, ctx, False):
            env[s["var"]] = v
            _run(s["body"], env, ctx)
            v += 1
        env.pop(s["var"], None)
    elif tag == "seq":
        _run(s["s1"], env, ctx)
        _run(s["s2"], env, ctx)
    elif tag == "alloc":
        dims = [_eval(d, env, ctx, False) for d in s["shape"]]
        name = s["buf"]
        ctx.bufs[name] = np.zeros(int(np.prod(dims)) if dims else 1,
                                  np.float64 if ctx.floating else np.int64)
        ctx.shapes[name] = dims
        ctx.local.add(name)
        try:
            _run(s["body"], env, ctx)
        finally:
            ctx.local.discard(name)
            del ctx.bufs[name], ctx.shapes[name]
    else:
        raise ValueError("unknown statement tag %r" % (tag,))


def run(stmt, buffers, shapes=None, layout="dense"):
    """Execute `stmt` over flat numpy buffers {name: 1-D array}, in place.

    shapes: {name: dims} for layout "dense" (row-major); layout "reference"
    uses the stride-1000 flat index. Each store computes in floating point
    when its own buffer or a buffer its value reads is floating point, in
    exact integers otherwise.
    """
    floating = any(b.dtype.kind == "f" for b in buffers.values())
    _run(stmt, {}, _Ctx(dict(buffers), dict(shapes or {}), layout, floating))
    return buffers
