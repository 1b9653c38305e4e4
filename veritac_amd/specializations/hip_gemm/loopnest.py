"""Loop-nest JSON -> HIP kernel for gfx950, compiled at run time.

The reference's CPU path takes a loop nest as `Stmt` JSON (README.md:456-503:
skip / bufWrite / loop / seq / alloc statements over lit / var / add / mul /
div / mod / bufRead expressions, loop annotations none / parallel /
vectorize / unrolled), parses it (specializations/cpu_gemm/lower.py:85-113)
and emits C (specializations/cpu_gemm/emit_c.py:83-155), then compiles that
with gcc and runs it (specializations/cpu_gemm/runner.py:65-108). This module
is the GPU counterpart: it reads the same JSON and emits one HIP kernel, which
the native library compiles in process with hipRTC (vt_rtc_compile) and
launches on the caller's stream (vt_rtc_launch).

Lowering, MI355X first
  * Thread mapping. Loops of the outermost perfect nest (a loop whose body
    is a loop, and so on) with constant bounds become GPU threads when they
    pass the two tests below: the product of their extents is linearised
    into one thread index, with the innermost mapped loop varying fastest
    so that neighbouring lanes of a wave touch neighbouring cells. Every
    other loop runs sequentially inside its thread, in its original order.
  * Independence is the reference's condition for `parallel` /
    `vectorize` (emit_c.py:60-80, "every buffer write mentions the loop
    variable"), tightened: every access, read or write, to a buffer written
    inside the loop must use one and the same index list, and that list must
    mention the variable. A reduction loop (C[i,j] += ... over k) fails it
    and stays sequential, which keeps each cell's additions in program
    order. Buffers allocated inside the loop are private to the iteration
    and do not count.
  * Mentioning the variable does not make cells disjoint (Y[i + j] over
    mapped i and j, Y[j % 2], or Y[j + i] under a sequential i all collide),
    so the mapped set must also pass threads_disjoint: each written
    buffer's flat index is affine in the loop variables and its
    coefficients separate the mapped variables like the digits of a mixed-
    radix number, whatever the sequential loops do. Threads then own
    disjoint cells and run what the sequential nest runs.
  * Annotations: a loop is mapped when it passes both tests, whatever its
    annotation; `parallel` / `vectorize` on a loop that does not is
    reported as suppressed (the reference writes the same "suppressed"
    comment instead of a pragma); `unrolled` adds `#pragma unroll` to a
    sequential loop.
  * Layouts. "reference": every buffer is flat with the reference's
    stride-1000 index, i0*1000^(d-1) + ... + i_{d-1} (emit_c.py:29-44), so
    buffers laid out for the reference's emitted C work unchanged. "dense":
    row-major with each buffer's declared shape.
  * Types. Buffers carry a dtype (int8, int32, int64, float32, float64).
    A store's value is evaluated in double when the stored-to buffer or a
    buffer read in the value (not in its indices) is floating point, else
    in 64-bit integers that wrap modulo 2^64; indices and loop bounds are
    always integers, and a floating value read there truncates toward zero.
    A store converts to the buffer's type (int32 stores wrap modulo 2^32,
    the contract's accumulator). The reference's CPU path uses double
    throughout, which is layout "reference" with float64 buffers.

Memory safety. An emitted kernel never touches memory outside the declared
buffers, whatever the nest computes: every access checks its flat index
against the buffer's declared size (the host checks each tensor holds at
least that many elements) and integer division or modulo by zero yields 0;
either event sets a bit in a status word (STATUS_RANGE, STATUS_DIV0) that
the call returns, and the offending store is skipped or read is 0.

Bounded work. Each GPU thread runs at most MAX_THREAD_ITERATIONS iterations
of sequential loops. Where interval arithmetic over the loop bounds gives an
upper bound on a thread's iterations, a nest above the cap is refused when
it is emitted. Where it cannot (a bound that reads memory), every
sequential loop counts its iterations, and a thread that reaches the cap
stops and sets STATUS_ITERATIONS. A nest therefore cannot hold the GPU
indefinitely, as an emitted C program on a CPU could run until killed.

Errors raise LoopNestError (a HipGemmError): unknown tags, unknown buffers,
unbound or shadowing loop variables, shapes that disagree with the index
count. Nothing falls back to the CPU.
"""
from __future__ import annotations

import ctypes
import re

from ... import _lib
from ..._lib import HipGemmError

BLOCK = 256
REFERENCE_STRIDE = 1000
STATUS_RANGE = 1   # an index fell outside its buffer
STATUS_DIV0 = 2    # an integer division or modulo by zero
STATUS_ITERATIONS = 4   # a thread reached MAX_THREAD_ITERATIONS and stopped
# Sequential loop iterations one GPU thread may run (about 0.1-1 s of one
# thread's time); the reference's largest benchmark nest (1000^3, one
# thread per output cell) runs 1000 per thread.
MAX_THREAD_ITERATIONS = 1 << 26
DTYPES = {"int8": "signed char", "int32": "int", "int64": "long long", "float32": "float",
          "float64": "double"}
FLOAT_DTYPES = ("float32", "float64")
ANNOTATIONS = ("none", "parallel", "vectorize", "unrolled")
_BINOPS = {"add": "+", "mul": "*", "div": "/", "mod": "%"}
_IDENT = re.compile(r"[A-Za-z_][A-Za-z0-9_]*\Z")
_INT64_MAX = 2**63 - 1


class LoopNestError(HipGemmError):
    """A loop nest the emitter cannot lower (malformed JSON, unknown buffer, ...)."""


# ---------------------------------------------------------------------------
# IR: expressions and statements as tuples
#   ("lit", v) ("var", name) (op, left, right) ("read", buf, (idx, ...))
#   ("skip",) ("write", buf, (idx, ...), value) ("seq", (stmt, ...))
#   ("loop", var, lo, hi, ann, body) ("alloc", buf, (dim, ...), body)
# ---------------------------------------------------------------------------

# Names the emitted C++ reserves: its own locals and helpers start with vt_.
_RESERVED = frozenset("""auto bool break case char const continue default do double else enum
extern float for goto if int long return short signed sizeof static struct switch typedef union
unsigned void volatile while class namespace template typename new delete this true false
private public protected operator friend virtual inline bool""".split())


def _name(value, what):
    if (not isinstance(value, str) or not _IDENT.match(value) or value.startswith("vt_")
            or value.startswith("__") or value in _RESERVED):
        raise LoopNestError("%s must be an identifier not starting with vt_ and not a C++ "
                            "keyword, got %r" % (what, value))
    return value


def parse_expr(node):
    """`SExpr` JSON -> IR (README.md:481-489)."""
    if not isinstance(node, dict) or "tag" not in node:
        raise LoopNestError("expression must be an object with a tag: %r" % (node,))
    tag = node["tag"]
    if tag == "lit":
        val = node.get("val")
        if (isinstance(val, bool) or not isinstance(val, int)
                or not -_INT64_MAX <= val <= _INT64_MAX):
            raise LoopNestError("lit value must be an integer within +-(2^63 - 1): %r" % (val,))
        return ("lit", val)
    if tag == "var":
        return ("var", _name(node.get("name"), "variable"))
    if tag in _BINOPS:
        return (tag, parse_expr(node.get("left")), parse_expr(node.get("right")))
    if tag == "bufRead":
        return ("read", _name(node.get("buf"), "buffer"),
                tuple(parse_expr(i) for i in node.get("indices", [])))
    raise LoopNestError("unknown expression tag %r" % (tag,))


def parse_stmt(node):
    """`Stmt` JSON -> IR (README.md:471-479); nested seqs are flattened."""
    if not isinstance(node, dict) or "tag" not in node:
        raise LoopNestError("statement must be an object with a tag: %r" % (node,))
    tag = node["tag"]
    if tag == "skip":
        return ("skip",)
    if tag == "bufWrite":
        return ("write", _name(node.get("buf"), "buffer"),
                tuple(parse_expr(i) for i in node.get("indices", [])), parse_expr(node.get("val")))
    if tag == "loop":
        ann = node.get("ann", "none")
        if ann not in ANNOTATIONS:
            raise LoopNestError("unknown loop annotation %r" % (ann,))
        return ("loop", _name(node.get("var"), "loop variable"), parse_expr(node.get("lo")),
                parse_expr(node.get("hi")), ann, parse_stmt(node.get("body")))
    if tag == "seq":
        parts = []
        for key in ("s1", "s2"):
            sub = parse_stmt(node.get(key))
            parts.extend(sub[1] if sub[0] == "seq" else (sub,))
        return ("seq", tuple(parts))
    if tag == "alloc":
        return ("alloc", _name(node.get("buf"), "buffer"),
                tuple(parse_expr(d) for d in node.get("shape", [])), parse_stmt(node.get("body")))
    raise LoopNestError("unknown statement tag %r" % (tag,))


def matmul_stmt(M, K, N):
    """The naive matmul nest as Stmt JSON: for i0 < M, i1 < N, i2 < K:
    C[i0,i1] = C[i0,i1] + A[i0,i2] * B[i2,i1]. Same nest as the reference's
    search starting point (Search/interface.py:66-116)."""
    def var(name):
        return {"tag": "var", "name": name}

    def read(buf, *idx):
        return {"tag": "bufRead", "buf": buf, "indices": [var(i) for i in idx]}

    def loop(name, hi, body):
        return {"tag": "loop", "var": name, "lo": {"tag": "lit", "val": 0},
                "hi": {"tag": "lit", "val": hi}, "ann": "none", "body": body}

    update = {"tag": "bufWrite", "buf": "C", "indices": [var("i0"), var("i1")],
              "val": {"tag": "add", "left": read("C", "i0", "i1"),
                      "right": {"tag": "mul", "left": read("A", "i0", "i2"),
                                "right": read("B", "i2", "i1")}}}
    return loop("i0", M, loop("i1", N, loop("i2", K, update)))


# ---------------------------------------------------------------------------
# Analysis
# ---------------------------------------------------------------------------

def _mentions(expr, name):
    kind = expr[0]
    if kind == "var":
        return expr[1] == name
    if kind == "lit":
        return False
    if kind == "read":
        return any(_mentions(i, name) for i in expr[2])
    return _mentions(expr[1], name) or _mentions(expr[2], name)


def _accesses(stmt, private, out):
    """Collect (buffer, indices, is_write) of every access in stmt, skipping
    buffers in `private` (allocated inside the region)."""
    def expr_acc(e):
        if e[0] == "read":
            if e[1] not in private:
                out.append((e[1], e[2], False))
            for i in e[2]:
                expr_acc(i)
        elif e[0] in _BINOPS:
            expr_acc(e[1])
            expr_acc(e[2])

    kind = stmt[0]
    if kind == "write":
        if stmt[1] not in private:
            out.append((stmt[1], stmt[2], True))
        for i in stmt[2]:
            expr_acc(i)
        expr_acc(stmt[3])
    elif kind == "loop":
        expr_acc(stmt[2])
        expr_acc(stmt[3])
        _accesses(stmt[5], private, out)
    elif kind == "seq":
        for sub in stmt[1]:
            _accesses(sub, private, out)
    elif kind == "alloc":
        for d in stmt[2]:
            expr_acc(d)
        _accesses(stmt[3], private | {stmt[1]}, out)
    return out


def independent(var, body):
    """True when the iterations of loop `var` over `body` touch disjoint cells
    of every buffer the body writes (the exact form of the reference's
    writes_local_to guard, emit_c.py:60-80)."""
    acc = _accesses(body, frozenset(), [])
    written = {buf for buf, _, is_write in acc if is_write}
    for buf in written:
        index_lists = {idx for b, idx, _ in acc if b == buf}
        if len(index_lists) != 1:
            return False
        (idx,) = index_lists
        if not any(_mentions(i, var) for i in idx):
            return False
    return True


def _const(expr):
    return expr[1] if expr[0] == "lit" else None


def _affine(e):
    """{var: coefficient, None: constant} of an integer expression that is
    affine in the loop variables (lit, var, add, mul by a constant), else
    None (division, modulo, buffer reads, products of two variables)."""
    kind = e[0]
    if kind == "lit":
        return {None: e[1]}
    if kind == "var":
        return {e[1]: 1}
    if kind not in ("add", "mul"):
        return None
    left, right = _affine(e[1]), _affine(e[2])
    if left is None or right is None:
        return None
    if kind == "add":
        out = dict(left)
        for v, c in right.items():
            out[v] = out.get(v, 0) + c
        return out
    for scale, form in ((left, right), (right, left)):
        if set(scale) <= {None}:
            k = scale.get(None, 0)
            return {v: c * k for v, c in form.items()}
    return None


def _interval(form, ranges):
    """(min, max) of an affine form over {var: (min, max)}, or None when a
    variable's range is unknown."""
    lo = hi = form.get(None, 0)
    for v, c in form.items():
        if v is None or c == 0:
            continue
        r = ranges.get(v)
        if r is None:
            return None
        a, b = c * r[0], c * r[1]
        lo, hi = lo + min(a, b), hi + max(a, b)
    return lo, hi


def _var_ranges(stmt, ranges):
    """Fill {var: (min, max) or None} with the values every loop variable can
    take, by interval arithmetic over the loop bounds (None where a bound is
    not affine). Sibling loops that reuse a name get the union; a loop that
    can never run leaves its variable (and those inside it) unknown."""
    kind = stmt[0]
    if kind == "loop":
        var, lo, hi, body = stmt[1], stmt[2], stmt[3], stmt[5]
        flo, fhi = _affine(lo), _affine(hi)
        ilo = None if flo is None else _interval(flo, ranges)
        ihi = None if fhi is None else _interval(fhi, ranges)
        r = None
        if ilo is not None and ihi is not None and ihi[1] - 1 >= ilo[0]:
            r = (ilo[0], ihi[1] - 1)
        if var in ranges:
            old = ranges[var]
            r = None if old is None or r is None else (min(old[0], r[0]), max(old[1], r[1]))
        ranges[var] = r
        _var_ranges(body, ranges)
    elif kind == "seq":
        for sub in stmt[1]:
            _var_ranges(sub, ranges)
    elif kind == "alloc":
        _var_ranges(stmt[3], ranges)
    return ranges


def thread_iterations(stmt, mapped_vars, ranges):
    """Upper bound on the sequential loop iterations one thread runs (mapped
    loops are the threads themselves), by interval arithmetic over the loop
    bounds with `ranges` from _var_ranges; None when a bound is not affine or
    its range is unknown."""
    kind = stmt[0]
    if kind == "loop":
        var, lo, hi, body = stmt[1], stmt[2], stmt[3], stmt[5]
        inner = thread_iterations(body, mapped_vars, ranges)
        if inner is None:
            return None
        if var in mapped_vars:
            return inner
        flo, fhi = _affine(lo), _affine(hi)
        ilo = None if flo is None else _interval(flo, ranges)
        ihi = None if fhi is None else _interval(fhi, ranges)
        if ilo is None or ihi is None:
            return None
        return max(0, ihi[1] - ilo[0]) * (1 + inner)
    if kind == "seq":
        total = 0
        for sub in stmt[1]:
            w = thread_iterations(sub, mapped_vars, ranges)
            if w is None:
                return None
            total += w
        return total
    if kind == "alloc":
        return thread_iterations(stmt[3], mapped_vars, ranges)
    return 0


def _flat_form(buf, idx, buffers, layout):
    """Affine form of the flat cell index of buf[idx], or None."""
    forms = [_affine(i) for i in idx]
    if any(f is None for f in forms):
        return None
    n = len(idx)
    if layout == "reference":
        strides = [REFERENCE_STRIDE ** (n - 1 - d) for d in range(n)]
    else:
        shape = tuple(buffers[buf]["shape"])
        if len(shape) != n:
            return None
        strides = [_prod(shape[d + 1:]) for d in range(n)]
    out = {}
    for form, stride in zip(forms, strides):
        for v, c in form.items():
            out[v] = out.get(v, 0) + c * stride
    return out


def threads_disjoint(stmt, mapped, buffers, layout="dense", ranges=None):
    """True when one thread per point of the mapped loops ({var: extent}),
    each running the rest of the nest sequentially, computes what the
    sequential nest computes.

    Sufficient condition, checked per buffer the nest writes (buffers
    allocated inside the nest are private to a thread and exempt):
      * every access to it, read or write, anywhere in the nest (loop bounds
        included) uses one and the same index list, so a thread touches only
        cells that list names;
      * the list's flat index F = c0 + sum(c_v * v) is affine in the loop
        variables, each mapped variable of extent > 1 has c_v != 0, and
        sorting the variables of nonzero coefficient and nonzero value range
        w_v by |c_v|, every variable from the first mapped one on satisfies
        |c_v| > sum(|c_u| * w_u) over the variables before it.
    Then F(m, s) == F(m', s') forces m == m': take the last variable in that
    order whose value differs between the two points; if any mapped value
    differs, it is that variable or comes after one, and its term alone
    outweighs every change the earlier ones can make. Threads therefore own
    disjoint cells, and each thread meets its own cells in program order.
    """
    if ranges is None:
        ranges = _var_ranges(stmt, {})
    acc = _accesses(stmt, frozenset(), [])
    for buf in {b for b, _, w in acc if w}:
        lists = {idx for b, idx, _ in acc if b == buf}
        if len(lists) != 1:
            return False
        form = _flat_form(buf, next(iter(lists)), buffers, layout)
        if form is None:
            return False
        if any(ext > 1 and form.get(v, 0) == 0 for v, ext in mapped.items()):
            return False
        terms = []
        for v, c in form.items():
            if v is None or c == 0:
                continue
            if v in mapped:
                width = mapped[v] - 1
            else:
                r = ranges.get(v)
                if r is None:
                    return False
                width = r[1] - r[0]
            if width > 0:
                terms.append((abs(c), v in mapped, width))
        span, seen_mapped = 0, False
        for c, is_mapped, width in sorted(terms, key=lambda t: t[0]):
            seen_mapped = seen_mapped or is_mapped
            if seen_mapped and c <= span:
                return False
            span += c * width
    return True


def plan_mapping(stmt, buffers, layout="dense"):
    """Split the outermost perfect nest into mapped and sequential loops.

    Loops are taken outermost first: a loop with constant bounds joins the
    mapped set when it is independent and the enlarged set still passes
    threads_disjoint. Returns (mapped, notes): mapped is a list of
    (var, lo, extent) from outermost to innermost; notes lists suppressed
    annotations.
    """
    mapped, notes = [], []
    ranges = _var_ranges(stmt, {})
    node = stmt
    while node[0] == "loop":
        var, lo, hi, ann, body = node[1], node[2], node[3], node[4], node[5]
        lo_c, hi_c = _const(lo), _const(hi)
        reason = "body writes cells not local to it"
        if lo_c is not None and hi_c is not None and independent(var, body):
            trial = mapped + [(var, lo_c, max(0, hi_c - lo_c))]
            if threads_disjoint(stmt, {m[0]: m[2] for m in trial}, buffers, layout, ranges):
                mapped = trial
                node = body
                continue
            reason = "iterations may write the same cell"
        if ann in ("parallel", "vectorize"):
            notes.append("%s suppressed on %s: %s" % (ann, var, reason))
        node = body
    return mapped, notes


def _walk_notes(stmt, mapped_vars, notes):
    """Suppression notes for annotated loops outside the mapped nest."""
    if stmt[0] == "loop":
        if stmt[1] not in mapped_vars and stmt[4] in ("parallel", "vectorize"):
            note = "%s suppressed on %s: body writes cells not local to it" % (stmt[4], stmt[1])
            if independent(stmt[1], stmt[5]):
                note = "%s on %s runs sequentially inside its thread" % (stmt[4], stmt[1])
            if note not in notes:
                notes.append(note)
        _walk_notes(stmt[5], mapped_vars, notes)
    elif stmt[0] == "seq":
        for sub in stmt[1]:
            _walk_notes(sub, mapped_vars, notes)
    elif stmt[0] == "alloc":
        _walk_notes(stmt[3], mapped_vars, notes)


# ---------------------------------------------------------------------------
# Emission
# ---------------------------------------------------------------------------

class _Emitter:
    guard = None   # cap on each thread's sequential iterations, when counted at run time

    def __init__(self, buffers, layout):
        self.buffers = buffers
        self.layout = layout
        self.locals = {}     # alloc'd buffer -> (shape exprs)
        self.lines = []

    def buf_dtype(self, buf):
        if buf in self.locals:
            return self.locals[buf][1]
        return self.buffers[buf]["dtype"]

    def size(self, buf):
        """Cells of a buffer as declared (guard bound of every access)."""
        if buf in self.locals:
            return _prod(_const(d) for d in self.locals[buf][0]) if self.locals[buf][0] else 1
        shape = tuple(self.buffers[buf]["shape"])
        return _max_index(shape, self.layout) + 1

    def guarded(self, buf, idx):
        """Index expression clamped into the buffer; out-of-range sets
        STATUS_RANGE and the caller skips the store / reads zero."""
        return "vt_idx(%s, %dLL, vt_status)" % (self.index(buf, idx), self.size(buf))

    def index(self, buf, idx):
        if buf not in self.buffers and buf not in self.locals:
            raise LoopNestError("buffer %r is not declared" % buf)
        if not idx:
            return "0LL"
        parts = [self.expr_int(i) for i in idx]
        if buf in self.locals:
            shape = [self.expr_int(d) for d in self.locals[buf][0]]
        elif self.layout == "reference":
            shape = None
        else:
            shape = [str(d) for d in self.buffers[buf]["shape"]]
            if len(shape) != len(idx):
                raise LoopNestError("buffer %r has %d dims, accessed with %d indices"
                                    % (buf, len(shape), len(idx)))
        flat = parts[0]
        for d in range(1, len(parts)):
            dim = "%dLL" % REFERENCE_STRIDE if shape is None else "(long long)(%s)" % shape[d]
            flat = "(%s) * %s + %s" % (flat, dim, parts[d])
        return flat

    def expr_int(self, e):
        return self.expr(e, "long long")

    def expr(self, e, ty):
        kind = e[0]
        if kind == "lit":
            return ("%d.0" % e[1]) if ty == "double" else ("%dLL" % e[1])
        if kind == "var":
            return "((%s)%s)" % (ty, e[1]) if ty == "double" else e[1]
        if kind == "read":
            # a read converts to the context's type; a floating value read
            # in integer context truncates toward zero, as a C cast does
            return "((%s)vt_rd(%s, %s))" % (ty, e[1], self.guarded(e[1], e[2]))
        left, right = self.expr(e[1], ty), self.expr(e[2], ty)
        if kind in ("div", "mod") and ty == "long long":
            return "vt_%s(%s, %s, vt_status)" % (kind, left, right)
        if kind == "mod":
            return "fmod(%s, %s)" % (left, right)
        return "(%s %s %s)" % (left, _BINOPS[kind], right)

    def value_type(self, stmt_buf, expr):
        bufs = {stmt_buf}

        def collect(x):
            if x[0] == "read":
                bufs.add(x[1])
            elif x[0] in _BINOPS:
                collect(x[1])
                collect(x[2])
        collect(expr)
        for b in bufs:
            if b not in self.buffers and b not in self.locals:
                raise LoopNestError("buffer %r is not declared" % b)
        return "double" if any(self.buf_dtype(b) in FLOAT_DTYPES for b in bufs) else "long long"

    def count_iteration(self, depth):
        if self.guard is not None:
            self.lines.append("%sif (++vt_iters > %dULL) { atomicOr(vt_status, %d); return; }"
                              % ("  " * depth, self.guard, STATUS_ITERATIONS))

    def stmt(self, s, depth):
        pad = "  " * depth
        kind = s[0]
        if kind == "skip":
            self.lines.append(pad + "/* skip */")
        elif kind == "write":
            buf, idx, val = s[1], s[2], s[3]
            ty = self.value_type(buf, val)
            ctype = DTYPES[self.buf_dtype(buf)]
            value = self.expr(val, ty)
            if self.buf_dtype(buf) == "int32" and ty == "long long":
                # int32 accumulator: keep the low 32 bits (two's complement wrap)
                value = "(int)(unsigned int)(unsigned long long)%s" % value
            else:
                value = "(%s)%s" % (ctype, value)
            self.lines.append("%s{ const long long vt_at = %s; if (vt_at >= 0) %s[vt_at] = %s; }"
                              % (pad, self.guarded(buf, idx), buf, value))
        elif kind == "loop":
            var, lo, hi, ann, body = s[1:]
            if ann == "unrolled":
                self.lines.append(pad + "#pragma unroll")
            self.lines.append("%sfor (long long %s = %s; %s < %s; ++%s) {"
                              % (pad, var, self.expr_int(lo), var, self.expr_int(hi), var))
            self.count_iteration(depth + 1)
            self.stmt(body, depth + 1)
            self.lines.append(pad + "}")
        elif kind == "seq":
            for sub in s[1]:
                self.stmt(sub, depth)
        elif kind == "alloc":
            buf, shape, body = s[1], s[2], s[3]
            if buf in self.buffers or buf in self.locals:
                raise LoopNestError("alloc of %r shadows another buffer" % buf)
            dims = [_const(d) for d in shape]
            if any(d is None or d <= 0 for d in dims) or (dims and _prod(dims) > 4096):
                raise LoopNestError("alloc %r needs constant positive dims (<= 4096 cells)" % buf)
            # local buffers are double, as in the reference's emitted C
            # (emit_c.py: `double buf[...]`), when any declared buffer is
            # floating point, else 64-bit integers
            floating = any(info["dtype"] in FLOAT_DTYPES for info in self.buffers.values())
            self.locals[buf] = (shape, "float64" if floating else "int64")
            self.lines.append("%s%s %s[%d] = {};" % (pad, DTYPES[self.locals[buf][1]], buf,
                                                     _prod(dims) if dims else 1))
            self.stmt(body, depth)
            del self.locals[buf]
        else:
            raise LoopNestError("unknown statement %r" % (kind,))


# Device helpers of every emitted kernel: guarded index, guarded read, and
# integer division / modulo that cannot trap or invoke undefined behaviour.
_PRELUDE = r"""__device__ __forceinline__ long long vt_idx(long long i, long long n, int *st) {
  if (i >= 0 && i < n) return i;
  atomicOr(st, 1);
  return -1;
}
template <typename T> __device__ __forceinline__ T vt_rd(const T *p, long long i) {
  return i >= 0 ? p[i] : T(0);
}
__device__ __forceinline__ long long vt_div(long long a, long long b, int *st) {
  if (b == 0 || (b == -1 && a == (-9223372036854775807LL - 1))) { atomicOr(st, 2); return 0; }
  return a / b;
}
__device__ __forceinline__ long long vt_mod(long long a, long long b, int *st) {
  if (b == 0 || b == -1) { if (b == 0) atomicOr(st, 2); return 0; }
  return a % b;
}"""


def _prod(values):
    out = 1
    for v in values:
        out *= v
    return out


def _expr_vars(e, out):
    if e[0] == "var":
        out.add(e[1])
    elif e[0] == "read":
        for i in e[2]:
            _expr_vars(i, out)
    elif e[0] in _BINOPS:
        _expr_vars(e[1], out)
        _expr_vars(e[2], out)
    return out


def _check_vars(stmt, bound):
    """Every variable is bound by an enclosing loop; no loop rebinds one."""
    def need(exprs):
        free = set()
        for e in exprs:
            _expr_vars(e, free)
        free -= bound
        if free:
            raise LoopNestError("unbound variables %s" % sorted(free))

    kind = stmt[0]
    if kind == "loop":
        if stmt[1] in bound:
            raise LoopNestError("loop variable %r shadows an enclosing loop" % stmt[1])
        need((stmt[2], stmt[3]))
        _check_vars(stmt[5], bound | {stmt[1]})
    elif kind == "seq":
        for sub in stmt[1]:
            _check_vars(sub, bound)
    elif kind == "alloc":
        need(stmt[2])
        _check_vars(stmt[3], bound)
    elif kind == "write":
        need(stmt[2] + (stmt[3],))


def _written(stmt):
    return {buf for buf, _, w in _accesses(stmt, frozenset(), []) if w}


def _used(stmt):
    return {buf for buf, _, _ in _accesses(stmt, frozenset(), [])}


def emit_kernel(stmt, buffers, name="loopnest", layout="dense",
                max_iterations=MAX_THREAD_ITERATIONS):
    """Lower a parsed (or JSON) loop nest to a HIP kernel.

    buffers: {name: {"dtype": one of DTYPES, "shape": (d0, ...)}} for every
    buffer the nest touches (shape is used by layout "dense" and for the
    parameter size checks). Returns a dict: source, kernel name, params (the
    buffer names in parameter order), mapped loops, threads, grid, block and
    the suppression notes. `max_iterations` caps each thread's sequential
    loop iterations (at most MAX_THREAD_ITERATIONS).
    """
    if isinstance(stmt, dict):
        stmt = parse_stmt(stmt)
    if not (isinstance(max_iterations, int) and 0 < max_iterations <= MAX_THREAD_ITERATIONS):
        raise LoopNestError("max_iterations must be an integer in [1, %d]" % MAX_THREAD_ITERATIONS)
    if layout not in ("dense", "reference"):
        raise LoopNestError("layout must be 'dense' or 'reference'")
    _name(name, "kernel name")
    for buf, info in buffers.items():
        _name(buf, "buffer")
        if info.get("dtype") not in DTYPES:
            raise LoopNestError("buffer %r: dtype must be one of %s" % (buf, sorted(DTYPES)))
    _check_vars(stmt, frozenset())
    used = _used(stmt)
    missing = sorted(used - set(buffers))
    if missing:
        raise LoopNestError("buffers used but not declared: %s" % missing)
    mapped, notes = plan_mapping(stmt, buffers, layout)
    _walk_notes(stmt, {m[0] for m in mapped}, notes)
    work = thread_iterations(stmt, {m[0] for m in mapped}, _var_ranges(stmt, {}))
    if work is not None and work > max_iterations:
        raise LoopNestError("each GPU thread would run up to %d sequential loop iterations, "
                            "beyond the cap of %d" % (work, max_iterations))
    if work is None:
        notes.append("loop bounds that read memory: each thread's sequential iterations are "
                     "counted and stop at %d (STATUS_ITERATIONS)" % max_iterations)
    written = _written(stmt)
    params = sorted(b for b in used if b in buffers)
    em = _Emitter(buffers, layout)
    em.guard = max_iterations if work is None else None
    # peel the mapped loops off the perfect nest
    node, seq_chain = stmt, []
    mapped_vars = {m[0] for m in mapped}
    while node[0] == "loop":
        if node[1] not in mapped_vars:
            seq_chain.append(node)
        node = node[5]
    inner = node
    total = _prod(m[2] for m in mapped) if mapped else 1
    sig = ", ".join(["%s%s *__restrict__ %s" % ("" if b in written else "const ",
                                               DTYPES[buffers[b]["dtype"]], b) for b in params]
                    + ["int *__restrict__ vt_status"])
    em.lines.append('extern "C" __global__ __launch_bounds__(%d) void %s(%s) {' % (BLOCK, name, sig))
    em.lines.append("  const long long vt_t = (long long)blockIdx.x * %d + threadIdx.x;" % BLOCK)
    em.lines.append("  if (vt_t >= %dLL) return;" % total)
    if em.guard is not None:
        em.lines.append("  unsigned long long vt_iters = 0;")
    if mapped:
        em.lines.append("  long long vt_rest = vt_t;")
        for var, lo, ext in reversed(mapped):
            # an empty mapped loop makes total 0 and this unreachable; the
            # divisor stays nonzero all the same
            em.lines.append("  const long long %s = %dLL + vt_rest %% %dLL;" % (var, lo, max(ext, 1)))
            em.lines.append("  vt_rest /= %dLL;" % max(ext, 1))
    # sequential loops of the chain, then the innermost body
    depth = 1
    for loop in seq_chain:
        var, lo, hi, ann = loop[1], loop[2], loop[3], loop[4]
        pad = "  " * depth
        if ann == "unrolled":
            em.lines.append(pad + "#pragma unroll")
        em.lines.append("%sfor (long long %s = %s; %s < %s; ++%s) {"
                        % (pad, var, em.expr_int(lo), var, em.expr_int(hi), var))
        depth += 1
        em.count_iteration(depth)
    em.stmt(inner, depth)
    for d in range(depth - 1, 0, -1):
        em.lines.append("  " * d + "}")
    em.lines.append("}")
    header = ["// Emitted by veritac_amd.specializations.hip_gemm.loopnest (layout %s)." % layout]
    header += ["// %s" % n for n in notes]
    header += [_PRELUDE]
    blocks = max(1, -(-total // BLOCK))
    if blocks > 2**31 - 1:
        raise LoopNestError("%d mapped iterations exceed the launch limit" % total)
    return {"source": "\n".join(header + em.lines) + "\n", "kernel": name, "params": params,
            "written": sorted(written), "mapped": [m[0] for m in mapped], "threads": total,
            "grid": (blocks, 1, 1), "block": (BLOCK, 1, 1), "notes": notes, "layout": layout}


# ---------------------------------------------------------------------------
# Compile and run
# ---------------------------------------------------------------------------

_TORCH_DTYPES = {"int8": "int8", "int32": "int32", "int64": "int64", "float32": "float32",
                 "float64": "float64"}


def _byte_span(t):
    """[first, last) byte addresses a contiguous tensor occupies."""
    start = t.data_ptr()
    return start, start + t.numel() * t.element_size()


def _max_index(shape, layout):
    if not shape:
        return 0
    if layout == "dense":
        return _prod(shape) - 1
    flat = 0
    for d in shape:
        flat = flat * REFERENCE_STRIDE + (d - 1)
    return flat


class LoopNestKernel:
    """An emitted loop nest, compiled for gfx950 by hipRTC."""

    def __init__(self, stmt, buffers, name="loopnest", layout="dense",
                 max_iterations=MAX_THREAD_ITERATIONS):
        self.info = emit_kernel(stmt, buffers, name=name, layout=layout,
                                max_iterations=max_iterations)
        self.buffers = {b: dict(v) for b, v in buffers.items()}
        self.program = _lib.RtcProgram(self.info["source"], self.info["kernel"])

    @property
    def source(self):
        return self.info["source"]

    def __call__(self, tensors, stream=None):
        """Run the nest over device tensors {buffer name: tensor}; written
        buffers are updated in place. Dtypes and sizes are checked against the
        declarations before the launch, and a written buffer may not share
        memory with another buffer (the kernel declares its pointers
        __restrict__, and the analysis assumes distinct buffers). `stream`
        is a raw hipStream_t handle, default torch's current stream; the
        call orders the status word's zeroing before the launch on it.
        Returns the int32 status tensor of the launch (0, or STATUS_RANGE |
        STATUS_DIV0 | STATUS_ITERATIONS bits; read it after the stream has
        synchronised)."""
        import torch
        for b in self.info["params"]:
            if b not in tensors:
                raise LoopNestError("missing tensor for buffer %r" % b)
            t = tensors[b]
            decl = self.buffers[b]
            if not isinstance(t, torch.Tensor) or not t.is_contiguous():
                raise LoopNestError("buffer %r must be a contiguous torch tensor" % b)
            if str(t.dtype).replace("torch.", "") != _TORCH_DTYPES[decl["dtype"]]:
                raise LoopNestError("buffer %r must be %s (got %s)" % (b, decl["dtype"], t.dtype))
            need = _max_index(tuple(decl["shape"]), self.info["layout"]) + 1
            if t.numel() < need:
                raise LoopNestError("buffer %r has %d elements; its %s layout needs %d"
                                    % (b, t.numel(), self.info["layout"], need))
        spans = {b: _byte_span(tensors[b]) for b in self.info["params"]}
        for w in self.info["written"]:
            for b in self.info["params"]:
                if b != w and spans[w][0] < spans[b][1] and spans[b][0] < spans[w][1]:
                    raise LoopNestError("written buffer %r overlaps buffer %r in memory" % (w, b))
        devices = {tensors[b].device for b in self.info["params"]}
        if any(d.type != "cuda" for d in devices):
            raise LoopNestError("buffers are on %s; loop nests run on the GPU only"
                                % sorted(str(d) for d in devices))
        if len(devices) > 1:
            raise LoopNestError("buffers are on different devices")
        # a nest that touches no buffer still runs (its loop bounds may divide
        # by zero), on the current device
        device = devices.pop() if devices else torch.device("cuda", torch.cuda.current_device())
        args = [ctypes.c_void_p(tensors[b].data_ptr()) for b in self.info["params"]]
        with torch.cuda.device(device):
            current = torch.cuda.current_stream(device)
            status = torch.zeros(1, dtype=torch.int32, device=device)
            if stream is None or stream == current.cuda_stream:
                stream = current.cuda_stream
            else:
                # zeroed on the current stream, used on the caller's: order the
                # two and keep the allocator from reusing the word too early
                ext = torch.cuda.ExternalStream(stream, device=device)
                ext.wait_stream(current)
                status.record_stream(ext)
        args.append(ctypes.c_void_p(status.data_ptr()))
        if self.info["threads"] > 0:
            self.program.launch(self.info["grid"], self.info["block"], args, stream)
        return status


# ---------------------------------------------------------------------------
# The reference's CPU benchmark, on the GPU
# ---------------------------------------------------------------------------

def benchmark_matmul(stmt_json, M, K, N, num_runs=5, stream=None):
    """Run a matmul loop nest the way the reference's benchmark_matmul does
    (specializations/cpu_gemm/runner.py:111-232), on the GPU.

    Same inputs and layout: A[i,k] = (i*K + k) % 7 and B[k,j] = (k*N + j) % 5
    as float64 in the stride-1000 flat layout, C zeroed before every run. The
    emitted kernel is compiled once (hipRTC); one warm-up, then `num_runs`
    launches timed with HIP events. The result is checked against numpy on
    every cell (the reference prints and compares four); all values are
    integers below 2^53, so float64 is exact and the comparison is equality.
    """
    import time
    import numpy as np
    import torch
    if min(M, K, N) <= 0 or max(M, K, N) > REFERENCE_STRIDE:
        raise LoopNestError("the stride-1000 layout needs 0 < M, K, N <= 1000")
    decl = {"A": {"dtype": "float64", "shape": (M, K)}, "B": {"dtype": "float64", "shape": (K, N)},
            "C": {"dtype": "float64", "shape": (M, N)}}
    kern = LoopNestKernel(stmt_json, decl, name="matmul", layout="reference")
    dev = torch.device("cuda", torch.cuda.current_device())
    A_np = np.fromfunction(lambda i, k: (i * K + k) % 7, (M, K), dtype=np.int64).astype(np.float64)
    B_np = np.fromfunction(lambda k, j: (k * N + j) % 5, (K, N), dtype=np.int64).astype(np.float64)
    bufs = {}
    for name, mat in (("A", A_np), ("B", B_np), ("C", np.zeros((M, N)))):
        rows, cols = mat.shape
        # flat buffer of the stride-1000 layout, and the logical matrix in it
        flat = torch.zeros(_max_index((rows, cols), "reference") + 1, dtype=torch.float64, device=dev)
        view = flat.as_strided((rows, cols), (REFERENCE_STRIDE, 1))
        view.copy_(torch.from_numpy(mat))
        bufs[name] = (flat, view)
    tensors = {name: flat for name, (flat, _) in bufs.items()}
    # the events go on the stream the kernel is launched on
    timed = torch.cuda.current_stream(dev) if stream is None else \
        torch.cuda.ExternalStream(stream, device=dev)
    statuses = [kern(tensors, stream=stream)]               # warm-up
    times = []
    for _ in range(num_runs):
        bufs["C"][0].zero_()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        timed.wait_stream(torch.cuda.current_stream(dev))
        e0.record(timed)
        statuses.append(kern(tensors, stream=stream))
        e1.record(timed)
        torch.cuda.synchronize(dev)
        times.append(e0.elapsed_time(e1))
    C_gpu = bufs["C"][1].cpu().numpy()
    t0 = time.perf_counter()
    for _ in range(num_runs):
        C_np = A_np @ B_np
    np_ms = (time.perf_counter() - t0) / num_runs * 1e3
    gpu_ms = sum(times) / len(times)
    cells = [(0, 0), (min(1, M - 1), 0), (M - 1, 0), (M - 1, N - 1)]
    st = 0
    for s in statuses:                                     # any run's events count
        st |= int(s.item())
    return {"gpu_time_ms": gpu_ms, "numpy_time_ms": np_ms,
            "speedup": np_ms / gpu_ms if gpu_ms else 0.0,
            "correct": bool(np.array_equal(C_gpu, C_np)) and st == 0,
            "gpu_first_values": [float(C_gpu[c]) for c in cells],
            "np_first_values": [float(C_np[c]) for c in cells],
            "status": st, "mapped_loops": kern.info["mapped"], "notes": kern.info["notes"]}
