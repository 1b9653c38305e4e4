"""Gemmini weight-stationary schedules: generators, modeled counts and the
symbolic program check.

The command streams that `replay.run_commands` executes on the GPU come
from here when they are not recorded ones:

  * `gen_baseline`, `gen_reuse_b`, `gen_commands` (specializations/
    gemmini_gemm/backend.py:267-324) and `gen_batched_reuse_b`
    (specializations/gemmini_gemm/lowering.py:18-40) emit the same commands,
    in the same order, as the reference's generators for a plan. All four are
    one tile walk (`_walk`) over blocks of 16-row output tiles that share one
    16-column block.
  * `modeled_counts` / `modeled_objective` (backend.py:330-367) count a stream;
    `make_plan` / `optimize` (backend.py:1064-1093) select a schedule by them.
  * `check_program` is the shape-parameterised translation validator the
    reference runs in Lean before it accepts a stream
    (VeriTac/Gemmini/Symbolic.lean:30-47 over the transitions of
    VeriTac/Gemmini/Engine.lean:38-84): every scratchpad tile names the input
    elements it holds, every accumulator tile carries its ordered list of
    products, and a stream is accepted only if every output cell holds exactly
    the products A[r, t] * B[t, c] for t = 0 .. k-1, in that order.

Commands are the dicts of a veritac_program_request_v1 (backend.py:902-906):
{"kind": ..., <fields>}, the form the replay reads.
"""
from __future__ import annotations

import numpy as np

from . import replay as _rp

DIM = _rp.DIM
GARBAGE_ADDR = _rp.GARBAGE_ADDR
ACCUMULATE_BIT = _rp.ACCUMULATE_BIT
# Accumulator-space, full-C output address of accumulator row 0; without the
# accumulate bit the compute overwrites the rows (backend.py:78-80).
ACC_OUT = _rp.ACC_SPACE_BIT | _rp.FULL_C_BIT
ACC_OUT_ACCUMULATE = ACC_OUT | ACCUMULATE_BIT
A_SPAD, B_SPAD = 0, DIM     # scratchpad rows of the streamed A tile and the B tile

SCHEDULES = _rp.SCHEDULES


def make_plan(m, n, k, schedule):
    """The smallest-capacity plan for a schedule (backend.py:1064-1069)."""
    plan = {"m": m, "n": n, "k": k, "dim": DIM, "schedule": schedule}
    plan["scratchpad_rows"], plan["accumulator_rows"] = _rp.required_resources(plan)
    return plan


def _preamble(plan):
    """Weight-stationary dataflow; row strides of C (int32), A and B (int8)."""
    m, n, k = plan["m"], plan["n"], plan["k"]
    return [{"kind": "config_ex", "dataflow": _rp.WEIGHT_STATIONARY},
            {"kind": "config_st", "stride_bytes": 4 * n},
            {"kind": "config_ld", "slot": 0, "stride_bytes": k, "scale": 1.0},
            {"kind": "config_ld", "slot": 1, "stride_bytes": n, "scale": 1.0}]


def _mvin(buf, offset, spad):
    return {"kind": "mvin", "slot": 0 if buf == "A" else 1, "buf": buf, "offset": offset,
            "spad_addr": spad, "cols": DIM, "rows": DIM}


def _walk(plan, blocks, b_per_tile):
    """Commands for `blocks`, a sequence of (j, rows): the 16-row tiles `rows`
    of column block j, computed into accumulator tiles 0, 1, ... in order.

    Over each 16-deep k step of a block, B(kk, j) is moved in once and latched
    by the block's first compute; the other rows retain it (compute
    accumulated). With b_per_tile (the baseline schedule, one row per block)
    A(i, kk) is moved in first, then B. The first k step overwrites each
    accumulator tile and later ones accumulate onto it; a tile leaves right
    after its last compute."""
    n, k = plan["n"], plan["k"]
    kt = k // DIM
    cmds = _preamble(plan)
    for j, rows in blocks:
        for kk in range(kt):
            b_in = _mvin("B", (kk * n + j) * DIM, B_SPAD)
            if not b_per_tile:
                cmds.append(b_in)
            for local, i in enumerate(rows):
                cmds.append(_mvin("A", (i * k + kk) * DIM, A_SPAD))
                if b_per_tile:
                    cmds.append(b_in)
                out = (ACC_OUT_ACCUMULATE if kk else ACC_OUT) + local * DIM
                retained = local > 0
                cmds.append({"kind": "preload", "bd_spad_addr": GARBAGE_ADDR if retained else B_SPAD,
                             "out_addr": out})
                cmds.append({"kind": "compute", "accumulated": retained, "a_spad_addr": A_SPAD,
                             "bd_spad_addr": GARBAGE_ADDR})
                if kk == kt - 1:
                    cmds.append({"kind": "mvout", "buf_offset": (i * n + j) * DIM,
                                 "acc_addr": ACC_OUT_ACCUMULATE + local * DIM,
                                 "cols": DIM, "rows": DIM})
    cmds.append({"kind": "fence"})
    return cmds


def gen_baseline(plan):
    """i, j, k order: A and B moved in for every output tile and k step; one
    accumulator tile live (backend.py:267-292)."""
    it, jt = plan["m"] // DIM, plan["n"] // DIM
    return _walk(plan, [(j, (i,)) for i in range(it) for j in range(jt)], True)


def gen_reuse_b(plan):
    """j, k, i order: each B tile moved in once per (j, k) and retained across
    all m / 16 row tiles, whose accumulators stay live (backend.py:295-324)."""
    it, jt = plan["m"] // DIM, plan["n"] // DIM
    return _walk(plan, [(j, tuple(range(it))) for j in range(jt)], False)


def gen_commands(plan):
    """The plan's own schedule (backend.py:327-330)."""
    return gen_baseline(plan) if plan["schedule"] == "baseline" else gen_reuse_b(plan)


def gen_batched_reuse_b(plan, batch_rows):
    """reuse_b over batches of `batch_rows` row tiles (the last batch may be
    shorter): B moved in once per (j, batch, k), batch_rows accumulator tiles
    live (lowering.py:18-40). The plan's schedule tag is not consulted; its
    accumulator_rows bound what the stream may touch, which the program
    check enforces, not this generator. Raises ValueError for an invalid plan
    or a batch that is not a positive int."""
    ok, why = _rp.validate_plan(plan)
    if not ok:
        raise ValueError(why)
    if type(batch_rows) is not int or batch_rows <= 0:
        raise ValueError("batch_rows must be a positive number of 16-row tiles")
    it, jt = plan["m"] // DIM, plan["n"] // DIM
    blocks = [(j, tuple(range(first, min(first + batch_rows, it))))
              for j in range(jt) for first in range(0, it, batch_rows)]
    return _walk(plan, blocks, False)


# ---------------------------------------------------------------------------
# Modeled counts (analytic, never a measurement)
# ---------------------------------------------------------------------------

_KINDS = ("config_ex", "config_ld", "config_st", "mvin", "preload", "compute", "mvout", "fence")


def modeled_counts(cmds):
    """Instruction and DMA counts of a stream (backend.py:330-356): per kind,
    A / B move-ins, preloaded / accumulated computes, int8 elements in, int32
    elements out, their bytes and the instruction total."""
    counts = dict.fromkeys(_KINDS, 0)
    counts.update(mvin_A=0, mvin_B=0, compute_preloaded=0, compute_accumulated=0)
    elems_in = elems_out = 0
    for c in cmds:
        kind = c["kind"]
        counts[kind] += 1
        if kind == "mvin":
            elems_in += c["rows"] * c["cols"]
            counts["mvin_" + c["buf"]] += 1
        elif kind == "mvout":
            elems_out += c["rows"] * c["cols"]
        elif kind == "compute":
            counts["compute_accumulated" if c["accumulated"] else "compute_preloaded"] += 1
    counts["dma_in_elems_int8"] = elems_in
    counts["dma_out_elems_int32"] = elems_out
    counts["dma_bytes"] = elems_in + 4 * elems_out
    counts["instructions"] = len(cmds)
    return counts


def modeled_objective(counts):
    """Least modeled DMA bytes, then fewest instructions (backend.py:359-362)."""
    return counts["dma_bytes"], counts["instructions"]


def optimize(m, n, k, *, scratchpad_rows=_rp.SCRATCHPAD_ROWS, accumulator_rows=_rp.ACC_ROWS):
    """Both schedules at the same target capacities, each plan validated and
    its generated stream put through `check_program`; the winner has the least
    modeled objective, then the fewest required accumulator rows
    (backend.py:1072-1093, with the program check standing in for the Lean
    plan check). Returns {"candidates": [...], "winner": plan or None}."""
    candidates = []
    for schedule in SCHEDULES:
        plan = make_plan(m, n, k, schedule)
        plan.update(scratchpad_rows=scratchpad_rows, accumulator_rows=accumulator_rows)
        ok, reason = _rp.validate_plan(plan)
        entry = {"plan": plan, "valid": ok, "invalid_reason": None if ok else reason,
                 "check": {"accepted": False, "reason": reason}, "counts": None,
                 "objective": None}
        if ok:
            cmds = gen_commands(plan)
            accepted, why, _ = check_program(plan, cmds)
            entry["check"] = {"accepted": accepted, "reason": why}
            if accepted:
                entry["counts"] = modeled_counts(cmds)
                entry["objective"] = modeled_objective(entry["counts"]) + \
                    (_rp.required_resources(plan)[1],)
        candidates.append(entry)
    eligible = [c for c in candidates if c["objective"] is not None]
    winner = min(eligible, key=lambda c: c["objective"])["plan"] if eligible else None
    return {"candidates": candidates, "winner": winner}


# ---------------------------------------------------------------------------
# Symbolic program check (translation validation against the GEMM)
# ---------------------------------------------------------------------------

EXECUTION_REJECTED = ("instruction execution rejected: check addresses, strides, "
                      "initialization, preload and retained weights")
NOT_DRAINED = "completion obligation failed: missing final fence"
OUTPUT_MISMATCH = ("GEMM output obligation failed: a cell is unwritten or its "
                   "input-product sequence differs from the specification")
ACCEPTED = "accepted"

_U32 = 1 << 32


class _Rejected(Exception):
    pass


def _nat(c, key):
    v = c[key]
    if not _rp._is_int(v) or v < 0:
        raise _Rejected("%s.%s must be a natural number" % (c["kind"], key))
    return v


def _tile_fits(row, capacity):
    return row % DIM == 0 and row + DIM <= capacity


def _acc_address(addr, capacity):
    """Accumulator space (bit 31), full-C width (bit 29) and an aligned
    in-range tile below bit 29 (Engine.lean:28-31)."""
    return addr < _U32 and addr >> 31 == 1 and (addr >> 29) & 1 == 1 and \
        _tile_fits(addr % (1 << 29), capacity)


class _Symbolic:
    """Engine.lean's state over symbolic values. A scratchpad tile is
    (buffer, offset, stride): element (r, c) is buffer[offset + r*stride + c].
    An accumulator tile is a tuple of (A tile, B tile) MACs, each adding
    A(r, t) * B(t, c) for t = 0..15 to cell (r, c) in that order. C cells
    record the mvout that last wrote them."""

    def __init__(self, plan):
        self.p = plan
        self.ws = False
        self.ld = {0: 0, 1: 0}
        self.st_stride = 0
        self.spad, self.acc = {}, {}
        self.pending = self.weights = None
        self.stores = []                                 # (acc tile, offset, stride)
        self.writer = np.full(plan["m"] * plan["n"], -1, np.int64)
        self.drained = True

    def step(self, c):
        kind = c.get("kind") if isinstance(c, dict) else None
        op = getattr(self, "_" + kind, None) if isinstance(kind, str) else None
        if op is None:
            raise _Rejected("unknown command kind %r" % (kind,))
        try:
            op(c)
        except KeyError as exc:
            raise _Rejected("%s command lacks field %s" % (kind, exc)) from None
        except TypeError:
            raise _Rejected("%s command has a field of the wrong type" % kind) from None

    def _config_ex(self, c):
        if c["dataflow"] != _rp.WEIGHT_STATIONARY:
            raise _Rejected("weight-stationary dataflow only")
        self.ws = True

    def _config_ld(self, c):
        if c["scale"] != 1.0:
            raise _Rejected("identity mvin scale only")
        slot, stride = c["slot"], _nat(c, "stride_bytes")
        if slot not in (0, 1):
            raise _Rejected("config_ld slot %r" % (slot,))
        self.ld[slot] = stride

    def _config_st(self, c):
        stride = _nat(c, "stride_bytes")
        if stride == 0 or stride % 4:
            raise _Rejected("config_st stride %d" % stride)
        self.st_stride = stride

    def _mvin(self, c):
        slot = c["slot"]
        if slot not in (0, 1):
            raise _Rejected("mvin slot %r" % (slot,))
        stride, buf = self.ld[slot], c["buf"]
        if buf not in ("A", "B"):
            raise _Rejected("mvin buffer %r" % (buf,))
        p = self.p
        size = p["m"] * p["k"] if buf == "A" else p["k"] * p["n"]
        off, row = _nat(c, "offset"), _nat(c, "spad_addr")
        if not (stride > 0 and c["cols"] == DIM and c["rows"] == DIM and
                off + 15 * stride + DIM <= size and _tile_fits(row, p["scratchpad_rows"])):
            raise _Rejected("mvin %s tile at %d (row %d)" % (buf, off, row))
        self.spad[row] = (buf, off, stride)
        self.drained = False

    def _preload(self, c):
        bd, out = _nat(c, "bd_spad_addr"), _nat(c, "out_addr")
        if not ((bd == GARBAGE_ADDR or _tile_fits(bd, self.p["scratchpad_rows"])) and
                _acc_address(out, self.p["accumulator_rows"])):
            raise _Rejected("preload operands")
        self.pending = (bd, out)

    def _compute(self, c):
        if not self.ws or c["bd_spad_addr"] != GARBAGE_ADDR or self.pending is None:
            raise _Rejected("compute without WS configuration, a pending preload and a garbage BD")
        b_row, out = self.pending
        a_tile = self.spad.get(c["a_spad_addr"])
        if c["accumulated"]:
            b_tile = self.weights if b_row == GARBAGE_ADDR else None
        else:
            b_tile = self.spad.get(b_row)
        if a_tile is None or b_tile is None:
            raise _Rejected("compute operand never moved in or no retained weights")
        row = out % (1 << 29)
        if (out >> 30) & 1:
            old = self.acc.get(row)
            if old is None:
                raise _Rejected("accumulation into an accumulator tile never computed")
        else:
            old = ()
        self.acc[row] = old + ((a_tile, b_tile),)
        self.weights, self.pending = b_tile, None
        self.drained = False

    def _mvout(self, c):
        p = self.p
        addr = _nat(c, "acc_addr")
        if c["cols"] != DIM or c["rows"] != DIM or self.st_stride == 0 or \
                not _acc_address(addr, p["accumulator_rows"]):
            raise _Rejected("mvout operands")
        stride, off = self.st_stride // 4, _nat(c, "buf_offset")
        if stride < DIM or off + 15 * stride + DIM > p["m"] * p["n"]:
            raise _Rejected("mvout range")
        tile = self.acc.get(addr % (1 << 29))
        if tile is None:
            raise _Rejected("mvout of an accumulator tile never computed")
        cells = off + (np.arange(DIM)[:, None] * stride + np.arange(DIM)[None, :]).reshape(-1)
        self.writer[cells] = len(self.stores)
        self.stores.append((tile, off, stride))
        self.drained = False

    def _fence(self, c):
        self.drained = True

    def first_wrong_cell(self):
        """Flat index of the first output cell that is unwritten or whose
        product sequence is not A[r, 0..k) . B[0..k), c] in order; None if
        there is none."""
        p = self.p
        n, k = p["n"], p["k"]
        bad = np.flatnonzero(self.writer < 0)
        worst = int(bad[0]) if bad.size else None
        rc = np.arange(DIM)
        for s in np.unique(self.writer[self.writer >= 0]):
            tile, off, stride = self.stores[s]
            cells = off + (rc[:, None] * stride + rc[None, :])       # (r, c) -> flat index
            mine = self.writer[cells] == s
            R, Cc = cells // n, cells % n
            ok = np.full(cells.shape, len(tile) * DIM == k)
            for j, ((abuf, aoff, astride), (bbuf, boff, bstride)) in enumerate(tile):
                # cell (r, c), t: A[aoff + r*astride + t] must be A[R*k + 16 j + t]
                # and B[boff + t*bstride + c] must be B[(16 j + t)*n + C], all t.
                if abuf != "A" or bbuf != "B" or bstride != n:
                    ok[:] = False
                    break
                ok &= (aoff + rc[:, None] * astride) == R * k + DIM * j
                ok &= (boff + rc[None, :]) == DIM * j * n + Cc
            wrong = cells[mine & ~ok]
            if wrong.size and (worst is None or wrong.min() < worst):
                worst = int(wrong.min())
        return worst


def check_program(plan, commands):
    """(accepted, reason, receipt) for a command stream under a Gemmini plan,
    the return shape of the reference's check_program (backend.py:989-997).
    Accepted: the plan is valid with dim 16, every command executes under
    Engine.lean's rules, the stream ends drained by a fence, and every output
    cell holds exactly its GEMM product sequence (Symbolic.lean:36-47). The
    reasons are the diagnostics of Symbolic.lean:39-47, with the failing
    command or cell appended. The receipt (None when refused) says what was
    checked; it is not a proof certificate, and the executable-byte half of
    the reference's check has no counterpart here."""
    ok, why = _rp.validate_plan(plan)
    if not ok:
        return False, why, None
    if not isinstance(commands, (list, tuple)):
        return False, EXECUTION_REJECTED + " (commands must be a list)", None
    s = _Symbolic(plan)
    for index, c in enumerate(commands):
        try:
            s.step(c)
        except _Rejected as exc:
            return False, "%s (command %d: %s)" % (EXECUTION_REJECTED, index, exc), None
    if not s.drained:
        return False, NOT_DRAINED, None
    cell = s.first_wrong_cell()
    if cell is not None:
        n = plan["n"]
        return (False, "%s (cell %d: row %d, col %d)" % (OUTPUT_MISMATCH, cell, cell // n, cell % n),
                None)
    m, n, k = plan["m"], plan["n"], plan["k"]
    return True, ACCEPTED, {"checker": "symbolic GEMM product sequences (Symbolic.lean:36-47)",
                            "commands": len(commands), "cells": m * n, "products_per_cell": k}
