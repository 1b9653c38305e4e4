"""Test-side loop-nest rewrites: the tactics of the reference's Lean CLI
(README.md:492-503: tile / reorder / parallel / vectorize / unroll), restated
on the JSON so the emitter can be checked on transformed nests without Lean.
Only the tests use these."""
import copy


def _subst(node, var, repl):
    if isinstance(node, dict):
        if node.get("tag") == "var" and node.get("name") == var:
            return copy.deepcopy(repl)
        return {k: _subst(v, var, repl) for k, v in node.items()}
    if isinstance(node, list):
        return [_subst(v, var, repl) for v in node]
    return node


def _lit(v):
    return {"tag": "lit", "val": v}


def _find(stmt, var, fn):
    """Apply fn to the loop over `var` (returns a new tree)."""
    if stmt.get("tag") == "loop":
        if stmt["var"] == var:
            return fn(stmt)
        return dict(stmt, body=_find(stmt["body"], var, fn))
    if stmt.get("tag") == "seq":
        return dict(stmt, s1=_find(stmt["s1"], var, fn), s2=_find(stmt["s2"], var, fn))
    if stmt.get("tag") == "alloc":
        return dict(stmt, body=_find(stmt["body"], var, fn))
    return stmt


def tile(stmt, var, size):
    """Split loop `var` (0 <= var < H, H % size == 0) into var_outer / var_inner."""
    def split(loop):
        assert loop["lo"] == _lit(0) and loop["hi"]["tag"] == "lit"
        hi = loop["hi"]["val"]
        assert hi % size == 0
        outer, inner = var + "_outer", var + "_inner"
        idx = {"tag": "add", "left": {"tag": "mul", "left": {"tag": "var", "name": outer},
                                      "right": _lit(size)},
               "right": {"tag": "var", "name": inner}}
        body = _subst(loop["body"], var, idx)
        return {"tag": "loop", "var": outer, "lo": _lit(0), "hi": _lit(hi // size),
                "ann": loop.get("ann", "none"),
                "body": {"tag": "loop", "var": inner, "lo": _lit(0), "hi": _lit(size),
                         "ann": "none", "body": body}}
    return _find(stmt, var, split)


def reorder(stmt, outer, inner):
    """Swap loop `outer` with the loop `inner` directly inside it."""
    def swap(loop):
        child = loop["body"]
        assert child["tag"] == "loop" and child["var"] == inner
        return dict(child, body=dict(loop, body=child["body"]))
    return _find(stmt, outer, swap)


def annotate(stmt, var, ann):
    return _find(stmt, var, lambda loop: dict(loop, ann=ann))
