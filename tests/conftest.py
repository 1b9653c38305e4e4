import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def golden():
    import json
    with open(os.path.join(ROOT, "tests", "golden", "spike_cout.json")) as fh:
        return json.load(fh)


@pytest.fixture(scope="session")
def commands():
    import json
    with open(os.path.join(ROOT, "tests", "golden", "gemmini_commands.json")) as fh:
        return json.load(fh)["streams"]


@pytest.fixture(scope="session")
def output_digests():
    import json
    with open(os.path.join(ROOT, "tests", "golden", "output_digests.json")) as fh:
        return json.load(fh)["runs"]


def winner_stream(streams, run_name):
    """The certified command stream of a recorded blind-search run."""
    name = "blind_search/%s/certification/winner" % run_name
    return next(s for s in streams if s["name"] == name)


def witness_inputs(stream):
    """The recorded counterexample input of a rejection witness: flat int8
    lists, all zero except the listed A / B indices, which are one."""
    p = stream["plan"]
    A = [0] * (p["m"] * p["k"])
    B = [0] * (p["k"] * p["n"])
    for buf, idx in stream["witness"]["sparse_inputs"]["ones"]:
        (A if buf == "a" else B)[idx] = 1
    return A, B


def decode_cout(hex_text):
    """8 hex digits per int32 (run_raw_spike.py:409-423 parse rule)."""
    vals = []
    for i in range(0, len(hex_text), 8):
        w = int(hex_text[i:i + 8], 16)
        vals.append(w - (1 << 32) if w >= (1 << 31) else w)
    return vals
