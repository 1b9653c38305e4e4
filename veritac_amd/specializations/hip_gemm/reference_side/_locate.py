"""Find the veritac_amd checkout for the reference-side hip_gemm modules.

VT_HIP_GEMM_REPO names the directory that holds veritac_amd/. Without it,
or when that directory has no veritac_amd package, importing the backend
fails (fail-closed, like the reference's missing-checker rule,
specializations/gemmini_gemm/backend.py:172-175): no module of this
specialization runs anything else instead.
"""
import os
import sys


def add_repo_to_path():
    repo = os.environ.get("VT_HIP_GEMM_REPO", "")
    if not repo or not os.path.isfile(os.path.join(repo, "veritac_amd", "__init__.py")):
        raise ImportError("hip_gemm: VT_HIP_GEMM_REPO must name the checkout that holds "
                          "veritac_amd/ (got %r); fail-closed" % repo)
    repo = os.path.abspath(repo)
    if repo not in sys.path:
        sys.path.insert(0, repo)
    return repo
