"""CPU oracle for the exact int8 x int8 -> int32 GEMM contract.

TEST INFRASTRUCTURE ONLY. Nothing in the product (``veritac_amd``,
``specializations``) imports, links or runs anything under ``oracle/``.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker or the timed CPU baseline.

Contents
--------
``gemm_oracle``  numpy / pure-Python restatements of the reference's scalar
                 oracles and deterministic input generators (each function
                 cites the reference file:line it restates).
``ref_gemm.c``   C restatement of the reference's emitted scalar kernel
                 ``veritac_scalar_ref`` with an optional initial partial sum
                 and OpenMP over output rows; built by ``oracle/Makefile``
                 into ``oracle/_build/libvt_oracle.so``.
``cref``         ctypes loader for that library.
``packed_b``     numpy restatement of the packed-B weight layout of the decode
                 path (include/vt_hip_gemm.h): pack, unpack, and the product
                 read under the MFMA operand convention.

Pinning (how each function is checked, see tests/test_oracle.py and
tests/test_packed_host.py):
  scalar_matmul / reference_matmul / gemm_i8 / ref_gemm.c
      - the 24 full-output Spike COUT vectors recorded by the reference
        (tests/golden/spike_cout.json, independent of the reference's Python);
      - the reference's hand known-answer tests (2x2 extrema, 2x2 mixed sign,
        [[19,22],[43,50]]);
      - brute force on tiny inputs, int64 matmul vs exact float64 BLAS,
        K-tiling invariance, a planted-mistake check (dropped partial sum).
  lcg8_stream / fill_inputs
      - the reference's own LCG known-answer test and the lcg COUT vectors.
  deterministic_inputs (every mode) / scalar_matmul
      - input/output vectors produced by the reference's own functions
        (tests/golden/lcg_inputs.json, written by
        tests/golden/make_lcg_vectors.py in the build container), which also
        tell the byte - 128 mapping from the two's-complement one;
      - the relation value = lcg8 byte - 128 for the same state sequence, and
        the C twin in ref_gemm.c (vt_ref_lcg_fill), which computes the value
        by a different formula (top bit flipped, read as int8).
  packed_b.pack_b / unpack_b / gemm_from_packed
      - round trip on ragged shapes; the product read under the
        v_mfma_i32_16x16x64_i8 operand convention equals the closed-form A.B;
        three planted layout mistakes fail both checks.
"""
