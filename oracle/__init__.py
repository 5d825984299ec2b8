"""CPU oracle for the TESM forward hot path -- TEST INFRASTRUCTURE ONLY.

Nothing under ``tesm_amd/`` imports this package.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it,
and only as the checker (or as the timed CPU baseline), never as a code path of
the product.

Contents
--------
* ``tesm_torch``  -- a restatement of the reference's in-module torch fallback
  (``kernel_backend='torch'``) for BitLinear, TESM_SISO, TESMMIMO_Optimized and
  the LM harness around them (WANGLILIN360/tesm, ``tesm_ssm/modules/tesm.py``,
  ``tesm_mimo.py``, ``block.py``, ``models/mixer_seq_simple.py``).  Every function
  cites the reference lines it follows.  It is pinned against golden vectors
  written by ``tests/golden/gen_fixtures.py`` from the reference itself, and
  against closed forms / brute force (``tests/test_oracle_*.py``).
* ``int_ref.c``   -- plain-C restatement of the integer/byte work on the path:
  per-token int8 activation codes, ternary weight codes, the canonical INT2
  packing, and the exact int32 BitLinear accumulators.  Built by
  ``oracle/Makefile`` into ``oracle/_build/liboracle_int.so`` and loaded by
  ``oracle.int_ref``.
* ``int2_export`` -- the reference's INT2 export format (``pack_int2_to_uint8``,
  ``unpack_uint8_to_int2``, ``export_model_to_int2``), the checker of the hip
  export and loader.
* ``brute``       -- tiny pure-Python/numpy brute-force versions of the scan and
  of the local-window ternary entanglement, used to pin ``tesm_torch``.

The reference's CUDA sources (``csrc/tesm_ops/*.cu``) need nvcc and are not the
torch path, so no ``oracle/_ref`` build of them exists.
"""
