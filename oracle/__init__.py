"""CPU oracle for the routed E8P expert path -- TEST INFRASTRUCTURE ONLY.

Nothing in ``keep_amd`` imports, links or runs anything from this package.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and only as the checker (or, for ``cpu_baseline``,
as the timed CPU restatement), never as the thing measured or shipped.

Modules:

- ``oracle.e8p``  -- E8P / E8 codebooks and decoders, restated from
  ``src/keep/vq/e8.py`` of the reference.
- ``oracle.rht``  -- random-sign Walsh-Hadamard transform, restated from
  ``src/keep/quant/rht.py``.
- ``oracle.ops``  -- dense float64 reference of every hot-path operator
  (projection mat-vec, routed gather, verify rows, sorted routes, nested
  tier, router, SwiGLU, MoE layer, route plan).
- ``oracle.cpu``  -- ctypes loader for ``cpu_ref.c``, the C/OpenMP
  restatement that decodes on the fly (the timed CPU baseline).

Parity status of each function is stated in its docstring; every function
here is pinned by a reference golden vector, a closed form or a brute-force
check in ``tests/test_oracle_*.py`` unless its docstring says
"parity unpinned".
"""
