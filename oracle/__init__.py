"""CPU integer oracle for the imie hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in plain numpy / Python big-ints (and a C/OpenMP twin in ``oracle/c``), the integer
algorithm of the reference engine's hot path:

* packed Q1_0 linear with the per-128-block floor and mod-2^64 wrap
  (``bonsai/src/trinote/infer_int/reference_bonsai.py:149-219``),
* fixed-point RMSNorm / 2^-f cubic softmax / sigmoid / SiLU
  (``bonsai/src/trinote/determinism/fixedpoint.py:31-179``),
* NeoX RoPE apply and the (YaRN) table builder (``bonsai/src/trinote/model/rope.py``, ``rope_v2.py``),
* fixed-point attention with its fail-loud bounds (``reference_bonsai.py:542-778``),
* the Q4_K / Q6_K integer codec and exact big-int linear (``north-mini-code/src/nmc/qk_codec.py``,
  ``north-mini-code/src/nmc/cohere2.py:102-188``).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this package, and
only as the checker. The product (``integer_inference_engine_amd``) never imports it and has no CPU fallback.

Pinning status of every function is listed in the module headers; a function whose only check would be a
retyping of its own formula is marked "parity unpinned" there.
"""
