"""CPU oracle for the wide-row workloads -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker / CPU baseline.
The product (``credit_amd``) never imports it and has no CPU fallback.

``oracle.reference`` restates every workload of the reference
(zhengxiongli08/CREDIT, ``dsmem_eval/workloads.py:40-154`` and the fp64
verifiers in ``src/workloads/*.cu``) and every BASELINE configuration in
float64 numpy.  How each function is pinned is listed in
``oracle/reference.py``'s module docstring; the pins themselves live in
``tests/test_oracle.py``.
"""
