"""CPU oracle for the fused-MoE path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker: the product path
(``vllm-xpu-kernels_amd/``) never imports it and fails loudly when its HIP
library is missing.
"""
