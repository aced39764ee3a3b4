"""CPU oracle for the hilda-kernel_amd hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in plain PyTorch on the CPU, the reference
implementations that kirsten-1/hilda-kernel checks its Triton kernels
against (each function cites the reference file:line it follows), plus the
seeded input generators of the benchmark configurations.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed CPU
baseline. The product (``hilda-kernel_amd/kernels``) never imports it and has
no CPU path.

Pinning (what independently checks each function here) is listed in the
docstring of ``oracle.reference``; every function is pinned.
"""
from .reference import *  # noqa: F401,F403
