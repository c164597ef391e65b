"""CPU oracle for the quantized-matmul path -- TEST INFRASTRUCTURE ONLY.

This package is the checker that the HIP library is held against. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it, and there only
to check or to time the reference algorithm; the product path (``splosh_amd``) never imports it.
"""
from .oracle import *  # noqa: F401,F403
