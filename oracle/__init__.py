"""CPU oracle for the fused-MoE hot path.

This package is TEST INFRASTRUCTURE. Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
answer GPU results are compared with (or the timed CPU baseline). The product path in ``flashinfer_amd``
never imports it and has no CPU fallback.
"""
