"""CPU oracle for the affine quantized-projection path (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the checker or the reported CPU baseline. The product path
(``metile_amd``) never imports it and fails loudly when its HIP library is missing.
"""
