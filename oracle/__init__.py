"""Oracle for the fused forward-Laplacian path: TEST INFRASTRUCTURE ONLY.

CPU restatements of the reference algorithm (``jet``: numpy closed forms; ``torch_ref``:
PyTorch forward Laplacian, eager autograd and recompute backward). Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use this package, and only
as the checker or the timed CPU baseline; the product never imports it.
"""
