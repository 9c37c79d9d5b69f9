"""CPU restatement of the reference's block-sparse attention hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the
checker or the reported CPU baseline.  The product (``dit_sparse_atten_amd``)
never imports it and has no CPU fallback.

Modules and the reference code each follows:
  attention     masked block-sparse softmax attention (flex.py:379-399,
                sparse.py:670-751), float64 closed form
"""
