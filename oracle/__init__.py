"""CPU oracle of the FP16 blocked-layout tensor path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker: the product
path (``thintnpu_amd``, ``thin_backend``) never imports, calls or links it.

Modules (each function cites the reference file:line it restates):
  numerics   -- fp16 ulp distance, floored relative error, bit views
  elementwise-- binary / sigmoid / SiLU / fused chains via PyTorch CPU
  movement   -- cat, upsample, NC1HWC0 pack/unpack, strided copies (numpy)
  reductions -- softmax, DFL softmax and expectation via PyTorch CPU
  selection  -- YOLO26 score keys, half->float bits, stable two-stage top-K

Pinning status of every function is listed in its module docstring.
"""
