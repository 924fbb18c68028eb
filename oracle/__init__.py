"""CPU oracle for the transformer-layer forward path -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (the ``tkmi`` package and its HIP library) may import,
call or link anything here.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker.

Modules
-------
``baseline``  fp32 PyTorch-on-CPU restatement of the reference's
              ``BaselineTransformer`` and harness helpers
              (``src/torch_transformer_benchmark.py``), plus per-kernel
              references (LayerNorm, add+LayerNorm, GELU, attention,
              masked softmax) and the query-chunked / row-sampled long-S
              references.
``twin64``    an independent float64 brute-force twin of the forward, written
              from the equations rather than from ``torch.nn`` modules, used to
              bound the fp32 oracle's own error on tiny shapes.

How each function is pinned (golden vectors from the reference, closed forms,
float64 twin, invariants) is listed in the module docstrings and exercised by
``tests/test_oracle.py``.
"""
