"""CPU restatement of the FlashLoop quantized-decode algorithm (test infrastructure only).

This package is the *checker* for the HIP kernels in ``flashloop_amd``.  It is imported
only by ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py``; the product path never imports it and fails loudly when the HIP library
is missing.

Every function cites the reference file:line it restates (paths relative to the
reference checkout of Superone77/FlashLoop v0.1.0).

Modules
-------
``codec``      int4 asymmetric min/max fake quantization and the residual chain
               (``flashloop_torch/kv_quantization.py``).
``attention``  dense decode attention, decode top-k, cached-mass sparse delta
               (``flashloop_torch/attention_utils.py``, ``flashloop/engine.py``).
``tokens``     token-sparse prefill selection and row gather/scatter
               (``flashloop_torch/token_updates.py``, ``flashloop/selection.py``).

Pinning status of each function is stated in its docstring ("pinned by: ...").
"""
