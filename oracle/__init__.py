"""CPU oracle for the RWKV7 hot path -- TEST INFRASTRUCTURE, never shipped.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or as the timed
CPU baseline). The HIP library and its Python host code never import it.

``oracle.rwkv7_ref`` restates yuyi2439/rwkv-tl's pure-torch model
(``demo/rwkv7_torch.py``, ``src/rwkv_tl/weight.py``, ``src/rwkv_tl/state.py``,
``demo/_rwkv7_abc.py``). Every function there cites the reference lines it
follows and the tests that pin it. ``oracle.sampling_ref`` restates the
reference's token sampling (``demo/sampling.py``) and the sampling kernel's
counter-based draw (Philox4x32-10), as the checker of ``rwkv7_sample``.
``oracle.quant_ref`` is the float64 checker of the int8 weight-only GEMV
(``rwkv7_gemv_i8``) and of the per-row int8 quantisation it reads.
"""
