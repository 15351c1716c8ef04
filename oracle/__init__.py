"""CPU oracle for the paged-KV decode path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithm of mlx-one's paged KV path
(``src/mlx_one/engine/paged.py`` and ``src/mlx_one/engine/paged_attention.py``)
so that the HIP implementation can be checked against it.  It is the checker,
never the thing measured or shipped:

* only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
  ``bench.py`` may import it;
* the product package (``mlx-one_amd/pkv``) never imports it and fails loudly
  when its HIP library is missing instead of falling back to this code.

Modules:

``numpy_ref``   numpy restatement: quantizer/dequantizer, reference page format,
                block-table gather, paged attention, log-sum-exp partition merge.
``cport``       ctypes loader for ``pkv_oracle.c`` (the same arithmetic in C, used
                for bit-exact quantization at full sizes and as the timed CPU
                baseline).

Parity status of each function (what pins it) is written in each docstring.
"""
