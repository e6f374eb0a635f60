"""The oracle: CPU restatements of the reference's algorithms. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import, call, link or execute anything here, and only as the checker
or the host baseline that is timed beside the GPU. The product package,
``nanocompile_amd``, never imports it and has no CPU fallback.

* ``reference.py``: NumPy restatement (quantizers, the per-token projection,
  rms_norm in both the reference's order and the GPU's stated order).
* ``nc_host.c`` (built by ``build.py`` into ``_lib/libnc_host.so``): the host
  C int8 path, both the bit-level oracle for fused-multiply-add orders that
  NumPy cannot express and the CPU baseline ``bench.py`` times.
"""
