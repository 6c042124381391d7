"""CPU oracle for the RFSN warm-tier quantized-KV decode path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``apple_amd`` imports this package.
It may be imported by ``tests/``, by ``__graft_entry__.smoke()`` (as the
checker) and by the ``cpu_baseline`` leg of ``bench.py`` (as the timed CPU
baseline).  It is never the thing measured on the GPU and never a fallback.

It restates, in numpy (and, for the timed baseline, torch-CPU), the
arithmetic of the reference files:

* ``quantization.py:92-157``  PQ distance, encode, decode        -> numerics.py
* ``quantization.py:206-275`` gated full-D RVQ encode/correction -> numerics.py
* ``quantization.py:305-319`` hybrid encode/decode               -> numerics.py
* ``quantization.py:330-403`` compressed-tensor helpers          -> numerics.py
* ``attention.py:16-105``     query positions, blockwise attention-> numerics.py
* ``cache.py:89-440``         tier fill, windows, stats, bytes   -> cache_model.py
* ``rfsn_v10_mlx_ane_complete.py:175-225`` PQ k-means           -> kmeans.py
* ``rfsn_v10_unified_mac_launcher.py:217-273`` torch-CPU form    -> cpu_baseline.py

Parity status per function is listed in each module's header.
"""
