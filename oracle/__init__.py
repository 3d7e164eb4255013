"""Test infrastructure: CPU restatement of the reference Mamba-3 hot path.

This package is the *checker*, never the product. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The product package ``mamba3_amd`` never imports it and has no CPU
fallback: its hot path runs only through the HIP library.

Modules:

* ``oracle.portable`` -- op-for-op restatement of the reference's portable
  PyTorch path (``mamba3/ops.py`` and ``mamba3/model.py`` of jreoka/mamba3),
  with the same low-precision rounding points, as pure functions over a
  parameter dictionary.
* ``oracle.recurrence`` -- an independent float64 per-token recurrence
  (numpy) used to pin the chunked scan, in the spirit of the reference's
  ``tests/test_scan.py:21-98``.

Pinning status of every function is listed in the header of each module.
"""
