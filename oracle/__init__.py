"""CPU oracle for the sparse-decode KV path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference's arithmetic on the CPU so that tests,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg can check
(or time, as a baseline) the HIP product.  The product never imports it.

* ``twilight_oracle.c`` -- scalar C restatement of the bit-exact parts (page
  metadata, INT4 pack/dequantize, Quest score order, top-k, row plan).
* ``oracle.py`` -- ctypes wrappers over the C library plus numpy float64
  references for the floating-point parts (decode attention).

Parity status of every function (what pins it) is recorded next to each
function and in the tests under tests/test_oracle_*.py.
"""

from .oracle import *  # noqa: F401,F403
