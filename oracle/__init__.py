"""CPU oracle (test infrastructure only).

ctypes bindings over two CPU libraries built by ``oracle/Makefile``:

* ``liboracle.so`` -- this repository's C restatement of the reference CPU path
  (``oracle/oracle.c``), the checker the GPU parity tests compare against;
* ``_ref/libaffref.so`` -- the reference's own sources compiled where they lie, plus a
  C-ABI forwarder (``oracle/ref_shim.cpp``); present only where it was built.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this package, and only as the checker. The product package ``affinity_amd`` never
imports it and fails loudly when its HIP library is missing.
"""
from .binding import Oracle, RefLib, load_oracle, load_ref, ref_available, build  # noqa: F401
