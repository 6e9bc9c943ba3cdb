"""CPU oracle for the route n-gram memory hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm of the route n-gram
memory (``ffnmem/memory``) and its self-drafting readers (``drafting/``).  It is
the checker the HIP kernels are compared against, and (for ``bench.py``'s
``cpu_baseline`` leg) the CPU path that is timed beside them.  Nothing in the
product package imports it; the product fails loudly when its HIP library is
missing instead of falling back here.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import, call, link or execute anything under ``oracle/``.

Modules
-------
- ``oracle.memory``   : codes, n-gram addresses, rows, route tokens, the memory
                        readout in the reference's op order (fp64 / fp32 / bf16),
                        router features, diagonal SSM.
- ``oracle.drafting`` : draft head, greedy/top-k drafter, code-keyed online
                        counts, tree structure / verify gather / acceptance.
- ``oracle.cint``     : ctypes loader of the C restatement of the integer parts
                        (``oracle/c/oracle_int.c``), built by ``oracle/Makefile``.
- ``oracle.cdrafter`` : ctypes loader of the C++ CPU drafter port
                        (``oracle/c/cpu_drafter.cpp``), the drafter CPU baseline.

Parity pinning (what checks each function against something other than itself)
is listed in each function's docstring and exercised in ``tests/test_oracle_*.py``.
"""
