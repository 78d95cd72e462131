"""CPU oracle for the parity tests (test infrastructure, not product code).

``oracle.ops`` restates Farx1/AKO's unfused reference operations in numpy.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker.
The reference itself is pure Python/PyTorch (no C or C++ path to compile),
so there is no ``oracle/_ref`` build.
"""

from oracle import ops

__all__ = ["ops"]
