"""Test-infrastructure package: the CPU oracle and the compiled reference.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may
import this package, and only as the checker.  The HIP product path never
imports it.
"""
