"""Test infrastructure: the CPU parity oracle and the reference build.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this package.  The product package (``laii_amd``) never does.
"""
