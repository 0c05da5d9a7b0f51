"""CPU oracle for the quantibbler-kernels hot paths (TEST INFRASTRUCTURE ONLY).

The checker the parity tests, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg compare the HIP library against.  The shipped package
``quantibbler_amd`` never imports this module.
"""
from .oracle import *  # noqa: F401,F403
