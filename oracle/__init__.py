"""CPU oracle for the quantized-decode path (test infrastructure only).

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this package, always as the checker.  The shipped library
(``ironmill_amd``) never imports it.
"""
from .oracle import *  # noqa: F401,F403
