"""CPU oracle for the low-bit projection path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package.  See ``lowbit_oracle.py``.
"""
from .lowbit_oracle import *  # noqa: F401,F403
