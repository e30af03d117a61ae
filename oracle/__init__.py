"""CPU oracle for the OSCAR INT2 KV-cache hot path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import this package, and only as the checker. The product package
``oscar_new_amd`` never imports it and has no CPU fallback.
"""

from .oscar_oracle import *  # noqa: F401,F403
