"""CPU oracle for the .gmdag sphere tracer — test infrastructure only.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker / CPU baseline. The
product path (``navi_amd``) never imports it.

Parity status of each function is listed in ``oracle/pyoracle.py``.
"""

from .pyoracle import *  # noqa: F401,F403
