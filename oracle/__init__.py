"""CPU oracle for the W4A16 MoE hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference's W4A16
mixture-of-experts path (``hybrid_agent/quantization.py`` and the router in
``hybrid_agent/backends.py``).  It exists to check the HIP implementation in
``hybridagent_amd``; it is never the thing measured or shipped.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker / CPU baseline.  The
product path (``hybridagent_amd``) never imports this package and has no CPU
fallback.

Pinning status of every function is listed in ``oracle/w4a16_oracle.py``'s
module docstring.
"""
from .w4a16_oracle import *  # noqa: F401,F403
