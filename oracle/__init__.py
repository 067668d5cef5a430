"""CPU oracle for the DeepSeek-V4-Flash MoE hot path (TEST INFRASTRUCTURE ONLY).

Nothing in the product path imports this package.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use it, and
only as the checker (or the timed CPU baseline), never as the measured path.
"""

from .moe_oracle import *  # noqa: F401,F403
