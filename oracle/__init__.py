"""CPU oracle for the native Qwen2 stage forward -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may use
this package, and only as the checker. The product (jetsonfabric_amd) never
imports it.
"""
from .jfo import *  # noqa: F401,F403
