"""CPU oracle for the MoE layer — TEST INFRASTRUCTURE ONLY (see moe_oracle.h).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package; the product (ffai_amd, libmoehip.so) never does.
"""
from .oracle import *  # noqa: F401,F403
from .oracle import build, lib  # noqa: F401
