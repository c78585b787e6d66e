"""CPU oracle of the LegoLink KV link step.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
CPU-baseline leg may import anything here, and only as the checker (or, for
bench.py, as the timed CPU baseline).  The product package ``legolink_amd``
never imports it.

Modules:
  ll_oracle.c / kv_link_oracle.py   the fused link arithmetic (R2) in C and numpy
  r1_torch.py                       the reference's eager torch path (R1)

Parity status of each function (how it is pinned) is listed in DESIGN.md.
"""
