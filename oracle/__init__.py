"""CPU oracle of the LegoLink KV link step.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
CPU-baseline leg may import anything here, and only to check results (or, for
bench.py, as the timed CPU baseline).  The product package ``legolink_amd``
never imports it.

Modules:
  ll_oracle.c / kv_link_oracle.py   the fused link arithmetic (R2) in C and numpy
  r1_torch.py                       the reference's eager torch path (R1)
  link_maps_oracle.py               a link's token maps (plan order, repair rows, prefix)

Each module's docstring names the reference lines it restates; the tests that
pin it are tests/test_oracle_pins.py and tests/test_link_maps.py.
"""
