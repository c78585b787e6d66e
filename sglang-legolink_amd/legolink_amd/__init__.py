"""legolink_amd: the LegoLink KV link step on MI355X (gfx950).

Hand-written HIP kernels behind a C ABI (``include/legolink_kv.h``), driven by
a Python host layer that mirrors the reference's operator and link-executor
interfaces:

* ``legolink_amd.kv_link``       fused_kv_link_inplace & co. (legolink_triton.py)
* ``legolink_amd.link_plan``     imp_indices / block_ranges derivation
* ``legolink_amd.link_runtime``  the batched link executor over a KV pool
* ``legolink_amd.rope``          cos/sin table
* ``legolink_amd.workloads``     seeded synthetic link workloads
"""

__all__ = ["kv_link", "link_plan", "link_runtime", "rope", "workloads"]
