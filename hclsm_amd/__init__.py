"""hclsm_amd: MI355X (gfx950) native hot path of RightNow-AI/hclsm's hclsm/kernels.

``hclsm_amd.kernels`` mirrors the reference package ``hclsm.kernels`` (same names,
signatures and return types) and runs every call on hand-written HIP kernels in
``libhclsm_amd.so`` through the C ABI of ``include/hclsm_amd.h``.
"""

__version__ = "0.1.0"
