"""genet5_amd — MI355X-native (gfx950) mixture-of-experts layer forward for GeneT5.

The drop-in module is `genet5_amd.moe.MoEFeedForward` (replaces FeedForward at
lib/blocks/encoder.py:69 of the reference); `genet5_amd.ops` holds functional
wrappers of each stage of the C ABI (include/g5moe.h), implemented by the HIP
kernels in genet5_amd/csrc and built into genet5_amd/libg5moe.so.
"""
__version__ = "0.1.0"
