"""Current paged MHA entry: hand-written CDNA4 kernels for MI355X.

Drop-in for the reference's operators/mha/current.py:7-9, which re-exports
build_kernel and mha_paged_decode of its default kernel module.
"""
from fgw_amd.operators.mha.kernels.mha_paged_decode_hip import build_kernel, mha_paged_decode

__all__ = ["build_kernel", "mha_paged_decode"]
