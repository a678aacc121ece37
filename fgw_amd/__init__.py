"""MI355X-native paged multi-head attention (drop-in for FGW's operators/mha).

Public entry: fgw_amd.operators.mha.current.{mha_paged_decode, build_kernel}.
Kernels: fgw_amd/csrc (HIP, gfx950), C ABI: include/fgw_mha.h.
"""
__version__ = "0.1.0"
