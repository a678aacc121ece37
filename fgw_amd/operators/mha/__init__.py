"""Paged multi-head attention operator (public entry: fgw_amd.operators.mha.current)."""
