"""Operators of the MI355X build (paged MHA)."""
