"""Case tables of the reference accuracy harness (tests/mha/test_mha_paged_accuracy.py:17-70).

Each case is (label, batch, queries, heads, head_dim, page_size, table_width);
the tables are kept identical so results compare one to one.
"""
QUICK = [
    ("tiny", 2, 2, 2, 16, 16, 2),
    ("non_power_two_dim", 3, 4, 2, 80, 32, 3),
    ("wide_head", 2, 2, 4, 256, 128, 2),
]
STANDARD = QUICK + [
    ("single_decode", 1, 1, 8, 64, 128, 4),
    ("dim32", 4, 2, 4, 32, 32, 4),
    ("dim128", 2, 4, 4, 128, 64, 4),
    ("many_queries", 2, 8, 2, 64, 16, 8),
    ("many_requests", 8, 2, 2, 64, 64, 4),
    ("page256", 2, 2, 4, 128, 256, 4),
    ("cache2048", 2, 2, 2, 64, 128, 16),
]
EXTENDED = STANDARD + [
    ("dim48", 2, 2, 2, 48, 48, 3),
    ("dim96", 2, 4, 2, 96, 64, 8),
    ("dim192", 2, 2, 2, 192, 128, 4),
    ("cache4096", 2, 2, 2, 128, 256, 16),
    ("cache8192", 2, 2, 2, 64, 256, 32),
]
CUBE = [
    ("cube_decode512", 1, 1, 8, 128, 128, 4),
    ("cube_decode2048", 2, 1, 4, 128, 256, 8),
    ("cube_query4", 2, 4, 4, 128, 128, 16),
    ("cube_q127", 1, 127, 2, 128, 128, 2),
    ("cube_q128", 1, 128, 2, 128, 128, 2),
    ("cube_q129", 1, 129, 2, 128, 128, 2),
    ("cube_q257", 1, 257, 2, 128, 128, 2),
    ("cube_direct_q1", 2, 1, 64, 128, 128, 2),
    ("cube_direct_q129", 2, 129, 64, 128, 128, 2),
    ("cube_direct_q1024", 2, 1024, 8, 128, 128, 2),
]
GENERAL = [
    ("general_d16_page16", 2, 2, 2, 16, 16, 3),
    ("general_d32_q31", 2, 31, 2, 32, 32, 2),
    ("general_d48_page48", 2, 4, 2, 48, 48, 3),
    ("general_d64_q33", 2, 33, 2, 64, 64, 2),
    ("general_d80", 2, 17, 2, 80, 32, 3),
    ("general_d96", 2, 32, 2, 96, 64, 2),
    ("general_d128_q129", 2, 129, 2, 128, 128, 2),
    ("general_d192", 2, 4, 2, 192, 128, 2),
    ("general_d256", 2, 4, 2, 256, 256, 2),
    ("general_decode", 1, 1, 2, 128, 128, 2),
]
SPLIT = [
    ("split_d16_q1", 2, 1, 2, 16, 16, 64),
    ("split_d48_q17", 2, 17, 2, 48, 48, 24),
    ("split_d128_q33", 2, 33, 2, 128, 128, 8),
    ("split_d256_q129", 2, 129, 2, 256, 256, 4),
]
SEEDS = (7, 42, 2026)
PATTERNS = ("mixed", "full", "empty")
ALL_CASES = {c[0]: c for c in EXTENDED + CUBE + GENERAL + SPLIT}
