"""Accuracy against the reference kernel's own records (MI355X only).

Every check the reference recorded in its accuracy reports (987 of them:
tests/golden/accuracy_report_ratios.json, written by
tests/golden/make_report_vectors.py from reports/mha/latest) is rerun on the
HIP kernel with the same seeded inputs (the harness recipe,
tests/mha/test_mha_paged_accuracy.py:73-101, :232-238): every one passes the
reference tolerances, the largest error / tolerance ratio is the reference's
own (0.639), and check by check the ratios agree on geometric mean. The
suite's worst BF16 checks, outside the reference's reports (causal CUBE
cases), reach the ratios that the reference's rounding points alone give
(oracle rounded_reference).
"""
import json
import math
import pathlib

import pytest
import torch

from oracle import mha_oracle as O
from tests import mha_cases as C

pytestmark = pytest.mark.gpu

RATIOS = pathlib.Path(__file__).with_name("golden") / "accuracy_report_ratios.json"


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    torch.cuda.set_device(0)


def _ratio(name, seed, dtype, causal, pattern, rtol, atol):
    from fgw_amd.operators.mha.current import mha_paged_decode
    case = C.ALL_CASES[name]
    q, k, v, table = O.make_inputs(case, seed, dtype)
    lengths = torch.tensor(O.lengths_for(case, pattern, seed), dtype=torch.int32)
    k, v = O.poison_unread(k, v, table, lengths, case[5])
    got = mha_paged_decode(*[x.cuda() for x in (q, k, v, table, lengths)], page_size=case[5],
                           is_causal=causal).cpu()
    exp = O.chunked_reference(q, k, v, table, lengths, case[5], causal, 128)
    return ((got.float() - exp.float()).abs() / (atol + rtol * exp.float().abs())).max().item(), (
        q, k, v, table, lengths, case[5], exp)


def test_every_recorded_reference_check():
    checks = json.loads(RATIOS.read_text())["checks"]
    assert len(checks) == 987
    ours, pairs = [], []
    for c in checks:
        r, _ = _ratio(c["case"], c["seed"], getattr(torch, c["dtype"]), c["causal"], c["pattern"],
                      c["rtol"], c["atol"])
        assert r <= 1.0, (c, r)
        ours.append(r)
        if c["max_tolerance_ratio"] > 0.05:
            pairs.append(r / c["max_tolerance_ratio"])
    ref_max = max(c["max_tolerance_ratio"] for c in checks)
    geo = math.exp(sum(map(math.log, pairs)) / len(pairs))
    not_above = sum(o <= c["max_tolerance_ratio"] for o, c in zip(ours, checks))
    print(f"reference checks: ours max {max(ours):.4f}, reference max {ref_max:.4f}, "
          f"ours / reference geomean {geo:.4f} over {len(pairs)}, ours <= reference on "
          f"{not_above} of {len(checks)}", flush=True)
    assert max(ours) <= ref_max + 0.005
    assert geo <= 1.02


@pytest.mark.parametrize("name,seed,causal,pattern", [
    ("cube_direct_q129", 42, True, "mixed"),
    ("cube_direct_q1024", 7, True, "mixed"),
    ("cube_q257", 2026, True, "full"),
])
def test_worst_suite_checks_are_the_rounding_points(name, seed, causal, pattern):
    rtol, atol = O.TOLERANCES[torch.bfloat16]
    r, (q, k, v, table, lengths, page, exp) = _ratio(name, seed, torch.bfloat16, causal, pattern,
                                                     rtol, atol)
    emu = O.rounded_reference(q, k, v, table, lengths, page, causal)
    r_emu = ((emu.float() - exp.float()).abs() / (atol + rtol * exp.float().abs())).max().item()
    print(f"{name} seed {seed}: kernel {r:.4f}, reference rounding points {r_emu:.4f}", flush=True)
    assert abs(r - r_emu) <= 0.01
