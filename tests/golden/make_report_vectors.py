"""Extract the accuracy-harness vectors the reference recorded in its reports.

Reads JSON reports under /root/reference/reports/mha/latest (data only; no
reference code is imported or run) and writes accuracy_report_vectors.json:
one entry per distinct (case, seed, pattern) with the shape, pool rows and the
per-request cache lengths the reference's harness generated
(tests/mha/test_mha_paged_accuracy.py:73-101, :219-222). These pin the
oracle's lengths_for / make_inputs restatements. It also writes
accuracy_report_ratios.json: every recorded check (case, seed, dtype, causal,
pattern) with the reference kernel's max error / tolerance ratio at the
harness tolerances (test_mha_paged_accuracy.py:259-273), the figures this
build's accuracy is compared with check by check.

Run once in the build container: python tests/golden/make_report_vectors.py
"""
import json
import pathlib
import sys

REPORTS = pathlib.Path("/root/reference/reports/mha/latest")
SOURCES = (
    "mha_cube_general_accuracy.json",
    "mha_cube_general_boundaries.json",
    "mha_cube_general_smoke.json",
    "mha_paged_accuracy_v7_report.json",
    "mha_persistent28_causal.json",
)
OUT = pathlib.Path(__file__).with_name("accuracy_report_vectors.json")
RATIOS = pathlib.Path(__file__).with_name("accuracy_report_ratios.json")


def main() -> int:
    seen, vectors, ratios = set(), [], []
    for name in SOURCES:
        report = json.loads((REPORTS / name).read_text(encoding="utf-8"))
        for entry in report["results"]:
            shape = entry["shape"]
            if entry.get("status") == "passed" and "max_tolerance_ratio" in entry:
                ratios.append({
                    "source": name, "case": entry["case"], "seed": entry["seed"],
                    "dtype": entry["dtype"].replace("torch.", ""), "causal": entry["causal"],
                    "pattern": entry["pattern"], "rtol": entry["rtol"], "atol": entry["atol"],
                    "max_tolerance_ratio": entry["max_tolerance_ratio"],
                })
            key = (entry["case"], entry["seed"], entry["pattern"])
            if key in seen:
                continue
            seen.add(key)
            vectors.append({
                "source": name, "case": entry["case"], "seed": entry["seed"],
                "pattern": entry["pattern"], "B": shape["B"], "Sq": shape["Sq"], "H": shape["H"],
                "D": shape["D"], "page_size": shape["page_size"],
                "table_width": shape["table_width"], "pool_rows": shape["pool_rows"],
                "lengths": entry["lengths"],
            })
    OUT.write_text(json.dumps({"note": "extracted from the reference's recorded accuracy reports",
                               "vectors": vectors}, indent=1) + "\n", encoding="utf-8")
    print(f"wrote {len(vectors)} vectors to {OUT}")
    lines = ",\n".join(json.dumps(r, separators=(",", ":")) for r in ratios)
    RATIOS.write_text('{"note": "per-check max error / tolerance of the reference kernel, from '
                      'its recorded accuracy reports",\n"checks": [\n' + lines + "\n]}\n",
                      encoding="utf-8")
    print(f"wrote {len(ratios)} checks to {RATIOS}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
