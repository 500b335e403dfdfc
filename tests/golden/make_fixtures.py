"""Transcribe the reference's own data fixtures into JSON golden files.

Reads (as text) the reference's ``tests/fixtures/shared_monomial_plan_v1.txt``
and writes its numbers to ``shared_monomial_plan_v1.json``.  Run once in a
container where the reference tree is mounted; the JSON is committed.
"""
import json
import sys

ARRAYS = ("monomial_counts", "output_offsets", "coefficient_terms", "coefficient_outputs",
          "coefficient_values", "input", "output_adjoint", "expected_output", "expected_input_adjoint")


def main(src="/root/reference/tests/fixtures/shared_monomial_plan_v1.txt",
         dst="tests/golden/shared_monomial_plan_v1.json"):
    data = {}
    for line in open(src):
        parts = line.split()
        if not parts or parts[0] == "end":
            continue
        key, rest = parts[0], parts[1:]
        if key in ARRAYS:
            n, vals = int(rest[0]), rest[1:]
            assert len(vals) == n, key
            data[key] = [float(v) if ("." in v or "e" in v) else int(v) for v in vals]
        else:
            data[key] = rest[0] if len(rest) == 1 else rest
    data["_source"] = ("reference tests/fixtures/shared_monomial_plan_v1.txt "
                       "(data transcribed by tests/golden/make_fixtures.py)")
    json.dump(data, open(dst, "w"), indent=1)


if __name__ == "__main__":
    main(*sys.argv[1:])
