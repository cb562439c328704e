"""The evaluator (python -m oztt_amd.evaluate) against the reference's validated quick run
(tools/validated/quick.csv:2-17, values copied into QUICK below): Scheme I outputs are the
reference's bit for bit (hash, effective bits, relative error); every Scheme II format plans the
reference's moduli (Info), FP8 (on the FP8 matrix cores, by default) and INT8 run the reference's partial
products and the others the 15 INT8 products of b = 54; every Scheme II output is the exact rounding at
b = 54."""
import csv

import pytest

from oztt_amd import evaluate

pytestmark = pytest.mark.gpu

# format: (I hash, I effective bits, I relative Frobenius error, I partial products, II moduli, II products); the
# II products of the formats carried by INT8 residues are the 15 int8 products the device runs at b = 54
QUICK = {
    "BF16": ("be6558fa9f435fa0", "54.2420686589", "4.69364573273e-17", 55, 12, 15),
    "FP16": ("be6558fa9f435fa0", "54.2420686589", "4.69364573273e-17", 55, 11, 15),
    "TF32": ("be6558fa9f435fa0", "54.2420686589", "4.69364573273e-17", 55, 11, 15),
    "BFP8": ("be6558fa9f435fa0", "54.2420686589", "4.69364573273e-17", 55, 12, 15),
    "FP8": ("4d24add106258287", "54.2417946941", "4.69453713108e-17", 78, 12, 36),
    "INT8": ("6c9693442bfc11b0", "54.243846521", "4.68786522126e-17", 36, 15, 15),
    "BFP4": ("f353dbd6b57f8b99", "54.2426979466", "4.69159886276e-17", 136, 14, 15),
    "BFP2": ("13cd8e69edca2911", "54.2388822441", "4.70402383076e-17", 1770, 18, 15),
}


def test_quick_table_suite_matches_reference_records(tmp_path):
    """FP8 runs the FP8 route's digits on the FP8 matrix cores, as the reference runs them (its partial
    product count)."""
    out = tmp_path / "results.csv"
    assert evaluate.main(["--quick", "--suite", "table", "--output", str(out)]) == 0
    rows = list(csv.DictReader(open(out)))
    assert [r["format"] for r in rows[::2]] == list(QUICK) and len(rows) == 16
    ii_bits = set()
    for r in rows:
        h, eb, rel, pp, mod, pp2 = QUICK[r["format"]]
        assert r["suite"] == "table" and r["n"] == "128" and r["phi"] == "-1" and r["timing"] == "quick"
        assert float(r["total_ms"]) > 0 and float(r["effective_tflops"]) > 0
        if r["scheme"] == "I":
            assert (r["output_hash"], r["effective_bits"], r["relative_fro"]) == (h, eb, rel), r["format"]
            assert int(r["partial_products"]) == pp
        else:
            assert r["integer_bits"] == "54" and r["passes"] == "1"
            if mod is not None:
                assert (int(r["moduli"]), int(r["partial_products"])) == (mod, pp2), r["format"]
            ii_bits.add(r["effective_bits"])
            assert r["fp64_equivalent"] == "yes"
    # one exact C' at b = 54 for every format: one output, at least as accurate as the reference's best row
    assert len(ii_bits) == 1 and float(ii_bits.pop()) >= 54.2439488749
