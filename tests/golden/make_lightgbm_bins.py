"""Writes ``lightgbm_bins_all_rows.json``: the ``feature_infos`` that LightGBM 3.3.5 recorded for the ``all_rows``
case of the reference's bin fixture (crates/silvic-core/src/data/fixtures/lightgbm_bins.json).

The fixture's features are built from silvic's ``mix32`` (gen_lightgbm_bins.py:54-99), and with 150,000 rows
LightGBM's bin sample is every row, so each numerical feature's ``[min:max]`` is the exact extreme of a column that
``mix32`` determines. Only these strings are kept: they are data, not code.

    python tests/golden/make_lightgbm_bins.py   # reads the reference checkout
"""

import json
import pathlib
import sys

SRC = pathlib.Path("/root/reference/crates/silvic-core/src/data/fixtures/lightgbm_bins.json")
OUT = pathlib.Path(__file__).with_name("lightgbm_bins_all_rows.json")


def main():
    src = json.loads(SRC.read_text())
    case = next(c for c in src["cases"] if c["name"] == "all_rows")
    out = {
        "source": "crates/silvic-core/src/data/fixtures/lightgbm_bins.json, case all_rows",
        "lightgbm": src["lightgbm"],
        "rows": case["rows"],
        "feature_infos": {f["name"]: f["feature_infos"] for f in case["features"]},
    }
    OUT.write_text(json.dumps(out, indent=2) + "\n")
    print(OUT)


if __name__ == "__main__":
    sys.exit(main())
