"""Copy the reference's request-contract fixtures and its option-label codebook into this repository.

    python tests/golden/make_contract_cases.py [/path/to/reference]

Both files are data held by the reference: tests/fixtures/contract_cases.json (48 requests with their
rows, rendered prompts, model probabilities and responses, plus 41 invalid requests; the reference's
tests/test_contract.py reads it) and mica/codebook_255.json (the 2 + 255 readout labels the model was
trained on).  They are rewritten as compact JSON with every value unchanged; nothing else is read.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parents[1] / "mica_amd"


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    ref = Path(argv[0]) if argv else Path("/root/reference")
    cases = json.loads((ref / "tests" / "fixtures" / "contract_cases.json").read_text(encoding="utf-8"))
    (HERE / "contract_cases.json").write_text(
        json.dumps(cases, ensure_ascii=False, separators=(",", ":")) + "\n", encoding="utf-8")
    book = json.loads((ref / "mica" / "codebook_255.json").read_text(encoding="utf-8"))
    (PKG / "codebook_255.json").write_text(json.dumps(book, ensure_ascii=False, indent=0) + "\n", encoding="utf-8")
    print(f"{len(cases['cases'])} cases, {len(cases['invalid'])} invalid requests; "
          f"{len(book['noul_labels'])} + {len(book['option_labels'])} labels")


if __name__ == "__main__":
    main()
