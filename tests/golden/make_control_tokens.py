"""Extract the control tokens the reference's prompt builder escapes into a fixture.

    python tests/golden/make_control_tokens.py [/path/to/reference]

Reads v0.5/serving/lib/contract.py as text (nothing is imported or run), takes the string literal of
its _SPECIAL_TEXT pattern (lib/contract.py:266-268), splits the alternation and writes the token list
to tests/golden/control_tokens.json.
"""
from __future__ import annotations

import ast
import json
import re
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    ref = Path(argv[0]) if argv else Path("/root/reference")
    text = (ref / "v0.5" / "serving" / "lib" / "contract.py").read_text(encoding="utf-8")
    m = re.search(r"_SPECIAL_TEXT = re\.compile\(\s*('(?:[^'\\]|\\.)*')\s*\)", text)
    pattern = ast.literal_eval(m.group(1))
    tokens = [re.sub(r"\\(.)", r"\1", alt) for alt in re.split(r"(?<!\\)\|", pattern)]
    (HERE / "control_tokens.json").write_text(json.dumps(sorted(tokens), indent=0) + "\n", encoding="utf-8")
    print(f"{len(tokens)} control tokens")


if __name__ == "__main__":
    main()
