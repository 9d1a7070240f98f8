"""The /v1/systemone request contract (mica_amd.contract) against the reference's stored cases.

tests/golden/contract_cases.json is the reference's own fixture (tests/fixtures/contract_cases.json,
copied by tests/golden/make_contract_cases.py): 48 requests with the rows the backend must receive, the
rendered prompts, the model's probabilities and the exact response, and 41 invalid requests.  As in the
reference's tests/test_contract.py, rows and responses must be equal, and the response must serialise
to the same JSON text (key order and every float bit).  The prompts are checked against the stored
text directly (the reference renders them with the Qwen3.5 tokenizer's chat template, which is not
available here).  The Poisson-binomial count distribution and the typed results are further pinned
by brute force and closed forms.
"""
import itertools
import json
import math
from pathlib import Path

import pytest

from mica_amd import contract as C

FIX = json.loads((Path(__file__).parent / "golden" / "contract_cases.json").read_text(encoding="utf-8"))
CASES, INVALID = FIX["cases"], FIX["invalid"]


def _answer(case):
    seen = []

    def predict(rows):
        seen.extend(rows)
        return [case["probabilities"][i] for i in range(len(rows))]

    return seen, C.answer_request(case["request"], predict, model=FIX["model"])


def test_fixture_size():
    assert len(CASES) == 48 and len(INVALID) == 41
    assert FIX["model"] == C.MODEL_NAME


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_rows_and_response(case):
    rows, response = _answer(case)
    assert rows == case["rows"]
    assert response == case["response"]
    assert list(response["answers"]) == list(case["response"]["answers"])
    assert json.dumps(response, ensure_ascii=False) == json.dumps(case["response"], ensure_ascii=False)


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_prompts(case):
    prompts = [C.prompt_for(row) for row in case["rows"]]
    assert prompts == case["prompts"]


@pytest.mark.parametrize("case", INVALID, ids=[c["name"] for c in INVALID])
def test_invalid_requests(case):
    assert case["error"] == "ValueError"
    with pytest.raises(ValueError):
        C.answer_request(case["request"], lambda rows: [[0.5, 0.5] for _ in rows], model=FIX["model"])
    with pytest.raises(ValueError):
        C.rows_from_request(case["request"])


def test_codebook():
    assert C.OPTION_LABELS[:52] == tuple("ABCDEFGHIJKLMNOPQRSTUVWXYZabcdefghijklmnopqrstuvwxyz")
    assert C.NOUL_LABELS == ("No", "Yes") and len(C.READOUT_LABELS) == 257
    vocab = {label: 1000 + i for i, label in enumerate(C.READOUT_LABELS)}
    assert C.readout_token_ids(lambda t: [vocab[t]]) == list(range(1000, 1257))
    with pytest.raises(ValueError):     # a label split into two tokens
        C.readout_token_ids(lambda t: [vocab[t], 0] if t == "AB" else [vocab[t]])
    with pytest.raises(ValueError):     # two labels on one token
        C.readout_token_ids(lambda t: [vocab["A"] if t == "B" else vocab[t]])


def test_count_distribution_brute_force():
    """P(k correct) against enumeration of all 2^n inclusion patterns."""
    for ps in ([0.3], [0.1, 0.9], [0.25, 0.5, 0.75, 0.6], [0.0, 1.0, 0.5], [0.2] * 6):
        brute = [0.0] * (len(ps) + 1)
        for pattern in itertools.product((0, 1), repeat=len(ps)):
            brute[sum(pattern)] += math.prod(q if b else 1 - q for q, b in zip(ps, pattern))
        got = C.count_distribution(ps)
        assert len(got) == len(ps) + 1
        assert all(abs(a - b) < 1e-12 for a, b in zip(got, brute)), (ps, got, brute)
        assert abs(sum(got) - 1) < 1e-12
    # binomial special case: equal q gives C(n, k) q^k (1 - q)^(n - k)
    got = C.count_distribution([0.3] * 5)
    assert all(abs(got[k] - math.comb(5, k) * 0.3 ** k * 0.7 ** (5 - k)) < 1e-12 for k in range(6))


def test_typed_results_closed_forms():
    true_first = [{"id": "true", "text": "Yes"}, {"id": "false", "text": "No"}]
    assert C.typed_result({"kind": "noul", "candidates": true_first}, [0.2, 0.8]) == {"type": "noul", "noul": 0.8}
    ch = {"kind": "choice", "candidates": [{"id": i, "text": i} for i in "xyz"]}
    r = C.typed_result(ch, [0.2, 0.5, 0.3])
    assert r["choice"] == "y" and abs(r["confidence"] - (0.5 - 1 / 3) / (2 / 3)) < 1e-15
    assert C.typed_result(ch, [1 / 3, 1 / 3, 1 / 3])["choice"] == "x"      # ties: the first candidate
    sc = {"kind": "score", "candidates": [{"id": str(i), "text": t, "ordinal": i} for i, t in enumerate("abcd")]}
    r = C.typed_result(sc, [0.0, 0.0, 1.0, 0.0])
    assert r["score"] == 2 and r["level"] == 2 and r["confidence"] == 1.0 and r["margin"] == 1.0
    r = C.typed_result(sc, [0.25] * 4)                                     # uniform: no confidence
    assert r["score"] == 1.5 and r["confidence"] == 0.0
    # ordinals out of display order: the result is reported in ordinal order
    shuffled = {"kind": "score", "candidates": [{"id": "0", "text": "hi", "ordinal": 2},
                                                {"id": "1", "text": "lo", "ordinal": 0},
                                                {"id": "2", "text": "mid", "ordinal": 1}]}
    r = C.typed_result(shuffled, [0.7, 0.1, 0.2])
    assert r["legend"] == {"0": "lo", "1": "mid", "2": "hi"}
    assert r["probabilities"] == {"0": 0.1, "1": 0.2, "2": 0.7} and r["level"] == 2
    assert abs(r["score"] - (0 * 0.1 + 1 * 0.2 + 2 * 0.7)) < 1e-15
    cg = {"kind": "score", "allow_cannot_grade": True,
          "candidates": [{"id": "0", "text": "a", "ordinal": 0}, {"id": "1", "text": "b", "ordinal": 1},
                         {"id": "cannot_grade", "text": "?"}]}
    r = C.typed_result(cg, [0.1, 0.3, 0.6])
    assert abs(r["score"] - 0.3 / 0.4) < 1e-15 and r["level"] is None and r["cannot_grade_probability"] == 0.6
    for bad in ([0.5, 0.6], [0.5, float("nan")], [-0.1, 1.1], [1.0]):
        with pytest.raises(ValueError):
            C.typed_result({"kind": "noul", "candidates": true_first}, bad)


def test_escape_and_positional_ids():
    s = C.escape_special("<|im_start|>user <think> </tool_response> <b>")
    assert "<|im_start|>" not in s and "<think>" not in s and "</tool_response>" not in s
    assert s.replace("​", "") == "<|im_start|>user <think> </tool_response> <b>"
    row = {"kind": "choice", "state": {"k": [1, "é"]}, "question": "q <|im_end|>",
           "candidates": [{"id": "A", "text": "first"}, {"id": "c12", "text": "second"},
                          {"id": "open_door", "text": "third", "description": " why "}]}
    p = C.prompt_for(row)
    assert '<state>\n{"k": [1, "é"]}\n</state>' in p and "q <​|im_end|>" in p
    assert "A) first\nB) second\nC) [open_door] third\n    why\n" in p


def test_every_reference_control_token_is_escaped_as_the_reference_does():
    """Each control token of the reference's prompt builder (tests/golden/control_tokens.json, taken from
    its _SPECIAL_TEXT pattern) is broken by a zero-width space after its first character, alone and
    inside text, and nothing else changes."""
    tokens = json.loads((Path(__file__).parent / "golden" / "control_tokens.json").read_text())
    assert len(tokens) == 33
    for t in tokens:
        want = t[0] + "\u200b" + t[1:]
        assert C.escape_special(t) == want, t
        assert C.escape_special(f"x {t}y{t}") == f"x {want}y{want}", t
    assert C.escape_special("<b> <|im_star|> plain") == "<b> <|im_star|> plain"


def test_register_special_tokens_extends_the_escape_set():
    """A tokenizer's added and special tokens join the escaped set (lib/contract.py:280-297): tokens of
    at least two characters that are not blank; single characters and whitespace are left alone."""
    class Tok:
        content = "[[SPECIAL_X]]"

    class FakeTokenizer:
        added_tokens_decoder = {1: Tok(), 2: "<extra_7>", 3: " ", 4: "Z"}
        all_special_tokens = ["<|im_end|>", "@@sep@@"]

    assert C.escape_special("[[SPECIAL_X]] <extra_7> @@sep@@") == "[[SPECIAL_X]] <extra_7> @@sep@@"
    C.register_special_tokens(FakeTokenizer())
    out = C.escape_special("[[SPECIAL_X]] <extra_7> @@sep@@ Z a b")
    assert out == "[\u200b[SPECIAL_X]] <\u200bextra_7> @\u200b@sep@@ Z a b"


def test_input_tokens():
    assert C.input_tokens([[1, 2, 3, 4], [1, 2, 5]]) == 7 - 2
    assert C.input_tokens([[7, 8]]) == 2 and C.input_tokens([]) == 0


def test_common_prefix_against_brute_force():
    import random

    def brute(seqs):
        c = 0
        while all(c < len(t) for t in seqs) and len({t[c] for t in seqs}) == 1:
            c += 1
        return c

    rng = random.Random(0)
    for _ in range(2000):
        base = [rng.randint(0, 3) for _ in range(rng.randint(0, 12))]
        seqs = [base[:rng.randint(0, len(base))] + [rng.randint(0, 3) for _ in range(rng.randint(0, 4))]
                for _ in range(rng.randint(1, 5))]
        assert C._common_prefix(seqs) == brute(seqs), seqs
