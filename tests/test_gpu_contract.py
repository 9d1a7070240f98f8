"""Requests end to end on the GPU: /v1/systemone request -> rows -> prompts -> tokens -> the prefill
engine (W8A8 stack, last-position label readout) -> typed answers.

The stack is a small random one with the reference model's layer computation, so the probabilities
mean nothing; what is checked is the plumbing
around them: every stored request gets a response with the stored answer ids, types and order; each
answer is the typed result of that row's own distribution, computed by running its prompt alone
(batching, padding and duplicate removal do not change a bit); Noul rows read the No / Yes slice and
Choice / Score rows the first n option labels; the usage count is the prompts' tokens with the common
prefix once; and a prompt longer than the limit is refused.  Tokens are UTF-8 bytes (no tokenizer
files are available); the stack's readout ids are a seeded sample of its vocabulary.
"""
import json
import sys
from pathlib import Path

import pytest
import torch

from mica_amd import contract as C
from mica_amd.engine import PrefillEngine
from mica_amd.model import StackConfig, W8A8Stack

pytestmark = pytest.mark.gpu

FIX = json.loads((Path(__file__).parent / "golden" / "contract_cases.json").read_text(encoding="utf-8"))


def _tokenize(text):
    return list(text.encode("utf-8"))


@pytest.fixture(scope="module")
def judge(gpu):
    # the reference model's computation at a small size: a GDN layer, then a full-attention layer with the
    # q_proj output gate, q / k head norm and partial RoPE (StackConfig.reference_model)
    cfg = StackConfig.reference_model(layers=2, hidden=512, intermediate=1024, heads=4, kv_heads=1, head_dim=256,
                                      vocab=4096, n_options=255, full_attention_interval=2, linear_k_heads=2,
                                      linear_v_heads=4)
    st = W8A8Stack(cfg, device=gpu, seed=11)
    return C.EngineJudge(PrefillEngine(st, graph=False), _tokenize, max_length=32768, max_batch=8)


def _alone(judge, row):
    """The row's distribution from its prompt run by itself (batch 1)."""
    ids = torch.tensor(_tokenize(C.prompt_for(row)), dtype=torch.long).to(judge.engine.device)
    kind = "noul" if row["kind"] == "noul" else "choice"
    n = 2 if kind == "noul" else len(row["candidates"])
    _, probs = judge.engine([ids], [kind], [n])
    return [float(v) for v in probs[0, :n].float().cpu().tolist()]


@pytest.mark.parametrize("case", FIX["cases"], ids=[c["name"] for c in FIX["cases"]])
def test_request_end_to_end(judge, case):
    print(f"[case] contract end to end {case['name']}", file=sys.stderr, flush=True)
    response = C.answer(case["request"], judge)
    want = case["response"]["answers"]
    assert list(response["answers"]) == list(want)
    for qid, ans in response["answers"].items():
        assert ans["type"] == want[qid]["type"] and set(ans) == set(want[qid]), qid
    rows = C.rows_from_request(case["request"])
    judged = [r for r in rows if not r.get("multi")] + [x for r in rows if r.get("multi") for x in C.inclusion_rows(r)]
    assert response["usage"] == {"input_tokens": C.input_tokens([_tokenize(C.prompt_for(r)) for r in judged]),
                                 "output_tokens": 0}
    dists = {r["id"]: _alone(judge, r) for r in judged}
    for r in rows:
        if r.get("multi"):
            incl = {x["multi_option"]: dists[x["id"]][1] for x in C.inclusion_rows(r)}
            assert response["answers"][r["id"]] == C.assemble(r, incl)
        else:
            expect = C.response_envelope([r], [dists[r["id"]]], model=C.MODEL_NAME)["answers"][r["id"]]
            assert response["answers"][r["id"]] == expect, r["id"]


def test_duplicate_questions_scored_once(judge):
    q = {"type": "choice", "instructions": "Which?", "criteria": {"a": "left", "b": "right", "c": "up"}}
    req = {"state": "s", "questions": {"x": q, "y": dict(q), "z": {"type": "noul", "instructions": "Is it?"}}}
    calls = []
    engine_call = judge.engine.__call__

    class Counting:
        def __init__(self, eng):
            self.eng, self.device, self.stack = eng, eng.device, eng.stack

        def __call__(self, reqs, kinds, counts, prefix=None):
            calls.append(len(reqs))
            return engine_call(reqs, kinds, counts, prefix=prefix)

    j2 = C.EngineJudge(Counting(judge.engine), _tokenize, max_length=32768)
    out = C.answer(req, j2)
    assert calls == [2]                                  # x and y share one readout
    assert out["answers"]["x"] == out["answers"]["y"]
    assert abs(sum(out["answers"]["x"]["probabilities"].values()) - 1) < 1e-5


def test_input_too_long(judge):
    short = C.EngineJudge(judge.engine, _tokenize, max_length=64)
    with pytest.raises(C.InputTooLongError):
        C.answer({"state": "s", "questions": {"q": {"type": "noul", "instructions": "i"}}}, short)


def test_questions_about_one_state_share_its_prefix(judge):
    """Several questions about one long state: the prompts' common start (system message and state)
    runs once, and every answer equals the one from its prompt run alone."""
    state = "Inventory log. " + " ".join(f"item {i}: {i * 7 % 13} units" for i in range(60))
    req = {"state": state, "questions": {
        "a": {"type": "noul", "instructions": "Is item 3 in stock?"},
        "b": {"type": "choice", "instructions": "Which item has most units?", "criteria": {"x": "item 1", "y": "item 2"}},
        "c": {"type": "score", "instructions": "How full is the store?", "criteria": ["empty", "half", "full"]}}}
    out = C.answer(req, judge)
    assert judge.shared_tokens >= 2 * 512
    for r in C.rows_from_request(req):
        expect = C.response_envelope([r], [_alone(judge, r)], model=C.MODEL_NAME)["answers"][r["id"]]
        assert out["answers"][r["id"]] == expect, r["id"]
