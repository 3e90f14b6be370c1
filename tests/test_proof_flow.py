"""The grading flow end to end on the CPU: tests/grade_gpu.py's grade_op() writes one log
per runner -- a correct one and each planted one (tests/planted_kernels.py OracleKernel)
-- and grader/ledger.py turns the logs into the verdict table: the correct runner passes,
each plant carries its label, and regrading the stored logs gives the same table."""
import json

import pytest

from cob_amd.grader import ledger
from oracle import exact
from planted_kernels import EXPECT, OracleKernel
from grade_gpu import grade_op


def _key(fault, op):
    return f"{'correct' if fault is None else 'planted_' + fault}__{op}"


@pytest.mark.parametrize("op", ["reward_to_go", "ppo_clip"])
def test_proof_flow_on_cpu(tmp_path, op):
    for fault in EXPECT:
        entry = grade_op(op, OracleKernel(op, fault), exact.reference_exact, passes=1, device="cpu",
                         key=_key(fault, op), log=lambda m: None)
        (tmp_path / f"{entry['kernel']}.json").write_text(json.dumps(entry))
    rows = {r["kernel"]: r for r in ledger.tables(tmp_path)}
    assert len(rows) == len(EXPECT)
    for fault, (status, label) in EXPECT.items():
        r = rows[_key(fault, op)]
        assert (r["status"], r["label"]) == (status, label), r
    assert rows[_key("nonrepeatable", op)]["repeat_identical"] is False
    table = (tmp_path / "table.md").read_text()
    assert table.count("\n") == len(EXPECT) + 2
    ledger.tables(tmp_path, recompute=True)
    assert (tmp_path / "table.md").read_text() == table


def test_proof_record_on_cpu(tmp_path):
    """proof() of grade_gpu.py: the drop-in's verdict and each plant's expected and actual
    verdict, counted as graders/grade.py:228-253 counts them; a plant that draws the
    wrong label is not counted as expected."""
    from grade_gpu import proof, proof_table
    from cob_amd.grader.plants import KINDS
    op = "reward_to_go"
    entry = grade_op(op, OracleKernel(op, None), exact.reference_exact, passes=1, device="cpu",
                     key=f"taskops_{op}", log=lambda m: None)
    (tmp_path / f"{entry['kernel']}.json").write_text(json.dumps(entry))
    planted = {}
    for kind in KINDS:
        key = f"planted_{op}__{kind}"
        entry = grade_op(op, OracleKernel(op, None if kind == "none" else kind), exact.reference_exact, passes=1,
                         device="cpu", key=key, log=lambda m: None)
        (tmp_path / f"{key}.json").write_text(json.dumps(entry))
        planted[f"{op}/{kind}"] = (key, kind)
    rows = {r["kernel"]: r for r in ledger.tables(tmp_path)}
    res = proof(rows, {op: f"taskops_{op}"}, planted, EXPECT, {"gpu": "cpu"})
    assert res["summary"] == {"references_pass": 1, "references": 1,
                              "planted_as_expected": len(KINDS), "planted": len(KINDS)}
    assert res["planted"][f"{op}/cached_result"]["label"] == "stale state"
    assert res["planted"][f"{op}/nonrepeatable"]["repeat_identical"] is False
    table = proof_table(res)
    assert table.startswith(f"references_pass 1/1, planted_as_expected {len(KINDS)}/{len(KINDS)}")
    # a wrong-value plant that passes, or a nonrepeatable plant with identical repeats, is not as expected
    rows[f"planted_{op}__wrong_value"] = dict(rows[f"planted_{op}__wrong_value"], status="pass", label=None)
    rows[f"planted_{op}__nonrepeatable"] = dict(rows[f"planted_{op}__nonrepeatable"], repeat_identical=True)
    res = proof(rows, {op: f"taskops_{op}"}, planted, EXPECT, {"gpu": "cpu"})
    assert res["summary"]["planted_as_expected"] == len(KINDS) - 2
    assert "| NO |" in proof_table(res)
