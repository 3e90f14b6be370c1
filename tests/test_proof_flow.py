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
