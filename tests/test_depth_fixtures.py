"""CPU: the engine's recorded runs at the 36-layer benchmark shapes whose teacher forcing is too
long for a GPU test -- config 4 (B=32 x 2048, 8 rows of 32, 8 tokens) and config 5 (B=4 x 8192,
all 4 rows, 32 tokens, tree verification with random drafts and plain decode) -- against the
CPU oracle teacher-forced on exactly those ids.

tests/golden/engine_runs.json holds the ids, recorded on MI355X by record_engine_runs.py;
tests/golden/depth.json "teacher" holds, per step, the oracle's top-2 gap and the emitted id's
deficit under the oracle's maximum along the engine's own prefix (make_depth_golden.py).  The
north-star token rule at 36 layers (tests/helpers.py): where the gap exceeds DEPTH_TIE the id is
the oracle's argmax; elsewhere it lies within DEPTH_TIE of it; and the near-tie substitutions
stay within the measured disagreement rate of two valid oracle restatements.
tests/test_gpu_depth.py checks that the engine still emits these ids.
"""

import json
import os

import pytest

from helpers import DEPTH_TIE, GOLDEN, allowance_bound

DEPTH = json.load(open(os.path.join(GOLDEN, "depth.json")))
RUNS = json.load(open(os.path.join(GOLDEN, "engine_runs.json")))


def _records():
    for name in ("config4", "config5"):
        t = DEPTH.get("teacher", {}).get(name)
        if t is None:
            continue
        for rec in t["rows"]:
            for kind in ("plain", "tree"):
                if kind in rec:
                    yield name, rec["row"], kind, rec[kind]


def test_teacher_records_cover_the_recorded_runs():
    assert "teacher" in DEPTH, "depth.json lacks the teacher-forced records"
    seen = {(n, r, k) for n, r, k, _ in _records()}
    assert {("config5", r, k) for r in range(4) for k in ("plain", "tree")} <= seen
    assert len([s for s in seen if s[0] == "config4"]) >= 8
    for name, row, kind, rec in _records():
        assert rec["tokens"] == RUNS[name][kind][row], (name, row, kind)
        assert len(rec["steps"]) == RUNS[name]["N"]
        assert DEPTH["teacher"][name]["engine_runs_library_sha256"] == RUNS["library_sha256"]


@pytest.mark.parametrize("name", ["config4", "config5"])
def test_recorded_runs_pass_the_margin_rule(name):
    steps = used = 0
    worst = 0.0
    for n, row, kind, rec in _records():
        if n != name:
            continue
        for i, st in enumerate(rec["steps"]):
            steps += 1
            if st["gap"] > DEPTH_TIE:
                assert st["deficit"] == 0, (name, row, kind, i, st)
            else:
                assert st["deficit"] <= DEPTH_TIE, (name, row, kind, i, st)
                used += st["deficit"] > 0
            worst = max(worst, st["deficit"])
    print(f"{name}: {steps} teacher-forced steps, near-tie substitutions {used} "
          f"(bound {allowance_bound(steps)}), worst deficit {worst:.4f}")
    assert steps > 0 and used <= allowance_bound(steps)
