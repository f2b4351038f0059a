"""In-launch hand-offs between workgroups against kernel boundaries
(tests/probe/si_handoff, test-only): every bounded wait ends without a
timeout, the counter protocol leaves its counters reset and the generation
protocol raises every workgroup's word once per launch.  The timings it
prints are the measured cost of each hand-off protocol."""
import json
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "probe", "si_handoff")


def test_handoff_protocols_end_and_stay_consistent():
    import torch  # noqa: F401  (the HIP runtime on this box; the probe runs on its own)
    assert os.path.exists(EXE), f"{EXE} missing: run __graft_entry__.build()"
    reps = 50
    r = subprocess.run([EXE, str(reps)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0
    rows = [json.loads(line) for line in r.stdout.splitlines() if line.startswith("{")]
    assert len(rows) == 3
    for row in rows:
        assert row["timeouts"] == 0, row
        assert row["counters_left"] == 0, row
        assert row["flag_generations"] == [6 * reps, 6 * reps], row
        assert row["us_four_kernels"] > 0 and row["us_one_launch_flags"] > 0
