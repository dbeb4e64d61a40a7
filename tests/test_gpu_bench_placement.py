"""bench.py --placement on the GPU: separately allocated caches of one
configuration, each timed alone; one JSON line with every cache's addresses
and a positive us/step (a child process, as a user would run it)."""
import json
import os
import subprocess
import sys

import pytest

from _util import REPO

pytestmark = pytest.mark.gpu


def test_placement_mode_reports_every_cache():
    env = dict(os.environ)
    r = subprocess.run([sys.executable, "bench.py", "--placement", "2", "--placement-steps", "5", "--warmup", "10",
                        "--config", "cfg0"], cwd=REPO, env=env, capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stderr[-2000:]
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["mode"] == "placement" and line["steps_per_cache"] == 5
    assert [c["cache"] for c in line["caches"]] == [0, 1]
    for c in line["caches"]:
        assert int(c["k"], 16) > 0 and int(c["v"], 16) > 0 and c["us_per_step"] > 0
    assert line["caches"][0]["k"] != line["caches"][1]["k"]
