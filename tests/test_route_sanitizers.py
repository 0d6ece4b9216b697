"""The host route builder under AddressSanitizer and UndefinedBehaviorSanitizer (CPU).

route.cpp restates omniweave/models/routing.py:40-198 with index arithmetic on flat tables; a
build of it with g++ -fsanitize=address,undefined drives ~200K plans (tests/sanitize/
route_sanitize.cpp: every H, W in a grid of 15 sizes, three routes, four window / shift
pairs, radix levels 0-3, seven channel counts, three spatial and four channel tiles), checks
each token / channel / space_to_depth table is a permutation padded as documented, checks that
invalid plans and arguments fail with an error, and must finish with no sanitizer report.  The
tables of a few plans are compared with the oracle.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

from oracle.routing import build_route_plan

REPO = Path(__file__).resolve().parent.parent
SAN_FLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]
PLANS = [(14, 14, 512, 16, 128, "radix", 1), (56, 56, 128, 16, 64, "shifted", 0), (7, 7, 1024, 16, 128, "local", 0),
         (13, 9, 200, 3, 16, "radix", 3), (5, 6, 96, 16, 64, "shifted", 0)]
ROUTE_CODE = {"local": 0, "shifted": 1, "radix": 2}


@pytest.fixture(scope="module")
def driver(tmp_path_factory) -> Path:
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("route_san") / "route_san"
    cmd = [gxx, "-std=c++17", "-O1", "-g", *SAN_FLAGS, f"-I{REPO / 'include'}", f"-I{REPO / 'omniwave_amd' / 'csrc'}",
           str(REPO / "omniwave_amd" / "csrc" / "route.cpp"), str(REPO / "tests" / "sanitize" / "route_sanitize.cpp"),
           "-o", str(exe)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0 and ("asan" in proc.stderr.lower() or "ubsan" in proc.stderr.lower()):
        pytest.skip(f"sanitizer runtime not available: {proc.stderr[-300:]}")
    assert proc.returncode == 0, proc.stderr
    return exe


def test_route_builder_is_clean_under_sanitizers(driver) -> None:
    args = [str(v if not isinstance(v, str) else ROUTE_CODE[v]) for plan in PLANS for v in plan]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1", UBSAN_OPTIONS="halt_on_error=1")
    proc = subprocess.run([str(driver), *args], capture_output=True, text=True, env=env, timeout=600)
    assert proc.returncode == 0, proc.stderr[-3000:]
    assert "ERROR: AddressSanitizer" not in proc.stderr and "runtime error" not in proc.stderr, proc.stderr[-3000:]
    lines = proc.stdout.splitlines()
    assert lines[0].startswith("tables ") and int(lines[0].split()[1]) > 100_000
    tables = [ln for ln in lines if ln.startswith("plan")]
    assert len(tables) == len(PLANS)
    for (h, w, c, g, d, route, level), line in zip(PLANS, tables):
        tok_s, ch_s = line[len("plan"):].split("|")
        plan = build_route_plan(h, w, c, g, d, route, level)
        assert [int(v) for v in tok_s.split()] == plan.token_indices.reshape(-1).tolist(), (h, w, c, route, level)
        assert [int(v) for v in ch_s.split()] == plan.channel_indices.reshape(-1).tolist(), (h, w, c, route, level)
