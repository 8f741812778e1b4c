"""The engine's page logic over the real HIP backend (tests/cpp/hip_engine_test.cpp, linked with libember_hip.so and
created through ember::create_backend("hip")): ten requests with fixed continuations run alone, then together on a
24-page cache (preemption and re-prefill, 40-token chunks, a shared system prompt from the prefix cache), then with
speculative verify (4 drafts, one in four wrong). Every logit row computed on a request's own context must equal the
alone run's within 2e-2 relative (rounding from the different kernel paths; a page or slot mistake moves it by O(1)),
recomputed rows likewise, and every page must be back in the pool at the end."""
import subprocess
from pathlib import Path

import pytest

from synthetic_model import write_model

pytestmark = pytest.mark.gpu

DRIVER = Path(__file__).resolve().parent / "cpp" / "_build" / "hip_engine_test"


def test_engine_page_logic_over_the_hip_backend(tmp_path):
    assert DRIVER.exists(), "build the C++ drivers first (__graft_entry__.build())"
    write_model(tmp_path, layers=4, vocab=8192)
    r = subprocess.run([str(DRIVER), str(tmp_path)], capture_output=True, text=True, timeout=240)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "hip engine ok" in r.stdout
