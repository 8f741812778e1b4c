"""The engine's page logic over the real HIP backend (tests/cpp/hip_engine_test.cpp, linked with libember_hip.so and
created through ember::create_backend("hip")): ten requests with fixed continuations run alone, then together on a
24-page cache (preemption and re-prefill, 40-token chunks, a shared system prompt from the prefix cache), then with
speculative verify (4 drafts, one in four wrong). Every logit row computed on a request's own context must equal the
alone run's within 2e-2 relative (rounding from the different kernel paths; a page or slot mistake moves it by O(1)),
recomputed rows likewise, and every page must be back in the pool at the end.

The alone runs are themselves checked against the oracle: the driver dumps their sequences and logit rows, and the
oracle's forward pass (its rmsnorm, linear, append and attention composed with the GPU path's f16 roundings) of four
of the requests, teacher-forced, must give the same rows within 2e-2 (max |d| / max |oracle|, as the backend test)."""
import subprocess
from pathlib import Path

import numpy as np
import pytest

from synthetic_model import OracleModel, write_model

pytestmark = pytest.mark.gpu

DRIVER = Path(__file__).resolve().parent / "cpp" / "_build" / "hip_engine_test"


def _read_dump(path):
    raw = np.fromfile(path, dtype=np.int32)
    at = 0

    def take(n):
        nonlocal at
        out = raw[at:at + n]
        at += n
        return out

    seqs = []
    for _ in range(int(take(1)[0])):
        plen, n = (int(x) for x in take(2))
        seqs.append((plen, take(n).copy()))
    rows, vocab = (int(x) for x in take(2))
    rec = {}
    for _ in range(rows):
        req, pos = (int(x) for x in take(2))
        rec[(req, pos)] = take(vocab).view(np.float32).copy()
    return seqs, rec


def test_engine_page_logic_over_the_hip_backend(tmp_path):
    assert DRIVER.exists(), "build the C++ drivers first (__graft_entry__.build())"
    w = write_model(tmp_path, layers=4, vocab=8192)
    dump = tmp_path / "alone.bin"
    r = subprocess.run([str(DRIVER), str(tmp_path), str(dump)], capture_output=True, text=True, timeout=240)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "hip engine ok" in r.stdout

    seqs, rec = _read_dump(dump)
    om = OracleModel(w, num_blocks=32)
    table = np.arange(32, dtype=np.int32)[None, :]
    worst, checked = 0.0, 0
    for req in (0, 1, 2, 3):  # requests 0 and 3 start with the shared system prompt
        plen, seq = seqs[req]
        rows = sorted(p for (q, p) in rec if q == req)
        assert rows and rows[0] == plen, "the dump lacks the request's first sampled position"
        toks = seq[:rows[-1]]
        assert len(toks) <= 32 * 16
        want = om.forward(toks.tolist(), np.arange(len(toks), dtype=np.int32), table, [p - 1 for p in rows])
        for i, p in enumerate(rows):
            got = rec[(req, p)]
            err = float(np.abs(got - want[i]).max() / np.abs(want[i]).max())
            worst = max(worst, err)
            checked += 1
    print(f"alone runs against the oracle: {checked} logit rows, worst relative difference {worst:.3e}")
    assert worst < 2e-2
