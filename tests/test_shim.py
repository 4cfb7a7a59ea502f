"""The reference-API C++ shim (include/mars/*.{h,cuh} + libmars_amd.so) driven by
tests/cpp/shim_driver.cpp, a driver written like the reference's own drivers."""
from __future__ import annotations

import subprocess

import numpy as np
import pytest

from conftest import ROOT

DRIVER = ROOT / "tests" / "cpp" / "shim_driver"


def test_shim_driver_host_checks():
    assert DRIVER.exists(), "built by mars_amd/build.py"
    r = subprocess.run([str(DRIVER), "host"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "host ok" in r.stdout, r.stdout + r.stderr


@pytest.mark.gpu
def test_shim_driver_matches_oracle():
    import oracle
    from mars_amd import corpus
    n, seed, q = 3000, 7, 12
    r = subprocess.run([str(DRIVER), "query", str(n), str(seed), str(q)], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    c = corpus.nsn_graph(corpus.make_corpus(n, 768, seed=seed))
    og = oracle.make_graph(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices, c.episode_ids)
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith(("global", "episode"))]
    assert len(lines) == 2 * q
    off = og.ep_offsets
    for ln in lines:
        head, tail = ln.split(" | ")
        parts = head.split()
        scope, node = parts[0], int(parts[1])
        res = [tuple(float(x) if i == 1 else int(x) for i, x in enumerate(p.split(":"))) for p in parts[2:]]
        ep = int(c.episode_ids[node])
        cfg = oracle.config(10, 2, 0.1, 0.5, -1, 15, 1 if scope == "episode" else 0, ep,
                            int(off[ep]) if scope == "episode" else 0,
                            int(off[ep + 1] - off[ep]) if scope == "episode" else 0)
        ref = oracle.query(og, c.embeddings[node], 600.0, cfg)
        want = ref["results"]
        assert len(res) == len(want)
        for got, w in zip(res, want):
            assert got[0] == w[0] or abs(got[1] - w[1]) <= 2e-5 * max(1.0, abs(w[1])), (scope, node, got, w)
            assert abs(got[1] - w[1]) <= 1e-5 * max(1.0, abs(w[1]))
        assert ("scanned=10 " in tail) == (scope == "episode")
        assert ("waves=0" in tail) == (scope == "episode")
