"""The reference's own kids-ball sweep driver (demos/embodied_scene/bench_kids_sweep.cu),
built by oracle/Makefile against this repository's drop-in headers (include/mars) and
libmars_amd.so, run unchanged apart from its two CUDA runtime calls.

The driver builds the kids corpus and NSN graph with the reference's host code, queries
256 IMAGE probes per N in {1K, 5K, 10K, 20K, 50K} through query_memory_fast for three
variants and writes its JSON summary (bench_kids_sweep.cu:700-745). Bars:
  * it runs to completion and writes every variant and N;
  * episode-scoped hit@15 is 1.0 at every N (the published value);
  * global hit@15 at 1K / 5K / 10K equals the oracle's on the same corpus, probes and
    configuration (the driver prints four decimals);
  * the 0.24 same-episode boost leaves the global hit rate unchanged, as published.
"""
from __future__ import annotations

import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle
from test_gpu_kids_sweep import D, kids_graph

ROOT = Path(__file__).resolve().parents[1]
DRIVER = ROOT / "oracle" / "_ref" / "bench_kids_sweep"

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not DRIVER.exists(), reason="oracle/_ref/bench_kids_sweep not built "
                                                             "(reference tree absent when the library was built)"),
              pytest.mark.skipif(oracle.ref is None, reason="oracle/_ref not built (reference tree absent)")]


def oracle_global_hit(n):
    """hit@15 of the global variant over the sweep's probes, from the oracle
    (bench_kids_sweep.cu:589-676: IMAGE probes, t = ts + 0.001 p, top_k 15, 96 results)."""
    emb, mods, ts, ep, row, col = kids_graph(n)
    og = oracle.make_graph(emb, mods, ts, row, col, ep)
    ocfg = oracle.config(15, 2, 8e-6, 0.55, -1, 96)
    img = np.nonzero(mods == 2)[0]
    probes = img[oracle.kids_probes(n, len(img), 256)]
    hits = 0
    for p, node in enumerate(probes):
        t = float(np.float32(ts[node]) + np.float32(p) * np.float32(0.001))
        ids = [r[0] for r in oracle.query(og, emb[node], t, ocfg)["results"]][:15]
        ms = {int(mods[v]) for v in ids if ep[v] == ep[node]}
        hits += 0 in ms and 1 in ms
    return hits / len(probes)


def test_reference_kids_driver(tmp_path):
    out = tmp_path / "sweep.json"
    r = subprocess.run([str(DRIVER), str(out)], cwd=tmp_path, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    doc = json.loads(out.read_text())
    assert doc["embedding_dim"] == D and doc["top_k"] == 15 and doc["num_probes_per_n"] == 256
    rows = {v["name"]: {c["N"]: c for c in v["configurations"]} for v in doc["variants"]}
    assert set(rows) == {"global_baseline", "global_episode_boost_0.24", "episode_scoped_no_bfs"}
    for name, by_n in rows.items():
        assert sorted(by_n) == [1000, 5000, 10000, 20000, 50000], name
        for n, c in by_n.items():
            print(f"{name} N={n}: wall p99 {c['wall_p99_ms']:.4f} ms, kernel p99 {c['kernel_p99_ms']:.4f} ms, "
                  f"hit@15 {c['episode_cross_modal_hit_rate_top15']:.4f}")
            assert c["wall_p99_ms"] > 0.0
    for n, c in rows["episode_scoped_no_bfs"].items():
        assert c["episode_cross_modal_hit_rate_top15"] == 1.0, n
    for n, c in rows["global_baseline"].items():
        assert (rows["global_episode_boost_0.24"][n]["episode_cross_modal_hit_rate_top15"] ==
                c["episode_cross_modal_hit_rate_top15"]), n
    for n in (1000, 5000, 10000):
        want = oracle_global_hit(n)
        got = rows["global_baseline"][n]["episode_cross_modal_hit_rate_top15"]
        assert abs(got - want) <= 5e-5, (n, got, want)
