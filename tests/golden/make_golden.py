"""Write the golden fixtures under tests/golden/ from the reference's own host code.

Runs in the build container only: it needs oracle/_ref/libref.so, which
oracle/Makefile compiles from the reference sources (src/memory_graph.cpp,
src/streaming.cpp) when the reference tree is present. The fixtures are data:
inputs and the reference's outputs.

  episode_csr.npz   build_episode_csr (src/memory_graph.cpp:12-44) on four id sets
  kids_small.npz    EmbodiedKidsBallCorpus::make(200, 64, 2026) + build_nsn_edges(6, 0.15)
                    (src/memory_graph.cpp:95-189, :241-295)
  stream_flush.npz  StreamingBuffer insert + flush of 10 nodes onto
                    MemoryGraph::synthetic(30,15,15,64) + NSN (src/streaming.cpp:13-163)

Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes as C
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle  # noqa: E402


def _p(a):
    return C.c_void_p(a.ctypes.data)


def ref_episode_csr(ids: np.ndarray):
    r = oracle.ref
    ids = np.ascontiguousarray(ids, np.int32)
    ne = C.c_int32()
    r.ref_build_episode_csr(_p(ids), len(ids), C.byref(ne), None, None)
    off = np.zeros(ne.value + 1, np.int32)
    mem = np.zeros(max(len(ids), 1), np.int32)
    m = r.ref_build_episode_csr(_p(ids), len(ids), C.byref(ne), _p(off), _p(mem))
    return ne.value, off, mem[:m]


def ref_graph_arrays(h):
    r = oracle.ref
    n, d, e = C.c_int32(), C.c_int32(), C.c_int32()
    r.ref_graph_sizes(h, C.byref(n), C.byref(d), C.byref(e))
    emb = np.zeros((n.value, d.value), np.float32)
    mods = np.zeros(n.value, np.int32)
    ts = np.zeros(n.value, np.float32)
    ep = np.zeros(n.value, np.int32)
    row = np.zeros(n.value + 1, np.int32)
    col = np.zeros(max(e.value, 1), np.int32)
    r.ref_graph_copy(h, _p(emb), _p(mods), _p(ts), _p(ep), _p(row), _p(col))
    return dict(emb=emb, mods=mods, ts=ts, ep=ep, row=row, col=col[: e.value])


def main() -> None:
    if oracle.ref is None:
        raise SystemExit("oracle/_ref/libref.so missing: run `make -C oracle` with the reference tree present")
    rng = np.random.default_rng(20261201)
    cases = {}
    # (a) the kids corpus ids of the reference test T19 (30 nodes)
    h = oracle.ref.ref_kids_make(30, 16, 99, 0, 0.0)
    cases["kids30"] = ref_graph_arrays(h)["ep"]
    oracle.ref.ref_graph_free(h)
    # (b) shuffled ids with empty episodes (gaps)
    cases["shuffled"] = rng.choice(np.arange(0, 97, 3), size=1000).astype(np.int32)
    # (c) one episode
    cases["single"] = np.zeros(7, np.int32)
    # (d) one node in episode 5 (episodes 0-4 empty)
    cases["one_node"] = np.array([5], np.int32)
    out = {}
    for name, ids in cases.items():
        ne, off, mem = ref_episode_csr(ids)
        out[f"{name}_ids"], out[f"{name}_num"] = ids, np.int32(ne)
        out[f"{name}_offsets"], out[f"{name}_members"] = off, mem
    np.savez_compressed(HERE / "episode_csr.npz", **out)

    h = oracle.ref.ref_kids_make(200, 64, 2026, 6, 0.15)
    g = ref_graph_arrays(h)
    oracle.ref.ref_graph_free(h)
    np.savez_compressed(HERE / "kids_small.npz", **g)

    h = oracle.ref.ref_synthetic_make(30, 15, 15, 64, 42, 6, 0.15)
    before = ref_graph_arrays(h)
    new_emb = rng.standard_normal((10, 64)).astype(np.float32)
    new_emb /= np.linalg.norm(new_emb, axis=1, keepdims=True)
    new_mods = (np.arange(10) % 3).astype(np.int32)
    new_ts = np.full(10, 2.0, np.float32)
    accepted = oracle.ref.ref_stream_flush(h, 64, 6, 10, _p(new_mods), _p(new_ts), _p(new_emb))
    after = ref_graph_arrays(h)
    oracle.ref.ref_graph_free(h)
    np.savez_compressed(HERE / "stream_flush.npz", accepted=np.int32(accepted),
                        **{f"before_{k}": v for k, v in before.items()},
                        **{f"after_{k}": v for k, v in after.items()},
                        new_emb=new_emb, new_mods=new_mods, new_ts=new_ts)
    print("wrote", *(p.name for p in sorted(HERE.glob("*.npz"))))


if __name__ == "__main__":
    main()
