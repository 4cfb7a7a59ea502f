"""The 5-phase NSN builder (mars_nsn_edges; MemoryGraph::build_nsn_edges in the C++
shim) against the reference's own builder, src/memory_graph.cpp:102-189, compiled
into oracle/_ref: the same CSR, edge for edge, over sizes, k, p, phase subsets and
modality mixes. Host code, no GPU."""
from __future__ import annotations

import ctypes as C
import subprocess

import numpy as np
import pytest

import oracle
from conftest import ROOT
from mars_amd import corpus

needs_ref = pytest.mark.skipif(oracle.ref is None, reason="oracle/_ref not built (reference tree absent)")


def ref_nsn(mods, k, p, phases):
    mods = np.ascontiguousarray(mods, np.int32)
    n = len(mods)
    row = np.zeros(n + 1, np.int32)
    cap = 64 * max(n, 1)
    col = np.empty(cap, np.int32)
    e = oracle.ref.ref_nsn_edges(n, C.c_void_p(mods.ctypes.data), k, p, phases, C.c_void_p(row.ctypes.data),
                                 C.c_void_p(col.ctypes.data), cap)
    assert e <= cap
    return row, col[:e]


@needs_ref
@pytest.mark.parametrize("n", [1, 2, 3, 5, 16, 97, 1000, 4099, 65537])
@pytest.mark.parametrize("k,p", [(6, 0.15), (2, 0.0), (8, 0.5), (4, 1.0)])
def test_nsn_matches_reference(n, k, p):
    mods = np.random.default_rng(n + k).integers(0, 3, n).astype(np.int32)
    row, col = corpus.nsn_edges(mods, k, p)
    rrow, rcol = ref_nsn(mods, k, p, corpus.NSN_ALL)
    np.testing.assert_array_equal(row, rrow)
    np.testing.assert_array_equal(col, rcol)


@needs_ref
@pytest.mark.parametrize("phases", [0x1, 0x2, 0x4, 0x8, 0x10, 0x9, 0x1B, 0x17, 0x0])
def test_nsn_phase_subsets(phases):
    mods = np.random.default_rng(3).integers(0, 3, 3001).astype(np.int32)
    row, col = corpus.nsn_edges(mods, 6, 0.3, phases)
    rrow, rcol = ref_nsn(mods, 6, 0.3, phases)
    np.testing.assert_array_equal(row, rrow)
    np.testing.assert_array_equal(col, rcol)


@needs_ref
def test_nsn_single_modality_and_invariants():
    mods = np.full(500, 2, np.int32)                  # no other modality: no bridges
    row, col = corpus.nsn_edges(mods)
    rrow, rcol = ref_nsn(mods, 6, 0.15, corpus.NSN_ALL)
    np.testing.assert_array_equal(col, rcol)
    # undirected, no self edges, rows strictly ascending
    for i in range(500):
        r = col[row[i]:row[i + 1]]
        assert np.all(np.diff(r) > 0) and i not in r
        for j in r:
            assert i in col[row[j]:row[j + 1]]


def test_nsn_rejects_bad_modalities():
    from mars_amd._lib import MarsError
    with pytest.raises(MarsError):
        corpus.nsn_edges(np.int32([0, 1, 3]))
    row, col = corpus.nsn_edges(np.int32([0, 1, 3]), phases=corpus.NSN_ALL & ~corpus.NSN_BRIDGES)
    assert row[-1] == len(col)
