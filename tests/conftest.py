"""Shared fixtures. Tests marked ``gpu`` need an MI355X; the rest run on CPU."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"

# Tolerances (fp32 path): |gpu - oracle| <= RTOL * max(|oracle|, scale), where
# scale = w * sum_d |e_d q_d| bounds the rounding error of a length-D fp32 dot
# product; the oracle accumulates in fp64. fp16 rows: the oracle reads the
# same RNE-rounded rows, so the same bound holds; against the fp32 oracle the
# fp16 path must agree within 2e-3 of that scale.
RTOL_F32 = 1e-5
RTOL_F16_VS_F32 = 2e-3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def golden():
    return GOLDEN


@pytest.fixture(scope="session")
def corpus_small():
    """N=2,000 D=768 corpus of the benchmark generator with its NSN graph (seed 11)."""
    from mars_amd import corpus
    c = corpus.make_corpus(2000, 768, seed=11)
    return corpus.nsn_graph(c)


@pytest.fixture(scope="session")
def corpus_10k():
    """N=10,000 D=768 corpus (the CPU-reference plumbing size) with its NSN graph (seed 2026)."""
    from mars_amd import corpus
    c = corpus.make_corpus(10000, 768, seed=2026)
    return corpus.nsn_graph(c)


def near_tie_ok(ids_a, ids_b, score_of, kth_score, tol) -> bool:
    """Top-K id sets equal except for ids whose reference score is within tol of the cut."""
    diff = set(map(int, ids_a)) ^ set(map(int, ids_b))
    return all(abs(score_of(i) - kth_score) <= tol for i in diff)


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
