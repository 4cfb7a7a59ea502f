"""Files on either side of the path: MARS v1 graph checkpoints (persistence.h:8-18)
and the KIDS binary corpus (bench_kids_sweep.cu:29-37).

Pinned by:
  * the published FNV-1a 64 test vectors ("", "a", "foobar");
  * the reference's own src/persistence.cpp (oracle/_ref: fnv1a_checksum, save_graph,
    load_graph): files written by either side are byte-identical, each side loads the
    other's files, and both reject the same damaged files;
  * the reference's KIDS reader layout (scripts/bench_kids_ball_cuvs_cagra.py:49-60),
    restated with numpy in read_kids_numpy below.
"""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np
import pytest

import mars_amd
import oracle
from mars_amd._lib import MarsError

FNV_VECTORS = [(b"", 0xCBF29CE484222325), (b"a", 0xAF63DC4C8601EC8C), (b"foobar", 0x85944171F73967E8)]
needs_ref = pytest.mark.skipif(oracle.ref is None, reason="oracle/_ref not built (reference tree absent)")


def _p(a):
    return C.c_void_p(a.ctypes.data)


def random_graph(rng, n, d, deg=6):
    deg_i = rng.integers(0, deg + 1, size=n)
    ro = np.zeros(n + 1, np.int32)
    ro[1:] = np.cumsum(deg_i)
    col = rng.integers(0, max(n, 1), size=int(ro[-1])).astype(np.int32)
    emb = rng.standard_normal((n, d)).astype(np.float32)
    mods = rng.integers(0, 3, size=n).astype(np.int32)
    ts = (rng.random(n) * 600).astype(np.float32)
    return mars_amd.MemoryGraph(n, d, ro, col, emb, mods, ts)


def ref_save(path, g):
    assert oracle.ref.ref_save_graph(str(path).encode(), g.num_nodes, g.num_edges, g.embedding_dim,
                                     _p(g.row_offsets), _p(g.col_indices), _p(g.embeddings), _p(g.modalities),
                                     _p(g.timestamps)) == 1


def ref_load(path):
    n, e, d = C.c_int32(), C.c_int32(), C.c_int32()
    if oracle.ref.ref_load_graph(str(path).encode(), C.byref(n), C.byref(e), C.byref(d),
                                 None, None, None, None, None) != 1:
        return None
    n, e, d = n.value, e.value, d.value
    ro, col = np.zeros(n + 1, np.int32), np.zeros(max(e, 1), np.int32)
    emb, mods, ts = np.zeros((n, d), np.float32), np.zeros(max(n, 1), np.int32), np.zeros(max(n, 1), np.float32)
    assert oracle.ref.ref_load_graph(str(path).encode(), C.byref(C.c_int32()), C.byref(C.c_int32()),
                                     C.byref(C.c_int32()), _p(ro), _p(col), _p(emb), _p(mods), _p(ts)) == 1
    return mars_amd.MemoryGraph(n, d, ro, col[:e], emb, mods[:n], ts[:n])


def same_graph(a, b):
    assert (a.num_nodes, a.num_edges, a.embedding_dim) == (b.num_nodes, b.num_edges, b.embedding_dim)
    for name in ("row_offsets", "col_indices", "embeddings", "modalities", "timestamps"):
        np.testing.assert_array_equal(getattr(a, name), getattr(b, name), err_msg=name)


def test_fnv1a_known_answers():
    for data, want in FNV_VECTORS:
        assert mars_amd.fnv1a64(data) == want


@needs_ref
def test_fnv1a_matches_reference(rng):
    for n in (0, 1, 7, 8, 9, 63, 1000, 3 << 20):
        buf = rng.integers(0, 256, size=max(n, 1), dtype=np.uint8)[:n]
        want = oracle.ref.ref_fnv1a(_p(buf) if n else None, n)
        assert mars_amd.fnv1a64(buf.tobytes()) == want, n


@needs_ref
@pytest.mark.parametrize("n,d", [(0, 16), (1, 3), (257, 64), (3000, 768)])
def test_graph_file_identical_to_reference(tmp_path, rng, n, d):
    g = random_graph(rng, n, d)
    mars_amd.save_graph(g, tmp_path / "ours.mars")
    ref_save(tmp_path / "ref.mars", g)
    assert (tmp_path / "ours.mars").read_bytes() == (tmp_path / "ref.mars").read_bytes()
    same_graph(mars_amd.load_graph(tmp_path / "ref.mars"), g)      # we read the reference's file
    same_graph(ref_load(tmp_path / "ours.mars"), g)                  # the reference reads ours


@needs_ref
def test_reference_kids_graph_round_trip(tmp_path):
    """The reference's own corpus and NSN graph (memory_graph.cpp) through both sides."""
    h = oracle.ref.ref_kids_make(2000, 128, 7, 6, 0.15)
    try:
        n, d, e = C.c_int32(), C.c_int32(), C.c_int32()
        oracle.ref.ref_graph_sizes(h, C.byref(n), C.byref(d), C.byref(e))
        n, d, e = n.value, d.value, e.value
        emb, mods, ts = np.zeros((n, d), np.float32), np.zeros(n, np.int32), np.zeros(n, np.float32)
        ep, ro, col = np.zeros(n, np.int32), np.zeros(n + 1, np.int32), np.zeros(e, np.int32)
        oracle.ref.ref_graph_copy(h, _p(emb), _p(mods), _p(ts), _p(ep), _p(ro), _p(col))
    finally:
        oracle.ref.ref_graph_free(h)
    g = mars_amd.MemoryGraph(n, d, ro, col, emb, mods, ts)
    ref_save(tmp_path / "ref.mars", g)
    same_graph(mars_amd.load_graph(tmp_path / "ref.mars"), g)
    mars_amd.save_graph(g, tmp_path / "ours.mars")
    assert (tmp_path / "ours.mars").read_bytes() == (tmp_path / "ref.mars").read_bytes()


def test_graph_file_rejects_damage(tmp_path, rng):
    g = random_graph(rng, 300, 32)
    good = tmp_path / "g.mars"
    mars_amd.save_graph(g, good)
    raw = bytearray(good.read_bytes())
    cases = {}
    flipped = bytearray(raw)
    flipped[20 + 4 * 150] ^= 0x01                        # a row offset
    cases["flipped"] = (flipped, -1)
    cases["truncated"] = (raw[:-3], -1)
    cases["extended"] = (raw + b"\0", -1)
    magic = bytearray(raw)
    magic[0:4] = b"MARX"
    cases["magic"] = (magic, -1)
    version = bytearray(raw)
    version[4:8] = struct.pack("<I", 2)
    cases["version"] = (version, -5)
    for name, (data, code) in cases.items():
        p = tmp_path / f"{name}.mars"
        p.write_bytes(bytes(data))
        with pytest.raises(MarsError) as e:
            mars_amd.load_graph(p)
        assert e.value.code == code, name
        if oracle.ref is not None:
            assert ref_load(p) is None, name               # the reference rejects the same files
    with pytest.raises(MarsError):
        mars_amd.load_graph(tmp_path / "absent.mars")


def read_kids_numpy(path):
    """The reference reader (scripts/bench_kids_ball_cuvs_cagra.py:49-60), restated."""
    with open(path, "rb") as f:
        magic = struct.unpack("<I", f.read(4))[0]
        assert magic == 0x5344494B
        struct.unpack("<I", f.read(4))
        n, d = struct.unpack("<ii", f.read(8))
        emb = np.fromfile(f, count=n * d, dtype=np.float32).reshape(n, d)
        ts = np.fromfile(f, count=n, dtype=np.float32)
        mod = np.fromfile(f, count=n, dtype=np.int32)
        epi = np.fromfile(f, count=n, dtype=np.int32)
    return emb, ts, mod, epi


def write_kids_numpy(path, emb, ts, mods, ep):
    """write_corpus_bin (bench_kids_sweep.cu:84-102), restated."""
    n, d = emb.shape
    with open(path, "wb") as f:
        f.write(struct.pack("<IIii", 0x5344494B, 1, n, d))
        f.write(np.ascontiguousarray(emb, np.float32).tobytes())
        f.write(np.ascontiguousarray(ts, np.float32).tobytes())
        f.write(np.ascontiguousarray(mods, np.int32).tobytes())
        f.write(np.ascontiguousarray(ep, np.int32).tobytes())


def test_kids_corpus(tmp_path, rng):
    from mars_amd import corpus
    c = corpus.make_corpus(1000, 768, seed=3)
    arrays = (c.embeddings, c.timestamps, c.modalities, c.episode_ids)
    mars_amd.write_kids_corpus(tmp_path / "ours.bin", *arrays)
    write_kids_numpy(tmp_path / "ref.bin", *arrays)
    assert (tmp_path / "ours.bin").read_bytes() == (tmp_path / "ref.bin").read_bytes()
    for got, want in zip(read_kids_numpy(tmp_path / "ours.bin"), arrays):
        np.testing.assert_array_equal(got, want)
    for got, want in zip(mars_amd.read_kids_corpus(tmp_path / "ref.bin"), arrays):
        np.testing.assert_array_equal(got, want)
    # empty corpus, damaged files
    mars_amd.write_kids_corpus(tmp_path / "empty.bin", np.zeros((0, 8), np.float32), [], [], [])
    emb, ts, mods, ep = mars_amd.read_kids_corpus(tmp_path / "empty.bin")
    assert emb.shape == (0, 8) and len(ts) == len(mods) == len(ep) == 0
    raw = (tmp_path / "ours.bin").read_bytes()
    (tmp_path / "short.bin").write_bytes(raw[:-4])
    (tmp_path / "magic.bin").write_bytes(b"SDIK" + raw[4:])
    for name in ("short.bin", "magic.bin"):
        with pytest.raises(MarsError):
            mars_amd.read_kids_corpus(tmp_path / name)
