"""mars_query_batch_static, the entry point that allocates nothing (its scratch is a static
device array of the library), against mars_query_batch, the entry point whose kernels it
shares: ids and scores identical on two calls in a row, the second with fewer queries
(the array keeps the first call's contents), per-query and uniform query times; sizes
beyond the static array rejected with MARS_ERR_CAPACITY before any launch."""
from __future__ import annotations

import numpy as np
import pytest

import mars_amd
from mars_amd import RetrievalConfig, corpus
from mars_amd._lib import MarsError

pytestmark = pytest.mark.gpu
N, D = 20000, 768


def static_call(dg, qs, tq, cfg, uniform):
    q = len(qs)
    bq = mars_amd.DeviceBuffer.from_array(np.ascontiguousarray(qs, np.float32))
    bt = mars_amd.DeviceBuffer.from_array(np.ascontiguousarray(tq, np.float32))
    bi = mars_amd.DeviceBuffer(q * cfg.top_k * 4)
    bs = mars_amd.DeviceBuffer(q * cfg.top_k * 4)
    try:
        mars_amd.query_batch_static(dg, bq.ptr, q, bt.ptr, cfg, bi.ptr, bs.ptr, uniform_tq=uniform)
        mars_amd.synchronize()
        return (bi.to_array(np.int32, q * cfg.top_k).reshape(q, cfg.top_k),
                bs.to_array(np.float32, q * cfg.top_k).reshape(q, cfg.top_k))
    finally:
        for b in (bq, bt, bi, bs):
            b.free()


def test_static_batch_matches_query_batch():
    mars_amd.init(0)
    c = corpus.make_corpus(N, D, seed=47)
    g = mars_amd.MemoryGraph(N, D, None, None, c.embeddings, c.modalities, c.timestamps)
    dg = mars_amd.upload_to_device(g)
    mars_amd.upload_fp16_embeddings(dg)
    ctx = mars_amd.create_query_context(N, D, 64)
    rng = np.random.default_rng(8)
    try:
        for q, k, uniform, filt in ((200, 10, True, -1), (37, 16, False, 1), (256, 5, False, -1)):
            nodes = corpus.pick_queries(c.modalities, q, seed=q)
            qs = c.embeddings[nodes]
            tq = np.full(q, corpus.QUERY_TIME, np.float32) if uniform else \
                rng.uniform(300, 600, size=q).astype(np.float32)
            cfg = RetrievalConfig(top_k=k, time_decay_lambda=corpus.DECAY_LAMBDA, modality_filter=filt)
            buf = mars_amd.DeviceBuffer.from_array(np.ascontiguousarray(qs))
            try:
                want_ids, want_sc = mars_amd.query_batch(dg, ctx, buf.ptr, q, tq, cfg)
            finally:
                buf.free()
            got_ids, got_sc = static_call(dg, qs, tq, cfg, uniform)
            np.testing.assert_array_equal(got_ids, want_ids)
            np.testing.assert_array_equal(got_sc.view(np.uint32), want_sc.view(np.uint32))
        with pytest.raises(MarsError) as e:
            static_call(dg, c.embeddings[:257], np.zeros(257, np.float32), RetrievalConfig(top_k=10), True)
        assert e.value.code == -4                      # MARS_ERR_CAPACITY
    finally:
        mars_amd.destroy_query_context(ctx)
        mars_amd.free_device(dg)


def _hip():
    """The HIP runtime libmars_amd.so links (the same library, so streams and graphs are
    shared with it)."""
    import ctypes as C
    h = C.CDLL("libamdhip64.so.7")
    vp = C.c_void_p
    for name, args in (("hipStreamCreate", [C.POINTER(vp)]), ("hipStreamBeginCapture", [vp, C.c_int]),
                       ("hipStreamEndCapture", [vp, C.POINTER(vp)]),
                       ("hipGraphInstantiate", [C.POINTER(vp), vp, vp, vp, C.c_size_t]),
                       ("hipGraphLaunch", [vp, vp]), ("hipStreamSynchronize", [vp]),
                       ("hipGraphExecDestroy", [vp]), ("hipGraphDestroy", [vp]), ("hipStreamDestroy", [vp])):
        getattr(h, name).argtypes = args
        getattr(h, name).restype = C.c_int
    return h


def _free_bytes():
    import ctypes as C
    from mars_amd._lib import check, lib
    free, total = C.c_size_t(), C.c_size_t()
    check(lib.mars_device_memory(C.byref(free), C.byref(total)), "mars_device_memory")
    return free.value


def test_static_batch_captured_in_a_hip_graph():
    """The call captured on a stream into a HIP graph, replayed three times with other
    work and new query vectors between the replays: every replay equals query_batch on
    the queries it read. Eager calls leave the device's free memory unchanged."""
    import ctypes as C
    mars_amd.init(0)
    c = corpus.make_corpus(N, D, seed=48)
    g = mars_amd.MemoryGraph(N, D, None, None, c.embeddings, c.modalities, c.timestamps)
    dg = mars_amd.upload_to_device(g)
    mars_amd.upload_fp16_embeddings(dg)
    ctx = mars_amd.create_query_context(N, D, 64)
    hip = _hip()
    q, k = 96, 10
    cfg = RetrievalConfig(top_k=k, time_decay_lambda=corpus.DECAY_LAMBDA)
    sets = [c.embeddings[corpus.pick_queries(c.modalities, q, seed=900 + i)] for i in range(3)]
    tq = np.full(q, corpus.QUERY_TIME, np.float32)
    bq = mars_amd.DeviceBuffer.from_array(np.ascontiguousarray(sets[0]))
    bt = mars_amd.DeviceBuffer.from_array(tq)
    bi, bs = mars_amd.DeviceBuffer(q * k * 4), mars_amd.DeviceBuffer(q * k * 4)
    s, graph, exe = C.c_void_p(), C.c_void_p(), C.c_void_p()
    try:
        # eager: no allocation (after one warm call that loads the kernels)
        mars_amd.query_batch_static(dg, bq.ptr, q, bt.ptr, cfg, bi.ptr, bs.ptr, uniform_tq=True)
        mars_amd.synchronize()
        free0 = _free_bytes()
        for _ in range(3):
            mars_amd.query_batch_static(dg, bq.ptr, q, bt.ptr, cfg, bi.ptr, bs.ptr, uniform_tq=True)
        mars_amd.synchronize()
        assert _free_bytes() == free0
        # capture
        assert hip.hipStreamCreate(C.byref(s)) == 0
        assert hip.hipStreamBeginCapture(s, 0) == 0                # hipStreamCaptureModeGlobal
        mars_amd.query_batch_static(dg, bq.ptr, q, bt.ptr, cfg, bi.ptr, bs.ptr, uniform_tq=True, stream=s.value)
        assert hip.hipStreamEndCapture(s, C.byref(graph)) == 0
        assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
        for i, qs in enumerate(sets):
            src = mars_amd.DeviceBuffer.from_array(np.ascontiguousarray(qs))
            try:
                from mars_amd._lib import check, lib
                check(lib.mars_copy_device(C.c_void_p(bq.ptr), C.c_void_p(src.ptr), qs.nbytes), "mars_copy_device")
                want_ids, want_sc = mars_amd.query_batch(dg, ctx, src.ptr, q, tq, cfg)   # eager work between
            finally:
                src.free()
            assert hip.hipGraphLaunch(exe, s) == 0
            assert hip.hipStreamSynchronize(s) == 0
            got_ids = bi.to_array(np.int32, q * k).reshape(q, k)
            got_sc = bs.to_array(np.float32, q * k).reshape(q, k)
            np.testing.assert_array_equal(got_ids, want_ids, err_msg=f"replay {i}")
            np.testing.assert_array_equal(got_sc.view(np.uint32), want_sc.view(np.uint32), err_msg=f"replay {i}")
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        if graph.value:
            hip.hipGraphDestroy(graph)
        if s.value:
            hip.hipStreamSynchronize(s)
            hip.hipStreamDestroy(s)
        for b in (bq, bt, bi, bs):
            b.free()
        mars_amd.destroy_query_context(ctx)
        mars_amd.free_device(dg)
