"""Benchmark of the retrieval hot path on one MI355X.

Workload (N=1M, D=768, K=10): the seeded episode corpus (4 IMAGE / 3 TEXT /
3 AUDIO per 10-node episode, decay lambda 0.1/s, query time 600 s), NSN graph
= intra-episode pairs + 8-NN, queries = IMAGE node embeddings resident in HBM.
A step is one Q=1 query. Timed: K global queries (fused scan + decay + top-K
+ depth-2 BFS, fp32 corpus), K episode-scoped queries, K global queries over
the fp16 corpus; each query is one C-ABI call whose host wall latency is taken
inside the library (steady_clock), p99 = sorted[floor(0.99 (n-1))].

One JSON line on stdout; progress on stderr.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "p99 query latency µs @N=1M D=768 K=10 (episode & global); HBM GB/s % peak"
HBM_PEAK_GBS = 8000.0


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def source_digest(name: str) -> str:
    """First 16 hex digits of the SHA-256 of a kernel source file of the package."""
    import hashlib
    return hashlib.sha256((ROOT / "mars_amd" / "csrc" / name).read_bytes()).hexdigest()[:16]


def scan_traffic(n: int, d: int, profile: str = "k_scan_fp32_1M.md"):
    """HBM bytes per scan launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    scaled by a plain-copy calibration) for this workload, from the committed profile, and
    where they come from. The profile names the kernel source it measured (file and
    SHA-256 prefix): a source that changed since makes the figure stale, and then no
    traffic is reported."""
    p = ROOT / "profiles" / profile
    if not p.exists():
        return None, f"no profile {profile}"
    kv = {}
    for line in p.read_text().splitlines():
        if ":" in line and not line.startswith(("#", " ", "|")):
            k, v = line.split(":", 1)
            kv[k.strip()] = v.split("(")[0].strip()
    if kv.get("workload") != f"N={n} D={d}":
        return None, f"profiles/{profile} measured {kv.get('workload')}, not N={n} D={d}"
    src = kv.get("kernel_source", "").split()
    if len(src) != 2 or source_digest(src[0]) != src[1]:
        return None, f"profiles/{profile} measured {' '.join(src) or 'an unnamed source'}; the source has changed since"
    return int(kv["traffic_bytes_per_launch"]), f"profiles/{profile} (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; " \
                                                 f"kernel source {src[0]} {src[1]})"


def checkpoint_pass(args, mars_amd, dg):
    """MARS v1 checkpoint of the device graph (mars_graph_save) and its reload through the
    file reader (FNV-1a checked); the file is removed afterwards."""
    path = Path(args.checkpoint_dir) / "bench_checkpoint.mars"
    t0 = time.perf_counter()
    mars_amd.save_device_graph(dg, path)
    t_save = time.perf_counter() - t0
    size = path.stat().st_size
    t0 = time.perf_counter()
    g = mars_amd.load_graph(path)
    t_load = time.perf_counter() - t0
    blob = np.zeros(256 << 20, np.uint8)
    t0 = time.perf_counter()
    mars_amd.fnv1a64(blob.tobytes())
    fnv = blob.size / (time.perf_counter() - t0) / 1e9
    path.unlink()
    res = dict(bytes=size, nodes=g.num_nodes, edges=g.num_edges, save_s=t_save, load_s=t_load,
               save_gbs=size / t_save / 1e9, load_gbs=size / t_load / 1e9, fnv1a_gbs=fnv)
    log(f"checkpoint: {size / 1e9:.2f} GB MARS v1, save {t_save:.2f} s ({res['save_gbs']:.2f} GB/s), "
        f"load + checksum {t_load:.2f} s ({res['load_gbs']:.2f} GB/s); FNV-1a alone {fnv:.2f} GB/s")
    return res


def maintenance_pass(mars_amd, dg, ctx, dq, first, count, D, gcfg, pctl, reps=200):
    """Importance update (decay every node + 10 boosts), novelty (top-1 raw dot on the
    graph's own certified context), edge-hit counting after a depth-2 global query, and
    the maintenance sweep; host wall time of each synchronous call."""
    from mars_amd import RetrievalStats
    dg.refresh()
    n = dg.num_nodes
    mars_amd.init_importance(dg)
    mars_amd.init_edge_hits(dg)
    rng = np.random.default_rng(5)
    t_imp, t_nov, t_hit, t_q = [], [], [], []
    for r in range(reps + 10):
        ids = rng.integers(0, n, 10).astype(np.int32)
        t0 = time.perf_counter()
        mars_amd.update_importance(dg, ids)
        t1 = time.perf_counter()
        qp = dq.ptr + (first + r % count) * D * 4
        mars_amd.compute_novelty(dg, device_ptr=qp)
        t2 = time.perf_counter()
        mars_amd.query_memory_fast_device(dg, ctx, qp, 600.0, gcfg, RetrievalStats())
        t3 = time.perf_counter()
        mars_amd.count_edge_hits(dg, ctx)
        t4 = time.perf_counter()
        if r >= 10:
            t_imp.append((t1 - t0) * 1e6)
            t_nov.append((t2 - t1) * 1e6)
            t_q.append((t3 - t2) * 1e6)
            t_hit.append((t4 - t3) * 1e6)
    hits = mars_amd.read_edge_hits(dg)
    touched = int(np.count_nonzero(hits))
    t0 = time.perf_counter()
    low = mars_amd.maintain_graph(dg, 0)
    t_sweep = (time.perf_counter() - t0) * 1e6
    t_again = []
    for _ in range(20):                      # the same pass over counters already zero
        t0 = time.perf_counter()
        mars_amd.maintain_graph(dg, 0)
        t_again.append((time.perf_counter() - t0) * 1e6)
    res = dict(nodes=n, edges=int(len(hits)),
               importance_update=dict(p50_us=pctl(t_imp, .5), p99_us=pctl(t_imp, .99), bytes=8 * n),
               novelty=dict(p50_us=pctl(t_nov, .5), p99_us=pctl(t_nov, .99), path="certified candidate scan, top-1"),
               edge_hit_count=dict(p50_us=pctl(t_hit, .5), p99_us=pctl(t_hit, .99),
                                   after="depth-2 global query (fp32 path)"),
               maintenance_sweep=dict(us=t_sweep, low_utility=low, edges_hit=touched,
                                      repeat_p50_us=pctl(t_again, .5)))
    log(f"maintenance at N={n:,}: importance update p50 {res['importance_update']['p50_us']:.1f} us, novelty p50 "
        f"{res['novelty']['p50_us']:.1f} us, edge-hit count p50 {res['edge_hit_count']['p50_us']:.1f} us, sweep "
        f"{t_sweep:.1f} us ({low:,} of {len(hits):,} edges never hit over {reps + 10} queries)")
    return res


def engine_pass(n_nodes, n_queries, D, pctl):
    """The JSON-line engine server (mars_amd/mars_engine) over its stdin/stdout pipe, with the
    reference server's edge policy (NSN graph rebuilt before a query after the node count
    doubled or grew by 1000): n_nodes ADDs of the benchmark corpus (each a one-node
    streaming insert), then n_queries QUERYs (top-10, depth-2 BFS, certified path; the
    first one builds the NSN graph) timed from the write of the request to the parsed
    response; requests are encoded before timing."""
    import subprocess
    from mars_amd import corpus as corp
    exe = ROOT / "mars_amd" / "mars_engine"
    c = corp.make_corpus(n_nodes, D, seed=11)
    p = subprocess.Popen([str(exe), "--dim", str(D), "--capacity", str(n_nodes)], stdin=subprocess.PIPE,
                         stdout=subprocess.PIPE, text=True, bufsize=1)

    def call(line):
        p.stdin.write(line)
        p.stdin.flush()
        return json.loads(p.stdout.readline())

    adds = [json.dumps({"cmd": "ADD", "id": i, "modality": int(c.modalities[i]), "embedding": c.embeddings[i].tolist(),
                        "timestamp": float(c.timestamps[i])}) + "\n" for i in range(n_nodes)]
    t0 = time.perf_counter()
    for line in adds:
        r = call(line)
        if r != {"ok": True}:
            raise RuntimeError(f"engine ADD failed: {r}")
    t_add = time.perf_counter() - t0
    qn = corp.pick_queries(c.modalities, n_queries, seed=12)
    qs = [json.dumps({"cmd": "QUERY", "embedding": c.embeddings[int(i)].tolist(), "top_k": 10, "bfs_max_hops": 2,
                      "timestamp": float(corp.QUERY_TIME)}) + "\n" for i in qn]
    lat, gpu = [], []
    for line in qs:
        t0 = time.perf_counter()
        r = call(line)
        lat.append((time.perf_counter() - t0) * 1e6)
        gpu.append(r["gpu_ms"] * 1e3)
        if len(r["results"]) != 10:
            raise RuntimeError(f"engine QUERY returned {len(r['results'])} results")
    st = call(json.dumps({"cmd": "STATS"}) + "\n")
    call(json.dumps({"cmd": "SHUTDOWN"}) + "\n")
    p.wait(timeout=60)
    res = dict(nodes=n_nodes, edges=st["edges"], add_per_s=n_nodes / t_add,
               query_rtt_p50_us=pctl(lat, .5), query_rtt_p99_us=pctl(lat, .99), query_gpu_p50_us=pctl(gpu, .5),
               request_bytes=len(qs[0]))
    log(f"engine server: {n_nodes:,} ADDs at {res['add_per_s']:.0f}/s ({st['edges']:,} undirected edges); QUERY "
        f"round trip p50 {res['query_rtt_p50_us']:.0f} us p99 {res['query_rtt_p99_us']:.0f} us (GPU p50 "
        f"{res['query_gpu_p50_us']:.0f} us, {len(qs[0]):,}-byte requests)")
    return res


def tiled_pass(args, mars_amd, corpus, c, qnodes, N, D, K, pctl, lat_resident, host_memory):
    """tiled_query contract over the corpus held in host RAM (pinned when the host grants it):
    tiles of --tiled-tile rows (the copy of tile i+1 overlaps the scan of tile i)."""
    from mars_amd import TiledQueryConfig
    bufs = [mars_amd.HostBuffer((N,), np.int32), mars_amd.HostBuffer((N,), np.float32)]
    tile = min(N, args.tiled_tile)
    tctx = mars_amd.create_tiled_context(tile, D, 64)
    try:
        bufs[0].array[:] = c.modalities
        bufs[1].array[:] = c.timestamps
        cfg = TiledQueryConfig(tile_size=tile, top_k=K, time_decay_lambda=corpus.DECAY_LAMBDA)
        tot, x, comp, gbs = [], [], [], []
        for i, node in enumerate(qnodes[:args.tiled_queries + 1]):
            st = mars_amd.TiledQueryStats()
            mars_amd.tiled_query(tctx, c.embeddings, bufs[0].array, bufs[1].array, c.embeddings[node],
                                 corpus.QUERY_TIME, cfg, st)
            if i:                                       # the first call warms the copy path
                tot.append(st.total_ms); x.append(st.transfer_ms); comp.append(st.compute_ms)
                gbs.append(st.h2d_gbs)
        res = dict(tile_rows=tile, tiles=(N + tile - 1) // tile, queries=len(tot), host_memory=host_memory,
                   total_ms_p50=pctl(tot, .5), total_ms_p99=pctl(tot, .99), transfer_ms_mean=float(np.mean(x)),
                   compute_ms_mean=float(np.mean(comp)), h2d_gbs_mean=float(np.mean(gbs)),
                   resident_global_p50_ms=pctl(lat_resident, .5) / 1e3,
                   speedup_resident_vs_tiled=pctl(tot, .5) / (pctl(lat_resident, .5) / 1e3))
        log(f"tiled comparator ({res['tiles']} tiles of {tile} rows, {host_memory} host RAM): total p50 "
            f"{res['total_ms_p50']:.1f} ms (H2D {res['transfer_ms_mean']:.1f} ms at {res['h2d_gbs_mean']:.1f} "
            f"GB/s, scan {res['compute_ms_mean']:.2f} ms) vs HBM-resident global p50 "
            f"{pctl(lat_resident, .5) / 1e3:.3f} ms ({res['speedup_resident_vs_tiled']:.0f}x)")
    finally:
        mars_amd.destroy_tiled_context(tctx)
        for b in bufs:
            b.free()
    return res


SERVE_MODES = {
    "auto": "q1 while one certified Q=1 query per arrival keeps the global server under half busy "
            "(measured Q=1 latency x global arrival rate < 0.5), link beyond",
    "q1": "one global query per call (certified candidate scan); each insert finds its own k-NN",
    "batch": "batched global calls; each insert finds its own k-NN",
    "link": "batched global calls that also find the k-NN of the nodes inserted since the last call "
            "(one corpus pass for both); inserts publish rows and episode edges only",
}


def serve_pass(args, mars_amd, corpus, lib, check, full, dg, ctx, qnodes, nq, ep_cfgs, gcfg, ctx_nodes, D, first_ins,
               M, mode, pctl):
    """Streaming: 10-node episodes inserted at 2,000 nodes/s on the graph's side stream while
    Q=1 queries arrive at 1,000/s, alternating global and episode-scoped. Episode queries
    are answered on their own thread and context as they arrive; global queries by a
    server thread (SERVE_MODES). Latency = completion - arrival (queueing included)."""
    max_batch = 1 if mode == "q1" else args.batch_max
    from mars_amd import _lib
    nq = min(nq, len(qnodes))
    ng, ne = (nq + 1) // 2, nq // 2
    rate = 1000.0
    g_arr = np.arange(ng, dtype=np.float64) * 2e6 / rate
    e_arr = g_arr[:ne] + 1e6 / rate
    gq = mars_amd.DeviceBuffer.from_array(np.ascontiguousarray(full.embeddings[qnodes[0:2 * ng:2]]))
    eq = mars_amd.DeviceBuffer.from_array(np.ascontiguousarray(full.embeddings[qnodes[1:2 * ne:2]]))
    ecf = ep_cfgs(qnodes[1:2 * ne:2])
    g1 = gcfg.to_c()
    ectx = mars_amd.create_query_context(ctx_nodes, D, 64, flags=0)
    ib = args.stream_insert_batch
    nb = (M + ib - 1) // ib
    ins = (_lib.InsertStatsC * max(1, nb))()
    istart = np.zeros(max(1, nb), np.float64)
    ilinked = np.zeros(max(1, nb), np.float64)
    g_done = np.zeros(ng, np.float64)
    g_batch = np.zeros(ng, np.int32)
    e_done = np.zeros(ne, np.float64)
    sl = slice(first_ins, first_ins + M)
    emb = np.ascontiguousarray(full.embeddings[sl])
    mods, ts = np.ascontiguousarray(full.modalities[sl]), np.ascontiguousarray(full.timestamps[sl])
    ep = np.ascontiguousarray(full.episode_ids[sl])
    pv = lambda a: a.ctypes.data
    b = _lib.ServeBenchC()
    b.t_q, b.max_batch = corpus.QUERY_TIME, max_batch
    b.g_queries, b.n_global, b.g_arrival_us, b.gcfg = gq.ptr, ng, pv(g_arr), C.cast(C.pointer(g1), C.c_void_p).value
    b.e_queries, b.n_episode, b.e_arrival_us, b.ecfgs = eq.ptr, ne, pv(e_arr), C.cast(ecf, C.c_void_p).value
    b.ins_emb, b.ins_mods, b.ins_ts, b.ins_ep = pv(emb), pv(mods), pv(ts), pv(ep)
    b.n_insert, b.insert_batch, b.insert_rate, b.knn_k = M, ib, 2000.0, args.knn_k
    b.g_done_us, b.g_batch, b.e_done_us = pv(g_done), pv(g_batch), pv(e_done)
    b.ins_stats, b.ins_start_us = C.cast(ins, C.c_void_p).value, pv(istart)
    b.link_deferred, b.max_link, b.ins_linked_us, b.link_wait_us = int(mode == "link"), 1024, pv(ilinked), 5000.0
    t0 = time.time()
    ctx.certified = True          # a global query answered alone uses the certified candidate scan
    try:
        check(lib.mars_bench_serve(dg.handle, ctx.handle, ectx.handle, C.byref(b)), "mars_bench_serve")
    finally:
        ctx.certified = False
        wall = time.time() - t0
        mars_amd.destroy_query_context(ectx)
        gq.free()
        eq.free()
    dg.refresh()
    lg, le = g_done - g_arr, e_done - e_arr
    res = dict(mode=mode, global_server=SERVE_MODES[mode], max_batch=max_batch, queries=nq, global_p50_us=pctl(lg, .5), global_p99_us=pctl(lg, .99),
               episode_p50_us=pctl(le, .5), episode_p99_us=pctl(le, .99),
               global_mean_batch=float(g_batch.mean()), global_q1_answers=int(b.g_uncertified),
               inserted_nodes=M, wall_s=wall)
    if M > 0:
        qa = np.array([s.queryable_us for s in ins[:nb]])
        li = ilinked[:nb] - istart[:nb]                    # insert call -> k-NN edges visible
        span = istart[nb - 1] + np.array([s.linked_us for s in ins[:nb]])[-1] - istart[0]
        res.update(insert_rate_achieved=M / (span / 1e6), queryable_p50_us=pctl(qa, .5),
                   queryable_p99_us=pctl(qa, .99), linked_p50_us=pctl(li, .5), linked_p99_us=pctl(li, .99),
                   rows_relocated=int(sum(s.rows_relocated for s in ins[:nb])),
                   rows_appended=int(sum(s.rows_appended for s in ins[:nb])))
        if mode == "link":
            res.update(link_calls=int(b.link_calls))
        else:
            res.update(knn_mean_us=float(np.mean([s.knn_us for s in ins[:nb]])))
    log(f"streaming [{mode}] ({M} nodes at 2000/s onto {first_ins}, {nq} queries at 1000/s 50/50): "
        f"global p50 {res['global_p50_us']:.0f} p99 {res['global_p99_us']:.0f} us (mean batch "
        f"{res['global_mean_batch']:.1f}), episode p50 {res['episode_p50_us']:.0f} p99 {res['episode_p99_us']:.0f} us"
        + (f"; time-to-queryable p50 {res['queryable_p50_us']:.0f} p99 {res['queryable_p99_us']:.0f} us; linked p50 "
           f"{res['linked_p50_us']:.0f} p99 {res['linked_p99_us']:.0f} us; {res['insert_rate_achieved']:.0f} nodes/s"
           if M > 0 else ""))
    return res


def compare_results(got, want, scl):
    """GPU results against oracle results from the same seeds: equal count; at each rank the
    same id with the same hops and a score within 1e-5 * max(|s|, its BFS-carried scale), or
    two ids whose scores are a near-tie under that bound."""
    if len(got) != len(want):
        return False
    for r, w in zip(got, want):
        tw = 1e-5 * max(abs(w[1]), scl[w[0]])
        if r.node_id == w[0]:
            if r.hops_from_seed != w[3] or abs(r.score - w[1]) > tw:
                return False
        elif abs(r.score - w[1]) > 2 * (tw + 1e-5 * max(abs(r.score), scl.get(r.node_id, float("inf")))):
            return False
    return True


def capture_answers(mars_amd, dg, ctx, dq, first, D, count, t_q, gcfg):
    """The GPU's answers to timed queries first .. first + count - 1, taken on the resident
    corpus before the streaming passes grow it: each query on the fp32-scan path (whose
    seeds the context keeps) and on the certified path (the one `value` times)."""
    out = []
    for i in range(count):
        ptr = dq.ptr + (first + i) * D * 4
        ctx.certified = False
        got = mars_amd.query_memory_fast_device(dg, ctx, ptr, t_q, gcfg)
        seeds = ctx.last_seeds()[0].copy()
        ctx.certified = True
        got_c = mars_amd.query_memory_fast_device(dg, ctx, ptr, t_q, gcfg)
        ctx.certified = False
        out.append((got, seeds, got_c))
    return out


def parity_check(oracle, first, og, c, qnodes, t_q, gcfg, ocfg, refs, answers):
    """The GPU's answers (capture_answers) to the queries the CPU baseline answered, against
    those oracle answers. The fp32 and certified answers must be bit-identical. The seed set
    must equal the oracle's up to near-ties at the K-th score (the oracle then runs again
    from the GPU's seeds); results as compare_results."""
    bad = []
    for i, ref in enumerate(refs):
        q = c.embeddings[qnodes[first + i]]
        got, seeds, got_c = answers[i]
        if got_c != got:
            bad.append(i)
            continue
        fin = ref["final"]
        _, scale = oracle.scores(og, q, t_q, gcfg.time_decay_lambda, gcfg.modality_filter)
        tol = 1e-5 * np.maximum(np.abs(fin), scale)
        kth = ref["seeds"][-1]
        diff = set(seeds.tolist()) ^ set(ref["seeds"].tolist())
        if any(abs(fin[j] - fin[kth]) > 2 * (tol[j] + tol[kth]) for j in diff):
            bad.append(i)
            continue
        if diff:                                   # near-tie seeds: the oracle from the GPU's seeds
            ref = oracle.query(og, q, t_q, ocfg, seeds_in=seeds)
        if not compare_results(got, ref["results"], oracle.result_scales(og, q, t_q, ocfg, ref)):
            bad.append(i)
    return {"queries": len(refs), "mismatched": len(bad), "mismatched_queries": bad[:10],
            "paths": "fp32 scan and MARS_CTX_CERTIFIED (bit-identical to each other)",
            "against": "the cpu_baseline oracle answers (fp64, same corpus, graph and query vectors)",
            "bar": "ids and hops exact, scores within 1e-5 * max(|s|, BFS-carried w * sum|e q|), near-ties allowed"}


def build_graph(mars_amd, corpus, n, D, seed, knn_k=8, threads=16):
    """A resident graph of the benchmark generator: fp32 rows with fp16 and int8 copies, the
    NSN graph (intra-episode pairs + knn_k-NN from the GPU builder), episode ids and CSR."""
    c = corpus.make_corpus(n, D, seed=seed, threads=threads)
    g = mars_amd.MemoryGraph(n, D, None, None, c.embeddings, c.modalities, c.timestamps)
    dg = mars_amd.upload_to_device(g)
    mars_amd.upload_fp16_embeddings(dg)
    mars_amd.upload_int8_embeddings(dg)
    knn = mars_amd.graph_knn(dg, knn_k) if knn_k > 0 else np.empty((n, 0), np.int32)
    corpus.nsn_graph(c, knn, threads=threads)
    mars_amd.set_csr(dg, c.row_offsets, c.col_indices)
    mars_amd.upload_episode_ids(dg, c.episode_ids)
    csr = mars_amd.build_episode_csr(c.episode_ids, n)
    mars_amd.upload_episode_csr(dg, csr)
    return c, dg, csr


def episode_cfgs(RetrievalConfig, RetrievalScope, RetrievalConfigC, corpus, c, csr, nodes, K, max_results=-1):
    """Episode-scoped configurations (one per query node) as a C array."""
    off = csr.ep_csr_offsets
    arr = (RetrievalConfigC * len(nodes))()
    for i, node in enumerate(nodes):
        ep = int(c.episode_ids[node])
        arr[i] = RetrievalConfig(top_k=K, time_decay_lambda=corpus.DECAY_LAMBDA, max_results_returned=max_results,
                                 retrieval_scope=RetrievalScope.EpisodeScoped, query_episode_id=ep,
                                 query_episode_member_begin=int(off[ep]),
                                 query_episode_member_count=int(off[ep + 1] - off[ep])).to_c()
    return arr


def bench_queries(lib, check, dg, ctx, dq_ptr, D, count, t_q, cfgs, n_cfg, K):
    """mars_bench_queries: `count` Q=1 queries on consecutive device vectors; per query the
    host wall latency (steady_clock inside the library) and, with the context's timing
    flag, the scan and post-scan kernel times (HIP events on the query stream)."""
    lat = np.zeros(count, np.float64)
    kern = np.zeros(count, np.float32)
    bfs = np.zeros(count, np.float32)
    nres = np.zeros(count, np.int32)
    check(lib.mars_bench_queries(dg.handle, ctx.handle, C.c_void_p(dq_ptr), D, count, C.c_float(t_q), cfgs, n_cfg,
                                 C.c_void_p(lat.ctypes.data), C.c_void_p(kern.ctypes.data),
                                 C.c_void_p(bfs.ctypes.data), C.c_void_p(nres.ctypes.data)), "mars_bench_queries")
    assert np.all(nres == K), "every query must return K results"
    return lat, kern, bfs


def config_100k_pass(args, mars_amd, corpus, lib, check, evict, pctl):
    """N=100,000 D=768: 10,000 Q=1 queries each global (certified and fp32 paths) and
    episode-scoped; scan GB/s both as measured back to back (the rows stay in the 256 MB
    Infinity Cache: cache-resident) and with a 1.5 GB read of another graph's rows between
    queries (evicted: L2 and Infinity Cache refilled from HBM); the CPU oracle on the same
    global queries."""
    from mars_amd import RetrievalConfig, RetrievalScope
    from mars_amd._lib import RetrievalConfigC
    n, D, K, S, W = 100_000, args.dim, 10, args.queries_100k, 200
    t = time.time()
    c, dg, csr = build_graph(mars_amd, corpus, n, D, args.seed)
    log(f"[100K] corpus + upload + 8-NN + NSN graph ({len(c.col_indices)} edges): {time.time() - t:.1f}s")
    ctx = mars_amd.create_query_context(n, D, 64, flags=0)
    qnodes = corpus.pick_queries(c.modalities, W + S, seed=args.query_seed)
    dq = mars_amd.DeviceBuffer.from_array(np.ascontiguousarray(c.embeddings[qnodes]))
    gcfg = RetrievalConfig(top_k=K, bfs_max_hops=2, time_decay_lambda=corpus.DECAY_LAMBDA, bfs_score_decay=0.5)
    g1 = gcfg.to_c()
    ec = episode_cfgs(RetrievalConfig, RetrievalScope, RetrievalConfigC, corpus, c, csr, qnodes, K)
    ec_t = (RetrievalConfigC * S).from_buffer(ec, W * C.sizeof(RetrievalConfigC))
    bytes_i8, bytes_f32 = n * D + 12 * n, n * D * 4 + 4 * n
    out = {"num_nodes": n, "dim": D, "queries": S, "num_edges": int(len(c.col_indices)),
           "nsn_graph": "intra-episode pairs + 8-NN"}
    try:
        def one(tag, cfgs, n_cfg, certified, nbytes):
            ctx.certified = certified
            ctx.timing = False
            bench_queries(lib, check, dg, ctx, dq.ptr, D, W, corpus.QUERY_TIME, cfgs if n_cfg == 1 else ec,
                          1 if n_cfg == 1 else W, K)
            t0 = time.time()
            lat, _, _ = bench_queries(lib, check, dg, ctx, dq.ptr + W * D * 4, D, S, corpus.QUERY_TIME, cfgs,
                                      n_cfg, K)
            wall = time.time() - t0
            ctx.timing = True
            _, kern, rest = bench_queries(lib, check, dg, ctx, dq.ptr + W * D * 4, D, min(S, 2000),
                                          corpus.QUERY_TIME, cfgs, min(n_cfg, 2000), K)
            r = dict(p50_us=pctl(lat, .5), p99_us=pctl(lat, .99), qps=S / wall, kernel_mean_us=float(kern.mean()),
                     after_scan_mean_us=float(rest.mean()))
            if nbytes:
                r.update(scan_gbs_cache_resident=nbytes / float(kern.mean()) / 1e3)
                # the same scan with the caches refilled from HBM: a 1.5 GB read before each query
                ev = []
                for i in range(200):
                    evict()
                    st = mars_amd.RetrievalStats()
                    mars_amd.query_memory_fast_device(dg, ctx, dq.ptr + (W + i) * D * 4, corpus.QUERY_TIME, gcfg, st)
                    ev.append(st.gpu_ms_similarity * 1e3)
                r.update(scan_kernel_evicted_mean_us=float(np.mean(ev)),
                         scan_gbs_evicted=nbytes / float(np.mean(ev)) / 1e3, scan_bytes_per_launch=nbytes)
            ctx.timing = False
            ctx.certified = False
            log(f"[100K] {tag}: p50 {r['p50_us']:.1f} us p99 {r['p99_us']:.1f} us; kernel mean {r['kernel_mean_us']:.1f} us"
                + (f" ({r['scan_gbs_cache_resident']:.0f} GB/s cache-resident, {r['scan_gbs_evicted']:.0f} GB/s "
                   f"evicted)" if nbytes else ""))
            return r

        out["global_certified"] = one("global certified (int8 candidates)", C.pointer(g1), 1, True, bytes_i8)
        out["global_fp32"] = one("global fp32", C.pointer(g1), 1, False, bytes_f32)
        out["episode"] = one("episode-scoped", ec_t, S, False, 0)
        out["cache_note"] = (f"cache-resident: queries back to back (int8 copy {bytes_i8 / 1e6:.0f} MB, fp32 rows "
                             f"{bytes_f32 / 1e6:.0f} MB against the 256 MB Infinity Cache); evicted: a 1.5 GB kernel "
                             f"read of another graph's rows before each timed query")
        if not args.no_cpu:
            import oracle
            answers = capture_answers(mars_amd, dg, ctx, dq, W, D, min(50, S), corpus.QUERY_TIME, gcfg)
            og = oracle.make_graph(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices)
            ocfg = oracle.config(K, 2, corpus.DECAY_LAMBDA, 0.5)
            nc = min(args.cpu_queries_100k, S)
            cl, refs = [], []
            for i, node in enumerate(qnodes[W:W + nc]):
                t0 = time.perf_counter()
                r = oracle.query(og, c.embeddings[node], corpus.QUERY_TIME, ocfg)
                cl.append((time.perf_counter() - t0) * 1e6)
                if i < len(answers):
                    refs.append(r)
            out["parity_checked"] = parity_check(oracle, W, og, c, qnodes, corpus.QUERY_TIME, gcfg, ocfg, refs,
                                                 answers)
            out["cpu_baseline"] = {"p50_us": pctl(cl, .5), "p99_us": pctl(cl, .99), "queries": nc,
                                   "cores": oracle.lib.oracle_num_threads(), "kind": "port"}
            log(f"[100K] cpu oracle ({out['cpu_baseline']['cores']} threads, {nc} queries): p50 {pctl(cl, .5):.0f} us "
                f"p99 {pctl(cl, .99):.0f} us; parity {out['parity_checked']['queries'] - out['parity_checked']['mismatched']}"
                f"/{out['parity_checked']['queries']}")
    finally:
        dq.free()
        mars_amd.destroy_query_context(ctx)
        mars_amd.free_device(dg)
    return out


def config_10k_recall_pass(args, mars_amd, corpus, pctl):
    """N=10,000 D=768: TEXT+AUDIO recall in the top 15 over 1,000 IMAGE queries (K=10, 15
    results; global depth-2 BFS and episode scope), from the GPU's answers and from the
    oracle's on the same queries."""
    from mars_amd import RetrievalConfig, RetrievalScope
    n, D, K, Q = 10_000, args.dim, 10, 1000
    c, dg, csr = build_graph(mars_amd, corpus, n, D, args.seed)
    ctx = mars_amd.create_query_context(n, D, 64, flags=0)
    nodes = corpus.pick_queries(c.modalities, Q, seed=args.seed)
    dq = mars_amd.DeviceBuffer.from_array(np.ascontiguousarray(c.embeddings[nodes]))
    off, mem = csr.ep_csr_offsets, csr.ep_csr_members
    gcfg = RetrievalConfig(top_k=K, bfs_max_hops=2, time_decay_lambda=corpus.DECAY_LAMBDA, bfs_score_decay=0.5,
                           max_results_returned=15)
    out = {"num_nodes": n, "queries": Q, "metric": "hit@15: the query's episode has a TEXT and an AUDIO node among "
           "the 15 results (bench_kids_sweep.cu:65-82); recall@15: fraction of the episode's 6 TEXT and AUDIO "
           "members among them"}
    per = {"global": [], "episode": []}
    lat = {"global": [], "episode": []}
    ctx.certified = True
    try:
        for i, node in enumerate(nodes):
            ep = int(c.episode_ids[node])
            members = mem[off[ep]:off[ep + 1]]
            ecfg = RetrievalConfig(top_k=K, time_decay_lambda=corpus.DECAY_LAMBDA, max_results_returned=15,
                                   retrieval_scope=RetrievalScope.EpisodeScoped, query_episode_id=ep,
                                   query_episode_member_begin=int(off[ep]),
                                   query_episode_member_count=int(off[ep + 1] - off[ep]))
            for scope, cfg in (("global", gcfg), ("episode", ecfg)):
                st = mars_amd.RetrievalStats()
                res = mars_amd.query_memory_fast_device(dg, ctx, dq.ptr + i * D * 4, corpus.QUERY_TIME, cfg, st)
                ids = [r.node_id for r in res]
                per[scope].append((ids, ep, members))
                lat[scope].append(st.wall_us)
        for scope in per:
            hit = [corpus.cross_modal_hit(ids, c.modalities, c.episode_ids, ep) for ids, ep, _ in per[scope]]
            rec = [corpus.cross_modal_recall(ids, c.modalities, c.episode_ids, ep, m) for ids, ep, m in per[scope]]
            out[scope] = {"hit_at_15": float(np.mean(hit)), "recall_at_15": float(np.mean(rec)),
                          "p50_us": pctl(lat[scope], .5), "p99_us": pctl(lat[scope], .99)}
        if not args.no_cpu:
            import oracle
            og = oracle.make_graph(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices,
                                   c.episode_ids)
            oh, orc, same = [], [], 0
            for i, node in enumerate(nodes):
                ids, ep, members = per["global"][i]
                ref = oracle.query(og, c.embeddings[node], corpus.QUERY_TIME,
                                   oracle.config(K, 2, corpus.DECAY_LAMBDA, 0.5, -1, 15))
                want = [w[0] for w in ref["results"]]
                same += set(want) == set(ids)
                oh.append(corpus.cross_modal_hit(want, c.modalities, c.episode_ids, ep))
                orc.append(corpus.cross_modal_recall(want, c.modalities, c.episode_ids, ep, members))
            out["global"]["oracle_hit_at_15"] = float(np.mean(oh))
            out["global"]["oracle_recall_at_15"] = float(np.mean(orc))
            out["global"]["same_result_sets"] = same
        log(f"[10K] {Q} IMAGE queries, top 15: global hit {out['global']['hit_at_15']:.4f} recall "
            f"{out['global']['recall_at_15']:.4f}" +
            (f" (oracle {out['global']['oracle_hit_at_15']:.4f} / {out['global']['oracle_recall_at_15']:.4f}, "
             f"same result sets {out['global']['same_result_sets']}/{Q})" if not args.no_cpu else "") +
            f"; episode scope hit {out['episode']['hit_at_15']:.4f} recall {out['episode']['recall_at_15']:.4f}")
    finally:
        ctx.certified = False
        dq.free()
        mars_amd.destroy_query_context(ctx)
        mars_amd.free_device(dg)
    return out


def pctl(v, p):
    v = np.sort(np.asarray(v, np.float64))
    return float(v[int(p * (len(v) - 1))]) if len(v) else 0.0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--dim", type=int, default=768)
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--query-seed", type=int, default=77)
    ap.add_argument("--cpu-queries", type=int, default=40)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--profile-only", action="store_true", help="only the global fp32 pass (for rocprofv3)")
    ap.add_argument("--stream-nodes", type=int, default=8000,
                    help="nodes inserted during the streaming pass (10-node episodes at 2,000 nodes/s)")
    ap.add_argument("--stream-queries", type=int, default=4000, help="queries of the streaming pass (1,000/s)")
    ap.add_argument("--tiled-queries", type=int, default=8, help="queries of the tiled out-of-core comparator")
    ap.add_argument("--tiled-tile", type=int, default=250_000, help="rows per tile of the tiled comparator")
    ap.add_argument("--knn-k", type=int, default=8,
                    help="nearest neighbours per node in the NSN graph (0: intra-episode pairs only)")
    ap.add_argument("--batch-q", default="64,256",
                    help="queries per batched MFMA scoring call, comma-separated (one pass each; 0: none)")
    ap.add_argument("--batch-max", type=int, default=64, help="most global queries per batched call when serving")
    ap.add_argument("--serve-modes", default="auto,q1,link",
                    help="servers of the streaming pass, one run each: auto, q1, batch, link (see SERVE_MODES)")
    ap.add_argument("--stream-insert-batch", type=int, default=10, help="nodes per insert call when streaming")
    ap.add_argument("--knn-block", type=int, default=0,
                    help="k-NN of the NSN graph within blocks of this many consecutive ids (0: exact, all pairs)")
    ap.add_argument("--candidates", choices=("int8", "fp16"), default="int8",
                    help="row copy the certified global query scans for candidates (the fp16 one is "
                         "also timed alongside)")
    ap.add_argument("--no-maintenance", action="store_true",
                    help="skip the importance / novelty / edge-hit maintenance pass")
    ap.add_argument("--maintenance-only", action="store_true",
                    help="only the maintenance pass (for rocprofv3)")
    ap.add_argument("--engine-nodes", type=int, default=0,
                    help="also drive the JSON-line engine server with this many ADDs and 500 QUERYs")
    ap.add_argument("--checkpoint-dir", default="",
                    help="also time a MARS v1 checkpoint of the device graph to this directory and its reload")
    ap.add_argument("--queries-100k", type=int, default=10000,
                    help="Q=1 queries per path of the N=100,000 pass (0: no such pass)")
    ap.add_argument("--cpu-queries-100k", type=int, default=10000,
                    help="global queries the CPU oracle answers in the N=100,000 pass")
    ap.add_argument("--no-recall-10k", action="store_true",
                    help="skip the N=10,000 TEXT+AUDIO recall pass")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU; --gpus above 1 is not supported here "
              "(the path would shard by node-id range: each GPU scans its share, then one all-gather of K keys)", file=sys.stderr)
        return 2

    import mars_amd
    from mars_amd import RetrievalConfig, RetrievalScope, corpus
    from mars_amd._lib import RetrievalConfigC, check, lib

    mars_amd.init(0)
    N, D, K = args.n, args.dim, 10
    M = 0 if args.profile_only else max(0, args.stream_nodes) // 10 * 10     # whole 10-node episodes
    t = time.time()
    # rows in pinned host memory when the host grants it (uploaded once, streamed again by the
    # tiled comparator), otherwise pageable
    try:
        host_rows = mars_amd.HostBuffer((N + M, D), np.float32)
    except mars_amd.MarsError as e:
        log(f"pinned host rows unavailable ({e}); using pageable memory")
        host_rows = None
    full = corpus.make_corpus(N + M, D, seed=args.seed,               # prefix-stable: rows >= N arrive later
                              out_emb=host_rows.array if host_rows else None)
    c = corpus.Corpus(full.embeddings[:N], full.modalities[:N], full.timestamps[:N], full.episode_ids[:N], args.seed)
    log(f"corpus N={N} D={D} seed={args.seed} (+{M} streamed): {time.time() - t:.1f}s")
    t = time.time()
    g = mars_amd.MemoryGraph(N, D, None, None, c.embeddings, c.modalities, c.timestamps)
    dg = mars_amd.upload_to_device(g, capacity_nodes=N + M)
    mars_amd.upload_fp16_embeddings(dg)
    if args.candidates == "int8":
        try:
            mars_amd.upload_int8_embeddings(dg)
        except mars_amd.MarsError as e:             # e.g. no room beside the fp32 and fp16 rows
            log(f"int8 copy unavailable ({e}); the certified query scans the fp16 rows")
            mars_amd.free_int8_embeddings(dg)
            args.candidates = "fp16"
    log(f"upload + fp16 copy" + (" + int8 copy" if args.candidates == "int8" else "") + f": {time.time() - t:.1f}s")
    t = time.time()
    if args.knn_k > 0:
        def knn_progress(done, total):
            if done % 10 == 0 or done == total or N > 2_000_000:
                log(f"{args.knn_k}-NN block {done}/{total}: {time.time() - t:.1f}s")
        # fp16 MFMA candidates + exact fp32 rescoring; above 2M rows the all-pairs build runs in
        # pieces of 1M query nodes (a progress line each)
        big = args.knn_block == 0 and N > 2_000_000
        knn = mars_amd.graph_knn(dg, args.knn_k, args.knn_block,
                                 knn_progress if (args.knn_block or big) else None)
        knn_unc, knn_res = getattr(dg, "knn_report", (0, 0))
        knn_s = time.time() - t
        log(f"{args.knn_k}-NN on the GPU" + (f" (blocks of {args.knn_block} ids)" if args.knn_block else "") +
            f": {knn_s:.1f}s; {N - knn_unc:,} of {N:,} lists certified exact, {knn_res:,} scanned again")
    else:
        knn = np.empty((N, 0), np.int32)
        knn_unc, knn_res, knn_s = 0, 0, 0.0
        log("NSN graph without k-NN edges (intra-episode pairs only)")
    t = time.time()
    corpus.nsn_graph(c, knn)
    mars_amd.set_csr(dg, c.row_offsets, c.col_indices)
    log(f"NSN graph: {len(c.col_indices)} directed edges, avg degree {len(c.col_indices) / N:.1f}: "
        f"{time.time() - t:.1f}s")
    mars_amd.upload_episode_ids(dg, c.episode_ids)
    csr = mars_amd.build_episode_csr(c.episode_ids, N)
    mars_amd.upload_episode_csr(dg, csr)
    ctx = mars_amd.create_query_context(N + M, D, 64, flags=0)

    batch_sizes = [int(x) for x in str(args.batch_q).split(",") if int(x) > 0]
    # every batched pass reads B consecutive query vectors, so the set holds at least the
    # largest batch
    nq = max(args.steps, args.stream_queries, *batch_sizes, 0) + args.warmup
    qnodes = corpus.pick_queries(c.modalities, nq, seed=args.query_seed)
    dq = mars_amd.DeviceBuffer.from_array(c.embeddings[qnodes])

    gcfg = RetrievalConfig(top_k=K, bfs_max_hops=2, time_decay_lambda=corpus.DECAY_LAMBDA, bfs_score_decay=0.5)
    if args.engine_nodes > 0 and args.maintenance_only:
        print(json.dumps({"engine": engine_pass(args.engine_nodes, 500, D, pctl)}), flush=True)
    if args.maintenance_only:
        m = maintenance_pass(mars_amd, dg, ctx, dq, 0, nq, D, gcfg, pctl)
        dq.free()
        mars_amd.destroy_query_context(ctx)
        mars_amd.free_device(dg)
        print(json.dumps({"maintenance": m}), flush=True)
        return 0
    off = csr.ep_csr_offsets

    def ep_cfgs(nodes):
        arr = (RetrievalConfigC * len(nodes))()
        for i, node in enumerate(nodes):
            ep = int(c.episode_ids[node])
            arr[i] = RetrievalConfig(top_k=K, time_decay_lambda=corpus.DECAY_LAMBDA,
                                     retrieval_scope=RetrievalScope.EpisodeScoped, query_episode_id=ep,
                                     query_episode_member_begin=int(off[ep]),
                                     query_episode_member_count=int(off[ep + 1] - off[ep])).to_c()
        return arr

    def run(first, count, cfgs, n_cfg):
        lat = np.zeros(count, np.float64)
        kern = np.zeros(count, np.float32)
        bfs = np.zeros(count, np.float32)
        nres = np.zeros(count, np.int32)
        ptr = dq.ptr + first * D * 4
        check(lib.mars_bench_queries(dg.handle, ctx.handle, C.c_void_p(ptr), D, count,
                                     C.c_float(corpus.QUERY_TIME), cfgs, n_cfg, C.c_void_p(lat.ctypes.data),
                                     C.c_void_p(kern.ctypes.data), C.c_void_p(bfs.ctypes.data),
                                     C.c_void_p(nres.ctypes.data)), "mars_bench_queries")
        assert np.all(nres == K), "every query must return K results"
        return lat, kern, bfs

    hq = np.ascontiguousarray(c.embeddings[qnodes])          # the same query vectors in host memory

    def run_host(first, count, cfgs, n_cfg):
        """query_memory_fast's contract: a host vector, copied to the device inside each call."""
        lat = np.zeros(count, np.float64)
        nres = np.zeros(count, np.int32)
        check(lib.mars_bench_queries_host(dg.handle, ctx.handle, C.c_void_p(hq.ctypes.data + first * D * 4), D, count,
                                          C.c_float(corpus.QUERY_TIME), cfgs, n_cfg, C.c_void_p(lat.ctypes.data),
                                          C.c_void_p(nres.ctypes.data)), "mars_bench_queries_host")
        assert np.all(nres == K), "every query must return K results"
        return lat

    W, S = args.warmup, args.steps
    KT = min(S, 2000)          # queries of the kernel-timing passes (HIP events on the query stream)
    g1 = gcfg.to_c()
    if args.profile_only:
        # a plain 1 GiB device copy: the HBM counters of a known byte count, used to
        # scale FETCH_SIZE / WRITE_SIZE of the scan kernel
        src, dst = mars_amd.DeviceBuffer(1 << 30), mars_amd.DeviceBuffer(1 << 30)
        check(lib.mars_copy_device(C.c_void_p(dst.ptr), C.c_void_p(src.ptr), 1 << 30), "mars_copy_device")
        src.free()
        dst.free()
    out = {}
    bytes_f32 = N * D * 4 + 4 * N
    bytes_f16 = N * D * 2 + 4 * N
    # the int8 candidate scan: bytes, per-row scale and bound, timestamps
    bytes_i8 = N * D + 8 * N + 4 * N
    cand = args.candidates
    bytes_cert = bytes_i8 if cand == "int8" else bytes_f16

    def timed(first, count, cfgs, n_cfg, events):
        ctx.timing = events
        t0 = time.time()
        r = run(first, count, cfgs, n_cfg)
        return r, time.time() - t0

    # ---- global fp32: latency pass (no events), then a kernel-timing pass
    ctx.use_fp16 = False
    run(0, W, C.pointer(g1), 1)
    (lat_g, _, _), wall_g = timed(W, S, C.pointer(g1), 1, False)
    (lat_gk, kern_g, bfs_g), _ = timed(W, KT, C.pointer(g1), 1, True)
    log(f"global fp32: p50 {pctl(lat_g, .5):.1f} us p99 {pctl(lat_g, .99):.1f} us; {S / wall_g:.0f} q/s; scan kernel "
        f"mean {kern_g.mean():.1f} us ({bytes_f32 / kern_g.mean() / 1e3:.0f} GB/s); finalize mean {bfs_g.mean():.1f} us")
    # the same queries replayed as a hipGraph (kernel-node arguments rewritten per query)
    ctx.use_cuda_graph = True
    run(0, W, C.pointer(g1), 1)
    (lat_gg, _, _), wall_gg = timed(W, S, C.pointer(g1), 1, False)
    ctx.use_cuda_graph = False
    log(f"global fp32 (graph replay): p50 {pctl(lat_gg, .5):.1f} us p99 {pctl(lat_gg, .99):.1f} us")
    # ---- global, certified candidate scan (results identical to the fp32 scan's)
    ctx.certified = True
    run(0, W, C.pointer(g1), 1)
    (lat_c, _, _), wall_c = timed(W, S, C.pointer(g1), 1, False)
    (lat_ck, kern_c, rest_c), _ = timed(W, KT, C.pointer(g1), 1, True)
    ctx.timing = False
    run_host(0, W, C.pointer(g1), 1)
    lat_ch = run_host(W, S, C.pointer(g1), 1)
    log(f"global certified, host query vectors (3 KB H2D inside each call): p50 {pctl(lat_ch, .5):.1f} us "
        f"p99 {pctl(lat_ch, .99):.1f} us")
    n_cert, n_samp = 0, min(S, 500)
    for i in range(n_samp):
        st = mars_amd.RetrievalStats()
        mars_amd.query_memory_fast_device(dg, ctx, dq.ptr + (W + i) * D * 4, corpus.QUERY_TIME, gcfg, st)
        n_cert += st.seeds_certified
    cph = []
    for node in qnodes[W:W + 200]:
        mars_amd.query_memory_fast(dg, ctx, c.embeddings[node], corpus.QUERY_TIME, gcfg)
        cph.append(ctx.last_phases(6))
    cph = np.array(cph).mean(0)
    ctx.certified = False
    log("certified phases (us, mean): merge {:.1f}  rescore+certify {:.1f}  bfs {:.1f}  mark {:.1f}  "
        "exact {:.1f}  results {:.1f}".format(*cph))
    log(f"global certified ({cand} scan, exact results): p50 {pctl(lat_c, .5):.1f} us p99 {pctl(lat_c, .99):.1f} us; "
        f"{S / wall_c:.0f} q/s; scan kernel mean {kern_c.mean():.1f} us ({bytes_cert / kern_c.mean() / 1e3:.0f} GB/s); "
        f"seeds + BFS + results {rest_c.mean():.1f} us; certified {n_cert}/{n_samp}")
    if cand == "int8" and not args.profile_only:
        # global queries in batches of 8 and 16 over one int8 pass (k_scan8m, certified seeds,
        # batched BFS), the answers identical to the Q=1 path's
        for B in (8, 16):
            ctx.timing = True
            rs = []
            for r in range(33):
                st = mars_amd.BatchStats()
                mars_amd.query_global_batch(dg, ctx, dq.ptr + (W + r * B) % (nq - B + 1) * D * 4, B,
                                            corpus.QUERY_TIME, gcfg, stats=st)
                if r >= 3:
                    rs.append((st.wall_us, st.gpu_ms_scan * 1e3, st.gpu_ms_seeds * 1e3, st.gpu_ms_bfs * 1e3,
                               st.batched, st.candidate_rows))
            ctx.timing = False
            a = np.array(rs)
            out[f"global_batch{B}_int8"] = dict(
                p50_us=pctl(a[:, 0], .5), p99_us=pctl(a[:, 0], .99), queries_per_s=B / (pctl(a[:, 0], .5) / 1e6),
                scan_kernel_mean_us=float(a[:, 1].mean()), certify_mean_us=float(a[:, 2].mean()),
                bfs_results_mean_us=float(a[:, 3].mean()), batched=int(a[:, 4].sum()), queries=B * len(rs),
                scan_vs_q1_scan=float(a[:, 1].mean()) / float(kern_c.mean()),
                candidate_rows=int(a[0, 5]), kernel="k_scan8m (int8 MFMA, 8 queries per A operand)")
            log(f"global batch of {B} (one int8 pass): p50 {pctl(a[:, 0], .5):.0f} us p99 {pctl(a[:, 0], .99):.0f} us; "
                f"scan {a[:, 1].mean():.1f} us ({a[:, 1].mean() / float(kern_c.mean()):.2f}x the Q=1 scan), certify "
                f"{a[:, 2].mean():.1f} us, BFS + results {a[:, 3].mean():.1f} us; {int(a[:, 4].sum())}/{B * len(rs)} "
                f"batched")
    cert16 = None
    if cand == "int8" and not args.profile_only:
        # the same queries certified over the fp16 copy (the int8 copy set aside, then rebuilt)
        mars_amd.free_int8_embeddings(dg)
        ctx.certified = True
        run(0, W, C.pointer(g1), 1)
        (lat_c16, _, _), _ = timed(W, min(S, 4000), C.pointer(g1), 1, False)
        (_, kern_c16, rest_c16), _ = timed(W, KT, C.pointer(g1), 1, True)
        ctx.timing = False
        ctx.certified = False
        t0 = time.perf_counter()
        mars_amd.upload_int8_embeddings(dg)           # k_convert_i8 over all rows, synchronous
        t_i8 = time.perf_counter() - t0
        log(f"int8 copy rebuilt (k_convert_i8 over {N:,} rows, allocation included): {t_i8 * 1e3:.2f} ms")
        out["int8_copy_build_ms"] = t_i8 * 1e3
        cert16 = dict(p50_us=pctl(lat_c16, .5), p99_us=pctl(lat_c16, .99), scan_kernel_mean_us=float(kern_c16.mean()),
                      seeds_bfs_results_mean_us=float(rest_c16.mean()),
                      scan_gbs=bytes_f16 / float(kern_c16.mean()) / 1e3, queries=min(S, 4000))
        log(f"global certified over the fp16 copy: p50 {cert16['p50_us']:.1f} us p99 {cert16['p99_us']:.1f} us; "
            f"scan kernel mean {kern_c16.mean():.1f} us; seeds + BFS + results {rest_c16.mean():.1f} us")
    # finalize phase breakdown (seed merge, BFS, selection) from the GPU realtime counter
    ctx.timing = False
    ph = []
    for node in qnodes[W:W + 200]:
        mars_amd.query_memory_fast(dg, ctx, c.embeddings[node], corpus.QUERY_TIME, gcfg)
        ph.append(ctx.last_phases())
    ph = np.array(ph)
    log(f"finalize phases (us, mean): seeds {ph[:, 0].mean():.1f}  bfs {ph[:, 1].mean():.1f}  "
        f"select {ph[:, 2].mean():.1f}")
    if not args.profile_only:
        # ---- episode-scoped
        ec = ep_cfgs(qnodes[:W + S])
        run(0, W, ec, W) if W else None
        ec_t = (RetrievalConfigC * S).from_buffer(ec, W * C.sizeof(RetrievalConfigC))
        (lat_e, _, _), wall_e = timed(W, S, ec_t, S, False)
        (_, kern_e, _), _ = timed(W, KT, ec_t, KT, True)
        log(f"episode: p50 {pctl(lat_e, .5):.1f} us p99 {pctl(lat_e, .99):.1f} us; {S / wall_e:.0f} q/s; kernel mean "
            f"{kern_e.mean():.1f} us")
        run_host(0, W, ec, W) if W else None
        lat_eh = run_host(W, S, ec_t, S)
        log(f"episode, host query vectors: p50 {pctl(lat_eh, .5):.1f} us p99 {pctl(lat_eh, .99):.1f} us")
        ctx.use_cuda_graph = True
        run(0, W, ec, W) if W else None
        (lat_eg, _, _), _ = timed(W, S, ec_t, S, False)
        ctx.use_cuda_graph = False
        log(f"episode (graph replay): p50 {pctl(lat_eg, .5):.1f} us p99 {pctl(lat_eg, .99):.1f} us")
        # ---- global fp16
        ctx.use_fp16 = True
        run(0, W, C.pointer(g1), 1)
        (lat_h, _, _), wall_h = timed(W, S, C.pointer(g1), 1, False)
        (_, kern_h, bfs_h), _ = timed(W, KT, C.pointer(g1), 1, True)
        ctx.use_fp16 = False
        log(f"global fp16: p50 {pctl(lat_h, .5):.1f} us p99 {pctl(lat_h, .99):.1f} us; scan kernel mean "
            f"{kern_h.mean():.1f} us ({bytes_f16 / kern_h.mean() / 1e3:.0f} GB/s)")
        # ---- batched global scoring on MFMA fp16 tiles (--batch-q 0 skips it). The scoring time
        # is the GPU time from the batch's first scoring launch to the end of its full corpus
        # pass (with more than 128 queries: the sampled floor pass and its merge included).
        for B in batch_sizes:
            ctx.timing = True
            reps = 30
            bl, bk = [], []
            for r in range(reps + 3):
                st = mars_amd.RetrievalStats()
                assert B <= nq
                mars_amd.query_batch(dg, ctx, dq.ptr + ((W + r * B) % (nq - B + 1)) * D * 4, B, corpus.QUERY_TIME,
                                     RetrievalConfig(top_k=K, time_decay_lambda=corpus.DECAY_LAMBDA), st)
                if r >= 3:
                    bl.append(st.wall_us)
                    bk.append(st.gpu_ms_similarity * 1e3)
            ctx.timing = False
            bkm = float(np.mean(bk))
            flops = 2.0 * B * N * D
            out[f"batch_q{B}_fp16"] = dict(p50_us=pctl(bl, .5), p99_us=pctl(bl, .99), queries_per_s=B / (pctl(bl, .5) / 1e6),
                                         scan_kernel_mean_us=bkm, tflops=flops / bkm / 1e6,
                                         mfma_util=flops / bkm / 1e6 / 2500.0,
                                         hbm_gbs=bytes_f16 / bkm / 1e3, hbm_frac=bytes_f16 / bkm / 1e3 / HBM_PEAK_GBS,
                                         kernel="k_batch_scan" if B <= 64 else "k_batch_rq")
            log(f"batch Q={B}: p50 {pctl(bl, .5):.0f} us; scan {bkm:.0f} us = {flops / bkm / 1e6:.0f} TFLOP/s "
                f"({flops / bkm / 1e6 / 25:.1f}% of 2.5 PF), {bytes_f16 / bkm / 1e3:.0f} GB/s")
        out["episode"] = dict(p50_us=pctl(lat_e, .5), p99_us=pctl(lat_e, .99), qps=S / wall_e,
                              host_vector_p50_us=pctl(lat_eh, .5), host_vector_p99_us=pctl(lat_eh, .99),
                              kernel_mean_us=float(kern_e.mean()),
                              graph_replay=dict(p50_us=pctl(lat_eg, .5), p99_us=pctl(lat_eg, .99)))
        out["global_fp16"] = dict(p50_us=pctl(lat_h, .5), p99_us=pctl(lat_h, .99), qps=S / wall_h,
                                  scan_kernel_mean_us=float(kern_h.mean()),
                                  scan_gbs=bytes_f16 / float(kern_h.mean()) / 1e3,
                                  scan_frac=bytes_f16 / float(kern_h.mean()) / 1e3 / HBM_PEAK_GBS)

    # the GPU's answers for the parity check against the CPU baseline, before any pass
    # below inserts nodes (the oracle holds the resident corpus)
    answers = None
    if not args.no_cpu and not args.profile_only:
        answers = capture_answers(mars_amd, dg, ctx, dq, W, D, min(args.cpu_queries, S), corpus.QUERY_TIME, gcfg)
    if args.checkpoint_dir and not args.profile_only:
        out["checkpoint"] = checkpoint_pass(args, mars_amd, dg)
    if not args.profile_only and args.tiled_queries > 0:
        out["tiled_comparator"] = tiled_pass(args, mars_amd, corpus, c, qnodes[W:], N, D, K, pctl, lat_g,
                                             "pinned" if host_rows else "pageable")
    # the streaming workload needs nodes to insert (--stream-nodes 0 measures the resident
    # corpus only)
    if args.stream_queries > 0 and args.serve_modes and not args.profile_only and M > 0:
        modes = [m for m in args.serve_modes.split(",") if m]
        runs, first = [], N
        per = M // len(modes) // 10 * 10                  # whole 10-node episodes per run
        per_q = args.stream_queries // len(modes)
        for i, m in enumerate(modes):
            chosen = m
            if m == "auto":
                # global queries arrive at half the query rate (1,000/s alternating global and episode)
                load = float(np.median(lat_c)) * 1e-6 * 500.0
                chosen = "q1" if load < 0.5 else "link"
                log(f"streaming [auto]: certified Q=1 p50 {np.median(lat_c):.0f} us x 500 global/s = "
                    f"{load:.0%} busy -> {chosen}")
            r = serve_pass(args, mars_amd, corpus, lib, check, full, dg, ctx, qnodes[W + i * per_q:], per_q,
                           ep_cfgs, gcfg, N + M, D, first, per, chosen, pctl)
            if m == "auto":
                r = dict(r, mode="auto", chosen=chosen, q1_load=round(load, 4))
            runs.append(r)
            first += per
        out["streaming"] = dict(base_nodes=N, insert_batch=args.stream_insert_batch, insert_rate_target=2000.0,
                                query_rate_target=1000.0, knn_k=args.knn_k,
                                latency="completion - arrival (queueing included)", runs=runs)
    if args.engine_nodes > 0 and not args.profile_only:
        out["engine_server"] = engine_pass(args.engine_nodes, 500, D, pctl)
    if not args.profile_only and not args.no_maintenance:
        out["maintenance"] = maintenance_pass(mars_amd, dg, ctx, dq, W, S - W, D, gcfg, pctl)

    traffic, traffic_src = scan_traffic(N, D, "k_scan_int8_1M.md" if cand == "int8" else "k_scan_fp16_1M.md")
    achieved = bytes_cert / float(kern_c.mean()) / 1e3      # GB/s of the certified path's candidate scan
    achieved32 = bytes_f32 / float(kern_g.mean()) / 1e3
    res = {
        "metric": METRIC,
        "value": round(pctl(lat_c, .99), 2),
        "unit": "us",
        "n_gpus": 1,
        "steps": S,
        "warmup": W,
        "ms_per_step": round(float(lat_c.mean()) / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"global Q=1 decay+top-K+depth-2 BFS over N={N:,} D={D}, K={K}: {cand} candidate "
                               f"scan with certified exact seeds and exact BFS scores (results bit-identical to the "
                               f"fp32 scan path, which answers any query the certificate does not cover); the "
                               f"fp32-scan path, the fp16-candidate certified path, episode-scoped and fp16 global "
                               f"reported alongside",
                   "global_path": "MARS_CTX_CERTIFIED", "candidate_rows": cand,
                   "num_nodes": N, "dim": D, "top_k": K, "bfs_hops": 2, "decay_lambda": corpus.DECAY_LAMBDA,
                   "corpus_seed": args.seed, "query_seed": args.query_seed, "num_edges": int(len(c.col_indices)),
                   "knn_lists_uncertified": knn_unc, "knn_lists_scanned_again": knn_res,
                   "knn_build_s": round(knn_s, 3),
                   "nsn_graph": (f"intra-episode pairs + {args.knn_k}-NN" +
                                 (f" within blocks of {args.knn_block} ids" if args.knn_block else "")
                                 if args.knn_k > 0 else "intra-episode pairs only (k-NN edges omitted)")},
        "global_certified": dict(p50_us=pctl(lat_c, .5), p99_us=pctl(lat_c, .99), qps=S / wall_c,
                                 host_vector_p50_us=pctl(lat_ch, .5), host_vector_p99_us=pctl(lat_ch, .99),
                                 p99_us_with_events=pctl(lat_ck, .99), scan_kernel_mean_us=float(kern_c.mean()),
                                 seeds_bfs_results_mean_us=float(rest_c.mean()),
                                 scan_gbs=achieved, scan_frac=achieved / HBM_PEAK_GBS,
                                 certified=n_cert, certified_sample=n_samp,
                                 candidate_rows=cand, scan_bytes_per_launch=bytes_cert,
                                 phases_us=dict(zip(("merge", "rescore_certify", "bfs", "mark", "exact", "results"),
                                                    [round(float(x), 2) for x in cph]))),
        **({"global_certified_fp16": cert16} if cert16 else {}),
        "global_fp32": dict(p50_us=pctl(lat_g, .5), p99_us=pctl(lat_g, .99), qps=S / wall_g,
                            p99_us_with_events=pctl(lat_gk, .99),
                            graph_replay=dict(p50_us=pctl(lat_gg, .5), p99_us=pctl(lat_gg, .99)),
                            scan_kernel_mean_us=float(kern_g.mean()), finalize_kernel_mean_us=float(bfs_g.mean()),
                            scan_gbs=achieved32, scan_frac=achieved32 / HBM_PEAK_GBS,
                            scan_traffic=scan_traffic(N, D)[0],
                            finalize_phases_us=dict(seed_merge=float(ph[:, 0].mean()), bfs=float(ph[:, 1].mean()),
                                                    select=float(ph[:, 2].mean()))),
        **out,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": (f"k_scan8<{D // 64},false> (int8 MFMA, 16 keys per workgroup, 64 candidates, keys = "
                                f"per-row upper bounds)"
                                if cand == "int8" else f"k_scan<__half,QF16<{D // 128}>,false> (16 candidates per "
                                                       f"workgroup)"),
                     "bytes_per_launch": bytes_cert},
    }
    if not args.profile_only:
        # a plain streaming read of the same fp16 rows, no arithmetic: the scan's practical ceiling
        ceiling = mars_amd.read_ceiling(dg, fp16=True, reps=20)
        res["read_ceiling"] = {"value": round(ceiling, 1), "unit": "GB/s", "rows": "fp16",
                               "kernel": "k_read_rows (16-byte non-temporal loads, 8 in flight per lane)",
                               "frac_of_peak": round(ceiling / HBM_PEAK_GBS, 4)}
        log(f"streaming-read ceiling (fp16 rows, no arithmetic): {ceiling:.0f} GB/s = "
            f"{ceiling / HBM_PEAK_GBS:.1%} of peak")
        if cand == "int8":
            # the same stream over the int8 copy (half the bytes): the int8 scan's own ceiling
            ceiling = mars_amd.read_pattern(dg, mars_amd.READ_STREAM_INT8, reps=20)
            res["read_ceiling"]["int8_rows"] = round(ceiling, 1)
            log(f"streaming-read ceiling (int8 rows): {ceiling:.0f} GB/s = {ceiling / HBM_PEAK_GBS:.1%} of peak")
        res["read_ceiling"]["scan_frac_of_ceiling"] = round(achieved / ceiling, 4)
        log(f"the certified scan runs at {achieved / ceiling:.1%} of its rows' streaming-read ceiling")
        # the batched scan's fragment pattern (16 rows x 64 B per load), ordinary and non-temporal
        frag = mars_amd.read_pattern(dg, mars_amd.READ_FRAGMENTS, reps=20)
        frag_nt = mars_amd.read_pattern(dg, mars_amd.READ_FRAGMENTS_NT, reps=20)
        res["read_ceiling"]["fragments_16x64B"] = round(frag, 1)
        res["read_ceiling"]["fragments_16x64B_nontemporal"] = round(frag_nt, 1)
        log(f"fragment-pattern read (16 rows x 64 B per load, no arithmetic): {frag:.0f} GB/s, "
            f"non-temporal {frag_nt:.0f} GB/s")

    if not args.no_cpu and not args.profile_only:
        import oracle
        og = oracle.make_graph(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices)
        ocfg = oracle.config(K, 2, corpus.DECAY_LAMBDA, 0.5)
        cl, refs = [], []
        nc = min(args.cpu_queries, S)
        for node in qnodes[W:W + nc]:
            t0 = time.perf_counter()
            refs.append(oracle.query(og, c.embeddings[node], corpus.QUERY_TIME, ocfg))
            cl.append((time.perf_counter() - t0) * 1e6)
        res_parity = parity_check(oracle, W, og, c, qnodes, corpus.QUERY_TIME, gcfg, ocfg, refs, answers)
        res["cpu_baseline"] = {"value": round(pctl(cl, .99), 1), "unit": "us", "cores": oracle.lib.oracle_num_threads(),
                               "kind": "port",
                               "sample": f"first {nc} of the timed global queries (same corpus, graph and query "
                                         f"vectors), fp64 C++ oracle with OpenMP over rows; p99 of {nc}",
                               "p50_us": round(pctl(cl, .5), 1)}
        log(f"cpu oracle ({res['cpu_baseline']['cores']} threads): p50 {pctl(cl, .5):.0f} us p99 {pctl(cl, .99):.0f} us")
        # the same oracle on one thread (a few queries: about 0.4 s each at 1M)
        threads = oracle.lib.oracle_num_threads()
        oracle.lib.oracle_set_num_threads(1)
        c1 = []
        for node in qnodes[W:W + 5]:
            t0 = time.perf_counter()
            oracle.query(og, c.embeddings[node], corpus.QUERY_TIME, ocfg)
            c1.append((time.perf_counter() - t0) * 1e6)
        oracle.lib.oracle_set_num_threads(threads)
        model = next((ln.split(":", 1)[1].strip() for ln in Path("/proc/cpuinfo").read_text().splitlines()
                      if ln.startswith("model name")), "unknown")
        res["parity_checked"] = res_parity
        res["cpu_baseline"]["single_thread"] = {"p50_us": round(pctl(c1, .5), 1), "queries": len(c1)}
        res["cpu_baseline"]["host"] = {"cpu": model, "nproc": os.cpu_count()}
        log(f"cpu oracle (1 thread, {len(c1)} queries): p50 {pctl(c1, .5):.0f} us; host {model}, nproc {os.cpu_count()}")
    dq.free()
    mars_amd.destroy_query_context(ctx)
    if not args.profile_only and args.dim == 768:
        # the two smaller configurations of the same generator, each on its own graph
        if args.queries_100k > 0:
            evict = lambda: mars_amd.read_pattern(dg, mars_amd.READ_FRAGMENTS, reps=1)
            res["config_100k"] = config_100k_pass(args, mars_amd, corpus, lib, check, evict, pctl)
        if not args.no_recall_10k:
            res["config_10k_recall"] = config_10k_recall_pass(args, mars_amd, corpus, pctl)
    mars_amd.free_device(dg)
    del c, full
    if host_rows:
        host_rows.free()
    print(json.dumps(res), flush=True)
    if res.get("config_100k", {}).get("parity_checked", {}).get("mismatched", 0):
        log("PARITY FAILURE at N=100,000")
        return 3
    if res.get("parity_checked", {}).get("mismatched", 0):
        log(f"PARITY FAILURE: {res['parity_checked']['mismatched']} of {res['parity_checked']['queries']} GPU answers "
            f"differ from the oracle's")
        return 3
    return 0


if __name__ == "__main__":
    sys.exit(main())
