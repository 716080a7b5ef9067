"""Benchmark of the flat exact-search hot path on one MI355X.

Workload (the headline configuration): exact cosine search over 1,000,000
unit-normalised 768-d f32 vectors (N(0,1) draws plus one of 256 cluster
offsets, then L2-normalised by the library's prepare step), 10,000 queries from
the same recipe in batches of 1,024. One step = one batch of 1,024 queries
searched from HBM-resident queries to HBM-resident results (k=10 for the
headline value; k=100 reported alongside).

Prints ONE JSON line with the contract fields plus `roofline` (dominant
kernel: the FP32-MFMA candidate GEMM, timed with HIP events on its own stream)
and `cpu_baseline` (the oracle's restatement of the reference CPU path on a
bounded sample of the same workload, on this host's cores; one-thread figures
beside it). Every leg also reports the host-pointer path (PCIe both ways) and
single-query latency (mean and p95, bench.rs:381-409); the sub-objects `c1`,
`ivfpq`, `sq8`, `kmeans` and `fixture` carry the other workloads.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "QPS exact k=10 @1M×768 f32 batch 1024; % MFMA/HBM roofline; IVF-PQ QPS"
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


GENERATOR = ("ChaCha8Rng::seed_from_u64(seed) counter-mode stream on the GPU, fixture.rs's Box-Muller "
             "(pxg_mixture_generate_device / pxg_uniform_generate_device)")


def mixture(torch, px, dev, n, dim, clusters, sigma, nq, drawn, seed):
    """Centres N(0,1), point i = centre[cluster(i)] + sigma * N(0,1), queries the
    same, from one seeded ChaCha8 stream (cluster(i) = i % clusters, or drawn
    from the stream)."""
    x = torch.empty((n, dim), dtype=torch.float32, device=dev)
    q = torch.empty((nq, dim), dtype=torch.float32, device=dev)
    px.mixture_generate_device(n, dim, clusters, 1.0, sigma, nq, drawn, seed, x, q)
    return x, q


def inputs_info(seed, recipe):
    return {"seed": seed, "generator": GENERATOR, "recipe": recipe}


def load_traffic(name):
    """HBM bytes per launch of `name` from the committed rocprofv3 PMC summary, if any."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(p) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


def cpu_model():
    """The host CPU's model string (from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_path(search_batch, batches_host, k, reps=3):
    """The host-pointer entry point a VectorIndex drop-in calls: queries copied
    over PCIe, results copied back, per batch (median of `reps` passes over the
    batches after one untimed pass)."""
    for b in batches_host:
        search_batch(b, k)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        for b in batches_host:
            search_batch(b, k)
        times.append((time.perf_counter() - t0) / len(batches_host))
    t = float(np.median(times))
    nq = batches_host[0].shape[0]
    return {"ms_per_batch": round(t * 1e3, 4), "queries_per_s": round(nq / t, 2), "batch": nq,
            "note": "host-pointer search: host queries in, host results out (PCIe both ways)"}


def latency_batch1(search_one, queries_host, k, repeats=200):
    """bench.rs:381-409: one untimed warm pass, then `repeats` single-query
    searches through the host-pointer entry point; mean and p95 (index
    len * 95 / 100 of the sorted samples)."""
    m = min(repeats, queries_host.shape[0])
    for i in range(m):
        search_one(queries_host[i], k)
    samples = []
    for i in range(m):
        t0 = time.perf_counter()
        search_one(queries_host[i], k)
        samples.append(time.perf_counter() - t0)
    samples.sort()
    return {"mean_us": round(1e6 * float(np.mean(samples)), 2), "p95_us": round(1e6 * samples[m * 95 // 100], 2),
            "samples": m, "note": "single queries, host pointers, after one untimed pass"}


def bench_c1(args, torch, px, dev):
    """Flat exact search, Euclidean, k=10: 100,000 x 128 f32 from a mixture of
    100 Gaussian clusters (centres N(0,1), sigma 0.15); 1,000 queries drawn
    fresh from the same mixture, searched as one batch of 1,000."""
    n, dim, nq, k = 100_000, 128, 1000, 10
    seed = args.seed + 3
    x, q = mixture(torch, px, dev, n, dim, 100, 0.15, nq, False, seed)
    ids = np.arange(n, dtype=np.uint64)
    idx = px.FlatIndex(px.VectorSpace(dim, px.Metric.EUCLIDEAN), n)
    idx.insert_device(ids, x)
    oi = torch.empty((nq, k), dtype=torch.int64, device=dev)
    od = torch.empty((nq, k), dtype=torch.float32, device=dev)
    oc = torch.empty((nq,), dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    for _ in range(5):
        idx.search_device(q, k, oi, od, oc, stream=stream)
    torch.cuda.synchronize()
    steps = args.c1_steps
    t0 = time.perf_counter()
    for _ in range(steps):
        idx.search_device(q, k, oi, od, oc, stream=stream)
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t0) / steps
    px.set_profiling(True)
    stages = []
    for _ in range(steps):
        idx.search_device(q, k, oi, od, oc, stream=stream)
        stages.append(px.last_timings())
    px.set_profiling(False)
    cand_ms = float(np.mean([t["candidates_ms"] for t in stages]))
    tflops = 2.0 * n * dim * nq / (cand_ms * 1e-3) / 1e12
    qh = q.cpu().numpy()
    log(f"[bench] c1: {step_s * 1e3:.3f} ms/batch = {nq / step_s:.0f} QPS; candidate GEMM {cand_ms:.3f} ms = "
        f"{tflops:.1f} TFLOP/s")
    if args.profile_core:
        return {"ms_per_step": round(step_s * 1e3, 4), "candidates_ms": round(cand_ms, 4)}
    out = {"value": round(nq / step_s, 2), "unit": "queries/s", "ms_per_step": round(step_s * 1e3, 4), "steps": steps,
           "config": {"workload": "flat exact search, Euclidean, 100k x 128 f32 (100 Gaussian clusters, sigma 0.15), "
                                  "1,000 queries in one batch, k=10", "n": n, "dim": dim, "batch": nq, "k": k,
                      "inputs": inputs_info(seed, "100 centres N(0,1)^128; x_i = centre[i % 100] + 0.15 N(0,1); "
                                                  "query q = centre[q % 100] + 0.15 N(0,1)")},
           "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(tflops / PEAK_FP32_MFMA_TFLOPS, 4),
                        "traffic": load_traffic("flat_mfma_candidates_c1"),
                        "kernel": "flat_mfma_candidates",
                        "timed": "the candidate stage: seeding pass, flat_seed_threshold and full pass",
                        "ms_per_launch": round(cand_ms, 4)},
           "stage_ms": {key: round(float(np.mean([t[key] for t in stages])), 4) for key in stages[0]},
           "host_path": host_path(idx.search_batch, [qh], k),
           "latency_batch1": latency_batch1(idx.search_all, qh, k)}
    if not args.no_cpu:
        from oracle import oracle as orc
        xh = x.cpu().numpy()
        t0 = time.perf_counter()
        wi, wd, wc = orc.flat_search(xh, ids, orc.EUCLIDEAN, qh, k, threads=args.cpu_threads)
        cpu_mt = time.perf_counter() - t0
        t0 = time.perf_counter()
        orc.flat_search(xh, ids, orc.EUCLIDEAN, qh, k, threads=1)
        cpu_1 = time.perf_counter() - t0
        gi, gd, gc = idx.search_batch(qh, k)
        same = int(sum(np.array_equal(gi[i], wi[i]) and np.array_equal(gd[i].view(np.uint32), wd[i].view(np.uint32))
                       for i in range(nq)))
        out["cpu_baseline"] = {"value": round(nq / cpu_mt, 2), "unit": "queries/s", "cores": args.cpu_threads,
                               "kind": "port", "sample": f"the whole workload (all {nq} queries over 100k x 128), "
                                                         f"oracle FlatIndex::search restatement, {cpu_mt:.2f}s"}
        out["cpu_baseline_1core"] = {"value": round(nq / cpu_1, 2), "unit": "queries/s", "cores": 1, "kind": "port",
                                     "sample": f"the whole workload on one thread, {cpu_1:.2f}s"}
        out["parity_sample"] = {"queries": nq, "bit_exact": same}
        log(f"[bench] c1 CPU {nq / cpu_mt:.0f} QPS ({args.cpu_threads} threads), {nq / cpu_1:.0f} QPS (1 thread); "
            f"GPU/oracle bit-exact {same}/{nq}")
    del idx, x
    return out


def bench_ivfpq(args, torch, px, dev):
    """IVF-PQ search, Euclidean, k=10: 10M x 128 f32 from 1,000 Gaussian clusters
    (centres N(0,1), sigma 0.15); nlist 4096, PQ 16 x 256, nprobe 32; 10,000
    queries from the same mixture in batches of 1,024. Trained on the GPU from
    the default 100,000-vector stride sample (seed 0x1FF9C0D, 25 iterations)."""
    n, dim, B, k, nprobe = args.ivf_n, 128, args.batch, 10, 32
    seed = args.seed + 7
    # cluster ids drawn from the stream: an `i % clusters` layout would alias
    # with the trainer's deterministic stride sample (stride 100 at 10M) and
    # show it only 10 of the 1,000 clusters
    x, queries = mixture(torch, px, dev, n, dim, 1000, 0.15, args.queries, True, seed)
    ids = np.arange(n, dtype=np.uint64)
    cfg = px.IvfPqConfig(4096, 16).with_nprobe(nprobe).with_train_threshold(1 << 63)
    idx = px.IvfPqIndex(px.VectorSpace(dim, px.Metric.EUCLIDEAN), cfg)
    t0 = time.time()
    idx.insert_device(ids, x)
    torch.cuda.synchronize()
    log(f"[bench] ivfpq: inserted {n}x{dim} in {time.time() - t0:.2f}s; training on the GPU")
    t0 = time.time()
    rep = idx.train()
    train_s = time.time() - t0
    log(f"[bench] ivfpq: trained in {train_s:.2f}s: {rep}")
    nb = args.queries // B
    batches = [queries[i * B:(i + 1) * B] for i in range(nb)]
    oi = torch.empty((B, k), dtype=torch.int64, device=dev)
    od = torch.empty((B, k), dtype=torch.float32, device=dev)
    oc = torch.empty((B,), dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    for s_ in range(3):
        idx.search_device(batches[s_ % nb], k, oi, od, oc, stream=stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s_ in range(args.ivf_steps):
        idx.search_device(batches[s_ % nb], k, oi, od, oc, stream=stream)
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t0) / args.ivf_steps
    px.set_profiling(True)
    stages, scanned = [], []
    for s_ in range(args.ivf_steps):
        idx.search_device(batches[s_ % nb], k, oi, od, oc, stream=stream)
        stages.append(px.last_timings())
        scanned.append(px.IvfPqIndex.last_scanned())
    px.set_profiling(False)
    scan_ms = float(np.mean([t["candidates_ms"] for t in stages]))
    entry_bytes = 16 + 4
    bytes_per_launch = float(np.mean(scanned)) * entry_bytes
    gbs = bytes_per_launch / (scan_ms * 1e-3) / 1e9
    log(f"[bench] ivfpq: {step_s * 1e3:.3f} ms/step = {B / step_s:.0f} QPS; scan {scan_ms:.3f} ms, "
        f"{bytes_per_launch / 1e9:.3f} GB/launch = {gbs:.0f} GB/s")
    if args.profile_core:
        return {"ms_per_step": round(step_s * 1e3, 4), "scan_ms": round(scan_ms, 4),
                "scanned_entries": float(np.mean(scanned))}
    # recall@10 against the exact GPU flat index over the same vectors
    m = 1024
    flat = px.FlatIndex(px.VectorSpace(dim, px.Metric.EUCLIDEAN), n)
    flat.insert_device(ids, x)
    qh = queries.cpu().numpy()
    ti, _, _ = flat.search_batch(qh[:m], k)
    del flat

    def recall_of(gi, gc):
        return float(np.mean([len(set(ti[i].tolist()) & set(gi[i, :gc[i]].tolist())) / k for i in range(m)]))

    gi, gd, gc = idx.search_batch(qh[:m], k)
    recall = recall_of(gi, gc)
    # the reference harness's dial (bench.rs:267-300): recall@10 and throughput
    # against nprobe, on the same index and batches
    sweep = []
    for npb in (1, 4, 16, 32, 64, 256):
        for s_ in range(2):
            idx.search_device(batches[s_ % nb], k, oi, od, oc, nprobe=npb, stream=stream)
        torch.cuda.synchronize()
        reps = max(3, min(args.ivf_steps, 10))
        t0 = time.perf_counter()
        for s_ in range(reps):
            idx.search_device(batches[s_ % nb], k, oi, od, oc, nprobe=npb, stream=stream)
        torch.cuda.synchronize()
        t = (time.perf_counter() - t0) / reps
        si, _, sc = idx.search_batch(qh[:m], k, nprobe=npb)
        sweep.append({"nprobe": npb, "queries_per_s": round(B / t, 2), "ms_per_step": round(t * 1e3, 4),
                      "recall_at_10_vs_exact": round(recall_of(si, sc), 4)})
        log(f"[bench] ivfpq nprobe {npb}: {t * 1e3:.3f} ms/step = {B / t:.0f} QPS, recall@10 {sweep[-1]['recall_at_10_vs_exact']:.4f}")
    # the same trained parts with an exact rerank of the best 100 ADC
    # candidates (IvfPqConfig::with_rerank, ivfpq.rs:1094-1109)
    rr = 100
    cents_h, books_h, codes_h, list_of_h = idx.parts()
    idx_rr = px.IvfPqIndex(px.VectorSpace(dim, px.Metric.EUCLIDEAN),
                           px.IvfPqConfig(4096, 16).with_nprobe(nprobe).with_rerank(rr).with_train_threshold(1 << 63))
    idx_rr.insert_device(ids, x)
    idx_rr.load_trained(cents_h, books_h, codes_h, list_of_h)
    del x
    torch.cuda.empty_cache()
    for s_ in range(3):
        idx_rr.search_device(batches[s_ % nb], k, oi, od, oc, stream=stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s_ in range(args.ivf_steps):
        idx_rr.search_device(batches[s_ % nb], k, oi, od, oc, stream=stream)
    torch.cuda.synchronize()
    rr_step = (time.perf_counter() - t0) / args.ivf_steps
    ri, _, rc = idx_rr.search_batch(qh[:m], k)
    recall_rr = recall_of(ri, rc)
    del idx_rr
    torch.cuda.empty_cache()
    log(f"[bench] ivfpq rerank {rr}: {rr_step * 1e3:.3f} ms/step = {B / rr_step:.0f} QPS, recall@10 {recall_rr:.4f}")
    host = host_path(idx.search_batch, [qh[i * B:(i + 1) * B] for i in range(3)], k)
    lat = latency_batch1(idx.search_all, qh, k)
    out = {"value": round(B / step_s, 2), "unit": "queries/s", "ms_per_step": round(step_s * 1e3, 4),
           "steps": args.ivf_steps,
           "config": {"workload": "IVF-PQ search, Euclidean, 10M x 128 f32, nlist 4096, PQ 16x256, nprobe 32, "
                                  "batch 1024, k=10", "n": n, "dim": dim, "nlist": 4096, "subspaces": 16,
                      "nprobe": nprobe, "batch": B, "k": k,
                      "inputs": inputs_info(seed, "1000 centres N(0,1)^128; each point and query takes a cluster "
                                                  "drawn from the stream, + 0.15 N(0,1)")},
           "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                        "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": load_traffic("ivf_scan")},
           "kernel": "ivf_scan", "scanned_entries_per_launch": float(np.mean(scanned)),
           "stage_ms": {key: round(float(np.mean([t[key] for t in stages])), 4) for key in stages[0]},
           "train_s": round(train_s, 2), "training_report": rep._asdict(), "recall_at_10_vs_exact": round(recall, 4),
           "recall_queries": m,
           "nprobe_sweep": sweep,
           "rerank100": {"value": round(B / rr_step, 2), "unit": "queries/s", "ms_per_step": round(rr_step * 1e3, 4),
                         "recall_at_10_vs_exact": round(recall_rr, 4),
                         "note": "same trained parts, exact rerank of the best 100 ADC candidates per query"},
           "host_path": host, "latency_batch1": lat}
    if not args.no_cpu:
        from oracle import oracle as orc
        cents, books, codes, list_of = cents_h, books_h, codes_h, list_of_h
        mq = args.queries
        log(f"[bench] ivfpq CPU baseline: oracle IVF-PQ search, {mq} queries, {args.cpu_threads} threads")
        t0 = time.perf_counter()
        wi, wd, wc = orc.ivf_search(0, cents, books, codes, list_of, ids, qh[:mq], k, nprobe, 16,
                                    threads=args.cpu_threads)
        cpu_s = time.perf_counter() - t0
        gi, gd, gc = idx.search_batch(qh[:mq], k)
        same = int(sum(np.array_equal(gi[i], wi[i]) and np.array_equal(gd[i].view(np.uint32), wd[i].view(np.uint32))
                       for i in range(mq)))
        out["cpu_baseline"] = {"value": round(mq / cpu_s, 2), "unit": "queries/s", "cores": args.cpu_threads,
                               "kind": "port", "sample": f"all {mq} queries, oracle IvfPqIndex::search restatement on "
                                                         f"the GPU-trained parts, {args.cpu_threads} threads, "
                                                         f"{cpu_s:.2f}s (includes its O(n) list build)"}
        m1 = args.ivf_cpu1_sample
        t0 = time.perf_counter()
        orc.ivf_search(0, cents, books, codes, list_of, ids, qh[:m1], k, nprobe, 16, threads=1)
        cpu_1 = time.perf_counter() - t0
        out["cpu_baseline_1core"] = {"value": round(m1 / cpu_1, 2), "unit": "queries/s", "cores": 1, "kind": "port",
                                     "sample": f"{m1} queries on one thread, {cpu_1:.2f}s (includes its O(n) list "
                                               f"build)"}
        out["parity_sample"] = {"queries": mq, "bit_exact": same}
        log(f"[bench] ivfpq CPU {mq / cpu_s:.1f} QPS ({args.cpu_threads} threads), {m1 / cpu_1:.1f} QPS (1 thread); "
            f"GPU/oracle bit-exact on {same}/{mq}")
    out["mutate_cycle"] = ivf_mutate_cycles(args, torch, px, dev, idx, batches, stream, k, cents_h, books_h)
    return out


def ivf_mutate_cycles(args, torch, px, dev, idx, batches, stream, k, cents, books):
    """IvfPqIndex insert/remove (ivfpq.rs:1129-1180) between searches at the
    full 10M size: each cycle removes 100 ids, inserts 100 new vectors from the
    same mixture and searches one 1,024-query batch. The list view is updated
    in place (appends, holes filled, regions moved when full), so a cycle
    costs its mutations plus one search, not a rebuild of the lists."""
    B, dim = batches[0].shape
    nb = len(batches)
    cycles, per = 20, 100
    oi = torch.empty((B, k), dtype=torch.int64, device=dev)
    od = torch.empty((B, k), dtype=torch.float32, device=dev)
    oc = torch.empty((B,), dtype=torch.int32, device=dev)
    new, _ = mixture(torch, px, dev, cycles * per, dim, 1000, 0.15, 0, True, args.seed + 8)
    ids, live = idx.slots()
    present = ids[live.astype(bool)]
    rng = np.random.default_rng(args.seed)
    victims = rng.choice(present, size=cycles * per, replace=False)
    next_id = int(ids.max()) + 1
    r0, m0 = idx.view_stats()
    t_rm = t_ins = t_srch = 0.0
    torch.cuda.synchronize()
    t_all = time.perf_counter()
    for c in range(cycles):
        t0 = time.perf_counter()
        for i in victims[c * per:(c + 1) * per]:
            idx.remove(int(i))
        t1 = time.perf_counter()
        idx.insert_device(np.arange(next_id, next_id + per, dtype=np.uint64), new[c * per:(c + 1) * per])
        next_id += per
        t2 = time.perf_counter()
        idx.search_device(batches[c % nb], k, oi, od, oc, stream=stream)
        torch.cuda.synchronize()
        t3 = time.perf_counter()
        t_rm += t1 - t0
        t_ins += t2 - t1
        t_srch += t3 - t2
    t_all = time.perf_counter() - t_all
    r1, m1 = idx.view_stats()
    res = {"cycles": cycles, "removed_per_cycle": per, "inserted_per_cycle": per,
           "ms_per_cycle": round(t_all / cycles * 1e3, 3), "remove_ms_per_id": round(t_rm / (cycles * per) * 1e3, 4),
           "insert_ms_per_batch": round(t_ins / cycles * 1e3, 3), "search_ms": round(t_srch / cycles * 1e3, 3),
           "view_rebuilds": r1 - r0, "view_region_moves": m1 - m0,
           "note": "remove 100 ids, insert 100 vectors (insert_device), search one batch of 1024, per cycle"}
    if not args.no_cpu:
        from oracle import oracle as orc
        ids, live = idx.slots()
        _, _, codes, list_of = idx.parts()
        qh = batches[0][:256].cpu().numpy()
        gi, gd, gc = idx.search_batch(qh, k)
        wi, wd, wc = orc.ivf_search(0, cents, books, codes, list_of, ids, qh, k, 32, 16, live=live,
                                    threads=args.cpu_threads)
        same = int(sum(np.array_equal(gi[i], wi[i]) and np.array_equal(gd[i].view(np.uint32), wd[i].view(np.uint32))
                       for i in range(qh.shape[0])))
        res["parity_after_mutations"] = {"queries": qh.shape[0], "bit_exact": same}
    log(f"[bench] ivfpq mutate cycle: {res['ms_per_cycle']} ms (remove {res['remove_ms_per_id']} ms/id, insert "
        f"{res['insert_ms_per_batch']} ms/100, search {res['search_ms']} ms); view rebuilds {r1 - r0}, "
        f"region moves {m1 - m0}; parity {res.get('parity_after_mutations')}")
    return res


PEAK_INT8_MFMA_TOPS = 5000.0


def bench_sq8(args, torch, px, dev):
    """SQ8 flat search, inner product, k=10: 10M x 96 f32 ~U(-1,1), per-dimension
    ranges calibrated on the first 100,000 vectors, I8 codes; 10,000 queries
    ~U(-1,1) quantised the same way, batches of 1,024. Score = -(float) of the
    exact int32 code dot product (integer MFMA)."""
    n, dim, B, k = args.sq8_n, 96, args.batch, 10
    seed = args.seed + 11
    xq = torch.empty((n + args.queries, dim), dtype=torch.float32, device=dev)
    px.uniform_generate_device(n + args.queries, dim, -1.0, 1.0, seed, xq)  # corpus rows, then the queries
    x, queries = xq[:n], xq[n:]
    ids = np.arange(n, dtype=np.uint64)
    idx = px.Sq8Index(px.VectorSpace(dim, px.Metric.INNER_PRODUCT), capacity=n)
    t0 = time.time()
    idx.train_device(x[:100_000].contiguous())
    idx.insert_device(ids, x)
    torch.cuda.synchronize()
    log(f"[bench] sq8: calibrated on 100000 and encoded {n}x{dim} in {time.time() - t0:.2f}s")
    nb = args.queries // B
    batches = [queries[i * B:(i + 1) * B] for i in range(nb)]
    oi = torch.empty((B, k), dtype=torch.int64, device=dev)
    od = torch.empty((B, k), dtype=torch.float32, device=dev)
    oc = torch.empty((B,), dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    for s_ in range(3):
        idx.search_device(batches[s_ % nb], k, oi, od, oc, stream=stream)
    torch.cuda.synchronize()
    fallbacks = 0
    t0 = time.perf_counter()
    for s_ in range(args.sq8_steps):
        idx.search_device(batches[s_ % nb], k, oi, od, oc, stream=stream)
        fallbacks += px.Sq8Index.last_fallbacks()
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t0) / args.sq8_steps
    px.set_profiling(True)
    stages = []
    for s_ in range(args.sq8_steps):
        idx.search_device(batches[s_ % nb], k, oi, od, oc, stream=stream)
        stages.append(px.last_timings())
    px.set_profiling(False)
    scan_ms = float(np.mean([t["candidates_ms"] for t in stages]))
    tops = 2.0 * n * dim * B / (scan_ms * 1e-3) / 1e12
    log(f"[bench] sq8: {step_s * 1e3:.3f} ms/step = {B / step_s:.0f} QPS; stage-2 scan {scan_ms:.3f} ms = "
        f"{tops:.0f} TOP/s; fallback queries {fallbacks}")
    if args.profile_core:
        return {"ms_per_step": round(step_s * 1e3, 4), "scan_ms": round(scan_ms, 4)}
    # recall@10 against exact f32 inner product over the same vectors
    m = 200
    qh = queries.cpu().numpy()
    flat = px.FlatIndex(px.VectorSpace(dim, px.Metric.INNER_PRODUCT), n)
    flat.insert_device(ids, x)
    ti, _, _ = flat.search_batch(qh[:m], k)
    del flat
    gi, gd, gc = idx.search_batch(qh[:m], k)
    recall = float(np.mean([len(set(ti[i].tolist()) & set(gi[i, :gc[i]].tolist())) / k for i in range(m)]))
    ri, _, rc = idx.search_batch(qh[:m], k, rescore=100)
    recall_rs = float(np.mean([len(set(ti[i].tolist()) & set(ri[i, :rc[i]].tolist())) / k for i in range(m)]))
    host = host_path(idx.search_batch, [qh[i * B:(i + 1) * B] for i in range(3)], k)
    lat = latency_batch1(idx.search_all, qh, k)
    x_host = None if args.no_cpu else x.cpu().numpy()
    del x
    torch.cuda.empty_cache()
    out = {"value": round(B / step_s, 2), "unit": "queries/s", "ms_per_step": round(step_s * 1e3, 4),
           "steps": args.sq8_steps,
           "config": {"workload": "SQ8 flat search, inner product, 10M x 96 f32 ~U(-1,1) as I8 codes, batch 1024, "
                                  "k=10", "n": n, "dim": dim, "batch": B, "k": k, "calibration": 100_000,
                      "inputs": inputs_info(seed, "U(-1,1) = -1 + 2 gen::<f32>(), corpus rows then the queries")},
           "roofline": {"bound": "mfma", "achieved": round(tops, 1), "peak": PEAK_INT8_MFMA_TOPS, "unit": "TOP/s",
                        "frac": round(tops / PEAK_INT8_MFMA_TOPS, 4), "traffic": load_traffic("sq8_mfma_scan")},
           "kernel": "sq8_mfma_scan (stage 2)", "fallback_queries": fallbacks,
           "stage_ms": {key: round(float(np.mean([t[key] for t in stages])), 4) for key in stages[0]},
           "recall_at_10_vs_f32_ip": round(recall, 4), "recall_at_10_rescore100": round(recall_rs, 4),
           "host_path": host, "latency_batch1": lat}
    if not args.no_cpu:
        from oracle import oracle as orc
        mn, sc, inv, _ = orc.sq_train(x_host[:100_000], True)
        qz = idx.quantizer()
        ranges_same = bool(np.array_equal(qz.min.view(np.uint32), mn.view(np.uint32)) and
                           np.array_equal(qz.inverse_scale.view(np.uint32), inv.view(np.uint32)))
        codes = orc.sq_encode(x_host, mn, inv, True, 1, threads=args.cpu_threads).view(np.int8)
        del x_host
        mq = args.sq8_cpu_sample
        qc = orc.sq_encode(qh[:mq], mn, inv, True, 1).view(np.int8)
        log(f"[bench] sq8 CPU baseline: oracle integer SQ8 scan, {mq} queries, {args.cpu_threads} threads")
        t0 = time.perf_counter()
        wi, wd, wc = orc.sq8_search(codes, ids, qc, k, threads=args.cpu_threads)
        cpu_s = time.perf_counter() - t0
        gi, gd, gc = idx.search_batch(qh[:mq], k)
        same = int(sum(np.array_equal(gi[i], wi[i]) and np.array_equal(gd[i].view(np.uint32), wd[i].view(np.uint32))
                       for i in range(mq)))
        out["cpu_baseline"] = {"value": round(mq / cpu_s, 3), "unit": "queries/s", "cores": args.cpu_threads,
                               "kind": "port", "sample": f"{mq} queries, each a full 10M x 96 integer scan, oracle "
                                                         f"SQ8 restatement, {args.cpu_threads} threads, {cpu_s:.2f}s"}
        m1 = args.sq8_cpu1_sample
        t0 = time.perf_counter()
        orc.sq8_search(codes, ids, qc[:m1], k, threads=1)
        cpu_1 = time.perf_counter() - t0
        out["cpu_baseline_1core"] = {"value": round(m1 / cpu_1, 3), "unit": "queries/s", "cores": 1, "kind": "port",
                                     "sample": f"{m1} queries on one thread, each a full 10M x 96 integer scan, "
                                               f"{cpu_1:.2f}s"}
        out["parity_sample"] = {"queries": mq, "bit_exact": same, "ranges_bit_exact": ranges_same}
        log(f"[bench] sq8 CPU {mq / cpu_s:.2f} QPS ({args.cpu_threads} threads), {m1 / cpu_1:.2f} QPS (1 thread); "
            f"GPU/oracle bit-exact on {same}/{mq}; ranges equal {ranges_same}")
    return out


def bench_kmeans(args, torch, px, dev):
    """k-means training (Lloyd): 2,000,000 x 128 f32 from 4,096 Gaussian clusters
    (centres N(0,1), sigma 0.2) into 4,096 centroids, k-means++ seeding from
    the seed, 10 Lloyd iterations; then PQ 16 x 256 trained on the residuals
    (25 iterations per subspace)."""
    n, dim, K, iters = args.km_n, 128, 4096, 10
    seed = args.seed + 13
    x, _ = mixture(torch, px, dev, n, dim, K, 0.2, 0, True, seed)
    seeds = torch.empty((K, dim), device=dev)
    cents = torch.empty((K, dim), device=dev)
    assign = torch.empty(n, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    px.kmeans_device(x, K, 0, args.seed, seeds)  # k-means++ seeding only
    t_seed = time.perf_counter() - t0
    inexact_seed = px.kmeans_last_stats()["inexact_sums"]
    t0 = time.perf_counter()
    inertia, its = px.kmeans_device(x, K, iters, args.seed, cents, assign, init=seeds)
    t_lloyd = time.perf_counter() - t0
    st = px.kmeans_last_stats()
    t_pq, pq_its = float("nan"), 0
    if not args.km_skip_pq:
        resid = (x - cents[assign.long()]).contiguous()
        books = torch.empty(dim * 256, device=dev)
        t0 = time.perf_counter()
        pq = px.ProductQuantizer.train_device(px.VectorSpace(dim, px.Metric.EUCLIDEAN), resid,
                                              px.PqConfig(16).with_seed(args.seed), books)
        t_pq = time.perf_counter() - t0
        pq_its = pq.training_iterations
    per_iter = t_lloyd / max(its, 1)
    flops = 2.0 * n * K * dim  # per assignment pass
    tflops = flops / per_iter / 1e12
    # the dominant kernel: the FP32-MFMA distance pass of the assignments
    # (HIP events around each launch, on the library's stream)
    mfma_ms = st["mfma_ms"] / max(st["mfma_passes"], 1)
    mfma_tflops = st["mfma_flops"] / max(st["mfma_ms"], 1e-9) / 1e9
    log(f"[bench] kmeans: seeding {t_seed:.2f}s, {its} Lloyd iterations {t_lloyd:.2f}s ({per_iter * 1e3:.1f} ms each, "
        f"{tflops:.1f} TFLOP/s by 2nKd per iteration), inertia {inertia:.1f}; MFMA distance pass "
        f"{mfma_ms:.2f} ms = {mfma_tflops:.1f} TFLOP/s over {st['mfma_passes']} passes, "
        f"{st['rescanned']} points rescanned exactly; PQ 16x256 on residuals "
        + ("skipped" if args.km_skip_pq else f"{t_pq:.2f}s ({pq_its} iterations)"))
    out = {"value": round(1.0 / per_iter, 3), "unit": "Lloyd iterations/s", "ms_per_iteration": round(per_iter * 1e3, 2),
           "config": {"workload": "k-means 2M x 128 f32 -> 4096, k-means++ then 10 Lloyd iterations; PQ 16x256 on "
                                  "the residuals", "n": n, "dim": dim, "k": K, "iterations": its,
                      "inputs": inputs_info(seed, "4096 centres N(0,1)^128; each point takes a cluster drawn from "
                                                  "the stream, + 0.2 N(0,1)"),
                      "kmeans_seed": args.seed, "pq_seed": args.seed},
           "roofline": {"bound": "mfma", "achieved": round(mfma_tflops, 2), "peak": PEAK_FP32_MFMA_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(mfma_tflops / PEAK_FP32_MFMA_TFLOPS, 4),
                        "traffic": load_traffic("km_mfma_reg"),
                        "kernel": "km_mfma_reg", "ms_per_launch": round(mfma_ms, 3),
                        "note": "2nKd per assignment pass over the FP32-MFMA approximate distances; winners are "
                                "certified and rescored with the reference's sequential f32 arithmetic"},
           "effective_tflops_per_iteration": round(tflops, 2),
           "mfma_passes": st["mfma_passes"], "rescanned_points": st["rescanned"],
           "inexact_sums": {"seeding": inexact_seed, "lloyd": st["inexact_sums"]},
           "seeding_s": round(t_seed, 3), "lloyd_s": round(t_lloyd, 3), "pq_train_s": None if args.km_skip_pq else round(t_pq, 3),
           "inertia": inertia}
    if not args.no_cpu:
        from oracle import oracle as orc
        ns = args.km_cpu_sample
        sample = x[:ns].cpu().numpy()
        init = seeds.cpu().numpy()
        log(f"[bench] kmeans CPU baseline: oracle assignment pass on {ns} points x {K} centroids, 1 thread")
        t0 = time.perf_counter()
        orc.kmeans_assign(sample, init)
        cpu_s = time.perf_counter() - t0
        cpu_iter = cpu_s * n / ns
        nmt = ns * args.cpu_threads // 2
        sample_mt = x[:nmt].cpu().numpy()
        t0 = time.perf_counter()
        orc.kmeans_assign(sample_mt, init, threads=args.cpu_threads)
        cpu_mt = time.perf_counter() - t0
        cpu_iter_mt = cpu_mt * n / nmt
        # full-size parity of the assignment pass on a slice: GPU kernel vs oracle, final centroids
        m = 4096
        ch = cents.cpu().numpy()
        ga, gd = px.kmeans_assign(x[:m].cpu().numpy(), ch)
        wa, wd = orc.kmeans_assign(x[:m].cpu().numpy(), ch)
        same = int(np.sum((ga == wa) & (gd.view(np.uint32) == wd.view(np.uint32))))
        out["cpu_baseline"] = {"value": round(1.0 / cpu_iter_mt, 6), "unit": "Lloyd iterations/s",
                               "cores": args.cpu_threads, "kind": "port",
                               "sample": f"the assignment pass of one Lloyd iteration (kmeans.rs:90-97 restatement; "
                                         f"the O(n d) update is left out) on {nmt} of the {n} points against the {K} "
                                         f"seeds, points split over {args.cpu_threads} threads: {cpu_mt:.2f}s, scaled "
                                         f"by n/{nmt}"}
        out["cpu_baseline_1core"] = {"value": round(1.0 / cpu_iter, 6), "unit": "Lloyd iterations/s", "cores": 1,
                                     "kind": "port", "sample": f"the same pass on {ns} points, one thread as the "
                                                               f"reference: {cpu_s:.2f}s, scaled by n/{ns}"}
        out["parity_sample"] = {"points": m, "assignments_and_distances_bit_exact": same}
        log(f"[bench] kmeans CPU {cpu_iter:.1f} s per full iteration (1 core), {cpu_iter_mt:.1f} s "
            f"({args.cpu_threads} threads); assignment parity {same}/{m}")
    return out


def bench_fixture(args, torch, px, dev):
    """fixture::generate (proxima-cli/src/fixture.rs:71-123) on the GPU: the
    reference bench harness's corpus generator, at 10M x 128 from 1000
    clusters with 10,000 queries. Bound by the HBM writes of the output."""
    n, dim, clusters, nq = args.fx_n, 128, 1000, 10_000
    v = torch.empty((n, dim), dtype=torch.float32, device=dev)
    q = torch.empty((nq, dim), dtype=torch.float32, device=dev)
    px.fixture_generate_device(n, dim, clusters, nq, args.seed, v, q)  # warm-up
    torch.cuda.synchronize()
    reps = 3
    t0 = time.perf_counter()
    for _ in range(reps):
        px.fixture_generate_device(n, dim, clusters, nq, args.seed, v, q)
    torch.cuda.synchronize()
    t = (time.perf_counter() - t0) / reps
    written = (n + nq) * dim * 4
    gbs = written / t / 1e9
    out = {"value": round(written / t / 2**20, 1), "unit": "MiB/s of f32 generated", "ms_per_run": round(t * 1e3, 3),
           "config": {"workload": "fixture::generate 10M x 128 f32, 1000 clusters, 10,000 queries", "count": n,
                      "dim": dim, "clusters": clusters, "queries": nq, "seed": args.seed},
           "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                        "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
                        "note": "bytes written per run over the host-timed run (3 launches + one host sync); "
                                "the kernels are bound by the f64 ln and cos of the Box-Muller step, not by HBM"}}
    log(f"[bench] fixture: {n}x{dim} + {nq} queries in {t * 1e3:.2f} ms = {gbs:.0f} GB/s written")
    if not args.no_cpu:
        from oracle import oracle as orc
        ns = 200_000
        t0 = time.perf_counter()
        wv, _ = orc.fixture_generate(ns, dim, clusters, 0, args.seed)
        cpu_s = time.perf_counter() - t0
        got = v[:ns].cpu().numpy()
        same = float(np.mean(got.view(np.uint32) == wv.view(np.uint32)))
        worst = float(np.max(np.abs(got.astype(np.float64) - wv.astype(np.float64))))
        out["cpu_baseline"] = {"value": round(ns * dim * 4 / cpu_s / 2**20, 1), "unit": "MiB/s of f32 generated",
                               "cores": 1, "kind": "port",
                               "sample": f"oracle fixture_generate restatement, {ns} x {dim} points, 1 thread, "
                                         f"{cpu_s:.2f}s (the reference draws every value from one sequential "
                                         f"ChaCha8 stream, so its CPU path has no multi-thread form)"}
        out["parity"] = {"points": ns, "bit_identical_fraction": round(same, 6), "max_abs_diff": worst}
        log(f"[bench] fixture CPU {ns * dim * 4 / cpu_s / 2**20:.1f} MiB/s (1 core); bit-identical {same:.6f} of "
            f"the first {ns} points, max |diff| {worst:.2e}")
    del v, q
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--dim", type=int, default=768)
    ap.add_argument("--queries", type=int, default=10_000)
    ap.add_argument("--batch", type=int, default=1024)
    ap.add_argument("--k", type=int, default=10)
    ap.add_argument("--seed", type=int, default=0x9E3779B9)
    ap.add_argument("--cpu-sample", type=int, default=2048)
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--skip-ivfpq", action="store_true")
    ap.add_argument("--ivf-only", action="store_true", help="run only the IVF-PQ leg (prints its JSON object)")
    ap.add_argument("--ivf-n", type=int, default=10_000_000)
    ap.add_argument("--ivf-steps", type=int, default=20)
    ap.add_argument("--skip-sq8", action="store_true")
    ap.add_argument("--sq8-only", action="store_true", help="run only the SQ8 leg (prints its JSON object)")
    ap.add_argument("--sq8-n", type=int, default=10_000_000)
    ap.add_argument("--sq8-steps", type=int, default=20)
    ap.add_argument("--sq8-cpu-sample", type=int, default=2048)
    ap.add_argument("--sq8-cpu1-sample", type=int, default=32)
    ap.add_argument("--ivf-cpu1-sample", type=int, default=1000)
    ap.add_argument("--cpu1-sample", type=int, default=32, help="queries of the one-thread CPU baseline of the 1M x 768 cosine search")
    ap.add_argument("--skip-c1", action="store_true")
    ap.add_argument("--c1-only", action="store_true", help="run only the 100k x 128 flat leg (prints its JSON object)")
    ap.add_argument("--c1-steps", type=int, default=50)
    ap.add_argument("--skip-kmeans", action="store_true")
    ap.add_argument("--kmeans-only", action="store_true", help="run only the k-means leg (prints its JSON object)")
    ap.add_argument("--km-n", type=int, default=2_000_000)
    ap.add_argument("--km-skip-pq", action="store_true",
                    help="k-means leg without the PQ training (one host thread; for counter profiling)")
    ap.add_argument("--km-cpu-sample", type=int, default=131072)
    ap.add_argument("--skip-fixture", action="store_true")
    ap.add_argument("--profile-core", action="store_true",
                    help="only the timed and stage-timed batches of the leg that runs (the flat cosine leg, or "
                         "the one --c1-only, --ivf-only or --sq8-only picks; for profiler runs)")
    ap.add_argument("--fixture-only", action="store_true", help="run only the fixture leg (prints its JSON object)")
    ap.add_argument("--fx-n", type=int, default=10_000_000)
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="also run one device copy of this size (a known-size kernel for scaling PMC byte counters)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: --gpus {args.gpus} is not supported "
              "(the flat search shards by database rows; that path is design-only here).", flush=True)
        sys.exit(2)

    import torch

    import proxima_amd as px

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_probe_mib:
        src = torch.empty(args.copy_probe_mib << 18, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copy probe: {args.copy_probe_mib} MiB device-to-device copy")
        del src, dst
        torch.cuda.empty_cache()
    if args.c1_only:
        print(json.dumps(bench_c1(args, torch, px, dev)), flush=True)
        return
    if args.ivf_only:
        print(json.dumps(bench_ivfpq(args, torch, px, dev)), flush=True)
        return
    if args.sq8_only:
        print(json.dumps(bench_sq8(args, torch, px, dev)), flush=True)
        return
    if args.kmeans_only:
        print(json.dumps(bench_kmeans(args, torch, px, dev)), flush=True)
        return
    if args.fixture_only:
        print(json.dumps(bench_fixture(args, torch, px, dev)), flush=True)
        return
    n, dim, B = args.n, args.dim, args.batch
    log(f"[bench] generating {n}x{dim} corpus + {args.queries} queries on the GPU")
    x, queries = mixture(torch, px, dev, n, dim, 256, 1.0, args.queries, False, args.seed)

    idx = px.FlatIndex(px.VectorSpace(dim, px.Metric.COSINE), n)
    t0 = time.time()
    idx.insert_device(np.arange(n, dtype=np.uint64), x)
    torch.cuda.synchronize()
    log(f"[bench] inserted {n} vectors in {time.time() - t0:.2f}s")
    x_host = None
    if not args.no_cpu:
        x_host = x.cpu().numpy()
    del x
    torch.cuda.empty_cache()

    nb = args.queries // B
    batches = [queries[i * B:(i + 1) * B] for i in range(nb)]

    def run(k, steps, warmup, prof=False):
        oi = torch.empty((B, k), dtype=torch.int64, device=dev)
        od = torch.empty((B, k), dtype=torch.float32, device=dev)
        oc = torch.empty((B,), dtype=torch.int32, device=dev)
        stream = torch.cuda.current_stream(dev).cuda_stream
        for s in range(warmup):
            idx.search_device(batches[s % nb], k, oi, od, oc, stream=stream)
        px.set_profiling(prof)
        stages = []
        fallbacks = 0
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for s in range(steps):
            idx.search_device(batches[s % nb], k, oi, od, oc, stream=stream)
            fallbacks += px.FlatIndex.last_fallbacks()
            if prof:
                stages.append(px.last_timings())
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        px.set_profiling(False)
        return (t1 - t0) / steps, stages, fallbacks

    log(f"[bench] k={args.k}: {args.warmup} warmup + {args.steps} timed steps of {B} queries")
    step_s, _, fb = run(args.k, args.steps, args.warmup)
    # the same steps again with stage events, for the dominant-kernel roofline
    _, stages, _ = run(args.k, args.steps, 1, prof=True)
    cand_ms = float(np.mean([s["candidates_ms"] for s in stages]))
    stage_mean = {key: round(float(np.mean([s[key] for s in stages])), 4) for key in stages[0]}
    flops = 2.0 * n * dim * B
    achieved = flops / (cand_ms * 1e-3) / 1e12
    log(f"[bench] k={args.k}: {step_s * 1e3:.3f} ms/step, candidate GEMM {cand_ms:.3f} ms = {achieved:.1f} TFLOP/s")
    if args.profile_core:
        print(json.dumps({"ms_per_step": round(step_s * 1e3, 4), "candidates_ms": round(cand_ms, 4)}), flush=True)
        return

    k2 = 100
    step100, stages100, fb100 = run(k2, max(5, args.steps // 2), 1, prof=True)
    log(f"[bench] k=100: {step100 * 1e3:.3f} ms/step")

    # the partial last batch of the 10,000 queries (9 x 1024 + 784)
    tail = queries[nb * B:]
    tail_info = None
    if tail.shape[0]:
        nt = tail.shape[0]
        toi = torch.empty((nt, args.k), dtype=torch.int64, device=dev)
        tod = torch.empty((nt, args.k), dtype=torch.float32, device=dev)
        toc = torch.empty((nt,), dtype=torch.int32, device=dev)
        stream = torch.cuda.current_stream(dev).cuda_stream
        idx.search_device(tail, args.k, toi, tod, toc, stream=stream)
        torch.cuda.synchronize()
        reps = 5
        t0 = time.perf_counter()
        for _ in range(reps):
            idx.search_device(tail, args.k, toi, tod, toc, stream=stream)
        torch.cuda.synchronize()
        tail_s = (time.perf_counter() - t0) / reps
        all_s = nb * step_s + tail_s
        tail_info = {"queries": nt, "ms": round(tail_s * 1e3, 4),
                     "all_queries_per_s": round(args.queries / all_s, 2),
                     "note": f"{nb} full batches at ms_per_step plus this tail: the whole {args.queries}-query set"}
        log(f"[bench] tail batch of {nt}: {tail_s * 1e3:.3f} ms; all {args.queries} queries at "
            f"{args.queries / all_s:.0f} QPS")
    qhost = queries.cpu().numpy()
    host = host_path(idx.search_batch, [qhost[i * B:(i + 1) * B] for i in range(2)], args.k, reps=5)
    lat = latency_batch1(idx.search_all, qhost, args.k, repeats=100)
    log(f"[bench] host path {host['ms_per_batch']} ms/batch; batch-1 latency mean {lat['mean_us']} us, "
        f"p95 {lat['p95_us']} us")

    cpu = None
    cpu1 = None
    parity = None
    if not args.no_cpu:
        from oracle import oracle as orc
        m = min(args.cpu_sample, args.queries)
        log(f"[bench] CPU baseline: oracle flat search, {m} queries, {args.cpu_threads} threads")
        xp = orc.prepare_rows(orc.COSINE, x_host, threads=args.cpu_threads)
        del x_host
        qh = queries[:m].cpu().numpy()
        qp = orc.prepare_rows(orc.COSINE, qh, threads=args.cpu_threads)
        ids = np.arange(n, dtype=np.uint64)
        t0 = time.perf_counter()
        wi, wd, wc = orc.flat_search(xp, ids, orc.COSINE, qp, args.k, threads=args.cpu_threads)
        cpu_s = time.perf_counter() - t0
        cpu = {"value": round(m / cpu_s, 3), "unit": "queries/s", "cores": args.cpu_threads, "kind": "port",
               "sample": f"{m} queries of the same workload (each a full 1M x 768 exact scan), oracle "
                         f"FlatIndex::search restatement, {args.cpu_threads} host threads, {cpu_s:.2f}s"}
        m1 = min(args.cpu1_sample, m)
        t0 = time.perf_counter()
        orc.flat_search(xp, ids, orc.COSINE, qp[:m1], args.k, threads=1)
        cpu_1 = time.perf_counter() - t0
        cpu1 = {"value": round(m1 / cpu_1, 3), "unit": "queries/s", "cores": 1, "kind": "port",
                "sample": f"{m1} queries on one thread (the reference's single-threaded scan), {cpu_1:.2f}s"}
        # parity of the GPU results on the same sample, full size
        gi, gd, gc = idx.search_batch(qh, args.k)
        same = int(sum(np.array_equal(gi[i], wi[i]) and np.array_equal(gd[i].view(np.uint32), wd[i].view(np.uint32))
                       for i in range(m)))
        parity = {"queries": m, "bit_exact": same}
        log(f"[bench] CPU {cpu['value']} QPS; GPU/oracle bit-exact on {same}/{m} sample queries")

    del idx
    torch.cuda.empty_cache()
    c1 = None
    if not args.skip_c1:
        c1 = bench_c1(args, torch, px, dev)
        torch.cuda.empty_cache()
    ivf = None
    if not args.skip_ivfpq:
        ivf = bench_ivfpq(args, torch, px, dev)
        torch.cuda.empty_cache()
    sq8 = None
    if not args.skip_sq8:
        sq8 = bench_sq8(args, torch, px, dev)
        torch.cuda.empty_cache()
    km = None
    if not args.skip_kmeans:
        km = bench_kmeans(args, torch, px, dev)
        torch.cuda.empty_cache()
    fx = None
    if not args.skip_fixture:
        fx = bench_fixture(args, torch, px, dev)

    out = {
        "metric": METRIC,
        "value": round(B / step_s, 2),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: N(0,1) + one of 256 N(0,1) cluster offsets (i % 256), L2-normalised by the index's "
                "prepare step; ChaCha8 stream from the recorded seed, generated on the GPU",
        "config": {"workload": "flat exact search, cosine, 1M x 768 f32, batch 1024, k=10", "n": n, "dim": dim,
                   "batch": B, "k": args.k, "metric": "cosine", "queries": args.queries,
                   "inputs": inputs_info(args.seed, "256 centres N(0,1)^768; x_i = centre[i % 256] + N(0,1); "
                                                    "query q = centre[q % 256] + N(0,1)")},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
                     "traffic": load_traffic("flat_mfma_candidates")},
        "cpu_baseline": cpu,
        "cpu_baseline_1core": cpu1,
        "host": {"cpu_model": cpu_model(), "cpu_count": os.cpu_count(), "cpu_threads_used": args.cpu_threads},
        "kernel": "flat_mfma_candidates",
        "stage_ms": stage_mean,
        "fallback_queries": fb,
        "k100": {"value": round(B / step100, 2), "ms_per_step": round(step100 * 1e3, 4),
                 "candidates_ms": round(float(np.mean([s["candidates_ms"] for s in stages100])), 4),
                 "fallback_queries": fb100},
        "parity_sample": parity,
        "tail_batch": tail_info,
        "host_path": host,
        "latency_batch1": lat,
        "c1": c1,
        "ivfpq": ivf,
        "sq8": sq8,
        "kmeans": km,
        "fixture": fx,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
