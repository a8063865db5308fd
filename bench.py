"""Benchmark: standard GPU Vamana build throughput on one MI355X.

A step is one full build (medoid, init, 4 x (search + online insert, reverse
merge, prune)) of the configured synthetic workload, with the vectors already
resident in HBM. value = vertices/s = N / seconds per build.

Prints ONE JSON line. Also reports recall@10 of the built graph (GPU
best-first search against exact ground truth on a query subset), the HBM roofline of the
dominant kernel (search + online insert; algorithmic bytes counted on device,
duration from HIP events on the build stream) and the CPU baseline (the CPU
oracle of the same algorithm on a bounded sample, on this host's cores).

--config c5f / c5s measure the label-filtered and stitched builds on the c5
workload (recall of label-filtered search against per-label exact ground
truth); the default run is the c3 standard build.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
# The filtered build's reference-format log goes to stdout, which carries the
# bench line here; its extra per-round work also stays out of the timed region.
os.environ.setdefault("DANCE_FILTERED_LOG", "0")

HBM_PEAK_GBS = 8000.0
WORKLOADS = {
    "c1": "c1: 100k x 96 fp32 N(0,I) L2-normalized, seed 42; R64 L100 C80 STEPS64 alpha1.2",
    "c2": "c2: 1M x 96 fp32 256-center Gaussian mixture sigma 0.3 L2-normalized, seed 42; R64 L100 C80 STEPS64 alpha1.2",
    "c3": "c3: 10M x 96 fp32 256-center Gaussian mixture sigma 0.3 L2-normalized, seed 42; R64 L100 C80 STEPS64 alpha1.2",
    "c4": "c4: 10M x 128 uint8 clip(round(64+24z)) 1024-center mixture, seed 42; R64 L100 C80 STEPS64 alpha1.2",
    "c5f": ("c5 filtered: 1M x 192 uint8 (c4 generator at 192 dims), 1-8 distinct labels/row Zipf(1.0) over 20k, "
            "GPU-FilteredVamana canonical_v2 R64 L=FL=100 alpha1.2 C750 (work C 128) STEPS64, 3 rounds"),
    "c5s": ("c5 stitched: the c5 vectors, 100 partitioned labels (one per row, uniform), StitchedVamana "
            "Rsmall32 Lsmall100 Rstitched64 C96 steps64"),
}
C5 = dict(n=1_000_000, dim=192, centers=1024, sigma=0.3, nq=10_000, vocab=20_000, min_labels=1, max_labels=8,
          R=64, L=100, FL=100, C=750, STEPS=64, alpha=1.2, parts=100, Rsmall=32, Lsmall=100, Rstitched=64, Cs=96)
# profiles that store float input as fp16 (dance_set_profile in include/dance_hip.h)
FP16_PROFILES = ("FAST_SMALL", "PRO6000_100M", "FILTERED_PAPER")
METRIC = "Vamana build seconds + vertices/sec at 10M×96 fp32 R64/L100; recall@10"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def ground_truth(base_t, base_np: np.ndarray, queries: np.ndarray, k: int = 10, rerank: int = 64) -> np.ndarray:
    """Exact top-k: fp32 Gram-form shortlist on the GPU, fp64 re-rank on the host."""
    import torch
    q = torch.from_numpy(queries.astype(np.float32)).to(base_t.device)
    bf = base_t.float()
    n = bf.shape[0]
    xn = (bf * bf).sum(1)
    best_d = torch.full((q.shape[0], rerank), float("inf"), device=q.device)
    best_i = torch.zeros((q.shape[0], rerank), dtype=torch.int64, device=q.device)
    chunk = 1 << 21
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        d = xn[s:e][None, :] - 2.0 * (q @ bf[s:e].T)
        dd, ii = torch.topk(d, min(rerank, e - s), dim=1, largest=False)
        cat_d = torch.cat([best_d, dd], 1)
        cat_i = torch.cat([best_i, ii + s], 1)
        best_d, pos = torch.topk(cat_d, rerank, dim=1, largest=False)
        best_i = torch.gather(cat_i, 1, pos)
    cand = best_i.cpu().numpy()
    out = np.empty((q.shape[0], k), np.uint32)
    for r in range(q.shape[0]):
        ids = np.unique(cand[r])
        rows = base_np[ids]
        dist = ((rows.astype(np.float64) - queries[r].astype(np.float64)) ** 2).sum(1)
        order = np.lexsort((ids, dist))[:k]
        out[r] = ids[order]
    return out


def label_starts_gpu(torch, base_t, ls):
    """Per label: the member nearest (fp64) to the label centroid, ties to the
    smaller id; INVALID for empty labels. Also the global start (nearest to
    the centroid of all points)."""
    from dance_amd import INVALID
    dev = base_t.device
    off, pts = ls.postings()
    nl = ls.num_labels
    cnt = np.diff(off).astype(np.int64)
    lab_of = torch.from_numpy(np.repeat(np.arange(nl), cnt)).to(dev)
    P = torch.from_numpy(pts.astype(np.int64)).to(dev)
    dim = base_t.shape[1]
    # per-label sums from prefix sums over the label-grouped memberships
    # (no atomics); fp64 prefix sums of uint8 rows are exact integers
    ends = np.cumsum(cnt) - 1
    at_end = torch.zeros((max(1, P.shape[0]), dim), dtype=torch.float64, device=dev)
    carry = torch.zeros(dim, dtype=torch.float64, device=dev)
    step = 1 << 20
    for s0 in range(0, P.shape[0], step):
        cs = torch.cumsum(base_t[P[s0:s0 + step]].double(), 0) + carry
        at_end[s0:s0 + cs.shape[0]] = cs
        carry = cs[-1]
    nz = cnt > 0
    sums = torch.zeros((nl, dim), dtype=torch.float64, device=dev)
    e_t = torch.from_numpy(ends[nz]).to(dev)
    b_t = torch.from_numpy((ends - cnt)[nz]).to(dev)
    hi = at_end[e_t]
    lo = torch.where((b_t >= 0)[:, None], at_end[b_t.clamp(min=0)], torch.zeros_like(hi))
    sums[torch.from_numpy(np.nonzero(nz)[0]).to(dev)] = hi - lo
    cent = sums / torch.from_numpy(np.maximum(cnt, 1)).to(dev).double()[:, None]
    d = torch.empty(P.shape[0], dtype=torch.float64, device=dev)
    for s0 in range(0, P.shape[0], step):
        diff = base_t[P[s0:s0 + step]].double() - cent[lab_of[s0:s0 + step]]
        d[s0:s0 + step] = (diff * diff).sum(1)
    o1 = torch.sort(d, stable=True).indices
    o2 = torch.sort(lab_of[o1], stable=True).indices
    best = P[o1[o2]].cpu().numpy()
    starts = np.full(max(1, nl), INVALID, np.uint32)
    nz = np.nonzero(cnt)[0]
    starts[nz] = best[off[nz]]
    mean = base_t.double().mean(0)
    gd = ((base_t.double() - mean) ** 2).sum(1)
    gstart = int(torch.nonzero(gd == gd.min())[0, 0])
    return starts, gstart


def label_ground_truth(torch, base_t, ls, queries, qlabels, k=10):
    """Exact top-k among the points carrying each query's label (uint8 rows:
    integer distances, exact in the fp32 Gram form), ties to the smaller id;
    INVALID pads labels with fewer than k points."""
    from dance_amd import INVALID
    dev = base_t.device
    off, pts = ls.postings()
    out = np.full((queries.shape[0], k), INVALID, np.uint32)
    xf = base_t.float()
    xn = (xf * xf).sum(1)
    for l in np.unique(qlabels):
        qi = np.nonzero(qlabels == l)[0]
        rows = torch.from_numpy(pts[off[l]:off[l + 1]].astype(np.int64)).to(dev)
        if rows.numel() == 0:
            continue
        q = torch.from_numpy(queries[qi].astype(np.float32)).to(dev)
        d = (xn[rows][None, :] + (q * q).sum(1)[:, None] - 2.0 * (q @ xf[rows].T)).round().long()
        key = d * (1 << 21) + rows[None, :]
        kk = min(k, rows.numel())
        top = torch.topk(key, kk, dim=1, largest=False).values
        out[qi, :kk] = (top % (1 << 21)).cpu().numpy().astype(np.uint32)
    return out


def copy_calibration(torch, dev, mib):
    """One device copy of known size before the build, so that a counter run
    (FETCH_SIZE / WRITE_SIZE) can scale its readings by what the counters
    report for the copy."""
    if mib <= 0:
        return
    nbytes = mib << 20
    src = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy calibration: {nbytes} bytes read + {nbytes} bytes written")
    del src, dst


BUCKET_LS = (20, 40, 80, 160, 320, 650, 1000)  # the reference's filtered recall sweep (REPRODUCIBILITY.md:96-104)


def label_reachability(graph: np.ndarray, deg: np.ndarray, ls, qlabels: np.ndarray, query_starts: list,
                       gt: np.ndarray) -> dict:
    """Per query: the fraction of its ground-truth points reachable from its
    start points through edges between carriers of its label (the only edges
    a label-filtered search can follow). Mean over queries, and the fraction
    of queries whose whole ground truth is reachable: the recall ceiling of
    the filtered search on this graph at any L."""
    from dance_amd import INVALID
    n, R = graph.shape
    off, pts = ls.postings()
    carrier = np.zeros(n, bool)
    vis = np.zeros(n, bool)
    col = np.arange(R)[None, :]
    fr, full = [], []
    by_label = {}
    for r, l in enumerate(qlabels):
        by_label.setdefault((int(l), tuple(query_starts[r])), []).append(r)
    for (l, starts), rows in by_label.items():
        c = pts[off[l]:off[l + 1]]
        carrier[c] = True
        front = np.array([s for s in starts if s < n], np.int64)
        vis[front] = True
        touched = [front]
        while front.size:
            nb = graph[front]
            nb = nb[col < deg[front][:, None]].astype(np.int64)
            nb = nb[nb < n]
            nb = np.unique(nb[carrier[nb]])
            nb = nb[~vis[nb]]
            vis[nb] = True
            touched.append(nb)
            front = nb
        for r in rows:
            t = gt[r][gt[r] != INVALID].astype(np.int64)
            if t.size:
                hit = vis[t]
                fr.append(float(hit.mean()))
                full.append(bool(hit.all()))
        carrier[c] = False
        for t in touched:
            vis[t] = False
    return {"mean_reachable_fraction": round(float(np.mean(fr)), 4) if fr else None,
            "queries_fully_reachable": round(float(np.mean(full)), 4) if full else None}


def label_subgraph_stats(graph: np.ndarray, deg: np.ndarray, ls, labels, starts) -> dict:
    """For each label: its carriers' out-edges to other carriers (the edges a
    filtered search can follow), the carriers with none, the start's own
    count, and the share of carriers reachable from the start; means over
    the labels."""
    n, R = graph.shape
    off, pts = ls.postings()
    col = np.arange(R)[None, :]
    carrier = np.zeros(n, bool)
    vis = np.zeros(n, bool)
    out = {"in_label_out_degree": [], "carriers_without_in_label_edge": [], "start_in_label_out_degree": [],
           "carriers_reachable_from_start": []}
    for l in labels:
        c = pts[off[l]:off[l + 1]].astype(np.int64)
        carrier[c] = True
        rows = graph[c]
        live = (col < deg[c][:, None]) & (rows < n)
        nb = np.where(live, rows, 0).astype(np.int64)
        inl = (live & carrier[nb]).sum(1)
        out["in_label_out_degree"].append(float(inl.mean()))
        out["carriers_without_in_label_edge"].append(float((inl == 0).mean()))
        s0 = int(starts[l])
        out["start_in_label_out_degree"].append(float(inl[np.searchsorted(c, s0)]) if s0 in set(c.tolist()) else 0.0)
        front = np.array([s0], np.int64)
        vis[front] = True
        touched = [front]
        while front.size:
            r = graph[front]
            r = r[col < deg[front][:, None]].astype(np.int64)
            r = r[r < n]
            r = np.unique(r[carrier[r]])
            r = r[~vis[r]]
            vis[r] = True
            touched.append(r)
            front = r
        out["carriers_reachable_from_start"].append(float(vis[c].mean()))
        carrier[c] = False
        for t in touched:
            vis[t] = False
    return {k: round(float(np.mean(v)), 4) for k, v in out.items()}


def cardinality_buckets(ls, names=(("P50", 50.0), ("P1", 1.0)), per_bucket: int = 5) -> dict:
    """The reference's query buckets (tools/prepare_multilabel_workload.py:
    243-253): per percentile of the label cardinalities, the per_bucket labels
    nearest to it (ties to the smaller label)."""
    off, _ = ls.postings()
    counts = np.diff(off).astype(np.int64)
    out = {}
    for name, p in names:
        target = float(np.percentile(counts, p))
        order = sorted(range(len(counts)), key=lambda l: (abs(counts[l] - target), l))[:per_bucket]
        out[name] = {"target_cardinality": target, "labels": order, "cardinalities": [int(counts[l]) for l in order]}
    return out


def run_c5(args, mode) -> int:
    import torch
    import dance_amd as D
    from dance_amd import INVALID
    from dance_amd import filtered as F

    c = C5
    n = args.n or c["n"]
    t0 = time.time()
    base = D.synth_u8(42, 0, n, c["dim"], c["centers"], c["sigma"])
    queries = D.synth_u8(42, 1, c["nq"], c["dim"], c["centers"], c["sigma"])
    dev = torch.device("cuda:0")
    base_t = torch.from_numpy(base).to(dev)
    if mode == "c5f":
        ls = F.synth_labels(n, c["vocab"], c["min_labels"], c["max_labels"], 1.0, seed=42)
        qlab = F.zipf_labels(c["nq"], c["vocab"], 1.0, seed=43)
    else:
        part = np.random.default_rng(44).integers(0, c["parts"], n)
        ls = F.LabelSet(np.arange(n + 1, dtype=np.uint32), part.astype(np.uint32), c["parts"])
        qlab = np.random.default_rng(45).integers(0, c["parts"], c["nq"]).astype(np.uint32)
    cstarts, gstart = label_starts_gpu(torch, base_t, ls)
    # label starts: DiskANN's load-balanced rule (build_memory_index's
    # default) or, with --label-starts centroid, the carrier nearest the
    # label centroid
    starts = cstarts if args.label_starts == "centroid" else F.balanced_label_starts(ls, INVALID, seed=1)
    log(f"generated {mode} N={n} labels={ls.labels.shape[0]} in {time.time() - t0:.1f}s")
    R = c["R"] if mode == "c5f" else c["Rsmall"]
    graph_t = torch.empty((n, c["R"]), dtype=torch.int32, device=dev)
    deg_t = torch.empty((n,), dtype=torch.int32, device=dev)
    stitched = {}

    def step_filtered():
        F.filtered_build_resident(base_t.data_ptr(), D.DTYPE_U8, n, c["dim"], ls, starts, c["R"], c["L"], c["FL"],
                                  c["C"], c["STEPS"], c["alpha"], INVALID, gstart, graph_t.data_ptr(),
                                  deg_t.data_ptr())

    off_s = pts_s = None
    if mode == "c5s":
        off_s, pts_s = ls.postings()  # label -> ascending points

    def step_stitched():
        # dance_stitched_build_resident: per label, the rows are gathered, built
        # (Rsmall) and remapped to global ids on the device
        medoids = D.stitched_build_resident(base_t.data_ptr(), D.DTYPE_U8, n, c["dim"], off_s, pts_s, c["Rsmall"],
                                            c["Lsmall"], c["Cs"], c["STEPS"], c["Rstitched"], c["R"],
                                            graph_t.data_ptr(), deg_t.data_ptr())
        stitched["medoids"] = medoids
        stitched["stats"] = D.last_stitched_stats()

    step = step_filtered if mode == "c5f" else step_stitched
    copy_calibration(torch, dev, args.copy_calibration_mib)
    for i in range(args.warmup):
        step()
        log(f"warmup {i + 1}/{args.warmup} done")
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for i in range(args.steps):
        step()
        log(f"step {i + 1}/{args.steps} done")
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    ms_per_step = elapsed * 1000.0 / args.steps
    value = n / (ms_per_step / 1000.0)

    # recall@10 of label-filtered search against exact per-label ground truth
    nq = min(args.recall_queries, c["nq"])
    recall = {}
    qs = queries[:nq]
    ql = qlab[:nq]
    if nq > 0:
        t1 = time.time()
        gt = label_ground_truth(torch, base_t, ls, qs, ql)
        ent = starts[ql] if mode == "c5f" else stitched["medoids"][ql]
        # row width of the built graph: R, or the published degree when
        # DISKANN_GPU_FILTERED_PUBLISH_DEGREE ran the publish step
        Rg = int(F.last_profile()["publish_degree"]) if mode == "c5f" else c["R"]
        for Ls in (10, 20, 50, 100, 200):
            found, _ = D.search_resident(base_t.data_ptr(), D.DTYPE_U8, n, c["dim"], graph_t.data_ptr(),
                                         deg_t.data_ptr(), Rg, ent, qs, 10, Ls, ls.offsets, ls.labels, ql)
            recall[f"L{Ls}"] = round(D.recall_at_k(found, gt, 10), 4)
        log(f"recall {recall} ({time.time() - t1:.1f}s)")
    analysis = None
    if nq > 0 and args.filtered_analysis:
        # what bounds label-filtered recall on this graph: the reachable share
        # of each query's ground truth, recall with the reference's extra
        # search starts, and the reference's P50 / P1 cardinality buckets
        t1 = time.time()
        Rg = int(F.last_profile()["publish_degree"]) if mode == "c5f" else c["R"]
        g_host = graph_t.view(-1)[:n * Rg].view(n, Rg).cpu().numpy().view(np.uint32)
        d_host = deg_t.cpu().numpy().view(np.uint32)
        primary = starts if mode == "c5f" else stitched["medoids"]
        one = [[int(primary[l])] for l in ql]
        extra = F.extra_label_starts(ls, primary, 16)
        many = F.query_starts(base, qs, ql, primary, extra)
        analysis = {"label_starts": args.label_starts,
                    "reachability": {"start": label_reachability(g_host, d_host, ls, ql, one, gt),
                                     "start_and_16_extra": label_reachability(g_host, d_host, ls, ql, many, gt)}}
        rec16 = {}
        for Ls in (10, 20, 50, 100, 200):
            found, _ = D.search_resident(base_t.data_ptr(), D.DTYPE_U8, n, c["dim"], graph_t.data_ptr(),
                                         deg_t.data_ptr(), Rg, many, qs, 10, Ls, ls.offsets, ls.labels, ql)
            rec16[f"L{Ls}"] = round(D.recall_at_k(found, gt, 10), 4)
        analysis["recall@10_start_and_16_extra"] = rec16
        buckets = cardinality_buckets(ls)
        bq = queries[:args.bucket_queries]
        for name, b in buckets.items():
            bl = np.repeat(np.array(b["labels"], np.uint32), bq.shape[0])
            bqs = np.tile(bq, (len(b["labels"]), 1))
            bgt = label_ground_truth(torch, base_t, ls, bqs, bl)
            bent = [[int(primary[l])] for l in bl]
            b["queries"] = int(bqs.shape[0])
            b["recall@10"] = {}
            for Ls in BUCKET_LS:
                found, _ = D.search_resident(base_t.data_ptr(), D.DTYPE_U8, n, c["dim"], graph_t.data_ptr(),
                                             deg_t.data_ptr(), Rg, bent, bqs, 10, Ls, ls.offsets, ls.labels, bl)
                b["recall@10"][f"L{Ls}"] = round(D.recall_at_k(found, bgt, 10), 4)
            b["reachability"] = label_reachability(g_host, d_host, ls, bl, bent, bgt)
            b["subgraph"] = label_subgraph_stats(g_host, d_host, ls, b["labels"], primary)
            bmany = [F.query_starts(base, bqs[r:r + 1], bl[r:r + 1], primary, extra)[0] for r in range(bl.size)]
            b["recall@10_start_and_16_extra"] = {}
            for Ls in BUCKET_LS:
                found, _ = D.search_resident(base_t.data_ptr(), D.DTYPE_U8, n, c["dim"], graph_t.data_ptr(),
                                             deg_t.data_ptr(), Rg, bmany, bqs, 10, Ls, ls.offsets, ls.labels, bl)
                b["recall@10_start_and_16_extra"][f"L{Ls}"] = round(D.recall_at_k(found, bgt, 10), 4)
        analysis["buckets"] = buckets
        log(f"filtered analysis {json.dumps(analysis)} ({time.time() - t1:.1f}s)")

    line = {"metric": ("filtered" if mode == "c5f" else "stitched") + " Vamana build vertices/sec (1M x 192 uint8)",
            "value": round(value, 1), "unit": "vertices/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_per_step, 2), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "u8", "data": "synthetic",
            "config": {"workload": WORKLOADS[mode] + (f" (N overridden to {n})" if args.n else ""), "N": n},
            "build_seconds": round(ms_per_step / 1000.0, 3), "recall@10": recall, "filtered_analysis": analysis}
    Rg = int(F.last_profile()["publish_degree"]) if mode == "c5f" else c["R"]
    line["graph_check"] = graph_check(torch, graph_t.view(-1)[:n * Rg].view(n, Rg), deg_t, n, Rg)
    if mode == "c5f":
        kp = F.last_profile()
        st = F.last_stats()
        V = c["dim"]
        # algorithmic bytes: vector rows of the distances, adjacency rows of
        # the expansions (4 R + 4 bytes: ids and degree) and the 32-byte label
        # rows of the membership tests
        adj = 4 * c["R"] + 4
        task_b = kp["task_dist"] * V + kp["task_expansions"] * adj + kp["task_label_reads"] * 32
        row_b = ((kp["union_dist"] + kp["work_dist"] + kp["prune_dist"]) * V + kp["union_expansions"] * adj
                 + kp["union_label_reads"] * 32)
        kernels = {"k_task_search": (kp["task_search_ms"], task_b), "k_row": (kp["row_ms"], row_b),
                   "k_csr": (kp["csr_ms"], (kp["csr_dist"] + kp["csr_prune_dist"]) * V)}
        name = max(kernels, key=lambda k: kernels[k][0])
        ms, by = kernels[name]
        rounds = kp["rounds"]
        avg_ms = ms / rounds
        algo_gbs = by / (ms * 1e-3) / 1e9 if ms > 0 else 0.0  # bytes and time summed over the rounds
        line["roofline"] = {"bound": "hbm", "achieved": None, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": None,
                            "traffic": None, "kernel": name, "avg_launch_ms": round(avg_ms, 3),
                            "algorithmic_bytes_per_launch": by / rounds, "algorithmic_GBps": round(algo_gbs, 1),
                            "vector_bytes_per_launch": kp["task_dist"] * V / rounds if name == "k_task_search"
                            else None}
        traffic_file = os.path.join(ROOT, "profiles", "traffic_c5f.json")
        if os.path.exists(traffic_file) and args.n is None:
            with open(traffic_file) as f:
                tj = json.load(f)
            per = [x["read_bytes"] + x["write_bytes"] for x in tj.get("kernels", {}).get(name, [])]
            if per:
                traffic = sum(per) / len(per)
                achieved = traffic / (avg_ms * 1e-3) / 1e9
                line["roofline"].update({"achieved": round(achieved, 1), "frac": round(achieved / HBM_PEAK_GBS, 4),
                                         "traffic": traffic, "traffic_source": tj["source"],
                                         "traffic_over_algorithmic": round(traffic / (by / rounds), 3)})
        if line["roofline"]["achieved"] is None:  # no measured traffic: the algorithmic rate
            line["roofline"].update({"achieved": round(algo_gbs, 1), "frac": round(algo_gbs / HBM_PEAK_GBS, 4)})
        line["stage_ms"] = {k: round(kp[k], 2) for k in ("backbone_ms", "task_search_ms", "row_ms", "reverse_ms",
                                                        "csr_ms", "publish_ms", "diagnostics_ms", "total_ms")}
        line["config"]["published_degree"] = kp["publish_degree"]
        line["counters"] = {k: kp[k] for k in ("task_dist", "union_dist", "work_dist", "prune_dist", "csr_dist",
                                               "csr_prune_dist", "merged_candidates", "quota_dropped",
                                               "reverse_edges", "touched_rows", "long_lists", "long_max_candidates",
                                               "task_expansions", "task_label_reads", "union_expansions",
                                               "union_label_reads")}
        line["diagnostics"] = {k: st[k] for k in ("invalid_neighbor_count", "self_loop_count", "out_degree_min",
                                                  "out_degree_max", "out_degree_avg", "avg_common_label_out_degree",
                                                  "low_common_label_degree_count")}
    else:
        sst = stitched["stats"]
        line["stitched"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in sst.items()}
    print(json.dumps(line), flush=True)
    return 0


LS = (10, 20, 50, 100, 200)
GATE_TOL = 0.005  # north star: recall@10 >= CPU Vamana - 0.005 at equal R, L, alpha


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def graph_check(torch, graph_t, deg_t, n: int, R: int) -> dict:
    """Counts what no valid graph may hold: neighbour ids >= N, self loops,
    repeated neighbours in a row, non-INVALID slots past the degree."""
    from dance_amd import INVALID
    g = graph_t.long() & 0xFFFFFFFF
    d = deg_t.long()
    col = torch.arange(R, device=g.device)[None, :]
    live = col < d[:, None]
    rows = torch.arange(n, device=g.device)[:, None]
    invalid = int((live & (g >= n)).sum())
    selfl = int((live & (g == rows)).sum())
    pad = int((~live & (g != INVALID)).sum())
    srt = torch.sort(torch.where(live, g, (-col - 1).expand_as(g)), dim=1).values
    dup = int((srt[:, 1:] == srt[:, :-1]).sum())
    del g, srt, live
    out = {"invalid": invalid, "self_loops": selfl, "duplicates": dup, "bad_padding": pad,
           "min_degree": int(d.min()), "max_degree": int(d.max()), "mean_degree": round(float(d.float().mean()), 3)}
    out["ok"] = invalid == selfl == dup == pad == 0 and out["max_degree"] <= R and out["min_degree"] >= 1
    out["digest"] = graph_digest(torch, graph_t, deg_t)
    return out


def graph_digest(torch, graph_t, deg_t) -> str:
    """A 64-bit position-weighted checksum of the graph and degree arrays
    (int64 arithmetic wraps), computed on the device: equal across builds iff
    (with overwhelming likelihood) every id, slot and degree is equal."""
    def mix(x):
        x = x.reshape(-1).long() & 0xFFFFFFFF
        pos = torch.arange(x.numel(), device=x.device, dtype=torch.int64)
        w = pos * -7046029254386353131 + 1442695040888963407  # odd multiplier, wraps
        return int(((x + 1) * (w | 1)).sum())
    return f"{(mix(graph_t) * 31 + mix(deg_t)) & 0xFFFFFFFFFFFFFFFF:016x}"


def recall_curve(D, data, graph, degree, start, queries, gt) -> dict:
    """recall@10 of GPU best-first search (dance_search) over a host graph."""
    out = {}
    for Ls in LS:
        found, _ = D.search(data, graph, degree, start, queries, 10, Ls)
        out[f"L{Ls}"] = round(D.recall_at_k(found, gt, 10), 4)
    return out


def gate(gpu: dict, cpu: dict) -> dict:
    delta = {k: round(gpu[k] - cpu[k], 4) for k in gpu}
    ok = {k: gpu[k] >= cpu[k] - GATE_TOL for k in gpu}
    return {"gpu": gpu, "cpu_vamana": cpu, "delta": delta, "pass": ok, "all_pass": all(ok.values())}


def cpu_leg(torch, D, O, cfg: dict, name: str, base: np.ndarray, queries: np.ndarray, m: int, nq: int,
            with_port: bool, alpha_from: int = -1) -> dict:
    """On the first m rows of a workload: times the CPU Vamana (and the CPU
    oracle of this algorithm), builds the same rows on the GPU through the C
    ABI, checks the GPU graph against the oracle's, and scores both graphs'
    recall@10 with the same GPU search against exact ground truth. With
    alpha_from >= 0 the GPU build is also scored under the reference's alpha
    schedule knob (DANCE_ALPHA_FROM_ITER: alpha from that iteration on)."""
    sample = np.ascontiguousarray(base[:m])
    R, L, C_, S = cfg["R"], cfg["L"], cfg["C"], cfg["STEPS"]
    os.environ["DANCE_ORACLE_PROGRESS"] = "1"  # the CPU build reports each tenth of its points
    t0 = time.perf_counter()
    gc, dc, sc = O.cpu_vamana_build(sample, R, L, 1.2, 750)
    t_cpu = time.perf_counter() - t0
    log(f"{name}: CPU Vamana on {m} rows in {t_cpu:.1f}s")
    res = D.vamana_build(sample, R, L, C_, S)
    out = {"rows": m, "cpu_vamana_seconds": round(t_cpu, 2)}
    if with_port:
        t0 = time.perf_counter()
        go, do, mo = O.vnew2_build(sample, R, L, C_, S)
        t_port = time.perf_counter() - t0
        log(f"{name}: CPU oracle on {m} rows in {t_port:.1f}s")
        out["oracle_seconds"] = round(t_port, 2)
        out["gpu_graph_equals_oracle"] = bool(np.array_equal(res.graph, go) and np.array_equal(res.degree, do)
                                              and res.medoid == mo)
    q = queries[:nq]
    st = torch.from_numpy(sample).to(torch.device("cuda:0"))
    gt = ground_truth(st, sample, q)
    del st
    cpu_rec = recall_curve(D, sample, gc, dc, sc, q, gt)
    out["recall_gate"] = gate(recall_curve(D, sample, res.graph, res.degree, res.medoid, q, gt), cpu_rec)
    log(f"{name}: gate {out['recall_gate']['delta']} pass={out['recall_gate']['all_pass']}")
    if alpha_from >= 0:
        os.environ["DANCE_ALPHA_FROM_ITER"] = str(alpha_from)
        try:
            ra = D.vamana_build(sample, R, L, C_, S)
        finally:
            del os.environ["DANCE_ALPHA_FROM_ITER"]
        g2 = gate(recall_curve(D, sample, ra.graph, ra.degree, ra.medoid, q, gt), cpu_rec)
        g2["schedule"] = f"alpha from iteration {alpha_from} (reference knob USE_ALPHA_FROM_FIRST_ITER / " \
                         "VAMANA_ALPHA_FINAL_FROM_ITER)"
        g2["gpu_build_seconds"] = round(ra.stats["gpu_build_seconds"], 3)
        out["recall_gate_alpha_schedule"] = g2
        log(f"{name}: gate with alpha from {alpha_from}: {g2['delta']} pass={g2['all_pass']}")
    return out


def parse_settings(text: str, C_: int, S: int) -> list:
    """'iters:alpha_from[:C[:STEPS]],...' -> [(iters, alpha_from or None, C,
    STEPS)]; alpha_from -1 (or empty) is the reference default, alpha in the
    last iteration; C and STEPS default to the workload's."""
    out = []
    for item in text.split(","):
        f = [x.strip() for x in item.strip().split(":")]
        a = int(f[1]) if len(f) > 1 and f[1] else -1
        c = int(f[2]) if len(f) > 2 and f[2] else C_
        st = int(f[3]) if len(f) > 3 and f[3] else S
        out.append((int(f[0]), None if a < 0 else a, c, st))
    return out


def run_gate(args) -> int:
    """bench.py --gate: score_gate on the workload of --config, one summary
    line on stdout."""
    rec = score_gate(args)
    print(json.dumps({"gate": args.config, "cpu_mean": rec["cpu_vamana"]["recall_mean"],
                      "spread": rec["cpu_vamana"]["recall_spread"],
                      "gpu": [(e["iters"], e["alpha_from"], e["C"], e["STEPS"], e["build_seconds"], e.get("all_pass"))
                              for e in rec["gpu"]]}), flush=True)
    return 0


def score_gate(args) -> dict:
    """The recall gate of the north star on a whole workload: recall@10 of the
    GPU graph >= the CPU Vamana's - 0.005 at equal R, L and alpha, both graphs
    scored by the same GPU search (dance_search_resident) against exact ground
    truth at L in LS. The GPU graph is built under each (iterations, alpha
    from) setting (the reference's VAMANA_ITERS and USE_ALPHA_FROM_FIRST_ITER /
    VAMANA_ALPHA_FINAL_FROM_ITER, here DANCE_VAMANA_ITERS and
    DANCE_ALPHA_FROM_ITER) and timed (warm, vectors resident). The CPU Vamana
    (oracle/cpu_baselines.cpp, every host thread) runs --gate-cpu-runs times,
    each timed; its insertion order depends on thread timing, so the record
    holds every run's recall, their mean and spread, and each setting passes
    per L against the mean. Writes the record to --gate-out (when set) after
    the GPU settings and after every CPU run, and returns it."""
    import torch
    import dance_amd as D
    from oracle import oracle as O  # the CPU comparator of the gate

    cfg = dict(D.CONFIGS[args.config])
    # The gate resolves recall differences of 0.005, so it scores
    # --gate-queries queries of the workload's query distribution even where
    # the workload itself has fewer (c1: 1k; the first 1k are the workload's).
    cfg["nq"] = max(cfg["nq"], args.gate_queries)
    n = args.n or cfg["n"]
    R, L, C_, S = cfg["R"], cfg["L"], cfg["C"], cfg["STEPS"]
    t0 = time.time()
    base, queries = D.make_workload(cfg, n=n)
    nq = min(args.gate_queries, queries.shape[0])
    q = queries[:nq]
    dev = torch.device("cuda:0")
    base_t = torch.from_numpy(base).to(dev)
    dcode = D.DTYPE_F32 if base.dtype == np.float32 else D.DTYPE_U8
    gt = ground_truth(base_t, base, q)
    log(f"gate {args.config}: N={n} queries={nq} workload and ground truth in {time.time() - t0:.1f}s")
    graph_t = torch.empty((n, R), dtype=torch.int32, device=dev)
    deg_t = torch.empty((n,), dtype=torch.int32, device=dev)

    def score(start) -> dict:
        out = {}
        for Ls in LS:
            found, _ = D.search_resident(base_t.data_ptr(), dcode, n, cfg["dim"], graph_t.data_ptr(),
                                         deg_t.data_ptr(), R, start, q, 10, Ls)
            out[f"L{Ls}"] = round(D.recall_at_k(found, gt, 10), 4)
        return out

    def set_env(iters, alpha_from):
        os.environ["DANCE_VAMANA_ITERS"] = str(iters)
        if alpha_from is None:
            os.environ.pop("DANCE_ALPHA_FROM_ITER", None)
        else:
            os.environ["DANCE_ALPHA_FROM_ITER"] = str(alpha_from)

    def build(c, st):
        D.vamana_build_resident(base_t.data_ptr(), dcode, n, cfg["dim"], R, L, c, st, graph_t.data_ptr(),
                                deg_t.data_ptr())

    settings = parse_settings(args.gate_settings, C_, S)
    gpu = []
    for k, (iters, af, c, st) in enumerate(settings):
        set_env(iters, af)
        if k == 0:
            build(c, st)  # untimed: loads the code objects
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        build(c, st)
        torch.cuda.synchronize()
        secs = time.perf_counter() - t1
        medoid = int(D.lib().gpu_vamana_vnew2_get_last_medoid())
        check = graph_check(torch, graph_t, deg_t, n, R)
        rec = score(medoid)
        e = {"iters": iters, "alpha_from": iters - 1 if af is None else af, "C": c, "STEPS": st,
             "reference_default": iters == 4 and af in (None, 3) and (c, st) == (C_, S), "build_seconds": round(secs, 3), "vertices_per_s": round(n / secs, 1), "digest": check["digest"],
             "graph_ok": check["ok"], "mean_degree": check["mean_degree"], "recall": rec}
        if n <= args.gate_oracle_max:
            og, od, om = O.vnew2_build(base, R, L, c, st, iters=iters, alpha_from=af)
            e["graph_equals_oracle"] = bool(om == medoid and np.array_equal(od, deg_t.cpu().numpy().view(np.uint32))
                                            and np.array_equal(og, graph_t.cpu().numpy().view(np.uint32)))
        gpu.append(e)
        log(f"gate {args.config}: GPU iters={iters} alpha_from={e['alpha_from']} C={c} STEPS={st} {secs:.3f}s "
            f"{rec}")
    os.environ.pop("DANCE_VAMANA_ITERS", None)
    os.environ.pop("DANCE_ALPHA_FROM_ITER", None)

    keys = [f"L{Ls}" for Ls in LS]
    runs, alt_runs = [], []

    def record() -> dict:
        """The gate record so far (rewritten after every CPU run, so a run
        cut short still leaves the finished parts)."""
        cpu_mean = spread = None
        if runs:
            cpu_mean = {k: round(float(np.mean([x["recall"][k] for x in runs])), 4) for k in keys}
            spread = {k: round(float(max(x["recall"][k] for x in runs) - min(x["recall"][k] for x in runs)), 4)
                      for k in keys}
            for e in gpu:
                e["delta_vs_cpu_mean"] = {k: round(e["recall"][k] - cpu_mean[k], 4) for k in keys}
                e["pass"] = {k: e["recall"][k] >= cpu_mean[k] - GATE_TOL for k in keys}
                e["all_pass"] = all(e["pass"].values())
                e["passes_every_cpu_run"] = all(e["recall"][k] >= x["recall"][k] - GATE_TOL
                                                for x in runs for k in keys)
        alt_mean = ({k: round(float(np.mean([x["recall"][k] for x in alt_runs])), 4) for k in keys}
                    if alt_runs else None)
        if alt_mean:
            for e in gpu:
                e["delta_vs_alt_pool_mean"] = {k: round(e["recall"][k] - alt_mean[k], 4) for k in keys}
        passing = [e for e in gpu if e.get("all_pass")]
        best = min(passing, key=lambda e: e["build_seconds"]) if passing else None
        rec = {"config": args.config,
               "workload": WORKLOADS[args.config] + (f" (N overridden to {n})" if args.n else ""),
               "N": n, "queries": nq, "tolerance": GATE_TOL,
               "rule": "GPU recall@10 >= mean CPU Vamana recall@10 - tolerance at every L; same GPU search, "
                       "exact ground truth (GPU fp32 shortlist, fp64 re-rank)",
               "cpu_vamana": {"what": "DiskANN's in-memory Vamana build restated in C++/OpenMP "
                                      "(oracle/cpu_baselines.cpp), R/L/alpha of the workload, maxc 750; Microsoft "
                                      "DiskANN is not available offline",
                              "pool": args.gate_cpu_pool,
                              "pools": {"diskann": "RobustPrune over the search's expanded points "
                                                   "(DiskANN's search_for_point_and_prune)",
                                        "paper": "RobustPrune over the expanded points and the point's current "
                                                 "neighbours (Alg. 2 of the DiskANN paper)"},
                              "threads": O.num_threads(), "cpu_model": cpu_model(), "runs": runs,
                              "recall_mean": cpu_mean, "recall_spread": spread,
                              "alt_pool_runs": alt_runs, "alt_pool_recall_mean": alt_mean},
               "gpu": gpu,
               "cheapest_passing": ({k: best[k] for k in ("iters", "alpha_from", "C", "STEPS", "build_seconds")}
                                    if best else None),
               "command": "python bench.py " + " ".join(sys.argv[1:]),
               "date": time.strftime("%Y-%m-%d %H:%M:%S")}
        if args.gate_out:
            os.makedirs(os.path.dirname(os.path.abspath(args.gate_out)), exist_ok=True)
            with open(args.gate_out, "w") as f:
                json.dump(rec, f, indent=1)
        return rec

    record()
    os.environ["DANCE_ORACLE_PROGRESS"] = "1"
    plan = [args.gate_cpu_pool] * args.gate_cpu_runs + [args.gate_cpu_alt_pool] * args.gate_cpu_alt_runs
    for r, pool in enumerate(plan):
        t1 = time.perf_counter()
        gc, dc, sc = O.cpu_vamana_build(base, R, L, 1.2, 750, pool=pool)
        secs = time.perf_counter() - t1
        graph_t.copy_(torch.from_numpy(gc.view(np.int32)))
        deg_t.copy_(torch.from_numpy(dc.view(np.int32)))
        rec = score(sc)
        (runs if pool == args.gate_cpu_pool else alt_runs).append(
            {"pool": pool, "seconds": round(secs, 2), "vertices_per_s": round(n / secs, 1),
             "mean_degree": round(float(dc.mean()), 3), "recall": rec})
        log(f"gate {args.config}: CPU Vamana ({pool} pool) run {r + 1} {secs:.1f}s {rec}")
        del gc, dc
        record()
    del base_t, graph_t, deg_t
    torch.cuda.empty_cache()
    return record()


def recorded_gate(config: str):
    """The committed whole-workload gate record of a config (bench.py --gate
    on the GPU box, copied to profiles/), or None."""
    path = os.path.join(ROOT, "profiles", f"recall_gate_{config}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)


def compact_gate(rec: dict, source: str | None = None) -> dict:
    """The parts of a gate record the bench line carries."""
    cv = rec["cpu_vamana"]
    out = {"N": rec["N"], "queries": rec["queries"], "tolerance": rec["tolerance"],
           "cpu_vamana": {"pool": cv.get("pool"), "threads": cv["threads"], "cpu_model": cv["cpu_model"],
                          "seconds": [r["seconds"] for r in cv["runs"]], "recall_mean": cv["recall_mean"],
                          "recall_spread": cv["recall_spread"], "alt_pool_recall_mean": cv.get("alt_pool_recall_mean")},
           "gpu": [{k: e.get(k) for k in ("iters", "alpha_from", "C", "STEPS", "build_seconds", "digest", "recall",
                                          "delta_vs_cpu_mean", "all_pass")} for e in rec["gpu"]],
           "cheapest_passing": rec.get("cheapest_passing"), "command": rec["command"], "date": rec["date"]}
    if source:
        out["source"] = source
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1)
    ap.add_argument("--warmup", type=int, default=1,
                    help="untimed builds first (the first also loads the code objects)")
    ap.add_argument("--config", default="c3", choices=sorted(WORKLOADS))
    ap.add_argument("--n", type=int, default=None, help="override N (parity/debug runs)")
    ap.add_argument("--recall-queries", type=int, default=1000)
    ap.add_argument("--cpu-sample", type=int, default=200_000,
                    help="rows of the workload in the CPU baseline sample (CPU Vamana and the CPU oracle, timed "
                         "on this host's cores; the recall gate is scored on it); 0 disables the CPU legs")
    ap.add_argument("--port-max", type=int, default=200_000,
                    help="largest sample on which the CPU oracle of this algorithm is also timed")
    ap.add_argument("--gate-c1", type=int, default=1, help="also score the recall gate on c1 (100k, CPU Vamana)")
    ap.add_argument("--gate-alpha-from", type=int, default=0,
                    help="also score the gates with alpha from this iteration on (the reference's "
                         "USE_ALPHA_FROM_FIRST_ITER at 0); -1 disables")
    ap.add_argument("--abi", type=int, default=1,
                    help="also time one build through the host-buffer C ABI (H2D and D2H included)")
    ap.add_argument("--profile", default="QUALITY")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="run one device copy of this size first (HBM counter calibration)")
    ap.add_argument("--label-starts", default="balanced", choices=("balanced", "centroid"),
                    help="c5 label entry points: DiskANN's load-balanced rule or the carrier nearest the centroid")
    ap.add_argument("--filtered-analysis", type=int, default=1,
                    help="c5: reachability, extra-start recall and the P50 / P1 cardinality buckets")
    ap.add_argument("--bucket-queries", type=int, default=200, help="c5: queries per bucket label")
    ap.add_argument("--gate", action="store_true",
                    help="score the recall gate on the whole workload instead of the bench line (run_gate)")
    ap.add_argument("--gate-settings", default="4:-1,5:-1,6:-1,4:0,5:0,6:0",
                    help="GPU settings iterations:alpha_from[:C[:STEPS]] (alpha_from -1 = the last iteration, the "
                         "reference default; C and STEPS default to the workload's)")
    ap.add_argument("--gate-cpu-runs", type=int, default=1, help="timed CPU Vamana runs (the gate's comparator)")
    ap.add_argument("--gate-cpu-pool", default="diskann", choices=("diskann", "paper"),
                    help="the comparator's RobustPrune candidates: the expanded points (DiskANN's code) or those "
                         "plus the point's current neighbours (the paper's Alg. 2)")
    ap.add_argument("--gate-cpu-alt-pool", default="paper", choices=("diskann", "paper"))
    ap.add_argument("--gate-cpu-alt-runs", type=int, default=0, help="CPU Vamana runs with the other pool, reported")
    ap.add_argument("--gate-queries", type=int, default=10_000)
    ap.add_argument("--gate-oracle-max", type=int, default=0,
                    help="largest N at which each GPU graph is also compared with the CPU oracle's")
    ap.add_argument("--gate-out", default="", help="JSON record of the gate")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build targets one GPU; sharding over several GPUs is a design only, "
              "so --gpus must be 1.", file=sys.stderr)
        return 2

    if args.config in ("c5f", "c5s"):
        return run_c5(args, args.config)
    if args.gate:
        return run_gate(args)

    import torch
    import dance_amd as D

    D.set_profile(args.profile)
    cfg = dict(D.CONFIGS[args.config])
    n = args.n or cfg["n"]
    R = cfg["R"]
    t0 = time.time()
    base, queries = D.make_workload(cfg, n=n)
    log(f"generated {args.config} N={n} dim={cfg['dim']} in {time.time() - t0:.1f}s")
    dev = torch.device("cuda:0")
    base_t = torch.from_numpy(base).to(dev)
    graph_t = torch.empty((n, R), dtype=torch.int32, device=dev)
    deg_t = torch.empty((n,), dtype=torch.int32, device=dev)
    dcode = D.DTYPE_F32 if base.dtype == np.float32 else D.DTYPE_U8
    torch.cuda.synchronize()

    def step():
        D.vamana_build_resident(base_t.data_ptr(), dcode, n, cfg["dim"], R, cfg["L"], cfg["C"],
                                cfg["STEPS"], graph_t.data_ptr(), deg_t.data_ptr())

    copy_calibration(torch, dev, args.copy_calibration_mib)
    for i in range(args.warmup):
        step()
        log(f"warmup {i + 1}/{args.warmup} done")
    torch.cuda.synchronize()
    profs = []
    t_start = time.perf_counter()
    for i in range(args.steps):
        step()
        profs.append(D.last_kernel_profile())
        log(f"step {i + 1}/{args.steps} done")
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    ms_per_step = elapsed * 1000.0 / args.steps
    value = n / (ms_per_step / 1000.0)
    kp = profs[-1]
    medoid = int(D.lib().gpu_vamana_vnew2_get_last_medoid())
    check = graph_check(torch, graph_t, deg_t, n, R)
    log(f"graph check {check}")

    # Roofline of the dominant kernel (search + online insert): measured HBM
    # bytes per launch (committed counter profile of the same workload) over
    # the live mean launch time; the device-counted algorithmic bytes are
    # reported beside it, with their ratio to the measured bytes.
    launches = kp["iterations"]
    avg_ms = kp["search_ms"] / launches
    algo = kp["search_bytes"] / launches
    roofline = {"bound": "hbm", "achieved": None, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": None,
                "traffic": None, "kernel": "k_search (search + online robust insert)",
                "avg_launch_ms": round(avg_ms, 3), "launches": launches,
                "algorithmic_bytes_per_launch": algo,
                "algorithmic_GBps": round(algo / (avg_ms * 1e-3) / 1e9, 1),
                "algorithmic_frac": round(algo / (avg_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "algorithmic_note": "cache-inclusive demand: every distance counts its whole row, every expansion "
                                    "its adjacency row; L2 and the MALL serve the part above 1"}
    traffic_file = os.path.join(ROOT, "profiles", f"traffic_{args.config}.json")
    if os.path.exists(traffic_file) and args.n is None and args.profile == "QUALITY":
        with open(traffic_file) as f:
            tj = json.load(f)
        per = [l["read_bytes"] + l["write_bytes"] for l in tj["search_launches"]]
        traffic = sum(per) / len(per)
        achieved = traffic / (avg_ms * 1e-3) / 1e9
        roofline.update({"achieved": round(achieved, 1), "frac": round(achieved / HBM_PEAK_GBS, 4),
                         "traffic": traffic, "traffic_source": tj["source"],
                         "traffic_measured": tj.get("measured"), "traffic_graph_digest": tj.get("graph_digest"),
                         "traffic_graph_is_this_graph": tj.get("graph_digest") == check["digest"],
                         "traffic_note": "fabric traffic (FETCH_SIZE + WRITE_SIZE, calibrated on a device copy) of a "
                                         "committed counter run: Infinity Cache hits included, so an upper bound on "
                                         "HBM bytes",
                         "algorithmic_over_traffic": round(algo / traffic, 3)})
    else:
        tj = None

    # Every search and prune launch on its own: live HIP-event time, the
    # device-counted algorithmic bytes, and (with a committed counter profile
    # of this workload) the measured HBM bytes, each as a rate and a fraction
    # of the HBM peak.
    def per_launch(stage, ms, algo_b, prof):
        out = []
        for i, (t, b) in enumerate(zip(ms, algo_b)):
            e = {"iteration": i, "ms": round(t, 2), "algorithmic_GB": round(b / 1e9, 2),
                 "algorithmic_frac": round(b / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)}
            if prof and i < len(prof):
                mb = prof[i]["read_bytes"] + prof[i]["write_bytes"]
                e.update({"measured_GB": round(mb / 1e9, 2),
                          "measured_frac": round(mb / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)})
            out.append(e)
        return out
    kernels = {"search": per_launch("search", kp["search_iter_ms"], kp["search_bytes_iter"],
                                    tj["search_launches"] if tj else None),
               "prune": per_launch("prune", kp["prune_iter_ms"], kp["prune_bytes_iter"],
                                   tj.get("prune_launches") if tj else None)}

    # Recall@10 of the resident graph on a query subset.
    nq = min(args.recall_queries, queries.shape[0])
    recall = {}
    if nq > 0:
        t0 = time.time()
        gt = ground_truth(base_t, base, queries[:nq])
        for Ls in LS:
            found, _ = D.search_resident(base_t.data_ptr(), dcode, n, cfg["dim"], graph_t.data_ptr(),
                                         deg_t.data_ptr(), R, medoid, queries[:nq], 10, Ls)
            recall[f"L{Ls}"] = round(D.recall_at_k(found, gt, 10), 4)
        log(f"recall {recall} ({time.time() - t0:.1f}s)")

    # The same build through the host-buffer C ABI (gpu_vamana_vnew2_build*),
    # whose time includes the H2D and D2H copies, as the reference's
    # gpu_build_seconds does (vnew2.cu:2174, 2838).
    abi = None
    if args.abi:
        t0 = time.perf_counter()
        res = D.vamana_build(base, R, cfg["L"], cfg["C"], cfg["STEPS"])
        wall = time.perf_counter() - t0
        st = res.stats
        same = bool(np.array_equal(res.degree, deg_t.cpu().numpy().view(np.uint32))
                    and np.array_equal(res.graph, graph_t.cpu().numpy().view(np.uint32)))
        abi = {"seconds": round(wall, 3), "gpu_build_seconds": round(st["gpu_build_seconds"], 3),
               "h2d_seconds": round(st["h2d_seconds"], 3), "d2h_seconds": round(st["d2h_seconds"], 3),
               "vertices_per_s": round(n / wall, 1), "graph_equals_resident": same}
        del res
        log(f"abi {abi}")

    cpu = None
    gates = {}
    if args.cpu_sample > 0:
        from oracle import oracle as O  # the CPU baseline legs only
        m = min(args.cpu_sample, n)
        leg = cpu_leg(torch, D, O, cfg, args.config, base, queries, m, nq or 1000, with_port=m <= args.port_max,
                      alpha_from=args.gate_alpha_from)
        port = None
        if "oracle_seconds" in leg:
            port = {"value": round(m / leg["oracle_seconds"], 1), "seconds": leg["oracle_seconds"],
                    "what": "CPU oracle of this build's algorithm (oracle/vamana_oracle.cpp), same sample, same cores",
                    "gpu_graph_equals_oracle": leg["gpu_graph_equals_oracle"]}
        cpu = {"value": round(m / leg["cpu_vamana_seconds"], 1), "unit": "vertices/s", "cores": O.num_threads(),
               "kind": "port", "cpu_model": cpu_model(),
               "sample": (f"first {m} rows of the {args.config} workload; DiskANN's in-memory Vamana build "
                          f"(R{R} L{cfg['L']} alpha 1.2, maxc 750) restated in C++/OpenMP "
                          "(oracle/cpu_baselines.cpp); Microsoft DiskANN itself is not available offline"),
               "seconds": leg["cpu_vamana_seconds"], "oracle_port": port}
        gates[f"{args.config}_first_{m}"] = leg["recall_gate"]
        if "recall_gate_alpha_schedule" in leg:
            gates[f"{args.config}_first_{m}_alpha_from_{args.gate_alpha_from}"] = leg["recall_gate_alpha_schedule"]
        if args.gate_c1 and args.config != "c1":
            # the whole c1 workload, live: the default schedule, 5 iterations
            # and alpha from iteration 0, against three CPU Vamana runs (one
            # run alone is within the gate's width of noise), 10k queries
            g1 = score_gate(argparse.Namespace(config="c1", n=None, gate_queries=10_000, gate_settings="4:-1,5:-1,4:0",
                                               gate_oracle_max=0, gate_cpu_pool="diskann", gate_cpu_alt_pool="paper",
                                               gate_cpu_runs=3, gate_cpu_alt_runs=0, gate_out=""))
            gates["c1 (live)"] = compact_gate(g1)
        full = recorded_gate(args.config)
        if full and cpu is not None:
            rs = full["cpu_vamana"]["runs"]
            secs = float(np.mean([r["seconds"] for r in rs]))
            cpu["full_n"] = {"value": round(full["N"] / secs, 1), "seconds": round(secs, 2), "runs": len(rs),
                             "cores": full["cpu_vamana"]["threads"], "N": full["N"],
                             "source": f"profiles/recall_gate_{args.config}.json (recorded {full['date']})"}
    for c in ("c1", "c2", "c3"):
        rec = recorded_gate(c)
        if rec:
            gates[f"{c} (recorded)"] = compact_gate(rec, f"profiles/recall_gate_{c}.json")

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "vertices/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 2), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        # float rows are stored and differenced in binary16 under the fp16 profiles
        "dtype": ("f16" if args.profile in FP16_PROFILES else "f32") if dcode == D.DTYPE_F32 else "u8",
        "data": "synthetic",
        "config": {"workload": WORKLOADS[args.config] + (f" (N overridden to {n})" if args.n else ""),
                   "N": n, "dim": cfg["dim"], "R": R, "L": cfg["L"], "C": cfg["C"], "STEPS": cfg["STEPS"],
                   "alpha": 1.2, "profile": args.profile},
        "build_seconds": round(ms_per_step / 1000.0, 3),
        "graph_check": check,
        "recall@10": recall,
        "recall_gate": gates or None,
        "abi": abi,
        "stage_ms": {k: round(kp[k], 2) for k in ("medoid_ms", "init_ms", "search_ms", "reverse_ms", "merge_ms",
                                                     "prune_ms", "total_ms")},
        "launch_ms": {"search": [round(v, 2) for v in kp["search_iter_ms"]],
                      "prune": [round(v, 2) for v in kp["prune_iter_ms"]]},
        "launch_counters": {k: list(kp[k]) for k in (
            "search_dist_iter", "insert_dist_iter", "expansions_iter", "bound_checks_iter", "bound_skips_iter",
            "merge_dist_iter", "prune_dist_iter", "prune_bound_checks_iter", "prune_bound_skips_iter",
            "insert_bound_checks_iter", "insert_bound_skips_iter")},
        "launch_algorithmic_GB": {"search": [round(v / 1e9, 2) for v in kp["search_bytes_iter"]],
                                  "prune": [round(v / 1e9, 2) for v in kp["prune_bytes_iter"]]},
        "kernels": kernels,
        "prune_rounds": {"rounds": kp["prune_rounds"], "exact_rounds": kp["prune_exact_rounds"]},
        "prune_cycles": ({k: kp[k] for k in ("cyc_prune_rank", "cyc_prune_gram", "cyc_prune_rounds",
                                             "cyc_prune_fill")} if kp["cyc_prune_rounds"] else None),
        "counters": {k: kp[k] for k in ("search_dist", "insert_dist", "expansions", "vis_skips", "merge_dist",
                                        "prune_dist", "reverse_edges", "bound_checks", "bound_skips",
                                        "prune_bound_checks", "prune_bound_skips", "insert_bound_checks",
                                        "insert_bound_skips")},
        "search_cycles": ({k: kp[k] for k in ("cyc_select", "cyc_insert", "cyc_dist", "cyc_pool", "cyc_seed",
                                              "cyc_total")} if kp["cyc_total"] else None),
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0 if check["ok"] else 1


if __name__ == "__main__":
    sys.exit(main())
