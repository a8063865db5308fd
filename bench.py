"""Benchmark: standard GPU Vamana build throughput on one MI355X.

A step is one full build (medoid, init, 4 x (search + online insert, reverse
merge, prune)) of the configured synthetic workload, with the vectors already
resident in HBM. value = vertices/s = N / seconds per build.

Prints ONE JSON line. Also reports recall@10 of the built graph (beam search
against exact ground truth on a query subset), the HBM roofline of the
dominant kernel (search + online insert; algorithmic bytes counted on device,
duration from HIP events on the build stream) and the CPU baseline (the CPU
oracle of the same algorithm on a bounded sample, on this host's cores).
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

HBM_PEAK_GBS = 8000.0
WORKLOADS = {
    "c1": "c1: 100k x 96 fp32 N(0,I) L2-normalized, seed 42; R64 L100 C80 STEPS64 alpha1.2",
    "c2": "c2: 1M x 96 fp32 256-center Gaussian mixture sigma 0.3 L2-normalized, seed 42; R64 L100 C80 STEPS64 alpha1.2",
    "c3": "c3: 10M x 96 fp32 256-center Gaussian mixture sigma 0.3 L2-normalized, seed 42; R64 L100 C80 STEPS64 alpha1.2",
    "c4": "c4: 10M x 128 uint8 clip(round(64+24z)) 1024-center mixture, seed 42; R64 L100 C80 STEPS64 alpha1.2",
}
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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1)
    ap.add_argument("--warmup", type=int, default=0)
    ap.add_argument("--config", default="c3", choices=sorted(WORKLOADS))
    ap.add_argument("--n", type=int, default=None, help="override N (parity/debug runs)")
    ap.add_argument("--recall-queries", type=int, default=1000)
    ap.add_argument("--cpu-sample", type=int, default=50_000, help="0 disables the CPU baseline")
    ap.add_argument("--profile", default="QUALITY")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="run one device copy of this size first (HBM counter calibration)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build targets one GPU; multi-GPU sharding is design-only "
              "(see DESIGN.md), so --gpus must be 1.", file=sys.stderr)
        return 2

    import torch
    import dance_amd as D

    D.set_profile(args.profile)
    cfg = dict(D.CONFIGS[args.config])
    n = args.n or cfg["n"]
    t0 = time.time()
    base, queries = D.make_workload(cfg, n=n)
    log(f"generated {args.config} N={n} dim={cfg['dim']} in {time.time() - t0:.1f}s")
    dev = torch.device("cuda:0")
    base_t = torch.from_numpy(base).to(dev)
    graph_t = torch.empty((n, cfg["R"]), dtype=torch.int32, device=dev)
    deg_t = torch.empty((n,), dtype=torch.int32, device=dev)
    dcode = D.DTYPE_F32 if base.dtype == np.float32 else D.DTYPE_U8
    torch.cuda.synchronize()

    def step():
        D.vamana_build_resident(base_t.data_ptr(), dcode, n, cfg["dim"], cfg["R"], cfg["L"], cfg["C"],
                                cfg["STEPS"], graph_t.data_ptr(), deg_t.data_ptr())

    if args.copy_calibration_mib > 0:
        nbytes = args.copy_calibration_mib << 20
        src = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: {nbytes} bytes read + {nbytes} bytes written")
        del src, dst
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
    stats = D.last_stats()

    # Roofline of the dominant kernel: search + online insert.
    search_launches = kp["iterations"]
    avg_ms = kp["search_ms"] / search_launches
    bytes_per_launch = kp["search_bytes"] / search_launches
    achieved = bytes_per_launch / (avg_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "k_search (search + online robust insert)",
                "avg_launch_ms": round(avg_ms, 3), "algorithmic_bytes_per_launch": bytes_per_launch}
    traffic_file = os.path.join(ROOT, "profiles", f"traffic_{args.config}.json")
    if os.path.exists(traffic_file) and args.n is None:
        with open(traffic_file) as f:
            roofline["traffic"] = json.load(f).get("search_hbm_bytes_per_launch")

    # Recall@10 on a query subset.
    from oracle import oracle as O
    nq = min(args.recall_queries, queries.shape[0])
    recall = {}
    if nq > 0:
        t0 = time.time()
        gt = ground_truth(base_t, base, queries[:nq])
        graph = graph_t.cpu().numpy().view(np.uint32)
        deg = deg_t.cpu().numpy().view(np.uint32)
        medoid = int(D.lib().gpu_vamana_vnew2_get_last_medoid())
        for Ls in (10, 20, 50, 100, 200):
            found = O.beam_search(base, graph, deg, medoid, queries[:nq], 10, Ls)
            recall[f"L{Ls}"] = round(O.recall_at_k(found, gt, 10), 4)
        log(f"recall {recall} ({time.time() - t0:.1f}s)")

    cpu = None
    if args.cpu_sample > 0:
        m = min(args.cpu_sample, n)
        sample = np.ascontiguousarray(base[:m])
        t0 = time.perf_counter()
        O.vnew2_build(sample, cfg["R"], cfg["L"], cfg["C"], cfg["STEPS"])
        dt = time.perf_counter() - t0
        cpu = {"value": round(m / dt, 1), "unit": "vertices/s", "cores": O.num_threads(), "kind": "port",
               "sample": f"first {m} vectors of the same workload, full vnew2 build (CPU oracle, OpenMP)",
               "seconds": round(dt, 2)}
        log(f"cpu baseline {cpu}")

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "vertices/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 2), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32" if dcode == D.DTYPE_F32 else "u8",
        "data": "synthetic",
        "config": {"workload": WORKLOADS[args.config] + (f" (N overridden to {n})" if args.n else ""),
                   "N": n, "dim": cfg["dim"], "R": cfg["R"], "L": cfg["L"], "C": cfg["C"], "STEPS": cfg["STEPS"],
                   "alpha": 1.2, "profile": args.profile},
        "build_seconds": round(ms_per_step / 1000.0, 3),
        "recall@10": recall,
        "stage_ms": {k: round(kp[k], 2) for k in ("medoid_ms", "init_ms", "search_ms", "reverse_ms", "merge_ms",
                                                     "prune_ms", "total_ms")},
        "counters": {k: kp[k] for k in ("search_dist", "insert_dist", "expansions", "vis_skips", "merge_dist",
                                        "prune_dist", "reverse_edges")},
        "search_cycles": ({k: kp[k] for k in ("cyc_select", "cyc_insert", "cyc_dist", "cyc_pool", "cyc_seed",
                                              "cyc_total")} if kp["cyc_total"] else None),
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
