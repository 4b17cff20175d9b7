#!/usr/bin/env python3
"""bench.py — JHQ IVF search throughput on one MI355X.

Workload ("config 2"): N=1,000,000 base and 10,000
query vectors, D=1024 fp32, drawn from a seeded 10,000-component Gaussian
mixture (per-component N(0, I) mean, diagonal std log-uniform in [0.1, 1],
uniform weights) and L2-normalised.  IVF nlist=4096 trained on the first
100,000 base vectors (the reference demo's protocol), M=128, B=8, Br=4,
alpha=4, k=10, query batch 64.  Ground truth is exact L2 brute force.

A "step" is one batch of 64 queries through the whole search path (rotate,
centroid scores, probe selection, byte LUT, ADC scan + top-ck, refine +
final top-k) with queries and results resident in device memory.  The nprobe
sweep {16, 32, 64} picks the fastest setting with recall@10 >= 0.95; `value`
is that setting's queries/s over exactly --steps timed steps.

Also reported: per-kernel HIP-event times, the ADC scan's HBM roofline
fraction, the reference's host-to-host QPS protocol, and the CPU baseline
(the oracle's scalar search, one query at a time, on the same GPU-built
index, timed on this host's cores).
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "QPS@recall@10>=0.95 (1Mx1024 IVF, batch 64); ADC-scan HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=0, help="timed steps (default: 5 passes)")
    ap.add_argument("--warmup", type=int, default=0, help="warmup steps (default: 1 pass)")
    ap.add_argument("--nprobe", type=str, default="16,32,64")
    ap.add_argument("--alpha", type=str, default="4,10",
                    help="short-list factors swept (ck = max(k, ceil(alpha*k)))")
    ap.add_argument("--scale", type=float, default=1.0, help="fraction of N (debug only)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--profile-batches", type=int, default=0,
                    help="profiling mode: build the index, run this many search batches at the "
                         "first --nprobe/--alpha plus one 256 MiB device copy (the counter "
                         "calibration kernel), print per-step times and exit")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=0x4A48510002)
    return ap.parse_args()


def gen_mixture(torch, dev, n, d, ncomp, seed, means=None, scales=None, chunk=100_000):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    if means is None:
        means = torch.randn(ncomp, d, device=dev, generator=g)
        scales = torch.exp(torch.empty(ncomp, d, device=dev).uniform_(math.log(0.1), 0.0,
                                                                     generator=g))
    out = torch.empty(n, d, device=dev)
    for i in range(0, n, chunk):
        m = min(chunk, n - i)
        c = torch.randint(0, ncomp, (m,), device=dev, generator=g)
        x = means[c] + scales[c] * torch.randn(m, d, device=dev, generator=g)
        out[i:i + m] = x / x.norm(dim=1, keepdim=True)
    return out, means, scales


def ground_truth(torch, base, q, k=10, width=100, short=200, chunk=256):
    """Exact L2 neighbours: an fp32 GEMM short list of `short`, re-ranked in
    float64.  Returns the top-`width` ids (the reference's GT files are 100
    wide, scripts/preprocess.py:231); column order is exact distance order."""
    bn = (base.double() ** 2).sum(1).float()
    gt = []
    for i in range(0, q.shape[0], chunk):
        qq = q[i:i + chunk]
        s = bn[None, :] - 2.0 * (qq @ base.T)
        cand = s.topk(short, dim=1, largest=False).indices
        xb = base[cand].double()
        dd = ((xb - qq.double()[:, None, :]) ** 2).sum(2)
        order = dd.argsort(dim=1, stable=True)[:, :width]
        gt.append(torch.gather(cand, 1, order).cpu().numpy())
    return np.concatenate(gt)


def recall_at(ids, gt, k=10):
    """Standard k@k recall: |returned top-k & true top-k| / k."""
    hits = 0
    for a, b in zip(ids, gt):
        hits += len(set(a[:k].tolist()) & set(b[:k].tolist()))
    return hits / (len(ids) * k)


def recall_ref_def(ids, gt, k=10):
    """The reference demos' definition: a returned id counts if it is anywhere
    in the ground-truth row (examples/demo_jhq_v14_streaming_add.cu:15-27,
    which loops over the GT file's full width)."""
    hits = 0
    for a, b in zip(ids, gt):
        hits += len(set(a[:k].tolist()) & set(b.tolist()))
    return hits / (len(ids) * k)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the JHQ engine is "
              "single-GPU and multi-GPU sharding is design-only in this build.", file=sys.stderr)
        sys.exit(2)
    import torch
    import jhq_gpu_amd as jg
    if not torch.cuda.is_available():
        print("no HIP device visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False

    N = int(1_000_000 * args.scale)
    D, NQ, NCOMP = 1024, 10_000, 10_000
    M, B, Br, NLIST, K, BATCH = 128, 8, 4, 4096, 10, 64
    if args.scale < 1.0:
        NLIST = max(64, int(NLIST * args.scale))
    nprobes = [int(x) for x in args.nprobe.split(",")]
    alphas = [float(x) for x in args.alpha.split(",")]

    t0 = time.time()
    base, means, scales = gen_mixture(torch, dev, N, D, NCOMP, args.seed)
    q, _, _ = gen_mixture(torch, dev, NQ, D, NCOMP, args.seed + 0x100, means, scales)
    torch.cuda.synchronize()
    log(f"data N={N} NQ={NQ} D={D} gen {time.time() - t0:.1f}s")
    hb = base.cpu().numpy()
    hq = q.cpu().numpy()

    gt = None
    if args.profile_batches <= 0:
        t0 = time.time()
        gt = ground_truth(torch, base, q, K)
        torch.cuda.synchronize()
        log(f"ground truth {time.time() - t0:.1f}s")

    p = jg.Params(M=M, B=B, Br=Br, alpha=alphas[0], nlist=NLIST, nprobe=nprobes[0],
                  ivf_iters=8, batch_size=BATCH, seed=42)
    t0 = time.time()
    ix = jg.JHQGpuIndex(D, p)
    t_create = time.time() - t0
    n_train = min(N, 100_000)
    t0 = time.time()
    ix.train(hb[:n_train])
    t_train = time.time() - t0
    log(f"create {t_create:.1f}s train {t_train:.1f}s")
    t0 = time.time()
    ix.add(hb)
    t_add = time.time() - t0
    log(f"add {t_add:.1f}s")
    del base
    torch.cuda.empty_cache()

    if args.profile_batches > 0:
        profile_mode(torch, dev, ix, q, K, BATCH, nprobes[0], alphas[0], args.profile_batches)
        return

    out_d = torch.empty((NQ, K), dtype=torch.float32, device=dev)
    out_i = torch.empty((NQ, K), dtype=torch.int32, device=dev)
    nb = (NQ + BATCH - 1) // BATCH

    def run_steps(nsteps):
        for s in range(nsteps):
            b = s % nb
            q0 = b * BATCH
            q1 = min(NQ, q0 + BATCH)
            ix.search_device(q[q0:q1], K, out_d[q0:q1], out_i[q0:q1])

    sweep = []
    for alpha in alphas:
        ix.set_alpha(alpha)
        for npb in nprobes:
            ix.set_nprobe(npb)
            run_steps(nb)
            torch.cuda.synchronize()
            t0 = time.time()
            run_steps(nb)
            torch.cuda.synchronize()
            dt = time.time() - t0
            ids_np = out_i.cpu().numpy()
            rec = recall_at(ids_np, gt, K)
            rec_ref = recall_ref_def(ids_np, gt, K)
            sweep.append(dict(alpha=alpha, nprobe=npb, qps=NQ / dt, recall_at_10=rec,
                              recall_ref_def=rec_ref))
            log(f"sweep alpha={alpha:g} nprobe={npb} qps={NQ / dt:.0f} recall@10={rec:.4f} "
                f"(reference definition, 10@100: {rec_ref:.4f})")
    ok = [s for s in sweep if s["recall_at_10"] >= 0.95]
    gate_met = bool(ok)
    if not ok:
        # the quantizer's recall ceiling is below the gate on this data: take
        # the fastest point within 0.001 of the best recall
        best = max(s["recall_at_10"] for s in sweep)
        ok = [s for s in sweep if s["recall_at_10"] >= best - 1e-3]
    chosen = max(ok, key=lambda s: s["qps"])
    npb, alpha = chosen["nprobe"], chosen["alpha"]
    ix.set_nprobe(npb)
    ix.set_alpha(alpha)

    W = args.warmup if args.warmup > 0 else nb
    Kst = args.steps if args.steps > 0 else 5 * nb
    run_steps(W)
    torch.cuda.synchronize()
    t0 = time.time()
    run_steps(Kst)
    torch.cuda.synchronize()
    elapsed = time.time() - t0
    queries_timed = sum(min(BATCH, NQ - (s % nb) * BATCH) for s in range(Kst))
    qps = queries_timed / elapsed
    ms_per_step = elapsed * 1000.0 / Kst
    rec = recall_at(out_i.cpu().numpy(), gt, K)
    rec_ref = recall_ref_def(out_i.cpu().numpy(), gt, K)
    log(f"timed nprobe={npb} steps={Kst} qps={qps:.0f} ms/step={ms_per_step:.4f} recall={rec:.4f}")

    # per-kernel HIP-event times over one pass (events on the kernels' stream)
    ix.set_timing(True)
    run_steps(nb)
    torch.cuda.synchronize()
    tm, nbat = ix.timing()
    ix.set_timing(False)
    step_us = {k2: v * 1000.0 / nbat for k2, v in tm.items()}
    log("per-batch us: " + " ".join(f"{k2}={v:.1f}" for k2, v in step_us.items()))

    # algorithmic scan bytes per launch: sum_q sum_{probed l} |l| * M
    dbg = ix.search_debug(hq, K)
    lists = ix.lists(include_payload=False)
    sizes = np.diff(lists["offsets"]).astype(np.int64)
    per_q = sizes[dbg["probes"]].sum(1)
    scan_bytes_per_launch = float(per_q.sum()) * M / nb
    scan_us = step_us["scan_topck"]
    achieved = scan_bytes_per_launch / (scan_us * 1e-6) / 1e9
    dominant = max(step_us, key=step_us.get)

    # HBM traffic per scan launch: FETCH_SIZE + WRITE_SIZE from the committed
    # rocprofv3 counter runs (scaled by the calibration kernel), when they were
    # taken at the operating point chosen above
    traffic, traffic_note = None, "no counter run at this operating point"
    tpath = os.path.join(ROOT, "profiles", "scan_topck_cfg2_traffic.json")
    if os.path.exists(tpath) and args.scale == 1.0:
        with open(tpath) as f:
            tj = json.load(f)
        if tj.get("nprobe") == npb and float(tj.get("alpha")) == float(alpha):
            traffic = int(tj["traffic_bytes_per_launch"])
            traffic_note = ("bytes per launch from %s (FETCH_SIZE x %.2f + WRITE_SIZE x %.2f)"
                            % (tj["source"], tj["fetch_scale"], tj["write_scale"]))

    # reference protocol: host arrays, warm-up + mean of 5 search() calls
    ix.search(hq, K)
    t0 = time.time()
    for _ in range(5):
        ix.search(hq, K)
    qps_host = NQ / ((time.time() - t0) / 5)
    log(f"host-to-host qps={qps_host:.0f}")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(ix, npb, alpha, hq, K, out_i.cpu().numpy(), args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": round(qps, 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": Kst,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded 10k-component Gaussian mixture, L2-normalised (torch Philox)",
        "config": {
            "workload": "cfg2 IVF-JHQ N=1M D=1024 fp32, nlist=4096, M=128 B=8 Br=4, alpha=%g, "
                        "k=10, batch=64, queries resident in HBM" % alpha,
            "N": N, "nq": NQ, "nlist": NLIST, "nprobe": npb, "alpha": alpha, "k": K,
            "batch": BATCH, "recall_at_10": round(rec, 4),
            "recall_gate_0.95_met": gate_met,
            "recall_at_10_reference_definition": round(rec_ref, 4),
            "recall_note": ("standard 10@10 against exact L2; the reference's published recalls "
                            "count a hit anywhere in a 100-wide GT row (10@100, reported "
                            "alongside). With M=128 B=8 Br=4 the JHQ estimate itself caps "
                            "10@10 below 0.95 on this data (refining every candidate reaches "
                            "0.8865 on a 50K sample), so the gate is unmet at every nprobe/alpha"),
            "sweep": [{k2: (round(v, 4) if isinstance(v, float) else v) for k2, v in s.items()}
                      for s in sweep],
            "qps_host_to_host": round(qps_host, 1),
            "build_s": {"create": round(t_create, 2), "train": round(t_train, 2),
                        "add": round(t_add, 2)},
            "step_us_per_batch": {k2: round(v, 2) for k2, v in step_us.items()},
        },
        "roofline": {
            "kernel": "scan_topck_kernel",
            "dominant_step": dominant,
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_note": traffic_note,
            "algorithmic_bytes_per_launch": int(scan_bytes_per_launch),
            "avg_launch_us": round(scan_us, 2),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def profile_mode(torch, dev, ix, q, k, batch, nprobe, alpha, nbatches):
    """A short, fixed workload for rocprofv3 counter runs: `nbatches` search
    batches over distinct queries, then one elementwise float32 kernel that
    reads and writes 256 MiB; its FETCH_SIZE / WRITE_SIZE readings calibrate
    the counters."""
    ix.set_nprobe(nprobe)
    ix.set_alpha(alpha)
    out_d = torch.empty((batch, k), dtype=torch.float32, device=dev)
    out_i = torch.empty((batch, k), dtype=torch.int32, device=dev)
    nq = q.shape[0]
    ix.set_timing(True)
    for s in range(nbatches):
        q0 = (s * batch) % max(1, nq - batch + 1)
        ix.search_device(q[q0:q0 + batch], k, out_d, out_i)
    torch.cuda.synchronize()
    tm, nb = ix.timing()
    ix.set_timing(False)
    # calibration: an elementwise float32 kernel that reads and writes 256 MiB
    src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    # algorithmic scan bytes of the profiled batches
    L = ix.lists(include_payload=False)
    sizes = np.diff(L["offsets"]).astype(np.int64)
    qs = [q[(s * batch) % max(1, nq - batch + 1):][:batch] for s in range(nbatches)]
    tot = 0
    for qq in qs:
        dbg = ix.search_debug(qq.cpu().numpy(), k)
        tot += int(sizes[dbg["probes"]].sum()) * ix.params.M
    print(json.dumps({"profile_batches": nbatches, "nprobe": nprobe, "alpha": alpha,
                      "scan_bytes_per_launch": tot / nbatches,
                      "step_us_per_batch": {k2: round(v * 1000.0 / nb, 2) for k2, v in tm.items()},
                      "calibration_kernel": "torch.mul(float32[64Mi], 1.0)",
                      "calibration_bytes_each_way": 256 << 20}), flush=True)


def cpu_baseline(ix, nprobe, alpha, hq, k, gpu_ids, seconds):
    """Oracle (scalar C restatement of the reference) on the GPU-built index."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as po
    cb = ix.codebooks()
    L = ix.lists()
    pp = ix.params
    pp.nprobe = nprobe
    pp.alpha = alpha
    o = po.OracleIndex.from_state(ix.dim, pp, cb["P"], cb["c1d"], cb["res_c1d"], cb["centroids"],
                                  cb["cent_norms"], L["offsets"], L["ids"], L["codes"], L["res"],
                                  L["corr"])
    n = 0
    ids = []
    t0 = time.time()
    while n < hq.shape[0] and (time.time() - t0) < seconds:
        _, i1 = o.search(hq[n:n + 1], k)
        ids.append(i1[0])
        n += 1
    dt = time.time() - t0
    ids = np.array(ids)
    same = float(np.mean([len(set(a) & set(b)) / k for a, b in zip(ids, gpu_ids[:n])]))
    log(f"cpu baseline: {n} queries in {dt:.1f}s ({n / dt:.1f} q/s), id overlap with GPU {same:.4f}")
    return {
        "value": round(n / dt, 2),
        "unit": "queries/s",
        "cores": 1,
        "kind": "port",
        "sample": f"first {n} of the 10k config-2 queries, one at a time, nprobe={nprobe}, "
                  f"alpha={alpha:g}, "
                  f"oracle search on the GPU-built index (id overlap with GPU {same:.4f})",
    }


if __name__ == "__main__":
    main()
