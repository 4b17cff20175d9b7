#!/usr/bin/env python3
"""bench.py — JHQ IVF search throughput on one MI355X.

Default run (the driver's `python bench.py --gpus 1 --steps K --warmup W`):

* Headline, BASELINE.json configs[1] ("config 2"): N=1,000,000 base and
  10,000 query vectors, D=1024 fp32, drawn from a seeded 10,000-component
  Gaussian mixture (per-component N(0, I) mean, diagonal std log-uniform in
  [0.1, 1], uniform weights) and L2-normalised.  IVF nlist=4096 trained on the
  first 100,000 base vectors (the reference demo's protocol), M=128, B=8,
  Br=4, k=10, query batch 64.  Ground truth is exact L2 brute force.  A
  "step" is one device search call over the 10,000 queries, resident in HBM
  with their results: the engine runs them in batches of 64 through the whole
  search path, consecutive batches on the search lanes that have hardware
  queues of their own (four of six streams; forked from and joined into the
  caller's stream; a lane takes two consecutive batches at a time, with one
  query-product launch for both).  The sweep nprobe {16, 32, 64} x
  alpha {4, 10} picks the fastest point with recall@10 >= 0.95; when no point
  reaches it (the codes' own recall ceiling, measured by ranking every vector
  by its full estimate, is below 0.95 on this data) the fastest point within
  0.001 of the best recall.  `value` is that point's queries/s over exactly
  --steps timed steps; the host-to-host rate of the reference's protocol
  (PCIe copies included) is reported beside it.
* HBM-streaming leg, configs[2] ("config 3"): 100M x 128 uint8, nlist 65,536,
  nprobe 64, M=16, batch 64 (1.6 GB of codes, streamed from HBM), under
  `hbm_streaming_leg` with its own roofline, counters and build check.

Each part reports per-kernel HIP-event times, the step's roofline (bytes and
int8 ops the step must move and compute over the timed pipelined step), the
measured HBM traffic from the committed counter run, and the CPU baseline
(the oracle's scalar search on the same GPU-built index, one query at a time
and over all host threads).  `--config N` runs one configuration alone.
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
INT8_PEAK_TOPS = 5000.0  # dense int8 MFMA


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=0,
                    help="timed steps, each one pass over the query set (default: 10; 3 for "
                         "configs 3-5)")
    ap.add_argument("--warmup", type=int, default=0, help="warmup steps (default: 1)")
    ap.add_argument("--config", type=int, default=None, choices=(1, 2, 3, 4, 5),
                    help="BASELINE.json workload alone: 2 (the metric's config), 1 (flat "
                         "100K x 1024, one query per batch), 3 (100M uint8 D=128), 4 (100M "
                         "int8 D=100), 5 (streaming add + search, D=768).  Default: config 2, "
                         "then config 3 as the HBM-streaming leg of the same JSON line")
    ap.add_argument("--no-hbm-leg", action="store_true",
                    help="default run: skip the config-3 leg")
    ap.add_argument("--nprobe", type=str, default=None,
                    help="nprobe values swept (default: 16,32,64 for config 2, the config's own "
                         "value otherwise)")
    ap.add_argument("--alpha", type=str, default=None,
                    help="short-list factors swept (ck = max(k, ceil(alpha*k))); default 4,10 "
                         "for config 2, 4 otherwise")
    ap.add_argument("--scale", type=float, default=1.0, help="fraction of N (debug only)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--profile-batches", type=int, default=0,
                    help="profiling mode: build the index, run this many search batches at the "
                         "first --nprobe/--alpha plus one 256 MiB device copy (the counter "
                         "calibration kernel), print per-step times and exit")
    ap.add_argument("--trace-steps", type=int, default=0,
                    help="kernel-trace mode: build the index, then run one warmup and this many "
                         "timed device-search calls over the whole query set at the first "
                         "--nprobe/--alpha (the pipelined step the headline times), print their "
                         "times and exit")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--index", type=str, default=None,
                    help="configs 3/4 with --profile-batches: load the index from this file "
                         "(jhq_save format) if it exists, else build it and save it there")
    ap.add_argument("--seed", type=int, default=None,
                    help="data seed (default 0x4A48510000 + config)")
    ap.add_argument("--scan-kind", type=int, default=0, choices=(0, 1, 2),
                    help="0 (default): the integer-MFMA pre-scan with exact re-check where it "
                         "applies and pays off; 1: the byte-LUT scans only; 2: the pre-scan "
                         "wherever it applies (same results)")
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
    if not torch.cuda.is_available():
        print("no HIP device visible", file=sys.stderr)
        sys.exit(1)
    torch.backends.cuda.matmul.allow_tf32 = False
    if args.config is None:
        # the headline (config 2), then the HBM-streaming workload (config 3,
        # 1.6 GB of codes, read from HBM) reported under its own key
        args.config = 2
        line = bench_float(args, FLOAT_CFGS[2])
        if not args.no_hbm_leg and args.profile_batches <= 0:
            import gc
            gc.collect()
            torch.cuda.empty_cache()
            a3 = argparse.Namespace(**vars(args))
            a3.config, a3.nprobe, a3.alpha, a3.seed = 3, None, None, None
            a3.cpu_seconds = min(args.cpu_seconds, 10.0)
            log("HBM-streaming leg: config 3")
            line["hbm_streaming_leg"] = bench_bytes(a3, LARGE[3])
    elif args.config in (1, 2):
        line = bench_float(args, FLOAT_CFGS[args.config])
    elif args.config in (3, 4):
        line = bench_bytes(args, LARGE[args.config])
    else:
        line = bench_streaming(args)
    if line is not None:
        print(json.dumps(line), flush=True)


FLOAT_CFGS = {
    # flat JHQ, one query at a time
    1: dict(name="cfg1", N=100_000, NQ=1_000, NCOMP=1_000, D=1024, M=128, NLIST=1, NPROBE="1",
            ALPHA="4", BATCH=1, seed=0x4A48510001,
            workload="cfg1 flat JHQ N=100K D=1024 fp32, nlist=1, M=128 B=8 Br=4, alpha=%g, "
                     "k=10, one query per batch, queries resident in HBM"),
    # the metric's config
    2: dict(name="cfg2", N=1_000_000, NQ=10_000, NCOMP=10_000, D=1024, M=128, NLIST=4096,
            NPROBE="16,32,64", ALPHA="4,10", BATCH=64, seed=0x4A48510002,
            workload="cfg2 IVF-JHQ N=1M D=1024 fp32, nlist=4096, M=128 B=8 Br=4, alpha=%g, "
                     "k=10, batch=64, queries resident in HBM"),
}


def bench_float(args, cf):
    import torch
    import jhq_gpu_amd as jg
    dev = torch.device("cuda:0")
    if args.seed is None:
        args.seed = cf["seed"]
    if args.nprobe is None:
        args.nprobe = cf["NPROBE"]
    if args.alpha is None:
        args.alpha = cf["ALPHA"]

    N = int(cf["N"] * args.scale)
    D, NQ, NCOMP = cf["D"], cf["NQ"], cf["NCOMP"]
    M, B, Br, NLIST, K, BATCH = cf["M"], 8, 4, cf["NLIST"], 10, cf["BATCH"]
    if args.scale < 1.0 and NLIST > 1:
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
    if args.profile_batches <= 0 and args.trace_steps <= 0:
        t0 = time.time()
        gt = ground_truth(torch, base, q, K)
        torch.cuda.synchronize()
        log(f"ground truth {time.time() - t0:.1f}s")

    p = jg.Params(M=M, B=B, Br=Br, alpha=alphas[0], nlist=NLIST, nprobe=nprobes[0],
                  ivf_iters=8, batch_size=BATCH, seed=42)
    t0 = time.time()
    ix = jg.JHQGpuIndex(D, p)
    ix.set_scan_kind(args.scan_kind)
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
        return None
    if args.trace_steps > 0:
        trace_mode(torch, dev, ix, q, K, BATCH, nprobes[0], alphas[0], args.trace_steps)
        return None

    out_d = torch.empty((NQ, K), dtype=torch.float32, device=dev)
    out_i = torch.empty((NQ, K), dtype=torch.int32, device=dev)
    nb = (NQ + BATCH - 1) // BATCH

    def run_steps(nsteps):
        for s in range(nsteps):
            ix.search_device(q, K, out_d, out_i)

    sweep = []
    for alpha in alphas:
        ix.set_alpha(alpha)
        for npb in nprobes:
            ix.set_nprobe(npb)
            run_steps(1)
            torch.cuda.synchronize()
            t0 = time.time()
            run_steps(2)
            torch.cuda.synchronize()
            dt = (time.time() - t0) / 2
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

    W = args.warmup if args.warmup > 0 else 1
    Kst = args.steps if args.steps > 0 else 10
    run_steps(W)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.time()
    ev0.record()
    run_steps(Kst)
    ev1.record()
    torch.cuda.synchronize()
    elapsed = time.time() - t0
    ev_ms = ev0.elapsed_time(ev1) / Kst
    qps = NQ * Kst / elapsed
    ms_per_step = elapsed * 1000.0 / Kst
    rec = recall_at(out_i.cpu().numpy(), gt, K)
    rec_ref = recall_ref_def(out_i.cpu().numpy(), gt, K)
    log(f"timed nprobe={npb} steps={Kst} qps={qps:.0f} ms/step={ms_per_step:.4f} recall={rec:.4f}")

    # per-kernel HIP-event times over one pass (events on the kernels' stream;
    # timing runs the batches one after another on one stream)
    ix.set_timing(True)
    run_steps(1)
    torch.cuda.synchronize()
    tm, nbat = ix.timing()
    ix.set_timing(False)
    step_us = {k2: v * 1000.0 / nbat for k2, v in tm.items()}
    log("per-batch us: " + " ".join(f"{k2}={v:.1f}" for k2, v in step_us.items()))

    roof = step_roofline(ix, hq, K, BATCH, step_us, ev_ms, cf["name"], npb, alpha,
                         use_profiles=args.scale == 1.0)

    # reference protocol: host arrays, warm-up + mean of 5 search() calls
    ix.search(hq, K)
    t0 = time.time()
    for _ in range(5):
        ix.search(hq, K)
    qps_host = NQ / ((time.time() - t0) / 5)
    log(f"host-to-host qps={qps_host:.0f}")

    # the quantizer's own ceiling: every base vector ranked by the full JHQ
    # estimate (primary + residual, i.e. ck = N)
    t0 = time.time()
    ceiling = recall_ceiling(torch, dev, ix, q, gt, K)
    log(f"recall ceiling (every vector refined) {ceiling:.4f} ({time.time() - t0:.1f}s)")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(ix, npb, alpha, hq, K, out_i.cpu().numpy(), args.cpu_seconds,
                           hb[:n_train], NLIST, n_train)

    metric = METRIC
    if not gate_met:
        metric += (" [value: queries/s with queries and results in HBM at recall@10 %.4f; the "
                   "0.95 gate is above these codes' recall ceiling %.4f]" % (rec, ceiling))
    line = {
        "metric": metric,
        "value": round(qps, 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": Kst,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 5),
        "ms_per_step_hip_events": round(ev_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded %d-component Gaussian mixture, L2-normalised (torch Philox)"
                % NCOMP,
        "config": {
            "workload": cf["workload"] % alpha,
            "N": N, "nq": NQ, "nlist": NLIST, "nprobe": npb, "alpha": alpha, "k": K,
            "batch": BATCH, "recall_at_10": round(rec, 4),
            "recall_gate_0.95_met": gate_met,
            "recall_at_10_ceiling_all_refined": round(ceiling, 4),
            "recall_at_10_reference_definition": round(rec_ref, 4),
            "recall_note": ("standard 10@10 against exact L2; the reference's published recalls "
                            "count a hit anywhere in a 100-wide GT row (10@100, reported "
                            "alongside). recall_at_10_ceiling_all_refined ranks every base "
                            "vector by the full JHQ estimate (ck = N): no nprobe/alpha can "
                            "exceed it, so the 0.95 gate is unreachable for M=128 B=8 Br=4 "
                            "codes on this data"),
            "sweep": [{k2: (round(v, 4) if isinstance(v, float) else v) for k2, v in s.items()}
                      for s in sweep],
            "qps_host_to_host": round(qps_host, 1),
            "qps_note": "value: queries and results resident in HBM (device search); "
                        "qps_host_to_host: the reference demo's protocol with PCIe copies",
            "build_s": {"create": round(t_create, 2), "train": round(t_train, 2),
                        "add": round(t_add, 2)},
            "step_us_per_batch": {k2: round(v, 2) for k2, v in step_us.items()},
            "query_product_fp32_mfma": query_product_rate(NQ, nb, D, NLIST, step_us),
        },
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    return line


def recall_ceiling(torch, dev, ix, q, gt, k, chunk=65536):
    """recall@k when every base vector is ranked by its full JHQ estimate
    ||q_rot - (yhat + rhat)||^2 (the composite distance minus ||q||^2): the
    best any nprobe / alpha can reach with these codes."""
    cb = ix.codebooks()
    L = ix.lists()
    pp = ix.params
    d, M = ix.dim, pp.M
    Ds = d // M
    K1D = cb["c1d"].size
    bpd = K1D.bit_length() - 1
    c1d = torch.from_numpy(cb["c1d"]).to(dev)
    rc = torch.from_numpy(np.asarray(cb["res_c1d"], np.float32).reshape(-1)).to(dev)
    P = torch.from_numpy(cb["P"]).to(dev)
    qr = q @ P.T
    qn = (qr * qr).sum(1, keepdim=True)
    shifts = torch.arange(Ds, device=dev, dtype=torch.int32) * bpd
    jj = torch.arange(d, device=dev)
    n = L["ids"].shape[0]
    best_d = torch.full((q.shape[0], k), float("inf"), device=dev)
    best_i = torch.full((q.shape[0], k), -1, dtype=torch.int64, device=dev)
    ids_all = torch.from_numpy(L["ids"]).to(dev).long()
    for c0 in range(0, n, chunk):
        codes = torch.from_numpy(L["codes"][c0:c0 + chunk]).to(dev).int()
        res = torch.from_numpy(L["res"][c0:c0 + chunk]).to(dev).int()
        dig = (codes[:, :, None] >> shifts) & (K1D - 1)
        yhat = c1d[dig.reshape(codes.shape[0], d).long()]
        if pp.Br == 4:
            r = (res[:, jj // 2] >> ((jj % 2) * 4)) & 15
        else:
            r = res
        cbo = ((jj // Ds) * (1 << pp.Br)) if pp.residual_per_subspace else 0
        xhat = yhat + rc[(r + cbo).long()]
        dd = qn - 2.0 * (qr @ xhat.T) + (xhat * xhat).sum(1)[None, :]
        cd = torch.cat([best_d, dd], 1)
        ci = torch.cat([best_i, ids_all[c0:c0 + chunk][None, :].expand(q.shape[0], -1)], 1)
        o = cd.topk(k, dim=1, largest=False).indices
        best_d, best_i = torch.gather(cd, 1, o), torch.gather(ci, 1, o)
        del codes, res, dig, yhat, xhat, dd, cd, ci
    return recall_at(best_i.cpu().numpy(), gt, k)


# ---------------------------------------------------------------------------
# configs 3 and 4: 100M byte vectors, the scan streaming codes from HBM
# ---------------------------------------------------------------------------
LARGE = {
    3: dict(name="cfg3", N=100_000_000, D=128, NQ=10_000, NCOMP=65_536, NLIST=65_536,
            NPROBE=64, M=16, BATCH=64, kind="uint8"),
    4: dict(name="cfg4", N=100_000_000, D=100, NQ=10_000, NCOMP=32_768, NLIST=32_768,
            NPROBE=48, M=25, BATCH=32, kind="int8"),
}


def gen_bytes(torch, dev, n, d, ncomp, seed, kind, means=None, chunk=2_000_000):
    """Byte-valued mixture rows on the device.
    uint8: component means ~ N(34, 60^2) per coordinate, per-coordinate std 20,
    rounded and clipped to 0..255 (about 30% of coordinates become 0).
    int8: means ~ N(0, 32^2), plus 16 * Student-t(nu=4) noise (a normal over
    sqrt(chi2_4 / 4)), rounded and clipped to -128..127."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    if means is None:
        mu, sd = (34.0, 60.0) if kind == "uint8" else (0.0, 32.0)
        means = mu + sd * torch.randn(ncomp, d, device=dev, generator=g)
    lo, hi, dt = (0, 255, torch.uint8) if kind == "uint8" else (-128, 127, torch.int8)
    out = torch.empty(n, d, dtype=dt, device=dev)
    for i in range(0, n, chunk):
        m = min(chunk, n - i)
        c = torch.randint(0, ncomp, (m,), device=dev, generator=g)
        z = torch.randn(m, d, device=dev, generator=g)
        if kind == "uint8":
            x = means[c] + 20.0 * z
        else:
            chi = (torch.randn(m, d, 4, device=dev, generator=g) ** 2).sum(2)
            x = means[c] + 16.0 * z / torch.sqrt(chi / 4.0)
        out[i:i + m] = torch.clamp(torch.round(x), lo, hi).to(dt)
        del x, z, c
    return out, means


def ground_truth_int(torch, base, q, width=100, bchunk=4_000_000, qchunk=1024):
    """Exact L2 neighbours of integer-valued data: ||x||^2 - 2<q,x> in fp32 is
    exact (every partial sum is an integer below 2^24 for these ranges), so an
    fp32 GEMM over base chunks with a running top-`width` is exact up to
    order among equal distances.  Returns (ids [nq, width], dists [nq, width])
    with dists = ||q - x||^2."""
    nq = q.shape[0]
    qn = (q.double() ** 2).sum(1)
    best_d = torch.full((nq, width), float("inf"), device=q.device)
    best_i = torch.full((nq, width), -1, dtype=torch.int64, device=q.device)
    for b0 in range(0, base.shape[0], bchunk):
        xb = base[b0:b0 + bchunk].float()
        xn = (xb * xb).sum(1)
        for q0 in range(0, nq, qchunk):
            qq = q[q0:q0 + qchunk]
            s = torch.addmm(xn.expand(qq.shape[0], -1), qq, xb.T, alpha=-2.0)
            dd, ii = s.topk(min(width, s.shape[1]), dim=1, largest=False)
            cd = torch.cat([best_d[q0:q0 + qchunk], dd], 1)
            ci = torch.cat([best_i[q0:q0 + qchunk], ii + b0], 1)
            o = cd.topk(width, dim=1, largest=False).indices
            best_d[q0:q0 + qchunk] = torch.gather(cd, 1, o)
            best_i[q0:q0 + qchunk] = torch.gather(ci, 1, o)
            del s, dd, ii, cd, ci
        del xb, xn
        log(f"ground truth: {min(b0 + bchunk, base.shape[0])} / {base.shape[0]} base rows")
    # ascending order, then add ||q||^2 back
    o = best_d.argsort(dim=1, stable=True)
    best_d = torch.gather(best_d, 1, o).double() + qn[:, None]
    best_i = torch.gather(best_i, 1, o)
    return best_i.cpu().numpy(), best_d.cpu().numpy()


def exact_dists(torch, base, q, ids):
    """||q - x_id||^2 in float64 for returned ids (-1 -> inf)."""
    t = torch.as_tensor(ids, device=q.device, dtype=torch.int64)
    ok = t >= 0
    x = base[t.clamp(min=0)].double()
    d = ((x - q.double()[:, None, :]) ** 2).sum(2)
    d[~ok] = float("inf")
    return d.cpu().numpy()


def recall_tie_aware(dist_ret, gt_d, k=10):
    """Hits are returned ids whose exact distance is <= the k-th true distance
    (integer data has exact ties, so id sets alone under-count)."""
    kth = gt_d[:, k - 1:k]
    return float(np.minimum((dist_ret[:, :k] <= kth * (1 + 1e-12)).sum(1), k).sum()) / (
        dist_ret.shape[0] * k)


def timed_search(torch, ix, q, out_d, out_i, k, batch, warmup, steps):
    """Queries/s, ms per step (host clock) and ms per step from HIP events on
    the caller's stream around the timed steps; a step is one device search
    over all of q (the engine batches it by its batch_size)."""
    nq = q.shape[0]

    def run(nsteps):
        for st in range(nsteps):
            ix.search_device(q, k, out_d, out_i)

    run(warmup)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.time()
    ev0.record()
    run(steps)
    ev1.record()
    torch.cuda.synchronize()
    el = time.time() - t0
    return nq * steps / el, el * 1000.0 / steps, ev0.elapsed_time(ev1) / steps


def step_times(torch, ix, q, out_d, out_i, k, batch):
    ix.set_timing(True)
    timed_search(torch, ix, q, out_d, out_i, k, batch, 0, 1)
    tm, nbat = ix.timing()
    ix.set_timing(False)
    return {k2: v * 1000.0 / nbat for k2, v in tm.items()}


FP32_MFMA_PEAK_TFLOPS = 157.3


def query_product_rate(nq, nb, d, nlist, step_us):
    """The query product (rotation and centroid scores in one fp32 MFMA
    product, 2 * B * d * (d + nlist) flops per batch) against the fp32 MFMA
    peak, over its HIP-event time on one stream."""
    flops = 2.0 * (nq / nb) * d * (d + nlist)
    us = step_us["query_gemm"]
    tf = flops / (us * 1e-6) / 1e12
    return {"flops_per_batch": int(flops), "us_per_batch": round(us, 2),
            "achieved_tflops": round(tf, 2), "peak_tflops": FP32_MFMA_PEAK_TFLOPS,
            "frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4),
            "note": "HIP events around the query product on one stream: the product "
                    "kernel, and the kernel that adds its split sums where the probe "
                    "selection does not (nlist > 8192; at nlist <= 8192 the selection adds "
                    "them)"}


def step_roofline(ix, hq, k, batch, step_us, ev_ms_per_step, workload, nprobe, alpha,
                  use_profiles=True):
    """The roofline of the search step at the current operating point.

    Time base: one batch's share of the timed pipelined run, ev_ms_per_step /
    batches per step (HIP events on the caller's stream bracket the timed steps;
    the engine forks its lanes from that stream and joins them back into it).

    Bytes and ops are what the dominant step's kernels must move and compute:
    * byte-LUT scans (scan_skew / scan_wave / scan_dump): every probed code is
      streamed once per query (sum_q sum_probed |l| * M), as the reference's
      scan does (v14/search.cu:138-151), plus the refine's ck * (bpv + 8)
      bytes per query;
    * the integer-MFMA pre-scan: the batch's distinct probed lists once
      (sum over distinct l of |l| * M), the I-value dump it writes (4 B per
      padded (query, candidate) slot + 4 B per tile minimum) and the least of
      it the re-check must read back (the tile minima + the 16 values of ck
      tiles per query), plus the refine's bytes; its int8 MFMA work is
      16 x 16 x D multiply-adds x 2 halves per 16-query x 16-candidate tile,
      priced against 5.0 POP/s.
    frac is the larger of bytes / time / 8 TB/s and ops / time / 5 POP/s, and
    `bound` names that roofline.  The counter run committed under profiles/
    for this operating point gives the measured HBM traffic per launch and
    what limits the kernels (`limiter`)."""
    dbg = ix.search_debug(hq, k)
    L = ix.lists(include_payload=False)
    sizes = np.diff(L["offsets"]).astype(np.int64)
    pad = (sizes + 15) // 16
    nq = hq.shape[0]
    nb = (nq + batch - 1) // batch
    M, D = ix.params.M, hq.shape[1]
    kernel, ck = ix.scan_plan(k)
    bpv = ix.dims()["bpv"]
    probes = dbg["probes"]
    codes_per_query = float(sizes[probes].sum()) * M / nb       # per batch, counted per query
    refine = float(nq) * ck * (bpv + 4 + 4) / nb
    t_batch = ev_ms_per_step * 1e3 / nb                          # us per batch, pipelined
    mfma = kernel == "mfma_scan_kernel"
    fused = mfma and ck <= 128
    alone_us = step_us["scan_topck"] + (0.0 if fused else step_us["refine_topk"])
    parts = {"refine": refine}
    ops = 0.0
    if mfma:
        distinct = rows = tiles = 0
        for b in range(nb):
            lists, cnt = np.unique(probes[b * batch:(b + 1) * batch], return_counts=True)
            distinct += int(sizes[lists].sum()) * M
            rows += int((((cnt + 15) // 16) * sizes[lists]).sum()) * M
            tiles += int((((cnt + 15) // 16) * pad[lists]).sum())
        qt = pad[probes].sum(1)                                  # tiles per query
        dump_w = float((qt * 16 * 4 + qt * 4).sum())
        dump_r = float((qt * 4 + np.minimum(qt, ck) * 16 * 4).sum())
        parts.update(codes_distinct_lists=distinct / nb, dump_write=dump_w / nb,
                     dump_read_min=dump_r / nb)
        ops = tiles / nb * 16.0 * 16.0 * D * 2 * 2
    else:
        parts["codes_per_query"] = codes_per_query
    step_bytes = sum(parts.values())
    gbs = step_bytes / (t_batch * 1e-6) / 1e9
    tops = ops / (t_batch * 1e-6) / 1e12
    f_hbm, f_mfma = gbs / HBM_PEAK_GBS, tops / INT8_PEAK_TOPS
    bound = "mfma" if f_mfma > f_hbm else "hbm"
    traffic, traffic_note, limiter = None, "no counter run at this operating point", None
    counters = None
    pdir = os.path.join(ROOT, "profiles")
    for fn in sorted(os.listdir(pdir)) if (use_profiles and os.path.isdir(pdir)) else []:
        if not fn.endswith("_traffic.json"):
            continue
        with open(os.path.join(pdir, fn)) as f:
            tj = json.load(f)
        if (tj.get("kernel") == kernel and tj.get("nprobe") == nprobe
                and float(tj.get("alpha")) == float(alpha)
                and tj.get("workload", "").startswith(workload)):
            traffic = int(tj["traffic_bytes_per_launch"])
            traffic_note = ("HBM bytes per launch of the step's kernels from %s (FETCH_SIZE x %.2f "
                            "+ WRITE_SIZE x %.2f, factors from a copy kernel of known size)"
                            % (tj["source"], tj["fetch_scale"], tj["write_scale"]))
            limiter = tj.get("limiter")
            counters = tj.get("counters")
    names = {"scan_dump_kernel": "scan_dump_kernel + select_query_kernel",
             "mfma_scan_kernel": "mfma_scan_kernel + mfma_recheck_kernel"
                                 + (" (re-check and refine)" if fused else "")}
    out = {
        "kernel": names.get(kernel, kernel),
        "dominant_step": max(step_us, key=step_us.get),
        "bound": bound,
        "achieved": round(tops if bound == "mfma" else gbs, 2 if bound == "mfma" else 1),
        "peak": INT8_PEAK_TOPS if bound == "mfma" else HBM_PEAK_GBS,
        "unit": "TOP/s" if bound == "mfma" else "GB/s",
        "frac": round(max(f_hbm, f_mfma), 4),
        "traffic": traffic,
        "time_base": "us per batch in the timed pipelined run: HIP events on the caller's "
                     "stream around the timed steps / batches per step",
        "us_per_batch_pipelined": round(t_batch, 2),
        "algorithmic_bytes_per_batch": int(step_bytes),
        "bytes_breakdown": {k2: int(v) for k2, v in parts.items()},
        "hbm": {"achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "frac": round(f_hbm, 4)},
        "traffic_note": traffic_note,
        "traffic_rate_over_step_gbs": (None if traffic is None
                                       else round(traffic / (t_batch * 1e-6) / 1e9, 1)),
        "limiter": limiter,
        "counters": counters,
        "kernel_alone": {
            "us_per_launch": round(alone_us, 2),
            "note": "the step's kernels on one stream (HIP events in a separate timing pass); "
                    "in the pipelined run other lanes' kernels run beside them",
            "frac_hbm": round(step_bytes / (alone_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        },
    }
    if mfma:
        out["int8_mfma"] = {"ops_per_batch": int(ops), "achieved_tops": round(tops, 2),
                            "peak_tops": INT8_PEAK_TOPS, "frac": round(f_mfma, 4)}
        out["tile_row_reads_per_batch"] = int(rows / nb)
        out["effective_per_query_codes"] = {
            "bytes_per_batch": int(codes_per_query),
            "gbs_over_step": round(codes_per_query / (t_batch * 1e-6) / 1e9, 1),
            "note": "codes counted once per (query, probed list) as the reference's scan "
                    "streams them; the pre-scan reads each list once per 16-query tile, so "
                    "this is an effective rate, not a bandwidth",
        }
    else:
        out["scan_kernel_alone"] = {
            "us_per_launch": round(step_us["scan_topck"], 2),
            "codes_bytes_per_launch": int(codes_per_query),
            "frac_hbm": round(codes_per_query / (step_us["scan_topck"] * 1e-6) / 1e9
                              / HBM_PEAK_GBS, 4),
        }
    return out


def bench_bytes(args, cf):
    os.environ.setdefault("JHQ_VERBOSE", "1")  # progress lines during the long build
    import torch
    import jhq_gpu_amd as jg
    dev = torch.device("cuda:0")
    seed = args.seed if args.seed is not None else 0x4A48510000 + args.config
    N = int(cf["N"] * args.scale)
    D, NQ, M, K, BATCH = cf["D"], cf["NQ"], cf["M"], 10, cf["BATCH"]
    NLIST = cf["NLIST"] if args.scale >= 1.0 else max(64, int(cf["NLIST"] * args.scale))
    NCOMP = cf["NCOMP"] if args.scale >= 1.0 else max(64, int(cf["NCOMP"] * args.scale))
    npb = int((args.nprobe or str(cf["NPROBE"])).split(",")[0])
    alpha = float((args.alpha or "4").split(",")[0])

    if (args.profile_batches > 0 or args.trace_steps > 0) and args.index and \
            os.path.exists(args.index):
        # counter runs over a saved index: only the queries are generated
        _, means = gen_bytes(torch, dev, 0, D, NCOMP, seed, cf["kind"])
        qb, _ = gen_bytes(torch, dev, NQ, D, NCOMP, seed + 0x100, cf["kind"], means)
        t0 = time.time()
        ix = jg.JHQGpuIndex.load(args.index)
        ix.set_scan_kind(args.scan_kind)
        log(f"loaded {args.index} ({ix.ntotal} vectors) in {time.time() - t0:.1f}s")
        if args.trace_steps > 0:
            trace_mode(torch, dev, ix, qb.float(), K, BATCH, npb, alpha, args.trace_steps)
        else:
            profile_mode(torch, dev, ix, qb.float(), K, BATCH, npb, alpha, args.profile_batches)
        return None
    t0 = time.time()
    base, means = gen_bytes(torch, dev, N, D, NCOMP, seed, cf["kind"])
    qb, _ = gen_bytes(torch, dev, NQ, D, NCOMP, seed + 0x100, cf["kind"], means)
    torch.cuda.synchronize()
    zero_frac = float((base[:1_000_000] == 0).float().mean())
    log(f"data {cf['kind']} N={N} D={D} gen {time.time() - t0:.1f}s zero fraction "
        f"{zero_frac:.3f}")
    t0 = time.time()
    hb = base.cpu().numpy()
    hq = qb.cpu().numpy()
    qf = qb.float()
    log(f"host copy {time.time() - t0:.1f}s")

    if args.profile_batches <= 0 and args.trace_steps <= 0:
        t0 = time.time()
        gt_i, gt_d = ground_truth_int(torch, base, qf)
        torch.cuda.synchronize()
        log(f"ground truth {time.time() - t0:.1f}s")

    p = jg.Params(M=M, B=8, Br=4, alpha=alpha, nlist=NLIST, nprobe=npb, ivf_iters=8,
                  batch_size=BATCH, seed=42)
    ix = jg.JHQGpuIndex(D, p)
    ix.set_scan_kind(args.scan_kind)
    n_train = min(N, max(100_000, 16 * NLIST))
    t0 = time.time()
    ix.train(hb[:n_train])
    t_train = time.time() - t0
    log(f"train n={n_train} {t_train:.1f}s")
    t0 = time.time()
    ix.add(hb)
    t_add = time.time() - t0
    log(f"add {t_add:.1f}s ({N / t_add / 1e6:.2f} M vectors/s)")
    x_sample = np.ascontiguousarray(hb[:min(N, 1_000_000)])
    del hb
    if args.profile_batches > 0 or args.trace_steps > 0:
        del base
        torch.cuda.empty_cache()
        if args.index:
            t0 = time.time()
            ix.save(args.index)
            log(f"saved {args.index} in {time.time() - t0:.1f}s")
        if args.trace_steps > 0:
            trace_mode(torch, dev, ix, qf, K, BATCH, npb, alpha, args.trace_steps)
        else:
            profile_mode(torch, dev, ix, qf, K, BATCH, npb, alpha, args.profile_batches)
        return None

    out_d = torch.empty((NQ, K), dtype=torch.float32, device=dev)
    out_i = torch.empty((NQ, K), dtype=torch.int32, device=dev)
    nb = (NQ + BATCH - 1) // BATCH
    W = args.warmup if args.warmup > 0 else 1
    Kst = args.steps if args.steps > 0 else 3
    qps, ms, ev_ms = timed_search(torch, ix, qf, out_d, out_i, K, BATCH, W, Kst)
    ids = out_i.cpu().numpy()
    rec = recall_at(ids, gt_i, K)
    rec_tie = recall_tie_aware(exact_dists(torch, base, qf, ids), gt_d, K)
    rec_ref = recall_ref_def(ids, gt_i, K)
    log(f"timed nprobe={npb} steps={Kst} qps={qps:.0f} ms/step={ms:.4f} recall@10={rec:.4f} "
        f"tie-aware={rec_tie:.4f} 10@100={rec_ref:.4f}")
    step_us = step_times(torch, ix, qf, out_d, out_i, K, BATCH)
    log("per-batch us: " + " ".join(f"{k2}={v:.1f}" for k2, v in step_us.items()))
    roof = step_roofline(ix, hq.astype(np.float32), K, BATCH, step_us, ev_ms, cf["name"], npb,
                         alpha, use_profiles=args.scale == 1.0)
    used, cap = ix.pool()
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(ix, npb, alpha, hq.astype(np.float32), K, ids, args.cpu_seconds,
                           x_sample=x_sample)
    line = {
        "metric": f"QPS ({N // 1_000_000}Mx{D} {cf['kind']} IVF, nprobe {npb}, batch {BATCH}); "
                  "ADC-scan HBM GB/s vs peak",
        "value": round(qps, 1), "unit": "queries/s", "n_gpus": 1, "steps": Kst, "warmup": W,
        "ms_per_step": round(ms, 5), "ms_per_step_hip_events": round(ev_ms, 5),
        "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": f"synthetic: seeded {NCOMP}-component {cf['kind']} mixture (torch Philox), "
                f"zero fraction {zero_frac:.3f}",
        "config": {
            "workload": f"{cf['name']} IVF-JHQ N={N} D={D} {cf['kind']}, nlist={NLIST}, M={M} "
                        f"B=8 Br=4, alpha={alpha:g}, k=10, batch={BATCH}, queries resident "
                        "in HBM",
            "N": N, "nq": NQ, "nlist": NLIST, "nprobe": npb, "alpha": alpha, "k": K,
            "batch": BATCH, "n_train": n_train,
            "recall_at_10": round(rec, 4), "recall_at_10_tie_aware": round(rec_tie, 4),
            "recall_at_10_reference_definition": round(rec_ref, 4),
            "build_s": {"train": round(t_train, 2), "add": round(t_add, 2)},
            "pool_slots": [used, cap],
            "step_us_per_batch": {k2: round(v, 2) for k2, v in step_us.items()},
            "query_product_fp32_mfma": query_product_rate(NQ, nb, D, NLIST, step_us),
        },
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    return line


# ---------------------------------------------------------------------------
# config 5: streaming add interleaved with search
# ---------------------------------------------------------------------------
def gen_mixture_chunks(torch, dev, n, d, ncomp, seed, chunk=1_000_000):
    """gen_mixture for large n: same distribution, built chunk by chunk into
    one device tensor."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
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


def ground_truth_f32(torch, base, q, width=100, short=300, qchunk=128, bchunk=2_000_000):
    """Exact L2 neighbours of float data: an fp32 GEMM short list of `short`
    per base chunk, merged, then re-ranked in float64."""
    nq = q.shape[0]
    bn = torch.cat([(base[i:i + bchunk].double() ** 2).sum(1).float()
                    for i in range(0, base.shape[0], bchunk)])
    gt = []
    for q0 in range(0, nq, qchunk):
        qq = q[q0:q0 + qchunk]
        s = torch.addmm(bn.expand(qq.shape[0], -1), qq, base.T, alpha=-2.0)
        cand = s.topk(short, dim=1, largest=False).indices
        del s
        xb = base[cand].double()
        dd = ((xb - qq.double()[:, None, :]) ** 2).sum(2)
        o = dd.argsort(dim=1, stable=True)[:, :width]
        gt.append(torch.gather(cand, 1, o).cpu().numpy())
        if (q0 // qchunk) % 20 == 19:
            log(f"ground truth: {q0 + qq.shape[0]} / {nq} queries")
    return np.concatenate(gt)


def bench_streaming(args):
    os.environ.setdefault("JHQ_VERBOSE", "1")
    import torch
    import jhq_gpu_amd as jg
    dev = torch.device("cuda:0")
    seed = args.seed if args.seed is not None else 0x4A48510005
    sc = args.scale
    N0, NINS, INS_B = int(10_000_000 * sc), int(1_000_000 * sc), 10_000
    D, NQ, M, K, BATCH, NCOMP = 768, 10_000, 96, 100, 128, 10_000
    NLIST = 8192 if sc >= 1.0 else max(64, int(8192 * sc))
    npb = int((args.nprobe or "32").split(",")[0])
    alpha = float((args.alpha or "4").split(",")[0])

    t0 = time.time()
    base, means, scales = gen_mixture_chunks(torch, dev, N0 + NINS, D, NCOMP, seed)
    q, _, _ = gen_mixture(torch, dev, NQ, D, NCOMP, seed + 0x100, means, scales)
    torch.cuda.synchronize()
    hb = base.cpu().numpy()
    log(f"data N0={N0} inserts={NINS} D={D} gen+copy {time.time() - t0:.1f}s")

    p = jg.Params(M=M, B=8, Br=4, alpha=alpha, nlist=NLIST, nprobe=npb, ivf_iters=8,
                  batch_size=BATCH, seed=42, residual_per_subspace=1)
    ix = jg.JHQGpuIndex(D, p)
    ix.set_scan_kind(args.scan_kind)
    n_train = min(N0, max(100_000, 16 * NLIST))
    t0 = time.time()
    ix.train(hb[:n_train])
    t_train = time.time() - t0
    t0 = time.time()
    ix.add(hb[:N0])
    t_add = time.time() - t0
    log(f"train n={n_train} {t_train:.1f}s, initial add {t_add:.1f}s")
    ix.reserve(K)  # device searches with k=100 run in the reserved workspace

    out_d = torch.empty((NQ, K), dtype=torch.float32, device=dev)
    out_i = torch.empty((NQ, K), dtype=torch.int32, device=dev)
    nb = (NQ + BATCH - 1) // BATCH
    # interleave: one insert batch, then one search batch
    t_ins = t_srch = 0.0
    nsearched = 0
    upto = N0
    t_all = time.time()
    for it in range(NINS // INS_B):
        t0 = time.time()
        ix.append(hb[upto:upto + INS_B])
        t_ins += time.time() - t0
        upto += INS_B
        b = it % nb
        q0, q1 = b * BATCH, min(NQ, b * BATCH + BATCH)
        t0 = time.time()
        ix.search_device(q[q0:q1], K, out_d[q0:q1], out_i[q0:q1])
        torch.cuda.synchronize()
        t_srch += time.time() - t0
        nsearched += q1 - q0
    t_all = time.time() - t_all
    nbatches = NINS // INS_B
    log(f"streaming: {nbatches} inserts of {INS_B} in {t_ins:.2f}s "
        f"({NINS / max(t_ins, 1e-9):.0f} vectors/s), {nsearched} queries in {t_srch:.3f}s")
    del hb

    W = args.warmup if args.warmup > 0 else 1
    Kst = args.steps if args.steps > 0 else 3
    qps, ms, ev_ms = timed_search(torch, ix, q, out_d, out_i, K, BATCH, W, Kst)
    t0 = time.time()
    gt = ground_truth_f32(torch, base, q)
    log(f"ground truth {time.time() - t0:.1f}s")
    ids = out_i.cpu().numpy()
    rec10 = recall_at(ids, gt, 10)
    rec100 = recall_at(ids, gt, 100)
    log(f"timed steps={Kst} qps={qps:.0f} ms/step={ms:.4f} recall@10={rec10:.4f} "
        f"recall@100={rec100:.4f}")
    step_us = step_times(torch, ix, q, out_d, out_i, K, BATCH)
    log("per-batch us: " + " ".join(f"{k2}={v:.1f}" for k2, v in step_us.items()))
    roof = step_roofline(ix, q.cpu().numpy(), K, BATCH, step_us, ev_ms, "cfg5", npb, alpha,
                         use_profiles=sc == 1.0)
    used, cap = ix.pool()
    line = {
        "metric": "QPS after streaming add (11Mx768 IVF, nprobe 32, k=100, batch 128); "
                  "ADC-scan HBM GB/s vs peak",
        "value": round(qps, 1), "unit": "queries/s", "n_gpus": 1, "steps": Kst, "warmup": W,
        "ms_per_step": round(ms, 5), "ms_per_step_hip_events": round(ev_ms, 5),
        "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: seeded 10k-component Gaussian mixture, L2-normalised (torch Philox)",
        "config": {
            "workload": f"cfg5 streaming: N0={N0} + {NINS} appends of {INS_B} interleaved with "
                        f"{BATCH}-query searches, D=768, nlist={NLIST}, M=96 per-subspace "
                        f"residual codebooks, alpha={alpha:g}, k=100",
            "N_final": upto, "nq": NQ, "nlist": NLIST, "nprobe": npb, "alpha": alpha, "k": K,
            "batch": BATCH, "n_train": n_train,
            "recall_at_10": round(rec10, 4), "recall_at_100": round(rec100, 4),
            "streaming": {"insert_batches": nbatches, "insert_vectors_per_s":
                          round(NINS / max(t_ins, 1e-9), 1),
                          "insert_ms_per_batch": round(t_ins * 1000 / max(nbatches, 1), 3),
                          "search_qps_interleaved": round(nsearched / max(t_srch, 1e-9), 1),
                          "wall_s": round(t_all, 2)},
            "build_s": {"train": round(t_train, 2), "initial_add": round(t_add, 2)},
            "pool_slots": [used, cap],
            "step_us_per_batch": {k2: round(v, 2) for k2, v in step_us.items()},
        },
        "roofline": roof,
        "cpu_baseline": None,
    }
    return line


def trace_mode(torch, dev, ix, q, k, batch, nprobe, alpha, nsteps):
    """The headline's timed step alone, for a kernel trace: one warmup and
    `nsteps` device searches over all of q (batches pipelined on the lanes),
    each bracketed by a host synchronisation so the trace shows whole calls."""
    ix.set_nprobe(nprobe)
    ix.set_alpha(alpha)
    nq = q.shape[0]
    out_d = torch.empty((nq, k), dtype=torch.float32, device=dev)
    out_i = torch.empty((nq, k), dtype=torch.int32, device=dev)
    ix.search_device(q, k, out_d, out_i)
    torch.cuda.synchronize()
    ms = []
    for _ in range(nsteps):
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        ix.search_device(q, k, out_d, out_i)
        ev1.record()
        torch.cuda.synchronize()
        ms.append(ev0.elapsed_time(ev1))
    print(json.dumps({"trace_steps": nsteps, "nprobe": nprobe, "alpha": alpha, "nq": nq,
                      "batches_per_step": (nq + batch - 1) // batch,
                      "scan_kernel": ix.scan_plan(k)[0],
                      "ms_per_step_hip_events": [round(x, 4) for x in ms]}), flush=True)


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


def cpu_info():
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        threads = len(os.sched_getaffinity(0))
    except AttributeError:
        threads = os.cpu_count() or 1
    return model, threads


def verify_sample(po, ix, L, cb, x_sample, n_assign, T):
    """The GPU-built lists against the oracle on the first len(x_sample) vectors
    (ids 0 ..): primary codes, residual codes and corrections bit for bit, and
    the IVF list of the first n_assign of them (the oracle's assignment is the
    expensive part at 65 536 lists)."""
    t0 = time.time()
    po.set_threads(T)
    pp = ix.params
    ids = L["ids"]
    pos = np.empty(ids.size, np.int64)
    pos[ids] = np.arange(ids.size, dtype=np.int64)
    ns = x_sample.shape[0]
    p = pos[:ns]
    y = po.rotate(cb["P"], np.ascontiguousarray(x_sample, np.float32))
    codes = po.primary_encode(y, pp.M, cb["c1d"])
    res, corr = po.residual_encode(y, codes, pp.M, cb["c1d"], cb["res_c1d"], pp.Br)
    bad_codes = int((L["codes"][p] != codes).any(1).sum())
    bad_res = int((L["res"][p] != res).any(1).sum())
    bad_corr = int((L["corr"][p].view(np.uint32) != corr.view(np.uint32)).sum())
    na = min(n_assign, ns)
    asg = po.assign(y[:na], cb["centroids"], cb["cent_norms"])
    lst = np.searchsorted(L["offsets"], p[:na], side="right") - 1
    bad_asg = int((lst != asg).sum())
    ok = bad_codes == 0 and bad_res == 0 and bad_corr == 0 and bad_asg == 0
    log(f"build check: {ns} vectors, codes/res/corr mismatches {bad_codes}/{bad_res}/{bad_corr}, "
        f"list mismatches {bad_asg} of {na} ({time.time() - t0:.1f}s)")
    return {"vectors_checked": ns, "assignments_checked": na, "bit_exact": ok,
            "mismatched_codes": bad_codes, "mismatched_residual_codes": bad_res,
            "mismatched_corrections": bad_corr, "mismatched_lists": bad_asg,
            "note": "ids 0.. of the GPU-built index against the oracle's rotation, encode and "
                    "assignment of the same input rows"}


def cpu_baseline(ix, nprobe, alpha, hq, k, gpu_ids, seconds, train_x=None, nlist=None,
                 n_train=None, x_sample=None, n_assign=10_000):
    """The reference's CPU path as the oracle restates it (scalar C, test
    infrastructure): host train on a bounded sample, then search on the
    GPU-built index, one query at a time on one thread and over all host
    threads.  Also measures how often the reference's approximate top-ck
    (4 candidates kept per thread, v14/search.cu:105-195) returns other ids
    than exact selection on the same queries."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as po
    model, T = cpu_info()
    T = max(1, min(T, 64))
    cb = ix.codebooks()
    L = ix.lists()
    pp = ix.params
    pp.nprobe = nprobe
    pp.alpha = alpha
    o = po.OracleIndex.from_state(ix.dim, pp, cb["P"], cb["c1d"], cb["res_c1d"], cb["centroids"],
                                  cb["cent_norms"], L["offsets"], L["ids"], L["codes"], L["res"],
                                  L["corr"])
    check = None
    if x_sample is not None:
        check = verify_sample(po, ix, L, cb, x_sample, n_assign, T)
    budget = max(1.0, seconds / 3.0)
    # 1. search, one query at a time on one thread
    po.set_threads(1)
    n1, ids1 = 0, []
    t0 = time.time()
    while n1 < hq.shape[0] and (time.time() - t0) < budget:
        _, i1 = o.search(hq[n1:n1 + 1], k)
        ids1.append(i1[0])
        n1 += 1
    dt1 = time.time() - t0
    qps1 = n1 / dt1
    # 2. search over T threads (queries in parallel), about the same budget
    nT = int(min(hq.shape[0], max(T, qps1 * T * budget)))
    po.set_threads(T)
    t0 = time.time()
    _, idsT = o.search(hq[:nT], k)
    dtT = time.time() - t0
    qpsT = nT / dtT
    same = float(np.mean([len(set(a) & set(b)) / k for a, b in zip(idsT, gpu_ids[:nT])]))
    # 3. the reference's approximate selection on the same queries
    _, idsA = o.search(hq[:nT], k, mode=1)
    q_diff = float(np.mean([set(a) != set(b) for a, b in zip(idsA, idsT)]))
    id_diff = float(np.mean([1.0 - len(set(a) & set(b)) / k for a, b in zip(idsA, idsT)]))
    # 4. host train (the oracle's restatement of the reference's train) on a
    # bounded sample: rotation QR, sigma, Lloyd-Max codebook, rotation of the
    # sample, IVF k-means with the lists scaled to the sample, residual 1-D k-means
    ns = nl_s = 0
    t_train = None
    if train_x is not None:
        ns = min(train_x.shape[0], 10_000)
        nl_s = max(1, int(round(nlist * ns / max(n_train, 1))))
        t0 = time.time()
        ot = po.OracleIndex(ix.dim, M=pp.M, B=pp.B, Br=pp.Br, alpha=alpha, nlist=nl_s,
                            nprobe=min(nprobe, nl_s), ivf_iters=pp.ivf_iters, seed=pp.seed)
        ot.train(np.ascontiguousarray(train_x[:ns], np.float32))
        t_train = time.time() - t0
    po.set_threads(1)
    log(f"cpu baseline: 1 thread {qps1:.1f} q/s ({n1} queries), {T} threads {qpsT:.1f} q/s "
        f"({nT} queries), id overlap with GPU {same:.4f}; reference approximate top-ck "
        f"differs on {q_diff:.4f} of queries ({id_diff:.5f} of ids); "
        + (f"train sample n={ns} nlist={nl_s}: {t_train:.1f}s on {T} threads; "
           if t_train is not None else "") + f"cpu {model}")
    return {
        "value": round(qpsT, 2),
        "unit": "queries/s",
        "cores": T,
        "kind": "port",
        "sample": f"first {nT} of the queries over {T} threads (and the first {n1} one at a "
                  f"time on 1 thread), nprobe={nprobe}, alpha={alpha:g}, oracle search on the "
                  f"GPU-built index (id overlap with GPU {same:.4f})",
        "single_thread_qps": round(qps1, 2),
        "cpu_model": model,
        "host_threads": T,
        "train_s": None if t_train is None else round(t_train, 2),
        "train_sample": (f"n_train={ns}, nlist={nl_s}, ivf_iters={pp.ivf_iters}, {T} threads"
                         if t_train is not None else None),
        "build_check": check,
        "reference_approx_topck": {
            "queries_with_other_ids": round(q_diff, 5),
            "ids_differing": round(id_diff, 6),
            "note": "the reference's scan keeps 4 candidates per thread (v14/search.cu:116,"
                    "153-161) then block-argmin; measured by the oracle in that mode against "
                    "exact selection on the same queries and index",
        },
    }


if __name__ == "__main__":
    main()
