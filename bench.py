"""Routed-expert layer benchmark on one MI355X.

Headline workload ("c2"): one MoE FFN layer, decode
batch 1, hidden 4096, expert FFN 1536, 128 experts, top-8 softmax routing,
gate/up Q2_K, down Q3_K, activations quantized to Q8_K.  A step is one full
layer forward (router -> Q8_K -> bucketing -> gate/up+SwiGLU -> down ->
weighted top-k sum) with fresh router logits (new expert ids) every step,
cycling over layer replicas so the working set exceeds the 256 MB
Infinity Cache; inputs are resident in HBM before the timed region.

Prints ONE JSON line.  The other configurations are reported under
"extras" (c1, c3 prefill tok/s, c4, c5 at S=1 and S=64, and the expert-record
unpack at c2's expert shape).  cpu_baseline times the CPU
restatement of ggml's MUL_MAT_ID layer (oracle/) on this host.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "routed-expert layer µs + HBM GB/s (% of peak) at batch 1; prefill tok/s"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_OPS = 5.0e15  # MI355X dense int8 MFMA, ops/s
Q2, Q3, Q4, Q5, Q6, IQ2, IQ3X, IQ4X = 10, 11, 12, 13, 14, 16, 18, 23
BB = {Q2: 84, Q3: 110, Q4: 144, Q5: 176, Q6: 210, IQ2: 66, IQ3X: 98, IQ4X: 136}

CONFIGS = {
    # name: H, F, E, K, S, type gate/up, type down, extra
    "c1": dict(H=2048, F=768, E=128, K=8, S=1, tg=Q4, td=Q4),
    "c2": dict(H=4096, F=1536, E=128, K=8, S=1, tg=Q2, td=Q3),
    "c3": dict(H=4096, F=1536, E=128, K=8, S=512, tg=Q4, td=Q4, logit_bias_sd=1.5),
    "c4": dict(H=5120, F=1536, E=160, K=8, S=4, tg=IQ2, td=IQ2),
    "c5": dict(H=7168, F=2048, E=256, K=8, S=1, tg=Q2, td=Q2, gating="sigmoid", n_slots=96, groups=8,
               groups_used=4, norm=True, scale=2.5, F_shared=2048, t_shared=Q4, router_gemv=True),
}
CONFIGS["c5_s64"] = dict(CONFIGS["c5"], S=64)
CONFIGS["q4k_q6k"] = dict(CONFIGS["c2"], tg=Q4, td=Q6)
CONFIGS["c3_q6k"] = dict(CONFIGS["c3"], td=Q6)
CONFIGS["iq4xs"] = dict(CONFIGS["c2"], tg=IQ4X, td=IQ4X)
CONFIGS["c3_iq4xs"] = dict(CONFIGS["c3"], tg=IQ4X, td=IQ4X)
CONFIGS["iq3xxs"] = dict(CONFIGS["c2"], tg=IQ3X, td=IQ3X)
CONFIGS["c3_iq2xxs"] = dict(CONFIGS["c3"], tg=IQ2, td=IQ2)
CONFIGS["c3_q5k"] = dict(CONFIGS["c3"], tg=Q5, td=Q5)
CONFIGS["c3_iq3xxs"] = dict(CONFIGS["c3"], tg=IQ3X, td=IQ3X)
WORKLOAD = {
    "c1": "decode S=1, H=2048 F=768 E=128 top-8 softmax, Q4_K",
    "c2": "decode S=1, H=4096 F=1536 E=128 top-8 softmax, gate/up Q2_K, down Q3_K",
    "c3": "prefill S=512, H=4096 F=1536 E=128 top-8 softmax + per-expert logit bias N(0,1.5), Q4_K",
    "c4": "small batch S=4, H=5120 F=1536 E=160 top-8 softmax, IQ2_XXS",
    "c5": "full block S=1, H=7168 F=2048, 256 routed Q2_K (96 resident slots) + shared Q4_K, sigmoid 8 groups/top-4",
    "iq4xs": "decode S=1 at c2's shape with IQ4_XS gate/up/down",
    "c3_iq2xxs": "prefill S=512 at c3's shape and routing with IQ2_XXS gate/up/down (stand-in grid)",
    "iq3xxs": "decode S=1 at c2's shape with IQ3_XXS gate/up/down (stand-in grid)",
    "c3_iq4xs": "prefill S=512 at c3's shape and routing with IQ4_XS gate/up/down",
    "c3_q5k": "prefill S=512 at c3's shape and routing with Q5_K gate/up/down",
    "c3_iq3xxs": "prefill S=512 at c3's shape and routing with IQ3_XXS gate/up/down (stand-in grid)",
    "c3_q6k": "prefill S=512 at c3's shape and routing with a Q6_K down projection (mixed-type layer)",
    "q4k_q6k": "decode S=1 at c2's shape with Q4_K gate/up and a Q6_K down projection (mixed-type layer)",
    "c5_s64": "full block S=64, H=7168 F=2048, 256 routed Q2_K (96 resident slots) + shared Q4_K, sigmoid 8 groups/top-4",
}


def row_bytes(t, n):
    return (n // 256) * BB[t]


def dev_random_blocks(torch, t, rows, n, gen, scale=0.02):
    """Random valid quantized rows built on the device (random bytes, finite
    fp16 scale fields of sensible size)."""
    nb = n // 256
    raw = torch.randint(0, 256, (rows, nb, BB[t]), dtype=torch.uint8, device="cuda", generator=gen)

    def put(off, lo, hi):
        v = (torch.rand((rows, nb), device="cuda", generator=gen) * (hi - lo) + lo).to(torch.float16)
        raw[:, :, off:off + 2] = v.view(torch.uint8).view(rows, nb, 2)

    if t == Q2:
        put(80, 0.5 * scale / 20, 1.5 * scale / 20)
        put(82, 0.5 * scale / 8, 1.5 * scale / 8)
    elif t == Q3:
        put(108, 0.5 * scale / 40, 1.5 * scale / 40)
    elif t == Q4:
        put(0, 0.5 * scale / 200, 1.5 * scale / 200)
        put(2, 0.5 * scale / 60, 1.5 * scale / 60)
    elif t == Q5:
        put(0, 0.5 * scale / 400, 1.5 * scale / 400)
        put(2, 0.5 * scale / 60, 1.5 * scale / 60)
    elif t == Q6:
        put(208, 0.5 * scale / 2000, 1.5 * scale / 2000)
    elif t == IQ4X:
        put(0, 0.5 * scale / 2000, 1.5 * scale / 2000)
    elif t == IQ3X:
        put(0, 0.5 * scale / 150, 1.5 * scale / 150)
    else:
        put(0, 0.5 * scale / 40, 1.5 * scale / 40)
    return raw.view(rows, nb * BB[t])


def expert_bytes(c):
    return c["F"] * row_bytes(c["tg"], c["H"]) * 2 + c["H"] * row_bytes(c["td"], c["F"])


def build_layers(torch, Z, c, replicas, seed):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    NS = c.get("n_slots") or c["E"]
    layers = []
    for r in range(replicas):
        wg = dev_random_blocks(torch, c["tg"], NS * c["F"], c["H"], gen).view(NS, c["F"], -1)
        wu = dev_random_blocks(torch, c["tg"], NS * c["F"], c["H"], gen).view(NS, c["F"], -1)
        wd = dev_random_blocks(torch, c["td"], NS * c["H"], c["F"], gen).view(NS, c["H"], -1)
        kw = {}
        if c.get("logit_bias_sd"):
            kw["logit_bias"] = torch.randn(c["E"], device="cuda", generator=gen) * c["logit_bias_sd"]
        if c.get("n_slots"):
            perm = torch.randperm(c["E"], device="cuda", generator=gen)
            rmap = torch.full((c["E"],), -1, dtype=torch.int32, device="cuda")
            rmap[perm[:NS]] = torch.arange(NS, dtype=torch.int32, device="cuda")
            kw["route_map"] = rmap
        if c.get("router_gemv"):
            kw["router_w"] = torch.randn((c["E"], c["H"]), device="cuda", generator=gen) * 0.02
        if c.get("F_shared"):
            ts, Fs = c["t_shared"], c["F_shared"]
            kw.update(F_shared=Fs, type_shared=ts, ws_gate=dev_random_blocks(torch, ts, Fs, c["H"], gen),
                      ws_up=dev_random_blocks(torch, ts, Fs, c["H"], gen),
                      ws_down=dev_random_blocks(torch, ts, c["H"], Fs, gen))
        layers.append(Z.MoELayer(H=c["H"], F=c["F"], n_experts=c["E"], topk=c["K"], type_gate=c["tg"],
                                 type_up=c["tg"], type_down=c["td"], w_gate=wg, w_up=wu, w_down=wd,
                                 gating=c.get("gating", "softmax"), n_groups=c.get("groups", 0),
                                 n_groups_used=c.get("groups_used", 0), weights_norm=c.get("norm", False),
                                 weights_scale=c.get("scale", 0.0), **kw))
    return layers


def run_config(torch, Z, name, steps, warmup, replicas, use_graph=True, kernel_launches=0):
    c = CONFIGS[name]
    S, H, E, K = c["S"], c["H"], c["E"], c["K"]
    layers = build_layers(torch, Z, c, replicas, seed=1234)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(99)
    total = steps + warmup
    xs = torch.randn((replicas, S, H), device="cuda", generator=gen)
    logits = torch.randn((total, S, E), device="cuda", generator=gen)
    out = torch.empty((S, H), device="cuda")
    ids = torch.empty((total, S, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((total, S, K), dtype=torch.float32, device="cuda")
    use_logits = not c.get("router_gemv")
    for L in layers:  # workspaces allocated before timing
        L.workspace(S, xs.device)

    def step(i):
        L = layers[i % replicas]
        L.forward(xs[i % replicas], logits[i] if use_logits else None, out=out, ids=ids[i], weights=wts[i])

    # Every step is a launch sequence recorded once into a HIP graph (the
    # layer's kernels take device pointers only), so the timed region measures
    # the device, not Python's per-call dispatch.  Warm-up steps run eagerly.
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    graph = None
    if use_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(warmup, total):
                step(i)
        graph.replay()  # first replay settles the graph's resources; not timed
        torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    if graph is not None:
        graph.replay()
    else:
        for i in range(warmup, total):
            step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / steps
    check_status(layers, S, name)
    # algorithmic bytes: each touched resident expert's gate+up+down once, plus
    # shared expert, fp32 router and f32 activations in/out
    ids_h = ids[warmup:].cpu().numpy().reshape(steps, -1)
    eb = expert_bytes(c)
    uniq = [len(set(int(v) for v in row if v >= 0)) for row in ids_h]
    mean_uniq = sum(uniq) / len(uniq)
    extra_bytes = 2 * S * H * 4 + S * E * 4
    if c.get("F_shared"):
        extra_bytes += c["F_shared"] * row_bytes(c["t_shared"], H) * 2 + H * row_bytes(c["t_shared"], c["F_shared"])
    if c.get("router_gemv"):
        extra_bytes += E * H * 4
    bytes_step = mean_uniq * eb + extra_bytes
    gbs = bytes_step / (ms * 1e-3) / 1e9
    res = dict(us_per_layer=ms * 1e3, ms_per_step=ms, GBps=gbs, frac_hbm_peak=gbs / HBM_PEAK_GBS,
               bytes_per_layer=bytes_step, unique_experts=mean_uniq, tok_per_s=S / (ms * 1e-3),
               wall_s=wall, replicas=replicas)
    if S >= 32:
        # algorithmic int8 ops (2 per multiply-add; gate, up and down of every
        # routed pair, plus the shared expert) against the dense int8 MFMA peak
        pairs = float((ids[warmup:] >= 0).sum().item()) / steps
        ops = 2 * 3 * H * c["F"] * pairs + (2 * 3 * H * c["F_shared"] * S if c.get("F_shared") else 0)
        res.update(int8_ops_per_layer=ops, int8_TOPs=ops / (ms * 1e-3) / 1e12,
                   mfma_frac=ops / (ms * 1e-3) / INT8_PEAK_OPS)
    if kernel_launches:
        res["kernel_us"] = time_launches(torch, step, warmup, min(steps, kernel_launches))
        check_status(layers, S, name)
    return res


def check_status(layers, S, name):
    """Every layer replica's error word after a timed region: a decode launch
    whose bounded wait expired writes NaN rows instead of results, and a
    number measured over such launches is not reported."""
    bad = {i: st for i, L in enumerate(layers) if (st := L.status(S)) != 0}
    if bad:
        print(f"bench.py: {name}: decode wait expired on layer replicas {bad}; no result is reported",
              file=sys.stderr)
        sys.exit(3)


def time_launches(torch, step, first, n):
    """Mean device time of one layer launch: a HIP event pair on the stream the
    library launches on (torch's current stream) around n back-to-back
    launches, queued behind a spin kernel so Python's dispatch never leaves the
    device idle between them.  For a layer that is one kernel (decode with
    given logits) this is that kernel's average duration, launch gaps included,
    as rocprofv3's kernel trace reports it."""
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    torch.cuda._sleep(50_000_000)  # spin ahead of the queue (long enough for n host dispatches)
    e0.record(stream)
    for i in range(n):
        step(first + i)
    e1.record(stream)
    torch.cuda.synchronize()
    return {"mean": e0.elapsed_time(e1) * 1e3 / n, "launches": n}


def run_unpack(torch, Z, steps, warmup, records=32):
    """Expert-record unpack at c2's expert shape: `records` [gate|up|down]
    records (6.83 MB each) split into the planar expert tensors by one
    launch_ggml_moe_unpack_scatter call (slots in reverse order).  Bytes moved =
    2 x record bytes (each read once, written once); a same-size device copy
    (hipMemcpyAsync via torch) is timed beside it as the practical ceiling."""
    c = CONFIGS["c2"]
    H, F = c["H"], c["F"]
    parts = (F * row_bytes(c["tg"], H), F * row_bytes(c["tg"], H), H * row_bytes(c["td"], F))
    rec = sum(parts)
    src = torch.randint(0, 256, (records * rec,), dtype=torch.uint8, device="cuda")
    dst = [torch.empty(records * p, dtype=torch.uint8, device="cuda") for p in parts]
    slots = torch.arange(records - 1, -1, -1, dtype=torch.int32, device="cuda")
    flat = torch.empty_like(src)

    def unpack(_):
        Z.moe_unpack(src, *dst, records, rec, parts, slots=slots)

    def copy(_):
        flat.copy_(src)

    for i in range(warmup):
        unpack(i)
        copy(i)
    n = max(20, steps)
    t_u = time_launches(torch, unpack, 0, n)["mean"]
    t_c = time_launches(torch, copy, 0, n)["mean"]
    moved = 2 * records * rec
    return {"us": t_u, "GBps": moved / (t_u * 1e-6) / 1e9, "frac": moved / (t_u * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "copy_us": t_c, "copy_GBps": moved / (t_c * 1e-6) / 1e9, "bytes_moved": moved, "records": records,
            "workload": f"unpack {records} c2 expert records (Q2_K gate/up, Q3_K down, {rec} B each) to planar "
                        f"tensors via the slot table"}


def cpu_baseline(seconds: float = 10.0):
    """Restatement of the reference's CPU expert path (ggml CPU MUL_MAT_ID on
    AVX-512: serial Q8_K of x on one thread, OpenMP over the output rows of
    gate+up and of down, one VNNI vec_dot per row; oracle/zm_oracle.c,
    zmo_moe_forward_fast, bit-identical to the oracle) at the c2 shape, S=1,
    on this host's cores: ids re-drawn every iteration over all 128 experts
    of the layer (875 MB of weights, beyond any host cache)."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import zm_oracle as O

    c = CONFIGS["c2"]
    H, F, K = c["H"], c["F"], c["K"]
    pool = c["E"]
    Wg = O.random_blocks(Q2, pool * F, H, seed=1).reshape(pool, F, -1)
    Wu = O.random_blocks(Q2, pool * F, H, seed=2).reshape(pool, F, -1)
    Wd = O.random_blocks(Q3, pool * H, F, seed=3).reshape(pool, H, -1)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, H)).astype(np.float32)
    # the GPU box's CPU share is 16 threads (OMP_NUM_THREADS there); never more
    threads = max(1, min(16, int(os.environ.get("OMP_NUM_THREADS", "16")), os.cpu_count() or 1))
    w = np.full((1, K), 1.0 / K, np.float32)
    avx = O.has_avx512()

    def one():
        ids = rng.permutation(pool)[:K][None].astype(np.int32)
        O.moe_forward(x, ids, w, Q2, Q2, Q3, Wg, Wu, Wd, nthreads=threads, fast=True)

    one()
    n, t0 = 0, time.perf_counter()
    while True:
        one()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds and n >= 3:
            break
    us = el / n * 1e6
    gbs = K * expert_bytes(c) / (us * 1e-6) / 1e9
    return {"value": round(us, 1), "unit": "us/layer", "GBps": round(gbs, 2), "cores": threads, "kind": "port",
            "nproc": os.cpu_count(), "avx512_vnni": avx,
            "sample": f"c2 layer S=1 (8 of the layer's {pool} experts per iteration, {pool * expert_bytes(c) / 1e6:.0f} MB), "
                      f"{n} iterations in {el:.1f} s; "
                      f"restatement of the reference CPU path ({'AVX-512 VNNI' if avx else 'scalar, no AVX-512 on this host'} "
                      f"Q2_K/Q3_K dots, serial Q8_K, OpenMP over output rows, {threads} threads of nproc={os.cpu_count()})"}


PMC_SUMMARY = os.path.join(ROOT, "profiles", "k_moe_decode_c2_hbm_traffic.txt")
COPY_PROBE_BYTES = 1 << 30


def copy_probe(torch):
    """A plain device copy of known size (1 GiB read + 1 GiB written): the
    scale for the FETCH_SIZE / WRITE_SIZE counters."""
    a = torch.ones(COPY_PROBE_BYTES // 4, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()


def _read_counters(d):
    """{(kernel name, counter): [value per dispatch]} from a rocprofv3 --pmc csv."""
    import csv
    import glob

    out = {}
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                out.setdefault((r["Kernel_Name"], r["Counter_Name"]), []).append(float(r["Counter_Value"]))
    return out


def pmc_summary(fetch_dir, write_dir, out_path, command, label="c2", pattern="k_moe_decode"):
    """Per-launch HBM traffic of one kernel (name containing `pattern`) from
    FETCH_SIZE / WRITE_SIZE (KiB per dispatch), each scaled by what the counter
    reads for the copy probe."""
    lines = [f"# HBM traffic per launch: {pattern}, {label} (bench.py --profile {label})", f"# command: {command}"]
    tot = 0.0
    for ctr, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        vals = _read_counters(d)
        dec = [v for (k, c), vs in vals.items() if c == ctr and pattern in k for v in vs]
        cp = [v for (k, c), vs in vals.items() if c == ctr and "copy" in k.lower() for v in vs]
        cp = [v for v in cp if v >= 0.9 * max(cp, default=0.0)]  # the 1 GiB probe, not smaller copies
        if not dec or not cp:
            raise SystemExit(f"pmc_summary: no {ctr} samples for {pattern} or the copy probe in {d}")
        probe = sum(cp) / len(cp)
        factor = (COPY_PROBE_BYTES / 1024) / probe
        kib = sum(dec) / len(dec)
        b = kib * 1024 * factor
        tot += b
        lines += [f"{ctr}_kib_per_launch: {kib:.1f}  (dispatches: {len(dec)})",
                  f"{ctr}_copy_probe_kib: {probe:.1f}  (expected {COPY_PROBE_BYTES // 1024}; factor {factor:.4f})",
                  f"{ctr}_bytes_per_launch: {b:.0f}"]
    lines.append(f"traffic_bytes_per_launch: {tot:.0f}")
    with open(out_path, "w") as fh:
        fh.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def mfma_summary(d, out_path, command, pattern="k_mmq", label="c3", peak_ops=5.0e15):
    """Counters of the kernels whose name contains `pattern` from one rocprofv3
    --pmc run: per kernel, the mean per dispatch of each counter and, when
    SQ_INSTS_VALU_MFMA_MOPS_I8 was collected, the int8 MFMA ops (it counts
    units of 512 ops) and their rate over the dispatch's duration against the
    dense int8 peak."""
    import csv
    import glob
    import re

    per = {}  # kernel -> {counter: [values]}, plus durations
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                if pattern not in r["Kernel_Name"]:
                    continue
                name = re.sub(r"\(.*", "", r["Kernel_Name"].replace("void ", ""))[:60]
                e = per.setdefault(name, {"_dur": {}})
                e.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
                e["_dur"][r["Dispatch_Id"]] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9
    if not per:
        raise SystemExit(f"mfma_summary: no {pattern} dispatches under {d}")
    lines = [f"# counters per dispatch of the {pattern} kernels ({label}, bench.py --profile {label})",
             f"# command: {command}"]
    for name, e in sorted(per.items()):
        durs = list(e.pop("_dur").values())
        dur = sum(durs) / len(durs)
        lines.append(f"{name}: dispatches {len(durs)}, mean duration under counters {dur * 1e6:.1f} us")
        for c, vs in sorted(e.items()):
            lines.append(f"  {c}: {sum(vs) / len(vs):.6g} per dispatch")
        if "SQ_INSTS_VALU_MFMA_MOPS_I8" in e:
            ops = sum(e["SQ_INSTS_VALU_MFMA_MOPS_I8"]) / len(e["SQ_INSTS_VALU_MFMA_MOPS_I8"]) * 512
            lines.append(f"  int8 MFMA ops: {ops / 1e9:.2f} G per dispatch -> {ops / dur / 1e12:.1f} TOP/s = "
                         f"{ops / dur / peak_ops:.4f} of {peak_ops / 1e15:.1f} POP/s")
    with open(out_path, "w") as fh:
        fh.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def stats_summary(d, out_path, command, top=8):
    """Top kernels of a rocprofv3 --kernel-trace --stats run, as text."""
    import csv
    import glob
    import re

    f = glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True)
    if not f:
        raise SystemExit(f"stats_summary: no kernel_stats.csv under {d}")
    with open(f[0]) as fh:
        rows = list(csv.DictReader(fh))
    lines = [f"# rocprofv3 kernel stats", f"# command: {command}",
             f"{'calls':>6} {'avg_us':>9} {'min_us':>9} {'max_us':>9} {'pct':>6}  kernel"]
    for r in rows[:top]:
        name = re.sub(r"\(.*", "", r["Name"].replace("void ", "").replace("(anonymous namespace)::", ""))[:100]
        lines.append(f"{int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:9.2f} {float(r['MinNs']) / 1e3:9.2f} "
                     f"{float(r['MaxNs']) / 1e3:9.2f} {float(r['Percentage']):6.2f}  {name}")
    with open(out_path, "w") as fh:
        fh.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def committed_traffic():
    try:
        with open(PMC_SUMMARY) as fh:
            for l in fh:
                if l.startswith("traffic_bytes_per_launch:"):
                    return float(l.split()[1])
    except OSError:
        pass
    return None


TRACE_SLOTS = [(0, "workgroup start"), (6, "routing wave done (tables stored)"), (7, "first x-quant worker done"),
               (1, "routed (routing barrier)"), (2, "gate/up rows done (workgroup)"), (3, "hand-off counted"),
               (4, "act quantized in LDS"), (5, "down rows done")]


def trace_summary(torch, Z, name, out_path, command, launches=40):
    """Phase trace of the fused decode kernel (ZEROMOE_TRACE=1: eight s_memrealtime
    stamps per workgroup, 100 MHz): percentiles over workgroups and launches, in us
    from the first workgroup's start of each launch."""
    import ctypes

    import numpy as np

    from zeromoe_amd import _lib

    os.environ["ZEROMOE_TRACE"] = "1"
    c = CONFIGS[name]
    S, H, E = c["S"], c["H"], c["E"]
    layers = build_layers(torch, Z, c, 4, seed=1234)
    xs = torch.randn((S, H), device="cuda")
    out = torch.empty((S, H), device="cuda")
    use_logits = not c.get("router_gemv")
    runs = []
    for it in range(launches + 8):
        lg = torch.randn((S, E), device="cuda") if use_logits else None
        layers[it % 4].forward(xs, lg, out=out)
        torch.cuda.synchronize()
        buf = (ctypes.c_uint64 * (4096 * 8))()
        n = _lib.lib().zm_debug_trace(buf, 4096 * 8)
        t = np.frombuffer(buf, dtype=np.uint64, count=n).reshape(-1, 8).astype(np.int64)
        t = t[t[:, 0] > 0]
        if it >= 8:
            runs.append((t - t[:, 0].min()) / 100.0)
    os.environ.pop("ZEROMOE_TRACE")
    status = [L.status(S) for L in layers]
    R = np.stack(runs)
    lines = [f"# phase trace of the fused decode kernel, {name} ({WORKLOAD[name]})",
             f"# command: {command}",
             f"# {R.shape[0]} launches x {R.shape[1]} workgroups; us from the first workgroup's start; status {status}",
             f"{'phase':36s} {'p10':>7s} {'p50':>7s} {'p90':>7s} {'max':>7s}"]
    for sl, label in TRACE_SLOTS:
        v = R[:, :, sl].ravel()
        lines.append(f"{label:36s} {np.percentile(v, 10):7.2f} {np.percentile(v, 50):7.2f} "
                     f"{np.percentile(v, 90):7.2f} {v.max():7.2f}")
    d = (R[:, :, 2] - R[:, :, 1]).ravel()
    lines.append(f"{'gate/up duration (done - routed)':36s} {np.percentile(d, 10):7.2f} {np.percentile(d, 50):7.2f} "
                 f"{np.percentile(d, 90):7.2f} {d.max():7.2f}")
    text = "\n".join(lines) + "\n"
    with open(out_path, "w") as f:
        f.write(text)
    print(text, end="")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--replicas", type=int, default=0, help="layer replicas (0 = enough to exceed the MALL)")
    ap.add_argument("--extras", default="c1,c3,c4,c5,c5_s64,q4k_q6k,c3_q6k,iq4xs,c3_iq4xs,iq3xxs,c3_iq2xxs", help="extra configs to report ('' for none)")
    ap.add_argument("--no-unpack", dest="unpack", action="store_false",
                    help="skip the expert-record unpack extra")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true", help="launch every step from Python instead of a HIP graph")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--profile", metavar="CFG", help="profiling run: CFG's layer launched eagerly --steps times, "
                    "then a 1 GiB copy probe; prints a short summary (for rocprofv3)")
    ap.add_argument("--pmc-summary", nargs=3, metavar=("FETCH_DIR", "WRITE_DIR", "OUT"),
                    help="summarize two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of --profile c2")
    ap.add_argument("--stats-summary", nargs=2, metavar=("DIR", "OUT"), help="summarize a rocprofv3 --stats run")
    ap.add_argument("--mfma-summary", nargs=2, metavar=("DIR", "OUT"),
                    help="int8 MFMA utilisation of the prefill kernels from a rocprofv3 --pmc run of --profile c3")
    ap.add_argument("--trace", nargs=2, metavar=("CFG", "OUT"),
                    help="phase trace of CFG's fused decode kernel (percentiles over workgroups) into OUT")
    ap.add_argument("--command", default="", help="command line recorded in a summary")
    ap.add_argument("--label", default="", help="configuration named in a --pmc-summary / --mfma-summary")
    ap.add_argument("--pattern", default="", help="kernel-name pattern of a --pmc-summary / --mfma-summary")
    args = ap.parse_args()
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary, args.command, args.label or "c2", args.pattern or "k_moe_decode")
        return
    if args.stats_summary:
        stats_summary(*args.stats_summary, args.command)
        return
    if args.mfma_summary:
        mfma_summary(*args.mfma_summary, args.command, args.pattern or "k_mmq", args.label or "c3")
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); the expert axis would "
              f"shard across GPUs as described in DESIGN.md, but no multi-GPU figure is produced.", file=sys.stderr)
        sys.exit(2)
    import torch

    import zeromoe_amd as Z

    torch.cuda.set_device(0)
    Z.init()

    def reps(name):
        if args.replicas:
            return args.replicas
        c = CONFIGS[name]
        NS = c.get("n_slots") or c["E"]
        per = NS * expert_bytes(c)
        return max(2, min(16, int(1.2e9 // per) + 2))

    if args.trace:
        trace_summary(torch, Z, args.trace[0], args.trace[1], args.command)
        return
    if args.profile == "unpack":
        r = run_unpack(torch, Z, args.steps, args.warmup)
        print(json.dumps({"profile": "unpack", "us": round(r["us"], 2), "GBps": round(r["GBps"], 1)}))
        return
    if args.profile:
        r = run_config(torch, Z, args.profile, args.steps, args.warmup, reps(args.profile), use_graph=False)
        copy_probe(torch)
        print(json.dumps({"profile": args.profile, "us_per_layer": round(r["us_per_layer"], 2),
                          "bytes_per_layer": int(r["bytes_per_layer"])}))
        return
    main_res = run_config(torch, Z, "c2", args.steps, args.warmup, reps("c2"), use_graph=not args.eager,
                          kernel_launches=100)
    kern = main_res["kernel_us"]
    kern_gbs = main_res["bytes_per_layer"] / (kern["mean"] * 1e-6) / 1e9
    traffic = committed_traffic()
    extras = {}
    for name in [n for n in args.extras.split(",") if n]:
        st = max(10, args.steps // 4) if name in ("c3", "c5_s64", "c3_q6k", "c3_iq4xs", "c3_iq2xxs", "c3_q5k", "c3_iq3xxs") else args.steps
        r = run_config(torch, Z, name, st, max(3, args.warmup // 2), reps(name), use_graph=not args.eager)
        extras[name] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()}
        extras[name]["workload"] = WORKLOAD[name]
    if args.unpack:
        r = run_unpack(torch, Z, args.steps, args.warmup)
        extras["unpack"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()}
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    line = {
        "metric": METRIC,
        "value": round(main_res["GBps"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_res["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (random valid Q2_K/Q3_K blocks, N(0,1) activations and logits)",
        "config": {"workload": "c2: " + WORKLOAD["c2"], "H": 4096, "F": 1536, "experts": 128, "topk": 8,
                   "tokens": 1, "replicas": main_res["replicas"]},
        "us_per_layer": round(main_res["us_per_layer"], 2),
        "roofline": {"bound": "hbm", "kernel": "zm::k_moe_decode<Q2_K,Q3_K> (the whole c2 layer is this one launch)",
                     "achieved": round(kern_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(kern_gbs / HBM_PEAK_GBS, 4),
                     "traffic": None if traffic is None else int(traffic),
                     "algorithmic_bytes_per_launch": int(main_res["bytes_per_layer"]),
                     "kernel_us": {k: (round(v, 2) if isinstance(v, float) else v) for k, v in kern.items()},
                     "traffic_source": "profiles/k_moe_decode_c2_hbm_traffic.txt (rocprofv3 --pmc FETCH_SIZE, "
                                       "WRITE_SIZE, scaled by a 1 GiB copy)"},
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
