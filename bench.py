"""Benchmark: batch-64 paged decode step (append + paged decode attention) on
one MI355X — BASELINE.json config 3.

A step appends one bf16 K/V row per sequence into its page (pkv_append) and
runs paged decode attention over every sequence's context
(pkv_attn_decode: key-range kernel + merge). Contexts are U[512, 8192] per
sequence (fresh seeded mix per run), pages scattered over a 65,536-page pool
(2 GiB of K + 2 GiB of V), Hq 16 / Hkv 4 / head_dim 256, page 16. Step i
appends at position ctx + i and attends ctx + i + 1 keys; the pages for every
step are reserved up front as the reference's admission does.

Prints one JSON line. `value` is the achieved HBM bandwidth of the whole step
in GB/s (algorithmic bytes / measured step time); us_per_step and the
fraction of the 8 TB/s peak ride along. `roofline` is for the dominant kernel
(the key-range decode kernel), timed with HIP events on the launch stream.
`cpu_baseline` times the oracle (a scalar C restatement) on the host.
`roofline.traffic` is the dominant kernel's HBM bytes per launch, from two
short child runs of the same workload under rocprofv3 --pmc (FETCH_SIZE,
WRITE_SIZE), copy-calibrated (--no-traffic skips them).

Other workloads: --config c2 (one sequence at 4096 context), c4 (chunked
prefill over a shared prefix, TFLOP/s), c5 (speculative verify at 32k-128k
context), attn (the reference's bench-attn: one prompt of --tokens tokens
after --context cached keys, the prompt kernel alone).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "pocket-engine_amd"))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA


class HipEvents:
    """Raw hipEvent_t pairs from the process's HIP runtime (the one torch
    loaded), for kernels that record events themselves."""

    def __init__(self, n):
        import ctypes
        self.hip = ctypes.CDLL("libamdhip64.so.7")  # resolves to the already-loaded runtime
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.pairs = []
        for _ in range(n):
            a, b = ctypes.c_void_p(), ctypes.c_void_p()
            assert self.hip.hipEventCreate(ctypes.byref(a)) == 0 and self.hip.hipEventCreate(ctypes.byref(b)) == 0
            self.pairs.append((a.value, b.value))

    def record(self, ev, stream):
        assert self.hip.hipEventRecord(ev, stream) == 0

    def elapsed_ms(self):
        import ctypes
        out = []
        for a, b in self.pairs:
            ms = ctypes.c_float()
            assert self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
            out.append(ms.value)
        return out

    def __del__(self):
        for a, b in getattr(self, "pairs", []):
            self.hip.hipEventDestroy(a)
            self.hip.hipEventDestroy(b)


def measure_traffic(args, seed, algorithmic_bytes, want=None):
    """HBM bytes per launch of the workload's dominant kernel, measured: the
    same workload (same seed, 1 warm-up + 3 steps) runs twice in a child
    process under rocprofv3 --pmc, once per counter (FETCH_SIZE, WRITE_SIZE;
    KiB per dispatch), and each counter is scaled by what it reads for the
    2 GiB device copies the child also runs (2 GiB read, 2 GiB written). The
    dominant kernel is this library's kernel with the largest FETCH_SIZE
    among those whose name holds `want` (any, if None); algorithmic_bytes is
    its per-launch figure over the child's steps 0 .. 3. Returns (bytes per
    launch or None, detail dict)."""
    import csv
    import glob
    import shutil
    import signal
    import subprocess
    import tempfile

    import numpy as np

    if args.no_traffic or args.traffic_child:
        return None, None
    prof = shutil.which("rocprofv3") or ("/opt/rocm/bin/rocprofv3" if os.path.exists("/opt/rocm/bin/rocprofv3")
                                          else None)
    if prof is None:
        return None, {"error": "rocprofv3 not found"}
    child = [sys.executable, "-u", os.path.abspath(__file__), "--traffic-child", "--no-traffic", "--no-cpu",
             "--no-graph", "--steps", "3", "--warmup", "1", "--seed", str(seed), "--config", args.config,
             "--kv", args.kv, "--q-heads", str(args.q_heads), "--batch", str(args.batch), "--pages", str(args.pages),
             "--prefix", str(args.prefix), "--tokens", str(args.tokens), "--context", str(args.context),
             "--seqs", str(args.seqs)]
    for flag in ("unfused", "with_prep", "refabi", "verify_kernel", "prefill_split"):
        if getattr(args, flag):
            child.append("--" + flag.replace("_", "-"))
    if args.wg_per_cu or args.min_range:
        child += ["--wg-per-cu", str(args.wg_per_cu or 1), "--min-range", str(args.min_range or 32)]
    per_kib, name = {}, None
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        out = tempfile.mkdtemp(prefix="pkv_traffic_", dir="/tmp")
        cmd = [prof, "--pmc", ctr, "--output-format", "csv", "-d", out, "-o", "run", "--"] + child
        proc = subprocess.Popen(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"), stdout=subprocess.DEVNULL,
                                stderr=subprocess.DEVNULL, start_new_session=True)
        try:
            proc.wait(timeout=120)
        except subprocess.TimeoutExpired:
            os.killpg(proc.pid, signal.SIGKILL)  # the process group this call started
            proc.wait()
            return None, {"error": f"rocprofv3 --pmc {ctr} run timed out"}
        files = glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True)
        if proc.returncode != 0 or not files:
            return None, {"error": f"rocprofv3 --pmc {ctr} run failed (exit {proc.returncode})"}
        rows = []
        for f in files:
            with open(f, newline="") as fh:
                rows += [r for r in csv.DictReader(fh) if r["Counter_Name"] == ctr]
        shutil.rmtree(out, ignore_errors=True)
        copies = sorted((float(r["Counter_Value"]) for r in rows if "copyBuffer" in r["Kernel_Name"]),
                        reverse=True)[:3]
        mine = {}
        for r in rows:
            k = r["Kernel_Name"]
            if ("pkv::" in k or k.startswith("attn_")) and (want is None or want in k):
                mine.setdefault(k, []).append(float(r["Counter_Value"]))
        if not copies or not mine:
            return None, {"error": f"no copy or library dispatches in the {ctr} run"}
        if name is None:  # the dominant kernel: largest median FETCH_SIZE
            name = max(mine, key=lambda k: float(np.median(mine[k])))
        if name not in mine:
            return None, {"error": f"{name} missing from the {ctr} run"}
        factor = (2 << 30) / (float(np.median(copies)) * 1024)
        per_kib[ctr] = (float(np.median(mine[name])), factor)
    rd = per_kib["FETCH_SIZE"][0] * 1024 * per_kib["FETCH_SIZE"][1]
    wr = per_kib["WRITE_SIZE"][0] * 1024 * per_kib["WRITE_SIZE"][1]
    return rd + wr, {
        "kernel": name.split("(")[0].replace("void ", ""), "read_bytes": round(rd), "write_bytes": round(wr),
        "read_factor": round(per_kib["FETCH_SIZE"][1], 4), "write_factor": round(per_kib["WRITE_SIZE"][1], 4),
        "algorithmic_bytes": round(algorithmic_bytes), "ratio": round((rd + wr) / algorithmic_bytes, 4),
        "source": "rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, over the same workload (same seed, 4 launches) in "
                  "child processes of this run; median per dispatch, scaled by the counter of 2 GiB device copies "
                  "in the same runs"}


def build_parser():
    """The command line of this script (the driver's contract: --gpus,
    --steps, --warmup; the rest selects and shapes the workload)."""
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--seed", type=int, default=None, help="length-mix seed (default: fresh per run)")
    ap.add_argument("--config", default="c3", choices=["c2", "c3", "c4", "c5", "attn"],
                    help="c3 (default, the metric): batch-64 decode step; c2: single-sequence decode at 4096 "
                         "context; c4: chunked prefill of 8 x 2048 tokens over a shared 16,384-token prefix; "
                         "c5: speculative verify of 4 drafts x 16 sequences at 32k..128k context")
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--tokens", type=int, default=4096, help="attn: prompt tokens per sequence")
    ap.add_argument("--context", type=int, default=0, help="attn: cached keys before the prompt")
    ap.add_argument("--seqs", type=int, default=1, help="attn: sequences")
    ap.add_argument("--prefill-split", action="store_true",
                    help="attn: the library through pkv_attn_prefill_split (keys split over workgroups when the "
                         "grid has fewer workgroups than CUs, then a merge launch)")
    ap.add_argument("--prefix", type=int, default=16384,
                    help="c4: shared prefix tokens (a multiple of 64 reaches the sequences through the prefix cache; "
                         "otherwise shared pages with the partial last page copied on write)")
    ap.add_argument("--pages", type=int, default=65536)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--wg-per-cu", type=int, default=None)
    ap.add_argument("--min-range", type=int, default=None)
    ap.add_argument("--no-graph", action="store_true",
                    help="report the eager step only (default: the K steps are also captured into one HIP graph and "
                         "replayed, as the reference engine replays its decode step, and value is the replayed step)")
    ap.add_argument("--passes", type=int, default=5,
                    help="timed passes over the K steps (eager with kernel events, then one graph replay, "
                         "alternating); the reported step and kernel times are medians over the passes")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run kernels of known traffic (2 GiB copy, read-only sum, fill; x3 each), to scale rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--verify-kernel", action="store_true",
                    help="c2/c3 unfused through the verify kernels (pkv_attn_verify) instead of decode")
    ap.add_argument("--refabi", action="store_true",
                    help="c2/c3 through the reference-ABI code object (pkv_kernels.hsaco: attn_paged_g4 + attn_merge "
                         "on the reference engine's grid) after pkv_append")
    ap.add_argument("--kv", default="bf16", choices=["bf16", "e4m3"],
                    help="c2/c3 cache type; e4m3: the step is pkv_attn_prep (E4M3 store) + pkv_attn_decode_e4m3")
    ap.add_argument("--with-prep", action="store_true",
                    help="c2/c3: the step's append is pkv_attn_prep (q/k RMSNorm + rotary + K/V slot writes, the "
                         "reference's attn_prep) on the raw qkv rows, followed by the key ranges and the merge")
    ap.add_argument("--q-heads", type=int, default=16,
                    help="query heads over the 4 kv heads (16: the configs' G = 4; 24: the reference's 27B shape, "
                         "G = 6, whose fused step is the verify kernel with the append fused in)")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the HBM traffic measurement (two short child runs of the same workload under "
                         "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, scaled by 2 GiB device copies in the same runs)")
    ap.add_argument("--traffic-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--no-others", action="store_true",
                    help="default run only: skip the short child runs of the other workloads (c2, c4, c5, bench-attn, "
                         "c3 at 24 query heads, c3 over an E4M3 cache) whose figures go into other_configs (also "
                         "skipped under rocprofv3)")
    ap.add_argument("--unfused", action="store_true",
                    help="append, key ranges and merge as three launches instead of the fused step")
    return ap


def main():
    args = build_parser().parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); the paged KV path shards by "
              "sequence with no exchange, so N-GPU throughput is N x the one-GPU figure. Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    if args.calibrate_copy:
        # Kernels of known traffic for scaling rocprofv3 FETCH_SIZE /
        # WRITE_SIZE: a device copy (reads 2 GiB, writes 2 GiB), an integer
        # sum (reads 2 GiB, writes 8 bytes) and a fill (writes 2 GiB), 3 each.
        src = torch.ones(1 << 30, dtype=torch.int16, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        for _ in range(3):
            src.view(torch.int64).sum()
        for _ in range(3):
            dst.fill_(7)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_bytes": 2 << 30, "copies": 3, "sums": 3, "fills": 3}))
        return

    if args.traffic_child:
        # calibration for the parent's counter runs: 2 GiB device copies
        # (2 GiB read + 2 GiB written each)
        src = torch.ones(1 << 30, dtype=torch.int16, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    import pkv
    from pkv import synth

    if args.config == "c4":
        return bench_prefill(args)
    if args.config == "c5":
        return bench_verify(args)
    if args.config == "attn":
        return bench_attn(args)

    if args.wg_per_cu or args.min_range:
        pkv.attn_decode_config(args.wg_per_cu or 1, args.min_range or 32)
    seed = args.seed if args.seed is not None else int(time.time()) % 100000
    dev = torch.device("cuda:0")
    Hq, Hkv, D, BS = args.q_heads, 4, 256, 16
    G = Hq // Hkv
    B, pages = args.batch, args.pages
    S = args.warmup + args.steps
    if args.config == "c2":
        B, pages = 1, 4096 + (S + 15) // 16 + 1
        lens = np.array([4096])
    else:
        lens = synth.c3_lengths(seed, batch=B)
    meta = synth.decode_meta(lens, pages, steps=S, seed=seed)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    e4m3 = args.kv == "e4m3"
    if e4m3:
        # random E4M3 bytes (NaN codes replaced) and scales amax/448-like
        kc = torch.randint(0, 256, (pages * BS, Hkv, D), device=dev, generator=gen, dtype=torch.int32).to(torch.uint8)
        vc = torch.randint(0, 256, (pages * BS, Hkv, D), device=dev, generator=gen, dtype=torch.int32).to(torch.uint8)
        for t in (kc, vc):
            t[(t & 0x7F) == 0x7F] = 0x7E
        kscale = torch.rand(pages * BS, Hkv, device=dev, generator=gen) * 0.004 + 0.001
        vscale = torch.rand(pages * BS, Hkv, device=dev, generator=gen) * 0.004 + 0.001
        args.with_prep = True
    else:
        kc = torch.empty(pages * BS, Hkv, D, dtype=torch.bfloat16, device=dev)
        vc = torch.empty_like(kc)
        for t in (kc, vc):  # N(0,1) * 0.5, in slices to bound temporaries
            for i in range(0, t.shape[0], 1 << 18):
                t[i:i + (1 << 18)] = torch.randn(t[i:i + (1 << 18)].shape, device=dev, generator=gen) * 0.5
    q = (torch.randn(B, Hq, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    qstride = synth.qkv_stride(Hq, Hkv)
    qkv = (torch.randn(B, qstride, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=dev)
    steps = [meta.step(i) for i in range(S)]
    pos_d = torch.from_numpy(np.stack([s["pos"] for s in steps])).to(dev)
    slot_d = torch.from_numpy(np.stack([s["slot_map"] for s in steps])).to(dev)
    ts = torch.from_numpy(steps[0]["tok_seq"]).to(dev)
    cu = torch.from_numpy(steps[0]["cu"]).to(dev)
    bt = torch.from_numpy(meta.block_table).to(dev)
    ws = torch.empty(max(pkv.attn_decode_workspace(B, Hq), pkv.attn_verify_workspace(B, Hq)), dtype=torch.uint8,
                     device=dev)
    if args.verify_kernel:
        args.unfused = True
    k_rows = qkv.data_ptr() + 2 * (2 * Hq * D)
    v_rows = k_rows + 2 * (Hkv * D)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream


    if args.with_prep:
        args.unfused = True
        qn = (1 + 0.1 * torch.randn(D, device=dev, generator=gen)).float()
        kn = (1 + 0.1 * torch.randn(D, device=dev, generator=gen)).float()
        inv_freq = (1.0 / 1e7 ** (torch.arange(32, device=dev, dtype=torch.float64) * 2 / 64)).float()
        rope_d = pos_d.unsqueeze(1).expand(-1, 3, -1).contiguous()  # [steps][3][B]: text tokens
    rk = None
    if args.refabi:
        from pkv import refabi
        rk = refabi.RefKernels()
        Z = refabi.split_ranges(B, Hkv, torch.cuda.get_device_properties(0).multi_processor_count)
        part = torch.empty(B * Z * Hq * (D + 2), dtype=torch.float32, device=dev) if Z > 1 else None
        P_, I_, F_ = refabi.P, refabi.I, refabi.F

    def step_on(i, strm, ev=None):
        s_ = strm.cuda_stream
        if args.refabi:
            if e4m3:
                pkv.attn_prep(qkv, qstride, Hq, Hkv, qn, kn, rope_d[i], B, 11, 11, slot_d[i], inv_freq, q, kc, vc,
                              1e-6, B, pages * BS, kscale=kscale, vscale=vscale, stream=s_)
            else:
                pkv.append(k_rows, v_rows, qstride * 2, slot_d[i], B, Hkv, D * 2, kc, vc, pages * BS, stream=s_)
            if ev:
                kev.record(ev[0], s_)
            rk.launch(f"attn_paged8_g{G}" if e4m3 else f"attn_paged_g{G}", (B, Hkv, Z), 128 if G >= 6 else 256, 0,
                      [P_(q), P_(kc), P_(vc), P_(kscale if e4m3 else None), P_(vscale if e4m3 else None), P_(qkv), I_(qstride), I_(Hq), I_(Hkv),
                       P_(pos_d[i]), P_(ts), P_(bt), I_(meta.max_blocks), I_(BS), P_(out), F_(1 / 16), P_(None),
                       P_(None), I_(0), I_(0), P_(cu), I_(0), I_(refabi.SPLIT_MIN_KEYS), P_(part), P_(None), I_(1)],
                      stream=s_)
            if ev:
                kev.record(ev[1], s_)
            if part is not None:
                rk.launch("attn_merge", (B, Hq, 1), 256, 0,
                          [P_(part), I_(Z), I_(refabi.SPLIT_MIN_KEYS), P_(qkv), I_(qstride), I_(Hq), P_(pos_d[i]),
                           P_(ts), P_(cu), I_(0), P_(out), P_(None), P_(None), I_(0), I_(0), P_(None), I_(1)],
                          stream=s_)
            return
        if e4m3:
            pkv.attn_prep(qkv, qstride, Hq, Hkv, qn, kn, rope_d[i], B, 11, 11, slot_d[i], inv_freq, q, kc, vc, 1e-6,
                          B, pages * BS, kscale=kscale, vscale=vscale, stream=s_)
            pkv.attn_decode_e4m3(q, kc, vc, kscale, vscale, qkv, qstride, Hq, Hkv, pos_d[i], ts, bt, meta.max_blocks,
                                 BS, out, 1 / 16, cu, 0, None, 1, B, pages, ws, stream=s_)
        elif args.with_prep:
            pkv.attn_prep(qkv, qstride, Hq, Hkv, qn, kn, rope_d[i], B, 11, 11, slot_d[i], inv_freq, q, kc, vc, 1e-6,
                          B, pages * BS, stream=s_)
            pkv.attn_decode(q, kc, vc, qkv, qstride, Hq, Hkv, pos_d[i], ts, bt, meta.max_blocks, BS, out, 1 / 16, cu,
                            0, None, 1, B, pages, ws, stream=s_)
        elif args.unfused:
            pkv.append(k_rows, v_rows, qstride * 2, slot_d[i], B, Hkv, D * 2, kc, vc, pages * BS, stream=s_)
            fn = pkv.attn_verify if args.verify_kernel else pkv.attn_decode
            fn(q, kc, vc, qkv, qstride, Hq, Hkv, pos_d[i], ts, bt, meta.max_blocks, BS, out, 1 / 16, cu,
                            0, None, 1, B, pages, ws, stream=s_)
        else:
            pkv.attn_decode_step(k_rows, v_rows, qstride * 2, slot_d[i], q, kc, vc, qkv, qstride, Hq, Hkv, pos_d[i], ts,
                                 bt, meta.max_blocks, BS, out, 1 / 16, cu, 0, None, 1, B, pages, ws, stream=s_)

    def step(i, ev=None):
        # ev: the key-range kernel records these HIP events at its own start
        # and end (hipExtLaunchKernelGGL), so no dispatch gap is counted.
        if ev and not args.refabi:
            pkv.time_next_range_kernel(ev[0], ev[1])
        step_on(i, stream, ev)

    P = max(1, args.passes)
    kev = HipEvents(args.steps * P)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    g = None
    if not args.no_graph:
        # The same K steps captured into one HIP graph (the reference engine
        # replays a captured graph per step, src/engine.rs:704-720); one
        # untimed replay before the timed passes.
        g = torch.cuda.CUDAGraph()
        cs = torch.cuda.Stream()
        cs.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cs):
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=cs):
                for k in range(args.steps):
                    step_on(args.warmup + k, cs)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
    # P timed passes, each over the same K steps (the appends rewrite the
    # same slots with the same rows, so every pass is the same workload):
    # an eager pass whose events bracket the dominant kernel of every step
    # (the fused step kernel, or the key-range kernel with --unfused), then
    # one replay of the graph, each bracketed by synchronize. Eager and graph
    # passes alternate so the kernel time and the step time are taken under
    # the same clocks; the reported figures are medians over the passes.
    eager_ms, graph_ms, kern_pass_ms, kern_ms = [], [], [], []
    for r in range(P):
        evs = kev.pairs[r * args.steps:(r + 1) * args.steps]
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record(stream)
        for k in range(args.steps):
            step(args.warmup + k, evs[k])
        t1.record(stream)
        torch.cuda.synchronize()
        eager_ms.append(t0.elapsed_time(t1))
        if g is not None:
            g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            g0.record(stream)
            g.replay()
            g1.record(stream)
            torch.cuda.synchronize()
            graph_ms.append(g0.elapsed_time(g1))
    all_kern = kev.elapsed_ms()
    for r in range(P):
        km = all_kern[r * args.steps:(r + 1) * args.steps]
        kern_ms += km
        kern_pass_ms.append(sum(km))
    med = lambda xs: float(np.median(np.asarray(xs)))
    total_ms = med(eager_ms)
    ms_step = total_ms / args.steps
    graph_us = None if g is None else 1e3 * med(graph_ms) / args.steps

    keys = [meta.keys(args.warmup + k) for k in range(args.steps)]
    if e4m3:
        step_bytes = [synth.algorithmic_bytes_decode(kk, B, Hq, Hkv, kv="e4m3") + synth.algorithmic_bytes_append(
            B, Hkv, kv="e4m3") for kk in keys]
    else:
        step_bytes = [synth.algorithmic_bytes_decode(kk, B, Hq, Hkv) + synth.algorithmic_bytes_append(B, Hkv)
                      for kk in keys]
    gbs_eager = sum(step_bytes) / (total_ms * 1e-3) / 1e9
    step_ms = ms_step if graph_us is None else graph_us * 1e-3  # the reported step
    gbs = sum(step_bytes) / (step_ms * args.steps * 1e-3) / 1e9
    if args.unfused or args.refabi:
        # key-range kernel: every key's K and V rows (all kv heads) + q; its
        # partials are overhead, not algorithmic.
        kern_bytes = [kk * Hkv * (D + 4 if e4m3 else D * 2) * 2 + B * Hq * D * 2 for kk in keys]
        kname = (f"attn_paged8_g{G} (reference ABI, E4M3 cache, after attn_prep)" if e4m3 and args.refabi else
                 f"decode_range8_kernel<{G}> (E4M3 cache, after attn_prep)" if e4m3 else
                 f"attn_paged_g{G} (reference ABI)" if args.refabi else
                 f"verify_range_kernel<{G}> (one row per segment)" if G != 4 else
                 "decode_range_kernel<4,false> (after attn_prep)" if args.with_prep else
                 "verify_range_kernel<4>" if args.verify_kernel else "decode_range_kernel<4,false>")
    else:
        kern_bytes = step_bytes  # the fused kernel does the whole step
        kname = (f"decode_range_kernel<4,true>" if G == 4 else f"verify_range_kernel<{G},true>") + \
            " (fused append + key ranges; the merge is a second launch)"
    kern_med_pass_ms = med(kern_pass_ms)  # the median pass's K kernel durations, summed
    kern_avg_us = 1e3 * kern_med_pass_ms / args.steps
    kern_gbs = sum(kern_bytes) / (kern_med_pass_ms * 1e-3) / 1e9

    copy_gbs, read_gbs = hbm_copy_probe(dev)
    # algorithmic bytes of the dominant kernel over the child's steps 0 .. 3
    # (the same formulas as kern_bytes)
    keys0 = [meta.keys(k) for k in range(4)]
    if args.unfused or args.refabi:
        alg0 = [kk * Hkv * (D + 4 if e4m3 else D * 2) * 2 + B * Hq * D * 2 for kk in keys0]
    else:
        alg0 = [synth.algorithmic_bytes_decode(kk, B, Hq, Hkv) + synth.algorithmic_bytes_append(B, Hkv) for kk in keys0]
    traffic, traffic_detail = measure_traffic(args, seed, float(np.mean(alg0)))
    cpu = None
    st0 = steps[args.warmup]
    if not args.no_cpu and args.config == "c3" and not e4m3:
        cpu = cpu_baseline(kc, vc, q, qkv, meta, st0, Hq, Hkv, qstride, dev)
    elif not args.no_cpu:
        # c2: its one row; c3 over E4M3: 16 of the 64 rows (every 4th)
        sample = np.arange(0, B, 4) if B > 1 else np.arange(1)
        cpu = cpu_baseline_rows(kc, vc, q, qkv, meta.block_table, st0["pos"], st0["tok_seq"], Hq, Hkv, qstride,
                                meta.max_blocks, sample, "every 4th sequence" if B > 1 else "the one sequence",
                                kscale=kscale if e4m3 else None, vscale=vscale if e4m3 else None,
                                append_rows=0 if e4m3 else B)

    line = {
        "metric": ("paged decode step us + achieved HBM GB/s (% of peak) at batch 64, 1 MI355X" if args.config == "c3"
                   else "paged decode step us + achieved HBM GB/s (% of peak), one sequence at 4096 context, "
                        "1 MI355X"),
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "us_per_step": round(step_ms * 1e3, 2),
        "pct_of_hbm_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
        "step_timing": (f"eager: median of {P} passes of the K steps" if graph_us is None else
                        f"HIP graph replay of the K steps: median of {P} replays, each alternating with an eager "
                        "pass that times the kernel"),
        "us_per_step_passes": [round(1e3 * x / args.steps, 2) for x in (graph_ms if graph_ms else eager_ms)],
        "kernel_us_passes": [round(1e3 * x / args.steps, 2) for x in kern_pass_ms],
        "us_per_step_eager": round(ms_step * 1e3, 2),
        "gbs_eager": round(gbs_eager, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3 KV (bf16 q/out, f32 accum)" if e4m3 else "bf16",
        "data": ("synthetic (random E4M3 bytes and scales, seeded N(0,1)*0.5 q, U[512,8192] contexts)" if e4m3 else
                 "synthetic (seeded N(0,1)*0.5 K/V/q, U[512,8192] contexts)"),
        "config": {"workload": ("c3: batch-64 paged decode step (append 1 token/seq + paged decode attention)"
                                if args.config == "c3" else
                                "c2: single-sequence paged decode step at 4096 context (append + attention)") +
                               (f", {Hq} query heads over {Hkv} kv heads (G = {G})" if G != 4 else "") +
                               (", E4M3 cache" if e4m3 else ""),
                   "kv": args.kv,
                   "path": ("attn_prep (E4M3 store), key ranges over the E4M3 cache, merge" if e4m3 else
                            f"reference-ABI code object (append, attn_paged_g{G}, attn_merge)" if args.refabi else
                            "attn_prep (norm + rotary + append), key ranges, merge" if args.with_prep else
                            "unfused (append, key ranges, merge)" if args.unfused else
                            "fused step (two launches: append + key ranges, then merge)"),
                   "batch": B, "ctx": "4096" if args.config == "c2" else "U[512,8192]", "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "page": BS,
                   "pool_pages": pages, "seed": seed, "mean_keys_per_step": round(float(np.mean(keys)), 1),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": kname, "achieved": round(kern_gbs, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(kern_gbs / PEAK_HBM_GBS, 4),
                     "avg_us": round(kern_avg_us, 2), "median_us": round(1e3 * float(np.median(kern_ms)), 2),
                     "hbm_copy_probe_gbs": round(copy_gbs, 1), "hbm_read_probe_gbs": round(read_gbs, 1),
                     "frac_of_read_probe": round(kern_gbs / read_gbs, 4),
                     "traffic": None if traffic is None else round(traffic),
                     "traffic_detail": traffic_detail},
        "cpu_baseline": cpu,
    }
    if default_workload(args):
        line["other_configs"] = other_configs()
    print(json.dumps(line), flush=True)


# The other workloads' short runs (child processes, after the metric's own
# run), as flags of this script. c3 at 24 query heads is the reference's 27B
# shape (G = 6); the E4M3 line is the step over an E4M3 cache.
OTHER_CONFIGS = [
    ("c2", ["--config", "c2", "--seed", "1"]),
    ("c4", ["--config", "c4", "--seed", "1", "--steps", "10", "--warmup", "2"]),
    ("c5", ["--config", "c5", "--seed", "1"]),
    ("attn", ["--config", "attn"]),
    ("c3_g6", ["--q-heads", "24", "--seed", "1"]),
    ("c3_e4m3", ["--kv", "e4m3", "--seed", "1"]),
]


def default_workload(args):
    """True for the metric's own workload with no flag that changes it (the
    run the driver makes), outside rocprofv3: under the profiler (whose
    launcher sets ROCPROF_OUTPUT_PATH for the program) the child runs would
    add their launches, some of the same kernels, to the command's trace."""
    return (args.config == "c3" and args.kv == "bf16" and args.q_heads == 16 and args.batch == 64
            and "ROCPROF_OUTPUT_PATH" not in os.environ
            and args.pages == 65536 and not args.no_others and not args.traffic_child
            and not (args.refabi or args.unfused or args.with_prep or args.verify_kernel)
            and args.wg_per_cu is None and args.min_range is None)


def other_configs():
    """Runs each OTHER_CONFIGS workload in a child process (no CPU leg, no
    counter runs; 200 s limit each) and keeps the headline fields of its JSON
    line, or the error."""
    import signal
    import subprocess

    out = {}
    for name, flags in OTHER_CONFIGS:
        cmd = [sys.executable, "-u", os.path.abspath(__file__), "--no-cpu", "--no-traffic", "--no-others"] + flags
        proc = subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.DEVNULL, start_new_session=True,
                                text=True)
        try:
            text, _ = proc.communicate(timeout=200)
        except subprocess.TimeoutExpired:
            os.killpg(proc.pid, signal.SIGKILL)  # the process group this call started
            proc.communicate()
            out[name] = {"flags": " ".join(flags), "error": "timed out after 200 s"}
            continue
        lines = [ln for ln in text.splitlines() if ln.startswith("{")]
        if proc.returncode != 0 or not lines:
            out[name] = {"flags": " ".join(flags), "error": f"exit {proc.returncode}"}
            continue
        d = json.loads(lines[-1])
        r = d.get("roofline") or {}
        out[name] = {"flags": " ".join(flags), "workload": (d.get("config") or {}).get("workload"),
                     "metric": d.get("metric"), "value": d.get("value"), "unit": d.get("unit"),
                     "ms_per_step": d.get("ms_per_step"), "vs_baseline": d.get("vs_baseline"),
                     "roofline": {k: r.get(k) for k in ("bound", "kernel", "achieved", "peak", "unit", "frac")}}
    return out


def bench_prefill(args):
    """Config 4: 8 sequences share a refcounted 16,384-token cached prefix,
    set up through the KV manager (pkv_kv: the seed's whole 64-token units
    cached, each sequence admitted with a prefix-cache hit so the same 1,024
    pages sit in every block table at refs 9; --prefix not a multiple of 64
    shares the seed's pages instead and copies the partial last page on
    write). Each step appends every sequence's 2,048-token chunk
    (pkv_append at the manager's slots) and runs causal paged attention of
    the chunk over prefix + chunk (pkv_attn_prefill). FLOPs = 4 * 256 * Hq *
    sum over query rows of keys attended (QK^T and PV, the reference
    bench-attn formula, src/main.rs:950-952). The append is timed on its own
    against the HBM roofline (bytes in + out)."""
    import numpy as np
    import torch

    import pkv
    from pkv import synth

    seed = args.seed if args.seed is not None else int(time.time()) % 100000
    dev = torch.device("cuda:0")
    Hq, Hkv, D, BS, B, P, N = args.q_heads, 4, 256, 16, 8, args.prefix, 2048
    per_seq = (P + N + BS - 1) // BS
    pages = (P + BS - 1) // BS + B * (per_seq - P // BS) + 8
    kv = pkv.Kv(pages, BS)
    plan = synth.c4_kv_plan(kv, P, N, B, seed=seed)
    st, mb = plan["step"], plan["max_blocks"]
    bt, pos, slot, cu = st["block_table"], st["pos"], st["slot_map"], st["cu"]
    prefix_refs = kv.refs(plan["seed_blocks"][0])
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    e4m3 = args.kv == "e4m3"
    if e4m3:
        # random E4M3 bytes (NaN codes replaced), scales amax/448-like; the
        # step is the prefill kernel alone (no bf16 append into this cache)
        kc = torch.randint(0, 256, (pages * BS, Hkv, D), device=dev, generator=gen, dtype=torch.int32).to(torch.uint8)
        vc = torch.randint(0, 256, (pages * BS, Hkv, D), device=dev, generator=gen, dtype=torch.int32).to(torch.uint8)
        for t_ in (kc, vc):
            t_[(t_ & 0x7F) == 0x7F] = 0x7E
        kscale = torch.rand(pages * BS, Hkv, device=dev, generator=gen) * 0.004 + 0.001
        vscale = torch.rand(pages * BS, Hkv, device=dev, generator=gen) * 0.004 + 0.001
    else:
        kc = (torch.randn(pages * BS, Hkv, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
        vc = (torch.randn(pages * BS, Hkv, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    if plan["cow"] and not e4m3:
        # the copies on write the manager asked for, before any chunk write
        cs = torch.from_numpy(np.array([c[0] for c in plan["cow"]], np.int32)).to(dev)
        cd = torch.from_numpy(np.array([c[1] for c in plan["cow"]], np.int32)).to(dev)
        pkv.page_copy(kc, vc, cs, cd, len(plan["cow"]), BS * Hkv * D * 2, pages)
    T = B * N
    q = (torch.randn(T, Hq, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    qstride = (2 * Hq + 2 * Hkv) * D
    qkv = (torch.randn(T, qstride, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    out = torch.empty(T, Hq, D, dtype=torch.bfloat16, device=dev)
    bt_d, pos_d, cu_d, slot_d = (torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in (bt, pos, cu, slot))
    k_rows = qkv.data_ptr() + 2 * (2 * Hq * D)
    v_rows = k_rows + 2 * Hkv * D
    stream = torch.cuda.current_stream()
    evs = HipEvents(args.steps)
    aevs = HipEvents(args.steps)

    if args.refabi:
        # the code object's prompt kernel, launched as the reference engine
        # launches it on gfx950 (fa_shape's attn_groupr_g4_t2_k32, model.rs:
        # 2438-2493); timed with events recorded around the launch
        from pkv import refabi
        from pkv.refabi import F, I, P as Pa
        rk = refabi.RefKernels()
        fname, fgrid, fthreads, fsmem = refabi.flash_launch(T, B, Hkv, g=Hq // Hkv, fp8=e4m3)
        fargs = [Pa(q), Pa(kc), Pa(vc), Pa(kscale if e4m3 else None), Pa(vscale if e4m3 else None), Pa(qkv), I(qstride), I(Hq), I(Hkv), Pa(pos_d), Pa(cu_d),
                 I(B), Pa(bt_d), I(mb), I(BS), Pa(out), F(1 / 16), Pa(None), I(1)]

    def step(ev=None, aev=None):
        if not e4m3:
            if aev:
                aevs.record(aev[0], stream.cuda_stream)
            pkv.append(k_rows, v_rows, qstride * 2, slot_d, T, Hkv, D * 2, kc, vc, pages * BS)
            if aev:
                aevs.record(aev[1], stream.cuda_stream)
        if args.refabi:
            if ev:
                evs.record(ev[0], stream.cuda_stream)
            rk.launch(fname, fgrid, fthreads, fsmem, fargs)
            if ev:
                evs.record(ev[1], stream.cuda_stream)
            return
        if ev:
            pkv.time_next_prefill_kernel(ev[0], ev[1])
        if e4m3:
            pkv.attn_prefill_e4m3(q, kc, vc, kscale, vscale, qkv, qstride, Hq, Hkv, pos_d, cu_d, B, bt_d, mb, BS,
                                  out, 1 / 16, None, 1, T, pages)
            return
        pkv.attn_prefill(q, kc, vc, qkv, qstride, Hq, Hkv, pos_d, cu_d, B, bt_d, mb, BS, out, 1 / 16, None, 1,
                         T, pages)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for k in range(args.steps):
        step(evs.pairs[k], aevs.pairs[k])
    t1.record(stream)
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / args.steps
    kern_ms = evs.elapsed_ms()
    flops = 4.0 * D * Hq * float((pos.astype(np.int64) + 1).sum())
    kern_us = 1e3 * sum(kern_ms) / len(kern_ms)
    tflops = flops / (kern_us * 1e-6) / 1e12
    append = None
    if not e4m3:
        app_ms = aevs.elapsed_ms()
        app_us = 1e3 * float(np.median(app_ms))
        app_bytes = synth.algorithmic_bytes_append(T, Hkv)
        append = {"kernel": "append_kernel (events around the launch)", "bytes": app_bytes,
                  "median_us": round(app_us, 2), "achieved": round(app_bytes / (app_us * 1e-6) / 1e9, 1),
                  "peak": PEAK_HBM_GBS, "unit": "GB/s",
                  "frac": round(app_bytes / (app_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}
    # algorithmic bytes of one prefill launch: every key of the prefix and
    # the chunks once (K and V, all kv heads; E4M3 bytes + scales), q, the
    # gate rows and the outputs
    key_bytes = Hkv * (D + 4) * 2 if e4m3 else Hkv * D * 2 * 2
    alg = (P + B * N) * key_bytes + 3 * T * Hq * D * 2
    traffic, traffic_detail = measure_traffic(args, seed, alg, want=fname if args.refabi else "prefill")
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_prefill(kc, vc, q, qkv, bt, pos, cu, B, Hq, Hkv, qstride, mb, flops, e4m3,
                                   kscale if e4m3 else None, vscale if e4m3 else None)
    line = {
        "metric": "chunked-prefill attention TFLOP/s over paged context (config 4), 1 MI355X",
        "value": round(tflops, 1),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3 KV (bf16 MFMA, f32 accum)" if e4m3 else "bf16",
        "data": ("synthetic (random E4M3 bytes and scales; q N(0,1)*0.5)" if e4m3 else
                 "synthetic (seeded N(0,1)*0.5)"),
        "config": {"workload": (f"c4: 8 seqs x 2048-token chunk over a shared {P}-token prefix through the KV "
                                f"manager ({'prefix-cache hits' if plan['via_cache'] else 'shared pages, partial page copied on write'}; "
                                + ("prefill kernel only, no append)" if e4m3 else "append + prefill)")),
                   "kv": args.kv, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "page": BS, "flop_per_step": flops,
                   "prefix": P, "prefix_page_refs": prefix_refs, "cow_copies": len(plan["cow"]),
                   "seed": seed, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": (f"{fname} (reference ABI, events around the launch)" if args.refabi
                                                  else f"prefill_e4m3_kernel<{Hq // Hkv}>" if e4m3 else f"prefill_kernel<{Hq // Hkv}>"),
                     "achieved": round(tflops, 1),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                     "avg_us": round(kern_us, 1), "traffic": None if traffic is None else round(traffic),
                     "traffic_detail": traffic_detail},
        "append": append,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_verify(args):
    """Config 5: 16 sequences with U[32768, 131072] cached tokens; a step
    appends 4 draft rows per sequence (pkv_append) and verifies them
    (pkv_attn_verify: each row attends causally, every page read once for
    the sequence's 4 rows), then the host rewinds each sequence to its
    accepted length (seeded a in 0..4: length += a + 1; pages stay reserved
    as the reference's finish does, src/sched.rs:1297-1327). Unique bytes
    per step = sum over sequences of (len + 4) keys x 4 KiB + append + q,
    gate, out. The same steps through per-token decode attention (each row
    re-reads its sequence's pages, as the reference) ride along."""
    import numpy as np
    import torch

    import pkv
    from pkv import synth

    seed = args.seed if args.seed is not None else int(time.time()) % 100000
    dev = torch.device("cuda:0")
    Hq, Hkv, D, BS, B, n = 16, 4, 256, 16, 16, 4
    S = args.warmup + args.steps
    rng = np.random.default_rng(seed)
    L0 = rng.integers(32768, 131072 + 1, size=B).astype(np.int64)
    acc = rng.integers(0, n + 1, size=(S, B))  # accepted drafts per step
    lens = L0 + np.concatenate([np.zeros((1, B), np.int64), np.cumsum(acc + 1, axis=0)[:-1]])  # [S][B]
    need = (lens[-1] + n + BS - 1) // BS
    pages = int(need.sum()) + 16
    mb = int(need.max())
    perm = rng.permutation(pages).astype(np.int32)
    bt = np.zeros((B, mb), np.int32)
    at = 0
    for s_ in range(B):
        bt[s_, :need[s_]] = perm[at:at + need[s_]]
        at += need[s_]
    pos = (lens[:, :, None] + np.arange(n)[None, None, :]).reshape(S, B * n).astype(np.int32)
    seqs = np.repeat(np.arange(B), n)
    slot = (bt[seqs[None, :], pos // BS] * BS + pos % BS).astype(np.int32)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    e4m3 = args.kv == "e4m3"
    if e4m3:
        # random E4M3 bytes (NaN codes replaced) and scales; the step is the
        # attention kernel and merge alone (no bf16 append into this cache)
        kc = torch.randint(0, 256, (pages * BS, Hkv, D), device=dev, generator=gen, dtype=torch.int32).to(torch.uint8)
        vc = torch.randint(0, 256, (pages * BS, Hkv, D), device=dev, generator=gen, dtype=torch.int32).to(torch.uint8)
        for t in (kc, vc):
            t[(t & 0x7F) == 0x7F] = 0x7E
        kscale = torch.rand(pages * BS, Hkv, device=dev, generator=gen) * 0.004 + 0.001
        vscale = torch.rand(pages * BS, Hkv, device=dev, generator=gen) * 0.004 + 0.001
    else:
        kc = torch.empty(pages * BS, Hkv, D, dtype=torch.bfloat16, device=dev)
        vc = torch.empty_like(kc)
        for t in (kc, vc):
            for i in range(0, t.shape[0], 1 << 18):
                t[i:i + (1 << 18)] = torch.randn(t[i:i + (1 << 18)].shape, device=dev, generator=gen) * 0.5
    T = B * n
    q = (torch.randn(T, Hq, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    qstride = synth.qkv_stride(Hq, Hkv)
    qkv = (torch.randn(T, qstride, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    out = torch.empty(T, Hq, D, dtype=torch.bfloat16, device=dev)
    pos_d, slot_d = torch.from_numpy(pos).to(dev), torch.from_numpy(slot).to(dev)
    ts = torch.from_numpy(seqs.astype(np.int32)).to(dev)
    cu = torch.from_numpy((np.arange(B + 1) * n).astype(np.int32)).to(dev)
    outs = torch.zeros(B, dtype=torch.int32, device=dev)  # every sequence verifies (spec rows)
    bt_d = torch.from_numpy(bt).to(dev)
    ws = torch.empty(max(pkv.attn_verify_workspace(T, Hq), pkv.attn_decode_workspace(T, Hq)), dtype=torch.uint8,
                     device=dev)
    k_rows = qkv.data_ptr() + 2 * (2 * Hq * D)
    v_rows = k_rows + 2 * Hkv * D
    stream = torch.cuda.current_stream()

    verify_fn, decode_fn = ((pkv.attn_verify_e4m3, pkv.attn_decode_e4m3) if e4m3 else
                            (pkv.attn_verify, pkv.attn_decode))

    def step(i, ev=None, fn=verify_fn):
        if not e4m3:
            pkv.append(k_rows, v_rows, qstride * 2, slot_d[i], T, Hkv, D * 2, kc, vc, pages * BS)
        if ev:
            pkv.time_next_range_kernel(ev[0], ev[1])
        if e4m3:
            fn(q, kc, vc, kscale, vscale, qkv, qstride, Hq, Hkv, pos_d[i], ts, bt_d, mb, BS, out, 1 / 16, cu, 1, outs,
               1, T, pages, ws)
            return
        fn(q, kc, vc, qkv, qstride, Hq, Hkv, pos_d[i], ts, bt_d, mb, BS, out, 1 / 16, cu, 1, outs, 1, T, pages, ws)

    def timed(fn, k0, K):
        evs = HipEvents(K)
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record(stream)
        for k in range(K):
            step(k0 + k, evs.pairs[k], fn)
        t1.record(stream)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1), evs.elapsed_ms()

    for i in range(args.warmup):
        step(i)
    total_ms, kern_ms = timed(verify_fn, args.warmup, args.steps)
    ms_step = total_ms / args.steps
    keys = [int((lens[args.warmup + k] + n).sum()) for k in range(args.steps)]  # unique keys per step
    key_bytes = Hkv * (D + 4) * 2 if e4m3 else Hkv * D * 2 * 2  # K + V (+ scales) per key
    step_bytes = [kk * key_bytes + 3 * T * Hq * D * 2 + (0 if e4m3 else synth.algorithmic_bytes_append(T, Hkv))
                  for kk in keys]
    gbs = sum(step_bytes) / (total_ms * 1e-3) / 1e9
    kern_bytes = [kk * key_bytes + T * Hq * D * 2 for kk in keys]
    kern_gbs = sum(kern_bytes) / (sum(kern_ms) * 1e-3) / 1e9
    kern_avg_us = 1e3 * sum(kern_ms) / len(kern_ms)
    # per-token decode attention on the same steps (each row re-reads its pages)
    Kd = min(args.steps, 20)
    dec_ms, _ = timed(decode_fn, args.warmup, Kd)
    # the verify kernel's algorithmic bytes over the child's steps 0 .. 3
    alg0 = float(np.mean([int((lens[k] + n).sum()) * key_bytes + T * Hq * D * 2 for k in range(4)]))
    traffic, traffic_detail = measure_traffic(args, seed, alg0, want="verify_range")
    cpu = None
    if not args.no_cpu:
        # every row of 4 of the 16 sequences (the 1st, 5th, 9th and 13th)
        sample = np.concatenate([np.arange(s_ * n, s_ * n + n) for s_ in range(0, B, 4)])
        cpu = cpu_baseline_rows(kc, vc, q, qkv, bt, pos[args.warmup], seqs.astype(np.int32), Hq, Hkv, qstride, mb,
                                sample, "every row of sequences 0, 4, 8, 12", kscale=kscale if e4m3 else None,
                                vscale=vscale if e4m3 else None, append_rows=0 if e4m3 else T)
    line = {
        "metric": "speculative verify step us + achieved HBM GB/s over unique KV bytes (config 5), 1 MI355X",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "us_per_step": round(ms_step * 1e3, 2),
        "pct_of_hbm_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
        "us_per_step_per_token_decode": round(1e3 * dec_ms / Kd, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3 KV (bf16 q/out, f32 accum)" if e4m3 else "bf16",
        "data": ("synthetic (random E4M3 bytes and scales, q N(0,1)*0.5, U[32768,131072] contexts, seeded accepted "
                 "counts)" if e4m3 else
                 "synthetic (seeded N(0,1)*0.5 K/V/q, U[32768,131072] contexts, seeded accepted counts)"),
        "config": {"workload": ("c5: 16 seqs x 4 draft rows over an E4M3 cache, verify attention + rewind (no append)"
                                if e4m3 else "c5: 16 seqs x 4 draft rows, append + verify attention + rewind"),
                   "kv": args.kv, "batch": B, "drafts": n, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "page": BS,
                   "pool_pages": pages, "seed": seed, "mean_unique_keys_per_step": round(float(np.mean(keys)), 1),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "verify_range8_kernel<4> (E4M3 cache, no append)" if e4m3 else
                     "verify_range_kernel<4>", "achieved": round(kern_gbs, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(kern_gbs / PEAK_HBM_GBS, 4),
                     "avg_us": round(kern_avg_us, 2), "traffic": None if traffic is None else round(traffic),
                     "traffic_detail": traffic_detail},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_attn(args):
    """The reference's bench-attn (src/main.rs:721-955), restated: --seqs
    sequences of --tokens prompt tokens after --context cached keys, 4 kv
    heads, G = --q-heads / 4, head_dim 256, inputs from bench-attn's hash
    (x = ((h % 2001) / 1000 - 1) * scale, h = (i ^ seed * 0x9e3779b9) *
    2654435761 mod 2^64, main.rs:738-746), each sequence's pages in reverse
    order (main.rs:755-763). Times the prompt kernel alone over 20 launches
    by wall clock after one warm-up, as bench-attn does (main.rs:938-955),
    for this library's pkv_attn_prefill and for the code object's kernel on
    the engine's grid (fa_shape's choice on gfx950); FLOPs 4 x 256 x Hq x
    attended keys. bench-attn --check's comparison with the decode kernel
    (main.rs:843-938) runs on sampled rows."""
    import numpy as np
    import torch

    import pkv
    from pkv import refabi
    from pkv.refabi import F, I, P as Pa

    dev = torch.device("cuda:0")
    D, BS, hkv = 256, 16, 4
    G = args.q_heads // hkv
    hq, seqs, tokens, context = G * hkv, args.seqs, args.tokens, args.context
    qstride = (2 * hq + 2 * hkv) * D
    t = seqs * tokens
    mb = (context + tokens + BS - 1) // BS
    slots = seqs * mb * BS
    two64 = (1 << 64) % 2001

    def rnd(n, seed, scale):
        # bench-attn's hash in unsigned 64-bit arithmetic (int64 wraps alike;
        # the remainder is corrected for the sign), in chunks on the device
        out = torch.empty(n, dtype=torch.bfloat16, device=dev)
        mul = torch.tensor(2654435761, dtype=torch.int64, device=dev)
        sd = (seed * 0x9E3779B9) & ((1 << 63) - 1)
        for a in range(0, n, 1 << 26):
            i = torch.arange(a, min(n, a + (1 << 26)), dtype=torch.int64, device=dev)
            h = torch.bitwise_xor(i, sd) * mul
            r = torch.remainder(h, 2001)
            r = torch.remainder(r + (h < 0).to(torch.int64) * two64, 2001)
            out[a:a + len(i)] = ((r.to(torch.float32) / 1000.0 - 1.0) * scale).to(torch.bfloat16)
        return out

    q = rnd(t * hq * D, 1, 1.0).view(t, hq, D)
    proj = rnd(t * qstride, 2, 1.0).view(t, qstride)
    kc = rnd(slots * hkv * D, 3, 1.0).view(slots, hkv, D)
    vc = rnd(slots * hkv * D, 4, 1.0).view(slots, hkv, D)
    bt = np.array([[s * mb + mb - 1 - b for b in range(mb)] for s in range(seqs)], np.int32)
    pos = np.array([context + i % tokens for i in range(t)], np.int32)
    cu = np.arange(seqs + 1, dtype=np.int32) * tokens
    bt_d, pos_d, cu_d = (torch.from_numpy(a).to(dev) for a in (bt, pos, cu))
    out = torch.zeros(t, hq, D, dtype=torch.bfloat16, device=dev)
    out_ref = torch.zeros_like(out)
    scale = 1.0 / 16.0
    flops = 4.0 * D * hq * seqs * float(sum(context + i + 1 for i in range(tokens)))

    ws_bytes = pkv.attn_prefill_workspace(t, hq, hkv, seqs) if args.prefill_split else 0
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev) if args.prefill_split else None

    def lib():
        pkv.attn_prefill(q, kc, vc, proj, qstride, hq, hkv, pos_d, cu_d, seqs, bt_d, mb, BS, out, scale, None, 1, t,
                         seqs * mb, workspace=ws)

    rk = refabi.RefKernels()
    fname, fgrid, fthreads, fsmem = refabi.flash_launch(t, seqs, hkv, g=G)
    fargs = [Pa(q), Pa(kc), Pa(vc), Pa(None), Pa(None), Pa(proj), I(qstride), I(hq), I(hkv), Pa(pos_d), Pa(cu_d),
             I(seqs), Pa(bt_d), I(mb), I(BS), Pa(out_ref), F(scale), Pa(None), I(1)]

    def ref():
        rk.launch(fname, fgrid, fthreads, fsmem, fargs)

    def wall_us(fn, n=20):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n * 1e6

    lib_us = min(wall_us(lib) for _ in range(3))
    ref_us = min(wall_us(ref) for _ in range(3))
    # the library kernel's own duration (events at its start and end)
    kev = HipEvents(20)
    for k in range(20):
        pkv.time_next_prefill_kernel(*kev.pairs[k])
        lib()
    torch.cuda.synchronize()
    kern_us = 1e3 * float(np.median(kev.elapsed_ms()))

    # --check: decode attention of sampled rows (every 64th token of each
    # sequence and its last) against the prompt kernels' rows
    rows = np.array(sorted({s * tokens + j for s in range(seqs) for j in list(range(0, tokens, 64)) + [tokens - 1]}),
                    np.int64)
    rows_d = torch.from_numpy(rows).to(dev)
    dq, dproj = q[rows_d].contiguous(), proj[rows_d].contiguous()
    dseq = (rows // tokens).astype(np.int32)
    dcu = np.searchsorted(dseq, np.arange(seqs + 1), side="left").astype(np.int32)
    dout = torch.zeros(len(rows), hq, D, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(max(pkv.attn_decode_workspace(len(rows), hq), pkv.attn_verify_workspace(len(rows), hq)),
                     dtype=torch.uint8, device=dev)
    pkv.attn_decode(dq, kc, vc, dproj, qstride, hq, hkv, torch.from_numpy(pos[rows]).to(dev),
                    torch.from_numpy(dseq).to(dev), bt_d, mb, BS, dout, scale, torch.from_numpy(dcu).to(dev), 0, None,
                    1, len(rows), seqs * mb, ws)
    torch.cuda.synchronize()
    check = {}
    for what, o in (("library", out), ("code object", out_ref)):
        got, want = o[rows_d].float(), dout.float()
        err = (got - want).abs()
        check[what] = {"max_abs": round(float(err.max()), 6),
                       "within_tolerance": bool((err <= 2e-3 + 1e-2 * want.abs()).all())}

    # CPU baseline: the oracle's prompt attention on 8 groups of 2 rows spread
    # over the prompt, scaled by FLOPs to the whole launch
    cpu = None
    if not args.no_cpu:
        import oracle
        (kc_h, vc_h), bt_h = _host_pages([kc, vc], bt, np.full(seqs, mb))
        q_h, proj_h = _bits(q), _bits(proj)
        items = [(s, np.array([s * tokens + j, s * tokens + j + 1]))
                 for s in range(seqs) for j in np.linspace(0, tokens - 2, 8).astype(int)]

        def run(it):
            s, r = it
            oracle.attn_prefill(np.ascontiguousarray(q_h[r]), kc_h, vc_h, np.ascontiguousarray(proj_h[r]), qstride,
                                hq, hkv, pos[r], np.array([0, 2], np.int32), 1, np.ascontiguousarray(bt_h[s:s + 1]),
                                mb, BS, scale, threads=1)

        rate1, rate_mt, nthr, detail = _cpu_rates(items, run, lambda it: 4.0 * D * hq * float(
            (pos[it[1]].astype(np.int64) + 1).sum()))
        cpu = {"value": round(flops / rate_mt * 1e6, 1), "unit": "us", "cores": nthr, "kind": "port",
               "sample": f"oracle prompt attention of {len(items)} groups of 2 rows spread over the prompt, scaled "
                         f"by FLOPs to the launch ({flops:.3e} FLOP); {detail}",
               "single_thread_us": round(flops / rate1 * 1e6, 1), "cpu": _cpu_model()}

    alg = seqs * (context + tokens) * hkv * D * 2 * 2 + 3 * t * hq * D * 2
    traffic, traffic_detail = measure_traffic(args, 0, alg, want="prefill_split" if ws_bytes else "prefill")
    published = {(4, 4096, 0, 1): 1160.0}  # bench-attn prefill g4 4096 tokens, RTX 5090
    base = published.get((G, tokens, context, seqs))
    tf = flops / (kern_us * 1e-6) / 1e12
    line = {
        "metric": f"bench-attn prefill us (group {G}, {tokens} tokens after {context}, {seqs} seq), 1 MI355X",
        "value": round(lib_us, 1),
        "unit": "us",
        "n_gpus": 1,
        "steps": 20,
        "warmup": 1,
        "ms_per_step": round(lib_us * 1e-3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None if base is None else round(lib_us / base, 4),
        "baseline_us": base,
        "baseline_note": None if base is None else "RTX 5090 (scripts/perf/nvidia-geforce-rtx-5090.json:2)",
        "tflops_wall": round(flops / (lib_us * 1e-6) / 1e12, 1),
        "code_object": {"kernel": fname, "grid": list(fgrid), "threads": fthreads, "smem": fsmem,
                        "us": round(ref_us, 1), "tflops": round(flops / (ref_us * 1e-6) / 1e12, 1),
                        "vs_baseline": None if base is None else round(ref_us / base, 4)},
        "dtype": "bf16",
        "data": "synthetic (bench-attn's hash inputs, reversed block table)",
        "config": {"workload": "bench-attn: prompt attention alone", "entry": ("pkv_attn_prefill_split ("
                   f"{ws_bytes} workspace bytes)" if args.prefill_split else "pkv_attn_prefill"), "q_heads": hq,
                   "kv_heads": hkv,
                   "head_dim": D, "page": BS, "seqs": seqs, "tokens": tokens, "context": context,
                   "flop_per_launch": flops, "parallelism": "single GPU"},
        "check": {"rows": len(rows), "against": "pkv_attn_decode of the same rows", **check},
        "roofline": {"bound": "mfma", "kernel": (f"prefill_split_kernel<{G}> (events at its start and end; the merge launch after it "
                                "is outside)" if ws_bytes else
                                f"the prompt kernel pkv_attn_prefill picks for G={G} (events at its start and end)"),
                     "achieved": round(tf, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / PEAK_BF16_TFLOPS, 4), "median_us": round(kern_us, 1),
                     "traffic": None if traffic is None else round(traffic), "traffic_detail": traffic_detail},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def hbm_copy_probe(dev):
    """A plain device copy of 2 GiB (read 2 GiB + write 2 GiB) timed with
    events over 10 copies after 2 warm-up copies (a copy kernel on the
    current stream), and a read-mostly reduction over the same bytes: the
    HBM GB/s plain library kernels reach on this box, beside the 8 TB/s
    spec figure."""
    import torch

    src = torch.ones(1 << 30, dtype=torch.int16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        dst.copy_(src)
    e1.record()
    e1.synchronize()
    gbs = 10 * 2 * (2 << 30) / (e0.elapsed_time(e1) * 1e-3) / 1e9
    # read-mostly: an integer sum over the same 2 GiB (reads only, a few
    # bytes written), the access decode makes
    words = src.view(torch.int64)
    for _ in range(2):
        words.sum()
    e0.record()
    for _ in range(10):
        words.sum()
    e1.record()
    e1.synchronize()
    read_gbs = 10 * (2 << 30) / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del src, dst, words
    torch.cuda.empty_cache()
    return gbs, read_gbs


def cpu_baseline(kc, vc, q, qkv, meta, st, Hq, Hkv, qstride, dev):
    """Scalar host code on the first timed step's workload — append + decode
    of all 64 sequences — timed on the host with 1 thread and with up to 16
    threads (the box's CPU share), tokens split into key-balanced sets (ctypes
    releases the GIL, so the C calls run in parallel). Two implementations:
    the one-pass f32 port (orc_attn_decode_f32: online softmax, K / V rows
    read once per kv-head group, f32 throughout), whose threaded figure is
    the line's value, and the f64 oracle (the checker: two passes, double
    sums), reported beside it."""
    import numpy as np
    import torch

    import oracle

    BS, D = 16, 256
    B = meta.B
    sel = list(range(B))
    bt = meta.block_table
    need = [(int(st["pos"][s]) + BS) // BS for s in sel]
    sub = np.concatenate([bt[s, :n] for s, n in zip(sel, need)])
    idx = torch.from_numpy(sub).to(dev).long()
    kc_h = kc.view(-1, BS, Hkv, D)[idx].cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1, Hkv, D)
    vc_h = vc.view(-1, BS, Hkv, D)[idx].cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1, Hkv, D)
    remap = {int(p): i for i, p in enumerate(sub)}
    bts = np.zeros((len(sel), meta.max_blocks), np.int32)
    for i, (s, n) in enumerate(zip(sel, need)):
        bts[i, :n] = [remap[int(p)] for p in bt[s, :n]]
    q_h = q[sel].cpu().view(torch.int16).numpy().view(np.uint16)
    qkv_h = qkv[sel].cpu().view(torch.int16).numpy().view(np.uint16)
    pos = st["pos"][sel]
    k_new = np.ascontiguousarray(qkv_h[:, 2 * Hq * D:2 * Hq * D + Hkv * D])
    v_new = np.ascontiguousarray(qkv_h[:, 2 * Hq * D + Hkv * D:2 * Hq * D + 2 * Hkv * D])
    slots = (bts[np.arange(len(sel)), pos // BS] * BS + pos % BS).astype(np.int32)
    sample_keys = int((pos + 1).sum())
    full_keys = int((st["pos"] + 1).sum())
    scale_f = full_keys / sample_keys

    # Threaded runs: longest-first assignment of tokens to the lightest set.
    import concurrent.futures
    nthr = max(1, min(16, os.cpu_count() or 1, len(sel)))
    sets = [[] for _ in range(nthr)]
    load = [0] * nthr
    for i in sorted(range(len(sel)), key=lambda i: -int(pos[i])):
        j = load.index(min(load))
        sets[j].append(i)
        load[j] += int(pos[i]) + 1
    parts = []
    for ids in sets:
        ids = np.array(sorted(ids), np.int64)
        parts.append((np.ascontiguousarray(k_new[ids]), np.ascontiguousarray(v_new[ids]), slots[ids].copy(),
                      np.ascontiguousarray(q_h[ids]), np.ascontiguousarray(qkv_h[ids]), pos[ids].copy(),
                      np.arange(len(ids), dtype=np.int32), np.ascontiguousarray(bts[ids])))

    def decode(f32, qq, qk, ps, ts, bt_):
        if f32:
            oracle.attn_decode_f32(qq, kc_h, vc_h, qk, qstride, Hq, Hkv, ps, ts, bt_, meta.max_blocks, BS, 1 / 16)
        else:
            oracle.attn_decode(qq, kc_h, vc_h, qk, qstride, Hq, Hkv, ps, ts, bt_, meta.max_blocks, BS, 1 / 16,
                               threads=1)

    def timed(f32, budget1, budget_mt):
        # The same step repeated (the append rewrites the same slots) to a
        # bounded sample, mean per step: 1 thread, then the threaded sets.
        reps, t = 0, time.perf_counter()
        while True:
            oracle.append(k_new, v_new, slots, kc_h, vc_h)
            decode(f32, q_h, qkv_h, pos, np.arange(len(sel), dtype=np.int32), bts)
            reps += 1
            total = time.perf_counter() - t
            if total >= budget1 or reps >= 8:
                break

        def run(part):
            kn, vn, sl, qq, qk, ps, ts, bt_ = part
            if len(ps) == 0:
                return
            oracle.append(kn, vn, sl, kc_h, vc_h)  # disjoint slots per set
            decode(f32, qq, qk, ps, ts, bt_)

        reps_mt, t = 0, time.perf_counter()
        with concurrent.futures.ThreadPoolExecutor(nthr) as ex:
            while True:
                list(ex.map(run, parts))
                reps_mt += 1
                total_mt = time.perf_counter() - t
                if total_mt >= budget_mt or reps_mt >= 16:
                    break
        return reps, total, reps_mt, total_mt

    r1, t1, rm, tm = timed(True, 5.0, 3.0)
    us1, usm = t1 / r1 * 1e6 * scale_f, tm / rm * 1e6 * scale_f
    r1d, t1d, rmd, tmd = timed(False, 5.0, 3.0)
    us1d, usmd = t1d / r1d * 1e6 * scale_f, tmd / rmd * 1e6 * scale_f
    return {"value": round(usm, 1), "unit": "us/step", "cores": nthr, "kind": "port",
            "arith": "f32 (one-pass scalar C port: online softmax, f32 scores, weights and sums)",
            "sample": f"append + decode of one full step: all {len(sel)} sequences, {sample_keys} keys; "
                      f"{nthr} threads (tokens split into key-balanced sets): {rm} repetitions in {tm:.1f} s; "
                      f"1 thread: {r1} repetitions in {t1:.1f} s, {us1 / 1e6:.2f} s per step (scale factor "
                      f"{scale_f:.3f})",
            "single_thread_us_per_step": round(us1, 1),
            "f64_oracle": {"value": round(usmd, 1), "cores": nthr, "single_thread_us_per_step": round(us1d, 1),
                           "arith": "f64 (the checker: scores, softmax and weighted sums in double)",
                           "sample": f"the same step: {rmd} repetitions in {tmd:.1f} s on {nthr} threads, {r1d} in "
                                     f"{t1d:.1f} s on 1"},
            "cpu": _cpu_model()}


def _host_pages(tensors, bt, need):
    """Host copies (numpy) of the pages sequence s uses (bt[s, :need[s]]) from
    device pools shaped [pages * 16][...], gathered once each, and bt
    remapped to them."""
    import numpy as np
    import torch

    rows = [bt[s, :int(n)] for s, n in enumerate(need)]
    sub = np.unique(np.concatenate(rows))
    out = []
    for t in tensors:
        idx = torch.from_numpy(sub.astype(np.int64)).to(t.device)
        x = t.view(-1, 16, *t.shape[1:])[idx].cpu()
        x = (x.view(torch.int16).numpy().view(np.uint16) if x.dtype == torch.bfloat16 else x.numpy())
        out.append(np.ascontiguousarray(x.reshape(-1, *t.shape[1:])))
    where = np.full(int(bt.max()) + 1, -1, np.int64)
    where[sub] = np.arange(len(sub))
    bt_h = np.zeros(bt.shape, np.int32)
    for s, r in enumerate(rows):
        bt_h[s, :len(r)] = where[r]
    return out, bt_h


def _bits(x):
    import numpy as np
    import torch
    return x.cpu().view(torch.int16).numpy().view(np.uint16)


def _cpu_rates(items, run, weight, budget1=10.0, budget_mt=5.0):
    """Oracle throughput in work units per second: on 1 thread (items in
    order, cycling, until budget1 seconds) and on up to 16 threads (items
    spread over a thread pool, ctypes releasing the GIL, until budget_mt).
    Returns (rate_1, rate_mt, threads, detail)."""
    import concurrent.futures
    nthr = max(1, min(16, os.cpu_count() or 1, len(items)))
    done, i, t = 0.0, 0, time.perf_counter()
    while True:
        run(items[i % len(items)])
        done += weight(items[i % len(items)])
        i += 1
        t1 = time.perf_counter() - t
        if t1 >= budget1:
            break
    rate1 = done / t1
    detail = f"1 thread: {i} units in {t1:.1f} s"
    if nthr == 1:
        return rate1, rate1, 1, detail
    done_mt, rounds, t = 0.0, 0, time.perf_counter()
    with concurrent.futures.ThreadPoolExecutor(nthr) as ex:
        while True:
            list(ex.map(run, items))
            done_mt += sum(weight(x) for x in items)
            rounds += 1
            tm = time.perf_counter() - t
            if tm >= budget_mt:
                break
    detail += f"; {nthr} threads: {rounds} rounds of {len(items)} units in {tm:.1f} s"
    return rate1, done_mt / tm, nthr, detail


def cpu_baseline_prefill(kc, vc, q, qkv, bt, pos, cu, B, Hq, Hkv, qstride, mb, flops, e4m3, kscale, vscale):
    """The oracle's chunked prefill (scalar C, f64 softmax) on a bounded
    sample of config 4: groups of 2 query rows spread over all sequences and
    positions, timed on 1 thread and on up to 16, scaled to the step's
    FLOPs; plus the oracle's append of the step's 16,384 K/V rows (timed
    once, added to both). E4M3 caches are not timed on the host (null)."""
    import numpy as np

    import oracle
    if e4m3:
        return None
    BS, D = 16, 256
    need = np.full(B, mb)
    (kc_h, vc_h), bt_h = _host_pages([kc, vc], bt, need)
    q_h, qkv_h = _bits(q), _bits(qkv)
    rng = np.random.default_rng(0)
    N = int(cu[1] - cu[0])
    items = []
    for s in range(B):
        for j in rng.choice(N // 2, 4, replace=False):
            rows = np.array([cu[s] + 2 * j, cu[s] + 2 * j + 1])
            items.append((s, rows))

    def run(it):
        s, rows = it
        oracle.attn_prefill(np.ascontiguousarray(q_h[rows]), kc_h, vc_h, np.ascontiguousarray(qkv_h[rows]), qstride,
                            Hq, Hkv, pos[rows], np.array([0, len(rows)], np.int32), 1,
                            np.ascontiguousarray(bt_h[s:s + 1]), mb, BS, 1 / 16, threads=1)

    def weight(it):
        return 4.0 * D * Hq * float((pos[it[1]].astype(np.int64) + 1).sum())

    rate1, rate_mt, nthr, detail = _cpu_rates(items, run, weight)
    T = len(pos)
    kn = np.ascontiguousarray(qkv_h[:, 2 * Hq * D:2 * Hq * D + Hkv * D])
    vn = np.ascontiguousarray(qkv_h[:, 2 * Hq * D + Hkv * D:2 * Hq * D + 2 * Hkv * D])
    slot_h = np.zeros(T, np.int32)  # the host pool holds the used pages only: append into its first slots
    slot_h[:] = np.arange(T) % (kc_h.shape[0])
    t = time.perf_counter()
    oracle.append(kn, vn, slot_h, kc_h, vc_h)
    app_s = time.perf_counter() - t
    us1 = (flops / rate1 + app_s) * 1e6
    us_mt = (flops / rate_mt + app_s) * 1e6
    return {"value": round(us_mt, 1), "unit": "us/step", "cores": nthr, "kind": "port",
            "sample": f"oracle prefill of {len(items)} groups of 2 query rows (4 per sequence, all 8 sequences) "
                      f"scaled by FLOPs to the full step ({flops:.3e} FLOP), plus the oracle append of all {T} "
                      f"K/V rows ({app_s * 1e3:.0f} ms); {detail}",
            "single_thread_us_per_step": round(us1, 1),
            "tflops_single_thread": round(rate1 / 1e12, 6), "tflops_threads": round(rate_mt / 1e12, 6),
            "cpu": _cpu_model()}


def cpu_baseline_rows(kc, vc, q, qkv, bt, pos, tok_seq, Hq, Hkv, qstride, mb, sample_rows, what, kscale=None,
                      vscale=None, append_rows=0):
    """The oracle's paged decode attention (per row, scalar C) on a bounded
    sample of the step's rows (sample_rows, each row one work unit weighted
    by its keys), timed on 1 thread and on up to 16 and scaled by keys to
    the whole step, plus the oracle append of append_rows K/V rows. E4M3
    caches (kscale given) run oracle.attn_decode8."""
    import numpy as np
    import torch

    import oracle
    BS, D = 16, 256
    seqs = np.unique(tok_seq[sample_rows])
    need = np.zeros(len(seqs), np.int64)
    for i, s in enumerate(seqs):
        need[i] = int(pos[sample_rows][tok_seq[sample_rows] == s].max()) // BS + 1
    tens = [kc, vc] + ([kscale, vscale] if kscale is not None else [])
    hosts, bt_h = _host_pages(tens, bt[seqs], need)
    remap = {int(s): i for i, s in enumerate(seqs)}
    q_h = _bits(q[torch.from_numpy(np.asarray(sample_rows)).to(q.device)])
    qkv_h = _bits(qkv[torch.from_numpy(np.asarray(sample_rows)).to(q.device)])
    items = list(range(len(sample_rows)))

    def run(i):
        r = sample_rows[i]
        args8 = (hosts[2], hosts[3]) if kscale is not None else ()
        fn = oracle.attn_decode8 if kscale is not None else oracle.attn_decode
        fn(np.ascontiguousarray(q_h[i:i + 1]), hosts[0], hosts[1], *args8, np.ascontiguousarray(qkv_h[i:i + 1]),
           qstride, Hq, Hkv, np.array([pos[r]], np.int32), np.array([remap[int(tok_seq[r])]], np.int32), bt_h, mb,
           BS, 1 / 16, threads=1)

    def weight(i):
        return float(pos[sample_rows[i]] + 1)

    rate1, rate_mt, nthr, detail = _cpu_rates(items, run, weight)
    keys = float((pos.astype(np.int64) + 1).sum())
    app_s = 0.0
    if append_rows and kscale is None:
        kn = np.ascontiguousarray(qkv_h[:1, 2 * Hq * D:2 * Hq * D + Hkv * D].repeat(append_rows, 0))
        slot_h = (np.arange(append_rows) % hosts[0].shape[0]).astype(np.int32)
        t = time.perf_counter()
        oracle.append(kn, kn, slot_h, hosts[0], hosts[1])
        app_s = time.perf_counter() - t
    us1 = (keys / rate1 + app_s) * 1e6
    us_mt = (keys / rate_mt + app_s) * 1e6
    return {"value": round(us_mt, 1), "unit": "us/step", "cores": nthr, "kind": "port",
            "sample": f"oracle {'E4M3 ' if kscale is not None else ''}decode attention of {len(sample_rows)} of the "
                      f"step's {len(pos)} rows ({what}), scaled by keys to the whole step ({int(keys)} keys)"
                      + (f", plus the oracle append of {append_rows} K/V rows" if append_rows else "")
                      + f"; {detail}",
            "single_thread_us_per_step": round(us1, 1),
            "cpu": _cpu_model()}


def _cpu_model():
    """The host CPU as /proc/cpuinfo names it (model name, family, model,
    stepping of the first processor entry) with the logical CPU count and
    the CPUs this process may run on."""
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            if not line.strip():
                break
            k, _, v = line.partition(":")
            fields[k.strip()] = v.strip()
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = None
    return (f"{fields.get('model name', 'unknown')} (family {fields.get('cpu family', '?')}, model "
            f"{fields.get('model', '?')}, stepping {fields.get('stepping', '?')}; {os.cpu_count()} logical CPUs, "
            f"{allowed} allowed to this process)")


if __name__ == "__main__":
    main()
