#!/usr/bin/env python3
"""Throughput of the BLT entropy-patching path on one MI355X.

One step = the full entropy-model forward (14 layers, dim 768, 12 heads,
FFN 2048 SwiGLU, vocab 260, window 512) over a [16, 8192] batch of synthetic
byte tokens plus the monotonic patch-boundary pass, with
every input already resident in HBM.  Prints one JSON line:
value = input bytes patched per second; roofline = the dominant kernel's
achieved MFMA rate (algorithmic FLOPs / its mean HIP-event duration on the
launch stream); cpu_baseline = the CPU oracle (C restatement of the
reference's NdArray path) on a bounded sample of the same workload.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0
METRIC = "input bytes/sec patched (BLT entropy model, bf16, T=8192); % of roofline"


def attention_pairs(T, window):
    """Visible (query, key) pairs of one causal row of length T."""
    if window <= 0:
        return T * (T + 1) // 2
    w = min(window, T)
    return w * (w + 1) // 2 + (T - w) * w


def stage_flops(stage, M, B, T, D, F, V, H, window):
    hd = D // H
    return {
        "qkv_gemm_rope": 2.0 * M * D * 3 * D,
        "o_gemm_residual": 2.0 * M * D * D,
        "w13_gemm_silu": 2.0 * M * D * 2 * F,
        "w2_gemm_residual": 2.0 * M * F * D,
        "head_gemm": 2.0 * M * D * V,
        "attention": 4.0 * hd * attention_pairs(T, window) * H * B,
    }.get(stage)


STAGE_OF_GEMM = ("qkv_gemm_rope", "o_gemm_residual", "w13_gemm_silu", "w2_gemm_residual")


def _dispatch_stages(names, layers):
    """Map the kernel names of one forward's dispatches, in order, to model stages."""
    out, g = [], 0
    for n in names:
        if "gemm_bf16" in n:
            out.append(STAGE_OF_GEMM[g % 4] if g < 4 * layers else "head_gemm")
            g += 1
        elif "attn_fwd_kernel" in n:
            out.append("attention")
        elif "head_entropy_kernel" in n:
            # the fused final RMSNorm + L2 + head + entropy (+ coherence)
            out.append("head_gemm")
        elif "rmsnorm" in n:
            out.append("rmsnorm")
        elif "entropy_" in n and "_kernel" in n:
            out.append("entropy")
        elif ("patch_boundary_kernel" in n or "patch_flags_kernel" in n or
              "patch_scan_kernel" in n or "patch_compact_kernel" in n):
            out.append("patch_boundaries")
        elif "embed_kernel" in n:
            out.append("embed")
        elif "coherence_kernel" in n:
            out.append("coherence")
        else:
            out.append(None)
    return out


def _forward_stages(names, layers):
    """_dispatch_stages over a run's dispatches: the run is split into forwards,
    each starting at its embed_kernel (dispatches before the first get None)."""
    starts = [i for i, n in enumerate(names) if "embed_kernel" in n] + [len(names)]
    out = [None] * starts[0]
    for a, b in zip(starts[:-1], starts[1:]):
        out += _dispatch_stages(names[a:b], layers)
    return out


def _read_counter_csv(path, counter):
    import csv
    rows = [r for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    return [(r["Kernel_Name"], float(r["Counter_Value"])) for r in rows]


def summarize_dirs(dirs, copy_bytes, L=14):
    """Per-stage HBM traffic per launch from rocprofv3 --pmc runs of
    `bench.py --steps 1 --warmup 0 --no-cpu` (FETCH_SIZE and WRITE_SIZE, KiB per
    dispatch), each scaled by the bytes a copy of copy_bytes reads/writes
    divided by what the counter reports for that copy.  dirs: the output
    directories of the fetch, write, copy-fetch and copy-write runs."""
    import glob
    find = lambda d: glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)[0]
    fetch = _read_counter_csv(find(dirs[0]), "FETCH_SIZE")
    write = _read_counter_csv(find(dirs[1]), "WRITE_SIZE")
    cf = max(v for _, v in _read_counter_csv(find(dirs[2]), "FETCH_SIZE"))
    cw = max(v for _, v in _read_counter_csv(find(dirs[3]), "WRITE_SIZE"))
    kf, kw = copy_bytes / (cf * 1024.0), copy_bytes / (cw * 1024.0)
    res = {"fetch_scale": kf, "write_scale": kw, "copy_bytes": copy_bytes,
           "copy_fetch_kib": cf, "copy_write_kib": cw, "stages": {}}
    counts = {}
    for lst, key, k in ((fetch, "fetch_bytes", kf), (write, "write_bytes", kw)):
        ours = [(n, v) for n, v in lst if "blt::" in n]
        for st, (n, v) in zip(_forward_stages([n for n, _ in ours], L), ours):
            if st is None:
                continue
            d = res["stages"].setdefault(st, {"launches": 0})
            d[key] = d.get(key, 0.0) + v * 1024.0 * k
            counts[(st, key)] = counts.get((st, key), 0) + 1
    # each counter's total over its own dispatches; a stage whose write pass
    # saw a different number of launches than its fetch pass says so
    for st, d in res["stages"].items():
        nf, nw = counts.get((st, "fetch_bytes"), 0), counts.get((st, "write_bytes"), 0)
        d["launches"] = nf
        if nw != nf:
            d["write_launches"] = nw
        d["fetch_bytes"] = round(d.get("fetch_bytes", 0.0) / max(nf, 1))
        d["write_bytes"] = round(d.get("write_bytes", 0.0) / max(nw, 1))
    return res


def summarize(args):
    """--summarize: summarize_dirs of the four given directories as JSON."""
    print(json.dumps(summarize_dirs(args.summarize, args.copy_bytes), indent=1))


def live_traffic(args, timeout_s=180):
    """Config 4's per-stage traffic measured in this run: the four rocprofv3
    --pmc passes that --summarize reads (one counter each: FETCH_SIZE, then
    WRITE_SIZE, over a one-step bench of the same shape, then both over the
    copy probe), each a child process; all four share one time limit of
    timeout_s seconds.  Called before this process touches the GPU.  Returns
    (summary, None) or (None, reason)."""
    import shutil
    import signal
    import subprocess
    import tempfile
    exe = shutil.which("rocprofv3")
    if exe is None:
        return None, "rocprofv3 not on PATH"
    tmp = tempfile.mkdtemp(prefix="blt_traffic_")
    step = ["--steps", "1", "--warmup", "0", "--no-cpu", "--telemetry-s", "0",
            "--traffic", "off", "--batch", str(args.batch), "--seq", str(args.seq),
            "--window", str(args.window), "--threshold", repr(args.threshold)]
    probe = ["--copy-probe", "--copy-bytes", repr(args.copy_bytes)]
    runs = (("tf", "FETCH_SIZE", step), ("tw", "WRITE_SIZE", step),
            ("cf", "FETCH_SIZE", probe), ("cw", "WRITE_SIZE", probe))
    deadline = time.monotonic() + timeout_s
    try:
        for d, counter, extra in runs:
            cmd = [exe, "--pmc", counter, "--output-format", "csv", "-d", os.path.join(tmp, d),
                   "-o", "p", "--", sys.executable, os.path.abspath(__file__)] + extra
            with open(os.path.join(tmp, d + ".log"), "w") as log:
                proc = subprocess.Popen(cmd, stdout=log, stderr=subprocess.STDOUT,
                                        start_new_session=True, cwd=tmp)
                try:
                    rc = proc.wait(timeout=max(deadline - time.monotonic(), 0.1))
                except subprocess.TimeoutExpired:
                    os.killpg(proc.pid, signal.SIGKILL)
                    proc.wait()
                    return None, "rocprofv3 --pmc passes over their %d s limit (at %s)" % (
                        timeout_s, counter)
            # rocprofv3 can exit non-zero after the program ended with its
            # results written; the checks below take them only when whole
            if rc != 0:
                print("bench: rocprofv3 --pmc %s exited %d" % (counter, rc), file=sys.stderr)
        try:
            res = summarize_dirs([os.path.join(tmp, d) for d, _, _ in runs], args.copy_bytes)
        except (IndexError, KeyError, ValueError, OSError) as e:
            return None, "no usable counter output (%s: %s)" % (type(e).__name__, e)
        partial = sorted(st for st, d in res["stages"].items() if "write_launches" in d)
        if partial:
            return None, "FETCH_SIZE and WRITE_SIZE passes saw different launches of %s" % (
                ", ".join(partial))
        return res, None
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def summarize_counters(dir1, dir2, layers=14):
    """Per-stage SQ counter means of two rocprofv3 --pmc passes over the same
    bench run (pass 1: SQ_WAVES, SQ_BUSY_CYCLES, SQ_ACTIVE_INST_VALU,
    SQ_VALU_MFMA_BUSY_CYCLES, SQ_VALU_MFMA_COEXEC_CYCLES; pass 2: SQ_INSTS_VALU,
    SQ_INSTS_MFMA, SQ_INSTS_SALU, SQ_INSTS_LDS, SQ_LDS_BANK_CONFLICT,
    SQ_ACTIVE_INST_LDS), as a markdown table.  MI355X has 32 shader engines
    and 1024 SIMDs: busy cycles per SE = SQ_BUSY_CYCLES / 32; MFMA busy =
    SQ_VALU_MFMA_BUSY_CYCLES / (busy * 1024); VALU busy = 4 *
    SQ_ACTIVE_INST_VALU (quad-cycles) / (busy * 1024); VALU beside MFMA =
    SQ_VALU_MFMA_COEXEC_CYCLES / (busy * 1024); instructions per wave =
    SQ_INSTS_* / SQ_WAVES."""
    import csv
    import glob

    def load(d):
        f = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)[0]
        disp = {}
        for r in csv.DictReader(open(f)):
            e = disp.setdefault(int(r["Dispatch_Id"]), {"name": r["Kernel_Name"]})
            e[r["Counter_Name"]] = float(r["Counter_Value"])
        ours = [v for _, v in sorted(disp.items()) if "blt::" in v["name"]]
        return list(zip(_forward_stages([v["name"] for v in ours], layers), ours))

    p1, p2 = load(dir1), load(dir2)
    if [st for st, _ in p1] != [st for st, _ in p2]:
        raise ValueError("the two passes saw different dispatches")
    tot, n = {}, {}
    for (st, a), (_, b) in zip(p1, p2):
        if st is None:
            continue
        t = tot.setdefault(st, {})
        for k, v in list(a.items()) + list(b.items()):
            if k != "name":
                t[k] = t.get(k, 0.0) + v
        n[st] = n.get(st, 0) + 1
    lines = ["| stage | launches | busy cycles / SE | MFMA busy | VALU busy | VALU beside MFMA | "
             "neither | VALU / wave | MFMA / wave | SALU / wave | LDS / wave | "
             "LDS conflict / LDS active |", "|---" * 12 + "|"]
    for st in sorted(tot, key=lambda k: -tot[k]["SQ_BUSY_CYCLES"]):
        m = {k: v / n[st] for k, v in tot[st].items()}
        busy = m["SQ_BUSY_CYCLES"] / 32.0
        mf = m["SQ_VALU_MFMA_BUSY_CYCLES"] / (busy * 1024)
        va = 4 * m["SQ_ACTIVE_INST_VALU"] / (busy * 1024)
        co = m["SQ_VALU_MFMA_COEXEC_CYCLES"] / (busy * 1024)
        w = m["SQ_WAVES"]
        lines.append("| %s | %d | %d | %.1f%% | %.1f%% | %.1f%% | %.1f%% | %d | %d | %d | %d | %.2f |" % (
            st, n[st], busy, 100 * mf, 100 * va, 100 * co, 100 * (1 - mf - va + co),
            m["SQ_INSTS_VALU"] / w, m["SQ_INSTS_MFMA"] / w, m["SQ_INSTS_SALU"] / w,
            m["SQ_INSTS_LDS"] / w, m["SQ_LDS_BANK_CONFLICT"] / max(m["SQ_ACTIVE_INST_LDS"], 1.0)))
    return "\n".join(lines)


def summarize_trace(path):
    """Per-stage mean kernel duration from a rocprofv3 --kernel-trace CSV of
    bench.py (stages recovered from the dispatch order of each forward)."""
    import csv
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Dispatch_Id"]))
    rows = [r for r in rows if "blt::" in r["Kernel_Name"]]
    names = [r["Kernel_Name"] for r in rows]
    agg = {}
    for st, r in zip(_forward_stages(names, 14), rows):
        if st is None:
            continue
        kn = r["Kernel_Name"]
        d = agg.setdefault(st, [0, 0.0, kn[:kn.rfind("(")]])
        d[0] += 1
        d[1] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    print("| stage | kernel | launches | mean us | total us |")
    print("|---|---|---|---|---|")
    for st, (n, us, k) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        print("| %s | `%s` | %d | %.1f | %.0f |" % (st, k, n, us / n, us))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--config", type=int, default=4, choices=(1, 2, 3, 4, 5),
                    help="4: [16, 8192] forward + boundaries (the headline metric); "
                         "1: fused entropy + patch boundaries over f32 logits [4, 8192, 260]; "
                         "2: RMSNorm + pre-norm L2 [32768, 768] and SiLU*gate [32768, 2048], "
                         "bf16; 3: causal RoPE attention B=8 T=4096 H=12 d=64 W=512; "
                         "5: streaming ingest of variable-length documents, end to end")
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (config 4: batches, default 10; config 5: passes over "
                         "the document sample, default 1)")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--ingest-mib", type=float, default=24.0,
                    help="config 5: MiB of the seeded 1 GiB document stream to ingest per pass")
    ap.add_argument("--ingest-segment-mib", type=float, default=64.0,
                    help="config 5: documents go to the ingest driver in document-aligned "
                         "segments of about this many MiB (bounds host memory for the "
                         "outputs; one progress line per segment on stderr)")
    ap.add_argument("--pipeline", action="store_true",
                    help="measure the streaming pipeline of pipeline.rs instead (4096-byte "
                         "chunks, 2048 context): the packed many-document form and the "
                         "one-forward-per-chunk form over a prefix of the config-5 documents")
    ap.add_argument("--pipeline-mib", type=float, default=8.0,
                    help="--pipeline: MiB of the seeded document stream per pass")
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--seq", type=int, default=8192)
    ap.add_argument("--window", type=int, default=512)
    ap.add_argument("--threshold", type=float, default=1.335)
    ap.add_argument("--cpu-seq", type=int, default=4096,
                    help="tokens of the CPU-oracle sample (B=1)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--telemetry-s", type=float, default=2.0,
                    help="config 4: seconds of extra steps after the timed ones with the "
                         "GPU's power, PPT residency and clocks recorded (0 = off)")
    ap.add_argument("--power-stages", action="store_true",
                    help="each config-4 stage alone (its kernel on config-4 shapes, back to "
                         "back for --stage-s seconds) with power, PPT residency and clocks; "
                         "one JSON line")
    ap.add_argument("--stage-s", type=float, default=1.5)
    ap.add_argument("--traffic", choices=("live", "file", "off"), default="live",
                    help="config 4's roofline.traffic: live = rocprofv3 --pmc passes run by "
                         "this bench before it starts (about 15 s; the committed file when "
                         "they fail or when bench.py itself runs under rocprofv3), file = "
                         "--traffic-file, off = null")
    ap.add_argument("--traffic-file", default=os.path.join(ROOT, "profiles",
                                                           "traffic_config4.json"),
                    help="per-stage HBM bytes per launch measured with rocprofv3 --pmc")
    ap.add_argument("--summarize", nargs=4, metavar=("FETCH_DIR", "WRITE_DIR", "COPY_FETCH_DIR",
                                                     "COPY_WRITE_DIR"),
                    help="print per-stage traffic from rocprofv3 --pmc output and exit")
    ap.add_argument("--copy-bytes", type=float, default=float(2 ** 30))
    ap.add_argument("--summarize-counters", nargs=2, metavar=("PASS1_DIR", "PASS2_DIR"),
                    help="print per-stage SQ counter means of two rocprofv3 --pmc passes")
    ap.add_argument("--summarize-trace", metavar="KERNEL_TRACE_CSV",
                    help="print per-stage kernel durations from rocprofv3 --kernel-trace output")
    ap.add_argument("--copy-probe", action="store_true",
                    help="run one device copy of --copy-bytes bytes (the counter calibration "
                         "kernel for --summarize) and exit")
    args = ap.parse_args()
    if args.copy_probe:
        import torch
        x = torch.ones(int(args.copy_bytes) // 4, device="cuda")
        y = torch.empty_like(x)
        torch.cuda.synchronize()
        y.copy_(x)
        torch.cuda.synchronize()
        print("copied %d bytes" % (x.numel() * 4))
        return
    if args.summarize_trace:
        summarize_trace(args.summarize_trace)
        return
    if args.summarize_counters:
        print(summarize_counters(*args.summarize_counters))
        return
    if args.summarize:
        summarize(args)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(rows and documents are independent, so more GPUs would each take a "
              "share of them with no collective). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    # config 4's traffic passes run first, while this process has not touched
    # the GPU (each pass is a child process of its own)
    live, live_err = None, None
    if (args.config == 4 and not (args.pipeline or args.power_stages) and args.traffic == "live"
            and (args.batch, args.seq, args.window) == (16, 8192, 512)):
        if "ROCPROF_OUTPUT_PATH" in os.environ:
            live_err = "bench.py runs under rocprofv3"
        else:
            live, live_err = live_traffic(args)

    import numpy as np
    import torch

    import __graft_entry__
    __graft_entry__.load_package()
    from blt_burn_amd import model as M, patcher, synth

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if args.pipeline:
        bench_pipeline(args)
        return
    if args.power_stages:
        bench_power_stages(args)
        return
    if args.config == 5:
        bench_ingest(args)
        return
    if args.config in (1, 2, 3):
        (bench_config1, bench_config2, bench_config3)[args.config - 1](args)
        return
    if args.steps is None:
        args.steps = 10
    dev = torch.device("cuda", 0)
    cfg = M.entropy_model_config()
    F, D, V, L, H = 2048, cfg.dim, cfg.vocab_size, cfg.n_layers, cfg.resolved_n_heads()
    B, T, W = args.batch, args.seq, args.window
    seed = synth.config_seed(4)
    weights = M.random_weights(cfg, seed, hidden=F)
    tok_np = synth.tokens(seed, (B, T))
    tok = torch.from_numpy(tok_np).to(dev)
    model = M.LMTransformer(cfg, weights, device=0, max_tokens=B * T, window=W)
    outs = {n: torch.empty(s, dtype=torch.float32, device=dev) for n, s in
            (("logits", (B, T, V)), ("pre_norm_embeddings", (B, T, D)),
             ("embedding_norms", (B, T)), ("entropies", (B, T)), ("coherence_scores", (B, T)))}
    bnd = tuple(torch.empty(s, dtype=torch.int32, device=dev)
                for s in ((B, T), (B, T), (B, T), (B,)))

    def step():
        o = model.forward_with_embeddings(tok, out=outs)
        patcher.patch_boundaries(o.entropies, args.threshold, patcher.PATCH_MONOTONIC, out=bnd)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    model.read_profile()
    model.set_profiling(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    prof = model.read_profile()
    model.set_profiling(False)
    sec = (t1 - t0) / max(args.steps, 1)
    value = B * T / sec

    Mtok = B * T
    layer_stages = ("qkv_gemm_rope", "attention", "o_gemm_residual", "w13_gemm_silu",
                    "w2_gemm_residual")
    total_flops = L * sum(stage_flops(s, Mtok, B, T, D, F, V, H, W) for s in layer_stages) \
        + stage_flops("head_gemm", Mtok, B, T, D, F, V, H, W)
    stage_ms = {s: round(ms / max(args.steps, 1), 4) for s, (ms, n) in prof.items() if n}
    mfma_stages = {s: v for s, v in prof.items() if stage_flops(s, Mtok, B, T, D, F, V, H, W)
                   and v[1]}
    dom = max(mfma_stages, key=lambda s: mfma_stages[s][0])
    ms_tot, launches = mfma_stages[dom]
    per_launch_ms = ms_tot / launches
    achieved = stage_flops(dom, Mtok, B, T, D, F, V, H, W) / (per_launch_ms * 1e-3) / 1e12
    traffic, traffic_st, traffic_src = None, None, None
    if live is not None and (live["stages"].get(dom) or {}).get("launches"):
        traffic_st = live["stages"][dom]
        traffic_src = "rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE in this run"
    elif (args.traffic != "off" and os.path.exists(args.traffic_file)
          and (B, T, W) == (16, 8192, 512)):
        traffic_st = json.load(open(args.traffic_file)).get("stages", {}).get(dom)
        traffic_src = os.path.relpath(args.traffic_file, ROOT) + " (committed)" + (
            "; live passes: " + live_err if live_err else "")
    if traffic_st:
        traffic = int(traffic_st["fetch_bytes"] + traffic_st["write_bytes"])
    roofline = {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2),
                "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                "launch_ms": round(per_launch_ms, 4)}
    if traffic_st:
        roofline.update({"traffic_fetch": int(traffic_st["fetch_bytes"]),
                         "traffic_write": int(traffic_st["write_bytes"]),
                         "traffic_source": traffic_src})
    step_tflops = total_flops / sec / 1e12
    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "bytes/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded Zipf(1.1) printable bytes + 5% uniform, +4 offset; "
                "random-init bf16 weights N(0,0.02), norms 1+N(0,0.02))",
        "config": {"workload": "config4: entropy-model forward_with_embeddings + monotonic "
                               "patch boundaries", "batch": B, "seq_len": T, "window": W,
                   "layers": L, "dim": D, "heads": H, "ffn_hidden": F, "vocab": V,
                   "threshold": args.threshold},
        "roofline": _with_achievable(roofline),
        "step_roofline": _with_achievable({"bound": "mfma", "achieved": round(step_tflops, 2),
                                           "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                                           "frac": round(step_tflops / PEAK_BF16_TFLOPS, 4),
                                           "flop_per_byte": round(total_flops / Mtok, 1)}),
        "stage_ms_per_step": stage_ms,
        "cpu_baseline": None,
    }
    if args.telemetry_s > 0:
        # after the timed steps, outside `value`: what the power manager did
        # while the same step ran back to back
        result["telemetry"] = telemetry_window(step, args.telemetry_s, sync_every=2)

    if not args.no_cpu:
        import oracle  # the checker / CPU baseline only
        cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
        os.environ["OMP_NUM_THREADS"] = str(cores)
        Tc = min(args.cpu_seq, T)
        f32 = {k: synth.bf16_to_f32(v) for k, v in weights.items()}
        ow = {"emb": f32["tok_embeddings"], "attn_norm": f32["attention_norm"],
              "ffn_norm": f32["ffn_norm"], "wq": f32["wq"], "wk": f32["wk"], "wv": f32["wv"],
              "wo": f32["wo"], "w1": f32["w1"], "w2": f32["w2"], "w3": f32["w3"],
              "norm": f32["norm"], "out": f32["output"]}
        sample = tok_np[:1, :Tc]
        oc = dict(dim=D, n_layers=L, n_heads=H, hidden=F, vocab=V, max_seqlen=cfg.max_seqlen,
                  norm_eps=cfg.norm_eps, rope_theta=cfg.rope_theta, window=W)
        c0 = time.perf_counter()
        ref = oracle.model_forward(oc, ow, sample)
        c1 = time.perf_counter()
        g = model.forward_with_embeddings(torch.from_numpy(np.ascontiguousarray(sample)).to(dev))
        Hg = g.entropies.cpu().numpy()
        ng = g.embedding_norms.cpu().numpy()
        result["cpu_baseline"] = {
            "value": round(Tc / (c1 - c0), 2), "unit": "bytes/s", "cores": cores,
            "kind": "port",
            "sample": "B=1, T=%d prefix of the config-4 token stream, same weights, "
                      "fp32 C restatement of the NdArray path (oracle/oracle.c, OpenMP), "
                      "%.1f s" % (Tc, c1 - c0),
            "parity_on_sample": {
                "entropy_max_abs": float(np.abs(Hg - ref["entropies"]).max()),
                "norm_max_rel": float((np.abs(ng - ref["embedding_norms"])
                                       / ref["embedding_norms"]).max())},
        }
    print(json.dumps(result), flush=True)


def _timed(fn, steps, warmup):
    """Mean ms of fn() over `steps` calls, bracketed by HIP events on the current
    stream (the stream the library launches on)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


_PEAKS = {}


def achievable_peaks():
    """The dense bf16 MFMA rate and the HBM copy bandwidth this GPU sustains
    (blt_probe_mfma_bf16 / blt_probe_copy, timed with HIP events): the
    published peaks assume a clock the chip does not hold under a full MFMA
    load, so fractions are also reported against these."""
    if _PEAKS:
        return _PEAKS
    import torch
    from blt_burn_amd import _lib
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks, iters = cus * 4, 2048
    sink = torch.empty(blocks * 256, device="cuda")
    ms = _timed(lambda: _lib.check(L.blt_probe_mfma_bf16(blocks, iters, sink.data_ptr(), stream),
                                   "probe_mfma"), 5, 2)
    _PEAKS["mfma_bf16_tflops"] = round(L.blt_probe_mfma_flops(blocks, iters) / (ms * 1e-3) / 1e12, 1)
    nbytes = 1 << 30
    src = torch.ones(nbytes // 4, device="cuda")
    dst = torch.empty_like(src)
    ms = _timed(lambda: _lib.check(L.blt_probe_copy(src.data_ptr(), dst.data_ptr(), nbytes, stream),
                                   "probe_copy"), 5, 2)
    _PEAKS["copy_gbs"] = round(2 * nbytes / (ms * 1e-3) / 1e9, 1)
    del src, dst, sink
    return _PEAKS


def _with_achievable(roof):
    """roofline object + the achievable peak of its bound and the fraction of it."""
    pk = achievable_peaks()
    ach = pk["mfma_bf16_tflops"] if roof["bound"] == "mfma" else pk["copy_gbs"]
    roof["achievable_peak"] = ach
    roof["frac_of_achievable"] = round(roof["achieved"] / ach, 4)
    return roof


def _amdsmi_handle():
    """amdsmi's handle of the GPU the bench runs on, or None when the module or
    the device's metrics table is not available."""
    try:
        import amdsmi
        amdsmi.amdsmi_init()
        hs = amdsmi.amdsmi_get_processor_handles()
        if not hs:
            return None
        amdsmi.amdsmi_get_gpu_metrics_info(hs[0])
        return hs[0]
    except Exception:  # no telemetry on this system: the bench line omits it
        return None


def _metric(m, key):
    v = m.get(key)
    return v if isinstance(v, (int, float)) else None


def telemetry_window(fn, seconds, sync_every=8):
    """Runs fn() back to back for about `seconds` and reports what the GPU's
    power manager saw meanwhile, from amdsmi's metrics table (the firmware
    refreshes it every few tens of ms; every figure below is a delta of its
    accumulators between the first and last table read inside the busy
    window, timed by the table's own clock):
      power_w        mean socket power: energy accumulator delta (times the
                     counter resolution) over system_clock_counter delta
      residency      fraction of the window each limiter was active
                     (<name>_residency_acc delta / accumulation_counter delta):
                     ppt = package power limit, prochot, socket_thm, vr_thm,
                     hbm_thm = thermal limits
      xcd_*          per XCD, fraction of the window its graphics clock was
                     held below the host limit (total, by PPT, by thermal) or
                     its utilisation was low, from xcp_stats
      gfxclk_mhz     current graphics clock of the 8 XCDs, read every 20 ms by
                     a host thread (mean, min, max over reads and XCDs)
      socket_power_samples_w  the table's current socket power over the reads
    plus ms per call of fn over the window.  None without amdsmi."""
    import threading
    import torch
    h = _amdsmi_handle()
    if h is None:
        return None
    import amdsmi
    try:
        res_uj = float(amdsmi.amdsmi_get_energy_count(h).get("counter_resolution", 15.259))
    except Exception:  # MI300-series energy unit
        res_uj = 15.259

    snaps = []  # (host time, metrics table)
    stop = threading.Event()

    def sample():
        while not stop.is_set():
            snaps.append((time.perf_counter(), amdsmi.amdsmi_get_gpu_metrics_info(h)))
            stop.wait(0.02)

    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    th = threading.Thread(target=sample, daemon=True)
    th.start()
    n = 0
    while time.perf_counter() - t0 < seconds:
        fn()
        n += 1
        if n % sync_every == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    stop.set()
    th.join()
    out = {"seconds": round(t1 - t0, 3), "calls": n, "ms_per_call": round((t1 - t0) * 1e3 / n, 4)}
    try:
        out["power_cap_w"] = round(amdsmi.amdsmi_get_power_info(h)["power_limit"] / 1e6, 1)
    except Exception:  # the cap is informational
        out["power_cap_w"] = None
    busy = [m for t, m in snaps if t0 + 0.1 < t < t1]  # past the ramp
    # distinct table refreshes only (the driver hands out a cached copy in between)
    uniq = []
    for m in busy:
        if not uniq or m.get("system_clock_counter") != uniq[-1].get("system_clock_counter"):
            uniq.append(m)
    out["table_refreshes"] = len(uniq)
    if len(uniq) >= 2:
        ma, mb = uniq[0], uniq[-1]

        def d(k):
            x, y = _metric(ma, k), _metric(mb, k)
            return None if x is None or y is None else y - x

        dt_ns, de = d("system_clock_counter"), d("energy_accumulator")
        if dt_ns and de is not None:
            out["power_w"] = round(de * res_uj * 1e-6 / (dt_ns * 1e-9), 1)
        da = d("accumulation_counter")
        if da:
            out["residency"] = {k: round(d(k + "_residency_acc") / da, 3)
                                for k in ("ppt", "prochot", "socket_thm", "vr_thm", "hbm_thm")
                                if d(k + "_residency_acc") is not None}
            for name, key in (("xcd_below_host_limit", "gfx_below_host_limit_total_acc"),
                              ("xcd_below_host_limit_ppt", "gfx_below_host_limit_ppt_acc"),
                              ("xcd_below_host_limit_thm", "gfx_below_host_limit_thm_acc"),
                              ("xcd_low_utilization", "gfx_low_utilization_acc")):
                k = "xcp_stats." + key
                if isinstance(ma.get(k), list) and isinstance(mb.get(k), list):
                    v = [round((y - x) / da, 3) for x, y in zip(ma[k][0], mb[k][0])
                         if isinstance(x, int) and isinstance(y, int)]
                    if v:
                        out[name] = v
    powers = [p for p in (_metric(m, "current_socket_power") for m in uniq) if p is not None]
    clocks = [x for m in busy for x in (m.get("current_gfxclks") or [])
              if isinstance(x, (int, float))]
    if powers:
        out["socket_power_samples_w"] = {"mean": round(sum(powers) / len(powers), 1),
                                         "max": max(powers), "n": len(powers)}
    if clocks:
        out["gfxclk_mhz"] = {"mean": round(sum(clocks) / len(clocks), 1), "min": min(clocks),
                             "max": max(clocks), "n": len(clocks)}
    return out


def bench_power_stages(args):
    """Each stage of the config-4 forward alone, on its config-4 shapes (M =
    16 x 8192 rows), run back to back for --stage-s seconds under
    telemetry_window: socket power, PPT residency and XCD clocks per stage,
    beside the MFMA loop probe (the matrix cores' power at full load), the
    device copy probe (HBM at full load) and the whole step.  Tells whether a
    stage is held by the package power limit and at what clock it runs."""
    import torch
    from blt_burn_amd import _lib, model as M, patcher, synth
    L = _lib.lib()
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream().cuda_stream
    B, T, W, D, F, Hh = args.batch, args.seq, args.window, 768, 2048, 12
    Mr = B * T
    g = torch.Generator(device=dev)
    g.manual_seed(synth.config_seed(4))

    def rnd(shape, std=1.0):
        return (torch.randn(shape, generator=g, device=dev) * std).to(torch.bfloat16)

    a768, h2048, qkv, attn = rnd((Mr, D)), rnd((Mr, F)), rnd((Mr, 3 * D)), rnd((Mr, D))
    w13, wqkv, wo, w2 = rnd((2 * F, D), 0.02), rnd((3 * D, D), 0.02), rnd((D, D), 0.02), \
        rnd((D, F), 0.02)
    resid = torch.randn((Mr, D), generator=g, device=dev)
    hout, qout = torch.empty((Mr, F), dtype=torch.bfloat16, device=dev), \
        torch.empty((Mr, 3 * D), dtype=torch.bfloat16, device=dev)
    cs = torch.empty((T, 32, 2), dtype=torch.float32, device=dev)
    _lib.check(L.blt_rope_table_f32(cs.data_ptr(), 64, T, 10000.0, stream), "rope_table")

    def gemm(A, Bt, C, N, K, ldc, epi, rope_cols=0):
        _lib.check(L.blt_gemm_bf16_epilogue(A.data_ptr(), Bt.data_ptr(), C.data_ptr(), Mr, N, K,
                                            K, K, ldc, epi, 0, rope_cols, T,
                                            cs.data_ptr() if rope_cols else None, stream), "gemm")

    def attention():
        _lib.check(L.blt_fused_attention_bf16(
            qkv.data_ptr(), qkv[:, D:].data_ptr(), qkv[:, 2 * D:].data_ptr(), attn.data_ptr(),
            B, Hh, T, 64, T * 3 * D, 64, 3 * D, T * 3 * D, 64, 3 * D, T * D, 64, D, 1, W, 0.0,
            None, stream), "attention")

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.empty(cus * 4 * 256, device=dev)
    src = torch.ones((1 << 30) // 4, device=dev)
    dst = torch.empty_like(src)
    cfg = M.entropy_model_config()
    seed = synth.config_seed(4)
    model = M.LMTransformer(cfg, M.random_weights(cfg, seed, hidden=F), device=0,
                            max_tokens=Mr, window=W)
    tok = torch.from_numpy(synth.tokens(seed, (B, T))).to(dev)
    outs = {n: torch.empty(sh, dtype=torch.float32, device=dev) for n, sh in
            (("logits", (B, T, 260)), ("pre_norm_embeddings", (B, T, D)),
             ("embedding_norms", (B, T)), ("entropies", (B, T)), ("coherence_scores", (B, T)))}

    def step():
        o = model.forward_with_embeddings(tok, out=outs)
        patcher.patch_boundaries(o.entropies, args.threshold, patcher.PATCH_MONOTONIC)

    stages = [
        ("w13_gemm_silu", lambda: gemm(a768, w13, hout, 2 * F, D, F, _lib.EPI_SILU_GATE), 8),
        ("qkv_gemm_rope", lambda: gemm(a768, wqkv, qout, 3 * D, D, 3 * D, _lib.EPI_QKV_ROPE,
                                       2 * D), 8),
        ("w2_gemm_residual", lambda: gemm(h2048, w2, resid, D, F, D, _lib.EPI_RESID_F32), 8),
        ("o_gemm_residual", lambda: gemm(attn, wo, resid, D, D, D, _lib.EPI_RESID_F32), 8),
        ("attention", attention, 8),
        ("mfma_probe", lambda: _lib.check(L.blt_probe_mfma_bf16(cus * 4, 2048, sink.data_ptr(),
                                                                stream), "probe"), 8),
        ("copy_probe", lambda: _lib.check(L.blt_probe_copy(src.data_ptr(), dst.data_ptr(),
                                                           1 << 30, stream), "copy"), 8),
        ("step", step, 2),
    ]
    res = {}
    for name, fn, sync_every in stages:
        print("power stage %s" % name, file=sys.stderr, flush=True)
        res[name] = telemetry_window(fn, args.stage_s, sync_every=sync_every)
        res[name]["event_ms"] = round(_timed(fn, 10, 2), 4)
    print(json.dumps({"power_stages": res, "shapes": {"rows": Mr, "dim": D, "ffn": F,
                                                     "heads": Hh, "window": W}}), flush=True)


def _cpu_cores():
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    os.environ["OMP_NUM_THREADS"] = str(cores)
    return cores


def _graph_launch_ms(fn, launches, replays=10):
    """Mean ms per call of fn() when `launches` calls are replayed back to back
    from a HIP graph (no host gaps between them), HIP events on the stream
    the graph is replayed on."""
    import torch
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(launches):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (replays * launches)


def bench_config1(args):
    """Config 1: softmax entropy over f32 logits [4, 8192, 260] ~ N(0, 2) and the
    global (H > 1.33) and monotonic (dH > 0.2) boundaries with their start
    indices and lengths, inputs in HBM.  One call of entropy_patch_boundaries
    per step (its prepared form, patcher.EntropyPatchPlan): a flags kernel
    reads the logits once and writes the entropies, both masks and per-tile
    counts, a compaction kernel writes the starts and lengths.  value =
    positions per second of the eager step; roofline = the
    call's HBM rate (its algorithmic bytes over its mean duration, calls
    replayed back to back from a HIP graph) against 8 TB/s."""
    import numpy as np
    import torch
    from blt_burn_amd import patcher, synth
    steps = args.steps or 50
    B, T, V = 4, 8192, 260
    logits_np = synth.normal_f32(synth.config_seed(1), (B, T, V), 0.0, 2.0)
    logits = torch.from_numpy(logits_np).cuda()
    rules = [(patcher.PATCH_GLOBAL, 1.33), (patcher.PATCH_MONOTONIC, 0.2)]
    bnd = [tuple(torch.empty(s, dtype=torch.int32, device="cuda")
                 for s in ((B, T), (B, T), (B, T), (B,))) for _ in range(2)]
    # the prepared form of entropy_patch_boundaries (outputs and arguments
    # bound once, as a serving loop calls it); the function form checks a
    # dozen tensors per call and is timed beside it as eager_function_ms
    plan = patcher.EntropyPatchPlan(B, T, V, rules)
    bnd = plan.outs
    Hbuf = torch.empty((B, T), dtype=torch.float32, device="cuda")

    def step_fn():
        patcher.entropy_patch_boundaries(logits, rules, out=bnd, entropies=Hbuf)

    def step():
        plan(logits)

    ms = _timed(step, steps, args.warmup)
    ms_fn = _timed(step_fn, steps, args.warmup)
    ms_k = _graph_launch_ms(step, 20)
    # the entropy kernel alone on the same logits (fused_entropy), for its HBM rate
    from blt_burn_amd import fused_ops
    ms_e = _graph_launch_ms(lambda: fused_ops.fused_entropy(logits, V), 20)
    n = B * T
    counts = [int(bnd[r][3].sum()) for r in range(2)]
    # logits read, entropies written, both masks, the starts and lengths written
    k_bytes = n * (V * 4 + 4) + 2 * n * 4 + 8 * sum(counts)
    gbs = k_bytes / (ms_k * 1e-3) / 1e9
    result = {
        "metric": "positions/sec through fused entropy + global and monotonic patch boundaries "
                  "(config 1, f32 logits [4, 8192, 260])",
        "value": round(n / (ms * 1e-3), 1), "unit": "positions/s", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: logits ~ N(0, 2.0), seed %d" % synth.config_seed(1),
        "config": {"workload": "config1: entropy + global (1.33) and monotonic (0.2) patch "
                               "boundaries, starts and lengths, one pass",
                   "batch": B, "seq_len": T, "vocab": V,
                   "host_call": "patcher.EntropyPatchPlan (prepared entropy_patch_boundaries)"},
        "eager_function_ms": round(ms_fn, 4),
        "roofline": _with_achievable({"bound": "hbm",
                                      "kernel": "entropy_flags_half_kernel<2, 1, 16> + "
                                                "patch_compact_kernel<1> (one call)",
                                      "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                      "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                                      "traffic": None, "launch_ms": round(ms_k, 5),
                                      "bytes_per_launch": k_bytes}),
        "starts": {"global": counts[0], "monotonic": counts[1]},
        "entropy_kernel_only": {"kernel": "entropy_half_kernel<float, 2, 1> (fused_entropy)",
                                "ms": round(ms_e, 5),
                                "GB/s": round(n * (V * 4 + 4) / (ms_e * 1e-3) / 1e9, 1),
                                "frac": round(n * (V * 4 + 4) / (ms_e * 1e-3) / 1e9 /
                                              PEAK_HBM_GBS, 4)},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        import oracle
        cores = _cpu_cores()
        Bs = B
        c0 = time.perf_counter()
        reps = 0
        while True:
            Hc = oracle.entropy(logits_np[:Bs])
            oracle.patch_mask(Hc, 1.33, 1)
            oracle.patch_mask(Hc, 0.2, 0)
            reps += 1
            c1 = time.perf_counter()
            if c1 - c0 > 2.0:
                break
        Hg = plan.entropies.cpu().numpy()[:Bs]
        m_g = bnd[1][0].cpu().numpy()[:Bs]
        result["cpu_baseline"] = {
            "value": round(reps * Bs * T / (c1 - c0), 1), "unit": "positions/s",
            "cores": cores, "kind": "port",
            "sample": "the whole [4, 8192, 260] input through the C oracle's entropy (OpenMP) "
                      "and both masks, %d passes in %.2f s" % (reps, c1 - c0),
            "parity_on_sample": {"entropy_max_abs": float(np.abs(Hg - Hc).max()),
                                 "monotonic_mask_equal": bool(
                                     (m_g == oracle.patch_mask(Hg, 0.2, 0)).all())}}
    print(json.dumps(result), flush=True)


def bench_config2(args):
    """Config 2: RMSNorm (eps 1e-5 after the root) with the pre-norm L2 norms over
    bf16 x [32768, 768], and SiLU(a) * b over bf16 [32768, 2048].  Both are
    HBM-bound: RMSNorm+L2 moves 1536 + 1536 + 4 B per row, SiLU*gate 6 B per
    element.  value = rows per second through both ops; roofline = each
    kernel's HBM rate against 8 TB/s (the slower of the two as `roofline`)."""
    import numpy as np
    import torch
    from blt_burn_amd import fused_ops, synth
    steps = args.steps or 50
    R, D, F = 32768, 768, 2048
    seed = synth.config_seed(2)
    x = torch.from_numpy(synth.normal_f32(seed, (1, R, D))).cuda().to(torch.bfloat16)
    w = torch.from_numpy(synth.normal_f32(seed + 1, (D,), 1.0, 0.02)).cuda().to(torch.bfloat16)
    a = torch.from_numpy(synth.normal_f32(seed + 2, (R, F))).cuda().to(torch.bfloat16)
    b = torch.from_numpy(synth.normal_f32(seed + 3, (R, F))).cuda().to(torch.bfloat16)
    l2 = torch.empty((1, R), dtype=torch.float32, device="cuda")
    keep = {}

    def rms():
        keep["y"] = fused_ops.fused_rms_norm(x, w, 1e-5, l2_out=l2)

    def silu():
        keep["s"] = fused_ops.fused_silu_gate(a, b)

    # the drop-in boundary: each op's C entry with its arguments bound once (as
    # a binding calls it); the Python functions, which check and allocate per
    # call and are host-bound next to an 18 us kernel, are timed beside it
    from blt_burn_amd import _lib
    from blt_burn_amd._torch import stream_ptr
    rms(), silu()
    torch.cuda.synchronize()
    L = _lib.lib()
    st = stream_ptr(x.device)
    y_c, s_c = torch.empty_like(x), torch.empty_like(a)
    rms_args = (x.data_ptr(), w.data_ptr(), y_c.data_ptr(), l2.data_ptr(), R, D, 1e-5,
                fused_ops.EPS_AFTER_SQRT, st)
    silu_args = (a.data_ptr(), b.data_ptr(), s_c.data_ptr(), R * F, st)
    f_rms, f_silu = L.blt_fused_rms_norm_bf16, L.blt_fused_silu_gate_bf16

    def rms_c():
        rc = f_rms(*rms_args)
        if rc:
            _lib.check(rc, "fused_rms_norm")

    def silu_c():
        rc = f_silu(*silu_args)
        if rc:
            _lib.check(rc, "fused_silu_gate")

    ms_rms = _timed(rms_c, steps, args.warmup)
    ms_silu = _timed(silu_c, steps, args.warmup)
    ms_rms_fn = _timed(rms, steps, args.warmup)
    ms_silu_fn = _timed(silu, steps, args.warmup)
    # the bound calls compute what the functions return
    if not (torch.equal(y_c, keep["y"]) and torch.equal(s_c, keep["s"])):
        raise RuntimeError("config 2: the C entries and the Python functions disagree")
    rms_bytes = R * (2 * D * 2 + 4) + D * 2
    silu_bytes = R * F * 6
    g_rms = rms_bytes / (ms_rms * 1e-3) / 1e9
    g_silu = silu_bytes / (ms_silu * 1e-3) / 1e9
    worst = ("rmsnorm_kernel", g_rms, ms_rms, rms_bytes) if g_rms < g_silu else \
        ("silu_gate_bf16_kernel", g_silu, ms_silu, silu_bytes)
    result = {
        "metric": "rows/sec through RMSNorm+L2 [., 768] and SiLU*gate [., 2048] (config 2, bf16)",
        "value": round(R / ((ms_rms + ms_silu) * 1e-3), 1), "unit": "rows/s", "n_gpus": 1,
        "steps": steps, "warmup": args.warmup, "ms_per_step": round(ms_rms + ms_silu, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: x, a, b ~ N(0, 1), w ~ 1 + N(0, 0.02), seed %d" % seed,
        "config": {"workload": "config2: fused_rms_norm (+pre-norm L2) and fused_silu_gate",
                   "rows": R, "dim": D, "ffn": F, "eps": 1e-5},
        "roofline": _with_achievable({"bound": "hbm", "kernel": worst[0],
                                      "achieved": round(worst[1], 1), "peak": PEAK_HBM_GBS,
                                      "unit": "GB/s", "frac": round(worst[1] / PEAK_HBM_GBS, 4),
                                      "traffic": None, "launch_ms": round(worst[2], 4),
                                      "bytes_per_launch": worst[3]}),
        "kernels": {"rmsnorm_l2": {"ms": round(ms_rms, 4), "GB/s": round(g_rms, 1),
                                   "frac": round(g_rms / PEAK_HBM_GBS, 4)},
                    "silu_gate": {"ms": round(ms_silu, 4), "GB/s": round(g_silu, 1),
                                  "frac": round(g_silu / PEAK_HBM_GBS, 4)}},
        "eager_function_ms": {"rmsnorm_l2": round(ms_rms_fn, 4),
                              "silu_gate": round(ms_silu_fn, 4)},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        import oracle
        cores = _cpu_cores()
        n = 4096
        xs = x[0, :n].float().cpu().numpy()
        ws = w.float().cpu().numpy()
        as_, bs = a[:n].float().cpu().numpy(), b[:n].float().cpu().numpy()
        c0 = time.perf_counter()
        reps = 0
        while True:
            yr = oracle.rms_norm(xs, ws, 1e-5, 0)
            lr = oracle.l2_norm(xs)
            sr = oracle.silu_gate(as_, bs)
            reps += 1
            c1 = time.perf_counter()
            if c1 - c0 > 2.0:
                break
        yg = keep["y"][0, :n].float().cpu().numpy()
        sg = keep["s"][:n].float().cpu().numpy()
        result["cpu_baseline"] = {
            "value": round(reps * n / (c1 - c0), 1), "unit": "rows/s", "cores": cores,
            "kind": "port",
            "sample": "first %d rows through the C oracle's rms_norm, l2_norm and silu_gate "
                      "(f32, OpenMP), %d passes in %.2f s" % (n, reps, c1 - c0),
            "parity_on_sample": {
                "rmsnorm_max_abs": float(np.abs(yg - yr).max()),
                "l2_max_rel": float((np.abs(l2[0, :n].cpu().numpy() - lr) / lr).max()),
                "silu_gate_max_abs": float(np.abs(sg - sr).max())}}
    print(json.dumps(result), flush=True)


def bench_config3(args):
    """Config 3: causal attention with RoPE (theta 10000, half-split) and a
    512-key window, bf16 q, k, v [8, 12, 4096, 64] ~ N(0, 1), f32 softmax.
    value = visible (query, key) pairs per second; roofline = 4 d = 256 FLOP
    per visible pair over the fused call (RoPE pre-pass + attention kernel)
    against 2.5 PFLOP/s bf16; the attention kernel alone is reported beside it."""
    import numpy as np
    import torch
    from blt_burn_amd import fused_ops, synth
    steps = args.steps or 20
    B, H, T, d, W = 8, 12, 4096, 64, 512
    seed = synth.config_seed(3)
    qkv = [torch.from_numpy(synth.normal_f32(seed + i, (B, H, T, d))).cuda().to(torch.bfloat16)
           for i in range(3)]
    keep = {}

    def run_rope():
        keep["o"] = fused_ops.fused_attention(*qkv, True, window=W, rope_theta=10000.0)

    def run_plain():
        fused_ops.fused_attention(*qkv, True, window=W, rope_theta=0.0)

    ms = _timed(run_rope, steps, args.warmup)
    ms_attn = _timed(run_plain, steps, args.warmup)
    pairs = attention_pairs(T, W) * B * H
    flops = 4.0 * d * pairs
    tf = flops / (ms * 1e-3) / 1e12
    tf_attn = flops / (ms_attn * 1e-3) / 1e12
    result = {
        "metric": "visible (query, key) pairs/sec of causal RoPE attention, window 512 "
                  "(config 3, bf16)",
        "value": round(pairs / (ms * 1e-3), 1), "unit": "pairs/s", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: q, k, v ~ N(0, 1), seed %d" % seed,
        "config": {"workload": "config3: fused_attention causal, RoPE theta 10000, window 512",
                   "batch": B, "heads": H, "seq_len": T, "head_dim": d, "window": W},
        "roofline": _with_achievable({"bound": "mfma", "kernel": "rope pre-pass + attn_fwd_kernel",
                                      "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS,
                                      "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                                      "traffic": None, "launch_ms": round(ms, 4),
                                      "flop_per_launch": flops}),
        "attention_kernel_only": {"ms": round(ms_attn, 4), "TFLOP/s": round(tf_attn, 2),
                                  "frac": round(tf_attn / PEAK_BF16_TFLOPS, 4)},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        import oracle
        cores = _cpu_cores()
        q, k, v = (t[:1].float().cpu().numpy() for t in qkv)
        c0 = time.perf_counter()
        ref = oracle.attention(q, k, v, True, W, 10000.0)
        c1 = time.perf_counter()
        got = keep["o"][:1].float().cpu().numpy()
        result["cpu_baseline"] = {
            "value": round(attention_pairs(T, W) * H / (c1 - c0), 1), "unit": "pairs/s",
            "cores": cores, "kind": "port",
            "sample": "batch row 0 (12 heads x 4096) through the C oracle's fp32 attention "
                      "(RoPE, window 512, OpenMP), %.2f s" % (c1 - c0),
            "parity_on_sample": {"max_abs": float(np.abs(got - ref).max())}}
    print(json.dumps(result), flush=True)


def _oracle_weights(weights):
    from blt_burn_amd import synth
    f32 = {k: synth.bf16_to_f32(v) for k, v in weights.items()}
    return {"emb": f32["tok_embeddings"], "attn_norm": f32["attention_norm"],
            "ffn_norm": f32["ffn_norm"], "wq": f32["wq"], "wk": f32["wk"], "wv": f32["wv"],
            "wo": f32["wo"], "w1": f32["w1"], "w2": f32["w2"], "w3": f32["w3"],
            "norm": f32["norm"], "out": f32["output"]}


def bench_ingest(args):
    """Config 5: seeded log-normal byte documents (median 2 KiB, clipped 256 B - 64 KiB,
    content as config 4) -> tokenizer -> native ingest (chunks of 8192 with 512
    overlap packed into [16, 8192] rows, pinned double-buffered copies) -> per-document
    entropies, norms, coherence, patch starts / lengths in host memory.  value =
    document bytes / second end to end (overlap recompute and padding are cost)."""
    import numpy as np

    from blt_burn_amd import ingest as I, model as M, synth, tokenizer as tk

    steps = args.steps if args.steps is not None else 1
    cfg = M.entropy_model_config()
    F, D, V, L, H = 2048, cfg.dim, cfg.vocab_size, cfg.n_layers, cfg.resolved_n_heads()
    B, T, W = args.batch, args.seq, args.window
    seed = synth.config_seed(5)
    weights = M.random_weights(cfg, seed, hidden=F)
    model = M.LMTransformer(cfg, weights, device=0, max_tokens=B * T, window=W)
    conf = I.BltConfig(threshold=args.threshold, max_seq_len=T, chunk_overlap=512)
    ing = I.StreamingIngest(model, conf, rows=B, row_len=T)
    nbytes = int(args.ingest_mib * 2 ** 20)
    data, off = synth.documents(seed, nbytes)
    wdata, woff = synth.documents(seed + 1, 2 ** 20)
    # documents go to the ingest driver in segments of about
    # --ingest-segment-mib; a background thread reads and tokenizes segment
    # i + 1 while segment i runs on the GPU (ingest.StreamingIngest.stream)
    seg = max(1, int(args.ingest_segment_mib * 2 ** 20))
    n_seg = max(1, -(-int(off[-1]) // seg))

    def docs(d, o):
        return ((str(i), d[o[i]:o[i + 1]].tobytes()) for i in range(o.size - 1))

    for _ in range(args.warmup):
        for _seg in ing.stream(docs(wdata, woff), seg):
            pass
    model.read_profile()
    model.set_profiling(True)
    st = {}
    t0 = time.perf_counter()
    for _ in range(steps):
        st = {}
        for k, (_ids, _toks, r) in enumerate(ing.stream(docs(data, off), seg)):
            if k == 0:
                res = r  # the parity sample below reads the first documents
            for name, v in ing.last_stats().items():
                st[name] = st.get(name, 0) + v
            if n_seg > 1:
                print("config 5: segment %d/~%d done, %.1f s" % (
                    k + 1, n_seg, time.perf_counter() - t0), file=sys.stderr, flush=True)
            del r
    t1 = time.perf_counter()
    prof = model.read_profile()
    model.set_profiling(False)
    sec = (t1 - t0) / steps
    gpu_ms = sum(ms for ms, n in prof.values()) / steps
    dom = "w13_gemm_silu"
    ms_tot, launches = prof[dom]
    per_launch_ms = ms_tot / launches
    Mtok = B * T
    achieved = stage_flops(dom, Mtok, B, T, D, F, V, H, W) / (per_launch_ms * 1e-3) / 1e12
    result = {
        "metric": "input bytes/sec ingested end to end (config 5 streaming ingest, BLT entropy "
                  "model, bf16)",
        "value": round(nbytes / sec, 1), "unit": "bytes/s", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: %.1f MiB prefix of the seeded config-5 document stream "
                "(%d documents, %d segment(s)), random-init bf16 weights" % (
                    nbytes / 2 ** 20, off.size - 1, n_seg),
        "config": {"workload": "config5: tokenize (background thread) + chunk/overlap + packed "
                               "forward + stitch + per-document monotonic boundaries, host in / "
                               "host out",
                   "rows": B, "row_len": T, "chunk_len": T, "overlap": 512, "window": W,
                   "threshold": args.threshold},
        "ingest": {"batches": st["batches"], "documents": st["documents"],
                   "tokens": st["tokens"], "tokens_computed": st["tokens_computed"],
                   "row_tokens": st["row_tokens"],
                   "useful_fraction": round(st["tokens"] / st["row_tokens"], 4),
                   "gpu_model_ms": round(gpu_ms, 1),
                   "gpu_model_busy_fraction": round(gpu_ms / (sec * 1e3), 4)},
        "roofline": _with_achievable({"bound": "mfma", "kernel": dom,
                                      "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                                      "unit": "TFLOP/s",
                                      "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                                      "traffic": None, "launch_ms": round(per_launch_ms, 4)}),
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        import oracle  # the checker / CPU baseline only
        cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
        os.environ["OMP_NUM_THREADS"] = str(cores)
        oc = dict(dim=D, n_layers=L, n_heads=H, hidden=F, vocab=V, max_seqlen=cfg.max_seqlen,
                  norm_eps=cfg.norm_eps, rope_theta=cfg.rope_theta, window=W)
        ow = _oracle_weights(weights)
        toks, toff = tk.tokenize_documents(data, off)
        n_docs, done_bytes, worst = 0, 0, 0.0
        c0 = time.perf_counter()
        while done_bytes < args.cpu_seq and n_docs < off.size - 1:
            ref = oracle.process_document(oc, ow, toks[toff[n_docs]:toff[n_docs + 1]], T, 512,
                                          args.threshold)
            worst = max(worst, float(np.abs(res.doc(n_docs)[0] - ref["entropies"]).max()))
            done_bytes += int(off[n_docs + 1] - off[n_docs])
            n_docs += 1
        c1 = time.perf_counter()
        result["cpu_baseline"] = {
            "value": round(done_bytes / (c1 - c0), 2), "unit": "bytes/s", "cores": cores,
            "kind": "port",
            "sample": "first %d documents (%d bytes) of the same stream through the fp32 C "
                      "restatement (oracle: per-chunk forward, stitch, boundaries), %.1f s"
                      % (n_docs, done_bytes, c1 - c0),
            "parity_on_sample": {"entropy_max_abs": worst}}
    print(json.dumps(result), flush=True)


def bench_pipeline(args):
    """The streaming pipeline (pipeline.rs:279-324) over a prefix of the config-5
    document stream: raw bytes (no +4 offset), 4096-byte chunks with 2048 bytes
    of context, the boundary pass over the accumulated entropies after each
    chunk, per-patch means.  value = document bytes / second of the packed
    many-document form (pipeline.process_documents: chunks of all documents as
    segments of [rows, 8192] forwards); the one-forward-per-chunk form
    (pipeline.process_document per document, as the reference runs it) is
    reported beside it.  Host memory in and out."""
    import numpy as np

    from blt_burn_amd import model as M, pipeline as P, synth

    steps = args.steps if args.steps is not None else 1
    cfg = M.entropy_model_config()
    F, D, V, L, H = 2048, cfg.dim, cfg.vocab_size, cfg.n_layers, cfg.resolved_n_heads()
    B, T, W = args.batch, args.seq, args.window
    seed = synth.config_seed(5)
    weights = M.random_weights(cfg, seed, hidden=F)
    model = M.LMTransformer(cfg, weights, device=0, max_tokens=B * T, window=W)
    nbytes = int(args.pipeline_mib * 2 ** 20)
    data, off = synth.documents(seed, nbytes)
    docs = [data[off[i]:off[i + 1]].tobytes() for i in range(off.size - 1)]
    wdata, woff = synth.documents(seed + 1, 2 ** 20)
    wdocs = [wdata[woff[i]:woff[i + 1]].tobytes() for i in range(woff.size - 1)]
    for _ in range(args.warmup):
        P.process_documents(wdocs, model, args.threshold, rows=B, row_len=T)
        for d in wdocs[:64]:
            P.process_document(d, model, threshold=args.threshold)
    model.read_profile()
    model.set_profiling(True)
    t0 = time.perf_counter()
    for _ in range(steps):
        packed = P.process_documents(docs, model, args.threshold, rows=B, row_len=T)
    t1 = time.perf_counter()
    prof = model.read_profile()
    model.set_profiling(False)
    sec = (t1 - t0) / steps
    dom = "w13_gemm_silu"
    ms_tot, launches = prof[dom]
    per_launch_ms = ms_tot / launches
    achieved = stage_flops(dom, B * T, B, T, D, F, V, H, W) / (per_launch_ms * 1e-3) / 1e12
    gpu_ms = sum(ms for ms, n in prof.values()) / steps
    c0 = time.perf_counter()
    single = [P.process_document(d, model, threshold=args.threshold) for d in docs]
    c1 = time.perf_counter()
    n_patches = sum(len(r.patches) for r in packed)
    worst = max(float(np.abs(a.entropies - b.entropies).max()) for a, b in zip(packed, single)
                if a.entropies.size)
    result = {
        "metric": "document bytes/sec through the streaming pipeline (pipeline.rs "
                  "process_document, BLT entropy model, bf16)",
        "value": round(nbytes / sec, 1), "unit": "bytes/s", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: %.1f MiB prefix of the seeded config-5 document stream (%d "
                "documents), raw bytes as tokens, random-init bf16 weights"
                % (nbytes / 2 ** 20, len(docs)),
        "config": {"workload": "pipeline.rs: 4096-byte chunks with 2048 bytes of context, "
                               "boundary pass over the accumulated entropies per chunk, "
                               "per-patch means; chunks of all documents packed into "
                               "[rows, row_len] forwards",
                   "rows": B, "row_len": T, "window": W, "threshold": args.threshold},
        "pipeline": {"patches_emitted": n_patches,
                     "per_chunk_form_bytes_per_s": round(nbytes / (c1 - c0), 1),
                     "per_chunk_form_s": round(c1 - c0, 3),
                     "packed_vs_per_chunk_entropy_max_abs": worst,
                     "gpu_model_ms": round(gpu_ms, 1),
                     "gpu_model_busy_fraction": round(gpu_ms / (sec * 1e3), 4)},
        "roofline": _with_achievable({"bound": "mfma", "kernel": dom,
                                      "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                                      "unit": "TFLOP/s",
                                      "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                                      "traffic": None, "launch_ms": round(per_launch_ms, 4)}),
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        import oracle  # the checker / CPU baseline only
        cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
        os.environ["OMP_NUM_THREADS"] = str(cores)
        oc = dict(dim=D, n_layers=L, n_heads=H, hidden=F, vocab=V, max_seqlen=cfg.max_seqlen,
                  norm_eps=cfg.norm_eps, rope_theta=cfg.rope_theta, window=W)
        ow = _oracle_weights(weights)

        def fwd(tokens, start):
            o = oracle.model_forward(oc, ow, tokens[None, :])
            return o["entropies"][0], o["embedding_norms"][0]
        n_docs, done_bytes, dH = 0, 0, 0.0
        c0 = time.perf_counter()
        while done_bytes < args.cpu_seq and n_docs < len(docs):
            ref = oracle.pipeline_process_document(docs[n_docs], fwd, args.threshold)
            dH = max(dH, float(np.abs(single[n_docs].entropies - ref["entropies"]).max()))
            done_bytes += len(docs[n_docs])
            n_docs += 1
        c1 = time.perf_counter()
        result["cpu_baseline"] = {
            "value": round(done_bytes / (c1 - c0), 2), "unit": "bytes/s", "cores": cores,
            "kind": "port",
            "sample": "first %d documents (%d bytes) of the same stream through the oracle's "
                      "restatement of process_document with the fp32 C forward, %.1f s"
                      % (n_docs, done_bytes, c1 - c0),
            "parity_on_sample": {"entropy_max_abs": dH}}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
