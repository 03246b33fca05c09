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
        elif "rmsnorm" in n:
            out.append("rmsnorm")
        elif "entropy_kernel" in n:
            out.append("entropy")
        elif "patch_boundary_kernel" in n:
            out.append("patch_boundaries")
        elif "embed_kernel" in n:
            out.append("embed")
        elif "coherence_kernel" in n:
            out.append("coherence")
        else:
            out.append(None)
    return out


def _read_counter_csv(path, counter):
    import csv
    rows = [r for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    return [(r["Kernel_Name"], float(r["Counter_Value"])) for r in rows]


def summarize(args):
    """Per-stage HBM traffic per launch from rocprofv3 --pmc runs of
    `bench.py --steps 1 --warmup 0 --no-cpu` (FETCH_SIZE and WRITE_SIZE, KiB per
    dispatch), each scaled by the bytes a copy of --copy-bytes reads/writes
    divided by what the counter reports for that copy.  Prints JSON."""
    import glob
    find = lambda d: glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)[0]
    fetch = _read_counter_csv(find(args.summarize[0]), "FETCH_SIZE")
    write = _read_counter_csv(find(args.summarize[1]), "WRITE_SIZE")
    cf = max(v for _, v in _read_counter_csv(find(args.summarize[2]), "FETCH_SIZE"))
    cw = max(v for _, v in _read_counter_csv(find(args.summarize[3]), "WRITE_SIZE"))
    kf, kw = args.copy_bytes / (cf * 1024.0), args.copy_bytes / (cw * 1024.0)
    L = 14
    res = {"fetch_scale": kf, "write_scale": kw, "copy_bytes": args.copy_bytes,
           "copy_fetch_kib": cf, "copy_write_kib": cw, "stages": {}}
    for lst, key, k in ((fetch, "fetch_bytes", kf), (write, "write_bytes", kw)):
        ours = [(n, v) for n, v in lst if "blt::" in n]
        for st, (n, v) in zip(_dispatch_stages([n for n, _ in ours], L), ours):
            if st is None:
                continue
            d = res["stages"].setdefault(st, {"launches": 0})
            d[key] = d.get(key, 0.0) + v * 1024.0 * k
            if key == "fetch_bytes":
                d["launches"] += 1
    for d in res["stages"].values():
        for key in ("fetch_bytes", "write_bytes"):
            d[key] = round(d.get(key, 0.0) / max(d["launches"], 1))
    print(json.dumps(res, indent=1))


def summarize_trace(path):
    """Per-stage mean kernel duration from a rocprofv3 --kernel-trace CSV of
    bench.py (stages recovered from the dispatch order of each forward)."""
    import csv
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Dispatch_Id"]))
    rows = [r for r in rows if "blt::" in r["Kernel_Name"]]
    names = [r["Kernel_Name"] for r in rows]
    # split into forwards: each starts with embed_kernel
    starts = [i for i, n in enumerate(names) if "embed_kernel" in n] + [len(names)]
    agg = {}
    for a, b in zip(starts[:-1], starts[1:]):
        for st, r in zip(_dispatch_stages(names[a:b], 14), rows[a:b]):
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
    ap.add_argument("--config", type=int, default=4, choices=(4, 5),
                    help="4: [16, 8192] forward + boundaries (the headline metric); "
                         "5: streaming ingest of variable-length documents, end to end")
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (config 4: batches, default 10; config 5: passes over "
                         "the document sample, default 1)")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--ingest-mib", type=float, default=24.0,
                    help="config 5: MiB of the seeded 1 GiB document stream to ingest per pass")
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--seq", type=int, default=8192)
    ap.add_argument("--window", type=int, default=512)
    ap.add_argument("--threshold", type=float, default=1.335)
    ap.add_argument("--cpu-seq", type=int, default=4096,
                    help="tokens of the CPU-oracle sample (B=1)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--traffic-file", default=os.path.join(ROOT, "profiles",
                                                           "traffic_config4.json"),
                    help="per-stage HBM bytes per launch measured with rocprofv3 --pmc")
    ap.add_argument("--summarize", nargs=4, metavar=("FETCH_DIR", "WRITE_DIR", "COPY_FETCH_DIR",
                                                     "COPY_WRITE_DIR"),
                    help="print per-stage traffic from rocprofv3 --pmc output and exit")
    ap.add_argument("--copy-bytes", type=float, default=float(2 ** 30))
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
    if args.summarize:
        summarize(args)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(rows shard with no collective; see DESIGN.md). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import __graft_entry__
    __graft_entry__.load_package()
    from blt_burn_amd import model as M, patcher, synth

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if args.config == 5:
        bench_ingest(args)
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
    traffic = None
    if os.path.exists(args.traffic_file) and (B, T, W) == (16, 8192, 512):
        st = json.load(open(args.traffic_file)).get("stages", {}).get(dom)
        if st:
            traffic = int(st["fetch_bytes"] + st["write_bytes"])
    roofline = {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2),
                "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                "launch_ms": round(per_launch_ms, 4)}
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
        "roofline": roofline,
        "step_roofline": {"bound": "mfma", "achieved": round(step_tflops, 2),
                          "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                          "frac": round(step_tflops / PEAK_BF16_TFLOPS, 4),
                          "flop_per_byte": round(total_flops / Mtok, 1)},
        "stage_ms_per_step": stage_ms,
        "cpu_baseline": None,
    }

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

    def one_pass(d, o):
        toks, toff = tk.tokenize_documents(d, o, conf.add_bos, conf.add_eos)
        return ing.run(toks, toff)

    for _ in range(args.warmup):
        one_pass(wdata, woff)
    model.read_profile()
    model.set_profiling(True)
    t0 = time.perf_counter()
    for _ in range(steps):
        res = one_pass(data, off)
    t1 = time.perf_counter()
    prof = model.read_profile()
    model.set_profiling(False)
    st = ing.last_stats()
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
                "(%d documents), random-init bf16 weights" % (nbytes / 2 ** 20, off.size - 1),
        "config": {"workload": "config5: tokenize + chunk/overlap + packed forward + stitch + "
                               "per-document monotonic boundaries, host in / host out",
                   "rows": B, "row_len": T, "chunk_len": T, "overlap": 512, "window": W,
                   "threshold": args.threshold},
        "ingest": {"batches": st["batches"], "documents": st["documents"],
                   "tokens": st["tokens"], "tokens_computed": st["tokens_computed"],
                   "row_tokens": st["row_tokens"],
                   "useful_fraction": round(st["tokens"] / st["row_tokens"], 4),
                   "gpu_model_ms": round(gpu_ms, 1),
                   "gpu_model_busy_fraction": round(gpu_ms / (sec * 1e3), 4)},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None,
                     "launch_ms": round(per_launch_ms, 4)},
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


if __name__ == "__main__":
    main()
