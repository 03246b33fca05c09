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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--seq", type=int, default=8192)
    ap.add_argument("--window", type=int, default=512)
    ap.add_argument("--threshold", type=float, default=1.335)
    ap.add_argument("--cpu-seq", type=int, default=4096,
                    help="tokens of the CPU-oracle sample (B=1)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
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
    roofline = {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2),
                "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None,
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


if __name__ == "__main__":
    main()
