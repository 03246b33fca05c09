"""The bench's profiler bookkeeping, on synthetic rocprofv3 CSVs: dispatches of
one forward mapped to model stages, and the per-stage HBM traffic per launch
(counter values scaled by what the same counter reads for a copy of known
size), which the bench line's roofline.traffic reports.  CPU only."""
import argparse
import csv
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
_spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
bench = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(bench)

L = 14
G = "void blt::gemm::gemm_bf16_dma_persistent_kernel<256, 256, 64, 2, 4, %d>(blt::GemmArgs)"


def _forward_names(layers):
    n = ["blt::embed_kernel(int const*)"]
    for _ in range(layers):
        n += [G % 3, "void blt::(anonymous namespace)::attn_fwd_kernel<1>(blt::AttnArgs)",
              G % 2, "blt::row_rstd_kernel(float const*)", G % 4, G % 2,
              "blt::row_rstd_kernel(float const*)"]
    n += ["void blt::rmsnorm_kernel<float, float, unsigned short, 4, 3>(float const*)",
          "void blt::gemm::gemm_bf16_kernel<128, 128, 32, 2, 2, 2, 3>(blt::GemmArgs)",
          "void blt::entropy_half_kernel<float, 2, 1>(float const*)",
          "blt::coherence_kernel(float const*)",
          "blt::(anonymous namespace)::patch_flags_kernel(blt::PatchKArgs)",
          "blt::(anonymous namespace)::patch_compact_kernel(blt::PatchKArgs)"]
    return n


def test_dispatch_stages_one_forward():
    st = bench._dispatch_stages(_forward_names(2), 2)
    assert st[0] == "embed"
    layer = ["qkv_gemm_rope", "attention", "o_gemm_residual", None, "w13_gemm_silu",
             "w2_gemm_residual", None]
    assert st[1:15] == layer * 2
    assert st[15:] == ["rmsnorm", "head_gemm", "entropy", "coherence", "patch_boundaries",
                       "patch_boundaries"]
    # the fused head replaces the final norm, head GEMM, entropy and coherence
    fused = _forward_names(2)[:15] + [
        "void blt::(anonymous namespace)::head_entropy_kernel<true>(float const*)",
        "blt::(anonymous namespace)::patch_flags_kernel(blt::PatchKArgs)"]
    assert bench._dispatch_stages(fused, 2)[15:] == ["head_gemm", "patch_boundaries"]
    assert bench._dispatch_stages(["blt::(anonymous namespace)::mfma_peak_kernel(int, float*)",
                                   "at::native::copy"], 2) == [None, None]


def _write_counters(d, counter, rows):
    os.makedirs(os.path.join(d, "host"), exist_ok=True)
    with open(os.path.join(d, "host", "p_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for i, (name, v) in enumerate(rows):
            w.writerow({"Dispatch_Id": i + 1, "Kernel_Name": name, "Counter_Name": counter,
                        "Counter_Value": v})


def test_summarize_scales_and_averages(tmp_path, capsys):
    names = _forward_names(L)
    # a peak probe before the forward (not a stage), then one forward; the
    # W1|W3 launches read 1000 + layer KiB and write 500 KiB each
    pre = [("blt::(anonymous namespace)::mfma_peak_kernel(int, float*)", 7.0)]
    fetch, write, layer = list(pre), list(pre), 0
    for n in names:
        f, wv = 10.0, 20.0
        if n == G % 4:
            f, wv = 1000.0 + layer, 500.0
            layer += 1
        fetch.append((n, f))
        write.append((n, wv))
    copy = 1 << 20  # bytes the copy probe moves
    _write_counters(str(tmp_path / "tf"), "FETCH_SIZE", fetch)
    _write_counters(str(tmp_path / "tw"), "WRITE_SIZE", write)
    # the copy reads half its bytes on FETCH_SIZE and all of them on WRITE_SIZE
    _write_counters(str(tmp_path / "cf"), "FETCH_SIZE", [("copy", copy / 2048.0)])
    _write_counters(str(tmp_path / "cw"), "WRITE_SIZE", [("copy", copy / 1024.0)])
    args = argparse.Namespace(summarize=[str(tmp_path / x) for x in ("tf", "tw", "cf", "cw")],
                              copy_bytes=float(copy))
    bench.summarize(args)
    import json
    res = json.loads(capsys.readouterr().out)
    assert res["fetch_scale"] == pytest.approx(2.0) and res["write_scale"] == pytest.approx(1.0)
    w13 = res["stages"]["w13_gemm_silu"]
    assert w13["launches"] == L
    assert w13["fetch_bytes"] == round((1000.0 + (L - 1) / 2.0) * 1024 * 2.0)
    assert w13["write_bytes"] == 500 * 1024
    assert res["stages"]["head_gemm"]["launches"] == 1
    assert res["stages"]["qkv_gemm_rope"]["fetch_bytes"] == 10 * 1024 * 2
    assert "mfma_peak" not in json.dumps(res["stages"])


def test_summarize_splits_forwards(tmp_path, capsys):
    # a run of three forwards (the timed step and two telemetry steps): every
    # forward's stages count, none of the later GEMMs is taken for the head
    fetch, write = [], []
    for fwd in range(3):
        for n in _forward_names(L):
            f = 1000.0 + fwd if n == G % 4 else (50.0 if "coherence" in n else 10.0)
            fetch.append((n, f))
            write.append((n, 20.0))
    _write_counters(str(tmp_path / "tf"), "FETCH_SIZE", fetch)
    _write_counters(str(tmp_path / "tw"), "WRITE_SIZE", write)
    _write_counters(str(tmp_path / "cf"), "FETCH_SIZE", [("copy", 1024.0)])
    _write_counters(str(tmp_path / "cw"), "WRITE_SIZE", [("copy", 1024.0)])
    args = argparse.Namespace(summarize=[str(tmp_path / x) for x in ("tf", "tw", "cf", "cw")],
                              copy_bytes=float(1 << 20))
    bench.summarize(args)
    import json
    st = json.loads(capsys.readouterr().out)["stages"]
    assert st["w13_gemm_silu"]["launches"] == 3 * L
    assert st["w13_gemm_silu"]["fetch_bytes"] == 1001 * 1024
    assert st["head_gemm"]["launches"] == 3 and st["embed"]["launches"] == 3
    assert st["attention"]["launches"] == 3 * L
    assert st["coherence"]["fetch_bytes"] == 50 * 1024


_FAKE_ROCPROF = r"""#!%(py)s
# stands in for rocprofv3 --pmc: writes a counter CSV for the command after --
import csv, os, sys, time
a = sys.argv[1:]
counter, out = a[a.index("--pmc") + 1], a[a.index("-d") + 1]
prog = a[a.index("--") + 1:]
mode = os.environ.get("FAKE_ROCPROF_MODE", "ok")
if mode == "hang":
    time.sleep(60)
if mode == "empty":
    sys.exit(0)
names = ["copy"] if "--copy-probe" in prog else %(names)r
if mode == "partial" and counter == "WRITE_SIZE" and "--copy-probe" not in prog:
    names = names[:len(names) // 2]
os.makedirs(os.path.join(out, "host"), exist_ok=True)
with open(os.path.join(out, "host", "p_counter_collection.csv"), "w", newline="") as f:
    w = csv.DictWriter(f, ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
    w.writeheader()
    for i, n in enumerate(names):
        v = 1024.0 if n == "copy" else (3000.0 if "4>" in n else 10.0)
        if counter == "WRITE_SIZE":
            v = 2048.0 if n == "copy" else v / 2
        w.writerow({"Dispatch_Id": i + 1, "Kernel_Name": n, "Counter_Name": counter,
                    "Counter_Value": v})
# rocprofv3 may exit non-zero after writing whole results
sys.exit(139 if mode == "segv" else 0)
"""


def _fake_rocprof(tmp_path, monkeypatch, mode):
    import sys as _sys
    d = tmp_path / "bin"
    d.mkdir()
    exe = d / "rocprofv3"
    exe.write_text(_FAKE_ROCPROF % {"py": _sys.executable, "names": _forward_names(L) * 2})
    exe.chmod(0o755)
    monkeypatch.setenv("PATH", str(d) + os.pathsep + os.environ.get("PATH", ""))
    monkeypatch.setenv("FAKE_ROCPROF_MODE", mode)
    return argparse.Namespace(batch=16, seq=8192, window=512, threshold=1.335,
                              copy_bytes=float(1 << 21))


@pytest.mark.parametrize("mode", ["ok", "segv"])
def test_live_traffic_runs_the_four_passes(tmp_path, monkeypatch, mode):
    args = _fake_rocprof(tmp_path, monkeypatch, mode)
    res, err = bench.live_traffic(args, timeout_s=60)
    assert err is None
    # copy: 2 MiB moved, FETCH_SIZE reads 1024 KiB (factor 2), WRITE_SIZE 2048 KiB (1)
    assert res["fetch_scale"] == pytest.approx(2.0) and res["write_scale"] == pytest.approx(1.0)
    w13 = res["stages"]["w13_gemm_silu"]
    assert w13["launches"] == 2 * L
    assert (w13["fetch_bytes"], w13["write_bytes"]) == (3000 * 1024 * 2, 1500 * 1024)


def test_summarize_averages_each_counter_over_its_own_launches(tmp_path, capsys):
    # the write pass lost the second forward's dispatches: its bytes are still
    # per launch, and the stage says how many launches each pass saw
    names = _forward_names(L)
    fetch = [(n, 1000.0 if n == G % 4 else 10.0) for n in names * 2]
    write = [(n, 500.0 if n == G % 4 else 20.0) for n in names]
    _write_counters(str(tmp_path / "tf"), "FETCH_SIZE", fetch)
    _write_counters(str(tmp_path / "tw"), "WRITE_SIZE", write)
    _write_counters(str(tmp_path / "cf"), "FETCH_SIZE", [("copy", 1024.0)])
    _write_counters(str(tmp_path / "cw"), "WRITE_SIZE", [("copy", 1024.0)])
    res = bench.summarize_dirs([str(tmp_path / x) for x in ("tf", "tw", "cf", "cw")],
                               float(1 << 20))
    w13 = res["stages"]["w13_gemm_silu"]
    assert (w13["launches"], w13["write_launches"]) == (2 * L, L)
    assert (w13["fetch_bytes"], w13["write_bytes"]) == (1000 * 1024, 500 * 1024)


def test_live_traffic_reports_failures(tmp_path, monkeypatch):
    args = _fake_rocprof(tmp_path, monkeypatch, "empty")
    res, err = bench.live_traffic(args, timeout_s=60)
    assert res is None and "no usable counter output" in err
    monkeypatch.setenv("FAKE_ROCPROF_MODE", "partial")
    res, err = bench.live_traffic(args, timeout_s=60)
    assert res is None and "different launches" in err
    monkeypatch.setenv("FAKE_ROCPROF_MODE", "hang")
    res, err = bench.live_traffic(args, timeout_s=2)
    assert res is None and "limit" in err
    monkeypatch.setenv("PATH", str(tmp_path / "nowhere"))
    res, err = bench.live_traffic(args)
    assert res is None and "not on PATH" in err


def _write_multi(d, rows):
    os.makedirs(os.path.join(d, "host"), exist_ok=True)
    with open(os.path.join(d, "host", "p_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for i, (name, counters) in enumerate(rows):
            for c, v in counters.items():
                w.writerow({"Dispatch_Id": i + 1, "Kernel_Name": name, "Counter_Name": c,
                            "Counter_Value": v})


def test_summarize_counters_normalises_per_stage(tmp_path):
    # W1|W3 launches: 32,000 busy cycles summed over 32 SEs (1,000 per SE); the
    # matrix core busy 512,000 SIMD cycles of 1,024,000 (50 %), VALU 64,000
    # quad-cycles (25 %), 102,400 cycles of both (10 %); 100 waves issuing 500
    # VALU, 120 MFMA, 300 SALU, 80 LDS instructions each
    names = _forward_names(L)
    p1, p2 = [], []
    for n in names:
        if n == G % 4:
            p1.append((n, {"SQ_WAVES": 100, "SQ_BUSY_CYCLES": 32000, "SQ_ACTIVE_INST_VALU": 64000,
                           "SQ_VALU_MFMA_BUSY_CYCLES": 512000,
                           "SQ_VALU_MFMA_COEXEC_CYCLES": 102400}))
            p2.append((n, {"SQ_INSTS_VALU": 50000, "SQ_INSTS_MFMA": 12000, "SQ_INSTS_SALU": 30000,
                           "SQ_INSTS_LDS": 8000, "SQ_LDS_BANK_CONFLICT": 5,
                           "SQ_ACTIVE_INST_LDS": 20}))
        else:
            p1.append((n, {"SQ_WAVES": 1, "SQ_BUSY_CYCLES": 32, "SQ_ACTIVE_INST_VALU": 0,
                           "SQ_VALU_MFMA_BUSY_CYCLES": 0, "SQ_VALU_MFMA_COEXEC_CYCLES": 0}))
            p2.append((n, {"SQ_INSTS_VALU": 1, "SQ_INSTS_MFMA": 0, "SQ_INSTS_SALU": 1,
                           "SQ_INSTS_LDS": 0, "SQ_LDS_BANK_CONFLICT": 0, "SQ_ACTIVE_INST_LDS": 0}))
    _write_multi(str(tmp_path / "a"), p1)
    _write_multi(str(tmp_path / "b"), p2)
    table = bench.summarize_counters(str(tmp_path / "a"), str(tmp_path / "b"), L)
    rows = {r.split("|")[1].strip(): [c.strip() for c in r.split("|")[2:-1]]
            for r in table.splitlines()[2:]}
    assert rows["w13_gemm_silu"] == ["%d" % L, "1000", "50.0%", "25.0%", "10.0%", "35.0%", "500",
                                     "120", "300", "80", "0.25"]
    assert list(rows)[0] == "w13_gemm_silu"  # most busy cycles first
    # passes over different dispatches are refused
    _write_multi(str(tmp_path / "c"), p2[:-1])
    with pytest.raises(ValueError):
        bench.summarize_counters(str(tmp_path / "a"), str(tmp_path / "c"), L)


def test_summarize_trace_means_per_stage(tmp_path, capsys):
    # a probe before the first forward, then two forwards: W1|W3 launches take
    # 700 us in the first and 800 us in the second, every other kernel 10 us
    rows, t, did = [], 0, 0
    seq = [("blt::(anonymous namespace)::mfma_peak_kernel(int, float*)", 0)]
    for fwd in range(2):
        seq += [(n, fwd) for n in _forward_names(L)]
    for n, fwd in seq:
        dur = (700 + 100 * fwd) * 1000 if n == G % 4 else 10 * 1000
        did += 1
        rows.append({"Dispatch_Id": did, "Kernel_Name": n, "Start_Timestamp": t,
                     "End_Timestamp": t + dur})
        t += dur + 5000
    p = tmp_path / "trace.csv"
    with open(p, "w", newline="") as f:
        w = csv.DictWriter(f, ["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        w.writerows(rows[::-1])  # the summary sorts by dispatch id itself
    bench.summarize_trace(str(p))
    lines = capsys.readouterr().out.splitlines()
    table = {c[1].strip(): c for c in (ln.split("|") for ln in lines[2:])}
    w13 = table["w13_gemm_silu"]
    assert w13[2].strip() == "`" + (G % 4)[:(G % 4).rfind("(")] + "`"
    assert (int(w13[3]), float(w13[4]), float(w13[5])) == (2 * L, 750.0, 2 * L * 750.0)
    assert lines[2].split("|")[1].strip() == "w13_gemm_silu"  # largest total first
    assert (int(table["head_gemm"][3]), float(table["head_gemm"][4])) == (2, 10.0)
    assert int(table["o_gemm_residual"][3]) == 2 * L
    assert "mfma_peak" not in "".join(lines)
