"""Parity of the gfx950 fused ops and patcher kernels with the CPU oracle
(bit-exact for boundaries/indices; tolerances stated per test), on the
reference tests' shapes and on BASELINE config 1/2/3 shapes."""
import ctypes
import json
import math
import os

import numpy as np
import pytest
import torch

import oracle
from blt_burn_amd import fused_ops as F
from blt_burn_amd import patcher, synth
from blt_burn_amd import _lib

pytestmark = pytest.mark.gpu
KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kat.json")))
DEV = "cuda:0"


def cuda(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def bf16(a):
    """f32 numpy -> (bf16 cuda tensor, the same values as f32 numpy)."""
    t = cuda(a.astype(np.float32)).to(torch.bfloat16)
    return t, t.float().cpu().numpy()


# ---------------------------------------------------------------- entropy
@pytest.mark.parametrize("case", KAT["entropy"], ids=lambda c: c["name"])
def test_entropy_kat(case):
    x = np.full(case["shape"], case["fill"], np.float32)
    if "hot" in case:
        x[..., 0] = case["hot"]
    H = F.fused_entropy(cuda(x), x.shape[-1]).cpu().numpy()
    assert H.shape == tuple(case["shape"][:-1])
    assert np.all(np.abs(H - case["expected"]) < case["tol"])


@pytest.mark.parametrize("shape,std,mean", [((2, 4, 10), 1.0, 0.0), ((2, 128, 260), 1.0, 0.0),
                                            ((1, 32, 260), 1.0, 0.0), ((4, 1, 260), 1.0, 0.0),
                                            ((1, 64, 260), 20.0, 50.0), ((3, 5, 1000), 2.0, 0.0),
                                            ((2, 7, 3000), 2.0, 0.0), ((2, 9, 97), 2.0, 0.0)])
def test_entropy_vs_oracle(shape, std, mean):
    x = synth.normal_f32(11, shape, mean, std)
    H = F.fused_entropy(cuda(x), shape[-1]).cpu().numpy()
    ref = oracle.entropy(x)
    assert np.all(np.isfinite(H)) and np.all(H >= -1e-6)
    np.testing.assert_allclose(H, ref, atol=1e-4)  # reference tests: 1e-4 / 1e-3


@pytest.mark.parametrize("n", [4, 64, 68, 128, 256, 260, 320, 512, 516, 1024, 1280])
@pytest.mark.parametrize("std", [0.5, 8.0])
def test_entropy_widths_vs_oracle(n, std):
    # every (full chunks, tail) split of the one-exponential kernel; std 8 gives
    # near one-hot rows, where H = lse - sum(p d) / s must not cancel badly
    x = synth.normal_f32(31 + n, (3, 17, n), 1.0, std)
    H = F.fused_entropy(cuda(x), n).cpu().numpy()
    np.testing.assert_allclose(H, oracle.entropy(x), atol=1e-4)
    xb, xf = bf16(x)
    np.testing.assert_allclose(F.fused_entropy(xb, n).cpu().numpy(), oracle.entropy(xf), atol=1e-4)


def test_entropy_config1_full_size():
    # logits f32 [4, 8192, 260] ~ N(0, 2)
    x = synth.normal_f32(synth.config_seed(1), (4, 8192, 260), 0.0, 2.0)
    H = F.fused_entropy(cuda(x), 260).cpu().numpy()
    np.testing.assert_allclose(H, oracle.entropy(x), atol=1e-4)


def test_entropy_bf16():
    xb, xf = bf16(synth.normal_f32(12, (8, 64, 260), 0.0, 2.0))
    H = F.fused_entropy(xb, 260).cpu().numpy()
    np.testing.assert_allclose(H, oracle.entropy(xf), atol=1e-4)


# ---------------------------------------------------------------- norms / elementwise
@pytest.mark.parametrize("mode", [F.EPS_AFTER_SQRT, F.EPS_INSIDE_SQRT])
@pytest.mark.parametrize("dim", [64, 768, 1000, 4100])
def test_rms_norm_f32(mode, dim):
    x = synth.normal_f32(13, (2, 8, dim))
    w = synth.normal_f32(14, dim, 1.0, 0.2)
    l2 = torch.empty((2, 8), dtype=torch.float32, device=DEV)
    y = F.fused_rms_norm(cuda(x), cuda(w), 1e-6, mode, l2_out=l2).cpu().numpy()
    np.testing.assert_allclose(y, oracle.rms_norm(x, w, 1e-6, mode), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(l2.cpu().numpy(), oracle.l2_norm(x), rtol=1e-5)


def test_rms_norm_bf16_config2():
    # x [32768, 768] ~ N(0,1), w ~ 1 + N(0, 0.02), eps 1e-5, bf16
    xb, xf = bf16(synth.normal_f32(synth.config_seed(2), (1, 32768, 768)))
    wb, wf = bf16(synth.normal_f32(synth.config_seed(2) + 1, 768, 1.0, 0.02))
    l2 = torch.empty((1, 32768), dtype=torch.float32, device=DEV)
    y = F.fused_rms_norm(xb, wb, 1e-5, F.EPS_AFTER_SQRT, l2_out=l2).float().cpu().numpy()
    ref = oracle.rms_norm(xf, wf, 1e-5, 0)
    # bf16 output: within one bf16 rounding (2^-8 relative) of the f32 oracle
    np.testing.assert_allclose(y, ref, rtol=2 ** -8, atol=1e-6)
    np.testing.assert_allclose(l2.cpu().numpy(), oracle.l2_norm(xf), rtol=1e-5)


@pytest.mark.parametrize("dim", [8, 64, 760, 768, 1024, 1032])
@pytest.mark.parametrize("rows", [1, 7, 130])
def test_rms_norm_bf16_widths(dim, rows):
    # the two-rows-per-wave bf16 kernel (n % 8 == 0, n <= 1024; odd row counts
    # leave a wave with one row) and the generic kernel beyond it
    xb, xf = bf16(synth.normal_f32(40 + dim, (1, rows, dim)))
    wb, wf = bf16(synth.normal_f32(41 + dim, dim, 1.0, 0.02))
    l2 = torch.empty((1, rows), dtype=torch.float32, device=DEV)
    y = F.fused_rms_norm(xb, wb, 1e-5, F.EPS_AFTER_SQRT, l2_out=l2).float().cpu().numpy()
    np.testing.assert_allclose(y, oracle.rms_norm(xf, wf, 1e-5, 0), rtol=2 ** -8, atol=1e-6)
    np.testing.assert_allclose(l2.cpu().numpy(), oracle.l2_norm(xf), rtol=1e-5)


def test_l2_norm():
    x = synth.normal_f32(15, (2, 16, 128))  # test_fused_ops.rs:63-94
    np.testing.assert_allclose(F.fused_l2_norm(cuda(x)).cpu().numpy(), oracle.l2_norm(x),
                               atol=1e-4)
    xb, xf = bf16(x)
    np.testing.assert_allclose(F.fused_l2_norm(xb).cpu().numpy(), oracle.l2_norm(xf), rtol=1e-5)


@pytest.mark.parametrize("shape", [(2, 8, 64), (2, 8, 32, 32), (3, 300), (2, 2, 5000)])
def test_softmax(shape):
    x = synth.normal_f32(16, shape)
    y = F.fused_softmax(cuda(x), shape[-1]).cpu().numpy()
    np.testing.assert_allclose(y, oracle.softmax(x), atol=1e-6)
    big = synth.normal_f32(17, (2, 8, 64), 50.0, 20.0)  # test_fused_ops.rs:269-287
    yb = F.fused_softmax(cuda(big), 64).cpu().numpy()
    assert np.all(np.isfinite(yb)) and np.all((yb >= 0) & (yb <= 1))


@pytest.mark.parametrize("n", [(2, 8, 256), (1, 16, 128), (3, 5, 7)])
def test_silu_gate(n):
    g, u = synth.normal_f32(18, n), synth.normal_f32(19, n)
    np.testing.assert_allclose(F.fused_silu_gate(cuda(g), cuda(u)).cpu().numpy(),
                               oracle.silu_gate(g, u), atol=1e-5)
    gb, gf = bf16(g)
    ub, uf = bf16(u)
    got = F.fused_silu_gate(gb, ub).float().cpu().numpy()
    np.testing.assert_allclose(got, oracle.silu_gate(gf, uf), rtol=2 ** -8, atol=1e-6)


def test_silu_gate_bf16_config2():
    gb, gf = bf16(synth.normal_f32(synth.config_seed(2) + 2, (32768, 2048)))
    ub, uf = bf16(synth.normal_f32(synth.config_seed(2) + 3, (32768, 2048)))
    got = F.fused_silu_gate(gb, ub).float().cpu().numpy()
    np.testing.assert_allclose(got, oracle.silu_gate(gf, uf), rtol=2 ** -8, atol=1e-6)


def test_coherence():
    n = synth.normal_f32(20, (4, 32), 5.0, 2.0)
    H = np.abs(synth.normal_f32(21, (4, 32), 2.5, 1.0)) + 0.1
    np.testing.assert_allclose(F.fused_coherence(cuda(n), cuda(H), 1e-6).cpu().numpy(),
                               oracle.coherence(n, H, 1e-6), rtol=1e-5)


# ---------------------------------------------------------------- patch boundaries
def _check_boundaries(H, thr, mode):
    mask, starts, lengths, counts = patcher.patch_boundaries(cuda(H), thr, mode)
    ref_mask = oracle.patch_mask(H, thr, mode)
    np.testing.assert_array_equal(mask.cpu().numpy(), ref_mask)
    ref_starts = oracle.patch_indices(ref_mask)
    ref_len = oracle.patch_lengths(ref_starts, H.shape[1])
    c = counts.cpu().numpy()
    st, ln = starts.cpu().numpy(), lengths.cpu().numpy()
    for b in range(H.shape[0]):
        assert c[b] == len(ref_starts[b])
        assert st[b, :c[b]].tolist() == ref_starts[b]
        assert ln[b, :c[b]].tolist() == ref_len[b]
        assert int(ln[b, :c[b]].sum()) == H.shape[1]


@pytest.mark.parametrize("case", KAT["patch"], ids=lambda c: c["name"])
def test_patch_kat(case):
    H = np.array(case["H"], np.float32)
    mode = patcher.PATCH_MONOTONIC if case["mode"] == "monotonic" else patcher.PATCH_GLOBAL
    mask, starts, lengths, counts = patcher.patch_boundaries(cuda(H), case["thr"], mode)
    assert mask.cpu().tolist() == case["mask"]
    c = counts.cpu().tolist()
    assert [starts[b, :c[b]].cpu().tolist() for b in range(len(c))] == case["starts"]
    assert [lengths[b, :c[b]].cpu().tolist() for b in range(len(c))] == case["lengths"]


@pytest.mark.parametrize("B,T", [(1, 0), (3, 1), (2, 2), (2, 3), (4, 8191), (4, 8192), (2, 8193),
                                 (1, 20000), (16, 8192)])
@pytest.mark.parametrize("mode,thr", [(0, 0.2), (1, 1.33), (0, 1.335)])
def test_patch_boundaries_vs_oracle(B, T, mode, thr):
    H = np.abs(synth.normal_f32(22 + T, (B, T), 1.4, 0.6))
    _check_boundaries(H, thr, mode)


def test_patch_boundaries_config1():
    # config 1: entropies of N(0, 2) logits; global (1.33) and monotonic (0.2) masks
    x = synth.normal_f32(synth.config_seed(1), (4, 8192, 260), 0.0, 2.0)
    Hd = F.fused_entropy(cuda(x), 260)
    H = Hd.cpu().numpy()
    _check_boundaries(H, 1.33, 1)
    _check_boundaries(H, 0.2, 0)
    # shifted-logit variant: scale rows so entropies straddle the global threshold
    xs = x * np.linspace(0.2, 4.0, 8192, dtype=np.float32)[None, :, None]
    Hs = F.fused_entropy(cuda(xs), 260).cpu().numpy()
    assert 0.05 < (Hs > 1.33).mean() < 0.95
    _check_boundaries(Hs, 1.33, 1)
    _check_boundaries(Hs, 0.2, 0)
    # mask API of the reference
    m = patcher.patch_start_mask_from_entropy_with_monotonicity(Hd, 0.2).cpu().numpy()
    np.testing.assert_array_equal(m, oracle.patch_mask(H, 0.2, 0))


def _check_rule_outputs(H, thr, mode, outs):
    mask, starts, lengths, counts = (t.cpu().numpy() for t in outs)
    ref_mask = oracle.patch_mask(H, thr, mode)
    np.testing.assert_array_equal(mask, ref_mask)
    ref_starts = oracle.patch_indices(ref_mask)
    ref_len = oracle.patch_lengths(ref_starts, H.shape[1])
    for b in range(H.shape[0]):
        assert counts[b] == len(ref_starts[b])
        assert starts[b, :counts[b]].tolist() == ref_starts[b]
        assert lengths[b, :counts[b]].tolist() == ref_len[b]


# shapes around the 64-position (fused) and 1024-position tiles, rows of more
# than 4096 tiles (the scan kernel), and T = 0, 1, 2
RULE_SHAPES = [(1, 0), (3, 1), (2, 2), (2, 3), (1, 63), (1, 64), (1, 65), (2, 1023), (2, 1024),
               (2, 1025), (4, 8191), (4, 8192), (2, 8193), (1, 20000), (16, 8192), (1, 70000),
               (3, 66 * 1024 + 5), (1, 4096 * 1024 + 3000)]


@pytest.mark.parametrize("B,T", RULE_SHAPES)
def test_patch_rules_two_rules_one_read(B, T):
    # monotonic and global rules from one read of H, bit-exact vs the oracle
    H = np.abs(synth.normal_f32(31 + T, (B, T), 1.4, 0.6))
    rules = [(patcher.PATCH_MONOTONIC, 0.2), (patcher.PATCH_GLOBAL, 1.33)]
    outs = patcher.patch_boundaries_rules(cuda(H), rules)
    for (mode, thr), o in zip(rules, outs):
        _check_rule_outputs(H, thr, mode, o)


def test_patch_rules_threshold_edges():
    # H on a 0.25 grid, so every f32 difference is exactly 0 or 0.25: a
    # difference equal to the threshold starts no patch, the next f32 below
    # it as threshold makes every step a start; the global rule sees the same
    # values against a threshold equal to one of them
    k = np.cumsum(synth.normal_f32(7, 5000) > 0.3).astype(np.float32)
    H = np.stack([0.25 * k, 0.25 * k[::-1].copy()]).astype(np.float32)
    below = float(np.nextafter(np.float32(0.25), np.float32(0)))
    for thr in (0.25, below):
        outs = patcher.patch_boundaries_rules(cuda(H), [(0, thr), (1, 10.0)])
        _check_rule_outputs(H, thr, 0, outs[0])
        _check_rule_outputs(H, 10.0, 1, outs[1])
        n_up = int((np.diff(H[0]) == 0.25)[1:].sum())
        assert int(outs[0][3][0]) == 2 + (0 if thr == 0.25 else n_up)


@pytest.mark.parametrize("V", [260, 256, 100, 4, 1024, 1000, 13, 1280])
@pytest.mark.parametrize("B,T", [(4, 8192), (2, 1025), (1, 1), (2, 0), (1, 9000), (2, 300000)])
def test_entropy_patch_boundaries_vs_oracle(V, B, T):
    # entropies (1e-4 abs vs the oracle, identical to fused_entropy) and both
    # rules bit-exact on those entropies; V 13 and 1280 take the two-kernel path
    if B * T * V > 40_000_000:
        T = 40_000_000 // (B * V)
    x = synth.normal_f32(41 + V + T, (B, T, V), 0.0, 2.0)
    xs = x * np.linspace(0.2, 4.0, max(T, 1), dtype=np.float32)[None, :T, None]
    rules = [(patcher.PATCH_GLOBAL, 1.33 if V > 8 else 0.5), (patcher.PATCH_MONOTONIC, 0.2)]
    Hd, outs = patcher.entropy_patch_boundaries(cuda(xs), rules)
    H = Hd.cpu().numpy()
    if T > 0:
        np.testing.assert_allclose(H, oracle.entropy(xs), atol=1e-4, rtol=0)
        assert torch.equal(Hd, F.fused_entropy(cuda(xs), V))
    for (mode, thr), o in zip(rules, outs):
        _check_rule_outputs(H, thr, mode, o)


def test_patch_rules_workspace_reused_across_sizes():
    # one workspace through calls of growing and shrinking size, one and two
    # rules, both kernels: every call matches the oracle
    for k, (B, T, n) in enumerate([(4, 8192, 2), (1, 100, 1), (2, 70000, 2), (3, 5, 1),
                                   (16, 8192, 1), (1, 65, 2)]):
        H = np.abs(synth.normal_f32(90 + k, (B, T), 1.4, 0.6))
        rules = [(patcher.PATCH_MONOTONIC, 0.2), (patcher.PATCH_GLOBAL, 1.33)][:n]
        outs = patcher.patch_boundaries_rules(cuda(H), rules)
        for (mode, thr), o in zip(rules, outs):
            _check_rule_outputs(H, thr, mode, o)
        x = synth.normal_f32(190 + k, (B, min(T, 3000), 260), 0.0, 2.0)
        Hd, outs = patcher.entropy_patch_boundaries(cuda(x), rules)
        for (mode, thr), o in zip(rules, outs):
            _check_rule_outputs(Hd.cpu().numpy(), thr, mode, o)


def test_entropy_patch_plan_matches_function():
    # the prepared call returns what the function returns, call after call, and
    # rejects logits of another shape, dtype or layout
    B, T, V = 3, 1000, 260
    rules = [(patcher.PATCH_GLOBAL, 1.33), (patcher.PATCH_MONOTONIC, 0.2)]
    plan = patcher.EntropyPatchPlan(B, T, V, rules)
    for k in range(3):
        x = cuda(synth.normal_f32(400 + k, (B, T, V), 0.0, 2.0))
        Hp, outs_p = plan(x)
        Hf, outs_f = patcher.entropy_patch_boundaries(x, rules)
        assert torch.equal(Hp, Hf)
        for op, of in zip(outs_p, outs_f):
            for a, b in zip(op, of):
                if a.dim() == 2:  # starts / lengths: the valid entries of each row
                    for r in range(B):
                        n = int(of[3][r])
                        assert torch.equal(a[r, :n], b[r, :n])
                else:
                    assert torch.equal(a, b)
        _check_rule_outputs(Hf.cpu().numpy(), 0.2, patcher.PATCH_MONOTONIC, outs_p[1])
    for bad in (x[:, :500], x.to(torch.float64), x.transpose(0, 1), x.cpu()):
        with pytest.raises(_lib.BltError):
            plan(bad)


def test_patch_boundaries_c_entry_one_block_per_row():
    # blt_patch_boundaries (no workspace, one block per row) against the oracle
    L = _lib.lib()
    for B, T in [(3, 1), (4, 8192), (2, 8193), (1, 20000)]:
        H = np.abs(synth.normal_f32(60 + T, (B, T), 1.4, 0.6))
        for mode, thr in ((0, 0.2), (1, 1.33)):
            outs = [torch.empty((B, T), dtype=torch.int32, device=DEV) for _ in range(3)]
            outs.append(torch.empty((B,), dtype=torch.int32, device=DEV))
            Hd = cuda(H)
            rc = L.blt_patch_boundaries(Hd.data_ptr(), B, T, ctypes.c_float(thr), mode,
                                        *[t.data_ptr() for t in outs],
                                        torch.cuda.current_stream().cuda_stream)
            assert rc == 0, _lib.last_error()
            _check_rule_outputs(H, thr, mode, outs)


# ---------------------------------------------------------------- GEMM and attention
@pytest.mark.parametrize("M,N,K", [(256, 256, 64), (1000, 320, 768), (4096, 2304, 768),
                                   (131072 // 8, 768, 2048)])
def test_gemm_vs_torch_fp32(M, N, K):
    a = torch.randn(M, K, device=DEV).to(torch.bfloat16)
    b = torch.randn(N, K, device=DEV).to(torch.bfloat16)
    c = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    _lib.check(_lib.lib().blt_gemm_bf16(a.data_ptr(), b.data_ptr(), c.data_ptr(), M, N, K,
                                        torch.cuda.current_stream().cuda_stream), "gemm")
    ref = a.float() @ b.float().t()
    err = (c.float() - ref).abs().max().item()
    assert err <= 2 ** -7 * ref.abs().max().item() + 1e-2, err


def _attn_case(B, H, T, causal, window, theta, seed=30):
    q, k, v = (synth.normal_f32(seed + i, (B, H, T, 64)) for i in range(3))
    qb, qf = bf16(q)
    kb, kf = bf16(k)
    vb, vf = bf16(v)
    o = F.fused_attention(qb, kb, vb, causal, window=window, rope_theta=theta).float().cpu().numpy()
    ref = oracle.attention(qf, kf, vf, causal, window, theta)
    return o, ref


def _assert_rows_close(o, ref, rel=2e-2, label=""):
    """Per query row: max |o - ref| <= rel * max |ref| of that row (+1e-4 for
    rows whose outputs are all near 0).  The output is stored in bf16 (unit
    roundoff 2^-8), q enters QK^T re-rounded after its log2(e)/8 scale, and P
    enters the PV product in bf16 with the row sum taken over the same rounded
    values, so the weights stay a convex combination within 2^-8 of the exact
    ones; every one of these errors scales with the row (measured: up to
    1.05e-2 of the row max over 2800 rows).  A per-(batch, head) bar against
    the head's largest output would be several times looser, since early rows
    average few keys and reach |v|.  The window edge itself is pinned exactly
    by test_attention_window_edge."""
    d = np.abs(o - ref).max(axis=-1)
    s = np.abs(ref).max(axis=-1)
    worst = float((d / (s + 1e-2)).max())
    print("%s attention: max|d| %.2e, worst row |d|/max|ref| %.2e" % (label, d.max(), worst))
    bad = d > rel * s + 1e-4
    assert not bad.any(), (np.argwhere(bad)[:5], d[bad][:5], s[bad][:5])


@pytest.mark.parametrize("B,H,T,causal,window,theta", [
    (1, 2, 64, True, 0, 0.0), (2, 3, 200, True, 0, 0.0), (1, 2, 333, True, 64, 0.0),
    (1, 1, 130, False, 0, 0.0), (1, 2, 300, True, 0, 10000.0), (2, 2, 700, True, 512, 10000.0),
    (1, 1, 1, True, 0, 10000.0), (1, 1, 97, True, 1, 0.0),
    # RoPE slices of uneven size: 3 batch slices; 4 head slices of 5 heads
    (3, 2, 300, True, 64, 10000.0), (1, 5, 200, True, 0, 10000.0),
    # window edges at any offset inside a 64-key tile
    (1, 2, 500, True, 100, 10000.0), (2, 1, 777, True, 333, 0.0)])
def test_attention_vs_oracle(B, H, T, causal, window, theta):
    o, ref = _attn_case(B, H, T, causal, window, theta)
    _assert_rows_close(o, ref, label="B%d H%d T%d w%d" % (B, H, T, window))


@pytest.mark.parametrize("W,val,periods", [(512, 512.0, (61, 63, 50)),
                                           (300, 256.0, (61, 63, 47))])
@pytest.mark.parametrize("theta", [0.0, 10000.0])
def test_attention_window_edge(theta, W, val, periods):
    # q = k = 0: every visible key gets the same weight, so row i of the output
    # is the mean of v over keys j in (i - W, i].  v[j] is one-hot in column
    # j % P (value val, exact in bf16) with a period P per head that does not
    # divide W, so including key i - W or dropping key i - W + 1 (or i) moves
    # some column of every row with i >= W by about val / W against outputs
    # of about val / P.  W = 300 puts the window edge at varying offsets inside
    # the 64-key tiles.  Expected values in closed form, independent of the
    # oracle.
    T, H = 1600, 3
    assert all(W % P for P in periods)
    v = np.zeros((1, H, T, 64), np.float32)
    for h, P in enumerate(periods):
        v[0, h, np.arange(T), np.arange(T) % P] = val
    z = torch.zeros((1, H, T, 64), dtype=torch.bfloat16, device=DEV)
    o = F.fused_attention(z, z, torch.from_numpy(v).to(DEV).to(torch.bfloat16), True,
                          window=W, rope_theta=theta).float().cpu().numpy()
    want = np.zeros_like(v)
    for h, P in enumerate(periods):
        for i in range(T):
            j = np.arange(max(0, i - W + 1), i + 1)
            want[0, h, i] = np.bincount(j % P, minlength=64)[:64] * val / len(j)
    np.testing.assert_allclose(o, want, rtol=2 ** -8, atol=1e-3)
    # the oracle agrees with the closed form (no rounding anywhere on its side)
    ref = oracle.attention(np.zeros_like(v), np.zeros_like(v), v, True, W, theta)
    np.testing.assert_allclose(ref, want, rtol=1e-6, atol=1e-4)


def test_attention_rope_64_query_waves():
    # long full-causal rows take the 64-queries-per-wave kernel; with RoPE its q
    # is rotated in registers as it is loaded.  Same result as handing it q and
    # k rotated beforehand (half-split pairs, the oracle's f32 table).
    B, H, T = 4, 16, 4096
    qb, _ = bf16(synth.normal_f32(81, (B, H, T, 64)))
    kb, _ = bf16(synth.normal_f32(82, (B, H, T, 64)))
    vb, _ = bf16(synth.normal_f32(83, (B, H, T, 64)))
    cs = torch.from_numpy(np.ascontiguousarray(oracle.rope_table(64, T, 10000.0))).to(DEV)
    cs = cs.reshape(T, 32, 2)
    c, s_ = cs[..., 0], cs[..., 1]

    def rot(x):
        x = x.float()
        x1, x2 = x[..., :32], x[..., 32:]
        return torch.cat([x1 * c - x2 * s_, x1 * s_ + x2 * c], dim=-1).to(torch.bfloat16)

    o = F.fused_attention(qb, kb, vb, True, rope_theta=10000.0).float()
    ref = F.fused_attention(rot(qb), rot(kb), vb, True).float()
    # the two paths differ only in where each rotated value was rounded to bf16
    assert float((o - ref).abs().max()) < 2e-2


def test_entropy_boundaries_graph_replay():
    # fused_entropy + both boundary passes captured as one HIP graph; every
    # replay (with eager work and syncs between them) matches the eager step
    B, T, V = 2, 3000, 260
    logits = cuda(synth.normal_f32(71, (B, T, V), 0.0, 2.0))
    outs = [tuple(torch.empty(s, dtype=torch.int32, device=DEV)
                  for s in ((B, T), (B, T), (B, T), (B,))) for _ in range(2)]
    held = {}

    def step():
        H = F.fused_entropy(logits, V)
        held["H"] = H
        patcher.patch_boundaries(H, 1.33, patcher.PATCH_GLOBAL, out=outs[0])
        patcher.patch_boundaries(H, 0.2, patcher.PATCH_MONOTONIC, out=outs[1])

    step()
    torch.cuda.synchronize()
    eager = [t.clone() for t in (held["H"],) + outs[0] + outs[1]]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for k in range(3):
        for t in outs[0] + outs[1]:
            t.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        got = (held["H"],) + outs[0] + outs[1]
        for i, (a, b) in enumerate(zip(eager, got)):
            if i in (2, 3, 6, 7):  # starts / lengths: only the first counts[b] entries are defined
                cnt = eager[4 if i < 4 else 8].cpu().numpy()
                for r in range(B):
                    np.testing.assert_array_equal(a[r, :cnt[r]].cpu().numpy(),
                                                  b[r, :cnt[r]].cpu().numpy())
            else:
                assert torch.equal(a, b), (k, i)
        # eager work between replays
        F.fused_entropy(cuda(synth.normal_f32(72 + k, (1, 64, V))), V)
        torch.cuda.synchronize()


@pytest.mark.parametrize("B,H,Tq,Tkv,d,causal", [(1, 2, 300, 300, 64, True),
                                                 (2, 3, 70, 200, 32, True),
                                                 (1, 2, 200, 70, 100, True),
                                                 (1, 1, 97, 130, 256, False),
                                                 (2, 2, 1, 33, 8, True),
                                                 (1, 4, 129, 129, 128, False)])
def test_attention_f32_reference_kernel(B, H, Tq, Tkv, d, causal):
    # f32 fused_attention is the reference kernel's computation (any head_dim,
    # seq_q != seq_kv) in f32: 1e-4 abs, far below one bf16 rounding of q, k, v
    q = synth.normal_f32(80 + d, (B, H, Tq, d))
    k = synth.normal_f32(81 + d, (B, H, Tkv, d))
    v = synth.normal_f32(82 + d, (B, H, Tkv, d))
    o = F.fused_attention(cuda(q), cuda(k), cuda(v), causal)
    assert o.dtype == torch.float32 and tuple(o.shape) == (B, H, Tq, d)
    np.testing.assert_allclose(o.cpu().numpy(), oracle.attention_kernel(q, k, v, causal),
                               atol=1e-4, rtol=0)


def test_attention_f32_rejects_wide_heads():
    q = cuda(synth.normal_f32(90, (1, 1, 8, 264)))
    with pytest.raises(_lib.BltError):
        F.fused_attention(q, q, q, True)


def test_attention_config3_b1():
    # config 3 shape at B=1 (the CPU comparison size): T=4096, 12 heads, window 512, RoPE
    o, ref = _attn_case(1, 12, 4096, True, 512, 10000.0, seed=synth.config_seed(3))
    _assert_rows_close(o, ref, label="config3 B1")


# ---------------------------------------------------------------- GEMM epilogues
def _gemm_epi(a, bt, c, epi, n_valid=0, rope_cols=0, seq_len=1, cs=None):
    M, K = a.shape
    N = bt.shape[0]
    _lib.check(_lib.lib().blt_gemm_bf16_epilogue(
        a.data_ptr(), bt.data_ptr(), c.data_ptr(), M, N, K, K, K, c.shape[1], epi, n_valid,
        rope_cols, seq_len, cs.data_ptr() if cs is not None else 0,
        torch.cuda.current_stream().cuda_stream), "gemm_epilogue")
    torch.cuda.synchronize()


@pytest.mark.parametrize("M,N,K", [(256, 768, 768), (1000, 768, 2048), (4096, 768, 768)])
def test_gemm_residual_epilogue(M, N, K):
    a = torch.randn(M, K, device=DEV).to(torch.bfloat16)
    bt = torch.randn(N, K, device=DEV).to(torch.bfloat16)
    r0 = torch.randn(M, N, device=DEV)
    c = r0.clone()
    _gemm_epi(a, bt, c, _lib.EPI_RESID_F32)
    ref = r0 + a.float() @ bt.float().t()
    assert (c - ref).abs().max().item() <= 2e-3 * ref.abs().max().item()


@pytest.mark.parametrize("M,N", [(256, 1024), (777, 4096)])
def test_gemm_silu_gate_epilogue(M, N):
    K = 768
    a = torch.randn(M, K, device=DEV).to(torch.bfloat16)
    bt = (0.1 * torch.randn(N, K, device=DEV)).to(torch.bfloat16)
    c = torch.empty(M, N // 2, device=DEV, dtype=torch.bfloat16)
    _gemm_epi(a, bt, c, _lib.EPI_SILU_GATE)
    y = a.float() @ bt.float().t()
    g = y.view(M, N // 64, 2, 32)[:, :, 0, :].reshape(M, N // 2)
    u = y.view(M, N // 64, 2, 32)[:, :, 1, :].reshape(M, N // 2)
    ref = torch.nn.functional.silu(g) * u
    assert (c.float() - ref).abs().max().item() <= 2 ** -7 * ref.abs().max().item() + 1e-3


@pytest.mark.parametrize("M,T", [(256, 256), (1000, 100), (8192, 4096)])
def test_gemm_qkv_rope_epilogue(M, T):
    K, N, rope_cols = 768, 2304, 1536
    a = torch.randn(M, K, device=DEV).to(torch.bfloat16)
    bt = (0.05 * torch.randn(N, K, device=DEV)).to(torch.bfloat16)
    cs = torch.from_numpy(oracle.rope_table(64, T, 10000.0)).to(DEV)
    c = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    _gemm_epi(a, bt, c, _lib.EPI_QKV_ROPE, rope_cols=rope_cols, seq_len=T, cs=cs)
    y = (a.float() @ bt.float().t()).cpu().numpy()
    ref = y.copy()
    pos = np.arange(M) % T
    q = y[:, :rope_cols].reshape(M, rope_cols // 64, 64)
    cos = cs.cpu().numpy()[pos, :, 0][:, None, :]
    sin = cs.cpu().numpy()[pos, :, 1][:, None, :]
    x1, x2 = q[..., :32], q[..., 32:]
    ref[:, :rope_cols] = np.concatenate([x1 * cos - x2 * sin, x1 * sin + x2 * cos],
                                        -1).reshape(M, rope_cols)
    err = np.abs(c.float().cpu().numpy() - ref).max()
    assert err <= 2 ** -7 * np.abs(ref).max() + 1e-3, err


@pytest.mark.parametrize("M,N", [(300, 260), (4096, 260)])
def test_gemm_f32_epilogue_partial_columns(M, N):
    K = 768
    a = torch.randn(M, K, device=DEV).to(torch.bfloat16)
    bt = torch.randn(N, K, device=DEV).to(torch.bfloat16)
    c = torch.full((M, N), 7.0, device=DEV)
    _gemm_epi(a, bt, c, _lib.EPI_F32, n_valid=N)
    ref = a.float() @ bt.float().t()
    assert (c - ref).abs().max().item() <= 2e-3 * ref.abs().max().item()


@pytest.mark.parametrize("K", [192, 768])
@pytest.mark.parametrize("epi", ["bf16", "resid", "f32", "silu", "qkv"])
def test_gemm_small_launch_tiles_bit_identical(epi, K):
    # A launch with fewer 256 x 256 tiles than CUs runs on 128 x 128 tiles; its
    # rows must equal the same rows of a launch that stays on 256 x 256 tiles,
    # bit for bit (the model's row-independence rests on it), also on the
    # column blocks whose K tiles run from the last one down (N > 1024).
    Mb, Ms = 256 * 256 + 64, 1000
    N = {"silu": 4096, "qkv": 2304}.get(epi, 768)
    torch.manual_seed(5)
    a = torch.randn(Mb, K, device=DEV).to(torch.bfloat16)
    bt = (0.05 * torch.randn(N, K, device=DEV)).to(torch.bfloat16)
    kw = {}
    if epi == "qkv":
        T = 512
        kw = dict(rope_cols=1536, seq_len=T,
                  cs=torch.from_numpy(oracle.rope_table(64, T, 10000.0)).to(DEV))
    if epi == "f32":
        kw = dict(n_valid=N)
    code = {"bf16": _lib.EPI_BF16, "resid": _lib.EPI_RESID_F32, "f32": _lib.EPI_F32,
            "silu": _lib.EPI_SILU_GATE, "qkv": _lib.EPI_QKV_ROPE}[epi]
    if epi in ("resid", "f32"):
        big = torch.randn(Mb, N, device=DEV)
    else:
        big = torch.zeros(Mb, N // 2 if epi == "silu" else N, device=DEV, dtype=torch.bfloat16)
    small = big[:Ms].clone()
    _gemm_epi(a, bt, big, code, **kw)
    _gemm_epi(a[:Ms].contiguous(), bt, small, code, **kw)
    assert torch.equal(small, big[:Ms])


# ---------------------------------------------------------------- measurement probes
def test_probe_copy_and_mfma():
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    x = torch.randn(1 << 20, device=DEV)
    y = torch.empty_like(x)
    _lib.check(L.blt_probe_copy(x.data_ptr(), y.data_ptr(), x.numel() * 4, stream), "probe_copy")
    sink = torch.zeros(8 * 256, device=DEV)
    _lib.check(L.blt_probe_mfma_bf16(8, 16, sink.data_ptr(), stream), "probe_mfma")
    torch.cuda.synchronize()
    assert torch.equal(x, y)
    assert sink.abs().sum().item() == 0.0  # the sink is never written
    assert L.blt_probe_mfma_flops(8, 16) == 8 * 4 * 16 * 4 * 32 * 32 * 16 * 2
    assert L.blt_probe_copy(x.data_ptr(), y.data_ptr(), 10, stream) != 0  # not a multiple of 16


# ---------------------------------------------------------------- persistent GEMM tile walks
@pytest.mark.parametrize("N", [512, 2304])
@pytest.mark.parametrize("K", [64, 192, 320, 768])
def test_gemm_persistent_many_tiles_odd_k_tiles(K, N):
    # More tiles than CUs (each block walks several tiles) with odd and even
    # numbers of 64-deep K tiles, so the LDS stage holding a tile's last K
    # tile alternates between tiles; a ragged last row tile.  Every epilogue
    # kind on the same operands.  N = 2304: column tiles 4-7 (first column
    # with bit 10 set) take their K tiles from the last one down, and the row
    # tiles go in groups of 8 whose odd members walk the columns in reverse
    # (134 row tiles: a partial last group), so a block's next tile can run
    # the other K direction, including with a single K tile.
    M = 256 * 133 + 17
    torch.manual_seed(K)
    a = torch.randn(M, K, device=DEV).to(torch.bfloat16)
    bt = (0.1 * torch.randn(N, K, device=DEV)).to(torch.bfloat16)
    y = a.float() @ bt.float().t()
    tol = lambda ref: 2 ** -7 * ref.abs().max().item() + 1e-3

    c = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    _gemm_epi(a, bt, c, _lib.EPI_BF16)
    assert (c.float() - y).abs().max().item() <= tol(y)

    r0 = torch.randn(M, N, device=DEV)
    r = r0.clone()
    _gemm_epi(a, bt, r, _lib.EPI_RESID_F32)
    ref = r0 + y
    assert (r - ref).abs().max().item() <= 2e-3 * ref.abs().max().item()

    h = torch.empty(M, N // 2, device=DEV, dtype=torch.bfloat16)
    _gemm_epi(a, bt, h, _lib.EPI_SILU_GATE)
    g = y.view(M, N // 64, 2, 32)[:, :, 0, :].reshape(M, N // 2)
    u = y.view(M, N // 64, 2, 32)[:, :, 1, :].reshape(M, N // 2)
    ref = torch.nn.functional.silu(g) * u
    assert (h.float() - ref).abs().max().item() <= tol(ref)


# ---------------------------------------------------------------- N % 128 == 64 column bound
def _gemm_epi_ld(a, bt, buf, ldc, epi, rope_cols=0, seq_len=1, cs=None):
    M, K = a.shape
    N = bt.shape[0]
    _lib.check(_lib.lib().blt_gemm_bf16_epilogue(
        a.data_ptr(), bt.data_ptr(), buf.data_ptr(), M, N, K, K, K, ldc, epi, 0, rope_cols,
        seq_len, cs.data_ptr() if cs is not None else 0,
        torch.cuda.current_stream().cuda_stream), "gemm_epilogue")
    torch.cuda.synchronize()


@pytest.mark.parametrize("N,pad", [(192, 0), (192, 64), (576, 0), (320, 64)])
def test_gemm_pair_epilogues_n_mod_128_is_64(N, pad):
    """N % 256 != 0 takes the 128 x 128 register-staged kernel; with N % 128 ==
    64 its last N tile overhangs N by 64 columns.  The RoPE and SiLU*gate pair
    epilogues must write nothing there: a sentinel-filled row padding (pad)
    and a guard region after the last row stay untouched."""
    M, K = 300, 256
    torch.manual_seed(N + pad)
    a = torch.randn(M, K, device=DEV).to(torch.bfloat16)
    bt = (0.1 * torch.randn(N, K, device=DEV)).to(torch.bfloat16)
    y = a.float() @ bt.float().t()
    sentinel = torch.tensor(-12345.0, dtype=torch.bfloat16)
    guard = 4096
    T = 100
    cs = torch.from_numpy(oracle.rope_table(64, T, 10000.0)).to(DEV)
    for epi in (_lib.EPI_QKV_ROPE, _lib.EPI_SILU_GATE):
        width = N if epi == _lib.EPI_QKV_ROPE else N // 2
        ldc = width + pad
        buf = torch.full((M * ldc + guard,), sentinel.item(), device=DEV, dtype=torch.bfloat16)
        rope_cols = (N // 64 // 2) * 64 if epi == _lib.EPI_QKV_ROPE else 0
        _gemm_epi_ld(a, bt, buf, ldc, epi, rope_cols=rope_cols, seq_len=T, cs=cs)
        c = buf[:M * ldc].view(M, ldc)
        assert torch.all(buf[M * ldc:] == sentinel), "wrote past the last row"
        if pad:
            assert torch.all(c[:, width:] == sentinel), "wrote into the row padding"
        out = c[:, :width].float()
        if epi == _lib.EPI_SILU_GATE:
            g = y.view(M, N // 64, 2, 32)[:, :, 0, :].reshape(M, N // 2)
            u = y.view(M, N // 64, 2, 32)[:, :, 1, :].reshape(M, N // 2)
            ref = torch.nn.functional.silu(g) * u
        else:
            yy = y.cpu().numpy()
            ref = yy.copy()
            pos = np.arange(M) % T
            q = yy[:, :rope_cols].reshape(M, rope_cols // 64, 64)
            cos = cs.cpu().numpy()[pos, :, 0][:, None, :]
            sin = cs.cpu().numpy()[pos, :, 1][:, None, :]
            x1, x2 = q[..., :32], q[..., 32:]
            ref[:, :rope_cols] = np.concatenate([x1 * cos - x2 * sin, x1 * sin + x2 * cos],
                                                -1).reshape(M, rope_cols)
            ref = torch.from_numpy(ref).to(DEV)
        err = (out - ref).abs().max().item()
        assert err <= 2 ** -7 * ref.abs().max().item() + 1e-3, (epi, err)
