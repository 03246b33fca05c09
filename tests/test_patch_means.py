"""Per-patch means (pipeline.rs:240-258 compute_mean_entropy /
compute_mean_prominence; huggingface_loader.rs:265-295 segment coherence):
the CPU oracle pinned by hand-worked vectors, exact closed forms and
invariants; the device kernel bit-exact against the oracle (gpu)."""
import math

import numpy as np
import pytest

import oracle


def _starts(rows, T):
    st = np.zeros((len(rows), max(T, 1)), np.int32)
    ct = np.zeros(len(rows), np.int32)
    for b, r in enumerate(rows):
        st[b, :len(r)] = r
        ct[b] = len(r)
    return st, ct


def test_hand_worked():
    H = np.array([[1, 2, 3, 4, 5], [0.5, 0.5, 4, 4, 4]], np.float32)
    N = np.array([[2, 4, 6, 8, 10], [1, 1, 1, 1, 1]], np.float32)
    C = np.array([[1, 1, 1, 1, 7], [2, 0, 2, 0, 2]], np.float32)
    st, ct = _starts([[0, 1, 3], [0, 2]], 5)
    mH, mN, mC = oracle.patch_means(H, N, st, ct, C)
    assert mH[0, :3].tolist() == [1.0, 2.5, 4.5] and mH[1, :2].tolist() == [0.5, 4.0]
    assert mN[0, :3].tolist() == [2.0, 5.0, 9.0] and mN[1, :2].tolist() == [1.0, 1.0]
    assert mC[0, :3].tolist() == [1.0, 1.0, 4.0] and mC[1, 0] == 1.0
    assert mC[1, 1] == np.float32(4.0) / np.float32(3.0)  # (2 + 0 + 2) / 3 in f32


def test_edges():
    # count 0, a start past the row end (clamped: empty patch -> 0), T = 1
    H = np.array([[3.0, 1.0, 2.0]], np.float32)
    st, ct = _starts([[0, 5]], 3)
    mH, mN, mC = oracle.patch_means(H, H, st, ct)
    assert mC is None and mH[0, :2].tolist() == [2.0, 0.0]
    st0, ct0 = _starts([[]], 3)
    mH0, _, _ = oracle.patch_means(H, H, st0, ct0)
    assert not mH0.any()
    mH1, _, _ = oracle.patch_means(np.array([[7.0]], np.float32), np.ones((1, 1), np.float32),
                                   *_starts([[0]], 1))
    assert mH1[0, 0] == 7.0


def test_constant_rows_and_invariants():
    rng = np.random.default_rng(5)
    B, T = 4, 3000
    # constants whose f32 running sums are exact: the mean is the constant
    Hc = np.full((B, T), 0.5, np.float32)
    Nc = np.full((B, T), 3.0, np.float32)
    rows = []
    for b in range(B):
        cuts = np.sort(rng.choice(np.arange(1, T), size=200 + 50 * b, replace=False))
        rows.append([0] + cuts.tolist())
    st, ct = _starts(rows, T)
    mH, mN, _ = oracle.patch_means(Hc, Nc, st, ct)
    for b in range(B):
        assert (mH[b, :ct[b]] == 0.5).all() and (mN[b, :ct[b]] == 3.0).all()
    # random rows: mean * length sums to the row total, and each mean is the
    # fp64 mean to f32 accuracy
    H = (rng.random((B, T)) * 5.5).astype(np.float32)
    N = (rng.random((B, T)) * 40).astype(np.float32)
    mH, mN, _ = oracle.patch_means(H, N, st, ct)
    for b in range(B):
        s = rows[b] + [T]
        lens = np.diff(s)
        assert abs(float(np.dot(mH[b, :ct[b]].astype(np.float64), lens)) - math.fsum(H[b])) \
            < 1e-5 * math.fsum(H[b])
        for i in range(ct[b]):
            ref = math.fsum(N[b, s[i]:s[i + 1]].tolist()) / lens[i]
            assert abs(mN[b, i] - ref) <= 4e-7 * abs(ref) * max(1, lens[i])


@pytest.mark.gpu
def test_device_bit_exact_vs_oracle():
    import torch
    from blt_burn_amd import patcher
    rng = np.random.default_rng(9)
    for B, T in ((1, 1), (2, 2), (3, 17), (16, 8192)):
        H = (rng.normal(3.0, 1.0, (B, T))).astype(np.float32)
        N = (rng.random((B, T)) * 30).astype(np.float32)
        C = (N * N / (H + 1e-6)).astype(np.float32)
        Hd = torch.from_numpy(H).cuda()
        _, starts, _, counts = patcher.patch_boundaries(Hd, 0.2, patcher.PATCH_MONOTONIC)
        st, ct = starts.cpu().numpy(), counts.cpu().numpy()
        mH, mN, mC = patcher.patch_means(Hd, torch.from_numpy(N).cuda(), starts, counts,
                                         torch.from_numpy(C).cuda())
        rH, rN, rC = oracle.patch_means(H, N, st, ct, C)
        torch.cuda.synchronize()
        print("patch_means B=%d T=%d patches=%d" % (B, T, int(ct.sum())))
        for b in range(B):
            n = ct[b]
            assert np.array_equal(mH.cpu().numpy()[b, :n], rH[b, :n])
            assert np.array_equal(mN.cpu().numpy()[b, :n], rN[b, :n])
            assert np.array_equal(mC.cpu().numpy()[b, :n], rC[b, :n])
    # no coherence; zero rows
    Hd = torch.rand(2, 64, device="cuda")
    _, s2, _, c2 = patcher.patch_boundaries(Hd, 0.1)
    a, b_, c = patcher.patch_means(Hd, Hd, s2, c2)
    assert c is None
    e = torch.empty(0, 5, device="cuda")
    patcher.patch_means(e, e, torch.empty(0, 5, dtype=torch.int32, device="cuda"),
                        torch.empty(0, dtype=torch.int32, device="cuda"))


@pytest.mark.gpu
@pytest.mark.parametrize("T", [5000, 8192, 20000])
def test_device_long_patches_bit_exact(T):
    """Patches longer than the kernel's 2048-position LDS tiles (their sums
    carried from tile to tile), patches ending or starting exactly on tile
    edges, and one patch over the whole row, bit-exact against the oracle."""
    import torch
    from blt_burn_amd import patcher
    rng = np.random.default_rng(T)
    rows = [[0], [0, 1], [0, 2047, 2048, 2049, 4095, 4096, 4097],
            [0, 1, 3000, T - 1], [0] + sorted(rng.choice(np.arange(1, T), 7, replace=False)
                                              .tolist()),
            [0] + sorted(rng.choice(np.arange(1, T), T // 3, replace=False).tolist())]
    B = len(rows)
    H = rng.normal(3.0, 1.0, (B, T)).astype(np.float32)
    N = (rng.random((B, T)) * 30).astype(np.float32)
    C = (N * N / (H + 1e-6)).astype(np.float32)
    st, ct = _starts(rows, T)
    mH, mN, mC = patcher.patch_means(torch.from_numpy(H).cuda(), torch.from_numpy(N).cuda(),
                                     torch.from_numpy(st).cuda(), torch.from_numpy(ct).cuda(),
                                     torch.from_numpy(C).cuda())
    rH, rN, rC = oracle.patch_means(H, N, st, ct, C)
    for b in range(B):
        n = ct[b]
        assert np.array_equal(mH.cpu().numpy()[b, :n], rH[b, :n]), (T, b)
        assert np.array_equal(mN.cpu().numpy()[b, :n], rN[b, :n]), (T, b)
        assert np.array_equal(mC.cpu().numpy()[b, :n], rC[b, :n]), (T, b)


@pytest.mark.gpu
def test_device_rejects_bad_out_tensors():
    import torch
    from blt_burn_amd import BltError, patcher
    Hd = torch.rand(2, 64, device="cuda")
    _, s, _, c = patcher.patch_boundaries(Hd, 0.1)
    good = torch.empty(2, 64, device="cuda")
    bad = [torch.empty(2, 63, device="cuda"),                   # too small
           torch.empty(2, 64, device="cuda", dtype=torch.float64),
           torch.empty(64, 2, device="cuda").t(),               # not contiguous
           torch.empty(2, 64)]                                  # host memory
    for t in bad:
        with pytest.raises(BltError):
            patcher.patch_means(Hd, Hd, s, c, out=(t, good, None))
        with pytest.raises(BltError):
            patcher.patch_means(Hd, Hd, s, c, out=(good, t, None))
    with pytest.raises(BltError):  # a coherence output without coherence input
        patcher.patch_means(Hd, Hd, s, c, out=(good, good.clone(), good.clone()))
    with pytest.raises(BltError):  # coherence given, no output for it
        patcher.patch_means(Hd, Hd, s, c, Hd, out=(good, good.clone(), None))
    mH, mN, _ = patcher.patch_means(Hd, Hd, s, c, out=(good, good.clone(), None))
    assert mH is good
