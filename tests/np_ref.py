"""Independent float64 NumPy statement of the reference's math, written from
the mathematics (materialised masks and score matrices, closed-form RoPE) to
pin the C oracle.  Test-only."""
import numpy as np


def entropy(logits):
    x = np.asarray(logits, np.float64)
    z = x - x.max(-1, keepdims=True)
    p = np.exp(z)
    p /= p.sum(-1, keepdims=True)
    with np.errstate(divide="ignore", invalid="ignore"):
        t = np.where(p > 0, p * np.log(p), 0.0)
    return -t.sum(-1)


def rms_norm(x, w, eps, mode=0):
    x = np.asarray(x, np.float64)
    rms2 = (x * x).mean(-1, keepdims=True)
    den = np.sqrt(rms2) + eps if mode == 0 else np.sqrt(rms2 + eps)
    return x / den * np.asarray(w, np.float64)


def l2_norm(x):
    x = np.asarray(x, np.float64)
    return np.sqrt((x * x).sum(-1))


def softmax(x):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def silu_gate(g, u):
    g = np.asarray(g, np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(u, np.float64)


def rope_angles(d, T, theta):
    i = np.arange(d // 2, dtype=np.float64)
    inv = theta ** (-2.0 * i / d)
    return np.arange(T, dtype=np.float64)[:, None] * inv[None, :]


def rotate(x, theta):
    """x [..., T, d] rotated with half-split pairs (x[m], x[m + d/2])."""
    x = np.asarray(x, np.float64)
    T, d = x.shape[-2], x.shape[-1]
    a = rope_angles(d, T, theta)
    c, s = np.cos(a), np.sin(a)
    x1, x2 = x[..., : d // 2], x[..., d // 2:]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], -1)


def mask_matrix(T, causal, window):
    i = np.arange(T)[:, None]
    j = np.arange(T)[None, :]
    vis = np.ones((T, T), bool)
    if causal:
        vis &= j <= i
        if window > 0:
            vis &= j > i - window
    return np.where(vis, 0.0, -np.inf)


def attention(q, k, v, causal=True, window=0, rope_theta=0.0):
    """[B, H, T, d] float64, materialised [T, T] scores."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    if rope_theta > 0:
        q, k = rotate(q, rope_theta), rotate(k, rope_theta)
    d = q.shape[-1]
    s = q @ np.swapaxes(k, -1, -2) / np.sqrt(d) + mask_matrix(q.shape[-2], causal, window)
    return softmax(s) @ v


def attention_qkv(q, k, v, causal=True):
    """[B, H, Tq, d] x [B, H, Tkv, d] float64 with a materialised mask (key j
    visible to query i iff j <= i); a query that sees no key gets 0."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    Tq, Tkv, d = q.shape[-2], k.shape[-2], q.shape[-1]
    s = q @ np.swapaxes(k, -1, -2) / np.sqrt(d)
    if causal:
        vis = np.arange(Tkv)[None, :] <= np.arange(Tq)[:, None]
        s = np.where(vis, s, -np.inf)
    with np.errstate(invalid="ignore"):
        mx = s.max(-1, keepdims=True)
        e = np.exp(s - np.where(np.isfinite(mx), mx, 0.0))
        w = e / np.maximum(e.sum(-1, keepdims=True), 1e-300)
    return np.nan_to_num(w) @ v


def model_forward(cfg, w, tokens):
    """cfg dict as oracle.model_forward; w: dict of float arrays in reference layouts."""
    D, L, Hn, F = cfg["dim"], cfg["n_layers"], cfg["n_heads"], cfg["hidden"]
    hd = D // Hn
    eps, theta, window = cfg["norm_eps"], cfg["rope_theta"], cfg.get("window", 0)
    W = {k: np.asarray(v, np.float64) for k, v in w.items()}
    tokens = np.asarray(tokens)
    B, T = tokens.shape
    x = W["emb"][tokens]
    for l in range(L):
        a = rms_norm(x, W["attn_norm"][l], eps)
        q = (a @ W["wq"][l]).reshape(B, T, Hn, hd).transpose(0, 2, 1, 3)
        k = (a @ W["wk"][l]).reshape(B, T, Hn, hd).transpose(0, 2, 1, 3)
        v = (a @ W["wv"][l]).reshape(B, T, Hn, hd).transpose(0, 2, 1, 3)
        o = attention(q, k, v, True, window, theta).transpose(0, 2, 1, 3).reshape(B, T, D)
        x = x + o @ W["wo"][l]
        f = rms_norm(x, W["ffn_norm"][l], eps)
        x = x + silu_gate(f @ W["w1"][l], f @ W["w3"][l]) @ W["w2"][l]
    pre = x
    norms = l2_norm(x)
    logits = rms_norm(x, W["norm"], eps) @ W["out"]
    H = entropy(logits)
    return {"logits": logits, "pre_norm_embeddings": pre, "embedding_norms": norms,
            "entropies": H, "coherence_scores": norms ** 2 / (H + 1e-6)}


def bf16_round(x):
    """float32 values rounded to the nearest bfloat16 (ties to even)."""
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


ROUNDING_POINTS = ("norm_in", "q", "k", "v", "p", "attn_out", "silu", "head_in")


def model_forward_bf16_operands(cfg, w, tokens, rounding=True, points=None):
    """model_forward in float32 with the GEMM and attention operands rounded to
    bf16 where a bf16-MFMA forward must round them: the RMSNorm-weighted
    activations x * w inside the layers (norm_in; the 1 / rms row factor
    applied to the GEMM output), q (scaled by 1 / sqrt(d) after RoPE), k and v,
    the softmax numerators P (p), the attention output (attn_out), the
    SiLU-gate product (silu) and the final norm's output (head_in).  `points`
    (a subset of ROUNDING_POINTS) rounds only those; rounding=False or an empty
    set is the float32 statement of the reference's math."""
    D, L, Hn = cfg["dim"], cfg["n_layers"], cfg["n_heads"]
    hd = D // Hn
    eps, theta, window = cfg["norm_eps"], cfg["rope_theta"], cfg.get("window", 0)
    if points is None:
        points = ROUNDING_POINTS if rounding else ()
    unknown = set(points) - set(ROUNDING_POINTS)
    assert not unknown, unknown

    def rp(name):
        return bf16_round if name in points else (lambda t: np.asarray(t, np.float32))
    W = {k: np.asarray(v, np.float32) for k, v in w.items()}
    tokens = np.asarray(tokens)
    B, T = tokens.shape
    ang = rope_angles(hd, T, theta).astype(np.float32)
    c, s = np.cos(ang), np.sin(ang)

    def rot(t):
        t1, t2 = t[..., : hd // 2], t[..., hd // 2:]
        return np.concatenate([t1 * c - t2 * s, t1 * s + t2 * c], -1)

    def heads(t):
        return t.reshape(B, T, Hn, hd).transpose(0, 2, 1, 3)

    def rstd(x):
        return 1.0 / (np.sqrt((x * x).mean(-1, keepdims=True)) + eps)

    mask = mask_matrix(T, True, window).astype(np.float32)
    x = W["emb"][tokens]
    for l in range(L):
        a, f = rp("norm_in")(x * W["attn_norm"][l]), rstd(x)
        q = rp("q")(rot(heads((a @ W["wq"][l]) * f)) / np.float32(np.sqrt(hd)))
        k = rp("k")(rot(heads((a @ W["wk"][l]) * f)))
        v = rp("v")(heads((a @ W["wv"][l]) * f))
        sc = q @ np.swapaxes(k, -1, -2) + mask
        p = rp("p")(np.exp(sc - sc.max(-1, keepdims=True)))
        o = (p @ v) / p.sum(-1, keepdims=True)
        x = x + rp("attn_out")(o.transpose(0, 2, 1, 3).reshape(B, T, D)) @ W["wo"][l]
        a, f = rp("norm_in")(x * W["ffn_norm"][l]), rstd(x)
        g, u = (a @ W["w1"][l]) * f, (a @ W["w3"][l]) * f
        x = x + rp("silu")(g / (1 + np.exp(-g)) * u) @ W["w2"][l]
    logits = rp("head_in")(x * rstd(x) * W["norm"]) @ W["out"]
    return {"logits": logits, "pre_norm_embeddings": x, "entropies": entropy(logits)}
