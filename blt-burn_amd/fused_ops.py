"""Fused ops with the reference's public signatures (src/fused_ops/mod.rs:155-236).

Each function takes torch tensors on the GPU, allocates its output like the
reference's CubeBackend impl (a fresh contiguous tensor, backend.rs:42-53),
and runs one gfx950 kernel through libblt_hip.so on the current stream.
Inputs are f32 (Burn's default float) or bf16.  Shape mismatches raise
(where the reference panics).
"""
import torch

from . import _lib
from ._lib import EPS_AFTER_SQRT, EPS_INSIDE_SQRT, BltError, check
from ._torch import contiguous, require_cuda, stream_ptr

__all__ = ["fused_entropy", "fused_rms_norm", "fused_softmax", "fused_l2_norm",
           "fused_silu_gate", "fused_coherence", "fused_attention", "EPS_AFTER_SQRT",
           "EPS_INSIDE_SQRT"]


def _dtype_ok(t):
    if t.dtype not in (torch.float32, torch.bfloat16):
        raise BltError("unsupported dtype %s (f32 or bf16)" % t.dtype)


def fused_entropy(logits, vocab_size):
    """[batch, seq, vocab] -> [batch, seq] f32 softmax entropy, natural log
    (mod.rs:155-159; NdArray form patcher.rs:38-63)."""
    require_cuda(logits)
    _dtype_ok(logits)
    if logits.dim() != 3:
        raise BltError("fused_entropy expects [batch, seq, vocab], got %s" % (tuple(logits.shape),))
    b, s, v = logits.shape
    if v != vocab_size:
        raise BltError("vocab_size %d does not match logits' last dim %d" % (vocab_size, v))
    x = contiguous(logits)
    out = torch.empty((b, s), dtype=torch.float32, device=x.device)
    f = (_lib.lib().blt_fused_entropy_f32 if x.dtype == torch.float32
         else _lib.lib().blt_fused_entropy_bf16)
    check(f(x.data_ptr(), out.data_ptr(), b * s, v, stream_ptr(x.device)), "fused_entropy")
    return out


def fused_rms_norm(input, weight, epsilon, eps_mode=EPS_AFTER_SQRT, l2_out=None):
    """[batch, seq, dim] x weight[dim] -> [batch, seq, dim] (mod.rs:162-176).

    eps_mode EPS_AFTER_SQRT is the model's formula x / (sqrt(mean x^2) + eps) * w
    (model.rs:758-770, and the reference's Fusion fallback backend.rs:502-506);
    EPS_INSIDE_SQRT is x / sqrt(mean x^2 + eps) * w (rms_norm_kernel.rs:40-43).
    l2_out, if given, is an f32 [batch, seq] tensor receiving sqrt(sum x^2)."""
    require_cuda(input, weight)
    _dtype_ok(input)
    if input.dim() != 3 or weight.dim() != 1 or weight.shape[0] != input.shape[-1]:
        raise BltError("fused_rms_norm expects x [batch, seq, dim] and weight [dim]")
    x = contiguous(input)
    w = contiguous(weight.to(x.dtype))
    y = torch.empty_like(x)
    rows, dim = x.numel() // x.shape[-1], x.shape[-1]
    l2p = 0
    if l2_out is not None:
        require_cuda(l2_out)
        if l2_out.dtype != torch.float32 or l2_out.numel() != rows or not l2_out.is_contiguous():
            raise BltError("l2_out must be a contiguous f32 tensor with one value per row")
        l2p = l2_out.data_ptr()
    f = (_lib.lib().blt_fused_rms_norm_f32 if x.dtype == torch.float32
         else _lib.lib().blt_fused_rms_norm_bf16)
    check(f(x.data_ptr(), w.data_ptr(), y.data_ptr(), l2p, rows, dim, float(epsilon), eps_mode,
            stream_ptr(x.device)), "fused_rms_norm")
    return y


def fused_softmax(input, dim_size):
    """Softmax over the last dim of an f32 tensor of any rank (mod.rs:179-185)."""
    require_cuda(input)
    if input.dtype != torch.float32:
        raise BltError("fused_softmax takes f32")
    if input.dim() == 0 or input.shape[-1] != dim_size:
        raise BltError("dim_size %d does not match the last dim" % dim_size)
    x = contiguous(input)
    y = torch.empty_like(x)
    check(_lib.lib().blt_fused_softmax_f32(x.data_ptr(), y.data_ptr(), x.numel() // dim_size,
                                           dim_size, stream_ptr(x.device)), "fused_softmax")
    return y


def fused_l2_norm(input):
    """[batch, seq, dim] -> [batch, seq] f32 sqrt(sum x^2) (mod.rs:188-192)."""
    require_cuda(input)
    _dtype_ok(input)
    if input.dim() != 3:
        raise BltError("fused_l2_norm expects [batch, seq, dim]")
    x = contiguous(input)
    b, s, d = x.shape
    out = torch.empty((b, s), dtype=torch.float32, device=x.device)
    f = (_lib.lib().blt_fused_l2_norm_f32 if x.dtype == torch.float32
         else _lib.lib().blt_fused_l2_norm_bf16)
    check(f(x.data_ptr(), out.data_ptr(), b * s, d, stream_ptr(x.device)), "fused_l2_norm")
    return out


def fused_silu_gate(gate_input, up_input):
    """silu(gate) * up, elementwise (mod.rs:195-205)."""
    require_cuda(gate_input, up_input)
    _dtype_ok(gate_input)
    if gate_input.shape != up_input.shape or gate_input.dtype != up_input.dtype:
        raise BltError("fused_silu_gate: gate and up must have one shape and dtype")
    g, u = contiguous(gate_input), contiguous(up_input)
    out = torch.empty_like(g)
    f = (_lib.lib().blt_fused_silu_gate_f32 if g.dtype == torch.float32
         else _lib.lib().blt_fused_silu_gate_bf16)
    check(f(g.data_ptr(), u.data_ptr(), out.data_ptr(), g.numel(), stream_ptr(g.device)),
          "fused_silu_gate")
    return out


def fused_coherence(norms, entropies, epsilon):
    """norms^2 / (entropies + epsilon), f32 (mod.rs:208-220)."""
    require_cuda(norms, entropies)
    if norms.dtype != torch.float32 or entropies.dtype != torch.float32:
        raise BltError("fused_coherence takes f32")
    if norms.shape != entropies.shape:
        raise BltError("fused_coherence: shapes differ")
    n, e = contiguous(norms), contiguous(entropies)
    out = torch.empty_like(n)
    check(_lib.lib().blt_fused_coherence_f32(n.data_ptr(), e.data_ptr(), out.data_ptr(),
                                             n.numel(), float(epsilon), stream_ptr(n.device)),
          "fused_coherence")
    return out


def fused_attention(q, k, v, use_causal_mask, window=0, rope_theta=0.0):
    """Scaled dot-product attention over [batch, heads, seq, head_dim] (mod.rs:225-236).

    f32 q, k, v without a window or RoPE: the reference kernel's semantics
    (attention_kernel.rs:20-125) in f32 throughout, any head_dim <= 256, k and v
    may have another seq length than q (causal: key j visible to query i iff
    j <= i).  bf16 inputs (or a window > 0 / rope_theta > 0, this build's
    extensions for the entropy model) take the MFMA path: head_dim 64, q, k, v
    of one shape, QK^T and PV on bf16 MFMA with an f32 softmax; f32 inputs are
    rounded to bf16 there and the output is returned in the input dtype."""
    require_cuda(q, k, v)
    _dtype_ok(q)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise BltError("fused_attention expects q, k, v [batch, heads, seq, head_dim]")
    if (q.dtype == torch.float32 and k.dtype == torch.float32 and v.dtype == torch.float32 and
            window == 0 and rope_theta == 0):
        B, H, Tq, d = q.shape
        if tuple(k.shape[:2]) != (B, H) or k.shape[3] != d or k.shape != v.shape:
            raise BltError("fused_attention: k and v must be [batch, heads, seq_kv, head_dim] "
                           "with q's batch, heads and head_dim")
        qc, kc, vc = (contiguous(t) for t in (q, k, v))
        o = torch.empty_like(qc)
        check(_lib.lib().blt_fused_attention_f32(
            qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), o.data_ptr(), B, H, Tq, kc.shape[2], d,
            1 if use_causal_mask else 0, stream_ptr(qc.device)), "fused_attention")
        return o
    if q.shape != k.shape or q.shape != v.shape:
        raise BltError("fused_attention (MFMA path) expects q, k, v of one shape "
                       "[batch, heads, seq, 64]")
    B, H, T, d = q.shape
    in_dtype = q.dtype
    qb, kb, vb = (contiguous(t.to(torch.bfloat16)) for t in (q, k, v))
    o = torch.empty_like(qb)
    ws = None
    if rope_theta > 0:
        nbytes = _lib.lib().blt_attention_workspace_bytes(B, H, T, d)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=qb.device)
    sb, sh, st = H * T * d, T * d, d
    check(_lib.lib().blt_fused_attention_bf16(
        qb.data_ptr(), kb.data_ptr(), vb.data_ptr(), o.data_ptr(), B, H, T, d,
        sb, sh, st, sb, sh, st, sb, sh, st, 1 if use_causal_mask else 0, int(window),
        float(rope_theta), ws.data_ptr() if ws is not None else 0, stream_ptr(qb.device)),
        "fused_attention")
    return o if in_dtype == torch.bfloat16 else o.to(in_dtype)
