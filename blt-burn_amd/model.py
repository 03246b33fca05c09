"""The BLT entropy model (src/model.rs) on gfx950.

LMTransformerConfig / entropy_model_config mirror model.rs:167-226 and
model_loader.rs:30-44; LMTransformer.forward_with_embeddings mirrors
model.rs:269-322 and returns a ModelOutput (model.rs:229-245).  The whole
forward is one call into libblt_hip.so (blt_model_forward); weights are
packed once onto the device by blt_model_create.
"""
import ctypes
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import _lib, synth
from ._lib import BltError, ModelConfig, ModelOutputs, ModelWeights, WEIGHT_FIELDS, check
from ._torch import require_cuda, stream_ptr

__all__ = ["LMTransformerConfig", "entropy_model_config", "ModelOutput", "LMTransformer",
           "random_weights"]


@dataclass
class LMTransformerConfig:
    """model.rs:167-180."""
    dim: int
    n_layers: int
    head_dim: Optional[int] = None
    n_heads: Optional[int] = None
    n_kv_heads: Optional[int] = None
    ffn_dim_multiplier: Optional[float] = None
    multiple_of: int = 256
    norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    max_seqlen: int = 8192
    vocab_size: int = 260

    def resolved_head_dim(self):
        # model.rs:184-186
        return self.head_dim or self.dim // (self.n_heads or 1)

    def resolved_n_heads(self):
        return self.n_heads or self.dim // self.resolved_head_dim()

    def ffn_hidden(self):
        """FFN width as TransformerBlockConfig::init computes it (model.rs:468-473):
        int(multiplier * dim) (4 * dim without a multiplier), rounded up to multiple_of."""
        f = int(self.ffn_dim_multiplier * self.dim) if self.ffn_dim_multiplier is not None \
            else 4 * self.dim
        return self.multiple_of * ((f + self.multiple_of - 1) // self.multiple_of)


def entropy_model_config():
    """model_loader.rs:30-44 (hidden resolves to 768; real weights carry 2048)."""
    return LMTransformerConfig(dim=768, n_layers=14, head_dim=None, n_heads=12, n_kv_heads=None,
                               ffn_dim_multiplier=1.0, multiple_of=256, norm_eps=1e-5,
                               rope_theta=10000.0, max_seqlen=8192, vocab_size=260)


@dataclass
class ModelOutput:
    """model.rs:229-245."""
    logits: torch.Tensor
    pre_norm_embeddings: torch.Tensor
    embedding_norms: torch.Tensor
    entropies: Optional[torch.Tensor]
    coherence_scores: Optional[torch.Tensor]


def random_weights(cfg, seed, hidden=None, std=0.02, norm_std=0.02):
    """Seeded random weights in the reference's layouts (Burn Linear = [in, out]),
    as bf16 bits (numpy uint16): linear and embedding weights ~ N(0, std), norm
    weights ~ 1 + N(0, norm_std).  `hidden` overrides the FFN width (2048 for the
    real facebook/blt-entropy shapes)."""
    D, L, V = cfg.dim, cfg.n_layers, cfg.vocab_size
    F = hidden or cfg.ffn_hidden()
    shapes = {
        "tok_embeddings": (V, D), "attention_norm": (L, D), "ffn_norm": (L, D),
        "wq": (L, D, D), "wk": (L, D, D), "wv": (L, D, D), "wo": (L, D, D),
        "w1": (L, D, F), "w2": (L, F, D), "w3": (L, D, F), "norm": (D,), "output": (D, V),
    }
    w = {}
    for i, name in enumerate(WEIGHT_FIELDS):
        is_norm = name in ("attention_norm", "ffn_norm", "norm")
        w[name] = synth.normal_bf16(seed * 64 + i, shapes[name], 1.0 if is_norm else 0.0,
                                    norm_std if is_norm else std)
    return w


class LMTransformer:
    """LMTransformerConfig::init + load_record on one GPU (model.rs:182-226)."""

    def __init__(self, cfg, weights, device=0, max_tokens=None, window=0, hidden=None):
        self.cfg = cfg
        self.device = torch.device("cuda", device) if isinstance(device, int) else device
        self.hidden = hidden or weights["w1"].shape[-1]
        self.window = window
        self.max_tokens = max_tokens or cfg.max_seqlen
        if cfg.n_kv_heads not in (None, cfg.resolved_n_heads()):
            raise BltError("grouped-query attention is not on this path (n_kv_heads == n_heads)")
        c = ModelConfig(cfg.dim, cfg.n_layers, cfg.resolved_n_heads(), self.hidden,
                        cfg.vocab_size, cfg.max_seqlen, cfg.norm_eps, cfg.rope_theta, window)
        keep = {n: np.ascontiguousarray(weights[n], dtype=np.uint16) for n in WEIGHT_FIELDS}
        w = ModelWeights(*[keep[n].ctypes.data for n in WEIGHT_FIELDS])
        h = ctypes.c_void_p()
        check(_lib.lib().blt_model_create(self.device.index or 0, ctypes.byref(c),
                                          ctypes.byref(w), self.max_tokens, ctypes.byref(h)),
              "blt_model_create")
        self._h = h

    @classmethod
    def from_safetensors(cls, path, cfg=None, device=0, max_tokens=None, window=0):
        """load_entropy_model (model_loader.rs:103-145) from a local safetensors
        checkpoint with facebook/blt-entropy tensor names: the config defaults to
        entropy_model_config() and the FFN width comes from the file."""
        from .safetensors_io import load_entropy_weights
        w, shp = load_entropy_weights(path)
        return cls._from_loaded(path, w, shp, cfg, device, max_tokens, window)

    @classmethod
    def from_mpk(cls, path, cfg=None, device=0, max_tokens=None, window=0):
        """load_entropy_model's `.mpk` branch (model_loader.rs:119-125): a Burn
        NamedMpkFileRecorder record of the module, Linear weights already in
        Burn's [d_input, d_output] layout."""
        from .mpk_io import load_entropy_weights_mpk
        w, shp = load_entropy_weights_mpk(path)
        return cls._from_loaded(path, w, shp, cfg, device, max_tokens, window)

    @classmethod
    def from_checkpoint(cls, path, cfg=None, device=0, max_tokens=None, window=0):
        """load_entropy_model (model_loader.rs:103-145): the format follows the
        file name, `.mpk` for a Burn record and safetensors otherwise."""
        if str(path).endswith(".mpk"):
            return cls.from_mpk(path, cfg, device, max_tokens, window)
        return cls.from_safetensors(path, cfg, device, max_tokens, window)

    @classmethod
    def _from_loaded(cls, path, w, shp, cfg, device, max_tokens, window):
        cfg = cfg or entropy_model_config()
        if (cfg.dim, cfg.n_layers, cfg.vocab_size) != (shp["dim"], shp["n_layers"], shp["vocab"]):
            raise BltError("checkpoint %s holds dim %d, %d layers, vocab %d; the config says "
                           "dim %d, %d layers, vocab %d" % (path, shp["dim"], shp["n_layers"],
                                                            shp["vocab"], cfg.dim, cfg.n_layers,
                                                            cfg.vocab_size))
        return cls(cfg, w, device=device, max_tokens=max_tokens, window=window,
                   hidden=shp["hidden"])

    def __del__(self):
        # pipeline buffers cached on this model hold handles into it: free them first
        for buf in self.__dict__.pop("_pipeline_cache", {}).values():
            buf.close()
        h = getattr(self, "_h", None)
        # at interpreter exit the module globals may already be gone
        if h is not None and h.value and _lib is not None and _lib._lib is not None:
            _lib.lib().blt_model_destroy(h)
            self._h = None

    def device_bytes(self):
        return _lib.lib().blt_model_device_bytes(self._h)

    def forward_with_embeddings(self, tokens, out=None, seg_start=None):
        """tokens: int32 [batch, seq] on this GPU.  Returns ModelOutput with logits
        [B, T, V] f32, pre_norm_embeddings [B, T, D] f32, embedding_norms [B, T],
        entropies [B, T], coherence_scores [B, T].  `out` may hold preallocated
        tensors under those names (reused, nothing allocated).

        seg_start (optional int32 [B, T] on this GPU): position of the first
        token of each token's segment, non-decreasing along a row.  Several
        independent sequences then share one row: attention stays inside a
        segment and RoPE positions restart at each segment start, so every
        segment's outputs equal a separate forward of that segment alone."""
        require_cuda(tokens)
        if tokens.dim() != 2:
            raise BltError("forward_with_embeddings expects tokens [batch, seq]")
        tok = tokens if (tokens.dtype == torch.int32 and tokens.is_contiguous()) \
            else tokens.to(torch.int32).contiguous()
        B, T = tok.shape
        D, V = self.cfg.dim, self.cfg.vocab_size
        shapes = {"logits": (B, T, V), "pre_norm_embeddings": (B, T, D),
                  "embedding_norms": (B, T), "entropies": (B, T), "coherence_scores": (B, T)}
        res = {}
        for n, shp in shapes.items():
            t = out.get(n) if out else None
            if t is None:
                t = torch.empty(shp, dtype=torch.float32, device=tok.device)
            elif tuple(t.shape) != shp or t.dtype != torch.float32 or not t.is_contiguous():
                raise BltError("output %s must be contiguous f32 %s" % (n, shp))
            res[n] = t
        o = ModelOutputs(*[res[n].data_ptr() for n in _lib.OUTPUT_FIELDS])
        if seg_start is None:
            check(_lib.lib().blt_model_forward(self._h, tok.data_ptr(), B, T, ctypes.byref(o),
                                               stream_ptr(tok.device)), "blt_model_forward")
        else:
            require_cuda(seg_start)
            if tuple(seg_start.shape) != (B, T) or seg_start.dtype != torch.int32 \
                    or not seg_start.is_contiguous():
                raise BltError("seg_start must be contiguous int32 [batch, seq]")
            check(_lib.lib().blt_model_forward_segments(
                self._h, tok.data_ptr(), seg_start.data_ptr(), B, T, ctypes.byref(o),
                stream_ptr(tok.device)), "blt_model_forward_segments")
        return ModelOutput(**res)

    def extract_embeddings(self, tokens, out=None):
        """LMTransformer::extract_embeddings (model.rs:325-345, 413-431): the
        pre-normalisation residual after the last layer, f32 [B, T, D].  No
        final norm, head, entropy or coherence is computed.  `out` may pass the
        result tensor preallocated (contiguous f32 [B, T, D] on this GPU)."""
        require_cuda(tokens)
        if tokens.dim() != 2:
            raise BltError("extract_embeddings expects tokens [batch, seq]")
        tok = tokens if (tokens.dtype == torch.int32 and tokens.is_contiguous()) \
            else tokens.to(torch.int32).contiguous()
        B, T = tok.shape
        shp = (B, T, self.cfg.dim)
        if out is None:
            out = torch.empty(shp, dtype=torch.float32, device=tok.device)
        elif (tuple(out.shape) != shp or out.dtype != torch.float32 or not out.is_contiguous()
              or out.device != tok.device):
            raise BltError("extract_embeddings: out must be contiguous f32 %s on the tokens' "
                           "device" % (shp,))
        check(_lib.lib().blt_model_extract_embeddings(self._h, tok.data_ptr(), B, T,
                                                      out.data_ptr(), stream_ptr(tok.device)),
              "blt_model_extract_embeddings")
        return out

    def set_profiling(self, on=True):
        """Record HIP events between the forward's kernels (per-stage timing)."""
        check(_lib.lib().blt_model_set_profiling(self._h, 1 if on else 0), "set_profiling")

    def read_profile(self):
        """{stage name: (total ms, launches)} since the last read; waits for the GPU."""
        n = _lib.NUM_STAGES
        ms = (ctypes.c_double * n)()
        cnt = (ctypes.c_int64 * n)()
        check(_lib.lib().blt_model_read_profile(self._h, ms, cnt, n), "read_profile")
        return {_lib.lib().blt_stage_name(i).decode(): (ms[i], cnt[i]) for i in range(n)}

    def forward(self, tokens):
        """Logits only (model.rs:263-266)."""
        return self.forward_with_embeddings(tokens).logits
