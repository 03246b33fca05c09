"""ctypes binding of libblt_hip.so (include/blt_hip.h).

The library is the product: every op in this package runs through it.  There
is no fallback — a missing library raises BltError.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libblt_hip.so")

c_i32, c_i64, c_f32, c_f64, c_u64 = (ctypes.c_int32, ctypes.c_int64, ctypes.c_float,
                                     ctypes.c_double, ctypes.c_uint64)
c_vp = ctypes.c_void_p

# blt_status / enums (include/blt_hip.h)
BLT_OK = 0
EPS_AFTER_SQRT, EPS_INSIDE_SQRT = 0, 1
PATCH_MONOTONIC, PATCH_GLOBAL = 0, 1
EPI_BF16, EPI_F32, EPI_RESID_F32, EPI_QKV_ROPE, EPI_SILU_GATE = 0, 1, 2, 3, 4
NUM_STAGES = 11

EXPORTS = {
    # name: (restype, argtypes)
    "blt_last_error": (ctypes.c_char_p, []),
    "blt_version": (ctypes.c_char_p, []),
    "blt_device_count": (c_i32, []),
    "blt_stream_sync": (c_i32, [c_vp]),
    "blt_fused_entropy_f32": (c_i32, [c_vp, c_vp, c_i64, c_i32, c_vp]),
    "blt_fused_entropy_bf16": (c_i32, [c_vp, c_vp, c_i64, c_i32, c_vp]),
    "blt_fused_rms_norm_f32": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i32, c_f32, c_i32, c_vp]),
    "blt_fused_rms_norm_bf16": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i32, c_f32, c_i32, c_vp]),
    "blt_fused_softmax_f32": (c_i32, [c_vp, c_vp, c_i64, c_i32, c_vp]),
    "blt_fused_l2_norm_f32": (c_i32, [c_vp, c_vp, c_i64, c_i32, c_vp]),
    "blt_fused_l2_norm_bf16": (c_i32, [c_vp, c_vp, c_i64, c_i32, c_vp]),
    "blt_fused_silu_gate_f32": (c_i32, [c_vp, c_vp, c_vp, c_i64, c_vp]),
    "blt_fused_silu_gate_bf16": (c_i32, [c_vp, c_vp, c_vp, c_i64, c_vp]),
    "blt_fused_coherence_f32": (c_i32, [c_vp, c_vp, c_vp, c_i64, c_f32, c_vp]),
    "blt_attention_workspace_bytes": (c_i64, [c_i64, c_i64, c_i64, c_i32]),
    "blt_fused_attention_bf16": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i32]
                                 + [c_i64] * 9 + [c_i32, c_i32, c_f32, c_vp, c_vp]),
    "blt_fused_attention_f32": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i32,
                                        c_i32, c_vp]),
    "blt_rope_table_f32": (c_i32, [c_vp, c_i32, c_i32, c_f64, c_vp]),
    "blt_patch_boundaries": (c_i32, [c_vp, c_i64, c_i64, c_f32, c_i32, c_vp, c_vp, c_vp, c_vp,
                                     c_vp]),
    "blt_patch_mask_starts": (c_i32, [c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp]),
    "blt_patch_means": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_vp,
                                c_vp]),
    "blt_patch_workspace_bytes": (c_i64, [c_i64, c_i64, c_i32]),
    "blt_patch_boundaries_rules": (c_i32, [c_vp, c_i64, c_i64, c_i32, c_vp, c_vp, c_i64, c_vp]),
    "blt_patch_boundaries_rules_noalloc": (c_i32, [c_vp, c_i64, c_i64, c_i32, c_vp, c_vp]),
    "blt_entropy_patch_boundaries": (c_i32, [c_vp, c_i64, c_i64, c_i32, c_vp, c_i32, c_vp, c_vp,
                                             c_i64, c_vp]),
    "blt_model_create": (c_i32, [c_i32, c_vp, c_vp, c_i64, ctypes.POINTER(c_vp)]),
    "blt_model_destroy": (c_i32, [c_vp]),
    "blt_model_device_bytes": (c_i64, [c_vp]),
    "blt_model_forward": (c_i32, [c_vp, c_vp, c_i64, c_i64, c_vp, c_vp]),
    "blt_model_forward_segments": (c_i32, [c_vp, c_vp, c_vp, c_i64, c_i64, c_vp, c_vp]),
    "blt_model_extract_embeddings": (c_i32, [c_vp, c_vp, c_i64, c_i64, c_vp, c_vp]),
    "blt_tokenize_bytes": (c_i32, [c_vp, c_i64, c_i32, c_i32, c_vp, c_i64, c_vp]),
    "blt_tokenize_documents": (c_i32, [c_vp, c_vp, c_i64, c_i32, c_i32, c_vp, c_i64, c_vp]),
    "blt_ingest_plan_chunks": (c_i32, [c_i64, c_i32, c_i32, c_vp, c_vp, c_vp, c_i64]),
    "blt_ingest_create": (c_i32, [c_vp, c_vp, c_vp]),
    "blt_ingest_destroy": (c_i32, [c_vp]),
    "blt_ingest_last_stats": (c_i32, [c_vp, c_vp]),
    "blt_ingest_run": (c_i32, [c_vp, c_vp, c_vp, c_i64] + [c_vp] * 7),
    "blt_ingest_run_patch_means": (c_i32, [c_vp, c_vp, c_vp, c_i64] + [c_vp] * 10),
    "blt_pipeline_create": (c_i32, [c_vp, c_f64, c_vp]),
    "blt_pipeline_destroy": (c_i32, [c_vp]),
    "blt_pipeline_process_chunk": (c_i32, [c_vp, c_vp, c_i64, c_i32, c_i64] + [c_vp] * 6),
    "blt_pipeline_reset": (c_i32, [c_vp]),
    "blt_pipeline_accumulated": (c_i32, [c_vp, c_vp]),
    "blt_pipeline_read": (c_i32, [c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp]),
    "blt_pipeline_process_documents": (c_i32, [c_vp, c_vp, c_vp, c_i64, c_i32, c_i32, c_vp, c_vp,
                                               c_i64] + [c_vp] * 6),
    "blt_model_set_profiling": (c_i32, [c_vp, c_i32]),
    "blt_model_read_profile": (c_i32, [c_vp, ctypes.POINTER(c_f64), ctypes.POINTER(c_i64), c_i32]),
    "blt_stage_name": (ctypes.c_char_p, [c_i32]),
    "blt_synth_normal_f32": (c_i32, [c_u64, c_vp, c_i64, c_f64, c_f64]),
    "blt_synth_normal_bf16": (c_i32, [c_u64, c_vp, c_i64, c_f64, c_f64]),
    "blt_synth_tokens": (c_i32, [c_u64, c_vp, c_i64, c_f64, c_f64, c_i32]),
    "blt_gemm_bf16": (c_i32, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp]),
    "blt_gemm_bf16_epilogue": (c_i32, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                       c_i32, c_i32, c_i32, c_i64, c_vp, c_vp]),
    "blt_probe_mfma_flops": (c_i64, [c_i32, c_i32]),
    "blt_probe_mfma_bf16": (c_i32, [c_i32, c_i32, c_vp, c_vp]),
    "blt_probe_copy": (c_i32, [c_vp, c_vp, c_i64, c_vp]),
}


class BltError(RuntimeError):
    """A non-zero blt_status from the library (the reference panics instead)."""


class ModelConfig(ctypes.Structure):
    _fields_ = [("dim", c_i32), ("n_layers", c_i32), ("n_heads", c_i32), ("ffn_hidden", c_i32),
                ("vocab", c_i32), ("max_seqlen", c_i32), ("norm_eps", c_f32),
                ("rope_theta", c_f32), ("window", c_i32)]


WEIGHT_FIELDS = ("tok_embeddings", "attention_norm", "ffn_norm", "wq", "wk", "wv", "wo", "w1",
                 "w2", "w3", "norm", "output")


class ModelWeights(ctypes.Structure):
    _fields_ = [(n, c_vp) for n in WEIGHT_FIELDS]


OUTPUT_FIELDS = ("logits", "pre_norm_embeddings", "embedding_norms", "entropies",
                 "coherence_scores")


class ModelOutputs(ctypes.Structure):
    _fields_ = [(n, c_vp) for n in OUTPUT_FIELDS]


class PatchRule(ctypes.Structure):
    """blt_patch_rule."""
    _fields_ = [("mode", c_i32), ("threshold", c_f32), ("mask", c_vp), ("starts", c_vp),
                ("lengths", c_vp), ("count", c_vp)]


class IngestStats(ctypes.Structure):
    """blt_ingest_stats."""
    _fields_ = [("batches", c_i64), ("documents", c_i64), ("tokens", c_i64),
                ("tokens_computed", c_i64), ("row_tokens", c_i64), ("long_documents", c_i64),
                ("long_documents_host", c_i64)]


class IngestConfig(ctypes.Structure):
    """blt_ingest_config."""
    _fields_ = [("rows", c_i32), ("row_len", c_i32), ("chunk_len", c_i32), ("overlap", c_i32),
                ("threshold", c_f32), ("mode", c_i32), ("with_embeddings", c_i32),
                ("long_arena_tokens", c_i32)]


_lib = None


def lib():
    """Load libblt_hip.so once; raise BltError when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise BltError("libblt_hip.so is not built (%s); run __graft_entry__.build()"
                           % LIB_PATH)
        # torch bundles its own libamdhip64.so.7; load it first so this library
        # binds to the same HIP runtime (one runtime, shared streams and memory)
        # instead of pulling a second copy from /opt/rocm.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in EXPORTS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def last_error():
    return lib().blt_last_error().decode(errors="replace")


def check(rc, what):
    if rc != BLT_OK:
        raise BltError("%s failed with status %d: %s" % (what, rc, last_error()))
