"""Host-side logic mirrored from the reference: model config resolution and the
CPU half of the patcher API.  CPU only."""
import json
import os

import pytest
import torch

from blt_burn_amd import model as M
from blt_burn_amd import patcher

KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kat.json")))


def test_entropy_model_config_matches_reference():
    c = M.entropy_model_config()  # model_loader.rs:30-44, test 158-164
    assert (c.dim, c.n_layers, c.vocab_size) == (768, 14, 260)
    assert c.resolved_head_dim() == 64 and c.resolved_n_heads() == 12
    # model.rs:468-473: ffn_dim = (1.0 * 768) rounded up to 256 -> 768 (not 2048)
    assert c.ffn_hidden() == 768
    c2 = M.LMTransformerConfig(dim=768, n_layers=1, n_heads=12, ffn_dim_multiplier=None)
    assert c2.ffn_hidden() == 3072
    c3 = M.LMTransformerConfig(dim=768, n_layers=1, n_heads=12, ffn_dim_multiplier=2048 / 768)
    assert c3.ffn_hidden() == 2048


@pytest.mark.parametrize("case", KAT["patch"], ids=lambda c: c["name"])
def test_indices_and_lengths_from_mask(case):
    mask = torch.tensor(case["mask"], dtype=torch.int32)
    starts = patcher.patch_start_indices_cpu(mask)
    assert starts == case["starts"]
    T = mask.shape[1]
    assert patcher.patch_lengths_from_start_indices(starts, T) == case["lengths"]


def test_random_weights_shapes():
    cfg = M.LMTransformerConfig(dim=128, n_layers=2, n_heads=2, ffn_dim_multiplier=2.0,
                                multiple_of=64, vocab_size=260)
    w = M.random_weights(cfg, 1)
    assert w["wq"].shape == (2, 128, 128) and w["w1"].shape == (2, 128, 256)
    assert w["w2"].shape == (2, 256, 128) and w["output"].shape == (128, 260)
    w2 = M.random_weights(cfg, 1, hidden=512)
    assert w2["w3"].shape == (2, 128, 512)
