"""Host-side logic that runs without a GPU: synthetic checkpoints, config parsing, rope tables,
the cap rule, and the engine's refusal to run without a GPU."""
import tempfile

import pytest
import torch

from dryft_amd import synth
from dryft_amd.engine import CAP_GRAN, Engine, build_rope_tables, rope_theta
from oracle.reference import OracleEngine
from oracle.reference import build_rope_tables as oracle_rope


def test_synth_is_deterministic_and_named_like_hf():
    cfg = synth.qwen3_config(num_hidden_layers=2, vocab_size=512, hidden_size=256,
                             intermediate_size=192, num_attention_heads=8, num_key_value_heads=2)
    a = synth.random_weights(cfg, seed=3)
    b = synth.random_weights(cfg, seed=3)
    c = synth.random_weights(cfg, seed=4)
    assert a.keys() == b.keys()
    assert all(torch.equal(a[k], b[k]) for k in a)
    assert not torch.equal(a["model.embed_tokens.weight"], c["model.embed_tokens.weight"])
    assert a["model.layers.0.self_attn.q_proj.weight"].shape == (8 * 128, 256)
    assert a["model.layers.1.mlp.down_proj.weight"].shape == (256, 192)
    assert "lm_head.weight" not in a                      # tied
    w = a["model.layers.0.mlp.up_proj.weight"].float()
    assert abs(w.std().item() - 0.02) < 0.002 and abs(w.mean().item()) < 0.002
    n = a["model.layers.0.input_layernorm.weight"].float()
    assert abs(n.mean().item() - 1.0) < 0.01


def test_synth_roundtrip_through_safetensors():
    cfg = synth.qwen3_config(num_hidden_layers=1, vocab_size=256, hidden_size=128,
                             intermediate_size=64, num_attention_heads=2, num_key_value_heads=1)
    w = synth.random_weights(cfg, seed=0)
    d = tempfile.mkdtemp()
    synth.write_model(d, cfg, w)
    ref_dir = OracleEngine(d)
    ref_mem = OracleEngine.from_state_dict(cfg, w)
    assert torch.equal(ref_dir.layers[0].wqkv, ref_mem.layers[0].wqkv)
    # q | k | v order of the fused projection (engine.py:300-302)
    assert torch.equal(ref_mem.layers[0].wqkv[:256], w["model.layers.0.self_attn.q_proj.weight"])
    assert torch.equal(ref_mem.layers[0].wqkv[256:384], w["model.layers.0.self_attn.k_proj.weight"])
    assert torch.equal(ref_mem.lm_head, ref_mem.embed)


def test_rope_theta_both_config_forms():
    assert rope_theta({"rope_theta": 5e6}) == 5e6
    assert rope_theta({"rope_parameters": {"rope_theta": 1e6, "rope_type": "default"}}) == 1e6


def test_engine_rope_tables_are_the_oracle_bits():
    cos, sin = build_rope_tables(5e6, 128, 1024)
    rc, rs = oracle_rope(5e6, 128, 1024)
    assert torch.equal(cos, rc) and torch.equal(sin, rs)


def test_cap_rule():
    # engine.py:707: cap = ceil((S + n) / 128) * 128
    for S, n, cap in ((512, 32, 640), (2048, 1024, 3072), (1, 1, 128), (127, 1, 128), (128, 1, 256)):
        assert -(-(S + n) // CAP_GRAN) * CAP_GRAN == cap


def test_engine_refuses_cpu():
    with pytest.raises(RuntimeError):
        Engine.from_state_dict(synth.qwen3_config(num_hidden_layers=1), {}, device="cpu")


@pytest.mark.parametrize("nh,nkv", [(4, 1), (8, 2), (32, 8), (64, 8), (32, 16)])
def test_qkv_head_grouped_order(nh, nkv):
    """The fused step's raw q|k|v slot is head-grouped (per kv head: its nh / nkv q heads, then
    k, then v, 128 columns each). FusedStep.qkv_natural must map it back to cat(q, k, v): applied
    to the head-grouped order of the column indices it gives 0, 1, 2, ... and it keeps every head
    of a group next to its own k and v (head h of group g is q head g * nh / nkv + h)."""
    from dryft_amd.step import FusedStep
    hd = 128
    g = nh // nkv
    n = (nh + 2 * nkv) * hd
    # head-grouped order written out head by head (the layout the step's QKV phase writes)
    order = []
    for kv in range(nkv):
        for h in range(g):
            order += range((kv * g + h) * hd, (kv * g + h + 1) * hd)
        order += range((nh + kv) * hd, (nh + kv + 1) * hd)
        order += range((nh + nkv + kv) * hd, (nh + nkv + kv + 1) * hd)
    grouped = torch.tensor(order).view(1, 1, n)
    assert sorted(order) == list(range(n))
    assert torch.equal(FusedStep.qkv_natural(grouped, nh, nkv).view(-1), torch.arange(n))
