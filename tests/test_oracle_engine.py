"""Pin the oracle's model restatement end to end (CPU only).

* Token-exact against HF ``Qwen3ForCausalLM.generate`` (greedy) on the reference's tiny fp32
  config (tests/test_vs_hf.py:13-45): weight names and q|k|v / gate|up concat order, tied
  lm_head, norms, rope, GQA mapping and the decode loop all have to be right for this to pass.
* No state leak across calls, ragged grouping, n = 0 (test_vs_hf.py:36-44).
* Verify-shaped forward == sequential decode (engine.py:549-627), per-row decode == per-sequence
  decode (engine.py:1093-1105 semantics).
"""
import tempfile

import pytest
import torch

from oracle.reference import OracleEngine


@pytest.fixture(scope="module")
def tiny():
    from transformers import Qwen3Config, Qwen3ForCausalLM
    torch.manual_seed(0)
    cfg = Qwen3Config(
        vocab_size=300, hidden_size=64, intermediate_size=128, num_hidden_layers=3,
        num_attention_heads=4, num_key_value_heads=2, head_dim=32,
        rope_theta=5e6, rms_norm_eps=1e-6, tie_word_embeddings=True,
        max_position_embeddings=4096,
    )
    model = Qwen3ForCausalLM(cfg).eval()
    d = tempfile.mkdtemp()
    model.save_pretrained(d)
    return model, OracleEngine(d, dtype=torch.float32)


@pytest.mark.parametrize("B,S,n", [(1, 20, 12), (3, 37, 9), (2, 130, 5)])
def test_oracle_matches_hf_greedy(tiny, B, S, n):
    model, eng = tiny
    g = torch.Generator().manual_seed(B * 1000 + S)
    ids = torch.randint(0, 300, (B, S), generator=g)
    with torch.inference_mode():
        ref = model.generate(ids, attention_mask=torch.ones_like(ids), do_sample=False,
                             max_new_tokens=n, min_new_tokens=n, eos_token_id=None,
                             pad_token_id=0)[:, S:]
    out = torch.tensor(list(eng.generate(ids.tolist(), n))).T
    assert torch.equal(ref, out)


def test_oracle_state_reuse_ragged_and_empty(tiny):
    _, eng = tiny
    ids = torch.randint(0, 300, (3, 37), generator=torch.Generator().manual_seed(7))
    a = list(eng.generate(ids.tolist(), 9))
    b = list(eng.generate(ids.tolist(), 9))
    assert a == b
    r = list(eng.generate([[1, 2, 3], [4, 5, 6, 7]], 4))
    assert len(r) == 4 and all(len(x) == 2 for x in r)
    # ragged == each sequence on its own
    solo0 = list(eng.generate([[1, 2, 3]], 4))
    solo1 = list(eng.generate([[4, 5, 6, 7]], 4))
    assert [x[0] for x in r] == [x[0] for x in solo0]
    assert [x[1] for x in r] == [x[0] for x in solo1]
    assert list(eng.generate([[1, 2, 3]], 0)) == []


def test_oracle_rows_and_verify_equal_sequential(tiny):
    _, eng = tiny
    torch.manual_seed(5)
    seqs = [torch.randint(0, 300, (L,)).tolist() for L in (11, 17)]
    W = 4
    # per-sequence reference: prefill, then teacher-forced decode of W tokens
    drafts = torch.randint(0, 300, (2, W))
    seq_logits = []
    for b, s in enumerate(seqs):
        st = eng.new_state(1, 128)
        eng.prefill(st, torch.tensor([s]))
        for j in range(W):
            _, lg = eng.forward(st, drafts[b, j:j + 1], 1, torch.tensor([len(s) + j]),
                                return_logits=True)
            seq_logits.append(lg[0])
    # verify-shaped forward over both sequences at their own start positions
    st = eng.new_state(2, 128)
    for b, s in enumerate(seqs):
        sub = eng.new_state(1, 128)
        sub.kc = [k[b:b + 1] for k in st.kc]
        sub.vc = [v[b:b + 1] for v in st.vc]
        eng.prefill(sub, torch.tensor([s]))
    lv = eng.verify_logits(st, drafts, torch.tensor([len(s) for s in seqs]))
    assert torch.allclose(lv, torch.stack(seq_logits), atol=1e-5)
    # per-row decode step == per-sequence decode step (fresh caches)
    st2 = eng.new_state(2, 128)
    firsts = []
    for b, s in enumerate(seqs):
        sub = eng.new_state(1, 128)
        sub.kc = [k[b:b + 1] for k in st2.kc]
        sub.vc = [v[b:b + 1] for v in st2.vc]
        eng.prefill(sub, torch.tensor([s]))
        firsts.append(int(sub.tok[0]))
    _, lr = eng.forward_rows(st2, torch.tensor(firsts), torch.tensor([len(s) for s in seqs]),
                             return_logits=True)
    for b, s in enumerate(seqs):
        st1 = eng.new_state(1, 128)
        eng.prefill(st1, torch.tensor([s]))
        _, l1 = eng.forward(st1, st1.tok, 1, torch.tensor([len(s)]), return_logits=True)
        assert torch.allclose(lr[b], l1[0], atol=1e-5)
