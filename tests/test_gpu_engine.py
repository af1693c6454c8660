"""End-to-end parity of the HIP decode engine against the CPU oracle on seeded random-init
Qwen3-shape models: greedy tokens, per-step logits (within 2.0, the reference's gate,
tests/bench.py:159-166), ragged batches vs per-sequence decoding, the verify-shaped multi-query
forward vs sequential decode, graph replay vs eager, and the self-test ladder
(test_selftest_fallback.py).

Greedy tokens are checked by teacher forcing: the oracle is re-run on the engine's own tokens
and every emitted token must be the oracle's argmax, or within 2 bf16 ulps of the oracle's max
logit (a near-tie, where one ulp of reduction-order difference legitimately flips argmax; small
random models have many). Strict identity with the oracle's free-running generation and the
first divergence step are reported as well.
"""
import math

import pytest
import torch

from dryft_amd import synth
from gpu_checks import near_tie, teacher_forced_check
from oracle.reference import OracleEngine

pytestmark = pytest.mark.gpu

# TINY is below the one-launch step's size class (I % 256 != 0): its states decode with the
# per-op HIP kernels. SMALL is the smallest geometry the one-launch step takes: its states decode
# with dd_decode_step, the bench's path. The engine-level tests run on both.
TINY = synth.qwen3_config(vocab_size=512, hidden_size=256, intermediate_size=192,
                          num_hidden_layers=3, num_attention_heads=8, num_key_value_heads=2,
                          head_dim=128)
SMALL = synth.qwen3_config(vocab_size=1024, hidden_size=1024, intermediate_size=512,
                           num_hidden_layers=3, num_attention_heads=4, num_key_value_heads=1,
                           head_dim=128)
MODELS = {"tiny-per-op": TINY, "small-fused": SMALL}


@pytest.fixture(scope="module", params=list(MODELS))
def tiny(cuda, request):
    """(oracle, engine) of one test model; the engine decodes with the path its name says."""
    from dryft_amd.engine import Engine
    cfg = MODELS[request.param]
    w = synth.random_weights(cfg, seed=0)
    ref = OracleEngine.from_state_dict(cfg, dict(w))
    eng = Engine.from_state_dict(cfg, {k: v.cuda() for k, v in w.items()})
    assert (eng.step is not None) == (request.param == "small-fused")
    return ref, eng


def first_divergence(a, b):
    for t, (x, y) in enumerate(zip(a, b)):
        if x != y:
            return t
    return None


def bf16_ulp(x):
    return 2.0 ** (math.floor(math.log2(max(abs(x), 2.0 ** -126))) - 7)


# (1, 120, 8) and (4, 100, 28) fill the 128-slot cache exactly: the last decode steps run at the
# cache's end, where the attention's key count (pos + max(W, 4)) is clamped to the capacity
@pytest.mark.parametrize("B,S,n", [(1, 20, 12), (3, 37, 9), (2, 130, 5), (16, 64, 8), (1, 120, 8),
                                   (4, 100, 28)])
def test_generate_matches_oracle(tiny, B, S, n):
    ref, eng = tiny
    g = torch.Generator().manual_seed(B * 1000 + S)
    ids = torch.randint(0, eng.cfg["vocab_size"], (B, S), generator=g).tolist()
    got = list(eng.generate(ids, n))
    assert len(got) == n and all(len(x) == B for x in got)
    flips = teacher_forced_check(ref, ids, got)
    want = list(ref.generate(ids, n))
    print(f"B={B} S={S} n={n}: identical={got == want} first divergence="
          f"{first_divergence(got, want)} near-tie flips={flips}")


def test_ragged_matches_per_sequence(tiny):
    ref, eng = tiny
    seqs = [[1, 2, 3], [4, 5, 6, 7], [8, 9, 10], [11, 12, 13, 14, 15]]
    n = 6
    got = list(eng.generate(seqs, n))
    teacher_forced_check(ref, seqs, got)      # reference semantics: each sequence on its own
    solo = [list(eng.generate([s], n)) for s in seqs]
    for b in range(len(seqs)):
        teacher_forced_check(ref, [seqs[b]], solo[b])


def test_state_reuse_single_token_and_empty(tiny):
    _, eng = tiny
    ids = torch.randint(0, 512, (3, 37), generator=torch.Generator().manual_seed(7)).tolist()
    a = list(eng.generate(ids, 9))
    b = list(eng.generate(ids, 9))
    assert a == b
    assert list(eng.generate([[1, 2, 3]], 0)) == []
    one = list(eng.generate([[1, 2, 3, 4, 5, 6]], 1))
    assert len(one) == 1
    cap = 128
    assert eng.states[(1, cap, 1, False)].graph is None      # n=1 captures no graph


def test_generate_raises_on_error_flag(tiny):
    """A step whose kernels flag an error (here: a row's position pushed to the cache capacity,
    flag 2) makes generate() raise instead of yielding tokens computed from it; the fused step
    and the per-op path both report through the state's error word."""
    _, eng = tiny
    prefill = eng._prefill

    def past_cache(ids, st):
        prefill(ids, st)
        st.pos.fill_(st.cap - 1)             # step 1 writes slot cap - 1, step 2 is past the cache
    eng._prefill = past_cache
    try:
        out = []
        with pytest.raises(RuntimeError, match="error flags 0x2"):
            for step in eng.generate([[1, 2, 3]], 5):
                out.append(step)
        assert len(out) == 2                  # the prefill token and step 1
    finally:
        del eng._prefill
    assert list(eng.generate([[1, 2, 3]], 3))  # the flag is cleared by the next generate


def test_verify_selftest_gate(tiny):
    """The load-time verify check of speculation (engine.py:549-627): the verify-shaped forward
    against step-by-step decode, B=1 W=5 and B=4 W=4 at distinct per-row positions, within the
    reference's 0.5 gate."""
    _, eng = tiny
    if eng.step is None:
        pytest.skip("per-op path: the verify check runs on the one-launch step")
    d1, d2 = eng._selftest_verify(4)
    print(f"verify selftest: B=1 W=5 {d1:.4f}, B=4 W=4 distinct positions {d2:.4f}")
    assert d1 <= 0.5 and d2 <= 0.5


@torch.inference_mode()
def test_counters_recovered_after_barrier_timeout(tiny):
    """Recovery from a grid-barrier timeout of the one-launch step (error flag 4), forced from
    the host so no kernel waits: the counters are poisoned the way a timed-out launch can leave
    them (attention-combine, argmax and split-down counts nonzero) and the state's error word
    carries flag 4; the next generate() must zero the counters first and produce the same
    tokens as a clean run, leaving every counter zero."""
    _, eng = tiny
    if eng.step is None:
        pytest.skip("per-op path: no one-launch step counters")
    ids = torch.randint(0, 1024, (3, 40), generator=torch.Generator().manual_seed(17)).tolist()
    want = list(eng.generate(ids, 6))
    st = eng.states[(3, 128, 1, True)]
    n = eng.step.L.dd_step_counters()
    poison = [0] * n
    for i in range(1024, n):                 # hand-off counters (not the barrier counters)
        poison[i] = 1 + i % 3
    eng.step.write_counters(st, poison)
    st.err.fill_(4)                          # what the timed-out launch reported
    got = list(eng.generate(ids, 6))
    assert got == want
    assert eng.step.counters(st) == [0] * n
    assert eng.error_flags() == 0


@torch.inference_mode()
def test_graph_replay_equals_eager(tiny):
    """The captured step must reproduce eager steps bit for bit (replayed several times, with
    eager work and syncs in between)."""
    _, eng = tiny
    ids = torch.randint(0, 512, (4, 50), generator=torch.Generator().manual_seed(9)).tolist()
    st = eng._state(4, 256, graph=True)
    eng._prefill(ids, st)
    snap = (st.tok.clone(), st.pos.clone(), [k.clone() for k in st.kc], [v.clone() for v in st.vc])
    graph_toks = []
    for _ in range(5):
        st.graph.replay()
        torch.cuda.synchronize()
        graph_toks.append(st.tok.clone())
    st.tok.copy_(snap[0]); st.pos.copy_(snap[1])
    for i in range(eng.L):
        st.kc[i].copy_(snap[2][i]); st.vc[i].copy_(snap[3][i])
    eager_toks = []
    for _ in range(5):
        eng._decode_body(st)
        torch.cuda.synchronize()
        eager_toks.append(st.tok.clone())
    for a, b in zip(graph_toks, eager_toks):
        assert torch.equal(a, b)


@torch.inference_mode()
def test_verify_shape_matches_sequential(tiny):
    """Verify-shaped forward (W=5 tokens per row at per-row start positions) vs the oracle's W
    sequential single-token decodes (engine.py:549-627 equivalence)."""
    ref, eng = tiny
    torch.manual_seed(11)
    B, W = 4, 5
    seqs = [torch.randint(0, 512, (L,)).tolist() for L in (30, 41, 17, 64)]
    drafts = torch.randint(0, 512, (B, W))
    spos = torch.tensor([len(s) for s in seqs])
    st = eng._new_state(B, 256, W=W)
    eng._prefill(seqs, st)
    got = eng.verify_logits(st, drafts.cuda(), spos.cuda()).float().cpu()
    rst = ref.new_state(B, 256)
    for b, s in enumerate(seqs):
        sub = ref.new_state(1, 256)
        sub.kc = [k[b:b + 1] for k in rst.kc]
        sub.vc = [v[b:b + 1] for v in rst.vc]
        ref.prefill(sub, torch.tensor([s]))
    want = ref.verify_logits(rst, drafts, spos).float()
    d = (got - want).abs().max().item()
    assert d <= 0.5, d                         # the reference's verify selftest gate (engine.py:579)
    for r in range(B * W):                     # argmax equal up to near-ties
        gap, tie = near_tie(want[r], int(got[r].argmax()), (got[r] - want[r]).abs().max().item())
        assert gap == 0 or tie, (r, gap)
    # K/V written at spos[b] + s, nothing past spos[b] + W. Layer 0 projects the draft tokens'
    # embedding rows (identical inputs: the per-kernel bar); deeper layers carry the earlier
    # layers' rounding differences (and the two prefills'), held to a sanity bound.
    for i in range(eng.L):
        for b in range(B):
            sl = slice(int(spos[b]), int(spos[b]) + W)
            for c, rc in ((st.kc[i], rst.kc[i]), (st.vc[i], rst.vc[i])):
                got_kv, want_kv = c[b, :, sl].float().cpu(), rc[b, :, sl].float()
                tol = 2e-2 if i == 0 else 0.5
                assert ((got_kv - want_kv).abs() <= tol + 2e-2 * want_kv.abs()).all(), (i, b)
                assert not c[b, :, int(spos[b]) + W:].any()


def test_qwen3_width_decode_logits(cuda):
    """Full Qwen3-4B widths (2 layers, reduced vocab): per-step logits within 2.0, and greedy
    tokens equal to the oracle's argmax wherever the oracle has no near-tie (teacher forced)."""
    from dryft_amd.engine import Engine
    cfg = synth.qwen3_config(num_hidden_layers=2, vocab_size=8192)
    w = synth.random_weights(cfg, seed=1)
    ref = OracleEngine.from_state_dict(cfg, dict(w))
    eng = Engine.from_state_dict(cfg, {k: v.cuda() for k, v in w.items()}, selftest=False)
    ids = torch.randint(0, 8192, (4, 96), generator=torch.Generator().manual_seed(3)).tolist()
    n = 6
    got = list(eng.generate(ids, n))
    flips = teacher_forced_check(ref, ids, got)
    want = list(ref.generate(ids, n))
    print(f"identical={got == want} first divergence={first_divergence(got, want)} flips={flips}")
    # teacher-forced eager decode steps: logits of every step within 2.0 of the oracle's
    st = eng._new_state(4, 256)
    eng._prefill(ids, st)
    rst = ref.new_state(4, 256)
    ref.prefill(rst, torch.tensor(ids))
    worst = 0.0
    for t in range(n - 1):
        forced = torch.tensor([x for x in want[t]])
        st.tok.copy_(forced.cuda())
        lg = eng._forward(st, st.tok, 1, st.pos).float().cpu()
        eng.ops.argmax_(lg.cuda().to(torch.bfloat16), st.tok, st.pos)
        _, rl = ref.forward(rst, forced, 1, torch.tensor([96 + t]), return_logits=True)
        worst = max(worst, (lg - rl.float()).abs().max().item())
    print(f"worst per-step logit diff over {n - 1} steps: {worst:.4f}")
    assert worst <= 2.0


def test_selftest_falls_back_without_gemv(cuda):
    """test_selftest_fallback.py:24-43: a GEMV that returns NaN at decode M=2 on layer 0's wqkv
    makes the engine keep the HIP ops with use_gemv=False."""
    from dryft_amd import hipops
    from dryft_amd.engine import Engine
    w = synth.random_weights(TINY, seed=2)
    orig = hipops.HipOps.linear

    def bad(self, x, wt):
        out = orig(self, x, wt)
        if self.use_gemv and x.shape[0] == 2 and wt is self.e.layers[0].wqkv:
            return torch.full_like(out, float("nan"))
        return out
    hipops.HipOps.linear = bad
    try:
        eng = Engine.from_state_dict(TINY, {k: v.cuda() for k, v in w.items()})
    finally:
        hipops.HipOps.linear = orig
    assert isinstance(eng.ops, hipops.HipOps)
    assert not eng.ops.use_gemv
