"""GPU parity of the in-graph speculative decoding (dd_spec_seed / dd_spec_draft /
dd_spec_accept around the verify-shaped step) against the CPU restatement (oracle/spec.py).

* kernels: table seeding, drafting and acceptance bit for bit against the oracle's functions
  on random tables, planted accepted prefixes and repeated tokens (T, rows, positions,
  confirmed tokens, the per-step record);
* engine: speculative generation on a model the one-launch step takes, every emitted token
  checked by teacher-forcing the CPU oracle (its argmax, or a near-tie within 2 bf16 ulps);
  graph replays equal eager steps; a table seeded with the true continuation is accepted.
"""
import pytest
import torch

from dryft_amd import synth
from gpu_checks import teacher_forced_check
from oracle.reference import OracleEngine
from oracle.spec import accept, draft, seed_table

pytestmark = pytest.mark.gpu


def _lib():
    from dryft_amd._lib import lib
    return lib()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _table_dict(row):
    return {i: int(v) for i, v in enumerate(row.tolist()) if v != 0}


def test_seed_kernel_matches_oracle(cuda):
    L = _lib()
    g = torch.Generator().manual_seed(1)
    V = 300
    lens = [1, 9, 40, 3]
    prompts = [torch.randint(0, 12, (n,), generator=g).tolist() for n in lens]   # many repeats
    first = torch.randint(0, V, (len(lens),), generator=g)
    starts = [0]
    for n in lens:
        starts.append(starts[-1] + n)
    T = torch.zeros(len(lens), V, dtype=torch.int32, device="cuda")
    ids = torch.tensor([t for p in prompts for t in p], dtype=torch.long, device="cuda")
    ss = torch.tensor(starts, dtype=torch.int32, device="cuda")
    fg = first.cuda()
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    assert L.dd_spec_seed(T.data_ptr(), V, ids.data_ptr(), ss.data_ptr(), len(lens), fg.data_ptr(),
                          err.data_ptr(), _stream()) == 0
    Tc = T.cpu()
    for b, p in enumerate(prompts):
        want = seed_table(p, int(first[b]))
        got = {i: int(v) for i, v in enumerate(Tc[b].tolist()) if i in want or v != 0}
        assert got == want, b
    assert err.item() == 0


@pytest.mark.parametrize("B,W", [(1, 2), (3, 4), (8, 5), (16, 3)])
def test_draft_accept_kernels_match_oracle(cuda, B, W):
    L = _lib()
    V = 64                                    # small vocabulary: repeated tokens in rows
    g = torch.Generator().manual_seed(B * 10 + W)
    T = torch.randint(0, V, (B, V), generator=g, dtype=torch.int32)
    tok = torch.randint(0, V, (B,), generator=g)
    gpos = torch.randint(0, 500, (B,), generator=g)
    limit = gpos + torch.randint(0, 6, (B,), generator=g)
    Td, tokd, gposd, limd = T.cuda(), tok.cuda(), gpos.cuda(), limit.cuda()
    rows = torch.zeros(B * W, dtype=torch.long, device="cuda")
    pos = torch.zeros(B, dtype=torch.long, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    err_fill = torch.tensor([0x40], dtype=torch.int32, device="cuda")     # copied into rec
    assert L.dd_spec_draft(Td.data_ptr(), V, tokd.data_ptr(), gposd.data_ptr(), B, W, rows.data_ptr(),
                           pos.data_ptr(), err.data_ptr(), _stream()) == 0
    tabs = [_table_dict(T[b]) for b in range(B)]
    want_rows = [draft(tabs[b], int(tok[b]), W) for b in range(B)]
    assert rows.view(B, W).cpu().tolist() == want_rows
    assert torch.equal(pos.cpu(), gpos)
    # verify outputs with a planted accepted prefix of length a_b (then a mismatch)
    out = torch.randint(0, V, (B, W), generator=g)
    for b in range(B):
        a = b % W
        for j in range(a):
            out[b, j] = want_rows[b][j + 1]
        if a < W - 1 and out[b, a] == want_rows[b][a + 1]:
            out[b, a] = (out[b, a] + 1) % V
    outd = out.reshape(-1).cuda()
    rec = torch.zeros(B * W + B + 1, dtype=torch.long, device="cuda")
    assert L.dd_spec_accept(rows.data_ptr(), outd.data_ptr(), Td.data_ptr(), V, B, W,
                            tokd.data_ptr(), gposd.data_ptr(), limd.data_ptr(), rec.data_ptr(),
                            err_fill.data_ptr(), _stream()) == 0
    recc = rec.cpu().tolist()
    for b in range(B):
        a, t, gp = accept(tabs[b], want_rows[b], out[b].tolist(), int(gpos[b]), int(limit[b]))
        assert a == b % W
        assert recc[B * W + b] == a
        assert int(tokd[b]) == t and int(gposd[b]) == gp
        got_tab = {i: int(v) for i, v in enumerate(Td[b].cpu().tolist()) if v != 0 or i in tabs[b]}
        assert got_tab == {k: v for k, v in tabs[b].items()}
    assert recc[:B * W] == out.reshape(-1).tolist()
    assert recc[-1] == 0x40
    assert err.item() == 0


SMALL = synth.qwen3_config(vocab_size=1024, hidden_size=1024, intermediate_size=512,
                           num_hidden_layers=3, num_attention_heads=4, num_key_value_heads=1,
                           head_dim=128)


@pytest.fixture(scope="module")
def small(cuda):
    from dryft_amd.engine import Engine
    w = synth.random_weights(SMALL, seed=0)
    ref = OracleEngine.from_state_dict(SMALL, dict(w))
    eng = Engine.from_state_dict(SMALL, {k: v.cuda() for k, v in w.items()})
    assert eng.step is not None
    return ref, eng


@pytest.mark.parametrize("B,W", [(1, 4), (2, 4), (3, 2), (4, 4)])
def test_verify_row0_is_the_decode_step(small, B, W):
    """A verify step of the 16-row instantiation (B W <= 16, W G <= 16) partitions and reduces
    like the decode step at the same positions, so its row 0 of every sequence gives the decode
    step's logits and K/V bit for bit (what makes speculation token-identical to plain decoding).
    Prompt lengths put positions on, just before and just past 32-key block boundaries."""
    ref, eng = small
    g = torch.Generator().manual_seed(100 * B + W)
    lens = [29, 32, 61, 95][:B]
    prompts = [torch.randint(0, 1024, (n,), generator=g).tolist() for n in lens]
    cap = 256
    sd = eng._new_state(B, cap)
    eng._prefill(prompts, sd)
    first = sd.tok.clone()
    spos = sd.pos.clone()
    dec = eng.step.run(sd).clone()
    sv = eng._new_state(B, cap, W=W)
    eng._prefill(prompts, sv)
    drafts = torch.randint(0, 1024, (B, W), generator=g)
    drafts[:, 0] = first.cpu()
    ver = eng.verify_logits(sv, drafts.cuda(), spos).clone()
    torch.cuda.synchronize()
    assert int(sd.err.item()) == 0 and int(sv.err.item()) == 0
    for b in range(B):
        assert torch.equal(ver[b * W], dec[b]), b
        p = int(spos[b])
        for i in range(eng.L):
            assert torch.equal(sv.kc[i][b, :, p], sd.kc[i][b, :, p]), (b, i)
            assert torch.equal(sv.vc[i][b, :, p], sd.vc[i][b, :, p]), (b, i)


@pytest.mark.parametrize("W", [2, 4, 5])
def test_spec_generate_matches_oracle(small, W):
    ref, eng = small
    sp = eng.speculator(W)
    g = torch.Generator().manual_seed(W)
    prompts = [torch.randint(0, 1024, (n,), generator=g).tolist() for n in (5, 33, 70)]
    n = 40
    stats = {}
    got = list(sp.generate(prompts, n, stats=stats))
    assert len(got) == n and all(len(r) == 3 for r in got)
    flips = teacher_forced_check(ref, prompts, got)
    plain = list(eng.generate(prompts, n))
    print(f"W={W}: {stats['steps']} verify steps, {stats['accepted_drafts']} accepted drafts, "
          f"identical to plain decode: {got == plain}, near-tie flips {flips}")
    # eager steps give the graph's tokens
    eager = list(sp.generate(prompts, n, graph=False))
    assert eager == got


def test_spec_accepts_true_continuation(small):
    """Seed the table with plain decode's own continuation: the drafts are the model's greedy
    tokens, so steps accept drafts and the output still passes the oracle check."""
    ref, eng = small
    W = 4
    sp = eng.speculator(W)
    g = torch.Generator().manual_seed(7)
    prompts = [torch.randint(0, 1024, (n,), generator=g).tolist() for n in (12, 50)]
    n = 48
    plain = list(eng.generate(prompts, n))
    st, first = sp.prepare(prompts, n)
    for b in range(len(prompts)):
        seq = [plain[t][b] for t in range(n)]
        for t in range(n - 1):
            st.T[b, seq[t]] = seq[t + 1]
    stats = {}
    got = list(sp.run(st, first, n, stats))
    teacher_forced_check(ref, prompts, got)
    print(f"true-continuation table: {stats['steps']} steps for {n - 1} tokens per row, "
          f"{stats['accepted_drafts']} accepted drafts, identical to plain: {got == plain}")
    assert stats["accepted_drafts"] > 0
    assert stats["steps"] < n - 1
