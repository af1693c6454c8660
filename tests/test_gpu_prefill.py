"""GPU parity of the HIP prefill (dd_qkv_post_prefill, dd_attn_prefill through HipOps) against the
CPU oracle, on packed ragged batches.

* qkv_post (engine.py:166-181 prefill branch, per prompt): V cache rows are the raw projection bit
  for bit; K and q heads equal the oracle's arithmetic bit for bit up to the 1/rms freedom the
  decode checks allow (an fp32 sum of 128 squares added in another order: 1/rms moved by at most
  RMS_ULPS fp32 ulps); every cache slot outside [0, len_b) and every other row is untouched;
  last_only writes the same K/V and the last rows' q.
* attention (engine.py:148-152 / fused.py:301-343): within 0.02 of a float64 causal loop
  (test_attn.py:40 of the reference uses the same bound), packed batch == each prompt alone bit
  for bit, last_only == the last rows of the full output bit for bit, keys past a prompt's length
  (filled with noise here) never seen.
* engine: a ragged batch prefilled in one packed pass gives each prompt the oracle's logits
  (within the reference's 2.0 gate) and its argmax up to near-ties; cache slots past each
  prompt stay zero.
"""
import types

import pytest
import torch

from dryft_amd import synth
from gpu_checks import RMS_ULPS, _oracle_k_heads, near_tie
from oracle.reference import OracleEngine, TorchOps, fake_engine

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
HD = 128


def _hip(e_cpu):
    from dryft_amd.hipops import HipOps
    e = types.SimpleNamespace(**vars(e_cpu))
    e.dev = torch.device("cuda")
    e.cos, e.sin = e_cpu.cos.cuda(), e_cpu.sin.cuda()
    return HipOps(e)


def _starts(lens):
    s = [0]
    for n in lens:
        s.append(s[-1] + n)
    return s


def _heads_bits_ok(e, w, raw, got, ph):
    """Every head of got [n, hd] equals the oracle's norm(w) + rope at positions ph [n] of raw
    [n, hd], with 1/rms moved by at most RMS_ULPS ulps. Returns the fraction exact at 0 ulps."""
    lay = types.SimpleNamespace(kn=w)
    ok = torch.zeros(raw.shape[0], dtype=torch.bool)
    exact = 0
    for dr in [0] + [d for k in range(1, RMS_ULPS + 1) for d in (k, -k)]:
        want = _oracle_k_heads(e, lay, raw, ph, dr)
        hit = (want.view(torch.int16) == got.view(torch.int16)).all(-1)
        if dr == 0:
            exact = int(hit.sum())
        ok |= hit
        if ok.all():
            break
    bad = (~ok).nonzero().flatten().tolist()
    assert not bad, ("heads not matching", bad[:6])
    return exact / raw.shape[0]


QKV_CASES = [((1, 17, 100, 130), 32, 8), ((64,), 32, 8), ((5, 33, 16, 1, 250), 16, 2),
             ((40, 3), 8, 8)]


@pytest.mark.parametrize("lens,NH,NKV", QKV_CASES)
def test_qkv_post_prefill_packed(cuda, lens, NH, NKV):
    B, cap = len(lens), 256
    e = fake_engine(nh=NH, nkv=NKV, hd=HD, rope_len=cap)
    hip = _hip(e)
    starts = _starts(lens)
    T = starts[-1]
    g = torch.Generator().manual_seed(sum(lens) + NH)
    qkv = torch.randn(T, (NH + 2 * NKV) * HD, generator=g).to(BF)
    qn = (1 + 0.1 * torch.randn(HD, generator=g)).to(BF)
    kn = (1 + 0.1 * torch.randn(HD, generator=g)).to(BF)
    lg = types.SimpleNamespace(qn=qn.cuda(), kn=kn.cuda())
    kc0 = torch.randn(B, NKV, cap, HD, generator=g).to(BF)
    vc0 = torch.randn(B, NKV, cap, HD, generator=g).to(BF)
    ss = torch.tensor(starts, dtype=torch.int32).cuda()
    kc, vc = kc0.cuda(), vc0.cuda()
    q = hip.qkv_post_packed(qkv.cuda(), lg, kc, vc, ss, B, T).cpu()        # [T, NH, HD]
    assert hip.err.item() == 0
    kcc, vcc = kc.cpu(), vc.cpu()
    written = torch.zeros(B, cap, dtype=torch.bool)
    for b, n in enumerate(lens):
        written[b, :n] = True
    for c, c0 in ((kcc, kc0), (vcc, vc0)):
        assert torch.equal(c.permute(0, 2, 1, 3)[~written], c0.permute(0, 2, 1, 3)[~written])
    # per token: V bits, K and q heads against the oracle arithmetic
    bidx = torch.cat([torch.full((n,), b) for b, n in enumerate(lens)])
    pidx = torch.cat([torch.arange(n) for n in lens])
    raw_q = qkv[:, :NH * HD].reshape(T * NH, HD)
    raw_k = qkv[:, NH * HD:(NH + NKV) * HD].reshape(T * NKV, HD)
    raw_v = qkv[:, (NH + NKV) * HD:].reshape(T, NKV, HD)
    assert torch.equal(vcc[bidx, :, pidx].view(torch.int16), raw_v.view(torch.int16))
    k_got = kcc[bidx, :, pidx].reshape(T * NKV, HD)
    fk = _heads_bits_ok(e, kn, raw_k, k_got, pidx.repeat_interleave(NKV))
    fq = _heads_bits_ok(e, qn, raw_q, q.reshape(T * NH, HD), pidx.repeat_interleave(NH))
    # and the oracle's own qkv_post, prompt by prompt, within bf16 rounding
    tor = TorchOps(e)
    lc = types.SimpleNamespace(qn=qn, kn=kn)
    rk, rv = kc0.clone(), vc0.clone()
    for b, n in enumerate(lens):
        rq = tor.qkv_post(qkv[starts[b]:starts[b + 1]], lc, rk[b:b + 1], rv[b:b + 1], 1, n, None)
        d = (rq[0].transpose(0, 1).float() - q[starts[b]:starts[b + 1]].float()).abs().max().item()
        assert d <= 0.02, d
    assert torch.equal(vcc, rv)
    assert (kcc.float() - rk.float()).abs().max().item() <= 0.02
    # last_only: same K/V bits, q of each prompt's last token at row b
    kc2, vc2 = kc0.cuda(), vc0.cuda()
    ql = hip.qkv_post_packed(qkv.cuda(), lg, kc2, vc2, ss, B, T, last_only=True).cpu()
    assert torch.equal(kc2.cpu(), kcc) and torch.equal(vc2.cpu(), vcc)
    assert torch.equal(ql, q[torch.tensor(starts[1:]) - 1])
    print(f"lens={lens} G={NH // NKV}: K heads exact at 0 ulps {fk:.3f}, q heads {fq:.3f}")


def _attn_ref_fp64(q, kc, vc, lens, starts, nh, nkv):
    """Causal GQA attention per prompt in float64: token at position p of prompt b sees keys
    0..p of cache row b. q [T, nh, hd] -> [T, nh*hd]."""
    G = nh // nkv
    T = q.shape[0]
    out = torch.zeros(T, nh, HD, dtype=torch.float64)
    for b, n in enumerate(lens):
        qb = q[starts[b]:starts[b + 1]].double()                      # [n, nh, hd]
        mask = torch.ones(n, n, dtype=torch.bool).tril()
        for h in range(nh):
            K = kc[b, h // G, :n].double()
            V = vc[b, h // G, :n].double()
            s = (qb[:, h] @ K.T) * HD ** -0.5
            s = s.masked_fill(~mask, float("-inf"))
            out[starts[b]:starts[b + 1], h] = torch.softmax(s, -1) @ V
    return out.reshape(T, nh * HD)


ATTN_CASES = [((1, 17, 100, 130), 32, 8, 256), ((2048,), 32, 8, 2048), ((5, 33, 16, 1, 250), 16, 2, 256),
              ((40, 3, 77), 8, 8, 128), ((31, 32, 33), 64, 8, 128), ((63, 64, 65, 129), 16, 8, 256),
              ((1, 2, 300), 32, 8, 384)]


@pytest.mark.parametrize("lens,NH,NKV,cap", ATTN_CASES)
def test_attn_prefill_packed(cuda, lens, NH, NKV, cap):
    B = len(lens)
    hip = _hip(fake_engine(nh=NH, nkv=NKV, hd=HD))
    starts = _starts(lens)
    T = starts[-1]
    g = torch.Generator().manual_seed(T * 7 + NH)
    q = torch.randn(T, NH, HD, generator=g).to(BF)
    kc = torch.randn(B, NKV, cap, HD, generator=g).to(BF)       # noise past each prompt's length
    vc = torch.randn(B, NKV, cap, HD, generator=g).to(BF)
    ss = torch.tensor(starts, dtype=torch.int32).cuda()
    qg, kg, vg = q.cuda(), kc.cuda(), vc.cuda()
    out = hip.attn_prefill_packed(qg, kg, vg, ss, B, T)
    ref = _attn_ref_fp64(q, kc, vc, lens, starts, NH, NKV)
    d = (out.double().cpu() - ref).abs().max().item()
    assert d < 0.02, d
    # each prompt alone gives the same bits
    for b, n in enumerate(lens):
        one = torch.tensor([0, n], dtype=torch.int32).cuda()
        ob = hip.attn_prefill_packed(qg[starts[b]:starts[b + 1]].contiguous(), kg[b:b + 1],
                                     vg[b:b + 1], one, 1, n)
        assert torch.equal(ob, out[starts[b]:starts[b + 1]]), b
    # last_only: q rows of the last tokens, output rows = the full output's last rows
    last = torch.tensor(starts[1:]) - 1
    ol = hip.attn_prefill_packed(qg[last.cuda()].contiguous(), kg, vg, ss, B, T, last_only=True)
    assert torch.equal(ol, out[last.cuda()])
    print(f"lens={lens} G={NH // NKV}: max|out - fp64| {d:.3g}")


def test_attn_prefill_dma_equals_register_staging(cuda):
    """G = 4 runs the LDS-DMA kernel when the cache capacity is a multiple of 32 and the
    register-staged kernel otherwise; both compute the same arithmetic, so the same prompts in a
    cache of 256 and of 264 slots give identical bits (and the fp64 bound holds for both)."""
    lens, NH, NKV = (1, 31, 32, 33, 200, 256), 32, 8
    B = len(lens)
    hip = _hip(fake_engine(nh=NH, nkv=NKV, hd=HD))
    starts = _starts(lens)
    T = starts[-1]
    g = torch.Generator().manual_seed(11)
    q = torch.randn(T, NH, HD, generator=g).to(BF)
    kc = torch.randn(B, NKV, 256, HD, generator=g).to(BF)
    vc = torch.randn(B, NKV, 256, HD, generator=g).to(BF)
    kc2 = torch.cat([kc, torch.randn(B, NKV, 8, HD, generator=g).to(BF)], dim=2)
    vc2 = torch.cat([vc, torch.randn(B, NKV, 8, HD, generator=g).to(BF)], dim=2)
    ss = torch.tensor(starts, dtype=torch.int32).cuda()
    qg = q.cuda()
    dma = hip.attn_prefill_packed(qg, kc.cuda(), vc.cuda(), ss, B, T)
    reg = hip.attn_prefill_packed(qg, kc2.cuda(), vc2.cuda(), ss, B, T)
    assert torch.equal(dma, reg)
    ref = _attn_ref_fp64(q, kc, vc, lens, starts, NH, NKV)
    assert (dma.double().cpu() - ref).abs().max().item() < 0.02
    last = torch.tensor(starts[1:]) - 1
    for k, v in ((kc, vc), (kc2, vc2)):
        ol = hip.attn_prefill_packed(qg[last].contiguous(), k.cuda(), v.cuda(), ss, B, T, last_only=True)
        assert torch.equal(ol, dma[last.cuda()])


def test_attn_prefill_through_reference_interface(cuda):
    """HipOps.qkv_post(pos=None) + attn_prefill (the reference's ops interface, B prompts of one
    length S) against the oracle's TorchOps on the same qkv."""
    NH, NKV, B, S, cap = 32, 8, 3, 70, 128
    e = fake_engine(nh=NH, nkv=NKV, hd=HD, rope_len=cap)
    hip, tor = _hip(e), TorchOps(e)
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(B * S, (NH + 2 * NKV) * HD, generator=g).to(BF)
    lc = types.SimpleNamespace(qn=(1 + 0.1 * torch.randn(HD, generator=g)).to(BF),
                               kn=(1 + 0.1 * torch.randn(HD, generator=g)).to(BF))
    lg = types.SimpleNamespace(qn=lc.qn.cuda(), kn=lc.kn.cuda())
    for last in (False, True):
        kc = torch.zeros(B, NKV, cap, HD, dtype=BF)
        vc = torch.zeros_like(kc)
        kg, vg = kc.cuda(), vc.cuda()
        q = hip.qkv_post(qkv.cuda(), lg, kg, vg, B, S, None, last_query_only=last)
        assert q.shape == (B, NH, 1 if last else S, HD)
        o = hip.attn_prefill(q, kg, vg, S, last_query_only=last).cpu()
        rq = tor.qkv_post(qkv, lc, kc, vc, B, S, None, last_query_only=last)
        ro = tor.attn_prefill(rq, kc, vc, S, last_query_only=last)
        assert o.shape == ro.shape
        d = (o.float() - ro.float()).abs().max().item()
        assert d <= 0.02, (last, d)
        assert torch.equal(vg.cpu(), vc)


TINY = synth.qwen3_config(vocab_size=512, hidden_size=256, intermediate_size=192,
                          num_hidden_layers=3, num_attention_heads=8, num_key_value_heads=2,
                          head_dim=128)


def test_engine_packed_prefill_matches_oracle(cuda):
    """Ragged prompts in one packed pass: per prompt the oracle's logits within 2.0 and its
    argmax up to near-ties; positions set to the lengths; cache slots past each prompt zero."""
    from dryft_amd.engine import Engine
    w = synth.random_weights(TINY, seed=3)
    ref = OracleEngine.from_state_dict(TINY, dict(w))
    eng = Engine.from_state_dict(TINY, {k: v.cuda() for k, v in w.items()})
    assert hasattr(eng.ops, "qkv_post_packed")                 # the HIP packed prefill runs
    g = torch.Generator().manual_seed(11)
    lens = [1, 19, 130, 64, 7]
    prompts = [torch.randint(0, TINY["vocab_size"], (n,), generator=g).tolist() for n in lens]
    st = eng._new_state(len(lens), 256)
    eng._dbg = []
    eng._prefill(prompts, st)
    logits = eng._dbg[-1]
    eng._dbg = None
    assert st.pos.tolist() == lens
    for i in range(eng.L):
        for c in (st.kc[i], st.vc[i]):
            for b, n in enumerate(lens):
                assert not c[b, :, n:].any()
    for b, p in enumerate(prompts):
        rs = ref.new_state(1, 256)
        ref._dbg = []
        ref.prefill(rs, torch.tensor([p]))
        rl = ref._dbg[-1][0]
        ref._dbg = None
        d = (logits[b] - rl).abs().max().item()
        assert d <= 2.0, (b, d)
        tok = int(st.tok[b])
        gap, tie = near_tie(rl, tok, d)
        assert tok == int(rl.argmax()) or tie, (b, tok, int(rl.argmax()), gap)
        print(f"prompt {b} len {lens[b]}: max|logit diff| {d:.4f}")
