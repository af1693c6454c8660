"""Teacher-forced correctness gate for generated tokens (the reference bench's check).

The reference benchmark accepts a generation only if, for every emitted token, an independent
implementation run over the prompt plus the tokens emitted before it puts that token within 2.0
logits of its own maximum (tests/bench.py:155-167 of the reference: HF transformers with SDPA,
``logits_to_keep=n``). Here the independent implementation is the reference's torch arithmetic
(``TorchOps``: ``F.linear`` on hipBLASLt, torch RMSNorm / RoPE, ``F.scaled_dot_product_attention``)
on the GPU, over the whole sequence at once like the reference's prefill (engine.py:459-503 with
every position kept), one sequence at a time. It shares no kernel with the HIP decode path.
"""
import torch

from .hipops import TorchOps

GAP_TOL = 2.0                  # reference tests/bench.py:162


class _Cache:
    pass


@torch.inference_mode()
def teacher_forced_logits(eng, ids, n):
    """Logits [n, V] (fp32) at the last n positions of the token sequence ``ids`` (list of
    int): row j predicts token len(ids) - n + j + 1."""
    ops = TorchOps(eng)
    S = len(ids)
    cap = -(-S // 128) * 128
    shape = (1, eng.nkv, cap, eng.hd)
    tokens = torch.tensor(ids, dtype=torch.long, device=eng.dev)
    h = eng.embed[tokens]
    a = ops.rms(h, eng.layers[0].ln1)
    last = eng.L - 1
    for i, l in enumerate(eng.layers):
        kc = torch.zeros(shape, dtype=eng.dtype, device=eng.dev)
        vc = torch.zeros(shape, dtype=eng.dtype, device=eng.dev)
        qkv = ops.linear(a, l.wqkv)
        q = ops.qkv_post(qkv, l, kc, vc, 1, S, None)
        o = ops.attn_prefill(q, kc, vc, S)
        h, a = ops.linear_add_norm(o, l.wo, h, l.ln2)
        m = ops.gate_up_silu(a, l.wgu)
        h, a = ops.linear_add_norm(m, l.wd, h, eng.layers[i + 1].ln1 if i < last else eng.norm)
    return ops.linear(a[S - n:], eng.lm_head).float()


@torch.inference_mode()
def gap_check(eng, prompts, steps, tol=GAP_TOL):
    """``steps``: [n][B] tokens emitted after ``prompts`` (steps[0] is the prefill's token).
    Returns (worst gap, number of tokens whose gap exceeds ``tol``, tokens checked); the gap of
    a token is the independent path's max logit minus its logit for that token."""
    n = len(steps)
    toks = torch.tensor(steps, dtype=torch.long).T            # [B, n]
    worst, bad = 0.0, 0
    for b, p in enumerate(prompts):
        seq = list(p) + toks[b, :-1].tolist()
        lg = teacher_forced_logits(eng, seq, n)                # row j predicts steps[j][b]
        t = toks[b].to(lg.device)
        if not torch.isfinite(lg).all():
            return float("inf"), n * len(prompts), n * len(prompts)
        gap = lg.max(-1).values - lg.gather(-1, t[:, None])[:, 0]
        worst = max(worst, gap.max().item())
        bad += int((gap > tol).sum())
    return worst, bad, n * len(prompts)


def _bf16_ulp(x):
    import math
    return 2.0 ** (math.floor(math.log2(max(abs(x), 2.0 ** -126))) - 7)


@torch.inference_mode()
def decode_trace(eng, prompts, n):
    """Greedy decode of ``prompts`` for n tokens through the engine's captured step (the
    product path), keeping every step's logits: returns (tokens [n][B], logits [n, B, V] bf16 on
    the device; row t holds the logits that chose tokens[t], row 0 the prefill's)."""
    B = len(prompts)
    S = max(len(p) for p in prompts)
    cap = -(-(S + n) // 128) * 128
    st = eng._state(B, cap, graph=n > 1)
    assert st.fused is not None, "decode_trace follows the one-launch decode step"
    st.err.zero_()
    V = eng.embed.shape[0]
    logits = torch.empty((n, B, V), dtype=torch.bfloat16, device=eng.dev)
    eng._dbg = []
    try:
        eng._prefill(prompts, st)
        logits[0].copy_(eng._dbg[-1].to(eng.dev, torch.bfloat16))
    finally:
        eng._dbg = None
    hist = torch.empty((n, B), dtype=torch.long, device=eng.dev)
    hist[0].copy_(st.tok[:B])
    for t in range(1, n):
        if st.graph is not None:
            st.graph.replay()
        else:
            eng._decode_body(st)
        hist[t].copy_(st.tok[:B])
        logits[t].copy_(st.fused.logits[:B])
    torch.cuda.synchronize()
    assert int(st.err.item()) == 0
    return hist.cpu().tolist(), logits


@torch.inference_mode()
def token_identity(eng, prompt, toks, logits=None):
    """Greedy token identity of one sequence's emitted tokens ``toks`` (list, toks[0] the
    prefill's) against the reference's torch arithmetic teacher-forced on prompt + toks: a flip
    is a token that is not that path's argmax. With the engine's own logits [n, V] (row t chose
    toks[t]) each step's noise is max |engine - torch| over the vocabulary, and a flip is a
    near-tie when the token's torch logit is below the torch maximum by no more than the larger
    of 2 bf16 ulps and that noise (the two paths add in different orders, so candidates closer
    than their disagreement may legitimately swap). Returns a dict: tokens, flips,
    first_flip (the first step where the engine leaves the torch path's own greedy run, or
    None), flip_detail [[step, gap, noise], ...], all_near_ties, worst_logit_diff."""
    n = len(toks)
    T = teacher_forced_logits(eng, list(prompt) + list(toks[:-1]), n)      # row t predicts toks[t]
    t_ = torch.tensor(toks, device=T.device)
    mx = T.max(-1).values
    gap = (mx - T.gather(-1, t_[:, None])[:, 0]).cpu().tolist()
    arg = T.argmax(-1).cpu().tolist()
    noise = None
    if logits is not None:
        noise = (logits.float() - T).abs().max(-1).values.cpu().tolist()
    mxl = mx.cpu().tolist()
    detail, all_near = [], True
    for t in range(n):
        if toks[t] != arg[t]:
            nz = noise[t] if noise is not None else 0.0
            near = gap[t] <= max(2 * _bf16_ulp(mxl[t]), nz)
            all_near = all_near and near
            detail.append([t, round(gap[t], 5), round(nz, 5) if noise is not None else None])
    return {"tokens": n, "flips": len(detail),
            "first_flip": detail[0][0] if detail else None,
            "flip_detail": detail[:32], "all_near_ties": all_near if noise is not None else None,
            "worst_logit_diff": round(max(noise), 5) if noise is not None else None}


@torch.inference_mode()
def first_divergence_check(eng, prompt, plain, plain_logits, other):
    """Where two emitted streams of one sequence part (``plain`` from the engine's decode step
    with its logits, ``other`` e.g. the speculative path's): the first step t with
    plain[t] != other[t], and whether both tokens there are acceptable greedy choices within the
    measured noise: the torch path teacher-forced on the common prefix, each token's logit below
    that path's maximum by no more than max(2 bf16 ulps, max |engine logits - torch logits| at
    that step). Returns None when the streams are identical, else a dict."""
    t = next((i for i, (a, b) in enumerate(zip(plain, other)) if a != b), None)
    if t is None:
        return None
    T = teacher_forced_logits(eng, list(prompt) + list(plain[:t]), 1)[0]
    noise = (plain_logits[t].float() - T).abs().max().item()
    mx = T.max().item()
    tol = max(2 * _bf16_ulp(mx), noise)
    gp, go = mx - T[plain[t]].item(), mx - T[other[t]].item()
    return {"step": t, "plain_token": plain[t], "other_token": other[t],
            "gap_plain": round(gp, 5), "gap_other": round(go, 5),
            "top2_margin": round(abs(T[plain[t]].item() - T[other[t]].item()), 5),
            "noise": round(noise, 5), "near_tie": gp <= tol and go <= tol}
