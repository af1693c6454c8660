"""CPU restatement of the reference engine's torch decode path (test infrastructure only).

Every function follows a region of ``engine/engine.py`` in KrishP147/Dryft-Challenge-HTN-2026;
the ``file:line`` citations point there. Rounding points (bf16 casts) are placed exactly where the
reference places them -- see the module docstring of ``oracle`` for how each one is pinned.

Nothing here runs on a GPU: every tensor is moved to the CPU first.
"""
import glob
import json
import os
import types

import torch
import torch.nn.functional as F

CAP_GRAN = 128          # engine.py:24 -- static cache capacity granule
ROPE_LEN = 32768        # engine.py:96 -- rows of the precomputed rope tables


def rope_theta(cfg):
    """RoPE base from an HF config: top-level ``rope_theta`` (transformers 4.x, what
    engine.py:258 reads) or ``rope_parameters.rope_theta`` (transformers 5.x)."""
    if "rope_theta" in cfg:
        return float(cfg["rope_theta"])
    return float(cfg["rope_parameters"]["rope_theta"])


def rms(x, w, eps):
    """engine.py:107-110: fp32 normalise, round to x.dtype, then multiply by w in x.dtype."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * xf.to(x.dtype)


def rope(x, cos, sin):
    """engine.py:113-115: x*cos + rotate_half(x)*sin with rotate_half = cat(-x[h:], x[:h])."""
    h = x.shape[-1] // 2
    return x * cos + torch.cat((-x[..., h:], x[..., :h]), -1) * sin


def build_rope_tables(theta, hd, n, dtype=torch.bfloat16):
    """engine.py:118-122: inv = 1/theta^(2j/hd) in fp32; emb = cat(f, f); cos/sin cast to dtype."""
    inv = 1.0 / (theta ** (torch.arange(0, hd, 2).float() / hd))
    fr = torch.outer(torch.arange(n).float(), inv)
    emb = torch.cat((fr, fr), -1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


class TorchOps:
    """The reference's ``_TorchOps`` (engine.py:125-187) plus ``add_rms`` (fused.py:1058-1059
    semantics: ``(h + d, rms(h + d))``), evaluated on the CPU.

    ``e`` carries ``eps, nh, nkv, hd, cos, sin`` like the reference's engine / fake engine
    (test_fused.py:20-22).
    """

    def __init__(self, e):
        self.e = e

    def linear(self, x, w):                          # engine.py:131-132
        return F.linear(x, w)

    def rms(self, h, w):                             # engine.py:134-135
        return rms(h, w, self.e.eps)

    def add_rms(self, h, d, w):                      # TritonOps.add_rms contract
        hn = h + d
        return hn, rms(hn, w, self.e.eps)

    def gate_up_silu(self, x, wgu):                  # engine.py:137-138
        return self.silu_mul(F.linear(x, wgu))

    def linear_add_norm(self, x, w, h, lnw):         # engine.py:140-142
        h = h + F.linear(x, w)
        return h, rms(h, lnw, self.e.eps)

    def silu_mul(self, gu):                          # engine.py:144-146
        g, u = gu.chunk(2, -1)
        return F.silu(g) * u

    def attn_prefill(self, q, kc, vc, S, last_query_only=False):   # engine.py:148-152
        e = self.e
        return F.scaled_dot_product_attention(
            q, kc[:, :, :S], vc[:, :, :S], is_causal=not last_query_only, enable_gqa=True
        ).transpose(1, 2).reshape(-1, e.nh * e.hd)

    def attn_decode(self, q, kc, vc, pos, W=1):      # engine.py:154-164 (scalar pos, W=1)
        e = self.e
        B, cap = q.shape[0], kc.shape[2]
        mask = (
            torch.zeros(cap, dtype=q.dtype)
            .masked_fill_(torch.arange(cap) > pos, float("-inf"))
            .view(1, 1, 1, cap)
        )
        return F.scaled_dot_product_attention(
            q.reshape(B, e.nkv, e.nh // e.nkv, e.hd), kc, vc, attn_mask=mask
        ).reshape(B, e.nh * e.hd)

    def qkv_post(self, qkv, l, kc, vc, B, S, pos, last_query_only=False):  # engine.py:166-187
        e = self.e
        nh, nkv, hd = e.nh, e.nkv, e.hd
        q, k, v = qkv.split([nh * hd, nkv * hd, nkv * hd], -1)
        q = q.reshape(B, S, nh, hd)
        if last_query_only:
            q = q[:, -1:, :, :]
        q = rms(q, l.qn, e.eps).transpose(1, 2)
        k = rms(k.reshape(B, S, nkv, hd), l.kn, e.eps).transpose(1, 2)
        v = v.reshape(B, S, nkv, hd).transpose(1, 2)
        if pos is None:
            cos, sin = e.cos[:S], e.sin[:S]
            qcos, qsin = (cos[-1:], sin[-1:]) if last_query_only else (cos, sin)
            q, k = rope(q, qcos, qsin), rope(k, cos, sin)
            kc[:, :, :S] = k
            vc[:, :, :S] = v
        else:
            cos, sin = e.cos.index_select(0, pos), e.sin.index_select(0, pos)
            q, k = rope(q, cos, sin), rope(k, cos, sin)
            kc.index_copy_(2, pos, k)
            vc.index_copy_(2, pos, v)
        return q

    # -- per-row extensions ------------------------------------------------------------------
    # The reference's torch ops take one scalar position for the whole batch; its ragged and
    # verify semantics are "each sequence on its own" (engine.py:1093-1105, 549-627). These
    # helpers apply the scalar-position ops row by row, which is exactly that semantics.

    def qkv_post_rows(self, qkv, l, kc, vc, pos):
        """Decode qkv_post with a per-row position ``pos[b]`` (S=1). Returns q [B, nh, 1, hd]."""
        B = qkv.shape[0]
        out = []
        for b in range(B):
            out.append(self.qkv_post(qkv[b:b + 1], l, kc[b:b + 1], vc[b:b + 1], 1, 1,
                                     pos[b:b + 1]))
        return torch.cat(out, 0)

    def attn_decode_rows(self, q, kc, vc, pos):
        """Decode attention with a per-row position ``pos[b]`` (W=1). -> [B, nh*hd]."""
        B = q.shape[0]
        return torch.cat([self.attn_decode(q[b:b + 1], kc[b:b + 1], vc[b:b + 1], pos[b:b + 1])
                          for b in range(B)], 0)


def attn_reference_fp64(q, kc, vc, pos, W, nh, nkv, hd):
    """Independent loop reference for GQA decode attention (restates test_attn.py:14-24 in
    float64). q: [B, nkv, W, G, hd]; token j of sequence b sees keys 0..pos[b]+j.
    Returns [B*W, nh*hd] float64."""
    B = q.shape[0]
    out = torch.zeros(B * W, nh * hd, dtype=torch.float64)
    for b in range(B):
        pb = int(pos[b if pos.numel() > 1 else 0])
        for j in range(W):
            L = pb + j + 1
            K = kc[b, :, :L].double()
            V = vc[b, :, :L].double()
            qj = q[b, :, j].double()
            p = torch.softmax(qj @ K.transpose(1, 2) * hd ** -0.5, -1)
            out[b * W + j] = (p @ V).reshape(-1)
    return out


class _Layer:
    pass


class _State:
    pass


class OracleEngine:
    """CPU restatement of ``Engine`` (engine.py:247-279, 282-316, 333-371, 459-540, 683-732,
    1093-1105) with the oracle flags of the plain greedy path: no speculation, no fp8, torch ops.

    Construct from a model directory (``config.json`` + ``*.safetensors`` with HF names) or from
    an in-memory ``(config, state_dict)`` pair via :meth:`from_state_dict`.
    """

    def __init__(self, model_path=None, dtype=torch.bfloat16, _cfg=None, _weights=None):
        self.dev = torch.device("cpu")
        self.dtype = dtype
        if _cfg is None:
            with open(os.path.join(model_path, "config.json")) as f:
                _cfg = json.load(f)
        cfg = _cfg
        self.L = cfg["num_hidden_layers"]
        self.nh = cfg["num_attention_heads"]
        self.nkv = cfg["num_key_value_heads"]
        self.hd = cfg.get("head_dim") or cfg["hidden_size"] // self.nh
        self.eps = cfg["rms_norm_eps"]
        self.theta = rope_theta(cfg)
        if _weights is None:
            from safetensors.torch import load_file
            _weights = {}
            for fn in sorted(glob.glob(os.path.join(model_path, "*.safetensors"))):
                _weights.update(load_file(fn, device="cpu"))
        self._load(dict(_weights))
        self.cos, self.sin = build_rope_tables(self.theta, self.hd, ROPE_LEN, self.dtype)
        self.ops = TorchOps(self)
        self._dbg = None

    @classmethod
    def from_state_dict(cls, cfg, weights, dtype=torch.bfloat16):
        return cls(None, dtype=dtype, _cfg=cfg, _weights=weights)

    def _load(self, w):
        """engine.py:282-308: fused wqkv = cat(q, k, v), wgu = cat(gate, up), tied lm_head."""
        g = lambda k: w.pop(k).to("cpu").to(self.dtype)
        self.embed = g("model.embed_tokens.weight")
        self.lm_head = g("lm_head.weight") if "lm_head.weight" in w else self.embed
        self.norm = g("model.norm.weight")
        self.layers = []
        for i in range(self.L):
            p = f"model.layers.{i}."
            l = _Layer()
            l.ln1 = g(p + "input_layernorm.weight")
            l.ln2 = g(p + "post_attention_layernorm.weight")
            l.qn = g(p + "self_attn.q_norm.weight")
            l.kn = g(p + "self_attn.k_norm.weight")
            l.wqkv = torch.cat([g(p + f"self_attn.{n}_proj.weight") for n in "qkv"], 0).contiguous()
            l.wo = g(p + "self_attn.o_proj.weight")
            l.wgu = torch.cat([g(p + "mlp.gate_proj.weight"), g(p + "mlp.up_proj.weight")], 0).contiguous()
            l.wd = g(p + "mlp.down_proj.weight")
            self.layers.append(l)

    def new_state(self, B, cap):
        """engine.py:343-349: zero-initialised static caches [B, nkv, cap, hd] per layer."""
        st = _State()
        st.B, st.cap = B, cap
        shape = (B, self.nkv, cap, self.hd)
        st.kc = [torch.zeros(shape, dtype=self.dtype) for _ in range(self.L)]
        st.vc = [torch.zeros(shape, dtype=self.dtype) for _ in range(self.L)]
        st.tok = torch.zeros(B, dtype=torch.long)
        st.pos = torch.zeros(1, dtype=torch.long)
        return st

    def forward(self, st, tokens, S, pos, return_logits=False):
        """engine.py:459-503 with plain torch ops. pos=None: prefill from position 0 (logits for
        each sequence's last token); pos=[1] tensor: one decode step (S=1)."""
        B = st.B
        ops = self.ops
        decode = pos is not None
        h = self.embed[tokens]
        a = ops.rms(h, self.layers[0].ln1)
        last = self.L - 1
        for i, l in enumerate(self.layers):
            kc, vc = st.kc[i], st.vc[i]
            qkv = ops.linear(a, l.wqkv)
            q = ops.qkv_post(qkv, l, kc, vc, B, S, pos, last_query_only=not decode and i == last)
            if decode:
                o = ops.attn_decode(q, kc, vc, pos, S)
            elif i == last:
                o = ops.attn_prefill(q, kc, vc, S, last_query_only=True)
                h = h[S - 1::S].contiguous()
            else:
                o = ops.attn_prefill(q, kc, vc, S)
            h, a = ops.linear_add_norm(o, l.wo, h, l.ln2)
            m = ops.gate_up_silu(a, l.wgu)
            h, a = ops.linear_add_norm(m, l.wd, h, self.layers[i + 1].ln1 if i < last else self.norm)
        logits = ops.linear(a, self.lm_head)
        if self._dbg is not None:
            self._dbg.append(logits.float())
        tok = logits.argmax(-1)
        return (tok, logits) if return_logits else tok

    def forward_rows(self, st, tokens, pos, return_logits=False):
        """One decode step where row b sits at its own position ``pos[b]`` -- the reference's
        ragged semantics (engine.py:1093-1105: each sequence decodes on its own)."""
        B = st.B
        ops = self.ops
        h = self.embed[tokens]
        a = ops.rms(h, self.layers[0].ln1)
        last = self.L - 1
        for i, l in enumerate(self.layers):
            qkv = ops.linear(a, l.wqkv)
            q = ops.qkv_post_rows(qkv, l, st.kc[i], st.vc[i], pos)
            o = ops.attn_decode_rows(q, st.kc[i], st.vc[i], pos)
            h, a = ops.linear_add_norm(o, l.wo, h, l.ln2)
            m = ops.gate_up_silu(a, l.wgu)
            h, a = ops.linear_add_norm(m, l.wd, h, self.layers[i + 1].ln1 if i < last else self.norm)
        logits = ops.linear(a, self.lm_head)
        tok = logits.argmax(-1)
        return (tok, logits) if return_logits else tok

    def prefill(self, st, ids):
        """engine.py:505-515 (eager branch): prompt pass, first token into st.tok."""
        B, S = ids.shape
        st.tok.copy_(self.forward(st, ids.reshape(-1), S, None))

    def decode_step(self, st):
        """engine.py:538-540: one decode step from st.tok at st.pos, then pos += 1."""
        st.tok.copy_(self.forward(st, st.tok, 1, st.pos))
        st.pos.add_(1)

    @torch.inference_mode()
    def generate(self, input_ids, max_new_tokens):
        """engine.py:683-732, plain greedy path (no speculation): yields one list[int] per step."""
        if max_new_tokens <= 0:
            return
        B = len(input_ids)
        S = len(input_ids[0])
        if any(len(x) != S for x in input_ids):
            yield from self.generate_ragged(input_ids, max_new_tokens)
            return
        n = max_new_tokens
        cap = -(-(S + n) // CAP_GRAN) * CAP_GRAN
        if cap > self.cos.shape[0]:
            self.cos, self.sin = build_rope_tables(self.theta, self.hd, cap, self.dtype)
        st = self.new_state(B, cap)
        ids = torch.tensor(input_ids, dtype=torch.long)
        self.prefill(st, ids)
        st.pos.fill_(S)
        yield st.tok.tolist()
        for _ in range(1, n):
            self.decode_step(st)
            yield st.tok.tolist()

    def generate_ragged(self, input_ids, n):
        """engine.py:1093-1105: group by prompt length, interleave per-group generators."""
        groups = {}
        for i, seq in enumerate(input_ids):
            groups.setdefault(len(seq), []).append(i)
        streams = [(idx, self.generate([input_ids[i] for i in idx], n)) for idx in groups.values()]
        for _ in range(n):
            step = [0] * len(input_ids)
            for idx, stream in streams:
                for i, t in zip(idx, next(stream)):
                    step[i] = t
            yield step

    @torch.inference_mode()
    def verify_logits(self, st, tokens, spos):
        """Verify-shaped forward (engine.py:542-547, S=W, per-row start ``spos[b]``) restated as
        W sequential single-token decodes per sequence -- the equivalence the reference's own
        ``_selftest_spec`` pins (engine.py:549-627). tokens: [B, W]. Returns logits [B*W, V]
        in (b, s) row order and writes K/V at spos[b]+s."""
        B, W = tokens.shape
        rows = []
        for b in range(B):
            sub = _State()
            sub.B = 1
            sub.kc = [k[b:b + 1] for k in st.kc]
            sub.vc = [v[b:b + 1] for v in st.vc]
            for s in range(W):
                pos = torch.tensor([int(spos[b]) + s])
                _, lg = self.forward(sub, tokens[b, s:s + 1], 1, pos, return_logits=True)
                rows.append(lg)
        return torch.cat(rows, 0)


def fake_engine(nh, nkv, hd, eps=1e-6, theta=5e6, rope_len=64, dtype=torch.bfloat16):
    """A namespace carrying what the ops read from an engine (test_fused.py:20-22)."""
    e = types.SimpleNamespace(dev=torch.device("cpu"), eps=eps, nh=nh, nkv=nkv, hd=hd, dtype=dtype)
    e.cos, e.sin = build_rope_tables(theta, hd, rope_len, dtype)
    return e
