"""Qwen3-shape greedy-decode engine on MI355X: static KV cache, hipGraph-captured decode step,
pipelined host loop, decode kernels from libdryft_decode.so.

Mirrors the reference ``Engine`` API (engine/engine.py:247-279, 683-732):
``Engine(model_path)`` loads an HF-named safetensors checkpoint, ``generate(input_ids, n)``
yields one ``list[int]`` (one token per sequence) per step. Greedy decoding; the reference's
in-graph speculation (exact acceptance only, ``speculate.py``) and fp8 prefill GEMMs are opt-in
with its own switches (``ENGINE_SPEC=1``, ``ENGINE_FP8=1``).

Differences by design (MI355X-first):
  * decode positions are per row (``st.pos`` is ``[B]``), so a ragged batch decodes in ONE state
    and one weight pass per step instead of the reference's per-length groups
    (engine.py:1093-1105); each row's tokens are the ones the reference produces for that
    sequence on its own;
  * one state (and one captured graph) serves every prompt length of a (B, cap) shape;
  * ``ops`` is :class:`HipOps`; a failed load-time self-test raises instead of falling back to
    torch (``ENGINE_OPS=torch`` selects the torch ops explicitly, for diagnostics).
"""
import glob
import json
import math
import os
import sys

import torch

from .hipops import HipOps, TorchOps
from .speculate import SPEC_W, Speculator
from .step import FusedStep

CAP_GRAN = 128        # engine.py:24
MAX_STATES = 6        # engine.py:94
# fp8 prefill GEMMs (engine.py:97-99, 451-457): tensorwise e4m3 for the QKV and gate/up
# projections of prompts of batches up to FP8_MAX_B. Opt-in (ENGINE_FP8=1): the outputs are not
# bf16-exact, and the reference's own notes (engine.py:100-104) record that its contract forbids
# quantised weights.
FP8_MAX_B = 8
ROPE_LEN = 32768      # engine.py:96


def rope_theta(cfg):
    """RoPE base from an HF config: top-level ``rope_theta`` (transformers 4.x, what
    engine.py:258 reads) or ``rope_parameters.rope_theta`` (transformers 5.x)."""
    if "rope_theta" in cfg:
        return float(cfg["rope_theta"])
    return float(cfg["rope_parameters"]["rope_theta"])


def build_rope_tables(theta, hd, n, dtype=torch.bfloat16):
    """engine.py:118-122, evaluated with torch on the CPU (then uploaded) so the tables are the
    same bits on every machine: inv = 1/theta^(2j/hd) fp32; emb = cat(f, f); cos/sin -> dtype."""
    inv = 1.0 / (theta ** (torch.arange(0, hd, 2).float() / hd))
    fr = torch.outer(torch.arange(n).float(), inv)
    emb = torch.cat((fr, fr), -1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


FLAG_NAMES = {1: "token id out of range", 2: "position outside the KV cache or rope table",
              4: "grid barrier timed out (decode kernel not fully resident)",
              8: "geometry rejected in the kernel"}


def describe_flags(flags):
    return ", ".join(v for k, v in FLAG_NAMES.items() if flags & k) or "unknown"


class _Layer:
    pass


class _State:
    pass


class _Mixed:
    """Diagnostics: HIP ops with some groups swapped for torch ops (ENGINE_OFF=attn,qkv,gemv);
    the reference's _Mixed contract (engine.py:221-236)."""

    GROUPS = {
        "attn": ("attn_decode",),
        "attnp": ("attn_prefill", "attn_prefill_packed"),
        "qkv": ("qkv_post", "qkv_post_packed"),
        "gemv": ("linear", "gate_up_silu", "linear_add_norm"),
    }

    def __init__(self, fused, ref, off):
        self.f, self.r = fused, ref
        self.off = {name for g in off for name in self.GROUPS.get(g, ())}

    def __getattr__(self, name):
        return getattr(self.r if name in self.off else self.f, name)


class Engine:
    def __init__(self, model_path=None, dtype=torch.bfloat16, device=None, selftest=True,
                 _cfg=None, _weights=None):
        self.dev = torch.device(device) if device is not None else torch.device("cuda")
        if self.dev.type != "cuda":
            raise RuntimeError("the HIP decode engine needs a GPU (device 'cuda')")
        self.dtype = dtype
        if _cfg is None:
            with open(os.path.join(model_path, "config.json")) as f:
                _cfg = json.load(f)
        cfg = _cfg
        self.cfg = cfg
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
                _weights.update(load_file(fn, device=str(self.dev)))
        self._load(dict(_weights))
        self.fp8 = os.environ.get("ENGINE_FP8", "0") == "1"
        if self.fp8:
            self._quantize_fp8()
        self._build_rope(ROPE_LEN)
        self.states = {}
        self._dbg = None
        self.pool = torch.cuda.graph_pool_handle()
        self.ops = None
        self.step = None
        self.ops = self._select_ops(selftest)
        self.step = self._select_step(selftest)
        self._specs = {}
        self.spec = None
        self.spec = self._select_spec(selftest)

    @classmethod
    def from_state_dict(cls, cfg, weights, **kw):
        return cls(None, _cfg=cfg, _weights=weights, **kw)

    # ---------------------------------------------------------------- weights
    def _load(self, w):
        """engine.py:282-308: fused wqkv = cat(q, k, v), wgu = cat(gate, up), tied lm_head."""
        g = lambda k: w.pop(k).to(device=self.dev, dtype=self.dtype)
        self.embed = g("model.embed_tokens.weight").contiguous()
        self.lm_head = g("lm_head.weight").contiguous() if "lm_head.weight" in w else self.embed
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
            l.wo = g(p + "self_attn.o_proj.weight").contiguous()
            l.wgu = torch.cat([g(p + "mlp.gate_proj.weight"), g(p + "mlp.up_proj.weight")],
                              0).contiguous()
            l.wd = g(p + "mlp.down_proj.weight").contiguous()
            self.layers.append(l)

    def _quantize_fp8(self):
        """engine.py:310-316: per-tensor scale s = amax / 448, w8 = e4m3(w / s), for the QKV and
        gate/up weights (the reference's default FP8_OPS)."""
        for l in self.layers:
            for name in ("wqkv", "wgu"):
                w = getattr(l, name)
                s = (w.abs().amax().clamp(min=1e-6) / 448.0).float().reshape(1, 1)
                setattr(l, name + "8", (w / s).to(torch.float8_e4m3fn).contiguous())
                setattr(l, name + "8s", s)

    def _build_rope(self, n):
        cos, sin = build_rope_tables(self.theta, self.hd, n, self.dtype)
        self.cos, self.sin = cos.to(self.dev), sin.to(self.dev)

    def _grow_rope(self, cap):
        """engine.py:322-331: rebuild the tables; graphs baked the old addresses, so drop them
        and start a fresh graph pool."""
        self.states.clear()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        self.pool = torch.cuda.graph_pool_handle()
        self._build_rope(cap)

    # ---------------------------------------------------------------- ops selection
    def _select_ops(self, selftest):
        if os.environ.get("ENGINE_OPS") == "torch":
            return TorchOps(self)
        ops = None
        errors = []
        candidates = (("full", True), ("without GEMV", False)) if selftest else (("full", True),)
        for label, use_gemv in candidates:
            cand = HipOps(self, use_gemv=use_gemv)
            if not selftest:
                ops = cand
                break
            try:
                diff = self._selftest(cand)
                print(f"[engine] HIP ops {label} selftest max logit diff {diff:.4f}",
                      file=sys.stderr)
                if diff <= 0.5:
                    ops = cand
                    break
                errors.append(f"{label}: diff {diff:.4f}")
            except Exception as ex:  # report and try the next rung
                errors.append(f"{label}: {ex!r}")
        if ops is None:
            raise RuntimeError("HIP decode ops failed their self-test: " + "; ".join(errors))
        off = [x for x in os.environ.get("ENGINE_OFF", "").split(",") if x]
        if off:
            ops = _Mixed(ops, TorchOps(self), off)
        return ops

    def _select_step(self, selftest):
        """The one-launch decode step (FusedStep) for states it takes (B <= 16, W == 1), checked
        like the ops: 3 teacher-forced steps against torch ops. ENGINE_STEP=0 turns it off;
        a failed check leaves the per-op HipOps graph in charge (also HIP)."""
        if os.environ.get("ENGINE_STEP") == "0" or isinstance(self.ops, (TorchOps, _Mixed)):
            return None
        try:
            step = FusedStep(self)
        except RuntimeError as ex:
            print(f"[engine] fused decode step unavailable: {ex}", file=sys.stderr)
            return None
        if selftest:
            diff = self._selftest(self.ops, step)
            print(f"[engine] fused decode step selftest max logit diff {diff:.4f}", file=sys.stderr)
            if not diff <= 0.5:
                print("[engine] fused decode step failed its self-test; using per-op kernels",
                      file=sys.stderr)
                return None
        return step

    def speculator(self, W=SPEC_W):
        """The in-graph speculative generator of verify width W (needs the one-launch step)."""
        sp = self._specs.get(W)
        if sp is None:
            sp = self._specs[W] = Speculator(self, W)
        return sp

    def _select_spec(self, selftest):
        """Speculation is opt-in (ENGINE_SPEC=1) and kept only if the verify-shaped forward
        matches sequential decode steps (engine.py:549-627, gate 0.5) and its generated tokens
        equal plain greedy decode on a small case (engine.py:1057-1091: B=3, S=48, n=10, eager)."""
        if os.environ.get("ENGINE_SPEC", "0") != "1" or self.step is None:
            return None
        try:
            sp = self.speculator()
            if selftest:
                d1, d2 = self._selftest_verify(sp.W)
                print(f"[engine] verify selftest max logit diff: B=1 W=5 {d1:.4f}, "
                      f"B=4 W={sp.W} at distinct positions {d2:.4f}", file=sys.stderr)
                if not (d1 <= 0.5 and d2 <= 0.5):
                    return None
                torch.manual_seed(3)
                high = min(5000, self.embed.shape[0])
                ids = torch.randint(min(100, high - 1), high, (3, 48)).tolist()
                plain = list(self.generate(ids, 10))
                got = list(sp.generate(ids, 10, graph=False))
                self.states.clear()
                print(f"[engine] speculative selftest B=3 S=48 n=10 W={sp.W} match={got == plain}",
                      file=sys.stderr)
                if got != plain:
                    return None
            return sp
        except RuntimeError as ex:
            print(f"[engine] speculation unavailable: {ex}", file=sys.stderr)
            return None

    @torch.inference_mode()
    def _selftest_verify(self, W2=4):
        """engine.py:549-627: the verify-shaped forward against step-by-step decode on the
        model's weights, two cases: B=1, W=5 at one position; B=4, W=W2 with each row's window at
        a different offset (0, 3, 7, 11) into one lock-step decode timeline, so rows sit at
        distinct positions (per-row position indexing). Returns the two max logit differences
        (the reference's gate is 0.5)."""
        torch.manual_seed(1)
        high = min(5000, self.embed.shape[0])
        low = min(100, high - 1)
        dev = self.dev

        def timeline(ids, B, S, n):
            st = self._new_state(B, 128)
            self._dbg = []
            try:
                self._prefill(ids, st)
                toks = [st.tok.clone()]
                for _ in range(n):
                    self._decode_body(st)
                    toks.append(st.tok.clone())
                return st, toks, self._dbg
            finally:
                self._dbg = None

        # B=1, W=5: row j is the token decode step j consumed, at position S + j
        B, S, W = 1, 96, 5
        ids = torch.randint(low, high, (B, S)).tolist()
        _, toks, plain = timeline(ids, B, S, W)
        sp = self._new_state(B, 128, W=W)
        self._prefill(ids, sp)
        got = self.verify_logits(sp, torch.stack(toks[:W], 1),
                                 torch.full((B,), S, dtype=torch.long, device=dev)).float().cpu()
        d1 = max((got[j] - plain[j + 1][0]).abs().max().item() for j in range(W))
        # B=4, W=W2, rows at distinct positions of one lock-step timeline
        B2, S2, offsets = 4, 96, (0, 3, 7, 11)
        ids2 = torch.randint(low, high, (B2, S2)).tolist()
        st2, toks2, plain2 = timeline(ids2, B2, S2, max(offsets) + W2)
        sp2 = self._new_state(B2, 128, W=W2)
        for i in range(self.L):
            sp2.kc[i].copy_(st2.kc[i])
            sp2.vc[i].copy_(st2.vc[i])
        rows = torch.stack([torch.stack([toks2[o + s][b] for s in range(W2)])
                            for b, o in enumerate(offsets)])
        spos = torch.tensor([S2 + o for o in offsets], dtype=torch.long, device=dev)
        got2 = self.verify_logits(sp2, rows, spos).float().cpu()
        d2 = max((got2[b * W2 + s] - plain2[o + s + 1][b]).abs().max().item()
                 for b, o in enumerate(offsets) for s in range(W2))
        return d1, d2

    def _selftest(self, candidate, step=None):
        """engine.py:629-680 contract: prefill B=2, S=96, then 3 teacher-forced decode steps with
        the candidate ops (and decode step) vs torch ops on the same weights; returns the max
        logit difference."""
        torch.manual_seed(0)
        B, S, n = 2, 96, 4
        high = min(5000, self.embed.shape[0])
        ids = torch.randint(min(100, high - 1), high, (B, S), device=self.dev)

        def run(ops, step, forced=None):
            saved = self.ops, self.step
            self.ops, self.step = ops, step
            try:
                st = self._new_state(B, 128)
                self._dbg, toks = [], []
                self._prefill(ids.tolist(), st)
                for t in range(n):
                    toks.append(st.tok.clone())
                    if t < n - 1:
                        if forced is not None:
                            st.tok.copy_(forced[t])
                        self._decode_body(st)
                return self._dbg, toks
            finally:
                self._dbg = None
                self.ops, self.step = saved

        ref, toks = run(TorchOps(self), None)
        got, _ = run(candidate, step, toks)
        diffs = [(r - g).abs().max().item() for r, g in zip(ref, got)]
        return max(diffs) if all(math.isfinite(d) for d in diffs) else float("inf")

    # ---------------------------------------------------------------- state
    def _new_state(self, B, cap, W=1):
        """engine.py:343-356 (zeros KV [B, nkv, cap, hd] per layer) with per-row positions."""
        st = _State()
        st.B, st.cap, st.W = B, cap, W
        shape = (B, self.nkv, cap, self.hd)
        # The cache starts as zeros: attention multiplies masked-out V rows by a zero weight,
        # and an uninitialised NaN there would survive the product.
        st.kc = [torch.zeros(shape, dtype=self.dtype, device=self.dev) for _ in range(self.L)]
        st.vc = [torch.zeros(shape, dtype=self.dtype, device=self.dev) for _ in range(self.L)]
        # tokens and the state's device error word share one buffer, so the host loop copies
        # both with one transfer per step: tok = tokbuf[:B*W], err = low 32 bits of tokbuf[B*W]
        st.tokbuf = torch.zeros(B * W + 1, dtype=torch.long, device=self.dev)
        st.tok = st.tokbuf[:B * W]
        st.err = st.tokbuf[B * W:].view(torch.int32)[:1]
        st.pos = torch.zeros(B, dtype=torch.long, device=self.dev)
        st.graph = None
        st.hcap = 0
        st.fused = None
        if self.step is not None and self.step.supports(B, W):
            self.step.bind(st)
        return st

    def _evict_for_new_state(self):
        """engine.py:339-341: at MAX_STATES cached states the oldest is dropped."""
        if len(self.states) >= MAX_STATES:
            del self.states[next(iter(self.states))]
            torch.cuda.empty_cache()

    def _state(self, B, cap, W=1, graph=True):
        key = (B, cap, W, graph)
        st = self.states.get(key)
        if st is not None:
            return st
        self._evict_for_new_state()
        st = self._new_state(B, cap, W)
        self.states[key] = st
        if graph:
            try:
                self._capture(st)
            except Exception as e:  # fall back to eager decode (engine.py:365-370)
                print(f"[engine] graph capture failed for {key}: {e!r}", file=sys.stderr)
                st.graph = None
        return st

    def _capture(self, st):
        """engine.py:380-396: warm up on a side stream, then capture one decode step. Positions
        are reset afterwards (the warm-ups and the capture advance them)."""
        st.pos.zero_()
        dbg, self._dbg = self._dbg, None       # no host copies inside the captured step
        try:
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for _ in range(3):
                    self._decode_body(st)
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=self.pool):
                self._decode_body(st)
            st.graph = g
            torch.cuda.synchronize()
        finally:
            self._dbg = dbg
        st.pos.zero_()
        st.tok.zero_()
        st.err.zero_()

    def _host_bufs(self, st, n):
        if st.hcap < n:
            st.hcap = max(n, 256)
            st.host = torch.empty((st.hcap, st.B * st.W + 1), dtype=torch.long, pin_memory=True)
            st.events = [torch.cuda.Event() for _ in range(st.hcap)]

    # ---------------------------------------------------------------- forward
    def _forward(self, st, tokens, S, pos):
        """engine.py:459-503 layer loop. pos=None: prefill from position 0 (logits of each
        sequence's last token); pos=[B] tensor: decode of S tokens per row starting at pos[b].
        Returns bf16 logits."""
        B = st.B
        ops = self.ops
        decode = pos is not None
        if decode and hasattr(ops, "embed_rms"):
            h, a = ops.embed_rms(tokens, self.embed, self.layers[0].ln1)
        else:
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
            self._dbg.append(logits.float().cpu())
        return logits

    def _decode_body(self, st):
        """engine.py:538-540: tok <- argmax(forward(tok, pos)); pos += 1. States bound to the
        fused step run it as one launch; others run the per-op kernels (argmax and pos += 1
        fused in one kernel)."""
        if st.fused is not None:
            logits = self.step.run(st)
            if self._dbg is not None:
                self._dbg.append(logits.float().cpu())
            return
        logits = self._forward(st, st.tok, st.W, st.pos)
        if hasattr(self.ops, "argmax_"):
            self.ops.argmax_(logits, st.tok, st.pos)
        else:
            st.tok.copy_(logits.argmax(-1))
            st.pos.add_(1)
        err = getattr(self.ops, "err", None)
        if err is not None:                   # per-op kernels flag into the ops' error word
            torch.bitwise_or(st.err, err, out=st.err)

    def _forward_packed(self, st, input_ids):
        """Prefill of B prompts of any lengths in one pass (engine.py:459-503 with pos = None,
        per prompt): the prompts' tokens packed end to end, the GEMMs over all of them at once,
        q/k norm + RoPE + cache write and causal attention per prompt from the packed offsets,
        the last layer on each prompt's last token only. Returns bf16 logits [B, V]."""
        ops = self.ops
        B = len(input_ids)
        lens = [len(x) for x in input_ids]
        starts = [0]
        for n in lens:
            starts.append(starts[-1] + n)
        T = starts[-1]
        dev = self.dev
        tokens = torch.tensor([t for x in input_ids for t in x], dtype=torch.long, device=dev)
        seq_start = torch.tensor(starts, dtype=torch.int32, device=dev)
        last_rows = seq_start[1:].long() - 1
        if hasattr(ops, "embed_rms"):
            h, a = ops.embed_rms(tokens, self.embed, self.layers[0].ln1)
        else:
            h = self.embed[tokens]
            a = ops.rms(h, self.layers[0].ln1)
        last = self.L - 1
        use8 = self.fp8 and B <= FP8_MAX_B and hasattr(ops, "fp8_linear")
        for i, l in enumerate(self.layers):
            qkv = ops.fp8_linear(a, l.wqkv8, l.wqkv8s, l.wqkv) if use8 else ops.linear(a, l.wqkv)
            q = ops.qkv_post_packed(qkv, l, st.kc[i], st.vc[i], seq_start, B, T, i == last)
            o = ops.attn_prefill_packed(q, st.kc[i], st.vc[i], seq_start, B, T, i == last)
            if i == last:
                h = h.index_select(0, last_rows)
            h, a = ops.linear_add_norm(o, l.wo, h, l.ln2)
            if use8:
                m = ops.silu_mul(ops.fp8_linear(a, l.wgu8, l.wgu8s, l.wgu))
            else:
                m = ops.gate_up_silu(a, l.wgu)
            h, a = ops.linear_add_norm(m, l.wd, h, self.layers[i + 1].ln1 if i < last else self.norm)
        logits = ops.linear(a, self.lm_head)
        if self._dbg is not None:
            self._dbg.append(logits.float().cpu())
        return logits

    def _prefill(self, input_ids, st):
        """Prompt pass (engine.py:505-515, eager). Ops with the packed prefill (HipOps): one pass
        over all prompts, equal or ragged. Others: equal lengths in one batched pass, ragged one
        pass per sequence into its own cache row. Sets st.tok and st.pos[b] = len(prompt b)."""
        lens = [len(x) for x in input_ids]
        if hasattr(self.ops, "qkv_post_packed") and hasattr(self.ops, "attn_prefill_packed"):
            st.tok[:len(input_ids)].copy_(self._forward_packed(st, input_ids).argmax(-1))
            err = getattr(self.ops, "err", None)
            if err is not None:               # prefill flags (token or position out of range)
                torch.bitwise_or(st.err, err, out=st.err)
        elif len(set(lens)) == 1:
            ids = torch.tensor(input_ids, dtype=torch.long, device=self.dev)
            B, S = ids.shape
            st.tok[:B].copy_(self._forward(st, ids.reshape(-1), S, None).argmax(-1))
        else:
            dbg = self._dbg
            rows = []
            for b, seq in enumerate(input_ids):
                sub = _State()
                sub.B = 1
                sub.kc = [k[b:b + 1] for k in st.kc]
                sub.vc = [v[b:b + 1] for v in st.vc]
                ids = torch.tensor([seq], dtype=torch.long, device=self.dev)
                self._dbg = [] if dbg is not None else None
                st.tok[b:b + 1].copy_(self._forward(sub, ids.reshape(-1), len(seq), None).argmax(-1))
                if dbg is not None:
                    rows.append(self._dbg[-1])
            self._dbg = dbg
            if dbg is not None:
                dbg.append(torch.cat(rows, 0))
        st.pos.copy_(torch.tensor(lens, dtype=torch.long, device=self.dev))

    # ---------------------------------------------------------------- generate
    @torch.inference_mode()
    def generate(self, input_ids, max_new_tokens):
        """engine.py:683-732 plain path: prefill, then n-1 graph replays; the host copies step t's
        tokens into pinned memory and yields step t-1 while step t runs. With speculation on
        (ENGINE_SPEC=1) shapes inside its gate go through the in-graph speculative path instead
        (engine.py:693-706)."""
        if max_new_tokens <= 0:
            return
        n = max_new_tokens
        B = len(input_ids)
        if self.spec is not None and self.spec.takes(B, n):
            yield from self.spec.generate(input_ids, n)
            return
        S = max(len(x) for x in input_ids)
        cap = -(-(S + n) // CAP_GRAN) * CAP_GRAN
        if cap > self.cos.shape[0]:
            self._grow_rope(cap)
        st = self._state(B, cap, graph=n > 1)
        self._host_bufs(st, n)
        if st.fused is not None:
            self.recover(int(st.err.item()))   # a barrier timeout left by an earlier call
        self._clear_errors(st)
        self._prefill(input_ids, st)
        host, ev = st.host, st.events
        host[0].copy_(st.tokbuf, non_blocking=True)
        ev[0].record()
        for t in range(1, n):
            if st.graph is not None:
                st.graph.replay()
            else:
                self._decode_body(st)
            host[t].copy_(st.tokbuf, non_blocking=True)
            ev[t].record()
            ev[t - 1].synchronize()
            yield self._checked(host[t - 1], t - 1)
        ev[n - 1].synchronize()
        yield self._checked(host[n - 1], n - 1)

    def _clear_errors(self, st):
        st.err.zero_()
        err = getattr(self.ops, "err", None)
        if err is not None:
            err.zero_()

    def recover(self, flags):
        """After a step that flagged a grid-barrier timeout (flag 4) the one-launch step's
        counters may be left nonzero (its workgroups stopped waiting, so hand-off counters that
        their last arrivers reset can keep a count): zero them before the next launch.
        Synchronises the device when it acts."""
        if flags & 4 and self.step is not None:
            self.step.reset_counters()

    def _checked(self, row, t):
        """Tokens of one step from the host ring, after its error word (the ring's last column):
        a step that flagged an error raises instead of yielding tokens computed from it."""
        flags = int(row[-1]) & 0xffffffff
        if flags:
            self.recover(flags)
            raise RuntimeError(f"decode step {t} reported error flags {flags:#x} ({describe_flags(flags)})")
        return row[:-1].tolist()

    # ---------------------------------------------------------------- verify shape
    @torch.inference_mode()
    def verify_logits(self, st, tokens, spos):
        """Multi-query (verify-shaped) forward: row (b, s) is token tokens[b, s] at position
        spos[b] + s, causal within the W rows (engine.py:542-547; fused.py:438-441, 492-503).
        Writes K/V at spos[b] + s and returns logits [B*W, V]."""
        B, W = tokens.shape
        if st.fused is not None:
            st.tok.copy_(tokens.reshape(-1))
            st.pos.copy_(spos)
            return self.step.run(st)
        return self._forward(st, tokens.reshape(-1).contiguous(), W, spos)

    def error_flags(self):
        """Device error words of the kernels, OR-ed over the ops and every cached state (1: token
        id out of range, 2: position outside the cache / rope table, 4: a grid barrier of the
        fused step timed out). Synchronises."""
        ops = self.ops.f if isinstance(self.ops, _Mixed) else self.ops
        flags = int(ops.err.item()) if hasattr(ops, "err") else 0
        for st in self.states.values():
            flags |= int(st.err.item())
        self.recover(flags)
        return flags
