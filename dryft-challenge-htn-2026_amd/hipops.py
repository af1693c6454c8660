"""``HipOps``: the engine's ops object backed by the gfx950 HIP kernels of libdryft_decode.so.

Drop-in for the reference's ``TritonOps`` (engine/fused.py:880-1059): same constructor
``HipOps(e, use_gemv=True)``, same methods, same argument meaning, same output layouts, and the
same fallback contract for inputs the kernels do not take (``F.linear`` for non-bf16,
non-contiguous or M > BM_MAX inputs, i.e. the prefill's GEMMs run on hipBLASLt; torch for
non-bf16 prefill). The prefill branch of ``qkv_post`` and ``attn_prefill`` run the HIP prefill
kernels; ``qkv_post_packed`` / ``attn_prefill_packed`` take a packed ragged batch (prompt b =
packed tokens ``seq_start[b] .. seq_start[b+1]-1``) so prompts of different lengths prefill in
one pass. ``e`` carries ``dev, eps, nh, nkv, hd, cos, sin`` like the reference's engine
(test_fused.py:20-22).

Every decode-step method calls the C ABI on torch's current stream; outputs and workspaces are
allocated with ``torch.empty`` (so they come from the graph pool under capture). A nonzero
status raises ``RuntimeError``.
"""
import json
import math
import os

import torch
import torch.nn.functional as F

from ._lib import check, lib

BM_MAX = 16  # largest activation-row count the skinny GEMV takes (fused.py:838 BM_MAX role)
GEMM_MIN_M = 256  # smallest row count sent to the tuned hipBLASLt GEMM (prefill-sized products)


def _ptr(t):
    return t.data_ptr() if t is not None else None


# hipBLASLt solution per prefill GEMM shape and row range (tune_gemm.py writes it on the GPU)
GEMM_TABLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_solutions.json")


def load_gemm_table(path=GEMM_TABLE):
    """{(N, K): [(M, solution), ...] sorted by M} from the committed table, or {} when it is
    absent (every shape then runs hipBLASLt's first heuristic candidate)."""
    try:
        with open(path) as f:
            doc = json.load(f)
    except (OSError, ValueError):
        return {}
    out = {}
    for key, rows in doc.get("shapes", {}).items():
        n, k = (int(v) for v in key.split("x"))
        out[(n, k)] = sorted((int(m), int(sol)) for m, sol in rows)
    return out


def gemm_solution(table, N, K, M):
    """The table's solution for an (N, K) product of M rows: the entry whose row count is
    nearest to M on a log scale (the smaller on a tie), or -1 (heuristic first) for shapes the
    table lacks."""
    rows = table.get((N, K))
    if not rows:
        return -1
    lm = math.log(M)
    return min(rows, key=lambda r: abs(math.log(r[0]) - lm))[1]


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _bf16_ok(*ts):
    return all(t.dtype == torch.bfloat16 and t.is_contiguous() and t.is_cuda for t in ts)


# -- torch helpers for the prefill branch (outside the decode step; same arithmetic as the
#    reference's _rms / _rope, engine.py:107-115) -----------------------------------------------
def _rms_t(x, w, eps):
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * xf.to(x.dtype)


def _rope_t(x, cos, sin):
    h = x.shape[-1] // 2
    return x * cos + torch.cat((-x[..., h:], x[..., :h]), -1) * sin


def _qkv_post_prefill_t(e, qkv, l, kc, vc, B, S, last_query_only):
    """Prefill branch of qkv_post (engine.py:172-181) in torch on the GPU: positions 0..S-1."""
    nh, nkv, hd = e.nh, e.nkv, e.hd
    q, k, v = qkv.split([nh * hd, nkv * hd, nkv * hd], -1)
    q = q.reshape(B, S, nh, hd)
    if last_query_only:
        q = q[:, -1:, :, :]
    q = _rms_t(q, l.qn, e.eps).transpose(1, 2)
    k = _rms_t(k.reshape(B, S, nkv, hd), l.kn, e.eps).transpose(1, 2)
    v = v.reshape(B, S, nkv, hd).transpose(1, 2)
    cos, sin = e.cos[:S], e.sin[:S]
    qcos, qsin = (cos[-1:], sin[-1:]) if last_query_only else (cos, sin)
    q, k = _rope_t(q, qcos, qsin), _rope_t(k, cos, sin)
    kc[:, :, :S] = k
    vc[:, :, :S] = v
    return q


class HipOps:
    """Ops object of the decode path on MI355X (gfx950)."""

    def __init__(self, e, use_gemv=True):
        self.e = e
        self.use_gemv = use_gemv
        assert e.hd & (e.hd - 1) == 0 and e.hd >= 2
        self.L = lib()  # raises when the library is missing: no silent fallback
        self._counters = None
        self._gemm_ws = None
        self._gemm_table = load_gemm_table()
        self._starts = {}
        self.err = torch.zeros(1, dtype=torch.int32, device=e.dev)

    # ---------------------------------------------------------------- helpers
    def _zeroed_counters(self, n, dev):
        """Zeroed int32 counters shared by every call on this stream (the kernels leave them
        zero). Allocated once, outside graph capture, and grown only when a larger op needs it."""
        c = self._counters
        if c is None or c.numel() < n or c.device != dev:
            self._counters = torch.zeros(max(n, 16384), dtype=torch.int32, device=dev)
        return self._counters

    def _gemv_ok(self, x, w):
        M, K = x.shape
        return (self.use_gemv and 1 <= M <= BM_MAX and _bf16_ok(x, w) and K % 8 == 0
                and x.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0)

    def _gemm_ok(self, x, w):
        """Prefill-sized bf16 products go to the library's hipBLASLt GEMM (dd_gemm_bf16) with the
        solution the committed table names for the shape; DD_TUNED_GEMM=0 keeps them on F.linear
        (diagnostics)."""
        return (x.dim() == 2 and x.shape[0] >= GEMM_MIN_M and _bf16_ok(x, w)
                and os.environ.get("DD_TUNED_GEMM", "1") != "0")

    def _gemm_lib(self, x, w, solution=None):
        M, K = x.shape
        N = w.shape[0]
        if solution is None:
            solution = gemm_solution(self._gemm_table, N, K, M)
        ws = self._gemm_ws
        if ws is None or ws.device != x.device:
            ws = self._gemm_ws = torch.empty(self.L.dd_gemm_ws_bytes(), dtype=torch.uint8,
                                             device=x.device)
        y = torch.empty((M, N), dtype=x.dtype, device=x.device)
        check(self.L.dd_gemm_bf16(_ptr(x), _ptr(w), _ptr(y), M, N, K, _ptr(ws), ws.numel(),
                                  solution, _stream(x.device)), "dd_gemm_bf16")
        return y

    def _gemm(self, x, w):
        """y = x . w^T on hipBLASLt with the table's solution for (N, K, M): a fixed choice per
        shape, so every process computes the same bits for the same operands."""
        return self._gemm_lib(x.contiguous(), w.contiguous())

    # ---------------------------------------------------------------- norms
    def rms(self, h, w):
        h = h.contiguous()
        if not _bf16_ok(h, w):
            return _rms_t(h, w, self.e.eps)
        M, N = h.reshape(-1, h.shape[-1]).shape
        y = torch.empty_like(h)
        check(self.L.dd_rmsnorm(_ptr(h), _ptr(w), _ptr(y), M, N, self.e.eps, _stream(h.device)),
              "dd_rmsnorm")
        return y

    def add_rms(self, h, d, w):
        h, d = h.contiguous(), d.contiguous()
        if not _bf16_ok(h, d, w):
            hn = h + d
            return hn, _rms_t(hn, w, self.e.eps)
        M, N = h.reshape(-1, h.shape[-1]).shape
        hn = torch.empty_like(h)
        y = torch.empty_like(h)
        check(self.L.dd_add_rmsnorm(_ptr(h), _ptr(d), _ptr(w), _ptr(hn), _ptr(y), M, N,
                                    self.e.eps, _stream(h.device)), "dd_add_rmsnorm")
        return hn, y

    def silu_mul(self, gu):
        gu = gu.contiguous()
        M, I2 = gu.shape
        out = torch.empty((M, I2 // 2), dtype=gu.dtype, device=gu.device)
        if not _bf16_ok(gu):
            g, u = gu.chunk(2, -1)
            return F.silu(g) * u
        check(self.L.dd_silu_mul(_ptr(gu), _ptr(out), M, I2 // 2, _stream(gu.device)),
              "dd_silu_mul")
        return out

    # ---------------------------------------------------------------- GEMV family
    def linear(self, x, w):
        if not self._gemv_ok(x, w):
            return self._gemm(x, w) if self._gemm_ok(x, w) else F.linear(x, w)
        M, K = x.shape
        N = w.shape[0]
        out = torch.empty((M, N), dtype=x.dtype, device=x.device)
        sk = self.L.dd_gemv_splitk(M, N, K)
        ws = cnt = None
        nbytes = self.L.dd_gemv_ws_bytes(M, N, K, sk)
        if nbytes:
            ws = torch.empty(nbytes // 4, dtype=torch.float32, device=x.device)
            cnt = self._zeroed_counters(self.L.dd_gemv_counters(N), x.device)
        check(self.L.dd_gemv(_ptr(x), _ptr(w), _ptr(out), M, N, K, sk, _ptr(ws), _ptr(cnt),
                             _stream(x.device)), "dd_gemv")
        return out

    def gate_up_silu(self, x, wgu):
        if not self._gemv_ok(x, wgu):
            return self.silu_mul(self.linear(x, wgu))
        M, K = x.shape
        I = wgu.shape[0] // 2
        out = torch.empty((M, I), dtype=x.dtype, device=x.device)
        check(self.L.dd_gate_up_silu(_ptr(x), _ptr(wgu), _ptr(out), M, I, K, _stream(x.device)),
              "dd_gate_up_silu")
        return out

    def linear_add_norm(self, x, w, h, lnw):
        """hn = h + x @ w^T ; returns (hn, rmsnorm(hn, lnw))"""
        if not (self._gemv_ok(x, w) and _bf16_ok(h, lnw)):
            return self.add_rms(h, self.linear(x, w), lnw)
        M, K = x.shape
        N = w.shape[0]
        sk = self.L.dd_gemv_splitk(M, N, K)
        ws = torch.empty(self.L.dd_gemv_add_rmsnorm_ws_bytes(M, N, K, sk) // 4,
                         dtype=torch.float32, device=x.device)
        cnt = self._zeroed_counters(self.L.dd_gemv_counters(N), x.device)
        hn = torch.empty_like(h)
        y = torch.empty_like(h)
        check(self.L.dd_gemv_add_rmsnorm(_ptr(x), _ptr(w), _ptr(h), _ptr(lnw), _ptr(hn), _ptr(y),
                                         M, N, K, self.e.eps, sk, _ptr(ws), _ptr(cnt),
                                         _stream(x.device)), "dd_gemv_add_rmsnorm")
        return hn, y

    # ---------------------------------------------------------------- attention block
    def qkv_post(self, qkv, l, kc, vc, B, S, pos, last_query_only=False):
        e = self.e
        if pos is None:
            return self._qkv_post_prefill(qkv, l, kc, vc, B, S, last_query_only)
        qkv = qkv.contiguous()
        q = torch.empty((B, e.nh, S, e.hd), dtype=qkv.dtype, device=qkv.device)
        pos_stride = 1 if pos.numel() > 1 else 0
        check(self.L.dd_qkv_post_decode(
            _ptr(qkv), _ptr(l.qn), _ptr(l.kn), _ptr(e.cos), _ptr(e.sin), e.cos.shape[0],
            _ptr(pos), pos_stride, _ptr(q), _ptr(kc), _ptr(vc), B, S, e.nh, e.nkv, e.hd,
            kc.shape[2], e.eps, _ptr(self.err), _stream(qkv.device)), "dd_qkv_post_decode")
        return q

    def attn_decode(self, q, kc, vc, pos, W=1):
        """q: [B, nkv, W, G, hd] (from qkv_post). Token j of seq b attends to
        kc/vc[b, :, :pos[b]+j+1]. -> [B*W, nh*hd]"""
        e = self.e
        B = q.shape[0]
        cap = kc.shape[2]
        chunk = self.L.dd_attn_chunk(B, e.nkv, cap)
        out = torch.empty((B * W, e.nh * e.hd), dtype=q.dtype, device=q.device)
        ws = torch.empty(max(1, self.L.dd_attn_ws_bytes(B, W, e.nh, e.nkv, e.hd, cap, chunk) // 4),
                         dtype=torch.float32, device=q.device)
        counters = self._zeroed_counters(B * e.nkv, q.device)
        pos_stride = 1 if pos.numel() > 1 else 0
        check(self.L.dd_attn_decode(_ptr(q.contiguous()), _ptr(kc), _ptr(vc), _ptr(pos), pos_stride,
                                    _ptr(out), _ptr(ws), _ptr(counters), B, W, e.nh, e.nkv, e.hd,
                                    cap, chunk, _stream(q.device)), "dd_attn_decode")
        return out

    # ---------------------------------------------------------------- fp8 prefill GEMMs
    def fp8_linear(self, x, w8, w_scale, w):
        """engine.py:451-457: y = x @ w^T with x quantised tensorwise to fp8 e4m3 by the HIP
        kernel and w8 / w_scale the weight's tensorwise fp8 copy, on hipBLASLt (torch._scaled_mm)
        with bf16 output. As in the reference's _fp8_lin, a row count that is not a multiple of
        16 (the fp8 GEMM's granule) takes the bf16 ``linear`` instead."""
        x = x.contiguous()
        M, K = x.shape
        if M % 16 != 0 or K % 16 != 0 or not _bf16_ok(x):
            return self.linear(x, w)
        xq = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=x.device)
        xs = torch.empty((1, 1), dtype=torch.float32, device=x.device)
        ws = torch.empty(self.L.dd_fp8_quant_ws_bytes(M * K) // 4, dtype=torch.float32,
                         device=x.device)
        check(self.L.dd_fp8_quant(_ptr(x), M * K, _ptr(xq), _ptr(xs), _ptr(ws), _stream(x.device)),
              "dd_fp8_quant")
        return torch._scaled_mm(xq, w8.t(), scale_a=xs, scale_b=w_scale, out_dtype=torch.bfloat16)

    # ---------------------------------------------------------------- prefill
    def _seq_start(self, B, S, dev):
        """Packed offsets of B prompts of length S (int32 [B+1]), kept per shape."""
        key = (B, S, dev)
        t = self._starts.get(key)
        if t is None:
            t = torch.arange(0, B * S + 1, S, dtype=torch.int32, device=dev)
            self._starts[key] = t
        return t

    def qkv_post_packed(self, qkv, l, kc, vc, seq_start, B, T, last_only=False):
        """Prefill qkv_post over a packed batch (fused.py:912-931 semantics, per prompt): k/v of
        every token to kc/vc[b, :, position]; returns q token-major [T, nh, hd], or [B, nh, hd]
        holding each prompt's last token when ``last_only``."""
        e = self.e
        qkv = qkv.contiguous()
        q = torch.empty((B if last_only else T, e.nh, e.hd), dtype=qkv.dtype, device=qkv.device)
        check(self.L.dd_qkv_post_prefill(
            _ptr(qkv), _ptr(l.qn), _ptr(l.kn), _ptr(e.cos), _ptr(e.sin), e.cos.shape[0],
            _ptr(seq_start), B, T, int(last_only), _ptr(q), _ptr(kc), _ptr(vc), e.nh, e.nkv, e.hd,
            kc.shape[2], e.eps, _ptr(self.err), _stream(qkv.device)), "dd_qkv_post_prefill")
        return q

    def attn_prefill_packed(self, q, kc, vc, seq_start, B, T, last_only=False):
        """Causal prefill attention over a packed batch (fused.py:943-959 semantics, per prompt).
        q from qkv_post_packed; returns [T, nh*hd] ([B, nh*hd] when ``last_only``)."""
        e = self.e
        q = q.contiguous()
        out = torch.empty((q.shape[0], e.nh * e.hd), dtype=q.dtype, device=q.device)
        check(self.L.dd_attn_prefill(_ptr(q), _ptr(kc), _ptr(vc), _ptr(seq_start), B, T,
                                     int(last_only), _ptr(out), e.nh, e.nkv, e.hd, kc.shape[2],
                                     _stream(q.device)), "dd_attn_prefill")
        return out

    def _qkv_post_prefill(self, qkv, l, kc, vc, B, S, last_query_only):
        """engine.py:172-181 / fused.py:912-931: q returned as a [B, nh, S', hd] view over a
        token-major [B, S', nh, hd] buffer (S' = 1 when last_query_only)."""
        e = self.e
        if not _bf16_ok(kc, vc) or qkv.dtype != torch.bfloat16:
            return _qkv_post_prefill_t(e, qkv, l, kc, vc, B, S, last_query_only)
        q = self.qkv_post_packed(qkv, l, kc, vc, self._seq_start(B, S, qkv.device), B, B * S,
                                 last_query_only)
        return q.view(B, 1 if last_query_only else S, e.nh, e.hd).transpose(1, 2)

    def attn_prefill(self, q, kc, vc, S, last_query_only=False):
        """Prefill attention (engine.py:148-152, fused.py:943-959): causal over keys 0..S-1 of
        each row, or the last query only. q: [B, nh, S', hd]. -> [B*S', nh*hd]."""
        e = self.e
        if not _bf16_ok(kc, vc) or q.dtype != torch.bfloat16:
            return F.scaled_dot_product_attention(
                q, kc[:, :, :S], vc[:, :, :S], is_causal=not last_query_only, enable_gqa=True
            ).transpose(1, 2).reshape(-1, e.nh * e.hd)
        B = q.shape[0]
        qtm = q.transpose(1, 2).contiguous()      # token-major (no copy for qkv_post's view)
        return self.attn_prefill_packed(qtm.view(-1, e.nh, e.hd), kc, vc,
                                        self._seq_start(B, S, q.device), B, B * S,
                                        last_query_only)

    # ---------------------------------------------------------------- step tail
    def argmax_(self, logits, tok, pos=None):
        """tok[:] = logits.argmax(-1); pos += 1 when given (engine.py:503, 539-540)."""
        M, V = logits.shape
        ws = torch.empty(self.L.dd_argmax_ws_bytes(M, V) // 4, dtype=torch.float32,
                         device=logits.device)
        cnt = self._zeroed_counters(M, logits.device)
        check(self.L.dd_argmax(_ptr(logits.contiguous()), M, V, _ptr(tok), _ptr(pos),
                               0 if pos is None else pos.numel(), _ptr(ws), _ptr(cnt),
                               _stream(logits.device)), "dd_argmax")
        return tok

    def embed_rms(self, tokens, embed, w):
        """h = embed[tokens]; a = rms(h, w) (engine.py:467-468). -> (h, a)"""
        M = tokens.numel()
        V, N = embed.shape
        h = torch.empty((M, N), dtype=embed.dtype, device=embed.device)
        a = torch.empty_like(h)
        check(self.L.dd_embed_rmsnorm(_ptr(tokens), _ptr(embed), V, _ptr(w), _ptr(h), _ptr(a), M,
                                      N, self.e.eps, _ptr(self.err), _stream(embed.device)),
              "dd_embed_rmsnorm")
        return h, a


class TorchOps:
    """The reference's torch arithmetic (``_TorchOps``, engine.py:125-187) on the GPU, extended
    to per-row positions ``pos[B]`` and verify widths W > 1. It is not the decode path: the
    engine uses it for its load-time self-test and when ``ENGINE_OPS=torch`` asks for it."""

    def __init__(self, e):
        self.e = e

    def linear(self, x, w):
        return F.linear(x, w)

    def rms(self, h, w):
        return _rms_t(h, w, self.e.eps)

    def add_rms(self, h, d, w):
        hn = h + d
        return hn, _rms_t(hn, w, self.e.eps)

    def gate_up_silu(self, x, wgu):
        return self.silu_mul(F.linear(x, wgu))

    def linear_add_norm(self, x, w, h, lnw):
        h = h + F.linear(x, w)
        return h, _rms_t(h, lnw, self.e.eps)

    def silu_mul(self, gu):
        g, u = gu.chunk(2, -1)
        return F.silu(g) * u

    def attn_prefill(self, q, kc, vc, S, last_query_only=False):
        e = self.e
        return F.scaled_dot_product_attention(
            q, kc[:, :, :S], vc[:, :, :S], is_causal=not last_query_only, enable_gqa=True
        ).transpose(1, 2).reshape(-1, e.nh * e.hd)

    def _positions(self, pos, B, S):
        p = pos.reshape(-1)
        p = p.expand(B) if p.numel() == 1 else p
        return p[:, None] + torch.arange(S, device=p.device)[None, :]      # [B, S]

    def attn_decode(self, q, kc, vc, pos, W=1):
        e = self.e
        B, cap = q.shape[0], kc.shape[2]
        G = e.nh // e.nkv
        P = self._positions(pos, B, W)                                      # [B, W]
        lim = P.repeat_interleave(G, dim=1)                                 # row r = s*G + g
        mask = torch.zeros((B, 1, W * G, cap), dtype=q.dtype, device=q.device)
        mask.masked_fill_(torch.arange(cap, device=q.device)[None, None, None, :]
                          > lim[:, None, :, None], float("-inf"))
        o = F.scaled_dot_product_attention(q.reshape(B, e.nkv, W * G, e.hd), kc, vc,
                                           attn_mask=mask)
        return o.reshape(B, e.nkv, W, G, e.hd).permute(0, 2, 1, 3, 4).reshape(B * W, e.nh * e.hd)

    def qkv_post(self, qkv, l, kc, vc, B, S, pos, last_query_only=False):
        e = self.e
        nh, nkv, hd = e.nh, e.nkv, e.hd
        if pos is None:
            return _qkv_post_prefill_t(e, qkv, l, kc, vc, B, S, last_query_only)
        q, k, v = qkv.split([nh * hd, nkv * hd, nkv * hd], -1)
        P = self._positions(pos, B, S)                                      # [B, S]
        cos, sin = e.cos[P][:, :, None, :], e.sin[P][:, :, None, :]         # [B, S, 1, hd]
        q = _rope_t(_rms_t(q.reshape(B, S, nh, hd), l.qn, e.eps), cos, sin)
        k = _rope_t(_rms_t(k.reshape(B, S, nkv, hd), l.kn, e.eps), cos, sin)
        v = v.reshape(B, S, nkv, hd)
        bi = torch.arange(B, device=qkv.device)[:, None].expand(B, S)
        kc[bi, :, P] = k
        vc[bi, :, P] = v
        G = nh // nkv
        qo = q.reshape(B, S, nkv, G, hd).permute(0, 2, 1, 3, 4).contiguous()  # [B, nkv, S, G, hd]
        return qo.view(B, nh, S, hd)
