"""``FusedStep``: the whole greedy decode step as ONE persistent kernel launch (dd_decode_step).

The reference runs a decode step as a CUDA graph of ~10 kernels per layer
(``Engine._capture``, engine/engine.py:380-396, replaying ``_decode_body`` engine.py:538-540
over ``_forward`` engine.py:459-503). On MI355X the per-kernel launch gaps and the tail of every
small GEMV cost more than the weight stream itself at decode batch sizes, so this path runs the
step's phases (embedding; per layer QKV+norm+RoPE+KV write, attention, O+residual,
gate/up+SiLU, down+residual; lm_head+argmax) inside one launch of one workgroup per CU, with
grid barriers between phases and every weight matrix streamed from a copy re-laid out once in
MFMA tile order (``dd_tile_weight``).

Same arithmetic and rounding points as ``HipOps`` / the reference ``_TorchOps``; it takes
``B <= 16`` sequences with one token each (a decode step, ``W == 1``) or up to 5 tokens each (the
verify-shaped step of speculation, engine.py:542-547: row ``b W + s`` is token s of sequence b at
position ``pos[b] + s``, causal within the W rows, and positions are not advanced). The engine
uses it for those states and the per-op ``HipOps`` graph otherwise (both are HIP; there is no
CPU path).
"""
import ctypes
import os

import torch

from ._lib import check, lib

MAXB = 16
MAXW = 5
HD = 128
NFIELD = 16


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


class FusedStep:
    """Tiled weights of one engine plus per-state buffers for ``dd_decode_step``."""

    def __init__(self, e):
        self.e = e
        self.L = lib()
        self._ctr = None
        self.grid = self.L.dd_step_grid()
        if self.grid <= 0:
            raise RuntimeError("dd_step_grid: the persistent decode kernel cannot be resident")
        if e.hd != HD:
            raise RuntimeError(f"fused decode step needs head_dim {HD}, got {e.hd}")
        self.H = e.embed.shape[1]
        self.V = e.lm_head.shape[0]
        self.I = e.layers[0].wd.shape[1]
        if not self.L.dd_step_supported(e.L, self.H, e.nh, e.nkv, self.I, self.V, MAXB, 1):
            raise RuntimeError("dd_step_supported: model geometry not taken by the fused step")
        # matrix kinds of dd_tile_weight: 0 wqkv (rows head-grouped: aux = kv heads), 1 wo,
        # 2 wgu (aux = I), 3 wd, 4 lm_head (each laid out for the workgroup split of its GEMV
        # phase on this device)
        with torch.no_grad():
            for l in e.layers:
                l.wqkv_t = self._tile(l.wqkv, 0, aux=e.nkv)
                l.wo_t = self._tile(l.wo, 1)
                l.wgu_t = self._tile(l.wgu, 2, aux=self.I)
                l.wd_t = self._tile(l.wd, 3)
            self.lm_t = self._tile(e.lm_head, 4)
        torch.cuda.synchronize(e.dev)

    def _counters(self):
        """The step's barrier and hand-off counters, one zeroed buffer shared by every state of
        this engine: each launch leaves them zero (a launch that timed out at a barrier may not;
        the engine then calls reset_counters), and the engine runs one launch at a time
        (launches that overlap in time must not share them). They live in uncached device
        memory allocated by the library (never freed), unless DD_UC_COUNTERS=0 asks for an
        ordinary zeroed tensor."""
        if self._ctr is None:
            if os.environ.get("DD_UC_COUNTERS", "1") != "0":
                ptr = ctypes.c_void_p()
                check(self.L.dd_step_counters_alloc(ctypes.byref(ptr)), "dd_step_counters_alloc")
                self._ctr = ptr.value
            else:
                self._ctr_t = torch.zeros(self.L.dd_step_counters(), dtype=torch.int32,
                                          device=self.e.dev)
                self._ctr = self._ctr_t.data_ptr()
        return self._ctr

    def reset_counters(self):
        """Zero the step's counters (synchronous): needed after a launch that set error flag 4
        (a grid barrier timed out), whose workgroups stopped waiting and may have left hand-off
        counters nonzero; every state of this engine shares them."""
        if self._ctr is not None:
            check(self.L.dd_step_counters_clear(self._ctr), "dd_step_counters_clear")

    def _tile(self, w, matrix, aux=0):
        N, K = w.shape
        out = torch.empty(self.L.dd_tiled_bytes(N, K) // 2, dtype=torch.bfloat16, device=w.device)
        check(self.L.dd_tile_weight(w.data_ptr(), out.data_ptr(), N, K, matrix, aux,
                                    _stream(w.device)), "dd_tile_weight")
        return out

    @staticmethod
    def qkv_natural(x, nh, nkv):
        """A head-grouped raw projection (last dim: per kv head its nh / nkv q heads, k, v; the
        step's qkv slot) in the reference's cat(q, k, v) column order."""
        g = nh // nkv
        t = x.unflatten(-1, (nkv, g + 2, HD))
        q = t[..., :g, :].flatten(-3)
        k = t[..., g, :].flatten(-2)
        v = t[..., g + 1, :].flatten(-2)
        return torch.cat([q, k, v], dim=-1)

    def supports(self, B, W):
        """Whether the one-launch step takes B sequences of W tokens for this model."""
        e = self.e
        return 1 <= B <= MAXB and 1 <= W <= MAXW and bool(
            self.L.dd_step_supported(e.L, self.H, e.nh, e.nkv, self.I, self.V, B, W))

    def bind(self, st):
        """Allocate the step's buffers for a state and build its layer table (the KV cache
        tensors of the state are baked in: one table per state)."""
        e, dev = self.e, self.e.dev
        B, W, H, I, V = st.B, st.W, self.H, self.I, self.V
        M = B * W
        bf = dict(dtype=torch.bfloat16, device=dev)
        f = _State()
        L = e.L
        # write-once activation slots (see dd_decode_step): h per producing phase, the others
        # per layer; h, attn and mbuf slots are k-step-major ([K/32][M][32]), qkv row-major and
        # head-grouped (qkv_natural)
        f.h = torch.empty(2 * L + 1, M, H, **bf)
        f.qkv = torch.empty(L, M, (e.nh + 2 * e.nkv) * HD, **bf)
        f.attn = torch.empty(L, M, e.nh * HD, **bf)
        f.mbuf = torch.empty(L, M, I, **bf)
        f.logits = torch.empty(M, V, **bf)
        ws = self.L.dd_step_ws_bytes(L, e.nh, e.nkv, W)
        if ws == 0:
            raise RuntimeError("dd_step_ws_bytes rejected the shape")
        f.ws = torch.empty(ws // 4, dtype=torch.float32, device=dev)
        f.counters_ptr = self._counters()
        f.err = st.err                       # the state's error word (next to its tokens)
        # the argmax of every row: a decode step writes it over its input tokens; a verify step
        # keeps its inputs (the drafts) and writes the argmax next to them
        f.otok = st.tok if W == 1 else torch.zeros(M, dtype=torch.long, device=dev)
        table = torch.zeros(e.L, NFIELD, dtype=torch.int64)
        for i, l in enumerate(e.layers):
            table[i, :10] = torch.tensor([
                l.wqkv_t.data_ptr(), l.wo_t.data_ptr(), l.wgu_t.data_ptr(), l.wd_t.data_ptr(),
                l.ln1.data_ptr(), l.ln2.data_ptr(), l.qn.data_ptr(), l.kn.data_ptr(),
                st.kc[i].data_ptr(), st.vc[i].data_ptr()], dtype=torch.int64)
        f.table = table.to(dev)
        st.fused = f

    def run(self, st, phase_begin=0, phase_end=None):
        """One step of the state. W == 1 (decode): st.tok <- argmax(logits(st.tok at st.pos)),
        st.pos += 1. W > 1 (verify): st.fused.otok <- the argmax of every row, positions kept.
        The logits stay in st.fused.logits."""
        e, f = self.e, st.fused
        if phase_end is None:
            phase_end = 2 + 5 * e.L
        check(self.L.dd_decode_step(
            f.table.data_ptr(), e.L, e.embed.data_ptr(), self.lm_t.data_ptr(), e.norm.data_ptr(),
            e.cos.data_ptr(), e.sin.data_ptr(), e.cos.shape[0], st.tok.data_ptr(),
            f.otok.data_ptr(), st.pos.data_ptr(), f.h.data_ptr(), f.qkv.data_ptr(),
            f.attn.data_ptr(), f.mbuf.data_ptr(), f.logits.data_ptr(), f.ws.data_ptr(),
            f.counters_ptr, f.err.data_ptr(), st.B, st.W, self.H, e.nh, e.nkv, self.I, self.V,
            st.cap, ctypes.c_float(e.eps), phase_begin, phase_end, _stream(e.dev)),
            "dd_decode_step")
        return f.logits


    def counters(self, st):
        """Host copy of a state's step counters (diagnostics: zero between steps)."""
        n = self.L.dd_step_counters()
        host = (ctypes.c_int * n)()
        check(self.L.dd_step_counters_read(st.fused.counters_ptr, host), "dd_step_counters_read")
        return list(host)

    def write_counters(self, st, values):
        """Overwrite a state's step counters from a host list (tests and diagnostics)."""
        n = self.L.dd_step_counters()
        host = (ctypes.c_int * n)(*values)
        check(self.L.dd_step_counters_write(st.fused.counters_ptr, host), "dd_step_counters_write")


class _State:
    pass
