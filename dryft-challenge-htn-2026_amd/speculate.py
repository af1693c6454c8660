"""In-graph speculative decoding with exact greedy acceptance.

The reference's gpu-mode speculation (engine/engine.py:862-1091: ``_gstate``, ``_gspec_body``,
``_generate_gspec``) drafts W - 1 tokens per sequence from a token-recycling table, verifies the
W rows in one multi-query forward and accepts, all inside one captured graph, so the host only
harvests results one step behind. Here a speculative step is three launches in one hipGraph:

  dd_spec_draft   rows[b] = (tok, T[tok], T[T[tok]], ...) at positions gpos[b] ..
  dd_decode_step  the verify-shaped step (W tokens per sequence, one launch): K/V written at
                  gpos[b] .. gpos[b] + W - 1 and out[b, j] = the argmax of row j
  dd_spec_accept  keep the longest prefix of drafts equal to the model's own argmax plus the
                  model's next token, recycle (row token -> argmax) into T, advance tok / gpos

Acceptance is exact greedy: the reference's margin acceptance (a draft within 1.25 logits of the
row's max, engine.py:923-929) is left out, so every emitted token is the verify forward's own
argmax. Sequences advance at their own pace (per-row positions; ragged prompts need no
grouping); the host yields a token row once every sequence has produced it.

Gate (engine.py:51, 61-64, 693-706): 1 <= B <= 8 and n >= 64, and the one-launch step must take
B x W rows; the engine turns speculation on only when ENGINE_SPEC=1 and the load-time check
(tokens identical to plain decode, engine.py:1057-1091) passes.
"""
import sys

import torch

from ._lib import check, lib

SPEC_W = 4            # verify rows per sequence: the last confirmed token and 3 drafts
SPEC_MAX_B = 8        # engine.py:51 (gpu-mode gate: 1 <= B <= 8)
SPEC_MIN_N = 64       # engine.py:51 (n >= 64)
CAP_GRAN = 128        # engine.py:24


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


class Speculator:
    """Speculative generation for one engine at one verify width W."""

    def __init__(self, eng, W=SPEC_W):
        if eng.step is None:
            raise RuntimeError("speculation needs the one-launch verify step")
        self.e = eng
        self.W = W
        self.L = lib()
        self.V = eng.embed.shape[0]

    def takes(self, B, n):
        return 1 <= B <= SPEC_MAX_B and n >= SPEC_MIN_N and self.e.step.supports(B, self.W)

    # ---------------------------------------------------------------- state
    def state(self, B, cap, graph=True):
        """engine.py:862-904: a W-wide state of the engine (KV cache, verify buffers) plus the
        table T [B, V] int32, the confirmed token / position per sequence, the position limits
        and the per-step record [out (B W) | accepted (B) | error word]."""
        e = self.e
        key = ("spec", B, cap, self.W, graph)
        st = e.states.get(key)
        if st is not None:
            return st
        st = e._new_state(B, cap, self.W)
        if st.fused is None:
            raise RuntimeError(f"the one-launch step does not take B={B} x W={self.W}")
        dev = e.dev
        st.T = torch.zeros(B, self.V, dtype=torch.int32, device=dev)
        st.gtok = torch.zeros(B, dtype=torch.long, device=dev)
        st.gpos = torch.zeros(B, dtype=torch.long, device=dev)
        st.limit = torch.zeros(B, dtype=torch.long, device=dev)
        st.rec = torch.zeros(B * self.W + B + 1, dtype=torch.long, device=dev)
        e._evict_for_new_state()
        e.states[key] = st
        if graph:
            try:
                self._capture(st)
            except Exception as ex:  # eager replays instead (engine.py:365-370 contract)
                print(f"[engine] speculative graph capture failed for {key}: {ex!r}",
                      file=sys.stderr)
                st.graph = None
        return st

    def body(self, st):
        """One speculative step (engine.py:889-943, exact acceptance)."""
        e, L, dev = self.e, self.L, self.e.dev
        B, W = st.B, self.W
        s = _stream(dev)
        check(L.dd_spec_draft(st.T.data_ptr(), self.V, st.gtok.data_ptr(), st.gpos.data_ptr(), B,
                              W, st.tok.data_ptr(), st.pos.data_ptr(), st.err.data_ptr(), s),
              "dd_spec_draft")
        e.step.run(st)
        check(L.dd_spec_accept(st.tok.data_ptr(), st.fused.otok.data_ptr(), st.T.data_ptr(),
                               self.V, B, W, st.gtok.data_ptr(), st.gpos.data_ptr(),
                               st.limit.data_ptr(), st.rec.data_ptr(), st.err.data_ptr(), s),
              "dd_spec_accept")

    def _capture(self, st):
        """engine.py:906-917: warm-ups on a side stream, then one step captured into the
        engine's pool. The warm-ups touch only the first W cache positions and the table, which
        every generate() re-seeds."""
        e = self.e
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):
                self.body(st)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=e.pool):
            self.body(st)
        st.graph = g
        torch.cuda.synchronize()

    # ---------------------------------------------------------------- generate
    def prepare(self, input_ids, n, graph=True):
        """Prefill the prompts into a W-wide state and seed its table (engine.py:945-976):
        T[b, prompt[i]] = prompt[i + 1], T[b, last prompt token] = first generated token.
        Returns (state, first tokens)."""
        e = self.e
        B = len(input_ids)
        lens = [len(x) for x in input_ids]
        cap = -(-(max(lens) + n + 2 * self.W) // CAP_GRAN) * CAP_GRAN
        if cap > e.cos.shape[0]:
            e._grow_rope(cap)
        st = self.state(B, cap, graph)
        e.recover(int(st.err.item()))              # a barrier timeout left by an earlier call
        e._clear_errors(st)
        e._prefill(input_ids, st)                  # first tokens in st.tok[:B]
        dev = e.dev
        st.gtok.copy_(st.tok[:B])
        st.gpos.copy_(torch.tensor(lens, dtype=torch.long))
        st.limit.copy_(torch.tensor([x + n - 1 for x in lens], dtype=torch.long))
        st.T.zero_()
        starts = [0]
        for x in lens:
            starts.append(starts[-1] + x)
        ids = torch.tensor([t for x in input_ids for t in x], dtype=torch.long, device=dev)
        seq_start = torch.tensor(starts, dtype=torch.int32, device=dev)
        check(self.L.dd_spec_seed(st.T.data_ptr(), self.V, ids.data_ptr(), seq_start.data_ptr(),
                                  B, st.gtok.data_ptr(), st.err.data_ptr(), _stream(dev)),
              "dd_spec_seed")
        flags = int(st.err.item())
        if flags:
            raise RuntimeError(f"speculative prefill reported error flags {flags:#x}")
        return st, st.gtok.tolist()

    def run(self, st, first, n, stats=None):
        """engine.py:977-1015: replay t + 1 is launched before step t's record is read; each
        sequence's stream is rebuilt from (out, accepted) and a token row is yielded once every
        sequence has it. ``stats``: optional dict that receives steps and accepted drafts."""
        B, W = st.B, self.W
        out = [[t] for t in first]
        yielded = 1
        yield list(first)
        if n <= 1:
            return
        max_steps = n - 1                           # every step confirms >= 1 token per row
        host = torch.empty((max_steps, st.rec.numel()), dtype=torch.long, pin_memory=True)
        ev = [torch.cuda.Event() for _ in range(max_steps)]

        def launch(t):
            if st.graph is not None:
                st.graph.replay()
            else:
                self.body(st)
            host[t].copy_(st.rec, non_blocking=True)
            ev[t].record()

        steps, accepted = 0, 0
        launch(0)
        t = 0
        while True:
            more = not all(len(x) >= n for x in out) and t + 1 < max_steps
            if more:
                launch(t + 1)
            ev[t].synchronize()
            row = host[t]
            flags = int(row[-1]) & 0xffffffff
            if flags:
                self.e.recover(flags)
                raise RuntimeError(f"speculative step {t} reported error flags {flags:#x}")
            o = row[:B * W].view(B, W).tolist()
            a = row[B * W:B * W + B].tolist()
            steps += 1
            for b in range(B):
                if len(out[b]) >= n:
                    continue
                take = min(a[b] + 1, n - len(out[b]))
                accepted += take - 1
                out[b] += o[b][:take]
            m = min(len(x) for x in out)
            while yielded < m:
                yield [out[b][yielded] for b in range(B)]
                yielded += 1
            if yielded >= n or not more:
                break
            t += 1
        if stats is not None:
            stats["steps"] = steps
            stats["accepted_drafts"] = accepted

    def generate(self, input_ids, n, graph=True, stats=None):
        if n <= 0:
            return
        st, first = self.prepare(input_ids, n, graph)
        yield from self.run(st, first, n, stats)
