"""dd_attn_decode_noalloc (the entry point that allocates nothing: split partials and counters in
a static device array) against dd_attn_decode with caller workspaces, through the C ABI.

Both launch the same kernel with the same key chunk, so the outputs must be identical bits. The
calls come in a row on one stream, the second with a smaller input than the first and the third
larger again, so each call starts from the array contents the previous one left."""
import pytest
import torch

from dryft_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(B, W, NH, NKV, cap, seed):
    G = NH // NKV
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(B, NKV, W, G, 128, generator=g, device="cuda").to(torch.bfloat16)
    kc = torch.randn(B, NKV, cap, 128, generator=g, device="cuda").to(torch.bfloat16)
    vc = torch.randn(B, NKV, cap, 128, generator=g, device="cuda").to(torch.bfloat16)
    pos = torch.randint(0, cap - W + 1, (B,), generator=g, device="cuda")
    return q, kc, vc, pos


def _with_workspace(L, q, kc, vc, pos, B, W, NH, NKV, cap):
    chunk = L.dd_attn_chunk(B, NKV, cap)
    ws = torch.empty(max(1, L.dd_attn_ws_bytes(B, W, NH, NKV, 128, cap, chunk) // 4),
                     dtype=torch.float32, device="cuda")
    counters = torch.zeros(B * NKV, dtype=torch.int32, device="cuda")
    out = torch.empty(B * W, NH * 128, dtype=torch.bfloat16, device="cuda")
    _lib.check(L.dd_attn_decode(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(), 1,
                                out.data_ptr(), ws.data_ptr(), counters.data_ptr(), B, W, NH, NKV,
                                128, cap, chunk, torch.cuda.current_stream().cuda_stream),
               "dd_attn_decode")
    return out


def _no_alloc(L, q, kc, vc, pos, B, W, NH, NKV, cap):
    out = torch.empty(B * W, NH * 128, dtype=torch.bfloat16, device="cuda")
    _lib.check(L.dd_attn_decode_noalloc(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(),
                                        1, out.data_ptr(), B, W, NH, NKV, 128, cap,
                                        torch.cuda.current_stream().cuda_stream),
               "dd_attn_decode_noalloc")
    return out


@pytest.mark.parametrize("shapes", [[(16, 5, 32, 8, 2048), (3, 1, 32, 8, 640), (16, 1, 32, 8, 8192)]])
def test_no_alloc_attention_matches_workspace_entry_point(cuda, shapes):
    L = _lib.lib()
    for i, (B, W, NH, NKV, cap) in enumerate(shapes):
        print(f"[no-alloc] call {i}: B={B} W={W} NH={NH} NKV={NKV} cap={cap}", flush=True)
        q, kc, vc, pos = _inputs(B, W, NH, NKV, cap, seed=i + 1)
        want = _with_workspace(L, q, kc, vc, pos, B, W, NH, NKV, cap)
        got = _no_alloc(L, q, kc, vc, pos, B, W, NH, NKV, cap)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (B, W, cap)


def test_no_alloc_first_call_under_capture(cuda):
    """A fresh process whose first no-allocation call is made under graph capture: the call is
    refused (hipErrorStreamCaptureUnsupported, 900) and records nothing; afterwards a call
    outside capture, then the same call captured and replayed three times (eager work between
    the replays), each equal bit for bit to dd_attn_decode with workspaces."""
    import os
    import subprocess
    import sys
    child = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_capture.py")
    print("[no-alloc] first call under capture (child process)", flush=True)
    r = subprocess.run([sys.executable, child], capture_output=True, text=True, timeout=300)
    line = [x for x in r.stdout.splitlines() if x.startswith("RESULT ")]
    assert r.returncode == 0 and line, r.stderr[-2000:]
    rc_first, untouched, rc_eager, eager_ok, rc_cap, replays_ok = map(int, line[0].split()[1:])
    assert rc_first == 900 and untouched == 1
    assert rc_eager == 0 and eager_ok == 1
    assert rc_cap == 0 and replays_ok == 3
