"""Child process of test_no_alloc_first_call_under_capture: a fresh process whose FIRST
dd_attn_decode_noalloc call on the device is made under hipGraph capture (it must refuse, launch
nothing and leave the capture usable), then a call outside capture, then a captured call
replayed three times with eager work between the replays; every result compared bit for bit
with dd_attn_decode on caller workspaces. Prints one RESULT line."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def main():
    import torch
    import __graft_entry__
    __graft_entry__.load_package()
    from dryft_amd import _lib
    from test_zz_no_alloc import _inputs, _with_workspace
    L = _lib.lib()
    B, W, NH, NKV, cap = 4, 1, 32, 8, 1024
    q, kc, vc, pos = _inputs(B, W, NH, NKV, cap, seed=7)
    want = _with_workspace(L, q, kc, vc, pos, B, W, NH, NKV, cap)
    out = torch.zeros(B * W, NH * 128, dtype=torch.bfloat16, device="cuda")

    def call():
        return L.dd_attn_decode_noalloc(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(),
                                        1, out.data_ptr(), B, W, NH, NKV, 128, cap,
                                        torch.cuda.current_stream().cuda_stream)

    torch.cuda.synchronize()
    g0 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g0):
        rc_first = call()                      # refused: nothing recorded
    g0.replay()
    torch.cuda.synchronize()
    untouched = int(out.abs().sum().item() == 0)
    rc_eager = call()
    torch.cuda.synchronize()
    eager_ok = int(torch.equal(out.view(torch.int16), want.view(torch.int16)))
    out.zero_()
    g1 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1):
        rc_cap = call()
    replays_ok = 0
    for _ in range(3):
        out.zero_()
        _with_workspace(L, q, kc, vc, pos, B, W, NH, NKV, cap)     # eager work between replays
        g1.replay()
        torch.cuda.synchronize()
        replays_ok += int(torch.equal(out.view(torch.int16), want.view(torch.int16)))
    print(f"RESULT {rc_first} {untouched} {rc_eager} {eager_ok} {rc_cap} {replays_ok}", flush=True)


if __name__ == "__main__":
    main()
