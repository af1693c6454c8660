"""Decode-step benchmark on one MI355X.

Workload: the full 36-layer Qwen3-4B-shape model with seeded
random-init bf16 weights (N(0, 0.02), norms 1 + N(0, 0.02), tied lm_head, vocab 151936),
B = 16 sequences with ragged prompt lengths U[64, 2048] (token ids uniform over the vocab),
greedy decode of 1024 tokens per sequence. A "step" is one hipGraph replay of the whole decode
step (all 16 rows, one weight pass, one persistent kernel launch).

Timed window: W warm-up steps, then exactly K timed steps. The window is placed at the middle of
the 1024-token generation whatever K and W are: each prompt is extended by
e = round(512 - W - (K + 1) / 2) further uniform ids (or shortened by -e when e < 0) before the
untimed prefill, so the K timed steps attend on average prompt + 512 keys per row -- the mean
context of configs[4]'s whole generation. Every step's tokens are recorded (one 128-byte copy per
step, inside the timed region) and afterwards checked with the reference benchmark's gate: an
independent torch path (hipBLASLt + SDPA, teacher-forced over prompt + emitted tokens) must put
every emitted token within 2.0 logits of its maximum (teacher.py).

One JSON line is printed with the contract fields plus
  roofline      the dominant kernel -- the one-launch decode step kernel, which is the whole
                step -- timed live with HIP events over the timed replays: algorithmic bytes
                (weights + attended K/V + new K/V + embedding rows) / average step time;
                ``traffic`` is the HBM bytes per launch measured with rocprofv3 --pmc on this
                same command (FETCH_SIZE + WRITE_SIZE, copy-kernel calibrated), reported with
                the algorithmic bytes of the profiled window it was measured against;
  cpu_baseline  the CPU oracle (this repo's restatement of the reference's torch path) timed on
                the host on a bounded sample: B=1 decode steps of the same 36-layer model at the
                window's mean context (the reference decodes ragged batches as independent
                B=1 streams, so its throughput is 1 token per B=1 step);
  extra         whole-step HBM accounting (bytes/step, achieved GB/s, fraction of the measured
                streaming-read ceiling and of the 8 TB/s spec), the B=1 configs[3] figure, the
                W=5 verify step, and the configs[1] / configs[2] microbenchmarks.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

SPEC_BW = 8.0e12          # MI355X HBM3E peak, B/s
KV_BYTES_TOKEN = 147456   # 36 layers x 2 (K, V) x 8 kv heads x 128 x 2 bytes


def weight_bytes(cfg):
    H, I, V, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"], cfg["num_hidden_layers"]
    nh, nkv, hd = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
    per_layer = ((nh + 2 * nkv) * hd * H + H * nh * hd + 2 * I * H + H * I) * 2
    return L * per_layer + V * H * 2


def measure_read_bw(torch, L, nbytes=4 << 30):
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    buf.fill_(1)
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    best = 0.0
    for grid, block in ((256, 512), (512, 256), (512, 512), (1024, 512), (2048, 256), (4096, 512)):
        for _ in range(2):
            L.dd_stream_read(buf.data_ptr(), nbytes, grid, block, sink.data_ptr(), st)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            L.dd_stream_read(buf.data_ptr(), nbytes, grid, block, sink.data_ptr(), st)
        e1.record()
        e1.synchronize()
        best = max(best, 5 * nbytes / (e0.elapsed_time(e1) * 1e-3))
    del buf
    return best


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_step_kernel_b16_configs4_traffic.json")


def measured_traffic(algo_bytes):
    """HBM bytes per launch of the step kernel from the committed rocprofv3 --pmc runs of this
    bench command (FETCH_SIZE + WRITE_SIZE per timed dispatch, scaled by the copy-kernel
    calibration), with the algorithmic bytes of the window those dispatches covered. Returns
    (bytes, basis algorithmic bytes), or (None, None) when the file is absent or was measured on
    a window whose algorithmic bytes differ from this run's by more than 0.5%."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        scale = t["copy_calibration"]["scale"] * 1024
        basis = float(t["algo_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None, None
    if abs(basis - algo_bytes) > 0.005 * algo_bytes:
        return None, basis
    return int((t["fetch_kib_per_dispatch"] + t["write_kib_per_dispatch"]) * scale), int(basis)


def step_roofline(ms, bytes_step, B):
    """The dominant (and only) kernel of a decode step is the one-launch step kernel: the timed
    region is K graph replays of one launch each, timed with HIP events on the stream they run
    on. Algorithmic bytes per launch: every weight matrix once (36 x [wqkv, wo, wgu, wd] +
    lm_head), the K/V cache rows each sequence attends (pos[b] + 1 per row), the new K/V rows,
    the embedding rows gathered; activations are a few MB and left out."""
    avg_s = ms * 1e-3
    traffic, basis = measured_traffic(bytes_step)
    return {"kernel": "dd::st::decode_step_kernel (whole decode step, one launch)",
            "bound": "hbm", "achieved": round(bytes_step / avg_s / 1e9, 1),
            "peak": SPEC_BW / 1e9, "unit": "GB/s", "frac": round(bytes_step / avg_s / SPEC_BW, 4),
            "traffic": traffic,
            "traffic_basis_algo_bytes": basis,
            "traffic_over_algo": round(traffic / basis, 4) if traffic else None,
            "avg_launch_us": round(avg_s * 1e6, 2),
            "algo_bytes_per_launch": int(bytes_step), "rows": B}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(torch, cfg, weights_gpu, mean_ctx, budget_s=20.0):
    """B=1 decode steps of the CPU oracle on the full model at the workload's mean context."""
    from oracle.reference import OracleEngine
    # the host's CPU share: OMP_NUM_THREADS when the environment sets it, else every core
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    w = {k: v.cpu() for k, v in weights_gpu.items()}
    ref = OracleEngine.from_state_dict(cfg, w)
    del w
    cap = -(-(mean_ctx + 64) // 128) * 128   # room for the timed steps (at most 21 positions)
    st = ref.new_state(1, cap)
    g = torch.Generator().manual_seed(0)
    for k, v in zip(st.kc, st.vc):            # a filled cache: timing does not depend on values
        k[:, :, :mean_ctx].copy_(torch.randn(k[:, :, :mean_ctx].shape, generator=g))
        v[:, :, :mean_ctx].copy_(torch.randn(v[:, :, :mean_ctx].shape, generator=g))
    st.pos.fill_(mean_ctx)
    st.tok.fill_(1)
    with torch.inference_mode():
        ref.decode_step(st)                   # warm-up
        t0 = time.perf_counter()
        n = 0
        while n < 3 or (time.perf_counter() - t0 < budget_s and n < 20):
            ref.decode_step(st)
            n += 1
            if time.perf_counter() - t0 > budget_s:
                break
        dt = (time.perf_counter() - t0) / n
    return {"value": round(1.0 / dt, 3), "unit": "tok/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{n} B=1 decode steps of the 36-layer model at context {mean_ctx} "
                      f"(mean context of the workload), {dt * 1e3:.0f} ms/step; the reference "
                      f"decodes ragged batches as independent B=1 streams (1 token per step)",
            "ms_per_step": round(dt * 1e3, 1), "host_cpus": os.cpu_count(),
            "cpu_model": cpu_model()}


def window_prompts(torch, prompts, warmup, steps, gen_len, vocab, seed):
    """Extend (or shorten) every prompt so that the K timed steps after W warm-up steps attend,
    on average, prompt + gen_len / 2 keys: the mean context of the whole generation."""
    e = int(round(gen_len / 2 - warmup - (steps + 1) / 2))
    g = torch.Generator().manual_seed(seed)
    out = []
    for p in prompts:
        if e >= 0:
            out.append(list(p) + torch.randint(0, vocab, (e,), generator=g).tolist())
        else:
            out.append(list(p)[:max(1, len(p) + e)])
    return out, e


def run_decode(torch, eng, prompts, warmup, steps):
    """Prefill, W warm-up replays, then K timed replays, recording every step's tokens.
    Returns (ms/step, algorithmic bytes/step, mean attended context, tokens [W+K+1][B])."""
    B = len(prompts)
    n = warmup + steps + 1
    S = max(len(p) for p in prompts)
    cap = -(-(S + n) // 128) * 128
    st = eng._state(B, cap, graph=True)
    assert st.graph is not None, "decode graph capture failed"
    assert st.fused is not None, "the one-launch decode step is not bound to this state"
    st.err.zero_()
    eng._prefill(prompts, st)
    hist = torch.empty((n, B), dtype=torch.long, device=st.tok.device)
    hist[0].copy_(st.tok)
    for i in range(warmup):
        st.graph.replay()
        hist[1 + i].copy_(st.tok)
    torch.cuda.synchronize()
    pos0 = st.pos.clone().cpu()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for i in range(steps):
        st.graph.replay()
        hist[1 + warmup + i].copy_(st.tok)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flags = int(st.err.item())
    assert flags == 0, f"kernel error flags {flags:#x}"
    # attended context of timed step t (1-based) for row b: pos0[b] + t keys
    ctx_sum = sum(int(p) * steps + steps * (steps + 1) // 2 for p in pos0)
    wb = weight_bytes(eng.cfg)
    H = eng.cfg["hidden_size"]
    bytes_step = wb + KV_BYTES_TOKEN * (ctx_sum / steps) + KV_BYTES_TOKEN * B + B * H * 2
    mean_ctx = ctx_sum / steps / B
    return ms, bytes_step, mean_ctx, hist.cpu().tolist()


def run_verify(torch, eng, prompts, W=5, steps=20):
    """configs[4]'s verify-shaped step: B rows x W tokens (1 + 4 draft ids) at per-row start
    positions through Engine.verify_logits (the reference's multi-query forward,
    engine.py:542-547), captured in a hipGraph and replayed; returns (ms/step, bytes/step)."""
    B = len(prompts)
    S = max(len(p) for p in prompts)
    cap = -(-(S + W + 1) // 128) * 128
    st = eng._new_state(B, cap, W=W)
    eng._prefill(prompts, st)
    g = torch.Generator().manual_seed(1)
    drafts = torch.randint(0, eng.cfg["vocab_size"], (B, W), generator=g).cuda()
    spos = torch.tensor([len(p) for p in prompts], dtype=torch.long).cuda()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            eng.verify_logits(st, drafts, spos)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        eng.verify_logits(st, drafts, spos)
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    ctx = sum(len(p) + W for p in prompts)
    bytes_step = weight_bytes(eng.cfg) + KV_BYTES_TOKEN * ctx + KV_BYTES_TOKEN * B * W
    del graph, st
    torch.cuda.empty_cache()
    return ms, bytes_step


def run_spec(torch, eng, prompts, n, W):
    """End-to-end generate() of n tokens (prefill included, host loop included), plain greedy
    decode vs in-graph speculation at verify width W; each timed after one untimed warm-up
    call. Returns (plain s, speculative s, verify steps, accepted drafts, plain tokens,
    speculative tokens)."""
    sp = eng.speculator(W)

    def timed(fn):
        list(fn())                                            # warm-up: states, graphs
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        toks = list(fn())
        torch.cuda.synchronize()
        return time.perf_counter() - t0, toks

    tp, plain = timed(lambda: eng.generate(prompts, n))
    stats = {}
    ts, spec = timed(lambda: sp.generate(prompts, n, stats=stats))
    return tp, ts, stats["steps"], stats["accepted_drafts"], plain, spec


def run_prefill(torch, eng, prompts, reps=3, first=None):
    """The prompt pass of configs[4]'s ragged batch: every prompt prefilled in one packed pass
    (GEMMs over all prompt tokens, per-prompt causal attention). Returns (ms, prompt tokens);
    with a dict `first`, also the untimed warm-up's own time (the first pass of these lengths in
    the process: host-side GEMM descriptors are created then) in first["ms"]."""
    import time as _t
    B = len(prompts)
    cap = -(-max(len(p) for p in prompts) // 128) * 128
    st = eng._new_state(B, cap)
    torch.cuda.synchronize()
    t0 = _t.time()
    eng._prefill(prompts, st)                                 # warm-up (allocator, GEMM plans)
    torch.cuda.synchronize()
    if first is not None:
        first["ms"] = (_t.time() - t0) * 1e3
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        eng._prefill(prompts, st)
    e1.record()
    torch.cuda.synchronize()
    assert int(st.err.item()) == 0
    del st
    torch.cuda.empty_cache()
    return e0.elapsed_time(e1) / reps, sum(len(p) for p in prompts)


def _time(torch, fn, reps):
    for _ in range(3):
        fn()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / reps * 1e-3


def micro_gemv(torch, eng):
    """the per-op skinny GEMV kernel (dd_gemv, MFMA, in-launch split-K) at the five
    Qwen3-4B projection shapes and M in {1, 4, 8, 16}; bf16 weights N(0, 0.02), x N(0, 1).
    Bytes per launch = N K 2 + M K 2 + M N 2. `us` / `GBps`: the op as generation runs it, inside
    a captured hipGraph (10 calls per graph, replayed; GPU time per call). `us_eager`: the same
    op called from Python, which the host's per-call work (two tensor allocations, the ctypes
    call) bounds at ~12 us whatever the shape."""
    ops = eng.ops.f if hasattr(eng.ops, "f") else eng.ops
    H, I, V = eng.cfg["hidden_size"], eng.cfg["intermediate_size"], eng.cfg["vocab_size"]
    shapes = {"qkv": ((eng.nh + 2 * eng.nkv) * eng.hd, H), "o": (H, eng.nh * eng.hd),
              "gate_up": (2 * I, H), "down": (H, I), "lm_head": (V, H)}
    g = torch.Generator(device="cuda").manual_seed(11)
    out = {}
    per_graph = 10
    for name, (N, K) in shapes.items():
        w = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
        row = {}
        for M in (1, 4, 8, 16):
            x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
            te = _time(torch, lambda: ops.linear(x, w), 20 if N < 100000 else 5)
            ref = ops.linear(x, w)
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                ops.linear(x, w)                      # workspace and counters outside capture
            torch.cuda.current_stream().wait_stream(side)
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                ys = [ops.linear(x, w) for _ in range(per_graph)]
            tg = _time(torch, gr.replay, 5 if N < 100000 else 2) / per_graph
            assert all(torch.equal(y, ref) for y in ys), f"graph replay differs from eager: {name} M={M}"
            nb = N * K * 2 + M * K * 2 + M * N * 2
            row[f"M{M}"] = {"us": round(tg * 1e6, 2), "GBps": round(nb / tg / 1e9, 1),
                            "us_eager": round(te * 1e6, 2)}
            del gr, ys
        out[name] = row
        del w
    return out


def micro_kv_layout(torch, L, lens, nkv=8, hd=128):
    """The KV-cache layout check: K and V rows 0 .. len_b - 1 of a [B, 8, cap, 128] bf16 cache
    (configs[4]'s window lengths) read one 32-key block per wave with the decode attention's
    access pattern (K as MFMA A operands: 16 keys x 64 bytes per wave load) and with 1 KB
    contiguous wave loads (dd_kv_read modes 0 and 1, same bytes). Equal rates mean the
    reference's [B, NKV, cap, 128] layout already streams at the contiguous rate."""
    B = len(lens)
    cap = -(-max(lens) // 128) * 128
    g = torch.Generator(device="cuda").manual_seed(3)
    kc = torch.randn(B, nkv, cap, hd, generator=g, device="cuda").to(torch.bfloat16)
    vc = torch.randn(B, nkv, cap, hd, generator=g, device="cuda").to(torch.bfloat16)
    ln = torch.tensor(lens, dtype=torch.long, device="cuda")
    nbytes = sum(-(-n // 32) * 32 for n in lens) * nkv * hd * 2 * 2
    s = torch.cuda.current_stream().cuda_stream
    out = {"bytes": nbytes}
    for mode, name in ((0, "attention_pattern"), (1, "contiguous_1KB")):
        t = _time(torch, lambda: L.dd_kv_read(kc.data_ptr(), vc.data_ptr(), ln.data_ptr(), B, nkv,
                                              cap, mode, None, s), 20)
        out[name + "_GBps"] = round(nbytes / t / 1e9, 1)
    del kc, vc
    torch.cuda.empty_cache()
    return out


def micro_attention(torch, cfg, synth, Engine, seed=0):
    """fused RoPE + q/k RMSNorm + K/V write followed by split-KV GQA attention at
    B=16 with ragged KV lengths U[512, 8192] (seeded), cache capacity 8192, q|k|v and cached K/V
    N(0, 1); one layer at Qwen3-4B widths. Times (a) the per-op pair dd_qkv_post_decode +
    dd_attn_decode and (b) the attention phase of the one-launch step run on its own
    (phase_begin = 2, phase_end = 3). Bytes per layer = 4,096 sum(ctx) (K/V read) + new K/V +
    q|k|v in + attention out."""
    c1 = synth.qwen3_config(num_hidden_layers=1, vocab_size=8192)
    w = synth.random_weights(c1, seed=seed, device="cuda")
    eng = Engine.from_state_dict(c1, w, selftest=False)
    B, cap = 16, 8192
    g = torch.Generator().manual_seed(seed + 1)
    ctx = torch.randint(512, 8193, (B,), generator=g)
    gd = torch.Generator(device="cuda").manual_seed(seed + 2)
    st = eng._new_state(B, cap)
    for c in (st.kc[0], st.vc[0]):
        c.copy_(torch.randn(c.shape, generator=gd, device="cuda").to(torch.bfloat16))
    pos = (ctx - 1).cuda()
    st.pos.copy_(pos)
    nqkv = (eng.nh + 2 * eng.nkv) * eng.hd
    qkv = torch.randn(B, nqkv, generator=gd, device="cuda").to(torch.bfloat16)
    ops, l = eng.ops, eng.layers[0]
    nbytes = 4096 * int(ctx.sum()) + B * (nqkv * 2 + eng.nh * eng.hd * 2)

    def per_op():
        q = ops.qkv_post(qkv, l, st.kc[0], st.vc[0], B, 1, st.pos)
        ops.attn_decode(q, st.kc[0], st.vc[0], st.pos, 1)
    t_op = _time(torch, per_op, 20)
    f = st.fused
    f.qkv[0].copy_(qkv)                          # the step's raw q|k|v slot (head-grouped)

    def phase():
        eng.step.run(st, 2, 3)
    st.pos.copy_(pos)
    t_ph = _time(torch, phase, 20)
    flags = int(st.err.item())
    del eng, st
    torch.cuda.empty_cache()
    return {"B": B, "cap": cap, "ctx_sum": int(ctx.sum()), "ctx_min": int(ctx.min()),
            "ctx_max": int(ctx.max()), "bytes_per_layer": nbytes, "error_flags": flags,
            "per_op_us_per_layer": round(t_op * 1e6, 2),
            "per_op_GBps": round(nbytes / t_op / 1e9, 1),
            "fused_phase_us_per_layer": round(t_ph * 1e6, 2),
            "fused_phase_GBps": round(nbytes / t_ph / 1e9, 1)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=23)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-b1", action="store_true")
    ap.add_argument("--no-verify", action="store_true")
    ap.add_argument("--no-micro", action="store_true")
    ap.add_argument("--no-check", action="store_true")
    ap.add_argument("--no-spec", action="store_true")
    ap.add_argument("--no-fp8", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the decode step is "
              "not sharded across GPUs in this build.", file=sys.stderr)
        sys.exit(2)

    import torch
    import __graft_entry__
    __graft_entry__.load_package()
    from dryft_amd import synth
    from dryft_amd.engine import Engine
    from dryft_amd.teacher import gap_check

    t0 = time.time()
    cfg = synth.qwen3_config(num_hidden_layers=args.layers)
    weights = synth.random_weights(cfg, seed=0, device="cuda")
    eng = Engine.from_state_dict(cfg, dict(weights), selftest=True)
    print(f"[bench] model ready in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    L = eng.ops.L

    read_bw = measure_read_bw(torch, L)
    print(f"[bench] streaming-read ceiling {read_bw / 1e9:.0f} GB/s", file=sys.stderr, flush=True)

    g = torch.Generator().manual_seed(0)
    B = args.batch
    V = cfg["vocab_size"]
    lens = torch.randint(64, 2049, (B,), generator=g).tolist()
    prompts = [torch.randint(0, V, (n,), generator=g).tolist() for n in lens]
    wprompts, ext = window_prompts(torch, prompts, args.warmup, args.steps, 1024, V, seed=5)
    ms, bytes_step, mean_ctx, toks = run_decode(torch, eng, wprompts, args.warmup, args.steps)
    tok_s = B / (ms * 1e-3)
    achieved = bytes_step / (ms * 1e-3)
    gen_mean = sum(lens) / B + 512
    print(f"[bench] B={B}: {ms:.3f} ms/step, {tok_s:.0f} tok/s, {achieved / 1e9:.0f} GB/s "
          f"({achieved / read_bw * 100:.1f}% of measured, {achieved / SPEC_BW * 100:.1f}% of spec); "
          f"window mean context {mean_ctx:.1f} (generation mean {gen_mean:.1f})",
          file=sys.stderr, flush=True)

    extra = {"bytes_per_step": int(bytes_step), "step_achieved_GBps": round(achieved / 1e9, 1),
             "measured_read_GBps": round(read_bw / 1e9, 1),
             "frac_of_measured": round(achieved / read_bw, 4),
             "frac_of_spec": round(achieved / SPEC_BW, 4),
             "prompt_lens": lens, "prompt_extension": ext,
             "window_mean_context": round(mean_ctx, 1),
             "generation_mean_context": round(gen_mean, 1)}

    if not args.no_check:                     # the reference bench's gate on every token
        t1 = time.time()
        worst, bad, n = gap_check(eng, wprompts, toks)
        extra["gap_check"] = {"tokens": n, "worst_gap": round(worst, 4), "over_2": bad,
                              "path": "teacher-forced torch (hipBLASLt + SDPA) over prompt + "
                                      "emitted tokens, warm-up and timed steps"}
        print(f"[bench] gap check: {n} tokens, worst gap {worst:.3f}, over 2.0: {bad} "
              f"({time.time() - t1:.1f}s)", file=sys.stderr, flush=True)
        assert bad == 0, f"{bad} emitted tokens exceed the 2-logit gap"

    if not args.no_b1:                        # configs[3]: B=1, prompt 128, 512 generated
        p1 = [torch.randint(0, V, (128,), generator=g).tolist()]
        w1, _ = window_prompts(torch, p1, 10, 500, 512, V, seed=6)
        ms1, bytes1, ctx1, toks1 = run_decode(torch, eng, w1, 10, 500)
        extra["b1"] = {"ms_per_step": round(ms1, 4), "tok_s": round(1e3 / ms1, 1),
                       "step_achieved_GBps": round(bytes1 / (ms1 * 1e-3) / 1e9, 1),
                       "frac_of_measured": round(bytes1 / (ms1 * 1e-3) / read_bw, 4),
                       "window_mean_context": round(ctx1, 1)}
        if not args.no_check:
            worst1, bad1, n1 = gap_check(eng, w1, toks1)
            extra["b1"]["gap_check"] = {"tokens": n1, "worst_gap": round(worst1, 4), "over_2": bad1}
            assert bad1 == 0, f"B=1: {bad1} emitted tokens exceed the 2-logit gap"
            # greedy identity against the reference's torch arithmetic (untimed replay of the
            # same generation keeping every step's logits; its tokens must be the timed run's)
            from dryft_amd.teacher import decode_trace, token_identity
            tr_toks, tr_logits = decode_trace(eng, w1, len(toks1))
            assert [x[0] for x in tr_toks] == [x[0] for x in toks1], "replay differs from timed run"
            ident = token_identity(eng, w1[0], [x[0] for x in toks1], tr_logits[:, 0])
            del tr_logits
            extra["b1"]["token_identity"] = dict(ident, path="vs the reference's torch arithmetic "
                                                 "(hipBLASLt + SDPA) teacher-forced on prompt + "
                                                 "emitted tokens; first_flip = first step off that "
                                                 "path's own greedy run")
            print(f"[bench] B=1 token identity: {ident['flips']} flips of {ident['tokens']} "
                  f"(first {ident['first_flip']}), all near-ties {ident['all_near_ties']}, "
                  f"worst logit diff {ident['worst_logit_diff']}", file=sys.stderr, flush=True)
        print(f"[bench] B=1: {ms1:.3f} ms/step, {1e3 / ms1:.0f} tok/s", file=sys.stderr, flush=True)

    if not args.no_verify:                    # configs[4] verify shape: W = 5 per row
        msv, bytesv = run_verify(torch, eng, prompts)
        extra["verify_w5"] = {"ms_per_step": round(msv, 4), "tokens_per_step": B * 5,
                              "tok_s": round(B * 5 / (msv * 1e-3), 1),
                              "step_achieved_GBps": round(bytesv / (msv * 1e-3) / 1e9, 1),
                              "path": "one-launch step kernel, verify instantiation "
                                      "(B x W = 80 query rows), hipGraph"}
        print(f"[bench] verify B={B} W=5: {msv:.3f} ms/step", file=sys.stderr, flush=True)

    if not args.no_spec:                      # in-graph speculation, configs[3]'s B=1 shape
        p1 = [torch.randint(0, V, (128,), generator=g).tolist()]
        tp, ts, nsteps, nacc, plain_t, spec_t = run_spec(torch, eng, p1, 512, 4)
        same = plain_t == spec_t
        div = None
        if not same:
            from dryft_amd.teacher import decode_trace, first_divergence_check
            tr_toks, tr_logits = decode_trace(eng, p1, 512)
            assert [x[0] for x in tr_toks] == [x[0] for x in plain_t]
            div = first_divergence_check(eng, p1[0], [x[0] for x in plain_t], tr_logits[:, 0],
                                         [x[0] for x in spec_t])
            del tr_logits
        extra["speculative_b1"] = {
            "tokens": 512, "W": 4, "plain_tok_s": round(512 / tp, 1),
            "spec_tok_s": round(512 / ts, 1), "verify_steps": nsteps,
            "accepted_drafts": nacc, "identical_to_plain": same, "first_divergence": div,
            "note": "end-to-end generate() incl. prefill; random-init weights and prompt ids, so "
                    "acceptance reflects this synthetic model's repetition, not natural text. "
                    "first_divergence: the first step where the speculative stream leaves the "
                    "plain one, with both tokens' distance below the torch path's maximum there "
                    "and the measured engine-vs-torch logit noise (near_tie: both within it)"}
        if div is not None:
            print(f"[bench] speculative stream leaves plain at step {div['step']}: "
                  f"near_tie={div['near_tie']} (gaps {div['gap_plain']} / {div['gap_other']}, "
                  f"noise {div['noise']})", file=sys.stderr, flush=True)
        print(f"[bench] speculative B=1 W=4: plain {512 / tp:.0f} tok/s, speculative "
              f"{512 / ts:.0f} tok/s ({nsteps} verify steps, {nacc} accepted drafts, "
              f"identical={same})", file=sys.stderr, flush=True)

    if not args.no_fp8:                       # opt-in fp8 prefill GEMMs (B <= 8)
        # The fp8 GEMMs take a packed row count that is a multiple of 16 (the reference's
        # _fp8_lin, engine.py:451-457, runs bf16 otherwise), so the last prompt is shortened by
        # the remainder: both legs then time the same 16k-row batch.
        p8 = [list(p) for p in prompts[:8]]
        p8[-1] = p8[-1][:len(p8[-1]) - sum(len(p) for p in p8) % 16]
        ms_bf, n8 = run_prefill(torch, eng, p8)
        eng._quantize_fp8()
        eng.fp8 = True
        ms_f8, _ = run_prefill(torch, eng, p8)
        eng.fp8 = False
        for l in eng.layers:
            del l.wqkv8, l.wqkv8s, l.wgu8, l.wgu8s
        torch.cuda.empty_cache()
        extra["prefill_fp8_b8"] = {"prompt_tokens": n8, "bf16_ms": round(ms_bf, 2),
                                   "fp8_ms": round(ms_f8, 2),
                                   "path": "first 8 configs[4] prompts, one packed pass; fp8 "
                                           "(e4m3, tensorwise) QKV and gate/up GEMMs on hipBLASLt "
                                           "after the HIP quantisation kernel (opt-in)"}
        print(f"[bench] prefill B=8 ({n8} tokens): bf16 {ms_bf:.1f} ms, fp8 {ms_f8:.1f} ms",
              file=sys.stderr, flush=True)

    # the same pass with every GEMM on F.linear (hipBLASLt's heuristic choice), then as built
    # (each prefill GEMM on the hipBLASLt solution the committed table names for its shape)
    os.environ["DD_TUNED_GEMM"] = "0"
    msp0, _ = run_prefill(torch, eng, prompts)
    os.environ.pop("DD_TUNED_GEMM")
    first = {}
    msp, ntok = run_prefill(torch, eng, prompts, first=first)
    from dryft_amd.hipops import gemm_solution
    ops = eng.ops.f if hasattr(eng.ops, "f") else eng.ops
    table = getattr(ops, "_gemm_table", {})
    H, I = cfg["hidden_size"], cfg["intermediate_size"]
    gshapes = {"qkv": ((eng.nh + 2 * eng.nkv) * eng.hd, H), "o": (H, eng.nh * eng.hd),
               "gate_up": (2 * I, H), "down": (H, I)}
    extra["prefill"] = {"prompt_tokens": ntok, "ms": round(msp, 2),
                        "tok_s": round(ntok / (msp * 1e-3), 1),
                        "first_pass_ms": round(first["ms"], 2),
                        "ms_gemms_on_f_linear": round(msp0, 2),
                        "gemm_solutions": {f"{k} {n}x{kk} rows={ntok}": gemm_solution(table, n, kk, ntok)
                                           for k, (n, kk) in gshapes.items()},
                        "path": "one packed pass over the 16 ragged prompts: hipBLASLt GEMMs "
                                "(the committed table's solution per shape, fixed per process), "
                                "HIP RMSNorm / q-k norm + RoPE + K/V write / causal flash "
                                "attention kernels"}
    print(f"[bench] prefill {ntok} prompt tokens: {msp:.1f} ms (first pass {first['ms']:.1f} ms; "
          f"GEMMs on F.linear: {msp0:.1f} ms)", file=sys.stderr, flush=True)

    if not args.no_micro:
        extra["kv_layout"] = micro_kv_layout(torch, L, [n + 512 for n in lens])
        print(f"[bench] KV layout {extra['kv_layout']}", file=sys.stderr, flush=True)
        try:                                  # the product's GEMV phases, profiled alone
            with open(os.path.join(ROOT, "profiles", "configs1_fused_phases.json")) as f:
                extra["configs1"] = dict(json.load(f)["phases"],
                                         source="profiles/configs1_fused_phases.json (rocprofv3 "
                                                "kernel trace of phase_bench.py: each phase of the "
                                                "one-launch step launched alone)")
        except (OSError, ValueError, KeyError):
            extra["configs1"] = None
        extra["configs1_per_op_gemv"] = dict(micro_gemv(torch, eng),
                                             path="dd_gemv, the per-op fallback for B > 16 and "
                                                  "geometries the one-launch step does not take")
        print(f"[bench] configs[1] per-op dd_gemv {extra['configs1_per_op_gemv']}", file=sys.stderr,
              flush=True)

    roof = step_roofline(ms, bytes_step, B)
    print(f"[bench] roofline {roof}", file=sys.stderr, flush=True)

    del eng
    torch.cuda.empty_cache()
    if not args.no_micro:
        extra["configs2_attention"] = micro_attention(torch, cfg, synth, Engine)
        print(f"[bench] configs[2] {extra['configs2_attention']}", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(torch, cfg, weights, int(round(mean_ctx)), args.cpu_budget)
        print(f"[bench] cpu baseline {cpu}", file=sys.stderr, flush=True)

    line = {
        "metric": "decode tok/s (Qwen3-4B-shape, B=16 ragged) + % of HBM roofline per step",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded random-init weights and prompt ids)",
        "config": {"workload": "configs[4]: Qwen3-4B-shape 36 layers, B=16 ragged prompts "
                               "U[64,2048], 1024 greedy tokens, hipGraph decode step; timed "
                               f"window at the generation's mean context ({mean_ctx:.0f} keys "
                               "per row on average)",
                   "global_batch": B, "layers": args.layers, "parallelism": "single GPU"},
        "roofline": roof, "cpu_baseline": cpu, "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
