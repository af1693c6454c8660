"""Decode-step benchmark on one MI355X.

Workload: the full 36-layer Qwen3-4B-shape model with seeded
random-init bf16 weights (N(0, 0.02), norms 1 + N(0, 0.02), tied lm_head, vocab 151936),
B = 16 sequences with ragged prompt lengths U[64, 2048] (token ids uniform over the vocab),
greedy decode of 1024 tokens per sequence. A "step" is one hipGraph replay of the whole decode
step (all 16 rows, one weight pass, one persistent kernel launch). Prefill is untimed; the first W decode steps are warm-up;
exactly K steps are timed (defaults W=23, K=1000: tokens 2..1024 of the generation).

One JSON line is printed with the contract fields plus
  roofline      the dominant kernel -- the one-launch decode step kernel, which is the whole
                step -- timed live with HIP events over the timed replays: algorithmic bytes
                (weights + attended K/V + new K/V) / average launch time;
  cpu_baseline  the CPU oracle (this repo's restatement of the reference's torch path) timed on
                the host on a bounded sample: B=1 decode steps of the same 36-layer model at the
                workload's mean context (the reference decodes ragged batches as independent
                B=1 streams, so its throughput is 1 token per B=1 step);
  extra         whole-step HBM accounting (bytes/step, achieved GB/s, fraction of the measured
                streaming-read ceiling and of the 8 TB/s spec) and the B=1 configs[3] figure.
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


def measured_traffic():
    """HBM bytes per launch of the step kernel from the committed rocprofv3 --pmc runs of this
    same workload (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the copy-kernel calibration);
    None when the file is absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    scale = t["copy_calibration"]["scale"] * 1024
    return int((t["fetch_kib_per_dispatch"] + t["write_kib_per_dispatch"]) * scale)


def step_roofline(ms, bytes_step, B):
    """The dominant (and only) kernel of a decode step is the one-launch step kernel: the timed
    region is K graph replays of one launch each, timed with HIP events on the stream they run
    on. Algorithmic bytes per launch: every weight matrix once (36 x [wqkv, wo, wgu, wd] +
    lm_head), the K/V cache rows each sequence attends (pos[b] + 1 per row), the new K/V rows,
    the embedding rows gathered; activations are a few MB and left out."""
    avg_s = ms * 1e-3
    return {"kernel": "dd::st::decode_step_kernel (whole decode step, one launch)",
            "bound": "hbm", "achieved": round(bytes_step / avg_s / 1e9, 1),
            "peak": SPEC_BW / 1e9, "unit": "GB/s", "frac": round(bytes_step / avg_s / SPEC_BW, 4),
            "traffic": measured_traffic() if B == 16 else None,
            "avg_launch_us": round(avg_s * 1e6, 2),
            "algo_bytes_per_launch": int(bytes_step), "rows": B}


def cpu_baseline(torch, cfg, weights_gpu, mean_ctx, budget_s=20.0):
    """B=1 decode steps of the CPU oracle on the full model at the workload's mean context."""
    from oracle.reference import OracleEngine
    # the host's CPU share: OMP_NUM_THREADS when the environment sets it, else every core
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    w = {k: v.cpu() for k, v in weights_gpu.items()}
    ref = OracleEngine.from_state_dict(cfg, w)
    del w
    cap = -(-(mean_ctx + 8) // 128) * 128
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
            "ms_per_step": round(dt * 1e3, 1), "host_cpus": os.cpu_count()}


def run_decode(torch, eng, prompts, warmup, steps):
    """Prefill, W warm-up replays, then K timed replays; returns (ms/step, bytes/step)."""
    B = len(prompts)
    n = warmup + steps + 1
    S = max(len(p) for p in prompts)
    cap = -(-(S + n) // 128) * 128
    st = eng._state(B, cap, graph=True)
    assert st.graph is not None, "decode graph capture failed"
    assert st.fused is not None, "the one-launch decode step is not bound to this state"
    eng._prefill(prompts, st)
    for _ in range(warmup):
        st.graph.replay()
    torch.cuda.synchronize()
    pos0 = st.pos.clone().cpu()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        st.graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    assert eng.error_flags() == 0, "kernel error flag set"
    # attended context of step t for row b: pos0[b] + t + 1 keys
    ctx_sum = sum(int(p) * steps + steps * (steps + 1) // 2 for p in pos0)
    wb = weight_bytes(eng.cfg)
    H = eng.cfg["hidden_size"]
    bytes_step = wb + KV_BYTES_TOKEN * (ctx_sum / steps) + KV_BYTES_TOKEN * B + B * H * 2
    return ms, bytes_step, float(pos0.float().mean()) + steps / 2


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
    lens = torch.randint(64, 2049, (B,), generator=g).tolist()
    prompts = [torch.randint(0, cfg["vocab_size"], (n,), generator=g).tolist() for n in lens]
    ms, bytes_step, mean_ctx = run_decode(torch, eng, prompts, args.warmup, args.steps)
    tok_s = B / (ms * 1e-3)
    achieved = bytes_step / (ms * 1e-3)
    print(f"[bench] B={B}: {ms:.3f} ms/step, {tok_s:.0f} tok/s, {achieved / 1e9:.0f} GB/s "
          f"({achieved / read_bw * 100:.1f}% of measured, {achieved / SPEC_BW * 100:.1f}% of spec)",
          file=sys.stderr, flush=True)

    extra = {"bytes_per_step": int(bytes_step), "step_achieved_GBps": round(achieved / 1e9, 1),
             "measured_read_GBps": round(read_bw / 1e9, 1),
             "frac_of_measured": round(achieved / read_bw, 4),
             "frac_of_spec": round(achieved / SPEC_BW, 4),
             "prompt_lens": lens, "mean_context": round(mean_ctx, 1)}

    if not args.no_b1:                        # configs[3]: B=1, prompt 128, 512 generated
        p1 = [torch.randint(0, cfg["vocab_size"], (128,), generator=g).tolist()]
        ms1, bytes1, _ = run_decode(torch, eng, p1, 10, 500)
        extra["b1"] = {"ms_per_step": round(ms1, 4), "tok_s": round(1e3 / ms1, 1),
                       "step_achieved_GBps": round(bytes1 / (ms1 * 1e-3) / 1e9, 1),
                       "frac_of_measured": round(bytes1 / (ms1 * 1e-3) / read_bw, 4)}
        print(f"[bench] B=1: {ms1:.3f} ms/step, {1e3 / ms1:.0f} tok/s", file=sys.stderr, flush=True)

    if not args.no_verify:                    # configs[4] verify shape: W = 5 per row
        msv, bytesv = run_verify(torch, eng, prompts)
        extra["verify_w5"] = {"ms_per_step": round(msv, 4), "tokens_per_step": B * 5,
                              "tok_s": round(B * 5 / (msv * 1e-3), 1),
                              "step_achieved_GBps": round(bytesv / (msv * 1e-3) / 1e9, 1),
                              "path": "per-op HIP kernels (q/k norm + RoPE + K/V write, "
                                      "attention) and hipBLASLt GEMMs at M=80, hipGraph"}
        print(f"[bench] verify B={B} W=5: {msv:.3f} ms/step", file=sys.stderr, flush=True)

    roof = step_roofline(ms, bytes_step, B)
    print(f"[bench] roofline {roof}", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu:
        del eng
        torch.cuda.empty_cache()
        cpu = cpu_baseline(torch, cfg, weights, int(mean_ctx), args.cpu_budget)
        print(f"[bench] cpu baseline {cpu}", file=sys.stderr, flush=True)

    line = {
        "metric": "decode tok/s (Qwen3-4B-shape, B=16 ragged) + % of HBM roofline per step",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded random-init weights and prompt ids)",
        "config": {"workload": "configs[4]: Qwen3-4B-shape 36 layers, B=16 ragged prompts "
                               "U[64,2048], 1024 greedy tokens, hipGraph decode step",
                   "global_batch": B, "layers": args.layers, "parallelism": "single GPU"},
        "roofline": roof, "cpu_baseline": cpu, "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
