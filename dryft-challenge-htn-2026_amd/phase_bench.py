"""Timing of the one-launch decode step's GEMV phases alone, and of the per-op kernels at the
BASELINE configs[1] / configs[2] shapes (the measurements behind bench.py's configs[1] line and
the rocprofv3 counter summaries of the per-op kernels).

Fused phases: dd_decode_step runs any sub-range of its 2 + 5L phases; a range of one phase
launches that phase alone, with no grid barrier. For M sequences (M in 1, 4, 8, 16) a state is
prefilled and run through one full step first (so every activation slot holds valid data), then
the embedding phase, each GEMV phase of layer 0 (QKV, O, gate/up, down) and the lm_head phase are
launched alone, one launch at a time, under a rocprofv3 kernel trace. ``--parse`` matches the
trace's step-kernel dispatches to the launch plan: a phase's own time is the median dispatch
duration of its launches minus the embedding phase's (a gather of M rows: the launch's fixed
set-up and exit). Bytes per phase follow configs[1]: N K 2 (weights) + M K 2 (activation) +
M N 2 (output).

Per-op kernels (``--per-op``): dd_gemv at the five projection shapes and M in 1, 4, 8, 16, then
dd_attn_decode at configs[2] (B = 16, ragged contexts U[512, 8192], cap 8192), a few launches
each, and three 1 GiB streaming reads (the byte counters' calibration), for
``rocprofv3 --kernel-trace --stats`` and ``--pmc`` runs.

  cd /tmp && rocprofv3 --kernel-trace --output-format csv -d <dir> -o phases -- \
      python3 <repo>/dryft-challenge-htn-2026_amd/phase_bench.py --plan <dir>/plan.json
  python3 dryft-challenge-htn-2026_amd/phase_bench.py --parse <dir>/phases_kernel_trace.csv \
      <dir>/plan.json
  python3 dryft-challenge-htn-2026_amd/phase_bench.py --layers 1 --per-op   (under rocprofv3
      --kernel-trace, then --pmc FETCH_SIZE, WRITE_SIZE and
      "SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_BF16 SQ_BUSY_CYCLES GRBM_GUI_ACTIVE")
  python3 dryft-challenge-htn-2026_amd/phase_bench.py --parse-per-op <trace dir> <pmc dirs...>
"""
import argparse
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _shapes(eng):
    cfg = eng.cfg
    H, I, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    return {"qkv": ((eng.nh + 2 * eng.nkv) * eng.hd, H), "o": (H, eng.nh * eng.hd),
            "gate_up": (2 * I, H), "down": (H, I), "lm_head": (V, H)}


PHASE_ORDER = ("embed", "qkv", "o", "gate_up", "down", "lm_head")


def launch_phases(torch, eng, Ms=(1, 4, 8, 16), reps=20, warm=3):
    """Launches, for each M, one full step, then `warm` + `reps` launches of each phase of
    PHASE_ORDER alone (the embedding phase, layer 0's QKV, O, gate/up and down, the lm_head
    phase); returns the launch plan [[M, phase, warm, reps], ...] in launch order."""
    L = eng.L
    q = {"embed": 0, "qkv": 1, "o": 3, "gate_up": 4, "down": 5, "lm_head": 1 + 5 * L}
    g = torch.Generator().manual_seed(21)
    V = eng.cfg["vocab_size"]
    plan = []
    for M in Ms:
        st = eng._new_state(M, 256)
        assert st.fused is not None, f"the one-launch step does not take B={M}"
        eng._prefill(torch.randint(0, V, (M, 64), generator=g).tolist(), st)
        eng.step.run(st)                                   # every slot valid
        plan.append([M, "full", 1, 0])
        for name in PHASE_ORDER:
            for _ in range(warm + reps):
                eng.step.run(st, q[name], q[name] + 1)
                torch.cuda.synchronize()                   # launches one at a time
            plan.append([M, name, warm, reps])
        assert int(st.err.item()) == 0
        del st
        torch.cuda.empty_cache()
    return plan


def parse_trace(trace_csv, plan, shapes):
    """Phase times from a rocprofv3 kernel trace of launch_phases: the decode-step dispatches
    in launch order are matched to the plan; per (M, phase) the median dispatch duration of its
    timed launches, minus the embedding phase's (the launch's fixed set-up and exit), is the
    phase's own time. Returns {phase: {"M<m>": {"us", "GBps"}}, "_embed_us": {...}}."""
    import csv
    rows = []
    with open(trace_csv) as f:
        for r in csv.DictReader(f):
            if "decode_step_kernel" in r.get("Kernel_Name", ""):
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    rows.sort()
    dur = [(e - b) / 1e3 for b, e in rows]                 # us
    i, med = 0, {}
    for M, name, warm, reps in plan:
        i += warm
        d = sorted(dur[i:i + reps])
        i += reps
        if reps:
            med[(M, name)] = d[len(d) // 2]
    assert i == len(dur), f"plan covers {i} dispatches, trace has {len(dur)}"
    out = {k: {} for k in PHASE_ORDER[1:]}
    out["_embed_us"] = {}
    for M in sorted({m for m, _ in med}):
        base = med[(M, "embed")]
        out["_embed_us"][f"M{M}"] = round(base, 2)
        for name in PHASE_ORDER[1:]:
            us = med[(M, name)] - base
            N, K = shapes[name]
            nbytes = N * K * 2 + M * K * 2 + M * N * 2
            out[name][f"M{M}"] = {"us": round(us, 2), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
    return out


def per_op(torch, eng, reps=10):
    """dd_gemv at the configs[1] shapes and dd_attn_decode at configs[2], `reps` launches each
    (for the profiler); returns {kernel: us per launch} from HIP events."""
    from dryft_amd._lib import check
    ops = eng.ops.f if hasattr(eng.ops, "f") else eng.ops
    res = {}
    g = torch.Generator(device="cuda").manual_seed(11)
    for name, (N, K) in _shapes(eng).items():
        w = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
        for M in (1, 4, 8, 16):
            x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
            ops.linear(x, w)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                ops.linear(x, w)
            e1.record()
            e1.synchronize()
            res[f"dd_gemv {name} M{M}"] = round(e0.elapsed_time(e1) * 1e3 / reps, 2)
        del w
    # B = 16, ragged contexts U[512, 8192], cap 8192, 32 q / 8 kv heads
    B, NH, NKV, HD, cap = 16, eng.nh, eng.nkv, eng.hd, 8192
    gc = torch.Generator().manual_seed(2)
    ctx = torch.randint(512, 8193, (B,), generator=gc)
    pos = (ctx - 1).cuda()
    q = torch.randn(B, NKV, 1, NH // NKV, HD, generator=g, device="cuda").to(torch.bfloat16)
    kc = torch.randn(B, NKV, cap, HD, generator=g, device="cuda").to(torch.bfloat16)
    vc = torch.randn(B, NKV, cap, HD, generator=g, device="cuda").to(torch.bfloat16)
    ops.attn_decode(q, kc, vc, pos, 1)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        ops.attn_decode(q, kc, vc, pos, 1)
    e1.record()
    e1.synchronize()
    res["dd_attn_decode configs[2]"] = round(e0.elapsed_time(e1) * 1e3 / reps, 2)
    res["dd_attn_decode configs[2] bytes"] = int(4096 * int(ctx.sum()))
    del kc, vc
    # a copy kernel of known size (1 GiB read) for the profiler's byte-counter calibration
    buf = torch.ones(1 << 30, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    for _ in range(3):
        check(eng.step.L.dd_stream_read(buf.data_ptr(), buf.numel(), 1024, 512, sink.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream), "dd_stream_read")
    torch.cuda.synchronize()
    return res


def parse_per_op(trace_dir, pmc_dirs, shapes, reps=10):
    """Per-kernel figures of a ``--per-op`` run from its rocprofv3 outputs: the kernel trace
    (dispatch durations) and --pmc passes (FETCH_SIZE, WRITE_SIZE in KiB; SQ_VALU_MFMA_BUSY_CYCLES,
    GRBM_GUI_ACTIVE). Dispatches are matched to the run's launch order (per dd_gemv shape and M:
    one warm-up and `reps` timed launches; then dd_attn_decode likewise; then three 1 GiB
    stream reads, whose FETCH_SIZE calibrates the byte counters). Returns rows of
    {kernel, us, algo_GBps, hbm_GBps, hbm_over_algo, mfma_util}."""
    import csv
    import glob

    def dispatches(path, name_filter, counter=None):
        names = (name_filter,) if isinstance(name_filter, str) else name_filter
        out = []
        with open(path) as f:
            for r in csv.DictReader(f):
                if (any(n in r["Kernel_Name"] for n in names)
                        and (counter is None or r["Counter_Name"] == counter)):
                    v = float(r["Counter_Value"]) if counter else (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
                    out.append((int(r.get("Dispatch_Id") or r.get("Correlation_Id") or 0), v))
        out.sort()
        return [v for _, v in out]

    trace = glob.glob(os.path.join(trace_dir, "*kernel_trace.csv"))[0]
    pmc = {}
    for d in pmc_dirs:
        f = glob.glob(os.path.join(d, "*counter_collection.csv"))[0]
        with open(f) as fh:
            names = {r["Counter_Name"] for r in csv.DictReader(fh)}
        for c in names:
            pmc[c] = f
    cal = dispatches(pmc["FETCH_SIZE"], "stream_read_kernel", "FETCH_SIZE")
    scale = (1 << 30) / 1024 / (sum(cal) / len(cal))         # true KiB / counted KiB
    rows = []
    # dd_gemv launches gemv_kernel, or gemv_multi_kernel (several W tiles per workgroup) for
    # unsplit shapes at M >= 8
    kinds = [(("gemv_kernel", "gemv_multi_kernel"), [(n, m) for n in shapes for m in (1, 4, 8, 16)]),
             ("attn_decode_kernel", [("configs[2]", 16)])]
    for kern, cases in kinds:
        us = dispatches(trace, kern)
        fetch = dispatches(pmc["FETCH_SIZE"], kern, "FETCH_SIZE")
        write = dispatches(pmc["WRITE_SIZE"], kern, "WRITE_SIZE")
        busy = dispatches(pmc["SQ_VALU_MFMA_BUSY_CYCLES"], kern, "SQ_VALU_MFMA_BUSY_CYCLES")
        gui = dispatches(pmc["GRBM_GUI_ACTIVE"], kern, "GRBM_GUI_ACTIVE")
        for i, (name, M) in enumerate(cases):
            sl = slice(i * (reps + 1) + 1, (i + 1) * (reps + 1))
            mean = lambda v: sum(v[sl]) / len(v[sl])
            t = mean(us)
            if "gemv_kernel" in kern:
                N, K = shapes[name]
                algo = N * K * 2 + M * K * 2 + M * N * 2
                label = f"dd_gemv {name} {N}x{K} M={M}"
            else:
                import torch
                ctx = torch.randint(512, 8193, (16,), generator=torch.Generator().manual_seed(2))
                algo = 4096 * int(ctx.sum())                   # K and V rows attended, all heads
                label = "dd_attn_decode configs[2] (B=16, ctx U[512,8192])"
            hbm = (mean(fetch) + mean(write)) * scale * 1024
            cyc = mean(gui) / 8                                # GRBM_GUI_ACTIVE summed over 8 XCDs
            rows.append({"kernel": label, "us": round(t, 2),
                         "algo_GBps": round(algo / (t * 1e-6) / 1e9, 1) if algo else None,
                         "hbm_bytes": int(hbm), "hbm_GBps": round(hbm / (t * 1e-6) / 1e9, 1),
                         "hbm_over_algo": round(hbm / algo, 3) if algo else None,
                         "mfma_util": round(mean(busy) / (cyc * 1024), 4) if cyc else None})
    return {"copy_calibration_scale": round(scale, 4), "rows": rows}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--per-op", action="store_true")
    ap.add_argument("--plan", help="write the fused-phase launch plan (JSON) here")
    ap.add_argument("--parse", nargs=2, metavar=("KERNEL_TRACE_CSV", "PLAN_JSON"),
                    help="phase times from a rocprofv3 kernel trace of a fused-phase run")
    ap.add_argument("--parse-per-op", nargs="+", metavar="DIR",
                    help="per-kernel figures of a --per-op run: its kernel-trace output folder, "
                         "then its --pmc output folders")
    args = ap.parse_args()
    if args.parse_per_op:
        shapes = {"qkv": (6144, 2560), "o": (2560, 4096), "gate_up": (19456, 2560),
                  "down": (2560, 9728), "lm_head": (151936, 2560)}
        print(json.dumps(parse_per_op(args.parse_per_op[0], args.parse_per_op[1:], shapes),
                         indent=1))
        return
    if args.parse:
        with open(args.parse[1]) as f:
            doc = json.load(f)
        print(json.dumps(parse_trace(args.parse[0], doc["plan"], doc["shapes"]), indent=1))
        return
    import torch
    sys.path.insert(0, ROOT)
    import __graft_entry__
    __graft_entry__.load_package()
    from dryft_amd import synth
    from dryft_amd.engine import Engine
    cfg = synth.qwen3_config(num_hidden_layers=args.layers)
    eng = Engine.from_state_dict(cfg, synth.random_weights(cfg, seed=0, device="cuda"),
                                 selftest=False)
    if args.per_op:
        print(json.dumps(per_op(torch, eng)), flush=True)
    else:
        plan = launch_phases(torch, eng, reps=args.reps)
        doc = {"plan": plan, "shapes": _shapes(eng)}
        if args.plan:
            with open(args.plan, "w") as f:
                json.dump(doc, f)
        print(json.dumps(doc), flush=True)


if __name__ == "__main__":
    main()
