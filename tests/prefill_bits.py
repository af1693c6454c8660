"""Child process of test_configs4_prefill_deterministic: builds the configs[4] engine (36 layers,
seed 0), prefills configs[4]'s 16 ragged prompts in one packed pass and prints the SHA-256 of the
first-token logits' bits and the first tokens, so the parent can compare another process's
prefill with its own bit for bit."""
import hashlib
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def prefill_digest(eng, prompts):
    """(SHA-256 hex of the packed prefill's bf16 logits, first tokens) on a fresh state."""
    import torch
    cap = -(-max(len(p) for p in prompts) // 128) * 128
    st = eng._new_state(len(prompts), cap)
    eng._dbg = []
    try:
        eng._prefill(prompts, st)
        logits = eng._dbg[-1]
    finally:
        eng._dbg = None
    assert int(st.err.item()) == 0
    bits = logits.to(torch.bfloat16).contiguous().view(torch.int16).numpy().tobytes()
    return hashlib.sha256(bits).hexdigest(), st.tok.cpu().tolist()


def main():
    import torch
    import __graft_entry__
    __graft_entry__.load_package()
    from dryft_amd import synth
    from dryft_amd.engine import Engine
    cfg = synth.qwen3_config()
    eng = Engine.from_state_dict(cfg, synth.random_weights(cfg, seed=0, device="cuda"),
                                 selftest=False)
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(64, 2049, (16,), generator=g).tolist()
    prompts = [torch.randint(0, cfg["vocab_size"], (n,), generator=g).tolist() for n in lens]
    digest, toks = prefill_digest(eng, prompts)
    print("PREFILL", digest, " ".join(map(str, toks)), flush=True)


if __name__ == "__main__":
    main()
