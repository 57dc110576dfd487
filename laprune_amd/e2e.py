"""End-to-end decode throughput on random-init Llama-3.1-8B (configs C4, C5).

The reference's decode benchmark (benchmarks/decode.py:16-108) times greedy
decode after a prefill: tok/s = batch * (decode_tokens - warmup_tokens) /
seconds.  Here the model is built from a local config with bf16 weights
N(0, 0.02) (no download), the prompt is uniform-random token ids, and the
codebooks are synthetic N(0, 0.02) [32, 256, 128] per LAPrune layer.

  C4: batch 1, 131072-token context, layers 0-1 dense and 2-31 LAPrune,
      4 sink + 64 local tokens, 64-token encode buffer, top-2048 per KV
      group, 256 decode tokens.
  C5: batch 16, per-sequence context lengths uniform in [16384, 32768]
      (ragged, prefilled one sequence at a time), top-1024, 128 tokens.

``--method dense`` decodes every layer with the same GPU's dense split-K
flash-decode (the comparator); ``both`` runs LAPrune, then dense, on the same
weights.  Each decode step is one replay of a captured graph (``--eager``:
host launches).  Prints one JSON line.

    python -m laprune_amd.e2e --config c4 --method both
"""
from __future__ import annotations

import argparse
import json
import sys
import time

import torch

CONFIGS = {
    "c4": dict(batch=1, ctx=(131072, 131072), topk=2048, decode=256, warmup=16),
    "c5": dict(batch=16, ctx=(16384, 32768), topk=1024, decode=128, warmup=8),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def run(model, cfg: dict, method: str, lengths: list[int], prompts: list[torch.Tensor],
        codebooks: dict, layers: int, graph: bool = True) -> dict:
    from .llama import LAPruneLlama, LAPruneSettings
    from .retrieval import RetrievalConfig
    apply = list(range(2, layers)) if method == "laprune" else []
    settings = LAPruneSettings(
        apply_layers=apply,
        retrieval=RetrievalConfig(sink_size=4, local_window=64, topk=cfg["topk"],
                                  select="group", score_dtype=torch.bfloat16),
        group_size=64)
    B = cfg["batch"]
    cap = max(lengths) + cfg["decode"] + 64
    lm = LAPruneLlama(model, {i: codebooks[i] for i in apply}, settings, batch=B, capacity=cap)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    last = []
    if len(set(lengths)) == 1:
        ids = torch.cat(prompts)
        logits = lm.prefill(ids[:, :-1])
        tok = ids[:, -1:]
    else:
        for b, p in enumerate(prompts):
            log(f"  prefill sequence {b} ({p.shape[1]} tokens)")
            lm.prefill_row(b, p[:, :-1])
            last.append(p[:, -1:])
        tok = torch.cat(last)
        logits = None
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    del logits
    log(f"  {method}: prefill {prefill_s:.2f} s; decoding {cfg['decode']} tokens")
    finite_flags = []
    t_warm = None
    generated = []
    for step in range(cfg["decode"]):
        if graph:  # one captured graph per step; the greedy token stays on the GPU
            logits = lm.decode_graph(tok if step == 0 else None)
            tok = lm.next_tokens().clone()
        else:
            logits = lm.decode(tok)
            tok = logits.argmax(dim=-1, keepdim=True)
        finite_flags.append(torch.isfinite(logits).all())
        generated.append(tok)
        if step + 1 == cfg["warmup"]:
            torch.cuda.synchronize()
            t_warm = time.perf_counter()
        if (step + 1) % 32 == 0:
            log(f"  {method}: {step + 1} tokens")
    torch.cuda.synchronize()
    secs = time.perf_counter() - t_warm
    finite = bool(torch.stack(finite_flags).all())
    measured = cfg["decode"] - cfg["warmup"]
    out = {"method": method, "graph": graph, "prefill_s": round(prefill_s, 3),
           "decode_s": round(secs, 4),
           "tokens_per_s": round(B * measured / secs, 3),
           "ms_per_step": round(secs / measured * 1e3, 3), "finite_logits": finite,
           "first_tokens": torch.cat(generated[:8], dim=1)[0].tolist()}
    del lm
    torch.cuda.empty_cache()
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--config", choices=sorted(CONFIGS), default="c4")
    ap.add_argument("--method", choices=["laprune", "dense", "both"], default="both")
    ap.add_argument("--layers", type=int, default=32, help="decoder layers (32 = Llama-3.1-8B)")
    ap.add_argument("--prompt-tokens", type=int, default=0,
                    help="override the context length (uniform across the batch)")
    ap.add_argument("--decode-tokens", type=int, default=0)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--eager", action="store_true",
                    help="launch every kernel from the host instead of replaying one "
                         "captured graph per decode step")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("e2e needs a GPU", file=sys.stderr)
        return 2
    from . import _native
    from .llama import llama31_8b_config, random_model
    _native.lib()
    cfg = dict(CONFIGS[args.config])
    if args.prompt_tokens:
        cfg["ctx"] = (args.prompt_tokens, args.prompt_tokens)
    if args.decode_tokens:
        cfg["decode"] = args.decode_tokens
        cfg["warmup"] = min(cfg["warmup"], args.decode_tokens // 4)
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(args.seed)
    lo, hi = cfg["ctx"]
    lengths = [lo] * cfg["batch"] if lo == hi else \
        torch.randint(lo, hi + 1, (cfg["batch"],), generator=g).tolist()
    config = llama31_8b_config(num_layers=args.layers)
    log(f"building random-init Llama-3.1-8B geometry, {args.layers} layers")
    model = random_model(config, dev, seed=args.seed)
    prompts = [torch.randint(0, config.vocab_size, (1, n), generator=g).to(dev) for n in lengths]
    codebooks = {i: (torch.randn(32, 256, 128, generator=g) * 0.02).to(dev)
                 for i in range(2, args.layers)}
    methods = ["laprune", "dense"] if args.method == "both" else [args.method]
    results = {m: run(model, cfg, m, lengths, prompts, codebooks, args.layers,
                      graph=not args.eager) for m in methods}
    line = {"config": args.config, "batch": cfg["batch"], "layers": args.layers,
            "context_lengths": lengths if len(set(lengths)) > 1 else lengths[0],
            "decode_tokens": cfg["decode"], "warmup_tokens": cfg["warmup"],
            "topk": cfg["topk"], "sink": 4, "local": 64, "encode_buffer": 64,
            "weights": "random N(0,0.02) bf16", "prompt": "uniform random ids",
            "results": results}
    if len(results) == 2:
        line["speedup_vs_dense"] = round(results["laprune"]["tokens_per_s"] /
                                         results["dense"]["tokens_per_s"], 3)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
