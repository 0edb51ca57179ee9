"""The 2-logit teacher-forced acceptance rule (bench/check_exact.py,
bench/margin.py of jeojdi1/EngineKernel).

A generated sequence is accepted when, replayed through a reference model
(prompt + generated tokens, one teacher-forced pass), every generated token is
the reference's greedy choice at its position or its logit is within LIMIT
(2.0) of the reference's top logit (check_exact.py:1-7, 96-99). Token equality
is stricter than this rule and fails on near-ties. `margins` returns the
per-position gaps (margin.py's worst-case report), `verdict` the summary.

The reference model is any callable mapping a [rows, n] int64 tensor of
token ids to [rows, n, vocab] logits; `hf_logits_fn` builds one from
transformers' AutoModelForCausalLM (bf16, SDPA), as the reference scripts do.

    python -m enginekernel_amd.acceptance --model DIR [--batch 1] [--in-len 512]
        [--out-len 32] [--mode random|text]

runs the engine on the model in DIR and checks its output that way
(check_exact.py:73-107); `text` mode needs the checkpoint's tokenizer files.
"""

from __future__ import annotations

import argparse
import os
import sys
from typing import Callable, Sequence

import torch

LIMIT = 2.0

TEXT = (
    "The history of computing hardware spans the development of machines able to "
    "perform arithmetic automatically. Early devices were mechanical; later ones "
    "used vacuum tubes, then transistors, then integrated circuits. Each step "
    "reduced cost and increased speed, which changed what problems were worth "
    "solving. Today the limiting factor for large language model inference is "
    "usually memory bandwidth rather than arithmetic throughput, because every "
    "generated token requires reading the entire set of model weights. "
)


def make_prompts(model_path: str | None, batch: int, in_len: int, mode: str) -> list[list[int]]:
    """check_exact.py:28-41: seeded random ids, or slices of a tokenized text."""
    if mode == "random":
        g = torch.Generator().manual_seed(0)
        return torch.randint(0, 151000, (batch, in_len), generator=g).tolist()
    from transformers import AutoTokenizer

    tok = AutoTokenizer.from_pretrained(model_path)
    ids = tok(TEXT * 200, return_tensors=None)["input_ids"]
    out = []
    for i in range(batch):
        s = (i * 37) % max(1, len(ids) - in_len - 1)
        out.append(ids[s:s + in_len])
    return out


@torch.inference_mode()
def margins(logits_fn: Callable[[torch.Tensor], torch.Tensor], prompts: Sequence[Sequence[int]],
            gen: Sequence[Sequence[int]], chunk: int = 2) -> list[tuple]:
    """check_exact.py:44-70: teacher-force prompt + generated tokens through
    the reference, rows of equal prompt length `chunk` at a time. gen[t][i] is
    row i's token at step t (the engine's yield order). Returns (row, step,
    ours, reference argmax, top logit - our token's logit) per position."""
    steps = len(gen)
    b = len(prompts)
    results = []
    lo = 0
    while lo < b:
        hi = min(lo + chunk, b)
        plen = len(prompts[lo])
        if any(len(prompts[i]) != plen for i in range(lo, hi)):   # ragged rows go one at a time
            hi = lo + 1
        rows = [list(prompts[i]) + [int(gen[t][i]) for t in range(steps)] for i in range(lo, hi)]
        logits = logits_fn(torch.as_tensor(rows, dtype=torch.long)).float()
        for i in range(hi - lo):
            for t in range(steps):
                lg = logits[i, plen + t - 1]
                ours = int(gen[t][lo + i])
                results.append((lo + i, t, ours, int(lg.argmax()), float(lg.max() - lg[ours])))
        lo = hi
    return results


def verdict(results: Sequence[tuple], limit: float = LIMIT) -> dict:
    """check_exact.py:94-107 and margin.py's worst margin: pass when no
    generated token sits more than `limit` below the reference's top logit."""
    diff = [r for r in results if r[2] != r[3]]
    over = [r for r in diff if r[4] > limit]
    gaps = [r[4] for r in results]
    return {"positions": len(results), "argmax_differs": len(diff), "over_limit": len(over),
            "worst_margin": max(gaps) if gaps else 0.0, "pass": not over, "first_failures": over[:8]}


def hf_logits_fn(model_path: str, device: str = "cuda"):
    """The reference scripts' replay model: transformers, bf16, SDPA."""
    from transformers import AutoModelForCausalLM

    model = AutoModelForCausalLM.from_pretrained(model_path, torch_dtype=torch.bfloat16,
                                                 attn_implementation="sdpa").to(device).eval()

    def fn(ids: torch.Tensor) -> torch.Tensor:
        out = model(input_ids=ids.to(device), use_cache=False).logits
        return out.float().cpu()
    return fn


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="the 2-logit teacher-forced acceptance rule")
    ap.add_argument("--model", required=True)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--in-len", type=int, default=512)
    ap.add_argument("--out-len", type=int, default=32)
    ap.add_argument("--mode", choices=["random", "text"], default="text")
    a = ap.parse_args(argv)
    prompts = make_prompts(a.model, a.batch, a.in_len, a.mode)

    from .engine import Engine
    eng = Engine(a.model)
    gen = list(eng.generate(prompts, a.out_len))
    del eng
    torch.cuda.empty_cache()
    v = verdict(margins(hf_logits_fn(a.model), prompts, gen))
    print(f"mode={a.mode} batch={a.batch} in={a.in_len} out={a.out_len}")
    print(f"  positions checked : {v['positions']}")
    print(f"  argmax differs    : {v['argmax_differs']}")
    print(f"  gap > {LIMIT} logits    : {v['over_limit']}")
    print(f"  worst margin      : {v['worst_margin']:.4f}")
    for r in v["first_failures"]:
        print(f"    {r}")
    print("VERDICT:", "PASS" if v["pass"] else "FAIL")
    return 0 if v["pass"] else 1


if __name__ == "__main__":
    sys.exit(main())
