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
import json
import os
import sys
from typing import Callable, Sequence

import torch

LIMIT = 2.0

# Prompt text for `--mode text`: any natural prose serves, since the rule
# compares the engine with the replay model on the same prompt.
CORPUS = (
    "A river delta forms where a slow current drops the silt it has carried for "
    "hundreds of kilometres. Each flood lays down a thin new layer, and over "
    "centuries the channels wander, split and rejoin across the plain. Farmers "
    "learned to read the colour of the water to judge when the next flood would "
    "come, and towns were built on the few ridges that stayed dry. Modern "
    "engineers measure the same process with sonar, satellite images and "
    "sediment cores, yet the basic pattern they record is the one the farmers "
    "knew: the land is always being rebuilt by the water that crosses it. "
)


def make_prompts(model_path: str | None, batch: int, in_len: int, mode: str,
                 vocab: int | None = None) -> list[list[int]]:
    """`batch` prompts of `in_len` token ids (the two prompt modes of
    check_exact.py:28-41). random: ids drawn uniformly from the checkpoint's
    vocabulary (config.json's vocab_size, or `vocab`), seed 20240; text: the
    tokenized corpus repeated as needed, row i starting i * in_len / batch
    tokens further along it, so that the rows overlap by less than a prompt."""
    if mode == "random":
        if vocab is None:
            with open(os.path.join(model_path, "config.json")) as f:
                vocab = int(json.load(f)["vocab_size"])
        g = torch.Generator().manual_seed(20240)
        return [torch.randint(0, vocab, (in_len,), generator=g).tolist() for _ in range(batch)]
    if mode != "text":
        raise ValueError(f"unknown prompt mode {mode!r}")
    from transformers import AutoTokenizer

    piece = AutoTokenizer.from_pretrained(model_path)(CORPUS, return_tensors=None)["input_ids"]
    step = max(1, in_len // max(1, batch))
    need = in_len + step * batch
    stream = piece * (need // max(1, len(piece)) + 1)
    return [stream[i * step:i * step + in_len] for i in range(batch)]


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


# command-line options: (flag, type, default, help); --model is required
_OPTIONS = (
    ("--model", str, None, "local HF checkpoint directory (config.json, safetensors, tokenizer for text mode)"),
    ("--batch", int, 1, "prompts decoded together"),
    ("--in-len", int, 512, "prompt length in tokens"),
    ("--out-len", int, 32, "tokens generated per prompt"),
    ("--mode", str, "text", "prompt source: random ids or the tokenized corpus"),
)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="the 2-logit teacher-forced acceptance rule")
    for flag, typ, default, text in _OPTIONS:
        kw = {"type": typ, "help": text}
        if default is None:
            kw["required"] = True
        else:
            kw["default"] = default
        if flag == "--mode":
            kw["choices"] = ["random", "text"]
        ap.add_argument(flag, **kw)
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
