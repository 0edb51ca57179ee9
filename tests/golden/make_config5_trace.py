"""Write the CPU oracle's config-5 trace (tests/golden/config5_trace.npz).

    python tests/golden/make_config5_trace.py [--steps 5] [--out PATH]

Config 5 of the benchmark at full depth: the random-init Qwen3-4B-
architecture model (checkpoint.random_weights(QWEN3_4B, seed=0)), the eight
ragged prompts bench.py decodes (microbench.batch8_prompts: lengths
U[64, 2048], ids U[0, vocab), seed 2), left-padded and prefilled as one
batch, then teacher-forced decode steps through the oracle (the reference's
torch fallback path restated: engine.py:721-743 over ek_model.py:280-416,
475-493). Step 0 is the prefill's token, steps 1.. the decode steps, each
fed the previous step's oracle ids. Per step and row the fixture holds the
argmax id and the 32 largest bf16 logits with their ids (ties in
first-index order).

It also records the oracle's own summation-order drift per step and row:
the same oracle re-run in lockstep (its own prefill and cache), fed the
same ids, with every projection of the prefill and of the decode steps
accumulated in another order (fp32 operands, one fp32 matmul, then bf16):
the largest |logit difference| over the whole vocabulary between the two
runs, and the reordered run's argmax. A GPU test judges its logits against
this drift, as the config-4 trace test does at batch 1. It runs on the
build container's CPU (the two prefills of 8 x 1805 padded tokens take most
of its time); nothing on the GPU box runs it.
"""

from __future__ import annotations

import argparse
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from enginekernel_amd import checkpoint as C  # noqa: E402
from enginekernel_amd.microbench import batch8_prompts  # noqa: E402
from oracle import ek_oracle as O  # noqa: E402

TOPK = 32


def top_entries(logits_row: torch.Tensor, k: int = TOPK):
    """The k largest logits of one row, ids ascending within equal values."""
    vals, idx = torch.sort(logits_row.float(), descending=True, stable=True)
    return idx[:k].to(torch.int32).numpy(), vals[:k].numpy()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--out", default=os.path.join(os.path.dirname(os.path.abspath(__file__)), "config5_trace.npz"))
    args = ap.parse_args()
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    cfg = dict(C.QWEN3_4B)
    t0 = time.perf_counter()
    tensors = C.random_weights(cfg, seed=0)
    print(f"weights in {time.perf_counter() - t0:.1f}s", flush=True)
    prompts = batch8_prompts(cfg["vocab_size"])
    b, n = len(prompts), args.steps
    model = O.OracleQwen3(O.OracleConfig(cfg), tensors)
    plain, plain_pre = model._proj, model._prefill_proj

    def reordered(x, layer, key):
        return torch.matmul(x.float(), layer[key].float().t()).to(torch.bfloat16)

    ids = np.zeros((n, b), dtype=np.int32)
    top_ids = np.zeros((n, b, TOPK), dtype=np.int32)
    top_logits = np.zeros((n, b, TOPK), dtype=np.float32)
    drift = np.zeros((n, b), dtype=np.float32)
    alt_ids = np.zeros((n, b), dtype=np.int32)
    forced = []   # ids fed to the reordered run (the main run's own tokens)
    main = O.generate_eager(model, prompts, n, record_logits=True)
    alt = O.generate_eager(model, prompts, n, record_logits=True, force=forced)
    t0 = time.perf_counter()
    for i in range(n):
        model._proj, model._prefill_proj = plain, plain_pre
        tok, logits = next(main)
        model._proj, model._prefill_proj = reordered, reordered
        _, alt_logits = next(alt)
        model._proj, model._prefill_proj = plain, plain_pre
        ids[i] = tok
        forced.append([int(t) for t in tok])
        for r in range(b):
            top_ids[i, r], top_logits[i, r] = top_entries(logits[r])
            assert top_ids[i, r, 0] == ids[i, r]
        drift[i] = (alt_logits.float() - logits.float()).abs().amax(dim=1).numpy()
        alt_ids[i] = torch.argmax(alt_logits, dim=-1).numpy()
        print(f"step {i}: ids {ids[i].tolist()}, drift max {drift[i].max():.4f}, reordered argmax differs in "
              f"{int((alt_ids[i] != ids[i]).sum())} rows ({time.perf_counter() - t0:.0f}s)", flush=True)
    lens = np.asarray([len(p) for p in prompts], dtype=np.int32)
    flat = np.asarray([t for p in prompts for t in p], dtype=np.int32)
    np.savez(args.out, prompt_lens=lens, prompt_ids=flat, ids=ids, top_ids=top_ids, top_logits=top_logits,
             drift=drift, alt_ids=alt_ids, seed=np.asarray([0, 2], dtype=np.int32))
    print(f"wrote {args.out}: {n} steps x {b} rows in {time.perf_counter() - t0:.0f}s")


if __name__ == "__main__":
    main()
