"""The acceptance rule (bench/check_exact.py) on CPU: transformers' own
greedy output passes with zero margin, a near-tie substitute passes, and a
token far below the top logit fails; ragged prompts replay row by row."""

import torch

from enginekernel_amd import acceptance as A
from enginekernel_amd import checkpoint as C
from tests.hf_ref import hf_greedy, hf_model


def _setup():
    cfg = dict(C.QWEN3_TINY)
    m = hf_model(cfg, C.random_weights(cfg, seed=0))

    def fn(ids):
        with torch.inference_mode():
            return m(input_ids=ids, use_cache=False).logits.float()
    return m, fn


def test_reference_greedy_passes_with_zero_margin():
    m, fn = _setup()
    g = torch.Generator().manual_seed(3)
    prompts = [torch.randint(0, 1024, (20,), generator=g).tolist() for _ in range(3)]
    gen = hf_greedy(m, prompts, 6)
    v = A.verdict(A.margins(fn, prompts, gen))
    assert v["pass"] and v["positions"] == 18 and v["argmax_differs"] == 0 and v["worst_margin"] == 0.0


def test_near_tie_passes_and_far_token_fails():
    m, fn = _setup()
    g = torch.Generator().manual_seed(4)
    prompts = [torch.randint(0, 1024, (16,), generator=g).tolist()]
    gen = hf_greedy(m, prompts, 4)
    # the runner-up at the last step sits within 2 logits of the top (a random-init model's logits are flat)
    ids = torch.as_tensor([prompts[0] + [t[0] for t in gen[:-1]]])
    last = fn(ids)[0, -1]
    top2 = torch.topk(last, 2).indices.tolist()
    worst = int(torch.argmin(last))
    near = [list(t) for t in gen]
    near[-1] = [top2[1]]
    v = A.verdict(A.margins(fn, prompts, near))
    assert v["pass"] and v["argmax_differs"] == 1 and 0 < v["worst_margin"] <= A.LIMIT
    far = [list(t) for t in gen]
    far[-1] = [worst]
    v = A.verdict(A.margins(fn, prompts, far), limit=float(last.max() - last[worst]) / 2)
    assert not v["pass"] and v["over_limit"] == 1 and v["first_failures"][0][1] == 3


def test_ragged_rows_replay_one_at_a_time():
    m, fn = _setup()
    prompts = [[5, 6, 7, 8, 9], [1, 2, 3]]
    gen = [[10, 11], [12, 13]]
    res = A.margins(fn, prompts, gen)
    assert [(r[0], r[1]) for r in res] == [(0, 0), (0, 1), (1, 0), (1, 1)]
    solo = A.margins(fn, [prompts[1]], [[11], [13]])
    assert [r[4] for r in res[2:]] == [r[4] for r in solo]
