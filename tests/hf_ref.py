"""transformers' own Qwen3ForCausalLM as an independent check of the oracle.

This is the comparison the reference's `bench/test_equivalence.py:34-59`
makes (HF greedy with attention_mask and position_ids = cumsum(mask) - 1),
built from the same HF-named tensors the oracle and the HIP path load.
"""

from __future__ import annotations

import torch


def hf_model(cfg: dict, tensors: dict):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    from enginekernel_amd.checkpoint import config_json

    kw = {k: v for k, v in config_json(cfg).items() if k not in ("architectures", "model_type", "torch_dtype")}
    m = Qwen3ForCausalLM(Qwen3Config(**kw)).to(torch.bfloat16).eval()
    missing, unexpected = m.load_state_dict(tensors, strict=False)
    assert not missing and not unexpected, (missing, unexpected)
    return m


def hf_greedy(m, prompts, n):
    """bench/test_equivalence.py:34-59: left-padded greedy decode with a KV cache."""
    lens = [len(p) for p in prompts]
    s, b = max(lens), len(prompts)
    ids = torch.zeros((b, s), dtype=torch.long)
    mask = torch.zeros((b, s), dtype=torch.long)
    for i, p in enumerate(prompts):
        ids[i, s - lens[i]:] = torch.as_tensor(p)
        mask[i, s - lens[i]:] = 1
    pos = (mask.cumsum(-1) - 1).clamp(min=0)
    past, cur, cur_pos, cur_mask = None, ids, pos, mask
    out = []
    with torch.inference_mode():
        for _ in range(n):
            o = m(input_ids=cur, attention_mask=cur_mask, position_ids=cur_pos, past_key_values=past, use_cache=True)
            past = o.past_key_values
            t = o.logits[:, -1, :].argmax(-1)
            out.append(t.tolist())
            cur = t.unsqueeze(1)
            cur_pos = cur_pos[:, -1:] + 1
            cur_mask = torch.cat([cur_mask, torch.ones((b, 1), dtype=torch.long)], dim=1)
    return out


def equivalence_cases(vocab: int, seed: int = 1):
    """The cases of bench/test_equivalence.py:67-71 plus BASELINE config 1."""
    g = torch.Generator().manual_seed(seed)
    return [
        ("uniform batch 1", [torch.randint(0, vocab, (37,), generator=g).tolist()], 12),
        ("uniform batch 4", [torch.randint(0, vocab, (29,), generator=g).tolist() for _ in range(4)], 10),
        ("ragged batch 3", [torch.randint(0, vocab, (n,), generator=g).tolist() for n in (31, 17, 24)], 8),
        ("config 1", [torch.randint(0, vocab, (n,), generator=g).tolist() for n in (5, 9, 16)], 32),
    ]
