"""The engine's greedy output under the 2-logit acceptance rule
(bench/check_exact.py), replayed through transformers' Qwen3ForCausalLM
built from the same tensors: the plain and the speculative paths, the tiny
model and every Qwen3-4B shape (two layers)."""

import pytest
import torch

from enginekernel_amd import acceptance as A
from enginekernel_amd import checkpoint as C
from enginekernel_amd.ek_model import Qwen3
from enginekernel_amd.engine import Engine
from tests.hf_ref import hf_model

pytestmark = pytest.mark.gpu


def _fn(m):
    def fn(ids):
        with torch.inference_mode():
            return m(input_ids=ids, use_cache=False).logits.float()
    return fn


@pytest.mark.parametrize("cfg_name", ["tiny", "4b_2layers"])
def test_engine_output_passes_acceptance(dev, cfg_name):
    cfg = dict(C.QWEN3_TINY) if cfg_name == "tiny" else dict(C.QWEN3_4B, num_hidden_layers=2)
    tensors = C.random_weights(cfg, seed=0)
    eng = Engine(model=Qwen3(None, dev, tensors=tensors, config=cfg))
    fn = _fn(hf_model(cfg, tensors))
    g = torch.Generator().manual_seed(9)
    vocab = cfg["vocab_size"]
    prompts = [torch.randint(0, vocab, (24,), generator=g).tolist()]
    for spec in (False, True):
        eng._impl.spec = spec
        gen = list(eng.generate(prompts, 12))
        v = A.verdict(A.margins(fn, prompts, gen))
        assert v["pass"] and v["positions"] == 12, (spec, v)
    # batch 3 (ragged), the plain path
    eng._impl.spec = False
    prompts = [torch.randint(0, vocab, (n,), generator=g).tolist() for n in (24, 17, 30)]
    gen = list(eng.generate(prompts, 8))
    v = A.verdict(A.margins(fn, prompts, gen))
    assert v["pass"] and v["positions"] == 24, v


def test_child_probes_and_probed_engine(dev, monkeypatch):
    """ek_probe in a child: the load-and-run probe and the attention launches
    of a decode and a verify shape; an engine that probes every new shape in
    a child before capturing it still generates the same tokens."""
    from enginekernel_amd import engine as E
    assert E._child_ok(["basic"])
    assert E._child_ok(["shape", 1, 3, 1024, 8, 32, 128])
    assert E._child_ok(["shape", 4, 0, 2048, 8, 32, 128])
    cfg = dict(C.QWEN3_TINY)
    tensors = C.random_weights(cfg, seed=0)
    plain = list(Engine(model=Qwen3(None, dev, tensors=tensors, config=cfg)).generate([[1, 2, 3, 4, 5]], 6))
    monkeypatch.setattr(E, "PROBE_CHILD", True)
    eng = Engine(model=Qwen3(None, dev, tensors=tensors, config=cfg))
    assert eng._impl.probe_child
    assert list(eng.generate([[1, 2, 3, 4, 5]], 6)) == plain
