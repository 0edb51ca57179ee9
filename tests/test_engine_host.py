"""Engine facade behaviour on the CPU (engine.py:770-830): no silent
degradation, explicit fallback at load, and replay-and-skip continuation
after a mid-stream failure. The fallback used here is the CPU oracle."""

import pytest
import torch

from enginekernel_amd import checkpoint as C
from enginekernel_amd import ek_kernels as K
from enginekernel_amd import engine as E
from oracle import ek_oracle as O

PROMPTS = [[3, 1, 4, 1, 5, 9, 2, 6], [5, 3, 5], [8, 9, 7, 9, 3, 2]]


class OracleEngine:
    def __init__(self, path):
        self.model = O.OracleQwen3.from_path(path)

    def generate(self, input_ids, max_new_tokens):
        yield from O.generate_eager(self.model, input_ids, max_new_tokens)


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    p = tmp_path_factory.mktemp("tiny")
    C.write_checkpoint(str(p), dict(C.QWEN3_TINY), seed=0)
    return str(p)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the GPU-less behaviour")
def test_no_gpu_raises_without_fallback(ckpt):
    with pytest.raises(K.HipUnavailable):
        E.Engine(ckpt)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the GPU-less behaviour")
def test_explicit_fallback_at_load(ckpt):
    eng = E.Engine(ckpt, fallback=lambda: OracleEngine(ckpt))
    assert eng.tier == "fallback"
    want = list(O.generate_eager(O.OracleQwen3.from_path(ckpt), PROMPTS, 6))
    assert list(eng.generate(PROMPTS, 6)) == want


def test_midstream_failure_replays_and_skips(ckpt, monkeypatch):
    ref = OracleEngine(ckpt)
    want = list(ref.generate(PROMPTS, 10))

    class Flaky:
        def __init__(self, model_path=None, model=None):
            self.calls = 0

        def generate(self, input_ids, n):
            for i, step in enumerate(ref.generate(input_ids, n)):
                if i == 4:
                    raise RuntimeError("injected device failure")
                yield step

    monkeypatch.setattr(E, "_FastEngine", Flaky)
    eng = E.Engine(ckpt, fallback=lambda: OracleEngine(ckpt))
    assert eng.tier == "hip"
    got = list(eng.generate(PROMPTS, 10))
    assert eng.tier == "fallback"
    assert got == want


def test_midstream_failure_without_fallback_propagates(ckpt, monkeypatch):
    class Broken:
        def __init__(self, model_path=None, model=None):
            pass

        def generate(self, input_ids, n):
            yield [0] * len(input_ids)
            raise RuntimeError("injected")

    monkeypatch.setattr(E, "_FastEngine", Broken)
    eng = E.Engine(ckpt)
    with pytest.raises(RuntimeError, match="injected"):
        list(eng.generate(PROMPTS, 4))


def test_rows_accepts_tensors_lists_and_arrays():
    import numpy as np
    assert E._rows(torch.tensor([[1, 2], [3, 4]])) == [[1, 2], [3, 4]]
    assert E._rows(np.array([[1, 2]])) == [[1, 2]]
    assert E._rows(((5, 6),)) == [[5, 6]]
