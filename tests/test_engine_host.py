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
    assert E._as_rows(torch.tensor([[1, 2], [3, 4]])) == [[1, 2], [3, 4]]
    assert E._as_rows(np.array([[1, 2]])) == [[1, 2]]
    assert E._as_rows(((5, 6),)) == [[5, 6]]
    assert E._as_rows([np.array([7, 8, 9]), torch.tensor([1])]) == [[7, 8, 9], [1]]


def test_tiles_split_rows_evenly():
    assert E._tiles(1, 8) == [(0, 1)]
    assert E._tiles(8, 8) == [(0, 8)]
    assert E._tiles(16, 8) == [(0, 8), (8, 16)]
    assert E._tiles(12, 8) == [(0, 6), (6, 12)]
    assert E._tiles(17, 8) == [(0, 5), (5, 11), (11, 17)]


@pytest.mark.parametrize("prompts", [[[1, 2, 3], [4, 5, 6]], PROMPTS, [[7], [1, 2, 3, 4, 5]], [[9, 9]]])
def test_pack_matches_the_oracle_layout(prompts):
    """engine.py:541-570's layout: left padding with id 0 at position 0, real
    positions 0..len-1, and for ragged batches the additive bf16 mask; the
    engine's numpy construction equals the oracle's loop, bit for bit."""
    holder = type("Holder", (), {"device": torch.device("cpu")})()
    ids, pos, pad, s, mask = E._FastEngine._pack(holder, prompts)
    r_ids, r_pos, r_pad, r_s, r_mask = O.pack(prompts)
    assert torch.equal(ids, r_ids) and torch.equal(pos, r_pos) and pad == r_pad and s == r_s
    assert (mask is None) == (r_mask is None)
    if mask is not None:
        assert mask.dtype == r_mask.dtype and torch.equal(mask, r_mask)
