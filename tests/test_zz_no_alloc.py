"""ek_decode_step_noalloc (the one-launch decode step on the library's static
per-device hand-over state) against ek_decode_step (the same step on a
caller-allocated arena and barrier block), both called through the C ABI.

Five calls in a row, each with a smaller hand-over arena than the one
before inside the same static array: 4 batch rows through 36 layers (the
batch kernel, an arena of 15.8 MiB, near the static 16 MiB), 2 rows through
three layers, then batch 1 -- a split-attention bucket of 4096 keys, then
attention-unit buckets with fewer layers and shorter contexts. Each runs
three consecutive steps on identical copies of the state and caches, and
everything the step writes must be bit-identical -- the step's logits,
tokens, out_buf rows, positions, slots and length, the step counter and
the new cache rows. The kernels are the same; only where the hand-over
words live differs.
"""

import pytest
import torch

from enginekernel_amd import _hip
from enginekernel_amd import checkpoint as C
from enginekernel_amd import ek_kernels as K
from enginekernel_amd.ek_model import Qwen3

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    _hip.load()
    return torch.device("cuda:0")


def _inputs(cfg, dev, ctx, s_cap, seed, b=1):
    g = torch.Generator().manual_seed(seed)
    shape = (b, cfg["num_key_value_heads"], s_cap, cfg["head_dim"])
    k = [(torch.randn(shape, generator=g) * 0.5).to(BF).to(dev) for _ in range(cfg["num_hidden_layers"])]
    v = [(torch.randn(shape, generator=g) * 0.5).to(BF).to(dev) for _ in range(cfg["num_hidden_layers"])]
    st = dict(tokens=torch.randint(0, cfg["vocab_size"], (b,), generator=g).to(dev),
              positions=torch.full((b,), ctx, dtype=torch.int64, device=dev),
              len_t=torch.full((1,), ctx, dtype=torch.int64, device=dev),
              slot_t=torch.zeros(b, dtype=torch.int64, device=dev),
              start_t=torch.zeros(b, dtype=torch.int32, device=dev),
              out_buf=torch.full((8, b), -7, dtype=torch.int32, device=dev),
              step_idx=torch.zeros(1, dtype=torch.int64, device=dev),
              err=torch.zeros(1, dtype=torch.int32, device=dev))
    return k, v, st


def _run(model, k, v, st, s_cap, steps, noalloc):
    cfg = model.cfg
    b = int(st["tokens"].numel())
    table = model._layer_table(k, v)
    out_tok = torch.zeros(b, dtype=torch.int64, device=k[0].device)
    logits = torch.empty(steps, b, cfg.vocab_size, dtype=BF, device=k[0].device)
    scratch = None
    if not noalloc:
        plan = K.decode_step_plan(cfg.hidden_size, cfg.intermediate_size, cfg.num_heads, cfg.num_kv_heads,
                                  cfg.head_dim, cfg.vocab_size, b, s_cap, cfg.num_layers)
        assert plan is not None
        scratch = K.StepScratch(plan, k[0].device)
    for i in range(steps):
        common = (table, cfg, model.embed, model.lm_head, model.final_norm, model.cos, model.sin, k[0], s_cap,
                  st["tokens"], st["positions"], st["len_t"], st["slot_t"], st["start_t"], st["out_buf"],
                  st["step_idx"])
        if noalloc:
            K.decode_step_noalloc(*common, st["err"], out_tok=out_tok, logits=logits[i])
        else:
            K.decode_step(*common, scratch, out_tok=out_tok, logits=logits[i], err=st["err"])
    torch.cuda.synchronize()
    return logits, out_tok


# (rows, layers, context, cache keys, seed, split attention at batch 1)
CALLS = [(4, 36, 100, 128, 8, None),     # the batch kernel, an arena of 15.8 MiB
         (2, 3, 200, 256, 9, None),      # the batch kernel at 2 rows
         (1, 3, 3000, 4096, 5, True),    # batch 1, split attention
         (1, 3, 300, 512, 7, False),
         (1, 2, 40, 64, 6, False)]


@pytest.mark.parametrize("call", range(len(CALLS)))
def test_noalloc_step_equals_the_arena_step(dev, call):
    b, layers, ctx, s_cap, seed, split = CALLS[call]
    cfg = dict(C.QWEN3_4B, num_hidden_layers=layers)
    model = Qwen3(None, dev, tensors=C.random_weights(cfg, seed=seed), config=cfg)
    plan = model.persistent_plan(b, s_cap)
    assert plan is not None
    if b == 1:
        assert (plan[1] > 0) == split
    sizes = K.decode_step_plan(cfg["hidden_size"], cfg["intermediate_size"], cfg["num_attention_heads"],
                               cfg["num_key_value_heads"], cfg["head_dim"], cfg["vocab_size"], b, s_cap, layers)
    assert sizes is not None and sizes[0] <= 16 << 20
    print(f"no-alloc step: call {call}, {b} rows, {layers} layers, context {ctx}, cache {s_cap}, "
          f"arena {sizes[0] / 2**20:.2f} MiB", flush=True)
    k_a, v_a, st_a = _inputs(cfg, dev, ctx, s_cap, seed, b)
    k_b, v_b = [t.clone() for t in k_a], [t.clone() for t in v_a]
    st_b = {n: t.clone() for n, t in st_a.items()}
    with torch.inference_mode():
        lg_a, tok_a = _run(model, k_a, v_a, st_a, s_cap, 3, noalloc=False)
        lg_b, tok_b = _run(model, k_b, v_b, st_b, s_cap, 3, noalloc=True)
    assert int(st_a["err"]) == 0 and int(st_b["err"]) == 0
    assert torch.equal(lg_a, lg_b)
    assert torch.equal(tok_a, tok_b)
    for n in st_a:
        assert torch.equal(st_a[n], st_b[n]), n
    assert int(st_b["step_idx"]) == 3 and int(st_b["len_t"]) == ctx + 3
    assert (st_b["out_buf"][:3] >= 0).all() and (st_b["out_buf"][3:] == -7).all()
    for a, b in zip(k_a + v_a, k_b + v_b):
        assert torch.equal(a, b)


def test_noalloc_rejects_an_arena_beyond_the_static_limit(dev):
    """A shape whose hand-over arena exceeds the static 16 MiB is refused
    with an error before anything is launched (4 rows through 40 layers of
    the 4B shape need about 17.6 MiB); the step's plan itself stops at 64
    layers (its layer table is held in LDS). Every
    pointer argument is NULL: were the size check lost, the launch would
    still be refused (null pointers), and the message would not name the
    16 MiB limit."""
    cfg = dict(C.QWEN3_4B)
    assert K.decode_step_plan(2560, 9728, 32, 8, 128, cfg["vocab_size"], 1, 64, 65) is None
    plan = K.decode_step_plan(2560, 9728, 32, 8, 128, cfg["vocab_size"], 4, 64, 40)
    assert plan is not None and plan[0] > 16 << 20
    lib = _hip.load()
    p = None
    rc = lib.ek_decode_step_noalloc(p, 40, 2560, 9728, 32, 8, 128, cfg["vocab_size"], 4, 1e-6, 0.088,
                                    p, 2560, p, p, p, p, 128, 64, 0, 0, 128, 64,
                                    p, p, p, p, p, p, p, 8, p, p, p, p)
    assert rc != 0
    assert b"16 MiB" in lib.ek_last_error()
