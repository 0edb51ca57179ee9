"""End-to-end parity of the HIP decode path with the CPU oracle.

Criteria: greedy token ids identical to the oracle's
torch-fallback loop; logits within 2e-2 of scale. The prefill is not part
of the hot path (it runs torch projections and an fp32 attention on the
GPU), so the decode-only tests start both sides from the oracle's own
prefill KV cache and teacher-force the oracle's tokens.
"""

import pytest
import torch

from enginekernel_amd import checkpoint as C
from enginekernel_amd import ek_kernels as K
from enginekernel_amd.ek_model import Qwen3
from enginekernel_amd.engine import Engine
from oracle import ek_oracle as O
from tests.hf_ref import equivalence_cases

pytestmark = pytest.mark.gpu
BF = torch.bfloat16

MID_4B = dict(C.QWEN3_4B, num_hidden_layers=2)   # every Qwen3-4B shape, two layers


def _ulp(x):
    a = x.abs().double().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


@pytest.fixture(scope="module")
def tiny_ckpt(tmp_path_factory):
    p = tmp_path_factory.mktemp("tiny")
    C.write_checkpoint(str(p), dict(C.QWEN3_TINY), seed=0)
    return str(p)


def test_engine_tiny_tokens_equal_oracle(dev, tiny_ckpt):
    eng = Engine(tiny_ckpt)
    assert eng.tier == "hip"
    om = O.OracleQwen3.from_path(tiny_ckpt)
    for name, prompts, n in equivalence_cases(1024):
        got = list(eng.generate(prompts, n))
        want = list(O.generate_eager(om, prompts, n))
        assert len(got) == n and all(len(s) == len(prompts) for s in got)
        assert got == want, name


def test_graph_path_equals_eager_hip_path(dev, tiny_ckpt):
    eng = Engine(tiny_ckpt)
    prompts = equivalence_cases(1024)[2][1]
    ids, pos, pad, s, bias = eng._impl._pack(prompts)
    eager = list(eng._impl._generate_eager(ids, pos, pad, s, bias, 12))
    assert list(eng.generate(prompts, 12)) == eager


def _decode_parity(cfg, tensors, prompts, steps, dev):
    """Both sides start from the oracle's prefill cache; the oracle's tokens
    are fed back to both. Returns per-step (rel logit error, tokens agree)."""
    om = O.OracleQwen3(O.OracleConfig(cfg), tensors)
    gm = Qwen3(None, dev, tensors=tensors, config=cfg)
    ids, pos, pad, s, bias = O.pack(prompts)
    b = len(prompts)
    total = s + steps + 1
    st = O.EagerState(om, b, s, pad, total)
    om.ensure_rope(total + 1)
    with torch.inference_mode():
        hidden = om.prefill(ids, pos, st.k, st.v, bias)
        tok = O.argmax_token(hidden, om.lm_head)
        kd = [t.to(dev) for t in st.k]
        vd = [t.to(dev) for t in st.v]
        positions = st.positions.to(dev)
        slot_t = torch.zeros(b, dtype=torch.int64, device=dev)
        len_t = torch.full((1,), s, dtype=torch.int64, device=dev)
        start_t = torch.as_tensor(pad, dtype=torch.int32, device=dev)
        ws = K.make_workspace(b, cfg["num_attention_heads"], cfg["num_key_value_heads"],
                              cfg.get("head_dim"), total, dev)
        out = []
        for _ in range(steps):
            h_ref = om.decode(tok, st.positions, st.k, st.v, st.slot_t, st.len_t, st.start_t)
            l_ref = O.lm_logits(h_ref, om.lm_head)
            h = gm.decode(tok.to(dev), positions, kd, vd, slot_t, len_t, start_t, ws)
            logits = torch.empty(b, cfg["vocab_size"], dtype=BF, device=dev)
            t_gpu = gm.argmax_token(h, logits=logits).cpu()
            err = (logits.cpu().float() - l_ref.float()).abs().max().item() / l_ref.float().abs().max().item()
            t_ref = torch.argmax(l_ref, -1)
            agree = torch.equal(t_gpu, t_ref)
            if not agree:     # only a near-tie of the oracle's own logits may differ
                for i in range(b):
                    if t_gpu[i] != t_ref[i]:
                        gap = (l_ref[i, t_ref[i]].float() - l_ref[i, t_gpu[i]].float()).item()
                        assert gap <= 2 * _ulp(l_ref[i, t_ref[i]].double()).item(), (gap, i)
            out.append((err, agree))
            tok = t_ref
            st.positions = st.positions + 1
            positions = positions + 1
        assert torch.equal(len_t.cpu(), st.len_t)
        # the prefill slots are untouched; the slots the decode wrote agree
        # with the oracle's. Layer 0 sees identical inputs (the embedding
        # rows), so its new values are the same rounded projections (>= 99%
        # bitwise); deeper layers inherit ulp-level residual differences and
        # are held to the scale bound
        n = int(st.len_t.item())
        for i in range(cfg["num_hidden_layers"]):
            for bi in range(b):
                for got_c, ref_c in ((kd[i], st.k[i]), (vd[i], st.v[i])):
                    assert torch.equal(got_c[bi, :, :s].cpu(), ref_c[bi, :, :s])
                    a = got_c[bi, :, s:n].cpu().float()
                    r = ref_c[bi, :, s:n].float()
                    assert (a - r).abs().max().item() <= 2e-2 * r.abs().max().item()
            a = vd[0][:, :, s:n].cpu()
            if i == 0:
                assert (a == st.v[0][:, :, s:n]).float().mean().item() >= 0.99
    return out


def test_decode_parity_tiny(dev):
    cfg = dict(C.QWEN3_TINY)
    tensors = C.random_weights(cfg, seed=0)
    prompts = equivalence_cases(1024)[3][1]      # config 1: lengths 5/9/16
    res = _decode_parity(cfg, tensors, prompts, 31, dev)
    assert max(e for e, _ in res) <= 2e-2
    assert all(a for _, a in res)


def test_decode_parity_4b_shapes(dev):
    """Every Qwen3-4B shape (H 2560, I 9728, 32/8 heads, D 128, vocab
    151936), two layers, batch 1 and a ragged batch of 3."""
    cfg = dict(MID_4B)
    tensors = C.random_weights(cfg, seed=0)
    g = torch.Generator().manual_seed(1)
    for prompts in ([torch.randint(0, 151936, (128,), generator=g).tolist()],
                    [torch.randint(0, 151936, (n,), generator=g).tolist() for n in (64, 100, 37)]):
        res = _decode_parity(cfg, tensors, prompts, 8, dev)
        assert max(e for e, _ in res) <= 2e-2, res


def test_engine_4b_shapes_tokens(dev):
    """Free-running greedy through the captured graph at the 4B shapes vs the
    oracle loop; a divergence is accepted only at a near-tie, and the
    teacher-forced test above pins every step's logits."""
    cfg = dict(MID_4B)
    tensors = C.random_weights(cfg, seed=0)
    model = Qwen3(None, dev, tensors=tensors, config=cfg)
    eng = Engine(model=model)
    om = O.OracleQwen3(O.OracleConfig(cfg), tensors)
    g = torch.Generator().manual_seed(2)
    prompts = [torch.randint(0, 151936, (32,), generator=g).tolist()]
    got = list(eng.generate(prompts, 16))
    want = list(O.generate_eager(om, prompts, 16))
    assert got[0] == want[0]              # the prefill's first token
    assert got == want


def test_decode_parity_full_depth_against_the_noise_floor(dev):
    """The full 36-layer Qwen3-4B shape, 12 teacher-forced steps. Through 36
    random-init layers an fp32 summation-order change alone moves the
    oracle's own logits by ~0.13 (0.03 at 2 layers): that drift, measured
    here by re-running the oracle with its projections accumulated in a
    different order (fp32 upcast matmul), is the noise floor. The HIP path
    must stay within 1.5x that floor plus 2 bf16 ulps, and may pick a
    different token only where the oracle's own top-2 gap is <= 2 ulps."""
    cfg = dict(C.QWEN3_4B)
    tensors = C.random_weights(cfg, seed=0)
    om = O.OracleQwen3(O.OracleConfig(cfg), tensors)
    gm = Qwen3(None, dev, tensors=tensors, config=cfg)
    g = torch.Generator().manual_seed(1)
    prompts = [torch.randint(0, 151936, (128,), generator=g).tolist()]
    ids, pos, pad, s, bias = O.pack(prompts)
    steps = 12
    total = s + steps + 1
    st = O.EagerState(om, 1, s, pad, total)
    with torch.inference_mode():
        hidden = om.prefill(ids, pos, st.k, st.v, bias)
        tok = O.argmax_token(hidden, om.lm_head)
        st2 = O.EagerState(om, 1, s, pad, total)
        st2.k = [t.clone() for t in st.k]
        st2.v = [t.clone() for t in st.v]
        kd = [t.to(dev) for t in st.k]
        vd = [t.to(dev) for t in st.v]
        positions = st.positions.to(dev)
        slot_t = torch.zeros(1, dtype=torch.int64, device=dev)
        len_t = torch.full((1,), s, dtype=torch.int64, device=dev)
        start_t = torch.zeros(1, dtype=torch.int32, device=dev)
        ws = K.make_workspace(1, 32, 8, 128, total, dev)
        proj = om._proj
        reordered = lambda x, layer, key: torch.matmul(x.float(), layer[key].float().t()).to(BF)
        agree = 0
        for _ in range(steps):
            om._proj = proj
            l_ref = O.lm_logits(om.decode(tok, st.positions, st.k, st.v, st.slot_t, st.len_t, st.start_t),
                                om.lm_head).float()[0]
            om._proj = reordered
            l_alt = O.lm_logits(om.decode(tok, st2.positions, st2.k, st2.v, st2.slot_t, st2.len_t,
                                          st2.start_t), om.lm_head).float()[0]
            h = gm.decode(tok.to(dev), positions, kd, vd, slot_t, len_t, start_t, ws)
            logits = torch.empty(1, 151936, dtype=BF, device=dev)
            t_gpu = int(gm.argmax_token(h, logits=logits)[0])
            floor = (l_alt - l_ref).abs().max().item()
            err = (logits.cpu().float()[0] - l_ref).abs().max().item()
            ulp = _ulp(l_ref.max().double()).item()
            assert err <= 1.5 * floor + 2 * ulp, (err, floor)
            t_ref = int(torch.argmax(l_ref))
            if t_gpu == t_ref:
                agree += 1
            else:
                assert (l_ref[t_ref] - l_ref[t_gpu]).item() <= 2 * ulp
            tok = torch.tensor([t_ref])
            for x in (st, st2):
                x.positions = x.positions + 1
            positions = positions + 1
        om._proj = proj
    assert agree >= steps - 2
