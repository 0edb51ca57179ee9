"""Speculative decoding on the HIP kernels against the CPU oracle.

The draft and accept kernels are integer work: bit-exact against the
oracle's restatement (engine.py:357-383, ek_kernels.py:618-680). The verify
attention is the prefill flash kernel with a per-row query offset: within a
few bf16 ulps of the oracle's verify attention (attn_torch, fp32 softmax). A
verify pass as a whole must give, at each of its positions, the token a
teacher-forced sequential decode gives (up to <= 2-ulp near-ties), and the
speculative engine the same greedy tokens as the plain one.
"""

import random

import pytest
import torch

from enginekernel_amd import checkpoint as C
from enginekernel_amd import ek_kernels as K
from enginekernel_amd.ek_model import Qwen3
from enginekernel_amd.engine import Engine
from oracle import ek_oracle as O

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
MID_4B = dict(C.QWEN3_4B, num_hidden_layers=2)


def _ulp(x):
    a = x.abs().double().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


@pytest.mark.parametrize("q", [2, 3, 5, 8, 16])
def test_ngram_draft_bit_exact(dev, q):
    rng = random.Random(q)
    b, h = 37, 512
    alphabet = [2, 3, 7, 151936]
    hist = torch.tensor([[rng.randrange(alphabet[r % 4]) for _ in range(h)] for r in range(b)], dtype=torch.int64)
    hist_len = torch.tensor([[1, 2, 3, h, h - 1][r] if r < 5 else rng.randint(3, h) for r in range(b)],
                            dtype=torch.int64)
    want = O.ngram_draft(hist, hist_len, q)
    tokens = torch.full((b, q), -7, dtype=torch.int64, device=dev)
    K.ngram_draft(hist.to(dev), hist_len.to(dev), tokens)
    assert torch.equal(tokens.cpu(), want)


@pytest.mark.parametrize("q", [2, 3, 8])
def test_spec_accept_bit_exact(dev, q):
    rng = random.Random(100 + q)
    b, h, steps = 29, 64, 6
    tokens = torch.tensor([[rng.randrange(4) for _ in range(q)] for _ in range(b)], dtype=torch.int64)
    am = torch.tensor([[rng.randrange(4) for _ in range(q)] for _ in range(b)], dtype=torch.int64)
    for r in range(0, b, 5):            # rows whose drafts all match
        am[r, : q - 1] = tokens[r, 1:]
    hist = torch.tensor([[rng.randrange(9) for _ in range(h)] for _ in range(b)], dtype=torch.int64)
    hist_len = torch.tensor([rng.choice([h - 1, h, 3, 30]) for _ in range(b)], dtype=torch.int64)
    len_b = torch.tensor([rng.randrange(1000) for _ in range(b)], dtype=torch.int64)
    pos_b = torch.tensor([rng.randrange(1000) for _ in range(b)], dtype=torch.int64)
    remaining = torch.tensor([rng.choice([0, 1, 2, 100]) for _ in range(b)], dtype=torch.int64)
    for step in (3, steps + 2):         # in range, and past the output ring (no output stores)
        want = [t.clone() for t in (hist, hist_len, len_b, pos_b, remaining)]
        w_tok = torch.zeros((steps, b, q), dtype=torch.int32)
        w_adv = torch.zeros((steps, b), dtype=torch.int32)
        O.spec_accept(tokens, am, *want, w_tok, w_adv, step)
        got = [t.to(dev) for t in (hist, hist_len, len_b, pos_b, remaining)]
        g_tok = torch.zeros((steps, b, q), dtype=torch.int32, device=dev)
        g_adv = torch.zeros((steps, b), dtype=torch.int32, device=dev)
        step_idx = torch.tensor([step], dtype=torch.int64, device=dev)
        K.spec_accept(tokens.to(dev), am.to(dev), *got, g_tok, g_adv, step_idx)
        for a, w in zip(got, want):
            assert torch.equal(a.cpu(), w)
        assert torch.equal(g_tok.cpu(), w_tok) and torch.equal(g_adv.cpu(), w_adv)
        assert int(step_idx) == step


@pytest.mark.parametrize("d,g,lens,starts,nq", [(128, 4, (57, 300), (0, 11), 3), (64, 2, (1, 200), (0, 0), 5),
                                                (32, 8, (31, 32), (3, 0), 8), (128, 1, (700, 129), (5, 40), 2)])
def test_attn_verify_matches_oracle(dev, d, g, lens, starts, nq):
    torch.manual_seed(d + g)
    b, n_kv, cap = 2, 2, 1024
    n_q = n_kv * g
    kc = torch.randn(b, n_kv, cap, d).to(BF)
    vc = torch.randn(b, n_kv, cap, d).to(BF)
    qkv = torch.randn(b * nq, (n_q + 2 * n_kv) * d).to(BF)
    q = qkv[:, : n_q * d].reshape(b * nq, n_q, d)
    len_b = torch.tensor(lens, dtype=torch.int64)
    start = torch.tensor(starts, dtype=torch.int32)
    scale = d ** -0.5
    outs = [K.attn_verify(qkv.to(dev), kc.to(dev), vc.to(dev), start.to(dev), len_b.to(dev), nq, n_q, scale,
                          splits=sp).cpu() for sp in (1, 3, None, 32)]
    got = outs[0]
    # float64 softmax attention over keys [start_b, len_b + j]
    want = torch.empty(b * nq, n_q * d, dtype=torch.float64)
    for r in range(b):
        for j in range(nq):
            hi = int(len_b[r]) + j + 1
            for hh in range(n_q):
                kv = hh // g
                sc = (kc[r, kv, int(start[r]):hi].double() @ q[r * nq + j, hh].double()) * scale
                want[r * nq + j, hh * d:(hh + 1) * d] = torch.softmax(sc, 0) @ vc[r, kv, int(start[r]):hi].double()
    # elementwise: probabilities are rounded to bf16 (2^-9 relative) before the value sum
    bound = 2.0 ** -7 * want.abs() + 2.0 ** -8 * vc.float().abs().max().item()
    err = (got.double() - want).abs()
    assert (err <= bound).all(), err.max().item()
    # and the oracle's restatement of the reference's torch form (bf16 scores)
    ref = O.verify_attn(q, kc, vc, len_b, start, scale, nq).float().reshape(b * nq, n_q * d)
    assert (got.float() - ref).abs().max().item() <= 2e-2 * ref.abs().max().item()
    # key splits (3, the default plan's, 32): the same bound against float64
    for o in outs[1:]:
        err = (o.double() - want).abs()
        assert (err <= bound).all(), err.max().item()


def test_verify_equals_teacher_forced_decode(dev):
    """A verify pass over [t, d1 .. d4] from the oracle's prefill cache gives,
    at each position, the oracle's argmax after a sequential decode of the
    same tokens (up to a <= 2-ulp near-tie), and writes the same K/V rows."""
    cfg = dict(MID_4B)
    tensors = C.random_weights(cfg, seed=0)
    om = O.OracleQwen3(O.OracleConfig(cfg), tensors)
    gm = Qwen3(None, dev, tensors=tensors, config=cfg)
    g = torch.Generator().manual_seed(5)
    prompt = torch.randint(0, cfg["vocab_size"], (61,), generator=g).tolist()
    nq = 5
    ids, pos, pad, s, bias = O.pack([prompt])
    st = O.EagerState(om, 1, s, pad, s + nq + 8)
    with torch.inference_mode():
        hidden = om.prefill(ids, pos, st.k, st.v, bias)
        first = O.argmax_token(hidden, om.lm_head)
        kd = [t.to(dev) for t in st.k]
        vd = [t.to(dev) for t in st.v]
        drafts = torch.randint(0, cfg["vocab_size"], (nq - 1,), generator=g).tolist()
        seq = [int(first[0])] + drafts
        refs = []
        for j, t in enumerate(seq):
            hid = om.decode(torch.tensor([t]), st.positions, st.k, st.v, st.slot_t, st.len_t, st.start_t)
            refs.append(O.lm_logits(hid, om.lm_head).float()[0])
            st.positions = st.positions + 1
        tokens = torch.tensor([seq], dtype=torch.int64, device=dev)
        pos_b = torch.tensor([s], dtype=torch.int64, device=dev)
        len_b = torch.tensor([s], dtype=torch.int64, device=dev)
        start_t = torch.zeros(1, dtype=torch.int32, device=dev)
        am = gm.verify(tokens, pos_b, kd, vd, len_b, start_t).cpu()[0].tolist()
    for j, l_ref in enumerate(refs):
        t_ref = int(torch.argmax(l_ref))
        if am[j] != t_ref:
            assert (l_ref[t_ref] - l_ref[am[j]]).item() <= 2 * _ulp(l_ref.max()).item(), (j, am[j], t_ref)
    for got_c, ref_c in ((kd[1], st.k[1]), (vd[1], st.v[1])):
        assert torch.equal(got_c[0, :, :s].cpu(), ref_c[0, :, :s])
        a = got_c[0, :, s:s + nq].cpu().float()
        r = ref_c[0, :, s:s + nq].float()
        assert (a - r).abs().max().item() <= 2e-2 * r.abs().max().item()


@pytest.fixture(scope="module")
def tiny_ckpt(tmp_path_factory):
    p = tmp_path_factory.mktemp("tiny_spec")
    C.write_checkpoint(str(p), dict(C.QWEN3_TINY), seed=0)
    return str(p)


@pytest.mark.parametrize("prompt_kind", ["repeating", "random"])
def test_speculative_generate_equals_plain(dev, tiny_ckpt, prompt_kind):
    """The speculative path emits the plain path's greedy tokens (and, on a
    repeating prompt, needs fewer verify steps than tokens)."""
    eng = Engine(tiny_ckpt)
    rng = random.Random(7)
    if prompt_kind == "repeating":
        prompt = [rng.randrange(1024) for _ in range(9)] * 6
    else:
        prompt = [rng.randrange(1024) for _ in range(50)]
    n = 48
    eng._impl.spec = False
    plain = list(eng.generate([prompt], n))
    eng._impl.spec = True
    spec = list(eng.generate([prompt], n))
    steps, target = eng._impl.last_stats
    assert spec == plain
    assert target == n - 1 and 1 <= steps <= target
    again = list(eng.generate([prompt], n))   # the captured graph, replayed for a second request
    assert again == plain


def test_speculative_capture_failure_falls_back_to_plain(dev, tiny_ckpt, monkeypatch):
    """engine.py:640-649: when the speculative graph cannot be built for a
    shape, the request runs on the plain captured step instead of failing."""
    from enginekernel_amd import engine as E
    eng = Engine(tiny_ckpt)
    prompt = [random.Random(3).randrange(1024) for _ in range(30)]
    eng._impl.spec = False
    plain = list(eng.generate([prompt], 24))

    def refuse(self, b, bucket):
        raise RuntimeError("speculative graph capture refused")

    monkeypatch.setattr(E._FastEngine, "_capture_spec", refuse)
    eng._impl.spec = True
    got = list(eng.generate([prompt], 24))
    assert got == plain
    assert not any(key[0] == "spec" for key in eng._impl.graphs)
    assert eng._impl.last_stats == (23, 23)          # plain steps: one replay per token


@pytest.mark.parametrize("prompt_kind", ["repeating", "random"])
def test_speculative_engine_4b_shapes_near_ties(dev, prompt_kind):
    """Free-running speculative greedy at the 4B shapes vs the oracle loop fed
    the same tokens (bench/check_exact.py's rule): every token is the oracle's
    argmax for its history, or within 2 bf16 ulps of the oracle's top logit."""
    cfg = dict(MID_4B)
    tensors = C.random_weights(cfg, seed=0)
    model = Qwen3(None, dev, tensors=tensors, config=cfg)
    eng = Engine(model=model)
    eng._impl.spec = True
    om = O.OracleQwen3(O.OracleConfig(cfg), tensors)
    g = torch.Generator().manual_seed(4)
    phrase = torch.randint(0, 151936, (8,), generator=g).tolist()
    prompt = phrase * 5 if prompt_kind == "repeating" else torch.randint(0, 151936, (40,), generator=g).tolist()
    got = list(eng.generate([prompt], 20))
    steps, target = eng._impl.last_stats
    assert target == 19 and 1 <= steps <= 19
    ref = list(O.generate_eager(om, [prompt], 20, record_logits=True, force=got[:-1]))
    agree = 0
    for j, (toks, logits) in enumerate(ref):
        top = int(torch.argmax(logits[0]))
        if got[j][0] == top:
            agree += 1
            continue
        lr = logits[0].float()
        assert float(lr[top] - lr[got[j][0]]) <= 2 * _ulp(logits[0, top].double()).item(), (j, got[j], toks)
    assert agree >= 18, agree
