"""Pins the CPU oracle (oracle/ek_oracle.py) before anything is compared to it.

Each oracle function is checked against something other than its own
formula: transformers' Qwen3ForCausalLM (token-exact greedy, the reference's
bench/test_equivalence.py check), transformers' Qwen3RMSNorm / rotary
embedding / apply_rotary_pos_emb (bitwise), float64 closed forms, brute-force
softmax, and attention special cases. The `planted_*` tests mutate the
oracle on the CPU and require the checks above to fail, so a dropped term,
a flipped sign or an off-by-one cannot pass unnoticed.
"""

import math

import pytest
import torch

from enginekernel_amd.checkpoint import QWEN3_TINY, random_weights
from oracle import ek_oracle as O
from tests.hf_ref import equivalence_cases, hf_greedy, hf_model

BF = torch.bfloat16


def _ulp(x):
    """bf16 spacing at each element's magnitude (fp64)."""
    a = x.abs().double().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


@pytest.fixture(scope="module")
def tiny():
    cfg = dict(QWEN3_TINY)
    t = random_weights(cfg, seed=0)
    return cfg, t, O.OracleQwen3(O.OracleConfig(cfg), t), hf_model(cfg, t)


@pytest.fixture(scope="module")
def ref_tiny():
    """The reference test's own tiny shape (vocab 512, I 256)."""
    cfg = dict(QWEN3_TINY, vocab_size=512, intermediate_size=256)
    t = random_weights(cfg, seed=0)
    return cfg, t, O.OracleQwen3(O.OracleConfig(cfg), t), hf_model(cfg, t)


# ----------------------------------------------------------------------------
# end to end: token-exact against transformers (bench/test_equivalence.py)
# ----------------------------------------------------------------------------
@pytest.mark.parametrize("which", ["tiny", "ref_tiny"])
def test_oracle_greedy_matches_transformers(which, request):
    cfg, _, om, hm = request.getfixturevalue(which)
    for name, prompts, n in equivalence_cases(cfg["vocab_size"]):
        got = list(O.generate_eager(om, prompts, n))
        want = hf_greedy(hm, prompts, n)
        assert got == want, name


def _teacher_forced_rel_errs(om, hm, vocab, n=6):
    """Per step: max |oracle logit - HF logit| / max |HF logit|, where HF
    runs a full forward (no cache) over the same prefix the oracle decoded."""
    prompts = equivalence_cases(vocab)[2][1]   # ragged batch 3
    steps = list(O.generate_eager(om, prompts, n, record_logits=True))
    toks = [st[0] for st in steps]
    b, s = len(prompts), max(len(p) for p in prompts)
    errs = []
    for j in range(n):
        rows = [prompts[i] + [toks[t][i] for t in range(j)] for i in range(b)]
        ids = torch.zeros((b, s + j), dtype=torch.long)
        mask = torch.zeros_like(ids)
        for i, r in enumerate(rows):
            ids[i, s + j - len(r):] = torch.as_tensor(r)
            mask[i, s + j - len(r):] = 1
        pos = (mask.cumsum(-1) - 1).clamp(min=0)
        with torch.inference_mode():
            ref = hm(input_ids=ids, attention_mask=mask, position_ids=pos).logits[:, -1, :].float()
        errs.append((steps[j][1].float() - ref).abs().max().item() / ref.abs().max().item())
    return errs


def test_oracle_logits_match_transformers_forward(tiny):
    """Teacher-forced: the oracle's per-step bf16 logits equal HF's full
    forward over the same prefix to ~1 bf16 ulp (observed 0.6% of scale)."""
    cfg, _, om, hm = tiny
    assert max(_teacher_forced_rel_errs(om, hm, cfg["vocab_size"])) <= 1e-2


# ----------------------------------------------------------------------------
# kernel-level closed forms
# ----------------------------------------------------------------------------
def test_rms_norm_closed_form_and_hf():
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm
    g = torch.Generator().manual_seed(0)
    for scale in (1.0, 1e-3):          # 1e-3: mean(x^2) ~ eps, so eps matters
        x = (torch.randn(64, 2560, generator=g) * scale).to(BF)
        w = (1 + 0.1 * torch.randn(2560, generator=g)).to(BF)
        y = O.rms_norm(x, w, 1e-6)
        x64 = x.double()
        ref = w.double() * (x64 / torch.sqrt(x64.pow(2).mean(-1, keepdim=True) + 1e-6))
        assert ((y.double() - ref).abs() <= 2 * _ulp(ref) + 1e-30).all()
        hf = Qwen3RMSNorm(2560, eps=1e-6)
        hf.weight.data = w.clone()
        assert torch.equal(hf(x), y)


def test_add_rms_norm_residual_is_bf16_add():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4, 256, generator=g).to(BF)
    r = torch.randn(4, 256, generator=g).to(BF)
    w = torch.ones(256, dtype=BF)
    _, r2 = O.add_rms_norm(x, r, w, 1e-6)
    assert torch.equal(r2, (x.float() + r.float()).to(BF))


def test_silu_mul_rounding_points():
    g = torch.Generator().manual_seed(2)
    gu = (torch.randn(8, 2 * 384, generator=g) * 3).to(BF)
    y = O.silu_mul(gu)
    gt, up = gu.double().chunk(2, -1)
    s = (gt / (1 + torch.exp(-gt))).to(torch.float32).to(BF).double()   # bf16(silu) rounding point
    ref = s * up
    assert ((y.double() - ref).abs() <= _ulp(ref) / 2 + 1e-30).all()


def test_rope_tables_match_transformers_and_closed_form():
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding
    for d, theta in ((32, 1e6), (128, 5e6)):
        cos, sin = O.build_rope(d, theta, 4096)
        cfg = Qwen3Config(head_dim=d, hidden_size=d * 4, num_attention_heads=4,
                          rope_parameters={"rope_type": "default", "rope_theta": theta})
        emb = Qwen3RotaryEmbedding(cfg)
        pos = torch.arange(4096)[None]
        hc, hs = emb(torch.zeros(1, dtype=BF), pos)
        assert torch.equal(cos, hc[0]) and torch.equal(sin, hs[0])
        t = torch.arange(64, dtype=torch.float64)[:, None]
        inv = theta ** (-torch.arange(0, d, 2, dtype=torch.float64) / d)
        ang = torch.cat([t * inv, t * inv], -1)
        assert ((cos[:64].double() - torch.cos(ang)).abs() <= _ulp(torch.cos(ang)) + 1e-6).all()


def _qkv_case(m=4, nq=4, nkv=2, d=32, seed=3):
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(m, (nq + 2 * nkv) * d, generator=g).to(BF)
    qn = (1 + 0.2 * torch.randn(d, generator=g)).to(BF)
    kn = (1 + 0.2 * torch.randn(d, generator=g)).to(BF)
    cos, sin = O.build_rope(d, 1e6, 64)
    pos = torch.randint(0, 64, (m,), generator=g)
    return qkv, qn, kn, cos[pos], sin[pos]


def test_qk_norm_rope_kv_matches_hf_and_writes_only_its_slots():
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm, apply_rotary_pos_emb
    nq, nkv, d, b = 4, 2, 32, 4
    qkv, qn, kn, cos, sin = _qkv_case(b, nq, nkv, d)
    kc = torch.zeros(b, nkv, 16, d, dtype=BF)
    vc = torch.zeros_like(kc)
    slot = torch.full((b,), 7, dtype=torch.int64)
    got = qkv.clone()
    O.qk_norm_rope_kv(got, qn, kn, cos, sin, kc, vc, slot, nq, nkv, 1e-6, 1)
    qnorm, knorm = Qwen3RMSNorm(d, 1e-6), Qwen3RMSNorm(d, 1e-6)
    qnorm.weight.data, knorm.weight.data = qn.clone(), kn.clone()
    q = qnorm(qkv[:, :nq * d].view(b, nq, d)).transpose(0, 1)        # [heads, b, d]
    k = knorm(qkv[:, nq * d:(nq + nkv) * d].view(b, nkv, d)).transpose(0, 1)
    qe, ke = apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=0)
    assert torch.equal(got[:, :nq * d].view(b, nq, d), qe.transpose(0, 1))
    assert torch.equal(kc[:, :, 7], ke.transpose(0, 1))
    assert torch.equal(vc[:, :, 7], qkv[:, (nq + nkv) * d:].view(b, nkv, d))
    others = torch.cat([kc[:, :, :7], kc[:, :, 8:], vc[:, :, :7], vc[:, :, 8:]], 2)
    assert not others.any()


def _attn_case(b=2, hq=4, hkv=2, d=32, s=48, seed=4):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, d, generator=g).to(BF)
    kc = torch.randn(b, hkv, s, d, generator=g).to(BF)
    vc = torch.randn(b, hkv, s, d, generator=g).to(BF)
    return q, kc, vc


def test_decode_attn_brute_force_fp64():
    q, kc, vc = _attn_case()
    start = torch.tensor([0, 5], dtype=torch.int32)
    n = 40
    got = O.decode_attn(q, kc, vc, n, start, 32 ** -0.5).double()
    for bi in range(2):
        for h in range(4):
            kv = h // 2
            keys = range(int(start[bi]), n)
            s = [float((q[bi, h].double() * kc[bi, kv, j].double()).sum()) * 32 ** -0.5 for j in keys]
            mx = max(s)
            e = [math.exp(v - mx) for v in s]
            tot = sum(e)
            o = sum((e[i] / tot) * vc[bi, kv, j].double() for i, j in enumerate(keys))
            assert (got[bi, h] - o).abs().max() <= 2e-2 * o.abs().max()


def test_decode_attn_special_cases():
    q, kc, vc = _attn_case()
    start = torch.tensor([0, 0], dtype=torch.int32)
    # one key: softmax is exactly 1 -> the value row itself
    assert torch.equal(O.decode_attn(q, kc, vc, 1, start, 0.17)[:, ::2], vc[:, :, 0])
    # start = len - 1: only the last key is visible
    st = torch.tensor([39, 39], dtype=torch.int32)
    assert torch.equal(O.decode_attn(q, kc, vc, 40, st, 0.17)[:, 1::2], vc[:, :, 39])
    # constant keys: uniform weights -> the mean of the values
    kc2 = kc.clone()
    kc2[:] = kc[:, :, :1]
    got = O.decode_attn(q, kc2, vc, 32, start, 0.17).double()
    mean = vc[:, :, :32].double().mean(2).repeat_interleave(2, 1)
    assert (got - mean).abs().max() <= 1e-2
    # masked keys never contribute, whatever they hold
    st = torch.tensor([10, 3], dtype=torch.int32)
    vc3 = vc.clone()
    vc3[0, :, :10] = 1e4
    vc3[1, :, :3] = -1e4
    assert torch.equal(O.decode_attn(q, kc, vc, 40, st, 0.17), O.decode_attn(q, kc, vc3, 40, st, 0.17))


def test_argmax_first_index_on_ties():
    h = torch.ones(2, 8, dtype=BF)
    e = torch.zeros(16, 8, dtype=BF)
    e[3] = 1
    e[9] = 1            # ties with row 3
    assert O.argmax_token(h, e).tolist() == [3, 3]


def test_pack_layout():
    ids, pos, pad, s, bias = O.pack([[5, 6, 7], [9]])
    assert s == 3 and pad == [0, 2]
    assert ids.tolist() == [[5, 6, 7], [0, 0, 9]]
    assert pos.tolist() == [[0, 1, 2], [0, 0, 0]]
    allow = (bias[:, 0] == 0)
    assert allow[1].tolist() == [[False] * 3, [False] * 3, [False, False, True]]
    assert O.pack([[1, 2], [3, 4]])[4] is None


def test_config_reads_both_rope_theta_locations():
    d = dict(QWEN3_TINY)
    assert O.OracleConfig(d).rope_theta == 1e6
    d2 = {k: v for k, v in d.items() if k != "rope_theta"}
    d2["rope_parameters"] = {"rope_type": "default", "rope_theta": 5e6}
    assert O.OracleConfig(d2).rope_theta == 5e6


# ----------------------------------------------------------------------------
# planted mistakes: each mutation of the oracle must fail the checks above
# ----------------------------------------------------------------------------
def _mismatches(om, hm, vocab):
    bad = 0
    for _, prompts, n in equivalence_cases(vocab):
        bad += list(O.generate_eager(om, prompts, n)) != hf_greedy(hm, prompts, n)
    return bad


def test_planted_rotate_half_sign_is_caught(tiny, monkeypatch):
    cfg, _, om, hm = tiny
    orig = O.qk_norm_rope_kv

    def wrong_sign(qkv, qn, kn, cos, sin, *a):
        return orig(qkv, qn, kn, cos, -sin, *a)   # (-sin) == rot with the sign flipped
    monkeypatch.setattr(O, "qk_norm_rope_kv", wrong_sign)
    assert _mismatches(om, hm, cfg["vocab_size"]) > 0


def test_planted_dropped_pad_mask_is_caught(tiny, monkeypatch):
    cfg, _, om, hm = tiny
    orig = O.decode_attn
    monkeypatch.setattr(O, "decode_attn", lambda q, kc, vc, n, st, sc: orig(q, kc, vc, n, st * 0, sc))
    prompts = equivalence_cases(cfg["vocab_size"])[2][1]   # ragged
    assert list(O.generate_eager(om, prompts, 8)) != hf_greedy(hm, prompts, 8)


def test_planted_position_off_by_one_is_caught(tiny, monkeypatch):
    """Random-init attention is nearly uniform, so a RoPE position shifted by
    one in decode leaves the greedy ids alone; the teacher-forced logits
    catch it (observed ~7% of scale against a 1% bound)."""
    cfg, _, om, hm = tiny
    orig = om.decode
    monkeypatch.setattr(om, "decode", lambda tok, pos, *a: orig(tok, pos + 1, *a))
    assert max(_teacher_forced_rel_errs(om, hm, cfg["vocab_size"])) > 2e-2


def test_planted_unrounded_softmax_probabilities_change_logits(tiny, monkeypatch):
    """The p -> bf16 rounding point (ek_model.py:487) is observable: without
    it the decode logits move, so a kernel that skips it is distinguishable."""
    cfg, _, om, _ = tiny
    prompts = equivalence_cases(cfg["vocab_size"])[0][1]
    base = [s[1] for s in O.generate_eager(om, prompts, 4, record_logits=True)]

    def fp32_p(q, kc, vc, n, start_t, sm_scale):
        rep = q.shape[1] // kc.shape[1]
        k = kc[:, :, :n].repeat_interleave(rep, 1).float()
        v = vc[:, :, :n].repeat_interleave(rep, 1).float()
        s = torch.einsum("bhd,bhsd->bhs", q.float(), k) * sm_scale
        s = s.masked_fill(torch.arange(n)[None, None] < start_t[:, None, None], float("-inf"))
        return torch.einsum("bhs,bhsd->bhd", torch.softmax(s, -1), v).to(q.dtype)
    monkeypatch.setattr(O, "decode_attn", fp32_p)
    alt = [s[1] for s in O.generate_eager(om, prompts, 4, record_logits=True)]
    assert any(not torch.equal(a, b) for a, b in zip(base[1:], alt[1:]))
