"""Pins the oracle's speculative-decoding restatements (CPU only).

- ngram_draft against an independent statement of its rule: search the
  trailing 3-gram, then 2-gram, then token, for its latest earlier
  occurrence, and continue from there (the oracle restates the reference's
  score arithmetic instead: (j + 1) + 2^20 [2-gram] + 2^21 [3-gram]);
- spec_accept against hand-worked cases;
- the verify attention against the single-query decode attention: query j
  of a verify step is a decode at length len + j + 1.
"""

import random

import torch

from oracle import ek_oracle as O


def _draft_by_search(row, hl, q, h):
    """The draft rule stated as a search: longest n-gram order first, then
    the latest position j <= hl - 2 where the trailing n-gram ends."""
    p = 0
    for n in (3, 2, 1):
        if hl < n:
            continue
        tail = row[hl - n:hl]
        found = [j for j in range(hl - 1) if j - n + 1 >= 0 and row[j - n + 1:j + 1] == tail]
        # order 2 and 3 also count a partial window at the row start as no match
        if found:
            p = max(found) + 1
            break
    span = max(hl - p, 1)
    return [row[hl - 1]] + [row[min(p + i % span, h - 1)] for i in range(q - 1)]


def test_ngram_draft_matches_search_rule():
    rng = random.Random(0)
    for trial in range(400):
        h = rng.choice([8, 16, 33, 64])
        alphabet = rng.choice([2, 3, 5, 50])
        b = rng.choice([1, 3])
        hist = torch.tensor([[rng.randrange(alphabet) for _ in range(h)] for _ in range(b)], dtype=torch.int64)
        hist_len = torch.tensor([rng.randint(3, h) for _ in range(b)], dtype=torch.int64)
        q = rng.choice([2, 3, 5, 8])
        got = O.ngram_draft(hist, hist_len, q)
        for r in range(b):
            want = _draft_by_search(hist[r].tolist(), int(hist_len[r]), q, h)
            assert got[r].tolist() == want, (trial, r)


def test_ngram_draft_cases():
    # no earlier occurrence: p = 0, the draft replays the row from its start
    hist = torch.tensor([[10, 11, 12, 13, 0, 0, 0, 0]])
    assert O.ngram_draft(hist, torch.tensor([4]), 4).tolist() == [[13, 10, 11, 12]]
    # a cycle of period 3: the latest 3-gram match is one period back and the
    # draft wraps around it
    hist = torch.tensor([[1, 2, 3, 1, 2, 3, 1, 2, 0, 0]])
    assert O.ngram_draft(hist, torch.tensor([8]), 5).tolist() == [[2, 3, 1, 2, 3]]
    # a 3-gram match beats a later 1-gram match
    hist = torch.tensor([[7, 8, 9, 4, 9, 5, 7, 8, 9]])
    assert O.ngram_draft(hist, torch.tensor([9]), 3).tolist() == [[9, 4, 9]]


def test_spec_accept_cases():
    def run(tokens, am, remaining, hist_len=5, h=8):
        tokens = torch.tensor([tokens])
        am = torch.tensor([am])
        hist = torch.zeros((1, h), dtype=torch.int64)
        hl = torch.tensor([hist_len])
        len_b = torch.tensor([100])
        pos_b = torch.tensor([50])
        rem = torch.tensor([remaining])
        out_tok = torch.zeros((4, 1, tokens.shape[1]), dtype=torch.int32)
        out_adv = torch.zeros((4, 1), dtype=torch.int32)
        O.spec_accept(tokens, am, hist, hl, len_b, pos_b, rem, out_tok, out_adv, 2)
        return hist[0].tolist(), int(hl[0]), int(len_b[0]), int(pos_b[0]), int(rem[0]), out_tok[2, 0].tolist(), \
            int(out_adv[2, 0])

    # drafts 5, 6 after token 4; the model says 5 after 4, 9 after 5: one accepted
    hist, hl, lb, pb, rem, ot, adv = run([4, 5, 6], [5, 9, 1], 100)
    assert adv == 2 and hl == 7 and lb == 102 and pb == 52 and rem == 98
    assert ot == [5, 9, 1] and hist[5:8] == [5, 9, 1]
    # all drafts accepted, capped by the budget
    *_, rem, ot, adv = run([4, 5, 6], [5, 6, 7], 2)
    assert adv == 2 and rem == 0
    # nothing accepted; a history slot past the row is not written
    hist, hl, *_, adv = run([4, 5, 6], [8, 6, 7], 10, hist_len=7, h=8)
    assert adv == 1 and hl == 8 and hist[7] == 8


def test_verify_attention_is_decode_at_each_length():
    torch.manual_seed(0)
    b, hq, hkv, d, cap, nq = 2, 4, 2, 16, 24, 3
    kc = torch.randn(b, hkv, cap, d).to(torch.bfloat16)
    vc = torch.randn(b, hkv, cap, d).to(torch.bfloat16)
    q = torch.randn(b * nq, hq, d).to(torch.bfloat16)
    len_b = [9, 13]
    start = torch.tensor([0, 4], dtype=torch.int32)
    got = O.verify_attn(q, kc, vc, len_b, start, 0.25, nq).float()
    for r in range(b):
        for j in range(nq):
            want = O.decode_attn(q[r * nq + j][None], kc[r:r + 1], vc[r:r + 1], len_b[r] + j + 1,
                                 start[r:r + 1], 0.25).float()[0]
            err = (got[r * nq + j] - want).abs().max().item()
            assert err <= 0.03 * want.abs().max().item(), (r, j, err)
    # a key past the query's length changes nothing; one inside does
    kc2 = kc.clone()
    kc2[0, :, len_b[0] + nq] += 5
    assert torch.equal(O.verify_attn(q, kc2, vc, len_b, start, 0.25, nq), O.verify_attn(q, kc, vc, len_b, start,
                                                                                        0.25, nq))
    kc2[0, :, len_b[0]] += 5
    assert not torch.equal(O.verify_attn(q, kc2, vc, len_b, start, 0.25, nq)[nq - 1],
                           O.verify_attn(q, kc, vc, len_b, start, 0.25, nq)[nq - 1])
