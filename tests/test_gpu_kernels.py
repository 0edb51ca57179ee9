"""Per-kernel parity of the HIP path against the CPU oracle and float64
references (mirrors the reference's bench/test_kernels.py, plus the
BASELINE GEMV and attention configurations).

Tolerances, stated per test, come from where the arithmetic can differ:
  * projections are checked against the exact float64 product: the bf16
    output must be the exact value rounded once (half an ulp) up to the
    fp32 accumulation error, bounded by 2^-18 * sum_k |x_k w_k|;
  * composite ops (norms, RoPE, SiLU*up, attention) are checked against the
    oracle, which has the same rounding points: most elements are bitwise
    equal; an fp32 sum taken in a different order (or a 1-ulp exp/rsqrt)
    can move one intermediate bf16 rounding, which shows as at most 2 ulps
    of the output, plus an absolute term where an output cancels to near 0.
"""

import pytest
import torch

from enginekernel_amd import ek_kernels as K
from oracle import ek_oracle as O

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _ulp(x):
    a = x.abs().double().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def assert_close_ulps(got, want, ulps=2, min_equal=0.999, name="", abs_tol=0.0):
    """Every element within `ulps` bf16 ulps (+ abs_tol) of the reference and
    at least `min_equal` of them bitwise equal."""
    got, want = got.detach().cpu(), want.detach().cpu()
    assert got.shape == want.shape, (name, got.shape, want.shape)
    diff = (got.double() - want.double()).abs()
    bound = ulps * _ulp(want) + abs_tol + 1e-30
    bad = diff > bound
    assert not bad.any(), f"{name}: {int(bad.sum())} elements beyond {ulps} ulp, max diff {diff.max().item():.3g}"
    eq = (got == want).float().mean().item()
    assert eq >= min_equal, f"{name}: only {eq:.5f} bitwise equal"


def assert_rounded(got, x, w, name="", min_equal=0.99):
    """A projection's bf16 output against the exact product x . w^T: the
    exact value rounded once, up to the fp32 accumulation error."""
    got = got.detach().cpu().double()
    exact = x.double() @ w.double().t()
    acc_err = 2.0 ** -18 * (x.double().abs() @ w.double().abs().t())
    mag = torch.maximum(got.abs(), exact.abs())
    bad = (got - exact).abs() > 0.5 * _ulp(mag) + acc_err
    assert not bad.any(), f"{name}: {int(bad.sum())} outputs are not the exact product rounded"
    eq = (got == exact.to(torch.float32).to(BF).double()).float().mean().item()
    assert eq >= min_equal, f"{name}: only {eq:.5f} equal to the correctly rounded product"


def check_scale(got, want, tol, name=""):
    """bench/test_kernels.py:18-33: max |err| / max |ref| <= tol."""
    got, want = got.detach().float().cpu(), want.detach().float().cpu()
    err = (got - want).abs().max().item()
    scale = max(want.abs().max().item(), 1e-6)
    assert err / scale <= tol, f"{name}: {err / scale:.3g} > {tol}"


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ----------------------------------------------------------------------------
# norms, SiLU, QK-norm/RoPE (bench/test_kernels.py:36-119)
# ----------------------------------------------------------------------------
@pytest.mark.parametrize("m", [1, 16, 8192])
def test_rms_norm_and_add_rms_norm(dev, m):
    g = _gen(m)
    x = torch.randn(m, 2560, generator=g).to(BF)
    w = torch.randn(2560, generator=g).to(BF)
    r = torch.randn(m, 2560, generator=g).to(BF)
    assert_close_ulps(K.rms_norm(x.to(dev), w.to(dev), 1e-6), O.rms_norm(x, w, 1e-6), name="rms_norm")
    rd = r.to(dev)
    y, r_out = K.add_rms_norm(x.to(dev), rd, w.to(dev), 1e-6)
    y_ref, r_ref = O.add_rms_norm(x, r, w, 1e-6)
    assert r_out.data_ptr() == rd.data_ptr()                      # updated in place
    assert torch.equal(r_out.cpu(), r_ref)                        # bf16 add: exact
    assert_close_ulps(y, y_ref, name="add_rms_norm")


@pytest.mark.parametrize("m", [1, 16, 8192])
def test_silu_mul(dev, m):
    gu = (torch.randn(m, 2 * 9728, generator=_gen(m)) * 2).to(BF)
    assert_close_ulps(K.silu_mul(gu.to(dev)), O.silu_mul(gu), name="silu_mul")


@pytest.mark.parametrize("b,mpb,d,nq,nkv", [(1, 1, 128, 32, 8), (4, 1, 128, 32, 8), (2, 16, 128, 32, 8),
                                             (3, 5, 32, 4, 2)])
def test_qk_norm_rope_kv(dev, b, mpb, d, nq, nkv):
    g = _gen(b * 100 + mpb)
    m, smax = b * mpb, 64
    qkv = torch.randn(m, (nq + 2 * nkv) * d, generator=g).to(BF)
    qn = torch.randn(d, generator=g).to(BF)
    kn = torch.randn(d, generator=g).to(BF)
    cos = torch.randn(m, d, generator=g).to(BF)
    sin = torch.randn(m, d, generator=g).to(BF)
    base = 7 if mpb == 1 else 0
    slot = torch.full((b,), base, dtype=torch.int64)
    kc = torch.zeros(b, nkv, smax, d, dtype=BF)
    vc = torch.zeros_like(kc)
    want = qkv.clone()
    O.qk_norm_rope_kv(want, qn, kn, cos, sin, kc, vc, slot, nq, nkv, 1e-6, mpb)
    got = qkv.to(dev)
    kcd, vcd = torch.zeros_like(kc).to(dev), torch.zeros_like(vc).to(dev)
    K.qk_norm_rope_kv(got, qn.to(dev), kn.to(dev), cos.to(dev), sin.to(dev), kcd, vcd, slot.to(dev),
                      nq, nkv, 1e-6, mpb)
    # q is rotated in place (bench/test_kernels.py:105 checks this slice); the
    # k and v slices of qkv stay raw, as in the reference's kernel (only its
    # torch fallback also rotates k inside qkv)
    assert_close_ulps(got[:, :nq * d], want[:, :nq * d], name="q in place")
    assert torch.equal(got[:, nq * d:].cpu(), qkv[:, nq * d:])
    assert_close_ulps(kcd, kc, name="k cache")                   # includes "elsewhere untouched"
    assert torch.equal(vcd.cpu(), vc)                             # raw v: exact


# ----------------------------------------------------------------------------
# projections (BASELINE config 2 shapes)
# ----------------------------------------------------------------------------
SHAPES = [("qkv", 6144, 2560), ("gate_up", 19456, 2560), ("o", 2560, 4096), ("down", 2560, 9728),
          ("lm_head", 151936, 2560)]


def _proj_ref(x, w):
    """bf16(x . w^T) from a float64 product on the CPU (the exact sum, rounded once)."""
    return (x.double() @ w.double().t()).to(torch.float32).to(BF)


@pytest.mark.parametrize("name,n,k", SHAPES)
@pytest.mark.parametrize("m", [1, 4])
def test_gemv_shapes(dev, name, n, k, m):
    g = _gen(n + m)
    x = (torch.randn(m, k, generator=g) * 0.02).to(BF)
    w = (torch.randn(n, k, generator=g) * 0.02).to(BF)
    got = K.gemv(x.to(dev), w.to(dev))
    assert_rounded(got, x, w, name=f"gemv {name} m={m}")
    check_scale(got, _proj_ref(x, w), 2e-2)


@pytest.mark.parametrize("m", [1, 4])
def test_gemv_swiglu_and_silu_epilogue(dev, m):
    """The fused gate/up projection with its SiLU*up epilogue on the 19456
    output (config 2) against the unfused composition."""
    g = _gen(7 + m)
    x = (torch.randn(m, 2560, generator=g) * 0.02).to(BF)
    w = (torch.randn(19456, 2560, generator=g) * 0.02).to(BF)
    want = O.silu_mul(_proj_ref(x, w))
    got = K.gemv_swiglu(x.to(dev), w.to(dev))
    tol = 2.0 ** -20 * want.abs().max().item()       # outputs that cancel to ~0
    assert_close_ulps(got, want, min_equal=0.99, name="gemv_swiglu", abs_tol=tol)
    got2 = K.silu_mul(K.gemv(x.to(dev), w.to(dev)))
    assert_close_ulps(got2, want, min_equal=0.99, name="gemv+silu_mul", abs_tol=tol)


@pytest.mark.parametrize("m,sk", [(1, 1), (1, 2), (4, 2), (8, 4)])
def test_gemv_parts_and_add_rms_norm_parts(dev, m, sk):
    g = _gen(11 + m)
    x = (torch.randn(m, 9728, generator=g) * 0.02).to(BF)
    w = (torch.randn(2560, 9728, generator=g) * 0.02).to(BF)
    r = (torch.randn(m, 2560, generator=g) * 0.5).to(BF)
    nw = (1 + 0.1 * torch.randn(2560, generator=g)).to(BF)
    parts = K.gemv_parts(x.to(dev), w.to(dev), sk=sk)
    assert parts.shape == (sk, m, 2560)
    exact = x.double() @ w.double().t()
    assert (parts.sum(0).double().cpu() - exact).abs().max() <= 1e-5 * exact.abs().max() + 1e-7
    rd = r.to(dev)
    y, r_out = K.add_rms_norm_parts(parts, rd, nw.to(dev), 1e-6)
    y_ref, r_ref = O.add_rms_norm(_proj_ref(x, w), r, nw, 1e-6)
    assert_close_ulps(r_out, r_ref, min_equal=0.99, name="residual")
    assert_close_ulps(y, y_ref, ulps=3, min_equal=0.99, name="norm")


@pytest.mark.parametrize("m", [1, 3, 8])
def test_norm_gemv_fused_prologues(dev, m):
    """norm_gemv (no add / add), parts_norm_gemv and embed_norm_gemv against
    the composition of the oracle's norms and an exact projection."""
    g = _gen(13 + m)
    H, N, I = 2560, 6144, 9728
    x = (torch.randn(m, H, generator=g) * 0.3).to(BF)
    r = (torch.randn(m, H, generator=g) * 0.3).to(BF)
    nw = (1 + 0.1 * torch.randn(H, generator=g)).to(BF)
    w = (torch.randn(N, H, generator=g) * 0.02).to(BF)
    wgu = (torch.randn(2 * I, H, generator=g) * 0.02).to(BF)
    d = lambda t: t.to(dev)
    # the normalised row is bitwise the oracle's (rare 1-ulp flips aside), so
    # the projection is checked as a rounded exact product of that row
    y, r1 = K.norm_gemv(d(x), None, d(nw), d(w), 1e-6)
    assert_rounded(y, O.rms_norm(x, nw, 1e-6), w, name="norm_gemv", min_equal=0.98)
    y, r2 = K.norm_gemv(d(x), d(r), d(nw), d(wgu), 1e-6, silu=True)
    xn, rr = O.add_rms_norm(x, r, nw, 1e-6)
    assert torch.equal(r2.cpu(), rr)
    want = O.silu_mul(_proj_ref(xn, wgu))
    assert_close_ulps(y, want, min_equal=0.98, name="norm_gemv silu", abs_tol=2.0 ** -20 * want.abs().max().item())
    # split-K partials as the addend
    parts = (torch.randn(2, m, H, generator=g) * 0.1)
    r_out = torch.empty(m, H, dtype=BF, device=dev)
    y = K.parts_norm_gemv(d(parts), d(r), r_out, d(nw), d(w), 1e-6)
    xsum = parts.sum(0).to(BF)
    xn, rr = O.add_rms_norm(xsum, r, nw, 1e-6)
    assert_close_ulps(r_out, rr, min_equal=0.999, name="parts residual")
    assert_rounded(y, xn, w, name="parts_norm_gemv", min_equal=0.98)
    # embedding gather + slot/length advance
    emb = (torch.randn(1000, H, generator=g) * 0.02).to(BF)
    tok = torch.randint(0, 1000, (m,), generator=g)
    slot = torch.zeros(m, dtype=torch.int64, device=dev)
    ln = torch.full((1,), 41, dtype=torch.int64, device=dev)
    y = K.embed_norm_gemv(d(tok), d(emb), r_out, d(nw), d(w), 1e-6, slot_t=slot, len_t=ln)
    assert torch.equal(r_out.cpu(), emb[tok])
    assert slot.tolist() == [41] * m and ln.item() == 42
    assert_rounded(y, O.rms_norm(emb[tok], nw, 1e-6), w, name="embed", min_equal=0.98)


@pytest.mark.parametrize("m,n,k", [(2, 1001, 128), (5, 4099, 384), (7, 777, 640), (8, 2560, 2432),
                                   (3, 2048, 2560), (6, 333, 3072), (2, 515, 4864)])
def test_matrix_core_gemv_matches_fma_kernel(dev, m, n, k):
    """The matrix-core GEMV (2..8 rows) against the exact product and the
    FMA kernel (forced with a negative rows-per-wave argument): ragged tile
    counts (N % 4 != 0), odd batch rows, one and two column groups, K / 128
    chunks per tile of 1, 3, 5, 19, 20, 24 and 38 (ring depths 1, 5, 8, 10,
    19, 20) and the bf16, SwiGLU, partials and argmax epilogues."""
    g = _gen(m * 7 + n)
    x = (torch.randn(m, k, generator=g) * 0.05).to(BF)
    w = (torch.randn(2 * n, k, generator=g) * 0.05).to(BF)
    xd, wd = x.to(dev), w.to(dev)
    ys = {}
    for rpw in (0, -1):                              # 0: matrix cores, -1: FMA kernel
        y = torch.empty(m, n, dtype=BF, device=dev)
        K.call("ek_gemv", K.ptr(xd), K.ptr(wd), K.ptr(y), m, n, k, k, k, n, rpw, 0, K.stream())
        a = torch.empty(m, n, dtype=BF, device=dev)
        K.call("ek_gemv_swiglu", K.ptr(xd), K.ptr(wd), K.ptr(a), m, n, k, k, k, n, rpw, 0, K.stream())
        sk = 2 if k % 256 == 0 else 1
        pt = torch.empty(sk, m, 2 * n, dtype=torch.float32, device=dev)
        K.call("ek_gemv_parts", K.ptr(xd), K.ptr(wd), K.ptr(pt), m, 2 * n, k, k, k, sk, rpw, 0, K.stream())
        scratch = K.ArgmaxScratch(m, 2 * n, dev)
        tok = torch.empty(m, dtype=torch.int64, device=dev)
        lg = torch.empty(m, 2 * n, dtype=BF, device=dev)
        K.call("ek_lm_head_argmax", K.ptr(xd), None, 0, None, None, 1e-6, K.ptr(wd), m, 2 * n, k, k, 0, k,
               K.ptr(lg), 2 * n, K.ptr(scratch.val), K.ptr(scratch.idx), scratch.cap, K.ptr(tok),
               None, None, None, None, 0, rpw, 0, K.stream())
        ys[rpw] = (y.cpu(), a.cpu(), pt.cpu(), tok.cpu(), lg.cpu())
    y, a, pt, tok, lg = ys[0]
    assert_rounded(y, x, w[:n], name=f"mfma gemv m={m} n={n} k={k}")
    want = O.silu_mul(_proj_ref(x, w))
    assert_close_ulps(a, want, min_equal=0.99, name="mfma swiglu", abs_tol=2.0 ** -20 * want.abs().max().item())
    exact = x.double() @ w.double().t()
    assert (pt.sum(0).double() - exact).abs().max() <= 1e-5 * exact.abs().max() + 1e-7
    assert_rounded(lg, x, w, name="mfma logits")
    assert tok.tolist() == torch.argmax(lg, -1).tolist()
    # the FMA kernel sums in another order: the same values up to fp32 rounding
    fy, fa, fpt, ftok, flg = ys[-1]
    assert_close_ulps(y, fy, ulps=2, min_equal=0.99, name="mfma vs fma")   # 1 ulp at a binade edge is 2 below it
    assert (pt.sum(0) - fpt.sum(0)).abs().max() <= 1e-5 * exact.abs().max() + 1e-7


# ----------------------------------------------------------------------------
# lm_head + argmax
# ----------------------------------------------------------------------------
@pytest.mark.parametrize("m", [1, 4])
def test_lm_head_argmax(dev, m):
    g = _gen(17 + m)
    V, H = 151936, 2560
    h = torch.randn(m, H, generator=g).to(BF)
    e = (torch.randn(V, H, generator=g) * 0.02).to(BF)
    # planted exact tie: the best row duplicated at a higher index must lose
    ref = _proj_ref(h, e)
    best = ref.float().argmax(-1)
    e[V - 5] = e[best[0]]
    ref = _proj_ref(h, e)
    scratch = K.ArgmaxScratch(m, V, dev)
    logits = torch.empty(m, V, dtype=BF, device=dev)
    tok = K.lm_head_argmax(h.to(dev), e.to(dev), scratch, logits=logits)
    assert_rounded(logits, h, e, name="logits")
    # exact on the kernel's own logits; equal to the reference unless a near-tie moved
    assert tok.tolist() == torch.argmax(logits.cpu(), -1).tolist()
    want = torch.argmax(ref, -1)
    for i in range(m):
        if tok[i].item() != want[i].item():
            gap = ref[i, want[i]].float() - ref[i, tok[i].item()].float()
            assert gap <= _ulp(ref[i, want[i]].double()), "argmax differs beyond a one-ulp near-tie"
    assert tok[0].item() == best[0].item()


def test_lm_head_argmax_step_state(dev):
    """The fused bookkeeping: tokens <- next, positions += 1,
    out_buf[step] <- next, step += 1 (engine.py:289-292)."""
    m, V, H = 2, 4096, 256
    g = _gen(3)
    h = torch.randn(m, H, generator=g).to(BF).to(dev)
    e = (torch.randn(V, H, generator=g) * 0.02).to(BF).to(dev)
    scratch = K.ArgmaxScratch(m, V, dev)
    tokens = torch.zeros(m, dtype=torch.int64, device=dev)
    pos = torch.tensor([5, 9], dtype=torch.int64, device=dev)
    out_buf = torch.full((4, m), -1, dtype=torch.int32, device=dev)
    step = torch.zeros(1, dtype=torch.int64, device=dev)
    for i in range(5):                                           # the 5th exceeds out_buf: guarded
        K.lm_head_argmax(h, e, scratch, state=(tokens, pos, out_buf, step))
    want = torch.argmax((h.float() @ e.float().t()).to(BF).float(), -1)
    assert tokens.tolist() == want.tolist()
    assert pos.tolist() == [10, 14] and step.item() == 5
    assert out_buf.tolist() == [want.tolist()] * 4


# ----------------------------------------------------------------------------
# attention (bench/test_kernels.py:122-155)
# ----------------------------------------------------------------------------
def _ref_attn64(q, kc, vc, seq_len, start):
    """bench/test_kernels.py:122-130 in float64 (no bf16 rounding of p)."""
    b, hq, d = q.shape
    rep = hq // kc.shape[1]
    k = kc[:, :, :seq_len].repeat_interleave(rep, 1).double()
    v = vc[:, :, :seq_len].repeat_interleave(rep, 1).double()
    s = torch.einsum("bhd,bhsd->bhs", q.double(), k) * (d ** -0.5)
    idx = torch.arange(seq_len)
    s = s.masked_fill(idx[None, None, :] < start[:, None, None], float("-inf"))
    return torch.einsum("bhs,bhsd->bhd", torch.softmax(s, -1), v)


def assert_attn_vs_oracle(got, want, vmax, fp32_p, name, min_equal=0.99):
    """An attention output against the oracle's fallback attention, which
    rounds each probability to bf16 after normalising (ek_model.py:475-488).
    The one-launch split form keeps p in fp32 and merges its splits by
    log-sum-exp, as the reference's split decode kernel does
    (ek_kernels.py:535-616, 989-1019): each oracle p is then off by at most
    half a bf16 ulp (2^-8 of p), and with the p summing to 1 the outputs
    differ by at most 2^-8 max|v| (plus their own 2-ulp rounding). The other
    forms round p where the oracle does and match it within 2 ulps and
    2^-13 max|v| (a p at a rounding boundary may go the other way)."""
    if fp32_p:
        assert_close_ulps(got, want, min_equal=0.0, name=name + " (fp32 p)", abs_tol=2.0 ** -8 * vmax)
    else:
        assert_close_ulps(got, want, min_equal=min_equal, name=name, abs_tol=2.0 ** -13 * vmax)


def _attn_form(ws, g, s_cap, run):
    """run() on workspace ws and the form of attn_decode that ran: "fused"
    (one split whose score rows fit in LDS), "pair" (the two launches: the
    only form that writes scores to the score scratch ws[7], zeroed first)
    or "one launch" (the split form on one grid: p in fp32)."""
    ws[7].zero_()
    out = run()
    if ws[4] == 1 and g * min(s_cap, ws[7].shape[2]) * 4 <= 32 * 1024:   # the score rows the kernel sees
        return out, "fused"
    return out, ("pair" if bool(ws[7].ne(0).any()) else "one launch")


def assert_attn_exact(got, q, kc, vc, seq_len, start, name):
    """The fp32-p form against the exact (float64) softmax attention rounded
    once to bf16: only its fp32 accumulation differs."""
    exact = _ref_attn64(q.cpu(), kc.cpu(), vc.cpu(), seq_len, start.cpu()).float().to(BF)
    assert_close_ulps(got, exact, min_equal=0.98, name=name + " vs exact", abs_tol=2.0 ** -13 * vc.abs().max().item())


# Rows whose scores fit in LDS (G * s_cap * 4 bytes <= 32 KiB: s_cap <= 2048 at
# G = 4) take the single-launch kernel; longer ones the two-phase pair.
ATTN_CASES = [(1, 1024, 600, 0), (4, 2048, 2048, 0), (16, 1024, 640, 0), (3, 1024, 97, 0), (2, 1024, 500, 37),
              (2, 4096, 1500, 37), (1, 4096, 4096, 0)]


@pytest.mark.parametrize("b,smax,slen,pad", ATTN_CASES)
def test_flash_decode_reference_cases(dev, b, smax, slen, pad):
    hq, hkv, d = 32, 8, 128
    g = _gen(b * 1000 + slen)
    q = torch.randn(b, hq, d, generator=g).to(BF)
    kc = torch.randn(b, hkv, smax, d, generator=g).to(BF)
    vc = torch.randn(b, hkv, smax, d, generator=g).to(BF)
    start = torch.full((b,), pad, dtype=torch.int32)
    splits, chunk, bn = K.plan_splits(b, hkv, smax)
    sp, gp = K._next_pow2(splits), K.group_pad(hq, hkv)
    ws = (torch.zeros(b, hkv, sp, gp, d, dtype=torch.float32, device=dev),
          torch.zeros(b, hkv, sp, gp, dtype=torch.float32, device=dev),
          torch.full((b, hkv, sp, gp), -1e30, dtype=torch.float32, device=dev),
          torch.empty(b, hq, d, dtype=BF, device=dev), splits, chunk, bn)     # the reference's 7-tuple
    got = K.flash_decode(q.to(dev), kc.to(dev), vc.to(dev), torch.tensor([slen], device=dev),
                         start.to(dev), ws, d ** -0.5)
    check_scale(got, _ref_attn64(q, kc, vc, slen, start), 3e-2, "vs fp64 softmax")
    # a probability whose fp32 value sits at a bf16 rounding boundary may
    # round the other way: at most 2^-8 * p * |v| for that key
    assert_close_ulps(got, O.decode_attn(q, kc, vc, slen, start, d ** -0.5), min_equal=0.99,
                      name="vs oracle (bf16 p)", abs_tol=2.0 ** -13 * vc.abs().max().item())


@pytest.mark.parametrize("L", [512, 4096, 16384, 32768])
def test_attention_config3_lengths_and_split_sweep(dev, L):
    """32/8 heads, D=128, capacity 32768, L filled, the
    split-count sweep. 4 and 32 splits run the one-launch form (fp32 p,
    log-sum-exp merge): they agree with each other and with the exact
    softmax up to fp32 summation order; 1 and 64 splits run the two-launch
    pair (p rounded as the oracle does): they agree with each other likewise.
    Every form and the planner's own split count agree with the oracle
    (assert_attn_vs_oracle; the oracle's fp32 softmax over 32 x 32768
    scores takes well under a second on the CPU)."""
    hq, hkv, d, cap = 32, 8, 128, 32768
    g = _gen(L)
    q = torch.randn(1, hq, d, generator=g).to(BF).to(dev)
    kc = torch.randn(1, hkv, cap, d, generator=g).to(BF).to(dev)
    vc = torch.randn(1, hkv, cap, d, generator=g).to(BF).to(dev)
    start = torch.zeros(1, dtype=torch.int32, device=dev)
    ln = torch.tensor([L], device=dev)
    outs, form = {}, {}
    for splits in (1, 4, 32, 64):
        ws = K.make_workspace(1, hq, hkv, d, cap, dev, splits=splits, chunk=-(-cap // splits))
        outs[splits], form[splits] = _attn_form(ws, hq // hkv, cap,
                                                lambda: K.flash_decode(q, kc, vc, ln, start, ws, d ** -0.5).clone())
    assert form == {1: "pair", 4: "one launch", 32: "one launch", 64: "pair"}, form
    one_launch = {k: v == "one launch" for k, v in form.items()}
    vmax = vc.abs().max().item()
    assert_close_ulps(outs[4], outs[32], min_equal=0.98, name="splits 4 vs 32", abs_tol=2.0 ** -13 * vmax)
    assert_close_ulps(outs[64], outs[1], min_equal=0.98, name="splits 64 vs 1", abs_tol=2.0 ** -13 * vmax)
    assert_attn_exact(outs[32], q, kc[:, :, :L], vc[:, :, :L], L, start, "32 splits")
    want = O.decode_attn(q.cpu(), kc.cpu()[:, :, :L], vc.cpu()[:, :, :L], L, start.cpu(), d ** -0.5)
    # every probability's bf16 rounding depends on the row's fp32 sum of exps
    # (L terms, summed in another order here): at 16K-32K keys about 1.3 % of
    # the outputs move by an ulp (measured 98.7 % bitwise equal at 32768)
    eq = 0.99 if L <= 4096 else 0.98
    for s_ in (1, 4, 32, 64):
        assert_attn_vs_oracle(outs[s_], want, vmax, one_launch[s_], f"splits {s_} vs oracle", min_equal=eq)
    bucket = -(-(L + 1) // 256) * 256
    ws = K.make_workspace(1, hq, hkv, d, bucket, dev)     # the planner's own split count
    assert K.ws_error(ws) is not None
    got, f = _attn_form(ws, hq // hkv, cap, lambda: K.flash_decode(q, kc, vc, ln, start, ws, d ** -0.5))
    assert_attn_vs_oracle(got, want, vmax, f == "one launch", f"planned splits ({ws[4]}, {f}) vs oracle",
                          min_equal=eq)
    K.check_error_word(K.ws_error(ws), "config 3 attention")


def test_split_combine_tickets_across_launches(dev):
    """The split combine's ticket block (arrival count + epoch per row and kv
    head) carries from launch to launch: repeated launches on one workspace
    are bitwise identical, the ticket ends each launch with zero arrivals and
    an epoch equal to the launch count, and the same buffers then serve a
    different split count."""
    b, hq, hkv, d, cap, L = 3, 32, 8, 128, 4096, 3001
    g = _gen(99)
    q = torch.randn(b, hq, d, generator=g).to(BF).to(dev)
    kc = torch.randn(b, hkv, cap, d, generator=g).to(BF).to(dev)
    vc = torch.randn(b, hkv, cap, d, generator=g).to(BF).to(dev)
    start = torch.tensor([0, 17, 900], dtype=torch.int32, device=dev)
    ln = torch.tensor([L], device=dev)
    ws = K.make_workspace(b, hq, hkv, d, cap, dev, splits=16, chunk=cap // 16)
    outs, f = _attn_form(ws, hq // hkv, cap,
                         lambda: [K.flash_decode(q, kc, vc, ln, start, ws, d ** -0.5).clone() for _ in range(3)])
    assert f == "one launch", f
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    t = ws[8].cpu()
    assert t[..., 0].eq(0).all() and t[..., 1].eq(3).all()
    ws4 = ws[:4] + (4, cap // 4) + ws[6:]                       # same buffers, four splits
    got4 = K.flash_decode(q, kc, vc, ln, start, ws4, d ** -0.5).clone()
    vmax = vc.abs().max().item()
    assert_close_ulps(got4, outs[0], min_equal=0.98, name="4 vs 16 splits", abs_tol=2.0 ** -13 * vmax)
    want = O.decode_attn(q.cpu(), kc.cpu()[:, :, :L], vc.cpu()[:, :, :L], L, start.cpu(), d ** -0.5)
    assert_attn_vs_oracle(outs[0], want, vmax, True, "vs oracle")
    assert_attn_exact(outs[0], q, kc[:, :, :L], vc[:, :, :L], L, start, "16 splits")
    assert ws[8].cpu()[..., 1].eq(4).all()


@pytest.mark.parametrize("b,d,nq,nkv,slen,pad,smax", [
    (1, 128, 32, 8, 129, 0, 1024), (3, 128, 32, 8, 300, 11, 1024), (3, 32, 4, 2, 17, 5, 1024),
    (8, 128, 32, 8, 700, 0, 1024), (1, 64, 16, 2, 333, 3, 1024), (1, 128, 32, 8, 1, 0, 256),
    (1, 128, 32, 8, 129, 0, 4096), (3, 128, 32, 8, 2000, 11, 4096), (2, 64, 16, 2, 333, 3, 2048)])
def test_rope_attn_decode(dev, b, d, nq, nkv, slen, pad, smax):
    """Fused QK-norm + RoPE + KV write + attention against the oracle's
    qk_norm_rope_kv followed by its fallback attention, on the single-launch
    kernel (short score rows) and on the two-phase pair (s_cap 4096 at G = 4,
    s_cap 2048 at G = 8)."""
    g = _gen(slen + b)
    qkv = torch.randn(b, (nq + 2 * nkv) * d, generator=g).to(BF)
    qn = (1 + 0.1 * torch.randn(d, generator=g)).to(BF)
    kn = (1 + 0.1 * torch.randn(d, generator=g)).to(BF)
    cos_t, sin_t = O.build_rope(d, 1e6, 2048)
    pos = torch.randint(0, 2000, (b,), generator=g)
    kc = torch.randn(b, nkv, smax, d, generator=g).to(BF)
    vc = torch.randn(b, nkv, smax, d, generator=g).to(BF)
    start = torch.full((b,), pad, dtype=torch.int32)
    # oracle: slot = slen - 1 (seq_len counts the new token)
    q_ref, kc_ref, vc_ref = qkv.clone(), kc.clone(), vc.clone()
    O.qk_norm_rope_kv(q_ref, qn, kn, cos_t[pos], sin_t[pos], kc_ref, vc_ref,
                      torch.full((b,), slen - 1, dtype=torch.int64), nq, nkv, 1e-6, 1)
    want = O.decode_attn(q_ref[:, :nq * d].view(b, nq, d), kc_ref, vc_ref, slen, start, d ** -0.5)
    kcd, vcd = kc.to(dev), vc.to(dev)
    ws = K.make_workspace(b, nq, nkv, d, smax, dev)
    got, f = _attn_form(ws, nq // nkv, smax, lambda: K.rope_attn_decode(
        qkv.to(dev), qn.to(dev), kn.to(dev), cos_t.to(dev), sin_t.to(dev), kcd, vcd,
        torch.tensor([slen], device=dev), start.to(dev), ws, d ** -0.5, nq, 1e-6, positions=pos.to(dev)))
    assert_attn_vs_oracle(got, want, vc.abs().max().item(), f == "one launch", f"rope_attn_decode ({f})")
    assert_close_ulps(kcd[:, :, slen - 1], kc_ref[:, :, slen - 1], name="new k")
    assert torch.equal(vcd[:, :, slen - 1].cpu(), vc_ref[:, :, slen - 1])
    keep = torch.ones(smax, dtype=torch.bool)
    keep[slen - 1] = False
    assert torch.equal(kcd[:, :, keep].cpu(), kc[:, :, keep]) and torch.equal(vcd[:, :, keep].cpu(), vc[:, :, keep])


@pytest.mark.parametrize("rope,b,d,nq,nkv,slen,pads,cap,splits", [
    (0, 1, 128, 32, 8, 4001, (0,), 8192, 16), (0, 3, 128, 32, 8, 3001, (0, 17, 900), 4096, 8),
    (1, 2, 128, 32, 8, 2000, (11, 0), 4096, 8), (1, 2, 64, 16, 2, 1500, (3, 700), 2048, 16)])
def test_attn_one_launch_and_pair(dev, rope, b, d, nq, nkv, slen, pads, cap, splits):
    """The two split forms of attn_decode on the same inputs, both against the
    oracle (assert_attn_vs_oracle): the one-launch form (the default
    workspace: its exchange words fit, and the grid is resident at once; p
    in fp32, log-sum-exp merge) and the two-launch pair (a workspace without
    the error word that the one-launch form's bounded waits need; p rounded
    as the oracle does). Which form ran shows in
    the buffers each writes: the one-launch form's tagged words, the pair's
    partial words in acc. With rope, both also write the same new K/V row."""
    g = _gen(slen + 7 * b + d)
    start = torch.tensor(pads, dtype=torch.int32)
    kc = torch.randn(b, nkv, cap, d, generator=g).to(BF)
    vc = torch.randn(b, nkv, cap, d, generator=g).to(BF)
    vmax = vc.abs().max().item()
    if rope:
        qkv = torch.randn(b, (nq + 2 * nkv) * d, generator=g).to(BF)
        qn = (1 + 0.1 * torch.randn(d, generator=g)).to(BF)
        kn = (1 + 0.1 * torch.randn(d, generator=g)).to(BF)
        cos_t, sin_t = O.build_rope(d, 1e6, 4096)
        pos = torch.randint(0, 4000, (b,), generator=g)
        q_ref, kc_ref, vc_ref = qkv.clone(), kc.clone(), vc.clone()
        O.qk_norm_rope_kv(q_ref, qn, kn, cos_t[pos], sin_t[pos], kc_ref, vc_ref,
                          torch.full((b,), slen - 1, dtype=torch.int64), nq, nkv, 1e-6, 1)
        want = O.decode_attn(q_ref[:, :nq * d].view(b, nq, d), kc_ref, vc_ref, slen, start, d ** -0.5)
    else:
        q = torch.randn(b, nq, d, generator=g).to(BF)
        want = O.decode_attn(q, kc, vc, slen, start, d ** -0.5)
    ws = K.make_workspace(b, nq, nkv, d, cap, dev, splits=splits, chunk=cap // splits)
    results = []
    for form, w in (("one launch", ws), ("pair", ws[:9])):
        kcd, vcd = kc.to(dev), vc.to(dev)
        if rope:
            run = lambda: K.rope_attn_decode(qkv.to(dev), qn.to(dev), kn.to(dev), cos_t.to(dev), sin_t.to(dev),
                                             kcd, vcd, torch.tensor([slen], device=dev), start.to(dev), w,
                                             d ** -0.5, nq, 1e-6, positions=pos.to(dev)).clone()
        else:
            run = lambda: K.flash_decode(q.to(dev), kcd, vcd, torch.tensor([slen], device=dev), start.to(dev), w,
                                         d ** -0.5).clone()
        got, ran = _attn_form(w, nq // nkv, cap, run)
        assert ran == form, (form, ran)
        if rope:
            assert_close_ulps(kcd[:, :, slen - 1], kc_ref[:, :, slen - 1], name=f"{form}: new k")
            assert torch.equal(vcd[:, :, slen - 1].cpu(), vc_ref[:, :, slen - 1])
        K.check_error_word(K.ws_error(ws), form)
        assert_attn_vs_oracle(got, want, vmax, form == "one launch", f"{form} vs oracle")
        results.append(got)
    vm = results[0].float().abs().max().item()
    assert (results[0].float() - results[1].float()).abs().max().item() <= 2.0 ** -6 * vm
    # every launch moved each (row, kv head)'s epoch on, whichever form ran
    assert ws[8].cpu()[..., 1].eq(2).all() and ws[8].cpu()[..., 0].eq(0).all()


@pytest.mark.parametrize("rope", [0, 1])
def test_attn_one_launch_unaligned_heads(dev, rope):
    """The one-launch kernel loads the heads as 16-byte pieces at entry when
    the q rows and heads are 16-byte aligned, else element by element. The
    same heads one element into a wider buffer (rows 2 bytes off 16, and an
    odd row stride) take the element path: the output (and with rope the new
    K/V row) must be bit-identical to the aligned call's, on two launches in
    a row (the second at a shorter length)."""
    b, d, nq, nkv, cap, splits = 2, 128, 32, 8, 4096, 16
    g = _gen(4242 + rope)
    start = torch.tensor([0, 33], dtype=torch.int32)
    kc = torch.randn(b, nkv, cap, d, generator=g).to(BF)
    vc = torch.randn(b, nkv, cap, d, generator=g).to(BF)
    width = (nq + 2 * nkv) * d if rope else nq * d
    x = torch.randn(b, width, generator=g).to(BF)
    wide = torch.zeros(b, width + 3, dtype=BF)
    wide[:, 1:width + 1] = x
    xa, xu = x.to(dev), wide.to(dev)[:, 1:width + 1]
    assert xu.data_ptr() % 16 and xu.stride(0) % 8
    qn = (1 + 0.1 * torch.randn(d, generator=g)).to(BF).to(dev)
    kn = (1 + 0.1 * torch.randn(d, generator=g)).to(BF).to(dev)
    cos_t, sin_t = (t.to(dev) for t in O.build_rope(d, 1e6, 4096))
    pos = torch.tensor([3000, 2999], device=dev)
    for slen in (3001, 1500):
        outs = []
        for src in (xa, xu):
            ws = K.make_workspace(b, nq, nkv, d, cap, dev, splits=splits, chunk=cap // splits)
            kcd, vcd = kc.to(dev), vc.to(dev)
            if rope:
                run = lambda: K.rope_attn_decode(src, qn, kn, cos_t, sin_t, kcd, vcd, torch.tensor([slen], device=dev),
                                                 start.to(dev), ws, d ** -0.5, nq, 1e-6, positions=pos).clone()
            else:
                run = lambda: K.flash_decode(src.view(b, nq, d), kcd, vcd, torch.tensor([slen], device=dev),
                                             start.to(dev), ws, d ** -0.5).clone()
            got, ran = _attn_form(ws, nq // nkv, cap, run)
            assert ran == "one launch", ran
            K.check_error_word(K.ws_error(ws), "unaligned heads")
            outs.append((got.cpu(), kcd[:, :, slen - 1].cpu(), vcd[:, :, slen - 1].cpu()))
        for a_, u_ in zip(*outs):
            assert torch.equal(a_, u_), (rope, slen)


# ----------------------------------------------------------------------------
# prefill attention (ek_model.py:315-323, SDPA with the _pack mask)
# ----------------------------------------------------------------------------
def _ref_prefill64(qkv, kc, vc, start, s, nq, d):
    """Causal GQA softmax attention in float64 over keys [start_b, t]; a
    padding token (t < start_b) attends to itself."""
    b, nkv = kc.shape[0], kc.shape[1]
    g = nq // nkv
    q = qkv[:, : nq * d].double().view(b, s, nq, d).transpose(1, 2)             # [b, nq, s, d]
    k = kc[:, :, :s].double().repeat_interleave(g, 1)
    v = vc[:, :, :s].double().repeat_interleave(g, 1)
    sc = q @ k.transpose(-1, -2) * d ** -0.5
    t = torch.arange(s)
    out = torch.empty(b, nq, s, d, dtype=torch.float64)
    for i in range(b):
        st = int(start[i])
        allow = (t[None, :] <= t[:, None]) & (t[None, :] >= st)
        allow |= (t[:, None] < st) & (t[None, :] == t[:, None])
        si = sc[i].masked_fill(~allow, float("-inf"))
        out[i] = torch.softmax(si, -1) @ v[i]
    return out.transpose(1, 2).reshape(b * s, nq * d)


@pytest.mark.parametrize("b,s,d,nq,nkv,pads,cap", [
    (1, 17, 128, 32, 8, [0], 32), (3, 100, 128, 32, 8, [0, 37, 99], 256), (2, 300, 64, 16, 2, [5, 0], 512),
    (2, 33, 32, 4, 2, [0, 10], 64), (1, 70, 128, 8, 8, [3], 96), (1, 2048, 128, 32, 8, [0], 4096)])
def test_attn_prefill_flash(dev, b, s, d, nq, nkv, pads, cap):
    """The prompt's causal GQA flash attention against a float64 softmax:
    ragged left padding (a row with one real token included), every group
    size G = 1, 2, 4, 8, head dims 32/64/128, partial 16-token blocks and a
    cache capacity above the prompt. Padding rows return their own value
    row exactly."""
    g = _gen(s + b + d)
    qkv = torch.randn(b * s, (nq + 2 * nkv) * d, generator=g).to(BF)
    kc = torch.randn(b, nkv, cap, d, generator=g).to(BF)
    vc = torch.randn(b, nkv, cap, d, generator=g).to(BF)
    start = torch.tensor(pads, dtype=torch.int32)
    got = K.attn_prefill(qkv.to(dev), kc.to(dev), vc.to(dev), start.to(dev), s, nq, d ** -0.5).cpu()
    want = _ref_prefill64(qkv, kc, vc, start, s, nq, d)
    check_scale(got, want, 1e-2, "vs float64 softmax")
    # elementwise: probabilities are rounded to bf16 (2^-9 relative) before the value sum
    bound = 2.0 ** -7 * want.abs() + 2.0 ** -8 * vc.float().abs().max().item()
    assert ((got.double() - want).abs() <= bound).float().mean().item() >= 0.999
    gg = nq // nkv
    for i, st in enumerate(pads):
        for t in range(min(st, s)):
            row = got.view(b, s, nq, d)[i, t]
            assert torch.equal(row, vc[i, :, t].repeat_interleave(gg, 0)), (i, t)


# ----------------------------------------------------------------------------
# graph capture of C-ABI launches
# ----------------------------------------------------------------------------
def test_graph_replay_matches_eager(dev):
    """A captured chain of C-ABI launches (no memset nodes) replays to the
    eager result every time, with eager work and syncs between replays."""
    g = _gen(5)
    x = (torch.randn(1, 2560, generator=g) * 0.3).to(BF).to(dev)
    w = (torch.randn(6144, 2560, generator=g) * 0.02).to(BF).to(dev)
    nw = torch.ones(2560, dtype=BF, device=dev)
    e = (torch.randn(4096, 6144, generator=g) * 0.02).to(BF).to(dev)
    scratch = K.ArgmaxScratch(1, 4096, dev)
    out = torch.empty(1, dtype=torch.int64, device=dev)

    def body():
        y, _ = K.norm_gemv(x, None, nw, w, 1e-6)
        return K.lm_head_argmax(y, e, scratch, out_tok=out)

    eager = body().clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body()
    for i in range(4):
        out.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        _ = (x.float() * 2).sum().item()                         # eager work between replays
