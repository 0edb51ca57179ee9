"""The reference's ek_kernels call surface, on hand-written gfx950 HIP kernels.

Same function names, argument order and return conventions as
jeojdi1/EngineKernel `engine/ek_kernels.py` (cited per function), so a caller
of that module can import this one instead. Every function launches through
the C ABI of libek_hip.so (include/ek_hip.h) on torch's current stream; none
has a CPU fallback: on CPU tensors or without the library they raise.

Shapes are checked on the host before any launch, so a wrong shape is a
Python exception rather than a kernel reading out of bounds.
"""

from __future__ import annotations

import os

import torch

from . import _hip
from ._hip import HipKernelError, HipUnavailable, call, ptr, stream

__all__ = [
    "has_hip", "probe_hip", "disable_hip", "has_triton", "probe_triton", "disable_triton",
    "rms_norm", "add_rms_norm", "silu_mul", "qk_norm_rope_kv", "gemv", "gemv_parts",
    "add_rms_norm_parts", "gemv_swiglu", "norm_gemv", "flash_decode", "rope_attn_decode",
    "plan_splits", "group_pad", "attn_warps", "make_workspace", "parts_norm_gemv",
    "embed_norm_gemv", "lm_head_argmax", "_next_pow2", "_cdiv", "_torch_rms_norm",
    "HipUnavailable", "HipKernelError",
]

_DISABLED = False
_BF16 = torch.bfloat16

# GEMV-family launch shape per (kernel, N, K[, rows]): (rows per wave, grid
# cap). (0, 0) is the library's default (1 row per wave, 4 workgroups per
# CU; lm_head 4 rows per wave). Results never depend on these. The entries
# below are the fastest of a rows-per-wave x grid-cap sweep on MI355X at
# batch 1 (weights rotated past the 256 MB Infinity Cache).
TUNE: dict = {
    ("parts_norm", 6144, 2560): (1, 512),        # add + RMSNorm + fused qkv
    ("parts_norm_silu", 9728, 2560): (1, 768),   # add + RMSNorm + gate_up + SwiGLU
    ("embed_norm", 6144, 2560): (1, 512),        # embedding + RMSNorm + qkv (layer 0)
    ("parts", 2560, 4096): (1, 1024),            # o_proj
    ("parts", 2560, 9728): (1, 512),             # down_proj
    ("lm_head", 151936, 2560): (1, 512),         # lm_head + argmax partials
}


def _tune(kind: str, n: int, k: int, m: int):
    return TUNE.get((kind, n, k, m), TUNE.get((kind, n, k), (0, 0)))


# ----------------------------------------------------------------------------
# availability (ek_kernels.py:44-70: has_triton / disable_triton / probe_triton)
# ----------------------------------------------------------------------------
def has_hip() -> bool:
    return not _DISABLED and _hip.available()


def disable_hip() -> None:
    global _DISABLED
    _DISABLED = True


def probe_hip() -> bool:
    """Load the library and run one kernel on the GPU (ek_kernels.py:53-70)."""
    global _DISABLED
    if _DISABLED or not torch.cuda.is_available():
        return False
    try:
        x = torch.ones(2, 64, device="cuda", dtype=_BF16)
        w = torch.ones(64, device="cuda", dtype=_BF16)
        y = rms_norm(x, w, 1e-6)
        torch.cuda.synchronize()
        if not torch.isfinite(y.float()).all():
            raise RuntimeError("bad output")
    except Exception:
        _DISABLED = True
    return not _DISABLED


# the reference's names for the same three functions
has_triton = has_hip
disable_triton = disable_hip
probe_triton = probe_hip


def _next_pow2(n: int) -> int:
    """ek_kernels.py:73-77."""
    p = 1
    while p < n:
        p <<= 1
    return p


def _cdiv(a: int, b: int) -> int:
    """ek_kernels.py:80-81."""
    return -(-a // b)


def _torch_rms_norm(x, w, eps):
    """The RMSNorm formula of ek_kernels.py:1025-1028, exported (as the
    reference exports it) for callers' own comparisons. No kernel path here
    calls it."""
    xf = x.float()
    xn = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * xn.to(x.dtype)


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _gpu(*ts) -> None:
    if _DISABLED:
        raise HipUnavailable("HIP kernels were disabled (disable_hip())")
    for t in ts:
        if t is not None and not t.is_cuda:
            raise HipUnavailable("enginekernel_amd kernels run on the GPU only; got a CPU tensor")


def _rows(t, name: str, dtype=_BF16):
    _need(t.dtype == dtype, f"{name}: expected {dtype}, got {t.dtype}")
    _need(t.dim() >= 1 and t.stride(-1) == 1, f"{name}: last dimension must be contiguous")
    return t


# ----------------------------------------------------------------------------
# norms and activations
# ----------------------------------------------------------------------------
def rms_norm(x, w, eps):
    """ek_kernels.py:1031-1042 -> y = w (x) bf16(x * rsqrt(mean(x^2) + eps))."""
    _gpu(x, w)
    shape = x.shape
    x2 = _rows(x.reshape(-1, shape[-1]), "rms_norm x")
    y = torch.empty(x2.shape, dtype=x.dtype, device=x.device)
    call("ek_rms_norm", ptr(x2), ptr(w.contiguous()), ptr(y), x2.shape[0], shape[-1], x2.stride(0),
         y.stride(0), float(eps), stream())
    return y.view(shape)


def add_rms_norm(x, residual, w, eps):
    """ek_kernels.py:1045-1059: residual += x (bf16, in place); returns
    (rmsnorm(residual) * w, residual)."""
    _gpu(x, residual, w)
    shape = x.shape
    x2 = _rows(x.reshape(-1, shape[-1]), "add_rms_norm x")
    r2 = _rows(residual.view(-1, shape[-1]), "add_rms_norm residual")
    y = torch.empty(x2.shape, dtype=x.dtype, device=x.device)
    call("ek_add_rms_norm", ptr(x2), ptr(r2), ptr(w.contiguous()), ptr(y), x2.shape[0], shape[-1],
         x2.stride(0), r2.stride(0), y.stride(0), float(eps), stream())
    return y.view(shape), residual


def silu_mul(gu):
    """ek_kernels.py:1062-1076: gu [..., 2I] -> bf16(silu(gate)) (x) up, [..., I]."""
    _gpu(gu)
    shape = list(gu.shape)
    n = shape[-1] // 2
    x2 = _rows(gu.reshape(-1, shape[-1]), "silu_mul")
    y = torch.empty(x2.shape[0], n, dtype=gu.dtype, device=gu.device)
    call("ek_silu_mul", ptr(x2), ptr(y), x2.shape[0], n, x2.stride(0), y.stride(0), stream())
    shape[-1] = n
    return y.view(shape)


def qk_norm_rope_kv(qkv, qn, kn, cos, sin, k_cache, v_cache, slot_base, n_q, n_kv, eps, m_per_batch):
    """ek_kernels.py:1110-1146: QK-norm + rotary on the fused QKV rows, q in
    place, rotated k and raw v written to the caches at slot_base[b] + row.
    Slots outside the cache are skipped."""
    _gpu(qkv, k_cache, v_cache, slot_base)
    d = qn.shape[0]
    m = qkv.shape[0]
    _rows(qkv, "qkv")
    _need(qkv.shape[1] >= (n_q + 2 * n_kv) * d, "qkv: too narrow for the head counts")
    _need(cos.shape[0] >= m and sin.shape[0] >= m and cos.stride(0) == sin.stride(0), "cos/sin rows")
    _need(k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride(), "k/v cache layouts differ")
    _need(k_cache.stride(-1) == 1 and k_cache.shape[1] == n_kv and k_cache.shape[3] == d, "cache shape")
    _need(m % m_per_batch == 0 and slot_base.dtype == torch.int64 and
          slot_base.numel() >= m // m_per_batch, "slot_base")
    _need(k_cache.shape[0] >= m // m_per_batch, "cache batch")
    call("ek_qk_norm_rope_kv", ptr(qkv), ptr(qn), ptr(kn), ptr(cos), ptr(sin), ptr(k_cache), ptr(v_cache),
         ptr(slot_base), m, qkv.stride(0), cos.stride(0), n_q, n_kv, d, k_cache.stride(0),
         k_cache.stride(1), k_cache.stride(2), k_cache.shape[2], m_per_batch, float(eps), stream())
    return qkv


# ----------------------------------------------------------------------------
# projections
# ----------------------------------------------------------------------------
def _check_proj(x, w, name):
    _gpu(x, w)
    _rows(x, name + " x")
    _rows(w, name + " w")
    _need(x.dim() == 2 and w.dim() == 2 and x.shape[1] == w.shape[1], f"{name}: x [M,K] and w [N,K] disagree")
    _need(x.shape[1] % 8 == 0, f"{name}: K must be a multiple of 8")


def gemv(x, w, out=None, cfg=None):
    """ek_kernels.py:1322-1347: x [M, K], w [N, K] -> bf16 [M, N] (fp32 accumulate).
    `cfg` (the reference's Triton block sizes) is accepted and ignored."""
    _check_proj(x, w, "gemv")
    m, k = x.shape
    n = w.shape[0]
    y = torch.empty(m, n, device=x.device, dtype=x.dtype) if out is None else out
    _need(y.shape == (m, n) and y.stride(-1) == 1, "gemv: out shape")
    call("ek_gemv", ptr(x), ptr(w), ptr(y), m, n, k, x.stride(0), w.stride(0), y.stride(0),
         *_tune("gemv", n, k, m), stream())
    return y


def gemv_parts(x, w, sk=None, out=None):
    """ek_kernels.py:1277-1293: fp32 split-K partials [sk, M, N] (M <= 8).
    sk defaults to the fewest splits whose activation rows fit the LDS
    stage (1 at batch 1: on gfx950 one wave streams a whole row of K). `out`
    (optional, contiguous fp32 [sk, M, N]) receives the partials."""
    _check_proj(x, w, "gemv_parts")
    m, k = x.shape
    n = w.shape[0]
    sk = int(sk or os.environ.get("ENGINE_SPLIT_K", "0") or parts_splits(m, k))
    _need(1 <= m <= 8, "gemv_parts: M must be 1..8")
    _need(k % (8 * sk) == 0, "gemv_parts: K must split into multiples of 8")
    parts = torch.empty(sk, m, n, device=x.device, dtype=torch.float32) if out is None else out
    _need(parts.shape == (sk, m, n) and parts.is_contiguous() and parts.dtype == torch.float32, "parts out")
    call("ek_gemv_parts", ptr(x), ptr(w), ptr(parts), m, n, k, x.stride(0), w.stride(0), sk,
         *_tune("parts", n, k, m), stream())
    return parts


ACT_STAGE_BYTES = 48 * 1024   # the kernels' per-workgroup activation stage


def parts_splits(m: int, k: int) -> int:
    """Smallest split-K count whose per-split activation rows (m padded to
    1/2/4/8, times K / sk bf16) fit the kernels' LDS activation stage."""
    bm = 1 if m <= 1 else 2 if m <= 2 else 4 if m <= 4 else 8
    sk = 1
    while bm * (k // sk) * 2 > ACT_STAGE_BYTES or (k % (8 * sk)):
        sk += 1
        if sk > k // 8:
            raise ValueError(f"no split of K={k} fits {m} rows")
    return sk


def add_rms_norm_parts(parts, residual, w, eps, out=None):
    """ek_kernels.py:1296-1304: residual += bf16(sum(parts)) in place;
    returns (norm * w, residual). `out` (optional, [M, N] bf16 rows)
    receives the normed rows."""
    _gpu(parts, residual, w)
    sk, m, n = parts.shape
    _need(parts.dtype == torch.float32 and parts.is_contiguous(), "parts: contiguous fp32 [sk, M, N]")
    _rows(residual, "residual")
    _need(residual.shape == (m, n), "residual shape")
    y = torch.empty(m, n, device=parts.device, dtype=residual.dtype) if out is None else out
    _need(y.shape == (m, n) and y.stride(-1) == 1 and y.dtype == residual.dtype, "add_rms_norm_parts: out")
    call("ek_add_rms_norm_parts", ptr(parts), ptr(residual), ptr(w), ptr(y), sk, m, n, residual.stride(0),
         y.stride(0), float(eps), stream())
    return y, residual


def gemv_swiglu(x, w, out=None):
    """ek_kernels.py:1247-1261: w is the fused [2I, K] gate/up matrix ->
    bf16(silu(bf16 gate)) (x) bf16(up), [M, I] (M <= 8). `out` (optional)
    receives the [M, I] rows."""
    _check_proj(x, w, "gemv_swiglu")
    m, k = x.shape
    i = w.shape[0] // 2
    _need(1 <= m <= 8, "gemv_swiglu: M must be 1..8")
    y = torch.empty(m, i, device=x.device, dtype=x.dtype) if out is None else out
    _need(y.shape == (m, i) and y.stride(-1) == 1, "gemv_swiglu: out")
    call("ek_gemv_swiglu", ptr(x), ptr(w), ptr(y), m, i, k, x.stride(0), w.stride(0), y.stride(0),
         *_tune("swiglu", i, k, m), stream())
    return y


def norm_gemv(x, residual, norm_w, w, eps, silu=False):
    """ek_kernels.py:1220-1244: y = proj(rmsnorm(x + residual)); returns
    (y, x + residual). residual=None: no add (the returned residual is x).
    silu=True: w is the fused [2I, K] gate/up matrix and y = silu(gate)*up."""
    _check_proj(x, w, "norm_gemv")
    m, k = x.shape
    _need(1 <= m <= 8, "norm_gemv: M must be 1..8")
    n = w.shape[0] // 2 if silu else w.shape[0]
    y = torch.empty(m, n, device=x.device, dtype=x.dtype)
    has_add = residual is not None
    r_out = torch.empty_like(x) if has_add else x
    if has_add:
        _rows(residual, "residual")
    call("ek_norm_gemv", ptr(x), ptr(residual) if has_add else None, ptr(r_out) if has_add else None,
         ptr(norm_w), ptr(w), ptr(y), m, n, k, x.stride(0), residual.stride(0) if has_add else 0,
         r_out.stride(0), w.stride(0), y.stride(0), float(eps), 1 if silu else 0,
         *_tune("norm_silu" if silu else "norm", n, k, m), stream())
    return y, r_out


def parts_norm_gemv(parts, residual, residual_out, norm_w, w, eps, silu=False, out=None):
    """The decode layer's fused consumer: r = bf16(residual + bf16(sum parts))
    -> residual_out; y = proj(rmsnorm(r) * norm_w) [+ SwiGLU]. The
    composition of add_rms_norm_parts (ek_kernels.py:1296) with gemv (:1322)
    or gemv_swiglu (:1247) in one launch. residual_out must not alias
    residual (other workgroups still read it)."""
    _gpu(parts, residual, residual_out, w)
    sk, m, k = parts.shape
    _need(parts.dtype == torch.float32 and parts.is_contiguous(), "parts: contiguous fp32")
    _need(residual.shape == (m, k) and residual_out.shape == (m, k), "residual shapes")
    _need(residual.data_ptr() != residual_out.data_ptr(), "residual_out must not alias residual")
    _need(w.shape[1] == k and w.stride(-1) == 1, "w shape")
    n = w.shape[0] // 2 if silu else w.shape[0]
    y = torch.empty(m, n, device=parts.device, dtype=_BF16) if out is None else out
    call("ek_parts_norm_gemv", ptr(parts), sk, ptr(residual), ptr(residual_out), ptr(norm_w), ptr(w), ptr(y),
         m, n, k, residual.stride(0), residual_out.stride(0), w.stride(0), y.stride(0), float(eps),
         1 if silu else 0, *_tune("parts_norm_silu" if silu else "parts_norm", n, k, m), stream())
    return y


def embed_norm_gemv(tokens, embed, residual_out, norm_w, w, eps, slot_t=None, len_t=None, out=None):
    """The decode step's first projection: residual_out = embed[tokens];
    y = proj(rmsnorm(residual_out) * norm_w). With slot_t/len_t it also
    performs the step's `slot_t <- len_t; len_t += 1` (ek_model.py:375-376)."""
    _gpu(tokens, embed, residual_out, w)
    m = tokens.shape[0]
    k = embed.shape[1]
    _need(tokens.dtype == torch.int64 and tokens.is_contiguous(), "tokens: int64")
    _need(w.shape[1] == k and residual_out.shape == (m, k), "shapes")
    if len_t is not None:
        _need(slot_t is not None and slot_t.dtype == torch.int64 and len_t.dtype == torch.int64
              and slot_t.numel() >= m, "slot_t/len_t")
    n = w.shape[0]
    y = torch.empty(m, n, device=tokens.device, dtype=_BF16) if out is None else out
    call("ek_embed_norm_gemv", ptr(tokens), ptr(embed), embed.stride(0), embed.shape[0], ptr(residual_out),
         ptr(norm_w), ptr(w), ptr(y), m, n, k, residual_out.stride(0), w.stride(0), y.stride(0), float(eps),
         ptr(slot_t) if len_t is not None else None, ptr(len_t), *_tune("embed_norm", n, k, m), stream())
    return y


class ArgmaxScratch:
    """Per-workgroup (value, index) partials of lm_head_argmax: room for the
    widest grid any launch shape can use (one row per wave)."""

    def __init__(self, m: int, vocab: int, device):
        self.cap = _cdiv(vocab, 4) * m
        self.val = torch.empty(self.cap, dtype=torch.float32, device=device)
        self.idx = torch.empty(self.cap, dtype=torch.int32, device=device)


def lm_head_argmax(hidden, lm_head, scratch: ArgmaxScratch, out_tok=None, logits=None,
                   parts=None, residual=None, norm_w=None, eps=1e-6, state=None, max_steps=0):
    """ek_model.py:490-493 argmax_token as one kernel: bf16 logits and the
    first-index argmax. With parts/residual/norm_w the final add + RMSNorm
    (ek_model.py:413-416) runs in its prologue instead of taking `hidden`.
    state = (tokens, positions, out_buf, step_idx) also performs the graph
    step's bookkeeping (engine.py:289-292)."""
    fused = parts is not None
    src = residual if fused else hidden
    _gpu(src, lm_head)
    m, k = src.shape
    vocab = lm_head.shape[0]
    _need(lm_head.shape[1] == k and lm_head.stride(-1) == 1, "lm_head shape")
    _need(1 <= m <= 8, "lm_head_argmax: M must be 1..8")
    _need(scratch.cap >= _cdiv(vocab, 4) * m, "argmax scratch too small")
    if out_tok is None:
        out_tok = torch.empty(m, dtype=torch.int64, device=src.device)
    if logits is not None:
        _need(logits.shape == (m, vocab) and logits.stride(-1) == 1 and logits.dtype == _BF16, "logits")
    st = (None,) * 4
    if state is not None:
        tokens, positions, out_buf, step_idx = state
        _need(out_buf.dtype == torch.int32 and out_buf.shape[1] == m and out_buf.is_contiguous(), "out_buf")
        st = (tokens, positions, out_buf, step_idx)
        max_steps = out_buf.shape[0]
    if fused:
        _need(parts.dtype == torch.float32 and parts.is_contiguous() and parts.shape[1:] == (m, k), "parts")
    call("ek_lm_head_argmax", ptr(hidden) if not fused else None, ptr(parts) if fused else None,
         parts.shape[0] if fused else 0, ptr(residual) if fused else None, ptr(norm_w) if fused else None,
         float(eps), ptr(lm_head), m, vocab, k, 0 if fused else hidden.stride(0),
         residual.stride(0) if fused else 0, lm_head.stride(0), ptr(logits),
         logits.stride(0) if logits is not None else 0, ptr(scratch.val), ptr(scratch.idx), scratch.cap,
         ptr(out_tok), ptr(st[0]), ptr(st[1]), ptr(st[2]), ptr(st[3]), max_steps,
         *_tune("lm_head", vocab, k, m), stream())
    return out_tok


# ----------------------------------------------------------------------------
# the whole decode step as one persistent launch
# ----------------------------------------------------------------------------
def decode_step_plan(hidden: int, inter: int, n_q: int, n_kv: int, head_dim: int, vocab: int, m: int,
                     s_cap: int, n_layers: int):
    """(arena bytes, long-context key split, barrier bytes, grid) when the
    persistent decode-step kernel handles this shape, else None (see
    decode_step). The split is 0 when each kv head's scores fit one attention
    unit's LDS (attention then runs on workgroups of its own beside the
    projections); otherwise every workgroup attends 1 / split of a kv head's
    keys and the splits combine through the arena."""
    import ctypes
    lib = _hip.load()
    sizes = (ctypes.c_int64 * 4)()
    rc = lib.ek_decode_step_plan(hidden, inter, n_q, n_kv, head_dim, vocab, m, s_cap, n_layers, sizes)
    if rc != 0:
        return None
    return tuple(int(v) for v in sizes)


class StepScratch:
    """Device state of the persistent decode step: the hand-over arena, the
    launch-state block and the error word, sized by decode_step_plan and
    zeroed once (the kernel keeps a launch epoch in them). One per (model,
    batch, arena size); launches sharing it must not overlap."""

    def __init__(self, sizes, device):
        arena_bytes, _, bar_bytes, grid = sizes
        self.arena = torch.zeros((arena_bytes + 7) // 8, dtype=torch.int64, device=device)
        self.barrier = torch.zeros((bar_bytes + 3) // 4, dtype=torch.int32, device=device)
        self.err = torch.zeros(1, dtype=torch.int32, device=device)
        self.arena_bytes, self.grid = arena_bytes, grid

    def reset(self) -> None:
        """Zero the arena, the launch state and the error word (after an
        abandoned launch)."""
        self.arena.zero_()
        self.barrier.zero_()
        self.err.zero_()

    def check(self) -> None:
        """Raise if a launch abandoned a hand-over wait (its outputs are invalid)."""
        if int(self.err.item()) != 0:
            self.reset()
            raise RuntimeError("decode_step: a hand-over wait timed out; the step's outputs are invalid")


def layer_table(layers, k_cache, v_cache, device) -> torch.Tensor:
    """The device pointer table [n_layers, 10] of decode_step: qkv, o, gu,
    down, ln1, ln2, qn, kn, k_cache, v_cache addresses per layer."""
    rows = [[lay["qkv"].data_ptr(), lay["o"].data_ptr(), lay["gu"].data_ptr(), lay["down"].data_ptr(),
             lay["ln1"].data_ptr(), lay["ln2"].data_ptr(), lay["qn"].data_ptr(), lay["kn"].data_ptr(),
             kc.data_ptr(), vc.data_ptr()] for lay, kc, vc in zip(layers, k_cache, v_cache)]
    return torch.tensor(rows, dtype=torch.int64).to(device)


def decode_step(table, cfg, embed, lm_head, final_norm, cos, sin, k_cache0, s_cap, tokens, positions, len_t,
                slot_t, start_t, out_buf, step_idx, scratch: StepScratch, out_tok=None, logits=None, err=None):
    """ek_model.py:360-416 + :490-493 + engine.py:288-292 (the captured step
    body) as ONE persistent launch: every layer, the final norm, lm_head, the
    first-index argmax and the step bookkeeping (tokens <- next, positions +=
    1, slot_t <- len, len += 1, out_buf[step_idx] <- next, step_idx += 1).
    Batch 1..8 rows (2..8: the batch form of the kernel); `table` from
    layer_table; k_cache0 gives the cache strides. logits: optional bf16
    tensor of rows x vocab elements that receives the step's logits. err: the error word to use (default: the scratch's own); a step
    that gives up, and every step launched while the word is set, writes
    token -1 and advances only step_idx."""
    if err is None:
        err = scratch.err
    args = _step_args(table, cfg, embed, lm_head, final_norm, cos, sin, k_cache0, s_cap, tokens, positions, len_t,
                      slot_t, start_t, out_buf, step_idx, out_tok, logits, err)
    call("ek_decode_step", *args, ptr(scratch.arena), scratch.arena_bytes, ptr(scratch.barrier), ptr(err), stream())
    return tokens


def decode_step_noalloc(table, cfg, embed, lm_head, final_norm, cos, sin, k_cache0, s_cap, tokens, positions,
                        len_t, slot_t, start_t, out_buf, step_idx, err, out_tok=None, logits=None):
    """decode_step on the library's static per-device hand-over state instead
    of a StepScratch: nothing is allocated, by the caller or the library.
    Shapes whose arena exceeds the static 16 MiB are rejected; calls that
    overlap on one device race (they share that device's state). err: the
    caller's error word, as for decode_step."""
    args = _step_args(table, cfg, embed, lm_head, final_norm, cos, sin, k_cache0, s_cap, tokens, positions, len_t,
                      slot_t, start_t, out_buf, step_idx, out_tok, logits, err)
    call("ek_decode_step_noalloc", *args, ptr(err), stream())
    return tokens


def _step_args(table, cfg, embed, lm_head, final_norm, cos, sin, k_cache0, s_cap, tokens, positions, len_t, slot_t,
               start_t, out_buf, step_idx, out_tok, logits, err):
    """The checked leading arguments shared by the two decode-step entry points."""
    _gpu(tokens, embed, lm_head, k_cache0)
    m = tokens.shape[0]
    _need(out_buf.dtype == torch.int32 and out_buf.shape[1] == m and out_buf.is_contiguous(), "out_buf")
    _need(positions.numel() >= m and slot_t.numel() >= m and start_t.numel() >= m and k_cache0.shape[0] >= m,
          "row state / cache rows")
    if logits is not None:
        _need(logits.dtype == _BF16 and logits.is_contiguous() and logits.numel() == m * cfg.vocab_size, "logits")
    _need(err.dtype == torch.int32 and err.numel() >= 1 and err.device == tokens.device, "err")
    _need(table.dtype == torch.int64 and table.shape == (cfg.num_layers, 10) and table.is_contiguous(), "table")
    _need(embed.stride(-1) == 1 and lm_head.stride(-1) == 1 and cos.stride(0) == sin.stride(0), "weights")
    return (ptr(table), cfg.num_layers, cfg.hidden_size, cfg.intermediate_size, cfg.num_heads,
            cfg.num_kv_heads, cfg.head_dim, cfg.vocab_size, m, float(cfg.rms_eps), float(cfg.head_dim ** -0.5),
            ptr(embed), embed.stride(0), ptr(lm_head), ptr(final_norm), ptr(cos), ptr(sin), cos.stride(0),
            cos.shape[0], k_cache0.stride(0), k_cache0.stride(1), k_cache0.stride(2), s_cap,
            ptr(tokens), ptr(positions), ptr(len_t), ptr(slot_t), ptr(start_t), ptr(out_buf), ptr(step_idx),
            out_buf.shape[0], ptr(out_tok), ptr(logits))


# ----------------------------------------------------------------------------
# attention
# ----------------------------------------------------------------------------
_SMS = None


def _sm_count() -> int:
    """Compute units of device 0 (ek_kernels.py:1158-1163); 256 on MI355X."""
    global _SMS
    if _SMS is None:
        _SMS = (torch.cuda.get_device_properties(0).multi_processor_count
                if torch.cuda.is_available() else 256)
    return _SMS


MIN_SPLIT_KEYS = 256    # keys per split at least (plan_splits)
FUSED_BUCKET = 1024     # buckets taking one split, the single-launch kernel


def group_pad(n_heads: int, n_kv: int) -> int:
    """ek_kernels.py:1350-1352 (the padded query-group size of the workspace)."""
    return max(16, _next_pow2(n_heads // n_kv))


def attn_warps() -> int:
    """ek_kernels.py:1384-1386. The HIP kernels always run 4 waves of 64."""
    return int(os.environ.get("ENGINE_ATTN_WARPS", "0")) or 4


def plan_splits(batch: int, n_kv: int, bucket: int, block_n: int = 0, target_cta: int = 0):
    """ek_kernels.py:1355-1381: (splits, chunk, block_n). Aims for a target
    number of workgroups across (batch x kv heads x splits); one split when
    batch x kv heads already covers 0.8 of the CUs; chunk is a multiple of
    block_n with splits * chunk >= bucket. The reference targets two
    workgroups per SM; on MI355X the split sweeps put the optimum at one per
    CU (config 3 at batch 1: 32 splits x 8 kv heads; config 5 at batch 8: 4
    splits, 7 % faster per step than 8), and two rules are added: a split
    gets at least MIN_SPLIT_KEYS keys (the split combine costs more than the
    parallelism gains below that), and buckets up to FUSED_BUCKET take one
    split (the single-launch kernel, which keeps the scores in LDS). The
    split count is then rounded down to a power of two, so that the
    one-launch split form of ek_attn_decode takes the row (its combine needs
    one; at batch 1 and a 2304-key bucket: 8 splits in one launch rather
    than 9 in the two-launch pair)."""
    sms = _sm_count()
    target_cta = target_cta or int(os.environ.get("ENGINE_ATTN_CTA", "0")) or sms
    base = batch * n_kv
    if base >= sms * float(os.environ.get("ENGINE_ATTN_FILL", "0.8")) or bucket <= FUSED_BUCKET:
        splits = 1
    else:
        splits = max(1, min(32, _cdiv(target_cta, base), bucket // MIN_SPLIT_KEYS))
    if not block_n:
        block_n = int(os.environ.get("ENGINE_ATTN_BLOCK", "0"))
    if not block_n:
        block_n = 128 if (splits == 1 and base <= sms) else 64
    splits = max(1, min(splits, _cdiv(bucket, block_n)))
    splits = 1 << (splits.bit_length() - 1)
    chunk = _cdiv(_cdiv(bucket, splits), block_n) * block_n
    return splits, chunk, block_n


def make_workspace(b: int, n_q: int, n_kv: int, head_dim: int, bucket: int, device, splits=None, chunk=None):
    """The attention workspace: the reference's 7-tuple (acc, lsum, mmax, out,
    splits, chunk, block_n) of engine.py:273-282, extended with the score
    scratch [B, n_q, bucket] fp32, the split combine's ticket block
    (int32 [B, n_kv, 2], zeroed; the kernels keep an arrival count and an
    epoch in it) and an error word (int32 [1]: set by a device-side wait
    that gave up, cleared by the caller; ws_error returns it), then the
    splits' exchange words (int64 [B, n_kv, SP, G (D + 2)]: partial outputs
    and per-split statistics as 64-bit {value, tag} words, enough for the
    one-launch split form; the reference's `acc` ([B, n_kv, SP, GP, D] fp32)
    is kept for its callers and holds the pair's partials when a 7-tuple
    workspace comes in)."""
    s, c, bn = plan_splits(b, n_kv, bucket)
    if splits is not None:
        s = splits
        c = chunk if chunk is not None else _cdiv(bucket, s)
    sp = _next_pow2(s)
    gp = group_pad(n_q, n_kv)
    acc = torch.zeros((b, n_kv, sp, gp, head_dim), dtype=torch.float32, device=device)
    lsum = torch.zeros((b, n_kv, sp, gp), dtype=torch.float32, device=device)
    mmax = torch.full((b, n_kv, sp, gp), -1e30, dtype=torch.float32, device=device)
    out = torch.empty((b, n_q, head_dim), dtype=_BF16, device=device)
    scores = torch.empty((b, n_q, bucket), dtype=torch.float32, device=device)
    ticket = torch.zeros((b, n_kv, 2), dtype=torch.int32, device=device)
    err = torch.zeros(1, dtype=torch.int32, device=device)
    g = n_q // n_kv
    words = torch.zeros((b, n_kv, sp, g * (head_dim + 2)), dtype=torch.int64, device=device)
    return (acc, lsum, mmax, out, s, c, bn, scores, ticket, err, words)


def ws_error(ws):
    """The workspace's error word (a 1-element int32 device tensor), or None
    for a reference-style workspace that has none."""
    return ws[9] if ws is not None and len(ws) >= 10 else None


def check_error_word(err, what: str = "a kernel") -> None:
    """Raise HipKernelError if the error word `err` (device int32) is set,
    i.e. a device-side wait of `what` gave up and its outputs are invalid.
    Reads the word back (waits for the work queued before it)."""
    if err is not None and int(err.reshape(-1)[0].item()) != 0:
        raise HipKernelError(what, 1, "a device-side wait gave up; the outputs are invalid")


_SCRATCH: dict = {}


def _attn_scratch(ws, b, n_q, n_kv, s_cap, device):
    """The score scratch and the ticket block; for a reference-style 7-tuple
    workspace they are allocated once per shape (eager callers only)."""
    if len(ws) >= 9:
        return ws[7], ws[8]
    key = (device, b, n_q, n_kv, s_cap)
    if key not in _SCRATCH:
        _SCRATCH[key] = (ws[7] if len(ws) >= 8 else torch.empty((b, n_q, s_cap), dtype=torch.float32, device=device),
                         torch.zeros((b, n_kv, 2), dtype=torch.int32, device=device))
    return _SCRATCH[key]


def _attn(q, ldq_b, ldq_h, rope, qn, kn, cos, sin, positions, k_cache, v_cache, seq_len_t, start_t,
          workspace, sm_scale, n_q, eps):
    acc, lsum, mmax, out, splits, chunk, _block_n = workspace[:7]
    b = out.shape[0]
    n_kv, s_cap, d = k_cache.shape[1], k_cache.shape[2], k_cache.shape[3]
    _need(k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride(), "k/v cache layouts differ")
    _need(k_cache.dtype == _BF16 and k_cache.stride(-1) == 1 and k_cache.shape[0] >= b, "cache")
    _need(n_q % n_kv == 0 and out.shape[1] == n_q and out.shape[2] == d, "head counts / workspace")
    _need(lsum.shape[:2] == (b, n_kv) and lsum.shape[2] >= splits and lsum.shape[3] >= n_q // n_kv
          and lsum.is_contiguous() and mmax.shape == lsum.shape and mmax.is_contiguous(), "lsum/mmax workspace")
    _need(splits * chunk >= 1, "splits/chunk")
    _need(seq_len_t.dtype == torch.int64 and start_t.dtype == torch.int32 and start_t.numel() >= b, "len/start")
    scores, ticket = _attn_scratch(workspace, b, n_q, n_kv, s_cap, out.device)
    _need(scores.shape[0] >= b and scores.shape[1] == n_q and scores.is_contiguous(), "score scratch")
    _need(ticket.dtype == torch.int32 and ticket.is_contiguous() and ticket.numel() >= 2 * b * n_kv, "ticket block")
    _need(acc.dtype == torch.float32 and acc.is_contiguous(), "acc (the splits' partial words)")
    part, part_words = (workspace[10], workspace[10].numel()) if len(workspace) >= 11 else (acc, acc.numel() // 2)
    _need(part.is_contiguous(), "exchange words")
    # the workspace bounds the attended length, as the reference's chunk plan does
    s_cap = min(s_cap, scores.shape[2])
    ld_cs = cos.stride(0) if cos is not None else 0
    rope_len = cos.shape[0] if cos is not None else 0
    call("ek_attn_decode", ptr(q), ldq_b, ldq_h, rope, ptr(qn), ptr(kn), ptr(cos), ptr(sin), ld_cs,
         ptr(positions), rope_len, ptr(k_cache), ptr(v_cache), k_cache.stride(0), k_cache.stride(1),
         k_cache.stride(2), s_cap, ptr(seq_len_t), ptr(start_t), ptr(scores), scores.stride(1),
         ptr(lsum), ptr(mmax), lsum.shape[2], lsum.shape[3], ptr(out), out.stride(0),
         out.stride(1), b, n_q, n_kv, d, splits, chunk, float(sm_scale), float(eps), ptr(part), part_words,
         ptr(ticket), ptr(ws_error(workspace)), stream())
    return out


def attn_prefill(qkv, k_cache, v_cache, start_t, s, n_q, sm_scale, out=None):
    """The prompt's causal GQA attention, ek_model.py:315-323 (SDPA with the
    _pack mask, engine.py:541-570): query heads from the fused rows qkv
    [B*S, (n_q + 2 n_kv) D] (already QK-normed and rotated), keys/values from
    the caches' slots [start_t[b], t] (written by qk_norm_rope_kv); padding
    tokens (t < start_t[b]) attend to themselves. Returns [B*S, n_q*D] bf16."""
    _gpu(qkv, k_cache, v_cache, start_t)
    _rows(qkv, "qkv")
    b, n_kv, s_cap, d = k_cache.shape
    _need(k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride(), "k/v cache layouts differ")
    _need(k_cache.dtype == _BF16 and k_cache.stride(-1) == 1, "cache")
    _need(qkv.shape[0] == b * s and qkv.shape[1] >= (n_q + 2 * n_kv) * d, "qkv rows [B*S, (n_q + 2 n_kv) D]")
    _need(start_t.dtype == torch.int32 and start_t.numel() >= b and start_t.is_contiguous(), "start_t: int32 [B]")
    y = torch.empty(b * s, n_q * d, device=qkv.device, dtype=_BF16) if out is None else out
    _need(y.shape == (b * s, n_q * d) and y.stride(-1) == 1, "attn_prefill: out")
    call("ek_attn_prefill", ptr(qkv), qkv.stride(0), ptr(k_cache), ptr(v_cache), k_cache.stride(0),
         k_cache.stride(1), k_cache.stride(2), s_cap, ptr(start_t), ptr(y), y.stride(0), b, s, n_q, n_kv, d,
         float(sm_scale), stream())
    return y


_VERIFY_PART: dict = {}


def verify_splits(s_cap: int) -> int:
    """Key splits of the verify attention: one per 64 cache rows (at most
    32; measured at the Qwen3-4B shape, 512-row cache: 4 / 8 / 16 splits ->
    3.49 / 3.33 / 3.37 ms per verify step); a split past a row's keys writes
    an empty partial and leaves at once."""
    return max(1, min(32, s_cap // 64))


def attn_verify(qkv, k_cache, v_cache, start_t, len_b, nq, n_q, sm_scale, out=None, splits=None):
    """The attention of a speculative verify step, ek_kernels.py:1419
    (flash_verify; torch form attn_torch, :1451): row b's nq query tokens
    (rows b*nq + j of the fused qkv [B*nq, (n_q + 2 n_kv) D], already
    QK-normed and rotated, their keys/values written at cache slots
    len_b[b] + j by qk_norm_rope_kv) see the keys at slots
    [start_t[b], len_b[b] + j]. Returns [B*nq, n_q*D] bf16."""
    _gpu(qkv, k_cache, v_cache, start_t, len_b)
    _rows(qkv, "qkv")
    b, n_kv, s_cap, d = k_cache.shape
    _need(k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride(), "k/v cache layouts differ")
    _need(k_cache.dtype == _BF16 and k_cache.stride(-1) == 1, "cache")
    _need(qkv.shape[0] == b * nq and qkv.shape[1] >= (n_q + 2 * n_kv) * d, "qkv rows [B*nq, (n_q + 2 n_kv) D]")
    _need(start_t.dtype == torch.int32 and start_t.numel() >= b and start_t.is_contiguous(), "start_t: int32 [B]")
    _need(len_b.dtype == torch.int64 and len_b.numel() >= b and len_b.is_contiguous(), "len_b: int64 [B]")
    y = torch.empty(b * nq, n_q * d, device=qkv.device, dtype=_BF16) if out is None else out
    _need(y.shape == (b * nq, n_q * d) and y.stride(-1) == 1, "attn_verify: out")
    sp = verify_splits(s_cap) if splits is None else int(splits)
    part = None
    if sp > 1:
        need = sp * b * nq * n_q * (d + 2)
        key = (qkv.device, need)
        part = _VERIFY_PART.get(key)
        if part is None:   # allocated once per shape, before any graph capture records the launch
            part = _VERIFY_PART[key] = torch.empty(need, dtype=torch.float32, device=qkv.device)
    call("ek_attn_verify", ptr(qkv), qkv.stride(0), ptr(k_cache), ptr(v_cache), k_cache.stride(0),
         k_cache.stride(1), k_cache.stride(2), s_cap, ptr(start_t), ptr(len_b), ptr(y), y.stride(0), b, nq, n_q,
         n_kv, d, float(sm_scale), ptr(part), part.numel() if part is not None else 0, sp, stream())
    return y


def ngram_draft(hist, hist_len, tokens):
    """ek_kernels.py:1510: tokens[B, Q] <- [last token, Q-1 n-gram drafts]
    per row of hist [B, H] (int64, first hist_len[b] entries valid)."""
    _gpu(hist, hist_len, tokens)
    _need(hist.dtype == torch.int64 and hist.dim() == 2 and hist.is_contiguous(), "hist: int64 [B, H]")
    b, h = hist.shape
    _need(hist_len.dtype == torch.int64 and hist_len.numel() >= b and hist_len.is_contiguous(), "hist_len")
    _need(tokens.dtype == torch.int64 and tokens.dim() == 2 and tokens.shape[0] == b and tokens.is_contiguous(),
          "tokens: int64 [B, Q]")
    call("ek_ngram_draft", ptr(hist), ptr(hist_len), ptr(tokens), b, h, tokens.shape[1], stream())
    return tokens


def spec_accept(tokens, am, hist, hist_len, len_b, pos_b, remaining, out_tok, out_adv, step_idx):
    """ek_kernels.py:1519: accept the longest draft prefix the model agrees
    with and do the step's bookkeeping (outputs at out_tok/out_adv[step_idx],
    history, lengths, positions, budget). step_idx is not advanced."""
    _gpu(tokens, am, hist, hist_len, len_b, pos_b, remaining, out_tok, out_adv, step_idx)
    b, q = tokens.shape
    for t, nm in ((tokens, "tokens"), (am, "am"), (hist, "hist"), (hist_len, "hist_len"), (len_b, "len_b"),
                  (pos_b, "pos_b"), (remaining, "remaining"), (step_idx, "step_idx")):
        _need(t.dtype == torch.int64 and t.is_contiguous(), f"spec_accept: {nm} must be contiguous int64")
    _need(am.shape == (b, q) and hist.dim() == 2 and hist.shape[0] == b, "spec_accept: am [B, Q], hist [B, H]")
    _need(out_tok.dtype == torch.int32 and out_tok.dim() == 3 and out_tok.shape[1:] == (b, q)
          and out_tok.is_contiguous(), "spec_accept: out_tok int32 [steps, B, Q]")
    _need(out_adv.dtype == torch.int32 and out_adv.shape == (out_tok.shape[0], b) and out_adv.is_contiguous(),
          "spec_accept: out_adv int32 [steps, B]")
    call("ek_spec_accept", ptr(tokens), ptr(am), ptr(hist), ptr(hist_len), ptr(len_b), ptr(pos_b),
         ptr(remaining), ptr(out_tok), ptr(out_adv), ptr(step_idx), b, hist.shape[1], q, out_tok.shape[0],
         stream())


def flash_decode(q, k_cache, v_cache, seq_len_t, start_t, workspace, sm_scale):
    """ek_kernels.py:1389-1416: q [B, HQ, D] (already rotated); caches
    [B, HKV, S, D]; seq_len_t (int64 [1]) / start_t (int32 [B]) on device.
    Keys [start_b, seq_len) are attended. Returns workspace's out [B, HQ, D]."""
    _gpu(q, k_cache, v_cache)
    _rows(q, "q")
    return _attn(q, q.stride(0), q.stride(1), 0, None, None, None, None, None, k_cache, v_cache,
                 seq_len_t, start_t, workspace, sm_scale, q.shape[1], 0.0)


def rope_attn_decode(qkv, qn, kn, cos, sin, k_cache, v_cache, seq_len_t, start_t, workspace,
                     sm_scale, n_q, eps, positions=None):
    """ek_kernels.py:1476-1507: QK-norm + rotary + cache write + decode
    attention from the raw fused QKV rows [B, (n_q + 2*n_kv)*D]; seq_len_t
    already counts the new token. cos/sin are per-row [B, D] tables, or the
    full tables when `positions` (int64 [B]) selects the rows."""
    _gpu(qkv, k_cache, v_cache)
    _rows(qkv, "qkv")
    n_kv, d = k_cache.shape[1], k_cache.shape[3]
    _need(qkv.shape[1] >= (n_q + 2 * n_kv) * d, "qkv too narrow")
    _need(cos.stride(0) == sin.stride(0) and cos.shape == sin.shape and cos.shape[1] >= d, "cos/sin")
    if positions is None:
        _need(cos.shape[0] >= qkv.shape[0], "cos/sin need a row per batch row")
    return _attn(qkv, qkv.stride(0), d, 1, qn, kn, cos, sin, positions, k_cache, v_cache, seq_len_t,
                 start_t, workspace, sm_scale, n_q, eps)
