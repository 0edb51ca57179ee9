"""Torch-on-CPU restatement of the reference fallback decode path (Appendix-A
arithmetic). TEST INFRASTRUCTURE ONLY; see oracle/__init__.py.

Every rounding point follows the reference's torch fallbacks:
`a (x) b` on bf16 tensors is one fp32 op rounded once to bf16; projections
are torch.matmul (fp32 accumulate, bf16 out); norms take fp32 statistics.
Citations are paths relative to the reference repository root.
"""

from __future__ import annotations

import json
import math
import os

import torch
import torch.nn.functional as F


# ----------------------------------------------------------------------------
# configuration -- engine/ek_model.py:26-42 (plus the transformers-5
# `rope_parameters.rope_theta` location, which the reference does not read)
# ----------------------------------------------------------------------------
class OracleConfig:
    def __init__(self, d: dict):
        self.hidden_size = d["hidden_size"]
        self.num_layers = d["num_hidden_layers"]
        self.num_heads = d["num_attention_heads"]
        self.num_kv_heads = d["num_key_value_heads"]
        self.head_dim = d.get("head_dim", self.hidden_size // self.num_heads)
        self.intermediate_size = d["intermediate_size"]
        self.vocab_size = d["vocab_size"]
        self.rms_eps = d.get("rms_norm_eps", 1e-6)
        theta = d.get("rope_theta")
        if theta is None:
            theta = (d.get("rope_parameters") or {}).get("rope_theta", 10000.0)
        self.rope_theta = float(theta)
        self.tie_embeddings = d.get("tie_word_embeddings", False)
        self.max_position = d.get("max_position_embeddings", 32768)
        self.q_size = self.num_heads * self.head_dim
        self.kv_size = self.num_kv_heads * self.head_dim

    @classmethod
    def from_path(cls, path: str) -> "OracleConfig":
        with open(os.path.join(path, "config.json")) as f:
            return cls(json.load(f))


# ----------------------------------------------------------------------------
# kernels' torch fallbacks -- engine/ek_kernels.py
# ----------------------------------------------------------------------------
def rms_norm(x, w, eps):
    """ek_kernels.py:1025-1028: w (x) bf16(x_f * rsqrt(mean(x_f^2) + eps))."""
    xf = x.float()
    xn = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * xn.to(x.dtype)


def add_rms_norm(x, residual, w, eps):
    """ek_kernels.py:1047-1049: residual = residual (+) x; (norm, residual)."""
    residual = residual + x
    return rms_norm(residual, w, eps), residual


def silu_mul(gu):
    """ek_kernels.py:1064-1066: bf16(silu_fp32(gate)) (x) up."""
    g, u = gu.chunk(2, dim=-1)
    return F.silu(g) * u


def qk_norm_rope_kv(qkv, qn, kn, cos, sin, k_cache, v_cache, slot_base,
                    n_q, n_kv, eps, m_per_batch):
    """ek_kernels.py:1119-1136: per-head RMSNorm, rotate-half RoPE in bf16,
    q rotated in place, rotated k and raw v written at slot_base[b] + row."""
    d = qn.shape[0]
    m = qkv.shape[0]
    b = m // m_per_batch
    half = d // 2
    q = qkv[:, : n_q * d].view(m, n_q, d)
    k = qkv[:, n_q * d: (n_q + n_kv) * d].view(m, n_kv, d)
    v = qkv[:, (n_q + n_kv) * d:].view(m, n_kv, d)
    c, sn = cos.unsqueeze(1), sin.unsqueeze(1)
    for t, w in ((q, qn), (k, kn)):
        tn = rms_norm(t, w, eps)
        rot = torch.cat((-tn[..., half:], tn[..., :half]), dim=-1)
        t.copy_(tn * c + rot * sn)
    ar = torch.arange(m_per_batch)
    slots = slot_base[:b, None] + ar[None, :]
    bi = torch.arange(b)[:, None].expand(b, m_per_batch)
    k_cache[bi, :, slots] = k.view(b, m_per_batch, n_kv, d)
    v_cache[bi, :, slots] = v.view(b, m_per_batch, n_kv, d)
    return qkv


def build_rope(head_dim: int, theta: float, max_len: int, dtype=torch.bfloat16):
    """ek_model.py:164-174: inv = 1/theta^(2i/D); emb = cat(t*inv, t*inv);
    cos/sin computed in fp32, then rounded to bf16."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    t = torch.arange(max_len, dtype=torch.float32)
    freqs = torch.outer(t, inv)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype).contiguous(), emb.sin().to(dtype).contiguous()


def decode_attn(q, kc, vc, seq_len: int, start_t, sm_scale: float):
    """ek_model.py:475-488: s = fp32(q.k)*scale, keys n < start_b masked,
    p = bf16(softmax_fp32(s)), o = bf16(sum_fp32 p*v). q: [B, HQ, D]."""
    n = int(seq_len)
    hq, hkv = q.shape[1], kc.shape[1]
    rep = hq // hkv
    k = kc[:, :, :n].repeat_interleave(rep, 1)
    v = vc[:, :, :n].repeat_interleave(rep, 1)
    scores = torch.einsum("bhd,bhsd->bhs", q.float(), k.float()) * sm_scale
    idx = torch.arange(n)
    scores = scores.masked_fill(idx[None, None, :] < start_t[:, None, None], float("-inf"))
    p = torch.softmax(scores, dim=-1).to(v.dtype)
    return torch.einsum("bhs,bhsd->bhd", p.float(), v.float()).to(q.dtype)


def lm_logits(hidden, lm_head):
    """ek_model.py:492: bf16(sum_fp32 h * E^T)."""
    return torch.matmul(hidden, lm_head.t())


def argmax_token(hidden, lm_head):
    """ek_model.py:490-493: first index of the max bf16 logit."""
    return torch.argmax(lm_logits(hidden, lm_head), dim=-1)


# ----------------------------------------------------------------------------
# model -- engine/ek_model.py (torch / ws=None branches)
# ----------------------------------------------------------------------------
class OracleQwen3:
    """The reference's Qwen3 on the torch fallback path, on CPU tensors.

    tensors: HF-named bf16 CPU tensors. q/k/v and gate/up are fused as in
    `ek_model.py:140-147`; the tied lm_head is the embedding (`:134`).
    """

    def __init__(self, cfg: OracleConfig, tensors: dict, rope_len: int | None = None):
        self.cfg = c = cfg
        self.embed = tensors["model.embed_tokens.weight"]
        self.final_norm = tensors["model.norm.weight"]
        self.lm_head = self.embed if c.tie_embeddings else tensors["lm_head.weight"]
        self.layers = []
        for i in range(c.num_layers):
            p = f"model.layers.{i}."
            self.layers.append({
                "qkv": torch.cat([tensors[p + "self_attn.q_proj.weight"],
                                  tensors[p + "self_attn.k_proj.weight"],
                                  tensors[p + "self_attn.v_proj.weight"]], 0).contiguous(),
                "gu": torch.cat([tensors[p + "mlp.gate_proj.weight"],
                                 tensors[p + "mlp.up_proj.weight"]], 0).contiguous(),
                "o": tensors[p + "self_attn.o_proj.weight"],
                "down": tensors[p + "mlp.down_proj.weight"],
                "ln1": tensors[p + "input_layernorm.weight"],
                "ln2": tensors[p + "post_attention_layernorm.weight"],
                "qn": tensors[p + "self_attn.q_norm.weight"],
                "kn": tensors[p + "self_attn.k_norm.weight"],
            })
        # ek_model.py:70 (then grown by ensure_rope, :176-178)
        n = rope_len or (c.max_position if c.max_position <= 16384 else 16384)
        self.cos, self.sin = build_rope(c.head_dim, c.rope_theta, n)
        self.rope_len = n
        self.sm_scale = c.head_dim ** -0.5

    @classmethod
    def from_path(cls, path: str, **kw) -> "OracleQwen3":
        from safetensors.torch import load_file
        import glob
        cfg = OracleConfig.from_path(path)
        tensors = {}
        for fn in sorted(glob.glob(os.path.join(path, "*.safetensors"))):
            tensors.update(load_file(fn))
        tensors = {k: v.to(torch.bfloat16) for k, v in tensors.items()}
        return cls(cfg, tensors, **kw)

    def ensure_rope(self, max_len: int):
        """ek_model.py:176-178."""
        if max_len > self.rope_len:
            self.rope_len = max(max_len, self.rope_len * 2)
            self.cos, self.sin = build_rope(self.cfg.head_dim, self.cfg.rope_theta, self.rope_len)

    def _proj(self, x, layer, key):
        """ek_model.py:203 (the torch.matmul branch)."""
        return torch.matmul(x, layer[key].t())

    def _prefill_proj(self, x, layer, key):
        """ek_model.py:298, :325 and :209 (the prefill's torch.matmul projections). A separate hook
        from _proj so that a fixture generator can re-run the prefill with
        another fp32 summation order without changing the decode's."""
        return torch.matmul(x, layer[key].t())

    def prefill(self, input_ids, positions, k_cache, v_cache, attn_bias=None):
        """ek_model.py:280-334, SDPA branch (:315-323). Writes cache slots
        [0, S); returns the final-normed hidden of the last position."""
        c = self.cfg
        b, s = input_ids.shape
        cos = self.cos.index_select(0, positions.reshape(-1))
        sin = self.sin.index_select(0, positions.reshape(-1))
        zero_slot = torch.zeros(b, dtype=torch.int64)
        h = F.embedding(input_ids, self.embed).reshape(b * s, c.hidden_size)
        residual = h
        x = None
        for i, layer in enumerate(self.layers):
            if i == 0:
                x = rms_norm(residual, layer["ln1"], c.rms_eps)
            else:
                x, residual = add_rms_norm(x, residual, layer["ln1"], c.rms_eps)
            qkv = self._prefill_proj(x, layer, "qkv")
            qk_norm_rope_kv(qkv, layer["qn"], layer["kn"], cos, sin,
                            k_cache[i], v_cache[i], zero_slot,
                            c.num_heads, c.num_kv_heads, c.rms_eps, s)
            q = qkv[:, : c.q_size].view(b, s, c.num_heads, c.head_dim).transpose(1, 2)
            k = k_cache[i][:, :, :s]
            v = v_cache[i][:, :, :s]
            o = F.scaled_dot_product_attention(q, k, v, attn_mask=attn_bias,
                                               is_causal=attn_bias is None,
                                               scale=self.sm_scale, enable_gqa=True)
            o = o.transpose(1, 2).reshape(b * s, c.q_size)
            x = self._prefill_proj(o, layer, "o")
            x, residual = add_rms_norm(x, residual, layer["ln2"], c.rms_eps)
            x = self._prefill_proj(silu_mul(self._prefill_proj(x, layer, "gu")), layer, "down")
        residual = residual + x
        last = residual.view(b, s, c.hidden_size)[:, -1, :]
        return rms_norm(last, self.final_norm, c.rms_eps)

    def decode(self, tokens, positions, k_cache, v_cache, slot_t, len_t, start_t):
        """ek_model.py:360-416 with ws=None: slot = len; len += 1; 36 layers
        of add+norm, fused qkv, QK-norm/RoPE/KV write, fallback attention,
        o_proj, add+norm, gate_up, SiLU*up, down; final add + norm."""
        c = self.cfg
        b = tokens.shape[0]
        cos = self.cos.index_select(0, positions)
        sin = self.sin.index_select(0, positions)
        slot_t.copy_(len_t.expand_as(slot_t))
        len_t.add_(1)
        residual = F.embedding(tokens, self.embed)
        x = None
        for i, layer in enumerate(self.layers):
            if i == 0:
                x = rms_norm(residual, layer["ln1"], c.rms_eps)
            else:
                x, residual = add_rms_norm(x, residual, layer["ln1"], c.rms_eps)
            qkv = self._proj(x, layer, "qkv")
            qk_norm_rope_kv(qkv, layer["qn"], layer["kn"], cos, sin,
                            k_cache[i], v_cache[i], slot_t,
                            c.num_heads, c.num_kv_heads, c.rms_eps, 1)
            q = qkv[:, : c.q_size].view(b, c.num_heads, c.head_dim)
            o = decode_attn(q, k_cache[i], v_cache[i], int(len_t.item()), start_t, self.sm_scale)
            o = o.reshape(b, c.q_size)
            x = self._proj(o, layer, "o")
            x, residual = add_rms_norm(x, residual, layer["ln2"], c.rms_eps)
            x = self._proj(silu_mul(self._proj(x, layer, "gu")), layer, "down")
        residual = residual + x
        return rms_norm(residual, self.final_norm, c.rms_eps)


# ----------------------------------------------------------------------------
# engine -- engine/engine.py
# ----------------------------------------------------------------------------
def pack(input_ids):
    """engine.py:541-570: left-pad to a rectangle; pad positions are 0, real
    positions 0..len_b-1; ragged batches get an additive bf16 -inf mask
    (causal AND key >= pad_b). Returns (ids, pos, pad, s, bias)."""
    rows = [list(map(int, r)) for r in input_ids]
    b = len(rows)
    lens = [len(r) for r in rows]
    s = max(lens)
    pad = [s - n for n in lens]
    if min(lens) == s:
        ids = torch.as_tensor(rows, dtype=torch.int64)
        pos = torch.arange(s, dtype=torch.int64).expand(b, s)
    else:
        ids = torch.zeros((b, s), dtype=torch.int64)
        pos = torch.zeros((b, s), dtype=torch.int64)
        for i, seq in enumerate(rows):
            ids[i, pad[i]:] = torch.as_tensor(seq, dtype=torch.int64)
            pos[i, pad[i]:] = torch.arange(lens[i], dtype=torch.int64)
    bias = None
    if max(pad) > 0:
        key_ok = torch.zeros((b, s), dtype=torch.bool)
        for i, p in enumerate(pad):
            key_ok[i, p:] = True
        allow = torch.ones((s, s), dtype=torch.bool).tril()[None] & key_ok[:, None, :]
        bias = torch.zeros((b, 1, s, s), dtype=torch.bfloat16)
        bias.masked_fill_(~allow.unsqueeze(1), float("-inf"))
    return ids, pos, pad, s, bias


class EagerState:
    """Device-free decode state of `_generate_eager` (engine.py:734-737)."""

    def __init__(self, model: OracleQwen3, b: int, s: int, pad, total: int):
        c = model.cfg
        shape = (b, c.num_kv_heads, total, c.head_dim)
        self.k = [torch.zeros(shape, dtype=torch.bfloat16) for _ in range(c.num_layers)]
        self.v = [torch.zeros(shape, dtype=torch.bfloat16) for _ in range(c.num_layers)]
        self.positions = torch.as_tensor([s - p for p in pad], dtype=torch.int64)
        self.slot_t = torch.zeros(b, dtype=torch.int64)
        self.len_t = torch.full((1,), s, dtype=torch.int64)
        self.start_t = torch.as_tensor(pad, dtype=torch.int32)


def generate_eager(model: OracleQwen3, input_ids, max_new_tokens: int,
                   record_logits: bool = False, force=None):
    """engine.py:721-743: zero caches, prefill, then (n-1) x decode + argmax.

    Yields list[int] of B token ids per step. With record_logits, yields
    (ids, bf16 logits [B, V]). `force` (list of per-step id lists) teacher-
    forces the fed-back tokens, as `bench/check_exact.py` does, so a near-tie
    at one step does not change every later step.
    """
    ids, pos, pad, s, bias = pack(input_ids)
    b = ids.shape[0]
    total = s + max_new_tokens
    model.ensure_rope(total + 1)
    st = EagerState(model, b, s, pad, total)
    with torch.inference_mode():
        hidden = model.prefill(ids, pos, st.k, st.v, bias)
        logits = lm_logits(hidden, model.lm_head)
        tok = torch.argmax(logits, dim=-1)
        yield (tok.tolist(), logits) if record_logits else tok.tolist()
        for step in range(1, max_new_tokens):
            if force is not None:
                tok = torch.as_tensor(force[step - 1], dtype=torch.int64)
            hidden = model.decode(tok, st.positions, st.k, st.v, st.slot_t, st.len_t, st.start_t)
            logits = lm_logits(hidden, model.lm_head)
            tok = torch.argmax(logits, dim=-1)
            st.positions = st.positions + 1
            yield (tok.tolist(), logits) if record_logits else tok.tolist()


def logit_gap(logits_row, a: int, b: int) -> float:
    """bench/check_exact.py rule helper: logit[a] - logit[b] in fp32."""
    r = logits_row.float()
    return float(r[a] - r[b])


def bf16_ulp(x: float) -> float:
    """Spacing of bf16 values at magnitude |x| (8 significant bits)."""
    x = abs(x)
    if x == 0:
        return 2.0 ** -133
    return 2.0 ** (math.floor(math.log2(x)) - 7)


# ----------------------------------------------------------------------------
# speculative decoding -- engine/engine.py:345-383 (the torch form of the
# draft/verify/accept step) and engine/ek_kernels.py:618-680 (the integer
# kernels that replace its draft and accept parts; where the two differ, at a
# full history, the kernels' behaviour is restated: no store past the row)
# ----------------------------------------------------------------------------
def ngram_draft(hist, hist_len, q: int):
    """engine.py:357-376 / ek_kernels.py:618-649: per row, [last token,
    q-1 drafts continuing the most recent earlier occurrence of the trailing
    3-gram (else 2-gram, else token), wrapping around a short cycle].
    hist [B, H] int64, hist_len [B] -> tokens [B, q] int64."""
    hist = torch.as_tensor(hist, dtype=torch.int64)
    b, h = hist.shape
    big = 1 << 20
    out = torch.empty((b, q), dtype=torch.int64)
    for r in range(b):
        hl = int(hist_len[r])
        row = hist[r].tolist()
        k_last, k_prev, k_pp = row[hl - 1], row[max(hl - 2, 0)], row[max(hl - 3, 0)]
        best = 0
        for j in range(0, hl - 1):                     # j <= hl - 2
            m1 = row[j] == k_last
            m2 = m1 and j >= 1 and row[j - 1] == k_prev
            m3 = m2 and j >= 2 and row[j - 2] == k_pp
            best = max(best, (j + 1 if m1 else 0) + (big if m2 else 0) + (2 * big if m3 else 0))
        p = best % big
        span = max(hl - p, 1)
        out[r, 0] = k_last
        for i in range(q - 1):
            out[r, i + 1] = row[min(p + i % span, h - 1)]
    return out


def spec_accept(tokens, am, hist, hist_len, len_b, pos_b, remaining, out_tok, out_adv, step: int):
    """engine.py:377-383 / ek_kernels.py:652-680, in place on CPU tensors:
    adv = min(1 + leading drafts equal to the argmax before them, remaining);
    outputs at out_tok/out_adv[step]; all q argmax tokens into hist[hl ..]
    inside the row; hist_len, len_b, pos_b += adv; remaining -= adv."""
    b, q = tokens.shape
    h = hist.shape[1]
    for r in range(b):
        nacc = 0
        while nacc < q - 1 and int(tokens[r, nacc + 1]) == int(am[r, nacc]):
            nacc += 1
        rem = int(remaining[r])
        adv = min(nacc + 1, rem)
        if 0 <= step < out_tok.shape[0]:
            out_tok[step, r] = am[r].to(torch.int32)
            out_adv[step, r] = adv
        hl = int(hist_len[r])
        for j in range(q):
            if hl + j < h:
                hist[r, hl + j] = am[r, j]
        hist_len[r] += adv
        len_b[r] += adv
        pos_b[r] += adv
        remaining[r] = rem - adv


def verify_attn(q, kc, vc, len_b, start_t, sm_scale: float, nq: int):
    """ek_kernels.py:1451-1475 (attn_torch, the verify attention's torch
    form): q [B*nq, HQ, D]; caches [B, HKV, S, D]; query j of row b sees
    keys [start_t[b], len_b[b] + j]; fp32 softmax, p rounded to bf16."""
    bq, hq, d = q.shape
    b = bq // nq
    hkv = kc.shape[1]
    g = hq // hkv
    bucket = kc.shape[2]
    qg = q.view(b, nq, hkv, g, d).permute(0, 2, 1, 3, 4).reshape(b, hkv, nq * g, d)
    scores = torch.matmul(qg, kc.transpose(-1, -2)).float() * sm_scale
    ar = torch.arange(bucket)
    qlen = torch.as_tensor(len_b, dtype=torch.int64)[:, None] + torch.arange(nq)[None, :] + 1
    qlen = qlen.repeat_interleave(g, dim=1)
    start = torch.as_tensor(start_t, dtype=torch.int64)
    ok = (ar[None, None, :] < qlen[:, :, None]) & (ar[None, None, :] >= start[:, None, None])
    scores = scores.masked_fill(~ok[:, None, :, :], float("-inf"))
    p = torch.softmax(scores, dim=-1).to(q.dtype)
    out = torch.matmul(p, vc)
    return out.view(b, hkv, nq, g, d).permute(0, 2, 1, 3, 4).reshape(bq, hq, d)
