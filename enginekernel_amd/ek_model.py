"""Qwen3 on the gfx950 decode kernels: the reference's ek_model API.

Same class names, constructor and methods as jeojdi1/EngineKernel
`engine/ek_model.py` (cited per method): Qwen3Config(path), Qwen3(path,
device, dtype) with .prefill, .decode, .argmax_token, .ensure_rope,
.use_gemv_for and the fused-weight layer dicts (qkv/o/gu/down and their
transposed views, ln1/ln2/qn/kn). Additions: Qwen3.from_random (seeded
random-init weights), Qwen3.step (the whole graph step, argmax and
bookkeeping included).

The decode step is six launches per layer, every one a hand-written HIP
kernel (ek_kernels):
    embed|parts+add+norm+qkv  ->  attention phase 1 (QK-norm, RoPE, KV write,
    scores)  ->  attention phase 2 (softmax, PV, split combine)  ->  o_proj
    ->  parts+add+norm+gate_up+SwiGLU  ->  down_proj
then one lm_head + final norm + argmax + step-advance launch. The residual
stream ping-pongs between two buffers so that the one workgroup writing the
new residual never races the workgroups still reading the old one.

The prefill (out of this build's hot-path scope) runs the same norms and
RoPE/KV-write kernels with torch (hipBLASLt) projections and an fp32 attention.
"""

from __future__ import annotations

import glob
import json
import os

import torch
import torch.nn.functional as F

from . import ek_kernels as K
from .checkpoint import random_weights


class Qwen3Config:
    """ek_model.py:26-42, plus transformers-5's `rope_parameters.rope_theta`
    (a config.json written by transformers 5 has no top-level rope_theta)."""

    def __init__(self, path: str | None = None, cfg: dict | None = None):
        if cfg is None:
            with open(os.path.join(path, "config.json")) as f:
                cfg = json.load(f)
        self.raw = dict(cfg)
        self.hidden_size = cfg["hidden_size"]
        self.num_layers = cfg["num_hidden_layers"]
        self.num_heads = cfg["num_attention_heads"]
        self.num_kv_heads = cfg["num_key_value_heads"]
        self.head_dim = cfg.get("head_dim", self.hidden_size // self.num_heads)
        self.intermediate_size = cfg["intermediate_size"]
        self.vocab_size = cfg["vocab_size"]
        self.rms_eps = cfg.get("rms_norm_eps", 1e-6)
        theta = cfg.get("rope_theta")
        if theta is None:
            theta = (cfg.get("rope_parameters") or {}).get("rope_theta", 10000.0)
        self.rope_theta = float(theta)
        self.tie_embeddings = cfg.get("tie_word_embeddings", False)
        self.max_position = cfg.get("max_position_embeddings", 32768)
        self.q_size = self.num_heads * self.head_dim
        self.kv_size = self.num_kv_heads * self.head_dim


def _safetensors_names(fn: str) -> list:
    """Tensor names in one .safetensors file, read from its header alone: an
    8-byte little-endian length, then that many bytes of JSON whose keys are
    the tensor names (plus an optional "__metadata__")."""
    with open(fn, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError(f"{fn}: truncated safetensors header")
        n = int.from_bytes(raw, "little")
        head = json.loads(f.read(n))
    return [k for k in head if k != "__metadata__"]


def shard_map(path: str) -> dict:
    """Tensor name -> shard file name of a local HF checkpoint (the lookup of
    ek_model.py:45-60): a sharded checkpoint's index names the file of every
    tensor; without one, each *.safetensors file's header lists its tensors.
    A name found in two files is an error rather than a silent override."""
    index = os.path.join(path, "model.safetensors.index.json")
    if os.path.isfile(index):
        with open(index) as f:
            return dict(json.load(f)["weight_map"])
    table: dict = {}
    for fn in sorted(glob.glob(os.path.join(path, "*.safetensors"))):
        base = os.path.basename(fn)
        for name in _safetensors_names(fn):
            if table.setdefault(name, base) != base:
                raise ValueError(f"tensor {name} is in both {table[name]} and {base}")
    if not table:
        raise FileNotFoundError(f"no safetensors under {path}")
    return table


def load_tensors(path: str, dtype=torch.bfloat16) -> dict:
    """Every tensor of a local HF checkpoint, on the CPU, as `dtype`."""
    from safetensors import safe_open

    wmap = shard_map(path)
    out = {}
    for fn in sorted(set(wmap.values())):
        with safe_open(os.path.join(path, fn), framework="pt", device="cpu") as f:
            for k in f.keys():
                out[k] = f.get_tensor(k).to(dtype)
    return out


def fuse_layer(tensors: dict, i: int) -> dict:
    """ek_model.py:139-160: q/k/v and gate/up concatenated along the output
    dimension ([out, in] row-major, a contiguous K per output row)."""
    p = f"model.layers.{i}."
    qkv = torch.cat([tensors[p + "self_attn.q_proj.weight"], tensors[p + "self_attn.k_proj.weight"],
                     tensors[p + "self_attn.v_proj.weight"]], dim=0).contiguous()
    gu = torch.cat([tensors[p + "mlp.gate_proj.weight"], tensors[p + "mlp.up_proj.weight"]], dim=0).contiguous()
    return {
        "qkv": qkv, "gu": gu,
        "o": tensors[p + "self_attn.o_proj.weight"].contiguous(),
        "down": tensors[p + "mlp.down_proj.weight"].contiguous(),
        "ln1": tensors[p + "input_layernorm.weight"].contiguous(),
        "ln2": tensors[p + "post_attention_layernorm.weight"].contiguous(),
        "qn": tensors[p + "self_attn.q_norm.weight"].contiguous(),
        "kn": tensors[p + "self_attn.k_norm.weight"].contiguous(),
    }


def rope_tables(head_dim: int, theta: float, max_len: int, dtype=torch.bfloat16):
    """ek_model.py:164-174, computed on the CPU (fp32, then rounded to bf16)
    so that every device sees the same bytes."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    t = torch.arange(max_len, dtype=torch.float32)
    freqs = torch.outer(t, inv)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype).contiguous(), emb.sin().to(dtype).contiguous()


class _StepBuffers:
    """Activations of one decode step at batch b (allocated once, reused by
    every step and by graph captures)."""

    def __init__(self, cfg: Qwen3Config, b: int, device):
        h = cfg.hidden_size
        bf = torch.bfloat16
        self.res = (torch.empty(b, h, dtype=bf, device=device), torch.empty(b, h, dtype=bf, device=device))
        self.qkv = torch.empty(b, cfg.q_size + 2 * cfg.kv_size, dtype=bf, device=device)
        self.sk_o = K.parts_splits(b, cfg.q_size)
        self.sk_down = K.parts_splits(b, cfg.intermediate_size)
        self.o_parts = torch.empty(self.sk_o, b, h, dtype=torch.float32, device=device)
        self.act = torch.empty(b, cfg.intermediate_size, dtype=bf, device=device)
        self.down_parts = torch.empty(self.sk_down, b, h, dtype=torch.float32, device=device)
        self.hidden = torch.empty(b, h, dtype=bf, device=device)
        self.xn = torch.empty(b, h, dtype=bf, device=device)       # normed rows (2..8-row path)
        self.att = torch.empty(b, cfg.q_size, dtype=bf, device=device)   # verify attention rows
        self.argmax = K.ArgmaxScratch(b, cfg.vocab_size, device)
        self.next_tok = torch.empty(b, dtype=torch.int64, device=device)
        self.step = None   # K.StepScratch of the persistent step's last launch, made on first use
        # every StepScratch made for this batch, by arena size (the long-context
        # plan's arena is larger); one a captured graph uses is never freed
        self.steps = {}


class Qwen3(torch.nn.Module):
    """ek_model.py:63-115 (constructor), on the HIP kernels only."""

    MAX_ROWS = 8   # rows per decode launch (the kernels' batch tile)

    def __init__(self, model_path: str | None, device: torch.device, dtype=torch.bfloat16, *,
                 tensors: dict | None = None, config: dict | None = None):
        super().__init__()
        device = torch.device(device)
        if device.type != "cuda":
            raise K.HipUnavailable("Qwen3 runs on the HIP kernels and needs a GPU device")
        if not K.has_hip():
            raise K.HipUnavailable("libek_hip.so is not loadable or no GPU is visible")
        self.cfg = Qwen3Config(model_path, config)
        self.device = device
        self.dtype = dtype
        if tensors is None:
            tensors = load_tensors(model_path, dtype)
        self._load(tensors)
        self._build_rope(self.cfg.max_position if self.cfg.max_position <= 16384 else 16384)
        self.sm_scale = self.cfg.head_dim ** -0.5
        self.zero_slot = torch.zeros(1024, dtype=torch.int64, device=device)
        self.arange_q = torch.arange(16, dtype=torch.int64, device=device)   # verify positions (<= 16 per row)
        self._bufs: dict = {}
        self._plans: dict = {}
        self._tables: dict = {}
        # the whole step as one persistent launch where its plan allows
        # (ENGINE_PERSISTENT=0 selects the per-kernel graph step everywhere),
        # up to persistent_rows rows (ENGINE_PERSISTENT_ROWS): at the
        # Qwen3-4B shape and config 5's prompts the one-launch step is the
        # faster one at every batch it takes (2, 4 and 8 rows: 2.19 / 2.62 /
        # 3.45 ms against 3.03 / 3.49 / 3.95 for the per-kernel graph)
        self.persistent = os.environ.get("ENGINE_PERSISTENT", "1") != "0"
        self.persistent_rows = int(os.environ.get("ENGINE_PERSISTENT_ROWS", "8"))
        # the prefill's hipBLASLt projections: no reduced-precision bf16 reductions
        torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction = False

    @classmethod
    def from_random(cls, config: dict, device, seed: int = 0, dtype=torch.bfloat16):
        """A seeded random-init model (weights ~N(0, 0.02), norm gains 1)."""
        return cls(None, device, dtype, tensors=random_weights(config, seed), config=config)

    # ------------------------------------------------------------------
    def _load(self, tensors: dict):
        """ek_model.py:117-162, from CPU tensors: fuse per layer, then upload."""
        c, dev = self.cfg, self.device
        self.embed = tensors["model.embed_tokens.weight"].to(dev, self.dtype).contiguous()
        self.final_norm = tensors["model.norm.weight"].to(dev, self.dtype).contiguous()
        self.lm_head = (self.embed if c.tie_embeddings
                        else tensors["lm_head.weight"].to(dev, self.dtype).contiguous())
        self.lm_head_t = self.lm_head.t()
        self.layers = []
        for i in range(c.num_layers):
            lay = {k: v.to(dev, self.dtype) for k, v in fuse_layer(tensors, i).items()}
            for key in ("qkv", "o", "gu", "down"):
                lay[key + "_t"] = lay[key].t()
            self.layers.append(lay)

    def _build_rope(self, max_len: int):
        cos, sin = rope_tables(self.cfg.head_dim, self.cfg.rope_theta, max_len, self.dtype)
        self.cos = cos.to(self.device)
        self.sin = sin.to(self.device)
        self.rope_len = max_len

    def ensure_rope(self, max_len: int):
        """ek_model.py:176-178."""
        if max_len > self.rope_len:
            self._build_rope(max(max_len, self.rope_len * 2))

    def use_gemv_for(self, rows: int) -> bool:
        """ek_model.py:214-266 chose Triton or cuBLAS by timing. Here the
        decode projections are always the HIP kernels, for 1..MAX_ROWS rows."""
        return 1 <= rows <= self.MAX_ROWS

    def buffers(self, b: int) -> _StepBuffers:
        if b not in self._bufs:
            self._bufs[b] = _StepBuffers(self.cfg, b, self.device)
        return self._bufs[b]

    # ------------------------------------------------------------------
    def prefill(self, input_ids, positions, k_cache, v_cache, attn_bias=None):
        """ek_model.py:280-334: input_ids/positions [B, S]; writes cache slots
        [0, S); returns the final-normed hidden of each row's last position.
        attn_bias is the prompt mask of engine._pack (causal, keys from each
        row's first real token) or None (causal); the attention is the HIP
        flash kernel (K.attn_prefill), the projections torch (hipBLASLt)."""
        c = self.cfg
        b, s = input_ids.shape
        cos = self.cos.index_select(0, positions.reshape(-1))
        sin = self.sin.index_select(0, positions.reshape(-1))
        zero_slot = self.zero_slot[:b] if b <= self.zero_slot.numel() else torch.zeros(
            b, dtype=torch.int64, device=self.device)
        residual = F.embedding(input_ids, self.embed).reshape(b * s, c.hidden_size)
        # the first visible key of each row: with the prompt mask (left
        # padding) it is S - len, read off the last position (len - 1)
        if attn_bias is None:
            start = torch.zeros(b, dtype=torch.int32, device=self.device)
        else:
            start = (s - 1 - positions[:, -1]).to(torch.int32).contiguous()
        x = None
        for i, layer in enumerate(self.layers):
            if i == 0:
                x = K.rms_norm(residual, layer["ln1"], c.rms_eps)
            else:
                x, residual = K.add_rms_norm(x, residual, layer["ln1"], c.rms_eps)
            qkv = torch.matmul(x, layer["qkv_t"])
            K.qk_norm_rope_kv(qkv, layer["qn"], layer["kn"], cos, sin, k_cache[i], v_cache[i], zero_slot,
                              c.num_heads, c.num_kv_heads, c.rms_eps, s)
            o = K.attn_prefill(qkv, k_cache[i], v_cache[i], start, s, c.num_heads, self.sm_scale)
            x = torch.matmul(o, layer["o_t"])
            x, residual = K.add_rms_norm(x, residual, layer["ln2"], c.rms_eps)
            x = torch.matmul(K.silu_mul(torch.matmul(x, layer["gu_t"])), layer["down_t"])
        residual = residual + x
        last = residual.view(b, s, c.hidden_size)[:, -1, :].contiguous()
        return K.rms_norm(last, self.final_norm, c.rms_eps)

    # ------------------------------------------------------------------
    def _layers(self, tokens, positions, k_cache, v_cache, slot_t, len_t, start_t, ws) -> _StepBuffers:
        """All layers of one decode step; leaves the last down_proj partials
        and the residual in the step buffers (final norm not applied)."""
        c = self.cfg
        b = tokens.shape[0]
        if not self.use_gemv_for(b):
            raise ValueError(f"decode batch {b} exceeds {self.MAX_ROWS} rows per launch")
        bufs = self.buffers(b)
        res_a, res_b = bufs.res
        # 1 row: the add + RMSNorm runs fused in each projection's prologue
        # (ping-pong residual rows); 2..8 rows: once per layer boundary in
        # add_rms_norm_parts (residual in res_a, in place), since the
        # matrix-core projections' workgroups would each repeat it over the
        # split-K partials
        split = b >= 2
        for i, layer in enumerate(self.layers):
            if i == 0:
                K.embed_norm_gemv(tokens, self.embed, res_a if split else res_b, layer["ln1"], layer["qkv"],
                                  c.rms_eps, slot_t=slot_t, len_t=len_t, out=bufs.qkv)
            elif split:
                K.add_rms_norm_parts(bufs.down_parts, res_a, layer["ln1"], c.rms_eps, out=bufs.xn)
                K.gemv(bufs.xn, layer["qkv"], out=bufs.qkv)
            else:
                K.parts_norm_gemv(bufs.down_parts, res_a, res_b, layer["ln1"], layer["qkv"], c.rms_eps,
                                  out=bufs.qkv)
            o = K.rope_attn_decode(bufs.qkv, layer["qn"], layer["kn"], self.cos, self.sin, k_cache[i],
                                   v_cache[i], len_t, start_t, ws, self.sm_scale, c.num_heads, c.rms_eps,
                                   positions=positions)
            K.gemv_parts(o.view(b, c.q_size), layer["o"], sk=bufs.sk_o, out=bufs.o_parts)
            if split:
                K.add_rms_norm_parts(bufs.o_parts, res_a, layer["ln2"], c.rms_eps, out=bufs.xn)
                K.gemv_swiglu(bufs.xn, layer["gu"], out=bufs.act)
            else:
                K.parts_norm_gemv(bufs.o_parts, res_b, res_a, layer["ln2"], layer["gu"], c.rms_eps, silu=True,
                                  out=bufs.act)
            K.gemv_parts(bufs.act, layer["down"], sk=bufs.sk_down, out=bufs.down_parts)
        return bufs

    def decode(self, tokens, positions, k_cache, v_cache, slot_t, len_t, start_t, ws=None):
        """ek_model.py:360-416: one decode step for tokens/positions [B];
        slot_t <- len_t; len_t += 1; returns the final-normed hidden [B, H].
        ws: the attention workspace (engine._make_ws); built on the fly if None."""
        if ws is None:
            ws = K.make_workspace(tokens.shape[0], self.cfg.num_heads, self.cfg.num_kv_heads,
                                  self.cfg.head_dim, k_cache[0].shape[2], self.device)
        bufs = self._layers(tokens, positions, k_cache, v_cache, slot_t, len_t, start_t, ws)
        res_a = bufs.res[0]
        hidden, _ = K.add_rms_norm_parts(bufs.down_parts, res_a, self.final_norm, self.cfg.rms_eps)
        return hidden

    def verify(self, tokens, pos_b, k_cache, v_cache, len_b, start_t, ws=None):
        """ek_model.py:418-472: score NQ tokens per sequence in one pass (the
        speculative verify). tokens [B, NQ] = the last emitted token and NQ-1
        drafts at positions pos_b[b] + j; their keys/values go to cache slots
        len_b[b] + j (what follows a rejected draft is overwritten by the next
        step). Returns the greedy token after each position, [B, NQ] int64.
        The HIP kernels of the 2..8-row decode at B*NQ rows, with the verify
        attention (K.attn_verify) in place of the decode attention; ws is
        accepted for the reference's signature and not used."""
        c = self.cfg
        b, nq = tokens.shape
        rows = b * nq
        if not self.use_gemv_for(rows):
            raise ValueError(f"verify: {rows} rows exceed {self.MAX_ROWS} rows per launch")
        positions = (pos_b[:, None] + self.arange_q[None, :nq]).reshape(-1).clamp(max=self.rope_len - 1)
        cos = self.cos.index_select(0, positions)
        sin = self.sin.index_select(0, positions)
        bufs = self.buffers(rows)
        res = bufs.res[0]
        tok = tokens.reshape(-1).contiguous()
        for i, layer in enumerate(self.layers):
            if i == 0:
                K.embed_norm_gemv(tok, self.embed, res, layer["ln1"], layer["qkv"], c.rms_eps, out=bufs.qkv)
            else:
                K.add_rms_norm_parts(bufs.down_parts, res, layer["ln1"], c.rms_eps, out=bufs.xn)
                K.gemv(bufs.xn, layer["qkv"], out=bufs.qkv)
            K.qk_norm_rope_kv(bufs.qkv, layer["qn"], layer["kn"], cos, sin, k_cache[i], v_cache[i], len_b,
                              c.num_heads, c.num_kv_heads, c.rms_eps, nq)
            o = K.attn_verify(bufs.qkv, k_cache[i], v_cache[i], start_t, len_b, nq, c.num_heads, self.sm_scale,
                              out=bufs.att)
            K.gemv_parts(o, layer["o"], sk=bufs.sk_o, out=bufs.o_parts)
            K.add_rms_norm_parts(bufs.o_parts, res, layer["ln2"], c.rms_eps, out=bufs.xn)
            K.gemv_swiglu(bufs.xn, layer["gu"], out=bufs.act)
            K.gemv_parts(bufs.act, layer["down"], sk=bufs.sk_down, out=bufs.down_parts)
        hidden, _ = K.add_rms_norm_parts(bufs.down_parts, res, self.final_norm, c.rms_eps, out=bufs.hidden)
        am = K.lm_head_argmax(hidden, self.lm_head, bufs.argmax, out_tok=bufs.next_tok)
        return am.view(b, nq)

    def argmax_token(self, hidden, logits=None):
        """ek_model.py:490-493: first index of the max bf16 logit, [B] int64."""
        b = hidden.shape[0]
        if not self.use_gemv_for(b):
            return torch.cat([self.argmax_token(hidden[i:i + self.MAX_ROWS].contiguous())
                              for i in range(0, b, self.MAX_ROWS)])
        bufs = self.buffers(b)
        out = torch.empty(b, dtype=torch.int64, device=hidden.device)
        return K.lm_head_argmax(hidden.contiguous(), self.lm_head, bufs.argmax, out_tok=out, logits=logits)

    def persistent_plan(self, b: int, s_cap: int):
        """decode_step_plan for this model at batch b and score capacity s_cap
        (None when the persistent step does not handle the shape)."""
        key = (b, s_cap)
        if key not in self._plans:
            c = self.cfg
            self._plans[key] = K.decode_step_plan(c.hidden_size, c.intermediate_size, c.num_heads,
                                                  c.num_kv_heads, c.head_dim, c.vocab_size, b, s_cap,
                                                  c.num_layers)
        return self._plans[key]

    def _layer_table(self, k_cache, v_cache):
        key = tuple(t.data_ptr() for t in k_cache) + tuple(t.data_ptr() for t in v_cache)
        tab = self._tables.get(key)
        if tab is None:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("decode_step: build the layer table (run one step) before capturing")
            tab = self._tables[key] = K.layer_table(self.layers, k_cache, v_cache, self.device)
        return tab

    def check_step_error(self) -> None:
        """Raise if a persistent step abandoned a hand-over wait."""
        for bufs in self._bufs.values():
            for scratch in bufs.steps.values():
                scratch.check()

    def step(self, tokens, positions, k_cache, v_cache, slot_t, len_t, start_t, ws, out_buf, step_idx,
             logits=None):
        """The whole graph step of engine.py:284-292: decode, final add + norm
        + lm_head + argmax, then tokens <- next, positions += 1, out_buf[step_idx]
        <- next, step_idx += 1. At batch 1 (and rows whose attention scores fit
        in LDS) it is one persistent launch (K.decode_step); otherwise HIP
        launches per layer with the last three fused into one kernel.
        logits: optional bf16 [B, vocab] that receives the step's logits.
        The device-side waits report a failure in the workspace's error word
        (K.ws_error(ws)); the persistent step then emits token -1."""
        b = tokens.shape[0]
        s_cap = k_cache[0].shape[2]
        if ws is not None and len(ws) >= 8:
            s_cap = min(s_cap, ws[7].shape[2])
        plan = self.persistent_plan(b, s_cap) if self.persistent and b <= self.persistent_rows else None
        if plan is not None:
            bufs = self.buffers(b)
            scratch = bufs.steps.get(plan[0])
            if scratch is None:
                if torch.cuda.is_current_stream_capturing():
                    raise RuntimeError("decode_step: run one step of this bucket before capturing it")
                scratch = bufs.steps[plan[0]] = K.StepScratch(plan, self.device)
            bufs.step = scratch
            K.decode_step(self._layer_table(k_cache, v_cache), self.cfg, self.embed, self.lm_head, self.final_norm,
                          self.cos, self.sin, k_cache[0], s_cap, tokens, positions, len_t, slot_t, start_t,
                          out_buf, step_idx, bufs.step, out_tok=bufs.next_tok, logits=logits,
                          err=K.ws_error(ws))
            return bufs.next_tok
        bufs = self._layers(tokens, positions, k_cache, v_cache, slot_t, len_t, start_t, ws)
        state = (tokens, positions, out_buf, step_idx)
        if b >= 2:
            K.add_rms_norm_parts(bufs.down_parts, bufs.res[0], self.final_norm, self.cfg.rms_eps, out=bufs.hidden)
            return K.lm_head_argmax(bufs.hidden, self.lm_head, bufs.argmax, out_tok=bufs.next_tok, logits=logits,
                                    state=state)
        return K.lm_head_argmax(None, self.lm_head, bufs.argmax, out_tok=bufs.next_tok, logits=logits,
                                parts=bufs.down_parts, residual=bufs.res[0], norm_w=self.final_norm,
                                eps=self.cfg.rms_eps, state=state)
