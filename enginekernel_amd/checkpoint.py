"""Seeded random-init Qwen3 checkpoints, in memory or as HF safetensors.

The benchmark and parity configurations are random-init (there is no network
for the real checkpoint), so the weights have to be reproducible bit for bit
wherever they are built: the HIP path and the CPU oracle must see identical
bf16 bytes. Every tensor is generated on the CPU by torch's CPU generator,
in fixed-size chunks whose seeds are a hash of (seed, tensor name, chunk
index). The bytes therefore depend only on the seed and the configuration,
never on the thread count, and chunks can be drawn on all host cores at once
(one stream of 4e9 normals takes ~90 s; the chunked draw is ~8x faster).

Tensor names and the config.json layout follow the HF Qwen3 checkpoint that
the reference loads (`engine/ek_model.py:26-42, 117-162`).
"""

from __future__ import annotations

import concurrent.futures as _cf
import hashlib
import json
import os

import torch

# The two model shapes of the benchmark (hidden/layers/heads/... as HF names).
QWEN3_4B = dict(
    architectures=["Qwen3ForCausalLM"], model_type="qwen3",
    hidden_size=2560, num_hidden_layers=36, num_attention_heads=32,
    num_key_value_heads=8, head_dim=128, intermediate_size=9728,
    vocab_size=151936, rms_norm_eps=1e-6, rope_theta=5000000.0,
    tie_word_embeddings=True, max_position_embeddings=40960,
    hidden_act="silu", torch_dtype="bfloat16",
)

QWEN3_TINY = dict(
    architectures=["Qwen3ForCausalLM"], model_type="qwen3",
    hidden_size=128, num_hidden_layers=2, num_attention_heads=4,
    num_key_value_heads=2, head_dim=32, intermediate_size=384,
    vocab_size=1024, rms_norm_eps=1e-6, rope_theta=1000000.0,
    tie_word_embeddings=True, max_position_embeddings=4096,
    hidden_act="silu", torch_dtype="bfloat16",
)

_CHUNK = 1 << 22   # elements per independently seeded chunk


def tensor_specs(cfg: dict):
    """[(hf_name, shape, kind)] for a Qwen3 config; kind is 'normal' or 'ones'."""
    h = cfg["hidden_size"]
    d = cfg.get("head_dim", h // cfg["num_attention_heads"])
    nq, nkv = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    inter, vocab = cfg["intermediate_size"], cfg["vocab_size"]
    out = [("model.embed_tokens.weight", (vocab, h), "normal")]
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        out += [
            (p + "self_attn.q_proj.weight", (nq * d, h), "normal"),
            (p + "self_attn.k_proj.weight", (nkv * d, h), "normal"),
            (p + "self_attn.v_proj.weight", (nkv * d, h), "normal"),
            (p + "self_attn.o_proj.weight", (h, nq * d), "normal"),
            (p + "self_attn.q_norm.weight", (d,), "ones"),
            (p + "self_attn.k_norm.weight", (d,), "ones"),
            (p + "mlp.gate_proj.weight", (inter, h), "normal"),
            (p + "mlp.up_proj.weight", (inter, h), "normal"),
            (p + "mlp.down_proj.weight", (h, inter), "normal"),
            (p + "input_layernorm.weight", (h,), "ones"),
            (p + "post_attention_layernorm.weight", (h,), "ones"),
        ]
    out.append(("model.norm.weight", (h,), "ones"))
    if not cfg.get("tie_word_embeddings", False):
        out.append(("lm_head.weight", (vocab, h), "normal"))
    return out


def _chunk_seed(seed: int, name: str, idx: int) -> int:
    dig = hashlib.sha256(f"{seed}/{name}/{idx}".encode()).digest()
    return int.from_bytes(dig[:8], "little") & ((1 << 63) - 1)


def _fill(dst: torch.Tensor, seed: int, name: str, idx: int, std: float) -> None:
    g = torch.Generator().manual_seed(_chunk_seed(seed, name, idx))
    v = torch.randn(dst.numel(), generator=g, dtype=torch.float32)
    dst.copy_(v.mul_(std))


def random_weights(cfg: dict, seed: int = 0, std: float = 0.02,
                   norm_init: str = "ones", threads: int | None = None) -> dict:
    """HF-named bf16 CPU tensors: linear/embedding ~N(0, std), norm gains 1.0.

    Norm gains are HF's init (1.0). norm_init="normal" draws them ~N(0, std)
    instead, which shrinks every activation and makes near-ties far more
    frequent; it exists only to show that effect.
    """
    specs = tensor_specs(cfg)
    out = {}
    jobs = []
    for name, shape, kind in specs:
        t = torch.empty(shape, dtype=torch.bfloat16)
        out[name] = t
        if kind == "ones" and norm_init == "ones":
            t.fill_(1.0)
            continue
        flat = t.view(-1)
        for idx, lo in enumerate(range(0, flat.numel(), _CHUNK)):
            jobs.append((flat[lo:lo + _CHUNK], name, idx))
    threads = threads or max(1, min(32, len(os.sched_getaffinity(0))))
    if len(jobs) <= 2 or threads == 1:
        for dst, name, idx in jobs:
            _fill(dst, seed, name, idx, std)
    else:
        prev = torch.get_num_threads()
        torch.set_num_threads(1)     # one chunk per pool thread
        # inference mode is per thread: the pool's threads take the caller's,
        # or they could not write tensors the caller made under it
        inference = torch.is_inference_mode_enabled()

        def fill(j):
            with torch.inference_mode(inference):
                _fill(j[0], seed, j[1], j[2], std)

        try:
            with _cf.ThreadPoolExecutor(threads) as ex:
                list(ex.map(fill, jobs))
        finally:
            torch.set_num_threads(prev)
    if cfg.get("tie_word_embeddings", False):
        out["lm_head.weight"] = out["model.embed_tokens.weight"]
    return out


def config_json(cfg: dict) -> dict:
    """config.json contents. rope_theta is written top-level (the reference's
    loader reads only that key, `ek_model.py:38`) and also in the
    transformers-5 `rope_parameters` block."""
    d = dict(cfg)
    d["rope_parameters"] = {"rope_type": "default", "rope_theta": float(cfg["rope_theta"])}
    return d


def write_checkpoint(path: str, cfg: dict, tensors: dict | None = None, seed: int = 0) -> str:
    """Write config.json + model.safetensors (HF names) under path."""
    from safetensors.torch import save_file

    os.makedirs(path, exist_ok=True)
    tensors = tensors if tensors is not None else random_weights(cfg, seed)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(config_json(cfg), f, indent=1)
    flat = {k: v.contiguous() for k, v in tensors.items()
            if not (k == "lm_head.weight" and cfg.get("tie_word_embeddings", False))}
    save_file(flat, os.path.join(path, "model.safetensors"))
    return path


def weight_bytes_per_token(cfg: dict) -> int:
    """Projection weight bytes one decode step streams (norm gains excluded):
    per layer qkv + o + gate_up + down, plus the lm_head."""
    h, i = cfg["hidden_size"], cfg["intermediate_size"]
    d = cfg.get("head_dim", h // cfg["num_attention_heads"])
    nq, nkv = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    per_layer = (nq + 2 * nkv) * d * h + h * nq * d + 2 * i * h + h * i
    return 2 * (cfg["num_hidden_layers"] * per_layer + cfg["vocab_size"] * h)
