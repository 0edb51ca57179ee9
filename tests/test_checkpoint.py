"""Random-init checkpoints and the load/fuse path (host logic, CPU)."""

import json

import torch

from enginekernel_amd import checkpoint as C
from enginekernel_amd.ek_model import Qwen3Config, fuse_layer, load_tensors, rope_tables, shard_map
from oracle import ek_oracle as O


def test_weight_bytes_match_the_published_per_token_figure():
    # README.md:14-15 / BASELINE: 36 x 201,850,880 + 777,912,320
    assert C.weight_bytes_per_token(C.QWEN3_4B) == 8_044_544_000


def test_random_weights_independent_of_thread_count():
    cfg = dict(C.QWEN3_TINY, vocab_size=4096 * 1025 // 128)     # > one 4M-element chunk in the embedding
    a = C.random_weights(cfg, seed=7, threads=1)
    b = C.random_weights(cfg, seed=7, threads=8)
    assert a.keys() == b.keys()
    for k in a:
        assert torch.equal(a[k], b[k]), k
    c = C.random_weights(cfg, seed=8, threads=4)
    assert not torch.equal(a["model.embed_tokens.weight"], c["model.embed_tokens.weight"])
    e = a["model.embed_tokens.weight"].float()
    assert abs(e.std().item() - 0.02) < 1e-3 and abs(e.mean().item()) < 1e-3
    assert torch.equal(a["model.norm.weight"], torch.ones_like(a["model.norm.weight"]))
    assert a["lm_head.weight"] is a["model.embed_tokens.weight"]


def test_checkpoint_roundtrip_and_config_styles(tmp_path):
    cfg = dict(C.QWEN3_TINY)
    t = C.random_weights(cfg, seed=0)
    C.write_checkpoint(str(tmp_path), cfg, t)
    d = json.load(open(tmp_path / "config.json"))
    assert d["rope_theta"] == d["rope_parameters"]["rope_theta"] == 1e6
    c = Qwen3Config(str(tmp_path))
    assert (c.hidden_size, c.num_layers, c.num_heads, c.num_kv_heads, c.head_dim, c.vocab_size) == \
        (128, 2, 4, 2, 32, 1024)
    del d["rope_theta"]                       # a transformers-5 style config.json
    json.dump(d, open(tmp_path / "config.json", "w"))
    assert Qwen3Config(str(tmp_path)).rope_theta == 1e6
    assert set(shard_map(str(tmp_path)).values()) == {"model.safetensors"}
    loaded = load_tensors(str(tmp_path))
    for k, v in loaded.items():
        assert torch.equal(v, t[k]), k


def test_fused_layer_is_byte_identical_to_separate_tensors():
    cfg = dict(C.QWEN3_TINY)
    t = C.random_weights(cfg, seed=0)
    lay = fuse_layer(t, 1)
    p = "model.layers.1."
    q, k, v = (t[p + f"self_attn.{n}_proj.weight"] for n in "qkv")
    assert torch.equal(lay["qkv"], torch.cat([q, k, v]))
    assert torch.equal(lay["qkv"][: q.shape[0]], q) and torch.equal(lay["qkv"][-v.shape[0]:], v)
    assert torch.equal(lay["gu"][:384], t[p + "mlp.gate_proj.weight"])
    assert torch.equal(lay["gu"][384:], t[p + "mlp.up_proj.weight"])
    assert lay["qkv"].is_contiguous() and lay["gu"].is_contiguous()


def test_rope_tables_equal_the_oracle():
    for d, th in ((32, 1e6), (128, 5e6)):
        a = rope_tables(d, th, 2048)
        b = O.build_rope(d, th, 2048)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_shard_map_reads_headers_of_unindexed_shards(tmp_path):
    from safetensors.torch import save_file

    save_file({"a": torch.zeros(2), "b": torch.ones(3)}, str(tmp_path / "x-1.safetensors"), metadata={"k": "v"})
    save_file({"c": torch.zeros(1)}, str(tmp_path / "x-2.safetensors"))
    assert shard_map(str(tmp_path)) == {"a": "x-1.safetensors", "b": "x-1.safetensors", "c": "x-2.safetensors"}
    save_file({"c": torch.zeros(1)}, str(tmp_path / "x-3.safetensors"))
    try:
        shard_map(str(tmp_path))
    except ValueError as e:
        assert "x-2" in str(e) and "x-3" in str(e)
    else:
        raise AssertionError("a tensor in two shards must be refused")
    json.dump({"weight_map": {"c": "x-3.safetensors"}}, open(tmp_path / "model.safetensors.index.json", "w"))
    assert shard_map(str(tmp_path)) == {"c": "x-3.safetensors"}
