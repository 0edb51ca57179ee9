"""The C-ABI library on the CPU: it loads, exports every symbol
include/ek_hip.h declares, reports argument errors without touching a GPU,
and the product path refuses CPU tensors (there is no CPU fallback)."""

import ctypes
import os

import pytest
import torch

from enginekernel_amd import _hip
from enginekernel_amd import ek_kernels as K


def test_library_exports_every_declared_symbol():
    lib = _hip.load()
    declared = _hip.declared_symbols()
    assert len(declared) == 24
    for name in declared:
        assert hasattr(lib, name), name
    # the ctypes signature table covers every kernel entry point
    assert set(_hip.SIGNATURES) == set(declared) - {"ek_version", "ek_last_error", "ek_device_info",
                                                     "ek_set_wait_limit"}
    assert lib.ek_version().startswith(b"enginekernel_amd")


def test_wait_limit_setting_round_trips():
    """ek_set_wait_limit returns the previous bound; <= 0 restores the defaults."""
    prev = _hip.set_wait_limit(123)
    try:
        assert _hip.set_wait_limit(7) == 123
        assert _hip.set_wait_limit(0) == 7
        assert _hip.set_wait_limit(-5) == 0
    finally:
        _hip.set_wait_limit(prev)


def test_signature_arity_matches_header():
    """Argument counts in the ctypes table equal the header prototypes."""
    import re
    text = open(_hip.HEADER).read()
    for name, argtypes in _hip.SIGNATURES.items():
        proto = re.search(name + r"\s*\(([^)]*)\)", text, flags=re.S).group(1)
        assert len([a for a in proto.split(",") if a.strip()]) == len(argtypes), name


def test_argument_errors_return_invalid_value_without_a_gpu():
    lib = _hip.load()
    # m = 0 is rejected by the host-side check before any HIP call
    rc = lib.ek_gemv(None, None, None, 0, 16, 64, 64, 64, 16, 0, 0, None)
    assert rc == 1
    assert b"empty" in lib.ek_last_error()
    zeros = [None if t is ctypes.c_void_p else 0.0 if t is ctypes.c_float else 0
             for t in _hip.SIGNATURES["ek_attn_decode"]]
    rc = lib.ek_attn_decode(*zeros)                                   # batch 0
    assert rc == 1 and b"head counts" in lib.ek_last_error()
    with pytest.raises(_hip.HipKernelError) as e:
        _hip.call("ek_silu_mul", None, None, 1, 7, 8, 8, None)      # n not a multiple of 8
    assert e.value.code == 1


def test_decode_step_plan_rejects_unsupported_shapes_without_a_gpu():
    lib = _hip.load()
    sizes = (ctypes.c_int64 * 4)()
    # 4B shape at batch 9: the persistent step takes 1 to 8 rows
    rc = lib.ek_decode_step_plan(2560, 9728, 32, 8, 128, 151936, 9, 768, 36, sizes)
    assert rc == 1 and b"batch" in lib.ek_last_error()
    # 32, 8 and 1 query heads per kv head: the persistent step takes groups of 2 and 4
    for n_q, n_kv in ((32, 1), (64, 8), (8, 8)):
        rc = lib.ek_decode_step_plan(2560, 9728, n_q, n_kv, 128, 151936, 1, 768, 36, sizes)
        assert rc == 1 and b"query heads" in lib.ek_last_error(), (n_q, n_kv)
    # 65 layers: the layer table held in LDS has 64 rows
    rc = lib.ek_decode_step_plan(2560, 9728, 32, 8, 128, 151936, 1, 768, 65, sizes)
    assert rc == 1 and b"64 layers" in lib.ek_last_error()
    zeros = [None if t is ctypes.c_void_p else 0.0 if t is ctypes.c_float else 0
             for t in _hip.SIGNATURES["ek_decode_step"]]
    assert lib.ek_decode_step(*zeros) == 1


def test_kernels_refuse_cpu_tensors():
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    w = torch.ones(64, dtype=torch.bfloat16)
    with pytest.raises(K.HipUnavailable):
        K.rms_norm(x, w, 1e-6)
    with pytest.raises(K.HipUnavailable):
        K.gemv(x, torch.zeros(8, 64, dtype=torch.bfloat16))


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_hip.HipUnavailable):
        _hip.load(str(tmp_path / "nope.so"))


def test_model_refuses_cpu_device():
    from enginekernel_amd.checkpoint import QWEN3_TINY
    from enginekernel_amd.ek_model import Qwen3
    with pytest.raises(K.HipUnavailable):
        Qwen3(None, torch.device("cpu"), tensors={}, config=dict(QWEN3_TINY))


@pytest.mark.parametrize("b,bucket", [(1, 768), (1, 32768), (4, 2048), (8, 8192), (16, 1024), (3, 256)])
def test_plan_splits_invariants(b, bucket):
    splits, chunk, block_n = K.plan_splits(b, 8, bucket)
    assert 1 <= splits <= 32 and chunk % block_n == 0
    assert splits * chunk >= bucket                      # every key of the bucket is covered
    assert (splits - 1) * chunk < bucket                 # no split starts past the bucket
    ws = K.make_workspace(b, 32, 8, 128, bucket, "cpu")
    assert ws[0].shape == (b, 8, K._next_pow2(splits), K.group_pad(32, 8), 128)
    assert ws[7].shape == (b, 32, bucket) and len(ws) == 11
    # the ticket block, the error word, and room for every split's partial as 64-bit words
    assert ws[8].shape == (b, 8, 2) and ws[8].dtype == torch.int32 and int(ws[8].abs().sum()) == 0
    assert K.ws_error(ws) is ws[9] and ws[9].shape == (1,) and int(ws[9]) == 0
    assert K.ws_error(ws[:7]) is None
    assert ws[0].numel() // 2 >= b * 8 * splits * (32 // 8) * 128
    # the exchange words of the one-launch split form: (max, sum) and a
    # partial output per split and query head
    assert ws[10].dtype == torch.int64 and ws[10].numel() >= b * 8 * splits * (32 // 8) * (128 + 2)


def test_group_pad_and_helpers():
    assert K.group_pad(32, 8) == 16 and K.group_pad(64, 2) == 32
    assert K._next_pow2(1) == 1 and K._next_pow2(17) == 32 and K._cdiv(7, 2) == 4
