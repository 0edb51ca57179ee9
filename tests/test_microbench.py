"""Host-side checks of the per-kernel measurements (bench.py --config 2/3/5):
the byte counts and floors they report, the cache-defeating copy counts and
config 5's prompt generator. No GPU needed."""

from enginekernel_amd import checkpoint as C
from enginekernel_amd import microbench as M


def test_gemv_floors_match_the_weight_stream():
    # the 8 TB/s floors of the five decode projections (weights only)
    floors = [round(M.gemv_floor_us(n, k), 2) for _, n, k, _, _ in M.GEMV_SHAPES]
    assert floors == [3.93, 12.45, 2.62, 6.23, 97.24]
    # all five per-layer projections plus lm_head are the weight bytes of a token
    per_layer = sum(2 * n * k for name, n, k, _, _ in M.GEMV_SHAPES if name != "lm_head")
    cfg = C.QWEN3_4B
    assert per_layer * cfg["num_hidden_layers"] + 2 * 151936 * 2560 == C.weight_bytes_per_token(cfg)


def test_gemv_bytes_count_each_operand_once():
    assert M.gemv_bytes("gemv", 6144, 2560, 1) == 2 * 6144 * 2560 + 2 * 2560 + 2 * 6144
    assert M.gemv_bytes("swiglu", 19456, 2560, 4) == 2 * 19456 * 2560 + 4 * 2 * 2560 + 4 * 2 * 9728
    assert M.gemv_bytes("parts", 2560, 9728, 4, sk=2) == 2 * 2560 * 9728 + 4 * 2 * 9728 + 2 * 4 * 4 * 2560


def test_every_timed_round_overflows_the_infinity_cache():
    for _, n, k, _, copies in M.GEMV_SHAPES:
        assert 2 * n * k * copies >= 512e6
    for length in M.ATTN_LENGTHS:
        per = M.attn_bytes(length)
        copies = max(4, -(-M.CACHE_DEFEAT // per))
        assert per * copies >= M.CACHE_DEFEAT


def test_attention_bytes_are_the_kv_rows():
    # 4096 bytes of K+V per key at 8 kv heads x 128 dims, plus q and out
    assert M.attn_bytes(32768) - M.attn_bytes(0) == 4096 * 32768
    assert [round(M.attn_bytes(l) / 8e12 * 1e6, 2) for l in M.ATTN_LENGTHS] == [0.26, 2.1, 8.39, 16.78]


def test_batch8_prompts_are_ragged_and_reproducible():
    a = M.batch8_prompts(151936)
    assert a == M.batch8_prompts(151936)
    assert len(a) == 8 and all(64 <= len(p) <= 2048 for p in a)
    assert len({len(p) for p in a}) > 1
    assert all(0 <= t < 151936 for p in a for t in p)


def test_batch8_bytes_add_the_attended_kv():
    kv_row = 2 * 36 * 8 * 128 * 2
    assert kv_row == 147456
    assert M.batch8_bytes(8_044_544_000, kv_row, 1000) == 8_044_544_000 + 147_456_000
