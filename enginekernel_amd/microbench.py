"""Per-kernel measurements of the decode path on one MI355X, beside the
batch-1 end-to-end figure of bench.py:

  config 2  the decode projections one launch at a time: each weight shape
            of the Qwen3-4B decode at batch 1 and 4, through the entry point
            the per-kernel decode uses for it (gemv, gemv_swiglu, gemv_parts),
            over enough distinct weight copies that every timed round reads
            at least 512 MB (the 256 MB Infinity Cache holds nothing of it).
  config 3  decode attention over one layer's cache: q [1, 32, 128], K/V
            bf16 ~N(0, 1) of capacity 32768 filled to L in {512, 4096,
            16384, 32768}, swept over the split count, again over copies
            that defeat the Infinity Cache.
  config 5  batch 8, left-padded prompts of U[64, 2048] random ids (seed 2),
            256 greedy tokens through the engine's captured graph (at 8
            rows the per-kernel graph, the faster form there), cache
            capacity 8192; also the prompt's prefill time (the first token).
  config 7  the step at 2, 4, 6 and 8 rows (the first rows of config 5's
            batch), one graph replay per step, in both forms: the one-launch
            batch kernel and the per-kernel graph.

Every figure is HIP-event time on the launching stream divided by the
launches inside the timed region; bytes are algorithmic (each weight, key,
value, activation and output byte once)."""

from __future__ import annotations

import math
import os
import time

PEAK_HBM = 8.0e12
CACHE_DEFEAT = 512 << 20   # bytes each timed round touches (> the 256 MB Infinity Cache)

# (name, N, K, kind, copies): kind "gemv" = bf16 out, "swiglu" = the fused
# gate/up with SiLU*up epilogue (N counts gate+up rows), "parts" = fp32 split-K
# partials. Copies as in the reference's sweep (gemv_sweep.py:94 analogue).
GEMV_SHAPES = (
    ("qkv", 6144, 2560, "gemv", 17),
    ("gate_up", 19456, 2560, "swiglu", 6),
    ("o", 2560, 4096, "parts", 25),
    ("down", 2560, 9728, "parts", 11),
    ("lm_head", 151936, 2560, "gemv", 1),
)
ATTN_LENGTHS = (512, 4096, 16384, 32768)
ATTN_SPLITS = (1, 2, 4, 8, 16, 32, 64, 128, 256)


def gemv_bytes(kind: str, n: int, k: int, b: int, sk: int = 1) -> int:
    """Algorithmic bytes of one launch: W once (2NK), x (2BK) and the output
    (bf16 [B, N], bf16 [B, N/2] after SwiGLU, or fp32 [sk, B, N] partials)."""
    out = {"gemv": 2 * b * n, "swiglu": 2 * b * (n // 2), "parts": 4 * sk * b * n}[kind]
    return 2 * n * k + 2 * b * k + out


def gemv_floor_us(n: int, k: int) -> float:
    """The weight stream alone at the 8 TB/s spec peak."""
    return 2 * n * k / PEAK_HBM * 1e6


def attn_bytes(length: int, n_q: int = 32, n_kv: int = 8, d: int = 128) -> int:
    """K and V rows of the attended keys plus q in and the output out."""
    return 2 * n_kv * d * 2 * length + 2 * (2 * n_q * d)


def _timed(fn, reps: int) -> float:
    """Seconds per call of fn: fn (a round of launches) is captured once as
    a HIP graph, so host launch overhead stays out of the figure, and the
    graph is replayed `reps` times between HIP events on the replay stream."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / 1e3 / reps


def gemv_sweep(batches=(1, 4), rounds: int = 10, log=print):
    """Config 2. Returns one record per (shape, batch)."""
    import torch
    from enginekernel_amd import ek_kernels as K

    dev = torch.device("cuda:0")
    out = []
    for name, n, k, kind, copies in GEMV_SHAPES:
        g = torch.Generator(device=dev).manual_seed(0)
        ws = [torch.empty(n, k, dtype=torch.bfloat16, device=dev).normal_(0, 0.02, generator=g)
              for _ in range(copies)]
        for b in batches:
            x = torch.empty(b, k, dtype=torch.bfloat16, device=dev).normal_(0, 0.02, generator=g)
            sk = K.parts_splits(b, k) if kind == "parts" else 1
            if kind == "gemv":
                y = torch.empty(b, n, dtype=torch.bfloat16, device=dev)
                call = lambda w: K.gemv(x, w, out=y)
            elif kind == "swiglu":
                call = lambda w: K.gemv_swiglu(x, w)
            else:
                p = torch.empty(sk, b, n, dtype=torch.float32, device=dev)
                call = lambda w: K.gemv_parts(x, w, sk=sk, out=p)

            def one_round():
                for w in ws:
                    call(w)

            t = _timed(one_round, rounds) / copies
            nbytes = gemv_bytes(kind, n, k, b, sk)
            rec = {"proj": name, "w": [n, k], "batch": b, "entry": {"gemv": "ek_gemv", "swiglu": "ek_gemv_swiglu",
                                                                    "parts": "ek_gemv_parts"}[kind],
                   "splits": sk, "copies": copies, "us": round(t * 1e6, 2),
                   "floor_us": round(gemv_floor_us(n, k), 2), "bytes": nbytes,
                   "GBps": round(nbytes / t / 1e9, 1), "frac": round(nbytes / t / PEAK_HBM, 4)}
            log(f"gemv {name:8s} B={b} {rec['us']:8.2f} us  {rec['GBps']:7.1f} GB/s  ({rec['frac']:.1%})")
            out.append(rec)
        del ws
        torch.cuda.empty_cache()
    return out


def attn_sweep(lengths=ATTN_LENGTHS, splits=ATTN_SPLITS, reps: int = 20, cap: int = 32768, log=print):
    """Config 3. One record per (L, splits). The caches have the config's
    capacity (head stride cap x 128): each copy is a [1, 8, L, 128] view of a
    [1, 8, cap, 128] pool, cap // L copies per pool, enough copies that a
    timed round reads at least 512 MB. splits = 1 at L <= 2048 takes the
    single-launch kernel, every other point the split pair."""
    import torch
    from enginekernel_amd import ek_kernels as K

    dev = torch.device("cuda:0")
    n_q, n_kv, d = 32, 8, 128
    scale = d ** -0.5
    out = []
    for length in lengths:
        per = attn_bytes(length)
        copies = max(4, math.ceil(CACHE_DEFEAT / per))
        per_pool = cap // length
        pools = math.ceil(copies / per_pool)
        g = torch.Generator(device=dev).manual_seed(0)
        kp = [torch.empty(1, n_kv, cap, d, dtype=torch.bfloat16, device=dev).normal_(generator=g) for _ in range(pools)]
        vp = [torch.empty(1, n_kv, cap, d, dtype=torch.bfloat16, device=dev).normal_(generator=g) for _ in range(pools)]
        caches = [(kp[c // per_pool][:, :, (c % per_pool) * length:(c % per_pool + 1) * length],
                   vp[c // per_pool][:, :, (c % per_pool) * length:(c % per_pool + 1) * length])
                  for c in range(copies)]
        q = torch.empty(1, n_q, d, dtype=torch.bfloat16, device=dev).normal_(generator=g)
        seq = torch.full((1,), length, dtype=torch.int64, device=dev)
        start = torch.zeros(1, dtype=torch.int32, device=dev)
        for sp in splits:
            if sp > length // 16:
                continue
            chunk = K._cdiv(length, sp)
            ws = K.make_workspace(1, n_q, n_kv, d, length, dev, splits=sp, chunk=chunk)
            fused = sp == 1 and 4 * length * 4 <= 32 * 1024

            def one_round():
                for kc, vc in caches:
                    K.flash_decode(q, kc, vc, seq, start, ws, scale)

            t = _timed(one_round, reps) / copies
            rec = {"L": length, "splits": sp, "path": "fused" if fused else "scores+pv",
                   "copies": copies, "us": round(t * 1e6, 2), "floor_us": round(per / PEAK_HBM * 1e6, 2),
                   "bytes": per, "GBps": round(per / t / 1e9, 1), "frac": round(per / t / PEAK_HBM, 4)}
            log(f"attn L={length:6d} splits={sp:4d} {rec['path']:10s} {rec['us']:8.2f} us  {rec['GBps']:7.1f} GB/s")
            out.append(rec)
        del caches, kp, vp
        torch.cuda.empty_cache()
    return out


def batch8_prompts(vocab: int, b: int = 8, seed: int = 2, lo: int = 64, hi: int = 2048):
    """Config 5's prompts: lengths U[lo, hi], ids U[0, vocab), one generator."""
    import torch
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (b,), generator=g).tolist()
    return [torch.randint(0, vocab, (n,), generator=g).tolist() for n in lens]


def batch8_bytes(w_bytes: int, kv_row: int, attended: int) -> int:
    """Algorithmic bytes of one batch step: every weight once, plus the K/V
    rows of every attended key of every row (kv_row bytes per key)."""
    return w_bytes + kv_row * attended


# HBM bytes per step of the batch kernel at config 5 (batch_step_kernel<128, 4, 8>), from two
# rocprofv3 PMC runs of `bench.py --config 5 --no-cpu` (FETCH_SIZE 4,529,238 KiB scaled by
# the 256 MiB device-copy calibration 0.500066, plus WRITE_SIZE 76,384 KiB), measured with the
# kernel sources of the commit named; re-measure when they change
BATCH8_TRAFFIC = 9_352_871_508
BATCH8_TRAFFIC_AT = "081d385"


def batch8_decode(tokens: int = 256, cap: int = 8192, log=print):
    """Config 5 on the Qwen3-4B architecture. Returns one record."""
    import torch
    from enginekernel_amd import checkpoint as C
    from enginekernel_amd.ek_model import Qwen3
    from enginekernel_amd.engine import _FastEngine

    dev = torch.device("cuda:0")
    cfg = dict(C.QWEN3_4B)
    t0 = time.perf_counter()
    model = Qwen3(None, dev, tensors=C.random_weights(cfg, seed=0), config=cfg)
    torch.cuda.synchronize()
    log(f"config 5: weights ready in {time.perf_counter() - t0:.1f}s")
    eng = _FastEngine(model=model)
    prompts = batch8_prompts(cfg["vocab_size"])
    b = len(prompts)
    steps = tokens - 1
    with torch.inference_mode():
        ids, pos, pad, s, bias = eng._pack(prompts)
        eng._ensure_cache(b, cap)
        graph = eng._get_graph(b, s + tokens)
        eng._first_token(ids, pos, b, s, bias)          # warm-up (library load, hipBLASLt plans)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        p0.record(stream)
        first = eng._first_token(ids, pos, b, s, bias)
        p1.record(stream)
        p1.synchronize()
        prefill_s = p0.elapsed_time(p1) / 1e3
        graph.begin(first, [s - p for p in pad], pad, s)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            graph.graph.replay()
        e1.record(stream)
        e1.synchronize()
        step_s = e0.elapsed_time(e1) / 1e3 / steps
        from enginekernel_amd import ek_kernels as K
        K.check_error_word(graph.err, "the timed batch-8 steps")
        if int(graph.step_idx.min()) != steps:
            raise RuntimeError("graph step counter out of step with the replays")
    w_bytes = C.weight_bytes_per_token(cfg)
    kv_row = 2 * cfg["num_hidden_layers"] * cfg["num_key_value_heads"] * cfg["head_dim"] * 2
    # step j (1-based) attends keys [pad_b, s + j) of row b
    attended = sum(sum(s + j - p for p in pad) for j in range(1, steps + 1)) / steps
    nbytes = batch8_bytes(w_bytes, kv_row, attended)
    rec = {"batch": b, "prompt_lens": [len(p) for p in prompts], "padded_len": s, "cache_cap": eng.cache_s,
           "graph_bucket": graph.bucket, "tokens": tokens, "timed_replays": steps,
           "ms_per_step": round(step_s * 1e3, 4), "tokens_per_s": round(b / step_s, 1),
           "bytes_per_step": int(nbytes), "weight_frac": round(w_bytes / step_s / PEAK_HBM, 4),
           "weight_kv_frac": round(nbytes / step_s / PEAK_HBM, 4),
           "prefill_ms": round(prefill_s * 1e3, 2), "prefill_tokens": b * s,
           "prefill_tokens_per_s": round(b * s / prefill_s, 0),
           # one kernel per replay: its launch time is the replay time
           "roofline": {"bound": "hbm", "kernel": "eks::batch_step_kernel<128,4,8> (the whole decode step, one launch)",
                        "achieved": round(nbytes / step_s / 1e9, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                        "frac": round(nbytes / step_s / PEAK_HBM, 4),
                        "traffic": BATCH8_TRAFFIC if (cap == 8192 and tokens == 256) else None,
                        "traffic_measured_at": BATCH8_TRAFFIC_AT if (cap == 8192 and tokens == 256) else None,
                        "bytes_per_launch": int(nbytes), "avg_launch_us": round(step_s * 1e6, 3),
                        "launches": steps}}
    log(f"config 5: prefill of {b} x {s} (padded) tokens in {prefill_s * 1e3:.2f} ms")
    log(f"config 5: {step_s * 1e3:.4f} ms/step, {rec['tokens_per_s']} tok/s, "
        f"weights {rec['weight_frac']:.1%} / weights+KV {rec['weight_kv_frac']:.1%} of 8 TB/s")
    return rec


def spec_decode(tokens: int = 256, log=print):
    """Batch-1 greedy decode at the Qwen3-4B shape (random-init weights,
    seed 0) through the engine, plain (one persistent step per token) and
    speculative (ENGINE_SPEC_Q tokens scored per verify step), on a random
    prompt and on a prompt that repeats a 16-token phrase. Time from the
    first token's arrival to the last (prefill excluded). Records where the
    two greedy sequences first differ, if they do (near-ties: the exact
    equality is tested on the tiny model and the verify pass position by
    position against the oracle)."""
    import time

    import torch

    from . import checkpoint as C
    from .ek_model import Qwen3
    from .engine import _FastEngine, _spec_q

    cfg = dict(C.QWEN3_4B)
    dev = torch.device("cuda:0")
    model = Qwen3(None, dev, tensors=C.random_weights(cfg, seed=0), config=cfg)
    eng = _FastEngine(model=model)
    g = torch.Generator().manual_seed(1)
    phrase = torch.randint(0, cfg["vocab_size"], (16,), generator=g).tolist()
    prompts = {"random": torch.randint(0, cfg["vocab_size"], (128,), generator=g).tolist(),
               "repeating": phrase * 8}
    out = []
    for name, prompt in prompts.items():
        rec = {"prompt": name, "prompt_len": len(prompt), "tokens": tokens, "q": _spec_q(1)}
        toks = {}
        for spec in (False, True):
            eng.spec = spec
            list(eng.generate([prompt], 16))          # capture the graphs outside the timing
            it = eng.generate([prompt], tokens)
            first = next(it)
            t0 = time.perf_counter()
            rest = list(it)
            dt = time.perf_counter() - t0
            toks[spec] = [first] + rest
            key = "spec" if spec else "plain"
            rec[key + "_ms_per_token"] = round(dt * 1e3 / (tokens - 1), 4)
            rec[key + "_tokens_per_s"] = round((tokens - 1) / dt, 1)
            if spec:
                steps, target = eng.last_stats
                rec["verify_steps"] = steps
                rec["tokens_per_verify"] = round(target / steps, 3)
                rec["ms_per_verify"] = round(dt * 1e3 / steps, 4)
        # greedy ties: the verify pass (3-row kernels, flash attention) and the
        # one-launch step round differently, and on a random-init model, whose
        # logits are flat, a near-tie flip makes the two sequences part ways
        div = next((i for i, (a, b) in enumerate(zip(toks[True], toks[False])) if a != b), None)
        rec["first_divergence"] = div
        rec["speedup"] = round(rec["plain_ms_per_token"] / rec["spec_ms_per_token"], 3)
        log(f"[bench] spec {name}: plain {rec['plain_ms_per_token']} ms/token, spec {rec['spec_ms_per_token']} "
            f"ms/token ({rec['tokens_per_verify']} tokens per {rec['ms_per_verify']} ms verify), "
            f"first divergence {rec['first_divergence']}")
        out.append(rec)
    eng.spec = False
    return out


def batch_sweep(rows=(2, 4, 6, 8), steps: int = 64, cap: int = 8192, log=print):
    """Config 7: the decode step at 2..8 rows, one captured graph replay per
    step, both forms: the one-launch batch kernel (every row count, whatever
    the default row limit) and the per-kernel graph. The batch is the first
    `b` of config 5's prompts (U[64, 2048] tokens, seed 2), cache 8192;
    bytes per step are the weights plus the K/V rows attended."""
    import torch
    from enginekernel_amd import checkpoint as C
    from enginekernel_amd import ek_kernels as K
    from enginekernel_amd.ek_model import Qwen3
    from enginekernel_amd.engine import _FastEngine

    dev = torch.device("cuda:0")
    cfg = dict(C.QWEN3_4B)
    model = Qwen3(None, dev, tensors=C.random_weights(cfg, seed=0), config=cfg)
    w_bytes = C.weight_bytes_per_token(cfg)
    kv_row = 2 * cfg["num_hidden_layers"] * cfg["num_key_value_heads"] * cfg["head_dim"] * 2
    out = []
    for b in rows:
        prompts = batch8_prompts(cfg["vocab_size"])[:b]
        rec = {"batch": b, "prompt_lens": [len(p) for p in prompts]}
        for persistent in (True, False):
            model.persistent = persistent
            model.persistent_rows = 8
            eng = _FastEngine(model=model)
            with torch.inference_mode():
                ids, pos, pad, s, bias = eng._pack(prompts)
                eng._ensure_cache(b, cap)
                graph = eng._get_graph(b, s + steps + 8)
                first = eng._first_token(ids, pos, b, s, bias)
                graph.begin(first, [s - p for p in pad], pad, s)
                for _ in range(4):
                    graph.graph.replay()
                torch.cuda.synchronize()
                stream = torch.cuda.current_stream()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(steps):
                    graph.graph.replay()
                e1.record(stream)
                e1.synchronize()
                step_s = e0.elapsed_time(e1) / 1e3 / steps
                K.check_error_word(graph.err, "the timed batch steps")
            attended = sum(s + 4 + j - p for p in pad for j in range(1, steps + 1)) / steps
            nbytes = batch8_bytes(w_bytes, kv_row, attended)
            key = "one_launch" if persistent else "per_kernel"
            rec[key + "_ms"] = round(step_s * 1e3, 4)
            rec[key + "_frac"] = round(nbytes / step_s / PEAK_HBM, 4)
            del eng, graph
            torch.cuda.empty_cache()
        log(f"config 7: batch {b}: one launch {rec['one_launch_ms']} ms, per-kernel {rec['per_kernel_ms']} ms")
        out.append(rec)
    model.persistent, model.persistent_rows = True, 8
    return out


def run(config: int, log=print) -> dict:
    """One JSON-ready record for config 2, 3, 5, 6 or 7."""
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("the microbenchmarks need a GPU")
    if config == 2:
        return {"metric": "decode GEMV per-launch time and HBM fraction (config 2)", "unit": "us",
                "higher_is_better": False, "dtype": "bf16", "data": "synthetic ~N(0,0.02), seed 0",
                "config": {"workload": "config 2: Qwen3-4B decode projections, B in {1, 4}"},
                "results": gemv_sweep(log=log)}
    if config == 3:
        return {"metric": "decode attention per-launch time and HBM fraction (config 3)", "unit": "us",
                "higher_is_better": False, "dtype": "bf16", "data": "synthetic q, K, V ~N(0,1), seed 0",
                "config": {"workload": "config 3: one layer, 32/8 heads, D 128, L swept, splits swept"},
                "results": attn_sweep(log=log)}
    if config == 5:
        rec = batch8_decode(log=log)
        return {"metric": "batch-8 decode tokens/s and % of HBM roofline (config 5)",
                "value": rec["tokens_per_s"], "unit": "tokens/s", "steps": rec["timed_replays"],
                "ms_per_step": rec["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                "dtype": "bf16", "data": "synthetic (random-init weights seed 0, prompts seed 2)",
                "config": {"workload": "config 5: Qwen3-4B architecture, batch 8 ragged, the engine's default step "
                                       "(the one-launch batch kernel, eks::batch_step_kernel<128, 4, 8>)"},
                "roofline": rec["roofline"], "results": [rec]}
    if config == 6:
        return {"metric": "batch-1 speculative decode tokens/s vs plain (config 6)", "unit": "tokens/s",
                "higher_is_better": True, "dtype": "bf16",
                "data": "synthetic (random-init weights seed 0; random and repeating prompts, seed 1)",
                "config": {"workload": "config 6: Qwen3-4B architecture, batch 1, n-gram draft + verify"},
                "results": spec_decode(log=log)}
    if config == 7:
        return {"metric": "decode step time at 2..8 rows, one-launch vs per-kernel (config 7)", "unit": "ms",
                "higher_is_better": False, "dtype": "bf16",
                "data": "synthetic (random-init weights seed 0, config 5 prompts seed 2)",
                "config": {"workload": "config 7: Qwen3-4B architecture, the first b of config 5's prompts, "
                                       "cache 8192, one graph replay per step"},
                "results": batch_sweep(log=log)}
    raise ValueError(f"no microbenchmark for config {config}")
