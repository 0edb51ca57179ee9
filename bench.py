"""Batch-1 Qwen3-4B-shape decode on one MI355X: tokens/s, ms/token and the
fraction of the HBM roofline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
    python bench.py --probe-traffic     (the launches the PMC traffic profile counts)
    python bench.py --config 2|3|5|6|7  (GEMV sweep, attention sweep, batch-8 decode,
                                         batch-1 speculative decode vs plain, 2..8-row step)

Workload: a random-init bf16 model of the Qwen3-4B
architecture (36 layers, hidden 2560, intermediate 9728, 32/8 heads, head
dim 128, vocab 151936, tied embeddings, QK-norm, RoPE theta 5e6, weights
~N(0, 0.02), seed 0), batch 1, a prompt of 128 random ids (seed 1),
greedy decode where every token is one replay of the captured HIP graph.
A step is one replay: the whole model streams once (8,044,544,000 weight
bytes). W untimed replays, then exactly K timed replays bracketed by
synchronisation; ms_per_step = time / K.

Also reported, on the same JSON line:
  roofline      the dominant kernel. On the default batch-1 path the whole
                step is ONE persistent kernel (eks::step_kernel), so the
                replay time is its launch time: achieved = the step's
                algorithmic bytes (weights, the KV rows it reads and writes,
                norm gains, the embedding row) / average replay time, HIP
                events on the replay stream. With ENGINE_PERSISTENT=0 (the
                per-kernel graph) it is the fused add + RMSNorm + gate_up +
                SwiGLU launch over all 36 layers' weights instead.
  cpu_baseline  the CPU oracle (the reference's torch fallback restated) decoding
                a bounded sample of the same workload on this host's cores,
                from the GPU's prefill KV cache and the same weights.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM = 8.0e12   # MI355X HBM3E, bytes/s (spec sheet)

# HBM bytes per launch, from two rocprofv3 PMC runs of `bench.py --probe-traffic`
# (FETCH_SIZE, then WRITE_SIZE), each scaled by what the same counter reads for a
# 256 MiB device copy (FETCH 0.50006, WRITE 1.0). Each constant names the commit
# whose kernel sources it was measured with; re-measure when those change.
#   gate_up (per-kernel path): gemv_kernel<PRO_PARTS, EPI_SWIGLU, 1, 5, 1> at batch 1
GATE_UP_TRAFFIC_B1 = 100_153_865
GATE_UP_TRAFFIC_AT = "1ea3e7e"
#   the persistent step kernel (step_kernel<128, 4, false>) at batch 1, context 137..146:
#   3,966,165 KiB / 0.500066 fetched + 4,418 KiB written per launch, 1.0075x its
#   8,065,954,304 algorithmic bytes (the rest is hand-over polling)
STEP_TRAFFIC_B1 = 8_126_157_727
STEP_TRAFFIC_AT = "081d385"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gate_up_bytes(b: int, h: int, inter: int, sk: int) -> int:
    """Algorithmic bytes of one fused gate_up launch: the [2I, H] weight, the
    prologue's fp32 partials + bf16 residual + gain, the bf16 residual it
    writes, and the [B, I] bf16 activation out."""
    return 2 * (2 * inter) * h + b * h * (4 * sk + 2 + 2) + 2 * h + 2 * b * inter


def step_bytes(cfg: dict, ctx_avg: float) -> int:
    """Algorithmic bytes of one batch-1 decode step: every weight once
    (8,044,544,000 at the Qwen3-4B shape), the cached K and V rows attended
    (2 x layers x kv heads x head dim x 2 B per key) and the new row written,
    the norm gains, the embedding row and the cos/sin rows."""
    from enginekernel_amd import checkpoint as C
    h, d, nl = cfg["hidden_size"], cfg["head_dim"], cfg["num_hidden_layers"]
    kv_row = 2 * nl * cfg["num_key_value_heads"] * d * 2
    gains = nl * (2 * h + 2 * d) * 2 + h * 2
    return int(C.weight_bytes_per_token(cfg) + kv_row * (ctx_avg + 1) + gains + 2 * h + 2 * 2 * d)


def time_dominant_kernel(model, b: int, reps: int = 3):
    """Average duration of the fused gate_up launch, measured with HIP
    events on the launching stream, over every layer's weights."""
    import torch
    from enginekernel_amd import ek_kernels as K

    bufs = model.buffers(b)
    c = model.cfg
    res_a, res_b = bufs.res
    bufs.o_parts.normal_(0, 0.05)
    res_b.normal_(0, 0.5)
    stream = torch.cuda.current_stream()

    def one_pass():
        for lay in model.layers:
            K.parts_norm_gemv(bufs.o_parts, res_b, res_a, lay["ln2"], lay["gu"], c.rms_eps, silu=True,
                              out=bufs.act)

    one_pass()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        one_pass()
    end.record(stream)
    end.synchronize()
    n = reps * len(model.layers)
    avg_s = start.elapsed_time(end) / 1e3 / n
    nbytes = gate_up_bytes(b, c.hidden_size, c.intermediate_size, bufs.sk_o)
    return avg_s, nbytes, n


def probe_traffic(b: int = 1, layers: int = 36) -> None:
    """The launches a `rocprofv3 --pmc FETCH_SIZE` (then `WRITE_SIZE`) run
    counts: one plain device copy of 256 MiB (the calibration: its
    algorithmic traffic is 256 MiB read + 256 MiB written), then 10 eager
    launches of the persistent decode step at the Qwen3-4B shape (batch 1,
    context 137..146; 8 GB of weights per launch, beyond the 256 MB Infinity
    Cache); with ENGINE_PERSISTENT=0, the fused gate_up launch over 36
    distinct weight copies instead."""
    import torch
    from enginekernel_amd import checkpoint as C
    from enginekernel_amd import ek_kernels as K

    dev = torch.device("cuda:0")
    h, inter = C.QWEN3_4B["hidden_size"], C.QWEN3_4B["intermediate_size"]
    src = torch.empty(128 << 20, dtype=torch.bfloat16, device=dev).normal_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    if os.environ.get("ENGINE_PERSISTENT", "1") != "0":
        from enginekernel_amd.ek_model import Qwen3
        from enginekernel_amd.engine import _FastEngine
        cfg = dict(C.QWEN3_4B)
        model = Qwen3(None, dev, tensors=C.random_weights(cfg, seed=0), config=cfg)
        eng = _FastEngine(model=model)
        s, steps = 136, 10
        with torch.inference_mode():
            eng._ensure_cache(1, s + steps + 1)
            g = eng._get_graph(1, s + steps + 1)
            g.begin(torch.ones(1, dtype=torch.int64, device=dev), [s], [0], s)
            kv = ([t[:1] for t in eng.k_cache], [t[:1] for t in eng.v_cache])
            torch.cuda.synchronize()
            for _ in range(steps):
                eng._step_body(g, kv)
            torch.cuda.synchronize()
        K.check_error_word(g.err, "the profiled decode steps")
        print(json.dumps({"probe": "traffic", "copy_bytes": 2 * src.numel(), "step_launches": steps,
                          "step_bytes": step_bytes(cfg, s + (steps + 1) / 2), "context": [s + 1, s + steps]}),
              flush=True)
        return
    g = torch.Generator(device=dev).manual_seed(0)
    ws = [torch.empty(2 * inter, h, dtype=torch.bfloat16, device=dev).normal_(0, 0.02, generator=g)
          for _ in range(layers)]
    sk = K.parts_splits(b, 4096)
    parts = torch.empty(sk, b, h, dtype=torch.float32, device=dev).normal_(0, 0.05, generator=g)
    res = torch.empty(b, h, dtype=torch.bfloat16, device=dev).normal_(0, 0.5, generator=g)
    res_out = torch.empty_like(res)
    nw = torch.ones(h, dtype=torch.bfloat16, device=dev)
    act = torch.empty(b, inter, dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    for w in ws:
        K.parts_norm_gemv(parts, res, res_out, nw, w, 1e-6, silu=True, out=act)
    torch.cuda.synchronize()
    print(json.dumps({"probe": "traffic", "copy_bytes": 2 * src.numel(), "gate_up_launches": layers,
                      "gate_up_bytes": gate_up_bytes(b, h, inter, sk), "sk": sk}), flush=True)


FIXTURE = os.path.join(ROOT, "tests", "golden", "config4_trace.npz")
CPU_STEPS = 64   # timed CPU decode steps (after one warm-up step), whatever --steps is


def cpu_baseline(tensors, cfg, kv, s, gpu_tokens, budget_s=60.0):
    """The oracle's decode loop (engine.py:721-743 restated) on this host's
    cores, from the GPU prefill's KV cache, teacher-forced with the committed
    config-4 fixture's ids (tests/golden/config4_trace.npz: the oracle's own
    greedy tokens for this prompt), so the sample is CPU_STEPS + 1 steps
    whatever --steps is. Times whole decode steps (argmax included), prefill
    excluded. Reports how many of its tokens equal the fixture's, and how many
    equal the GPU's over the steps where the GPU's free-running tokens still
    follow the fixture (after a GPU near-tie flip the contexts differ)."""
    import numpy as np
    import torch
    from oracle import ek_oracle as O

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    ids = np.load(FIXTURE)["ids"].astype(np.int64)
    n = CPU_STEPS + 1
    om = O.OracleQwen3(O.OracleConfig(cfg), tensors)
    k_cpu, v_cpu = kv
    b = 1
    st = O.EagerState.__new__(O.EagerState)
    st.k, st.v = k_cpu, v_cpu
    st.positions = torch.tensor([s], dtype=torch.int64)
    st.slot_t = torch.zeros(b, dtype=torch.int64)
    st.len_t = torch.full((1,), s, dtype=torch.int64)
    st.start_t = torch.zeros(b, dtype=torch.int32)
    # the GPU's tokens follow the fixture up to its first differing step
    follow = next((i for i in range(len(gpu_tokens)) if gpu_tokens[i] != ids[i + 1]), len(gpu_tokens))
    times, agree_fx, agree_gpu = [], 0, 0
    t_start = time.perf_counter()
    with torch.inference_mode():
        for i in range(n):
            t0 = time.perf_counter()
            hidden = om.decode(torch.tensor([int(ids[i])], dtype=torch.int64), st.positions, st.k, st.v,
                               st.slot_t, st.len_t, st.start_t)
            nxt = int(O.argmax_token(hidden, om.lm_head).item())
            times.append(time.perf_counter() - t0)
            agree_fx += int(nxt == ids[i + 1])
            if i < follow:
                agree_gpu += int(nxt == gpu_tokens[i])
            st.positions = st.positions + 1
            if time.perf_counter() - t_start > budget_s and i >= 3:
                break
    timed = times[1:] if len(times) > 2 else times      # the first step warms caches
    per = sum(timed) / len(timed)
    cpu_model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(b / per, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
        "ms_per_token": round(per * 1e3, 2),
        "sample": (f"{len(timed)} timed decode steps (of {len(times)} run) of config 4 at context "
                   f"{s + 1}..{s + len(times)}, batch 1, teacher-forced with the committed fixture's ids, "
                   f"torch CPU oracle, {cpu_model}"),
        "agree_with_fixture": f"{agree_fx}/{len(times)}",
        "agree_with_gpu": f"{agree_gpu}/{min(follow, len(times))}",
    }


def cpu_config1():
    """BASELINE config 1 end to end on the CPU oracle: the tiny random-init
    Qwen3 (seed 0), three left-padded prompts of 5 / 9 / 16 ids (seed 1),
    32 greedy tokens (prefill + 31 decode steps), timed whole."""
    import torch
    from enginekernel_amd import checkpoint as C
    from oracle import ek_oracle as O

    cfg = dict(C.QWEN3_TINY)
    tensors = C.random_weights(cfg, seed=0)
    g = torch.Generator().manual_seed(1)
    prompts = [torch.randint(0, cfg["vocab_size"], (n,), generator=g).tolist() for n in (5, 9, 16)]
    om = O.OracleQwen3(O.OracleConfig(cfg), tensors)
    with torch.inference_mode():
        list(O.generate_eager(om, prompts, 4))          # warm-up
        t0 = time.perf_counter()
        out = list(O.generate_eager(om, prompts, 32))
        dt = time.perf_counter() - t0
    return {"config1_ms": round(dt * 1e3, 2), "config1_tokens_per_s": round(3 * len(out) / dt, 1),
            "config1_sample": "BASELINE config 1 whole: tiny Qwen3, 3 left-padded prompts (5/9/16), 32 greedy "
                              "tokens each (prefill + 31 decode steps), torch CPU oracle"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=511)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--layers", type=int, default=0, help="override the layer count (diagnostics only)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-budget", type=float, default=60.0)
    ap.add_argument("--probe-traffic", action="store_true", help="run only the launches of the PMC traffic profile")
    ap.add_argument("--config", type=int, default=4, choices=(2, 3, 4, 5, 6, 7),
                    help="4 (default): the batch-1 decode line; 2 / 3 / 5 / 6 / 7: the GEMV sweep, the attention "
                         "sweep, the batch-8 decode, batch-1 speculative vs plain decode, or the 2..8-row step in "
                         "both forms, one JSON line each (enginekernel_amd.microbench)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)
    if args.probe_traffic:
        probe_traffic()
        return
    if args.config != 4:
        from enginekernel_amd import microbench
        print(json.dumps(dict(microbench.run(args.config, log=log), n_gpus=1)), flush=True)
        return

    import torch
    from enginekernel_amd import checkpoint as C
    from enginekernel_amd import ek_kernels as K
    from enginekernel_amd.ek_model import Qwen3
    from enginekernel_amd.engine import MAX_STEPS, _FastEngine

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    cfg = dict(C.QWEN3_4B)
    if args.layers:
        cfg["num_hidden_layers"] = args.layers
    w_bytes = C.weight_bytes_per_token(cfg)
    K_steps, W = args.steps, args.warmup
    if W + K_steps + 1 > MAX_STEPS:
        sys.exit(f"warmup + steps must stay below {MAX_STEPS}")

    t0 = time.perf_counter()
    tensors = C.random_weights(cfg, seed=0)
    log(f"random weights generated in {time.perf_counter() - t0:.1f}s")
    t0 = time.perf_counter()
    model = Qwen3(None, dev, tensors=tensors, config=cfg)
    torch.cuda.synchronize()
    log(f"weights uploaded in {time.perf_counter() - t0:.1f}s")
    eng = _FastEngine(model=model)

    b, s = 1, args.prompt
    g = torch.Generator().manual_seed(1)
    prompt = [torch.randint(0, cfg["vocab_size"], (s,), generator=g).tolist()]
    total = s + W + K_steps + 1
    with torch.inference_mode():
        ids, pos, pad, s, bias = eng._pack(prompt)
        eng._ensure_cache(b, total)
        model.ensure_rope(total + 1)
        t0 = time.perf_counter()
        graph = eng._get_graph(b, total)
        log(f"graph captured in {time.perf_counter() - t0:.1f}s (bucket {graph.bucket})")
        first = eng._first_token(ids, pos, b, s, bias)
        graph.begin(first, [s], [0], s)
        for _ in range(W):
            graph.graph.replay()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t_wall = time.perf_counter()
        ev0.record(stream)
        for _ in range(K_steps):
            graph.graph.replay()
        ev1.record(stream)
        ev1.synchronize()
        wall = time.perf_counter() - t_wall
        step_s = ev0.elapsed_time(ev1) / 1e3 / K_steps
        log(f"{K_steps} replays: {step_s * 1e3:.4f} ms/step (wall {wall / K_steps * 1e3:.4f})")
        tokens = graph.out_buf[: W + K_steps, 0].cpu().tolist()
        if graph.step_idx.item() != W + K_steps:
            raise RuntimeError("graph step counter out of step with the replays")

        persistent = model.buffers(b).step is not None
        K.check_error_word(graph.err, "the timed decode steps")
        if persistent:
            # one kernel per replay: its launch time is the replay time
            ctx_avg = s + W + 1 + (K_steps - 1) / 2
            dom_s, dom_bytes, dom_n = step_s, step_bytes(cfg, ctx_avg), K_steps
            split = model.persistent_plan(b, graph.bucket)[1]
            dom_name = (f"eks::step_kernel<128,4,{'true' if split else 'false'}> (the whole decode step, one launch"
                        + (f"; every workgroup attends 1/{split} of a kv head's keys)" if split else ")"))
            # the PMC figure is for the default workload only
            dom_traffic = STEP_TRAFFIC_B1 if (not split and args.prompt == 128 and not args.layers) else None
            traffic_at = STEP_TRAFFIC_AT if dom_traffic else None
        else:
            dom_s, dom_bytes, dom_n = time_dominant_kernel(model, b)
            dom_name = "gemv_kernel<PRO_PARTS,EPI_SWIGLU> (add+RMSNorm+gate_up+SwiGLU)"
            dom_traffic = GATE_UP_TRAFFIC_B1 if b == 1 else None
            traffic_at = GATE_UP_TRAFFIC_AT if dom_traffic else None
            log(f"gate_up kernel: {dom_s * 1e6:.2f} us over {dom_n} launches")

        cpu = None
        if not args.no_cpu and args.prompt == 128 and not args.layers:
            # the GPU prefill's KV cache of the prompt (rows [0, s)), with room
            # for the sampled steps
            room = CPU_STEPS + 2
            kv = ([t[0:1, :, :s].cpu().clone() for t in eng.k_cache],
                  [t[0:1, :, :s].cpu().clone() for t in eng.v_cache])
            kv = ([torch.cat([t, torch.zeros(1, t.shape[1], room, t.shape[3], dtype=t.dtype)], 2) for t in kv[0]],
                  [torch.cat([t, torch.zeros(1, t.shape[1], room, t.shape[3], dtype=t.dtype)], 2) for t in kv[1]])
            log("timing the CPU oracle baseline")
            # GPU step 1 decoded token `first` (fixture id 0) at context s+1 and emitted tokens[0]
            cpu = cpu_baseline(tensors, cfg, kv, s, tokens, budget_s=args.cpu_budget)
            cpu.update(cpu_config1())

    achieved = dom_bytes / dom_s
    line = {
        "metric": "batch-1 decode tokens/sec + ms/token and % of HBM roofline, Qwen3-4B shape",
        "value": round(b / step_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K_steps,
        "warmup": W,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights ~N(0,0.02) seed 0, random prompt ids seed 1)",
        "config": {
            "workload": ("config 4: Qwen3-4B-architecture bf16 greedy decode, one hipGraph replay per token"
                         + (" (one persistent kernel per step)" if persistent else " (per-kernel graph)")),
            "batch": b, "prompt_len": s, "context_at_timed_steps": [s + W + 1, s + W + K_steps],
            "layers": cfg["num_hidden_layers"], "hidden": cfg["hidden_size"],
            "intermediate": cfg["intermediate_size"], "heads": [cfg["num_attention_heads"], cfg["num_key_value_heads"]],
            "vocab": cfg["vocab_size"],
        },
        "ms_per_token": round(step_s * 1e3, 4),
        "weight_bytes_per_token": w_bytes,
        "hbm_roofline_frac": round(w_bytes / step_s / PEAK_HBM, 4),
        "roofline": {
            "bound": "hbm", "kernel": dom_name,
            "achieved": round(achieved / 1e9, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM, 4), "traffic": dom_traffic, "traffic_measured_at": traffic_at,
            "bytes_per_launch": dom_bytes, "avg_launch_us": round(dom_s * 1e6, 3), "launches": dom_n,
        },
        "cpu_baseline": cpu,
        "first_tokens": tokens[:8],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
