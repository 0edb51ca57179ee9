"""CPU oracle for the Qwen3 decode hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in plain torch on the CPU, the reference's torch
fallback path (jeojdi1/EngineKernel `engine/ek_kernels.py`,
`engine/ek_model.py`, `engine/engine.py`; file:line cited per function in
`ek_oracle.py`). It is the checker the HIP path is compared against.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import it, and only as the checker or the timed CPU baseline.
The product package `enginekernel_amd` never imports it and has no CPU
fallback: its kernels fail loudly when the HIP library is missing.

How each function is pinned (so that a dropped term, a wrong sign or a
transposed operand fails a test) is listed in `tests/test_oracle.py`:
transformers' own Qwen3ForCausalLM greedy decode (token-exact, the
reference's `bench/test_equivalence.py` check), float64 closed forms for the
norms, RoPE and attention, the HF rotary formula, brute-force softmax on
tiny inputs, and attention special cases (one key, constant keys). The
speculative draft is pinned against a search by n-gram order then position
(an independent statement of its score), the accept step against hand-worked
cases, and the verify attention against the single-query decode attention
(each verify query equals a decode at its own length).
"""
