"""Out-of-process probes of the HIP library (the reference's ek_probe.py,
called through engine._child_ok, engine.py:47-77, 439-470).

    python -m enginekernel_amd.ek_probe basic
        load libek_hip.so and run one kernel (ek_kernels.probe_hip)
    python -m enginekernel_amd.ek_probe shape B Q BUCKET N_KV N_Q HEAD_DIM
        run the attention launches of one decode shape on random data: the
        decode attention at batch B over a BUCKET-slot cache (the graph's
        plan of splits), and with Q > 0 the verify attention of Q tokens per
        row; the outputs must be finite
    python -m enginekernel_amd.ek_probe noop
        exit 0 (checks that a child can be started at all)

Exit status 0 means the probe ran cleanly. A crash, a hang or a failed check
in the child costs the parent nothing but the answer; the engine then
refuses the shape (HipUnavailable) and the Engine facade's fallback, if any,
takes over.
"""

from __future__ import annotations

import sys


def _basic() -> int:
    from . import ek_kernels as K
    return 0 if K.probe_hip() else 1


def _shape(b: int, q: int, bucket: int, n_kv: int, n_q: int, d: int) -> int:
    import torch

    from . import ek_kernels as K
    if not K.probe_hip():
        return 1
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    bf = torch.bfloat16
    kc = torch.randn(b, n_kv, bucket, d, generator=g, device=dev).to(bf)
    vc = torch.randn(b, n_kv, bucket, d, generator=g, device=dev).to(bf)
    start = torch.zeros(b, dtype=torch.int32, device=dev)
    ws = K.make_workspace(b, n_q, n_kv, d, bucket, dev)
    qd = torch.randn(b, n_q, d, generator=g, device=dev).to(bf)
    seq_len = torch.full((1,), max(1, bucket - max(q, 1)), dtype=torch.int64, device=dev)
    outs = [K.flash_decode(qd, kc, vc, seq_len, start, ws, d ** -0.5)]
    if q > 0:
        qkv = torch.randn(b * q, (n_q + 2 * n_kv) * d, generator=g, device=dev).to(bf)
        len_b = torch.full((b,), bucket - q, dtype=torch.int64, device=dev)
        outs.append(K.attn_verify(qkv, kc, vc, start, len_b, q, n_q, d ** -0.5))
    torch.cuda.synchronize()
    return 0 if all(bool(torch.isfinite(o.float()).all()) for o in outs) else 1


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    if not argv:
        return 2
    if argv[0] == "noop":
        return 0
    if argv[0] == "basic":
        return _basic()
    if argv[0] == "shape" and len(argv) == 7:
        return _shape(*(int(a) for a in argv[1:]))
    return 2


if __name__ == "__main__":
    sys.exit(main())
