"""enginekernel_amd: the Qwen3 per-token decode hot path of
jeojdi1/EngineKernel, rebuilt on hand-written gfx950 (MI355X) HIP kernels.

    enginekernel_amd.ek_kernels   the reference's kernel call surface
    enginekernel_amd.ek_model     Qwen3Config / Qwen3
    enginekernel_amd.engine       Engine (graph-captured greedy decode)
    enginekernel_amd.checkpoint   seeded random-init checkpoints
    enginekernel_amd.build        hipcc build of libek_hip.so

Submodules are imported on use so that `import enginekernel_amd` needs
neither a GPU nor the built library.
"""

__all__ = ["ek_kernels", "ek_model", "engine", "checkpoint", "build"]
