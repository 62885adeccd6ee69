"""MI355X (gfx950) quantized MoE expert path behind the C ABI of include/rvmoe.h.

`rosevine_amd.hip` is the safe host view of librvmoe.so (the reference's runtime/src/hip.rs),
`rosevine_amd.moe` the all-device MoE layer dispatch (runtime/src/hip_exec.rs:780-843) and
`rosevine_amd.synth` the seeded synthetic workloads. The compute path is HIP only: without the
built library every entry point raises.
"""
from . import hip, moe, synth  # noqa: F401

__all__ = ["hip", "moe", "synth"]
