"""rie-hip: RIE's per-token forward loop (CpuBackend::forward_impl,
crates/rie-core/src/model/cpu.rs:210-409) as hand-written HIP for MI355X
(gfx950), behind a C ABI that mirrors RIE's Backend trait (include/rie_hip.h).
"""
from . import synth
from ._lib import build, lib
from .backend import HipBackend, KvType, RieError
from .engine import Engine, argmax

__all__ = ["HipBackend", "KvType", "RieError", "Engine", "argmax", "synth", "build", "lib"]
