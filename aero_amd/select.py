"""Per-op selection of the GPU path for a model loop.

The reference's model loop (engine/model.py:550-754, src/model.cpp:166-342)
calls each elementwise op at a fixed site; this module is the switch such a
site consults: AERO_GPU_OPS=rmsnorm,rope,act,embed (or "all" / "none"),
overridable per call site with a keyword. The selector only answers "is this
op on the GPU?"; the caller keeps its own code for the ops it leaves off.

    from aero_amd import select
    if select.enabled("rmsnorm"):
        h = aero_amd.transformer_native.rmsnorm_rows(x, w, eps)
    else:
        h = transformer.rms_norm(x, w, eps)           # the caller's own path

Unknown names in AERO_GPU_OPS raise ValueError, so a typo cannot silently
leave an op on the CPU.
"""
from __future__ import annotations

import os

OPS = ("rmsnorm", "qk_norm", "gated_norm", "rope", "act", "embed", "dequant")
ENV = "AERO_GPU_OPS"

# Fusions a device-resident loop may use when every op they join is on the
# GPU: the embedding gather with the first norm, the norms (and residual
# adds) folded into the projections that consume them, the act-mul folded
# into the gate/up projection, RoPE (and the per-head norm) folded into the
# q/k projection's epilogue, the embedding rows read by the first q/k/v
# projection's pre-pass, a DeltaNet layer's conv folded into its input
# projections' epilogue at one token. AERO_GPU_FUSE=none turns them off (the
# same ops then run as separate kernels); unset means all on.
FUSIONS = ("embed_norm", "norm_gemm", "act_gemm", "rope_gemm", "conv_gemm", "embed_gemm")
FUSE_ENV = "AERO_GPU_FUSE"


class HostPathRequired(RuntimeError):
    """An op is off the GPU (AERO_GPU_OPS) and the caller gave no host code
    for it: a device-resident loop has no CPU path of its own."""


def parse(spec: str | None, names: tuple = OPS, env: str = ENV) -> frozenset:
    if spec is None:
        return frozenset()
    spec = spec.strip().lower()
    if spec in ("", "none", "0", "off"):
        return frozenset()
    if spec in ("all", "1", "on"):
        return frozenset(names)
    got = {s.strip() for s in spec.split(",") if s.strip()}
    unknown = got - set(names)
    if unknown:
        raise ValueError(f"{env}: unknown name(s) {sorted(unknown)}; choose from {names}")
    return frozenset(got)


def enabled_ops() -> frozenset:
    return parse(os.environ.get(ENV))


def enabled(op: str, override: bool | None = None, default: bool = False) -> bool:
    """True when `op` should run on the GPU: the call-site override if given,
    else AERO_GPU_OPS, else `default` when AERO_GPU_OPS is unset."""
    if op not in OPS:
        raise ValueError(f"unknown op {op!r}; choose from {OPS}")
    if override is not None:
        return bool(override)
    if os.environ.get(ENV) is None:
        return bool(default)
    return op in enabled_ops()


def fusion_enabled(name: str, override: bool | None = None) -> bool:
    """True when fusion `name` may be used: the override if given, else
    AERO_GPU_FUSE (unset: every fusion)."""
    if name not in FUSIONS:
        raise ValueError(f"unknown fusion {name!r}; choose from {FUSIONS}")
    if override is not None:
        return bool(override)
    spec = os.environ.get(FUSE_ENV)
    if spec is None:
        return True
    return name in parse(spec, FUSIONS, FUSE_ENV)
