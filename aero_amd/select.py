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


def parse(spec: str | None) -> frozenset:
    if spec is None:
        return frozenset()
    spec = spec.strip().lower()
    if spec in ("", "none", "0", "off"):
        return frozenset()
    if spec in ("all", "1", "on"):
        return frozenset(OPS)
    names = {s.strip() for s in spec.split(",") if s.strip()}
    unknown = names - set(OPS)
    if unknown:
        raise ValueError(f"{ENV}: unknown op(s) {sorted(unknown)}; choose from {OPS}")
    return frozenset(names)


def enabled_ops() -> frozenset:
    return parse(os.environ.get(ENV))


def enabled(op: str, override: bool | None = None) -> bool:
    """True when `op` should run on the GPU: the call-site override if given,
    else AERO_GPU_OPS."""
    if op not in OPS:
        raise ValueError(f"unknown op {op!r}; choose from {OPS}")
    if override is not None:
        return bool(override)
    return op in enabled_ops()
