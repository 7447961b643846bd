"""Swap the reference op for the MI355X one, in place.

The reference's GDN layers bind the op by name at import time
(``from ...gated_delta_rule import chunk_gated_delta_rule`` in
fla/layers/gated_deltanet.py:16 and gated_deltanet_with_tp.py:17), the same
way Kairos' own engine swap monkey-patches the DiT (kairos_ext/kairos_engine_patch.py:1773).
``install()`` rebinds that name in every already-imported module that holds
it, so the layers call this build's kernels; ``uninstall()`` restores the
originals.
"""
from __future__ import annotations

import sys

from .chunk import chunk_gated_delta_rule

# module names (pip fla and the copy vendored under kairos/third_party) that bind the op
SITES = (
    "fla.ops.gated_delta_rule",
    "fla.ops.gated_delta_rule.chunk",
    "fla.layers.gated_deltanet",
    "fla.layers.gated_deltanet_with_tp",
    "kairos.third_party.fla.ops.gated_delta_rule",
    "kairos.third_party.fla.ops.gated_delta_rule.chunk",
    "kairos.third_party.fla.layers.gated_deltanet",
    "kairos.third_party.fla.layers.gated_deltanet_with_tp",
)

_saved: dict[str, object] = {}


def install(sites=SITES) -> list[str]:
    """Rebind ``chunk_gated_delta_rule`` in the imported modules among ``sites``; returns the patched names."""
    patched = []
    for name in sites:
        mod = sys.modules.get(name)
        if mod is None or not hasattr(mod, "chunk_gated_delta_rule"):
            continue
        cur = getattr(mod, "chunk_gated_delta_rule")
        if cur is chunk_gated_delta_rule:
            patched.append(name)
            continue
        _saved.setdefault(name, cur)
        setattr(mod, "chunk_gated_delta_rule", chunk_gated_delta_rule)
        patched.append(name)
    return patched


def uninstall() -> list[str]:
    """Restore every binding ``install`` replaced; returns the restored names."""
    restored = []
    for name, fn in list(_saved.items()):
        mod = sys.modules.get(name)
        if mod is not None:
            setattr(mod, "chunk_gated_delta_rule", fn)
            restored.append(name)
        del _saved[name]
    return restored
