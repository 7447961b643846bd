"""Swap the reference op (and the layer's output norm) for the MI355X ones, in place.

The reference's GDN layers bind the ops by name at import time
(``from ...gated_delta_rule import chunk_gated_delta_rule, fused_recurrent_gated_delta_rule`` in
fla/layers/gated_deltanet.py:16 and gated_deltanet_with_tp.py:17), the same
way Kairos' own engine swap monkey-patches the DiT (kairos_ext/kairos_engine_patch.py:1773).
The layer's output norm and short-convolution classes are bound the same way
(``from ...modules import FusedRMSNormGated, RMSNorm, ShortConvolution``,
gated_deltanet.py:15) and instantiated in the layer's constructor (:176-197).  ``install()`` rebinds those
names in every already-imported module that holds them, so the layers call
this build's kernels (layers constructed afterwards get the MI355X norm and convolutions);
``uninstall()`` restores the originals.
"""
from __future__ import annotations

import sys

from .chunk import chunk_gated_delta_rule
from .conv import ShortConvolution
from .norm import FusedRMSNormGated
from .recurrent import fused_recurrent_gated_delta_rule

# module names (pip fla and the copy vendored under kairos/third_party) that bind the op or the norm
SITES = (
    "fla.ops.gated_delta_rule",
    "fla.ops.gated_delta_rule.chunk",
    "fla.ops.gated_delta_rule.fused_recurrent",
    "fla.layers.gated_deltanet",
    "fla.layers.gated_deltanet_with_tp",
    "kairos.third_party.fla.ops.gated_delta_rule",
    "kairos.third_party.fla.ops.gated_delta_rule.chunk",
    "kairos.third_party.fla.ops.gated_delta_rule.fused_recurrent",
    "kairos.third_party.fla.layers.gated_deltanet",
    "kairos.third_party.fla.layers.gated_deltanet_with_tp",
)
# the names install() rebinds, with their replacements
REPLACEMENTS = {
    "chunk_gated_delta_rule": chunk_gated_delta_rule,
    "fused_recurrent_gated_delta_rule": fused_recurrent_gated_delta_rule,
    "FusedRMSNormGated": FusedRMSNormGated,
    "ShortConvolution": ShortConvolution,
}

_saved: dict[tuple[str, str], object] = {}


def install(sites=SITES, names=tuple(REPLACEMENTS)) -> list[str]:
    """Rebind ``names`` (default: both ops, the norm and the convolution class) in the imported modules among
    ``sites``; returns the patched ``module.name`` entries."""
    patched = []
    for mod_name in sites:
        mod = sys.modules.get(mod_name)
        if mod is None:
            continue
        for attr in names:
            if not hasattr(mod, attr):
                continue
            new = REPLACEMENTS[attr]
            cur = getattr(mod, attr)
            if cur is not new:
                _saved.setdefault((mod_name, attr), cur)
                setattr(mod, attr, new)
            patched.append(f"{mod_name}.{attr}")
    return patched


def uninstall() -> list[str]:
    """Restore every binding ``install`` replaced; returns the restored ``module.name`` entries."""
    restored = []
    for (mod_name, attr), obj in list(_saved.items()):
        mod = sys.modules.get(mod_name)
        if mod is not None:
            setattr(mod, attr, obj)
            restored.append(f"{mod_name}.{attr}")
        del _saved[(mod_name, attr)]
    return restored
