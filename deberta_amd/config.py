"""The attention-kernel selector: the plugin seam the reference exposes as
``model.hf.attention_kernel`` (config.py:96-104, normalised at :1204-1216 via
:1105-1126).

The reference's three choices (``dynamic``, ``cached_bmm``, ``stable``) are
three eager formulations of one function (its tests pin them equal at
rtol 1e-5); this package computes that function once, in the fused HIP
kernels, and adds ``fused`` as the explicit name.  All four names (and the
reference's aliases) select the fused kernels, so a reference config loads
unchanged.  Invalid names raise the reference's error text.
"""

from __future__ import annotations

ATTENTION_KERNEL_CHOICES = frozenset({"dynamic", "cached_bmm", "stable", "fused"})
ATTENTION_KERNEL_ALIASES = {
    "default": "dynamic",
    "cache": "cached_bmm",
    "cached": "cached_bmm",
    "safe": "stable",
    "compile_safe": "stable",
    "hip": "fused",
    "flash": "fused",
}


def normalize_attention_kernel(value: object) -> str:
    """Canonical kernel name: lower-case, ``-`` to ``_``, aliases resolved;
    ``ValueError('model.hf.attention_kernel must be one of: ...')`` otherwise."""
    v = str(value).strip().lower().replace("-", "_")
    v = ATTENTION_KERNEL_ALIASES.get(v, v)
    if v not in ATTENTION_KERNEL_CHOICES:
        allowed = "|".join(sorted(ATTENTION_KERNEL_CHOICES))
        raise ValueError(f"model.hf.attention_kernel must be one of: {allowed}. Got: {value}")
    return v


def normalize_pos_att_type(raw: object) -> list[str]:
    """``"c2p|p2c"`` / ``"c2p,p2c"`` / list -> ``["c2p", "p2c"]`` (lower case,
    empty chunks dropped), as deberta_v2_native.py:28-48."""
    if raw is None:
        return []
    if isinstance(raw, str):
        chunks = raw.replace(",", "|").split("|")
    elif isinstance(raw, (list, tuple, set)):
        chunks = [str(x) for x in raw]
    else:
        chunks = [str(raw)]
    out: list[str] = []
    for chunk in chunks:
        value = str(chunk).strip().lower()
        if value:
            out.append(value)
    return out
