"""qengine_amd: MI355X-native (gfx950) gated-attention decode path for qengine.

``qengine_amd._C`` exposes the reference's ``qengine._C`` ops with the same signatures
(``attn_prep``, ``attn_decode``, the rest of the decode step, ``gdn_step_n``, plus the reference's
PDL / L2 / GDN A/B switches as no-ops), backed by hand-written HIP kernels in ``libqe_attn.so``
(C ABI: ``include/qe_*.h``). There is no CPU fallback: importing
this package fails if the native libraries are not built.
"""
from __future__ import annotations

import math

# torch first: it loads its own HIP runtime, and our libraries then bind to that same copy
# (both are named libamdhip64.so.7).
import torch  # noqa: F401

try:
    from . import _C  # noqa: F401
except ImportError as exc:  # pragma: no cover - exercised only on an unbuilt tree
    raise ImportError(
        "qengine_amd native extension is not built; run `python qengine_amd/_build.py`"
    ) from exc

from ._C import (  # noqa: E402,F401
    accept,
    argmax,
    attn_decode,
    attn_decode_combine,
    attn_decode_fp8,
    attn_decode_fp8_partials,
    attn_decode_partials,
    attn_prefill,
    attn_prep,
    attn_prep_chunk,
    attn_prep_decode,
    attn_prep_fp8,
    commit,
    embed,
    gdn_step_n,
    gemv_bf16,
    l2_persist_limit,
    mtp_select,
    rmsnorm1p,
    set_gdn_early,
    set_gdn_phases,
    set_pdl_launch,
    set_pdl_trigger,
    split_size,
    stream_window,
    swiglu,
    version,
)

HEAD_DIM = 256
MIN_SLICE = 32  # one wave step of cache positions


def compute_units(device=None) -> int:
    """Compute units of the GPU (256 on MI355X)."""
    try:
        return torch.cuda.get_device_properties(device or torch.cuda.current_device()).multi_processor_count
    except (RuntimeError, AssertionError):
        return 256


def default_splits(max_len: int, hkv: int = 4, cus: int | None = None) -> int:
    """Split count NS (part_o.size(2)) for a cache of ``max_len`` positions: one workgroup per
    compute unit when the whole cache is attended (NS * Hkv = CUs), never slices shorter than
    32 positions. Measured on MI355X, this is the fastest choice from 4k to 128k positions:
    fewer slices leave CUs idle, more slices cost a second round of workgroups and more partials.
    NS is fixed when the scratch is allocated, so graphs stay static; a row attending L
    positions uses slices of split_size(L, NS), so about NS slices hold work at every length."""
    cus = cus or compute_units()
    return max(1, min(math.ceil(max_len / MIN_SLICE), max(1, cus // hkv)))


def alloc_partials(n_rows: int, hq: int, ns: int, device="cuda"):
    """Caller-owned split-KV scratch (part_o, part_ml) for up to ``n_rows`` rows."""
    po = torch.empty(n_rows, hq, ns, HEAD_DIM, dtype=torch.float32, device=device)
    pml = torch.empty(n_rows, hq, ns, 2, dtype=torch.float32, device=device)
    return po, pml
