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


def default_splits(max_len: int, hkv: int = 4, cus: int | None = None, kv8: bool = False) -> int:
    """Split count NS (part_o.size(2)) for a cache of ``max_len`` positions: 13/16 of the compute
    units in workgroups when the whole cache is attended (NS * Hkv = 13/16 CUs, 52 at Hkv 4 on 256
    CUs), never slices shorter than 32 positions. Measured on MI355X with the look-ahead tile loop
    (one row, 24 Q / 4 KV heads, partials µs at 4k / 16k / 32k / 128k): NS 52 6.97 / 13.48 / 23.08
    / 79.8; NS 48 6.98 / 13.91 / 23.49 / 80.3; NS 64 7.08 / 13.94 / 24.18 / 83.8; 40, 44, 56 and
    60 lie between or above. The workgroups' fixed tail (last tile, merge, stores) is spread over
    longer slices than at one workgroup per CU; more slices cost a second round of workgroups and
    more partials. An fp8 cache (``kv8``) streams half the bytes per slice and keeps one workgroup
    per CU (NS 64: 9.34 / 14.36 µs at 16k / 32k against 9.52 / 14.23 at NS 52, 9.55 / 15.08 at
    NS 48). NS is fixed when the scratch is allocated, so graphs stay static; a row attending L
    positions uses slices of split_size(L, NS), so about NS slices hold work at every length."""
    cus = cus or compute_units()
    per_head = cus // hkv if kv8 else (13 * cus) // (16 * hkv)
    return max(1, min(math.ceil(max_len / MIN_SLICE), max(1, per_head)))


def alloc_partials(n_rows: int, hq: int, ns: int, device="cuda"):
    """Caller-owned split-KV scratch (part_o, part_ml) for up to ``n_rows`` rows."""
    po = torch.empty(n_rows, hq, ns, HEAD_DIM, dtype=torch.float32, device=device)
    pml = torch.empty(n_rows, hq, ns, 2, dtype=torch.float32, device=device)
    return po, pml
