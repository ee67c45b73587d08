"""ctypes binding of the C ABI in include/qe_attn.h, include/qe_gemv.h, include/qe_step.h and
include/qe_gdn.h (libqe_attn.so), without the torch extension.

This is the binding a non-torch host (or a test that must go through the C ABI) uses. Tensor
arguments may be torch tensors (their data_ptr is passed) or raw integer device addresses.
Streams are raw hipStream_t values (0 = the null stream; torch:
``torch.cuda.current_stream().cuda_stream``).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (loads torch's HIP runtime first; see qengine_amd/__init__.py)

LIB_PATH = Path(__file__).resolve().parent / "libqe_attn.so"

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_long
_F = ctypes.c_float

SIGNATURES = {
    "qe_attn_prep": (_I, [_P, _P, _P, _L, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P]),
    "qe_attn_decode": (_I, [_P, _P, _P, _P, _P, _L, _P, _P, _P, _L, _I, _I, _I, _I, _I, _F, _P]),
    "qe_attn_decode_partials": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P]),
    "qe_attn_decode_noalloc": (_I, [_P, _P, _P, _P, _P, _L, _P, _L, _I, _I, _I, _I, _I, _F, _P]),
    "qe_attn_decode_combine": (_I, [_P, _P, _P, _P, _L, _P, _L, _I, _I, _I, _I, _P]),
    "qe_attn_prefill": (_I, [_P, _P, _P, _P, _P, _L, _P, _L, _I, _I, _I, _I, _F, _P]),
    "qe_attn_prefill_fp8": (_I, [_P, _P, _P, _P, _P, _L, _P, _L, _I, _I, _I, _I, _F, _F, _F, _P]),
    "qe_attn_prep_decode": (_I, [_P, _P, _P, _L, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L, _I, _I,
                                 _I, _I, _I, _I, _F, _F, _P]),
    "qe_attn_split_size": (_I, [_I, _I]),
    "qe_kv_stream_probe": (_I, [_P, _P, _P, _I, _I, _I, _P, _P]),
    "qe_kv_stream_sweep": (_I, [_P, _P, _P, _I, _I, _I, _I, _P, _P]),
    "qe_launch_probe": (_I, [_P]),
    "qe_attn_version": (ctypes.c_char_p, []),
    "qe_set_pdl_trigger": (None, [_I]),
    "qe_set_pdl_launch": (None, [_I]),
    "qe_attn_prep_fp8": (_I, [_P, _P, _P, _L, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F,
                              _F, _P]),
    "qe_attn_decode_fp8": (_I, [_P, _P, _P, _P, _P, _L, _P, _P, _P, _L, _I, _I, _I, _I, _I, _F, _F,
                                _F, _P]),
    "qe_attn_decode_fp8_partials": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _F, _P]),
    "qe_gemv_bf16": (_I, [_P, _P, _P, _I, _I, _I, _L, _L, _P]),
    "qe_gemv_kparts": (_I, [_I, _I]),
    "qe_gemv_tile_rows": (_I, [_I, _I]),
    "qe_hbm_read_probe": (_I, [_P, ctypes.c_size_t, _P, _P]),
    "qe_embed": (_I, [_P, _P, _P, _I, _I, _I, _L, _P]),
    "qe_rmsnorm1p": (_I, [_P, _P, _P, _P, _I, _I, _L, _L, _L, _F, _P]),
    "qe_swiglu": (_I, [_P, _P, _I, _I, _L, _L, _P]),
    "qe_argmax": (_I, [_P, _I, _I, _L, _P, _P, _I, _P, _P, _P]),
    "qe_accept": (_I, [_P, _P, _I, _P, _P, _P, _I, _P]),
    "qe_commit": (_I, [_P, _P, _P, _P, _I, _P]),
    "qe_mtp_select": (_I, [_P, _P, _I, _P, _L, _P, _I, _P, _P, _P]),
    "qe_l2_persist_limit": (_I, [ctypes.c_size_t]),
    "qe_stream_access_window": (_I, [ctypes.c_size_t, ctypes.c_size_t, _F, _P]),
    "qe_gdn_step_n": (_I, [_P, _P, _P, _P, _L, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L, _I, _I,
                           _I, _F, _P]),
}

HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1

_lib = None


def load() -> ctypes.CDLL:
    """Load libqe_attn.so and declare every exported entry point (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise OSError(f"{LIB_PATH} is not built; run `python qengine_amd/_build.py`")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _ptr(x) -> int | None:
    if x is None:
        return None
    return x.data_ptr() if hasattr(x, "data_ptr") else int(x)


def _stream(stream) -> int | None:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return int(stream)


def prep(qg, k, v, ldp, qnw, knw, inv_freq, pos, q_out, kc, vc, n, hq, hkv, max_len, rd, eps,
         stream=None) -> int:
    return load().qe_attn_prep(_ptr(qg), _ptr(k), _ptr(v), ldp, _ptr(qnw), _ptr(knw),
                               _ptr(inv_freq), _ptr(pos), _ptr(q_out), _ptr(kc), _ptr(vc), n, hq,
                               hkv, max_len, rd, eps, _stream(stream))


def decode(q, kc, vc, pos, qg, ldp, part_o, part_ml, out, ldo, n, hq, hkv, max_len, ns,
           scale=1.0 / 16, stream=None) -> int:
    return load().qe_attn_decode(_ptr(q), _ptr(kc), _ptr(vc), _ptr(pos), _ptr(qg), ldp,
                                 _ptr(part_o), _ptr(part_ml), _ptr(out), ldo, n, hq, hkv, max_len,
                                 ns, scale, _stream(stream))


NOALLOC_MAX_SLOTS = 12288  # QE_NOALLOC_MAX_SLOTS in include/qe_attn.h


def decode_noalloc(q, kc, vc, pos, qg, ldp, out, ldo, n, hq, hkv, max_len, ns, scale=1.0 / 16,
                   stream=None) -> int:
    """qe_attn_decode with the library's own device scratch (no caller part_o / part_ml)."""
    return load().qe_attn_decode_noalloc(_ptr(q), _ptr(kc), _ptr(vc), _ptr(pos), _ptr(qg), ldp,
                                         _ptr(out), ldo, n, hq, hkv, max_len, ns, scale,
                                         _stream(stream))


def prep_decode(qg, k, v, ldp, qnw, knw, inv_freq, pos, q_out, kc, vc, part_o, part_ml, out, ldo,
                n, hq, hkv, max_len, rd, ns, scale=1.0 / 16, eps=1e-6, stream=None) -> int:
    return load().qe_attn_prep_decode(_ptr(qg), _ptr(k), _ptr(v), ldp, _ptr(qnw), _ptr(knw),
                                      _ptr(inv_freq), _ptr(pos), _ptr(q_out), _ptr(kc), _ptr(vc),
                                      _ptr(part_o), _ptr(part_ml), _ptr(out), ldo, n, hq, hkv,
                                      max_len, rd, ns, scale, eps, _stream(stream))


def decode_partials(q, kc, vc, pos, part_o, part_ml, n, hq, hkv, max_len, ns, scale=1.0 / 16,
                    stream=None) -> int:
    return load().qe_attn_decode_partials(_ptr(q), _ptr(kc), _ptr(vc), _ptr(pos), _ptr(part_o),
                                          _ptr(part_ml), n, hq, hkv, max_len, ns, scale,
                                          _stream(stream))


def decode_combine(part_o, part_ml, pos, qg, ldp, out, ldo, n, hq, max_len, ns,
                   stream=None) -> int:
    return load().qe_attn_decode_combine(_ptr(part_o), _ptr(part_ml), _ptr(pos), _ptr(qg), ldp,
                                         _ptr(out), ldo, n, hq, max_len, ns, _stream(stream))


def prefill(q, kc, vc, pos, qg, ldp, out, ldo, T, hq, hkv, max_len, scale=1.0 / 16,
            stream=None) -> int:
    return load().qe_attn_prefill(_ptr(q), _ptr(kc), _ptr(vc), _ptr(pos), _ptr(qg), ldp, _ptr(out),
                                  ldo, T, hq, hkv, max_len, scale, _stream(stream))


def prefill_fp8(q, kc8, vc8, pos, qg, ldp, out, ldo, T, hq, hkv, max_len, k_scale, v_scale,
                scale=1.0 / 16, stream=None) -> int:
    return load().qe_attn_prefill_fp8(_ptr(q), _ptr(kc8), _ptr(vc8), _ptr(pos), _ptr(qg), ldp,
                                      _ptr(out), ldo, T, hq, hkv, max_len, scale, k_scale, v_scale,
                                      _stream(stream))


def split_size(L: int, ns: int) -> int:
    """Slice size of a row attending L positions with ns partial slots (qe_attn_split_size)."""
    return load().qe_attn_split_size(L, ns)


def kv_stream_probe(kc, vc, pos, hkv, max_len, ns, sink, stream=None) -> int:
    """Measurement only: stream the K/V bytes of a 1-row decode at device position pos with the
    partials kernel's grid and slicing, no arithmetic (qe_kv_stream_probe)."""
    return load().qe_kv_stream_probe(_ptr(kc), _ptr(vc), _ptr(pos), hkv, max_len, ns, _ptr(sink),
                                     _stream(stream))


def kv_stream_sweep(kc, vc, pos, hkv, max_len, grid_per_head, depth, sink, stream=None) -> int:
    """Measurement only: the same K/V bytes on a (grid_per_head, hkv) grid with depth + depth
    loads in flight per thread (qe_kv_stream_sweep)."""
    return load().qe_kv_stream_sweep(_ptr(kc), _ptr(vc), _ptr(pos), hkv, max_len, grid_per_head,
                                     depth, _ptr(sink), _stream(stream))


def launch_probe(stream=None) -> int:
    """Measurement only: one empty kernel (qe_launch_probe)."""
    return load().qe_launch_probe(_stream(stream))


def version() -> str:
    return load().qe_attn_version().decode()


def gemv_bf16(W, x, out, nr, N, K, ldx, ldo, stream=None) -> int:
    return load().qe_gemv_bf16(_ptr(W), _ptr(x), _ptr(out), nr, N, K, ldx, ldo, _stream(stream))


def gemv_kparts(N: int, K: int) -> int:
    return load().qe_gemv_kparts(N, K)


def gemv_tile_rows(N: int, K: int) -> int:
    return load().qe_gemv_tile_rows(N, K)


def hbm_read_probe(buf, nbytes: int, sink, stream=None) -> int:
    return load().qe_hbm_read_probe(_ptr(buf), nbytes, _ptr(sink), _stream(stream))


def rmsnorm1p(x, delta, w, out, rows, H, ldx, ldd, ldo, eps, stream=None) -> int:
    return load().qe_rmsnorm1p(_ptr(x), _ptr(delta), _ptr(w), _ptr(out), rows, H, ldx, ldd, ldo,
                               eps, _stream(stream))


def argmax(x, rows, n, ldx, pv, pi, nb, out, idmap=None, stream=None) -> int:
    return load().qe_argmax(_ptr(x), rows, n, ldx, _ptr(pv), _ptr(pi), nb, _ptr(out), _ptr(idmap),
                            _stream(stream))


def gdn_step_n(qkv, z, b, a, ldp, ring, conv_w, A_log, dt_bias, norm_w, S, st_k, st_v, st_g, ctl,
               out, ldo, n, Hk, Hv, eps, stream=None) -> int:
    return load().qe_gdn_step_n(_ptr(qkv), _ptr(z), _ptr(b), _ptr(a), ldp, _ptr(ring), _ptr(conv_w),
                                _ptr(A_log), _ptr(dt_bias), _ptr(norm_w), _ptr(S), _ptr(st_k),
                                _ptr(st_v), _ptr(st_g), _ptr(ctl), _ptr(out), ldo, n, Hk, Hv, eps,
                                _stream(stream))
