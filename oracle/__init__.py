"""CPU oracle for the gated-attention decode path. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package. They use it as the checker or as the CPU baseline. It is never the thing
measured or shipped. The product path (``qengine_amd``) never imports it, and it fails loudly
when its HIP library is missing instead of falling back to the CPU.

Parity status per function (each is pinned by checks in ``tests/test_oracle.py``):
  rope_inv_freq, rope_cos_sin, apply_rope, rmsnorm1p, attention_qkv_from_proj,
  attention_core, attention_core_grouped, attn_prep, attn_decode, attn_prefill,
  flash_decode_fp64                                   -> pinned (closed forms, brute force,
                                                         invariants, bf16 rounding model; the
                                                         whole layer against HF transformers'
                                                         Qwen3_5Attention in
                                                         tests/test_oracle_hf.py)
  gemv_exact, gemv_bound, gemv_bf16_ref               -> pinned (brute-force loops, one-hot and
                                                         identity closed forms, NaN, the bound)
  step_oracle: embed, residual_rmsnorm1p, swiglu, argmax, accept, commit, mtp_select
                                                      -> pinned (closed forms, torch's own ops,
                                                         hand-worked step scenarios)
  kv8_oracle: decode, encode, dequantize              -> pinned (torch's float8_e4m3fn, closed
                                                         forms, ties, saturation)
  gdn_oracle: conv_silu, gates, l2norm, delta_update, gated_rmsnorm, GdnLayer.step_n / keep
                                                      -> pinned (HF transformers' qwen3_5 decode
                                                         functions, HF's chunked delta rule, the
                                                         fp64 matrix form, numpy convolution,
                                                         closed forms, rollback invariants)
"""
from .attn_oracle import *  # noqa: F401,F403
from .gemv_oracle import gemv_bf16_ref, gemv_bound, gemv_exact  # noqa: F401
from . import gdn_oracle, kv8_oracle, step_oracle  # noqa: F401
