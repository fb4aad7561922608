"""Drop-in ``custom_kernel(data)`` for the mixed-mla entry point.

Mirrors mixed-mla/submission.py:626-644: same ``data`` tuple, same
``[total_q, H, 512]`` bf16 result.  Instead of routing on
``(batch_size, kv_seq_len)`` to AITER/Triton paths it always runs the gfx950
HIP pipeline (FP8 Q quant -> on-device split plan -> decode -> LSE combine)
from libmla_mi355x.so, and it honours ``config["sm_scale"]`` (the reference
ignores it, mixed-mla/submission.py:37) plus the optional ``num_heads``,
``kv_indices`` and ``kv_mode`` keys.  There is no fallback: a missing library
or an unsupported shape raises.
"""
from __future__ import annotations

import math

import torch

from . import ops
from .task import input_t, output_t

DEFAULT_SM_SCALE = 1.0 / math.sqrt(576.0)


def custom_kernel(data: input_t) -> output_t:
    q, kv_data, qo_indptr, kv_indptr, config = data
    q_seq_len = int(config.get("q_seq_len", 1))
    if q_seq_len != 1:
        raise NotImplementedError("only decode (q_seq_len == 1) is implemented")
    num_heads = q.shape[1]
    if int(config.get("num_heads", num_heads)) != num_heads:
        raise ValueError("config['num_heads'] does not match q.shape[1]")
    sm_scale = float(config.get("sm_scale", DEFAULT_SM_SCALE))
    kv_mode = config.get("kv_mode", "fp8")
    kv_indices = config.get("kv_indices")
    if q.shape[0] != kv_indptr.numel() - 1:
        raise ValueError("q.shape[0] must equal batch (q_seq_len == 1)")
    return ops.decode_fwd(q, kv_data, kv_indptr, kv_indices, sm_scale, kv_mode)
