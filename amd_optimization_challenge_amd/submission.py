"""Drop-in ``custom_kernel(data)`` for the mixed-mla entry point.

Mirrors mixed-mla/submission.py:626-644: same ``data`` tuple, same
``[total_q, H, 512]`` bf16 result.  Instead of routing on
``(batch_size, kv_seq_len)`` to AITER/Triton paths it always runs the gfx950
HIP pipeline (FP8 Q quant -> on-device split plan -> decode -> LSE combine)
from libmla_mi355x.so, and it honours ``config["sm_scale"]`` (the reference
ignores it, mixed-mla/submission.py:37) plus the optional ``num_heads``,
``kv_indices`` and ``kv_mode`` keys.  ``config["q_seq_len"] > 1`` runs the
reference's causal multi-token decode (uniform qo length,
competitor_submissions/mi355x_reference/reference.py:188-193; ``qo_indptr``
is taken to be ``arange * q_seq_len`` as generate_input makes it, :330), and
``config["return_lse"]`` also returns the f32 log-sum-exp
(mixed-mla/asm_dumps/aiter_mla.py:367-371).  ``config["page_size"] > 1`` takes
a paged cache the way AITER's mla_decode_fwd does (aiter_mla.py:149-175): the
caches shaped [pages, page_size, 1, row], ``kv_indptr`` over pages,
``config["kv_indices"]`` the page ids and ``config["kv_last_page_lens"]``.
``config["q_dtype"] = "bf16"`` takes the reference's a16w8 route (bf16 Q, fp8
cache, 16 heads; TASK/reference.py:55-58 Q_DTYPE) instead of a8w8.
``config["kv_mode"] = "auto"`` picks the cache by speed, as the reference's
custom_kernel routes each (batch, kv_len) to its fastest path
(mixed-mla/submission.py:626-644, MXFP4 Triton for the small shapes): see
``auto_kv_mode``.  Without the key the route is a8w8 over the fp8 cache, the
one the north-star tolerance (2e-2) holds for on every shape.
There is no fallback: a missing library or an unsupported shape raises.

The result lives in a buffer the operator keeps per (shape, device), as the
reference's own output cache does (mixed-mla/submission.py:115, 346-351): the
next call of the same shape on the same device overwrites it, so a caller that
keeps a result past that call clones it.  The evaluation harness reads each
result before the next call and then drops it (eval.py:243-248).  With the
workspace cached the same way, a call in steady state allocates nothing.
"""
from __future__ import annotations

import math

import torch

from . import ops
from .task import input_t, output_t

DEFAULT_SM_SCALE = 1.0 / math.sqrt(576.0)


def auto_kv_mode(num_heads: int, kv_data: dict) -> str:
    """The fastest route whose cache is present.  At 16 heads the MXFP4 cache
    (e2m1 K and V, 306 bytes a token against 576) wins on every task shape under
    the leaderboard protocol (MI355X, whole call: 4 x 8192 38.9 us against 40.4
    for fp8, 64 x 8192 90.1 against 130.9, 256 x 1024 62.1 against 84.3; 4 x
    1024 ties at 25.9 / 25.5) and passes the task's check (rtol = atol = 0.1,
    competitor_submissions/mi355x_reference/reference.py:372); bf16 Q (a16w8)
    was slower than a8w8 on all eight.  At 128 heads the fp8 cache is the one
    that reads fewest bytes (the mixed route reads both caches)."""
    if num_heads == 16 and "mxfp4" in kv_data:
        return "mxfp4"
    if "fp8" in kv_data:
        return "fp8"
    raise ValueError("kv_mode 'auto' needs the fp8 or (at 16 heads) the mxfp4 cache in kv_data")


# (rows, heads, device, return_lse) -> (out, lse or None)
_out_cache: dict = {}


def _outputs(rows: int, heads: int, device: torch.device, return_lse: bool):
    key = (rows, heads, device, return_lse)
    bufs = _out_cache.get(key)
    if bufs is None:
        out = torch.empty((rows, heads, ops.V_DIM), dtype=torch.bfloat16, device=device)
        lse = torch.empty((rows, heads), dtype=torch.float32, device=device) if return_lse else None
        bufs = _out_cache[key] = (out, lse)
    return bufs


def custom_kernel(data: input_t) -> output_t:
    q, kv_data, qo_indptr, kv_indptr, config = data
    q_seq_len = int(config.get("q_seq_len", 1))
    num_heads = q.shape[1]
    if int(config.get("num_heads", num_heads)) != num_heads:
        raise ValueError("config['num_heads'] does not match q.shape[1]")
    sm_scale = float(config.get("sm_scale", DEFAULT_SM_SCALE))
    kv_mode = config.get("kv_mode", "fp8")
    q_dtype = config.get("q_dtype", "fp8")
    if kv_mode == "auto":
        kv_mode = auto_kv_mode(num_heads, kv_data)
        # 16 heads: Q quantized per head row in the decode, which for <= 256
        # query rows also plans its own work (decode + combine: no amax pass)
        q_dtype = config.get("q_dtype", "fp8_row" if num_heads == 16 else "fp8")
    kv_indices = config.get("kv_indices")
    if q.shape[0] != (kv_indptr.numel() - 1) * q_seq_len:
        raise ValueError("q.shape[0] must equal batch * q_seq_len")
    if qo_indptr is not None and qo_indptr.numel() != kv_indptr.numel():
        raise ValueError("qo_indptr and kv_indptr must both have batch + 1 entries")
    page_size = int(config.get("page_size", 1))
    return_lse = bool(config.get("return_lse", False))
    out, lse = _outputs(q.shape[0], num_heads, q.device, return_lse)
    return ops.decode_fwd(q, kv_data, kv_indptr, kv_indices, sm_scale, kv_mode, out=out, q_seq_len=q_seq_len,
                          return_lse=return_lse, page_size=page_size,
                          kv_last_page_lens=config.get("kv_last_page_lens"),
                          q_dtype=q_dtype, lse=lse)
