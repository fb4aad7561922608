"""The steps on either side of the absorbed decode (DeepSeek-style MLA).

Upstream, W_UK absorption turns a head's no-rope query into the latent space
the cache lives in: q_latent[b, h] = q_nope[b, h] @ W_UK[h] (128 -> 512), and
the decode's Q row is [q_latent, q_rope] (512 + 64 = 576).  Downstream, the
decode's latent output is lifted back by v_up_proj: y[b, h] = o[b, h] @ W_UV[h]
(512 -> 128), optionally quantized to per-tensor FP8 for the next GEMM (the
fusion vLLM does for this layer, mixed-mla/README.md:213-217).  The shared
MXFP4 quantizer of the mxfp4-mm / mxfp4-moe tasks is ``ops.pack_mxfp4`` (any
[rows, cols] bf16 with cols % 32 == 0).

Both products are per-head batched GEMMs with M = batch (tens to hundreds of
rows), dominated by streaming the weights once.  Each is one launch of this
package's HIP kernel (``mla_absorb_q`` / ``mla_v_up_proj``: a work-group owns
a head and 64 output columns, holds that weight slice in LDS and runs every
batch row over it on bf16 MFMAs with f32 accumulation); absorb_q also writes
the rope columns, and v_up_proj hands its per-work-group maxima straight to the
bit-exact per-tensor FP8 quantizer.
"""
from __future__ import annotations

import torch

from . import _lib
from .ops import _ptr, _stream

QK_NOPE = 128   # DeepSeek-V3/R1 qk_nope_head_dim
QK_ROPE = 64    # qk_rope_head_dim
LATENT = 512    # kv_lora_rank
V_HEAD = 128    # v_head_dim


def _check(*args) -> None:
    """args: (tensor, name, shape) triples; dtypes and shapes first, then devices."""
    for x, name, shape in args:
        if x.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bfloat16")
        if x.dim() != len(shape) or any(d != s for d, s in zip(x.shape, shape)):
            raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(x.shape)}")
    for x, name, _ in args:
        if x.device.type != "cuda":
            raise ValueError(f"{name} must be a CUDA (HIP) tensor")


def absorb_q(q_nope: torch.Tensor, q_rope: torch.Tensor, w_uk: torch.Tensor) -> torch.Tensor:
    """q_nope [B, H, 128], q_rope [B, H, 64], w_uk [H, 128, 512] (bf16) -> the
    decode's Q [B, H, 576] bf16 = [q_nope[b, h] @ w_uk[h], q_rope[b, h]]."""
    B, H = q_nope.shape[0], q_nope.shape[1]
    _check((q_nope, "q_nope", (B, H, QK_NOPE)), (q_rope, "q_rope", (B, H, QK_ROPE)),
           (w_uk, "w_uk", (H, QK_NOPE, LATENT)))
    q_nope, q_rope, w_uk = q_nope.contiguous(), q_rope.contiguous(), w_uk.contiguous()
    out = torch.empty((B, H, LATENT + QK_ROPE), dtype=torch.bfloat16, device=q_nope.device)
    with torch.cuda.device(q_nope.device):
        _lib.check(_lib.load().mla_absorb_q(_ptr(q_nope), _ptr(q_rope), _ptr(w_uk), B, H, _ptr(out),
                                            _stream()), "mla_absorb_q")
    return out


def v_up_proj(o: torch.Tensor, w_uv: torch.Tensor, quant_fp8: bool = False):
    """o [B, H, 512] (the decode output), w_uv [H, 512, 128] (bf16) ->
    y [B, H, 128] bf16 = o[b, h] @ w_uv[h]; with ``quant_fp8`` the pair
    (float8_e4m3fn [B, H, 128], f32 scale [1]) from the per-tensor quantizer."""
    B, H = o.shape[0], o.shape[1]
    _check((o, "o", (B, H, LATENT)), (w_uv, "w_uv", (H, LATENT, V_HEAD)))
    o, w_uv = o.contiguous(), w_uv.contiguous()
    y = torch.empty((B, H, V_HEAD), dtype=torch.bfloat16, device=o.device)
    q8 = scale = scratch = None
    if quant_fp8:
        q8 = torch.empty((B, H, V_HEAD), dtype=torch.float8_e4m3fn, device=o.device)
        scale = torch.empty(1, dtype=torch.float32, device=o.device)
        scratch = torch.empty(8192, dtype=torch.uint8, device=o.device)
    with torch.cuda.device(o.device):
        _lib.check(_lib.load().mla_v_up_proj(_ptr(o), _ptr(w_uv), B, H, _ptr(y), _ptr(q8), _ptr(scale),
                                             _ptr(scratch), 0 if scratch is None else scratch.numel(),
                                             _stream()), "mla_v_up_proj")
    return (q8, scale) if quant_fp8 else y
